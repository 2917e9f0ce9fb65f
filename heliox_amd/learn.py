"""Learning-signal capture and LRDS gradient replay on a ``heliox_amd.Sim``.

The public names, dataclass fields and call signatures are those of the
reference's ``heliox_learn.signals`` module (signals.py:9-276), so callers of
that module run unchanged.  Underneath, every call goes straight to the C ABI
(``include/heliox.h``):

  capture_signals_cached           -> hx_simulate_and_capture_mapped_signals_cached
  replay_grads_from_cached_signals -> hx_replay_compute_dw[_dx]_from_cached_signals_into
  replay_dw_from_cached_signals    -> hx_replay_compute_dw_from_cached_signals_into

The library keeps the captured (T, N) signals in HBM between the capture and
the replays; the host only sees the per-step output voltages and the gradients.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping, Optional, Sequence, Tuple

import numpy as np

# The three channels a capture can carry, in the order the C ABI takes them.
CHANNELS: Tuple[str, str, str] = ("pure_i", "didv", "didvpre")


@dataclass(frozen=True)
class MappedSignal:
    """One captured channel: at each capture point the values behind ``handles``
    (variable handles of the Sim) are rounded to fp32, multiplied by ``scale`` and
    added into column ``dest`` of an N-column signal (signals.py:9-38)."""

    name: str
    handles: Sequence[int]
    dest: np.ndarray   # int32, one column index per handle
    scale: np.ndarray  # float32, one factor per handle

    def __post_init__(self) -> None:
        nh = len(self.handles)
        for field_name, want in (("dest", np.int32), ("scale", np.float32)):
            arr = getattr(self, field_name)
            if not isinstance(arr, np.ndarray) or arr.ndim != 1:
                raise ValueError(f"signal {self.name!r}: {field_name} has to be a one-dimensional ndarray")
            if arr.shape[0] != nh:
                raise ValueError(f"signal {self.name!r}: {nh} handles but {arr.shape[0]} {field_name} entries")
            if arr.dtype != want:
                raise TypeError(f"signal {self.name!r}: {field_name} is {arr.dtype}, expected {np.dtype(want)}")


def empty_signal(name: str) -> MappedSignal:
    """A channel with no handles (it contributes nothing to the signal)."""
    return MappedSignal(name, (), np.empty(0, np.int32), np.empty(0, np.float32))


@dataclass(frozen=True)
class CaptureSpec:
    """One forward run with capture (signals.py:52-71).  The ``pure_i`` channel's
    largest dest sets N; ``didv``/``didvpre`` are used when ``percise`` is set."""

    output_v_handles: Sequence[int]
    signals: Mapping[str, MappedSignal]
    tstop_ms: float
    k_mul: int
    percise: bool
    v_init: float


@dataclass(frozen=True)
class CapturedPack:
    """What a capture returns to the host; the signals themselves stay on the device."""

    output_vs_tn: np.ndarray   # float32, (total_steps + 1, n_output)
    k_mul: int
    percise: bool

    @property
    def total_steps(self) -> int:
        rows, _ = self.output_vs_tn.shape
        return rows - 1

    @property
    def n_output(self) -> int:
        _, cols = self.output_vs_tn.shape
        return cols

    @property
    def ksteps_total(self) -> int:
        # learning-rate ticks: one per k_mul steps, the partial tail dropped
        return divmod(self.total_steps, int(self.k_mul))[0]


@dataclass(frozen=True)
class ReplayGrads:
    dw_out_n: np.ndarray               # float32, (N,)
    dx_lr_it: Optional[np.ndarray]     # float32, (n_input, ksteps_total), or None without inputs


def _sim(manager):
    """The Sim behind ``manager``: a Sim itself, or a wrapper holding it as ``client``
    (the reference's HelioXManager) or ``sim``."""
    for attr in ("client", "sim"):
        inner = getattr(manager, attr, None)
        if inner is not None:
            return inner
    return manager


def _vector(values, dtype, what: str) -> np.ndarray:
    out = np.ascontiguousarray(np.asarray(values, dtype=dtype))
    if out.ndim != 1:
        raise ValueError(f"{what}: expected a one-dimensional array, got shape {out.shape}")
    return out


def _channel_args(signals: Mapping[str, MappedSignal]) -> list:
    """Per channel (in CHANNELS order): handles, dest, scale as the Sim binding takes them."""
    unknown = set(signals) - set(CHANNELS)
    if unknown:
        raise ValueError(f"capture: unknown signal channel(s) {sorted(unknown)}; known: {list(CHANNELS)}")
    args = []
    for name in CHANNELS:
        sig = signals.get(name)
        if sig is None:
            sig = empty_signal(name)
        args += [np.fromiter((int(h) for h in sig.handles), np.int32, len(sig.handles)), sig.dest, sig.scale]
    return args


def _raise_on_failure(rc: int, sim, call: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{call} returned {rc}: {sim.last_error()}")


def capture_signals_cached(manager, spec: CaptureSpec, *, total_steps: int, dtype=np.float32) -> CapturedPack:
    """finitialize(v_init), then ``total_steps`` steps; the output handles are sampled
    after finitialize and after every step, the mapped channels every ``k_mul`` steps
    into the device-side signal cache (signals.py:222-276)."""
    sim = _sim(manager)
    outs = _vector(spec.output_v_handles, np.int32, "capture output_v_handles")
    steps, k_mul = int(total_steps), int(spec.k_mul)
    if outs.size == 0:
        raise ValueError("capture: no output voltage handles")
    if steps < 1 or k_mul < 1:
        raise ValueError(f"capture: total_steps ({steps}) and k_mul ({k_mul}) have to be at least 1")
    if np.dtype(dtype) != np.float32:
        raise TypeError("capture: the library writes float32 outputs")
    output_vs_tn = np.zeros((steps + 1, outs.size), np.float32)
    rc = sim.simulate_and_capture_mapped_signals_cached(
        output_vs_tn, outs, *_channel_args(spec.signals), float(spec.tstop_ms), k_mul, bool(spec.percise),
        float(spec.v_init))
    _raise_on_failure(rc, sim, "simulate_and_capture_mapped_signals_cached")
    return CapturedPack(output_vs_tn, k_mul, bool(spec.percise))


def replay_grads_from_cached_signals(manager, *, dLtdv_lr_ot, poutput, pre_of_col, dt_ms: float, percise: bool,
                                     pinput=None, grad_scale: float = 1.0, eps: float = 1e-6,
                                     grad_l2norm_threshold: float = 1e6, clip_strategy: int = 1,
                                     clip_check_every: int = 1) -> ReplayGrads:
    """dw over the N replay columns, and dx for the ``pinput`` columns when there are
    any, from the signals of the last cached capture (signals.py:102-183)."""
    sim = _sim(manager)
    dl = np.ascontiguousarray(np.asarray(dLtdv_lr_ot, dtype=np.float32))
    if dl.ndim != 2:
        raise ValueError(f"replay: dLtdv_lr_ot has to be (ksteps_total, n_output), got shape {dl.shape}")
    outs = _vector(poutput, np.int32, "replay poutput")
    pre = _vector(pre_of_col, np.int32, "replay pre_of_col")
    ins = None if pinput is None else _vector(pinput, np.int32, "replay pinput")
    knobs = {"dt_ms": float(dt_ms), "percise": bool(percise), "grad_scale": float(grad_scale), "eps": float(eps),
             "grad_l2norm_threshold": float(grad_l2norm_threshold), "clip_strategy": int(clip_strategy),
             "clip_check_every": int(clip_check_every)}
    dw = np.zeros(pre.size, np.float32)
    if ins is None or ins.size == 0:
        rc = sim.replay_compute_dw_from_cached_signals_into(dl, outs, pre, dw, **knobs)
        _raise_on_failure(rc, sim, "replay_compute_dw_from_cached_signals_into")
        return ReplayGrads(dw, None)
    dx = np.zeros((ins.size, dl.shape[0]), np.float32)
    rc = sim.replay_compute_dw_dx_from_cached_signals_into(dl, outs, ins, pre, dw, dx, **knobs)
    _raise_on_failure(rc, sim, "replay_compute_dw_dx_from_cached_signals_into")
    return ReplayGrads(dw, dx)


def replay_dw_from_cached_signals(manager, *, dLtdv_lr_ot, poutput, pre_of_col, dt_ms: float, percise: bool,
                                  grad_scale: float = 1.0, eps: float = 1e-6, grad_l2norm_threshold: float = 1e6,
                                  clip_strategy: int = 1, clip_check_every: int = 1) -> np.ndarray:
    """Only dw (signals.py:186-219)."""
    grads = replay_grads_from_cached_signals(
        manager, dLtdv_lr_ot=dLtdv_lr_ot, poutput=poutput, pre_of_col=pre_of_col, dt_ms=dt_ms, percise=percise,
        grad_scale=grad_scale, eps=eps, grad_l2norm_threshold=grad_l2norm_threshold, clip_strategy=clip_strategy,
        clip_check_every=clip_check_every)
    return grads.dw_out_n
