"""Learning-signal capture and LRDS replay on a ``heliox_amd.Sim``.

Mirror of the reference's ``heliox_learn.signals`` surface (signals.py:9-276):
the same dataclasses and wrapper functions, calling the library's
``simulate_and_capture_mapped_signals_cached`` and
``replay_compute_dw[_dx]_from_cached_signals_into`` (LearnRuntime.cpp:1619-2457).
A ``manager`` is a ``Sim`` or anything exposing one as ``.client``.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping, Sequence

import numpy as np


@dataclass(frozen=True)
class MappedSignal:
    """A gather + scatter-add channel: the values of ``handles`` times ``scale``
    summed into columns ``dest`` of an N-column signal (signals.py:9-38)."""

    name: str
    handles: Sequence[int]
    dest: np.ndarray   # int32, (len(handles),)
    scale: np.ndarray  # float32, (len(handles),)

    def __post_init__(self) -> None:
        if self.dest.ndim != 1 or self.scale.ndim != 1:
            raise ValueError(f"MappedSignal({self.name}): dest/scale must be 1D arrays")
        n = len(self.handles)
        if int(self.dest.shape[0]) != n or int(self.scale.shape[0]) != n:
            raise ValueError(f"MappedSignal({self.name}): size mismatch: handles={n} "
                             f"dest={self.dest.shape[0]} scale={self.scale.shape[0]}")
        if self.dest.dtype != np.int32:
            raise TypeError(f"MappedSignal({self.name}): dest must be int32 (got {self.dest.dtype})")
        if self.scale.dtype != np.float32:
            raise TypeError(f"MappedSignal({self.name}): scale must be float32 (got {self.scale.dtype})")


def empty_signal(name: str) -> MappedSignal:
    return MappedSignal(name=name, handles=(), dest=np.zeros((0,), np.int32), scale=np.zeros((0,), np.float32))


@dataclass(frozen=True)
class CaptureSpec:
    """One forward pass with learning-signal capture (signals.py:52-71).
    ``signals['pure_i']`` must be non-empty: it fixes N."""

    output_v_handles: Sequence[int]
    signals: Mapping[str, MappedSignal]
    tstop_ms: float
    k_mul: int
    percise: bool
    v_init: float


@dataclass(frozen=True)
class CapturedPack:
    """Host outputs of a capture; the signals stay cached on the device."""

    output_vs_tn: np.ndarray   # float32, (total_steps + 1, n_output)
    k_mul: int
    percise: bool

    @property
    def total_steps(self) -> int:
        return int(self.output_vs_tn.shape[0]) - 1

    @property
    def n_output(self) -> int:
        return int(self.output_vs_tn.shape[1])

    @property
    def ksteps_total(self) -> int:
        return int(self.total_steps // int(self.k_mul))


@dataclass(frozen=True)
class ReplayGrads:
    dw_out_n: np.ndarray               # float32, (N,)
    dx_lr_it: np.ndarray | None        # float32, (n_input, ksteps_total)


def _client(manager):
    return getattr(manager, "client", manager)


def capture_signals_cached(manager, spec: CaptureSpec, *, total_steps: int, dtype=np.float32) -> CapturedPack:
    """Run finitialize + total_steps steps, capturing outputs every step and the
    mapped signals every k_mul steps (signals.py:222-276)."""
    client = _client(manager)
    n_output = len(spec.output_v_handles)
    if n_output <= 0:
        raise ValueError("capture_signals_cached: output_v_handles is empty")
    if total_steps <= 0:
        raise ValueError("capture_signals_cached: total_steps must be positive")
    if int(spec.k_mul) <= 0:
        raise ValueError("capture_signals_cached: k_mul must be positive")
    output_vs_tn = np.empty((int(total_steps) + 1, n_output), dtype=dtype, order="C")
    pure_i = spec.signals.get("pure_i") or empty_signal("pure_i")
    didv = spec.signals.get("didv") or empty_signal("didv")
    didvpre = spec.signals.get("didvpre") or empty_signal("didvpre")
    rc = client.simulate_and_capture_mapped_signals_cached(
        output_vs_tn, [int(h) for h in spec.output_v_handles],
        [int(h) for h in pure_i.handles], pure_i.dest, pure_i.scale,
        [int(h) for h in didv.handles], didv.dest, didv.scale,
        [int(h) for h in didvpre.handles], didvpre.dest, didvpre.scale,
        float(spec.tstop_ms), int(spec.k_mul), bool(spec.percise), float(spec.v_init))
    if rc != 0:
        raise RuntimeError(f"simulate_and_capture_mapped_signals_cached failed (rc={rc}): {client.last_error()}")
    return CapturedPack(output_vs_tn=output_vs_tn, k_mul=int(spec.k_mul), percise=bool(spec.percise))


def replay_grads_from_cached_signals(manager, *, dLtdv_lr_ot, poutput, pre_of_col, dt_ms: float, percise: bool,
                                     pinput=None, grad_scale: float = 1.0, eps: float = 1e-6,
                                     grad_l2norm_threshold: float = 1e6, clip_strategy: int = 1,
                                     clip_check_every: int = 1) -> ReplayGrads:
    """dw (and dx when pinput is given) from the cached signals (signals.py:102-183)."""
    client = _client(manager)
    dLtdv_lr_ot = np.asarray(dLtdv_lr_ot, dtype=np.float32, order="C")
    poutput = np.asarray(poutput, dtype=np.int32, order="C")
    pre_of_col = np.asarray(pre_of_col, dtype=np.int32, order="C")
    if dLtdv_lr_ot.ndim != 2:
        raise ValueError("replay_grads_from_cached_signals: dLtdv_lr_ot must be 2D")
    if poutput.ndim != 1 or pre_of_col.ndim != 1:
        raise ValueError("replay_grads_from_cached_signals: poutput/pre_of_col must be 1D")
    ksteps_total = int(dLtdv_lr_ot.shape[0])
    N = int(pre_of_col.shape[0])
    dw_out_n = np.zeros((N,), dtype=np.float32)
    if pinput is None:
        n_input = 0
    else:
        pinput = np.asarray(pinput, dtype=np.int32, order="C")
        if pinput.ndim != 1:
            raise ValueError("replay_grads_from_cached_signals: pinput must be 1D")
        n_input = int(pinput.shape[0])
    common = dict(dt_ms=float(dt_ms), percise=bool(percise), grad_scale=float(grad_scale), eps=float(eps),
                  grad_l2norm_threshold=float(grad_l2norm_threshold), clip_strategy=int(clip_strategy),
                  clip_check_every=int(clip_check_every))
    if n_input <= 0:
        rc = client.replay_compute_dw_from_cached_signals_into(dLtdv_lr_ot, poutput, pre_of_col, dw_out_n, **common)
        if rc != 0:
            raise RuntimeError(f"replay_compute_dw_from_cached_signals_into failed (rc={rc}): {client.last_error()}")
        return ReplayGrads(dw_out_n=dw_out_n, dx_lr_it=None)
    dx_lr_it = np.zeros((n_input, ksteps_total), dtype=np.float32)
    rc = client.replay_compute_dw_dx_from_cached_signals_into(dLtdv_lr_ot, poutput, pinput, pre_of_col, dw_out_n,
                                                              dx_lr_it, **common)
    if rc != 0:
        raise RuntimeError(f"replay_compute_dw_dx_from_cached_signals_into failed (rc={rc}): {client.last_error()}")
    return ReplayGrads(dw_out_n=dw_out_n, dx_lr_it=dx_lr_it)


def replay_dw_from_cached_signals(manager, *, dLtdv_lr_ot, poutput, pre_of_col, dt_ms: float, percise: bool,
                                  grad_scale: float = 1.0, eps: float = 1e-6, grad_l2norm_threshold: float = 1e6,
                                  clip_strategy: int = 1, clip_check_every: int = 1) -> np.ndarray:
    """dw only (signals.py:186-219)."""
    return replay_grads_from_cached_signals(
        manager, dLtdv_lr_ot=dLtdv_lr_ot, poutput=poutput, pre_of_col=pre_of_col, dt_ms=dt_ms, percise=percise,
        pinput=None, grad_scale=grad_scale, eps=eps, grad_l2norm_threshold=grad_l2norm_threshold,
        clip_strategy=clip_strategy, clip_check_every=clip_check_every).dw_out_n
