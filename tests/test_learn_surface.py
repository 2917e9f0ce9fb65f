"""The Python learn surface (heliox_amd.learn) on the CPU: validation, and what it
hands the Sim binding, with a recording stand-in for the Sim (no GPU calls)."""
import numpy as np
import pytest

from heliox_amd import learn


class RecordingSim:
    def __init__(self, rc=0):
        self.calls = []
        self.rc = rc

    def last_error(self):
        return "recorded failure"

    def simulate_and_capture_mapped_signals_cached(self, out, outs, *rest):
        self.calls.append(("capture", out, outs, rest))
        out[:] = 1.5
        return self.rc

    def replay_compute_dw_from_cached_signals_into(self, dl, po, pre, dw, **kw):
        self.calls.append(("dw", dl, po, pre, kw))
        dw[:] = 2.0
        return self.rc

    def replay_compute_dw_dx_from_cached_signals_into(self, dl, po, pin, pre, dw, dx, **kw):
        self.calls.append(("dwdx", dl, po, pin, pre, kw))
        dw[:] = 3.0
        dx[:] = 4.0
        return self.rc


def sig(name, n, dest_dtype=np.int32, scale_dtype=np.float32):
    return learn.MappedSignal(name, list(range(n)), np.arange(n).astype(dest_dtype), np.ones(n, scale_dtype))


def test_mapped_signal_validation():
    sig("pure_i", 3)
    with pytest.raises(TypeError):
        sig("pure_i", 3, dest_dtype=np.int64)
    with pytest.raises(TypeError):
        sig("pure_i", 3, scale_dtype=np.float64)
    with pytest.raises(ValueError):
        learn.MappedSignal("x", [1, 2], np.zeros(3, np.int32), np.zeros(2, np.float32))
    with pytest.raises(ValueError):
        learn.MappedSignal("x", [1], np.zeros((1, 1), np.int32), np.zeros(1, np.float32))
    e = learn.empty_signal("didv")
    assert e.name == "didv" and len(e.handles) == 0 and e.dest.dtype == np.int32 and e.scale.dtype == np.float32


def test_captured_pack_properties():
    p = learn.CapturedPack(np.zeros((101, 3), np.float32), k_mul=4, percise=True)
    assert (p.total_steps, p.n_output, p.ksteps_total) == (100, 3, 25)
    p = learn.CapturedPack(np.zeros((11, 1), np.float32), k_mul=3, percise=False)
    assert p.ksteps_total == 3


def test_capture_marshalling_and_missing_channels():
    s = RecordingSim()
    spec = learn.CaptureSpec(output_v_handles=[7, 8], signals={"pure_i": sig("pure_i", 4)}, tstop_ms=1.0, k_mul=2,
                             percise=False, v_init=-65.0)
    pack = learn.capture_signals_cached(s, spec, total_steps=10)
    assert pack.output_vs_tn.shape == (11, 2) and np.all(pack.output_vs_tn == 1.5)
    _, out, outs, rest = s.calls[0]
    assert outs.dtype == np.int32 and list(outs) == [7, 8]
    # three channels of (handles, dest, scale), then tstop, k_mul, percise, v_init
    assert len(rest) == 13
    assert list(rest[0]) == [0, 1, 2, 3] and rest[3].size == 0 and rest[6].size == 0
    assert rest[9:] == (1.0, 2, False, -65.0)


class Manager:            # the reference's manager object exposes the Sim as .client
    def __init__(self, sim):
        self.client = sim


def test_capture_errors():
    s = RecordingSim(rc=-1)
    spec = learn.CaptureSpec([1], {"pure_i": sig("pure_i", 1)}, 1.0, 1, False, -65.0)
    with pytest.raises(RuntimeError, match="recorded failure"):
        learn.capture_signals_cached(Manager(s), spec, total_steps=4)
    with pytest.raises(ValueError):
        learn.capture_signals_cached(s, learn.CaptureSpec([], {}, 1.0, 1, False, -65.0), total_steps=4)
    with pytest.raises(ValueError):
        learn.capture_signals_cached(s, spec, total_steps=0)
    with pytest.raises(ValueError):
        learn.capture_signals_cached(s, learn.CaptureSpec([1], {"bogus": sig("bogus", 1)}, 1.0, 1, False, -65.0),
                                     total_steps=4)


def test_replay_dispatch():
    s = RecordingSim()
    dl = np.zeros((5, 2))
    g = learn.replay_grads_from_cached_signals(s, dLtdv_lr_ot=dl, poutput=[0, 1], pre_of_col=[-1, 0, 1],
                                               dt_ms=0.1, percise=True)
    assert g.dx_lr_it is None and np.all(g.dw_out_n == 2.0) and g.dw_out_n.shape == (3,)
    kind, dl_c, po, pre, kw = s.calls[-1]
    assert kind == "dw" and dl_c.dtype == np.float32 and kw["percise"] is True and kw["clip_strategy"] == 1
    g = learn.replay_grads_from_cached_signals(s, dLtdv_lr_ot=dl, poutput=[0, 1], pre_of_col=[-1, 0, 1],
                                               dt_ms=0.1, percise=False, pinput=[2])
    assert g.dx_lr_it.shape == (1, 5) and np.all(g.dx_lr_it == 4.0) and np.all(g.dw_out_n == 3.0)
    # an empty pinput is the dw-only call
    learn.replay_grads_from_cached_signals(s, dLtdv_lr_ot=dl, poutput=[0], pre_of_col=[0], dt_ms=0.1,
                                           percise=False, pinput=[])
    assert s.calls[-1][0] == "dw"
    dw = learn.replay_dw_from_cached_signals(s, dLtdv_lr_ot=dl, poutput=[0], pre_of_col=[0, 1], dt_ms=0.1,
                                             percise=False)
    assert dw.shape == (2,)
    with pytest.raises(ValueError):
        learn.replay_dw_from_cached_signals(s, dLtdv_lr_ot=np.zeros(5), poutput=[0], pre_of_col=[0], dt_ms=0.1,
                                            percise=False)
    with pytest.raises(RuntimeError):
        learn.replay_dw_from_cached_signals(RecordingSim(rc=-1), dLtdv_lr_ot=dl, poutput=[0], pre_of_col=[0],
                                            dt_ms=0.1, percise=False)
