"""Helpers for comparing the HIP path with the CPU oracle on the same model."""
import ctypes
import dataclasses

import numpy as np

import oracle
from heliox_amd import Sim

V_TOL = 1e-4      # mV, max abs on fp64 voltage traces


def run_both(spec, tstop, v_init=-65.0, fusion=True, monitors=None, chunks=None):
    o = oracle.OracleSim(spec, monitors=monitors)
    o.finitialize(v_init)
    g = Sim()
    if monitors is not None:
        spec = dataclasses.replace(spec, monitors=list(monitors))
    g.set_fusion(fusion)
    g.load_model_from_spec(spec)
    g.finitialize(v_init)
    if chunks:
        for c in chunks:
            o.continue_run(c)
            g.continue_run(c)
    else:
        o.run(tstop)
        g.run(tstop)
    return o, g


def sorted_spikes(t, gid):
    order = np.lexsort((gid, t))
    return t[order], gid[order]


def compare_spikes(o, g, dt):
    ot, og = sorted_spikes(*o.spikes())
    gt, gg = sorted_spikes(*g.spikes())
    assert ot.size == gt.size, f"spike counts differ: oracle {ot.size}, gpu {gt.size}"
    for gid in np.unique(og):
        a = ot[og == gid]
        b = gt[gg == gid]
        assert a.size == b.size, f"gid {gid}: {a.size} vs {b.size} spikes"
        if a.size:
            assert np.max(np.abs(a - b)) <= dt * 1.000001, f"gid {gid}: spike times differ by more than dt"
    return ot.size


def device_free_bytes() -> int:
    """Free device memory after the device has drained (hipDeviceSynchronize, hipMemGetInfo)
    from the HIP runtime the library is linked against, already loaded in the process."""
    hip = ctypes.CDLL("libamdhip64.so.7")
    assert hip.hipDeviceSynchronize() == 0
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return int(free.value)

