"""The allocation-free LRDS replay (hx_replay_compute_dw_dx_from_signals_into_noalloc)
against the allocating entry point, through the C ABI: identical dw and dx bits on two
calls in a row (the second smaller), the size limit refused with an error, and a
clipped, non-percise case.  The same kernels run over buffers carved from the
library's fixed scratch array, so the results are bit-identical."""
import ctypes as C

import numpy as np
import pytest

from heliox_amd import Sim, build_config, lib

pytestmark = pytest.mark.gpu

_F = C.POINTER(C.c_float)
_I = C.POINTER(C.c_int)


def fp(a):
    return a.ctypes.data_as(_F)


def ip(a):
    return a.ctypes.data_as(_I)


def problem(seed, bns, K_len, ksteps, n_out=7, n_in=3):
    rng = np.random.default_rng(seed)
    N = int(sum(bns))
    T = ksteps + 1
    blocks = [(rng.normal(0, 1, (bn, bn, K_len)) * 0.3 / np.sqrt(bn)).astype(np.float32) for bn in bns]
    sig = [rng.normal(0, s, (N, T)).astype(np.float32) for s in (1.0, 0.3, 0.3)]
    for x in sig:
        x[:, 0] = 0
    pre = np.where(rng.random(N) < 0.6, rng.integers(0, N, N), -1).astype(np.int32)
    po = np.sort(rng.choice(N, min(N, n_out), replace=False)).astype(np.int32)
    pin = np.sort(rng.choice(N, n_in, replace=False)).astype(np.int32)
    dL = rng.normal(0, 1, (ksteps, po.size)).astype(np.float32)
    return N, T, blocks, sig, pre, po, pin, dL


def call(sim, entry, N, T, sig, pre, po, pin, dL, percise, thr):
    dw = np.full(N, np.nan, np.float32)
    dx = np.full((pin.size, T - 1), np.nan, np.float32)
    rc = getattr(lib(), entry)(sim._h, fp(sig[0]), fp(sig[1]), fp(sig[2]), N, T, fp(dL), T - 1, po.size, ip(po),
                               ip(pin), pin.size, ip(pre), fp(dw), fp(dx), 0.1, int(percise), 1.3, 0.5, thr, 1, 1)
    return rc, dw, dx


@pytest.fixture(scope="module")
def sim(gpu_lib):
    g = Sim()
    g.load_model_from_spec(build_config(1, 2, 10.0))
    return g


CASES = [
    # (bns, K_len, ksteps, percise, thr): a large call, then a smaller one, on the same scratch
    [((96, 64, 33), 8, 40, True, 1e6), ((37,), 3, 9, True, 1e6)],
    [((70, 58), 6, 25, False, 0.05), ((40, 24), 1, 7, True, 0.05)],
]


@pytest.mark.parametrize("pair", CASES)
def test_noalloc_replay_equals_allocating_replay(sim, pair):
    for bns, K_len, ksteps, percise, thr in pair:
        N, T, blocks, sig, pre, po, pin, dL = problem(ksteps, bns, K_len, ksteps)
        print(f"case noalloc replay bns={bns} K_len={K_len} ksteps={ksteps} percise={percise} thr={thr}", flush=True)
        assert sim.set_dense_blocks_f32(blocks) == K_len
        rc, dw_a, dx_a = call(sim, "hx_replay_compute_dw_dx_from_signals_into", N, T, sig, pre, po, pin, dL,
                              percise, thr)
        assert rc == 0, sim.last_error()
        rc, dw_n, dx_n = call(sim, "hx_replay_compute_dw_dx_from_signals_into_noalloc", N, T, sig, pre, po, pin,
                              dL, percise, thr)
        assert rc == 0, sim.last_error()
        assert np.all(np.isfinite(dw_a)) and np.all(np.isfinite(dx_a))
        assert np.array_equal(dw_n, dw_a) and np.array_equal(dx_n, dx_a)
        assert np.max(np.abs(dw_a)) > 0


def test_noalloc_replay_refuses_problems_beyond_its_scratch(sim):
    # N = 1024, K_len = 16, percise: the two history rings alone are 2 x 17 x 4 MiB
    N, T = 1024, 6
    blocks = [np.zeros((512, 512, 16), np.float32), np.zeros((512, 512, 16), np.float32)]
    assert sim.set_dense_blocks_f32(blocks) == 16
    sig = [np.zeros((N, T), np.float32) for _ in range(3)]
    pre = np.full(N, -1, np.int32)
    po = np.arange(4, dtype=np.int32)
    pin = np.arange(2, dtype=np.int32)
    dL = np.zeros((T - 1, 4), np.float32)
    rc, _, _ = call(sim, "hx_replay_compute_dw_dx_from_signals_into_noalloc", N, T, sig, pre, po, pin, dL, True, 1e6)
    assert rc != 0
    assert "scratch" in sim.last_error()


def test_noalloc_replay_allocates_nothing(sim):
    """After one call, further calls with other tick counts, with and without the precise
    term and clipping, leave the free device memory unchanged (hipMemGetInfo).  The dense blocks are set before the measured region: setting them allocates."""
    from parity_util import device_free_bytes

    N, T, blocks, sig, pre, po, pin, dL = problem(11, (48, 40), 5, 20)
    assert sim.set_dense_blocks_f32(blocks) == 5
    rc, _, _ = call(sim, "hx_replay_compute_dw_dx_from_signals_into_noalloc", N, T, sig, pre, po, pin, dL, True, 1e6)
    assert rc == 0, sim.last_error()
    free0 = device_free_bytes()
    for t_cut, percise, thr in [(T, True, 1e6), (T - 4, False, 0.5), (T - 11, True, 0.05), (T, False, 1e6)] * 3:
        sub = [x[:, :t_cut].copy() for x in sig]
        rc, dw, _ = call(sim, "hx_replay_compute_dw_dx_from_signals_into_noalloc", N, t_cut, sub, pre, po, pin,
                         dL[: t_cut - 1].copy(), percise, thr)
        assert rc == 0, sim.last_error()
        assert np.all(np.isfinite(dw))
    free1 = device_free_bytes()
    print(f"  free device memory before {free0} after {free1}", flush=True)
    assert free1 == free0
