"""LRDS replay and learning-signal capture on the GPU against the oracle.

Tolerance: the device computes in fp32 (as the reference does) while the
oracle computes in fp64; dw, dx and the signals are compared with
|gpu - oracle| <= RTOL * max|oracle| + ATOL per array."""
import numpy as np
import pytest

import oracle
from oracle import lrds
from heliox_amd import Sim, build_config
from heliox_amd import learn

pytestmark = pytest.mark.gpu

RTOL = 2e-4
ATOL = 1e-7


def close(gpu, ref, rtol=RTOL, atol=ATOL):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = float(np.max(np.abs(gpu - ref))) if ref.size else 0.0
    return err <= rtol * scale + atol, err, scale


@pytest.fixture(scope="module")
def sim(gpu_lib):
    g = Sim()
    g.load_model_from_spec(build_config(1, 2, 10.0))
    return g


def problem(seed, bns, K_len, ksteps, pre_frac=0.6, gain=0.3):
    rng = np.random.default_rng(seed)
    N = int(sum(bns))
    T = ksteps + 1
    blocks = [(rng.normal(0, 1, (bn, bn, K_len)) * gain / np.sqrt(bn)).astype(np.float32) for bn in bns]
    it = rng.normal(0, 1, (N, T)).astype(np.float32)
    dv = rng.normal(0, 0.3, (N, T)).astype(np.float32)
    dp = rng.normal(0, 0.3, (N, T)).astype(np.float32)
    it[:, 0] = dv[:, 0] = dp[:, 0] = 0
    pre = np.where(rng.random(N) < pre_frac, rng.integers(0, N, N), -1).astype(np.int32)
    return N, T, blocks, it, dv, dp, pre


CASES = [
    # bns, K_len, ksteps, percise, n_input, clip_thr
    ((37,), 3, 9, True, 2, 1e6),
    ((64, 70, 5), 8, 20, True, 4, 1e6),
    ((129, 31), 5, 12, True, 0, 1e6),
    ((40, 24), 1, 7, True, 3, 1e6),
    ((96, 33), 6, 14, False, 3, 1e6),
    ((50, 50), 4, 11, True, 3, 0.05),      # the threshold clips
]


@pytest.mark.parametrize("bns,K_len,ksteps,percise,n_input,thr", CASES)
def test_replay_from_signals_matches_oracle(sim, bns, K_len, ksteps, percise, n_input, thr):
    N, T, blocks, it, dv, dp, pre = problem(hash((bns, K_len)) % 1000, bns, K_len, ksteps)
    print(f"case from-signals bns={bns} K_len={K_len} ksteps={ksteps} percise={percise} thr={thr}", flush=True)
    rng = np.random.default_rng(1)
    po = np.sort(rng.choice(N, min(N, 9), replace=False)).astype(np.int32)
    pin = np.sort(rng.choice(N, max(n_input, 1), replace=False)).astype(np.int32)
    dL = rng.normal(0, 1, (ksteps, po.size)).astype(np.float32)
    assert sim.set_dense_blocks_f32(blocks) == K_len
    dw = np.zeros(N, np.float32)
    dx = np.zeros((pin.size, ksteps), np.float32)
    # eps keeps dx's division well conditioned (|dvtdw| < 0.2 in these problems)
    rc = sim.replay_compute_dw_dx_from_signals_into(it, dv, dp, dL, po, pin, pre, dw, dx, 0.1, percise,
                                                    grad_scale=1.3, eps=0.5, grad_l2norm_threshold=thr)
    assert rc == 0, sim.last_error()
    rdw, rdx, hist = lrds.replay(it, dv, dp, blocks, dL, po, pre, dt=0.1, percise=percise, pinput=pin,
                                 grad_scale=1.3, eps=0.5, grad_l2norm_threshold=thr, clip_strategy=1,
                                 variant="signals", keep_history=True)
    assert min(np.min(np.abs(h[:, pin] + 0.5)) for h in hist) > 0.2
    if thr < 1.0:
        assert max(np.linalg.norm(h) for h in hist) <= thr * (1 + 1e-6)
    ok, err, scale = close(dw, rdw)
    print(f"  dw max err {err:.3e} scale {scale:.3e}", flush=True)
    assert ok
    ok, err, scale = close(dx, rdx, rtol=5e-4)
    print(f"  dx max err {err:.3e} scale {scale:.3e}", flush=True)
    assert ok


def test_cached_capture_and_replay_match_oracle(sim):
    """Capture ExpSyn currents (pure_i), conductances (didv) and the cell's soma
    voltage (didvpre) on a config-2 model, then replay with dw and dx."""
    spec = build_config(2, 3, 20.0)
    spec.netcons["ExpSyn"].weight = spec.netcons["ExpSyn"].weight * 20
    g = Sim()
    g.load_model_from_spec(spec, add_monitors=False)
    es = spec.mechs["ExpSyn"]
    nsyn = es.nodes.size
    cell = spec.cell_of_node()[es.nodes]
    roots = np.arange(spec.ncell)
    out_vars = [("global", "v", int(r)) for r in roots]
    pure_vars = [("ExpSyn", "i", k) for k in range(nsyn)]
    didv_vars = [("ExpSyn", "g", k) for k in range(nsyn)]
    pre_vars = [("global", "v", int(cell[k])) for k in range(nsyn)]
    handles = lambda vs: [g.get_variable_handle(*v) for v in vs]
    ho, hp, hd, hq = handles(out_vars), handles(pure_vars), handles(didv_vars), handles(pre_vars)
    dest = np.arange(nsyn, dtype=np.int32)
    scale = np.linspace(0.5, 1.5, nsyn).astype(np.float32)
    k_mul, total = 4, 800
    blocks = [(np.random.default_rng(b).normal(0, 0.05, (n, n, 6))).astype(np.float32)
              for b, n in enumerate([nsyn // 2, nsyn - nsyn // 2])]
    assert g.set_dense_blocks_f32(blocks) == 6
    spec_c = learn.CaptureSpec(output_v_handles=ho, signals={
        "pure_i": learn.MappedSignal("pure_i", hp, dest, scale),
        "didv": learn.MappedSignal("didv", hd, dest, np.ones(nsyn, np.float32)),
        "didvpre": learn.MappedSignal("didvpre", hq, dest, np.full(nsyn, 1e-3, np.float32))},
        tstop_ms=total * spec.dt, k_mul=k_mul, percise=True, v_init=-65.0)
    print("case cached capture config-2 3 cells", flush=True)
    pack = learn.capture_signals_cached(g, spec_c, total_steps=total)
    # the same capture into host buffers
    T = total // k_mul + 1
    bufs = [np.zeros((T, nsyn), np.float32) for _ in range(3)]
    out2 = np.zeros_like(pack.output_vs_tn)
    assert g.simulate_and_capture_mapped_signals_into(out2, *bufs, ho, hp, dest, scale, hd, dest,
                                                      np.ones(nsyn, np.float32), hq, dest,
                                                      np.full(nsyn, 1e-3, np.float32), total * spec.dt, k_mul,
                                                      True, -65.0) == 0, g.last_error()
    assert np.array_equal(out2, pack.output_vs_tn)
    # oracle samples of the same variables
    mons = out_vars + pure_vars + didv_vars + pre_vars
    o = oracle.OracleSim(spec, monitors=mons)
    o.finitialize(-65.0)
    o.run(total * spec.dt)
    samples = o.traces()
    assert samples.shape[1] == total + 1
    chans = [(dest, scale), (dest, np.ones(nsyn)), (dest, np.full(nsyn, 1e-3))]
    ref_out, ref_sig = lrds.capture_from_samples(samples, len(out_vars), chans, k_mul, nsyn)
    assert np.max(np.abs(pack.output_vs_tn - ref_out)) < 1e-3
    for b, r in zip(bufs, ref_sig):
        ok, err, sc = close(b, r, rtol=1e-6, atol=1e-9)
        assert ok, (err, sc)
    assert np.count_nonzero(bufs[0]) > 0, "no synaptic current was captured"
    # replay over the cached signals
    rng = np.random.default_rng(5)
    po = np.arange(0, nsyn, 3, dtype=np.int32)
    pin = np.array([1, nsyn - 2], np.int32)
    pre = np.where(rng.random(nsyn) < 0.5, rng.integers(0, nsyn, nsyn), -1).astype(np.int32)
    dL = rng.normal(0, 1, (T - 1, po.size)).astype(np.float32)
    _, _, hist = lrds.replay(ref_sig[0].T, ref_sig[1].T, ref_sig[2].T, blocks, dL, po, pre, dt=0.1, percise=True,
                             keep_history=True)
    eps = float(np.float32(2.0 * max(np.max(np.abs(h[:, pin])) for h in hist) + 0.1))   # well-conditioned dx
    grads = learn.replay_grads_from_cached_signals(g, dLtdv_lr_ot=dL, poutput=po, pre_of_col=pre, dt_ms=0.1,
                                                   percise=True, pinput=pin, eps=eps)
    rdw, rdx, _ = lrds.replay(ref_sig[0].T, ref_sig[1].T, ref_sig[2].T, blocks, dL, po, pre, dt=0.1, percise=True,
                              pinput=pin, eps=eps)
    for name, a, r in (("dw", grads.dw_out_n, rdw), ("dx", grads.dx_lr_it, rdx)):
        ok, err, sc = close(a, r, rtol=5e-4)
        print(f"  {name} max err {err:.3e} scale {sc:.3e}", flush=True)
        assert ok
    # dw-only gives the same dw as dw+dx
    dw_only = learn.replay_dw_from_cached_signals(g, dLtdv_lr_ot=dL, poutput=po, pre_of_col=pre, dt_ms=0.1,
                                                  percise=True, eps=eps)
    assert np.array_equal(dw_only, grads.dw_out_n)
    # the streaming entry point (its own capture, then the replay) reproduces the
    # cached capture + replay exactly
    dw_c = np.zeros(nsyn, np.float32)
    dx_c = np.zeros((pin.size, T - 1), np.float32)
    assert g.replay_compute_dw_dx_from_cached_signals_into(dL, po, pin, pre, dw_c, dx_c, spec.dt, True,
                                                          eps=eps) == 0, g.last_error()
    dw_s = np.zeros(nsyn, np.float32)
    dx_s = np.zeros((pin.size, T - 1), np.float32)
    assert g.simulate_and_replay_dw_dx_streaming_into(
        dL, po, pin, pre, dw_s, dx_s, hp, dest, scale, hd, dest, np.ones(nsyn, np.float32), hq, dest,
        np.full(nsyn, 1e-3, np.float32), total * spec.dt, k_mul, True, -65.0, spec.dt, eps=eps) == 0, g.last_error()
    assert np.array_equal(dw_s, dw_c) and np.array_equal(dx_s, dx_c)
    assert np.count_nonzero(dw_s) > 0


def test_full_size_rows_match_oracle(sim):
    """N = 2048 in 16 blocks of 128, K_len = 64, 80 ticks (the ring wraps): every
    row of dv/dw is its own recurrence, so a few rows of dw are checked against
    the oracle restricted to them; dw scales exactly with dLtdv."""
    bns = (128,) * 16
    N, T, blocks, it, dv, dp, pre = problem(21, bns, 64, 80, gain=0.5)
    rng = np.random.default_rng(2)
    po = np.sort(rng.choice(N, 64, replace=False)).astype(np.int32)
    dL = rng.normal(0, 1, (T - 1, po.size)).astype(np.float32)
    assert sim.set_dense_blocks_f32(blocks) == 64
    print("case full-size replay N=2048 K_len=64 ksteps=80", flush=True)
    dw = np.zeros(N, np.float32)
    dx = np.zeros((1, T - 1), np.float32)
    pin = np.array([0], np.int32)
    assert sim.replay_compute_dw_dx_from_signals_into(it, dv, dp, dL, po, pin, pre, dw, dx, 0.025, True,
                                                      clip_strategy=0) == 0, sim.last_error()
    rows = np.array([0, 127, 128, 1000, 2047])
    rdw, _, _ = lrds.replay(it, dv, dp, blocks, dL, po, pre, dt=0.025, percise=True, clip_strategy=0, rows=rows)
    ok, err, sc = close(dw[rows], rdw)
    print(f"  rows {rows.tolist()} max err {err:.3e} scale {sc:.3e}", flush=True)
    assert ok
    dw2 = np.zeros(N, np.float32)
    assert sim.replay_compute_dw_dx_from_signals_into(it, dv, dp, 2.0 * dL, po, pin, pre, dw2, dx, 0.025, True,
                                                      clip_strategy=0) == 0
    assert np.array_equal(dw2, 2.0 * dw)


def test_replay_errors(sim):
    N, T, blocks, it, dv, dp, pre = problem(3, (8,), 2, 4)
    dL = np.zeros((T - 1, 1), np.float32)
    dw = np.zeros(N, np.float32)
    dx = np.zeros((1, T - 1), np.float32)
    po, pin = np.array([0], np.int32), np.array([1], np.int32)
    sim.clear_dense_blocks()
    assert sim.replay_compute_dw_dx_from_signals_into(it, dv, dp, dL, po, pin, pre, dw, dx, 0.1, True) == -1
    assert "dense blocks not set" in sim.last_error()
    assert sim.set_dense_blocks_f32([np.zeros((3, 3, 2), np.float32), np.zeros((5, 5, 4), np.float32)]) == -1
    assert "K_len mismatch" in sim.last_error()
    assert sim.set_dense_blocks_f32(blocks) == 2
    bad = pre.copy()
    bad[2] = N
    assert sim.replay_compute_dw_dx_from_signals_into(it, dv, dp, dL, po, pin, bad, dw, dx, 0.1, True) == -1
    assert "out of range" in sim.last_error()
    assert sim.replay_compute_dw_dx_from_signals_into(it, dv, dp, dL[:-1], po, pin, pre, dw, dx[:, :-1], 0.1,
                                                      True) == -1
    assert "ksteps_total mismatch" in sim.last_error()
    assert sim.set_dense_blocks_f32([blocks[0][:4, :4]]) == 2
    assert sim.replay_compute_dw_dx_from_signals_into(it, dv, dp, dL, po, pin, pre, dw, dx, 0.1, True) == -1
    assert "total N mismatch" in sim.last_error()
    # a cached replay before any capture
    assert sim.set_dense_blocks_f32(blocks) == 2
    assert sim.replay_compute_dw_from_cached_signals_into(dL, po, pre, dw, 0.1, True) == -1
    assert "cached capture buffers not initialized" in sim.last_error()
