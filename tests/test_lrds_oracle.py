"""Pinning of the LRDS replay oracle (oracle/lrds.py) on the CPU.

The replay computes dv/dw of a linear recurrent network.  The main check
builds that network explicitly: currents I_k(s) = gs w_k It[k, s] (direct) and
dIt/dv[k, s] V_k(s-1) + dIt/dvpre[k, s] V_pre(k)(s-1) (feedback) drive
voltages through the block kernels,

  V_c(t) = dt sum_{s = t-tw+1..t} ( sum_{i in blk(c)} K_b[i][c][L-1-(t-s)] gs w_i It[i, s]
                                 + sum_{k in blk(c)} K_b[c][k][L-1-(t-s)] (feedback of k at s) ),

and simulates it forward once per unit weight w = e_i: V(t) is then exactly
row i of dvtdw_t.  Nothing in that simulation shares code with the oracle's
windowed, slot-ring formulation.
"""
import numpy as np
import pytest

from oracle import lrds


def make_problem(seed, bns, K_len, ksteps, pre_frac=0.6, cross=True):
    rng = np.random.default_rng(seed)
    N = int(sum(bns))
    T = ksteps + 1
    blocks = [rng.normal(0, 1.0, (bn, bn, K_len)) * 0.3 for bn in bns]
    it = rng.normal(0, 1, (N, T))
    dv = rng.normal(0, 0.3, (N, T))
    dp = rng.normal(0, 0.3, (N, T))
    it[:, 0] = dv[:, 0] = dp[:, 0] = 0.0
    pre = np.full(N, -1, np.int64)
    has = rng.random(N) < pre_frac
    pre[has] = rng.integers(0, N, has.sum()) if cross else np.arange(N)[has]
    return N, T, blocks, it, dv, dp, pre


def linear_network_rows(N, T, blocks, it, dv, dp, pre, dt, gs, K_len):
    """Forward simulation of the linear network for each unit weight: J[t][i] = V(t) with w = e_i."""
    starts, bns = lrds.block_layout(blocks)
    blk = np.repeat(np.arange(len(blocks)), bns)
    ks = T - 1
    J = np.zeros((ks + 1, N, N))
    for i in range(N):
        V = np.zeros((ks + 1, N))
        Id = np.zeros((ks + 1, N))
        Ifb = np.zeros((ks + 1, N))
        for t in range(1, ks + 1):
            Id[t, i] = gs * it[i, t]
            vp = np.where(pre >= 0, V[t - 1][np.maximum(pre, 0)], 0.0)
            Ifb[t] = dv[:, t] * V[t - 1] + dp[:, t] * vp
            for c in range(N):
                b = blk[c]
                S, bn = starts[b], bns[b]
                K = blocks[b]
                acc = 0.0
                for s in range(max(1, t - K_len + 1), t + 1):
                    tap = K_len - 1 - (t - s)
                    for k in range(S, S + bn):
                        acc += K[k - S, c - S, tap] * Id[s, k] + K[c - S, k - S, tap] * Ifb[s, k]
                V[t, c] = dt * acc
        J[:, i, :] = V
    return J


@pytest.mark.parametrize("bns,K_len,ksteps", [((3, 2, 4), 4, 9), ((5,), 1, 4), ((2, 3), 6, 5)])
def test_replay_equals_linear_network_jacobian(bns, K_len, ksteps):
    dt, gs = 0.025 * 4, 1.7
    N, T, blocks, it, dv, dp, pre = make_problem(7, bns, K_len, ksteps)
    rng = np.random.default_rng(3)
    po = np.array([0, N - 1, N // 2])
    dL = rng.normal(0, 1, (ksteps, po.size))
    dw, dx, hist = lrds.replay(it, dv, dp, blocks, dL, po, pre, dt=dt, percise=True, grad_scale=gs,
                               clip_strategy=0, keep_history=True)
    J = linear_network_rows(N, T, blocks, it, dv, dp, pre, dt, gs, K_len)
    for t in range(1, ksteps + 1):
        assert np.allclose(hist[t - 1], J[t], rtol=1e-12, atol=1e-13), t
    # dw is the gradient of L = (1/ks) sum_t sum_o dL[t-1, o] V_po(t)
    want = sum(J[t][:, po] @ dL[t - 1] for t in range(1, ksteps + 1)) / ksteps
    assert np.allclose(dw, want, rtol=1e-12, atol=1e-14)


def test_base_term_alone_is_a_windowed_convolution():
    """Without the precise correction dvtdw is block diagonal: a causal
    convolution of each row's It with the kernel taps K[i][j][L-1-lag]."""
    N, T, blocks, it, dv, dp, pre = make_problem(11, (4, 3), 5, 12)
    dt, gs = 0.1, 0.5
    _, _, hist = lrds.replay(it, None, None, blocks, np.zeros((T - 1, 1)), [0], pre, dt=dt, percise=False,
                             grad_scale=gs, clip_strategy=0, keep_history=True)
    starts, bns = lrds.block_layout(blocks)
    for b, K in enumerate(blocks):
        S, bn = starts[b], bns[b]
        for i in range(bn):
            for j in range(bn):
                kern = K[i, j, ::-1]          # lag 0 first
                conv = np.convolve(it[S + i], kern)[:T]
                for t in range(1, T):
                    # lags reaching back to column 0 (outside the window) are excluded;
                    # column 0 of It is zero, so the full convolution agrees
                    assert abs(hist[t - 1][S + i, S + j] - dt * gs * conv[t]) < 1e-12
    # off-diagonal blocks stay zero
    assert np.all(hist[-1][:4, 4:] == 0) and np.all(hist[-1][4:, :4] == 0)


def test_clipping_scales_by_running_minimum_of_threshold_ratios():
    """With eps = 0 the clipped replay is the unclipped one times
    c_T = min(1, min_t thr / ||dvtdw_t||), for dw and dx alike."""
    N, T, blocks, it, dv, dp, pre = make_problem(5, (6,), 3, 8)
    rng = np.random.default_rng(2)
    it = np.abs(it) + 0.5                   # dense, non-zero columns (dx divides by them)
    it[:, 0] = 0
    dv *= 0.1
    dp *= 0.1
    dL = rng.normal(0, 1, (T - 1, 2))
    po = [1, 4]
    pin = [0, 3, 5]
    kw = dict(dt=0.2, percise=True, pinput=pin, eps=0.0)
    dw_u, dx_u, hist_u = lrds.replay(it, dv, dp, blocks, dL, po, pre, clip_strategy=0, keep_history=True, **kw)
    norms = np.array([np.linalg.norm(h) for h in hist_u])
    thr = float(np.float32(np.median(norms)))
    dw_c, dx_c, hist_c = lrds.replay(it, dv, dp, blocks, dL, po, pre, clip_strategy=1, keep_history=True,
                                     grad_l2norm_threshold=thr, **kw)
    c = np.minimum.accumulate(np.minimum(1.0, thr / norms))
    assert c[-1] < 1.0, "the threshold should clip"
    for t in range(T - 1):
        assert np.allclose(hist_c[t], c[t] * hist_u[t], rtol=1e-6)
        assert np.linalg.norm(hist_c[t]) <= thr * (1 + 1e-6)
    assert np.allclose(dw_c, c[-1] * dw_u, rtol=1e-6)
    assert np.allclose(dx_c, c[-1] * dx_u, rtol=1e-6)


def test_clip_schedule_by_variant():
    """cached: strategy 1 checks every tick, others every clip_check_every;
    from-signals: only strategy 1, every clip_check_every (LearnRuntime.cpp:2238, 663)."""
    due = lrds._clip_due
    assert [due("cached", 1, 3, t) for t in range(1, 5)] == [True] * 4
    assert [due("cached", 2, 3, t) for t in range(1, 7)] == [False, False, True, False, False, True]
    assert [due("signals", 1, 2, t) for t in range(1, 5)] == [False, True, False, True]
    assert not any(due("signals", 2, 1, t) for t in range(1, 5))
    assert not any(due("cached", 0, 1, t) for t in range(1, 5))


def test_dx_single_column_closed_form():
    """N = 1, K_len = 1, no correction: dvtdw_t = dt gs K It_t, w_t = dvtdw_t dL_t,
    dx_t = w_t / (dvtdw_t + eps) * dvtdw_t."""
    K = np.array([[[1.5]]])
    it = np.array([[0.0, 0.4, -1.0, 2.0]])
    dL = np.array([[0.5], [2.0], [-1.0]])
    dt, gs, eps = 0.1, 2.0, 1e-3
    dw, dx, _ = lrds.replay(it, None, None, [K], dL, [0], [-1], dt=dt, percise=False, grad_scale=gs, pinput=[0],
                            eps=eps, clip_strategy=0)
    d = dt * gs * 1.5 * it[0, 1:]
    w = d * dL[:, 0]
    assert np.allclose(dx[0], w / (d + eps) * d, rtol=1e-14)
    assert np.isclose(dw[0], w.mean(), rtol=1e-14)


def test_dw_linear_in_loss_gradient():
    N, T, blocks, it, dv, dp, pre = make_problem(9, (3, 3), 4, 7)
    rng = np.random.default_rng(4)
    a, b = rng.normal(0, 1, (T - 1, 2)), rng.normal(0, 1, (T - 1, 2))
    f = lambda L: lrds.replay(it, dv, dp, blocks, L, [0, 5], pre, dt=0.1, percise=True, clip_strategy=0)[0]
    assert np.allclose(f(2.0 * a - 3.0 * b), 2.0 * f(a) - 3.0 * f(b), rtol=1e-11, atol=1e-13)


def test_row_restricted_replay_matches_full_rows():
    N, T, blocks, it, dv, dp, pre = make_problem(13, (4, 2, 3), 5, 10)
    dL = np.random.default_rng(1).normal(0, 1, (T - 1, 3))
    full, _, _ = lrds.replay(it, dv, dp, blocks, dL, [0, 4, 8], pre, dt=0.1, percise=True, clip_strategy=0)
    rows = np.array([1, 5, 8])
    part, _, _ = lrds.replay(it, dv, dp, blocks, dL, [0, 4, 8], pre, dt=0.1, percise=True, clip_strategy=0,
                             rows=rows)
    assert np.allclose(part, full[rows], rtol=1e-13, atol=1e-15)


def test_capture_reduces_to_samples():
    """One item per column with scale 1: the captured signal is the fp32 sample
    every k_mul steps, row 0 zero; outputs are fp32 samples of every step."""
    rng = np.random.default_rng(0)
    samples = rng.normal(0, 10, (5, 13))
    out, (sig,) = lrds.capture_from_samples(samples, 2, [(np.array([2, 0, 1]), np.ones(3))], 4, 3)
    assert np.array_equal(out, samples[:2].T.astype(np.float32))
    assert sig.shape == (4, 3) and np.all(sig[0] == 0)
    for lr in range(1, 4):
        assert np.array_equal(sig[lr], samples[[3, 4, 2], lr * 4].astype(np.float32))
    # two items into one column are summed in input order with fp32 rounding
    _, (sig2,) = lrds.capture_from_samples(samples[:3], 1, [(np.array([0, 0]), np.array([0.5, 2.0]))], 2, 1)
    v = samples[1:3, 2].astype(np.float32)
    assert sig2[1, 0] == np.float32(np.float32(v[0] * np.float32(0.5)) + np.float32(v[1] * np.float32(2.0)))
