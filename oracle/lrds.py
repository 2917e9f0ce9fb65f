"""LRDS replay and learning-signal capture -- TEST INFRASTRUCTURE ONLY.

numpy restatement of the reference's learn gradient surface.  Only tests and
the CPU-baseline leg of the benchmark use it.

  capture_from_samples .. LearnRuntime::simulate_and_capture_mapped_signals_cached
                          (LearnRuntime.cpp:1619-1984): per-step fp32 gather of the
                          output handles, every k_mul steps a gather + scale +
                          scatter-add of each mapped channel into column N
                          (batch_gather.cu:5-10, batch_scatter_add.cu:4-13)
  replay ................ LearnRuntime::replay_compute_dw_dx_from_cached_signals_impl_
                          (LearnRuntime.cpp:1986-2296) and
                          replay_compute_dw_dx_from_signals_into (:372-727), with the
                          kernels of replay_dw_dx.cu: base term (:227-274), precise
                          correction (:282-325), Frobenius clip (:28-93, driver
                          :2238-2262 / :663-689), w_tick (:96-114), dx (:445-501).
                          One deliberate difference: for K_len = 1 the previous
                          tick's slice is kept (the reference writes past its
                          one-slice history there and reads zeros at tick 2)

Parity status (tests/test_lrds_oracle.py):
  replay dvtdw / dw ..... pinned: equals the exact Jacobian of a linear network
                          simulated forward with unit weights (non-symmetric K,
                          cross-block pre links, grad_scale != 1)
  clipping .............. pinned: with eps = 0 a clipped replay is the unclipped
                          one times min(1, min_t thr / ||dvtdw_t||)
  dx .................... pinned: single-column closed form; the eps = 0 clip
                          scaling above
  capture ............... pinned: reduces to the oracle step loop's own samples
"""
from __future__ import annotations

import numpy as np


def block_layout(blocks):
    """Block starts and sizes; blocks partition the columns contiguously
    (LearnRuntime.cpp:2134-2152)."""
    bns = [int(b.shape[0]) for b in blocks]
    starts = np.concatenate([[0], np.cumsum(bns)[:-1]]).astype(np.int64)
    return starts, np.array(bns, dtype=np.int64)


def _clip_due(variant, clip_strategy, every, t_lr):
    if clip_strategy == 0:
        return False
    if variant == "cached":      # LearnRuntime.cpp:2238-2239
        return clip_strategy == 1 or (t_lr % every) == 0
    # replay_compute_dw_dx_from_signals_into: LearnRuntime.cpp:663-665
    return clip_strategy == 1 and (t_lr % every) == 0


def replay(it_nt, ditdv_nt, ditdvpre_nt, blocks, dLtdv, poutput, pre_of_col, *, dt, percise,
           pinput=None, grad_scale=1.0, eps=1e-6, grad_l2norm_threshold=1e6, clip_strategy=1,
           clip_check_every=1, variant="cached", rows=None, keep_history=False):
    """Replay dv/dw over the LR ticks and return (dw, dx, history).

    it_nt, ditdv_nt, ditdvpre_nt: (N, T) signals, T = ksteps + 1 (column 0 unused).
    blocks: list of (bn, bn, K_len) arrays partitioning the N columns.
    dLtdv: (ksteps, n_output).  Computed in float64.

    rows: restrict the computation to these rows of dv/dw (a row of dvtdw only
    depends on its own row of the history), which is exact when no clipping and
    no dx are requested.  history: list of per-tick dvtdw (rows x N) when
    keep_history is set.
    """
    it = np.asarray(it_nt, np.float64)
    dv_sig = None if ditdv_nt is None else np.asarray(ditdv_nt, np.float64)
    dp_sig = None if ditdvpre_nt is None else np.asarray(ditdvpre_nt, np.float64)
    dL = np.asarray(dLtdv, np.float64)
    N, T = it.shape
    ksteps = dL.shape[0]
    if ksteps != T - 1:
        raise ValueError("ksteps_total mismatch")
    K_len = int(blocks[0].shape[2])
    starts, bns = block_layout(blocks)
    if int(bns.sum()) != N:
        raise ValueError("dense blocks do not cover N")
    Ks = [np.asarray(b, np.float64) for b in blocks]
    pre = np.asarray(pre_of_col, np.int64)
    po = np.asarray(poutput, np.int64)
    need_dx = pinput is not None and len(pinput) > 0
    if rows is None:
        rows = np.arange(N)
    else:
        rows = np.asarray(rows, np.int64)
        if need_dx or clip_strategy != 0:
            raise ValueError("row-restricted replay needs clip_strategy 0 and no dx")
    R = rows.size
    thr_f = float(np.float32(grad_l2norm_threshold))
    gs = float(grad_scale)

    # The reference's ring has K_len slices with the first write at slice 1; for
    # K_len = 1 that write lands one slice past the buffer (LearnRuntime.cpp:2202,
    # 2278-2280) and tick 2 then reads zeros.  Two slices keep the previous
    # tick's slice instead, which is what every K_len >= 2 ring does.
    nslot = max(K_len, 2)
    hist = np.zeros((nslot, R, N))
    dw_acc = np.zeros(R)
    dx = np.zeros((len(pinput), ksteps)) if need_dx else None
    history = []
    dV_pos = 1                                   # slot 0 stays the zero slice (LearnRuntime.cpp:2202)
    for t_lr in range(1, ksteps + 1):
        tw = min(t_lr, K_len)
        it_t0 = t_lr - tw + 1
        k_t0 = K_len - tw
        dv = np.zeros((R, N))
        # base term: dvtdw[s+bi, s+bj] = dt*gs * sum_t K[bi,bj,k_t0+t] * It[s+bi, it_t0+t]
        for b, K in enumerate(Ks):
            s, bn = int(starts[b]), int(bns[b])
            sel = np.nonzero((rows >= s) & (rows < s + bn))[0]
            if sel.size == 0:
                continue
            bi = rows[sel] - s
            Kw = K[bi][:, :, k_t0:K_len]                       # (nsel, bn, tw)
            itw = it[rows[sel], it_t0:it_t0 + tw]              # (nsel, tw)
            dv[sel, s:s + bn] = np.einsum("rjt,rt->rj", Kw, itw) * dt * gs
        if percise:
            win = [(dV_pos - tw + t) % nslot for t in range(tw)]
            H = hist[win]                                      # (tw, R, N)
            for b, K in enumerate(Ks):
                s, bn = int(starts[b]), int(bns[b])
                cols = np.arange(s, s + bn)
                D = H[:, :, s:s + bn]                          # dV[i, col_k]
                pb = pre[s:s + bn]
                P = np.where(pb[None, None, :] >= 0, H[:, :, np.maximum(pb, 0)], 0.0)
                a = dv_sig[cols, it_t0:it_t0 + tw].T           # (tw, bn): dItdv[col_k, it_t]
                c = dp_sig[cols, it_t0:it_t0 + tw].T
                X = D * a[:, None, :] + P * c[:, None, :]      # (tw, R, bn) over (t, i, k)
                Kw = K[:, :, k_t0:K_len]                       # (j, k, t)
                dv[:, s:s + bn] += np.tensordot(X, Kw, axes=([0, 2], [2, 1])) * dt
        if _clip_due(variant, clip_strategy, clip_check_every, t_lr):
            fin = np.isfinite(dv)
            if not fin.all():
                dv[~fin] = 0.0
            l2 = float(np.sqrt(max(0.0, float(np.sum(dv * dv)))))
            if l2 > thr_f and np.isfinite(l2):
                sc = float(np.float32(thr_f / l2))
                dv *= sc
                hist *= sc
                dw_acc *= sc
                if need_dx:
                    dx *= sc
                gs *= sc
        w_tick = dv[:, po] @ dL[t_lr - 1]
        dw_acc += w_tick
        if need_dx:
            colv = dv[:, np.asarray(pinput, np.int64)]         # (N, n_input)
            s_ = np.sum(w_tick[:, None] / (colv + eps), axis=0)
            b_ = np.sum(colv, axis=0)
            dx[:, t_lr - 1] = s_ * b_
        hist[dV_pos] = dv
        dV_pos = (dV_pos + 1) % nslot
        if keep_history:
            history.append(dv.copy())
    dw = dw_acc / ksteps
    return dw, dx, history


def capture_from_samples(samples, n_output, channels, k_mul, N):
    """Expected capture buffers from per-step samples of the captured variables.

    samples: (nvar, nstep + 1) fp64 values after finitialize (column 0) and after
    each step; rows 0..n_output-1 are the output handles, then each channel's
    handles in order.  channels: list of (dest, scale) per mapped channel
    (pure_i, didv, didvpre), aligned with their handle rows.

    Returns output_vs (nstep+1, n_output) fp32 and one (T, N) fp32 array per
    channel, T = nstep // k_mul + 1, filled by in-order fp32 scatter-add
    (value rounded to fp32, times scale rounded, added rounded)."""
    samples = np.asarray(samples, np.float64)
    nstep = samples.shape[1] - 1
    ks = nstep // k_mul
    out = samples[:n_output].T.astype(np.float32)
    res = []
    row = n_output
    for dest, scale in channels:
        dest = np.asarray(dest, np.int64)
        scale = np.asarray(scale, np.float32)
        buf = np.zeros((ks + 1, N), np.float32)
        for lr in range(1, ks + 1):
            vals = samples[row:row + dest.size, lr * k_mul].astype(np.float32)
            for q in range(dest.size):
                buf[lr, dest[q]] = np.float32(buf[lr, dest[q]] + np.float32(vals[q] * scale[q]))
        res.append(buf)
        row += dest.size
    return out, res
