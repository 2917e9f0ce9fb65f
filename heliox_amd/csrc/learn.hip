// HIP kernels of the learn gradient surface for gfx950: learning-signal
// capture and the LRDS replay (replay_dw_dx.cu:9-731 is the reference's CUDA
// version of the same arithmetic).
//
// Per LR tick t (window tw = min(t, K_len), signal times it_t0 = t - tw + 1 ...
// t, kernel taps k_t0 = K_len - tw ... K_len - 1) the replay forms
//
//   dvtdw_t[i, s+j] = [i in block] (sum_u K_b[i-s][j][k_t0+u] It[it_t0+u][i]) dt gs
//                   + dt sum_{u,k} K_b[j][k][k_t0+u] X_u[i, k]
//   X_u[i, k] = dvtdw_{t-tw+u}[i, s+k] dIt/dv[it_t0+u][s+k]
//             + dvtdw_{t-tw+u}[i, pre(s+k)] dIt/dvpre[it_t0+u][s+k]
//
// (base term replay_dw_dx.cu:227-274, correction :282-325).  The correction is
// a GEMM per block, (N x bn*tw) X times (bn*tw x bn) K: k_rp_corr computes it
// with v_mfma_f32_32x32x2f32, forming X on the fly from the history slices as
// it stages each 128-row x 32-tap chunk through LDS.  The pre(s+k) operand is
// read from a column-gathered copy of each slice made once when the slice is
// written (k_rp_pregather), so every history read is a contiguous row segment.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "learn.h"

namespace hx {
namespace {

typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;

// ---------------------------------------------------------------- capture
// batch_gather.cu:5-10 and batch_scatter_add.cu:4-13: outputs are gathered
// every step; every k_mul steps each channel's items are rounded to fp32,
// multiplied by their scale and summed per destination column.  Items of one
// column are summed in input order (the reference's atomics leave that order
// open), so the result is reproducible.
__global__ void k_lr_capture(CaptureArgs C, int sample, int lr) {
    int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g < C.n_out) {
        C.out_vs[static_cast<size_t>(sample) * C.n_out + g] = static_cast<float>(*C.out_ptr[g]);
        return;
    }
    if (lr <= 0) return;
    g -= C.n_out;
    const int ch = g / max(C.N, 1);
    const int col = g - ch * C.N;
    if (ch >= C.nch) return;
    const CaptureChannel& Q = C.ch[ch];
    float acc = 0.f;
    for (int q = Q.begin[col]; q < Q.begin[col + 1]; ++q)
        acc = __fadd_rn(acc, __fmul_rn(static_cast<float>(*Q.ptr[q]), Q.scale[q]));
    Q.buf[static_cast<size_t>(lr) * C.N + col] = acc;
}

// ---------------------------------------------------------------- base term
// replay_base_blocks_kernel (replay_dw_dx.cu:227-274): one thread per (i, j)
// of a diagonal block, taps summed in time order with fused multiply-adds.
__global__ void k_rp_base(ReplayBaseArgs A) {
    const int b = blockIdx.y;
    const int bn = A.bn[b];
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (b == 0 && e == 0) A.slot_scale[A.cur] = 1.f;
    if (e >= bn * bn) return;
    const int bi = e / bn;
    const int row = A.start[b] + bi;
    const float* K = A.kt1 + A.koff[b];
    const size_t plane = static_cast<size_t>(bn) * bn;
    float sum = 0.f;
    for (int u = 0; u < A.tw; ++u)
        sum = fmaf(K[static_cast<size_t>(A.k_t0 + u) * plane + e],
                   A.it[static_cast<size_t>(A.it_t0 + u) * A.N + row], sum);
    A.base[A.boff[b] + e] = sum * A.dt * (*A.gs);
}

// ---------------------------------------------------------------- correction GEMM
// Workgroup tile: 128 rows x TJ columns of one block (TJ = 64 or 128) with NT
// threads, the waves arranged as WR row groups x (NT/64/WR) column groups; a
// wave owns a (128/WR) x (TJ/WC) sub-tile, held as 32 x 32 accumulators of
// v_mfma_f32_32x32x2f32.  The reduction runs over (tap u, chunk of KC columns
// k).  Each chunk stages X -- formed from the history slice D and its
// column-gathered copy G, both read as contiguous row segments -- and the K
// taps through LDS, double-buffered, with the next chunk's global loads in
// flight while the MFMAs run.
// Measured on MI355X (N = 2048, 16 blocks of 128, K_len 64): 64-tap chunks
// (one 130 KB workgroup per CU) beat 32- and 16-tap chunks, and 8 waves of
// 32 x 64 sub-tiles beat 4 waves of 64 x 64.
constexpr int kCorrThreads = 512;
constexpr int kTI = 128;
constexpr int kKC = 64;
constexpr int kWR = 4;
constexpr int kAPad = kTI + 1;

template <int TJ>
__global__ __launch_bounds__(kCorrThreads) void k_rp_corr(ReplayCorrArgs A) {
    constexpr int NW = kCorrThreads / 64;               // waves
    constexpr int WC = NW / kWR;                        // column groups of waves
    constexpr int WTI = kTI / kWR, WTJ = TJ / WC;       // wave sub-tile
    constexpr int MR = WTI / 32, NC = WTJ / 32;         // accumulators per wave
    static_assert(MR >= 1 && NC >= 1 && WTI % 32 == 0 && WTJ % 32 == 0, "wave sub-tile must be 32-aligned");
    constexpr int ASTEP = kCorrThreads / kKC;           // A rows covered per pass
    constexpr int RA = kTI / ASTEP;                     // A elements per thread and array
    constexpr int BSTEP = kCorrThreads / TJ;            // B taps covered per pass
    constexpr int BR = kKC / BSTEP;                     // B elements per thread
    __shared__ float As[2][kKC][kAPad];                 // X chunk, [k][i]
    __shared__ float Bs[2][kKC][TJ];                    // K chunk, [k][j]
    __shared__ double red_s[NW];
    __shared__ int red_f[NW];

    const int2 tl = A.tiles[blockIdx.x];
    const int b = tl.x, j0 = tl.y;
    const int s = A.start[b], bn = A.bn[b];
    const int N = A.N;
    const int i0 = blockIdx.y * kTI;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave / WC, wc = wave % WC;
    const float* Kb = A.kt2 + A.koff[b];
    const size_t plane = static_cast<size_t>(bn) * bn;
    const int nkc = (bn + kKC - 1) / kKC;
    const int nchunk = A.tw * nkc;

    // staging coordinates: A element (row ai + ASTEP r, tap ak), B element (tap bk + BSTEP r, column bj)
    const int ak = tid % kKC, ai = tid / kKC;
    const int bj = tid % TJ, bk = tid / TJ;
    float rd[RA], rg[RA], rb[BR];
    float ca = 0.f, cp = 0.f;

    auto fetch = [&](int c) {
        const int u = c / nkc;
        const int k0 = (c - u * nkc) * kKC;
        const int h = (A.t_lr - A.tw + u) % A.R;
        const size_t hoff = static_cast<size_t>(h) * A.slice;
        const float* D = A.hist + hoff;
        const float* G = A.ghist + hoff;
        const int kc = k0 + ak;
        const bool kin = kc < bn;
        const int col = s + kc;
        const size_t tau = static_cast<size_t>(A.it_t0 + u);
        ca = 0.f;
        cp = 0.f;
        if (kin) {
            const float sig = A.slot_scale[h];
            ca = sig * A.dv[tau * N + col];
            cp = sig * A.dp[tau * N + col];
        }
#pragma unroll
        for (int r = 0; r < RA; ++r) {
            const int i = i0 + ai + ASTEP * r;
            float x = 0.f, y = 0.f;
            if (kin && i < N) {
                const size_t o = static_cast<size_t>(i) * N + col;
                // the history window streams through once per tick: keep it out of
                // the caches so the K taps, reused by every row tile, stay in L2
                x = __builtin_nontemporal_load(D + o);
                y = __builtin_nontemporal_load(G + o);
            }
            rd[r] = x;
            rg[r] = y;
        }
        const float* Kt = Kb + static_cast<size_t>(A.k_t0 + u) * plane;
        const int jj = j0 + bj;
#pragma unroll
        for (int r = 0; r < BR; ++r) {
            const int k = k0 + bk + BSTEP * r;
            rb[r] = (jj < bn && k < bn) ? Kt[static_cast<size_t>(k) * bn + jj] : 0.f;
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int r = 0; r < RA; ++r) As[buf][ak][ai + ASTEP * r] = rd[r] * ca + rg[r] * cp;
#pragma unroll
        for (int r = 0; r < BR; ++r) Bs[buf][bk + BSTEP * r][bj] = rb[r];
    };

    f16v acc[MR][NC];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int n = 0; n < NC; ++n)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[m][n][r] = 0.f;

    if (nchunk > 0) {
        fetch(0);
        stage(0);
        __syncthreads();
        const int kr = lane >> 5;
        const int ia = wr * WTI + (lane & 31);
        const int jb = wc * WTJ + (lane & 31);
        for (int c = 0; c < nchunk; ++c) {
            const int buf = c & 1;
            if (c + 1 < nchunk) fetch(c + 1);
#pragma unroll
            for (int q = 0; q < kKC / 2; ++q) {
                float av[MR], bv[NC];
#pragma unroll
                for (int m = 0; m < MR; ++m) av[m] = As[buf][2 * q + kr][ia + 32 * m];
#pragma unroll
                for (int n = 0; n < NC; ++n) bv[n] = Bs[buf][2 * q + kr][jb + 32 * n];
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int n = 0; n < NC; ++n)
                        acc[m][n] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[m], bv[n], acc[m][n], 0, 0, 0);
            }
            if (c + 1 < nchunk) stage(buf ^ 1);
            __syncthreads();
        }
    }

    // epilogue: accumulator (m, n) of a lane holds rows 32m + 8(r/4) + 4(lane/32) + r%4
    // and column 32n + lane%32 of its wave's sub-tile
    double sq = 0.0;
    int bad = 0;
    const float* base = A.base + A.boff[b];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int n = 0; n < NC; ++n) {
            const int jw = j0 + wc * WTJ + 32 * n + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = i0 + wr * WTI + 32 * m + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= N || jw >= bn) continue;
                float v = acc[m][n][r] * A.dt;
                if (row >= s && row < s + bn) v = base[static_cast<size_t>(row - s) * bn + jw] + v;
                if (A.sanitize) {
                    if (!isfinite(v)) {
                        v = 0.f;
                        bad = 1;
                    }
                    sq += static_cast<double>(v) * v;
                }
                A.out[static_cast<size_t>(row) * N + s + jw] = v;
            }
        }
    if (A.sanitize) {
        for (int o = 32; o > 0; o >>= 1) {
            sq += __shfl_xor(sq, o);
            bad |= __shfl_xor(bad, o);
        }
        if (lane == 0) {
            red_s[wave] = sq;
            red_f[wave] = bad;
        }
        __syncthreads();
        if (tid == 0) {
            double t = 0.0;
            int f = 0;
            for (int w = 0; w < NW; ++w) {
                t += red_s[w];
                f |= red_f[w];
            }
            const int wg = blockIdx.y * gridDim.x + blockIdx.x;
            A.norm_part[wg] = t;
            A.flag_part[wg] = f;
        }
    }
}

// G[i][c] = D[i][pre(c)] (0 without a pre column): the column-gathered copy of
// a new history slice, so the correction reads both operands row-contiguous.
__global__ void k_rp_pregather(const float* D, const int* pre, int N, float* G) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= N) return;
    const size_t row = static_cast<size_t>(blockIdx.y) * N;
    const int p = pre[c];
    G[row + c] = p >= 0 ? D[row + p] : 0.f;
}

// ---------------------------------------------------------------- clip
// replay_frobenius_*_kernel (replay_dw_dx.cu:28-93) and the driver's decision
// (LearnRuntime.cpp:2238-2262): l2 over the finite entries; above the
// threshold the tick's slice, the history, the accumulators and the grad
// scale are all multiplied by thr / l2.  The decision stays on the device.
__global__ void k_rp_clip(const double* part, const int* flag, int n, float thr, float* gs, float* slot_scale,
                          int R, float* tick_scale) {
    __shared__ double sh[kThreads];
    __shared__ float sc_sh;
    const int tid = threadIdx.x;
    double acc = 0.0;
    for (int q = tid; q < n; q += kThreads) acc += part[q];
    sh[tid] = acc;
    __syncthreads();
    for (int st = kThreads / 2; st > 0; st >>= 1) {
        if (tid < st) sh[tid] += sh[tid + st];
        __syncthreads();
    }
    if (tid == 0) {
        const double l2 = sqrt(fmax(0.0, sh[0]));
        float sc = 1.f;
        if (l2 > static_cast<double>(thr) && isfinite(l2)) sc = static_cast<float>(static_cast<double>(thr) / l2);
        *tick_scale = sc;
        if (sc != 1.f) *gs *= sc;
        sc_sh = sc;
    }
    __syncthreads();
    const float sc = sc_sh;
    if (sc != 1.f)
        for (int r = tid; r < R; r += kThreads) slot_scale[r] *= sc;
    (void)flag;
}

// ---------------------------------------------------------------- w_tick
// replay_compute_w_tick_kernel (replay_dw_dx.cu:96-114): one wave per row.
__global__ void k_rp_wtick(const float* cur, const float* slot_scale, int cur_slot, int N, const int* po,
                           int n_out, const float* dl, int clip_ran, const float* tick_scale, float* w_tick,
                           float* dw_acc) {
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;
    const float sig = slot_scale[cur_slot];
    const float* r = cur + static_cast<size_t>(row) * N;
    float acc = 0.f;
    for (int o = lane; o < n_out; o += 64) acc = fmaf(r[po[o]] * sig, dl[o], acc);
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) {
        const float ts = clip_ran ? *tick_scale : 1.f;
        w_tick[row] = acc;
        dw_acc[row] = dw_acc[row] * ts + acc;
    }
}

// ---------------------------------------------------------------- dx
// replay_dx_reduce_kernel / replay_dx_finalize_kernel (replay_dw_dx.cu:445-501):
// one workgroup per input column, fixed-order reduction.  A clip at this tick
// also rescales the input's earlier dx entries (LearnRuntime.cpp:2257).
__global__ void k_rp_dx(const float* cur, const float* slot_scale, int cur_slot, int N, const int* pin, int n_in,
                        const float* w_tick, float eps, int t_idx, int ksteps, int clip_ran, const float* tick_scale,
                        float* dx) {
    __shared__ float s_sh[kThreads], b_sh[kThreads];
    const int j = blockIdx.x;
    const int tid = threadIdx.x;
    if (j >= n_in) return;
    const int p = pin[j];
    const float sig = slot_scale[cur_slot];
    float s = 0.f, bsum = 0.f;
    for (int i = tid; i < N; i += kThreads) {
        const float v = cur[static_cast<size_t>(i) * N + p] * sig;
        bsum += v;
        s += w_tick[i] / (v + eps);
    }
    s_sh[tid] = s;
    b_sh[tid] = bsum;
    __syncthreads();
    for (int st = kThreads / 2; st > 0; st >>= 1) {
        if (tid < st) {
            s_sh[tid] += s_sh[tid + st];
            b_sh[tid] += b_sh[tid + st];
        }
        __syncthreads();
    }
    float* row = dx + static_cast<size_t>(j) * ksteps;
    if (clip_ran) {
        const float ts = *tick_scale;
        if (ts != 1.f)
            for (int t = tid; t < t_idx; t += kThreads) row[t] *= ts;
    }
    if (tid == 0) row[t_idx] = s_sh[0] * b_sh[0];
}

__global__ void k_rp_scale_into(const float* src, float scale, float* dst, long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src[i] * scale;
}

__global__ void k_fill_f32(float* p, float v, long long n) {
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<long long>(gridDim.x) * blockDim.x)
        p[i] = v;
}

// (N, T) -> (T, N) through a 32 x 33 LDS tile
__global__ void k_transpose_nt_tn(const float* src, float* dst, int N, int T) {
    __shared__ float tile[32][33];
    const int t = blockIdx.x * 32 + threadIdx.x;
    const int n = blockIdx.y * 32 + threadIdx.y;
    if (n < N && t < T) tile[threadIdx.y][threadIdx.x] = src[static_cast<size_t>(n) * T + t];
    __syncthreads();
    const int n2 = blockIdx.y * 32 + threadIdx.x;
    const int t2 = blockIdx.x * 32 + threadIdx.y;
    if (n2 < N && t2 < T) dst[static_cast<size_t>(t2) * N + n2] = tile[threadIdx.x][threadIdx.y];
}

}  // namespace

void launch_lr_capture(const CaptureArgs& a, int sample, int lr, hipStream_t s) {
    const long long n = a.n_out + (lr > 0 ? static_cast<long long>(a.nch) * a.N : 0);
    if (n <= 0) return;
    hipLaunchKernelGGL(k_lr_capture, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                       s, a, sample, lr);
}

void launch_rp_base(const ReplayBaseArgs& a, int nblk, int max_bn, hipStream_t s) {
    const long long e = static_cast<long long>(max_bn) * max_bn;
    hipLaunchKernelGGL(k_rp_base, dim3(static_cast<unsigned>((e + kThreads - 1) / kThreads), nblk), dim3(kThreads),
                       0, s, a);
}

int rp_corr_row_tiles(int N) { return (N + kTI - 1) / kTI; }

void launch_rp_corr(const ReplayCorrArgs& a, int ntiles, int tile_cols, hipStream_t s) {
    const dim3 grid(ntiles, rp_corr_row_tiles(a.N));
    if (tile_cols == 128)
        hipLaunchKernelGGL(k_rp_corr<128>, grid, dim3(kCorrThreads), 0, s, a);
    else
        hipLaunchKernelGGL(k_rp_corr<64>, grid, dim3(kCorrThreads), 0, s, a);
}

void launch_rp_pregather(const float* D, const int* pre, int N, float* G, hipStream_t s) {
    hipLaunchKernelGGL(k_rp_pregather, dim3((N + kThreads - 1) / kThreads, N), dim3(kThreads), 0, s, D, pre, N, G);
}

void launch_rp_clip(const double* part, const int* flag, int n, float thr, float* gs, float* slot_scale, int R,
                    float* tick_scale, hipStream_t s) {
    hipLaunchKernelGGL(k_rp_clip, dim3(1), dim3(kThreads), 0, s, part, flag, n, thr, gs, slot_scale, R, tick_scale);
}

void launch_rp_wtick(const float* cur, const float* slot_scale, int cur_slot, int N, const int* po, int n_out,
                     const float* dl, int clip_ran, const float* tick_scale, float* w_tick, float* dw_acc,
                     hipStream_t s) {
    const int rows_per = kThreads / 64;
    hipLaunchKernelGGL(k_rp_wtick, dim3((N + rows_per - 1) / rows_per), dim3(kThreads), 0, s, cur, slot_scale,
                       cur_slot, N, po, n_out, dl, clip_ran, tick_scale, w_tick, dw_acc);
}

void launch_rp_dx(const float* cur, const float* slot_scale, int cur_slot, int N, const int* pin, int n_in,
                  const float* w_tick, float eps, int t_idx, int ksteps, int clip_ran, const float* tick_scale,
                  float* dx, hipStream_t s) {
    if (n_in <= 0) return;
    hipLaunchKernelGGL(k_rp_dx, dim3(n_in), dim3(kThreads), 0, s, cur, slot_scale, cur_slot, N, pin, n_in, w_tick,
                       eps, t_idx, ksteps, clip_ran, tick_scale, dx);
}

void launch_rp_scale_into(const float* src, float scale, float* dst, long long n, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_rp_scale_into, dim3(static_cast<unsigned>((n + kThreads - 1) / kThreads)), dim3(kThreads),
                       0, s, src, scale, dst, n);
}

void launch_fill_f32(float* p, float v, long long n, hipStream_t s) {
    if (n <= 0) return;
    const long long blocks = std::min<long long>((n + kThreads - 1) / kThreads, 4096);
    hipLaunchKernelGGL(k_fill_f32, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s, p, v, n);
}

void launch_transpose_nt_tn(const float* src_nt, float* dst_tn, int N, int T, hipStream_t s) {
    if (N <= 0 || T <= 0) return;
    hipLaunchKernelGGL(k_transpose_nt_tn, dim3((T + 31) / 32, (N + 31) / 32), dim3(32, 32), 0, s, src_nt, dst_tn, N,
                       T);
}

}  // namespace hx
