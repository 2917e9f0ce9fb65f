// Per-chunk steps of the tree solve, shared by the wavefront kernel (one lane
// per chunk) and the host emulation used by the CPU tests.
//
// For node i with parent p and children C (reference: assembly
// simulate.cpp:527-555, capacitance capac.cpp:68-80, elimination and back
// substitution simulate.cpp:558-581):
//   D_i = (dm_i + cfac cm_i) - b_i - sum_c (a_c + (a_c/D_c) b_c)
//   R_i = rm_i - b_i (v_p - v_i) + sum_c (a_c (v_i - v_c) - (a_c/D_c) R_c)
//   x_root = R_root / D_root,  x_i = (R_i - b_i x_p) / D_i,  v_i += x_i
// Inside a chunk the child of node k is node k+1 and is carried in registers;
// node k of the chunk lives at idx[k] (position-major round layout: see the
// scheduler);
// the head's pair (a + p b, a dv - p R) goes to the LDS slot of the chunk and
// is summed by the parent chunk's tail.  After elimination, d and rhs hold D
// and R (as the reference's in-place arrays do after triangularization).
#pragma once
#include "hx_internal.h"

namespace hx {

// Keeps the staged loads of a chunk together: the compiler would otherwise sink
// each load next to its use in the serial recurrence and pay one memory
// latency per node instead of one per chunk.
__host__ __device__ __forceinline__ void pin(double& x) {
#ifdef __HIP_DEVICE_COMPILE__
    asm volatile("" : "+v"(x));
#else
    (void)x;
#endif
}

__host__ __device__ __forceinline__ void chunk_forward(const ChunkDesc& q, const int* idx, int nb, double* v,
                                                       double* d, double* rhs, const double* a, const double* b,
                                                       const double* cm, double cfac, double* slots) {
    double dm[kChunk], rm[kChunk], av[kChunk], bv[kChunk], vv[kChunk], cmv[kChunk];
    const bool head_has_parent = q.head_parent != kNone;
    // parent voltage of the head; unconditional (own head when there is no parent)
    // so that every load of the burst is consumed on every path
    double vpar = v[head_has_parent ? nb + q.head_parent : idx[0]];
    // unconditional loads from a clamped index: straight-line code, one latency
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        const int kk = idx[k < q.len ? k : q.len - 1];
        dm[k] = d[kk];
        rm[k] = rhs[kk];
        av[k] = a[kk];
        bv[k] = b[kk];
        vv[k] = v[kk];
        cmv[k] = cm[kk];
    }
    pin(vpar);
#pragma unroll
    for (int k = 0; k < kChunk; ++k) { pin(dm[k]); pin(rm[k]); pin(av[k]); pin(bv[k]); pin(vv[k]); pin(cmv[k]); }
    double accd = 0.0, accr = 0.0;
    for (int ch = 0; ch < q.child_count; ++ch) {
        accd += slots[2 * (q.child_begin + ch)];
        accr += slots[2 * (q.child_begin + ch) + 1];
    }
#pragma unroll
    for (int k = kChunk - 1; k >= 0; --k) {
        if (k < q.len) {
            const bool has_parent = k > 0 || head_has_parent;
            const double vp = k > 0 ? vv[k - 1] : vpar;
            double D = dm[k] + cfac * cmv[k];
            double R = rm[k];
            double dv = 0.0;
            if (has_parent) {
                dv = vp - vv[k];
                R -= bv[k] * dv;
                D -= bv[k];
            }
            D -= accd;
            R += accr;
            d[idx[k]] = D;
            rhs[idx[k]] = R;
            if (has_parent) {
                const double p = av[k] / D;
                accd = av[k] + p * bv[k];
                accr = av[k] * dv - p * R;
            }
        }
    }
    if (head_has_parent) {
        slots[2 * q.slot] = accd;
        slots[2 * q.slot + 1] = accr;
    }
}

// Returns the tail's solution, to be stored in the chunk's slot after the round.
__host__ __device__ __forceinline__ double chunk_back(const ChunkDesc& q, const int* idx, double* v, const double* d,
                                                      const double* rhs, const double* b, const double* slots) {
    double Dv[kChunk], Rv[kChunk], bv[kChunk], vv[kChunk];
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        const int kk = idx[k < q.len ? k : q.len - 1];
        Dv[k] = d[kk];
        Rv[k] = rhs[kk];
        bv[k] = b[kk];
        vv[k] = v[kk];
    }
#pragma unroll
    for (int k = 0; k < kChunk; ++k) { pin(Dv[k]); pin(Rv[k]); pin(bv[k]); pin(vv[k]); }
    const bool head_has_parent = q.head_parent != kNone;
    double x = head_has_parent ? slots[2 * q.parent_slot] : 0.0;
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        if (k < q.len) {
            if (k == 0 && !head_has_parent) x = Rv[0] / Dv[0];
            else x = (Rv[k] - bv[k] * x) / Dv[k];
            v[idx[k]] = vv[k] + x;
        }
    }
    return x;
}

}  // namespace hx
