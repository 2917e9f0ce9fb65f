// Per-chunk arithmetic of the tree solve, shared by the wavefront kernel and the
// host emulation used by the CPU tests.
//
// The system is the reference's (assembly simulate.cpp:527-555, capacitance
// capac.cpp:68-80, elimination and back substitution simulate.cpp:558-581):
// for node i with parent p and children C,
//   D_i = (dm_i + cfac cm_i) - b_i - sum_c (a_c + (a_c/D_c) b_c)
//   R_i = rm_i - b_i (v_p - v_i) + sum_c (a_c (v_i - v_c) - (a_c/D_c) R_c)
//   x_root = R_root / D_root,  x_i = (R_i - b_i x_p) / D_i,  v_i += x_i.
//
// A chunk is an unbranched run of nodes 0 (head) .. len-1 (tail); node k+1 is
// the only child of node k, the chunks hanging off the tail are its other
// children.  Three rearrangements take the divisions off the serial chain:
//
// * Elimination inside a chunk is the continued fraction
//     D_k = Db_k - a_{k+1} - a_{k+1} b_{k+1} / D_{k+1},
//   which is carried as D_k = P_k / P_{k+1} with the linear recurrence
//     P_k = (Db_k - a_{k+1}) P_{k+1} - a_{k+1} b_{k+1} P_{k+2}
//   (P_len = 1), so the chain costs one fma per node and the reciprocals
//   1/P_k are independent of each other.
// * Elimination has u = R/D and w = b/D, and back substitution is
//   x_k = u_k - w_k x_{k-1}.  In terms of the new voltages vn_k = v_k + x_k that is
//   vn_k = s_k - w_k vn_{k-1} with s_k = v_k + u_k + w_k v_{k-1}, so elimination
//   stores s and w and back substitution reads just those two (one fma per
//   node, no reload of v); x is vn - v where a caller needs it.
// * The head's parent voltage v_p enters R_head only through -b_head v_p.
//   Leaving it out, the head hands its parent the pair (cd, ce) with
//   cd = a + (a/D) b and ce = -a v_head - (a/D) R'_head, and the parent's tail
//   takes -sum cd into its diagonal and v_tail * sum cd + sum ce into its
//   right-hand side (exactly the reference's child terms).  In back
//   substitution the missing -w_head v_p term is added back together with
//   -w_head x_p as -w_head (v_p + x_p), i.e. with the parent's updated
//   voltage.  Elimination therefore never reads another chunk's voltages.
//
// The child terms are added to the tail's inputs before the chunk runs
// (tail_inject), so the per-node loop has no special cases.  Nodes k >= len
// are padding with the neutral values db = 1, rm = a = b = v = 0; they leave
// every quantity of the real nodes unchanged, so the loops run all kChunk
// nodes without branches.  The results agree with the reference's serial
// order to rounding.
#pragma once
#include <cmath>

#include "hx_internal.h"

namespace hx {

// arrays of a round stage; elimination reads DB RM A B V and produces D, s and w;
// back substitution reads s (RM), w (A) and, where x is wanted, the old v (V)
enum StageArr { SA_DB = 0, SA_RM = 1, SA_A = 2, SA_B = 3, SA_V = 4 };

struct FwdNode {
    double db, rm, a, b, v;    // db = dm + cfac cm
};
struct BackNode {
    double s, w, v;            // v: the voltage before the step (read only when x is stored)
};

// The tail's inputs after adding the chunk's children: acd = sum cd,
// ace = sum ce over the chunks hanging off the tail.
__host__ __device__ __forceinline__ void tail_inject(double& db, double& rm, double v, double acd, double ace) {
    db = db - acd;
    rm = rm + (v * acd + ace);
}

// Prefetch distance of the chunk loops: node k's inputs are requested kAhead
// nodes before they are used, so a caller reading from a buffer with some
// latency (LDS) keeps several reads in flight behind the arithmetic.
constexpr int kAhead = 4;

// The chunk loops walk KM node slots (KM <= kChunk), without branches.  A
// round whose chunks are all at most KM long runs the KM variant: node slots
// k >= KM are padding on every lane, and a padding node maps the recurrence
// state (P1 = 1, r1 = 1, a1 = ab1 = accr = 0) onto itself, so leaving them out
// changes no result.  dispatch_chunk_bound calls f with the smallest of the
// compiled bounds that covers maxlen.
template <int KM>
struct ChunkBound {
    static constexpr int value = KM;
};
template <class F>
__host__ __device__ __forceinline__ void dispatch_chunk_bound(int maxlen, F&& f) {
    if (maxlen <= 8) f(ChunkBound<8>{});
    else if (maxlen <= 12) f(ChunkBound<12>{});
    else f(ChunkBound<kChunk>{});
}

// in.fwd(k): node k's inputs (neutral for k >= len, tail already injected);
// rcp(x) returns 1/x.  out(k, D, s, w) receives node k's results for every
// slot k < KM (the caller drops those of padding nodes): the pivot D, s and w.
// cd, ce: this chunk's pair for its parent.
template <int KM, class In, class Out, class Rcp>
__host__ __device__ __forceinline__ void chunk_forward_math(bool has_parent, const In& in, Out&& out, Rcp rcp,
                                                            double& cd, double& ce) {
    static_assert(KM >= 1 && KM <= kChunk, "chunk bound out of range");
    double P1 = 1.0, P2 = 0.0, r1 = 1.0, a1 = 0.0, ab1 = 0.0, accr = 0.0;
    cd = 0.0;
    ce = 0.0;
    FwdNode buf[KM];
    // the walk runs k = KM-1 down to 0; its first kAhead nodes are requested up front
#pragma unroll
    for (int j = KM - 1; j >= 0 && j >= KM - kAhead; --j) buf[j] = in.fwd(j);
#pragma unroll
    for (int k = KM - 1; k >= 0; --k) {
        if (k - kAhead >= 0) buf[k - kAhead] = in.fwd(k - kAhead);
        const FwdNode& cur = buf[k];
        double a = cur.a, b = cur.b;
        if (k == 0 && !has_parent) {
            a = 0.0;
            b = 0.0;
        }
        const double dv = (k > 0 ? buf[k - 1].v : 0.0) - cur.v;
        const double Db = cur.db - b;
        const double Rb = fma(-b, dv, cur.rm);
        const double P = fma(Db - a1, P1, -(ab1 * P2));
        const double r = rcp(P);
        const double rD = P1 * r;     // 1 / D_k
        const double R = Rb + accr;
        const double p = a * rD;
        accr = fma(a, dv, -(p * R));
        const double w = b * rD;
        out(k, P * r1, fma(w, k > 0 ? buf[k - 1].v : 0.0, cur.v + R * rD), w);
        if (k == 0) {
            cd = fma(p, b, a);
            ce = accr;
        }
        P2 = P1;
        P1 = P;
        r1 = r;
        a1 = a;
        ab1 = a * b;
    }
}

// in.back(k): node k's (s, w, v) (neutral for k >= len); vpar_new: updated
// voltage of the head's parent (0 for the root chunk, whose w_0 is 0).
// out(k, v_new, v_old) for every slot k < KM.
template <int KM, class In, class Out>
__host__ __device__ __forceinline__ void chunk_back_math(const In& in, Out&& out, double vpar_new) {
    static_assert(KM >= 1 && KM <= kChunk, "chunk bound out of range");
    double vn = vpar_new;
    BackNode buf[KM];
#pragma unroll
    for (int j = 0; j < kAhead && j < KM; ++j) buf[j] = in.back(j);
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        if (k + kAhead < KM) buf[k + kAhead] = in.back(k + kAhead);
        vn = fma(-buf[k].w, vn, buf[k].s);
        out(k, vn, buf[k].v);
    }
}

}  // namespace hx
