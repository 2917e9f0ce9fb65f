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
// * Elimination stores u = R/D and w = b/D, so back substitution is
//   x_k = u_k - w_k x_{k-1}: one fma per node.
// * The head's parent voltage v_p enters R_head only through -b_head v_p.
//   Leaving it out, the head hands its parent the pair (cd, ce) with
//   cd = a + (a/D) b and ce = -a v_head - (a/D) R'_head, and the parent's tail
//   adds v_tail * sum cd + sum ce to its R (this is exactly the reference's
//   child term).  In back substitution the missing -w_head v_p term is added
//   back together with -w_head x_p as -w_head (v_p + x_p), i.e. with the
//   parent's updated voltage.  Elimination therefore never reads another
//   chunk's voltages.
//
// Nodes k >= len are padding with the neutral values dm = 1, rm = a = b = v = 0;
// they leave every quantity of the real nodes unchanged, so the loops run
// all kChunk nodes without branches.  The results agree with the reference's
// serial order to rounding.
#pragma once
#include <cmath>

#include "hx_internal.h"

namespace hx {

// arrays of a round stage; elimination reads DB RM A B V and writes D into
// DB, u into RM and w into B; back substitution reads u (RM), w (A) and v (V)
// and writes x into RM and the new v into V
enum StageArr { SA_DB = 0, SA_RM = 1, SA_A = 2, SA_B = 3, SA_V = 4 };

// In(arr, k): node k's value of stage array arr (neutral for k >= len); rcp(x)
// returns 1/x.  Out(k, D, u, w) receives node k's results (ignored by the
// caller for k >= len).  acd and ace: sums of cd and ce over the chunks hanging
// off the tail.  cd and ce: this chunk's pair for its parent.
template <class In, class Out, class Rcp>
__host__ __device__ __forceinline__ void chunk_forward_math(int len, bool has_parent, const In& in, Out&& out,
                                                            Rcp rcp, double acd, double ace, double& cd,
                                                            double& ce) {
    double P1 = 1.0, P2 = 0.0, r1 = 1.0, a1 = 0.0, ab1 = 0.0, accr = 0.0;
    cd = 0.0;
    ce = 0.0;
#pragma unroll
    for (int k = kChunk - 1; k >= 0; --k) {
        double a = in(SA_A, k), b = in(SA_B, k);
        if (k == 0 && !has_parent) {
            a = 0.0;
            b = 0.0;
        }
        const double v = in(SA_V, k);
        const double dv = (k > 0 ? in(SA_V, k - 1) : 0.0) - v;
        const bool tail = k == len - 1;
        const double Db = in(SA_DB, k) - b - (tail ? acd : 0.0);
        const double Rb = in(SA_RM, k) - b * dv + (tail ? v * acd + ace : 0.0);
        const double P = (Db - a1) * P1 - ab1 * P2;
        const double r = rcp(P);
        const double rD = P1 * r;     // 1 / D_k
        const double D = P * r1;      // P_k / P_{k+1}
        const double R = Rb + accr;
        const double p = a * rD;
        accr = a * dv - p * R;
        out(k, D, R * rD, b * rD);
        if (k == 0) {
            cd = a + p * b;
            ce = accr;
        }
        P2 = P1;
        P1 = P;
        r1 = r;
        a1 = a;
        ab1 = a * b;
    }
}

// In(arr, k) as above (RM = u, A = w, V = v); vpar_new: updated voltage of the
// head's parent (0 for the root chunk, whose w_0 is 0).  Out(k, v_new, x).
// Returns the tail's updated voltage.
template <class In, class Out>
__host__ __device__ __forceinline__ double chunk_back_math(int len, const In& in, Out&& out, double vpar_new) {
    double x = vpar_new, vtail = 0.0;
#pragma unroll
    for (int k = 0; k < kChunk; ++k) {
        const double u = in(SA_RM, k), w = in(SA_A, k), v = in(SA_V, k);
        x = u - w * x;
        const double vn = v + x;
        out(k, vn, x);
        if (k == len - 1) vtail = vn;
    }
    return vtail;
}

}  // namespace hx
