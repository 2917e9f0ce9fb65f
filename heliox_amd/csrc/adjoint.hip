// Adjoint (vector-Jacobian) backward step of the fixed-step simulation, for
// models made of pas, hh, Ca_HVA, hd_la (Ih), CaDynamics_E2, ExpSyn, Exp2Syn,
// IClamp and the ions (na, k with fixed reversal potentials; ca with a fixed
// eca or eca from cai by the Nernst equation every step).  No reference code
// exists for this; it differentiates the step the forward kernels take
// (simulate.cpp:410-442 order).
//
// Step n maps (v^n, x^n, g^n) to (v^{n+1}, x^{n+1}, g^{n+1}):
//   g_eff = g^n + sum of the weights delivered at step n         (ExpSyn)
//   M (v^{n+1} - v^n) = -I(v^n) - K v^n,  M = C + G + K           (tree solve)
//     C = 1e-3 cm / dt, G = membrane conductance (all mechanisms here are
//     linear in v, so the FD Jacobian is G), K = the axial matrix
//   x^{n+1} = cnexp(x^n, v^{n+1})                                 (hh gates)
//   g^{n+1} = g_eff exp(-dt / tau)                                (ExpSyn decay)
// With I linear in v:  dv^{n+1}/dv^n = M^{-1} C  and, for anything p that G
// depends on,  dv^{n+1}/dp = -M^{-1} dG/dp (v^{n+1} - E).  So with
// mu = M^{-T} lambda_v^{n+1}:
//   lambda_v^n = C mu (+ loss term),
//   dL/dp     += -mu_i dI_i/dp evaluated at v^{n+1},
// and the gates add their cnexp derivative (dual numbers through the rate
// functions) to lambda_v^{n+1} before the solve.  M^T is solved with the same
// tree kernel by swapping a and b and correcting the diagonal (the kernel
// assembles it from a and b).
//
// Calcium.  Ca_HVA's current is g (v - eca) with g = gbar m^2 h and eca =
// (ktf / 2) ln(cao / cai^n) (ion style 0100) or fixed.  CaDynamics_E2 then takes
//   cai^{n+1} = cai^n + (1 - e)(decay drive(ica^n) + minCai - cai^n),
//   e = exp(-dt / decay), drive = -1e4 ica gamma / (2 F depth),
// with ica^n = g (v^n - eca) at the voltage of step n's current pass.  So
//   lambda_cai^n = e lambda_cai^{n+1} + (terms through eca),
//   lambda_ica^n = (1 - e) decay (-1e4 gamma / (2 F depth)) lambda_cai^{n+1},
// and lambda_ica^n reaches v^n, the Ca_HVA gates, gbar and (through eca) cai^n.
// Through the solve, eca enters like any reversal potential: d/dcai of G E.
//
// Exp2Syn: g = B_eff - A_eff (events add w factor to both), A and B decay by
// exp(-dt / tau1), exp(-dt / tau2) after the solve; a delivered event's weight
// gets factor (lambda_A + lambda_B).
//
// Gap junctions (HalfGap, an electrode current i = g (vgap - v) x 1e2/area): a
// conductance G = g 1e2/area with reversal potential vgap, which is the source
// node's v^n (the transfer after the previous step's solve) or, without a source,
// a constant.  So G joins M's diagonal like any membrane conductance, dL/dg +=
// -mu 1e2/area (v^{n+1} - vgap), and v^{n+1} = M^-1 (C v^n + G vgap) gives the
// source node lambda_v^n += G mu at the instance's node.
#include "hx_internal.h"
#include "mech_math.h"

namespace hx {
namespace {

__device__ __forceinline__ int ion_of(const MechDev& m, int which, int j) {
    return m.ion[which] ? m.ion[which][j] : j;
}

// Per-instance bodies of the density mechanisms.  Each takes the instance j and
// its node, updates the mechanism's own adjoints and returns what it adds to the
// node's lambda_v or d, so the per-mechanism kernels and the node-parallel kernels
// below add the same terms in the same order (the same bits either way).

// hh gates: lambda_x <- alpha lambda_x; returns dx^{n+1}/dv^{n+1} . lambda_x
__device__ __forceinline__ double hh_state_at(const AdjStep& A, int j, int node) {
    const Dual v1{A.v1[node], 1.0};
    Dual minf, mtau, hinf, htau, ninf, ntau;
    hh_rates(v1, A.hh_q10, minf, mtau, hinf, htau, ninf, ntau);
    const double x0[3] = {A.x0[j], A.x0[A.xstride + j], A.x0[2 * A.xstride + j]};
    const Dual xn[3] = {hh_cnexp(x0[0], minf, mtau, A.dt), hh_cnexp(x0[1], hinf, htau, A.dt),
                        hh_cnexp(x0[2], ninf, ntau, A.dt)};
    const double tau[3] = {mtau.v, htau.v, ntau.v};
    double dv = 0.0;
    for (int g = 0; g < 3; ++g) {
        const double lx = A.lam_x[g * A.xstride + j];
        dv += xn[g].d * lx;
        A.lam_x[g * A.xstride + j] = exp(A.dt * (-1.0 / tau[g])) * lx;   // d cnexp / d x
    }
    return dv;
}

// Ca_HVA gates (cnexp at v^{n+1}): lambda_x <- exp(-dt/tau) lambda_x; returns dx/dv lambda_x
__device__ __forceinline__ double cahva_state_at(const AdjStep& A, int j, int node) {
    const Dual v1{A.v1[node], 1.0};
    Dual mInf, mTau, hInf, hTau;
    cahva_rates_t(v1, mInf, mTau, hInf, hTau);
    const Dual mn = cnexp_t(A.c0[j], mInf, mTau, A.dt);
    const Dual hn = cnexp_t(A.c0[A.cstride + j], hInf, hTau, A.dt);
    const double lm = A.lam_c[j], lh = A.lam_c[A.cstride + j];
    A.lam_c[j] = exp(-A.dt / mTau.v) * lm;
    A.lam_c[A.cstride + j] = exp(-A.dt / hTau.v) * lh;
    return mn.d * lm + hn.d * lh;
}

// hd_la gate
__device__ __forceinline__ double hdla_state_at(const AdjStep& A, int j, int node) {
    const MechDev& m = A.m[M_HDLA];
    const Dual v1{A.v1[node], 1.0};
    Dual linf, taul;
    hdla_rate_t(v1, m.col(HD_VHALFL)[j], m.col(HD_TAU)[j], A.c, linf, taul);
    const Dual ln = cnexp_t(A.l0[j], linf, taul, A.dt);
    const double ll = A.lam_l[j];
    A.lam_l[j] = exp(-A.dt / taul.v) * ll;
    return ln.d * ll;
}

// CaDynamics_E2: lambda_ica^n from lambda_cai^{n+1}, then lambda_cai^n <- e lambda_cai^{n+1}
__device__ __forceinline__ void cadyn_at(const AdjStep& A, int j) {
    const MechDev& m = A.m[M_CADYN];
    const int ci = ion_of(m, 2, j);
    const double decay = m.col(CD_DECAY)[j];
    const double e = exp(A.dt * (-1.0 / decay));
    const double lc = A.lam_cai[ci];
    A.lam_ica[ci] = (1.0 - e) * decay * (-(10000.0) * m.col(CD_GAMMA)[j] / (2.0 * kFaradayCaDyn * m.col(CD_DEPTH)[j])) * lc;
    A.lam_cai[ci] = e * lc;
}

// membrane conductances G at step n
__device__ __forceinline__ double cond_pas_at(const AdjStep& A, int j) { return A.m[M_PAS].col(PAS_G)[j]; }

__device__ __forceinline__ double cond_hh_at(const AdjStep& A, int j) {
    const MechDev& m = A.m[M_HH];
    const double mm = A.x0[j], hh = A.x0[A.xstride + j], nn = A.x0[2 * A.xstride + j];
    return m.col(HH_GNABAR)[j] * mm * mm * mm * hh + m.col(HH_GKBAR)[j] * nn * nn * nn * nn + m.col(HH_GL)[j];
}

__device__ __forceinline__ double cond_cahva_at(const AdjStep& A, int j) {
    const double mm = A.c0[j], hh = A.c0[A.cstride + j];
    return A.m[M_CAHVA].col(CH_GBAR)[j] * mm * mm * hh;
}

__device__ __forceinline__ double cond_hdla_at(const AdjStep& A, int j) {
    return A.m[M_HDLA].col(HD_GHDBAR)[j] * A.l0[j];
}

__device__ __forceinline__ void hh_param_at(const AdjStep& A, int j, int node) {
    const MechDev& m = A.m[M_HH];
    const double mu = A.mu[node], v1 = A.v1[node];
    const double ena = A.m[M_NA_ION].col(ION_EREV)[ion_of(m, 0, j)];
    const double ek = A.m[M_K_ION].col(ION_EREV)[ion_of(m, 1, j)];
    const double mm = A.x0[j], hh = A.x0[A.xstride + j], nn = A.x0[2 * A.xstride + j];
    const double gnabar = m.col(HH_GNABAR)[j], gkbar = m.col(HH_GKBAR)[j];
    A.lam_x[j] -= mu * 3.0 * gnabar * mm * mm * hh * (v1 - ena);
    A.lam_x[A.xstride + j] -= mu * gnabar * mm * mm * mm * (v1 - ena);
    A.lam_x[2 * A.xstride + j] -= mu * 4.0 * gkbar * nn * nn * nn * (v1 - ek);
    A.grad_gnabar[j] -= mu * mm * mm * mm * hh * (v1 - ena);
    A.grad_gkbar[j] -= mu * nn * nn * nn * nn * (v1 - ek);
}

__device__ __forceinline__ void pas_param_at(const AdjStep& A, int j, int node) {
    A.grad_gpas[j] -= A.mu[node] * (A.v1[node] - A.m[M_PAS].col(PAS_E)[j]);
}

// eca of step n at ca_ion instance ci and d eca / d cai (0 where eca is fixed)
__device__ __forceinline__ double eca_of(const AdjStep& A, int ci, double& deca) {
    const MechDev& ca = A.m[M_CA_ION];
    if (ca.iontype[ci] & 0100) {
        const double c = A.cai0[ci];
        deca = -A.c.ktf / 2.0 / c;
        return nernst(c, ca.col(ION_CONCO)[ci], 2.0, A.c.ktf);
    }
    deca = 0.0;
    return ca.col(ION_EREV)[ci];
}

// Ca_HVA: through the solve (at v^{n+1}) and through the ica CaDynamics_E2 read (at v^n);
// lnew is the node's lambda_v^n
__device__ __forceinline__ void cahva_param_at(const AdjStep& A, int j, int node, double* lnew) {
    const MechDev& m = A.m[M_CAHVA];
    const int ci = ion_of(m, 2, j);
    double deca;
    const double eca = eca_of(A, ci, deca);
    const double gbar = m.col(CH_GBAR)[j];
    const double mm = A.c0[j], hh = A.c0[A.cstride + j];
    const double g = gbar * mm * mm * hh;
    // solve: dL/dq += -mu dG/dq (v^{n+1} - eca) + mu G deca/dq
    const double mu = A.mu[node];
    const double d1 = A.v1[node] - eca;
    double lm = -mu * 2.0 * gbar * mm * hh * d1;
    double lh = -mu * gbar * mm * mm * d1;
    double gg = -mu * mm * mm * hh * d1;
    double lcai = mu * g * deca;
    // ica^n = G (v^n - eca): its adjoint from CaDynamics_E2
    const double li = A.lam_ica ? A.lam_ica[ci] : 0.0;
    if (li != 0.0) {
        const double d0 = A.v0[node] - eca;
        *lnew += g * li;
        lm += 2.0 * gbar * mm * hh * d0 * li;
        lh += gbar * mm * mm * d0 * li;
        gg += mm * mm * hh * d0 * li;
        lcai -= g * deca * li;
    }
    A.lam_c[j] += lm;
    A.lam_c[A.cstride + j] += lh;
    A.grad_cgbar[j] += gg;
    if (A.lam_cai) A.lam_cai[ci] += lcai;
}

__device__ __forceinline__ void hdla_param_at(const AdjStep& A, int j, int node) {
    const MechDev& m = A.m[M_HDLA];
    const double mu = A.mu[node], d1 = A.v1[node] - A.c.hd_ehd;
    A.lam_l[j] -= mu * m.col(HD_GHDBAR)[j] * d1;
    A.grad_ghdbar[j] -= mu * A.l0[j] * d1;
}

// synapse decay adjoints: lambda_geff = exp(-dt/tau) lambda_g (ExpSyn, in place),
// lambda_{A,B eff} = exp(-dt/tau_{1,2}) lambda_{A,B} (Exp2Syn)
__device__ __forceinline__ void syn_state_at(const AdjStep& A, int j) {
    A.lam_g[j] = exp(-A.dt / A.m[M_EXPSYN].col(ES_TAU)[j]) * A.lam_g[j];
}

__device__ __forceinline__ void syn2_state_at(const AdjStep& A, int j) {
    const MechDev& m = A.m[M_EXP2SYN];
    A.lam_ab[j] *= exp(A.dt * (-1.0 / m.col(E2_TAU1)[j]));
    A.lam_ab[m.n + j] *= exp(A.dt * (-1.0 / m.col(E2_TAU2)[j]));
}

// conductance of node group q (the synapses on one node): sum of g_eff x 1e2/area (ExpSyn),
// of (B_eff - A_eff) x 1e2/area (Exp2Syn)
__device__ __forceinline__ double cond_syn_at(const AdjStep& A, int q, int node) {
    const MechDev& m = A.m[M_EXPSYN];
    double g = 0.0;
    for (int j = m.grp_begin[q]; j < m.grp_begin[q + 1]; ++j) g += A.geff[j];
    return g * (1.e2 / A.area[node]);
}

__device__ __forceinline__ double cond_syn2_at(const AdjStep& A, int q, int node) {
    const MechDev& m = A.m[M_EXP2SYN];
    double g = 0.0;
    for (int j = m.grp_begin[q]; j < m.grp_begin[q + 1]; ++j) g += A.ab0[m.n + j] - A.ab0[j];
    return g * (1.e2 / A.area[node]);
}

// lambda_geff += -mu (v^{n+1} - e) 1e2/area
__device__ __forceinline__ void syn_param_at(const AdjStep& A, int j) {
    const MechDev& m = A.m[M_EXPSYN];
    const int node = m.node[j];
    A.lam_g[j] -= A.mu[node] * (A.v1[node] - m.col(ES_E)[j]) * (1.e2 / A.area[node]);
}

// Exp2Syn: lambda_{A,eff} += mu (v^{n+1} - e) 1e2/area, lambda_{B,eff} -= the same
__device__ __forceinline__ void syn2_param_at(const AdjStep& A, int j) {
    const MechDev& m = A.m[M_EXP2SYN];
    const int node = m.node[j];
    const double t = A.mu[node] * (A.v1[node] - m.col(E2_E)[j]) * (1.e2 / A.area[node]);
    A.lam_ab[j] += t;
    A.lam_ab[m.n + j] -= t;
}

// ---- per-mechanism kernels (instance-parallel; one density instance per node) ----
#define HX_ADJ_INSTANCE(MECH)                                  \
    const MechDev& m = A.m[MECH];                              \
    const int j = blockIdx.x * blockDim.x + threadIdx.x;       \
    if (j >= m.n) return;                                      \
    const int node = m.node[j];                                \
    (void)node

__global__ void k_adj_hh_state(AdjStep A) { HX_ADJ_INSTANCE(M_HH); A.lam_v[node] += hh_state_at(A, j, node); }
__global__ void k_adj_cahva_state(AdjStep A) { HX_ADJ_INSTANCE(M_CAHVA); A.lam_v[node] += cahva_state_at(A, j, node); }
__global__ void k_adj_hdla_state(AdjStep A) { HX_ADJ_INSTANCE(M_HDLA); A.lam_v[node] += hdla_state_at(A, j, node); }
__global__ void k_adj_cadyn(AdjStep A) { HX_ADJ_INSTANCE(M_CADYN); cadyn_at(A, j); }
__global__ void k_adj_cond_pas(AdjStep A) { HX_ADJ_INSTANCE(M_PAS); A.dT[node] += cond_pas_at(A, j); }
__global__ void k_adj_cond_hh(AdjStep A) { HX_ADJ_INSTANCE(M_HH); A.dT[node] += cond_hh_at(A, j); }
__global__ void k_adj_cond_cahva(AdjStep A) { HX_ADJ_INSTANCE(M_CAHVA); A.dT[node] += cond_cahva_at(A, j); }
__global__ void k_adj_cond_hdla(AdjStep A) { HX_ADJ_INSTANCE(M_HDLA); A.dT[node] += cond_hdla_at(A, j); }
__global__ void k_adj_hh_param(AdjStep A) { HX_ADJ_INSTANCE(M_HH); hh_param_at(A, j, node); }
__global__ void k_adj_pas_param(AdjStep A) { HX_ADJ_INSTANCE(M_PAS); pas_param_at(A, j, node); }
__global__ void k_adj_cahva_param(AdjStep A) { HX_ADJ_INSTANCE(M_CAHVA); cahva_param_at(A, j, node, A.lam_v_new + node); }
__global__ void k_adj_hdla_param(AdjStep A) { HX_ADJ_INSTANCE(M_HDLA); hdla_param_at(A, j, node); }
#undef HX_ADJ_INSTANCE

// ---- node-parallel kernels ----
// Before the solve: the gate adjoints of the mechanisms in fuse_state (one instance on
// every node, instance i at node i), then the transposed system d = C + delta + G,
// rhs = lambda_v, v = 0, with the conductances of the mechanisms in fuse_cond.  The host
// runs every other mechanism's kernel so that each node's sums keep the order
// hh, Ca_HVA, hd_la (lambda_v) and pas, hh, Ca_HVA, hd_la (d).
__global__ void k_adj_before_nodes(AdjStep A) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= A.N) {
        // with fold_syn, threads N.. take the synapses' decay adjoints (ExpSyn, then Exp2Syn)
        if (!A.fold_syn) return;
        const int j = i - A.N, nes = A.m[M_EXPSYN].n;
        if (j < nes) syn_state_at(A, j);
        else if (j - nes < A.m[M_EXP2SYN].n) syn2_state_at(A, j - nes);
        return;
    }
    const unsigned fs = A.fuse_state, fc = A.fuse_cond;
    double lv = A.lam_v[i];
    if (fs & kAdjHH) lv += hh_state_at(A, i, i);
    if (fs & kAdjCaHVA) lv += cahva_state_at(A, i, i);
    if (fs & kAdjHdla) lv += hdla_state_at(A, i, i);
    if (fs & kAdjCaDyn) cadyn_at(A, i);
    double d = A.cfac * A.cm[i] + A.delta[i];
    if (fc & kAdjPas) d += cond_pas_at(A, i);
    if (fc & kAdjHH) d += cond_hh_at(A, i);
    if (fc & kAdjCaHVA) d += cond_cahva_at(A, i);
    if (fc & kAdjHdla) d += cond_hdla_at(A, i);
    if (A.fold_syn) {   // after every density conductance, as the group kernels add theirs
        if (A.es_grp) {
            const int q = A.es_grp[i];
            if (q >= 0) d += cond_syn_at(A, q, i);
        }
        if (A.e2_grp) {
            const int q = A.e2_grp[i];
            if (q >= 0) d += cond_syn2_at(A, q, i);
        }
    }
    A.dT[i] = d;
    A.rhsT[i] = lv;
}

// After the solve: lambda_v^n = C mu, then the parameter terms of the mechanisms in
// fuse_param (only Ca_HVA's adds to lambda_v^n, after C mu as in its own kernel), then
// the loss term when the host hands it over (no kernel after this one adds to lambda_v^n).
__global__ void k_adj_after_nodes(AdjStep A) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= A.N) {
        // with fold_syn, threads N.. take the synapses' parameter terms
        if (!A.fold_syn) return;
        const int j = i - A.N, nes = A.m[M_EXPSYN].n;
        if (j < nes) syn_param_at(A, j);
        else if (j - nes < A.m[M_EXP2SYN].n) syn2_param_at(A, j - nes);
        return;
    }
    const unsigned fp = A.fuse_param;
    double lnew = A.cfac * A.cm[i] * A.mu[i];
    if (fp & kAdjHH) hh_param_at(A, i, i);
    if (fp & kAdjPas) pas_param_at(A, i, i);
    if (fp & kAdjCaHVA) cahva_param_at(A, i, i, &lnew);
    if (fp & kAdjHdla) hdla_param_at(A, i, i);
    if (A.loss_v) {   // the loss term of v^n, last, as k_adj_loss adds it
        const int j = A.loss_of_node[i];
        if (j >= 0) lnew += 2.0 * A.loss_scale * (A.loss_v[i] - A.loss_tgt[j]);
    }
    A.lam_v_new[i] = lnew;
}

#define HX_ADJ_SYN(MECH)                                       \
    const MechDev& m = A.m[MECH];                              \
    const int j = blockIdx.x * blockDim.x + threadIdx.x;       \
    if (j >= m.n) return
#define HX_ADJ_GROUP(MECH)                                     \
    const MechDev& m = A.m[MECH];                              \
    const int q = blockIdx.x * blockDim.x + threadIdx.x;       \
    if (q >= m.ngrp) return

__global__ void k_adj_syn_state(AdjStep A) { HX_ADJ_SYN(M_EXPSYN); syn_state_at(A, j); }

// Instance tasks side by side in one launch, each on its own run of blocks.  The host
// puts tasks together only where their outputs are disjoint: at most one of them adds to
// a node's lambda_v, the others write their mechanism's own adjoints and gradients.
enum AdjTask : int { AT_HH_STATE, AT_SYN_STATE, AT_SYN2_STATE, AT_HH_PARAM, AT_PAS_PARAM, AT_SYN_PARAM, AT_SYN2_PARAM };
constexpr int kAdjSideMax = 4;
struct AdjSide {
    int task[kAdjSideMax];
    int begin[kAdjSideMax + 1];   // first block of each task, then the end
    int n;
};
__global__ void __launch_bounds__(kBlock) k_adj_side(AdjStep A, AdjSide S) {
    int t = 0;
    while (t + 1 < S.n && static_cast<int>(blockIdx.x) >= S.begin[t + 1]) ++t;
    const int j = (static_cast<int>(blockIdx.x) - S.begin[t]) * kBlock + static_cast<int>(threadIdx.x);
    switch (S.task[t]) {
        case AT_HH_STATE:
            if (j < A.m[M_HH].n) {
                const int node = A.m[M_HH].node[j];
                A.lam_v[node] += hh_state_at(A, j, node);
            }
            break;
        case AT_SYN_STATE:
            if (j < A.m[M_EXPSYN].n) syn_state_at(A, j);
            break;
        case AT_SYN2_STATE:
            if (j < A.m[M_EXP2SYN].n) syn2_state_at(A, j);
            break;
        case AT_HH_PARAM:
            if (j < A.m[M_HH].n) hh_param_at(A, j, A.m[M_HH].node[j]);
            break;
        case AT_PAS_PARAM:
            if (j < A.m[M_PAS].n) pas_param_at(A, j, A.m[M_PAS].node[j]);
            break;
        case AT_SYN_PARAM:
            if (j < A.m[M_EXPSYN].n) syn_param_at(A, j);
            break;
        case AT_SYN2_PARAM:
            if (j < A.m[M_EXP2SYN].n) syn2_param_at(A, j);
            break;
        default:
            break;
    }
}
__global__ void k_adj_syn2_state(AdjStep A) { HX_ADJ_SYN(M_EXP2SYN); syn2_state_at(A, j); }
__global__ void k_adj_syn_param(AdjStep A) { HX_ADJ_SYN(M_EXPSYN); syn_param_at(A, j); }
__global__ void k_adj_syn2_param(AdjStep A) { HX_ADJ_SYN(M_EXP2SYN); syn2_param_at(A, j); }
__global__ void k_adj_cond_syn(AdjStep A) {
    HX_ADJ_GROUP(M_EXPSYN);
    const int node = m.grp_node[q];
    A.dT[node] += cond_syn_at(A, q, node);
}
__global__ void k_adj_cond_syn2(AdjStep A) {
    HX_ADJ_GROUP(M_EXP2SYN);
    const int node = m.grp_node[q];
    A.dT[node] += cond_syn2_at(A, q, node);
}
#undef HX_ADJ_SYN
#undef HX_ADJ_GROUP

// HalfGap conductances of node group q (the instances on one node, in instance order)
__global__ void k_adj_cond_gap(AdjStep A) {
    const MechDev& m = A.m[M_HALFGAP];
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= m.ngrp) return;
    const int node = m.grp_node[q];
    double g = 0.0;
    for (int j = m.grp_begin[q]; j < m.grp_begin[q + 1]; ++j) g += m.col(HG_G)[j];
    A.dT[node] += g * (1.e2 / A.area[node]);
}

// dL/dg of each HalfGap instance
__global__ void k_adj_gap_param(AdjStep A) {
    const MechDev& m = A.m[M_HALFGAP];
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= m.n) return;
    const int node = m.node[j];
    const int src = A.gap_partner[j];
    const double vgap = src >= 0 ? A.v0[src] : m.col(HG_VGAP)[j];
    A.grad_ggap[j] -= A.mu[node] * (1.e2 / A.area[node]) * (A.v1[node] - vgap);
}

// lambda_v^n of each source node += G mu at the nodes of the instances it feeds, summed in
// instance order by one thread per source
__global__ void k_adj_gap_cross(AdjStep A) {
    const MechDev& m = A.m[M_HALFGAP];
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= A.ngap_src) return;
    double acc = 0.0;
    for (int e = A.gap_begin[q]; e < A.gap_begin[q + 1]; ++e) {
        const int j = A.gap_inst[e];
        const int node = m.node[j];
        acc += m.col(HG_G)[j] * (1.e2 / A.area[node]) * A.mu[node];
    }
    A.lam_v_new[A.gap_src[q]] += acc;
}

// events delivered at step n: ExpSyn dL/dw += lambda_geff, Exp2Syn dL/dw += factor
// (lambda_A + lambda_B) (one block)
__global__ void __launch_bounds__(256) k_adj_events(AdjStep A) {
    const int cnt = A.ev_count[0];
    for (int e = threadIdx.x; e < cnt; e += blockDim.x) {
        const int packed = A.ev[e];
        const int inst = packed & 0x3fffffff;
        if ((packed >> 30) == 0) {
            atomicAdd(&A.grad_w[inst], A.lam_g[inst]);
        } else {
            const MechDev& m = A.m[M_EXP2SYN];
            atomicAdd(&A.grad_w2[inst], m.col(E2_FACTOR)[inst] * (A.lam_ab[inst] + A.lam_ab[m.n + inst]));
        }
    }
}

// loss term of v^n: lambda_v^n[node] += 2 scale (v^n - target^n_j) for every loss index j
// of the node, one thread per distinct node adding its terms in list order
__global__ void k_adj_loss(const double* v, const int* nodes, const int* begin, const int* idx, int n,
                           const double* target, double scale, double* lam) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= n) return;
    const int node = nodes[q];
    const double vn = v[node];
    double acc = lam[node];
    for (int e = begin[q]; e < begin[q + 1]; ++e) acc += 2.0 * scale * (vn - target[idx[e]]);
    lam[node] = acc;
}

// out[r * nnodes + j] = tape_v[r * row + nodes[j]]
__global__ void k_adj_gather(const double* tape_v, long long row, const int* nodes, int nnodes, int nrows,
                             double* out) {
    const long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= static_cast<long long>(nnodes) * nrows) return;
    const long long r = t / nnodes;
    const int j = static_cast<int>(t - r * nnodes);
    out[t] = tape_v[r * row + nodes[j]];
}

// Adam: one thread per tied group (optimizer.cpp:351-393, optimizer_kernels.cu:173-195)
__global__ void k_adam(AdamArgs A) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= A.ngroup) return;
    const int b0 = A.begin[g], b1 = A.begin[g + 1];
    if (b1 <= b0) return;
    double sum = 0.0;
    for (int k = b0; k < b1; ++k) sum += *A.grad[k];
    const double avg = sum / static_cast<double>(b1 - b0);
    const double sg = avg * A.impedance[g] * A.inv_record_steps;
    double w;
    if (A.type == 0) {
        w = *A.w[b0] - A.lr * sg;
    } else if (A.type == 1) {
        const double vel = A.momentum * A.m[g] - A.lr * sg;
        A.m[g] = vel;
        w = *A.w[b0] + vel;
    } else {
        const double m = A.beta1 * A.m[g] + (1.0 - A.beta1) * sg;
        const double v = A.beta2 * A.v[g] + (1.0 - A.beta2) * sg * sg;
        A.m[g] = m;
        A.v[g] = v;
        const double mhat = m / (1.0 - pow(A.beta1, static_cast<double>(A.step)));
        const double vhat = v / (1.0 - pow(A.beta2, static_cast<double>(A.step)));
        w = *A.w[b0] - A.lr * mhat / (sqrt(vhat) + A.eps);
    }
    for (int k = b0; k < b1; ++k) {
        *A.w[k] = w;
        *A.grad[k] = 0.0;
    }
}

inline dim3 grid_of(long long n, int block = kBlock) {
    long long g = (n + block - 1) / block;
    return dim3(static_cast<unsigned>(g > 0 ? g : 1));
}

}  // namespace

// Kernels of one mechanism touch only that mechanism's adjoints, except for the
// per-node lambda_v and d (one density instance per node; point processes go by
// node groups) and lambda_cai / lambda_ica (one CaDynamics_E2 per ca_ion instance,
// written by it before the solve and by Ca_HVA after), so no two launches race.
// The node-parallel kernels take the mechanisms in a.fuse_*; the rest keep their own
// kernels, launched where each node's sums keep their order.
static void launch_adj_before_nodes_and_cond(const AdjStep& a, hipStream_t s);
static void launch_adj_events_and_gaps(const AdjStep& a, hipStream_t s);

// Launches the tasks of S (blocks per task from the instance counts) as one k_adj_side.
static void launch_side(const AdjStep& a, AdjSide S, hipStream_t s) {
    auto count = [&](int task) {
        switch (task) {
            case AT_HH_STATE: case AT_HH_PARAM: return a.m[M_HH].n;
            case AT_SYN_STATE: case AT_SYN_PARAM: return a.m[M_EXPSYN].n;
            case AT_SYN2_STATE: case AT_SYN2_PARAM: return a.m[M_EXP2SYN].n;
            case AT_PAS_PARAM: return a.m[M_PAS].n;
            default: return 0;
        }
    };
    int b = 0;
    for (int t = 0; t < S.n; ++t) {
        S.begin[t] = b;
        b += (count(S.task[t]) + kBlock - 1) / kBlock;
    }
    S.begin[S.n] = b;
    if (b > 0) hipLaunchKernelGGL(k_adj_side, dim3(b), dim3(kBlock), 0, s, a, S);
}

void launch_adj_before_solve(const AdjStep& a, hipStream_t s) {
    auto own = [&](int id, unsigned bit, unsigned fused) { return a.m[id].n > 0 && !(fused & bit); };
    // hh's state adjoint (the only one adding to lambda_v here) and the synapses' decay
    // adjoints side by side in one launch, when no other mechanism keeps its own kernels
    if (!own(M_CAHVA, kAdjCaHVA, a.fuse_state) && !own(M_HDLA, kAdjHdla, a.fuse_state) &&
        !own(M_CADYN, kAdjCaDyn, a.fuse_state) && !a.fold_syn) {
        AdjSide S{};
        if (own(M_HH, kAdjHH, a.fuse_state)) S.task[S.n++] = AT_HH_STATE;
        if (a.m[M_EXPSYN].n > 0) S.task[S.n++] = AT_SYN_STATE;
        if (a.m[M_EXP2SYN].n > 0) S.task[S.n++] = AT_SYN2_STATE;
        if (S.n > 1) {
            launch_side(a, S, s);
            launch_adj_before_nodes_and_cond(a, s);
            return;
        }
    }
    if (own(M_HH, kAdjHH, a.fuse_state)) hipLaunchKernelGGL(k_adj_hh_state, grid_of(a.m[M_HH].n), dim3(kBlock), 0, s, a);
    if (own(M_CAHVA, kAdjCaHVA, a.fuse_state))
        hipLaunchKernelGGL(k_adj_cahva_state, grid_of(a.m[M_CAHVA].n), dim3(kBlock), 0, s, a);
    if (own(M_HDLA, kAdjHdla, a.fuse_state))
        hipLaunchKernelGGL(k_adj_hdla_state, grid_of(a.m[M_HDLA].n), dim3(kBlock), 0, s, a);
    if (own(M_CADYN, kAdjCaDyn, a.fuse_state))
        hipLaunchKernelGGL(k_adj_cadyn, grid_of(a.m[M_CADYN].n), dim3(kBlock), 0, s, a);
    const long long nsyn = a.fold_syn ? static_cast<long long>(a.m[M_EXPSYN].n) + a.m[M_EXP2SYN].n : 0;
    if (!a.fold_syn && a.m[M_EXPSYN].n > 0)
        hipLaunchKernelGGL(k_adj_syn_state, grid_of(a.m[M_EXPSYN].n), dim3(kBlock), 0, s, a);
    if (!a.fold_syn && a.m[M_EXP2SYN].n > 0)
        hipLaunchKernelGGL(k_adj_syn2_state, grid_of(a.m[M_EXP2SYN].n), dim3(kBlock), 0, s, a);
    (void)nsyn;
    launch_adj_before_nodes_and_cond(a, s);
}

// The node-parallel kernel before the solve and the conductance kernels after it.
static void launch_adj_before_nodes_and_cond(const AdjStep& a, hipStream_t s) {
    auto own = [&](int id, unsigned bit, unsigned fused) { return a.m[id].n > 0 && !(fused & bit); };
    const long long nsyn = a.fold_syn ? static_cast<long long>(a.m[M_EXPSYN].n) + a.m[M_EXP2SYN].n : 0;
    hipLaunchKernelGGL(k_adj_before_nodes, grid_of(a.N + nsyn), dim3(kBlock), 0, s, a);
    if (own(M_PAS, kAdjPas, a.fuse_cond))
        hipLaunchKernelGGL(k_adj_cond_pas, grid_of(a.m[M_PAS].n), dim3(kBlock), 0, s, a);
    if (own(M_HH, kAdjHH, a.fuse_cond)) hipLaunchKernelGGL(k_adj_cond_hh, grid_of(a.m[M_HH].n), dim3(kBlock), 0, s, a);
    if (own(M_CAHVA, kAdjCaHVA, a.fuse_cond))
        hipLaunchKernelGGL(k_adj_cond_cahva, grid_of(a.m[M_CAHVA].n), dim3(kBlock), 0, s, a);
    if (own(M_HDLA, kAdjHdla, a.fuse_cond))
        hipLaunchKernelGGL(k_adj_cond_hdla, grid_of(a.m[M_HDLA].n), dim3(kBlock), 0, s, a);
    if (!a.fold_syn && a.m[M_EXPSYN].ngrp > 0)
        hipLaunchKernelGGL(k_adj_cond_syn, grid_of(a.m[M_EXPSYN].ngrp), dim3(kBlock), 0, s, a);
    if (!a.fold_syn && a.m[M_EXP2SYN].ngrp > 0)
        hipLaunchKernelGGL(k_adj_cond_syn2, grid_of(a.m[M_EXP2SYN].ngrp), dim3(kBlock), 0, s, a);
    if (a.m[M_HALFGAP].ngrp > 0)
        hipLaunchKernelGGL(k_adj_cond_gap, grid_of(a.m[M_HALFGAP].ngrp), dim3(kBlock), 0, s, a);
}

void launch_adj_after_solve(const AdjStep& a, hipStream_t s) {
    auto own = [&](int id, unsigned bit) { return a.m[id].n > 0 && !(a.fuse_param & bit); };
    const long long nsyn = a.fold_syn ? static_cast<long long>(a.m[M_EXPSYN].n) + a.m[M_EXP2SYN].n : 0;
    hipLaunchKernelGGL(k_adj_after_nodes, grid_of(a.N + nsyn), dim3(kBlock), 0, s, a);
    // hh's and pas's parameter terms and the synapses' (none adds to lambda_v) side by side
    // in one launch, when Ca_HVA and hd_la (which do) run in the node-parallel kernel or not at all
    if (!own(M_CAHVA, kAdjCaHVA) && !own(M_HDLA, kAdjHdla) && !a.fold_syn) {
        AdjSide S{};
        if (own(M_HH, kAdjHH)) S.task[S.n++] = AT_HH_PARAM;
        if (own(M_PAS, kAdjPas)) S.task[S.n++] = AT_PAS_PARAM;
        if (a.m[M_EXPSYN].n > 0) S.task[S.n++] = AT_SYN_PARAM;
        if (a.m[M_EXP2SYN].n > 0) S.task[S.n++] = AT_SYN2_PARAM;
        if (S.n > 1) {
            launch_side(a, S, s);
            launch_adj_events_and_gaps(a, s);
            return;
        }
    }
    if (own(M_HH, kAdjHH)) hipLaunchKernelGGL(k_adj_hh_param, grid_of(a.m[M_HH].n), dim3(kBlock), 0, s, a);
    if (own(M_PAS, kAdjPas)) hipLaunchKernelGGL(k_adj_pas_param, grid_of(a.m[M_PAS].n), dim3(kBlock), 0, s, a);
    if (own(M_CAHVA, kAdjCaHVA))
        hipLaunchKernelGGL(k_adj_cahva_param, grid_of(a.m[M_CAHVA].n), dim3(kBlock), 0, s, a);
    if (own(M_HDLA, kAdjHdla)) hipLaunchKernelGGL(k_adj_hdla_param, grid_of(a.m[M_HDLA].n), dim3(kBlock), 0, s, a);
    if (!a.fold_syn && a.m[M_EXPSYN].n > 0)
        hipLaunchKernelGGL(k_adj_syn_param, grid_of(a.m[M_EXPSYN].n), dim3(kBlock), 0, s, a);
    if (!a.fold_syn && a.m[M_EXP2SYN].n > 0)
        hipLaunchKernelGGL(k_adj_syn2_param, grid_of(a.m[M_EXP2SYN].n), dim3(kBlock), 0, s, a);
    launch_adj_events_and_gaps(a, s);
}

// The events' weight terms and the gap junctions' terms, after the parameter terms.
static void launch_adj_events_and_gaps(const AdjStep& a, hipStream_t s) {
    if (a.m[M_EXPSYN].n > 0 || a.m[M_EXP2SYN].n > 0) hipLaunchKernelGGL(k_adj_events, dim3(1), dim3(256), 0, s, a);
    if (a.m[M_HALFGAP].n > 0) {
        hipLaunchKernelGGL(k_adj_gap_param, grid_of(a.m[M_HALFGAP].n), dim3(kBlock), 0, s, a);
        if (a.ngap_src > 0) hipLaunchKernelGGL(k_adj_gap_cross, grid_of(a.ngap_src), dim3(kBlock), 0, s, a);
    }
}

void launch_adj_loss(const double* v, const int* nodes, const int* begin, const int* idx, int n,
                     const double* target, double scale, double* lam, hipStream_t s) {
    if (n > 0)
        hipLaunchKernelGGL(k_adj_loss, grid_of(n), dim3(kBlock), 0, s, v, nodes, begin, idx, n, target, scale, lam);
}

void launch_adj_gather(const double* tape_v, long long row, const int* nodes, int nnodes, int nrows, double* out,
                       hipStream_t s) {
    const long long n = static_cast<long long>(nnodes) * nrows;
    if (n > 0) hipLaunchKernelGGL(k_adj_gather, grid_of(n), dim3(kBlock), 0, s, tape_v, row, nodes, nnodes, nrows, out);
}

void launch_adam(const AdamArgs& a, hipStream_t s) {
    if (a.ngroup > 0) hipLaunchKernelGGL(k_adam, grid_of(a.ngroup), dim3(kBlock), 0, s, a);
}

}  // namespace hx
