// HIP kernels of the per-step simulation core (CDNA4 / gfx950, wave64).
//
// One fixed step (reference order: simulate.cpp:410-442, simulate.cu:722-771):
//   deliver events -> t+dt/2 -> VecPlay -> currents (FD Jacobian) -> capacitance
//   + axial terms -> tree solve -> v += dv -> gap copy -> t+dt/2 -> VecPlay ->
//   states (ion writers first) -> record.
//
// Kernels here:
//   k_dense ........ node-parallel fused mechanisms; optionally finishes the
//                    previous step's cnexp state update before evaluating this
//                    step's currents, so each state is read and written once
//   k_sparse<M> .... the same arithmetic for mechanisms present on a subset of
//                    nodes (instance-parallel, gather v / update d, rhs)
//   k_point<M> ..... point-process currents (IClamp, ExpSyn, Exp2Syn, HalfGap),
//                    scaled by 1e2/area and accumulated with fp64 atomics
//   k_solve ........ one wavefront per solve unit (a few consecutive cells):
//                    capacitance + axial assembly, the
//                    Hines elimination over chunked unbranched runs, back
//                    substitution and v update; junction values through LDS
//   k_solve_res .... the same for units small enough to be held whole in LDS:
//                    read once, solved in LDS records, written once
//   k_spike ........ threshold detection, wave-ballot compaction into the spike
//                    log, fan-out of deliveries into the device event ring
//   k_input ........ VecStim trains (sorted on the host) entering the ring;
//                    k_input_set: several cell groups sharing a stream, one launch
//   k_netstim ...... NetStims that receive events: the step's delivery loop for them
//   k_deliver ...... NET_RECEIVE of the events due this step
//   k_vecplay, k_record, k_gap, init kernels.
#include <algorithm>

#include <hip/hip_ext.h>

#include "hx_internal.h"
#include "mech_math.h"
#include "random123.h"
#include "solve_chunk.h"

namespace hx {

namespace {


__device__ __forceinline__ int ion_index(const MechDev& m, int which, int j) {
    const int* p = m.ion[which];
    return p ? p[j] : j;
}

// ---------------------------------------------------------------------------
// per-mechanism state updates (shared by the dense and sparse kernels).  Each
// takes the state it updates as values and returns the new values (also
// stored), so a kernel that goes on to the current evaluation keeps them in
// registers instead of reading back what it just wrote.
// ---------------------------------------------------------------------------
struct HHState { double m, h, n; };
struct CaHVAState { double m, h; };

// Per-compartment parameters and states are touched once per step, and a step
// moves far more data than L2 and the Infinity Cache hold: they are read and
// written with the non-temporal hint, which leaves the caches to the node
// arrays (v, d, rhs) that the tree solve reads right after the node kernel
// (config 3: 0.84 -> 0.80 ms per step).
__device__ __forceinline__ double lds_(const double* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void sts_(double* p, double v) { __builtin_nontemporal_store(v, p); }

// Parameter column c of instance j.  A column with one value for every instance
// is read once per wave from uval (a scalar load) instead of once per instance
// from HBM; the mask is uniform, so the choice is a scalar branch.
__device__ __forceinline__ double ldp(const MechDev& m, int c, int j) {
    if ((m.umask >> c) & 1u) return m.uval[c];
    return lds_(m.col(c) + j);
}

__device__ __forceinline__ HHState hh_load(const MechDev& m, int j) {
    return {lds_(m.col(HH_M) + j), lds_(m.col(HH_H) + j), lds_(m.col(HH_N) + j)};
}
__device__ __forceinline__ CaHVAState cahva_load(const MechDev& m, int j) {
    return {lds_(m.col(CH_M) + j), lds_(m.col(CH_H) + j)};
}

// wr: also store the update's rates (minf, mtau, ...); wa: also store the current's
// assigned outputs (i, ina, gna, ...).
__device__ __forceinline__ void hh_store(const StepArgs& A, const MechDev& m, int j, double v, const HHState& s,
                                         bool wr) {
    sts_(m.col(HH_M) + j, s.m);
    sts_(m.col(HH_H) + j, s.h);
    sts_(m.col(HH_N) + j, s.n);
    if (wr) {
        double minf, mtau, hinf, htau, ninf, ntau;
        hh_rates(v, A.c.hh_q10, minf, mtau, hinf, htau, ninf, ntau);
        sts_(m.col(HH_MINF) + j, minf); sts_(m.col(HH_MTAU) + j, mtau);
        sts_(m.col(HH_HINF) + j, hinf); sts_(m.col(HH_HTAU) + j, htau);
        sts_(m.col(HH_NINF) + j, ninf); sts_(m.col(HH_NTAU) + j, ntau);
    }
}
__device__ __forceinline__ HHState hh_state(const StepArgs& A, const MechDev& m, int j, double v, HHState s,
                                            bool wr) {
    hh_gates_r(v, A.c.hh_q10, A.dt, s.m, s.h, s.n);
    hh_store(A, m, j, v, s, wr);
    return s;
}

__device__ __forceinline__ void cahva_store(const MechDev& m, int j, double v, const CaHVAState& s,
                                            const double* ca_erev, int ci, bool wr) {
    sts_(m.col(CH_M) + j, s.m);
    sts_(m.col(CH_H) + j, s.h);
    if (wr) {
        double mInf, mTau, mAlpha, mBeta, hInf, hTau, hAlpha, hBeta;
        cahva_rates(v, mInf, mTau, mAlpha, mBeta, hInf, hTau, hAlpha, hBeta);
        sts_(m.col(CH_ECA) + j, ca_erev[ci]);
        sts_(m.col(CH_MINF) + j, mInf); sts_(m.col(CH_MTAU) + j, mTau); sts_(m.col(CH_MALPHA) + j, mAlpha); sts_(m.col(CH_MBETA) + j, mBeta);
        sts_(m.col(CH_HINF) + j, hInf); sts_(m.col(CH_HTAU) + j, hTau); sts_(m.col(CH_HALPHA) + j, hAlpha); sts_(m.col(CH_HBETA) + j, hBeta);
    }
}
__device__ __forceinline__ CaHVAState cahva_state(const StepArgs& A, const MechDev& m, int j, double v,
                                                  CaHVAState s, const double* ca_erev, int ci, bool wr) {
    cahva_gates_r(v, A.dt, s.m, s.h);
    cahva_store(m, j, v, s, ca_erev, ci, wr);
    return s;
}

__device__ __forceinline__ void hdla_store(const StepArgs& A, const MechDev& m, int j, double v, double l,
                                           double vhalfl, double tau, bool wr) {
    sts_(m.col(HD_L) + j, l);
    if (wr) {
        double linf, taul;
        hdla_rate(v, vhalfl, tau, A.c, linf, taul);
        sts_(m.col(HD_LINF) + j, linf); sts_(m.col(HD_TAUL) + j, taul);
    }
}
__device__ __forceinline__ double hdla_state(const StepArgs& A, const MechDev& m, int j, double v, double l, bool wr) {
    const double vhalfl = ldp(m, HD_VHALFL, j), tau = ldp(m, HD_TAU, j);
    l = hdla_gate_r(v, l, vhalfl, tau, A.c, A.dt);
    hdla_store(A, m, j, v, l, vhalfl, tau, wr);
    return l;
}

// returns the new cai (the caller stores it)
__device__ __forceinline__ double cadyn_state(const StepArgs& A, const MechDev& m, int j, double cai, double ica) {
    if (A.c.cd_uniform) return cadyn_uniform(cai, ica, A.c);
    return cadyn_step_r(cai, ica, ldp(m, CD_GAMMA, j), ldp(m, CD_DECAY, j), ldp(m, CD_DEPTH, j),
                        ldp(m, CD_MINCAI, j), A.dt);
}

// ---------------------------------------------------------------------------
// per-mechanism FD currents: returns I(v), sets g = (I(v+0.001) - I(v)) / 0.001
// (mech_template.cuh:616-626); ion currents of the I(v) evaluation are
// returned for the caller to accumulate
// ---------------------------------------------------------------------------
__device__ __forceinline__ double pas_cur(const MechDev& m, int j, double v, double& g, bool wa) {
    double gp = ldp(m, PAS_G, j), ep = ldp(m, PAS_E, j);
    double v1 = v + 0.001;
    double i1 = gp * (v1 - ep);
    double i0 = gp * (v - ep);
    g = (i1 - i0) * 1000.0;   // / 0.001
    if (wa) sts_(m.col(PAS_I) + j, i0);
    return i0;
}

__device__ __forceinline__ double hh_cur(const MechDev& m, int j, double v, const HHState& s, double ena, double ek,
                                         double& g, double& ina, double& ik, bool wa) {
    double gnabar = ldp(m, HH_GNABAR, j), gkbar = ldp(m, HH_GKBAR, j);
    double gl = ldp(m, HH_GL, j), el = ldp(m, HH_EL, j);
    double gna, gk, il;
    double v1 = v + 0.001;
    double i1 = hh_current(v1, gnabar, gkbar, gl, el, s.m, s.h, s.n, ena, ek, gna, ina, gk, ik, il);
    double i0 = hh_current(v, gnabar, gkbar, gl, el, s.m, s.h, s.n, ena, ek, gna, ina, gk, ik, il);
    g = (i1 - i0) * 1000.0;   // / 0.001
    if (wa) {
        sts_(m.col(HH_ENA) + j, ena); sts_(m.col(HH_EK) + j, ek); sts_(m.col(HH_INA) + j, ina); sts_(m.col(HH_IK) + j, ik);
        sts_(m.col(HH_IL) + j, il); sts_(m.col(HH_GNA) + j, gna); sts_(m.col(HH_GK) + j, gk);
    }
    return i0;
}

__device__ __forceinline__ double cahva_cur(const MechDev& m, int j, double v, const CaHVAState& s, double eca,
                                            double& g, bool wa) {
    double gbar = ldp(m, CH_GBAR, j);
    double v1 = v + 0.001;
    double gg = gbar * s.m * s.m * s.h;
    double i1 = gg * (v1 - eca);
    double i0 = gg * (v - eca);
    g = (i1 - i0) * 1000.0;   // / 0.001
    if (wa) {
        sts_(m.col(CH_ECA) + j, eca); sts_(m.col(CH_G) + j, gg); sts_(m.col(CH_ICA) + j, i0); sts_(m.col(CH_IMECH) + j, i0);
    }
    return i0;
}

__device__ __forceinline__ double hdla_cur(const StepArgs& A, const MechDev& m, int j, double v, double l,
                                           double& g, bool wa) {
    double ghd = ldp(m, HD_GHDBAR, j) * l;
    double v1 = v + 0.001;
    double i1 = ghd * (v1 - A.c.hd_ehd);
    double i0 = ghd * (v - A.c.hd_ehd);
    g = (i1 - i0) * 1000.0;   // / 0.001
    if (wa) { sts_(m.col(HD_GHD) + j, ghd); sts_(m.col(HD_I) + j, i0); }
    return i0;
}

// Per-step part of an ion (eion.cuh:155-166): zero cur and dcurdv, and
// recompute erev from the concentrations when iontype has 0100.  Used by the
// instance-parallel ion kernel; the fused kernel keeps cur in registers.
__device__ __forceinline__ void ion_cur(const MechDev& m, int j, double z, double ktf, int write_dcurdv) {
    sts_(m.col(ION_CUR) + j, 0.);
    if (write_dcurdv) sts_(m.col(ION_DCURDV) + j, 0.);
    if (m.iontype[j] & 0100)
        sts_(m.col(ION_EREV) + j, nernst_r(m.col(ION_CONCI)[j], m.col(ION_CONCO)[j], z, ktf));
}

// erev of ion x at dense instance i for this step's current evaluation.  ci:
// the inside concentration when the caller already holds it (have_ci).
__device__ __forceinline__ double dense_ion_erev(const StepArgs& A, const MechDev& ion, int x, int i, double z,
                                                 bool have_ci, double ci) {
    const int type = A.ion_type[x] >= 0 ? A.ion_type[x] : ion.iontype[i];
    if (type & 0100) {
        const double e = nernst_r(have_ci ? ci : lds_(ion.col(ION_CONCI) + i), ldp(ion, ION_CONCO, i), z, A.c.ktf);
        if (A.ion_store & (2u << (2 * x))) sts_(ion.col(ION_EREV) + i, e);
        return e;
    }
    return ldp(ion, ION_EREV, i);
}

__device__ __forceinline__ void dense_ion_store(const StepArgs& A, const MechDev& ion, int x, int i, double cur,
                                                bool wdc) {
    if (A.ion_store & (1u << (2 * x))) sts_(ion.col(ION_CUR) + i, cur);
    if (wdc) sts_(ion.col(ION_DCURDV) + i, 0.);
}

// Point-process currents of one mechanism on the nodes of this block, summed
// in instance order (instances are sorted by node).  s_first / s_last: LDS
// tables of kBlock ints.  Every thread of the block must call it.
template <int MECH>
__device__ __forceinline__ void fold_point(const StepArgs& A, int i, bool live, double v, int* s_first,
                                           int* s_last, double& rhs, double& d, int store);

// What one node-kernel launch does.  RtPass reads it from the launch's arguments;
// SteadyPass<MASK, FOLD> fixes it at compile time for a steady step (the previous
// step's state update and this step's currents, with CaDynamics_E2 updated right
// after its ica, storing nothing but states, d and rhs), so that instance has no
// branches on flags and the compiler schedules its loads and arithmetic freely.
// Both run the same arithmetic in the same order: same bits.
struct RtPass {
    const StepArgs& A;
    __device__ bool has(int b) const { return (A.dense_mask >> b) & 1u; }
    __device__ bool folds(int b) const { return (A.fold_mask >> b) & 1u; }
    __device__ bool do_state() const { return A.do_state != 0; }
    __device__ bool do_current() const { return A.do_current != 0; }
    __device__ bool cadyn_skip() const { return A.cadyn_skip != 0; }
    __device__ bool cadyn_after() const { return A.cadyn_after != 0; }
    __device__ bool write_assigned() const { return A.write_assigned != 0; }
    __device__ bool write_rates() const { return A.write_rates != 0; }
    __device__ bool write_dcurdv() const { return A.write_dcurdv != 0; }
    __device__ int point_assigned() const { return A.point_assigned; }
};

template <unsigned MASK, unsigned FOLD>
struct SteadyPass {
    static constexpr bool has(int b) { return (MASK >> b) & 1u; }
    static constexpr bool folds(int b) { return (FOLD >> b) & 1u; }
    static constexpr bool do_state() { return true; }
    static constexpr bool do_current() { return true; }
    static constexpr bool cadyn_skip() { return has(M_CADYN); }
    static constexpr bool cadyn_after() { return has(M_CADYN); }
    static constexpr bool write_assigned() { return false; }
    static constexpr bool write_rates() { return false; }
    static constexpr bool write_dcurdv() { return false; }
    static constexpr int point_assigned() { return 0; }
};

// Whether a launch's arguments are the steady step SteadyPass<MASK, FOLD> fixes.
template <unsigned MASK, unsigned FOLD>
bool is_steady(const StepArgs& a) {
    const bool cd = (MASK >> M_CADYN) & 1u;
    return a.dense_mask == MASK && a.fold_mask == FOLD && a.do_state && a.do_current &&
           (a.cadyn_skip != 0) == cd && (a.cadyn_after != 0) == cd && !a.write_assigned && !a.write_rates &&
           !a.write_dcurdv && !a.point_assigned;
}

// ---------------------------------------------------------------------------
// fused node-parallel kernel for dense mechanisms: the previous step's state
// update (ion writers first, simulate.cpp:822-834) and this step's currents in
// CoreNEURON mechanism order, with the synapse (ExpSyn, Exp2Syn) currents of
// the block's nodes added in their place.  Ion currents are summed in
// registers and each ion array is written once.
// ---------------------------------------------------------------------------
template <class P>
__device__ __forceinline__ void dense_node(const StepArgs& A, const P& p, int* s_first, int* s_last) {
    const int i = A.node0 + blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = i < A.N;
    const double v = live ? A.v[i] : 0.0;
    const MechDev& na = A.m[M_NA_ION];
    const MechDev& kk = A.m[M_K_ION];
    const MechDev& ca = A.m[M_CA_ION];
    HHState hs{};
    CaHVAState cs{};
    double hl = 0.0, cai = 0.0;
    const bool have_cai = p.do_state() && p.has(M_CADYN) && !p.cadyn_skip();
    const bool wr = p.write_rates(), wa = p.write_assigned();
    if (live) {
        if (p.do_state()) {
            // every state load ahead of the first state store: a load written after a
            // store (which may alias it, as far as the compiler can tell) waits for it
            double* conci = ca.col(ION_CONCI);
            double ci0 = 0.0, ica0 = 0.0, l0 = 0.0;
            HHState h0{};
            CaHVAState c0{};
            if (have_cai) {
                ci0 = lds_(conci + i);
                ica0 = lds_(ca.col(ION_CUR) + i);
            }
            if (p.has(M_HH)) h0 = hh_load(A.m[M_HH], i);
            if (p.has(M_CAHVA)) c0 = cahva_load(A.m[M_CAHVA], i);
            if (p.has(M_HDLA)) l0 = lds_(A.m[M_HDLA].col(HD_L) + i);
            if (have_cai) {
                cai = cadyn_state(A, A.m[M_CADYN], i, ci0, ica0);
                sts_(conci + i, cai);
            }
            if (p.has(M_HH)) hs = hh_state(A, A.m[M_HH], i, v, h0, wr);
            if (p.has(M_CAHVA)) cs = cahva_state(A, A.m[M_CAHVA], i, v, c0, ca.col(ION_EREV), i, wr);
            if (p.has(M_HDLA)) hl = hdla_state(A, A.m[M_HDLA], i, v, l0, wr);
        } else if (p.do_current()) {
            if (p.has(M_HH)) hs = hh_load(A.m[M_HH], i);
            if (p.has(M_CAHVA)) cs = cahva_load(A.m[M_CAHVA], i);
            if (p.has(M_HDLA)) hl = lds_(A.m[M_HDLA].col(HD_L) + i);
        }
    }
    if (!p.do_current()) return;
    // the capacitance term of the diagonal (capac.cpp:68-80) is added here,
    // ahead of the membrane conductances, so the solve reads one diagonal
    double rhs = 0.0, d = live ? A.cfac * (A.cm_uniform ? A.cm_value : A.cm[i]) : 0.0, g, cur;
    double prhs = 0.0, pd = 0.0;
    if (p.folds(M_EXPSYN))
        fold_point<M_EXPSYN>(A, i, live, v, s_first, s_last, prhs, pd, p.point_assigned());
    if (p.folds(M_EXP2SYN))
        fold_point<M_EXP2SYN>(A, i, live, v, s_first, s_last, prhs, pd, p.point_assigned());
    if (!live) return;
    double ena = 0.0, ek = 0.0, eca = 0.0, ina = 0.0, ik = 0.0, ica = 0.0;
    if (p.has(M_PAS)) { cur = pas_cur(A.m[M_PAS], i, v, g, wa); rhs -= cur; d += g; }
    if (p.has(M_NA_ION)) ena = dense_ion_erev(A, na, 0, i, 1.0, false, 0.0);
    if (p.has(M_K_ION)) ek = dense_ion_erev(A, kk, 1, i, 1.0, false, 0.0);
    if (p.has(M_HH)) {
        double ina_h, ik_h;
        cur = hh_cur(A.m[M_HH], i, v, hs, ena, ek, g, ina_h, ik_h, wa);
        ina += ina_h;
        ik += ik_h;
        rhs -= cur; d += g;
    }
    rhs += prhs;   // ExpSyn, Exp2Syn (mechanism types 5, 6)
    d += pd;
    // cai for the Nernst potential and, when CaDynamics_E2 runs after this pass, for its update
    const bool need_ci = p.has(M_CADYN) && p.cadyn_after();
    const double ci = have_cai ? cai : (need_ci ? lds_(ca.col(ION_CONCI) + i) : 0.0);
    if (p.has(M_CA_ION)) eca = dense_ion_erev(A, ca, 2, i, 2.0, have_cai || need_ci, ci);
    if (p.has(M_CAHVA)) {
        cur = cahva_cur(A.m[M_CAHVA], i, v, cs, eca, g, wa);
        ica += cur;
        rhs -= cur; d += g;
    }
    if (p.has(M_HDLA)) { cur = hdla_cur(A, A.m[M_HDLA], i, v, hl, g, wa); rhs -= cur; d += g; }
    A.d[i] = d;
    // with every d and rhs term of the step in this pass, rhs + d v makes the solve's
    // unknown the new voltage itself: the axial terms cancel, so the solve never reads v
    A.rhs[i] = A.yform ? fma(d, v, rhs) : rhs;
    const bool wdc = p.write_dcurdv();
    if (p.has(M_NA_ION)) dense_ion_store(A, na, 0, i, ina, wdc);
    if (p.has(M_K_ION)) dense_ion_store(A, kk, 1, i, ik, wdc);
    if (p.has(M_CA_ION)) dense_ion_store(A, ca, 2, i, ica, wdc);
    if (need_ci) sts_(ca.col(ION_CONCI) + i, cadyn_state(A, A.m[M_CADYN], i, ci, ica));
}

__global__ void __launch_bounds__(kBlock) k_dense(StepArgs A) {
    __shared__ int s_first[kBlock], s_last[kBlock];
    dense_node(A, RtPass{A}, s_first, s_last);
}

template <unsigned MASK, unsigned FOLD>
__global__ void __launch_bounds__(kBlock) k_dense_steady(StepArgs A) {
    __shared__ int s_first[kBlock], s_last[kBlock];
    dense_node(A, SteadyPass<MASK, FOLD>{}, s_first, s_last);
}

// ---------------------------------------------------------------------------
// sparse density mechanisms: instance-parallel, at most one instance per node
// ---------------------------------------------------------------------------
template <int MECH>
__global__ void __launch_bounds__(kBlock) k_sparse(StepArgs A) {
    const MechDev& m = A.m[MECH];
    const int j = A.pt0 + blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= m.n || j >= A.pt1) return;
    const int node = m.node[j];
    const double v = A.v[node];
    if (MECH == M_NA_ION || MECH == M_K_ION || MECH == M_CA_ION) {
        if (A.do_current) ion_cur(m, j, MECH == M_CA_ION ? 2.0 : 1.0, A.c.ktf, A.write_dcurdv);
        return;
    }
    const MechDev& na = A.m[M_NA_ION];
    const MechDev& kk = A.m[M_K_ION];
    const MechDev& ca = A.m[M_CA_ION];
    HHState hs{};
    CaHVAState cs{};
    double hl = 0.0;
    if (A.do_state) {
        if (MECH == M_CADYN) {
            const int ci = ion_index(m, 2, j);
            double* conci = ca.col(ION_CONCI);
            conci[ci] = cadyn_state(A, m, j, conci[ci], ca.col(ION_CUR)[ci]);
        }
        if (MECH == M_HH) hs = hh_state(A, m, j, v, hh_load(m, j), A.write_rates);
        if (MECH == M_CAHVA)
            cs = cahva_state(A, m, j, v, cahva_load(m, j), ca.col(ION_EREV), ion_index(m, 2, j), A.write_rates);
        if (MECH == M_HDLA) hl = hdla_state(A, m, j, v, m.col(HD_L)[j], A.write_rates);
    } else if (A.do_current) {
        if (MECH == M_HH) hs = hh_load(m, j);
        if (MECH == M_CAHVA) cs = cahva_load(m, j);
        if (MECH == M_HDLA) hl = m.col(HD_L)[j];
    }
    if (!A.do_current || MECH == M_CADYN) return;
    double g = 0.0, cur = 0.0;
    if (MECH == M_PAS) cur = pas_cur(m, j, v, g, A.write_assigned);
    if (MECH == M_HH) {
        const int ni = ion_index(m, 0, j), ki = ion_index(m, 1, j);
        double ina, ik;
        cur = hh_cur(m, j, v, hs, na.col(ION_EREV)[ni], kk.col(ION_EREV)[ki], g, ina, ik, A.write_assigned);
        if (A.hh_owns_ions) {         // the only writer of these currents: no ion kernel zeroed them
            na.col(ION_CUR)[ni] = ina;
            kk.col(ION_CUR)[ki] = ik;
            if (A.write_dcurdv) {
                na.col(ION_DCURDV)[ni] = 0.0;
                kk.col(ION_DCURDV)[ki] = 0.0;
            }
        } else {
            na.col(ION_CUR)[ni] += ina;
            kk.col(ION_CUR)[ki] += ik;
        }
    }
    if (MECH == M_CAHVA) {
        const int ci = ion_index(m, 2, j);
        cur = cahva_cur(m, j, v, cs, ca.col(ION_EREV)[ci], g, A.write_assigned);
        ca.col(ION_CUR)[ci] += cur;
    }
    if (MECH == M_HDLA) cur = hdla_cur(A, m, j, v, hl, g, A.write_assigned);
    A.rhs[node] -= cur;
    A.d[node] += g;
}

// ---------------------------------------------------------------------------
// point processes: FD current x 1e2/area (mech_template.cuh:616-646).  One
// thread per node that carries instances of the mechanism sums them and
// updates d and rhs of that node once, so no atomics are needed (each launch
// covers one mechanism; launches are ordered on the stream).
// ---------------------------------------------------------------------------
template <int MECH>
__device__ __forceinline__ void point_current(const StepArgs& A, const MechDev& m, int j, double v, double& i0,
                                              double& g, int store) {
    const double v1 = v + 0.001;
    double i1 = 0.0;
    i0 = 0.0;
    if (MECH == M_ICLAMP) {
        const double del = m.col(IC_DELAY)[j], dur = m.col(IC_DUR)[j];
        double cur = 0.0;
        if (A.t < del + dur && A.t >= del) cur = m.col(IC_AMP)[j];
        i1 = cur;
        i0 = cur;
        if (store) m.col(IC_I)[j] = cur;
    } else if (MECH == M_HALFGAP) {
        const double vg = m.col(HG_VGAP)[j], gg = m.col(HG_G)[j];
        i1 = (vg - v1) * gg;
        i0 = (vg - v) * gg;
        if (store) m.col(HG_I)[j] = i0;
    } else if (MECH == M_EXPSYN) {
        const double gg = m.col(ES_G)[j], e = m.col(ES_E)[j];
        i1 = gg * (v1 - e);
        i0 = gg * (v - e);
        if (store) m.col(ES_I)[j] = i0;
    } else if (MECH == M_EXP2SYN) {
        const double gg = m.col(E2_B)[j] - m.col(E2_A)[j];
        const double e = m.col(E2_E)[j];
        i1 = gg * (v1 - e);
        i0 = gg * (v - e);
        if (store) { m.col(E2_G)[j] = gg; m.col(E2_I)[j] = i0; }
    }
    g = (i1 - i0) * 1000.0;   // / 0.001
}

template <int MECH>
__device__ __forceinline__ void fold_point(const StepArgs& A, int i, bool live, double v, int* s_first,
                                           int* s_last, double& rhs, double& d, int store) {
    const MechDev& m = A.m[MECH];
    const int b0 = A.node0 + blockIdx.x * kBlock;   // blk_begin covers the launch's blocks
    const int s0 = m.blk_begin[blockIdx.x], s1 = m.blk_begin[blockIdx.x + 1];
    if (s1 == s0) return;                        // same for the whole block
    const int t = threadIdx.x;
    s_first[t] = 0;
    s_last[t] = 0;
    __syncthreads();
    for (int s = s0 + t; s < s1; s += kBlock) {
        const int node = m.node[s];
        if (s == s0 || m.node[s - 1] != node) s_first[node - b0] = s;
        if (s == s1 - 1 || m.node[s + 1] != node) s_last[node - b0] = s + 1;
    }
    __syncthreads();
    const int f = s_first[t], l = s_last[t];
    if (live && l > f) {
        const double mfact = 1.e2 / A.area[i];
        for (int j = f; j < l; ++j) {
            double i0, g;
            point_current<MECH>(A, m, j, v, i0, g, store);
            rhs -= i0 * mfact;
            d += g * mfact;
        }
    }
    __syncthreads();                             // the tables are reused by the next mechanism
}

template <int MECH>
__device__ __forceinline__ void point_group(const StepArgs& A, int q, double v, double mfact, double& rhs,
                                            double& d) {
    const MechDev& m = A.m[MECH];
    rhs = 0.0;
    d = 0.0;
    for (int j = m.grp_begin[q]; j < m.grp_begin[q + 1]; ++j) {
        double i0, g;
        point_current<MECH>(A, m, j, v, i0, g, A.point_assigned);
        g *= mfact;
        i0 *= mfact;
        if (MECH == M_ICLAMP || MECH == M_HALFGAP) {   // ELECTRODE_CURRENT: the sign flips
            rhs += i0;
            d -= g;
        } else {
            rhs -= i0;
            d += g;
        }
    }
}

template <int MECH>
__global__ void __launch_bounds__(kBlock) k_point(StepArgs A) {
    const MechDev& m = A.m[MECH];
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= m.ngrp) return;
    const int node = m.grp_node[q];
    double rhs, d;
    point_group<MECH>(A, q, A.v[node], 1.e2 / A.area[node], rhs, d);
    A.rhs[node] += rhs;
    A.d[node] += d;
}

// IClamp and HalfGap in one launch, one thread per node carrying either: the node's
// IClamp sum is added to its rhs and d first, then its HalfGap sum, the additions the
// two single-mechanism launches make one after the other (same bits).
__global__ void __launch_bounds__(kBlock) k_point_electrodes(StepArgs A, PointUnion U) {
    const int u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= U.n) return;
    const int node = U.node[u];
    const double v = A.v[node];
    const double mfact = 1.e2 / A.area[node];
    double r = A.rhs[node], dd = A.d[node], rhs, d;
    if (U.grp[0][u] >= 0) {
        point_group<M_ICLAMP>(A, U.grp[0][u], v, mfact, rhs, d);
        r += rhs;
        dd += d;
    }
    if (U.grp[1][u] >= 0) {
        point_group<M_HALFGAP>(A, U.grp[1][u], v, mfact, rhs, d);
        r += rhs;
        dd += d;
    }
    A.rhs[node] = r;
    A.d[node] = dd;
}

template <int MECH>
__global__ void __launch_bounds__(kBlock) k_point_state(StepArgs A) {
    const MechDev& m = A.m[MECH];
    const int j = A.pt0 + blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= m.n || j >= A.pt1) return;
    if (MECH == M_EXPSYN) {
        double* g = m.col(ES_G);
        g[j] = expsyn_decay(g[j], m.col(ES_TAU)[j], A.dt);
    } else if (MECH == M_EXP2SYN) {
        double* a = m.col(E2_A);
        double* b = m.col(E2_B);
        double aa = a[j], bb = b[j];
        a[j] = exp2syn_decay(aa, m.col(E2_TAU1)[j], A.dt);
        b[j] = exp2syn_decay(bb, m.col(E2_TAU2)[j], A.dt);
    }
}

// ---------------------------------------------------------------------------
// finitialize: mechanism INITIAL blocks (mech_template.cuh:552-585, eion.cuh:183-197)
// ---------------------------------------------------------------------------
template <int MECH>
__global__ void __launch_bounds__(kBlock) k_init(StepArgs A) {
    const MechDev& m = A.m[MECH];
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= m.n) return;
    if (MECH == M_NA_ION || MECH == M_K_ION || MECH == M_CA_ION) {
        const double z = MECH == M_CA_ION ? 2.0 : 1.0;
        const int x = MECH == M_NA_ION ? 0 : (MECH == M_K_ION ? 1 : 2);
        const double ci0 = kIonConciInit[x];
        const double co0 = kIonConcoInit[x];
        int it = m.iontype[j];
        if (it & 04) { m.col(ION_CONCI)[j] = ci0; m.col(ION_CONCO)[j] = co0; }
        if (it & 040) m.col(ION_EREV)[j] = nernst(m.col(ION_CONCI)[j], m.col(ION_CONCO)[j], z, A.c.ktf);
        return;
    }
    const int node = m.dense ? j : m.node[j];
    const double v = A.v[node];
    if (MECH == M_HH) {
        const MechDev& na = A.m[M_NA_ION];
        const MechDev& kk = A.m[M_K_ION];
        double minf, mtau, hinf, htau, ninf, ntau;
        hh_rates(v, A.c.hh_q10, minf, mtau, hinf, htau, ninf, ntau);
        m.col(HH_ENA)[j] = na.col(ION_EREV)[ion_index(m, 0, j)];
        m.col(HH_EK)[j] = kk.col(ION_EREV)[ion_index(m, 1, j)];
        m.col(HH_MINF)[j] = minf; m.col(HH_MTAU)[j] = mtau; m.col(HH_HINF)[j] = hinf;
        m.col(HH_HTAU)[j] = htau; m.col(HH_NINF)[j] = ninf; m.col(HH_NTAU)[j] = ntau;
        m.col(HH_M)[j] = minf; m.col(HH_H)[j] = hinf; m.col(HH_N)[j] = ninf;
    } else if (MECH == M_CAHVA) {
        double mInf, mTau, mAlpha, mBeta, hInf, hTau, hAlpha, hBeta;
        cahva_rates(v, mInf, mTau, mAlpha, mBeta, hInf, hTau, hAlpha, hBeta);
        m.col(CH_ECA)[j] = A.m[M_CA_ION].col(ION_EREV)[ion_index(m, 2, j)];
        m.col(CH_MINF)[j] = mInf; m.col(CH_MTAU)[j] = mTau; m.col(CH_MALPHA)[j] = mAlpha; m.col(CH_MBETA)[j] = mBeta;
        m.col(CH_HINF)[j] = hInf; m.col(CH_HTAU)[j] = hTau; m.col(CH_HALPHA)[j] = hAlpha; m.col(CH_HBETA)[j] = hBeta;
        m.col(CH_M)[j] = mInf;
        m.col(CH_H)[j] = hInf;
    } else if (MECH == M_HDLA) {
        double linf, taul;
        hdla_rate(v, m.col(HD_VHALFL)[j], m.col(HD_TAU)[j], A.c, linf, taul);
        m.col(HD_LINF)[j] = linf;
        m.col(HD_TAUL)[j] = taul;
        m.col(HD_L)[j] = linf;
    } else if (MECH == M_ICLAMP) {
        m.col(IC_I)[j] = 0.0;
    } else if (MECH == M_HALFGAP) {
        m.col(HG_I)[j] = 0.0;
    } else if (MECH == M_EXPSYN) {
        m.col(ES_G)[j] = 0;
    } else if (MECH == M_EXP2SYN) {
        double tau1 = m.col(E2_TAU1)[j], tau2 = m.col(E2_TAU2)[j];
        if (tau1 / tau2 > 0.9999) { tau1 = 0.9999 * tau2; m.col(E2_TAU1)[j] = tau1; }
        if (tau1 / tau2 < 1e-9) { tau1 = tau2 * 1e-9; m.col(E2_TAU1)[j] = tau1; }
        m.col(E2_A)[j] = 0.0;
        m.col(E2_B)[j] = 0.0;
        double tp = (tau1 * tau2) / (tau2 - tau1) * log(tau2 / tau1);
        m.col(E2_FACTOR)[j] = 1.0 / (-exp(-tp / tau1) + exp(-tp / tau2));
    }
    // CaDynamics_E2 keeps cai in the ca_ion conci column (its INITIAL copies it
    // back unchanged, CaDynamics_E2.cu:87-96); pas has no INITIAL block.
}

__global__ void k_set_v(double* v, int n, double val) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) v[i] = val;
}

// ---------------------------------------------------------------------------
// Tree solve: one wavefront per solve unit, a forest of a few consecutive
// cells (a wavefront issues the same instructions however many of its lanes
// carry a chunk, so packing cells into one wavefront divides the issue work
// of the whole solve).  Forward rounds run leaves -> root, each
// lane eliminating one chunk (an unbranched run of <= kChunk nodes) into its
// parent; the head's contribution to the parent chunk's tail is passed through
// an LDS slot.  Back substitution runs the rounds in reverse.
//   assembly: simulate.cpp:527-555, capacitance capac.cpp:68-80
//   elimination / back substitution: simulate.cpp:558-581
// ---------------------------------------------------------------------------
// The workgroup is exactly one wavefront: LDS accesses of a wavefront execute
// in program order, so a round boundary only needs the compiler not to move
// LDS accesses across it (a workgroup barrier would also wait for the round's
// global stores to land).
__device__ __forceinline__ void round_boundary() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

constexpr int kNeutral = kRoundMax;       // stage entry holding the padding value

// 1/x: hardware reciprocal estimate refined by two Newton-Raphson steps
// (each step squares the relative error), correct to about an ulp.
__device__ __forceinline__ double rcp_nr(double x) {
    double r = __builtin_amdgcn_rcp(x);
    double e = __builtin_fma(-x, r, 1.0);
    r = __builtin_fma(r, e, r);
    e = __builtin_fma(-x, r, 1.0);
    return __builtin_fma(r, e, r);
}

// A RoundInfo on its way in: every lane loads the same 32 bytes with vector
// loads issued a round ahead of use (the schedule's scalar reads would have
// to wait for the round's vector stores), then moves them to uniform
// registers.
struct RoundV {
    uint4 x0, x1, x2;
};
static_assert(sizeof(RoundV) == sizeof(RoundInfo), "RoundV mirrors RoundInfo");
struct RoundU {
    int desc_begin, desc_count, node_base, node_count, maxlen;
    uint32_t off[kChunk / 2];      // off[k] in half k % 2 of off[k / 2]
    __device__ __forceinline__ int offset(int k) const { return (off[k >> 1] >> (16 * (k & 1))) & 0xFFFF; }
};
__device__ __forceinline__ RoundV load_round(const RoundInfo* rounds, int r) {
    const uint4* p = reinterpret_cast<const uint4*>(rounds + r);
    return {p[0], p[1], p[2]};
}
__device__ __forceinline__ RoundU uniform_round(const RoundV& v) {
    RoundU u;
    const uint32_t w0 = __builtin_amdgcn_readfirstlane(v.x0.x);
    const uint32_t w1 = __builtin_amdgcn_readfirstlane(v.x0.y);
    u.desc_begin = w0 & 0xFFFF;
    u.desc_count = w0 >> 16;
    u.node_base = w1 & 0xFFFF;
    u.node_count = w1 >> 16;
    u.off[0] = __builtin_amdgcn_readfirstlane(v.x0.z);
    u.off[1] = __builtin_amdgcn_readfirstlane(v.x0.w);
    u.off[2] = __builtin_amdgcn_readfirstlane(v.x1.x);
    u.off[3] = __builtin_amdgcn_readfirstlane(v.x1.y);
    u.off[4] = __builtin_amdgcn_readfirstlane(v.x1.z);
    u.off[5] = __builtin_amdgcn_readfirstlane(v.x1.w);
    u.off[6] = __builtin_amdgcn_readfirstlane(v.x2.x);
    u.off[7] = __builtin_amdgcn_readfirstlane(v.x2.y);
    u.maxlen = __builtin_amdgcn_readfirstlane(v.x2.z) & 0xFF;
    return u;
}

// Round data in flight: every lane loads kPer elements of each array of the
// round's contiguous node block (coalesced, unconditional, clamped to the
// block) plus its chunk descriptor, so each round issues the same number of
// vector-memory instructions and the compiler's wait counts stay static.
struct FwdBuf {
    double x[5][kPer];    // d rhs a b v
    uint2 q;              // ChunkDesc
    RoundU ri;
};
template <int kX>
struct BackBuf {
    double x[2 + kX][kPer];   // s (in rhs), w [, the old v]
    uint2 q;
    RoundU ri;
};

struct SolveCtx {
    const SolveArgs& S;
    // Not __restrict__: with it the compiler proves the tables unwritten and turns
    // their uniform reads into scalar loads, whose waits share the LDS counter
    // and drain it; as vector loads they are requested a round ahead.
    const RoundInfo* rounds;                // this unit's rounds
    const uint2* desc;                      // this unit's descriptors
    int nb;                                 // first node of the unit
    int nn;                                 // nodes of the unit
    double* slots;                          // LDS, 2 per chunk
    double* stage;                          // LDS, kStageArrays x kStageStride
    int lane;
};

// Results leave the solve as raw buffer stores on a descriptor that spans the
// unit's nodes; a store whose offset lies past the descriptor's range is
// dropped by the hardware, which is how padding slots are masked without a
// branch (kDrop is far past any unit: units hold at most 65535 nodes).
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
constexpr int kBufferConfig = 0x00020000;   // raw buffer, 32-bit data format (CDNA)
constexpr int kDrop = static_cast<int>(0x80000000u);
__device__ __forceinline__ __amdgpu_buffer_rsrc_t cell_buffer(double* base, int nnode) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, nnode * static_cast<int>(sizeof(double)), kBufferConfig);
}
__device__ __forceinline__ void store_f64(__amdgpu_buffer_rsrc_t r, int byte_offset, double x) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, x), r, byte_offset, 0, 0);
}

// Stage positions of the first KM slots of the lane's chunk (the neutral
// entry past the chunk's length), byte offsets of its nodes in the unit (kDrop
// past the length) and tp, the position of the tail.
template <int KM>
__device__ __forceinline__ void round_positions(const RoundU& ri, int len, int lane, int* rp, int* wo, int& tp) {
    tp = kNeutral;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        const int p = ri.offset(k) + lane;
        rp[k] = k < len ? p : kNeutral;
        wo[k] = k < len ? (ri.node_base + p) * static_cast<int>(sizeof(double)) : kDrop;
        if (k == len - 1) tp = p;
    }
}

// A chunk hands its parent the pair (cd, ce) through one 16-byte LDS slot.
struct SlotPair {
    double cd, ce;
};

struct StageIn {
    const double* st;
    const int* rp;
    __device__ __forceinline__ double at(int arr, int k) const { return st[arr * kStageStride + rp[k]]; }
    __device__ __forceinline__ FwdNode fwd(int k) const {
        return {at(SA_DB, k), at(SA_RM, k), at(SA_A, k), at(SA_B, k), at(SA_V, k)};
    }
    __device__ __forceinline__ BackNode back(int k) const { return {at(SA_RM, k), at(SA_A, k), 0.0}; }
};
// back substitution that also reports x = vn - v: the old voltages are staged too
struct StageInX : StageIn {
    __device__ __forceinline__ BackNode back(int k) const { return {at(SA_RM, k), at(SA_A, k), at(SA_V, k)}; }
};

__device__ __forceinline__ unsigned clamp_index(int lane, int j, int count) {
    const unsigned e = static_cast<unsigned>(lane + kWave * j);
    const unsigned last = static_cast<unsigned>(count - 1);
    return e < last ? e : last;
}

__device__ __forceinline__ uint2 load_desc(const SolveCtx& C, const RoundU& ri) {
    const int top = ri.desc_count > 0 ? ri.desc_count - 1 : 0;   // padding rounds: any descriptor
    return C.desc[ri.desc_begin + (C.lane < top ? C.lane : top)];
}

__device__ __forceinline__ void fwd_load(const SolveCtx& C, FwdBuf& B, const RoundV& rv) {
    const RoundU ri = uniform_round(rv);
    const int base = C.nb + ri.node_base;
    const double* d = C.S.d + base;
    const double* rhs = C.S.rhs + base;
    const double* a = C.S.a + base;
    const double* b = C.S.b + base;
    const double* v = C.S.v + base;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const unsigned e = clamp_index(C.lane, j, ri.node_count);
        B.x[0][j] = d[e];
        B.x[1][j] = rhs[e];
        B.x[2][j] = a[e];
        B.x[3][j] = b[e];
    }
    // v enters elimination only through the axial terms, which rhs + d v already holds
    if (C.S.yform) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) B.x[4][j] = 0.0;
    } else {
#pragma unroll
        for (int j = 0; j < kPer; ++j) B.x[4][j] = v[clamp_index(C.lane, j, ri.node_count)];
    }
    B.q = load_desc(C, ri);
    B.ri = ri;
}

// Solves the round held in B; once B is staged, the next round (table entry
// `next`, already loaded) is requested into N.  kX: the pivots D go to d (the
// reference leaves them there; only read back through the API).
template <int kX>
__device__ __forceinline__ void fwd_round(const SolveCtx& C, const FwdBuf& B, FwdBuf& N, const RoundV& next) {
    const RoundU& ri = B.ri;
    const uint2 q = B.q;
    double* st = C.stage;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int e = C.lane + kWave * j;
        st[SA_DB * kStageStride + e] = B.x[0][j];
        st[SA_RM * kStageStride + e] = B.x[1][j];
        st[SA_A * kStageStride + e] = B.x[2][j];
        st[SA_B * kStageStride + e] = B.x[3][j];
        st[SA_V * kStageStride + e] = B.x[4][j];
    }
    round_boundary();
    fwd_load(C, N, next);
    const bool act = C.lane < ri.desc_count;
    const int slot = q.x & 0xFFFF;
    const bool has_parent = (q.x >> 16) != kNone;
    const int child_begin = q.y & 0xFFFF;
    const int len = act ? (q.y >> 16) & 0xFF : 0;
    const int nchild = act ? q.y >> 24 : 0;
    SlotPair* pairs = reinterpret_cast<SlotPair*>(C.slots);
    // the children's terms, summed in child order (the first two unrolled)
    double acd = 0.0, ace = 0.0;
    if (nchild > 0) {
        const SlotPair p0 = pairs[child_begin];
        acd = p0.cd;
        ace = p0.ce;
        if (nchild > 1) {
            const SlotPair p1 = pairs[child_begin + 1];
            acd += p1.cd;
            ace += p1.ce;
            for (int ch = 2; ch < nchild; ++ch) {
                const SlotPair pc = pairs[child_begin + ch];
                acd += pc.cd;
                ace += pc.ce;
            }
        }
    }
    // results go straight to HBM: node k of the lane's chunk sits at offset(k) + lane
    // of the round's block, so each store instruction writes contiguous memory
    const __amdgpu_buffer_rsrc_t rd = cell_buffer(C.S.d + C.nb, C.nn);
    const __amdgpu_buffer_rsrc_t ru = cell_buffer(C.S.rhs + C.nb, C.nn);
    const __amdgpu_buffer_rsrc_t rw = cell_buffer(C.S.w + C.nb, C.nn);
    double cd, ce;
    // the serial chunk arithmetic alone runs at raised issue priority (the same wave at
    // raised priority throughout takes too many issue slots from the waves beside it)
    __builtin_amdgcn_s_setprio(3);
    dispatch_chunk_bound(ri.maxlen, [&](auto km) {
        constexpr int KM = decltype(km)::value;
        int rp[KM], wo[KM], tp;
        round_positions<KM>(ri, len, C.lane, rp, wo, tp);
        if (nchild > 0) {
            double db = st[SA_DB * kStageStride + tp], rm = st[SA_RM * kStageStride + tp];
            tail_inject(db, rm, st[SA_V * kStageStride + tp], acd, ace);
            st[SA_DB * kStageStride + tp] = db;
            st[SA_RM * kStageStride + tp] = rm;
        }
        auto out = [&](int k, double D, double sv, double w) {
            if constexpr (kX != 0) store_f64(rd, wo[k], D);
            store_f64(ru, wo[k], sv);
            store_f64(rw, wo[k], w);
        };
        chunk_forward_math<KM>(has_parent, StageIn{st, rp}, out, rcp_nr, cd, ce);
    });
    __builtin_amdgcn_s_setprio(0);
    if (act && has_parent) pairs[slot] = SlotPair{cd, ce};
    round_boundary();
}

template <int kX>
__device__ __forceinline__ void back_load(const SolveCtx& C, BackBuf<kX>& B, const RoundV& rv) {
    const RoundU ri = uniform_round(rv);
    const int base = C.nb + ri.node_base;
    const double* sv = C.S.rhs + base;
    const double* w = C.S.w + base;
    const double* v = C.S.v + base;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const unsigned e = clamp_index(C.lane, j, ri.node_count);
        B.x[0][j] = sv[e];
        B.x[1][j] = w[e];
        if constexpr (kX != 0) B.x[2][j] = v[e];
    }
    B.q = load_desc(C, ri);
    B.ri = ri;
}

// kX: x = vn - v goes to rhs (the reference leaves the solution there), and the old
// voltage to w, where an outputs-only node pass after the call reads it.
template <int kX>
__device__ __forceinline__ void back_round(const SolveCtx& C, const BackBuf<kX>& B, BackBuf<kX>& N,
                                           const RoundV& next) {
    const RoundU& ri = B.ri;
    const uint2 q = B.q;
    double* st = C.stage;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int e = C.lane + kWave * j;
        st[SA_RM * kStageStride + e] = B.x[0][j];
        st[SA_A * kStageStride + e] = B.x[1][j];
        if constexpr (kX != 0) st[SA_V * kStageStride + e] = B.x[2][j];
    }
    round_boundary();
    back_load<kX>(C, N, next);
    const bool act = C.lane < ri.desc_count;
    const int slot = q.x & 0xFFFF;
    const int parent_slot = q.x >> 16;
    const int len = act ? (q.y >> 16) & 0xFF : 0;
    const double vpar = (act && parent_slot != kNone) ? C.slots[2 * parent_slot] : 0.0;
    const __amdgpu_buffer_rsrc_t rv = cell_buffer(C.S.v + C.nb, C.nn);
    const __amdgpu_buffer_rsrc_t rx = cell_buffer(C.S.rhs + C.nb, C.nn);
    const __amdgpu_buffer_rsrc_t rw = cell_buffer(C.S.w + C.nb, C.nn);
    double vtail = 0.0;
    __builtin_amdgcn_s_setprio(3);
    dispatch_chunk_bound(ri.maxlen, [&](auto km) {
        constexpr int KM = decltype(km)::value;
        int rp[KM], wo[KM], tp;
        round_positions<KM>(ri, len, C.lane, rp, wo, tp);
        auto out = [&](int k, double vn, double vo) {
            store_f64(rv, wo[k], vn);
            if constexpr (kX != 0) {
                store_f64(rx, wo[k], vn - vo);
                store_f64(rw, wo[k], vo);   // w (read for this node already) keeps the old voltage
            }
            if (k == len - 1) vtail = vn;
        };
        if constexpr (kX != 0) chunk_back_math<KM>(StageInX{{st, rp}}, out, vpar);
        else chunk_back_math<KM>(StageIn{st, rp}, out, vpar);
    });
    __builtin_amdgcn_s_setprio(0);
    if (act) C.slots[2 * slot] = vtail;   // the tail's new voltage
    round_boundary();
}

// Waits for every outstanding vector-memory access (s_waitcnt vmcnt(0); the
// other counters are left alone).  Used once before each sweep's loop, so the
// compiler's wait counts at the loop head only have to cover the loop's own
// steady state (one round's stores after the buffer's loads).
__device__ __forceinline__ void drain_vector_memory() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// One wavefront per unit.  Elimination walks the rounds from the leaves
// (round nround-1) to the root, back substitution from the root out.  While a
// round is solved from one register buffer, the next round's data is loaded
// into the other (a round takes longer than an HBM round trip); the round-table
// entry is fetched a round earlier still.  A unit's round count is even (the
// schedule appends a padding round with no chunks when needed), so each loop
// trip solves two rounds and the buffers never trade registers.  Round indices
// past either end are clamped to a real round, whose loads are issued but
// never used.
// A workgroup holds S.waves units, one wavefront each, with an LDS region each; there
// is no workgroup barrier, so a wavefront whose unit finishes early just exits.
template <int kX>
__global__ void __launch_bounds__(kWave * kSolveMaxWaves) k_solve(SolveArgs S, const RoundInfo* rounds_all,
                                                                  const uint2* desc, int max_chunks) {
    extern __shared__ double lds[];
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int c = blockIdx.x * S.waves + wv;
    if (c >= S.nunit) return;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int rb = S.unit_round_begin[c];
    const int nround = S.unit_round_begin[c + 1] - rb;
    const int last = nround - 1;
    double* slots = lds + static_cast<size_t>(wv) * solve_lds_doubles(max_chunks);
    double* stage = slots + 2 * max_chunks;
    if (lane < kStageArrays) stage[lane * kStageStride + kNeutral] = lane == SA_DB ? 1.0 : 0.0;
    round_boundary();
    const RoundInfo* rounds = rounds_all + rb;
    const SolveCtx C{S,
                     rounds,
                     desc + S.unit_desc_begin[c],
                     S.unit_node_begin[c],
                     S.unit_node_begin[c + 1] - S.unit_node_begin[c],
                     slots,
                     stage,
                     lane};
    auto fwd_idx = [&](int r) { return r > 0 ? r : 0; };
    auto back_idx = [&](int r) { return r < last ? r : last; };

    {
        FwdBuf x, y;
        fwd_load(C, x, load_round(rounds, last));
        RoundV nx = load_round(rounds, last - 1);
        drain_vector_memory();
        for (int r = last; r > 0; r -= 2) {
            RoundV n = load_round(rounds, fwd_idx(r - 2));
            fwd_round<kX>(C, x, y, nx);
            nx = load_round(rounds, fwd_idx(r - 3));
            fwd_round<kX>(C, y, x, n);
        }
    }
    {
        BackBuf<kX> x, y;
        back_load<kX>(C, x, load_round(rounds, 0));
        RoundV nx = load_round(rounds, 1);
        drain_vector_memory();
        for (int r = 0; r < last; r += 2) {
            RoundV n = load_round(rounds, back_idx(r + 2));
            back_round<kX>(C, x, y, nx);
            nx = load_round(rounds, back_idx(r + 3));
            back_round<kX>(C, y, x, n);
        }
    }
}

// ---------------------------------------------------------------------------
// tree solve with the unit held in LDS
// ---------------------------------------------------------------------------
// A unit whose nodes, round table and descriptors fit kResUnitBudget of LDS (cells of a
// few hundred nodes) is read from HBM once: d, rhs, a, b and v of each node go to one
// 40-byte LDS record, elimination and back substitution run over the same rounds and
// chunks as k_solve with s, w, the pivots and the new voltages kept in the records, and
// the results are written once.  The per-chunk arithmetic and the order of every sum are
// k_solve's, so the results are the same bits.  A round then waits on LDS instead of an
// HBM round trip and has no staging, and s and w never go to HBM (48 instead of 80 bytes
// per node).  A record's fields sit at fixed offsets, so one address serves a node's five
// reads.

// Node k of the lane's chunk reads record rp[k] (in doubles: record index x 5; the
// neutral record past the chunk's length) and writes record wp[k] (the sink record past
// the length, so that padding slots leave the neutral record as it is).
template <int kY>
struct ResIn {
    const double* st;
    const int* rp;
    __device__ __forceinline__ FwdNode fwd(int k) const {
        const double* r = st + rp[k];
        return {r[SA_DB], r[SA_RM], r[SA_A], r[SA_B], kY ? 0.0 : r[SA_V]};
    }
    __device__ __forceinline__ BackNode back(int k) const {
        const double* r = st + rp[k];
        return {r[SA_RM], r[SA_A], 0.0};
    }
};

template <int KM>
__device__ __forceinline__ void res_positions(const RoundU& ri, int len, int lane, int neutral, int* rp, int* wp,
                                              int& tp) {
    tp = neutral * kStageArrays;
#pragma unroll
    for (int k = 0; k < KM; ++k) {
        const int p = ri.node_base + ri.offset(k) + lane;
        rp[k] = (k < len ? p : neutral) * kStageArrays;
        wp[k] = (k < len ? p : neutral + 1) * kStageArrays;
        if (k == len - 1) tp = p * kStageArrays;
    }
}

// Round r's table entry (every lane reads the same 48 bytes) and the lane's descriptor.
__device__ __forceinline__ RoundU res_round(const uint4* rtab, int r) {
    const uint4* p = rtab + 3 * r;
    return uniform_round(RoundV{p[0], p[1], p[2]});
}
__device__ __forceinline__ uint2 res_desc(const uint2* dtab, int ndesc, const RoundU& ri, int lane) {
    const int top = ri.desc_count > 0 ? ri.desc_count - 1 : 0;
    const int e = ri.desc_begin + (lane < top ? lane : top);
    return dtab[e < ndesc ? e : ndesc - 1];    // padding rounds: any descriptor of the unit
}

constexpr int kResBatch = 4;    // nodes a lane moves per batch at the start and the end

// One wavefront per unit, S.waves units per workgroup, each with its own LDS region.
// kY: rhs holds rhs + d v (SolveArgs::yform), so elimination takes v as 0; v is then read
// only where x = v_new - v is stored (kX).
template <int kX, int kY>
__global__ void __launch_bounds__(kWave * kSolveMaxWaves) k_solve_res(SolveArgs S, const RoundInfo* rounds_all,
                                                                      const uint2* desc_all, int max_chunks) {
    extern __shared__ double lds[];
    const int wv = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int c = blockIdx.x * S.waves + wv;
    if (c >= S.nunit) return;
    const int lane = static_cast<int>(threadIdx.x) % kWave;
    const int rb = S.unit_round_begin[c];
    const int nround = S.unit_round_begin[c + 1] - rb;
    const int db0 = S.unit_desc_begin[c];
    const int ndesc = S.unit_desc_begin[c + 1] - db0;
    const int nb = S.unit_node_begin[c];
    const int nn = S.unit_node_begin[c + 1] - nb;
    const int neutral = S.res_nodes;                  // the sink record is neutral + 1
    double* slots = lds + static_cast<size_t>(wv) * res_lds_doubles(S.res_nodes, max_chunks, S.res_rounds);
    double* st = slots + 2 * max_chunks;
    uint4* rtab = reinterpret_cast<uint4*>(st + res_record_doubles(S.res_nodes));
    uint2* dtab = reinterpret_cast<uint2*>(rtab + 3 * S.res_rounds);

    // the unit's round table, descriptors and node records into LDS
    {
        const uint4* rsrc = reinterpret_cast<const uint4*>(rounds_all + rb);
        for (int i = lane; i < 3 * nround; i += kWave) rtab[i] = rsrc[i];
        for (int i = lane; i < ndesc; i += kWave) dtab[i] = desc_all[db0 + i];
        const double* src[kStageArrays] = {S.d + nb, S.rhs + nb, S.a + nb, S.b + nb, S.v + nb};
        for (int i0 = 0; i0 < nn; i0 += kWave * kResBatch) {
            double x[kStageArrays][kResBatch];
#pragma unroll
            for (int j = 0; j < kResBatch; ++j) {
                const int i = i0 + j * kWave + lane;
                const int e = i < nn ? i : nn - 1;
#pragma unroll
                for (int q = 0; q < kStageArrays; ++q)
                    x[q][j] = (q != SA_V || !kY || kX) ? lds_(src[q] + e) : 0.0;
            }
#pragma unroll
            for (int j = 0; j < kResBatch; ++j) {
                const int i = i0 + j * kWave + lane;
                if (i < nn) {
#pragma unroll
                    for (int q = 0; q < kStageArrays; ++q) st[i * kStageArrays + q] = x[q][j];
                }
            }
        }
        if (lane < 2 * kStageArrays) {     // the neutral record (db 1, the rest 0) and the sink
            const int q = lane % kStageArrays;
            st[(neutral + lane / kStageArrays) * kStageArrays + q] = q == SA_DB ? 1.0 : 0.0;
        }
    }
    round_boundary();

    // elimination, leaves to root: s to RM, w to A, the pivot D (kX) to DB
    SlotPair* pairs = reinterpret_cast<SlotPair*>(slots);
    for (int r = nround - 1; r >= 0; --r) {
        const RoundU ri = res_round(rtab, r);
        const uint2 q = res_desc(dtab, ndesc, ri, lane);
        const bool act = lane < ri.desc_count;
        const int slot = q.x & 0xFFFF;
        const bool has_parent = (q.x >> 16) != kNone;
        const int child_begin = q.y & 0xFFFF;
        const int len = act ? (q.y >> 16) & 0xFF : 0;
        const int nchild = act ? q.y >> 24 : 0;
        double acd = 0.0, ace = 0.0;
        if (nchild > 0) {
            const SlotPair p0 = pairs[child_begin];
            acd = p0.cd;
            ace = p0.ce;
            if (nchild > 1) {
                const SlotPair p1 = pairs[child_begin + 1];
                acd += p1.cd;
                ace += p1.ce;
                for (int ch = 2; ch < nchild; ++ch) {
                    const SlotPair pc = pairs[child_begin + ch];
                    acd += pc.cd;
                    ace += pc.ce;
                }
            }
        }
        double cd, ce;
        __builtin_amdgcn_s_setprio(3);
        dispatch_chunk_bound(ri.maxlen, [&](auto km) {
            constexpr int KM = decltype(km)::value;
            int rp[KM], wp[KM], tp;
            res_positions<KM>(ri, len, lane, neutral, rp, wp, tp);
            if (nchild > 0) {
                double db = st[tp + SA_DB], rm = st[tp + SA_RM];
                tail_inject(db, rm, kY ? 0.0 : st[tp + SA_V], acd, ace);
                st[tp + SA_DB] = db;
                st[tp + SA_RM] = rm;
            }
            auto out = [&](int k, double D, double sv, double w) {
                double* o = st + wp[k];
                if constexpr (kX != 0) o[SA_DB] = D;
                o[SA_RM] = sv;
                o[SA_A] = w;
            };
            chunk_forward_math<KM>(has_parent, ResIn<kY>{st, rp}, out, rcp_nr, cd, ce);
        });
        __builtin_amdgcn_s_setprio(0);
        if (act && has_parent) pairs[slot] = SlotPair{cd, ce};
        round_boundary();
    }

    // back substitution, root to leaves: the new voltages to B (free after elimination)
    for (int r = 0; r < nround; ++r) {
        const RoundU ri = res_round(rtab, r);
        const uint2 q = res_desc(dtab, ndesc, ri, lane);
        const bool act = lane < ri.desc_count;
        const int slot = q.x & 0xFFFF;
        const int parent_slot = q.x >> 16;
        const int len = act ? (q.y >> 16) & 0xFF : 0;
        const double vpar = (act && parent_slot != kNone) ? slots[2 * parent_slot] : 0.0;
        double vtail = 0.0;
        __builtin_amdgcn_s_setprio(3);
        dispatch_chunk_bound(ri.maxlen, [&](auto km) {
            constexpr int KM = decltype(km)::value;
            int rp[KM], wp[KM], tp;
            res_positions<KM>(ri, len, lane, neutral, rp, wp, tp);
            auto out = [&](int k, double vn, double) {
                st[wp[k] + SA_B] = vn;
                if (k == len - 1) vtail = vn;
            };
            chunk_back_math<KM>(ResIn<kY>{st, rp}, out, vpar);
        });
        __builtin_amdgcn_s_setprio(0);
        if (act) slots[2 * slot] = vtail;   // the tail's new voltage
        round_boundary();
    }

    // results: v; with kX also D in d, x = vn - v in rhs and the old voltage in w
    for (int i0 = 0; i0 < nn; i0 += kWave * kResBatch) {
#pragma unroll
        for (int j = 0; j < kResBatch; ++j) {
            const int i = i0 + j * kWave + lane;
            if (i < nn) {
                const double* rec = st + i * kStageArrays;
                const double vn = rec[SA_B];
                S.v[nb + i] = vn;
                if constexpr (kX != 0) {
                    const double vo = rec[SA_V];
                    S.d[nb + i] = rec[SA_DB];
                    S.rhs[nb + i] = vn - vo;
                    S.w[nb + i] = vo;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// events
// ---------------------------------------------------------------------------
__device__ __forceinline__ int delivery_step(const double* ttab, int k, int kmax, double T, double half_dt) {
    // first step m >= k whose receive window t_m + dt/2 covers T (postsyn.cpp:43-61)
    int m = k;
    const double est = (T - ttab[k]) / (2.0 * half_dt);
    if (est > 2.0) m = est - 1.0 < static_cast<double>(kmax - k) ? k + static_cast<int>(est) - 1 : kmax;
    while (m < kmax && ttab[m] + half_dt < T) ++m;
    while (m > k && ttab[m - 1] + half_dt >= T) --m;
    return m;
}

__device__ __forceinline__ void ring_push(const EventRing& R, int m, int packed) {
    const int slot = m & (R.nslot - 1);
    const int pos = atomicAdd(&R.count[slot], 1);
    if (pos < R.cap) R.entry[static_cast<long long>(slot) * R.cap + pos] = packed;
    else atomicOr(R.overflow, 1);
}

__device__ __forceinline__ void inbox_push(const NsInbox& B, int m, int j, double T, int round) {
    const int slot = m & (B.nslot - 1);
    const int pos = atomicAdd(&B.count[slot], 1);
    if (pos < B.cap) {
        const long long at = static_cast<long long>(slot) * B.cap + pos;
        B.entry[at] = (round << kNsRoundShift) | j;
        B.time[at] = T;
    } else {
        atomicOr(B.error, 1);
    }
}

// One fan-out target of a spike at time ts emitted in pass `round` of step k's delivery
// loop: synapses take it from the event ring at their delivery step; a NetStim takes it
// from its inbox, in the next pass of step k when it is due in step k, else in the first
// pass of its step (by then it waits in the NetStim's queue).
__device__ __forceinline__ void fan_out(const EventRing& R, const NsInbox& B, const double* ttab, int k, int kmax,
                                        double half_dt, double ts, int round, int target, double delay) {
    const double T = ts + delay;
    const int m = delivery_step(ttab, k, kmax, T, half_dt);
    if (target_kind(target) == kTargetNetStim) inbox_push(B, m, target_inst(target), T, m == k ? round + 1 : 1);
    else ring_push(R, m, target);
}

// detector i (every lane of the wavefront takes part: the log slots are compacted per wave)
__device__ __forceinline__ void spike_detect(const SpikeArgs& S, int i) {
    bool fire = false;
    if (i < S.npre) {
        const double vv = S.v[S.node[i]];
        const double th = S.thr[i];
        if (vv > th && !S.flag[i]) {           // presyn.cpp:140-157
            fire = true;
            S.flag[i] = 1;
        } else if (vv <= th) {
            S.flag[i] = 0;
        }
    }
    // wave-level compaction of the spikes into the log
    const unsigned long long ballot = __ballot(fire);
    const int lane = __lane_id();
    int base = 0;
    if (ballot) {
        if (lane == __ffsll(static_cast<long long>(ballot)) - 1)
            base = atomicAdd(S.log_count, __popcll(ballot));
        base = __shfl(base, __ffsll(static_cast<long long>(ballot)) - 1);
    }
    if (!fire) return;
    const int pos = base + __popcll(ballot & ((1ull << lane) - 1ull));
    if (pos < S.log_cap) {
        S.log_t[pos] = S.t;
        S.log_gid[pos] = S.gid[i];
    }
    // detected spikes are in place before the delivery loop's first pass
    for (int e = S.fo.begin[i]; e < S.fo.begin[i + 1]; ++e)
        fan_out(S.ring, S.ib, S.ttab, S.k, S.kmax, S.half_dt, S.t, 0, S.fo.target[e], S.fo.delay[e]);
}

__global__ void __launch_bounds__(kBlock) k_spike(SpikeArgs S) { spike_detect(S, blockIdx.x * blockDim.x + threadIdx.x); }

__device__ __forceinline__ void input_task(const InputArgs& I) {
    int cur = *I.cursor;
    for (;;) {
        const int idx = cur + static_cast<int>(threadIdx.x);
        const bool take = idx < I.n && I.eff_time[idx] <= I.tcut;
        const int cnt = __syncthreads_count(take);
        if (take) {
            const int s = I.inst[idx];
            const int round = I.round ? I.round[idx] : 1;
            for (int e = I.fo.begin[s]; e < I.fo.begin[s + 1]; ++e)
                fan_out(I.ring, I.ib, I.ttab, I.k, I.kmax, I.half_dt, I.t, round, I.fo.target[e], I.fo.delay[e]);
        }
        cur += cnt;
        if (cnt < static_cast<int>(blockDim.x)) break;
    }
    if (threadIdx.x == 0) *I.cursor = cur;
}

__global__ void __launch_bounds__(kBlock) k_input(InputArgs I) { input_task(I); }

// one workgroup per cell group
__global__ void __launch_bounds__(kBlock) k_input_set(InputSet S) { input_task(S.a[blockIdx.x]); }

// The delivery loop of step k (simulate.cpp:916-939) for the NetStims that receive
// events, in one workgroup.  Pass r hands each instance the events that reach it in
// that pass (inbox entries of round r) and its self events due by t_k + dt/2 that were
// sent before pass r, and processes them in time order as NET_RECEIVE
// (netstim.cpp:247-290, one stream per instance):
//   init event:  if on, init_sequence, self event at t;
//   self event:  if on, ispike += 1, spike at t, next_invl, if still on self event at
//                t + event;
//   netcon event with int(weight) > 0 while off: init_sequence, next_invl,
//                event -= interval (1 - noise), self event at t + event;
//                int(weight) < 0: off.
// A spike fans out at once; what it brings to a NetStim in this step arrives in pass
// r + 1.  Passes repeat while any instance has something due, as the reference's loop
// repeats while anything was sent (at most kNsRounds).  Events of one instance at equal
// times go self events first, then netcon events.
__device__ __forceinline__ double ns_invl(Stream123& rng, bool& rng_live, const unsigned* rng_words,
                                          double interval, double noise) {
    if (interval <= 0.0) interval = 0.01;                  // netstim.cpp:140-155
    if (noise == 0) return interval;
    if (!rng_live) {
        rng.load(rng_words);
        rng_live = true;
    }
    return (1.0 - noise) * interval + noise * interval * rng.negexp();
}

__device__ bool ns_process(const NsArgs& A, int j, int r, long long off, double tcut) {
    constexpr int kMax = kNsQueue + kNsMini;
    double bt[kMax];
    int bk[kMax];                                          // 0 netcon event, 1 self, 2 init
    int nb = 0;
    const long long q0 = static_cast<long long>(j) * kNsQueue;
    const int qn = A.q_n[j];
    const long long born_now = static_cast<long long>(A.k) << 8;
    int keep = 0;
    for (int q = 0; q < qn; ++q) {
        const double tq = A.q_t[q0 + q];
        const long long born = A.q_born[q0 + q];
        const int kind = A.q_kind[q0 + q];
        if (tq <= tcut && born < born_now + r) {
            bt[nb] = tq;
            bk[nb] = kind == 1 ? 2 : 1;
            ++nb;
        } else {
            A.q_t[q0 + keep] = tq;
            A.q_born[q0 + keep] = born;
            A.q_kind[q0 + keep] = kind;
            ++keep;
        }
    }
    const int nm = min(atomicExch(&A.mini_n[j], 0), kNsMini);
    for (int p = 0; p < nm; ++p) {
        bt[nb] = A.ib.time[off + A.mini_e[j * kNsMini + p]];
        bk[nb] = 0;
        ++nb;
    }
    bool due = false;
    if (nb > 0) {
        for (int a = 1; a < nb; ++a) {                     // stable: self events stay ahead
            const double x = bt[a];
            const int y = bk[a];
            int b = a - 1;
            while (b >= 0 && bt[b] > x) {
                bt[b + 1] = bt[b];
                bk[b + 1] = bk[b];
                --b;
            }
            bt[b + 1] = x;
            bk[b + 1] = y;
        }
        const int inst = A.inst[j];
        const double interval = A.interval[j], number = A.number[j], noise = A.noise[j];
        double on = A.on[j], ispike = A.ispike[j], event = A.event[j];
        Stream123 rng;
        bool rng_live = false;
        const unsigned* rw = A.rng + static_cast<long long>(j) * kNsRng;
        const double t = A.t;
        auto send_self = [&](double T, int kind) {
            if (keep < kNsQueue) {
                A.q_t[q0 + keep] = T;
                A.q_born[q0 + keep] = born_now + r;
                A.q_kind[q0 + keep] = kind;
                ++keep;
            } else {
                atomicOr(A.error, 8);
            }
        };
        auto init_sequence = [&]() {
            if (number > 0.0) {
                event = 0.0;
                on = 1.0;
                ispike = 0.0;
            }
        };
        auto next_invl = [&]() {
            if (number > 0) event = ns_invl(rng, rng_live, rw, interval, noise);
            if (ispike >= number) on = 0.0;
        };
        for (int b = 0; b < nb; ++b) {
            if (bk[b] == 2) {
                if (on == 1.0) {
                    init_sequence();
                    send_self(t + 0.0, 0);
                }
            } else if (bk[b] == 1) {
                if (on == 1.0) {
                    ispike += 1.0;
                    const int pos = atomicAdd(A.log_count, 1);
                    if (pos < A.log_cap) {
                        A.log_t[pos] = t;
                        A.log_inst[pos] = inst;
                    }
                    for (int e = A.fo.begin[j]; e < A.fo.begin[j + 1]; ++e)
                        fan_out(A.ring, A.ib, A.ttab, A.k, A.kmax, A.half_dt, t, r, A.fo.target[e], A.fo.delay[e]);
                    next_invl();
                    if (on == 1.0) send_self(t + event, 0);
                }
            } else {
                const int w = static_cast<int>(A.weight[j]);
                if (w > 0 && on == 0.0) {
                    init_sequence();
                    next_invl();
                    event -= interval * (1. - noise);
                    send_self(t + event, 0);
                } else if (w < 0) {
                    on = 0.0;
                }
            }
        }
        A.on[j] = on;
        A.ispike[j] = ispike;
        A.event[j] = event;
        if (rng_live) rng.save(A.rng + static_cast<long long>(j) * kNsRng);
    }
    A.q_n[j] = keep;
    for (int q = 0; q < keep; ++q) due |= A.q_t[q0 + q] <= tcut;
    return due;
}

__global__ void __launch_bounds__(1024) k_netstim(NsArgs A) {
    __shared__ int s_more, s_later, s_cnt;
    const int slot = A.k & (A.ib.nslot - 1);
    const long long off = static_cast<long long>(slot) * A.ib.cap;
    const double tcut = A.t + A.half_dt;
    auto slot_count = [&]() {
        return min(__hip_atomic_load(&A.ib.count[slot], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), A.ib.cap);
    };
    if (threadIdx.x == 0) {
        s_more = 0;
        s_later = 0;
        s_cnt = slot_count();
    }
    __syncthreads();
    // every thread takes every decision below from the same shared values, so all of
    // them run the same passes and meet at every barrier
    for (int r = 1;; ++r) {
        const int cnt = s_cnt;
        for (int e = threadIdx.x; e < cnt; e += blockDim.x) {
            const int packed = A.ib.entry[off + e];
            const int round = packed >> kNsRoundShift;
            if (round > r) s_later = 1;
            if (round != r) continue;
            const int j = packed & ((1 << kNsRoundShift) - 1);
            const int p = atomicAdd(&A.mini_n[j], 1);
            if (p < kNsMini) A.mini_e[j * kNsMini + p] = e;
            else atomicOr(A.error, 2);
        }
        __syncthreads();
        for (int j = threadIdx.x; j < A.n; j += blockDim.x)
            if (ns_process(A, j, r, off, tcut)) s_more = 1;
        __syncthreads();
        if (threadIdx.x == 0) {
            const int cnt2 = slot_count();
            s_more = (s_more || s_later || cnt2 > cnt) ? 1 : 0;
            s_later = 0;
            s_cnt = cnt2;
        }
        __syncthreads();
        const bool more = s_more != 0;
        __syncthreads();                                   // every thread has read s_more
        if (!more) break;
        if (r == kNsRounds) {
            if (threadIdx.x == 0) atomicOr(A.error, 4);
            break;
        }
        if (threadIdx.x == 0) s_more = 0;
        __syncthreads();
    }
    // the step's entries are consumed (a second loop for the same step, finitialize's then
    // the first step's, sees only what arrives in between)
    if (threadIdx.x == 0) A.ib.count[slot] = 0;
}

// ---------------------------------------------------------------------------
// VecPlay continuous playback (vecplay.cu:19-111)
// ---------------------------------------------------------------------------
__device__ __forceinline__ void vecplay_item(VecPlayDev* items, int n, double t, int do_play, int i) {
    if (i >= n) return;
    VecPlayDev it = items[i];
    const double* tv = it.tvec;
    const double* yv = it.yvec;
    if (do_play) {
        for (;;) {
            if (it.done || it.next_time > t) break;
            it.last_index = it.next_idx;
            if (it.next_idx < it.len - 1) { it.next_idx++; it.next_time = tv[it.next_idx]; }
            else it.done = 1;
        }
    }
    double val;
    if (t >= tv[it.next_idx]) {
        it.last_index = it.next_idx;
        if (it.last_index == 0) { val = yv[0]; goto store; }
    } else if (t <= tv[0]) {
        it.last_index = 0;
        val = yv[0];
        goto store;
    } else {
        while (t < tv[it.last_index]) --it.last_index;
        while (t >= tv[it.last_index]) ++it.last_index;
    }
    {
        const double x0 = yv[it.last_index - 1], x1 = yv[it.last_index];
        const double t0 = tv[it.last_index - 1], t1 = tv[it.last_index];
        if (t0 == t1) val = (x0 + x1) / 2.;
        else val = x0 + (x1 - x0) * ((t - t0) / (t1 - t0));
    }
store:
    *it.target = val;
    items[i] = it;
}

// NET_RECEIVE of the events of step k's ring slot (expsyn.cpp net_receive,
// exp2syn_temp.cuh:62-67): ExpSyn g += w, Exp2Syn A, B += w factor, in any order
// (fp64 atomics), as on the reference's GPU path.  The workgroups stride over the
// slot, so a burst spreads over the chip; each counts itself done after its loop (which
// used the count it read), and the last one empties the slot, so a second launch for
// the same step (finitialize's, then the first step's) delivers only what was pushed
// in between.
// Block b of the nb blocks delivering ring R's slot of step D.k.
__device__ __forceinline__ void deliver_task(const DeliverArgs& D, const EventRing& R, int b, int nb) {
    const int slot = D.k & (R.nslot - 1);
    int cnt = R.count[slot];
    if (cnt > R.cap) cnt = R.cap;
    const long long off = static_cast<long long>(slot) * R.cap;
    for (int e = b * blockDim.x + threadIdx.x; e < cnt; e += nb * blockDim.x) {
        const int packed = R.entry[off + e];
        const int type = target_kind(packed);
        const int inst = packed & 0x3fffffff;
        if (type == 0) {
            atomicAdd(&D.es.col(ES_G)[inst], D.es_weight[inst]);
        } else if (type == kTargetPlugin) {   // counted; the plugin's NET_RECEIVE kernel follows
            atomicAdd(&D.plugin_recv[(inst >> kPostsynSlotShift) & (kMaxPostsyn - 1)]
                                    [inst & ((1 << kPostsynSlotShift) - 1)], 1);
        } else if (type == 1) {            // (NetStim targets go to their own inbox)
            const double wf = D.e2_weight[inst] * D.e2.col(E2_FACTOR)[inst];
            atomicAdd(&D.e2.col(E2_A)[inst], wf);
            atomicAdd(&D.e2.col(E2_B)[inst], wf);
        }
        if (D.log) {          // the adjoint's record of the step's deliveries (packed as in the ring)
            const int pos = atomicAdd(D.log_count, 1);
            if (pos < D.log_cap) D.log[pos] = packed;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0 && (nb == 1 || atomicAdd(R.done, 1u) == nb - 1u)) {
        R.count[slot] = 0;
        if (nb > 1) *R.done = 0u;
    }
}

__global__ void __launch_bounds__(1024) k_deliver(DeliverArgs D) {
    if (static_cast<int>(blockIdx.x) >= D.ndeliver) {      // the VecPlay task's blocks
        vecplay_item(D.vp, D.nvp, D.t_vp, 1, (blockIdx.x - D.ndeliver) * blockDim.x + threadIdx.x);
        return;
    }
    deliver_task(D, D.ring, blockIdx.x, D.ndeliver);
}

// D.ndeliver blocks per ring of S, then the VecPlay task's blocks
__global__ void __launch_bounds__(1024) k_deliver_set(DeliverArgs D, RingSet S) {
    const int g = static_cast<int>(blockIdx.x) / D.ndeliver;
    if (g >= S.n) {
        vecplay_item(D.vp, D.nvp, D.t_vp, 1, (blockIdx.x - S.n * D.ndeliver) * blockDim.x + threadIdx.x);
        return;
    }
    deliver_task(D, S.r[g], blockIdx.x - g * D.ndeliver, D.ndeliver);
}

__global__ void k_vecplay(VecPlayDev* items, int n, double t, int do_play) {
    vecplay_item(items, n, t, do_play, blockIdx.x * blockDim.x + threadIdx.x);
}

// The work after a step's solve in one launch, each task on its own run of blocks:
// gap transfers (the model's, then those added at run time), threshold detection of the
// next step, VecPlay at the step's end time, and the synapses' state update.  The tasks
// touch disjoint data (the host keeps VecPlay out of it unless every target is an IClamp
// variable), so running them side by side gives the bits of the separate launches.
__global__ void __launch_bounds__(kBlock) k_after_solve(AfterSolve P) {
    const int b = blockIdx.x;
    const int tid = threadIdx.x;
    if (b < P.b_ptr) {
        const int i = b * kBlock + tid;
        if (i < P.ngap) P.vgap[P.gap_inst[i]] = P.v[P.gap_src[i]];
    } else if (b < P.b_spike) {
        const int i = (b - P.b_ptr) * kBlock + tid;
        if (i < P.nptr) *P.pdst[i] = *P.psrc[i];
    } else if (b < P.b_vp) {
        spike_detect(P.S, (b - P.b_spike) * kBlock + tid);
    } else if (b < P.b_es) {
        vecplay_item(P.vp, P.nvp, P.t, 0, (b - P.b_vp) * kBlock + tid);
    } else if (b < P.b_e2) {
        const int j = P.es0 + (b - P.b_es) * kBlock + tid;
        if (j < P.es1) {
            const double g = P.es_g[j];
            if (P.es_tape) P.es_tape[j] = g;
            P.es_g[j] = expsyn_decay(g, P.es_tau[j], P.dt);
        }
    } else if (b < P.b_tape) {
        const int j = P.e20 + (b - P.b_e2) * kBlock + tid;
        if (j < P.e21) {
            const double aa = P.e2_a[j], bb = P.e2_b[j];
            if (P.e2_tape_a) {
                P.e2_tape_a[j] = aa;
                P.e2_tape_b[j] = bb;
            }
            P.e2_a[j] = exp2syn_decay(aa, P.e2_tau1[j], P.dt);
            P.e2_b[j] = exp2syn_decay(bb, P.e2_tau2[j], P.dt);
        }
    } else {
        const long long i = static_cast<long long>(b - P.b_tape) * kBlock + tid;
        const long long stride = static_cast<long long>(gridDim.x - P.b_tape) * kBlock;
        for (int sg = 0; sg < P.tape.nseg; ++sg)
            for (long long j = i; j < P.tape.n[sg]; j += stride) P.tape.dst[sg][j] = P.tape.src[sg][j];
    }
}

__global__ void k_vecplay_reset(VecPlayDev* items, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    VecPlayDev it = items[i];
    it.last_index = 0;
    it.next_idx = 0;
    it.done = 0;
    if (it.len > 0) it.next_time = it.tvec[0];
    else { it.next_time = 0.0; it.done = 1; }
    items[i] = it;
}

__global__ void k_record(double* const* ptrs, int n, double* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = *ptrs[i];
}

__global__ void k_gap(const double* v, const int* src_node, double* vgap, const int* inst, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) vgap[inst[i]] = v[src_node[i]];
}

// Gap junctions added at run time (simulate.cpp:953-966 gap_transfer): *dst[i] = *src[i].
__global__ void k_copy_ptrs(double* const* src, double* const* dst, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) *dst[i] = *src[i];
}

__global__ void k_status(StatusArgs a) {
    int ov = 0;
    for (int g = 0; g < a.ngroups; ++g) ov |= *a.ring_overflow[g];
    a.out[0] = ov;
    a.out[1] = a.ns_error ? *a.ns_error : 0;
    a.out[2] = *a.spk_count;
}

__global__ void __launch_bounds__(kBlock) k_tape(TapeCopy T) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (int s = 0; s < T.nseg; ++s)
        for (long long j = i; j < T.n[s]; j += stride) T.dst[s][j] = T.src[s][j];
}

__global__ void k_clear_ints(int* p, long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

inline dim3 grid_for(long long n, int block = kBlock) {
    return dim3(static_cast<unsigned>((n + block - 1) / block));
}

}  // namespace

// ---------------------------------------------------------------------------
// launch wrappers
// ---------------------------------------------------------------------------
// Mechanism sets with a compile-time steady-step instance of the node kernel: every
// density mechanism of the pyramidal-cell model (pas, hh, Ca_HVA, Ih, CaDynamics_E2 and
// the three ions on every node) and pas alone (hh on part of the nodes runs
// instance-parallel), each with the synapse folds a model may have.
constexpr unsigned kMaskPyr = (1u << M_PAS) | (1u << M_NA_ION) | (1u << M_K_ION) | (1u << M_HH) |
                              (1u << M_CA_ION) | (1u << M_CADYN) | (1u << M_CAHVA) | (1u << M_HDLA);
constexpr unsigned kMaskPas = 1u << M_PAS;
constexpr unsigned kFoldES = 1u << M_EXPSYN, kFoldE2 = 1u << M_EXP2SYN;

template <unsigned MASK>
bool launch_steady(const StepArgs& a, dim3 grid, hipStream_t s, hipEvent_t e0, hipEvent_t e1) {
    for (unsigned fold : {0u, kFoldES, kFoldE2, kFoldES | kFoldE2}) {
        if (fold == 0u && is_steady<MASK, 0u>(a))
            hipExtLaunchKernelGGL((k_dense_steady<MASK, 0u>), grid, dim3(kBlock), 0, s, e0, e1, 0, a);
        else if (fold == kFoldES && is_steady<MASK, kFoldES>(a))
            hipExtLaunchKernelGGL((k_dense_steady<MASK, kFoldES>), grid, dim3(kBlock), 0, s, e0, e1, 0, a);
        else if (fold == kFoldE2 && is_steady<MASK, kFoldE2>(a))
            hipExtLaunchKernelGGL((k_dense_steady<MASK, kFoldE2>), grid, dim3(kBlock), 0, s, e0, e1, 0, a);
        else if (fold == (kFoldES | kFoldE2) && is_steady<MASK, kFoldES | kFoldE2>(a))
            hipExtLaunchKernelGGL((k_dense_steady<MASK, kFoldES | kFoldE2>), grid, dim3(kBlock), 0, s, e0, e1, 0, a);
        else
            continue;
        return true;
    }
    return false;
}

int launch_dense(const StepArgs& a, hipStream_t s, bool steady, hipEvent_t e0, hipEvent_t e1) {
    if (a.N - a.node0 <= 0) return 0;
    const dim3 grid = grid_for(a.N - a.node0);
    if (steady && (launch_steady<kMaskPyr>(a, grid, s, e0, e1) || launch_steady<kMaskPas>(a, grid, s, e0, e1)))
        return 2;
    hipExtLaunchKernelGGL(k_dense, grid, dim3(kBlock), 0, s, e0, e1, 0, a);
    return 1;
}

void launch_sparse(int mech, const StepArgs& a, hipStream_t s) {
    const int n = std::min(a.m[mech].n, a.pt1) - a.pt0;
    if (n <= 0) return;
    switch (mech) {
        case M_PAS: hipLaunchKernelGGL(k_sparse<M_PAS>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_NA_ION: hipLaunchKernelGGL(k_sparse<M_NA_ION>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_K_ION: hipLaunchKernelGGL(k_sparse<M_K_ION>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_HH: hipLaunchKernelGGL(k_sparse<M_HH>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_CA_ION: hipLaunchKernelGGL(k_sparse<M_CA_ION>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_CADYN: hipLaunchKernelGGL(k_sparse<M_CADYN>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_CAHVA: hipLaunchKernelGGL(k_sparse<M_CAHVA>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_HDLA: hipLaunchKernelGGL(k_sparse<M_HDLA>, grid_for(n), dim3(kBlock), 0, s, a); break;
        default: break;
    }
}

void launch_point_current(int mech, const StepArgs& a, hipStream_t s) {
    const int n = a.m[mech].ngrp;
    if (n <= 0) return;
    switch (mech) {
        case M_ICLAMP: hipLaunchKernelGGL(k_point<M_ICLAMP>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_EXPSYN: hipLaunchKernelGGL(k_point<M_EXPSYN>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_EXP2SYN: hipLaunchKernelGGL(k_point<M_EXP2SYN>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_HALFGAP: hipLaunchKernelGGL(k_point<M_HALFGAP>, grid_for(n), dim3(kBlock), 0, s, a); break;
        default: break;
    }
}

void launch_after_solve(AfterSolve p, hipStream_t s) {
    auto nb = [](long long n) { return static_cast<int>(n > 0 ? (n + kBlock - 1) / kBlock : 0); };
    p.b_ptr = nb(p.ngap);
    p.b_spike = p.b_ptr + nb(p.nptr);
    p.b_vp = p.b_spike + nb(p.S.npre);
    p.b_es = p.b_vp + nb(p.nvp);
    p.b_e2 = p.b_es + nb(p.es1 - p.es0);
    p.b_tape = p.b_e2 + nb(p.e21 - p.e20);
    long long most = 0;
    for (int k = 0; k < p.tape.nseg; ++k) most = std::max(most, p.tape.n[k]);
    const int end = p.b_tape + static_cast<int>(std::min<long long>(nb(most), 4096));
    if (end > 0) hipLaunchKernelGGL(k_after_solve, dim3(end), dim3(kBlock), 0, s, p);
}

void launch_point_electrodes(const StepArgs& a, const PointUnion& u, hipStream_t s) {
    if (u.n > 0) hipLaunchKernelGGL(k_point_electrodes, grid_for(u.n), dim3(kBlock), 0, s, a, u);
}

void launch_point_state(int mech, const StepArgs& a, hipStream_t s) {
    const int n = std::min(a.m[mech].n, a.pt1) - a.pt0;
    if (n <= 0) return;
    if (mech == M_EXPSYN) hipLaunchKernelGGL(k_point_state<M_EXPSYN>, grid_for(n), dim3(kBlock), 0, s, a);
    if (mech == M_EXP2SYN) hipLaunchKernelGGL(k_point_state<M_EXP2SYN>, grid_for(n), dim3(kBlock), 0, s, a);
}

void launch_init(int mech, const StepArgs& a, hipStream_t s) {
    const int n = a.m[mech].n;
    if (n <= 0) return;
    switch (mech) {
        case M_NA_ION: hipLaunchKernelGGL(k_init<M_NA_ION>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_K_ION: hipLaunchKernelGGL(k_init<M_K_ION>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_CA_ION: hipLaunchKernelGGL(k_init<M_CA_ION>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_HH: hipLaunchKernelGGL(k_init<M_HH>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_CAHVA: hipLaunchKernelGGL(k_init<M_CAHVA>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_HDLA: hipLaunchKernelGGL(k_init<M_HDLA>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_ICLAMP: hipLaunchKernelGGL(k_init<M_ICLAMP>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_HALFGAP: hipLaunchKernelGGL(k_init<M_HALFGAP>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_EXPSYN: hipLaunchKernelGGL(k_init<M_EXPSYN>, grid_for(n), dim3(kBlock), 0, s, a); break;
        case M_EXP2SYN: hipLaunchKernelGGL(k_init<M_EXP2SYN>, grid_for(n), dim3(kBlock), 0, s, a); break;
        default: break;
    }
}

void launch_set_v(double* v, int n, double val, hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(k_set_v, grid_for(n), dim3(kBlock), 0, s, v, n, val);
}

void launch_solve(const SolveArgs& a, int max_chunks, hipStream_t s) {
    if (a.nunit <= 0) return;
    SolveArgs b = a;
    b.waves = std::min(std::max(a.waves, 1), kSolveMaxWaves);
    if (b.res_nodes > 0) {
        const size_t lds = res_lds_bytes(b.res_nodes, max_chunks, b.res_rounds) * b.waves;
        const dim3 grid((a.nunit + b.waves - 1) / b.waves), block(kWave * b.waves);
        const uint2* desc = reinterpret_cast<const uint2*>(b.desc);
        if (a.store_dx && a.yform)
            hipLaunchKernelGGL((k_solve_res<1, 1>), grid, block, lds, s, b, b.rounds, desc, max_chunks);
        else if (a.store_dx)
            hipLaunchKernelGGL((k_solve_res<1, 0>), grid, block, lds, s, b, b.rounds, desc, max_chunks);
        else if (a.yform)
            hipLaunchKernelGGL((k_solve_res<0, 1>), grid, block, lds, s, b, b.rounds, desc, max_chunks);
        else
            hipLaunchKernelGGL((k_solve_res<0, 0>), grid, block, lds, s, b, b.rounds, desc, max_chunks);
        return;
    }
    const size_t lds = solve_lds_bytes(max_chunks) * b.waves;
    const dim3 grid((a.nunit + b.waves - 1) / b.waves), block(kWave * b.waves);
    if (a.store_dx)
        hipLaunchKernelGGL(k_solve<1>, grid, block, lds, s, b, b.rounds, reinterpret_cast<const uint2*>(b.desc),
                           max_chunks);
    else
        hipLaunchKernelGGL(k_solve<0>, grid, block, lds, s, b, b.rounds, reinterpret_cast<const uint2*>(b.desc),
                           max_chunks);
}

// Streaming ceiling of the node kernel's access mix: each thread reads R fp64 columns
// and writes W at its index, with the node kernel's non-temporal hints.  A measurement
// of what this GPU moves for that mix, not part of any step.
template <int R, int W>
__global__ void __launch_bounds__(kBlock) k_stream(const double* __restrict__ in, double* __restrict__ out,
                                                   long long n) {
    const long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n) return;
    double x[R];
#pragma unroll
    for (int r = 0; r < R; ++r) x[r] = __builtin_nontemporal_load(in + r * n + i);
    double acc = 0.0;
#pragma unroll
    for (int r = 0; r < R; ++r) acc += x[r];
#pragma unroll
    for (int w = 0; w < W; ++w) __builtin_nontemporal_store(acc + w, out + w * n + i);
}

bool launch_stream(int nread, int nwrite, const double* in, double* out, long long n, hipStream_t s) {
    const dim3 g(static_cast<unsigned>((n + kBlock - 1) / kBlock));
    if (nread == 1 && nwrite == 1) hipLaunchKernelGGL((k_stream<1, 1>), g, dim3(kBlock), 0, s, in, out, n);
    else if (nread == 11 && nwrite == 9) hipLaunchKernelGGL((k_stream<11, 9>), g, dim3(kBlock), 0, s, in, out, n);
    else if (nread == 26 && nwrite == 9) hipLaunchKernelGGL((k_stream<26, 9>), g, dim3(kBlock), 0, s, in, out, n);
    else return false;
    return true;
}

void launch_spike(const SpikeArgs& a, hipStream_t s) {
    if (a.npre > 0) hipLaunchKernelGGL(k_spike, grid_for(a.npre), dim3(kBlock), 0, s, a);
}

void launch_input(const InputArgs& a, hipStream_t s) {
    if (a.n > 0) hipLaunchKernelGGL(k_input, dim3(1), dim3(kBlock), 0, s, a);
}

void launch_netstim(const NsArgs& a, hipStream_t s) {
    if (a.n > 0) hipLaunchKernelGGL(k_netstim, dim3(1), dim3(1024), 0, s, a);
}

void launch_deliver(const DeliverArgs& a, int nblk, hipStream_t s) {
    DeliverArgs d = a;
    d.ndeliver = std::max(1, nblk);
    const int nvp_blk = d.nvp > 0 ? (d.nvp + 1023) / 1024 : 0;
    hipLaunchKernelGGL(k_deliver, dim3(d.ndeliver + nvp_blk), dim3(1024), 0, s, d);
}

void launch_input_set(const InputSet& a, hipStream_t s) {
    if (a.n > 0) hipLaunchKernelGGL(k_input_set, dim3(a.n), dim3(kBlock), 0, s, a);
}

void launch_deliver_set(const DeliverArgs& a, const RingSet& rings, int nblk, hipStream_t s) {
    if (rings.n <= 0) return;
    DeliverArgs d = a;
    d.ndeliver = std::max(1, nblk);
    const int nvp_blk = d.nvp > 0 ? (d.nvp + 1023) / 1024 : 0;
    hipLaunchKernelGGL(k_deliver_set, dim3(d.ndeliver * rings.n + nvp_blk), dim3(1024), 0, s, d, rings);
}

void launch_vecplay(VecPlayDev* items, int n, double t, int do_play, hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(k_vecplay, grid_for(n, 64), dim3(64), 0, s, items, n, t, do_play);
}

void launch_vecplay_reset(VecPlayDev* items, int n, hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(k_vecplay_reset, grid_for(n, 64), dim3(64), 0, s, items, n);
}

void launch_record(double* const* ptrs, int n, double* out, hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(k_record, grid_for(n), dim3(kBlock), 0, s, ptrs, n, out);
}

void launch_gap(const double* v, const int* src_node, double* vgap_col, const int* halfgap_inst, int n,
                hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(k_gap, grid_for(n), dim3(kBlock), 0, s, v, src_node, vgap_col, halfgap_inst, n);
}

void launch_copy_ptrs(double* const* src, double* const* dst, int n, hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(k_copy_ptrs, grid_for(n), dim3(kBlock), 0, s, src, dst, n);
}

void launch_clear_ints(int* p, long long n, hipStream_t s) {
    if (n > 0) hipLaunchKernelGGL(k_clear_ints, grid_for(n), dim3(kBlock), 0, s, p, n);
}

void launch_status(const StatusArgs& a, hipStream_t s) { hipLaunchKernelGGL(k_status, dim3(1), dim3(1), 0, s, a); }

void launch_tape(const TapeCopy& t, hipStream_t s) {
    long long most = 0;
    for (int k = 0; k < t.nseg; ++k) most = std::max(most, t.n[k]);
    if (most <= 0) return;
    const long long blocks = std::min<long long>((most + kBlock - 1) / kBlock, 4096);
    hipLaunchKernelGGL(k_tape, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0, s, t);
}

}  // namespace hx
