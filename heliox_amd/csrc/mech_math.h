// Device-side mechanism arithmetic.
//
// The reference forms below keep the algebraic form of the reference mechanism
// (the reference is compiled with -ffp-contract=off on the host; this library
// uses the same flag); the forward step uses the rearranged forms further down,
// which differ from them by a few ulps:
//   hh ............ src/mech/user-mech/hh_templated.cu:76-164
//   pas ........... src/mech/user-mech/pas_templated.cu:27-31
//   IClamp ........ src/mech/user-mech/iclamp_templated.cu:29-40
//   Ca_HVA ........ src/mech/user-mech/CA_HVA.cu:97-178
//   hd_la ......... src/mech/user-mech/hd_la.cu:80-128
//   CaDynamics_E2 . src/mech/user-mech/CaDynamics_E2.cu:101-139
//   HalfGap ....... src/mech/user-mech/HalfGap.cu:61-68
//   ExpSyn ........ src/spike/postsyn_mech/expsyn.cu:9-70 / expsyn.cpp
//   Exp2Syn ....... src/spike/user_postsyn_mech/exp2syn_temp.cuh:29-67
//   ions .......... src/mech/eion.cuh:39-57,155-197
#pragma once
#include <hip/hip_runtime.h>
#include "hx_internal.h"
#include "fastmath.h"

namespace hx {


__device__ __forceinline__ double nernst(double ci, double co, double z, double ktf) {
    if (z == 0) return 0.;
    if (ci <= 0.) return 1e6;
    else if (co <= 0.) return -1e6;
    else return ktf / z * log(co / ci);
}

// The same with the forward step's logarithm (fastmath.h log_pos, within a few ulps of
// log); the form above stays in use at finitialize and in the adjoint.
__device__ __forceinline__ double nernst_r(double ci, double co, double z, double ktf) {
    if (z == 0) return 0.;
    if (ci <= 0.) return 1e6;
    else if (co <= 0.) return -1e6;
    const double q = co / ci;
    const bool normal = q >= 2.2250738585072014e-308 && q <= 1.7976931348623157e308;
    return ktf / z * (normal ? log_pos(q) : log(q));
}

// ---------------- hh ----------------
// The rate functions are templates so that the adjoint can evaluate them on
// dual numbers (value + derivative) and get d/dv of exactly these formulas.
struct Dual {
    double v, d;
};
__host__ __device__ __forceinline__ Dual operator+(Dual a, Dual b) { return {a.v + b.v, a.d + b.d}; }
__host__ __device__ __forceinline__ Dual operator-(Dual a, Dual b) { return {a.v - b.v, a.d - b.d}; }
__host__ __device__ __forceinline__ Dual operator-(Dual a) { return {-a.v, -a.d}; }
__host__ __device__ __forceinline__ Dual operator*(Dual a, Dual b) { return {a.v * b.v, a.d * b.v + a.v * b.d}; }
__host__ __device__ __forceinline__ Dual operator/(Dual a, Dual b) {
    return {a.v / b.v, (a.d * b.v - a.v * b.d) / (b.v * b.v)};
}
__host__ __device__ __forceinline__ Dual operator+(Dual a, double b) { return {a.v + b, a.d}; }
__host__ __device__ __forceinline__ Dual operator+(double a, Dual b) { return {a + b.v, b.d}; }
__host__ __device__ __forceinline__ Dual operator-(Dual a, double b) { return {a.v - b, a.d}; }
__host__ __device__ __forceinline__ Dual operator-(double a, Dual b) { return {a - b.v, -b.d}; }
__host__ __device__ __forceinline__ Dual operator*(Dual a, double b) { return {a.v * b, a.d * b}; }
__host__ __device__ __forceinline__ Dual operator*(double a, Dual b) { return {a * b.v, a * b.d}; }
__host__ __device__ __forceinline__ Dual operator/(Dual a, double b) { return {a.v / b, a.d / b}; }
__host__ __device__ __forceinline__ Dual operator/(double a, Dual b) { return {a / b.v, -a * b.d / (b.v * b.v)}; }
__device__ __forceinline__ Dual exp(Dual a) {
    const double e = ::exp(a.v);
    return {e, e * a.d};
}
// keeps the library exp visible next to the Dual overload inside this namespace
__device__ __forceinline__ double exp(double a) { return ::exp(a); }
__host__ __device__ __forceinline__ double value_of(double a) { return a; }
__host__ __device__ __forceinline__ double value_of(Dual a) { return a.v; }

template <class T>
__device__ __forceinline__ T hh_vtrap(T x, double y) {
    if (fabs(value_of(x) / y) < 1e-6) return y * (1 - x / y / 2);
    else return x / (exp(x / y) - 1);
}

template <class T>
__device__ __forceinline__ void hh_rates(T volt, double q10, T& minf, T& mtau, T& hinf, T& htau, T& ninf,
                                         T& ntau) {
    T alpha, beta, sum;
    alpha = 0.1 * hh_vtrap(-(volt + 40), 10);
    beta = 4 * exp(-(volt + 65) / 18);
    sum = alpha + beta;
    mtau = 1.0 / (q10 * sum);
    minf = alpha / sum;
    alpha = 0.07 * exp(-(volt + 65) / 20);
    beta = 1.0 / (exp(-(volt + 35) / 10) + 1);
    sum = alpha + beta;
    htau = 1.0 / (q10 * sum);
    hinf = alpha / sum;
    alpha = 0.01 * hh_vtrap(-(volt + 55), 10);
    beta = 0.125 * exp(-(volt + 65) / 80);
    sum = alpha + beta;
    ntau = 1.0 / (q10 * sum);
    ninf = alpha / sum;
}

template <class T>
__device__ __forceinline__ T hh_cnexp(double x, T xinf, T xtau, double dt) {
    return x + (1.0 - exp(dt * (-1.0 / xtau))) * ((xinf / xtau) / (1.0 / xtau) - x);
}

// total current and the two ion currents at `volt`
__device__ __forceinline__ double hh_current(double volt, double gnabar, double gkbar, double gl, double el,
                                             double m, double h, double n, double ena, double ek,
                                             double& gna, double& ina, double& gk, double& ik, double& il) {
    gna = gnabar * m * m * m * h;
    ina = gna * (volt - ena);
    gk = gkbar * n * n * n * n;
    ik = gk * (volt - ek);
    il = gl * (volt - el);
    return ina + ik + il;
}

// ---------------- Ca_HVA ----------------
__device__ __forceinline__ double cahva_vtrap(double _lx, double _ly) {
    double _lvtrap;
    if (fabs(_lx / _ly) < 1e-6) _lvtrap = _ly * (1.0 - _lx / _ly / 2.0);
    else _lvtrap = _lx / (exp(_lx / _ly) - 1.0);
    return _lvtrap;
}

__device__ __forceinline__ void cahva_rates(double volt, double& mInf, double& mTau, double& mAlpha, double& mBeta,
                                            double& hInf, double& hTau, double& hAlpha, double& hBeta) {
    mAlpha = 0.055 * cahva_vtrap(-27.0 - volt, 3.8);
    mBeta = 0.94 * exp((-75.0 - volt) / 17.0);
    mInf = mAlpha / (mAlpha + mBeta);
    mTau = 1.0 / (mAlpha + mBeta);
    hAlpha = 0.000457 * exp((-13.0 - volt) / 50.0);
    hBeta = 0.0065 / (exp((-volt - 15.0) / 28.0) + 1.0);
    hInf = hAlpha / (hAlpha + hBeta);
    hTau = 1.0 / (hAlpha + hBeta);
}

// ---------------- hd_la (Ih) ----------------
__device__ __forceinline__ void hdla_rate(double v, double vhalfl, double tau, const MechConsts& c,
                                          double& linf, double& taul) {
    double a = exp(0.0378 * c.hd_zetat * (v - c.hd_vhalft));
    linf = 1.0 / (1.0 + exp(-(v - vhalfl) / c.hd_kl));
    double bett = exp(0.0378 * c.hd_zetat * c.hd_gmt * (v - c.hd_vhalft));
    taul = tau * bett / (c.hd_qtl * c.hd_qt * c.hd_a0t * (1.0 + a));
}

// Reference forms as templates, for the adjoint: evaluated on dual numbers they
// give d/dv of exactly these formulas (CA_HVA.cu:97-113, hd_la.cu:80-101, the
// cnexp updates CA_HVA.cu:170-177 and hd_la.cu:123-127).
template <class T>
__device__ __forceinline__ T cahva_vtrap_t(T x, double y) {
    if (fabs(value_of(x) / y) < 1e-6) return y * (1.0 - x / y / 2.0);
    else return x / (exp(x / y) - 1.0);
}

template <class T>
__device__ __forceinline__ void cahva_rates_t(T volt, T& mInf, T& mTau, T& hInf, T& hTau) {
    const T mAlpha = 0.055 * cahva_vtrap_t(-27.0 - volt, 3.8);
    const T mBeta = 0.94 * exp((-75.0 - volt) / 17.0);
    mInf = mAlpha / (mAlpha + mBeta);
    mTau = 1.0 / (mAlpha + mBeta);
    const T hAlpha = 0.000457 * exp((-13.0 - volt) / 50.0);
    const T hBeta = 0.0065 / (exp((-volt - 15.0) / 28.0) + 1.0);
    hInf = hAlpha / (hAlpha + hBeta);
    hTau = 1.0 / (hAlpha + hBeta);
}

template <class T>
__device__ __forceinline__ void hdla_rate_t(T v, double vhalfl, double tau, const MechConsts& c, T& linf, T& taul) {
    const T a = exp(0.0378 * c.hd_zetat * (v - c.hd_vhalft));
    linf = 1.0 / (1.0 + exp(-(v - vhalfl) / c.hd_kl));
    const T bett = exp(0.0378 * c.hd_zetat * c.hd_gmt * (v - c.hd_vhalft));
    taul = tau * bett / (c.hd_qtl * c.hd_qt * c.hd_a0t * (1.0 + a));
}

// x + (1 - exp(-dt / tau)) (inf - x)
template <class T>
__device__ __forceinline__ T cnexp_t(double x, T inf, T tau, double dt) {
    return x + (1.0 - exp(-dt / tau)) * (inf - x);
}

// ---------------- CaDynamics_E2 ----------------
__device__ __forceinline__ double cadyn_step(double cai, double ica, double gamma, double decay, double depth,
                                             double minCai, double dt) {
    double drive_ica = -(10000.0) * (ica * gamma) / (2.0 * kFaradayCaDyn * depth);
    double exp_factor = exp(dt * (-1.0 / decay));
    double steady_term = -(drive_ica - (-minCai) / decay) / (-1.0 / decay);
    return cai + (1.0 - exp_factor) * (steady_term - cai);
}

// ---------------- rearranged forms for the forward step ----------------
// The same mathematics as the reference forms above, with the divisions that the
// reference's expressions spell out but the algebra does not need taken out (an
// fp64 division costs about ten instructions, a multiplication one; the node
// kernel is close to its instruction-issue limit).  The cnexp update with
// tau = 1/(k (a+b)) and inf = a/(a+b),
//     x + (1 - exp(dt (-1/tau))) ((inf/tau)/(1/tau) - x),
// is x + (1 - exp(-dt k (a+b))) (a/(a+b) - x); divisions by constants become
// multiplications by their reciprocals.  Results differ from the reference
// forms by a few ulps.  The reference forms stay in use where their
// intermediate values are outputs (assigned variables) and in the adjoint.
// a / b from the hardware reciprocal, two Newton steps and a remainder correction: within
// one ulp of the rounded quotient, for the normal, finite operands the rates produce.  An
// infinite or subnormal divisor (a rate's exp overflowing at an extreme voltage) makes the
// Newton steps give NaN; such lanes take the IEEE division instead, so a / inf is 0 as in
// the reference forms.
__device__ __forceinline__ double div_r(double a, double b) {
    double r = __builtin_amdgcn_rcp(b);
    double e = fma(-b, r, 1.0);
    r = fma(r, e, r);
    e = fma(-b, r, 1.0);
    r = fma(r, e, r);
    const double q = a * r;
    const double res = fma(fma(-b, q, a), r, q);
    if (__builtin_expect(!__builtin_isfinite(res), 0)) return a / b;
    return res;
}

__device__ __forceinline__ double vtrap_r(double x, double y, double inv_y) {
    const double r = x * inv_y;                      // x / y
    if (fabs(r) < 1e-6) return y * (1 - r * 0.5);
    return div_r(x, exp(r) - 1);
}

__device__ __forceinline__ double gate_step(double x, double a, double b, double k, double dt) {
    const double sum = a + b;
    return x + (1.0 - exp(-dt * (k * sum))) * (div_r(a, sum) - x);
}

// hh: the three gates of one compartment
// The rates hold six exponentials of v; three of them are the others times
// constants: with E = exp(-(v + 40) / 10) and F = exp(-(v + 65) / 80),
//     exp(-(v + 35) / 10) = E e^(1/2),  exp(-(v + 55) / 10) = E e^(-3/2),
//     exp(-(v + 65) / 20) = F^4,
// which leaves three exp calls (a few ulps from the six-call form).
__device__ __forceinline__ double vtrap_e(double x, double y, double inv_y, double ex) {   // ex = exp(x / y)
    const double r = x * inv_y;
    if (fabs(r) < 1e-6) return y * (1 - r * 0.5);
    return div_r(x, ex - 1);
}

__device__ __forceinline__ void hh_gates_r(double v, double q10, double dt, double& m, double& h, double& n) {
    constexpr double kExpHalf = 1.6487212707001282;        // e^(1/2)
    constexpr double kExpMinus3Half = 0.22313016014842982; // e^(-3/2)
    const double E = exp(-(v + 40) * 0.1);
    const double F = exp(-(v + 65) * 0.0125);
    const double F2 = F * F;
    const double am = 0.1 * vtrap_e(-(v + 40), 10.0, 0.1, E);
    const double bm = 4 * exp(-(v + 65) * (1.0 / 18));
    const double ah = 0.07 * (F2 * F2);
    const double bh = div_r(1.0, E * kExpHalf + 1);
    const double an = 0.01 * vtrap_e(-(v + 55), 10.0, 0.1, E * kExpMinus3Half);
    const double bn = 0.125 * F;
    m = gate_step(m, am, bm, q10, dt);
    h = gate_step(h, ah, bh, q10, dt);
    n = gate_step(n, an, bn, q10, dt);
}

// Ca_HVA: m, h
__device__ __forceinline__ void cahva_gates_r(double v, double dt, double& m, double& h) {
    const double ma = 0.055 * vtrap_r(-27.0 - v, 3.8, 1.0 / 3.8);
    const double mb = 0.94 * exp((-75.0 - v) * (1.0 / 17.0));
    const double ha = 0.000457 * exp((-13.0 - v) * 0.02);
    const double hb = div_r(0.0065, exp((-v - 15.0) * (1.0 / 28.0)) + 1.0);
    m = gate_step(m, ma, mb, 1.0, dt);
    h = gate_step(h, ha, hb, 1.0, dt);
}

// hd_la: l + (1 - exp(-dt / taul)) (linf - l) with -dt / taul folded into one division
// With gmt = 0.4 (the model's value), bett = G^2 and a = G^5 for G = exp(0.0378 zetat
// (v - vhalft) / 5): one exponential instead of two, a few ulps from the two-call form.
__device__ __forceinline__ double hdla_gate_r(double v, double l, double vhalfl, double tau, const MechConsts& c,
                                              double dt) {
    double a, bett;
    if (c.hd_pow) {
        const double G = exp(c.hd_k5 * (v - c.hd_vhalft));
        bett = G * G;
        a = bett * bett * G;
    } else {
        a = exp(0.0378 * c.hd_zetat * (v - c.hd_vhalft));
        bett = exp(0.0378 * c.hd_zetat * c.hd_gmt * (v - c.hd_vhalft));
    }
    const double linf = div_r(1.0, 1.0 + exp(-(v - vhalfl) * c.hd_inv_kl));
    const double rate = div_r(c.hd_qtl * c.hd_qt * c.hd_a0t * (1.0 + a), tau * bett);   // 1 / taul
    return l + (1.0 - exp(-dt * rate)) * (linf - l);
}

// CaDynamics_E2: steady_term = -(drive - (-minCai)/decay) / (-1/decay) = drive decay + minCai
// (with its parameters one value over the model, cadyn_uniform below)
__device__ __forceinline__ double cadyn_step_r(double cai, double ica, double gamma, double decay, double depth,
                                               double minCai, double dt) {
    const double drive_ica = -(10000.0) * (ica * gamma) / (2.0 * kFaradayCaDyn * depth);
    const double exp_factor = exp(-dt / decay);
    const double steady_term = drive_ica * decay + minCai;
    return cai + (1.0 - exp_factor) * (steady_term - cai);
}

// The same update with its per-model constants made on the host (MechConsts::cd_*):
// cai + c1 (ica g + minCai - cai); a few ulps from cadyn_step_r.
__device__ __forceinline__ double cadyn_uniform(double cai, double ica, const MechConsts& c) {
    return cai + c.cd_c1 * (ica * c.cd_g + c.cd_min - cai);
}

// ---------------- synapses ----------------
__device__ __forceinline__ double expsyn_decay(double g, double tau, double dt) {
    return g + (1. - exp(dt * ((-1.0) / tau))) * (-(0.0) / ((-1.0) / tau) - g);
}

__device__ __forceinline__ double exp2syn_decay(double x, double tau, double dt) {
    return x + (1.0 - exp(dt * (-1.0 / tau))) * (-0.0 / (-1.0 / tau) - x);
}

}  // namespace hx
