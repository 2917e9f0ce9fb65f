// Device-side mechanism arithmetic.
//
// Every expression keeps the algebraic form of the reference mechanism so that
// the fp64 results track the reference CPU path to rounding (the reference is
// compiled with -ffp-contract=off on the host; this library uses the same flag):
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

namespace hx {

constexpr double kFaradayCaDyn = 96485.3321233100184;   // CaDynamics_E2.cu:109

__device__ __forceinline__ double nernst(double ci, double co, double z, double ktf) {
    if (z == 0) return 0.;
    if (ci <= 0.) return 1e6;
    else if (co <= 0.) return -1e6;
    else return ktf / z * log(co / ci);
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

// ---------------- CaDynamics_E2 ----------------
__device__ __forceinline__ double cadyn_step(double cai, double ica, double gamma, double decay, double depth,
                                             double minCai, double dt) {
    double drive_ica = -(10000.0) * (ica * gamma) / (2.0 * kFaradayCaDyn * depth);
    double exp_factor = exp(dt * (-1.0 / decay));
    double steady_term = -(drive_ica - (-minCai) / decay) / (-1.0 / decay);
    return cai + (1.0 - exp_factor) * (steady_term - cai);
}

// ---------------- synapses ----------------
__device__ __forceinline__ double expsyn_decay(double g, double tau, double dt) {
    return g + (1. - exp(dt * ((-1.0) / tau))) * (-(0.0) / ((-1.0) / tau) - g);
}

__device__ __forceinline__ double exp2syn_decay(double x, double tau, double dt) {
    return x + (1.0 - exp(dt * (-1.0 / tau))) * (-0.0 / (-1.0 / tau) - x);
}

}  // namespace hx
