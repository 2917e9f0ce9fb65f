// syn_record: an AMPA + NMDA (w > 0) or GABA (w <= 0) double-exponential synapse, a
// point process that netcons target (reference: src/spike/user_postsyn_mech/
// syn_record.cuh:8-203, registered there with REGISTER_POSTSYN), added through the
// mechanism plugin seam.  Columns: the reference's parameters (its VarNames 0-18), the
// six states, then the assigned variables; the arithmetic keeps the reference's forms.
#include <cmath>

#include "../plugin_kernels.h"

namespace {

struct SynRecord {
    static constexpr const char* kName = "syn_record";
    static constexpr const char* kCols[] = {
        "AMPA_tau1", "AMPA_tau2", "NMDA_tau1", "NMDA_tau2", "GABA_tau1", "GABA_tau2", "AMPA_e", "NMDA_e", "GABA_e",
        "NMDA_C", "NMDA_rho", "w", "r_na", "dv", "Use_e", "Use_i", "Dep", "Fac", "u0",
        "AMPA_A", "AMPA_B", "NMDA_A", "NMDA_B", "GABA_A", "GABA_B",
        "i", "AMPA_g", "NMDA_g", "GABA_g", "v_prev", "didv", "pure_i", "g_mul", "dgdv", "dgdg", "Use",
        "AMPA_factor", "NMDA_factor", "GABA_factor"};
    static constexpr double kDefault[] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1.0, 2.0, 1e-3, 1.0, 1.0, 0, 0, 0,
                                          0, 0, 0, 0, 0, 0,
                                          0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    static constexpr int kParams = 19, kStates = 6;
    static constexpr unsigned kFlags = hx::plugin::kPoint | hx::plugin::kPostsyn;
    static constexpr unsigned kIonRead = 0, kIonWrite = 0;
    enum {
        AMPA_TAU1 = 0, AMPA_TAU2, NMDA_TAU1, NMDA_TAU2, GABA_TAU1, GABA_TAU2, AMPA_E, NMDA_E, GABA_E, NMDA_C,
        NMDA_RHO, W, R_NA, DV, USE_E, USE_I, DEP, FAC, U0,
        AMPA_A, AMPA_B, NMDA_A, NMDA_B, GABA_A, GABA_B,
        I, AMPA_G, NMDA_G, GABA_G, V_PREV, DIDV, PURE_I, G_MUL, DGDV, DGDG, USE, AMPA_FACTOR, NMDA_FACTOR,
        GABA_FACTOR
    };
    using Inst = hx::plugin::Inst;

    __device__ static double sigma(double v, const Inst& x) {   // NMDA magnesium block
        return 1.0 / (1.0 + x[NMDA_C] * exp(-x[NMDA_RHO] * v));
    }
    // tau1 kept below tau2, A = B = 0, factor normalising the peak (syn_record.cuh:104-125)
    __device__ static void pair(Inst& x, int tau1, int tau2, int a, int b, int factor) {
        double t1 = x[tau1];
        const double t2 = x[tau2];
        if (t1 / t2 > 0.9999) { t1 = 0.9999 * t2; x[tau1] = t1; }
        if (t1 / t2 < 1e-9) { t1 = 1e-9 * t2; x[tau1] = t1; }
        x[a] = 0.0;
        x[b] = 0.0;
        const double tp = (t1 * t2) / (t2 - t1) * log(t2 / t1);
        x[factor] = 1.0 / (-exp(-tp / t1) + exp(-tp / t2));
    }
    __device__ static void init(Inst& x, double, const hx::plugin::IonIO&, const hx::plugin::Env&) {
        pair(x, AMPA_TAU1, AMPA_TAU2, AMPA_A, AMPA_B, AMPA_FACTOR);
        pair(x, NMDA_TAU1, NMDA_TAU2, NMDA_A, NMDA_B, NMDA_FACTOR);
        pair(x, GABA_TAU1, GABA_TAU2, GABA_A, GABA_B, GABA_FACTOR);
        x[USE] = x[W] > 0.0 ? x[USE_E] : x[USE_I];
    }
    // nA (syn_record.cuh:128-148)
    __device__ static double current(Inst& x, double v, hx::plugin::IonIO&, const hx::plugin::Env&) {
        x[V_PREV] = v;
        double cur;
        if (x[W] > 0.0) {
            x[AMPA_G] = x[AMPA_B] - x[AMPA_A];
            x[NMDA_G] = x[NMDA_B] - x[NMDA_A];
            const double s = sigma(v, x);
            cur = fabs(x[W]) * (x[AMPA_G] * (v - x[AMPA_E]) + x[NMDA_G] * s * (v - x[NMDA_E]));
        } else {
            x[GABA_G] = x[GABA_B] - x[GABA_A];
            cur = fabs(x[W]) * x[GABA_G] * (v - x[GABA_E]);
        }
        x[I] = cur;
        return cur;
    }
    // decays and the diagnostic gradients the reference records (syn_record.cuh:151-178)
    __device__ static void state(Inst& x, double v, const hx::plugin::IonIO&, const hx::plugin::Env& e) {
        const double dt = e.dt;
        x[AMPA_A] *= exp(-dt / x[AMPA_TAU1]);
        x[AMPA_B] *= exp(-dt / x[AMPA_TAU2]);
        x[NMDA_A] *= exp(-dt / x[NMDA_TAU1]);
        x[NMDA_B] *= exp(-dt / x[NMDA_TAU2]);
        x[GABA_A] *= exp(-dt / x[GABA_TAU1]);
        x[GABA_B] *= exp(-dt / x[GABA_TAU2]);
        const double w = x[W];
        if (w > 0.0) {
            x[DIDV] = fabs(w) * (x[AMPA_G] + x[NMDA_G] * sigma(x[V_PREV], x));
            x[PURE_I] = x[AMPA_G] * (v - x[AMPA_E]) + x[NMDA_G] * sigma(x[V_PREV], x) * (v - x[NMDA_E]);
            x[G_MUL] = fabs(w) * x[NMDA_G] * (v - x[NMDA_E]);
            x[DGDV] = (sigma(x[V_PREV] + x[DV], x) - sigma(x[V_PREV], x)) / x[DV];
            x[DGDG] = 0.0;
        } else {
            x[DIDV] = fabs(w) * x[GABA_G];
            x[PURE_I] = -x[GABA_G] * (v - x[GABA_E]);
            x[G_MUL] = 0.0;
            x[DGDV] = 0.0;
            x[DGDG] = 0.0;
        }
    }
    // one event of weight w_event (syn_record.cuh:181-199)
    __device__ static void net_receive(Inst& x, double w_event, double, const hx::plugin::Env&) {
        if (x[W] > 0.0) {
            const double ra = x[R_NA];
            const double a_fac = w_event * x[AMPA_FACTOR] / (1.0 + ra);
            const double n_fac = w_event * x[NMDA_FACTOR] * ra / (1.0 + ra);
            x[AMPA_A] += a_fac;
            x[AMPA_B] += a_fac;
            x[NMDA_A] += n_fac;
            x[NMDA_B] += n_fac;
        } else {
            const double g_fac = w_event * x[GABA_FACTOR];
            x[GABA_A] += g_fac;
            x[GABA_B] += g_fac;
        }
    }
};

HX_REGISTER_MECHANISM(SynRecord);

}  // namespace
