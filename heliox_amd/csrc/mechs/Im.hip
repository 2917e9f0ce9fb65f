// Im: the muscarinic K current of the Blue Brain models (reference:
// src/mech/user-mech/Im.cu:9-130), added through the mechanism plugin seam.
// Columns follow the reference's VarNames order; ek is read from k_ion and ik added
// to it.
#include <cmath>

#include "../plugin_kernels.h"

namespace {

struct Im {
    static constexpr const char* kName = "Im";
    static constexpr const char* kCols[] = {"gImbar", "m", "ik", "gIm", "ek", "mInf", "mTau", "mAlpha", "mBeta"};
    static constexpr double kDefault[] = {0.00001, 0, 0, 0, 0, 0, 0, 0, 0};
    static constexpr int kParams = 1, kStates = 1;
    static constexpr unsigned kFlags = 0;
    static constexpr unsigned kIonRead = hx::plugin::kK, kIonWrite = hx::plugin::kK;
    enum { GIMBAR = 0, M, IK, GIM, EK, MINF, MTAU, MALPHA, MBETA };

    // rates (Im.cu:63-70); the temperature factor is fixed at 34 C, as in the model
    __device__ static void rates(const hx::plugin::Inst& x, double v) {
        const double qt = pow(2.3, (34.0 - 21.0) / 10.0);
        x[MALPHA] = 3.3e-3 * exp(2.5 * 0.04 * (v - (-35.0)));
        x[MBETA] = 3.3e-3 * exp(-2.5 * 0.04 * (v - (-35.0)));
        x[MINF] = x[MALPHA] / (x[MALPHA] + x[MBETA]);
        x[MTAU] = (1.0 / (x[MALPHA] + x[MBETA])) / qt;
    }
    __device__ static void init(hx::plugin::Inst& x, double v, const hx::plugin::IonIO& io, const hx::plugin::Env&) {
        x[EK] = io.erev[1];
        rates(x, v);
        x[M] = x[MINF];
    }
    __device__ static double current(hx::plugin::Inst& x, double v, hx::plugin::IonIO& io, const hx::plugin::Env&) {
        x[EK] = io.erev[1];
        x[GIM] = x[GIMBAR] * x[M];
        x[IK] = x[GIM] * (v - x[EK]);
        io.cur[1] += x[IK];
        return x[IK];
    }
    // cnexp in the model's form (Im.cu:95-100)
    __device__ static void state(hx::plugin::Inst& x, double v, const hx::plugin::IonIO& io,
                                 const hx::plugin::Env& e) {
        x[EK] = io.erev[1];
        rates(x, v);
        const double tau = x[MTAU];
        x[M] = x[M] + (1.0 - exp(e.dt * ((-1.0) / tau))) * (-(x[MINF] / tau) / ((-1.0) / tau) - x[M]);
    }
};

HX_REGISTER_MECHANISM(Im);

}  // namespace
