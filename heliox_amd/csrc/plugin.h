// Mechanism plugins: the seam through which a mechanism outside the built-in set
// is added to the library and becomes insertable by name (hx_model_insert), as the
// reference's MechanismFactory registers a MechTemp-derived class under its name
// (mechanism.h:125-197, mech_reg.cu:60-75, author contract mech_template.cuh:104-126).
//
// A plugin is a struct with
//   static constexpr const char* kName;              the name models use
//   static constexpr const char* kCols[];            columns: parameters, then states,
//   static constexpr double kDefault[];              then assigned variables, with defaults
//   static constexpr int kParams, kStates;
//   static constexpr unsigned kFlags;                kPoint (values per instance scaled by
//                                                    1e2/area), kElectrode (sign of an
//                                                    electrode current)
//   static constexpr unsigned kIonRead, kIonWrite;   ions (kNa, kK, kCa bits) whose erev /
//                                                    concentrations it reads, whose current
//                                                    it adds to
//   __device__ static void init(Inst&, double v, const IonIO&, const Env&);
//   __device__ static double current(Inst&, double v, IonIO&, const Env&);
//       returns the membrane current (mA/cm2, or nA for a point process) at v and adds
//       its ion currents to io.cur[ion]; it may store assigned variables
//   __device__ static void state(Inst&, double v, const IonIO&, const Env&);
// and, with kPostsyn in kFlags (a synapse that netcons target; the reference's
// REGISTER_POSTSYN, mechanism.h:173 / postsyn_template.cuh:6-51),
//   __device__ static void net_receive(Inst&, double weight, double delay, const Env&);
// It is registered in a source file under csrc/mechs/ with HX_REGISTER_MECHANISM(Struct)
// (plugin_kernels.h).  The library then runs it with instance-parallel kernels: the
// finite-difference Jacobian of the current (mech_template.cuh:616-646), the current and
// ion current accumulation after the built-in mechanisms of each current pass, the state
// update after the solve of each step, and, for a synapse, NET_RECEIVE of the step's
// events after the built-in synapses' delivery.
#pragma once
#include <hip/hip_runtime.h>

#include "hx_internal.h"

namespace hx {

namespace plugin {
constexpr unsigned kPoint = 1u, kElectrode = 2u, kPostsyn = 4u;
constexpr unsigned kNa = 1u, kK = 2u, kCa = 4u;   // ion bits, in the ion index order na, k, ca

// One instance's columns: x[c] is column c of this instance.
struct Inst {
    double* base;
    long long stride;
    int j;
    __device__ double& operator[](int c) const { return base[c * stride + j]; }
};

// Ion values at the instance's node: erev and concentrations of the ions it reads
// (0 for ions absent there), and the ion currents its current evaluation adds.
struct IonIO {
    double erev[3], conci[3], conco[3];
    double cur[3];
};

struct Env {
    double t, dt, celsius;
};
}  // namespace plugin

// Device view of one plugin's instances and what its kernels touch.
struct PluginArgs {
    MechDev m;                    // columns, solver-order node, ion instance maps
    MechDev ion[3];               // na, k, ca ion columns
    double* v;
    double* d;
    double* rhs;
    const double* area;
    double t, dt, celsius;
    // synapses: events of the step per instance (counted by the delivery kernel), and the
    // weight and delay of each instance's netcon (one netcon per instance)
    int* recv_count;
    const double* recv_w;
    const double* recv_delay;
};

// What the registration records: the metadata the builder and the handles need, and
// the launchers of the plugin's kernels (instantiated in the plugin's source file).
struct PluginMeta {
    const char* name;
    int ncol, nparam, nstate;
    const char* const* cols;
    const double* dflt;
    unsigned flags, ion_read, ion_write;
    void (*launch_init)(const PluginArgs&, hipStream_t);
    void (*launch_current)(const PluginArgs&, hipStream_t);
    void (*launch_state)(const PluginArgs&, hipStream_t);
    void (*launch_receive)(const PluginArgs&, hipStream_t);   // synapses only, else nullptr
};

// Registers a plugin (from a static initializer); returns true.
bool register_plugin(const PluginMeta& meta);
// The plugin registered under name, or nullptr.
const PluginMeta* find_plugin(const char* name);
// Every registered plugin, in registration order.
int plugin_count();
const PluginMeta& plugin_at(int k);

}  // namespace hx
