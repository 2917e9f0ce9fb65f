// The generic kernels every mechanism plugin runs with, and the registration macro.
// Included by the plugin sources under csrc/mechs/ (each instantiates these kernels for
// its own struct).  One thread per instance.
#pragma once
#include "plugin.h"

namespace hx {
namespace plugin_detail {

template <class M>
__device__ __forceinline__ plugin::IonIO ion_view(const PluginArgs& P, int j) {
    plugin::IonIO io{};
    constexpr unsigned use = M::kIonRead | M::kIonWrite;
#pragma unroll
    for (int x = 0; x < 3; ++x) {
        if (!(use & (1u << x))) continue;
        const int ci = P.m.ion[x] ? P.m.ion[x][j] : -1;
        if (ci < 0) continue;
        io.erev[x] = P.ion[x].col(ION_EREV)[ci];
        io.conci[x] = P.ion[x].col(ION_CONCI)[ci];
        io.conco[x] = P.ion[x].col(ION_CONCO)[ci];
    }
    return io;
}

template <class M>
__global__ void __launch_bounds__(kBlock) k_plugin_init(PluginArgs P) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P.m.n) return;
    plugin::Inst x{P.m.base, P.m.stride, j};
    const plugin::IonIO io = ion_view<M>(P, j);
    M::init(x, P.v[P.m.node[j]], io, plugin::Env{P.t, P.dt, P.celsius});
}

// FD Jacobian (mech_template.cuh:616-646): I(v + 0.001) first, then I(v), whose assigned
// values stay and whose ion currents are added to the ions; g = (I1 - I0) / 0.001.
// A point process scales both by 1e2/area; an electrode current enters with the other
// sign.  Density instances are one per node (plain read-modify-write); point-process
// instances of one node may share it, so they add with atomics.
template <class M>
__global__ void __launch_bounds__(kBlock) k_plugin_current(PluginArgs P) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P.m.n) return;
    const int node = P.m.node[j];
    const double v = P.v[node];
    plugin::Inst x{P.m.base, P.m.stride, j};
    const plugin::Env env{P.t, P.dt, P.celsius};
    plugin::IonIO io1 = ion_view<M>(P, j);
    plugin::IonIO io0 = io1;
    const double i1 = M::current(x, v + 0.001, io1, env);
    const double i0 = M::current(x, v, io0, env);
    double g = (i1 - i0) / 0.001;
    double rhs = i0;
    if (M::kFlags & plugin::kPoint) {
        const double mfact = 1.e2 / P.area[node];
        g *= mfact;
        rhs *= mfact;
    }
    if (M::kFlags & plugin::kElectrode) {
        rhs = -rhs;
        g = -g;
    }
    if (M::kFlags & plugin::kPoint) {
        atomicAdd(&P.rhs[node], -rhs);
        atomicAdd(&P.d[node], g);
    } else {
        P.rhs[node] -= rhs;
        P.d[node] += g;
    }
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        if (!(M::kIonWrite & (1u << q))) continue;
        const int ci = P.m.ion[q] ? P.m.ion[q][j] : -1;
        if (ci >= 0) atomicAdd(&P.ion[q].col(ION_CUR)[ci], io0.cur[q]);
    }
}

template <class M>
__global__ void __launch_bounds__(kBlock) k_plugin_state(PluginArgs P) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P.m.n) return;
    plugin::Inst x{P.m.base, P.m.stride, j};
    const plugin::IonIO io = ion_view<M>(P, j);
    M::state(x, P.v[P.m.node[j]], io, plugin::Env{P.t, P.dt, P.celsius});
}

// NET_RECEIVE (postsyn_template.cuh:20-51): an instance has one netcon, so the step's
// events into it are alike; they are received one after another, as many as arrived.
template <class M>
__global__ void __launch_bounds__(kBlock) k_plugin_receive(PluginArgs P) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= P.m.n) return;
    const int n = P.recv_count[j];
    if (n == 0) return;
    plugin::Inst x{P.m.base, P.m.stride, j};
    const plugin::Env env{P.t, P.dt, P.celsius};
    for (int e = 0; e < n; ++e) M::net_receive(x, P.recv_w[j], P.recv_delay[j], env);
    P.recv_count[j] = 0;
}

inline dim3 plugin_grid(int n) { return dim3(static_cast<unsigned>(n > 0 ? (n + kBlock - 1) / kBlock : 1)); }

template <class M>
void launch_init(const PluginArgs& P, hipStream_t s) {
    if (P.m.n > 0) hipLaunchKernelGGL(k_plugin_init<M>, plugin_grid(P.m.n), dim3(kBlock), 0, s, P);
}
template <class M>
void launch_current(const PluginArgs& P, hipStream_t s) {
    if (P.m.n > 0) hipLaunchKernelGGL(k_plugin_current<M>, plugin_grid(P.m.n), dim3(kBlock), 0, s, P);
}
template <class M>
void launch_state(const PluginArgs& P, hipStream_t s) {
    if (P.m.n > 0) hipLaunchKernelGGL(k_plugin_state<M>, plugin_grid(P.m.n), dim3(kBlock), 0, s, P);
}

template <class M>
void launch_receive(const PluginArgs& P, hipStream_t s) {
    if (P.m.n > 0) hipLaunchKernelGGL(k_plugin_receive<M>, plugin_grid(P.m.n), dim3(kBlock), 0, s, P);
}

template <class M>
PluginMeta meta_of() {
    static_assert(sizeof(M::kCols) / sizeof(M::kCols[0]) == sizeof(M::kDefault) / sizeof(M::kDefault[0]),
                  "one default per column");
    static_assert(M::kParams + M::kStates <= static_cast<int>(sizeof(M::kCols) / sizeof(M::kCols[0])),
                  "parameters and states are columns");
    void (*recv)(const PluginArgs&, hipStream_t) = nullptr;
    if constexpr ((M::kFlags & plugin::kPostsyn) != 0) recv = &launch_receive<M>;
    return PluginMeta{M::kName, static_cast<int>(sizeof(M::kCols) / sizeof(M::kCols[0])), M::kParams, M::kStates,
                      M::kCols, M::kDefault, M::kFlags, M::kIonRead, M::kIonWrite, &launch_init<M>,
                      &launch_current<M>, &launch_state<M>, recv};
}

}  // namespace plugin_detail
}  // namespace hx

// Registration by name at library load (the reference's REGISTER_MECHANISM, mechanism.h:167-171).
#define HX_REGISTER_MECHANISM(STRUCT) \
    static const bool hx_plugin_registered_##STRUCT = ::hx::register_plugin(::hx::plugin_detail::meta_of<STRUCT>())
