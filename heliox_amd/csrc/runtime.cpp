// Host runtime of the HIP simulation core: model storage, HBM layout, the
// per-step launch pipeline and the C ABI declared in include/heliox.h.
//
// The step pipeline reproduces Simulate::fadvance (simulate.cpp:410-442,
// simulate.cu:722-771).  Two schedules are used:
//   fused:  step k launches the dense/sparse mechanism kernels with the state
//           update of step k-1 folded in front of the current of step k, so a
//           mechanism's state columns are read and written once per step;
//   split:  the reference order (currents ... solve ... states) as separate
//           passes.  Used when a VecPlay targets a density-mechanism variable,
//           when a monitor samples an assigned variable, or when an
//           ion-writing mechanism (CaDynamics_E2) is not on every node.
// Both give the same values at every observable point (end of a run call,
// every recorded sample).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <iterator>
#include <functional>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <limits>
#include <map>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <set>
#include <tuple>
#include <unordered_map>
#include <vector>

#include "heliox.h"
#include "h5out.h"
#include "hx_internal.h"
#include "learn.h"
#include "plugin.h"
#include "random123.h"
#include "fastmath.h"
#include "schedule.h"
#include "solve_chunk.h"

// ---------------------------------------------------------------------------
// mechanism plugins registered at library load (plugin.h)
// ---------------------------------------------------------------------------
namespace hx {
namespace {
std::vector<PluginMeta>& plugin_registry() {
    static std::vector<PluginMeta> r;
    return r;
}
}  // namespace
bool register_plugin(const PluginMeta& meta) {
    plugin_registry().push_back(meta);
    return true;
}
const PluginMeta* find_plugin(const char* name) {
    for (const auto& m : plugin_registry())
        if (std::strcmp(m.name, name) == 0) return &m;
    return nullptr;
}
int plugin_count() { return static_cast<int>(plugin_registry().size()); }
const PluginMeta& plugin_at(int k) { return plugin_registry()[k]; }
}  // namespace hx

using namespace hx;

namespace {

// ---------------------------------------------------------------------------
// mechanism registry (the reference's MechanismFactory, mechanism.h:125-164)
// ---------------------------------------------------------------------------
struct MechMeta {
    const char* name;
    int ncol;
    int nparam;
    int nstate;
    std::vector<const char*> cols;
    std::vector<double> dflt;
    bool point;
    bool ion;
    bool artificial;
    bool write_ion;     // WRITE_EION_IN_STATE (mech_template_utils.cuh:26-33)
    int ion_use;        // bit0 na, bit1 k, bit2 ca
    bool has_state;
};

const std::vector<MechMeta>& registry() {
    static const std::vector<MechMeta> R = [] {
        std::vector<MechMeta> r(M_COUNT);
        r[M_PAS] = {"pas", PAS_NCOL, 2, 0, {"g_pas", "e_pas", "i"}, {0.00016666, -60, 0}, false, false, false, false, 0, false};
        r[M_NA_ION] = {"na_ion", ION_NCOL, 3, 0, {"erev", "conci", "conco", "cur", "dcurdv"}, {0, 10.0, 140.0, 0, 0},
                       false, true, false, false, 0, false};
        r[M_K_ION] = {"k_ion", ION_NCOL, 3, 0, {"erev", "conci", "conco", "cur", "dcurdv"}, {0, 140.0, 4.0, 0, 0},
                      false, true, false, false, 0, false};
        r[M_HH] = {"hh", HH_NCOL, 4, 3,
                   {"gnabar", "gkbar", "gl", "el", "m", "h", "n", "ena", "ek", "ina", "ik", "il", "gna", "gk", "minf",
                    "hinf", "ninf", "mtau", "htau", "ntau"},
                   {0.25, 0.036, 0.00016666, -60.0, 0, 0, 0, 50, -77, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0},
                   false, false, false, false, 3, true};
        r[M_ICLAMP] = {"IClamp", IC_NCOL, 3, 0, {"delay", "dur", "amp", "i"}, {0, 0, 0, 0}, true, false, false, false, 0,
                       false};
        r[M_EXPSYN] = {"ExpSyn", ES_NCOL, 2, 1, {"tau", "e", "g", "i"}, {0.1, 0, 0, 0}, true, false, false, false, 0, true};
        r[M_EXP2SYN] = {"Exp2Syn", E2_NCOL, 3, 2, {"tau1", "tau2", "e", "A", "B", "factor", "g", "i"},
                        {0.1, 10.0, 0, 0, 0, 0, 0, 0}, true, false, false, false, 0, true};
        r[M_VECSTIM] = {"VecStim", 0, 0, 0, {}, {}, true, false, true, false, 0, false};
        r[M_CA_ION] = {"ca_ion", ION_NCOL, 3, 0, {"erev", "conci", "conco", "cur", "dcurdv"}, {0, 5.e-5, 2.0, 0, 0},
                       false, true, false, false, 0, false};
        r[M_CADYN] = {"CaDynamics_E2", CD_NCOL, 4, 0, {"gamma", "decay", "depth", "minCai"}, {0.05, 80.0, 0.1, 1e-4},
                      false, false, false, true, 4, true};
        r[M_CAHVA] = {"Ca_HVA", CH_NCOL, 1, 2,
                      {"gbar", "m", "h", "eca", "ica", "g", "i_mech", "mInf", "mTau", "mAlpha", "mBeta", "hInf", "hTau",
                       "hAlpha", "hBeta"},
                      {0.1, 0, 0, 140.0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0}, false, false, false, false, 4, true};
        r[M_HALFGAP] = {"HalfGap", HG_NCOL, 2, 0, {"g", "vgap", "i"}, {0, 0, 0}, true, false, false, false, 0, false};
        r[M_HDLA] = {"hd_la", HD_NCOL, 3, 1, {"ghdbar", "vhalfl", "tau", "l", "i", "linf", "taul", "ghd"},
                     {0.0001, -81.0, 1.0, 0, 0, 0, 0, 0}, false, false, false, false, 0, true};
        // defaults of netstim.cpp reg_node_indices (interval 10, number 10, start 50, noise 0)
        r[M_NETSTIM] = {"NetStim", NS_NCOL, NS_NCOL, 0, {"interval", "number", "start", "noise", "id1", "id2", "id3"},
                        {10.0, 10.0, 50.0, 0.0, -1.0, 0.0, 0.0}, true, false, true, false, 0, false};
        return r;
    }();
    return R;
}

int mech_id(const std::string& name) {
    const auto& R = registry();
    for (int i = 0; i < M_COUNT; ++i)
        if (name == R[i].name) return i;
    return -1;
}

int col_id(int mech, const std::string& var) {
    const auto& m = registry()[mech];
    for (int c = 0; c < m.ncol; ++c)
        if (var == m.cols[c]) return c;
    return -1;
}

struct HipError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define HXC(x)                                                                              \
    do {                                                                                    \
        hipError_t e_ = (x);                                                                \
        if (e_ != hipSuccess)                                                               \
            throw HipError(std::string(#x) + ": " + hipGetErrorString(e_));                 \
    } while (0)

template <class T>
T* dalloc(std::vector<void*>& owned, size_t n) {
    void* p = nullptr;
    HXC(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    owned.push_back(p);
    return static_cast<T*>(p);
}

template <class T>
T* dupload(std::vector<void*>& owned, const std::vector<T>& h) {
    T* p = dalloc<T>(owned, h.size());
    if (!h.empty()) HXC(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return p;
}

// ---------------------------------------------------------------------------
// host model
// ---------------------------------------------------------------------------
struct HostMech {
    bool present = false;
    int n = 0;
    std::vector<int> node;                     // user node per user instance
    std::vector<std::vector<double>> col;      // user-order columns (load time)
    std::vector<int> iontype;
    // layout
    std::vector<int> perm;                     // user instance -> device instance
    std::vector<int> iperm;                    // device instance -> user instance
    bool dense = false;
    MechDev dev;
};

// mech: a MechId, or kPluginMechBase + the index of a synapse plugin in the model
struct NetCon { int src_kind; int src; int mech; int inst; double weight; double delay; };
constexpr int kPluginMechBase = 1000;

struct VecPlayHost {
    std::string mech, var;
    int idx;
    std::vector<double> tvec, yvec;
    double* target = nullptr;
    double* d_t = nullptr;
    double* d_y = nullptr;
};

// klass 0 param/state, 1 assigned; point: a point-process column (its values
// change at event delivery, which the fused schedule runs before the record)
struct Ref {
    double* dev = nullptr;
    int klass = 0;
    bool point = false;
    int ab = 0;           // 1: node coefficient a, 2: b (the solver keeps its own copy)
    int node = -1;        // user node of an a / b reference
    int ns_col = -1;      // NetStim parameter (the host keeps the copy its trains come from)
    int ns_inst = -1;
};

struct Timer {
    std::vector<hipEvent_t> pool;
    std::vector<std::pair<int, int>> pending;   // (start, stop) indices into pool
    size_t used = 0;
    double ms = 0;
    long long launches = 0;
};

const char* kTimerNames[] = {"mech", "sparse", "point", "solve", "spike", "events", "other"};
enum TimerId { T_MECH = 0, T_SPARSE, T_POINT, T_SOLVE, T_SPIKE, T_EVENTS, T_OTHER, T_COUNT };

}  // namespace

// Parameters the adjoint differentiates: a mechanism's parameter column, or the
// weight of the netcon into a synapse instance.  Their gradients are addressable
// as variables "grad_<var>" of the mechanism (and "grad_weight").
struct Trainable {
    int mech;
    const char* var;
};
constexpr int kNumTrainable = 8;
constexpr Trainable kTrainable[kNumTrainable] = {
    {M_HH, "gnabar"}, {M_HH, "gkbar"}, {M_PAS, "g_pas"}, {M_EXPSYN, "weight"},
    {M_CAHVA, "gbar"}, {M_HDLA, "ghdbar"}, {M_EXP2SYN, "weight"}, {M_HALFGAP, "g"}};
enum TrainableId { T_GNABAR = 0, T_GKBAR, T_GPAS, T_WES, T_CGBAR, T_GHDBAR, T_WE2, T_GGAP };

inline int trainable_id(int mech, const std::string& var) {
    for (int k = 0; k < kNumTrainable; ++k)
        if (kTrainable[k].mech == mech && var == kTrainable[k].var) return k;
    return -1;
}

struct hx_sim {
    // A device block that a repeated call refills: it is reallocated only to grow, the
    // old block freed once the library stream has drained, so loops of such calls
    // (finitialize, adjoint, optimizer and monitor changes) hold one block each.
    struct DevSlot {
        void* p = nullptr;
        size_t bytes = 0;
    };
    std::string err;
    double dt = 0.025;
    bool dt_set = false;                 // set by the caller (else a CoreNEURON export's dt is taken)
    double celsius = 6.3;
    std::string data_path;               // CoreNEURON export read by hx_load_model
    int user_mod_num = 1000;             // artificial presyns are -(type + index * user_mod_num)
    // nodes (user order)
    int ncell = 0, nnode = 0;
    std::vector<int> parent;
    std::vector<double> a, b, area, cm;
    HostMech mech[M_COUNT];
    std::map<std::string, double> globals[M_COUNT];
    // mechanisms added through the plugin seam, in insertion order
    struct PluginInst {
        const PluginMeta* meta = nullptr;
        HostMech h;
        int slot = -1;                            // synapse plugins: slot of the packed targets
        int* d_recv_count = nullptr;              // events of the step per instance
        double* d_recv_w = nullptr;               // the instance's netcon weight and delay
        double* d_recv_delay = nullptr;
    };
    bool has_postsyn_plugins() const {
        for (const auto& p : plugins)
            if (p.meta->flags & plugin::kPostsyn) return true;
        return false;
    }
    std::vector<PluginInst> plugins;
    PluginInst* plugin_named(const std::string& name) {
        for (auto& p : plugins)
            if (name == p.meta->name) return &p;
        return nullptr;
    }
    unsigned plugin_ions() const {     // ions some plugin reads or writes (bit 0 na, 1 k, 2 ca)
        unsigned u = 0;
        for (const auto& p : plugins) u |= p.meta->ion_read | p.meta->ion_write;
        return u;
    }
    PluginArgs plugin_args(const PluginInst& p, double tcur) const;
    void launch_plugin_inits(double tcur);
    void launch_plugin_currents(double tcur);
    void launch_plugin_states(double tcur);
    std::vector<int> pre_gid, pre_node;
    std::vector<double> pre_thr;
    std::vector<std::vector<double>> vecstim;
    // the trains the current run reads: vecstim at finitialize, then what VecStim.play
    // calls during the run leave (vecstim_play)
    std::vector<std::vector<double>> vecstim_run;
    bool vecstim_run_differs = false;
    int vecstim_play(int inst, const double* times, int n);
    // NetStim trains (self-event times), made on the host up to step ns_horizon
    std::vector<std::vector<double>> netstim;
    int ns_horizon = 0;
    void make_netstim_trains(int horizon);
    std::vector<NetCon> netcons;
    std::vector<std::pair<int, int>> gaps;     // (src node, halfgap inst)
    std::vector<std::pair<int, int>> gaps_eff; // the gaps the transfers use: the last of each instance
    std::vector<VecPlayHost> vecplay;
    int event_cap_request = 0;
    int fusion_allowed = 1;
    int dense_steady = 1;                      // compile-time node-kernel instances for steady steps
    long long steady_launches = 0;             // node-kernel launches that ran such an instance
    hipEvent_t mech_end_mark = nullptr;        // the last mechanism pass's node-kernel timer end, if
                                               // nothing was launched after it (else nullptr)
    int* d_syn_grp[2] = {nullptr, nullptr};   // adjoint: node -> ExpSyn / Exp2Syn group
    // adjoint loss: nodes and targets per call, the distinct nodes with their loss
    // indices (node -> first index of its list), and node -> loss index when distinct
    DevSlot adj_ln_slot, adj_tgt_slot, adj_samp_slot, adj_un_slot, adj_ubeg_slot, adj_uidx_slot, adj_lmap_slot;
    DevSlot adj_gp_slot, adj_gs_slot, adj_gb_slot, adj_gi_slot;   // gap junctions (HalfGap)
    std::vector<int> adj_lmap_nodes;             // the loss nodes adj_lmap_slot holds the map of
    unsigned adj_fuse_bits = 0;          // last hx_adjoint's node-parallel masks (state | cond << 8 | param << 16)
    bool uniform_on = true;              // parameter columns with one value read as scalars
    bool cm_uniform = false;             // cm holds one value on every node (as the columns above)
    double cm_value = 0.0;
    bool loaded = false;

    // layout
    std::vector<int> node_perm, node_iperm;    // user <-> solver order
    std::vector<int> ion_at[3];                // na/k/ca: solver-order node -> device ion instance (-1: none)
    // solve units: runs of consecutive cells, each solved by one wavefront
    std::vector<int> unit_cell_begin, unit_node_begin, unit_desc_begin, unit_round_begin;
    int nunit = 0;
    int unit_cells = 1;                  // cells per unit of the current layout
    int unit_request = 0;                // 0: the library's choice
    int solve_waves_request = 0;         // units per solve workgroup (0: the library's choice)
    int solve_waves = 1;                 // in use (set at load)
    bool solve_resident_allowed = true;  // units that fit kResUnitBudget are solved held in LDS
    bool solve_voltage_allowed = true;   // the solve may take rhs + d v and yield v_new itself
    bool solve_voltage = false;          // in use: every d and rhs term of a step is the node kernel's
    int pass_yform = 0;                  // the node pass being launched stores rhs + d v
    int res_nodes = 0;                   // in use (set at load): nodes of the largest unit, 0: streamed
    // the solver's tree (user node indices) and its coupling coefficients
    std::vector<int> solve_parent;
    std::vector<double> solve_a, solve_b;
    bool solve_root_centre = true;
    std::vector<RoundInfo> rounds;       // all units' rounds, unit by unit
    std::vector<ChunkDesc> descs;
    int max_slots = 0, max_rounds = 0;
    int ion_type_uniform[3] = {-1, -1, -1};
    unsigned dense_mask = 0;
    bool fused = false;
    bool hh_owns_ions = false;           // sparse hh stores the na / k currents (see the layout)
    PointUnion point_union;              // IClamp / HalfGap nodes for the one-launch electrode currents
    bool vecplay_iclamp_only = true;     // every VecPlay target is an IClamp variable
    AfterSolve after_solve_args(double tn, int knext, int grp) const;
    SpikeArgs spike_args(int kk, double tk, int pre0, int pre1, const EventRing& ring) const;
    void upload_gap_ptrs();
    std::vector<int> point_grp_node[2];  // host copies of the IClamp / HalfGap group nodes
    // CaDynamics_E2 updated by the current pass that computes its ica (see k_dense):
    // allowed when nothing samples calcium between the two passes
    bool cadyn_eager = false;
    bool cadyn_done = false;      // the last current pass already did this step's update
    int pass_cadyn_skip = 0, pass_cadyn_after = 0;
    void refresh_cadyn_eager();
    bool write_assigned = false;
    bool init_pass = false;              // finitialize's current pass is running

    bool need_split_for_monitor = false;

    // device
    std::vector<void*> owned;
    hipStream_t stream = nullptr;
    void* slot_reserve(DevSlot& s, size_t bytes);
    template <class T>
    T* slot_upload(DevSlot& s, const std::vector<T>& h);
    double *d_sa = nullptr, *d_sb = nullptr;   // solver coefficients (solver tree), node order
    double *d_v = nullptr, *d_d = nullptr, *d_rhs = nullptr, *d_a = nullptr, *d_b = nullptr, *d_cm = nullptr,
           *d_area = nullptr, *d_w = nullptr;
    int *d_unit_node_begin = nullptr, *d_unit_desc_begin = nullptr, *d_unit_round_begin = nullptr;
    RoundInfo* d_rounds = nullptr;
    ChunkDesc* d_desc = nullptr;
    // spikes / events
    int npre = 0;
    std::vector<int> h_pre_node_dev;          // solver-order node of each device detector
    bool pre_fanout_empty = true;             // no netcon is driven by a detector
    std::vector<int> syn_node[2];             // solver-order node of each ExpSyn / Exp2Syn instance
    std::vector<int> inst_node[M_COUNT];      // the same for every mechanism outside the node kernel
    int *d_pre_node = nullptr, *d_pre_flag = nullptr, *d_pre_gid = nullptr;
    double* d_pre_thr = nullptr;
    int *d_pre_fo_begin = nullptr, *d_pre_fo_target = nullptr;
    double* d_pre_fo_delay = nullptr;
    double *d_es_weight = nullptr, *d_e2_weight = nullptr;
    double max_delay = 0;
    // NetStims that receive netcons run on the device (k_netstim); the others are trains
    // made on the host
    std::vector<int> ns_dyn;                  // NetStim instance -> index among these, or -1
    std::vector<int> ns_dyn_inst;             // index -> NetStim instance
    std::vector<double> ns_dyn_w;             // weight of its incoming netcon
    NsArgs nsa{};                             // device state (nsa.n == 0: none)
    int ns_log_cap = 0;
    void upload_ns_dyn_state();
    double* d_spk_t = nullptr;
    int* d_spk_gid = nullptr;
    int* d_spk_count = nullptr;
    int* const* d_ring_overflow = nullptr;   // each group's ring overflow flag
    int* h_status = nullptr;                 // pinned: StatusArgs::out
    double* h_mon = nullptr;                 // pinned: the monitor samples of a call
    size_t h_mon_cap = 0;                    // doubles
    int spk_cap = 0;
    bool inputs_dirty = true;
    // Cell groups.  Cells are split into contiguous groups, each with its own
    // event ring, VecStim input list and fan-out (targets inside the group).
    // When nothing couples the groups (no detector netcons, gaps or VecPlay,
    // every density mechanism in the node kernel, synapses folded) and the run
    // allows it, each group's step chain -- events, node kernel, solve,
    // detection, synapse decay -- is issued on a stream of its own, so one
    // group's latency-bound solve overlaps another group's HBM-bound node pass.
    struct CellGroup {
        int node0 = 0, node1 = 0, cell0 = 0, cell1 = 0, unit0 = 0, unit1 = 0;
        int pre0 = 0, pre1 = 0;                   // detectors (sorted by node)
        int es0 = 0, es1 = 0, e20 = 0, e21 = 0;   // ExpSyn / Exp2Syn instances
        int inst0[M_COUNT] = {}, inst1[M_COUNT] = {};   // instances of mechanisms outside the node kernel
        int* d_blk_es = nullptr;                  // fold tables over the group's node blocks
        int* d_blk_e2 = nullptr;
        EventRing ring{};
        double* d_in_time = nullptr;
        int* d_in_inst = nullptr;
        int* d_in_round = nullptr;                // pass of the delivery loop that emits each input
        DevSlot in_time_slot, in_inst_slot, in_round_slot;
        int* d_in_cursor = nullptr;
        int n_in = 0;
        int *d_vs_fo_begin = nullptr, *d_vs_fo_target = nullptr;
        double* d_vs_fo_delay = nullptr;
        std::vector<char> vs_used;                // VecStim instance has a target in the group
        int mon0 = 0, mon1 = 0;                   // monitor buffer columns of the group
        hipStream_t s = nullptr;
        hipEvent_t done = nullptr;
        hipEvent_t pass = nullptr;                // this group's node pass of the latest step issued
        hipEvent_t pass_mark = nullptr;           // what marks it: `pass`, or the node-kernel timer's end
    };
    std::vector<CellGroup> groups;                // one group unless the model decouples
    int group_request = 0;                        // hx_set_cell_groups (0: automatic)
    bool groups_coupled = true;                   // structural: something couples the groups
    bool multi_stream = false;                    // the current run issues groups on their streams
    bool last_multi_stream = false;
    bool group_streams_allowed = true;            // hx_set_group_streams
    hipEvent_t ev_main = nullptr;
    hipEvent_t ev_stagger = nullptr;     // group g's first node pass of a run, awaited by group g+1
    bool stagger_next = false;           // the next grouped step starts the groups half a step apart
    int stagger_groups = 1;              // 0: all groups start together
    int group_turns = 1;                 // hx_set_group_turns: the groups' node passes take turns
    bool turns_prev = false;             // a grouped step of this run was issued (its passes are recorded)
    // time table
    std::vector<double> ttab;
    double* d_ttab = nullptr;
    DevSlot ttab_slot;
    int ttab_cap = 0;
    int ttab_up = 0;                 // entries of ttab already in d_ttab (the table only grows)
    // gap
    int* d_gap_src = nullptr;
    int* d_gap_inst = nullptr;
    // vecplay
    VecPlayDev* d_vecplay = nullptr;
    DevSlot vecplay_slot;
    std::vector<std::tuple<std::string, std::string, int>> vecplay_keys;
    bool vecplay_dirty = true;
    // recorder
    std::vector<std::pair<std::string, std::string>> mon_name;
    std::vector<int> mon_idx;
    std::vector<Ref> mon_ref;
    std::vector<int> mon_col;       // sample-buffer column of each monitor (grouped by cell group)
    bool mon_all_v = true;          // every monitor samples a node voltage
    std::vector<std::vector<double>> mon_data;
    double** d_mon_ptr = nullptr;
    double* d_mon_buf = nullptr;
    DevSlot mon_ptr_slot, mon_buf_slot;
    long long mon_buf_cap = 0;     // samples
    long long mon_buf_fill = 0;
    bool mon_dirty = true;
    // handles
    std::vector<Ref> handles;
    // spike output (host)
    std::vector<std::pair<double, int>> spikes;
    // Spikes logged by the detection that follows a call's last step carry the time t the
    // next step starts at; the reference detects them at the start of that step, so they
    // are published once a step has been taken past them (finitialize's, at t = 0, at once).
    std::vector<std::pair<double, int>> spikes_held;
    std::unordered_map<int, std::vector<double>> spk_by_gid;
    // time stepping
    double t = 0.0;
    int k = 0;                       // step index since finitialize
    bool state_pending = false;
    // A run/continue_run/fadvance call may end with its last state update still pending
    // (close_deferral, default on): the next call's first node pass applies it as every
    // step applies the previous one, and any other entry point first completes it with
    // the closing pass the call would have run (settle).  Only those three entry points
    // set defer_allowed around their steps.
    bool close_deferral = true;
    bool defer_allowed = false;
    bool pending_sampled = false;   // the pending step's (voltage) samples are already recorded
    // A call that may defer its closing pass, on a model whose density mechanisms all run
    // in the node kernel, also leaves that kernel's assigned outputs of its last step
    // (ina, ica, i, ion cur and erev, ...) unstored (lazy_outputs_run); they are made when
    // something reads them (outputs_pending, settle) by an outputs-only node pass over the
    // last step's voltages, which the solve keeps in w, and its states, still pending.
    bool lazy_outputs_run = false;
    bool outputs_pending = false;
    bool final_step = false;   // the last step of a run call also stores every assigned variable
    bool initialized = false;
    // adjoint tape (hx_tape_begin): row n holds v^{n+1} (after step n's solve); the
    // states step n's current pass used: hh, Ca_HVA and hd_la gates, cai per ca_ion
    // instance, ExpSyn g_eff and Exp2Syn A_eff, B_eff (events of the step included);
    // and the synapse instances that received events at step n.  v^0 is kept apart.
    bool tape_on = false;
    int tape_cap = 0, tape_n = 0, tape_evcap = 0;
    double *d_tape_v = nullptr, *d_tape_x = nullptr, *d_tape_g = nullptr;
    int *d_tape_evn = nullptr, *d_tape_ev = nullptr;
    // adjoint work arrays and per-instance gradients (hx_adjoint)
    double *d_adj_delta = nullptr, *d_lv = nullptr, *d_lv2 = nullptr, *d_lx = nullptr, *d_lg = nullptr,
           *d_dT = nullptr, *d_rhsT = nullptr, *d_vT = nullptr, *d_wT = nullptr;
    // per-instance gradients of the trainable parameters (kTrainable order)
    double* d_grad[kNumTrainable] = {};
    // extra tape rows and adjoint work arrays of Ca_HVA, hd_la, CaDynamics_E2 and Exp2Syn
    double *d_tape_v0 = nullptr, *d_tape_c = nullptr, *d_tape_l = nullptr, *d_tape_cai = nullptr,
           *d_tape_ab = nullptr;
    double *d_lc = nullptr, *d_ll = nullptr, *d_lcai = nullptr, *d_lica = nullptr, *d_lab = nullptr;
    bool have_grad = false;
    bool adj_delta_dirty = true;
    struct AdamHost {
        int type = 2;        // 0 SGD, 1 momentum, 2 Adam
        double momentum = 0.9;
        double beta1 = 0.9, beta2 = 0.999, eps = 1e-8;
        long long step = 0;
        double* d_ext = nullptr;     // external gradients (one per registered weight)
        int n_ext = 0;
        std::vector<int> begin{0};
        std::vector<double*> w, g;
        std::vector<double> imp, m, v;
        bool dirty = true;
        int* d_begin = nullptr;
        double** d_w = nullptr;
        double** d_g = nullptr;
        double *d_imp = nullptr, *d_m = nullptr, *d_v = nullptr;
        DevSlot s_begin, s_w, s_g, s_imp, s_m, s_v;
    };
    std::vector<AdamHost> adams;
    // gap junctions added at run time (Simulate::add_gap_source/target, simulate.cpp:998-1100)
    struct GapMeta {
        std::string mech, var;
        int idx = 0;
        std::vector<std::tuple<std::string, std::string, int>> targets;
    };
    std::map<int, GapMeta> gap_meta;
    int next_sid = 0;
    std::vector<double*> dg_src, dg_dst;
    double** d_dg_src = nullptr;
    double** d_dg_dst = nullptr;
    DevSlot dg_src_slot, dg_dst_slot;
    bool dg_dirty = false;
    bool static_gaps_on = true;       // cleared by hx_clear_all_gap_junctions
    void launch_gap_transfers();
    // spk.dat after each run call (SimWrapper::run / continue_run, SimWrapper.cpp:46-84)
    bool spike_output = false;
    std::string output_dir = "output";          // Simulate's default (simulate.cpp:30)
    int after_run();
    void ensure_grad_arrays();
    int opt_add_group(int opt, const std::vector<double*>& w, const std::vector<double*>& g, double impedance);
    void tape_free() {
        for (void* p : {static_cast<void*>(d_tape_v), static_cast<void*>(d_tape_x), static_cast<void*>(d_tape_g),
                        static_cast<void*>(d_tape_evn), static_cast<void*>(d_tape_ev), static_cast<void*>(d_tape_v0),
                        static_cast<void*>(d_tape_c), static_cast<void*>(d_tape_l), static_cast<void*>(d_tape_cai),
                        static_cast<void*>(d_tape_ab)})
            if (p) (void)hipFree(p);
        d_tape_v = d_tape_x = d_tape_g = nullptr;
        d_tape_v0 = d_tape_c = d_tape_l = d_tape_cai = d_tape_ab = nullptr;
        d_tape_evn = d_tape_ev = nullptr;
        tape_cap = 0;
    }
    void tape_record();
    TapeCopy tape_row(bool syn) const;
    double grad_sq(int which);
    // profiling
    bool profiling = false;
    unsigned prof_mask = ~0u;   // timed kernel classes (bit = TimerId)
    Timer timers[T_COUNT];

    // learn gradient surface (capture + LRDS replay), created on first use
    std::unique_ptr<LearnRuntime> learn;
    // monitor samples appended to <output_dir>/sim_out.h5 after every call that syncs them
    bool h5_on = false;
    std::unique_ptr<H5Recorder> h5;
    std::vector<size_t> h5_written;            // samples of each monitor already in the file
    void h5_append();
    LearnRuntime& learn_rt() {
        if (!learn) learn.reset(new LearnRuntime(stream));
        return *learn;
    }
    void require_sample_point(const Ref& r);
    void mirror_ab(const Ref& r, double value);

    ~hx_sim() {
        learn.reset();
        tape_free();
        for (auto& g : groups) {
            if (g.done) (void)hipEventDestroy(g.done);
            if (g.pass) (void)hipEventDestroy(g.pass);
            if (g.s) (void)hipStreamDestroy(g.s);
        }
        if (ev_main) (void)hipEventDestroy(ev_main);
        if (ev_stagger) (void)hipEventDestroy(ev_stagger);
        for (auto& tm : timers)
            for (auto e : tm.pool) (void)hipEventDestroy(e);
        for (void* p : owned) (void)hipFree(p);
        if (h_status) (void)hipHostFree(h_status);
        if (h_mon) (void)hipHostFree(h_mon);
        if (stream) (void)hipStreamDestroy(stream);
    }

    // drops what the model builder holds (a failed read of an export)
    void reset_model(size_t keep_vecplay) {
        ncell = nnode = 0;
        parent.clear(); a.clear(); b.clear(); area.clear(); cm.clear();
        for (int k = 0; k < M_COUNT; ++k) {
            mech[k] = HostMech();
            globals[k].clear();
        }
        pre_gid.clear(); pre_node.clear(); pre_thr.clear();
        vecstim.clear();
        vecstim_run.clear();
        vecstim_run_differs = false;
        netcons.clear();
        gaps.clear();
        if (vecplay.size() > keep_vecplay) vecplay.resize(keep_vecplay);
    }

    int fail(const char* fmt, ...) {
        char buf[1024];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof(buf), fmt, ap);
        va_end(ap);
        err = buf;
        return -1;
    }

    // ------------------------------------------------------------ timing
    void tbegin(int id, hipStream_t on = nullptr) {
        if (!profiling || !(prof_mask & (1u << id))) return;
        Timer& tm = timers[id];
        while (tm.pool.size() < tm.used + 2) {
            hipEvent_t e;
            HXC(hipEventCreate(&e));
            tm.pool.push_back(e);
        }
        HXC(hipEventRecord(tm.pool[tm.used], on ? on : stream));
        tm.pending.push_back({static_cast<int>(tm.used), static_cast<int>(tm.used + 1)});
        tm.used += 2;
    }
    // A start/end pair for a launch that sets them itself as part of its dispatch
    // (hipExtLaunchKernel): false, and no events, when the class is not timed.  The pair
    // counts once tcommit says the launch happened.
    bool treserve(int id, hipEvent_t& e0, hipEvent_t& e1) {
        e0 = e1 = nullptr;
        if (!profiling || !(prof_mask & (1u << id))) return false;
        Timer& tm = timers[id];
        while (tm.pool.size() < tm.used + 2) {
            hipEvent_t e;
            HXC(hipEventCreate(&e));
            tm.pool.push_back(e);
        }
        e0 = tm.pool[tm.used];
        e1 = tm.pool[tm.used + 1];
        return true;
    }
    void tcommit(int id) {
        Timer& tm = timers[id];
        tm.pending.push_back({static_cast<int>(tm.used), static_cast<int>(tm.used + 1)});
        tm.used += 2;
    }
    // returns the event recorded (nullptr when the class is not timed)
    hipEvent_t tend(int id, hipStream_t on = nullptr) {
        if (!profiling || !(prof_mask & (1u << id))) return nullptr;
        Timer& tm = timers[id];
        hipEvent_t e = tm.pool[tm.pending.back().second];
        HXC(hipEventRecord(e, on ? on : stream));
        return e;
    }
    void tcollect() {
        for (auto& tm : timers) {
            for (auto& pr : tm.pending) {
                float ms = 0;
                HXC(hipEventElapsedTime(&ms, tm.pool[pr.first], tm.pool[pr.second]));
                tm.ms += ms;
                tm.launches++;
            }
            tm.pending.clear();
            tm.used = 0;
        }
    }

    // ------------------------------------------------------------ layout
    void build_layout();
    void recompute_fused();
    bool node_kernel_owns_matrix() const;
    void upload();
    void upload_inputs();
    void upload_vecplay();
    void upload_monitors();
    void ensure_ttab(int kneed);
    void ensure_mon_rows(long long rows);
    Ref resolve(const std::string& mechname, const std::string& var, int idx);
    StepArgs step_args(double tcur, int do_state, int do_current) const;
    unsigned ion_store_bits(bool assigned) const;
    // ------------------------------------------------------------ stepping
    void launch_mech_pass(int do_state, int do_current, double tcur, int grp = -1, hipStream_t on = nullptr);
    void launch_point_currents(double tcur);
    // vp_t >= 0: the delivery launch also runs VecPlay at time vp_t (and returns true)
    bool launch_events(int kk, double tk, double vp_t = -1.0);
    bool launch_events_group(int g, int kk, double tk, hipStream_t on, double vp_t = -1.0);
    InputArgs input_args(int g, int kk, double tk) const;
    DeliverArgs deliver_args(int kk, double vp_t) const;
    int deliver_blocks(int cap) const { return pre_fanout_empty ? 1 : std::min(64, (cap + 8191) / 8192); }
    void launch_detect(int kk, double tk);
    void launch_record();
    void build_groups(const std::vector<std::vector<std::pair<int, double>>>& vs_fo, long long ntgt);
    bool want_multi_stream() const;
    // The tree solve leaves the pivots in d and the solution x in rhs, as the reference
    // does, on the last step of a call (read back through the API) and on every step
    // when a handle, monitor or transfer may read them; otherwise neither is stored.
    bool store_dx() const { return final_step || write_assigned || !dg_src.empty(); }
    void step_once_groups();
    void step_once();
    void finish_pending();
    bool can_defer_close() const;
    bool close_may_defer() const;
    bool lazy_outputs_ok() const;
    void launch_outputs_pass();
    void sample_pending_step();
    int settle();
    int run_steps(int nstep);
    void sync_outputs();
    void finitialize(double v_init);
};

void* hx_sim::slot_reserve(DevSlot& s, size_t bytes) {
    bytes = std::max<size_t>(bytes, 1);
    if (s.p && s.bytes >= bytes) return s.p;
    if (s.p) {
        HXC(hipStreamSynchronize(stream));     // queued kernels may still read the old block
        owned.erase(std::find(owned.begin(), owned.end(), s.p));
        void* old = s.p;
        s.p = nullptr;
        s.bytes = 0;
        HXC(hipFree(old));
    }
    HXC(hipMalloc(&s.p, bytes));
    owned.push_back(s.p);
    s.bytes = bytes;
    return s.p;
}

template <class T>
T* hx_sim::slot_upload(DevSlot& s, const std::vector<T>& h) {
    T* p = static_cast<T*>(slot_reserve(s, h.size() * sizeof(T)));
    if (!h.empty()) {
        HXC(hipStreamSynchronize(stream));     // queued kernels may still read the block
        HXC(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    }
    return p;
}

// ===========================================================================
// layout
// ===========================================================================
namespace {

// Midpoint of the longest path of a tree given by parent links (parent < child).
int tree_centre(const std::vector<int>& lp) {
    const int n = static_cast<int>(lp.size());
    if (n <= 2) return 0;
    std::vector<std::vector<int>> adj(n);
    for (int j = 1; j < n; ++j) {
        adj[j].push_back(lp[j]);
        adj[lp[j]].push_back(j);
    }
    std::vector<int> dist(n), prev(n);
    auto bfs = [&](int s) {
        std::fill(dist.begin(), dist.end(), -1);
        std::vector<int> q{s};
        dist[s] = 0;
        prev[s] = -1;
        int far = s;
        for (size_t h = 0; h < q.size(); ++h) {
            const int u = q[h];
            if (dist[u] > dist[far]) far = u;
            for (int w : adj[u])
                if (dist[w] < 0) {
                    dist[w] = dist[u] + 1;
                    prev[w] = u;
                    q.push_back(w);
                }
        }
        return far;
    };
    const int x = bfs(0);
    const int y = bfs(x);
    std::vector<int> path;
    for (int u = y; u >= 0; u = prev[u]) path.push_back(u);
    return path[path.size() / 2];
}

// Re-root a tree at `root`: bfs lists the nodes in BFS order, and spl[j] is
// the parent of bfs[j] as an index into bfs (-1 for the root), so parent < child.
void reroot_tree(const std::vector<int>& lp, int root, std::vector<int>& bfs, std::vector<int>& spl) {
    const int n = static_cast<int>(lp.size());
    std::vector<std::vector<int>> adj(n);
    for (int j = 1; j < n; ++j) {
        adj[j].push_back(lp[j]);
        adj[lp[j]].push_back(j);
    }
    std::vector<int> label(n, -1);
    bfs.assign(1, root);
    spl.assign(1, -1);
    label[root] = 0;
    for (size_t h = 0; h < bfs.size(); ++h) {
        const int u = bfs[h];
        for (int w : adj[u])
            if (label[w] < 0) {
                label[w] = static_cast<int>(bfs.size());
                bfs.push_back(w);
                spl.push_back(static_cast<int>(h));
            }
    }
}

}  // namespace

void hx_sim::build_layout() {
    const auto& R = registry();
    // per-cell node lists (user order, increasing)
    std::vector<int> cell_of(nnode);
    for (int i = 0; i < ncell; ++i) cell_of[i] = i;
    for (int i = ncell; i < nnode; ++i) cell_of[i] = cell_of[parent[i]];
    std::vector<int> cnt(ncell, 0);
    for (int i = 0; i < nnode; ++i) cnt[cell_of[i]]++;
    std::vector<int> cbeg(ncell + 1, 0);
    for (int c = 0; c < ncell; ++c) cbeg[c + 1] = cbeg[c] + cnt[c];
    std::vector<int> cnodes(nnode), fill(cbeg.begin(), cbeg.end() - 1);
    for (int i = 0; i < nnode; ++i) cnodes[fill[cell_of[i]]++] = i;   // increasing user index per cell
    std::vector<int> local(nnode);
    // The solve may eliminate toward any node of a cell: the matrix and its
    // solution do not depend on the root, and the axial assembly is the same
    // once a and b trade places on every reversed edge.  Each cell is rooted at
    // the midpoint of its longest path, which shortens the chain of rounds
    // (config 3: 62 -> about 48).
    solve_parent.assign(nnode, -1);
    solve_a.assign(nnode, 0.0);
    solve_b.assign(nnode, 0.0);
    std::vector<std::vector<int>> cbfs(ncell), cspl(ncell);   // per cell: BFS order, solver-local parents
    for (int c = 0; c < ncell; ++c) {
        const int n = cnt[c];
        std::vector<int> lp(n);
        for (int j = 0; j < n; ++j) local[cnodes[cbeg[c] + j]] = j;
        for (int j = 0; j < n; ++j) {
            const int u = cnodes[cbeg[c] + j];
            lp[j] = (j == 0) ? -1 : local[parent[u]];
        }
        // solver tree: BFS from the root, relabelled so that parent < child
        const int root = solve_root_centre ? tree_centre(lp) : 0;
        std::vector<int>& bfs = cbfs[c];
        std::vector<int>& spl = cspl[c];
        reroot_tree(lp, root, bfs, spl);
        for (int j = 0; j < n; ++j) {
            if (spl[j] < 0) continue;
            const int u = cnodes[cbeg[c] + bfs[j]];
            const int q = cnodes[cbeg[c] + bfs[spl[j]]];
            solve_parent[u] = q;
            if (parent[u] == q) {          // same orientation as the model's tree
                solve_a[u] = a[u];
                solve_b[u] = b[u];
            } else {                       // reversed edge: the coefficients of q's old link trade places
                solve_a[u] = b[q];
                solve_b[u] = a[q];
            }
        }
    }
    // Solve units: runs of consecutive cells, each solved by one wavefront as
    // a forest.  By default a unit holds about ncell / kSolveUnitTarget cells,
    // so the whole solve runs about one wavefront per SIMD; a unit whose
    // schedule would need more than kUnitLdsBudget of LDS is split further.
    auto build_units = [&](int U) {
        node_perm.assign(nnode, -1);
        node_iperm.assign(nnode, -1);
        nunit = (ncell + U - 1) / U;
        unit_cell_begin.assign(nunit + 1, 0);
        unit_node_begin.assign(nunit + 1, 0);
        unit_desc_begin.assign(nunit + 1, 0);
        unit_round_begin.assign(nunit + 1, 0);
        rounds.clear();
        descs.clear();
        max_slots = 0;
        max_rounds = 0;
        int pos = 0;
        for (int k = 0; k < nunit; ++k) {
            const int c0 = k * U, c1 = std::min(ncell, c0 + U);
            std::vector<int> fp;                 // forest parents, cells one after another
            std::vector<int> fnode;              // forest index -> user node
            for (int c = c0; c < c1; ++c) {
                const int off = static_cast<int>(fp.size());
                for (size_t j = 0; j < cbfs[c].size(); ++j) {
                    fp.push_back(cspl[c][j] < 0 ? -1 : off + cspl[c][j]);
                    fnode.push_back(cnodes[cbeg[c] + cbfs[c][j]]);
                }
            }
            UnitSchedule us;
            build_unit_schedule(fp, kChunk, kWave, kRoundMax, us);
            if (U > 1 && solve_lds_bytes(us.nchunk) > kUnitLdsBudget) return false;
            unit_cell_begin[k] = c0;
            unit_node_begin[k] = pos;
            unit_desc_begin[k] = static_cast<int>(descs.size());
            unit_round_begin[k] = static_cast<int>(rounds.size());
            const int n = static_cast<int>(fp.size());
            for (int s = 0; s < n; ++s) {
                const int u = fnode[us.order[s]];
                node_perm[u] = pos + s;
                node_iperm[pos + s] = u;
            }
            pos += n;
            for (auto& d : us.desc) descs.push_back(d);
            for (auto& r : us.rounds) rounds.push_back(r);
            max_slots = std::max(max_slots, us.nchunk);
            max_rounds = std::max(max_rounds, us.nround);
        }
        unit_cell_begin[nunit] = ncell;
        unit_node_begin[nunit] = pos;
        unit_desc_begin[nunit] = static_cast<int>(descs.size());
        unit_round_begin[nunit] = static_cast<int>(rounds.size());
        return true;
    };
    int U = unit_request > 0 ? unit_request
                             : std::max(1, static_cast<int>(std::lround(static_cast<double>(ncell) / kSolveUnitTarget)));
    U = std::max(1, std::min(U, ncell));
    while (!build_units(U)) {
        if (unit_request > 0)
            throw std::runtime_error("solve units of " + std::to_string(U) + " cells need more than " +
                                     std::to_string(kUnitLdsBudget) + " B of LDS; use fewer cells per unit");
        U = std::max(1, U / 2);
    }
    unit_cells = U;

    // mechanism instance order: by solver-order node (stable); artificial cells
    // sit on no node and keep their own order
    for (int id = 0; id < M_COUNT; ++id) {
        HostMech& m = mech[id];
        if (!m.present) continue;
        std::vector<int> idx(m.n);
        std::iota(idx.begin(), idx.end(), 0);
        if (!R[id].artificial)
            std::stable_sort(idx.begin(), idx.end(),
                             [&](int x, int y) { return node_perm[m.node[x]] < node_perm[m.node[y]]; });
        m.iperm = idx;
        m.perm.assign(m.n, 0);
        for (int j = 0; j < m.n; ++j) m.perm[idx[j]] = j;
        m.dense = false;
        if (!R[id].point && !R[id].artificial && m.n == nnode) {
            bool ok = true;
            for (int j = 0; j < m.n && ok; ++j) ok = node_perm[m.node[idx[j]]] == j;
            m.dense = ok;
        }
    }
    for (auto& p : plugins) {
        HostMech& m = p.h;
        std::vector<int> idx(m.n);
        std::iota(idx.begin(), idx.end(), 0);
        std::stable_sort(idx.begin(), idx.end(), [&](int x, int y) { return node_perm[m.node[x]] < node_perm[m.node[y]]; });
        m.iperm = idx;
        m.perm.assign(m.n, 0);
        for (int j = 0; j < m.n; ++j) m.perm[idx[j]] = j;
    }
    // a mechanism that reads an ion can be fused only if the ion is dense too
    dense_mask = 0;
    for (int id = 0; id < M_COUNT; ++id) {
        HostMech& m = mech[id];
        if (!m.present || !m.dense) continue;
        int use = R[id].ion_use;
        bool ok = true;
        if ((use & 1) && !mech[M_NA_ION].dense) ok = false;
        if ((use & 2) && !mech[M_K_ION].dense) ok = false;
        if ((use & 4) && !mech[M_CA_ION].dense) ok = false;
        if (ok) dense_mask |= 1u << id;
        else m.dense = false;
    }
    // A sparse hh whose na and k currents no other mechanism adds to stores them itself
    // instead of adding to currents the ion kernels zeroed, and the two ion launches are
    // left out of the stepping current passes (with no 0100 style there is nothing else for
    // them to do; ion instances without hh keep the 0 the finitialize pass stored).
    {
        auto plain_ion = [&](int id) {
            const HostMech& m = mech[id];
            if (!m.present || (dense_mask & (1u << id))) return false;
            for (int t : m.iontype)
                if (t & 0100) return false;
            return true;
        };
        hh_owns_ions = mech[M_HH].present && mech[M_HH].n > 0 && !(dense_mask & (1u << M_HH)) &&
                       plain_ion(M_NA_ION) && plain_ion(M_K_ION) && !(plugin_ions() & 3u);
    }
    recompute_fused();
}

// the density mechanisms in the order of their kernels when they are not fused
static const int kSparseOrder[] = {M_PAS, M_NA_ION, M_K_ION, M_HH, M_CA_ION, M_CADYN, M_CAHVA, M_HDLA};

// Fusing the state update of step k-1 into the current pass of step k is exact
// unless something observes or changes density-mechanism values between the two.
void hx_sim::recompute_fused() {
    const auto& R = registry();
    bool fuse = fusion_allowed != 0;
    if (mech[M_CADYN].present && !(dense_mask & (1u << M_CADYN))) fuse = false;
    for (auto& vp : vecplay) {
        int id = mech_id(vp.mech);
        if (id >= 0 && !R[id].point) fuse = false;
        if (id < 0) fuse = false;   // node / capacitance variables
    }
    if (need_split_for_monitor) fuse = false;
    fused = fuse;
    solve_voltage = solve_voltage_allowed && node_kernel_owns_matrix();
}

// True when a stepping current pass takes every term of d and rhs from the node kernel:
// no density mechanism on a kernel of its own, no IClamp or HalfGap instance (synapses are
// folded into the node kernel), no plugin.  The node kernel can then store rhs + d v, and
// the solve yields the new voltage without reading v: (D + L) x = r - L v, with D the node
// kernel's diagonal and L the axial couplings, is (D + L) v_new = r + D v.
bool hx_sim::node_kernel_owns_matrix() const {
    if (dense_mask == 0 || !plugins.empty()) return false;
    for (int id : kSparseOrder)
        if (mech[id].present && !(dense_mask & (1u << id))) return false;
    for (int id : {M_ICLAMP, M_HALFGAP})
        if (mech[id].present && mech[id].n > 0) return false;
    return true;
}

// CaDynamics_E2's state depends on ica and cai only, so in the fused schedule
// the current pass that computes ica can apply the step's update at once (one
// calcium read and write per step instead of also storing and reloading ica).
// Exact unless something samples calcium between the current and state passes:
// a monitor on ca_ion or CaDynamics_E2, taping or signal capture.
void hx_sim::refresh_cadyn_eager() {
    bool ok = fused && mech[M_CADYN].present && (dense_mask & (1u << M_CADYN)) && !tape_on &&
              !(learn && learn->capturing()) && !(plugin_ions() & plugin::kCa);   // a plugin's ica comes later
    for (size_t i = 0; ok && i < mon_name.size(); ++i)
        if (mon_name[i].first == "ca_ion" || mon_name[i].first == "CaDynamics_E2") ok = false;
    cadyn_eager = ok;
}

void hx_sim::upload() {
    point_grp_node[0].clear();
    point_grp_node[1].clear();
    const auto& R = registry();
    if (!stream) HXC(hipStreamCreate(&stream));
    auto perm_nodes = [&](const std::vector<double>& u) {
        std::vector<double> g(nnode);
        for (int i = 0; i < nnode; ++i) g[node_perm[i]] = u[i];
        return g;
    };
    d_v = dalloc<double>(owned, nnode);
    d_d = dalloc<double>(owned, nnode);
    d_rhs = dalloc<double>(owned, nnode);
    HXC(hipMemset(d_v, 0, sizeof(double) * nnode));
    HXC(hipMemset(d_d, 0, sizeof(double) * nnode));
    HXC(hipMemset(d_rhs, 0, sizeof(double) * nnode));
    d_w = dalloc<double>(owned, nnode);
    d_a = dupload(owned, perm_nodes(a));
    d_b = dupload(owned, perm_nodes(b));
    d_sa = dupload(owned, perm_nodes(solve_a));
    d_sb = dupload(owned, perm_nodes(solve_b));
    d_cm = dupload(owned, perm_nodes(cm));
    cm_uniform = nnode > 0;
    for (int i = 1; i < nnode && cm_uniform; ++i) cm_uniform = std::memcmp(&cm[i], &cm[0], sizeof(double)) == 0;
    cm_value = nnode > 0 ? cm[0] : 0.0;
    d_area = dupload(owned, perm_nodes(area));
    d_unit_node_begin = dupload(owned, unit_node_begin);
    d_unit_desc_begin = dupload(owned, unit_desc_begin);
    d_unit_round_begin = dupload(owned, unit_round_begin);
    d_rounds = dupload(owned, rounds);
    d_desc = dupload(owned, descs);
    {
        int dev = 0;
        hipDeviceProp_t prop;
        HXC(hipGetDevice(&dev));
        HXC(hipGetDeviceProperties(&prop, dev));
        const size_t lds = solve_lds_bytes(max_slots);
        if (lds > prop.sharedMemPerBlock)
            throw std::runtime_error("a solve unit has " + std::to_string(max_slots) + " chunks; its " + std::to_string(lds) +
                                     " B solver schedule exceeds the " + std::to_string(prop.sharedMemPerBlock) +
                                     " B of LDS per workgroup");
        // units small enough are held whole in LDS (k_solve_res), the others streamed
        int max_unit_nodes = 0;
        for (int u = 0; u < nunit; ++u)
            max_unit_nodes = std::max(max_unit_nodes, unit_node_begin[u + 1] - unit_node_begin[u]);
        const size_t rlds = res_lds_bytes(max_unit_nodes, max_slots, max_rounds);
        const bool resident = solve_resident_allowed && rlds <= kResUnitBudget && rlds <= prop.sharedMemPerBlock;
        res_nodes = resident ? max_unit_nodes : 0;
        // as many units per workgroup as asked (default kSolveMaxWaves) and the LDS allows
        const int want = solve_waves_request > 0 ? solve_waves_request : kSolveMaxWaves;
        const size_t unit_lds = resident ? rlds : lds;
        solve_waves = std::max(1, std::min<int>(want, static_cast<int>(prop.sharedMemPerBlock / unit_lds)));
    }

    // ion node -> device instance maps
    const int ion_ids[3] = {M_NA_ION, M_K_ION, M_CA_ION};
    for (int x = 0; x < 3; ++x) {
        ion_at[x].assign(nnode, -1);
        HostMech& im = mech[ion_ids[x]];
        if (!im.present) continue;
        for (int j = 0; j < im.n; ++j) ion_at[x][node_perm[im.node[im.iperm[j]]]] = j;
    }
    // plugin mechanisms: columns in device instance order, solver-order nodes, and the
    // instances of the ions they use (which must be present on their nodes)
    for (auto& p : plugins) {
        HostMech& m = p.h;
        MechDev& d = m.dev;
        d = MechDev();
        d.n = m.n;
        d.stride = ((m.n + 63) / 64) * 64;
        const int ncol = p.meta->ncol;
        std::vector<double> blk(static_cast<size_t>(std::max(ncol, 1)) * std::max<long long>(d.stride, 1), 0.0);
        for (int c = 0; c < ncol; ++c)
            for (int j = 0; j < m.n; ++j) blk[c * d.stride + j] = m.col[c][m.iperm[j]];
        d.base = dupload(owned, blk);
        std::vector<int> nodes(m.n);
        for (int j = 0; j < m.n; ++j) nodes[j] = node_perm[m.node[m.iperm[j]]];
        d.node = dupload(owned, nodes);
        const unsigned use = p.meta->ion_read | p.meta->ion_write;
        static const char* ion_names[3] = {"na_ion", "k_ion", "ca_ion"};
        for (int x = 0; x < 3; ++x) {
            if (!(use & (1u << x))) continue;
            std::vector<int> map(m.n);
            for (int j = 0; j < m.n; ++j) {
                map[j] = ion_at[x][nodes[j]];
                if (map[j] < 0)
                    throw std::runtime_error(std::string(p.meta->name) + " uses " + ion_names[x] + ", which node " +
                                             std::to_string(m.node[m.iperm[j]]) + " does not have");
            }
            d.ion[x] = dupload(owned, map);
        }
    }
    std::vector<double> uval_host(static_cast<size_t>(M_COUNT) * kUniformCols, 0.0);
    for (int id = 0; id < M_COUNT; ++id) {
        HostMech& m = mech[id];
        MechDev& d = m.dev;
        d = MechDev();
        if (!m.present) continue;
        d.n = m.n;
        d.dense = m.dense ? 1 : 0;
        const int ncol = R[id].ncol;
        d.stride = ((m.n + 63) / 64) * 64;
        if (ncol > 0) {
            std::vector<double> blk(static_cast<size_t>(ncol) * d.stride, 0.0);
            for (int c = 0; c < ncol; ++c)
                for (int j = 0; j < m.n; ++j) blk[c * d.stride + j] = m.col[c][m.iperm[j]];
            d.base = dupload(owned, blk);
        }
        // parameters holding one value, for the mechanisms whose parameters the node
        // kernels read through ldp (ion columns may be written by kernels; point
        // processes read theirs elsewhere): compared bit for bit, so a uniform
        // column is exactly its value
        const bool scalar_reads = id == M_PAS || id == M_HH || id == M_HDLA || id == M_CAHVA || id == M_CADYN;
        if (R[id].ion && m.n > 0) {
            // the node kernel reads an ion's erev, or its conco when the style has 0100
            // (Nernst each step); erev is written by kernels under styles 040 (init) and
            // 0100, conco under 04 (init); conci is a state of calcium dynamics
            int any = 0;
            for (int t : m.iontype) any |= t;
            const int cols[2] = {ION_EREV, ION_CONCO};
            const bool ok[2] = {!(any & (040 | 0100)), (any & 0100) != 0};
            // conco as the steps read it: finitialize sets it to the ion's default outside
            // concentration where the style has 04 (k_init), and nothing writes it after that
            const int x = id == M_NA_ION ? 0 : id == M_K_ION ? 1 : 2;
            std::vector<double> after_init(m.col[ION_CONCO]);
            for (int j = 0; j < m.n; ++j)
                if (m.iontype[j] & 04) after_init[j] = kIonConcoInit[x];
            for (int k = 0; k < 2; ++k) {
                if (!ok[k]) continue;
                const int c = cols[k];
                const std::vector<double>& col = c == ION_CONCO ? after_init : m.col[c];
                const double x0 = col[0];
                bool same = true;
                for (int j = 1; j < m.n && same; ++j) same = std::memcmp(&col[j], &x0, sizeof(double)) == 0;
                if (same) {
                    d.umask |= 1u << c;
                    uval_host[static_cast<size_t>(id) * kUniformCols + c] = x0;
                }
            }
        }
        if (scalar_reads && m.n > 0)
            for (int c = 0; c < std::min(R[id].nparam, kUniformCols); ++c) {
                const double x0 = m.col[c][0];
                bool same = true;
                for (int j = 1; j < m.n && same; ++j) same = std::memcmp(&m.col[c][j], &x0, sizeof(double)) == 0;
                if (same) {
                    d.umask |= 1u << c;
                    uval_host[static_cast<size_t>(id) * kUniformCols + c] = x0;
                }
            }
        std::vector<int> nodes(m.n);
        for (int j = 0; j < m.n; ++j) nodes[j] = node_perm[m.node[m.iperm[j]]];
        d.node = dupload(owned, nodes);
        if (id == M_EXPSYN) syn_node[0] = nodes;
        if (id == M_EXP2SYN) syn_node[1] = nodes;
        inst_node[id].clear();
        if (!m.dense) inst_node[id] = nodes;
        if (R[id].point && m.n > 0) {
            std::vector<int> gnode, gbeg;
            for (int j = 0; j < m.n; ++j)
                if (j == 0 || nodes[j] != nodes[j - 1]) {
                    gnode.push_back(nodes[j]);
                    gbeg.push_back(j);
                }
            gbeg.push_back(m.n);
            d.ngrp = static_cast<int>(gnode.size());
            d.grp_node = dupload(owned, gnode);
            d.grp_begin = dupload(owned, gbeg);
            if (id == M_ICLAMP) point_grp_node[0] = gnode;
            if (id == M_HALFGAP) point_grp_node[1] = gnode;
            if (id == M_EXPSYN || id == M_EXP2SYN) {
                const int nblk = (nnode + kBlock - 1) / kBlock;
                std::vector<int> bb(nblk + 1);
                for (int b = 0; b <= nblk; ++b)
                    bb[b] = static_cast<int>(std::lower_bound(nodes.begin(), nodes.end(), b * kBlock) - nodes.begin());
                d.blk_begin = dupload(owned, bb);
            }
        }
        if (R[id].ion) {
            std::vector<int> it(m.n);
            for (int j = 0; j < m.n; ++j) it[j] = m.iontype[m.iperm[j]];
            d.iontype = dupload(owned, it);
            const int x = id == M_NA_ION ? 0 : (id == M_K_ION ? 1 : 2);
            ion_type_uniform[x] = -1;
            if (m.n > 0 && std::all_of(it.begin(), it.end(), [&](int t) { return t == it[0]; }))
                ion_type_uniform[x] = it[0];
        }
        for (int x = 0; x < 3; ++x) {
            if (!(R[id].ion_use & (1 << x))) continue;
            std::vector<int> map(m.n);
            bool ident = true;
            for (int j = 0; j < m.n; ++j) {
                map[j] = ion_at[x][nodes[j]];
                if (map[j] < 0)
                    throw std::runtime_error(std::string(R[id].name) + " instance without " + R[ion_ids[x]].name +
                                             " at its node");
                ident = ident && map[j] == j;
            }
            if (!ident) d.ion[x] = dupload(owned, map);
        }
    }
    {
        const double* d_uval = dupload(owned, uval_host);
        for (int id = 0; id < M_COUNT; ++id) mech[id].dev.uval = d_uval + static_cast<size_t>(id) * kUniformCols;
    }

    // nodes carrying IClamp or HalfGap, with their group of each (the loop above made the
    // groups)
    point_union = PointUnion{};
    if (!point_grp_node[0].empty() && !point_grp_node[1].empty()) {
        std::vector<int> un;
        std::set_union(point_grp_node[0].begin(), point_grp_node[0].end(), point_grp_node[1].begin(),
                       point_grp_node[1].end(), std::back_inserter(un));
        std::vector<int> g[2];
        for (int x = 0; x < 2; ++x) {
            g[x].assign(un.size(), -1);
            const std::vector<int>& gn = point_grp_node[x];
            for (size_t q = 0; q < gn.size(); ++q)
                g[x][std::lower_bound(un.begin(), un.end(), gn[q]) - un.begin()] = static_cast<int>(q);
        }
        point_union.n = static_cast<int>(un.size());
        point_union.node = dupload(owned, un);
        point_union.grp[0] = dupload(owned, g[0]);
        point_union.grp[1] = dupload(owned, g[1]);
    }

    // spike detectors, in solver-node order so a cell group's detectors are a
    // contiguous range (the gid travels with each detector)
    npre = static_cast<int>(pre_node.size());
    std::vector<int> pre_dev(npre), pre_order(npre);
    std::iota(pre_order.begin(), pre_order.end(), 0);
    std::stable_sort(pre_order.begin(), pre_order.end(),
                     [&](int x, int y) { return node_perm[pre_node[x]] < node_perm[pre_node[y]]; });
    {
        std::vector<int> pn(npre), pg(npre);
        std::vector<double> pt(npre);
        for (int r = 0; r < npre; ++r) {
            const int u = pre_order[r];
            pre_dev[u] = r;
            pn[r] = node_perm[pre_node[u]];
            pg[r] = pre_gid[u];
            pt[r] = pre_thr[u];
        }
        h_pre_node_dev = pn;
        d_pre_node = dupload(owned, pn);
        d_pre_thr = dupload(owned, pt);
        d_pre_gid = dupload(owned, pg);
    }
    d_pre_flag = dalloc<int>(owned, npre);
    HXC(hipMemset(d_pre_flag, 0, sizeof(int) * std::max(npre, 1)));

    // netcons: the last one per synapse instance wins (coredat_to_innerdat.cpp:356-364)
    std::map<std::pair<int, int>, NetCon> by_syn;
    for (auto& nc : netcons) by_syn[{nc.mech, nc.inst}] = nc;
    // input sources: VecStim instances, then NetStim instances
    const int nvs = mech[M_VECSTIM].present ? mech[M_VECSTIM].n : 0;
    const int nns = mech[M_NETSTIM].present ? mech[M_NETSTIM].n : 0;
    // NetStims with an incoming netcon run on the device; the rest stay host-made trains
    ns_dyn.assign(nns, -1);
    ns_dyn_inst.clear();
    ns_dyn_w.clear();
    for (auto& kv : by_syn)
        if (kv.second.mech == M_NETSTIM) {
            ns_dyn[kv.second.inst] = static_cast<int>(ns_dyn_inst.size());
            ns_dyn_inst.push_back(kv.second.inst);
            ns_dyn_w.push_back(kv.second.weight);
        }
    const int ndyn = static_cast<int>(ns_dyn_inst.size());
    if (ndyn >= (1 << kNsRoundShift)) throw std::runtime_error("too many NetStims receive netcons");
    std::vector<std::vector<std::pair<int, double>>> pre_fo(npre), vs_fo(nvs + nns), dyn_fo(ndyn);
    std::vector<double> esw(mech[M_EXPSYN].present ? mech[M_EXPSYN].n : 0, 0.0);
    std::vector<double> e2w(mech[M_EXP2SYN].present ? mech[M_EXP2SYN].n : 0, 0.0);
    // synapse plugins: a slot each, and their instances' netcon weights and delays
    std::vector<std::vector<double>> plugin_w, plugin_delay;
    for (auto& p : plugins) {
        p.slot = -1;
        if (!(p.meta->flags & plugin::kPostsyn)) continue;
        p.slot = static_cast<int>(plugin_w.size());
        if (p.slot >= kMaxPostsyn)
            throw std::runtime_error("a model may use at most " + std::to_string(kMaxPostsyn) + " synapse plugins");
        if (p.h.n >= (1 << kPostsynSlotShift)) throw std::runtime_error("too many instances of a synapse plugin");
        plugin_w.emplace_back(p.h.n, 0.0);
        plugin_delay.emplace_back(p.h.n, 0.0);
    }
    max_delay = 0;
    for (auto& kv : by_syn) {
        const NetCon& nc = kv.second;
        int packed;
        if (nc.mech >= kPluginMechBase) {
            PluginInst& p = plugins[nc.mech - kPluginMechBase];
            const int dinst = p.h.perm[nc.inst];
            packed = pack_target(kTargetPlugin, (p.slot << kPostsynSlotShift) | dinst);
            plugin_w[p.slot][dinst] = nc.weight;
            plugin_delay[p.slot][dinst] = nc.delay;
        } else if (nc.mech == M_NETSTIM) {
            packed = pack_target(kTargetNetStim, ns_dyn[nc.inst]);
        } else {
            const int dinst = mech[nc.mech].perm[nc.inst];
            packed = pack_target(nc.mech == M_EXP2SYN ? 1 : 0, dinst);
            if (nc.mech == M_EXPSYN) esw[dinst] = nc.weight;
            else e2w[dinst] = nc.weight;
        }
        if (nc.src_kind == 0) pre_fo[pre_dev[nc.src]].push_back({packed, nc.delay});
        else if (nc.src_kind == 1) vs_fo[nc.src].push_back({packed, nc.delay});
        else if (ns_dyn[nc.src] >= 0) dyn_fo[ns_dyn[nc.src]].push_back({packed, nc.delay});
        else vs_fo[nvs + nc.src].push_back({packed, nc.delay});
        max_delay = std::max(max_delay, nc.delay);
    }
    // every packed target decodes to an instance of its kind (the kernels index with it)
    {
        const int nes = mech[M_EXPSYN].present ? mech[M_EXPSYN].n : 0;
        const int ne2 = mech[M_EXP2SYN].present ? mech[M_EXP2SYN].n : 0;
        auto check = [&](const std::vector<std::vector<std::pair<int, double>>>& fo) {
            for (const auto& v : fo)
                for (const auto& pr : v) {
                    const int kind = target_kind(pr.first);
                    int inst = target_inst(pr.first), lim = 0;
                    if (kind == 0) lim = nes;
                    else if (kind == 1) lim = ne2;
                    else if (kind == kTargetNetStim) lim = ndyn;
                    else {
                        const int slot = inst >> kPostsynSlotShift;
                        inst &= (1 << kPostsynSlotShift) - 1;
                        for (const auto& p : plugins)
                            if (p.slot == slot) lim = p.h.n;
                    }
                    if (inst < 0 || inst >= lim) throw std::runtime_error("internal: bad fan-out target");
                }
        };
        check(pre_fo);
        check(vs_fo);
        check(dyn_fo);
    }
    long long ntgt = 0;
    {
        std::vector<int> b(pre_fo.size() + 1, 0), tg;
        std::vector<double> de;
        for (size_t i = 0; i < pre_fo.size(); ++i) {
            for (auto& pr : pre_fo[i]) { tg.push_back(pr.first); de.push_back(pr.second); }
            b[i + 1] = static_cast<int>(tg.size());
        }
        d_pre_fo_begin = dupload(owned, b);
        d_pre_fo_target = dupload(owned, tg);
        d_pre_fo_delay = dupload(owned, de);
        ntgt += static_cast<long long>(tg.size());
        pre_fanout_empty = tg.empty();
    }
    d_es_weight = dupload(owned, esw);
    d_e2_weight = dupload(owned, e2w);
    for (auto& p : plugins) {
        if (p.slot < 0) continue;
        p.d_recv_w = dupload(owned, plugin_w[p.slot]);
        p.d_recv_delay = dupload(owned, plugin_delay[p.slot]);
        p.d_recv_count = dalloc<int>(owned, std::max(p.h.n, 1));
        HXC(hipMemset(p.d_recv_count, 0, sizeof(int) * std::max(p.h.n, 1)));
    }
    nsa = NsArgs{};
    nsa.n = ndyn;
    if (ndyn > 0) {
        nsa.inst = dupload(owned, ns_dyn_inst);
        nsa.weight = dupload(owned, ns_dyn_w);
        nsa.interval = dalloc<double>(owned, ndyn);
        nsa.number = dalloc<double>(owned, ndyn);
        nsa.noise = dalloc<double>(owned, ndyn);
        nsa.on = dalloc<double>(owned, ndyn);
        nsa.ispike = dalloc<double>(owned, ndyn);
        nsa.event = dalloc<double>(owned, ndyn);
        nsa.q_t = dalloc<double>(owned, static_cast<size_t>(ndyn) * kNsQueue);
        nsa.q_kind = dalloc<int>(owned, static_cast<size_t>(ndyn) * kNsQueue);
        nsa.q_born = dalloc<long long>(owned, static_cast<size_t>(ndyn) * kNsQueue);
        nsa.q_n = dalloc<int>(owned, ndyn);
        nsa.rng = dalloc<unsigned>(owned, static_cast<size_t>(ndyn) * kNsRng);
        nsa.mini_n = dalloc<int>(owned, ndyn);
        nsa.mini_e = dalloc<int>(owned, static_cast<size_t>(ndyn) * kNsMini);
        std::vector<int> b(ndyn + 1, 0), tg;
        std::vector<double> de;
        for (int j = 0; j < ndyn; ++j) {
            for (auto& pr : dyn_fo[j]) { tg.push_back(pr.first); de.push_back(pr.second); }
            b[j + 1] = static_cast<int>(tg.size());
        }
        nsa.fo = FanOut{dupload(owned, b), dupload(owned, tg), dupload(owned, de)};
        ns_log_cap = std::max(1 << 20, 64 * ndyn);
        nsa.log_t = dalloc<double>(owned, ns_log_cap);
        nsa.log_inst = dalloc<int>(owned, ns_log_cap);
        nsa.log_count = dalloc<int>(owned, 1);
        nsa.log_cap = ns_log_cap;
        nsa.error = dalloc<int>(owned, 1);
    }

    spk_cap = std::max(1 << 20, npre * 64);
    d_spk_t = dalloc<double>(owned, spk_cap);
    d_spk_gid = dalloc<int>(owned, spk_cap);
    d_spk_count = dalloc<int>(owned, 1);
    HXC(hipMemset(d_spk_count, 0, sizeof(int)));
    build_groups(vs_fo, ntgt);

    // gap transfers.  The reference copies them one after the other, so a HalfGap instance
    // named by several gaps ends with the last one's source; the transfer kernel copies
    // them side by side, so only that last gap of each instance is kept (gaps_eff).
    {
        std::vector<int> last(mech[M_HALFGAP].present ? mech[M_HALFGAP].n : 0, -1);
        for (size_t e = 0; e < gaps.size(); ++e) last[gaps[e].second] = static_cast<int>(e);
        gaps_eff.clear();
        for (size_t e = 0; e < gaps.size(); ++e)
            if (last[gaps[e].second] == static_cast<int>(e)) gaps_eff.push_back(gaps[e]);
    }
    std::vector<int> gs, gi;
    for (auto& g : gaps_eff) { gs.push_back(node_perm[g.first]); gi.push_back(mech[M_HALFGAP].perm[g.second]); }
    d_gap_src = dupload(owned, gs);
    d_gap_inst = dupload(owned, gi);

    inputs_dirty = true;
    vecplay_dirty = true;
    mon_dirty = true;
    ttab_cap = 0;
}

// Cell groups (see CellGroup).  Groups are contiguous cell ranges of about
// equal node count; each owns the VecStim fan-out into its synapses, an event
// ring, its detectors and its synapse instances.
void hx_sim::build_groups(const std::vector<std::vector<std::pair<int, double>>>& vs_fo, long long ntgt) {
    for (auto& g : groups) {
        if (g.done) (void)hipEventDestroy(g.done);
        if (g.pass) (void)hipEventDestroy(g.pass);
        if (g.s) (void)hipStreamDestroy(g.s);
    }
    groups.clear();
    const auto& R = registry();
    bool coupled = !pre_fanout_empty || !gaps.empty() || !plugins.empty() || nsa.n > 0;
    for (int id = 0; id < M_COUNT; ++id) {
        if (!mech[id].present || mech[id].n == 0) continue;
        if (id == M_ICLAMP || id == M_HALFGAP) coupled = true;        // point currents outside the node kernel
    }
    (void)R;
    groups_coupled = coupled;
    int G = 1;
    if (!coupled) {
        G = group_request > 0 ? group_request : 2;
        G = std::min(G, std::max(1, std::min(ncell / 8, nunit)));
    }
    // event ring geometry: one slot per step, enough slots to cover the longest delay
    const int steps = static_cast<int>(std::ceil(max_delay / dt)) + 4;
    int nslot = 8;
    while (nslot < steps) nslot <<= 1;
    groups.resize(G);
    // groups are runs of whole solve units of about equal node count
    int u0 = 0;
    for (int g = 0; g < G; ++g) {
        CellGroup& cg = groups[g];
        int u1 = nunit;
        if (g < G - 1) {
            const long long target = static_cast<long long>(nnode) * (g + 1) / G;
            u1 = static_cast<int>(std::lower_bound(unit_node_begin.begin(), unit_node_begin.begin() + nunit, target) -
                                  unit_node_begin.begin());
            u1 = std::min(std::max(u1, u0 + 1), nunit - (G - 1 - g));
        }
        cg.unit0 = u0;
        cg.unit1 = u1;
        cg.cell0 = unit_cell_begin[u0];
        cg.cell1 = unit_cell_begin[u1];
        cg.node0 = unit_node_begin[u0];
        cg.node1 = unit_node_begin[u1];
        u0 = u1;
        auto range = [&](const std::vector<int>& nodes, int& b, int& e) {
            b = static_cast<int>(std::lower_bound(nodes.begin(), nodes.end(), cg.node0) - nodes.begin());
            e = static_cast<int>(std::lower_bound(nodes.begin(), nodes.end(), cg.node1) - nodes.begin());
        };
        range(h_pre_node_dev, cg.pre0, cg.pre1);
        range(syn_node[0], cg.es0, cg.es1);
        range(syn_node[1], cg.e20, cg.e21);
        for (int id = 0; id < M_COUNT; ++id) range(inst_node[id], cg.inst0[id], cg.inst1[id]);
        // synapse fold tables over the group's node blocks
        auto fold_table = [&](const std::vector<int>& nodes) {
            const int nb = (cg.node1 - cg.node0 + kBlock - 1) / kBlock;
            std::vector<int> bb(nb + 1);
            for (int b = 0; b < nb; ++b)
                bb[b] = static_cast<int>(std::lower_bound(nodes.begin(), nodes.end(), cg.node0 + b * kBlock) -
                                         nodes.begin());
            bb[nb] = static_cast<int>(std::lower_bound(nodes.begin(), nodes.end(), cg.node1) - nodes.begin());
            return dupload(owned, bb);
        };
        if (!syn_node[0].empty()) cg.d_blk_es = fold_table(syn_node[0]);
        if (!syn_node[1].empty()) cg.d_blk_e2 = fold_table(syn_node[1]);
        // VecStim fan-out restricted to the group's synapses
        std::vector<int> b(vs_fo.size() + 1, 0), tg;
        std::vector<double> de;
        cg.vs_used.assign(vs_fo.size(), 0);
        for (size_t i = 0; i < vs_fo.size(); ++i) {
            for (auto& pr : vs_fo[i]) {
                const int type = target_kind(pr.first), inst = target_inst(pr.first);
                // (a NetStim target makes the model one group)
                if (G > 1 && (syn_node[type][inst] < cg.node0 || syn_node[type][inst] >= cg.node1)) continue;
                tg.push_back(pr.first);
                de.push_back(pr.second);
                cg.vs_used[i] = 1;
            }
            b[i + 1] = static_cast<int>(tg.size());
        }
        cg.d_vs_fo_begin = dupload(owned, b);
        cg.d_vs_fo_target = dupload(owned, tg);
        cg.d_vs_fo_delay = dupload(owned, de);
        const long long ng = static_cast<long long>(tg.size()) + (g == 0 ? ntgt : 0);
        const long long cap =
            event_cap_request > 0 ? event_cap_request : std::max<long long>(4096, std::min<long long>(ng, 1 << 20));
        cg.ring.nslot = nslot;
        cg.ring.cap = static_cast<int>(cap);
        cg.ring.count = dalloc<int>(owned, nslot);
        cg.ring.entry = dalloc<int>(owned, static_cast<size_t>(nslot) * cap);
        cg.ring.overflow = dalloc<int>(owned, 1);
        cg.ring.done = dalloc<unsigned>(owned, 1);
        HXC(hipMemset(cg.ring.count, 0, sizeof(int) * nslot));
        HXC(hipMemset(cg.ring.overflow, 0, sizeof(int)));
        HXC(hipMemset(cg.ring.done, 0, sizeof(unsigned)));
        cg.d_in_cursor = dalloc<int>(owned, 1);
        HXC(hipMemset(cg.d_in_cursor, 0, sizeof(int)));
        if (G > 1) {
            HXC(hipStreamCreate(&cg.s));
            HXC(hipEventCreateWithFlags(&cg.done, hipEventDisableTiming));
            HXC(hipEventCreateWithFlags(&cg.pass, hipEventDisableTiming));
        }
    }
    {
        std::vector<int*> ov;
        for (auto& cg : groups) ov.push_back(cg.ring.overflow);
        d_ring_overflow = dupload(owned, ov);
    }
    if (G > 1 && !ev_main) HXC(hipEventCreateWithFlags(&ev_main, hipEventDisableTiming));
    if (G > 1 && !ev_stagger) HXC(hipEventCreateWithFlags(&ev_stagger, hipEventDisableTiming));
    if (nsa.n > 0) {
        // the NetStim inbox has the event ring's slots; a step's entries are bounded by
        // each instance's one source firing a few times per step
        NsInbox& ib = nsa.ib;
        ib.nslot = nslot;
        ib.cap = static_cast<int>(std::min<long long>(1 << 22, std::max<long long>(4096, 8LL * nsa.n)));
        ib.count = dalloc<int>(owned, nslot);
        ib.entry = dalloc<int>(owned, static_cast<size_t>(nslot) * ib.cap);
        ib.time = dalloc<double>(owned, static_cast<size_t>(nslot) * ib.cap);
        ib.error = nsa.error;
        HXC(hipMemset(ib.count, 0, sizeof(int) * nslot));
    }
}

// NetStim (netstim.cpp:211-330, one random stream per instance) as a train of
// self-event times, for instances that receive no events.  INITIAL schedules
// the init event at start + invl - interval (1 - noise) (0 if negative); that
// event starts the sequence with a self event at the same time, and every self
// event emits a spike at the step time t_m of the step that delivers it, draws
// the next interval and, until `number` spikes are out, schedules the next self
// event at t_m + interval.  A train element is therefore delivered exactly as
// a VecStim element: at the first step whose window t_m + dt/2 reaches it.
// Each instance draws from its own stream, ids (id1, id2, id3) with id1 < 0
// meaning the instance index, sequence 0 at every finitialize (the reference
// shares one stream among all instances and redraws every instance's interval
// on any event, netstim.cpp:118-161; each instance's draws here are the ones
// it would make alone).  Elements past step `horizon` are left for later.
constexpr int kNetStimHorizon0 = 4096;   // steps of NetStim train made at finitialize

namespace {

struct NetStimParams {
    double interval, number, start, noise;
    uint32_t id1, id2, id3;
};

// The train of one instance up to step `horizon` of the step-time table ttab.
void netstim_train(const std::vector<double>& ttab, int horizon, double dt, const NetStimParams& P,
                   std::vector<double>& train) {
    train.clear();
    const double half = dt / 2;
    const double t_end = ttab[horizon];
    const double interval = P.interval, number = P.number, start = P.start;
    const double noise = std::min(1.0, std::max(0.0, P.noise));
    Stream123 rng;
    rng.set_ids(P.id1, P.id2, P.id3);
    rng.set_seq(0, 0);
    auto invl = [&](double mean) {   // netstim.cpp:140-155
        if (mean <= 0.0) mean = 0.01;
        if (noise == 0) return mean;
        return (1.0 - noise) * mean + noise * mean * rng.negexp();
    };
    if (!(start >= 0.0 && number > 0)) return;
    double T = start + invl(interval) - interval * (1.0 - noise);
    if (T < 0.0) T = 0.0;
    int mstep = 0;
    double ispike = 0.0;
    while (T <= t_end) {
        while (ttab[mstep] + half < T) ++mstep;   // delivering step
        train.push_back(T);
        if (train.size() > 64 * static_cast<size_t>(horizon + 1))
            throw std::runtime_error("a NetStim fires more than 64 times per step (interval too small)");
        ispike += 1.0;
        const double e = invl(interval);
        if (ispike >= number) break;
        T = ttab[mstep] + e;
    }
}

// t of every step since finitialize, accumulated exactly as Simulate::fadvance
// does (t += 0.5*dt twice, simulate.cpp:417,774).
void extend_step_times(std::vector<double>& ttab, int n, double dt) {
    if (ttab.empty()) ttab.push_back(0.0);
    while (static_cast<int>(ttab.size()) < n) {
        double x = ttab.back();
        x += 0.5 * dt;
        x += 0.5 * dt;
        ttab.push_back(x);
    }
}

}  // namespace

// NetStim (netstim.cpp:211-330, one random stream per instance) as a train of
// self-event times, for instances that receive no events.  INITIAL schedules
// the init event at start + invl - interval (1 - noise) (0 if negative); that
// event starts the sequence with a self event at the same time, and every self
// event emits a spike at the step time t_m of the step that delivers it, draws
// the next interval and, until `number` spikes are out, schedules the next self
// event at t_m + interval.  A train element is therefore delivered exactly as
// a VecStim element: at the first step whose window t_m + dt/2 reaches it.
// Each instance draws from its own stream, ids (id1, id2, id3) with id1 < 0
// meaning the instance index, sequence 0 at every finitialize (the reference
// shares one stream among all instances and redraws every instance's interval
// on any event, netstim.cpp:118-161; each instance's draws here are the ones
// it would make alone).  Elements past step `horizon` are left for later.
void hx_sim::make_netstim_trains(int horizon) {
    const HostMech& m = mech[M_NETSTIM];
    const int nns = m.present ? m.n : 0;
    netstim.assign(nns, {});
    ensure_ttab(horizon + 1);
    for (int j = 0; j < nns; ++j) {
        if (j < static_cast<int>(ns_dyn.size()) && ns_dyn[j] >= 0) continue;   // runs on the device
        const double id1 = m.col[NS_ID1][j];
        const NetStimParams P{m.col[NS_INTERVAL][j], m.col[NS_NUMBER][j], m.col[NS_START][j], m.col[NS_NOISE][j],
                              id1 < 0 ? static_cast<uint32_t>(j) : static_cast<uint32_t>(id1),
                              static_cast<uint32_t>(m.col[NS_ID2][j]), static_cast<uint32_t>(m.col[NS_ID3][j])};
        netstim_train(ttab, horizon, dt, P, netstim[j]);
    }
    ns_horizon = horizon;
}

// VecStim trains -> globally sorted effective event times.  A train element is
// processed at the first step whose window t+dt/2 reaches it, but never before
// the previous element of the same train (vecevent.cpp:172-199 chains the
// self-events), hence the running maximum.
//
// Each element also carries the pass of its step's delivery loop that emits its spike
// (simulate.cpp:916-939 repeats the loop while anything was sent), which orders what a
// NetStim receiving these spikes sees within one step: a VecStim element is processed in
// pass 1 when its self event was queued in an earlier step, else in the pass after its
// predecessor's; a NetStim's first spike comes in pass 2 (the init event in pass 1 sends
// a self event at t), later ones like VecStim elements.
void hx_sim::upload_inputs() {
    struct In {
        double t;
        int src, round;
    };
    std::vector<In> ev;
    const int nvs = mech[M_VECSTIM].present ? mech[M_VECSTIM].n : 0;
    const int nns = mech[M_NETSTIM].present ? mech[M_NETSTIM].n : 0;
    const double half = dt / 2;
    auto step_of = [&](double T) {   // first step m with t_m + dt/2 >= T
        int m = std::max(0, static_cast<int>(std::floor(T / dt)) - 2);
        if (static_cast<int>(ttab.size()) < m + 8) extend_step_times(ttab, m + 64, dt);
        while (m > 0 && ttab[m - 1] + half >= T) --m;
        while (ttab[m] + half < T) {
            ++m;
            if (m + 1 >= static_cast<int>(ttab.size())) extend_step_times(ttab, m + 64, dt);
        }
        return m;
    };
    auto add_train = [&](const std::vector<double>& train, int s, int first_round) {
        double prev = -INFINITY;
        int round = 0;
        for (size_t i = 0; i < train.size(); ++i) {
            const double cur = std::max(prev, train[i]);
            if (i == 0) round = first_round;
            // only an element this close can share its predecessor's step
            else if (cur - prev <= 2 * dt && cur / dt < 5e7) round = step_of(cur) == step_of(prev) ? round + 1 : 1;
            else round = 1;
            prev = cur;
            ev.push_back({cur, s, std::min(round, kNsRounds - 1)});
        }
    };
    for (int s = 0; s < nvs && s < static_cast<int>(vecstim_run.size()); ++s) add_train(vecstim_run[s], s, 1);
    for (int j = 0; j < nns && j < static_cast<int>(netstim.size()); ++j) add_train(netstim[j], nvs + j, 2);
    std::stable_sort(ev.begin(), ev.end(), [](const In& x, const In& y) { return x.t < y.t; });
    for (auto& cg : groups) {
        // each group keeps the events of the VecStims that drive its synapses
        std::vector<double> tt;
        std::vector<int> ii, rr;
        for (auto& e : ev)
            if (e.src < static_cast<int>(cg.vs_used.size()) && cg.vs_used[e.src]) {
                tt.push_back(e.t);
                ii.push_back(e.src);
                rr.push_back(e.round);
            }
        cg.n_in = static_cast<int>(tt.size());
        cg.d_in_time = slot_upload(cg.in_time_slot, tt);
        cg.d_in_inst = slot_upload(cg.in_inst_slot, ii);
        cg.d_in_round = slot_upload(cg.in_round_slot, rr);
    }
    inputs_dirty = false;
}

// VecEvent::play -> update_sequence (vecevent.cpp:280-309): the instance's vector becomes
// `times`, read from its first element by the next finitialize (INITIAL, vecevent.cpp:
// 94-107).  A run already initialised keeps what the instance has read: element()
// (vecevent.cpp:123-156) has taken D + 1 elements after D deliveries and queued the
// self event of the last, so the run delivers that one and then times[D + 1],
// times[D + 2], ...; an instance that has read past its end takes nothing more.
// The deliveries so far are the elements whose effective time (the running maximum,
// as upload_inputs orders them) lies within the window of the last delivery, that of
// finitialize or of step k - 1; those entries keep their place at the head of the
// sorted input list, so the device's input cursor stays valid when the list is rebuilt.
int hx_sim::vecstim_play(int inst, const double* times, int n) {
    vecstim[inst].assign(times, times + n);
    if (!initialized) {
        inputs_dirty = true;
        return 0;
    }
    std::vector<double>& run = vecstim_run[inst];
    const double cut = ttab[k > 0 ? k - 1 : 0] + dt / 2;
    size_t D = 0;
    double prev = -INFINITY;
    while (D < run.size()) {
        const double cur = std::max(prev, run[D]);
        if (cur > cut) break;
        prev = cur;
        ++D;
    }
    if (D == run.size()) return 0;              // nothing queued: index -1 (or an empty vector)
    run.resize(D + 1);
    for (int i = static_cast<int>(D) + 1; i < n; ++i) run.push_back(times[i]);
    vecstim_run_differs = true;
    upload_inputs();
    return 0;
}

void hx_sim::upload_vecplay() {
    // keep the playback position of items that were already on the device
    std::map<std::tuple<std::string, std::string, int>, VecPlayDev> prev;
    if (d_vecplay && !vecplay_keys.empty()) {
        std::vector<VecPlayDev> old(vecplay_keys.size());
        HXC(hipMemcpy(old.data(), d_vecplay, sizeof(VecPlayDev) * old.size(), hipMemcpyDeviceToHost));
        for (size_t i = 0; i < old.size(); ++i) prev[vecplay_keys[i]] = old[i];
    }
    std::vector<VecPlayDev> items;
    vecplay_keys.clear();
    for (auto& vp : vecplay) {
        if (!vp.d_t) {
            vp.d_t = dupload(owned, vp.tvec);
            vp.d_y = dupload(owned, vp.yvec);
        }
        VecPlayDev it{};
        it.target = vp.target;
        it.tvec = vp.d_t;
        it.yvec = vp.d_y;
        it.len = static_cast<int>(vp.tvec.size());
        it.next_time = vp.tvec.empty() ? 0.0 : vp.tvec[0];
        auto key = std::make_tuple(vp.mech, vp.var, vp.idx);
        auto pv = prev.find(key);
        if (pv != prev.end() && pv->second.tvec == it.tvec && pv->second.len == it.len) {
            it.last_index = pv->second.last_index;
            it.next_idx = pv->second.next_idx;
            it.done = pv->second.done;
            it.next_time = pv->second.next_time;
        }
        vecplay_keys.push_back(key);
        items.push_back(it);
    }
    d_vecplay = slot_upload(vecplay_slot, items);
    vecplay_iclamp_only = true;
    for (const auto& vp : vecplay) vecplay_iclamp_only = vecplay_iclamp_only && vp.mech == "IClamp";
    vecplay_dirty = false;
}

void hx_sim::upload_monitors() {
    // sample-buffer columns are ordered by cell group (voltage monitors; the
    // rest last) so a group records its columns as one contiguous range
    const int nm = static_cast<int>(mon_ref.size());
    const int G = static_cast<int>(groups.size());
    std::vector<int> grp(nm, G);
    mon_all_v = true;
    for (int i = 0; i < nm; ++i) {
        const double* p = mon_ref[i].dev;
        if (p >= d_v && p < d_v + nnode) {
            const int node = static_cast<int>(p - d_v);
            for (int g = 0; g < G; ++g)
                if (node >= groups[g].node0 && node < groups[g].node1) grp[i] = g;
        } else {
            mon_all_v = false;
        }
    }
    std::vector<int> order(nm);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return grp[x] < grp[y]; });
    mon_col.assign(nm, 0);
    std::vector<double*> ptrs(nm);
    for (int q = 0; q < nm; ++q) {
        mon_col[order[q]] = q;
        ptrs[q] = mon_ref[order[q]].dev;
    }
    for (int g = 0; g < G; ++g) {
        groups[g].mon0 = static_cast<int>(std::lower_bound(order.begin(), order.end(), g,
                                                           [&](int m, int gg) { return grp[m] < gg; }) - order.begin());
        groups[g].mon1 = static_cast<int>(std::lower_bound(order.begin(), order.end(), g + 1,
                                                           [&](int m, int gg) { return grp[m] < gg; }) - order.begin());
    }
    d_mon_ptr = slot_upload(mon_ptr_slot, ptrs);
    mon_dirty = false;
}

// Step-time table long enough for kneed steps plus the longest netcon delay.
void hx_sim::ensure_ttab(int kneed) {
    const int margin = static_cast<int>(std::ceil(max_delay / dt)) + 8;
    const int want = kneed + margin;
    if (static_cast<int>(ttab.size()) < want + 1) {
        // grown geometrically, so most calls find their steps in the table already
        const int have = static_cast<int>(ttab.size());
        extend_step_times(ttab, std::max(want + 1, std::max(2 * have, 1024)), dt);
    }
    if (ttab_cap < static_cast<int>(ttab.size())) {
        ttab_cap = static_cast<int>(ttab.size()) * 2;
        d_ttab = static_cast<double*>(slot_reserve(ttab_slot, sizeof(double) * ttab_cap));
        ttab_up = 0;
    }
    // only new entries travel: a call whose steps the table already covers copies nothing
    const int n = static_cast<int>(ttab.size());
    if (ttab_up < n) {
        HXC(hipMemcpy(d_ttab + ttab_up, ttab.data() + ttab_up, sizeof(double) * (n - ttab_up),
                      hipMemcpyHostToDevice));
        ttab_up = n;
    }
}

// Monitor sample rows: a call of n steps records n rows (finitialize one).  The buffer
// grows geometrically, from at least 1024 rows while that stays within 64 MB, so calls
// of similar length do not allocate.
void hx_sim::ensure_mon_rows(long long rows) {
    if (mon_ref.empty() || mon_buf_cap >= rows) return;
    const long long nm = static_cast<long long>(mon_ref.size());
    long long want = std::max(rows, 2 * mon_buf_cap);
    want = std::max(want, std::min<long long>(1024, std::max<long long>(1, (64LL << 20) / (8 * nm))));
    mon_buf_cap = want;
    d_mon_buf = static_cast<double*>(slot_reserve(mon_buf_slot, sizeof(double) * static_cast<size_t>(want * nm)));
    mon_buf_fill = 0;
}

Ref hx_sim::resolve(const std::string& mn, const std::string& var, int idx) {
    Ref r;
    if (mn == "global" || mn == "node") {
        if (idx < 0 || idx >= nnode) return r;
        const int g = node_perm[idx];
        if (var == "v") r.dev = d_v + g;
        else if (var == "d") { r.dev = d_d + g; r.klass = 1; }
        else if (var == "rhs") { r.dev = d_rhs + g; r.klass = 1; }
        else if (var == "a") { r.dev = d_a + g; r.ab = 1; r.node = idx; }
        else if (var == "b") { r.dev = d_b + g; r.ab = 2; r.node = idx; }
        else if (var == "area") r.dev = d_area + g;
        return r;
    }
    if (mn == "capacitance") {
        if (idx < 0 || idx >= nnode || var != "cm") return r;
        r.dev = d_cm + node_perm[idx];
        cm_uniform = false;              // a handle may write it: read per node from now on
        return r;
    }
    int id = mech_id(mn);
    if (id < 0) {
        PluginInst* p = plugin_named(mn);
        if (!p || idx < 0 || idx >= p->h.n) return r;
        for (int c = 0; c < p->meta->ncol; ++c)
            if (var == p->meta->cols[c]) {
                r.dev = p->h.dev.col(c) + p->h.perm[idx];
                r.klass = c >= p->meta->nparam + p->meta->nstate ? 1 : 0;
                r.point = (p->meta->flags & plugin::kPoint) != 0;
            }
        return r;
    }
    if (!mech[id].present) return r;
    const auto& M = registry()[id];
    HostMech& m = mech[id];
    if (M.ion) {
        if (idx < 0 || idx >= nnode) return r;
        const int x = id == M_NA_ION ? 0 : id == M_K_ION ? 1 : 2;
        const int inst = ion_at[x][node_perm[idx]];
        const int c = col_id(id, var);
        if (inst < 0 || c < 0) return r;
        r.dev = m.dev.col(c) + inst;
        m.dev.umask &= ~(1u << c);       // a handle may write the column
        r.klass = (c == ION_CONCI || c == ION_CONCO) ? 0 : 1;
        return r;
    }
    // gradients of the adjoint (grad_<parameter>) and netcon weights, addressable by
    // handles so optimizers can be given (weight, gradient) pairs
    if (var.compare(0, 5, "grad_") == 0) {
        const int tk = trainable_id(id, var.substr(5));
        if (tk < 0 || idx < 0 || idx >= m.n) return r;
        ensure_grad_arrays();
        r.dev = d_grad[tk] + m.perm[idx];
        return r;
    }
    if ((id == M_EXPSYN || id == M_EXP2SYN) && var == "weight") {
        if (idx < 0 || idx >= m.n) return r;
        r.dev = (id == M_EXPSYN ? d_es_weight : d_e2_weight) + m.perm[idx];
        return r;
    }
    if (id == M_CADYN && (var == "cai" || var == "ica")) {
        // CaDynamics_E2 keeps cai / ica in the ca_ion columns of its node
        if (idx < 0 || idx >= m.n) return r;
        return resolve("ca_ion", var == "cai" ? "conci" : "cur", m.node[idx]);
    }
    if (id == M_NETSTIM && (var == "on" || var == "ispike" || var == "event")) {
        // state of a NetStim that receives events (the others are trains made on the host)
        if (idx < 0 || idx >= static_cast<int>(ns_dyn.size()) || ns_dyn[idx] < 0) return r;
        const int j = ns_dyn[idx];
        r.dev = (var == "on" ? nsa.on : var == "ispike" ? nsa.ispike : nsa.event) + j;
        r.point = true;        // changes at delivery, which the fused schedule runs before the record
        return r;
    }
    const int c = col_id(id, var);
    if (c < 0 || idx < 0 || idx >= m.n) return r;
    r.dev = m.dev.col(c) + m.perm[idx];
    // a handle may write the column: from now on the kernels read it per instance
    if (c < 32) m.dev.umask &= ~(1u << c);
    r.klass = c >= M.nparam + M.nstate ? 1 : 0;
    r.point = M.point;
    if (id == M_NETSTIM) {           // parameters only: nothing changes them during a step
        r.point = false;
        r.ns_col = c;
        r.ns_inst = idx;
    }
    if (id == M_EXP2SYN && c == E2_FACTOR) r.klass = 0;   // written by INITIAL
    if (id == M_HALFGAP && c == HG_VGAP) r.klass = 0;     // written by the gap transfer
    return r;
}

// An ion's cur and erev are stored when something outside the fused kernel reads
// them: a mechanism run instance-parallel, CaDynamics_E2 (reads ica in the next
// state update) or a handle/monitor on an assigned variable (assigned).
unsigned hx_sim::ion_store_bits(bool assigned) const {
    const auto& R = registry();
    unsigned need = 0;
    for (int id = 0; id < M_COUNT; ++id)
        if (mech[id].present && !(dense_mask & (1u << id))) need |= static_cast<unsigned>(R[id].ion_use);
    need |= plugin_ions();     // plugins read erev and add their currents after the node kernel
    unsigned bits = 0;
    for (int x = 0; x < 3; ++x) {
        const bool ext = assigned || (need & (1u << x));
        if (ext || (x == 2 && mech[M_CADYN].present && !pass_cadyn_after)) bits |= 1u << (2 * x);
        if (ext) bits |= 2u << (2 * x);
    }
    return bits;
}

StepArgs hx_sim::step_args(double tcur, int do_state, int do_current) const {
    StepArgs A{};
    A.N = nnode;
    A.node0 = 0;
    A.pt0 = 0;
    A.pt1 = std::numeric_limits<int>::max();
    A.v = d_v;
    A.d = d_d;
    A.rhs = d_rhs;
    A.area = d_area;
    A.cm = d_cm;
    A.cm_uniform = (cm_uniform && uniform_on) ? 1 : 0;
    A.cm_value = cm_value;
    A.cfac = 0.001 * (1.0 / dt);
    for (int id = 0; id < M_COUNT; ++id) {
        A.m[id] = mech[id].dev;
        if (!uniform_on) A.m[id].umask = 0;
    }
    A.dense_mask = dense_mask;
    A.yform = pass_yform;
    A.hh_owns_ions = (hh_owns_ions && !init_pass) ? 1 : 0;
    A.do_state = do_state;
    A.cadyn_skip = do_state ? pass_cadyn_skip : 0;
    A.cadyn_after = do_current ? pass_cadyn_after : 0;
    A.do_current = do_current;
    // A call whose outputs are made on demand (lazy_final) stores none of the node kernel's
    // assigned outputs on its last step; the synapses' outputs are stored as usual.
    const bool lazy_final = final_step && lazy_outputs_run && do_current;
    const bool assigned = write_assigned || (final_step && !lazy_final);
    A.write_assigned = assigned ? 1 : 0;
    A.point_assigned = (assigned || lazy_final) ? 1 : 0;
    // A call's last step stores the rates once, in its closing state pass (the fused
    // pass before it updates the previous step's states, whose rates that pass
    // overwrites).  dcurdv holds the 0 that finitialize's pass stored unless a handle
    // made every step store the assigned variables.
    A.write_rates = (write_assigned || (final_step && !do_current)) ? 1 : 0;
    A.ion_store = ion_store_bits(assigned);
    for (int x = 0; x < 3; ++x) A.ion_type[x] = ion_type_uniform[x];
    A.write_dcurdv = (write_assigned || init_pass) ? 1 : 0;
    A.fold_mask = 0;
    for (int id : {M_EXPSYN, M_EXP2SYN})
        if (mech[id].present && mech[id].n > 0) A.fold_mask |= 1u << id;
    A.t = tcur;
    A.dt = dt;
    auto G = [&](int id, const char* k, double dflt) {
        auto it = globals[id].find(k);
        return it == globals[id].end() ? dflt : it->second;
    };
    const double hh_cel = G(M_HH, "celsius", celsius);
    A.c.hh_q10 = std::pow(3.0, (hh_cel - 6.3) / 10);
    const double hd_cel = G(M_HDLA, "celsius", celsius);
    A.c.hd_qt = std::pow(G(M_HDLA, "q10", 4.5), ((hd_cel - 33.0) / 10.0));
    A.c.hd_ehd = G(M_HDLA, "ehd", -30.0);
    A.c.hd_kl = G(M_HDLA, "kl", -8.0);
    A.c.hd_inv_kl = 1.0 / A.c.hd_kl;
    A.c.hd_vhalft = G(M_HDLA, "vhalft", -75.0);
    A.c.hd_a0t = G(M_HDLA, "a0t", 0.011);
    A.c.hd_zetat = G(M_HDLA, "zetat", 2.2);
    A.c.hd_gmt = G(M_HDLA, "gmt", 0.4);
    A.c.hd_qtl = G(M_HDLA, "qtl", 1.0);
    A.c.hd_pow = A.c.hd_gmt == 0.4 ? 1 : 0;
    A.c.hd_k5 = 0.0378 * A.c.hd_zetat * 0.2;
    {
        const HostMech& cd = mech[M_CADYN];
        const unsigned all = (1u << CD_GAMMA) | (1u << CD_DECAY) | (1u << CD_DEPTH) | (1u << CD_MINCAI);
        A.c.cd_uniform = cd.present && cd.n > 0 && uniform_on && (cd.dev.umask & all) == all ? 1 : 0;
        if (A.c.cd_uniform) {
            const double gamma = cd.col[CD_GAMMA][0], decay = cd.col[CD_DECAY][0];
            const double depth = cd.col[CD_DEPTH][0];
            A.c.cd_c1 = 1.0 - std::exp(-dt / decay);
            A.c.cd_g = -(10000.0) * gamma / (2.0 * kFaradayCaDyn * depth) * decay;
            A.c.cd_min = cd.col[CD_MINCAI][0];
        }
    }
    const double R = 1.380649e-23 * 6.02214076e+23, F = 1.602176634e-19 * 6.02214076e+23;
    A.c.ktf = 1000. * R * (celsius + 273.15) / F;
    return A;
}

// ===========================================================================
// stepping
// ===========================================================================

// The mechanism pass over the whole model, or over one cell group (nodes,
// synapse fold tables and instance ranges of that group) on stream `on`.
void hx_sim::launch_mech_pass(int do_state, int do_current, double tcur, int grp, hipStream_t on) {
    StepArgs A = step_args(tcur, do_state, do_current);
    const CellGroup* cg = grp >= 0 ? &groups[grp] : nullptr;
    hipStream_t s = on ? on : stream;
    if (cg) {
        A.node0 = cg->node0;
        A.N = cg->node1;
        A.m[M_EXPSYN].blk_begin = cg->d_blk_es;
        A.m[M_EXP2SYN].blk_begin = cg->d_blk_e2;
    }
    // the node kernel's timer events are set by its own dispatch, with no marker packets
    // around it; the end event then also marks the pass for the cell groups' turns
    hipEvent_t e0, e1;
    const bool timed = treserve(T_MECH, e0, e1);
    const int launched = (do_current || dense_mask) ? launch_dense(A, s, dense_steady != 0, e0, e1) : 0;
    if (launched == 2) ++steady_launches;
    if (timed && launched) tcommit(T_MECH);
    mech_end_mark = timed && launched ? e1 : nullptr;
    bool any_sparse = false;
    for (int id : kSparseOrder) any_sparse |= mech[id].present && !(dense_mask & (1u << id));
    if (!any_sparse) return;
    auto sparse = [&](int id) {
        StepArgs B = A;
        if (cg) {
            B.pt0 = cg->inst0[id];
            B.pt1 = cg->inst1[id];
        }
        launch_sparse(id, B, s);
    };
    mech_end_mark = nullptr;        // launches follow the node kernel's timer end
    tbegin(T_SPARSE, s);
    // an ion's kernel only zeroes its current (and makes erev under style 0100): nothing
    // to do in a state pass, nor in a stepping current pass when hh stores its ions
    auto is_ion = [](int id) { return id == M_NA_ION || id == M_K_ION || id == M_CA_ION; };
    if (do_state && !do_current) {
        // ion writers first (simulate.cpp:822-834)
        if (mech[M_CADYN].present && !(dense_mask & (1u << M_CADYN))) sparse(M_CADYN);
        for (int id : kSparseOrder)
            if (id != M_CADYN && !is_ion(id) && mech[id].present && !(dense_mask & (1u << id))) sparse(id);
    } else {
        const bool skip_nak = hh_owns_ions && !init_pass;
        for (int id : kSparseOrder) {
            if (skip_nak && (id == M_NA_ION || id == M_K_ION)) continue;
            if (mech[id].present && !(dense_mask & (1u << id))) sparse(id);
        }
    }
    tend(T_SPARSE, s);
}

void hx_sim::launch_point_currents(double tcur) {
    StepArgs A = step_args(tcur, 0, 1);
    const int pts[] = {M_ICLAMP, M_EXPSYN, M_EXP2SYN, M_HALFGAP};   // CoreNEURON order
    bool any = false;
    for (int id : pts) any |= mech[id].present && mech[id].n > 0 && !(A.fold_mask & (1u << id));
    if (!any) return;
    tbegin(T_POINT);
    // IClamp and HalfGap in one launch when no synapse current comes between them
    const bool pair = point_union.n > 0 && !(mech[M_EXPSYN].present && !(A.fold_mask & (1u << M_EXPSYN))) &&
                      !(mech[M_EXP2SYN].present && !(A.fold_mask & (1u << M_EXP2SYN)));
    if (pair) {
        launch_point_electrodes(A, point_union, stream);
    } else {
        for (int id : pts)   // synapse currents are added by the node kernel
            if (mech[id].present && !(A.fold_mask & (1u << id))) launch_point_current(id, A, stream);
    }
    tend(T_POINT);
}

PluginArgs hx_sim::plugin_args(const PluginInst& p, double tcur) const {
    PluginArgs P{};
    P.m = p.h.dev;
    P.ion[0] = mech[M_NA_ION].dev;
    P.ion[1] = mech[M_K_ION].dev;
    P.ion[2] = mech[M_CA_ION].dev;
    P.v = d_v;
    P.d = d_d;
    P.rhs = d_rhs;
    P.area = d_area;
    P.t = tcur;
    P.dt = dt;
    P.celsius = celsius;
    P.recv_count = p.d_recv_count;
    P.recv_w = p.d_recv_w;
    P.recv_delay = p.d_recv_delay;
    return P;
}

// Plugins run after the built-in mechanisms: their currents after the node kernel and
// the point processes (CoreNEURON order puts user mechanisms after the built-in
// ones), their states after the solve, before the step's record.
void hx_sim::launch_plugin_inits(double tcur) {
    for (const auto& p : plugins) p.meta->launch_init(plugin_args(p, tcur), stream);
}
void hx_sim::launch_plugin_currents(double tcur) {
    if (plugins.empty()) return;
    tbegin(T_OTHER);
    for (const auto& p : plugins) p.meta->launch_current(plugin_args(p, tcur), stream);
    tend(T_OTHER);
}
void hx_sim::launch_plugin_states(double tcur) {
    if (plugins.empty()) return;
    tbegin(T_OTHER);
    for (const auto& p : plugins) p.meta->launch_state(plugin_args(p, tcur), stream);
    tend(T_OTHER);
}

bool hx_sim::launch_events(int kk, double tk, double vp_t) {
    const int G = static_cast<int>(groups.size());
    if (G > 1 && G <= kMaxMergedGroups && nsa.n == 0 && !has_postsyn_plugins()) {
        // the groups share the library stream: one input and one delivery launch for all
        // of them (each group keeps its own trains, cursor and ring)
        if (!mech[M_EXPSYN].present && !mech[M_EXP2SYN].present) return false;
        tbegin(T_EVENTS, stream);
        InputSet in{};
        RingSet rs{};
        int cap = 0;
        for (int g = 0; g < G; ++g) {
            if (groups[g].n_in > 0) in.a[in.n++] = input_args(g, kk, tk);
            rs.r[rs.n++] = groups[g].ring;
            cap = std::max(cap, groups[g].ring.cap);
        }
        launch_input_set(in, stream);
        launch_deliver_set(deliver_args(kk, vp_t), rs, deliver_blocks(cap), stream);
        tend(T_EVENTS, stream);
        return vp_t >= 0.0;
    }
    bool vp_done = false;
    for (int g = 0; g < static_cast<int>(groups.size()); ++g)
        vp_done |= launch_events_group(g, kk, tk, stream, g == 0 ? vp_t : -1.0);
    return vp_done;
}

// VecStim input and delivery of step kk for one cell group's synapses.
bool hx_sim::launch_events_group(int g, int kk, double tk, hipStream_t on, double vp_t) {
    const bool psyn = has_postsyn_plugins();
    const bool syn = mech[M_EXPSYN].present || mech[M_EXP2SYN].present || psyn;
    if (!syn && nsa.n == 0) return false;
    CellGroup& cg = groups[g];
    tbegin(T_EVENTS, on);
    if (cg.n_in > 0) launch_input(input_args(g, kk, tk), on);
    if (nsa.n > 0) {                 // NetStims receiving events: one group, the main stream
        NsArgs A = nsa;
        A.ring = cg.ring;
        A.ttab = d_ttab;
        A.kmax = static_cast<int>(ttab.size()) - 1;
        A.half_dt = dt / 2;
        A.t = tk;
        A.k = kk;
        launch_netstim(A, on);
    }
    if (!syn) {
        tend(T_EVENTS, on);
        return false;
    }
    DeliverArgs D = deliver_args(kk, vp_t);
    D.ring = cg.ring;
    // Workgroups: spike-driven netcons can put up to a whole fan-out of every cell into
    // one step, so a burst is spread over one 1024-thread workgroup per 8192 entries of
    // slot capacity (at most 64); with only VecStim inputs a step's events are few, and
    // one workgroup starts soonest beside the other cell group's kernels (measured:
    // config 3 ran 2.5% slower with the grid and a merged input kernel, and 3% slower
    // with 256-thread workgroups).
    launch_deliver(D, deliver_blocks(cg.ring.cap), on);
    // the synapse plugins' NET_RECEIVE of what was counted (one group: plugins couple the model)
    for (const auto& p : plugins)
        if (p.slot >= 0) p.meta->launch_receive(plugin_args(p, tk), on);
    tend(T_EVENTS, on);
    return vp_t >= 0.0;
}

// Group g's VecStim input of step kk (time tk).
InputArgs hx_sim::input_args(int g, int kk, double tk) const {
    const CellGroup& cg = groups[g];
    InputArgs I{};
    I.eff_time = cg.d_in_time;
    I.inst = cg.d_in_inst;
    I.round = cg.d_in_round;
    I.ib = nsa.ib;
    I.n = cg.n_in;
    I.cursor = cg.d_in_cursor;
    I.tcut = tk + dt / 2;
    I.t = tk;
    I.k = kk;
    I.fo = FanOut{cg.d_vs_fo_begin, cg.d_vs_fo_target, cg.d_vs_fo_delay};
    I.ring = cg.ring;
    I.ttab = d_ttab;
    I.kmax = static_cast<int>(ttab.size()) - 1;
    I.half_dt = dt / 2;
    return I;
}

// The delivery of step kk without its ring; VecPlay at vp_t on blocks of its own when
// vp_t >= 0.
DeliverArgs hx_sim::deliver_args(int kk, double vp_t) const {
    DeliverArgs D{};
    D.k = kk;
    D.es = mech[M_EXPSYN].dev;
    D.e2 = mech[M_EXP2SYN].dev;
    D.es_weight = d_es_weight;
    D.e2_weight = d_e2_weight;
    for (const auto& p : plugins)
        if (p.slot >= 0) D.plugin_recv[p.slot] = p.d_recv_count;
    if (tape_on && tape_n < tape_cap) {
        D.log_count = d_tape_evn + tape_n;
        D.log = d_tape_ev + static_cast<size_t>(tape_n) * tape_evcap;
        D.log_cap = tape_evcap;
    }
    if (vp_t >= 0.0) {
        D.vp = d_vecplay;
        D.nvp = static_cast<int>(vecplay.size());
        D.t_vp = vp_t;
    }
    return D;
}

// Threshold detection of detectors [pre0, pre1) at step kk (time tk), fanning out into
// `ring` (detector netcons exist only with a single group).
SpikeArgs hx_sim::spike_args(int kk, double tk, int pre0, int pre1, const EventRing& ring) const {
    SpikeArgs S{};
    S.npre = pre1 - pre0;
    S.v = d_v;
    S.node = d_pre_node + pre0;
    S.thr = d_pre_thr + pre0;
    S.flag = d_pre_flag + pre0;
    S.gid = d_pre_gid + pre0;
    S.t = tk;
    S.k = kk;
    S.log_t = d_spk_t;
    S.log_gid = d_spk_gid;
    S.log_count = d_spk_count;
    S.log_cap = spk_cap;
    S.fo = FanOut{d_pre_fo_begin + pre0, d_pre_fo_target, d_pre_fo_delay};
    S.ring = ring;
    S.ib = nsa.ib;
    S.ttab = d_ttab;
    S.kmax = static_cast<int>(ttab.size()) - 1;
    S.half_dt = dt / 2;
    return S;
}

void hx_sim::launch_detect(int kk, double tk) {
    if (npre == 0) return;
    tbegin(T_SPIKE);
    launch_spike(spike_args(kk, tk, 0, npre, groups[0].ring), stream);
    tend(T_SPIKE);
}

// The work after the solve of the step ending at tn (the next step is knext), as one
// launch: for cell group grp (its detectors and synapses; the groups have no gaps and no
// VecPlay) or, with grp < 0, the whole model.
AfterSolve hx_sim::after_solve_args(double tn, int knext, int grp) const {
    AfterSolve P{};
    P.v = d_v;
    P.dt = dt;
    P.t = tn;
    if (grp < 0) {
        if (static_gaps_on && !gaps.empty()) {
            P.gap_src = d_gap_src;
            P.gap_inst = d_gap_inst;
            P.vgap = mech[M_HALFGAP].dev.col(HG_VGAP);
            P.ngap = static_cast<int>(gaps_eff.size());
        }
        P.psrc = d_dg_src;
        P.pdst = d_dg_dst;
        P.nptr = static_cast<int>(dg_src.size());
        if (npre > 0) P.S = spike_args(knext, tn, 0, npre, groups[0].ring);
        P.vp = d_vecplay;
        P.nvp = static_cast<int>(vecplay.size());
    } else {
        const CellGroup& cg = groups[grp];
        if (cg.pre1 > cg.pre0) P.S = spike_args(knext, tn, cg.pre0, cg.pre1, cg.ring);
    }
    const MechDev& es = mech[M_EXPSYN].dev;
    if (mech[M_EXPSYN].present && es.n > 0) {
        P.es_g = es.col(ES_G);
        P.es_tau = es.col(ES_TAU);
        P.es0 = grp < 0 ? 0 : groups[grp].es0;
        P.es1 = grp < 0 ? es.n : groups[grp].es1;
    }
    const MechDev& e2 = mech[M_EXP2SYN].dev;
    if (mech[M_EXP2SYN].present && e2.n > 0) {
        P.e2_a = e2.col(E2_A);
        P.e2_b = e2.col(E2_B);
        P.e2_tau1 = e2.col(E2_TAU1);
        P.e2_tau2 = e2.col(E2_TAU2);
        P.e20 = grp < 0 ? 0 : groups[grp].e20;
        P.e21 = grp < 0 ? e2.n : groups[grp].e21;
    }
    return P;
}

void hx_sim::launch_record() {
    if (learn && learn->capturing()) learn->sample();
    if (mon_ref.empty()) return;
    if (mon_buf_fill >= mon_buf_cap) throw std::runtime_error("monitor buffer exhausted");
    tbegin(T_OTHER);
    hx::launch_record(d_mon_ptr, static_cast<int>(mon_ref.size()), d_mon_buf + mon_buf_fill * mon_ref.size(), stream);
    tend(T_OTHER);
    mon_buf_fill++;
}

// A write to a node's a or b also reaches the solver's copy: at the same node
// when the solver's tree keeps the link's orientation, else, with a and b
// trading places, at the node's parent (which the solver hangs below it).
void hx_sim::mirror_ab(const Ref& r, double value) {
    if (r.ns_col >= 0) {   // NetStim trains are made from the host copy at the next finitialize
        mech[M_NETSTIM].col[r.ns_col][r.ns_inst] = value;
        return;
    }
    if (!r.ab || r.node < 0) return;
    const int u = r.node;
    (r.ab == 1 ? a : b)[u] = value;
    const int p = parent[u];
    if (p < 0) return;
    int at;
    bool a_side;
    if (solve_parent[u] == p) {
        at = u;
        a_side = r.ab == 1;
    } else {
        at = p;
        a_side = r.ab == 2;
    }
    (a_side ? solve_a : solve_b)[at] = value;
    HXC(hipMemcpy((a_side ? d_sa : d_sb) + node_perm[at], &value, sizeof(double), hipMemcpyHostToDevice));
    adj_delta_dirty = true;   // rebuilt by the next adjoint
}

// A sampled assigned variable (klass 1) or point-process variable is only
// valid at the reference's record point under the split schedule.
void hx_sim::require_sample_point(const Ref& r) {
    if ((r.klass == 1 || r.point) && !need_split_for_monitor) {
        need_split_for_monitor = true;
        write_assigned = write_assigned || r.klass == 1;
        fused = false;
        if (state_pending) { finish_pending(); sync_outputs(); }
    }
}

// The step's tape row (v after the solve and the states its current pass used), as one
// launch of its own.
void hx_sim::tape_record() {
    launch_tape(tape_row(true), stream);
    ++tape_n;
}

// The next tape row's copies (the synapse states among them when syn, else the decay
// tasks of the after-solve launch tape those).
TapeCopy hx_sim::tape_row(bool syn) const {
    if (tape_n >= tape_cap)
        throw std::runtime_error("adjoint tape full (" + std::to_string(tape_cap) + " steps): call hx_tape_begin "
                                 "with more steps");
    const size_t n = static_cast<size_t>(tape_n);
    TapeCopy T{};
    auto seg = [&](const double* src, double* dst, long long cnt) {
        T.src[T.nseg] = src;
        T.dst[T.nseg] = dst;
        T.n[T.nseg] = cnt;
        ++T.nseg;
    };
    seg(d_v, d_tape_v + n * nnode, nnode);
    if (mech[M_HH].present && mech[M_HH].n > 0) {
        const MechDev& h = mech[M_HH].dev;   // columns m, h, n are consecutive
        seg(h.col(HH_M), d_tape_x + n * 3 * h.stride, 3 * h.stride);
    }
    if (syn && mech[M_EXPSYN].present && mech[M_EXPSYN].n > 0) {
        const MechDev& e = mech[M_EXPSYN].dev;
        seg(e.col(ES_G), d_tape_g + n * e.n, e.n);
    }
    if (d_tape_c) {            // Ca_HVA m, h are consecutive columns
        const MechDev& c = mech[M_CAHVA].dev;
        seg(c.col(CH_M), d_tape_c + n * 2 * c.stride, 2 * c.stride);
    }
    if (d_tape_l) {
        const MechDev& h = mech[M_HDLA].dev;
        seg(h.col(HD_L), d_tape_l + n * h.n, h.n);
    }
    if (d_tape_cai) {
        const MechDev& ca = mech[M_CA_ION].dev;
        seg(ca.col(ION_CONCI), d_tape_cai + n * ca.n, ca.n);
    }
    if (syn && d_tape_ab) {
        const MechDev& e = mech[M_EXP2SYN].dev;
        seg(e.col(E2_A), d_tape_ab + n * 2 * e.n, e.n);
        seg(e.col(E2_B), d_tape_ab + (n * 2 + 1) * e.n, e.n);
    }
    return T;
}

// Gap transfers after the update (and at finitialize): the model's HalfGap
// sources, then the transfers added at run time.
void hx_sim::launch_gap_transfers() {
    const bool stat = static_gaps_on && !gaps.empty();
    if (!stat && dg_src.empty()) return;
    upload_gap_ptrs();
    tbegin(T_OTHER);
    if (stat)
        launch_gap(d_v, d_gap_src, mech[M_HALFGAP].dev.col(HG_VGAP), d_gap_inst, static_cast<int>(gaps_eff.size()), stream);
    launch_copy_ptrs(d_dg_src, d_dg_dst, static_cast<int>(dg_src.size()), stream);
    tend(T_OTHER);
}

void hx_sim::upload_gap_ptrs() {
    if (dg_dirty) {
        d_dg_src = dg_src.empty() ? nullptr : slot_upload(dg_src_slot, dg_src);
        d_dg_dst = dg_dst.empty() ? nullptr : slot_upload(dg_dst_slot, dg_dst);
        dg_dirty = false;
    }
}

bool hx_sim::want_multi_stream() const {
    return group_streams_allowed && groups.size() > 1 && fused && vecplay.empty() && !tape_on && dg_src.empty() &&
           !(learn && learn->capturing()) && (mon_ref.empty() || mon_all_v);
}

// One fadvance with each cell group's chain on its own stream: the same
// launches as step_once, restricted to the group's nodes, cells, detectors and
// synapses, in the same order.
void hx_sim::step_once_groups() {
    const double tk = t;
    const double tmid = tk + 0.5 * dt;
    double tn = tk;
    tn += 0.5 * dt;
    tn += 0.5 * dt;
    const bool pending = state_pending;
    const bool sample = pending && !pending_sampled;   // a deferred call end sampled already
    const size_t nm = mon_ref.size();
    if (sample && nm && mon_buf_fill >= mon_buf_cap) throw std::runtime_error("monitor buffer exhausted");
    // the last step of a call with outputs on demand leaves calcium to the state update,
    // so the outputs pass reads the concentration its current evaluation used
    const bool eager = cadyn_eager && !(final_step && lazy_outputs_run);
    pass_cadyn_skip = cadyn_done ? 1 : 0;
    pass_cadyn_after = eager ? 1 : 0;
    // First step of a run: each group starts once the previous group's node pass is
    // done, so from then on one group's tree solve (latency-bound) runs beside the
    // other's node pass (HBM-bound) instead of two node passes and then two solves
    // running together.  With turns (the default) every step keeps that order: a
    // group's step waits for the previous group's node pass (group 0 for the last
    // group's pass of the step before).  The wait sits ahead of the group's event
    // kernels, so when a node pass ends, its group's solve (the next launch on that
    // stream) is dispatched before the next group's node pass, which otherwise fills
    // every CU first and leaves the solve's workgroups waiting for room.  The ordering
    // is through events only: results are unchanged.
    const bool turns = group_turns != 0;
    const bool stagger = stagger_next && !turns;
    stagger_next = false;
    const int G = static_cast<int>(groups.size());
    for (int g = 0; g < G; ++g) {
        CellGroup& cg = groups[g];
        hipStream_t s = cg.s;
        // the group's voltage samples (every monitor samples a voltage here, and the node
        // pass leaves v as it finds it)
        auto record = [&]() {
            if (sample && cg.mon1 > cg.mon0)
                hx::launch_record(d_mon_ptr + cg.mon0, cg.mon1 - cg.mon0, d_mon_buf + mon_buf_fill * nm + cg.mon0, s);
        };
        if (turns) {
            // the events and samples do not touch the other groups: they run during the
            // previous group's node pass, and only the node pass waits.  The wait's own
            // latency keeps this node pass behind the previous group's solve, which follows
            // its node pass directly (measured: a solve launched that way is dispatched
            // 10-15 us ahead; with the delivery after the wait as well the step was 1% slower)
            launch_events_group(g, k, tk, s);
            record();
            if (g > 0) HXC(hipStreamWaitEvent(s, groups[g - 1].pass_mark, 0));
            else if (turns_prev) HXC(hipStreamWaitEvent(s, groups[G - 1].pass_mark, 0));
            pass_yform = solve_voltage ? 1 : 0;
            launch_mech_pass(pending ? 1 : 0, 1, tmid, g, s);
            pass_yform = 0;
            // the next group waits for this mark; when the node kernel is timed, its end event
            // (set by the kernel's dispatch, nothing launched after it) marks the same point
            cg.pass_mark = mech_end_mark;
            if (!cg.pass_mark) {
                HXC(hipEventRecord(cg.pass, s));
                cg.pass_mark = cg.pass;
            }
        } else {
            if (stagger && g > 0) HXC(hipStreamWaitEvent(s, ev_stagger, 0));
            launch_events_group(g, k, tk, s);
            pass_yform = solve_voltage ? 1 : 0;
            launch_mech_pass(pending ? 1 : 0, 1, tmid, g, s);
            pass_yform = 0;
            if (stagger && g + 1 < G) HXC(hipEventRecord(ev_stagger, s));
            record();
        }
        SolveArgs S{};
        S.waves = solve_waves;
        S.nunit = cg.unit1 - cg.unit0;
        S.unit_node_begin = d_unit_node_begin + cg.unit0;
        S.unit_desc_begin = d_unit_desc_begin + cg.unit0;
        S.unit_round_begin = d_unit_round_begin + cg.unit0;
        S.rounds = d_rounds;
        S.desc = d_desc;
        S.v = d_v;
        S.d = d_d;
        S.rhs = d_rhs;
        S.w = d_w;
        S.a = d_sa;
        S.b = d_sb;
        S.store_dx = store_dx() ? 1 : 0;
        S.res_nodes = res_nodes;
        S.res_rounds = max_rounds;
        S.yform = solve_voltage ? 1 : 0;
        tbegin(T_SOLVE, s);
        launch_solve(S, max_slots, s);
        tend(T_SOLVE, s);
        // the group's detection of the next step and its synapses' decay, one launch
        tbegin(T_SPIKE, s);
        launch_after_solve(after_solve_args(tn, k + 1, g), s);
        tend(T_SPIKE, s);
    }
    turns_prev = turns;
    if (sample && nm) mon_buf_fill++;
    pending_sampled = false;
    cadyn_done = eager;
    pass_cadyn_skip = pass_cadyn_after = 0;
    t = tn;
    k += 1;
    state_pending = true;
}

// One Simulate::fadvance (simulate.cpp:410-442).  On entry spikes for step k
// have been detected (end of the previous step or finitialize).
void hx_sim::step_once() {
    // a full tape stops the call before the step issues anything, so the model stays at
    // the last taped step
    if (tape_on && tape_n >= tape_cap)
        throw std::runtime_error("adjoint tape full (" + std::to_string(tape_cap) + " steps): call hx_tape_begin "
                                 "with more steps");
    if (multi_stream) {
        step_once_groups();
        return;
    }
    const double tk = t;
    const double tmid = tk + 0.5 * dt;
    const bool has_vp = !vecplay.empty();
    const int nvp = static_cast<int>(vecplay.size());
    if (fused) {
        // events and VecPlay touch only point processes here (a non-point VecPlay
        // target selects the split schedule), so they may precede the previous
        // step's deferred state update; the node kernel then adds the synapse
        // currents with this step's deliveries in place
        // VecPlay writing only IClamp variables, which delivery never touches, runs on blocks
        // of the delivery launch
        const bool vp_in_events = has_vp && vecplay_iclamp_only;
        const bool vp_done = launch_events(k, tk, vp_in_events ? tmid : -1.0);
        if (has_vp && !vp_done) { tbegin(T_OTHER); launch_vecplay(d_vecplay, nvp, tmid, 1, stream); tend(T_OTHER); }
        const bool eager = cadyn_eager && !(final_step && lazy_outputs_run);   // as in step_once_groups
        pass_cadyn_skip = cadyn_done ? 1 : 0;
        pass_cadyn_after = eager ? 1 : 0;
        pass_yform = solve_voltage ? 1 : 0;
        launch_mech_pass(state_pending ? 1 : 0, 1, tmid);
        pass_yform = 0;
        cadyn_done = eager;
        pass_cadyn_skip = pass_cadyn_after = 0;
        if (state_pending && !pending_sampled) launch_record();
        pending_sampled = false;
    } else {
        launch_events(k, tk);
        if (has_vp) { tbegin(T_OTHER); launch_vecplay(d_vecplay, nvp, tmid, 1, stream); tend(T_OTHER); }
        pass_yform = solve_voltage ? 1 : 0;
        launch_mech_pass(0, 1, tmid);
        pass_yform = 0;
    }
    launch_point_currents(tmid);
    launch_plugin_currents(tmid);
    SolveArgs S{};
    S.waves = solve_waves;
    S.nunit = nunit;
    S.unit_node_begin = d_unit_node_begin;
    S.unit_desc_begin = d_unit_desc_begin;
    S.unit_round_begin = d_unit_round_begin;
    S.rounds = d_rounds;
    S.desc = d_desc;
    S.v = d_v;
    S.d = d_d;
    S.rhs = d_rhs;
    S.w = d_w;
    S.a = d_sa;
    S.b = d_sb;
    S.store_dx = store_dx() ? 1 : 0;
    S.res_nodes = res_nodes;
    S.res_rounds = max_rounds;
    S.yform = solve_voltage ? 1 : 0;
    tbegin(T_SOLVE);
    launch_solve(S, max_slots, stream);
    tend(T_SOLVE);
    // gap transfers, detection of the next step (spike_deliver detects on v_{k}), VecPlay
    // at the step's end and the synapses' decay: one launch when VecPlay writes only IClamp
    // variables, which none of the others touch, and no transfer added at run time (which
    // may name any variable) is in the step; the step's tape row then rides on it too
    const bool one_launch = (!has_vp || vecplay_iclamp_only) && dg_src.empty();
    if (tape_on && !one_launch) tape_record();
    if (!one_launch) launch_gap_transfers();
    // t += dt/2 twice, exactly as the reference accumulates it
    double tn = tk;
    tn += 0.5 * dt;
    tn += 0.5 * dt;
    t = tn;
    k += 1;
    if (one_launch) {
        upload_gap_ptrs();
        AfterSolve P = after_solve_args(t, k, -1);
        if (tape_on) {
            const size_t n = static_cast<size_t>(tape_n);
            P.tape = tape_row(false);
            if (P.es_g) P.es_tape = d_tape_g + n * mech[M_EXPSYN].dev.n;
            if (P.e2_a && d_tape_ab) {
                const size_t ne2 = static_cast<size_t>(mech[M_EXP2SYN].dev.n);
                P.e2_tape_a = d_tape_ab + n * 2 * ne2;
                P.e2_tape_b = d_tape_ab + (n * 2 + 1) * ne2;
            }
            ++tape_n;
        }
        tbegin(T_SPIKE);
        launch_after_solve(P, stream);
        tend(T_SPIKE);
    } else {
        launch_detect(k, t);
        tbegin(T_OTHER);
        launch_vecplay(d_vecplay, nvp, t, 0, stream);
        tend(T_OTHER);
        StepArgs A = step_args(t, 1, 0);
        if (mech[M_EXPSYN].present || mech[M_EXP2SYN].present) {
            tbegin(T_POINT);
            launch_point_state(M_EXPSYN, A, stream);
            launch_point_state(M_EXP2SYN, A, stream);
            tend(T_POINT);
        }
    }
    launch_plugin_states(t);
    if (fused) {
        state_pending = true;
    } else {
        launch_mech_pass(1, 0, t);
        launch_record();
    }
}

void hx_sim::finish_pending() {
    if (!state_pending) return;
    pass_cadyn_skip = cadyn_done ? 1 : 0;
    struct Reset {   // the pending pass completes this step's updates
        hx_sim* s;
        ~Reset() { s->pass_cadyn_skip = 0; s->cadyn_done = false; }
    } reset{this};
    if (multi_stream) {
        const size_t nm = mon_ref.size();
        if (nm && mon_buf_fill >= mon_buf_cap) throw std::runtime_error("monitor buffer exhausted");
        for (int g = 0; g < static_cast<int>(groups.size()); ++g) {
            CellGroup& cg = groups[g];
            launch_mech_pass(1, 0, t, g, cg.s);
            if (!pending_sampled && cg.mon1 > cg.mon0)
                hx::launch_record(d_mon_ptr + cg.mon0, cg.mon1 - cg.mon0, d_mon_buf + mon_buf_fill * nm + cg.mon0,
                                  cg.s);
        }
        if (nm && !pending_sampled) mon_buf_fill++;
        pending_sampled = false;
        state_pending = false;
        return;
    }
    launch_mech_pass(1, 0, t);
    if (!pending_sampled) launch_record();
    pending_sampled = false;
    state_pending = false;
}

// The closing pass may wait for the next call when nothing samples the states
// inside the step loop: every monitor samples a voltage (taken at the call's end,
// sample_pending_step), no tape and no signal capture.
bool hx_sim::close_may_defer() const {
    return defer_allowed && close_deferral && fused && (mon_ref.empty() || mon_all_v) && !tape_on &&
           !(learn && learn->capturing());
}
bool hx_sim::can_defer_close() const { return state_pending && close_may_defer(); }

// Outputs on demand need the node kernel to make every density mechanism's outputs
// (an instance-parallel mechanism or a plugin adds ion currents after it) and no
// handle or transfer that reads outputs inside the step loop.
bool hx_sim::lazy_outputs_ok() const {
    if (!close_may_defer() || write_assigned || !dg_src.empty() || !plugins.empty()) return false;
    for (int id : kSparseOrder)
        if (mech[id].present && !(dense_mask & (1u << id))) return false;
    return dense_mask != 0;
}

// The node kernel's assigned outputs of the call's last step: its current evaluation
// again, on the voltages before that step's solve (kept in w by k_solve<1>) and the
// states it used (their update is still pending).  Its d and rhs go to w too (each
// thread reads its own voltage there before it stores), so the solve's pivots and x
// stay in d and rhs.
void hx_sim::launch_outputs_pass() {
    const bool f = final_step, l = lazy_outputs_run;
    final_step = true;
    lazy_outputs_run = false;      // this pass stores the outputs
    pass_cadyn_after = 0;
    StepArgs A = step_args(t - 0.5 * dt, 0, 1);
    final_step = f;
    lazy_outputs_run = l;
    A.v = d_w;
    A.d = d_w;
    A.rhs = d_w;
    A.fold_mask = 0;
    A.point_assigned = 0;
    tbegin(T_MECH);
    launch_dense(A, stream, dense_steady != 0);
    tend(T_MECH);
    outputs_pending = false;
}

// A deferred call end still records the last step's samples: a voltage after the
// solve, which the pending state update does not change.
void hx_sim::sample_pending_step() {
    const size_t nm = mon_ref.size();
    if (nm == 0) return;
    if (mon_buf_fill >= mon_buf_cap) throw std::runtime_error("monitor buffer exhausted");
    if (multi_stream) {
        for (auto& cg : groups)
            if (cg.mon1 > cg.mon0)
                hx::launch_record(d_mon_ptr + cg.mon0, cg.mon1 - cg.mon0, d_mon_buf + mon_buf_fill * nm + cg.mon0,
                                  cg.s);
        mon_buf_fill++;
    } else {
        launch_record();
    }
    pending_sampled = true;
}

// Completes a deferred state update with the pass the call would have closed with
// (it also stores the rates, as a call's closing pass does) and waits for it.
int hx_sim::settle() {
    if (!state_pending) return 0;
    const bool prof = profiling;
    profiling = false;                 // the kernel timers cover stepping calls only
    try {
        if (outputs_pending) launch_outputs_pass();
        final_step = true;
        finish_pending();
        final_step = false;
        HXC(hipStreamSynchronize(stream));
    } catch (const std::exception& e) {
        final_step = false;
        profiling = prof;
        return fail("%s", e.what());
    }
    profiling = prof;
    return 0;
}

void hx_sim::sync_outputs() {
    if (!d_spk_count || !d_ring_overflow) {   // no model loaded
        HXC(hipStreamSynchronize(stream));
        return;
    }
    // one kernel gathers the flags and the spike count into pinned host memory, so the
    // host reads them after the synchronisation without a copy each
    if (!h_status) HXC(hipHostMalloc(reinterpret_cast<void**>(&h_status), 4 * sizeof(int), hipHostMallocDefault));
    // the call's monitor samples travel behind it on the stream, into pinned memory
    const size_t nmon = mon_ref.empty() ? 0 : static_cast<size_t>(mon_buf_fill) * mon_ref.size();
    if (nmon > 0) {
        if (h_mon_cap < nmon) {
            if (h_mon) HXC(hipHostFree(h_mon));
            h_mon = nullptr;
            h_mon_cap = std::max(nmon, 2 * h_mon_cap);
            HXC(hipHostMalloc(reinterpret_cast<void**>(&h_mon), sizeof(double) * h_mon_cap, hipHostMallocDefault));
        }
        HXC(hipMemcpyAsync(h_mon, d_mon_buf, sizeof(double) * nmon, hipMemcpyDeviceToHost, stream));
    }
    StatusArgs sa{d_ring_overflow, static_cast<int>(groups.size()), nsa.n > 0 ? nsa.error : nullptr, d_spk_count,
                  h_status};
    launch_status(sa, stream);
    HXC(hipGetLastError());
    HXC(hipStreamSynchronize(stream));
    if (profiling) tcollect();
    if (h_status[0]) throw std::runtime_error("event ring overflow: raise the per-step capacity with hx_set_event_capacity");
    if (nsa.n > 0) {
        const int e = h_status[1];
        if (e & 1) throw std::runtime_error("NetStim event inbox overflow");
        if (e & 2) throw std::runtime_error("more than 8 events reached one NetStim in one pass of a step");
        if (e & 4) throw std::runtime_error("a step's delivery loop needed more than 64 passes (NetStim interval too small?)");
        if (e & 8) throw std::runtime_error("a NetStim has more than 8 pending self events");
    }
    const int ns = h_status[2];
    if (ns > spk_cap) throw std::runtime_error("spike log overflow");
    {
        std::vector<std::pair<double, int>> fresh;
        fresh.swap(spikes_held);
        if (ns > 0) {
            std::vector<double> st(ns);
            std::vector<int> sg(ns);
            HXC(hipMemcpy(st.data(), d_spk_t, sizeof(double) * ns, hipMemcpyDeviceToHost));
            HXC(hipMemcpy(sg.data(), d_spk_gid, sizeof(int) * ns, hipMemcpyDeviceToHost));
            for (int i = 0; i < ns; ++i) fresh.push_back({st[i], sg[i]});
            HXC(hipMemset(d_spk_count, 0, sizeof(int)));
        }
        const double edge = t - 0.5 * dt;      // spikes at the current t belong to the step not yet taken
        for (auto& e : fresh) {
            if (k > 0 && e.first > edge) {
                spikes_held.push_back(e);
                continue;
            }
            spikes.push_back(e);
            spk_by_gid[e.second].push_back(e.first);
        }
    }
    if (nmon > 0) {
        const size_t nm = mon_ref.size();
        for (long long s = 0; s < mon_buf_fill; ++s)
            for (size_t i = 0; i < nm; ++i) mon_data[i].push_back(h_mon[s * nm + mon_col[i]]);
        mon_buf_fill = 0;
    }
    if (h5_on) h5_append();
}

// The new samples of every monitor go to its dataset /group_0/<mech>/<var>/<idx>; a
// (mech, var, idx) monitored twice has one dataset, written from its first monitor.
void hx_sim::h5_append() {
    if (!h5) h5.reset(new H5Recorder());
    if (!h5->is_open()) h5->open(output_dir);
    h5_written.resize(mon_data.size(), 0);
    std::set<std::tuple<std::string, std::string, int>> seen;
    for (size_t i = 0; i < mon_data.size(); ++i) {
        if (!seen.insert({mon_name[i].first, mon_name[i].second, mon_idx[i]}).second) continue;
        const size_t have = mon_data[i].size();
        if (have > h5_written[i])
            h5->append(mon_name[i].first, mon_name[i].second, mon_idx[i], mon_data[i].data() + h5_written[i],
                       have - h5_written[i]);
        h5_written[i] = have;
    }
}

int hx_sim::run_steps(int nstep) {
    if (!initialized) throw std::runtime_error("finitialize must be called before stepping");
    ensure_ttab(k + nstep + 1);
    refresh_cadyn_eager();
    if (mech[M_NETSTIM].present && mech[M_NETSTIM].n > 0 && k + nstep + 2 > ns_horizon) {
        // longer trains: the streams restart, so the events already delivered come
        // out the same and only events past the old horizon are added
        make_netstim_trains(std::max(2 * ns_horizon, k + nstep + 2 + kNetStimHorizon0));
        upload_inputs();
    }
    if (mon_dirty) upload_monitors();
    if (vecplay_dirty) upload_vecplay();
    ensure_mon_rows(nstep + 2);
    // Assigned variables (ion currents and reversal potentials, hh ina, minf,
    // ...) with no reader inside the step are not stored on every step; the
    // last step of the call stores them all, so they read back as after the
    // reference's last step.
    final_step = false;
    outputs_pending = false;           // this call's last step makes new ones
    lazy_outputs_run = lazy_outputs_ok();
    // cell groups on their own streams: they start after everything already on
    // the library stream, and the library stream waits for all of them
    multi_stream = want_multi_stream();
    last_multi_stream = multi_stream;
    if (multi_stream) {
        HXC(hipEventRecord(ev_main, stream));
        for (auto& cg : groups) HXC(hipStreamWaitEvent(cg.s, ev_main, 0));
        stagger_next = stagger_groups != 0;
        turns_prev = false;
    }
    try {
        for (int s = 0; s < nstep; ++s) {
            final_step = s == nstep - 1;
            step_once();
        }
        if (can_defer_close()) {
            sample_pending_step();
            outputs_pending = lazy_outputs_run;
        } else {
            if (lazy_outputs_run) launch_outputs_pass();
            finish_pending();
        }
    } catch (...) {
        if (multi_stream) {
            for (auto& cg : groups) (void)hipStreamSynchronize(cg.s);
            multi_stream = false;
        }
        throw;
    }
    if (multi_stream) {
        for (auto& cg : groups) {
            HXC(hipEventRecord(cg.done, cg.s));
            HXC(hipStreamWaitEvent(stream, cg.done, 0));
        }
        multi_stream = false;
    }
    final_step = false;
    sync_outputs();
    return 0;
}

// INITIAL of the NetStims that receive events (netstim.cpp:211-246, one stream per
// instance, sequence 0): noise clamped to [0, 1]; with start >= 0 and number > 0 the
// instance is on and its init event waits at start + invl - interval (1 - noise) (0 if
// negative).  Parameters are taken from the host copy, as the trains of the others are.
void hx_sim::upload_ns_dyn_state() {
    const int n = nsa.n;
    if (n == 0) return;
    HXC(hipStreamSynchronize(stream));      // nothing of an earlier run still uses the state
    const HostMech& m = mech[M_NETSTIM];
    std::vector<double> interval(n), number(n), noise(n), on(n, 0.0), ispike(n, 0.0), event(n, 0.0);
    std::vector<double> qt(static_cast<size_t>(n) * kNsQueue, 0.0);
    std::vector<int> qkind(static_cast<size_t>(n) * kNsQueue, 0), qn(n, 0);
    std::vector<long long> qborn(static_cast<size_t>(n) * kNsQueue, 0);
    std::vector<unsigned> rw(static_cast<size_t>(n) * kNsRng);
    for (int j = 0; j < n; ++j) {
        const int i = ns_dyn_inst[j];
        interval[j] = m.col[NS_INTERVAL][i];
        number[j] = m.col[NS_NUMBER][i];
        noise[j] = std::min(1.0, std::max(0.0, m.col[NS_NOISE][i]));
        Stream123 rng;
        const double id1 = m.col[NS_ID1][i];
        rng.set_ids(id1 < 0 ? static_cast<uint32_t>(i) : static_cast<uint32_t>(id1),
                    static_cast<uint32_t>(m.col[NS_ID2][i]), static_cast<uint32_t>(m.col[NS_ID3][i]));
        rng.set_seq(0, 0);
        const double start = m.col[NS_START][i];
        if (start >= 0.0 && number[j] > 0) {
            on[j] = 1.0;
            double mean = interval[j] <= 0.0 ? 0.01 : interval[j];
            if (noise[j] != 0) mean = (1.0 - noise[j]) * mean + noise[j] * mean * rng.negexp();
            event[j] = start + mean - interval[j] * (1.0 - noise[j]);
            if (event[j] < 0.0) event[j] = 0.0;
            qt[static_cast<size_t>(j) * kNsQueue] = event[j];
            qkind[static_cast<size_t>(j) * kNsQueue] = 1;
            qn[j] = 1;
        }
        rng.save(&rw[static_cast<size_t>(j) * kNsRng]);
    }
    auto up = [&](auto* dst, const auto& v) {
        HXC(hipMemcpy(dst, v.data(), sizeof(v[0]) * v.size(), hipMemcpyHostToDevice));
    };
    up(nsa.interval, interval);
    up(nsa.number, number);
    up(nsa.noise, noise);
    up(nsa.on, on);
    up(nsa.ispike, ispike);
    up(nsa.event, event);
    up(nsa.q_t, qt);
    up(nsa.q_kind, qkind);
    up(nsa.q_born, qborn);
    up(nsa.q_n, qn);
    up(nsa.rng, rw);
    HXC(hipMemset(nsa.mini_n, 0, sizeof(int) * n));
    HXC(hipMemset(nsa.log_count, 0, sizeof(int)));
    HXC(hipMemset(nsa.error, 0, sizeof(int)));
    HXC(hipMemset(nsa.ib.count, 0, sizeof(int) * nsa.ib.nslot));
}

// Simulate::finitialize (simulate.cpp:106-141, 271-339)
void hx_sim::finitialize(double v_init) {
    if (mech[M_NETSTIM].present && mech[M_NETSTIM].n > 0) {
        make_netstim_trains(std::max(ns_horizon, kNetStimHorizon0));
        inputs_dirty = true;
    }
    if (inputs_dirty || vecstim_run_differs) {   // every VecStim starts its own vector again
        vecstim_run = vecstim;
        vecstim_run_differs = false;
        inputs_dirty = true;
    }
    if (inputs_dirty) upload_inputs();
    if (vecplay_dirty) upload_vecplay();
    if (mon_dirty) upload_monitors();
    t = 0.0;
    k = 0;
    state_pending = false;
    pending_sampled = false;
    outputs_pending = false;
    lazy_outputs_run = false;
    cadyn_done = false;
    pass_cadyn_skip = pass_cadyn_after = 0;
    ensure_ttab(1);
    ensure_mon_rows(2);
    mon_buf_fill = 0;
    for (auto& md : mon_data) md.clear();
    h5_written.assign(mon_data.size(), 0);     // the file keeps growing across finitialize
    // the spike record keeps growing across finitialize, as the reference's rec_spikes and
    // per-gid spk_output do (simulate.cpp:880, presyn.cpp:155; nothing clears them); a
    // crossing found after the last step belongs to a step that is not taken now
    spikes_held.clear();
    const int nvp = static_cast<int>(vecplay.size());
    if (nvp) {
        launch_vecplay_reset(d_vecplay, nvp, stream);
        launch_vecplay(d_vecplay, nvp, 0.0, 1, stream);
    }
    for (auto& cg : groups) {
        launch_clear_ints(cg.ring.count, cg.ring.nslot, stream);
        launch_clear_ints(cg.ring.overflow, 1, stream);
        launch_clear_ints(reinterpret_cast<int*>(cg.ring.done), 1, stream);
        launch_clear_ints(cg.d_in_cursor, 1, stream);
    }
    launch_clear_ints(d_pre_flag, npre, stream);
    launch_clear_ints(d_spk_count, 1, stream);
    for (const auto& p : plugins)
        if (p.d_recv_count) launch_clear_ints(p.d_recv_count, p.h.n, stream);
    upload_ns_dyn_state();
    if (tape_on) {
        tape_n = 0;
        launch_clear_ints(d_tape_evn, tape_cap, stream);
    }
    launch_set_v(d_v, nnode, v_init, stream);
    if (tape_on)
        HXC(hipMemcpyAsync(d_tape_v0, d_v, sizeof(double) * nnode, hipMemcpyDeviceToDevice, stream));
    launch_gap_transfers();
    StepArgs A = step_args(0.0, 0, 0);
    for (int id = 0; id < M_COUNT; ++id)           // CoreNEURON order, ions before their users
        if (mech[id].present) launch_init(id, A, stream);
    launch_plugin_inits(0.0);
    launch_record();
    launch_detect(0, 0.0);
    launch_events(0, 0.0);
    final_step = true;
    init_pass = true;
    launch_mech_pass(0, 1, 0.0);
    launch_point_currents(0.0);
    launch_plugin_currents(0.0);
    init_pass = false;
    final_step = false;
    initialized = true;
    sync_outputs();
}

// ===========================================================================
// C ABI
// ===========================================================================
#define API_BEGIN try {
#define API_END                                         \
    }                                                   \
    catch (const std::exception& e) {                   \
        return sim->fail("%s", e.what());               \
    }

namespace hx {
int read_coredat(hx_sim* sim, const std::string& dir, int user_mod_num, bool take_dt, std::string& err);
}

namespace {
uint64_t fnv1a(const void* p, size_t n, uint64_t h = 1469598103934665603ull) {
    const unsigned char* c = static_cast<const unsigned char*>(p);
    for (size_t i = 0; i < n; ++i) h = (h ^ c[i]) * 1099511628211ull;
    return h;
}
template <class T>
uint64_t fnv_vec(const std::vector<T>& v) { return fnv1a(v.data(), v.size() * sizeof(T)); }
}  // namespace

// The stepping entry points (run, continue_run, fadvance) may leave their last state
// update pending; every other entry point that takes a handle completes it first.
#define HX_SETTLE(sim)                                                  \
    do {                                                                \
        if ((sim) && (sim)->state_pending && (sim)->settle() != 0) return -1; \
    } while (0)

struct DeferScope {
    hx_sim* s;
    explicit DeferScope(hx_sim* sim) : s(sim) { s->defer_allowed = true; }
    ~DeferScope() { s->defer_allowed = false; }
};

static bool check_loaded(hx_sim* sim) {
    if (!sim->loaded) { sim->fail("model not loaded (call hx_load_model)"); return false; }
    return true;
}

extern "C" {

int hx_create(hx_sim** out) {
    if (!out) return -1;
    try {
        *out = new hx_sim();
        return 0;
    } catch (...) {
        return -1;
    }
}

void hx_destroy(hx_sim* sim) { delete sim; }

const char* hx_last_error(hx_sim* sim) { return sim ? sim->err.c_str() : "null handle"; }

int hx_set_device(hx_sim* sim, const char* dev) {
    HX_SETTLE(sim);
    if (!dev || std::string(dev) != "gpu")
        return sim->fail("device '%s' is not served by this library (only \"gpu\")", dev ? dev : "");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return sim->fail("no HIP device visible");
    return 0;
}

int hx_set_dt(hx_sim* sim, double dt) {
    HX_SETTLE(sim);
    if (!(dt > 0)) return sim->fail("dt must be positive");
    sim->dt_set = true;
    if (sim->loaded && dt != sim->dt) {
        sim->dt = dt;
        sim->ttab.clear();
        sim->ttab_cap = 0;
        return 0;
    }
    sim->dt = dt;
    return 0;
}

double hx_get_dt(hx_sim* sim) { return sim->dt; }

int hx_set_celsius(hx_sim* sim, double c) {
    HX_SETTLE(sim);
    sim->celsius = c;
    return 0;
}

int hx_set_data_path(hx_sim* sim, const char* path) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("cannot set the data path after the model is loaded");
    if (!path || !*path) return sim->fail("empty data path");
    sim->data_path = path;
    return 0;
}

int hx_set_user_mod_num(hx_sim* sim, int num) {
    HX_SETTLE(sim);
    if (num <= 0) return sim->fail("user_mod_num must be positive");
    sim->user_mod_num = num;
    return 0;
}

int hx_model_set_nodes(hx_sim* sim, int ncell, int nnode, const int* parent, const double* a, const double* b,
                       const double* area) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded");
    if (ncell <= 0 || nnode < ncell || !parent || !a || !b || !area) return sim->fail("invalid node arrays");
    for (int i = 0; i < ncell; ++i)
        if (parent[i] != -1) return sim->fail("nodes [0, ncell) must be roots");
    for (int i = ncell; i < nnode; ++i)
        if (parent[i] < 0 || parent[i] >= i) return sim->fail("node %d: parent must satisfy 0 <= parent < node", i);
    sim->ncell = ncell;
    sim->nnode = nnode;
    sim->parent.assign(parent, parent + nnode);
    sim->a.assign(a, a + nnode);
    sim->b.assign(b, b + nnode);
    sim->area.assign(area, area + nnode);
    sim->cm.assign(nnode, 1.0);
    return 0;
}

int hx_model_insert(hx_sim* sim, const char* mech, int n, const int* nodes) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded");
    if (sim->nnode == 0) return sim->fail("set nodes before inserting mechanisms");
    const int id = mech_id(mech ? mech : "");
    if (id < 0) {
        const PluginMeta* pm = find_plugin(mech ? mech : "");
        if (!pm) return sim->fail("unknown mechanism '%s'", mech ? mech : "");
        if (sim->plugin_named(pm->name)) return sim->fail("mechanism '%s' inserted twice", mech);
        if (n < 0 || (n > 0 && !nodes)) return sim->fail("invalid instance list");
        std::vector<char> seen(sim->nnode, 0);
        for (int j = 0; j < n; ++j) {
            if (nodes[j] < 0 || nodes[j] >= sim->nnode) return sim->fail("%s: node index out of range", mech);
            if (!(pm->flags & plugin::kPoint)) {
                if (seen[nodes[j]]) return sim->fail("%s: density mechanism twice on node %d", mech, nodes[j]);
                seen[nodes[j]] = 1;
            }
        }
        hx_sim::PluginInst pi;
        pi.meta = pm;
        pi.h.present = true;
        pi.h.n = n;
        pi.h.node.assign(nodes, nodes + n);
        pi.h.col.assign(pm->ncol, {});
        for (int c = 0; c < pm->ncol; ++c) pi.h.col[c].assign(n, pm->dflt[c]);
        sim->plugins.push_back(std::move(pi));
        return 0;
    }
    HostMech& m = sim->mech[id];
    if (m.present) return sim->fail("mechanism '%s' inserted twice", mech);
    if (n < 0 || (n > 0 && !nodes)) return sim->fail("invalid instance list");
    const auto& M = registry()[id];
    std::vector<char> seen(sim->nnode, 0);
    for (int j = 0; j < n; ++j) {
        if (nodes[j] < 0 || nodes[j] >= sim->nnode) return sim->fail("%s: node index out of range", mech);
        if (!M.point) {
            if (seen[nodes[j]]) return sim->fail("%s: density mechanism twice on node %d", mech, nodes[j]);
            seen[nodes[j]] = 1;
        }
    }
    if (n >= (1 << 30)) return sim->fail("too many instances");
    m.present = true;
    m.n = n;
    m.node.assign(nodes, nodes + n);
    m.col.assign(M.ncol, {});
    for (int c = 0; c < M.ncol; ++c) m.col[c].assign(n, M.dflt[c]);
    if (M.ion) m.iontype.assign(n, 0);
    if (id == M_VECSTIM) sim->vecstim.assign(n, {});
    return 0;
}

int hx_model_set_param(hx_sim* sim, const char* mech, const char* var, int n, const double* vals) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded; use variable handles");
    std::string mn = mech ? mech : "", vn = var ? var : "";
    if (mn == "capacitance" && vn == "cm") {
        if (n != sim->nnode) return sim->fail("cm needs one value per node");
        sim->cm.assign(vals, vals + n);
        return 0;
    }
    const int id = mech_id(mn);
    if (id < 0) {
        hx_sim::PluginInst* p = sim->plugin_named(mn);
        if (!p) return sim->fail("mechanism '%s' not inserted", mn.c_str());
        int c = -1;
        for (int k = 0; k < p->meta->ncol; ++k)
            if (vn == p->meta->cols[k]) c = k;
        if (c < 0) return sim->fail("%s has no variable '%s'", mn.c_str(), vn.c_str());
        if (n != p->h.n) return sim->fail("%s.%s: expected %d values", mn.c_str(), vn.c_str(), p->h.n);
        p->h.col[c].assign(vals, vals + n);
        return 0;
    }
    if (!sim->mech[id].present) return sim->fail("mechanism '%s' not inserted", mn.c_str());
    const int c = col_id(id, vn);
    if (c < 0) return sim->fail("%s has no variable '%s'", mn.c_str(), vn.c_str());
    if (n != sim->mech[id].n) return sim->fail("%s.%s: expected %d values", mn.c_str(), vn.c_str(), sim->mech[id].n);
    sim->mech[id].col[c].assign(vals, vals + n);
    return 0;
}

int hx_model_set_global(hx_sim* sim, const char* mech, const char* var, double value) {
    HX_SETTLE(sim);
    const int id = mech_id(mech ? mech : "");
    if (id != M_HH && id != M_HDLA) return sim->fail("mechanism '%s' has no globals", mech ? mech : "");
    static const char* hh_g[] = {"celsius"};
    static const char* hd_g[] = {"celsius", "ehd", "kl", "vhalft", "a0t", "zetat", "gmt", "q10", "qtl"};
    bool ok = false;
    if (id == M_HH) for (auto g : hh_g) ok |= std::string(var) == g;
    if (id == M_HDLA) for (auto g : hd_g) ok |= std::string(var) == g;
    if (!ok) return sim->fail("%s has no global '%s'", mech, var);
    sim->globals[id][var] = value;
    return 0;
}

int hx_model_set_iontype(hx_sim* sim, const char* ion, int n, const int* it) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded");
    const int id = mech_id(ion ? ion : "");
    if (id < 0 || !registry()[id].ion || !sim->mech[id].present) return sim->fail("ion '%s' not inserted", ion ? ion : "");
    if (n != sim->mech[id].n) return sim->fail("iontype needs one value per ion instance");
    sim->mech[id].iontype.assign(it, it + n);
    return 0;
}

int hx_model_add_presyn(hx_sim* sim, int gid, int node, double thr) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded");
    if (node < 0 || node >= sim->nnode) return sim->fail("presyn node out of range");
    sim->pre_gid.push_back(gid);
    sim->pre_node.push_back(node);
    sim->pre_thr.push_back(thr);
    return static_cast<int>(sim->pre_node.size()) - 1;
}

int hx_model_set_vecstim(hx_sim* sim, int inst, int n, const double* times) {
    HX_SETTLE(sim);
    HostMech& m = sim->mech[M_VECSTIM];
    if (!m.present || inst < 0 || inst >= m.n) return sim->fail("VecStim instance %d does not exist", inst);
    if (n < 0 || (n > 0 && !times)) return sim->fail("invalid spike-time array");
    sim->vecstim[inst].assign(times, times + n);
    sim->inputs_dirty = true;
    return 0;
}

int hx_call_mech_func(hx_sim* sim, const char* mech, const char* func, int inst, int n, const double* data) {
    HX_SETTLE(sim);
    API_BEGIN
    const std::string mn = mech ? mech : "", fn = func ? func : "";
    // the reference's FunctionRegistry holds one function (vecevent.h:42-45)
    if (mn != "VecStim" || fn != "play") return sim->fail("function not registered: %s.%s", mn.c_str(), fn.c_str());
    HostMech& m = sim->mech[M_VECSTIM];
    if (!m.present || inst < 0 || inst >= m.n) return sim->fail("VecStim instance %d does not exist", inst);
    if (n <= 0) return 0;                       // update_sequence returns without a change
    if (!data) return sim->fail("VecStim.play: null spike-time array");
    return sim->vecstim_play(inst, data, n);
    API_END
}

int hx_model_add_netcon(hx_sim* sim, int src_kind, int src, const char* target, int inst, double w, double delay) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded");
    int id = mech_id(target ? target : "");
    if (id < 0) {                     // a synapse plugin
        hx_sim::PluginInst* p = sim->plugin_named(target ? target : "");
        if (!p || !(p->meta->flags & plugin::kPostsyn))
            return sim->fail("netcon target must be ExpSyn, Exp2Syn, NetStim or a synapse plugin");
        if (inst < 0 || inst >= p->h.n) return sim->fail("netcon target instance out of range");
        id = kPluginMechBase + static_cast<int>(p - sim->plugins.data());
    } else {
        if (id != M_EXPSYN && id != M_EXP2SYN && id != M_NETSTIM)
            return sim->fail("netcon target must be ExpSyn, Exp2Syn, NetStim or a synapse plugin");
        if (!sim->mech[id].present || inst < 0 || inst >= sim->mech[id].n)
            return sim->fail("netcon target instance out of range");
    }
    if (src_kind == 0 && (src < 0 || src >= static_cast<int>(sim->pre_node.size())))
        return sim->fail("netcon source detector out of range");
    if (src_kind == 1 && (!sim->mech[M_VECSTIM].present || src < 0 || src >= sim->mech[M_VECSTIM].n))
        return sim->fail("netcon source VecStim out of range");
    if (src_kind == 2 && (!sim->mech[M_NETSTIM].present || src < 0 || src >= sim->mech[M_NETSTIM].n))
        return sim->fail("netcon source NetStim out of range");
    if (src_kind < 0 || src_kind > 2) return sim->fail("src_kind must be 0, 1 or 2");
    if (!(delay >= 0)) return sim->fail("netcon delay must be >= 0");
    sim->netcons.push_back({src_kind, src, id, inst, w, delay});
    return 0;
}

int hx_model_add_gap(hx_sim* sim, int src_node, int hg) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded");
    if (src_node < 0 || src_node >= sim->nnode) return sim->fail("gap source node out of range");
    if (!sim->mech[M_HALFGAP].present || hg < 0 || hg >= sim->mech[M_HALFGAP].n)
        return sim->fail("HalfGap instance out of range");
    sim->gaps.push_back({src_node, hg});
    return 0;
}

int hx_model_digest(hx_sim* sim, char* out, int cap) {
    HX_SETTLE(sim);
    std::string d;
    char buf[512];
    auto add = [&](const char* fmt, auto... args) {
        snprintf(buf, sizeof(buf), fmt, args...);
        d += buf;
    };
    add("ncell %d nnode %d dt %.17g celsius %.17g\n", sim->ncell, sim->nnode, sim->dt, sim->celsius);
    add("nodes parent %016llx a %016llx b %016llx area %016llx cm %016llx\n",
        (unsigned long long)fnv_vec(sim->parent), (unsigned long long)fnv_vec(sim->a),
        (unsigned long long)fnv_vec(sim->b), (unsigned long long)fnv_vec(sim->area),
        (unsigned long long)fnv_vec(sim->cm));
    const auto& R = registry();
    for (int id = 0; id < M_COUNT; ++id) {
        const HostMech& m = sim->mech[id];
        if (!m.present) continue;
        // artificial cells sit on no node: their node list is not part of the model
        add("mech %s n %d node %016llx", R[id].name, m.n,
            (unsigned long long)(R[id].artificial ? 0 : fnv_vec(m.node)));
        for (size_t c = 0; c < m.col.size(); ++c) add(" c%zu %016llx", c, (unsigned long long)fnv_vec(m.col[c]));
        if (!m.iontype.empty()) add(" style %016llx", (unsigned long long)fnv_vec(m.iontype));
        for (const auto& g : sim->globals[id]) add(" %s=%.17g", g.first.c_str(), g.second);
        d += "\n";
    }
    add("presyn %zu gid %016llx node %016llx thr %016llx\n", sim->pre_node.size(),
        (unsigned long long)fnv_vec(sim->pre_gid), (unsigned long long)fnv_vec(sim->pre_node),
        (unsigned long long)fnv_vec(sim->pre_thr));
    uint64_t h = 1469598103934665603ull;
    size_t nt = 0;
    for (const auto& v : sim->vecstim) {
        const size_t n = v.size();
        h = fnv1a(&n, sizeof(n), h);
        h = fnv1a(v.data(), n * sizeof(double), h);
        nt += n;
    }
    add("vecstim %zu times %zu %016llx\n", sim->vecstim.size(), nt, (unsigned long long)h);
    // netcons in (target, instance) order: only the last one per instance acts
    std::map<std::pair<int, int>, NetCon> last;
    for (const auto& nc : sim->netcons) last[{nc.mech, nc.inst}] = nc;
    h = 1469598103934665603ull;
    for (const auto& e : last) {
        const NetCon& nc = e.second;
        const int iv[4] = {nc.src_kind, nc.src, nc.mech, nc.inst};
        const double dv[2] = {nc.weight, nc.delay};
        h = fnv1a(iv, sizeof(iv), h);
        h = fnv1a(dv, sizeof(dv), h);
    }
    add("netcon %zu %016llx\n", last.size(), (unsigned long long)h);
    // one transfer per HalfGap instance: their order does not matter
    auto gaps = sim->gaps;
    std::sort(gaps.begin(), gaps.end(), [](const auto& x, const auto& y) {
        return x.second != y.second ? x.second < y.second : x.first < y.first;
    });
    h = fnv1a(gaps.data(), gaps.size() * sizeof(gaps[0]));
    add("gap %zu %016llx\n", sim->gaps.size(), (unsigned long long)h);
    for (const auto& vp : sim->vecplay)
        add("vecplay %s.%s[%d] %zu t %016llx y %016llx\n", vp.mech.c_str(), vp.var.c_str(), vp.idx, vp.tvec.size(),
            (unsigned long long)fnv_vec(vp.tvec), (unsigned long long)fnv_vec(vp.yvec));
    if (out && cap > 0) {
        const size_t n = std::min(d.size(), static_cast<size_t>(cap - 1));
        memcpy(out, d.data(), n);
        out[n] = 0;
    }
    return static_cast<int>(d.size()) + 1;
}

int hx_model_read_export(hx_sim* sim) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded");
    if (sim->data_path.empty()) return sim->fail("no data path set");
    if (sim->nnode != 0) return sim->fail("the model already has nodes");
    std::string err;
    const bool dt_set = sim->dt_set;
    const double dt = sim->dt, celsius = sim->celsius;
    const size_t nvp = sim->vecplay.size();
    if (hx::read_coredat(sim, sim->data_path, sim->user_mod_num, !dt_set, err) != 0) {
        const std::string msg = sim->data_path + ": " + err;
        sim->reset_model(nvp);
        sim->dt_set = dt_set;
        sim->dt = dt;
        sim->celsius = celsius;
        return sim->fail("%s", msg.c_str());
    }
    sim->data_path.clear();     // read: hx_load_model builds from what is now in the builder
    return 0;
}

int hx_load_model(hx_sim* sim) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("model already loaded");
    if (!sim->data_path.empty() && hx_model_read_export(sim) != 0) return -1;
    if (sim->nnode == 0) return sim->fail("no nodes");
    API_BEGIN
    sim->build_layout();
    sim->upload();
    sim->loaded = true;
    // resolve vecplay targets / monitors registered before load
    for (auto& vp : sim->vecplay) {
        Ref r = sim->resolve(vp.mech, vp.var, vp.idx);
        if (!r.dev) return sim->fail("vecplay target %s.%s[%d] not found", vp.mech.c_str(), vp.var.c_str(), vp.idx);
        vp.target = r.dev;
    }
    for (size_t i = 0; i < sim->mon_name.size(); ++i) {
        Ref r = sim->resolve(sim->mon_name[i].first, sim->mon_name[i].second, sim->mon_idx[i]);
        if (!r.dev) return sim->fail("monitor %s.%s[%d] not found", sim->mon_name[i].first.c_str(),
                                     sim->mon_name[i].second.c_str(), sim->mon_idx[i]);
        sim->mon_ref[i] = r;
        if (r.klass == 1 || r.point) {
            // assigned outputs are sampled where the reference records them: split passes
            sim->need_split_for_monitor = true;
            sim->write_assigned = true;
        }
    }
    sim->recompute_fused();
    return 0;
    API_END
}

int hx_finitialize(hx_sim* sim, double v_init) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    sim->finitialize(v_init);
    return 0;
    API_END
}

int hx_run(hx_sim* sim, double tstop) {
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    int nstep = static_cast<int>(tstop / sim->dt);   // simulate.cpp:345 (int nstep = tstop / dt)
    // Simulate::run restarts t at 0 without re-initializing (simulate.cpp:346)
    if (sim->k != 0) {
        sim->t = 0.0;
        sim->k = 0;
    }
    DeferScope ds(sim);
    if (nstep > 0) sim->run_steps(nstep);
    return sim->after_run();
    API_END
}

int hx_continue_run(hx_sim* sim, double runtime) {
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    int nstep = static_cast<int>(runtime / sim->dt);
    DeferScope ds(sim);
    if (nstep > 0) sim->run_steps(nstep);
    return sim->after_run();
    API_END
}

int hx_sim::after_run() { return spike_output ? hx_output_spikes(this, output_dir.c_str()) : 0; }

int hx_set_spike_output_enabled(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    sim->spike_output = enable != 0;
    return 0;
}

int hx_is_spike_output_enabled(hx_sim* sim) { return sim->spike_output ? 1 : 0; }

int hx_set_output_dir(hx_sim* sim, const char* dir) {
    HX_SETTLE(sim);
    if (!dir || !*dir) return sim->fail("set_output_dir: empty directory");
    sim->output_dir = dir;
    return 0;
}

// ---- gap junctions at run time (simulate.cpp:998-1100) ----
int hx_add_gap_source(hx_sim* sim, int sid, const char* mech, const char* var, int idx) {
    HX_SETTLE(sim);
    if (!mech || !var) return sim->fail("add_gap_source: null variable name");
    if (sid < 0) {
        sid = sim->next_sid++;
        while (sim->gap_meta.count(sid)) sid = sim->next_sid++;
    } else {
        if (sim->gap_meta.count(sid)) return sim->fail("Gap junction with sid %d already exists", sid);
        if (sid >= sim->next_sid) sim->next_sid = sid + 1;
    }
    hx_sim::GapMeta g;
    g.mech = mech;
    g.var = var;
    g.idx = idx;
    sim->gap_meta[sid] = g;
    return sid;
}

int hx_add_gap_target(hx_sim* sim, int sid, const char* mech, const char* var, int idx) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    auto it = sim->gap_meta.find(sid);
    if (it == sim->gap_meta.end()) return sim->fail("Gap junction with sid %d does not exist", sid);
    if (!mech || !var) return sim->fail("add_gap_target: null variable name");
    API_BEGIN
    const Ref src = sim->resolve(it->second.mech, it->second.var, it->second.idx);
    const Ref dst = sim->resolve(mech, var, idx);
    if (!src.dev || !dst.dev) return sim->fail("Failed to resolve variable pointers");
    it->second.targets.emplace_back(mech, var, idx);
    sim->dg_src.push_back(src.dev);
    sim->dg_dst.push_back(dst.dev);
    sim->dg_dirty = true;
    return 0;
    API_END
}

int hx_clear_all_gap_junctions(hx_sim* sim) {
    HX_SETTLE(sim);
    sim->gap_meta.clear();
    sim->next_sid = 0;
    sim->dg_src.clear();
    sim->dg_dst.clear();
    sim->dg_dirty = true;
    sim->static_gaps_on = false;     // the reference clears the model's transfers too
    return 0;
}

int hx_get_next_available_sid(hx_sim* sim) {
    HX_SETTLE(sim);
    int sid = sim->next_sid;
    while (sim->gap_meta.count(sid)) ++sid;
    return sid;
}

int hx_get_gap_junction_sids(hx_sim* sim, int* sids, int cap) {
    HX_SETTLE(sim);
    int n = 0;
    for (auto& kv : sim->gap_meta) {
        if (sids && n < cap) sids[n] = kv.first;
        ++n;
    }
    return n;
}

int hx_get_gap_junction(hx_sim* sim, int sid, char* mech, int mech_cap, char* var, int var_cap, int* idx,
                        int* num_targets) {
    HX_SETTLE(sim);
    auto it = sim->gap_meta.find(sid);
    if (it == sim->gap_meta.end()) return -1;
    auto put = [](char* dst, int cap, const std::string& src) {
        if (!dst || cap <= 0) return;
        std::snprintf(dst, static_cast<size_t>(cap), "%s", src.c_str());
    };
    put(mech, mech_cap, it->second.mech);
    put(var, var_cap, it->second.var);
    if (idx) *idx = it->second.idx;
    if (num_targets) *num_targets = static_cast<int>(it->second.targets.size());
    return 0;
}

// ---- monitor and VecPlay lookups (SimRuntimeCore get_monitor_handle, get_vecplay_keys) ----
int hx_get_monitor_handle(hx_sim* sim, const char* mech, const char* var, int idx) {
    HX_SETTLE(sim);
    if (!mech || !var) return -1;
    for (size_t i = 0; i < sim->mon_name.size(); ++i)
        if (sim->mon_name[i].first == mech && sim->mon_name[i].second == var && sim->mon_idx[i] == idx)
            return static_cast<int>(i);
    return -1;
}

int hx_get_vecplay_keys(hx_sim* sim, char* buf, int cap) {
    HX_SETTLE(sim);
    std::string all;
    for (auto& vp : sim->vecplay) all += vp.mech + "\t" + vp.var + "\t" + std::to_string(vp.idx) + "\n";
    if (buf && cap > 0) std::snprintf(buf, static_cast<size_t>(cap), "%s", all.c_str());
    return static_cast<int>(all.size()) + 1;
}

int hx_fadvance(hx_sim* sim) {
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    DeferScope ds(sim);
    sim->run_steps(1);
    return 0;
    API_END
}

double hx_get_t(hx_sim* sim) { return sim->t; }

int hx_add_monitor(hx_sim* sim, const char* mech, const char* var, int idx) {
    HX_SETTLE(sim);
    if (!mech || !var) return sim->fail("null monitor name");
    Ref r;
    if (sim->loaded) {
        API_BEGIN
        r = sim->resolve(mech, var, idx);
        if (!r.dev) return sim->fail("monitor %s.%s[%d] not found", mech, var, idx);
        sim->require_sample_point(r);
        API_END
    }
    sim->mon_name.push_back({mech, var});
    sim->mon_idx.push_back(idx);
    sim->mon_ref.push_back(r);
    sim->mon_data.emplace_back();
    sim->mon_dirty = true;
    sim->mon_buf_cap = 0;
    return static_cast<int>(sim->mon_name.size()) - 1;
}

int hx_get_monitor_len(hx_sim* sim, int h) {
    HX_SETTLE(sim);
    if (h < 0 || h >= static_cast<int>(sim->mon_data.size())) return sim->fail("bad monitor handle");
    return static_cast<int>(sim->mon_data[h].size());
}

int hx_get_monitor_data(hx_sim* sim, int h, double* out, int cap) {
    HX_SETTLE(sim);
    if (h < 0 || h >= static_cast<int>(sim->mon_data.size())) return sim->fail("bad monitor handle");
    auto& d = sim->mon_data[h];
    int n = std::min<int>(cap, static_cast<int>(d.size()));
    if (n > 0) std::memcpy(out, d.data(), sizeof(double) * n);
    return n;
}

int hx_flush_recorders(hx_sim* sim) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    sim->sync_outputs();
    if (sim->h5) sim->h5->flush();
    return 0;
    API_END
}

int hx_mechanism_names(char* buf, int cap) {
    std::string out;
    auto line = [&](const char* name, const char* kind, int ncol, int nparam, int nstate, const char* const* cols) {
        out += name;
        out += '\t';
        out += kind;
        out += '\t' + std::to_string(nparam) + '\t' + std::to_string(nstate) + '\t';
        for (int c = 0; c < ncol; ++c) {
            if (c) out += ',';
            out += cols[c];
        }
        out += '\n';
    };
    const auto& R = registry();
    for (int id = 0; id < M_COUNT; ++id)
        line(R[id].name, "builtin", R[id].ncol, R[id].nparam, R[id].nstate, R[id].cols.data());
    for (int k = 0; k < plugin_count(); ++k) {
        const PluginMeta& m = plugin_at(k);
        line(m.name, "plugin", m.ncol, m.nparam, m.nstate, m.cols);
    }
    if (buf && cap > 0) {
        const size_t n = std::min(out.size(), static_cast<size_t>(cap - 1));
        std::memcpy(buf, out.data(), n);
        buf[n] = '\0';
    }
    return static_cast<int>(out.size()) + 1;
}

int hx_set_hdf5_enabled(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    API_BEGIN
    if (!enable) {
        sim->h5_on = false;
        sim->h5.reset();          // closes the file
        return 0;
    }
    std::string why;
    if (!H5Recorder::available(why)) return sim->fail("set_hdf5_enabled: %s", why.c_str());
    sim->h5_on = true;
    return 0;
    API_END
}

int hx_is_hdf5_enabled(hx_sim* sim) { return sim->h5_on ? 1 : 0; }

int hx_get_variable_handle(hx_sim* sim, const char* mech, const char* var, int idx) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    Ref r = sim->resolve(mech ? mech : "", var ? var : "", idx);
    if (!r.dev) return sim->fail("variable %s.%s[%d] not found", mech, var, idx);
    if (r.klass == 1) sim->write_assigned = true;
    sim->handles.push_back(r);
    return static_cast<int>(sim->handles.size()) - 1;
    API_END
}

int hx_get_variable_by_handle(hx_sim* sim, int h, double* out) {
    HX_SETTLE(sim);
    if (h < 0 || h >= static_cast<int>(sim->handles.size()) || !out) return sim->fail("bad variable handle");
    API_BEGIN
    HXC(hipStreamSynchronize(sim->stream));
    HXC(hipMemcpy(out, sim->handles[h].dev, sizeof(double), hipMemcpyDeviceToHost));
    return 0;
    API_END
}

int hx_set_variable_by_handle(hx_sim* sim, int h, double value) {
    HX_SETTLE(sim);
    if (h < 0 || h >= static_cast<int>(sim->handles.size())) return sim->fail("bad variable handle");
    API_BEGIN
    HXC(hipStreamSynchronize(sim->stream));
    HXC(hipMemcpy(sim->handles[h].dev, &value, sizeof(double), hipMemcpyHostToDevice));
    sim->mirror_ab(sim->handles[h], value);
    return 0;
    API_END
}

int hx_get_variables_by_handles(hx_sim* sim, int n, const int* hs, double* out) {
    HX_SETTLE(sim);
    for (int i = 0; i < n; ++i)
        if (hx_get_variable_by_handle(sim, hs[i], out + i) != 0) return -1;
    return 0;
}

int hx_get_variables_by_handles_f32_into(hx_sim* sim, int n, const int* hs, float* out) {
    HX_SETTLE(sim);
    for (int i = 0; i < n; ++i) {
        double x;
        if (hx_get_variable_by_handle(sim, hs[i], &x) != 0) return -1;
        out[i] = static_cast<float>(x);
    }
    return 0;
}

int hx_set_variables_by_handles(hx_sim* sim, int n, const int* hs, const double* vals) {
    HX_SETTLE(sim);
    for (int i = 0; i < n; ++i)
        if (hx_set_variable_by_handle(sim, hs[i], vals[i]) != 0) return -1;
    return 0;
}

int hx_get_variable_value(hx_sim* sim, const char* mech, const char* var, int idx, double* out) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    Ref r = sim->resolve(mech ? mech : "", var ? var : "", idx);
    if (!r.dev) return sim->fail("variable %s.%s[%d] not found", mech, var, idx);
    HXC(hipStreamSynchronize(sim->stream));
    HXC(hipMemcpy(out, r.dev, sizeof(double), hipMemcpyDeviceToHost));
    return 0;
    API_END
}

int hx_set_variable_value(hx_sim* sim, double value, const char* mech, const char* var, int idx) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    Ref r = sim->resolve(mech ? mech : "", var ? var : "", idx);
    if (!r.dev) return sim->fail("variable %s.%s[%d] not found", mech, var, idx);
    HXC(hipStreamSynchronize(sim->stream));
    HXC(hipMemcpy(r.dev, &value, sizeof(double), hipMemcpyHostToDevice));
    sim->mirror_ab(r, value);
    return 0;
    API_END
}

int hx_get_array(hx_sim* sim, const char* mech, const char* var, double* out, int cap) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    std::string mn = mech ? mech : "", vn = var ? var : "";
    HXC(hipStreamSynchronize(sim->stream));
    if (mn == "global" || mn == "node" || mn == "capacitance") {
        double* src = nullptr;
        if (mn == "capacitance") src = vn == "cm" ? sim->d_cm : nullptr;
        else if (vn == "v") src = sim->d_v;
        else if (vn == "d") src = sim->d_d;
        else if (vn == "rhs") src = sim->d_rhs;
        else if (vn == "a") src = sim->d_a;
        else if (vn == "b") src = sim->d_b;
        else if (vn == "area") src = sim->d_area;
        if (!src) return sim->fail("node variable '%s' not found", vn.c_str());
        if (cap < sim->nnode) return sim->fail("output too small");
        std::vector<double> g(sim->nnode);
        HXC(hipMemcpy(g.data(), src, sizeof(double) * sim->nnode, hipMemcpyDeviceToHost));
        for (int i = 0; i < sim->nnode; ++i) out[i] = g[sim->node_perm[i]];
        return sim->nnode;
    }
    int id = mech_id(mn);
    if (id < 0) {
        hx_sim::PluginInst* p = sim->plugin_named(mn);
        if (!p) return sim->fail("mechanism '%s' not present", mn.c_str());
        int c = -1;
        for (int k = 0; k < p->meta->ncol; ++k)
            if (vn == p->meta->cols[k]) c = k;
        if (c < 0) return sim->fail("%s has no variable '%s'", mn.c_str(), vn.c_str());
        const HostMech& m = p->h;
        if (cap < m.n) return sim->fail("output too small");
        std::vector<double> g(m.n);
        if (m.n) HXC(hipMemcpy(g.data(), m.dev.col(c), sizeof(double) * m.n, hipMemcpyDeviceToHost));
        for (int j = 0; j < m.n; ++j) out[j] = g[m.perm[j]];
        return m.n;
    }
    if (!sim->mech[id].present) return sim->fail("mechanism '%s' not present", mn.c_str());
    if (id == M_CADYN && (vn == "cai" || vn == "ica")) {
        // CaDynamics_E2 keeps cai / ica in the ca_ion column of its node: one copy of
        // that column, then a gather through the node -> ion instance map
        HostMech& m = sim->mech[id];
        HostMech& ca = sim->mech[M_CA_ION];
        if (cap < m.n) return sim->fail("output too small");
        std::vector<double> col(ca.n);
        if (ca.n)
            HXC(hipMemcpy(col.data(), ca.dev.col(vn == "cai" ? ION_CONCI : ION_CUR), sizeof(double) * ca.n,
                          hipMemcpyDeviceToHost));
        for (int j = 0; j < m.n; ++j) {
            const int inst = sim->ion_at[2][sim->node_perm[m.node[j]]];
            if (inst < 0) return sim->fail("CaDynamics_E2 instance %d has no ca_ion on its node", j);
            out[j] = col[inst];
        }
        return m.n;
    }
    const int c = col_id(id, vn);
    if (c < 0) return sim->fail("%s has no variable '%s'", mn.c_str(), vn.c_str());
    HostMech& m = sim->mech[id];
    if (cap < m.n) return sim->fail("output too small");
    std::vector<double> g(m.n);
    if (m.n) HXC(hipMemcpy(g.data(), m.dev.col(c), sizeof(double) * m.n, hipMemcpyDeviceToHost));
    for (int j = 0; j < m.n; ++j) out[j] = g[m.perm[j]];
    return m.n;
    API_END
}

int hx_add_vecplay(hx_sim* sim, const char* mech, const char* var, int idx, int n, const double* tv, const double* yv) {
    HX_SETTLE(sim);
    if (n <= 0 || !tv || !yv) return sim->fail("vecplay needs at least one (t, y) point");
    if (hx_has_vecplay(sim, mech, var, idx) == 1) return hx_update_vecplay(sim, mech, var, idx, n, tv, yv);
    VecPlayHost vp;
    vp.mech = mech;
    vp.var = var;
    vp.idx = idx;
    vp.tvec.assign(tv, tv + n);
    vp.yvec.assign(yv, yv + n);
    if (sim->loaded) {
        API_BEGIN
        Ref r = sim->resolve(mech, var, idx);
        if (!r.dev) return sim->fail("vecplay target %s.%s[%d] not found", mech, var, idx);
        vp.target = r.dev;
        API_END
    }
    sim->vecplay.push_back(std::move(vp));
    if (sim->loaded) {
        API_BEGIN
        if (sim->state_pending) { sim->finish_pending(); sim->sync_outputs(); }
        sim->recompute_fused();
        API_END
    }
    sim->vecplay_dirty = true;
    return 0;
}

int hx_update_vecplay(hx_sim* sim, const char* mech, const char* var, int idx, int n, const double* tv, const double* yv) {
    HX_SETTLE(sim);
    for (auto& vp : sim->vecplay)
        if (vp.mech == mech && vp.var == var && vp.idx == idx) {
            vp.tvec.assign(tv, tv + n);
            vp.yvec.assign(yv, yv + n);
            vp.d_t = vp.d_y = nullptr;
            sim->vecplay_dirty = true;
            return 0;
        }
    return sim->fail("vecplay %s.%s[%d] not found", mech, var, idx);
}

int hx_remove_vecplay(hx_sim* sim, const char* mech, const char* var, int idx) {
    HX_SETTLE(sim);
    for (size_t i = 0; i < sim->vecplay.size(); ++i) {
        auto& vp = sim->vecplay[i];
        if (vp.mech == mech && vp.var == var && vp.idx == idx) {
            sim->vecplay.erase(sim->vecplay.begin() + i);
            sim->vecplay_dirty = true;
            return 0;
        }
    }
    return sim->fail("vecplay %s.%s[%d] not found", mech, var, idx);
}

int hx_has_vecplay(hx_sim* sim, const char* mech, const char* var, int idx) {
    HX_SETTLE(sim);
    for (auto& vp : sim->vecplay)
        if (vp.mech == mech && vp.var == var && vp.idx == idx) return 1;
    return 0;
}

int hx_get_spike_count(hx_sim* sim) { return static_cast<int>(sim->spikes.size()); }

int hx_get_spikes(hx_sim* sim, double* t, int* gid, int cap) {
    int n = std::min<int>(cap, static_cast<int>(sim->spikes.size()));
    for (int i = 0; i < n; ++i) {
        t[i] = sim->spikes[i].first;
        gid[i] = sim->spikes[i].second;
    }
    return n;
}

// Spikes of every NetStim since finitialize, ordered by time then instance: those of
// host-made trains (an element's spike is at the step time t_m of the first step whose
// window t_m + dt/2 reaches it, once that step's delivery loop has run) and those logged
// by the device for the NetStims that receive events.
int hx_get_netstim_spikes(hx_sim* sim, double* t, int* inst, int cap) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    std::vector<std::pair<double, int>> all;
    if (sim->initialized) {
        const int last = std::max(sim->k - 1, 0);
        sim->ensure_ttab(last + 1);
        const double half = sim->dt / 2;
        const auto& tt = sim->ttab;
        for (int j = 0; j < static_cast<int>(sim->netstim.size()); ++j) {
            double run = -INFINITY;
            for (double e : sim->netstim[j]) {
                run = std::max(run, e);
                const auto it = std::lower_bound(tt.begin(), tt.begin() + last + 1, run,
                                                 [&](double tm, double T) { return tm + half < T; });
                if (it == tt.begin() + last + 1) break;
                all.push_back({*it, j});
            }
        }
        if (sim->nsa.n > 0) {
            HXC(hipStreamSynchronize(sim->stream));
            int c = 0;
            HXC(hipMemcpy(&c, sim->nsa.log_count, sizeof(int), hipMemcpyDeviceToHost));
            if (c > sim->ns_log_cap) throw std::runtime_error("NetStim spike log overflow");
            std::vector<double> lt(c);
            std::vector<int> li(c);
            if (c > 0) {
                HXC(hipMemcpy(lt.data(), sim->nsa.log_t, sizeof(double) * c, hipMemcpyDeviceToHost));
                HXC(hipMemcpy(li.data(), sim->nsa.log_inst, sizeof(int) * c, hipMemcpyDeviceToHost));
            }
            for (int i = 0; i < c; ++i) all.push_back({lt[i], li[i]});
        }
    }
    std::sort(all.begin(), all.end());
    const int n = std::min<int>(std::max(cap, 0), static_cast<int>(all.size()));
    for (int i = 0; i < n; ++i) {
        t[i] = all[i].first;
        inst[i] = all[i].second;
    }
    return static_cast<int>(all.size());
    API_END
}

// Simulate::output_spikes (simulate.cpp:892-909): <folder>/spk.dat, one "%.8g\t%d" line per
// spike, ordered by time and then gid, spikes of negative gids left out.
int hx_output_spikes(hx_sim* sim, const char* folder) {
    if (!folder || !*folder) return sim->fail("output_spikes: no folder given");
    std::error_code ec;
    std::filesystem::create_directories(folder, ec);
    if (ec) return sim->fail("output_spikes: cannot create %s: %s", folder, ec.message().c_str());
    std::vector<std::pair<double, int>> s = sim->spikes;
    std::sort(s.begin(), s.end(), [](const auto& x, const auto& y) {
        return x.first == y.first ? x.second < y.second : x.first < y.first;
    });
    const std::string path = std::string(folder) + "/spk.dat";
    FILE* fp = std::fopen(path.c_str(), "w");
    if (!fp) return sim->fail("output_spikes: cannot open %s", path.c_str());
    for (auto& e : s)
        if (e.second > -1) std::fprintf(fp, "%.8g\t%d\n", e.first, e.second);
    if (std::fclose(fp) != 0) return sim->fail("output_spikes: write to %s failed", path.c_str());
    return 0;
}

int hx_get_spk_by_gid(hx_sim* sim, int gid, double* out, int cap) {
    auto it = sim->spk_by_gid.find(gid);
    if (it == sim->spk_by_gid.end()) return 0;
    int n = std::min<int>(cap, static_cast<int>(it->second.size()));
    for (int i = 0; i < n; ++i) out[i] = it->second[i];
    return n;
}

int hx_set_event_capacity(hx_sim* sim, int per_step) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("set the event capacity before hx_load_model");
    if (per_step <= 0) return sim->fail("capacity must be positive");
    sim->event_cap_request = per_step;
    return 0;
}

int hx_set_cell_groups(hx_sim* sim, int ngroup) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("set the cell groups before hx_load_model");
    if (ngroup < 0) return sim->fail("group count must be >= 0");
    sim->group_request = ngroup;
    return 0;
}

int hx_set_solver_root(hx_sim* sim, int centre) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("set the solver root before hx_load_model");
    sim->solve_root_centre = centre != 0;
    return 0;
}

int hx_set_solve_unit_cells(hx_sim* sim, int cells) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("set the solve unit size before hx_load_model");
    if (cells < 0) return sim->fail("solve unit size must be >= 0 (0: the library's choice)");
    sim->unit_request = cells;
    return 0;
}

int hx_set_solve_waves(hx_sim* sim, int waves) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("set the solve units per workgroup before hx_load_model");
    if (waves < 0 || waves > kSolveMaxWaves)
        return sim->fail("solve units per workgroup must be 0..%d (0: the library's choice)", kSolveMaxWaves);
    sim->solve_waves_request = waves;
    return 0;
}

int hx_set_solve_resident(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    if (sim->loaded) return sim->fail("choose the tree solve's kernel before hx_load_model");
    sim->solve_resident_allowed = enable != 0;
    return 0;
}

int hx_set_solve_voltage(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    sim->solve_voltage_allowed = enable != 0;
    if (sim->loaded) sim->recompute_fused();
    return 0;
}

int hx_set_group_streams(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    sim->group_streams_allowed = enable != 0;
    return 0;
}

int hx_set_uniform_columns(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    sim->uniform_on = enable != 0;
    return 0;
}

int hx_set_fusion(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    sim->fusion_allowed = enable ? 1 : 0;
    if (sim->loaded) {
        API_BEGIN
        if (sim->state_pending) { sim->finish_pending(); sim->sync_outputs(); }
        sim->recompute_fused();
        API_END
    }
    return 0;
}

int hx_set_group_turns(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    sim->group_turns = enable ? 1 : 0;
    return 0;
}

int hx_set_dense_steady(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    sim->dense_steady = enable ? 1 : 0;
    return 0;
}

int hx_set_close_deferral(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    sim->close_deferral = enable != 0;
    return 0;
}

// The kernel timers are host state: these three neither read nor change the model, so
// they leave a pending state update pending (a timed call then starts as every call does).
int hx_measure_stream(int nread, int nwrite, long long n, int reps, double* ms) {
    if (n <= 0 || reps <= 0 || !ms) return -1;
    double *in = nullptr, *out = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = -1;
    if (hipMalloc(&in, sizeof(double) * nread * n) == hipSuccess &&
        hipMalloc(&out, sizeof(double) * nwrite * n) == hipSuccess &&
        hipMemset(in, 0, sizeof(double) * nread * n) == hipSuccess && hipEventCreate(&e0) == hipSuccess &&
        hipEventCreate(&e1) == hipSuccess && launch_stream(nread, nwrite, in, out, n, nullptr)) {
        (void)hipEventRecord(e0, nullptr);
        for (int k = 0; k < reps; ++k) launch_stream(nread, nwrite, in, out, n, nullptr);
        (void)hipEventRecord(e1, nullptr);
        float t = 0.f;
        if (hipEventSynchronize(e1) == hipSuccess && hipEventElapsedTime(&t, e0, e1) == hipSuccess) {
            *ms = static_cast<double>(t) / reps;
            rc = 0;
        }
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (in) (void)hipFree(in);
    if (out) (void)hipFree(out);
    return rc;
}

int hx_set_profiling(hx_sim* sim, int enable) {
    sim->profiling = enable != 0;
    sim->prof_mask = ~0u;
    for (auto& tm : sim->timers) { tm.ms = 0; tm.launches = 0; }
    return 0;
}

int hx_set_profiling_classes(hx_sim* sim, const char* classes) {
    unsigned mask = 0;
    std::string all = classes ? classes : "";
    size_t pos = 0;
    while (pos <= all.size()) {
        size_t e = all.find(',', pos);
        if (e == std::string::npos) e = all.size();
        const std::string name = all.substr(pos, e - pos);
        if (!name.empty()) {
            int id = -1;
            for (int i = 0; i < T_COUNT; ++i)
                if (name == kTimerNames[i]) id = i;
            if (id < 0) return sim->fail("unknown kernel class '%s'", name.c_str());
            mask |= 1u << id;
        }
        pos = e + 1;
    }
    sim->profiling = mask != 0;
    sim->prof_mask = mask;
    for (auto& tm : sim->timers) { tm.ms = 0; tm.launches = 0; }
    return 0;
}

int hx_get_kernel_time(hx_sim* sim, const char* kernel, double* ms, long long* launches) {
    for (int i = 0; i < T_COUNT; ++i)
        if (kernel && std::string(kernel) == kTimerNames[i]) {
            if (ms) *ms = sim->timers[i].ms;
            if (launches) *launches = sim->timers[i].launches;
            return 0;
        }
    return sim->fail("unknown kernel class '%s'", kernel ? kernel : "");
}

// Host emulation of one device tree solve over the same chunk schedule: for
// every cell, rounds in the kernel's order, each lane's chunk in turn, with the
// kernel's per-chunk arithmetic (reciprocals here are plain divisions).  Lanes
// of a round touch disjoint nodes and slots, so running them one after the
// other is what the wavefront computes.
int hx_fastmath_log(const double* x, double* y, int n) {
    if (n < 0 || (n > 0 && (!x || !y))) return -1;
    for (int i = 0; i < n; ++i) {
        if (!(x[i] >= 2.2250738585072014e-308 && x[i] <= 1.7976931348623157e308)) return -1;
        y[i] = hx::log_pos(x[i]);
    }
    return 0;
}

int hx_random123_philox4x32(const uint32_t* ctr, const uint32_t* key, uint32_t* out) {
    if (!ctr || !key || !out) return -1;
    Philox4x32::block(ctr, key, out);
    return 0;
}

int hx_netstim_train(double dt, double t_end, double interval, double number, double start, double noise,
                     unsigned id1, unsigned id2, unsigned id3, double* out, int cap) {
    try {
        if (!(dt > 0) || !(t_end >= 0) || cap < 0 || (cap > 0 && !out)) return -1;
        std::vector<double> ttab;
        const int horizon = static_cast<int>(std::ceil(t_end / dt));
        extend_step_times(ttab, horizon + 1, dt);
        std::vector<double> train;
        netstim_train(ttab, horizon, dt, NetStimParams{interval, number, start, noise, id1, id2, id3}, train);
        const int n = static_cast<int>(train.size());
        for (int i = 0; i < std::min(n, cap); ++i) out[i] = train[i];
        return n;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "hx_netstim_train: %s\n", e.what());
        return -1;
    }
}

int hx_emulate_tree_solve(int ncell, int nnode, const int* parent, const double* a, const double* b,
                          const double* cm, double cfac, double* v, const double* d, const double* rhs,
                          int* nchunk_max, int* nround_max) {
    return hx_emulate_tree_solve_units(ncell, nnode, parent, a, b, cm, cfac, v, d, rhs, 0, nchunk_max, nround_max);
}

int hx_emulate_tree_solve_units(int ncell, int nnode, const int* parent, const double* a, const double* b,
                                const double* cm, double cfac, double* v, const double* d, const double* rhs,
                                int unit_cells, int* nchunk_max, int* nround_max) {
    try {
        hx_sim tmp;
        if (hx_model_set_nodes(&tmp, ncell, nnode, parent, a, b, a) != 0) return -1;
        tmp.unit_request = std::max(0, unit_cells);
        tmp.build_layout();
        const int N = nnode;
        // solver-order arrays: DB RM A B V (the kernel's stage arrays) and w
        std::vector<double> arr[kStageArrays], gw(N);
        for (auto& x : arr) x.assign(N, 0.0);
        for (int i = 0; i < N; ++i) {
            const int g = tmp.node_perm[i];
            arr[SA_DB][g] = d[i] + cfac * cm[i];
            arr[SA_RM][g] = rhs[i];
            arr[SA_A][g] = tmp.solve_a[i];   // the solver's tree and coefficients, as uploaded
            arr[SA_B][g] = tmp.solve_b[i];
            arr[SA_V][g] = v[i];
        }
        const double neutral[kStageArrays] = {1.0, 0.0, 0.0, 0.0, 0.0};
        std::vector<double> slots(2 * static_cast<size_t>(std::max(tmp.max_slots, 1)));
        bool bound_mismatch = false;
        auto rcp = [](double x) { return 1.0 / x; };
        for (int c = 0; c < tmp.nunit; ++c) {
            const int nb = tmp.unit_node_begin[c];
            const ChunkDesc* cd = tmp.descs.data() + tmp.unit_desc_begin[c];
            const RoundInfo* ri = tmp.rounds.data() + tmp.unit_round_begin[c];
            const int nround = tmp.unit_round_begin[c + 1] - tmp.unit_round_begin[c];
            int idx[kChunk];
            auto positions = [&](int r, int l, int len) {
                for (int k = 0; k < kChunk; ++k) idx[k] = k < len ? nb + ri[r].node_base + ri[r].off[k] + l : -1;
            };
            // kernel stage arrays: DB RM A B V; back substitution reads s from RM, w from w, v from V
            auto val = [&](int x, int k) { return idx[k] >= 0 ? arr[x][idx[k]] : neutral[x]; };
            struct In {
                std::function<double(int, int)> f;
                std::function<double(int)> w;
                FwdNode fwd(int k) const { return {f(SA_DB, k), f(SA_RM, k), f(SA_A, k), f(SA_B, k), f(SA_V, k)}; }
                BackNode back(int k) const { return {f(SA_RM, k), w(k), f(SA_V, k)}; }
            };
            const In in{val, [&](int k) { return idx[k] >= 0 ? gw[idx[k]] : 0.0; }};
            for (int r = nround - 1; r >= 0; --r)
                for (int l = 0; l < ri[r].desc_count; ++l) {
                    const ChunkDesc& q = cd[ri[r].desc_begin + l];
                    positions(r, l, q.len);
                    if (q.child_count > 0) {
                        double acd = 0.0, ace = 0.0;
                        for (int ch = 0; ch < q.child_count; ++ch) {
                            acd += slots[2 * (q.child_begin + ch)];
                            ace += slots[2 * (q.child_begin + ch) + 1];
                        }
                        const int t = idx[q.len - 1];
                        tail_inject(arr[SA_DB][t], arr[SA_RM][t], arr[SA_V][t], acd, ace);
                    }
                    // results are written after the chunk is done (the kernel writes
                    // in place; a node's inputs are read before its outputs exist)
                    double D[kChunk], U[kChunk], W[kChunk], cdd, cee;
                    dispatch_chunk_bound(ri[r].maxlen, [&](auto km) {
                        chunk_forward_math<decltype(km)::value>(
                            q.parent_slot != kNone, in,
                            [&](int k, double Dk, double sk, double wk) { D[k] = Dk; U[k] = sk; W[k] = wk; }, rcp,
                            cdd, cee);
                    });
                    {
                        // the round's length bound skips padding iterations only:
                        // the full-length recurrence gives the same bits
                        double D2[kChunk], U2[kChunk], W2[kChunk], cd2, ce2;
                        chunk_forward_math<kChunk>(
                            q.parent_slot != kNone, in,
                            [&](int k, double Dk, double sk, double wk) { D2[k] = Dk; U2[k] = sk; W2[k] = wk; }, rcp,
                            cd2, ce2);
                        bool same = std::memcmp(&cd2, &cdd, sizeof cdd) == 0 && std::memcmp(&ce2, &cee, sizeof cee) == 0;
                        for (int k = 0; k < q.len; ++k)
                            same = same && std::memcmp(&D2[k], &D[k], 8) == 0 && std::memcmp(&U2[k], &U[k], 8) == 0 &&
                                   std::memcmp(&W2[k], &W[k], 8) == 0;
                        if (!same || q.len > ri[r].maxlen) bound_mismatch = true;
                    }
                    for (int k = 0; k < q.len; ++k) {
                        arr[SA_DB][idx[k]] = D[k];
                        arr[SA_RM][idx[k]] = U[k];
                        gw[idx[k]] = W[k];
                    }
                    if (q.parent_slot != kNone) {
                        slots[2 * q.slot] = cdd;
                        slots[2 * q.slot + 1] = cee;
                    }
                }
            for (int r = 0; r < nround; ++r)
                for (int l = 0; l < ri[r].desc_count; ++l) {
                    const ChunkDesc& q = cd[ri[r].desc_begin + l];
                    positions(r, l, q.len);
                    const double vpar = q.parent_slot != kNone ? slots[2 * q.parent_slot] : 0.0;
                    double VN[kChunk], X[kChunk], VN2[kChunk], X2[kChunk];
                    dispatch_chunk_bound(ri[r].maxlen, [&](auto km) {
                        chunk_back_math<decltype(km)::value>(
                            in, [&](int k, double vn, double vo) { VN[k] = vn; X[k] = vn - vo; }, vpar);
                    });
                    chunk_back_math<kChunk>(in, [&](int k, double vn, double vo) { VN2[k] = vn; X2[k] = vn - vo; },
                                            vpar);
                    for (int k = 0; k < q.len; ++k)
                        if (std::memcmp(&VN[k], &VN2[k], 8) != 0 || std::memcmp(&X[k], &X2[k], 8) != 0)
                            bound_mismatch = true;
                    for (int k = 0; k < q.len; ++k) {
                        arr[SA_V][idx[k]] = VN[k];
                        arr[SA_RM][idx[k]] = X[k];
                    }
                    slots[2 * q.slot] = VN[q.len - 1];
                }
        }
        if (bound_mismatch) return -2;
        std::vector<double>& gv = arr[SA_V];
        for (int i = 0; i < N; ++i) v[i] = gv[tmp.node_perm[i]];
        if (nchunk_max) *nchunk_max = tmp.max_slots;
        if (nround_max) *nround_max = tmp.max_rounds;
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "hx_emulate_tree_solve: %s\n", e.what());
        return -1;
    } catch (...) {
        return -1;
    }
}

long long hx_get_info(hx_sim* sim, const char* key) {
    std::string k = key ? key : "";
    if (k == "nnode") return sim->nnode;
    if (k == "ncell") return sim->ncell;
    if (k == "nchunk_max") return sim->max_slots;
    if (k == "nround_max") return sim->max_rounds;
    if (k == "dense_mask") return sim->dense_mask;
    if (k == "steady_launches") return sim->steady_launches;
    if (k == "electrode_nodes") return sim->point_union.n;
    if (k == "fused") return sim->fused ? 1 : 0;
    if (k == "adjoint_fused") return sim->adj_fuse_bits;
    if (k == "nround_total") return static_cast<long long>(sim->rounds.size());
    if (k == "solve_units") return sim->nunit;
    if (k == "handles") return static_cast<long long>(sim->handles.size());
    if (k == "solve_unit_cells") return sim->unit_cells;
    if (k == "solve_waves") return sim->solve_waves;
    if (k == "solve_resident") return sim->res_nodes > 0 ? 1 : 0;
    if (k == "solve_voltage") return sim->solve_voltage ? 1 : 0;
    if (k == "nchunk_total") return static_cast<long long>(sim->descs.size());
    if (k == "event_slots") return sim->groups.empty() ? 0 : sim->groups[0].ring.nslot;
    if (k == "event_cap") return sim->groups.empty() ? 0 : sim->groups[0].ring.cap;
    if (k == "cell_groups") return static_cast<long long>(sim->groups.size());
    if (k == "multi_stream") return sim->last_multi_stream ? 1 : 0;
    if (k == "state_pending") return sim->state_pending ? 1 : 0;
    if (k == "outputs_pending") return sim->outputs_pending ? 1 : 0;
    if (k == "uniform_columns" || k == "uniform_bytes") {
        long long cols = 0, bytes = 0;
        for (int id = 0; id < M_COUNT; ++id) {
            if (!sim->mech[id].present || !sim->uniform_on) continue;
            const int nb = __builtin_popcount(sim->mech[id].dev.umask);
            cols += nb;
            bytes += 8LL * nb * sim->mech[id].n;
        }
        if (sim->cm_uniform && sim->uniform_on) {
            cols += 1;
            bytes += 8LL * sim->nnode;
        }
        return k == "uniform_columns" ? cols : bytes;
    }
    return -1;
}

// ---------------------------------------------------------------------------
// adjoint (no reference counterpart) and Adam
// ---------------------------------------------------------------------------
int hx_tape_begin(hx_sim* sim, int max_steps) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    sim->tape_on = false;
    sim->tape_n = 0;
    if (max_steps <= 0) {
        sim->tape_free();
        return 0;
    }
    const auto& R = registry();
    if (!sim->plugins.empty()) {
        return sim->fail("the adjoint does not support plugin mechanisms (the model has %s)",
                         sim->plugins[0].meta->name);
    }
    for (int x : {M_NA_ION, M_K_ION})
        if (sim->mech[x].present)
            for (int t : sim->mech[x].iontype)
                if (t & 0100) return sim->fail("the adjoint needs fixed reversal potentials (%s iontype 0100)",
                                               R[x].name);
    // VecPlay into IClamp variables changes currents that do not depend on v or on any
    // trained parameter; any other target would need its values on the tape
    if (!sim->vecplay.empty() && !sim->vecplay_iclamp_only)
        return sim->fail("the adjoint supports VecPlay into IClamp variables only");
    sim->tape_free();
    const size_t cap = static_cast<size_t>(max_steps);
    HXC(hipMalloc(&sim->d_tape_v, sizeof(double) * cap * sim->nnode));
    HXC(hipMalloc(&sim->d_tape_v0, sizeof(double) * sim->nnode));
    auto has = [&](int id) { return sim->mech[id].present && sim->mech[id].n > 0; };
    if (has(M_CAHVA)) HXC(hipMalloc(&sim->d_tape_c, sizeof(double) * cap * 2 * sim->mech[M_CAHVA].dev.stride));
    if (has(M_HDLA)) HXC(hipMalloc(&sim->d_tape_l, sizeof(double) * cap * sim->mech[M_HDLA].n));
    if (has(M_CA_ION)) HXC(hipMalloc(&sim->d_tape_cai, sizeof(double) * cap * sim->mech[M_CA_ION].n));
    if (has(M_EXP2SYN)) HXC(hipMalloc(&sim->d_tape_ab, sizeof(double) * cap * 2 * sim->mech[M_EXP2SYN].n));
    if (sim->mech[M_HH].present && sim->mech[M_HH].n > 0)
        HXC(hipMalloc(&sim->d_tape_x, sizeof(double) * cap * 3 * sim->mech[M_HH].dev.stride));
    if (sim->mech[M_EXPSYN].present && sim->mech[M_EXPSYN].n > 0)
        HXC(hipMalloc(&sim->d_tape_g, sizeof(double) * cap * sim->mech[M_EXPSYN].n));
    sim->tape_evcap = 0;
    for (auto& cg : sim->groups) sim->tape_evcap += cg.ring.cap;   // every group appends to one row per step
    sim->tape_evcap = std::max(sim->tape_evcap, 1);
    HXC(hipMalloc(&sim->d_tape_evn, sizeof(int) * cap));
    HXC(hipMalloc(&sim->d_tape_ev, sizeof(int) * cap * sim->tape_evcap));
    HXC(hipMemsetAsync(sim->d_tape_evn, 0, sizeof(int) * cap, sim->stream));
    sim->tape_cap = max_steps;
    sim->tape_on = true;
    return 0;
    API_END
}

int hx_tape_length(hx_sim* sim) { return sim->tape_on ? sim->tape_n : 0; }

int hx_adjoint(hx_sim* sim, int nloss, const int* loss_nodes, const double* target, int nsample, double* loss) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    if (!sim->tape_on || sim->tape_n == 0) return sim->fail("no taped steps (hx_tape_begin, finitialize, run)");
    if (!sim->dg_src.empty()) return sim->fail("the adjoint does not support gap transfers added at run time");
    if (nsample != sim->tape_n)
        return sim->fail("target has %d samples, the tape holds %d steps", nsample, sim->tape_n);
    if (nloss <= 0) return sim->fail("no loss nodes");
    const int N = sim->nnode;
    std::vector<int> ln(nloss);
    for (int j = 0; j < nloss; ++j) {
        if (loss_nodes[j] < 0 || loss_nodes[j] >= N) return sim->fail("loss node %d out of range", loss_nodes[j]);
        ln[j] = sim->node_perm[loss_nodes[j]];
    }
    hipStream_t st = sim->stream;
    auto& owned = sim->owned;
    int* d_ln = sim->slot_upload(sim->adj_ln_slot, ln);
    std::vector<double> tgt(target, target + static_cast<size_t>(nsample) * nloss);
    double* d_tgt = sim->slot_upload(sim->adj_tgt_slot, tgt);
    // a node listed more than once gets each of its loss terms, in list order, from
    // one thread: the distinct nodes, and for each the positions it has in the list
    std::vector<int> un, ubeg, uidx;
    {
        std::vector<int> order(nloss);
        std::iota(order.begin(), order.end(), 0);
        std::stable_sort(order.begin(), order.end(), [&](int x, int y) { return ln[x] < ln[y]; });
        for (int q = 0; q < nloss; ++q) {
            if (q == 0 || ln[order[q]] != ln[order[q - 1]]) {
                un.push_back(ln[order[q]]);
                ubeg.push_back(q);
            }
            uidx.push_back(order[q]);
        }
        ubeg.push_back(nloss);
    }
    const int nun = static_cast<int>(un.size());
    int* d_un = sim->slot_upload(sim->adj_un_slot, un);
    int* d_ubeg = sim->slot_upload(sim->adj_ubeg_slot, ubeg);
    int* d_uidx = sim->slot_upload(sim->adj_uidx_slot, uidx);
    // loss: mean over samples 1..nsample and loss nodes of (v - target)^2
    double* d_samp = static_cast<double*>(
        sim->slot_reserve(sim->adj_samp_slot, sizeof(double) * static_cast<size_t>(nsample) * nloss));
    launch_adj_gather(sim->d_tape_v, N, d_ln, nloss, nsample, d_samp, st);
    std::vector<double> samp(static_cast<size_t>(nsample) * nloss);
    HXC(hipMemcpyAsync(samp.data(), d_samp, sizeof(double) * samp.size(), hipMemcpyDeviceToHost, st));
    HXC(hipStreamSynchronize(st));
    const double scale = 1.0 / (static_cast<double>(nsample) * nloss);
    double L = 0.0;
    for (size_t k = 0; k < samp.size(); ++k) L += (samp[k] - tgt[k]) * (samp[k] - tgt[k]);
    if (loss) *loss = L * scale;
    // diagonal correction of the transposed solve: the tree kernel assembles
    // d - b_i - sum_c a_c from the (swapped) coefficients, M^T needs the original
    if (!sim->d_adj_delta) {
        sim->d_adj_delta = dalloc<double>(owned, N);
        sim->adj_delta_dirty = true;
        for (double** p : {&sim->d_lv, &sim->d_lv2, &sim->d_dT, &sim->d_rhsT, &sim->d_vT, &sim->d_wT})
            *p = dalloc<double>(owned, N);
        const HostMech& hh = sim->mech[M_HH];
        const HostMech& es = sim->mech[M_EXPSYN];
        const HostMech& pas = sim->mech[M_PAS];
        sim->d_lx = dalloc<double>(owned, std::max<long long>(1, 3 * (hh.present ? hh.dev.stride : 0)));
        sim->d_lg = dalloc<double>(owned, std::max(1, es.present ? es.n : 0));
        auto cnt = [&](int id, long long per) {
            const HostMech& m = sim->mech[id];
            return std::max<long long>(1, m.present ? per : 0);
        };
        sim->d_lc = dalloc<double>(owned, cnt(M_CAHVA, 2 * sim->mech[M_CAHVA].dev.stride));
        sim->d_ll = dalloc<double>(owned, cnt(M_HDLA, sim->mech[M_HDLA].n));
        sim->d_lcai = dalloc<double>(owned, cnt(M_CA_ION, sim->mech[M_CA_ION].n));
        sim->d_lica = dalloc<double>(owned, cnt(M_CA_ION, sim->mech[M_CA_ION].n));
        sim->d_lab = dalloc<double>(owned, cnt(M_EXP2SYN, 2 * static_cast<long long>(sim->mech[M_EXP2SYN].n)));
        sim->ensure_grad_arrays();
    }
    if (!sim->d_adj_delta || sim->adj_delta_dirty) {
        // diagonal correction on the solver's tree, with the solver's coefficients
        std::vector<double> delta(N, 0.0);
        for (int i = 0; i < N; ++i) {
            const int q = sim->solve_parent[i];
            if (q < 0) continue;
            delta[i] += sim->solve_a[i] - sim->solve_b[i];
            delta[q] += sim->solve_b[i] - sim->solve_a[i];
        }
        std::vector<double> g(N);
        for (int i = 0; i < N; ++i) g[sim->node_perm[i]] = delta[i];
        HXC(hipMemcpy(sim->d_adj_delta, g.data(), sizeof(double) * N, hipMemcpyHostToDevice));
        sim->adj_delta_dirty = false;
    }
    const HostMech& hh = sim->mech[M_HH];
    const HostMech& es = sim->mech[M_EXPSYN];
    const HostMech& pas = sim->mech[M_PAS];
    const long long xs = hh.present ? hh.dev.stride : 0;
    HXC(hipMemsetAsync(sim->d_lv, 0, sizeof(double) * N, st));
    HXC(hipMemsetAsync(sim->d_lx, 0, sizeof(double) * std::max<long long>(1, 3 * xs), st));
    HXC(hipMemsetAsync(sim->d_lg, 0, sizeof(double) * std::max(1, es.present ? es.n : 0), st));
    (void)pas;
    for (int k = 0; k < kNumTrainable; ++k) {
        const HostMech& m = sim->mech[kTrainable[k].mech];
        HXC(hipMemsetAsync(sim->d_grad[k], 0, sizeof(double) * std::max(1, m.present ? m.n : 0), st));
    }
    const HostMech& cah = sim->mech[M_CAHVA];
    const HostMech& hdl = sim->mech[M_HDLA];
    const HostMech& cai = sim->mech[M_CA_ION];
    const HostMech& e2 = sim->mech[M_EXP2SYN];
    const bool with_c = cah.present && cah.n > 0, with_l = hdl.present && hdl.n > 0;
    const bool with_ca = cai.present && cai.n > 0, with_e2 = e2.present && e2.n > 0;
    const long long cs = with_c ? cah.dev.stride : 0;
    HXC(hipMemsetAsync(sim->d_lc, 0, sizeof(double) * std::max<long long>(1, 2 * cs), st));
    HXC(hipMemsetAsync(sim->d_ll, 0, sizeof(double) * std::max(1, with_l ? hdl.n : 0), st));
    HXC(hipMemsetAsync(sim->d_lcai, 0, sizeof(double) * std::max(1, with_ca ? cai.n : 0), st));
    HXC(hipMemsetAsync(sim->d_lica, 0, sizeof(double) * std::max(1, with_ca ? cai.n : 0), st));
    HXC(hipMemsetAsync(sim->d_lab, 0, sizeof(double) * std::max(1, with_e2 ? 2 * e2.n : 0), st));
    const StepArgs SA = sim->step_args(sim->t, 0, 0);
    AdjStep A{};
    A.N = N;
    A.dt = sim->dt;
    A.cfac = SA.cfac;
    A.hh_q10 = SA.c.hh_q10;
    A.cm = sim->d_cm;
    A.area = sim->d_area;
    A.delta = sim->d_adj_delta;
    for (int id = 0; id < M_COUNT; ++id) A.m[id] = SA.m[id];
    A.xstride = xs;
    A.lam_x = sim->d_lx;
    A.lam_g = sim->d_lg;
    A.dT = sim->d_dT;
    A.rhsT = sim->d_rhsT;
    A.mu = sim->d_vT;     // the solve's new voltage (solved for directly) is x = M^-T lambda
    A.grad_gnabar = sim->d_grad[T_GNABAR];
    A.grad_gkbar = sim->d_grad[T_GKBAR];
    A.grad_gpas = sim->d_grad[T_GPAS];
    A.grad_w = sim->d_grad[T_WES];
    A.c = SA.c;
    A.cstride = cs;
    A.lam_c = sim->d_lc;
    A.lam_l = sim->d_ll;
    A.lam_cai = with_ca ? sim->d_lcai : nullptr;
    A.lam_ica = (with_ca && sim->mech[M_CADYN].present && sim->mech[M_CADYN].n > 0) ? sim->d_lica : nullptr;
    A.lam_ab = sim->d_lab;
    A.grad_cgbar = sim->d_grad[T_CGBAR];
    A.grad_ghdbar = sim->d_grad[T_GHDBAR];
    A.grad_w2 = sim->d_grad[T_WE2];
    A.grad_ggap = sim->d_grad[T_GGAP];
    // gap junctions: each HalfGap instance's source node (solver order; -1: none) and the
    // distinct sources with the instances they feed, in instance order
    if (sim->mech[M_HALFGAP].present && sim->mech[M_HALFGAP].n > 0) {
        const HostMech& hg = sim->mech[M_HALFGAP];
        std::vector<int> partner(hg.n, -1);
        std::vector<std::pair<int, int>> by_src;        // (source node, device instance)
        for (const auto& gp : sim->gaps_eff) {
            const int j = hg.perm[gp.second], src = sim->node_perm[gp.first];
            partner[j] = src;
            by_src.push_back({src, j});
        }
        std::sort(by_src.begin(), by_src.end());
        std::vector<int> srcs, beg, inst;
        for (size_t e = 0; e < by_src.size(); ++e) {
            if (e == 0 || by_src[e].first != by_src[e - 1].first) {
                srcs.push_back(by_src[e].first);
                beg.push_back(static_cast<int>(e));
            }
            inst.push_back(by_src[e].second);
        }
        beg.push_back(static_cast<int>(by_src.size()));
        A.gap_partner = sim->slot_upload(sim->adj_gp_slot, partner);
        A.ngap_src = static_cast<int>(srcs.size());
        if (!srcs.empty()) {
            A.gap_src = sim->slot_upload(sim->adj_gs_slot, srcs);
            A.gap_begin = sim->slot_upload(sim->adj_gb_slot, beg);
            A.gap_inst = sim->slot_upload(sim->adj_gi_slot, inst);
        }
    }
    // The node-parallel kernels take the mechanisms with one instance on every node (the
    // node kernel's layout): gate adjoints only as the tail of hh, Ca_HVA, hd_la and
    // conductances only as the head of pas, hh, Ca_HVA, hd_la, so that every node's sums
    // keep the per-mechanism kernels' order.  hx_set_fusion(0) leaves every mechanism to
    // its own kernels.
    if (sim->fusion_allowed) {
        auto has = [&](int id) { return sim->mech[id].present && sim->mech[id].n > 0; };
        auto dense = [&](int id) { return has(id) && (sim->dense_mask & (1u << id)) != 0; };
        const int st_id[3] = {M_HH, M_CAHVA, M_HDLA};
        const unsigned st_bit[3] = {kAdjHH, kAdjCaHVA, kAdjHdla};
        for (int k = 2; k >= 0; --k) {
            if (!has(st_id[k])) continue;
            if (!dense(st_id[k])) break;
            A.fuse_state |= st_bit[k];
        }
        if (dense(M_CADYN)) A.fuse_state |= kAdjCaDyn;
        const int cd_id[4] = {M_PAS, M_HH, M_CAHVA, M_HDLA};
        const unsigned cd_bit[4] = {kAdjPas, kAdjHH, kAdjCaHVA, kAdjHdla};
        for (int k = 0; k < 4; ++k) {
            if (!has(cd_id[k])) continue;
            if (!dense(cd_id[k])) break;
            A.fuse_cond |= cd_bit[k];
        }
        for (int k = 0; k < 4; ++k)
            if (dense(cd_id[k])) A.fuse_param |= cd_bit[k];
        // the synapses join when every density conductance is in the node kernel, so that
        // their grouped conductances still come after the density ones on each node
        bool all_cond = true;
        for (int k = 0; k < 4; ++k) all_cond = all_cond && (!has(cd_id[k]) || (A.fuse_cond & cd_bit[k]));
        if (all_cond && (has(M_EXPSYN) || has(M_EXP2SYN))) {
            A.fold_syn = 1;
            // node -> its group (instances sorted by node, one group per node)
            int* maps[2] = {nullptr, nullptr};
            for (int k = 0; k < 2; ++k) {
                const int id = k == 0 ? M_EXPSYN : M_EXP2SYN;
                if (!has(id)) continue;
                if (!sim->d_syn_grp[k]) sim->d_syn_grp[k] = dalloc<int>(owned, N);
                std::vector<int> g(N, -1);
                const std::vector<int>& nodes = sim->syn_node[k];
                int q = -1;
                for (size_t j = 0; j < nodes.size(); ++j) {
                    if (j == 0 || nodes[j] != nodes[j - 1]) ++q;
                    g[nodes[j]] = q;
                }
                HXC(hipMemcpyAsync(sim->d_syn_grp[k], g.data(), sizeof(int) * N, hipMemcpyHostToDevice, st));
                HXC(hipStreamSynchronize(st));
                maps[k] = sim->d_syn_grp[k];
            }
            A.es_grp = maps[0];
            A.e2_grp = maps[1];
        }
    }
    // the loss term joins k_adj_after_nodes when no later kernel adds to lambda_v^n (Ca_HVA's
    // own parameter kernel would) and the loss nodes are distinct (one thread per node)
    int* d_lmap = nullptr;
    if (sim->fusion_allowed) {
        const HostMech& ch = sim->mech[M_CAHVA];
        if (!(ch.present && ch.n > 0) || (A.fuse_param & kAdjCaHVA)) {
            if (nun == nloss) {           // distinct nodes
                if (sim->adj_lmap_nodes != ln || !sim->adj_lmap_slot.p) {
                    std::vector<int> lmap(N, -1);
                    for (int j = 0; j < nloss; ++j) lmap[ln[j]] = j;
                    sim->slot_upload(sim->adj_lmap_slot, lmap);
                    sim->adj_lmap_nodes = ln;
                }
                d_lmap = static_cast<int*>(sim->adj_lmap_slot.p);
            }
        }
    }
    A.loss_of_node = d_lmap;
    A.loss_scale = scale;
    sim->adj_fuse_bits = A.fuse_state | (A.fuse_cond << 8) | (A.fuse_param << 16) |
                         (static_cast<unsigned>(A.fold_syn) << 24) | ((d_lmap ? 1u : 0u) << 25);
    SolveArgs S{};
    S.waves = sim->solve_waves;
    S.nunit = sim->nunit;
    S.unit_node_begin = sim->d_unit_node_begin;
    S.unit_desc_begin = sim->d_unit_desc_begin;
    S.unit_round_begin = sim->d_unit_round_begin;
    S.rounds = sim->d_rounds;
    S.desc = sim->d_desc;
    S.v = sim->d_vT;
    S.d = sim->d_dT;
    S.rhs = sim->d_rhsT;
    S.w = sim->d_wT;
    S.a = sim->d_sb;      // M^T: the coefficients trade places
    S.b = sim->d_sa;
    S.store_dx = 0;       // D and x are not needed
    S.yform = 1;          // the transposed system's unknown starts at 0: the solve reads no v,
                          // and the new v it writes is the solution itself
    S.res_nodes = sim->res_nodes;
    S.res_rounds = sim->max_rounds;
    double* lv = sim->d_lv;
    double* lv2 = sim->d_lv2;
    const size_t row = static_cast<size_t>(N);
    launch_adj_loss(sim->d_tape_v + (nsample - 1) * row, d_un, d_ubeg, d_uidx, nun,
                    d_tgt + static_cast<size_t>(nsample - 1) * nloss, scale, lv, st);
    for (int n = nsample - 1; n >= 0; --n) {
        A.v1 = sim->d_tape_v + n * row;
        A.x0 = sim->d_tape_x ? sim->d_tape_x + static_cast<size_t>(n) * 3 * xs : nullptr;
        A.geff = sim->d_tape_g ? sim->d_tape_g + static_cast<size_t>(n) * es.n : nullptr;
        A.ev_count = sim->d_tape_evn + n;
        A.ev = sim->d_tape_ev + static_cast<size_t>(n) * sim->tape_evcap;
        A.v0 = n >= 1 ? sim->d_tape_v + (n - 1) * row : sim->d_tape_v0;
        A.c0 = with_c ? sim->d_tape_c + static_cast<size_t>(n) * 2 * cs : nullptr;
        A.l0 = with_l ? sim->d_tape_l + static_cast<size_t>(n) * hdl.n : nullptr;
        A.cai0 = with_ca ? sim->d_tape_cai + static_cast<size_t>(n) * cai.n : nullptr;
        A.ab0 = with_e2 ? sim->d_tape_ab + static_cast<size_t>(n) * 2 * e2.n : nullptr;
        A.lam_v = lv;
        A.lam_v_new = lv2;
        A.loss_v = (d_lmap && n >= 1) ? sim->d_tape_v + (n - 1) * row : nullptr;
        A.loss_tgt = n >= 1 ? d_tgt + static_cast<size_t>(n - 1) * nloss : nullptr;
        launch_adj_before_solve(A, st);
        launch_solve(S, sim->max_slots, st);
        launch_adj_after_solve(A, st);
        if (n >= 1 && !d_lmap)
            launch_adj_loss(sim->d_tape_v + (n - 1) * row, d_un, d_ubeg, d_uidx, nun,
                            d_tgt + static_cast<size_t>(n - 1) * nloss, scale, lv2, st);
        std::swap(lv, lv2);
    }
    HXC(hipStreamSynchronize(st));
    sim->have_grad = true;
    return 0;
    API_END
}

int hx_get_gradient(hx_sim* sim, const char* mech, const char* var, double* out, int cap) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    if (!sim->have_grad) return sim->fail("no gradients (call hx_adjoint)");
    const std::string mn = mech ? mech : "", vn = var ? var : "";
    const int id = mech_id(mn);
    const int tk = id < 0 ? -1 : trainable_id(id, vn);
    if (tk < 0 || !sim->mech[id].present) return sim->fail("no gradient for %s.%s", mn.c_str(), vn.c_str());
    double* src = sim->d_grad[tk];
    const HostMech& m = sim->mech[id];
    if (cap < m.n) return sim->fail("output too small");
    std::vector<double> g(m.n);
    HXC(hipMemcpy(g.data(), src, sizeof(double) * m.n, hipMemcpyDeviceToHost));
    for (int j = 0; j < m.n; ++j) out[m.iperm[j]] = g[j];
    return m.n;
    API_END
}

int hx_adam_create(hx_sim* sim, double beta1, double beta2, double eps) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    hx_sim::AdamHost o;
    o.beta1 = beta1;
    o.beta2 = beta2;
    o.eps = eps;
    sim->adams.push_back(o);
    return static_cast<int>(sim->adams.size()) - 1;
}

int hx_adam_add_group(hx_sim* sim, int opt, const char* mech, const char* var, int n, const int* inst,
                      double impedance) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("bad optimizer id");
    if (n <= 0) return sim->fail("empty parameter group");
    const std::string mn = mech ? mech : "", vn = var ? var : "";
    sim->ensure_grad_arrays();
    const int id = mech_id(mn);
    const int tk = id < 0 ? -1 : trainable_id(id, vn);
    if (tk < 0 || !sim->mech[id].present) return sim->fail("no trainable parameter %s.%s", mn.c_str(), vn.c_str());
    double* grad = sim->d_grad[tk];
    const HostMech& m = sim->mech[id];
    std::vector<double*> w, g;
    for (int k = 0; k < n; ++k) {
        if (inst[k] < 0 || inst[k] >= m.n) return sim->fail("instance %d out of range", inst[k]);
        const int dj = m.perm[inst[k]];
        w.push_back(id == M_EXPSYN ? sim->d_es_weight + dj
                    : id == M_EXP2SYN ? sim->d_e2_weight + dj
                                      : sim->resolve(mn, vn, inst[k]).dev);
        g.push_back(grad + dj);
    }
    return sim->opt_add_group(opt, w, g, impedance);
    API_END
}

int hx_adam_step(hx_sim* sim, int opt, double lr, double inv_record_steps) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("bad optimizer id");
    auto& o = sim->adams[opt];
    auto& owned = sim->owned;
    const int ng = static_cast<int>(o.imp.size());
    if (o.dirty) {   // (re)upload the groups; the host copies of m and v are current
        o.d_begin = sim->slot_upload(o.s_begin, o.begin);
        o.d_w = sim->slot_upload(o.s_w, o.w);
        o.d_g = sim->slot_upload(o.s_g, o.g);
        o.d_imp = sim->slot_upload(o.s_imp, o.imp);
        o.d_m = sim->slot_upload(o.s_m, o.m);
        o.d_v = sim->slot_upload(o.s_v, o.v);
        o.dirty = false;
    }
    ++o.step;
    AdamArgs A{};
    A.type = o.type;
    A.momentum = o.momentum;
    A.ngroup = ng;
    A.begin = o.d_begin;
    A.w = o.d_w;
    A.grad = o.d_g;
    A.impedance = o.d_imp;
    A.m = o.d_m;
    A.v = o.d_v;
    A.lr = lr;
    A.inv_record_steps = inv_record_steps;
    A.beta1 = o.beta1;
    A.beta2 = o.beta2;
    A.eps = o.eps;
    A.step = o.step;
    launch_adam(A, sim->stream);
    HXC(hipMemcpyAsync(o.m.data(), o.d_m, sizeof(double) * ng, hipMemcpyDeviceToHost, sim->stream));
    HXC(hipMemcpyAsync(o.v.data(), o.d_v, sizeof(double) * ng, hipMemcpyDeviceToHost, sim->stream));
    HXC(hipStreamSynchronize(sim->stream));
    return 0;
    API_END
}

int hx_adam_get_state(hx_sim* sim, int opt, long long* step, double* m, double* v, int cap) {
    HX_SETTLE(sim);
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("bad optimizer id");
    const auto& o = sim->adams[opt];
    const int ng = static_cast<int>(o.imp.size());
    if (step) *step = o.step;
    if ((m || v) && cap < ng) return sim->fail("output too small");
    for (int g = 0; g < ng; ++g) {
        if (m) m[g] = o.m[g];
        if (v) v[g] = o.v[g];
    }
    return ng;
}


void hx_sim::ensure_grad_arrays() {
    if (d_grad[0]) return;
    for (int k = 0; k < kNumTrainable; ++k) {
        const HostMech& m = mech[kTrainable[k].mech];
        const int n = std::max(1, m.present ? m.n : 0);
        d_grad[k] = dalloc<double>(owned, n);
        HXC(hipMemset(d_grad[k], 0, sizeof(double) * n));
    }
}

int hx_sim::opt_add_group(int opt, const std::vector<double*>& w, const std::vector<double*>& g, double impedance) {
    auto& o = adams[opt];
    for (size_t k = 0; k < w.size(); ++k) {
        o.w.push_back(w[k]);
        o.g.push_back(g[k]);
    }
    o.begin.push_back(static_cast<int>(o.w.size()));
    o.imp.push_back(impedance);
    o.m.push_back(0.0);
    o.v.push_back(0.0);
    o.dirty = true;
    return static_cast<int>(o.imp.size()) - 1;
}

// ---------------------------------------------------------------------------
// optimizers with the reference's interface (SimWrapper.cpp:159-460,
// simulate.cpp:1150-1260): parameters are (weight, gradient) variable handles,
// a batch is one tied group (mean gradient, one update broadcast to every
// weight), gradients are zeroed after each step
// ---------------------------------------------------------------------------
int hx_create_optimizer(hx_sim* sim, const char* type) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    std::string t = type ? type : "";
    std::transform(t.begin(), t.end(), t.begin(), [](unsigned char c) { return std::tolower(c); });
    hx_sim::AdamHost o;
    if (t == "sgd") o.type = 0;
    else if (t == "momentum" || t == "sgdmomentum" || t == "sgd_momentum") o.type = 1;
    else if (t == "adam") o.type = 2;
    else return sim->fail("Unsupported optimizer type: %s", type ? type : "");
    sim->adams.push_back(o);
    return static_cast<int>(sim->adams.size()) - 1;
}

int hx_configure_optimizer(hx_sim* sim, int opt, double momentum, double beta1, double beta2, double eps) {
    HX_SETTLE(sim);
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer %d not found", opt);
    auto& o = sim->adams[opt];
    o.momentum = momentum;
    o.beta1 = beta1;
    o.beta2 = beta2;
    o.eps = eps;
    return 0;
}

int hx_optimizer_add_param_batch(hx_sim* sim, int opt, int n, const int* weight_handles, const int* grad_handles,
                                 double impedance) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer %d not found", opt);
    if (n <= 0 || !weight_handles || !grad_handles)
        return sim->fail("optimizer_add_param_batch: handle lists must be non-empty and have equal length");
    std::vector<double*> w(n), g(n);
    const int nh = static_cast<int>(sim->handles.size());
    for (int i = 0; i < n; ++i) {
        if (weight_handles[i] < 0 || weight_handles[i] >= nh)
            return sim->fail("optimizer_add_param_batch: invalid weight handle %d", weight_handles[i]);
        if (grad_handles[i] < 0 || grad_handles[i] >= nh)
            return sim->fail("optimizer_add_param_batch: invalid grad handle %d", grad_handles[i]);
        w[i] = sim->handles[weight_handles[i]].dev;
        g[i] = sim->handles[grad_handles[i]].dev;
    }
    return sim->opt_add_group(opt, w, g, impedance);
}

int hx_optimizer_add_param(hx_sim* sim, int opt, int weight_handle, int grad_handle, double impedance) {
    HX_SETTLE(sim);
    return hx_optimizer_add_param_batch(sim, opt, 1, &weight_handle, &grad_handle, impedance);
}

int hx_optimizer_step_with_inv_record_steps(hx_sim* sim, int opt, double lr, double inv_record_steps) {
    HX_SETTLE(sim);
    return hx_adam_step(sim, opt, lr, inv_record_steps);
}

int hx_optimizer_step(hx_sim* sim, int opt, double lr, double record_time, double dt) {
    HX_SETTLE(sim);
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer_step: optimizer %d not found", opt);
    if (record_time <= 0.0 || dt <= 0.0)
        return sim->fail("optimizer_step: invalid record_time (%f) or dt (%f)", record_time, dt);
    return hx_adam_step(sim, opt, lr, dt / record_time);   // simulate.cpp:1198-1211
}

int hx_optimizer_add_external_grads(hx_sim* sim, int opt, int n, const int* weight_handles, double impedance) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer %d not found", opt);
    if (n <= 0 || !weight_handles) return sim->fail("optimizer_add_external_grads: empty weight_handles");
    if (!(impedance > 0.0)) return sim->fail("optimizer_add_external_grads: invalid impedance (%f)", impedance);
    auto& o = sim->adams[opt];
    const int nh = static_cast<int>(sim->handles.size());
    for (int i = 0; i < n; ++i)
        if (weight_handles[i] < 0 || weight_handles[i] >= nh)
            return sim->fail("optimizer_add_external_grads: invalid weight handle %d", weight_handles[i]);
    o.d_ext = dalloc<double>(sim->owned, n);
    o.n_ext = n;
    HXC(hipMemset(o.d_ext, 0, sizeof(double) * n));
    for (int i = 0; i < n; ++i)      // one group per weight (SimWrapper.cpp:284-353)
        sim->opt_add_group(opt, {sim->handles[weight_handles[i]].dev}, {o.d_ext + i}, impedance);
    return 0;
    API_END
}

int hx_optimizer_set_external_grads_f32(hx_sim* sim, int opt, int n, const float* grads) {
    HX_SETTLE(sim);
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer %d not found", opt);
    auto& o = sim->adams[opt];
    if (!o.d_ext) return sim->fail("optimizer_set_external_grads_f32: optimizer %d has no external grads binding", opt);
    if (n != o.n_ext || !grads)
        return sim->fail("optimizer_set_external_grads_f32: grads shape mismatch (got %d expected %d)", n, o.n_ext);
    API_BEGIN
    std::vector<double> g(grads, grads + n);
    HXC(hipStreamSynchronize(sim->stream));
    HXC(hipMemcpy(o.d_ext, g.data(), sizeof(double) * n, hipMemcpyHostToDevice));
    return 0;
    API_END
}

int hx_optimizer_clear_external_grads(hx_sim* sim, int opt) {
    HX_SETTLE(sim);
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer %d not found", opt);
    auto& o = sim->adams[opt];
    if (!o.d_ext) return 0;
    API_BEGIN
    HXC(hipStreamSynchronize(sim->stream));
    HXC(hipMemset(o.d_ext, 0, sizeof(double) * o.n_ext));
    return 0;
    API_END
}

int hx_optimizer_reset_state(hx_sim* sim, int opt) {
    HX_SETTLE(sim);
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer %d not found", opt);
    auto& o = sim->adams[opt];
    if (o.type == 2) o.step = 0;
    std::fill(o.m.begin(), o.m.end(), 0.0);
    std::fill(o.v.begin(), o.v.end(), 0.0);
    o.dirty = true;
    return 0;
}

int hx_optimizer_get_adam_state(hx_sim* sim, int opt, long long* step, double* m, double* v, int cap, double* beta1,
                                double* beta2, double* eps) {
    HX_SETTLE(sim);
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer %d not found", opt);
    const auto& o = sim->adams[opt];
    if (o.type != 2) return sim->fail("optimizer %d is not Adam", opt);
    if (beta1) *beta1 = o.beta1;
    if (beta2) *beta2 = o.beta2;
    if (eps) *eps = o.eps;
    return hx_adam_get_state(sim, opt, step, m, v, cap);
}

int hx_optimizer_set_adam_state(hx_sim* sim, int opt, long long step, int n, const double* m, const double* v,
                                double beta1, double beta2, double eps) {
    HX_SETTLE(sim);
    if (opt < 0 || opt >= static_cast<int>(sim->adams.size())) return sim->fail("optimizer %d not found", opt);
    auto& o = sim->adams[opt];
    if (o.type != 2) return sim->fail("optimizer %d is not Adam", opt);
    if (n != static_cast<int>(o.imp.size()) || (n > 0 && (!m || !v)))
        return sim->fail("optimizer_set_adam_state: state size %d does not match %zu parameters", n, o.imp.size());
    if (step < 0) return sim->fail("optimizer_set_adam_state: negative step count");
    o.step = step;
    o.m.assign(m, m + n);
    o.v.assign(v, v + n);
    o.beta1 = beta1;
    o.beta2 = beta2;
    o.eps = eps;
    o.dirty = true;
    return 0;
}

// ---------------------------------------------------------------------------
// learn gradient surface (LearnRuntime.cpp:197-2457)
// ---------------------------------------------------------------------------
int hx_set_dense_blocks_f32(hx_sim* sim, int nblk, const float* const* blocks, const int* bn, const int* k_len) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    if (nblk < 0 || (nblk > 0 && (!blocks || !bn || !k_len))) return sim->fail("set_dense_blocks_f32: bad arguments");
    LearnRuntime& L = sim->learn_rt();
    const int r = L.set_dense_blocks(nblk, blocks, bn, k_len);
    if (r < 0) return sim->fail("%s", L.err.c_str());
    return r;
    API_END
}

int hx_clear_dense_blocks(hx_sim* sim) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    sim->learn_rt().clear_dense_blocks();
    return 0;
    API_END
}

namespace {

bool resolve_handles(hx_sim* sim, const char* fn, const char* what, int n, const int* hs, std::vector<double*>& out) {
    out.resize(n);
    for (int i = 0; i < n; ++i) {
        if (hs[i] < 0 || hs[i] >= static_cast<int>(sim->handles.size())) {
            sim->fail("%s: invalid %s handle", fn, what);
            return false;
        }
        const Ref& r = sim->handles[hs[i]];
        sim->require_sample_point(r);
        out[i] = r.dev;
    }
    return true;
}

// Steps from a run length, with the reference's tstop check
// (LearnRuntime.cpp:1719-1725, 286-292).
bool check_tstop(hx_sim* sim, const char* fn, int total_steps, double tstop_ms) {
    const double from_steps = static_cast<double>(total_steps) * sim->dt;
    if (tstop_ms > 0.0 && std::abs(tstop_ms - from_steps) > sim->dt * 0.5) {
        sim->fail("%s: tstop mismatch (tstop_ms=%f, steps*dt=%f)", fn, tstop_ms, from_steps);
        return false;
    }
    return true;
}

}  // namespace

int hx_simulate_output_vs_into(hx_sim* sim, float* output_vs_tn, int t_steps_plus1, int n_output,
                               const int* output_v_handles, double tstop_ms, double v_init) {
    HX_SETTLE(sim);
    static const char* fn = "simulate_output_vs_into";
    if (!check_loaded(sim)) return -1;
    if (!output_vs_tn) return sim->fail("%s: output buffer is null", fn);
    if (!(sim->dt > 0.0)) return sim->fail("%s: invalid dt", fn);
    if (n_output <= 0 || !output_v_handles) return sim->fail("%s: output handles mismatch", fn);
    if (t_steps_plus1 < 2) return sim->fail("%s: invalid steps", fn);
    API_BEGIN
    const int total_steps = t_steps_plus1 - 1;
    if (!check_tstop(sim, fn, total_steps, tstop_ms)) return -1;
    std::vector<double*> outp;
    if (!resolve_handles(sim, fn, "output", n_output, output_v_handles, outp)) return -1;
    LearnRuntime& L = sim->learn_rt();
    L.begin_capture(t_steps_plus1, outp, 0, 0, 1, false, nullptr, 0, LearnRuntime::SINK_CACHE);
    try {
        sim->finitialize(v_init);
        sim->run_steps(total_steps);
    } catch (...) {
        L.end_capture(nullptr);
        throw;
    }
    L.end_capture(output_vs_tn);
    return 0;
    API_END
}

namespace {

// simulate_and_capture_mapped_signals_{cached,into}: N_into > 0 gives N and T
// and copies the signals to to_host[3] instead of caching them.
int capture_common(hx_sim* sim, const char* fn, float* output_vs_tn, int total_steps_plus1, int n_output,
                   const int* output_v_handles, int n_pure_i, const int* pure_i_handles, const int* pure_i_dest,
                   const float* pure_i_scale, int n_didv, const int* didv_handles, const int* didv_dest,
                   const float* didv_scale, int n_didvpre, const int* didvpre_handles, const int* didvpre_dest,
                   const float* didvpre_scale, double tstop_ms, int k_mul, int percise, double v_init, int N_into,
                   int T_into, float* const* to_host) {
    if (k_mul <= 0) return sim->fail("%s: k_mul must be positive", fn);
    if (!(sim->dt > 0.0)) return sim->fail("%s: invalid dt", fn);
    if (!output_vs_tn) return sim->fail("%s: output_vs_tn is null", fn);
    if (n_output <= 0 || !output_v_handles) return sim->fail("%s: output_v_handles size mismatch", fn);
    if (total_steps_plus1 < 2) return sim->fail("%s: total_steps_plus1 must be >= 2", fn);
    const int total_steps = total_steps_plus1 - 1;
    const int ksteps = total_steps / k_mul;
    if (ksteps <= 0) return sim->fail("%s: ksteps_total must be positive", fn);
    if (n_pure_i < 0 || n_didv < 0 || n_didvpre < 0) return sim->fail("%s: negative channel size", fn);
    // cached: N is the largest pure_i destination + 1 (LearnRuntime.cpp:1671-1682)
    int N = N_into;
    if (!to_host) {
        N = 0;
        for (int i = 0; i < n_pure_i; ++i) N = std::max(N, pure_i_dest[i] + 1);
        if (N <= 0) return sim->fail("%s: inferred N is non-positive", fn);
    } else if (N <= 0) {
        return sim->fail("%s: N must be positive", fn);
    } else if (T_into < 2) {
        return sim->fail("%s: ksteps_total_plus1 must be >= 2", fn);
    }
    const int* hs[3] = {pure_i_handles, didv_handles, didvpre_handles};
    const int* ds[3] = {pure_i_dest, didv_dest, didvpre_dest};
    const float* sc[3] = {pure_i_scale, didv_scale, didvpre_scale};
    const int cnt[3] = {n_pure_i, n_didv, n_didvpre};
    const char* names[3] = {"pure_i", "didv", "didvpre"};
    const int nch = percise ? 3 : 1;
    for (int c = 0; c < nch; ++c) {
        if (cnt[c] > 0 && (!hs[c] || !ds[c] || !sc[c])) return sim->fail("%s: %s handles/dest/scale missing", fn, names[c]);
        for (int i = 0; i < cnt[c]; ++i)
            if (ds[c][i] < 0 || ds[c][i] >= N)
                return sim->fail("%s: %s_dest out of range at %d (%d)", fn, names[c], i, ds[c][i]);
    }
    API_BEGIN
    if (!check_tstop(sim, fn, total_steps, tstop_ms)) return -1;
    std::vector<double*> outp;
    if (!resolve_handles(sim, fn, "output", n_output, output_v_handles, outp)) return -1;
    LearnRuntime::Channel ch[3];
    for (int c = 0; c < nch; ++c) {
        if (!resolve_handles(sim, fn, names[c], cnt[c], hs[c], ch[c].ptr)) return -1;
        ch[c].dest.assign(ds[c], ds[c] + cnt[c]);
        ch[c].scale.assign(sc[c], sc[c] + cnt[c]);
    }
    LearnRuntime& L = sim->learn_rt();
    L.begin_capture(total_steps_plus1, outp, N, T_into, k_mul, percise != 0, ch, nch,
                    to_host ? LearnRuntime::SINK_HOST : LearnRuntime::SINK_CACHE);
    try {
        sim->finitialize(v_init);
        sim->run_steps(total_steps);
    } catch (...) {
        L.end_capture(nullptr);
        throw;
    }
    L.end_capture(output_vs_tn, to_host);
    return 0;
    API_END
}

}  // namespace

int hx_simulate_and_capture_mapped_signals_cached(
    hx_sim* sim, float* output_vs_tn, int total_steps_plus1, int n_output, const int* output_v_handles, int n_pure_i,
    const int* pure_i_handles, const int* pure_i_dest, const float* pure_i_scale, int n_didv, const int* didv_handles,
    const int* didv_dest, const float* didv_scale, int n_didvpre, const int* didvpre_handles, const int* didvpre_dest,
    const float* didvpre_scale, double tstop_ms, int k_mul, int percise, double v_init) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    return capture_common(sim, "simulate_and_capture_mapped_signals_cached", output_vs_tn, total_steps_plus1,
                          n_output, output_v_handles, n_pure_i, pure_i_handles, pure_i_dest, pure_i_scale, n_didv,
                          didv_handles, didv_dest, didv_scale, n_didvpre, didvpre_handles, didvpre_dest,
                          didvpre_scale, tstop_ms, k_mul, percise, v_init, 0, 0, nullptr);
}

int hx_simulate_and_capture_mapped_signals_into(
    hx_sim* sim, float* output_vs_tn, int total_steps_plus1, int n_output, float* it_lr_tn, float* ditdv_lr_tn,
    float* ditdvpre_lr_tn, int ksteps_total_plus1, int N, const int* output_v_handles, int n_pure_i,
    const int* pure_i_handles, const int* pure_i_dest, const float* pure_i_scale, int n_didv, const int* didv_handles,
    const int* didv_dest, const float* didv_scale, int n_didvpre, const int* didvpre_handles, const int* didvpre_dest,
    const float* didvpre_scale, double tstop_ms, int k_mul, int percise, double v_init) {
    HX_SETTLE(sim);
    static const char* fn = "simulate_and_capture_mapped_signals_into";
    if (!check_loaded(sim)) return -1;
    if (!output_vs_tn || !it_lr_tn || !ditdv_lr_tn || !ditdvpre_lr_tn)
        return sim->fail("%s: output buffers must be non-null", fn);
    float* host[3] = {it_lr_tn, ditdv_lr_tn, ditdvpre_lr_tn};
    return capture_common(sim, fn, output_vs_tn, total_steps_plus1, n_output, output_v_handles, n_pure_i,
                          pure_i_handles, pure_i_dest, pure_i_scale, n_didv, didv_handles, didv_dest, didv_scale,
                          n_didvpre, didvpre_handles, didvpre_dest, didvpre_scale, tstop_ms, k_mul, percise, v_init,
                          N, ksteps_total_plus1, host);
}

namespace {

int replay_common(hx_sim* sim, const char* fn, LearnRuntime::Source src, const float* dL, int ksteps, int n_output,
                  const int* poutput, const int* pinput, int n_input, const int* pre_of_col, int n_pre,
                  float* dw_out_n, float* dx_lr_it, double dt_ms, int percise, double grad_scale, double eps,
                  double thr, int clip_strategy, int clip_every, const float* const* noalloc_sig = nullptr,
                  int noalloc_T = 0) {
    LearnRuntime& L = sim->learn_rt();
    if (L.k_len() <= 0) return sim->fail("%s: dense blocks not set (call set_dense_blocks_f32)", fn);
    const bool cached = src == LearnRuntime::SRC_CACHE;
    const int N = cached ? L.capture_N() : n_pre;
    if (cached) {
        if (L.capture_N() <= 0 || L.capture_T() < 2) return sim->fail("%s: cached capture buffers not initialized", fn);
        if (percise && !L.capture_percise())
            return sim->fail("%s: percise requested but cached didv buffers missing", fn);
        if (ksteps != L.capture_T() - 1)
            return sim->fail("%s: ksteps_total mismatch (%d vs %d)", fn, ksteps, L.capture_T() - 1);
    }
    if (!dL || !poutput || !pre_of_col || !dw_out_n || (n_input > 0 && (!pinput || !dx_lr_it)))
        return sim->fail("%s: null input/output pointer", fn);
    if (n_output <= 0) return sim->fail("%s: empty poutput/pinput", fn);
    if (n_pre != N) return sim->fail("%s: pre_of_col has %d entries, N is %d", fn, n_pre, N);
    // indices are checked here: the kernels gather with them
    for (int o = 0; o < n_output; ++o)
        if (poutput[o] < 0 || poutput[o] >= N) return sim->fail("%s: poutput[%d]=%d out of range", fn, o, poutput[o]);
    for (int j = 0; j < n_input; ++j)
        if (pinput[j] < 0 || pinput[j] >= N) return sim->fail("%s: pinput[%d]=%d out of range", fn, j, pinput[j]);
    for (int i = 0; i < N; ++i)
        if (pre_of_col[i] < -1 || pre_of_col[i] >= N)
            return sim->fail("%s: pre_of_col[%d]=%d out of range", fn, i, pre_of_col[i]);
    int sum_bn = 0;
    for (int b = 0; b < static_cast<int>(L.block_sizes().size()); ++b) sum_bn += L.block_sizes()[b];
    if (sum_bn != N) return sim->fail("%s: dense blocks total N mismatch (sum=%d vs N=%d)", fn, sum_bn, N);
    LearnRuntime::ReplayIn in;
    in.dl = dL;
    in.ksteps = ksteps;
    in.n_out = n_output;
    in.n_in = n_input;
    in.po = poutput;
    in.pin = pinput;
    in.pre = pre_of_col;
    in.dw_out = dw_out_n;
    in.dx_out = dx_lr_it;
    in.dt = dt_ms;
    in.grad_scale = grad_scale;
    in.eps = eps;
    in.thr = thr;
    in.percise = percise != 0;
    in.clip_strategy = clip_strategy;
    in.clip_every = std::max(1, clip_every);
    in.source = src;
    in.cached_clip_rule = src != LearnRuntime::SRC_HOST;
    // host signals given here: the allocation-free replay over the library's scratch array
    const int rc = noalloc_sig
                       ? L.replay_from_host_noalloc(in, noalloc_sig[0], noalloc_sig[1], noalloc_sig[2], N, noalloc_T)
                       : L.replay(in);
    if (rc != 0) return sim->fail("%s: %s", fn, L.err.c_str());
    return 0;
}

}  // namespace

int hx_replay_compute_dw_from_cached_signals_into(hx_sim* sim, const float* dLtdv_lr_to, int ksteps_total,
                                                  int n_output, const int* poutput, const int* pre_of_col, int n_pre,
                                                  float* dw_out_n, double dt_ms, int percise, double grad_scale,
                                                  double eps, double grad_l2norm_threshold, int clip_strategy,
                                                  int clip_check_every) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    return replay_common(sim, "replay_compute_dw_from_cached_signals_into", LearnRuntime::SRC_CACHE, dLtdv_lr_to,
                         ksteps_total,
                         n_output, poutput, nullptr, 0, pre_of_col, n_pre, dw_out_n, nullptr, dt_ms, percise,
                         grad_scale, eps, grad_l2norm_threshold, clip_strategy, clip_check_every);
    API_END
}

int hx_replay_compute_dw_dx_from_cached_signals_into(hx_sim* sim, const float* dLtdv_lr_to, int ksteps_total,
                                                     int n_output, const int* poutput, const int* pinput, int n_input,
                                                     const int* pre_of_col, int n_pre, float* dw_out_n,
                                                     float* dx_lr_it, double dt_ms, int percise, double grad_scale,
                                                     double eps, double grad_l2norm_threshold, int clip_strategy,
                                                     int clip_check_every) {
    HX_SETTLE(sim);
    static const char* fn = "replay_compute_dw_dx_from_cached_signals_into";
    if (!check_loaded(sim)) return -1;
    if (n_input <= 0) return sim->fail("%s: empty poutput/pinput", fn);
    API_BEGIN
    return replay_common(sim, fn, LearnRuntime::SRC_CACHE, dLtdv_lr_to, ksteps_total, n_output, poutput, pinput,
                         n_input, pre_of_col,
                         n_pre, dw_out_n, dx_lr_it, dt_ms, percise, grad_scale, eps, grad_l2norm_threshold,
                         clip_strategy, clip_check_every);
    API_END
}

int hx_replay_compute_dw_dx_from_signals_into(hx_sim* sim, const float* it_lr_nt, const float* ditdv_lr_nt,
                                              const float* ditdvpre_lr_nt, int N, int T, const float* dLtdv_lr_to,
                                              int ksteps_total, int n_output, const int* poutput, const int* pinput,
                                              int n_input, const int* pre_of_col, float* dw_out_n, float* dx_lr_it,
                                              double dt_ms, int percise, double grad_scale, double eps,
                                              double grad_l2norm_threshold, int clip_strategy, int clip_check_every) {
    HX_SETTLE(sim);
    static const char* fn = "replay_compute_dw_dx_from_signals_into";
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    LearnRuntime& L = sim->learn_rt();
    // LearnRuntime.cpp:402-450
    if (L.k_len() <= 0) return sim->fail("%s: dense blocks not set (call set_dense_blocks_f32)", fn);
    if (!it_lr_nt || !dLtdv_lr_to || !poutput || !pinput || !pre_of_col || !dw_out_n || !dx_lr_it)
        return sim->fail("%s: null pointer input/output", fn);
    if (N <= 0 || T < 2) return sim->fail("%s: invalid it_lr_nt shape (%d, %d)", fn, N, T);
    if (ksteps_total != T - 1) return sim->fail("%s: ksteps_total mismatch (%d vs T-1=%d)", fn, ksteps_total, T - 1);
    if (n_output <= 0 || n_input <= 0) return sim->fail("%s: empty poutput/pinput", fn);
    if (!(dt_ms > 0.0) || !(eps > 0.0)) return sim->fail("%s: invalid dt_ms/eps", fn);
    if (!(grad_l2norm_threshold > 0.0)) return sim->fail("%s: invalid grad_l2norm_threshold", fn);
    clip_strategy = std::max(0, clip_strategy);
    clip_check_every = std::max(1, clip_check_every);
    if (percise && (!ditdv_lr_nt || !ditdvpre_lr_nt))
        return sim->fail("%s: percise requested but ditdv buffers are null", fn);
    int sum_bn = 0;
    for (int bn : L.block_sizes()) sum_bn += bn;
    if (sum_bn != N) return sim->fail("%s: dense blocks total N mismatch (sum=%d vs N=%d)", fn, sum_bn, N);
    if (L.load_signals(it_lr_nt, ditdv_lr_nt, ditdvpre_lr_nt, N, T, percise != 0) != 0)
        return sim->fail("%s", L.err.c_str());
    return replay_common(sim, fn, LearnRuntime::SRC_HOST, dLtdv_lr_to, ksteps_total, n_output, poutput, pinput,
                         n_input, pre_of_col,
                         N, dw_out_n, dx_lr_it, dt_ms, percise, grad_scale, eps, grad_l2norm_threshold,
                         clip_strategy, clip_check_every);
    API_END
}

int hx_replay_compute_dw_dx_from_signals_into_noalloc(
    hx_sim* sim, const float* it_lr_nt, const float* ditdv_lr_nt, const float* ditdvpre_lr_nt, int N, int T,
    const float* dLtdv_lr_to, int ksteps_total, int n_output, const int* poutput, const int* pinput, int n_input,
    const int* pre_of_col, float* dw_out_n, float* dx_lr_it, double dt_ms, int percise, double grad_scale, double eps,
    double grad_l2norm_threshold, int clip_strategy, int clip_check_every) {
    HX_SETTLE(sim);
    static const char* fn = "replay_compute_dw_dx_from_signals_into_noalloc";
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    LearnRuntime& L = sim->learn_rt();
    // the same checks as the allocating entry point
    if (L.k_len() <= 0) return sim->fail("%s: dense blocks not set (call set_dense_blocks_f32)", fn);
    if (!it_lr_nt || !dLtdv_lr_to || !poutput || !pinput || !pre_of_col || !dw_out_n || !dx_lr_it)
        return sim->fail("%s: null pointer input/output", fn);
    if (N <= 0 || T < 2) return sim->fail("%s: invalid it_lr_nt shape (%d, %d)", fn, N, T);
    if (ksteps_total != T - 1) return sim->fail("%s: ksteps_total mismatch (%d vs T-1=%d)", fn, ksteps_total, T - 1);
    if (n_output <= 0 || n_input <= 0) return sim->fail("%s: empty poutput/pinput", fn);
    if (!(dt_ms > 0.0) || !(eps > 0.0)) return sim->fail("%s: invalid dt_ms/eps", fn);
    if (!(grad_l2norm_threshold > 0.0)) return sim->fail("%s: invalid grad_l2norm_threshold", fn);
    clip_strategy = std::max(0, clip_strategy);
    clip_check_every = std::max(1, clip_check_every);
    if (percise && (!ditdv_lr_nt || !ditdvpre_lr_nt))
        return sim->fail("%s: percise requested but ditdv buffers are null", fn);
    const float* sig[3] = {it_lr_nt, ditdv_lr_nt, ditdvpre_lr_nt};
    return replay_common(sim, fn, LearnRuntime::SRC_HOST, dLtdv_lr_to, ksteps_total, n_output, poutput, pinput,
                         n_input, pre_of_col, N, dw_out_n, dx_lr_it, dt_ms, percise, grad_scale, eps,
                         grad_l2norm_threshold, clip_strategy, clip_check_every, sig, T);
    API_END
}

// LearnRuntime::simulate_and_replay_dw_dx_streaming_into (LearnRuntime.cpp:729-1288): the
// reference keeps only a K_len ring of signals and replays while it steps; with
// 288 GB of HBM the whole run's signals are captured first and replayed after,
// with the same windows, taps and clip schedule as a cached replay.
int hx_simulate_and_replay_dw_dx_streaming_into(
    hx_sim* sim, const float* dLtdv_lr_to, int ksteps_total, int n_output, const int* poutput, const int* pinput,
    int n_input, int N, const int* pre_of_col, float* dw_out_n, float* dx_lr_it, int n_pure_i,
    const int* pure_i_handles, const int* pure_i_dest, const float* pure_i_scale, int n_didv, const int* didv_handles,
    const int* didv_dest, const float* didv_scale, int n_didvpre, const int* didvpre_handles, const int* didvpre_dest,
    const float* didvpre_scale, double tstop_ms, int k_mul, int percise, double v_init, double dt_ms,
    double grad_scale, double eps, double grad_l2norm_threshold, int clip_strategy, int clip_check_every) {
    HX_SETTLE(sim);
    static const char* fn = "simulate_and_replay_dw_dx_streaming_into";
    if (!check_loaded(sim)) return -1;
    API_BEGIN
    LearnRuntime& L = sim->learn_rt();
    // LearnRuntime.cpp:767-866
    if (L.k_len() <= 0) return sim->fail("%s: dense blocks not set (call set_dense_blocks_f32)", fn);
    if (k_mul <= 0) return sim->fail("%s: k_mul must be positive", fn);
    if (!(sim->dt > 0.0)) return sim->fail("%s: invalid dt", fn);
    if (dt_ms > 0.0 && std::abs(dt_ms - sim->dt) > sim->dt * 0.5)
        return sim->fail("%s: dt_ms mismatch (dt_ms=%f, sim->dt=%f)", fn, dt_ms, sim->dt);
    if (clip_check_every <= 0) clip_check_every = 1;
    if (N <= 0) return sim->fail("%s: pre_of_col must be non-empty", fn);
    if (n_output <= 0 || n_input <= 0) return sim->fail("%s: empty poutput/pinput", fn);
    if (ksteps_total <= 0) return sim->fail("%s: dLtdv_lr_to must have at least 1 tick", fn);
    if (!dLtdv_lr_to || !poutput || !pinput || !pre_of_col || !dw_out_n || !dx_lr_it)
        return sim->fail("%s: null pointer input/output", fn);
    int sum_bn = 0;
    for (int bn : L.block_sizes()) sum_bn += bn;
    if (sum_bn != N) return sim->fail("%s: dense block sum mismatch (sum=%d N=%d)", fn, sum_bn, N);
    const int* hs[3] = {pure_i_handles, didv_handles, didvpre_handles};
    const int* ds[3] = {pure_i_dest, didv_dest, didvpre_dest};
    const float* sc[3] = {pure_i_scale, didv_scale, didvpre_scale};
    const int cnt[3] = {n_pure_i, n_didv, n_didvpre};
    const char* names[3] = {"pure_i", "didv", "didvpre"};
    const int nch = percise ? 3 : 1;
    for (int c = 0; c < nch; ++c) {
        if (cnt[c] < 0 || (cnt[c] > 0 && (!hs[c] || !ds[c] || !sc[c])))
            return sim->fail("%s: %s handles/dest/scale size mismatch", fn, names[c]);
        for (int i = 0; i < cnt[c]; ++i)
            if (ds[c][i] < 0 || ds[c][i] >= N)
                return sim->fail("%s: %s_dest out of range at %d (%d)", fn, names[c], i, ds[c][i]);
    }
    const int total_steps = ksteps_total * k_mul;
    if (!check_tstop(sim, fn, total_steps, tstop_ms)) return -1;
    LearnRuntime::Channel ch[3];
    for (int c = 0; c < nch; ++c) {
        if (!resolve_handles(sim, fn, names[c], cnt[c], hs[c], ch[c].ptr)) return -1;
        ch[c].dest.assign(ds[c], ds[c] + cnt[c]);
        ch[c].scale.assign(sc[c], sc[c] + cnt[c]);
    }
    L.begin_capture(total_steps + 1, {}, N, ksteps_total + 1, k_mul, percise != 0, ch, nch,
                    LearnRuntime::SINK_STREAM);
    try {
        sim->finitialize(v_init);
        sim->run_steps(total_steps);
    } catch (...) {
        L.end_capture(nullptr);
        throw;
    }
    L.end_capture(nullptr);
    return replay_common(sim, fn, LearnRuntime::SRC_STREAM, dLtdv_lr_to, ksteps_total, n_output, poutput, pinput,
                         n_input, pre_of_col, N, dw_out_n, dx_lr_it, dt_ms, percise, grad_scale, eps,
                         grad_l2norm_threshold, clip_strategy, clip_check_every);
    API_END
}

int hx_set_replay_timing(hx_sim* sim, int enable) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    sim->learn_rt().timing = enable != 0;
    return 0;
}

int hx_get_replay_kernel_time(hx_sim* sim, double* ms, long long* launches) {
    HX_SETTLE(sim);
    if (!check_loaded(sim)) return -1;
    LearnRuntime& L = sim->learn_rt();
    if (ms) *ms = L.corr_ms;
    if (launches) *launches = L.corr_launches;
    return 0;
}

}  // extern "C"
