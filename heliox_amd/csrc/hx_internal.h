// Internal types shared by the host runtime and the HIP kernels.
//
// HBM layout (one model per handle):
//   * node arrays (v, d, rhs, a, b, cm, area) are stored in solver order:
//     cells are gathered into solve units of a few consecutive cells, units
//     are contiguous, and inside a unit its cells' nodes are grouped in chunks
//     (unbranched runs of at most kChunk nodes) ordered root-round first;
//   * every mechanism is a structure of arrays: column c of mechanism m lives
//     at base + c * stride (stride = instance count rounded up to 64), and
//     instances are sorted by solver-order node index;
//   * a mechanism that has one instance on every node is "dense": instance i
//     sits on node i and is processed by the fused node-parallel kernel;
//     the others are "sparse" and run instance-parallel.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace hx {

// Mechanism ids in CoreNEURON type order: currents are accumulated in this
// order (coredat_to_innerdat.cpp:176-181 keeps CoreNEURON's order).
enum MechId : int {
    M_PAS = 0, M_NA_ION, M_K_ION, M_HH, M_ICLAMP, M_EXPSYN, M_EXP2SYN, M_VECSTIM,
    M_CA_ION, M_CADYN, M_CAHVA, M_HALFGAP, M_HDLA, M_NETSTIM, M_COUNT
};

// Column layouts: parameters, then states, then assigned variables.
enum PasCol { PAS_G = 0, PAS_E, PAS_I, PAS_NCOL };
enum IonCol { ION_EREV = 0, ION_CONCI, ION_CONCO, ION_CUR, ION_DCURDV, ION_NCOL };
enum HHCol {
    HH_GNABAR = 0, HH_GKBAR, HH_GL, HH_EL, HH_M, HH_H, HH_N, HH_ENA, HH_EK, HH_INA, HH_IK, HH_IL,
    HH_GNA, HH_GK, HH_MINF, HH_HINF, HH_NINF, HH_MTAU, HH_HTAU, HH_NTAU, HH_NCOL
};
enum IClampCol { IC_DELAY = 0, IC_DUR, IC_AMP, IC_I, IC_NCOL };
enum ExpSynCol { ES_TAU = 0, ES_E, ES_G, ES_I, ES_NCOL };
enum Exp2SynCol { E2_TAU1 = 0, E2_TAU2, E2_E, E2_A, E2_B, E2_FACTOR, E2_G, E2_I, E2_NCOL };
enum CaDynCol { CD_GAMMA = 0, CD_DECAY, CD_DEPTH, CD_MINCAI, CD_NCOL };
enum CaHVACol {
    CH_GBAR = 0, CH_M, CH_H, CH_ECA, CH_ICA, CH_G, CH_IMECH, CH_MINF, CH_MTAU, CH_MALPHA, CH_MBETA,
    CH_HINF, CH_HTAU, CH_HALPHA, CH_HBETA, CH_NCOL
};
enum HalfGapCol { HG_G = 0, HG_VGAP, HG_I, HG_NCOL };
enum HdLaCol { HD_GHDBAR = 0, HD_VHALFL, HD_TAU, HD_L, HD_I, HD_LINF, HD_TAUL, HD_GHD, HD_NCOL };
// NetStim (src/spike/netstim.cpp): parameters only; its spike trains are made on
// the host.  id1 < 0 stands for the instance index.
enum NetStimCol { NS_INTERVAL = 0, NS_NUMBER, NS_START, NS_NOISE, NS_ID1, NS_ID2, NS_ID3, NS_NCOL };

// Per-mechanism device view.
constexpr int kUniformCols = 32;   // parameter columns a mechanism may serve as one value

struct MechDev {
    double* base = nullptr;       // column c at base + c * stride
    long long stride = 0;
    int n = 0;
    int dense = 0;                // instance i on node i for every node
    const int* node = nullptr;    // solver-order node of each instance
    const int* ion[3] = {nullptr, nullptr, nullptr};   // na, k, ca instance of each instance
    const int* iontype = nullptr; // ions only
    // point processes: instances grouped by node (instances are sorted by node):
    // group g is node grp_node[g] with instances [grp_begin[g], grp_begin[g+1])
    const int* grp_node = nullptr;
    const int* grp_begin = nullptr;
    int ngrp = 0;
    // synapses folded into the node kernel: instances on the nodes of node-kernel
    // block b are [blk_begin[b], blk_begin[b+1])
    const int* blk_begin = nullptr;
    // parameter columns that hold one value for every instance: bit c set means
    // column c is uval[c] everywhere (the full column in HBM holds the same values)
    unsigned umask = 0;
    const double* uval = nullptr;
    __host__ __device__ double* col(int c) const { return base + c * stride; }
};

// Global constants of the hot-path mechanisms, computed once on the host
// with the same expressions the reference evaluates per call.
constexpr double kFaradayCaDyn = 96485.3321233100184;   // CaDynamics_E2.cu:109
// Default concentrations of na, k and ca (mM) that INITIAL sets where an ion's style has
// 04 (eion.cuh:183-197)
constexpr double kIonConciInit[3] = {10.0, 140.0, 5.e-5};
constexpr double kIonConcoInit[3] = {140.0, 4.0, 2.0};

struct MechConsts {
    double hh_q10;                // pow(3, (celsius - 6.3) / 10)            hh_templated.cu:87
    double hd_qt;                 // pow(q10, (celsius - 33) / 10)           hd_la.cu:94
    double hd_ehd, hd_kl, hd_vhalft, hd_a0t, hd_zetat, hd_gmt, hd_qtl;
    double hd_inv_kl;             // 1 / hd_kl
    int hd_pow;                   // gmt is 0.4: the two exponentials of the rate are G^5 and G^2
    double hd_k5;                 // 0.0378 zetat / 5, G = exp(hd_k5 (v - vhalft))
    double ktf;                   // 1000 R (celsius + 273.15) / F           eion.cuh:33-36
    // CaDynamics_E2 with gamma, decay, depth and minCai each one value over the model: its
    // update is cai + cd_c1 (ica cd_g + cd_min - cai), c1 = 1 - exp(-dt / decay),
    // g = -1e4 gamma decay / (2 F depth)
    int cd_uniform;
    double cd_c1, cd_g, cd_min;
};

struct StepArgs {
    int N;                        // node kernels cover nodes [node0, N)
    int node0;                    // first node (a cell group's range; 0 for the whole model)
    int pt0, pt1;                 // synapse-decay launches cover instances [pt0, min(pt1, n))
    double* v;
    double* d;
    double* rhs;
    const double* area;
    const double* cm;             // capacitance, added to d by the current pass
    int cm_uniform;               // cm holds cm_value on every node: read as that value
    double cm_value;
    double cfac;                  // 1e-3 * cj (capac.cpp:68-80)
    MechDev m[M_COUNT];
    unsigned dense_mask;          // mechanisms processed by the fused node kernel
    int hh_owns_ions;             // sparse hh stores the na / k currents (the ion kernels do not run)
    int do_state;                 // finish the previous step's state update first
    int cadyn_skip;               // ... except CaDynamics_E2, already updated by the last current pass
    int yform;                    // store rhs + d v in rhs: the solve then yields v_new itself (every
                                  // d and rhs term of the step comes from this pass)
    int cadyn_after;              // update CaDynamics_E2 right after this pass's ica (its state
                                  // depends on ica and cai only, so this is the step's own update)
    int do_current;
    int write_assigned;           // also store the current's assigned outputs (i, ina, gna, ...)
    int point_assigned;           // the node kernel's synapse fold stores the synapses' outputs (i, g)
    int write_rates;              // also store the state update's rates (minf, mtau, ...)
    int write_dcurdv;             // store the ions' dcurdv (0: it still holds the 0 stored at init)
    unsigned ion_store;           // ion x (0 na, 1 k, 2 ca): bit 2x stores cur, bit 2x+1 stores erev
    unsigned fold_mask;           // point processes whose currents the node kernel adds (bit = MechId)
    int ion_type[3];              // iontype shared by every instance of ion x, or -1 (read per instance)
    double t;                     // time of the current evaluation (t_n + dt/2)
    double dt;
    MechConsts c;
};

// Nodes carrying IClamp or HalfGap instances (sorted), with each node's group of either
// mechanism (MechDev::grp_node / grp_begin index) or -1: one launch adds both currents.
struct PointUnion {
    int n = 0;
    const int* node = nullptr;
    const int* grp[2] = {nullptr, nullptr};   // IClamp, HalfGap
};

// Chunked tree-solve schedule (one wavefront per solve unit: a few
// consecutive cells solved as one forest).  Indices are relative to the unit
// (units are limited to 65535 nodes and 65535 chunks), so a descriptor packs
// into 8 bytes.
constexpr int kBlock = 256;       // threads per block of the node-parallel kernels
constexpr uint16_t kNone = 0xFFFF;
constexpr int kChunk = 16;        // max nodes per chunk (one lane's serial run)
constexpr int kWave = 64;
constexpr int kMaxCellNodes = 65535;
constexpr int kRoundMax = 384;    // max nodes per round (one LDS stage)
constexpr int kPer = kRoundMax / kWave;   // stage elements per lane per array

struct ChunkDesc {
    uint16_t slot;         // junction slot of this chunk (its breadth-first id)
    uint16_t parent_slot;  // slot of the chunk whose tail is the head's parent (kNone for the root chunk)
    uint16_t child_begin;  // slots of the chunks hanging off the tail: [child_begin, +child_count)
    uint8_t len;           // nodes in the chunk (<= kChunk); a round's chunks are sorted by len, longest first
    uint8_t child_count;
};
static_assert(sizeof(ChunkDesc) == 8, "ChunkDesc must stay 8 bytes");

// One round of a unit's schedule: its descriptors and its contiguous,
// position-major block of nodes (all unit-relative).  Node k of the chunk on
// lane l sits at node_base + off[k] + l, where off[k] = sum_{j<k} W_j and W_j
// is the number of the round's chunks longer than j.
struct alignas(16) RoundInfo {
    uint16_t desc_begin;
    uint16_t desc_count;
    uint16_t node_base;
    uint16_t node_count;
    uint16_t off[kChunk];
    uint8_t maxlen;        // longest chunk of the round (0 for a padding round)
    uint8_t pad8[3];
    uint32_t pad;
};
static_assert(sizeof(RoundInfo) == 48, "RoundInfo must stay 48 bytes");

struct SolveArgs {
    int nunit;
    const int* unit_node_begin;   // [nunit+1] first solver-order node of each solve unit
    const int* unit_desc_begin;   // [nunit+1] first descriptor of each unit
    const int* unit_round_begin;  // [nunit+1] first round of each unit
    const RoundInfo* rounds;
    const ChunkDesc* desc;
    double* v;
    double* d;                    // in: membrane + capacitance diagonal; out (store_dx): eliminated diagonal D
    double* rhs;                  // in: membrane right-hand side; between the sweeps s; out (store_dx): solution x
    double* w;                    // scratch: b / D per node, written by elimination
    const double* a;
    const double* b;
    int store_dx;                 // 1: leave D in d and x = vn - v in rhs (as the reference does); 0: neither
    int waves;                    // solve units per workgroup, one wavefront each (1..kSolveMaxWaves)
    int yform;                    // 1: rhs holds rhs + d v, so elimination takes v as 0 and back
                                  // substitution yields v_new directly (v is read only for x)
    int res_nodes;                // > 0: each unit is solved held whole in LDS, sized for this many nodes
    int res_rounds;               //   and this many rounds (the largest unit's); 0: rounds streamed from HBM
};

// Event ring: one slot per delivery step (mod nslot), fixed capacity per slot.
struct EventRing {
    int* count;                   // [nslot]
    int* entry;                   // [nslot * cap], packed (type << 30) | instance
    int nslot;                    // power of two
    int cap;
    int* overflow;                // set to 1 when a slot overflowed
    unsigned* done;               // workgroups of the delivery launch that have finished (then back to 0)
};

// A packed fan-out target: bits 30-31 its kind (0 ExpSyn, 1 Exp2Syn, 2 NetStim, 3 a synapse
// plugin), bits 0-29 the instance (for kind 3: bits 26-29 the plugin's synapse slot, bits
// 0-25 the instance).  Kinds 2 and 3 set the sign bit, so the kind is read with an unsigned
// shift.
constexpr int kTargetNetStim = 2;
constexpr int kTargetPlugin = 3;
constexpr int kMaxPostsyn = 4;          // synapse plugins one model may use
constexpr int kPostsynSlotShift = 26;
__host__ __device__ inline int pack_target(int kind, int inst) {
    return static_cast<int>((static_cast<unsigned>(kind) << 30) | static_cast<unsigned>(inst));
}
__host__ __device__ inline int target_kind(int packed) { return static_cast<int>(static_cast<unsigned>(packed) >> 30); }
__host__ __device__ inline int target_inst(int packed) { return packed & 0x3fffffff; }

// Fan-out tables: source -> synapse targets (packed type|instance) with delays.
struct FanOut {
    const int* begin;             // [nsrc+1]
    const int* target;
    const double* delay;
};

// Events into NetStims that receive netcons, by delivery step: entry (round << 24) |
// instance and its delivery time.  The round is the pass of the step's delivery loop
// in which the event reaches the NetStim (1: it was there when the step began).
struct NsInbox {
    int* count;                   // [nslot]
    int* entry;                   // [nslot * cap]
    double* time;                 // [nslot * cap]
    int nslot;
    int cap;
    int* error;                   // bit 0: a slot overflowed
};
constexpr int kNsRoundShift = 24;

// What the host checks after a call: the event rings' overflow flags, the NetStim error
// bits and the spike count, gathered by one kernel into pinned host memory.
struct StatusArgs {
    const int* const* ring_overflow;   // [ngroups]
    int ngroups;
    const int* ns_error;               // null without event-receiving NetStims
    const int* spk_count;
    int* out;                          // host: [0] overflow (OR), [1] NetStim error, [2] spikes
};

struct SpikeArgs {
    int npre;
    const double* v;
    const int* node;              // solver-order node of each detector
    const double* thr;
    int* flag;
    const int* gid;
    double t;                     // step start time t_k
    int k;                        // step index (delivery slot base)
    double* log_t;                // spike log
    int* log_gid;
    int* log_count;
    int log_cap;
    FanOut fo;
    EventRing ring;
    NsInbox ib;                   // fan-out targets of type 2 (NetStims)
    const double* ttab;           // t of every step since finitialize
    int kmax;                     // last valid ttab index
    double half_dt;
};

struct VecPlayDev;

// The work after a step's solve, one launch (k_after_solve); the launcher sets the
// block offsets from the counts.  A task with no items gets no blocks.
// Up to kTapeSegs device-to-device copies in one launch (a step's tape row).
constexpr int kTapeSegs = 8;
struct TapeCopy {
    const double* src[kTapeSegs];
    double* dst[kTapeSegs];
    long long n[kTapeSegs];
    int nseg;
};
struct AfterSolve {
    int b_ptr, b_spike, b_vp, b_es, b_e2;   // first block of each task (gap transfers from 0)
    const double* v;
    const int* gap_src;                     // gap transfers of the model: vgap[gap_inst[i]] = v[gap_src[i]]
    double* vgap;
    const int* gap_inst;
    int ngap;
    double* const* psrc;                    // transfers added at run time: *pdst[i] = *psrc[i]
    double* const* pdst;
    int nptr;
    SpikeArgs S;                            // threshold detection of the next step (npre 0: none)
    VecPlayDev* vp;                         // VecPlay at the step's end time (nvp 0: none)
    int nvp;
    double t;
    double* es_g;                           // ExpSyn decay over instances [es0, es1)
    const double* es_tau;
    int es0, es1;
    double *e2_a, *e2_b;                    // Exp2Syn decay over instances [e20, e21)
    const double *e2_tau1, *e2_tau2;
    int e20, e21;
    double dt;
    // the adjoint tape's row of the step (nseg 0: none): the segments are copied on blocks
    // of their own; the synapse states, which the decay tasks change, are taped by those
    // tasks before they decay them (es_tape[j], e2_tape_a[j], e2_tape_b[j]; null: not taped)
    TapeCopy tape;
    double* es_tape;
    double *e2_tape_a, *e2_tape_b;
    int b_tape;
};

struct InputArgs {
    const double* eff_time;       // sorted effective VecStim event times
    const int* inst;              // VecStim instance of each event
    const int* round;             // pass of the delivery loop that emits each event's spike
    int n;
    int* cursor;                  // first unprocessed event
    double tcut;                  // t_k + dt/2
    double t;                     // t_k
    int k;
    FanOut fo;
    EventRing ring;
    NsInbox ib;
    const double* ttab;
    int kmax;
    double half_dt;
};

// NetStims that receive events (netstim.cpp:211-330 with one stream per instance),
// run on the device by k_netstim: per instance its state, its pending self events and
// its random stream; instance j of these is NetStim instance inst[j].
constexpr int kNsQueue = 8;       // pending self events per instance
constexpr int kNsMini = 8;        // events reaching one instance in one pass
constexpr int kNsRounds = 64;     // passes of one step's delivery loop
constexpr int kNsRng = 10;        // words of stream state per instance
struct NsArgs {
    int n;
    const int* inst;
    double* interval;
    double* number;
    double* noise;                // clamped to [0, 1] at finitialize
    const double* weight;         // weight of the instance's incoming netcon
    double* on;
    double* ispike;
    double* event;
    double* q_t;                  // [n * kNsQueue] self-event times
    int* q_kind;                  // 0 self event, 1 init event
    long long* q_born;            // (step << 8) | pass that sent it (pass 0: finitialize)
    int* q_n;
    unsigned* rng;                // [n * kNsRng]: counter, block, word index, key
    int* mini_n;                  // [n]
    int* mini_e;                  // [n * kNsMini]
    NsInbox ib;
    FanOut fo;                    // outputs of each of these instances
    EventRing ring;
    const double* ttab;
    int kmax;
    double half_dt;
    double t;                     // t_k
    int k;
    double* log_t;                // spikes of these NetStims: time and NetStim instance
    int* log_inst;
    int* log_count;
    int log_cap;
    int* error;                   // bit 1: a pass brought more than kNsMini events to one
                                  // instance; bit 2: more than kNsRounds passes; bit 3: a
                                  // self-event queue overflowed
};

struct DeliverArgs {
    EventRing ring;
    int k;
    int* plugin_recv[kMaxPostsyn];    // events per instance of each synapse plugin (kind 3)
    MechDev es;                   // ExpSyn
    MechDev e2;                   // Exp2Syn
    const double* es_weight;
    const double* e2_weight;
    int* log_count;               // when set: every delivered event (packed as in the ring) is appended
    int* log;                     // to log[0 .. *log_count) (capacity log_cap), for the adjoint
    int log_cap;
    // VecPlay at the current evaluation's time on blocks of their own (nvp 0: none); only
    // for targets delivery never touches (IClamp variables), so the two tasks are independent
    VecPlayDev* vp;
    int nvp;
    double t_vp;
    int ndeliver;                 // blocks of the delivery task (set by launch_deliver)
};

// The cell groups' VecStim input and delivery of one step in one launch each, when the
// groups share one stream: each group keeps its own trains, cursor and ring.
constexpr int kMaxMergedGroups = 8;
struct InputSet {
    InputArgs a[kMaxMergedGroups];
    int n;
};
struct RingSet {
    EventRing r[kMaxMergedGroups];
    int n;
};

// One backward step of the adjoint (adjoint.hip).  v1, x0, geff: the taped
// v^{n+1} (node order), hh gates x^n (3 columns of xstride) and ExpSyn g_eff^n.
struct AdjStep {
    int N;
    double dt, cfac, hh_q10;
    MechConsts c;
    const double* cm;
    const double* area;
    const double* delta;          // diagonal correction of the transposed solve
    MechDev m[M_COUNT];
    const double* v1;
    const double* x0;
    long long xstride;
    const double* geff;
    double* lam_v;                // adjoint of v^{n+1}
    double* lam_v_new;            // adjoint of v^n
    double* lam_x;                // adjoint of the gates (x^{n+1} in, x^n out)
    double* lam_g;                // adjoint of ExpSyn g (g^{n+1} in, g^n out)
    double* dT;
    double* rhsT;
    const double* mu;             // M^{-T} lam_v (the transposed solve's solution)
    double* grad_gnabar;
    double* grad_gkbar;
    double* grad_gpas;
    double* grad_w;               // ExpSyn netcon weights
    const int* ev_count;          // events delivered at step n
    const int* ev;                // packed (type << 30) | instance, as in the event ring
    // Ca_HVA, hd_la, CaDynamics_E2 (+ ca_ion) and Exp2Syn
    const double* v0;             // v^n, the voltage of step n's current pass (ica uses it)
    const double* c0;             // Ca_HVA m^n, h^n (2 columns of cstride)
    long long cstride;
    double* lam_c;                // adjoint of the Ca_HVA gates
    const double* l0;             // hd_la l^n
    double* lam_l;
    const double* cai0;           // cai^n per ca_ion instance
    double* lam_cai;              // adjoint of cai (cai^{n+1} in, cai^n out)
    double* lam_ica;              // per ca_ion instance: adjoint of the ica that CaDynamics_E2 reads
    const double* ab0;            // Exp2Syn A_eff^n, B_eff^n (2 columns of the instance count)
    double* lam_ab;               // adjoint of A, B (step n+1 in, step n out)
    double* grad_cgbar;           // Ca_HVA gbar
    double* grad_ghdbar;          // hd_la ghdbar
    double* grad_w2;              // Exp2Syn netcon weights
    // mechanisms the node-parallel adjoint kernels take (kAdj* bits; each has one instance
    // on every node, instance i at node i): gate adjoints and CaDynamics_E2 (fuse_state),
    // conductances (fuse_cond), parameter terms (fuse_param)
    unsigned fuse_state, fuse_cond, fuse_param;
    // fold_syn: the node-parallel kernels also take the synapses (decay adjoints and
    // parameter terms on threads N.., each node's grouped conductances after its density
    // ones); es_grp / e2_grp map a node to its ExpSyn / Exp2Syn group (-1: none)
    int fold_syn;
    const int* es_grp;
    const int* e2_grp;
    // loss term of lambda_v^n added by k_adj_after_nodes (loss_v null: by k_adj_loss):
    // node i adds 2 loss_scale (loss_v[i] - loss_tgt[loss_of_node[i]]) where that index is >= 0
    const double* loss_v;
    const double* loss_tgt;
    const int* loss_of_node;
    double loss_scale;
    // gap junctions (HalfGap): the source node of each instance's vgap (-1: none, vgap is a
    // constant), and the distinct source nodes with the instances they feed
    // (gap_inst[gap_begin[q] .. gap_begin[q+1]) for source gap_src[q])
    const int* gap_partner;
    int ngap_src;
    const int* gap_src;
    const int* gap_begin;
    const int* gap_inst;
    double* grad_ggap;            // HalfGap g
};
constexpr unsigned kAdjPas = 1, kAdjHH = 2, kAdjCaHVA = 4, kAdjHdla = 8, kAdjCaDyn = 16;

// Adam over tied parameter groups (optimizer.cpp:351-393): group g covers
// entries [begin[g], begin[g+1]) of the weight and gradient pointer lists.
// Optimizer step over tied parameter groups (optimizer.cpp:102-135 SGD, 190-240
// momentum, 351-413 Adam): type 0 SGD, 1 momentum (m holds the velocity), 2 Adam.
struct AdamArgs {
    int type;
    double momentum;
    int ngroup;
    const int* begin;
    double* const* w;
    double* const* grad;
    const double* impedance;
    double* m;
    double* v;
    double lr, inv_record_steps, beta1, beta2, eps;
    long long step;
};

struct VecPlayDev {
    double* target;
    const double* tvec;
    const double* yvec;
    int len;
    int last_index;
    int next_idx;
    int done;
    double next_time;
};

// LDS of the solve kernel: two junction values per chunk, then one round
// stage of kStageArrays arrays, each with a neutral entry after its kRoundMax
// nodes.
constexpr int kStageArrays = 5;
constexpr int kStageStride = kRoundMax + 1;
// Solve units: the default unit size aims at about kSolveUnitTarget units in
// all (one wavefront per SIMD of the chip), and a unit's LDS stays within
// kUnitLdsBudget so that four units fit in a CU's 160 KB.
constexpr int kSolveUnitTarget = 1024;
constexpr size_t kUnitLdsBudget = 40 * 1024;
// A workgroup of the tree solve holds up to kSolveMaxWaves units, one wavefront each:
// the CU spreads a workgroup's wavefronts over its four SIMDs, so four units in one
// workgroup put one solve wavefront on each SIMD.
constexpr int kSolveMaxWaves = 4;
// LDS of one unit in doubles (junction pairs, then the stage), rounded to 16 bytes so
// that every unit's pairs stay 16-byte aligned inside a multi-unit workgroup.
__host__ __device__ inline int solve_lds_doubles(int max_chunks) {
    const int mc = max_chunks > 0 ? max_chunks : 1;
    return (2 * mc + kStageArrays * kStageStride + 1) & ~1;
}
inline size_t solve_lds_bytes(int max_chunks) {
    return static_cast<size_t>(solve_lds_doubles(max_chunks)) * sizeof(double);
}
// A unit held whole in LDS: junction pairs, then one record of kStageArrays doubles per
// node (max_nodes records, a neutral record and a sink record, rounded to an even count so
// that what follows stays 16-byte aligned), the unit's round table (6 doubles a round) and
// its chunk descriptors (one double each; a unit has one descriptor per chunk).  Units are
// solved this way when this stays within kResUnitBudget, so four fit in a CU's 160 KB.
constexpr size_t kResUnitBudget = 40 * 1024;
__host__ __device__ inline int res_record_doubles(int max_nodes) { return ((max_nodes + 2) * kStageArrays + 1) & ~1; }
__host__ __device__ inline int res_lds_doubles(int max_nodes, int max_chunks, int max_rounds) {
    const int mc = max_chunks > 0 ? max_chunks : 1;
    return (2 * mc + res_record_doubles(max_nodes) + 6 * max_rounds + mc + 1) & ~1;
}
inline size_t res_lds_bytes(int max_nodes, int max_chunks, int max_rounds) {
    return static_cast<size_t>(res_lds_doubles(max_nodes, max_chunks, max_rounds)) * sizeof(double);
}

// launch wrappers (kernels.hip)
// steady: a launch whose flags are a steady step of a mechanism set with a compile-time
// instance runs that instance (same bits as the generic kernel).  e0, e1 (may be null):
// events set to the kernel's start and end as part of its dispatch (no marker of their
// own on the stream).  Returns 0 if nothing was launched, 1 for the generic kernel, 2 for
// a steady instance.
int launch_dense(const StepArgs& a, hipStream_t s, bool steady, hipEvent_t e0 = nullptr, hipEvent_t e1 = nullptr);
void launch_sparse(int mech, const StepArgs& a, hipStream_t s);
void launch_point_current(int mech, const StepArgs& a, hipStream_t s);
void launch_point_electrodes(const StepArgs& a, const PointUnion& u, hipStream_t s);
void launch_after_solve(AfterSolve p, hipStream_t s);
void launch_point_state(int mech, const StepArgs& a, hipStream_t s);
void launch_init(int mech, const StepArgs& a, hipStream_t s);
void launch_set_v(double* v, int n, double val, hipStream_t s);
void launch_solve(const SolveArgs& a, int max_chunks, hipStream_t s);
void launch_input_set(const InputSet& a, hipStream_t s);
void launch_deliver_set(const DeliverArgs& a, const RingSet& rings, int nblk, hipStream_t s);
// streaming probe (nread, nwrite) in {(1,1), (11,9), (26,9)}; false for other mixes
bool launch_stream(int nread, int nwrite, const double* in, double* out, long long n, hipStream_t s);
void launch_adj_before_solve(const AdjStep& a, hipStream_t s);
void launch_adj_after_solve(const AdjStep& a, hipStream_t s);
void launch_adj_loss(const double* v, const int* nodes, const int* begin, const int* idx, int n,
                     const double* target, double scale, double* lam, hipStream_t s);
void launch_adj_gather(const double* tape_v, long long row, const int* nodes, int nnodes, int nrows, double* out,
                       hipStream_t s);
void launch_adam(const AdamArgs& a, hipStream_t s);
void launch_spike(const SpikeArgs& a, hipStream_t s);
void launch_input(const InputArgs& a, hipStream_t s);
void launch_netstim(const NsArgs& a, hipStream_t s);
void launch_deliver(const DeliverArgs& a, int nblk, hipStream_t s);
void launch_vecplay(VecPlayDev* items, int n, double t, int do_play, hipStream_t s);
void launch_vecplay_reset(VecPlayDev* items, int n, hipStream_t s);
void launch_record(double* const* ptrs, int n, double* out, hipStream_t s);
void launch_gap(const double* v, const int* src_node, double* vgap_col, const int* halfgap_inst, int n,
                hipStream_t s);
void launch_clear_ints(int* p, long long n, hipStream_t s);
void launch_status(const StatusArgs& a, hipStream_t s);
void launch_tape(const TapeCopy& t, hipStream_t s);
void launch_copy_ptrs(double* const* src, double* const* dst, int n, hipStream_t s);

}  // namespace hx
