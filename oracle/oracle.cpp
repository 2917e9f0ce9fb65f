// oracle/oracle.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A CPU restatement of the HelioX reference CPU step loop, used as the parity
// checker for the HIP path and as the timed CPU baseline.  Nothing in the
// product links, loads or executes this file; only tests, the smoke check and
// the CPU-baseline leg of the benchmark do.
//
// It follows the reference CPU path literally (serial loops, the same
// expression forms, the same call order), compiled with -ffp-contract=off as
// the reference host code is (CMakeLists.txt:26-44):
//   step loop ............ src/simulate.cpp:343-449 (run/continue_run/fadvance_cpu)
//   finitialize .......... src/simulate.cpp:271-339
//   setup_tree_matrix .... src/simulate.cpp:455-556
//   solve_serial ......... src/simulate.cpp:558-581
//   update / last_part ... src/simulate.cpp:759-852
//   spike send/receive ... src/simulate.cpp:858-939, src/spike/presyn.cpp:133-177,
//                          src/spike/postsyn.cpp:43-113, src/spike/spike.h:113-136
//   gap transfer ......... src/simulate.cpp:953-966
//   FD current loop ...... src/mech/mech_template.cuh:589-648 (state 676-698)
//   ions ................. src/mech/eion.cuh:155-214 (+ units.h:22-24)
//   capacitance .......... src/mech/build-in-mech/capac.cpp:54-80
//   hh ................... src/mech/user-mech/hh_templated.cu:76-164
//   pas .................. src/mech/user-mech/pas_templated.cu:27-31
//   IClamp ............... src/mech/user-mech/iclamp_templated.cu:15-40
//   Ca_HVA ............... src/mech/user-mech/CA_HVA.cu:97-178
//   hd_la (Ih) ........... src/mech/user-mech/hd_la.cu:80-128
//   CaDynamics_E2 ........ src/mech/user-mech/CaDynamics_E2.cu:78-139
//   HalfGap .............. src/mech/user-mech/HalfGap.cu:52-68
//   ExpSyn ............... src/spike/postsyn_mech/expsyn.cpp (current/state/net_receive)
//   Exp2Syn .............. src/spike/user_postsyn_mech/exp2syn_temp.cuh:29-67
//   VecStim .............. src/spike/vecevent.cpp:94-217, src/spike/articell.cpp:18-35
//   NetStim .............. src/spike/netstim.cpp:211-330 with one stream per instance
//                          (src/utils/nrnran123.cpp:23-110; Philox4x32-10 as published
//                          by Salmon et al., SC11), netcon events included; every
//                          processed event keeps the delivery loop going
//   Im ................... src/mech/user-mech/Im.cu:9-130
//   syn_record ........... src/spike/user_postsyn_mech/syn_record.cuh:8-203
//   VecPlay .............. src/vecplay.cu:19-111
//   Adam ................. src/optimizer/optimizer.cpp:351-413
//
// Mechanism order: the reference evaluates currents in CoreNEURON type order
// (coredat_to_innerdat.cpp:176-181).  The oracle uses the fixed order of
// kMechOrder below, which is the NEURON built-in type order followed by the
// user mechanisms; the HIP path documents its own accumulation order.
//
// Pinning: every function above is checked, in tests/test_oracle_pinning.py,
// tests/test_netstim.py and tests/test_lrds_oracle.py, against closed forms, textbook
// rates, known-answer vectors or brute force chosen so that a plausible slip (a dropped
// term, a wrong sign, index or exponent) fails one of them; no function is left with
// parity unpinned.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <queue>
#include <string>
#include <vector>
#include <algorithm>

namespace {

constexpr double kFaraday = 1.602176634e-19 * 6.02214076e+23;   // units.h:22
constexpr double kGasConst = 1.380649e-23 * 6.02214076e+23;     // units.h:24

double ktf(double celsius) { return 1000. * kGasConst * (celsius + 273.15) / kFaraday; }

double nrn_nernst(double ci, double co, double z, double celsius) {   // eion.cuh:39-57
    if (z == 0) return 0.;
    if (ci <= 0.) return 1e6;
    else if (co <= 0.) return -1e6;
    else return ktf(celsius) / z * std::log(co / ci);
}

struct Model;

// ---------------------------------------------------------------------------
// Mechanism base: per-instance SoA columns addressed by name.
// ---------------------------------------------------------------------------
struct Mech {
    std::string name;
    int n = 0;
    std::vector<int> node;                       // node index of each instance
    std::map<std::string, std::vector<double>> col;  // per-instance variables
    std::map<std::string, double> glob;          // mechanism globals
    bool point_process = false, electrode = false, write_state_ion = false, is_ion = false;
    Model* m = nullptr;
    virtual ~Mech() = default;
    virtual void alloc() {}
    virtual void bind() {}
    virtual void init(const double* v) {}
    virtual void current(const double* v, double* d, double* rhs, double t) {}
    virtual void state(const double* v, double dt, double t) {}
    std::vector<double>& C(const char* k) { return col[k]; }
    void ensure(const char* k, double dflt) {
        auto& c = col[k];
        if ((int)c.size() != n) c.assign(n, dflt);
    }
};

// ---------------------------------------------------------------------------
// Ions: one instance per node that uses the ion (eion.cuh:69-338).
// ---------------------------------------------------------------------------
struct Ion : Mech {
    double charge, conci0, conco0;
    std::vector<int> iontype;
    std::vector<int> node2inst;   // node -> instance (or -1)
    Ion(const char* nm, double z, double ci0, double co0) : charge(z), conci0(ci0), conco0(co0) {
        name = nm; is_ion = true;
    }
    void alloc() override {
        ensure("erev", 0.0); ensure("conci", conci0); ensure("conco", conco0);
        ensure("cur", 0.0); ensure("dcurdv", 0.0);
        if ((int)iontype.size() != n) iontype.assign(n, 0);
    }
    double *erev, *conci, *conco, *cur, *dcurdv;
    void bind() override {
        erev = C("erev").data(); conci = C("conci").data(); conco = C("conco").data();
        cur = C("cur").data(); dcurdv = C("dcurdv").data();
    }
    void init(const double*) override;                 // eion.cuh:183-197
    void current(const double*, double*, double*, double) override;   // eion.cuh:155-166
};

// ---------------------------------------------------------------------------
// Templated density/point mechanisms: FD current loop of mech_template.cuh.
// Derived classes provide cur(i, volt, t, updateIon) returning the current.
// ---------------------------------------------------------------------------
struct TMech : Mech {
    virtual double cur(int i, double volt, double t, bool updateIon) = 0;
    void current(const double* v, double* d, double* rhs, double t) override;
};

struct Model {
    int ncell = 0, len = 0;
    std::vector<int> parent;
    std::vector<double> a, b, area, v, d, rhs, cm;
    double cj = 0, t = 0, dt = 0.025, celsius = 6.3;

    std::map<std::string, std::unique_ptr<Mech>> mechs;
    std::vector<Mech*> current_list;     // CoreNEURON order
    std::vector<Mech*> state_ion_first;  // write_state_ion mechanisms
    std::vector<Mech*> state_rest;       // mechanism_list minus write_state_ion, no ions

    // spikes (spike.h, presyn.cpp, postsyn.cpp, articell.cpp)
    struct Spike {
        int gid = -1, pre_node_id = -1, syn_type = -1, syn_id = -1;
        int flag = -1;
        double deliver_time = -1.0;
    };
    struct Cmp {
        bool operator()(const Spike& e1, const Spike& e2) const {   // spike.h:113-134
            bool result = false;
            if (std::fabs(e1.deliver_time - e2.deliver_time) > 1e-9)
                result = e1.deliver_time > e2.deliver_time;
            else {
                if (e1.syn_type != e2.syn_type) result = e1.syn_type > e2.syn_type;
                else if (e1.syn_id != e2.syn_id) result = e1.syn_id > e2.syn_id;
                else result = e1.pre_node_id > e2.pre_node_id;
            }
            return result;
        }
    };
    using SpikeBuffer = std::priority_queue<Spike, std::vector<Spike>, Cmp>;
    enum { INVALID = -1, NORMAL_EVENT = 0, SELF_EVENT = 1, NETSTIM_INIT_EVENT = 2 };

    // real presyns occupy spike slots [0, npre); VecStim instance k occupies npre + k
    std::vector<int> pre_node, pre_gid;
    std::vector<double> pre_thr;
    std::vector<char> pre_flag;
    std::vector<Spike> spk_vec;
    std::vector<int> spk_flags;
    std::vector<std::pair<double, int>> rec_spikes;
    std::vector<std::vector<double>> spk_output;

    static constexpr uint32_t kNoSource = 0xffffffffu;
    struct PostSynState {             // PostSyn_trait (postsyn.h)
        Mech* mech = nullptr;
        int type_id = 0;
        std::vector<uint32_t> spk_vec_idx;
        std::vector<double> delay, weight;
        SpikeBuffer buffer;
        std::vector<uint32_t> receive_idx;
        std::vector<int> receive_flag;
        int receive_count = 0;
        bool artificial = false;
    };
    std::vector<PostSynState> postsyns;   // in CoreNEURON type order

    // VecStim (vecevent.cpp)
    std::vector<std::vector<double>> vs_times;
    std::vector<int> vs_index;
    std::vector<double> vs_etime;
    int vs_postsyn = -1;
    // NetStim (netstim.cpp): spike slots after the VecStim ones
    int ns_postsyn = -1;
    std::vector<std::pair<double, int>> ns_spikes;   // (time, instance) of every NetStim spike
    void net_send_netstim(uint32_t idx, double tt, int flag);
    void netstim_init();
    bool netstim_receive(int isyn, int flag);

    // VecPlay (vecplay.cu)
    struct VecPlayItem {
        double* target;
        std::vector<double> tvec, yvec;
        int len, last_index, next_idx;
        bool done;
        double next_time;
        void play(double tt) {                      // vecplay.cu:19-45
            while (1) {
                if (done || next_time > tt) return;
                last_index = next_idx;
                if (next_idx < len - 1) { next_idx++; next_time = tvec[next_idx]; }
                else done = true;
            }
        }
        void search(double tt) {                    // vecplay.cu:81-90
            while (tt < tvec[last_index]) --last_index;
            while (tt >= tvec[last_index]) ++last_index;
        }
        double interpolate(double tt) {             // vecplay.cu:57-79
            if (tt >= tvec[next_idx]) {
                last_index = next_idx;
                if (last_index == 0) return yvec[last_index];
            } else if (tt <= tvec[0]) {
                last_index = 0;
                return yvec[0];
            } else {
                search(tt);
            }
            double x0 = yvec[last_index - 1], x1 = yvec[last_index];
            double t0 = tvec[last_index - 1], t1 = tvec[last_index];
            if (t0 == t1) return (x0 + x1) / 2.;
            double th = (tt - t0) / (t1 - t0);
            return x0 + (x1 - x0) * th;
        }
        void continuous(double tt) { *target = interpolate(tt); }
        void reset() {                              // vecplay.cu:95-111
            last_index = 0; next_idx = 0; done = false;
            if (len > 0) next_time = tvec[0];
            else { next_time = 0.0; done = true; }
        }
    };
    std::vector<VecPlayItem> vecplay;

    // gap transfer: *dst = *src after update (simulate.cpp:953-966)
    std::vector<std::pair<double*, double*>> gaps;   // (src, dst)

    // recorder
    std::vector<double*> rec_ptr;
    std::vector<std::vector<double>> rec_data;

    // Adam state (optimizer.cpp:351-413)
    struct AdamParam { std::vector<double*> w, g; double impedance; };
    std::vector<AdamParam> adam_params;
    std::vector<double> adam_m, adam_v;
    long long adam_step = 0;
    double beta1 = 0.9, beta2 = 0.999, eps = 1e-8;

    bool finalized = false;

    // ---- step pieces -------------------------------------------------------
    void setup_tree_matrix();
    void solve_serial();
    void update();
    void last_part();
    void nonvint();
    void spike_deliver();
    void network_spike_send();
    void network_spike_receive();
    void gap_transfer() { for (auto& g : gaps) *g.second = *g.first; }
    void log_data() { for (size_t i = 0; i < rec_ptr.size(); ++i) rec_data[i].push_back(*rec_ptr[i]); }
    void finitialize(double v_init);
    void fadvance();
    void net_send_vecstim(uint32_t idx, double tt, int flag);
    void vecstim_element(int inode);
    double* var_ptr(const std::string& mech, const std::string& var, int idx);
};

void Ion::init(const double*) {
    for (int i = 0; i < n; ++i) {
        int it = iontype[i];
        if (it & 04) { conci[i] = conci0; conco[i] = conco0; }
        if (it & 040) erev[i] = nrn_nernst(conci[i], conco[i], charge, m->celsius);
    }
}

void Ion::current(const double*, double*, double*, double) {
    for (int i = 0; i < n; ++i) {
        int it = iontype[i];
        cur[i] = 0.;
        dcurdv[i] = 0.;
        if (it & 0100) erev[i] = nrn_nernst(conci[i], conco[i], charge, m->celsius);
    }
}

void TMech::current(const double* v, double* vd, double* vrhs, double t) {
    // mech_template.cuh:589-648
    for (int i = 0; i < n; ++i) {
        int ni = node[i];
        double _v = v[ni];
        double _g = cur(i, _v + 0.001, t, false);
        double _rhs = cur(i, _v, t, true);
        _g = (_g - _rhs) / 0.001;
        if (point_process) {
            double nd_area = m->area[ni];
            _g *= 1.e2 / nd_area;
            _rhs *= 1.e2 / nd_area;
        }
        if (electrode) { vrhs[ni] += _rhs; vd[ni] -= _g; }
        else { vrhs[ni] -= _rhs; vd[ni] += _g; }
    }
}

// ion lookup: instance of ion `ion` at the node of instance i of mechanism `mm`
static int ion_inst(Model* m, const char* ion, int nodeidx) {
    auto it = m->mechs.find(ion);
    if (it == m->mechs.end()) return -1;
    return static_cast<Ion*>(it->second.get())->node2inst[nodeidx];
}

// ---------------------------------------------------------------------------
// hh (hh_templated.cu)
// ---------------------------------------------------------------------------
struct HH : TMech {
    std::vector<int> na, k;
    double *gnabar, *gkbar, *gl, *el, *ena, *ek, *m_, *h_, *n_, *ina, *ik, *il, *gna, *gk;
    double *minf, *hinf, *ninf, *mtau, *htau, *ntau;
    double *na_erev, *na_cur, *k_erev, *k_cur;
    HH() { name = "hh"; }
    void alloc() override {
        ensure("gnabar", 0.25); ensure("gkbar", 0.036); ensure("gl", 0.00016666); ensure("el", -60.0);
        ensure("ena", 50); ensure("ek", -77);
        for (auto k2 : {"m", "h", "n", "ina", "ik", "il", "gna", "gk", "minf", "hinf", "ninf", "mtau", "htau", "ntau"})
            ensure(k2, 0.0);
        if (!glob.count("celsius")) glob["celsius"] = m->celsius;
    }
    void bind() override {
        gnabar = C("gnabar").data(); gkbar = C("gkbar").data(); gl = C("gl").data(); el = C("el").data();
        ena = C("ena").data(); ek = C("ek").data(); m_ = C("m").data(); h_ = C("h").data(); n_ = C("n").data();
        ina = C("ina").data(); ik = C("ik").data(); il = C("il").data(); gna = C("gna").data(); gk = C("gk").data();
        minf = C("minf").data(); hinf = C("hinf").data(); ninf = C("ninf").data();
        mtau = C("mtau").data(); htau = C("htau").data(); ntau = C("ntau").data();
        na.resize(n); k.resize(n);
        for (int i = 0; i < n; ++i) { na[i] = ion_inst(m, "na_ion", node[i]); k[i] = ion_inst(m, "k_ion", node[i]); }
        na_erev = m->mechs["na_ion"]->col["erev"].data(); na_cur = m->mechs["na_ion"]->col["cur"].data();
        k_erev = m->mechs["k_ion"]->col["erev"].data(); k_cur = m->mechs["k_ion"]->col["cur"].data();
    }
    static double vtrap(double x, double y) {
        if (std::fabs(x / y) < 1e-6) return y * (1 - x / y / 2);
        else return x / (std::exp(x / y) - 1);
    }
    static void rates(double volt, double& minf, double& mtau, double& hinf, double& htau,
                      double& ninf, double& ntau, double celsius) {
        double q10, alpha, beta, sum;
        q10 = std::pow(3.0, (celsius - 6.3) / 10);
        alpha = 0.1 * vtrap(-(volt + 40), 10);
        beta = 4 * std::exp(-(volt + 65) / 18);
        sum = alpha + beta;
        mtau = 1.0 / (q10 * sum);
        minf = alpha / sum;
        alpha = 0.07 * std::exp(-(volt + 65) / 20);
        beta = 1.0 / (std::exp(-(volt + 35) / 10) + 1);
        sum = alpha + beta;
        htau = 1.0 / (q10 * sum);
        hinf = alpha / sum;
        alpha = 0.01 * vtrap(-(volt + 55), 10);
        beta = 0.125 * std::exp(-(volt + 65) / 80);
        sum = alpha + beta;
        ntau = 1.0 / (q10 * sum);
        ninf = alpha / sum;
    }
    void init(const double* v) override {
        double cel = glob["celsius"];
        for (int i = 0; i < n; ++i) {
            ena[i] = na_erev[na[i]];
            ek[i] = k_erev[k[i]];
            rates(v[node[i]], minf[i], mtau[i], hinf[i], htau[i], ninf[i], ntau[i], cel);
            m_[i] = minf[i];
            h_[i] = hinf[i];
            n_[i] = ninf[i];
        }
    }
    double cur(int i, double volt, double, bool updateIon) override {
        ena[i] = na_erev[na[i]];
        ek[i] = k_erev[k[i]];
        double _m = m_[i], _h = h_[i], _n = n_[i];
        gna[i] = gnabar[i] * _m * _m * _m * _h;
        ina[i] = gna[i] * (volt - ena[i]);
        gk[i] = gkbar[i] * _n * _n * _n * _n;
        ik[i] = gk[i] * (volt - ek[i]);
        il[i] = gl[i] * (volt - el[i]);
        double current = ina[i] + ik[i] + il[i];
        if (updateIon) {
            na_cur[na[i]] += ina[i];
            k_cur[k[i]] += ik[i];
        }
        return current;
    }
    void state(const double* v, double dt, double) override {
        double cel = glob["celsius"];
        for (int i = 0; i < n; ++i) {
            rates(v[node[i]], minf[i], mtau[i], hinf[i], htau[i], ninf[i], ntau[i], cel);
            double _minf = minf[i], _mtau = mtau[i];
            double _hinf = hinf[i], _htau = htau[i];
            double _ninf = ninf[i], _ntau = ntau[i];
            m_[i] = m_[i] + (1.0 - std::exp(dt * (-1.0 / _mtau))) * ((_minf / _mtau) / (1.0 / _mtau) - m_[i]);
            h_[i] = h_[i] + (1.0 - std::exp(dt * (-1.0 / _htau))) * ((_hinf / _htau) / (1.0 / _htau) - h_[i]);
            n_[i] = n_[i] + (1.0 - std::exp(dt * (-1.0 / _ntau))) * ((_ninf / _ntau) / (1.0 / _ntau) - n_[i]);
        }
    }
};

// ---------------------------------------------------------------------------
// pas (pas_templated.cu)
// ---------------------------------------------------------------------------
struct Pas : TMech {
    Pas() { name = "pas"; }
    double *g_pas, *e_pas, *i_;
    void alloc() override { ensure("g_pas", 0.00016666); ensure("e_pas", -60); ensure("i", 0.0); }
    void bind() override { g_pas = C("g_pas").data(); e_pas = C("e_pas").data(); i_ = C("i").data(); }
    double cur(int i, double volt, double, bool) override {
        double current = g_pas[i] * (volt - e_pas[i]);
        i_[i] = current;
        return current;
    }
};

// ---------------------------------------------------------------------------
// IClamp (iclamp_templated.cu): POINT_PROCESS + ELECTRODE_CURRENT
// ---------------------------------------------------------------------------
struct IClamp : TMech {
    IClamp() { name = "IClamp"; point_process = true; electrode = true; }
    double *amp, *delay, *dur, *i_;
    void alloc() override { ensure("amp", 0.0); ensure("delay", 0.0); ensure("dur", 0.0); ensure("i", 0.0); }
    void bind() override { amp = C("amp").data(); delay = C("delay").data(); dur = C("dur").data(); i_ = C("i").data(); }
    void init(const double*) override { for (int i = 0; i < n; ++i) i_[i] = 0.0; }
    double cur(int i, double, double t, bool) override {
        double _current = 0.0;
        double _dur = dur[i], _del = delay[i];
        if (t < _del + _dur && t >= _del) _current = amp[i];
        i_[i] = _current;
        return _current;
    }
};

// ---------------------------------------------------------------------------
// Ca_HVA (CA_HVA.cu)
// ---------------------------------------------------------------------------
struct CaHVA : TMech {
    std::vector<int> ca;
    double *gbar, *eca, *i_mech, *ica, *g, *m_, *h_, *mInf, *mTau, *mAlpha, *mBeta, *hInf, *hTau, *hAlpha, *hBeta;
    double *ca_erev, *ca_cur;
    CaHVA() { name = "Ca_HVA"; }
    void alloc() override {
        ensure("gbar", 0.1); ensure("eca", 140.0);
        for (auto k2 : {"i_mech", "ica", "g", "m", "h", "mInf", "mTau", "mAlpha", "mBeta", "hInf", "hTau", "hAlpha", "hBeta"})
            ensure(k2, 0.0);
    }
    void bind() override {
        gbar = C("gbar").data(); eca = C("eca").data(); i_mech = C("i_mech").data(); ica = C("ica").data();
        g = C("g").data(); m_ = C("m").data(); h_ = C("h").data();
        mInf = C("mInf").data(); mTau = C("mTau").data(); mAlpha = C("mAlpha").data(); mBeta = C("mBeta").data();
        hInf = C("hInf").data(); hTau = C("hTau").data(); hAlpha = C("hAlpha").data(); hBeta = C("hBeta").data();
        ca.resize(n);
        for (int i = 0; i < n; ++i) ca[i] = ion_inst(m, "ca_ion", node[i]);
        ca_erev = m->mechs["ca_ion"]->col["erev"].data(); ca_cur = m->mechs["ca_ion"]->col["cur"].data();
    }
    static double vtrap(double _lx, double _ly) {
        double _lvtrap;
        if (std::fabs(_lx / _ly) < 1e-6) _lvtrap = _ly * (1.0 - _lx / _ly / 2.0);
        else _lvtrap = _lx / (std::exp(_lx / _ly) - 1.0);
        return _lvtrap;
    }
    static void rates(double volt, double& mInf, double& mTau, double& mAlpha, double& mBeta,
                      double& hInf, double& hTau, double& hAlpha, double& hBeta) {
        mAlpha = 0.055 * vtrap(-27.0 - volt, 3.8);
        mBeta = 0.94 * std::exp((-75.0 - volt) / 17.0);
        mInf = mAlpha / (mAlpha + mBeta);
        mTau = 1.0 / (mAlpha + mBeta);
        hAlpha = 0.000457 * std::exp((-13.0 - volt) / 50.0);
        hBeta = 0.0065 / (std::exp((-volt - 15.0) / 28.0) + 1.0);
        hInf = hAlpha / (hAlpha + hBeta);
        hTau = 1.0 / (hAlpha + hBeta);
    }
    void store_rates(int i, double volt, double& mi, double& mt, double& hi, double& ht) {
        double ma, mb, ha, hb;
        rates(volt, mi, mt, ma, mb, hi, ht, ha, hb);
        mInf[i] = mi; mTau[i] = mt; mAlpha[i] = ma; mBeta[i] = mb;
        hInf[i] = hi; hTau[i] = ht; hAlpha[i] = ha; hBeta[i] = hb;
    }
    void init(const double* v) override {
        for (int i = 0; i < n; ++i) {
            eca[i] = ca_erev[ca[i]];
            double mi, mt, hi, ht;
            store_rates(i, v[node[i]], mi, mt, hi, ht);
            m_[i] = mi;
            h_[i] = hi;
        }
    }
    double cur(int i, double volt, double, bool updateIon) override {
        eca[i] = ca_erev[ca[i]];
        double _m = m_[i], _h = h_[i];
        g[i] = gbar[i] * _m * _m * _h;
        ica[i] = g[i] * (volt - eca[i]);
        i_mech[i] = ica[i];
        double current = i_mech[i];
        if (updateIon) ca_cur[ca[i]] += ica[i];
        return current;
    }
    void state(const double* v, double dt, double) override {
        for (int i = 0; i < n; ++i) {
            eca[i] = ca_erev[ca[i]];
            double mi, mt, hi, ht;
            store_rates(i, v[node[i]], mi, mt, hi, ht);
            m_[i] = m_[i] + (1.0 - std::exp(-dt / mt)) * (mi - m_[i]);
            h_[i] = h_[i] + (1.0 - std::exp(-dt / ht)) * (hi - h_[i]);
        }
    }
};

// ---------------------------------------------------------------------------
// hd_la, Ih (hd_la.cu); globals are the NEURON defaults of the Ih mod file
// (the reference reads them from globals.dat, hd_la.cu:65-73)
// ---------------------------------------------------------------------------
struct HdLa : TMech {
    double *ghdbar, *vhalfl, *tau, *l, *i_, *linf, *taul, *ghd;
    HdLa() { name = "hd_la"; }
    void alloc() override {
        ensure("ghdbar", 0.0001); ensure("vhalfl", -81.0); ensure("tau", 1.0);
        for (auto k2 : {"l", "i", "linf", "taul", "ghd", "Dl", "_g"}) ensure(k2, 0.0);
        const std::pair<const char*, double> dflt[] = {
            {"ehd", -30.0}, {"kl", -8.0}, {"vhalft", -75.0}, {"a0t", 0.011}, {"zetat", 2.2},
            {"gmt", 0.4}, {"q10", 4.5}, {"qtl", 1.0}};
        for (auto& p : dflt) if (!glob.count(p.first)) glob[p.first] = p.second;
        if (!glob.count("celsius")) glob["celsius"] = m->celsius;
    }
    double ehd, kl, vhalft, a0t, zetat, gmt, q10, qtl, celsius;
    void bind() override {
        ghdbar = C("ghdbar").data(); vhalfl = C("vhalfl").data(); tau = C("tau").data(); l = C("l").data();
        i_ = C("i").data(); linf = C("linf").data(); taul = C("taul").data(); ghd = C("ghd").data();
        ehd = glob["ehd"]; kl = glob["kl"]; vhalft = glob["vhalft"]; a0t = glob["a0t"]; zetat = glob["zetat"];
        gmt = glob["gmt"]; q10 = glob["q10"]; qtl = glob["qtl"]; celsius = glob["celsius"];
    }
    // alpt / bett / rate (hd_la.cu:80-101)
    double alpt(double v) { return std::exp(0.0378 * zetat * (v - vhalft)); }
    double bett(double v) { return std::exp(0.0378 * zetat * gmt * (v - vhalft)); }
    void rate(int i, double v) {
        double a, qt;
        qt = std::pow(q10, ((celsius - 33.0) / 10.0));
        a = alpt(v);
        linf[i] = 1.0 / (1.0 + std::exp(-(v - vhalfl[i]) / kl));
        taul[i] = tau[i] * bett(v) / (qtl * qt * a0t * (1.0 + a));
    }
    void init(const double* v) override {
        for (int i = 0; i < n; ++i) { rate(i, v[node[i]]); l[i] = linf[i]; }
    }
    double cur(int i, double volt, double, bool) override {
        ghd[i] = ghdbar[i] * l[i];
        i_[i] = ghd[i] * (volt - ehd);
        return i_[i];
    }
    void state(const double* v, double dt, double) override {
        for (int i = 0; i < n; ++i) {
            rate(i, v[node[i]]);
            l[i] = l[i] + (1.0 - std::exp(-dt / taul[i])) * (linf[i] - l[i]);
        }
    }
};

// ---------------------------------------------------------------------------
// CaDynamics_E2 (CaDynamics_E2.cu): no current; state writes cai
// ---------------------------------------------------------------------------
struct CaDyn : Mech {
    std::vector<int> ca;
    double *gamma, *decay, *depth, *minCai, *ica, *cai, *ca_cur, *ca_conci;
    CaDyn() { name = "CaDynamics_E2"; write_state_ion = true; }
    void alloc() override {
        ensure("gamma", 0.05); ensure("decay", 80.0); ensure("depth", 0.1); ensure("minCai", 1e-4);
        ensure("ica", 0.0); ensure("cai", 0.0);
    }
    void bind() override {
        gamma = C("gamma").data(); decay = C("decay").data(); depth = C("depth").data(); minCai = C("minCai").data();
        ica = C("ica").data(); cai = C("cai").data();
        ca.resize(n);
        for (int i = 0; i < n; ++i) ca[i] = ion_inst(m, "ca_ion", node[i]);
        ca_cur = m->mechs["ca_ion"]->col["cur"].data(); ca_conci = m->mechs["ca_ion"]->col["conci"].data();
    }
    void init(const double*) override {
        for (int i = 0; i < n; ++i) {
            ica[i] = ca_cur[ca[i]];
            cai[i] = ca_conci[ca[i]];
            ca_conci[ca[i]] = cai[i];
        }
    }
    void state(const double*, double dt, double) override {
        const double FARADAY = 96485.3321233100184;
        for (int i = 0; i < n; ++i) {
            ica[i] = ca_cur[ca[i]];
            cai[i] = ca_conci[ca[i]];
            double gamma_val = gamma[i], decay_val = decay[i];
            double depth_val = depth[i], minCai_val = minCai[i];
            double ica_val = ica[i], cai_val = cai[i];
            double drive_ica = -(10000.0) * (ica_val * gamma_val) / (2.0 * FARADAY * depth_val);
            double exp_factor = std::exp(dt * (-1.0 / decay_val));
            double steady_term = -(drive_ica - (-minCai_val) / decay_val) / (-1.0 / decay_val);
            cai[i] = cai_val + (1.0 - exp_factor) * (steady_term - cai_val);
            ca_conci[ca[i]] = cai[i];
        }
    }
};

// ---------------------------------------------------------------------------
// HalfGap (HalfGap.cu): POINT_PROCESS + ELECTRODE_CURRENT
// ---------------------------------------------------------------------------
struct HalfGap : TMech {
    double *g, *vgap, *i_;
    HalfGap() { name = "HalfGap"; point_process = true; electrode = true; }
    void alloc() override { ensure("g", 0.0); ensure("vgap", 0.0); ensure("i", 0.0); }
    void bind() override { g = C("g").data(); vgap = C("vgap").data(); i_ = C("i").data(); }
    void init(const double*) override { for (int i = 0; i < n; ++i) i_[i] = 0.0; }
    double cur(int i, double volt, double, bool) override {
        double current = (vgap[i] - volt) * g[i];
        i_[i] = current;
        return current;
    }
};

// ---------------------------------------------------------------------------
// ExpSyn (expsyn.cpp): POINT_PROCESS; its own FD loop with mfact
// ---------------------------------------------------------------------------
struct ExpSyn : Mech {
    double *tau, *e, *g, *i_;
    ExpSyn() { name = "ExpSyn"; point_process = true; }
    void alloc() override { ensure("tau", 0.1); ensure("e", 0.0); ensure("g", 0.0); ensure("i", 0.0); }
    void bind() override { tau = C("tau").data(); e = C("e").data(); g = C("g").data(); i_ = C("i").data(); }
    void init(const double*) override { for (int i = 0; i < n; ++i) g[i] = 0; }
    double cal(double v, int i) {
        double _current = g[i] * (v - e[i]);
        i_[i] = _current;
        return _current;
    }
    void current(const double* vv, double* vd, double* vrhs, double) override {
        for (int i = 0; i < n; ++i) {
            int ni = node[i];
            double nd_area = m->area[ni];
            double mfact = 1.0e2 / nd_area;
            double _v = vv[ni];
            double _g = cal(_v + 0.001, i);
            double _rhs = cal(_v, i);
            _g = (_g - _rhs) / 0.001;
            _g *= mfact;
            _rhs *= mfact;
            vrhs[ni] -= _rhs;
            vd[ni] += _g;
        }
    }
    void state(const double*, double dt, double) override {
        for (int i = 0; i < n; ++i)
            g[i] = g[i] + (1. - std::exp(dt * ((-1.0) / tau[i]))) * (-(0.0) / ((-1.0) / tau[i]) - g[i]);
    }
    void receive(int isyn, double w) { g[isyn] += w; }
};

// ---------------------------------------------------------------------------
// Exp2Syn (exp2syn_temp.cuh)
// ---------------------------------------------------------------------------
struct Exp2Syn : TMech {
    double *tau1, *tau2, *e, *factor, *A, *B, *g, *i_;
    Exp2Syn() { name = "Exp2Syn"; point_process = true; }
    void alloc() override {
        ensure("tau1", 0.1); ensure("tau2", 10.0); ensure("e", 0.0);
        for (auto k2 : {"factor", "A", "B", "g", "i"}) ensure(k2, 0.0);
    }
    void bind() override {
        tau1 = C("tau1").data(); tau2 = C("tau2").data(); e = C("e").data(); factor = C("factor").data();
        A = C("A").data(); B = C("B").data(); g = C("g").data(); i_ = C("i").data();
    }
    void init(const double*) override {
        for (int i = 0; i < n; ++i) {
            double _tau1 = tau1[i], _tau2 = tau2[i];
            if (_tau1 / _tau2 > 0.9999) { _tau1 = 0.9999 * _tau2; tau1[i] = _tau1; }
            if (_tau1 / _tau2 < 1e-9) { _tau1 = _tau2 * 1e-9; tau1[i] = _tau1; }
            A[i] = 0.0;
            B[i] = 0.0;
            double tp = (_tau1 * _tau2) / (_tau2 - _tau1) * std::log(_tau2 / _tau1);
            factor[i] = 1.0 / (-std::exp(-tp / _tau1) + std::exp(-tp / _tau2));
        }
    }
    double cur(int i, double volt, double, bool) override {
        double _g = B[i] - A[i];
        g[i] = _g;
        double _current = _g * (volt - e[i]);
        i_[i] = _current;
        return _current;
    }
    void state(const double*, double dt, double) override {
        for (int i = 0; i < n; ++i) {
            double _tau1 = tau1[i], _tau2 = tau2[i];
            double _A = A[i], _B = B[i];
            A[i] = _A + (1.0 - std::exp(dt * (-1.0 / _tau1))) * (-0.0 / (-1.0 / _tau1) - _A);
            B[i] = _B + (1.0 - std::exp(dt * (-1.0 / _tau2))) * (-0.0 / (-1.0 / _tau2) - _B);
        }
    }
    void receive(int isyn, double w) {
        double _factor = factor[isyn];
        A[isyn] = A[isyn] + w * _factor;
        B[isyn] = B[isyn] + w * _factor;
    }
};

// VecStim has no current/state; it is an artificial cell driven through the queue.
struct VecStim : Mech {
    VecStim() { name = "VecStim"; point_process = true; }
};

// nrnran123 stream (nrnran123.cpp: setids, setseq, ipick, dblpick, negexp) over
// Philox4x32-10: 10 rounds with multipliers 0xD2511F53 / 0xCD9E8D57 on counter
// words 0 / 2 and key increments 0x9E3779B9 / 0xBB67AE85 (Salmon et al., SC11).
struct Ran123 {
    uint32_t c[4] = {0, 0, 0, 0}, r[4] = {0, 0, 0, 0};
    int which = 0;
    static void philox(const uint32_t in[4], uint32_t out[4]) {
        uint32_t x0 = in[0], x1 = in[1], x2 = in[2], x3 = in[3], k0 = 0, k1 = 0;   // global index 0
        for (int rnd = 0; rnd < 10; ++rnd) {
            if (rnd > 0) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
            uint64_t a = (uint64_t)0xD2511F53u * x0, b = (uint64_t)0xCD9E8D57u * x2;
            uint32_t y0 = (uint32_t)(b >> 32) ^ x1 ^ k0, y1 = (uint32_t)b;
            uint32_t y2 = (uint32_t)(a >> 32) ^ x3 ^ k1, y3 = (uint32_t)a;
            x0 = y0; x1 = y1; x2 = y2; x3 = y3;
        }
        out[0] = x0; out[1] = x1; out[2] = x2; out[3] = x3;
    }
    void setids(uint32_t id1, uint32_t id2, uint32_t id3) { c[1] = id3; c[2] = id1; c[3] = id2; }
    void setseq(uint32_t seq, int w) { which = (w > 3 || w < 0) ? 0 : w; c[0] = seq; philox(c, r); }
    uint32_t ipick() {
        uint32_t v = r[which++];
        if (which > 3) {
            which = 0;
            if (++c[0] == 0 && ++c[1] == 0 && ++c[2] == 0) ++c[3];
            philox(c, r);
        }
        return v;
    }
    double dblpick() { static const double SHIFT32 = 1.0 / 4294967297.0; return ((double)ipick() + 1.0) * SHIFT32; }
    double negexp() { return -std::log(dblpick()); }
};

// NetStim: artificial cell driven through the queue (netstim.cpp), each
// instance with its own stream (ids id1 / id2 / id3, id1 < 0: the instance index).
struct NetStim : Mech {
    std::vector<Ran123> rng;
    NetStim() { name = "NetStim"; point_process = true; }
    void alloc() override {
        ensure("interval", 10.0); ensure("number", 10.0); ensure("start", 50.0); ensure("noise", 0.0);
        ensure("id1", -1.0); ensure("id2", 0.0); ensure("id3", 0.0);
        ensure("event", 0.0); ensure("on", 0.0); ensure("ispike", 0.0);
        rng.assign(n, Ran123());
    }
    double invl(int i, double mean) {              // netstim.cpp:140-155
        if (mean <= 0.0) mean = 0.01;
        double noise = C("noise")[i];
        if (noise == 0) return mean;
        return (1.0 - noise) * mean + noise * mean * rng[i].negexp();
    }
    void init_sequence(int i) {                    // netstim.cpp:127-139, this instance only
        if (C("number")[i] > 0.0) { C("event")[i] = 0.0; C("on")[i] = 1.0; C("ispike")[i] = 0.0; }
    }
    void next_invl(int i) {                        // netstim.cpp:156-172, this instance only
        if (C("number")[i] > 0) C("event")[i] = invl(i, C("interval")[i]);
        if (C("ispike")[i] >= C("number")[i]) C("on")[i] = 0.0;
    }
};

// ---------------------------------------------------------------------------
// Im, the muscarinic K current (user-mech/Im.cu:9-130); run by the library through its
// mechanism plugin seam
// ---------------------------------------------------------------------------
struct ImMech : TMech {
    std::vector<int> k;
    double *gImbar, *ik, *gIm, *m_, *ek, *mInf, *mTau, *mAlpha, *mBeta, *k_erev, *k_cur;
    ImMech() { name = "Im"; }
    void alloc() override {
        ensure("gImbar", 0.00001);
        for (auto k2 : {"ik", "gIm", "m", "ek", "mInf", "mTau", "mAlpha", "mBeta"}) ensure(k2, 0.0);
    }
    void bind() override {
        gImbar = C("gImbar").data(); ik = C("ik").data(); gIm = C("gIm").data(); m_ = C("m").data();
        ek = C("ek").data(); mInf = C("mInf").data(); mTau = C("mTau").data(); mAlpha = C("mAlpha").data();
        mBeta = C("mBeta").data();
        k.resize(n);
        for (int i = 0; i < n; ++i) k[i] = ion_inst(m, "k_ion", node[i]);
        k_erev = m->mechs["k_ion"]->col["erev"].data(); k_cur = m->mechs["k_ion"]->col["cur"].data();
    }
    void rates(int i, double v) {                       // Im.cu:63-70
        double qt = std::pow(2.3, ((34.0 - 21.0) / 10.0));
        mAlpha[i] = 3.3e-3 * std::exp(2.5 * 0.04 * (v - (-35.0)));
        mBeta[i] = 3.3e-3 * std::exp(-2.5 * 0.04 * (v - (-35.0)));
        mInf[i] = mAlpha[i] / (mAlpha[i] + mBeta[i]);
        mTau[i] = (1.0 / (mAlpha[i] + mBeta[i])) / qt;
    }
    void init(const double* v) override {
        for (int i = 0; i < n; ++i) {
            ek[i] = k_erev[k[i]];
            m_[i] = 0.0;
            rates(i, v[node[i]]);
            m_[i] = mInf[i];
        }
    }
    double cur(int i, double volt, double, bool updateIon) override {
        ek[i] = k_erev[k[i]];
        gIm[i] = gImbar[i] * m_[i];
        ik[i] = gIm[i] * (volt - ek[i]);
        if (updateIon) k_cur[k[i]] += ik[i];
        return ik[i];
    }
    void state(const double* v, double dt, double) override {
        for (int i = 0; i < n; ++i) {
            ek[i] = k_erev[k[i]];
            rates(i, v[node[i]]);
            m_[i] = m_[i] + (1.0 - std::exp(dt * ((-1.0) / mTau[i]))) *
                                (-(mInf[i] / mTau[i]) / ((-1.0) / mTau[i]) - m_[i]);
        }
    }
};

// ---------------------------------------------------------------------------
// syn_record: AMPA + NMDA (excitatory, w > 0) or GABA (w <= 0) double-exponential
// synapse, a postsyn point process (user_postsyn_mech/syn_record.cuh:8-203); run by the
// library through its mechanism plugin seam
// ---------------------------------------------------------------------------
struct SynRecord : TMech {
    SynRecord() { name = "syn_record"; point_process = true; }
    void alloc() override {
        for (auto c : {"AMPA_tau1", "AMPA_tau2", "NMDA_tau1", "NMDA_tau2", "GABA_tau1", "GABA_tau2", "AMPA_e",
                       "NMDA_e", "GABA_e", "NMDA_C", "NMDA_rho"})
            ensure(c, 0.0);
        ensure("w", 1.0); ensure("r_na", 2.0); ensure("dv", 1e-3); ensure("Use_e", 1.0); ensure("Use_i", 1.0);
        ensure("Dep", 0.0); ensure("Fac", 0.0); ensure("u0", 0.0);
        for (auto c : {"i", "AMPA_g", "NMDA_g", "GABA_g", "v_prev", "didv", "pure_i", "g_mul", "dgdv", "dgdg", "Use",
                       "AMPA_A", "AMPA_B", "NMDA_A", "NMDA_B", "GABA_A", "GABA_B", "AMPA_factor", "NMDA_factor",
                       "GABA_factor"})
            ensure(c, 0.0);
    }
    double& X(const char* c, int i) { return C(c)[i]; }
    double sigma(double v, int i) { return 1.0 / (1.0 + X("NMDA_C", i) * std::exp(-X("NMDA_rho", i) * v)); }
    void init(const double*) override {                 // syn_record.cuh:104-125
        for (int i = 0; i < n; ++i) {
            auto pair = [&](const char* tau1, const char* tau2, const char* A, const char* B, const char* factor) {
                double t1 = X(tau1, i), t2 = X(tau2, i);
                if (t1 / t2 > 0.9999) { t1 = 0.9999 * t2; X(tau1, i) = t1; }
                if (t1 / t2 < 1e-9) { t1 = 1e-9 * t2; X(tau1, i) = t1; }
                X(A, i) = 0.0; X(B, i) = 0.0;
                double tp = (t1 * t2) / (t2 - t1) * std::log(t2 / t1);
                X(factor, i) = 1.0 / (-std::exp(-tp / t1) + std::exp(-tp / t2));
            };
            pair("AMPA_tau1", "AMPA_tau2", "AMPA_A", "AMPA_B", "AMPA_factor");
            pair("NMDA_tau1", "NMDA_tau2", "NMDA_A", "NMDA_B", "NMDA_factor");
            pair("GABA_tau1", "GABA_tau2", "GABA_A", "GABA_B", "GABA_factor");
            X("Use", i) = X("w", i) > 0.0 ? X("Use_e", i) : X("Use_i", i);
        }
    }
    double cur(int i, double v, double, bool) override {   // syn_record.cuh:128-148
        X("v_prev", i) = v;
        double current = 0.0;
        if (X("w", i) > 0.0) {
            X("AMPA_g", i) = X("AMPA_B", i) - X("AMPA_A", i);
            X("NMDA_g", i) = X("NMDA_B", i) - X("NMDA_A", i);
            double s = sigma(v, i);
            current = std::fabs(X("w", i)) *
                      (X("AMPA_g", i) * (v - X("AMPA_e", i)) + X("NMDA_g", i) * s * (v - X("NMDA_e", i)));
        } else {
            X("GABA_g", i) = X("GABA_B", i) - X("GABA_A", i);
            current = std::fabs(X("w", i)) * X("GABA_g", i) * (v - X("GABA_e", i));
        }
        X("i", i) = current;
        return current;
    }
    void state(const double* vv, double dt, double) override {   // syn_record.cuh:151-178
        for (int i = 0; i < n; ++i) {
            auto decay = [&](const char* x, const char* tau) { X(x, i) *= std::exp(-dt / X(tau, i)); };
            decay("AMPA_A", "AMPA_tau1"); decay("AMPA_B", "AMPA_tau2");
            decay("NMDA_A", "NMDA_tau1"); decay("NMDA_B", "NMDA_tau2");
            decay("GABA_A", "GABA_tau1"); decay("GABA_B", "GABA_tau2");
            const double v = vv[node[i]];
            const double w = X("w", i);
            if (w > 0.0) {
                X("didv", i) = std::fabs(w) * (X("AMPA_g", i) + X("NMDA_g", i) * sigma(X("v_prev", i), i));
                X("pure_i", i) = X("AMPA_g", i) * (v - X("AMPA_e", i)) +
                                 X("NMDA_g", i) * sigma(X("v_prev", i), i) * (v - X("NMDA_e", i));
                X("g_mul", i) = std::fabs(w) * X("NMDA_g", i) * (v - X("NMDA_e", i));
                X("dgdv", i) = (sigma(X("v_prev", i) + X("dv", i), i) - sigma(X("v_prev", i), i)) / X("dv", i);
                X("dgdg", i) = 0.0;
            } else {
                X("didv", i) = std::fabs(w) * X("GABA_g", i);
                X("pure_i", i) = -X("GABA_g", i) * (v - X("GABA_e", i));
                X("g_mul", i) = X("dgdv", i) = X("dgdg", i) = 0.0;
            }
        }
    }
    void receive(int isyn, double w_event) {            // syn_record.cuh:181-199
        if (X("w", isyn) > 0.0) {
            double ra = X("r_na", isyn);
            double a_fac = w_event * X("AMPA_factor", isyn) / (1.0 + ra);
            double n_fac = w_event * X("NMDA_factor", isyn) * ra / (1.0 + ra);
            X("AMPA_A", isyn) += a_fac; X("AMPA_B", isyn) += a_fac;
            X("NMDA_A", isyn) += n_fac; X("NMDA_B", isyn) += n_fac;
        } else {
            double g_fac = w_event * X("GABA_factor", isyn);
            X("GABA_A", isyn) += g_fac; X("GABA_B", isyn) += g_fac;
        }
    }
};

// CoreNEURON type order used by the oracle (NEURON built-ins, then user mechanisms).
const char* kMechOrder[] = {"pas", "na_ion", "k_ion", "hh", "IClamp", "ExpSyn", "Exp2Syn", "VecStim", "NetStim",
                            "ca_ion", "CaDynamics_E2", "Ca_HVA", "HalfGap", "hd_la", "Im", "syn_record"};

std::unique_ptr<Mech> make_mech(const std::string& nm) {
    if (nm == "na_ion") return std::make_unique<Ion>("na_ion", 1.0, 10.0, 140.0);
    if (nm == "k_ion") return std::make_unique<Ion>("k_ion", 1.0, 140.0, 4.0);
    if (nm == "ca_ion") return std::make_unique<Ion>("ca_ion", 2.0, 5.e-5, 2.0);
    if (nm == "hh") return std::make_unique<HH>();
    if (nm == "pas") return std::make_unique<Pas>();
    if (nm == "IClamp") return std::make_unique<IClamp>();
    if (nm == "Ca_HVA") return std::make_unique<CaHVA>();
    if (nm == "hd_la") return std::make_unique<HdLa>();
    if (nm == "CaDynamics_E2") return std::make_unique<CaDyn>();
    if (nm == "HalfGap") return std::make_unique<HalfGap>();
    if (nm == "ExpSyn") return std::make_unique<ExpSyn>();
    if (nm == "Exp2Syn") return std::make_unique<Exp2Syn>();
    if (nm == "VecStim") return std::make_unique<VecStim>();
    if (nm == "NetStim") return std::make_unique<NetStim>();
    if (nm == "Im") return std::make_unique<ImMech>();
    if (nm == "syn_record") return std::make_unique<SynRecord>();
    return nullptr;
}

// ---------------------------------------------------------------------------
// Step pieces
// ---------------------------------------------------------------------------
void Model::setup_tree_matrix() {             // simulate.cpp:455-556
    std::fill(rhs.begin(), rhs.end(), 0.0);
    std::fill(d.begin(), d.end(), 0.0);
    for (auto* mm : current_list) mm->current(v.data(), d.data(), rhs.data(), t);
    double cfac = 0.001 * cj;                 // capac.cpp:68-80
    for (int i = 0; i < len; ++i) d[i] += cfac * cm[i];
    for (int i = ncell; i < len; i++) {
        double dv = v[parent[i]] - v[i];
        rhs[i] -= b[i] * dv;
        rhs[parent[i]] += a[i] * dv;
    }
    for (int i = ncell; i < len; i++) {
        d[i] -= b[i];
        d[parent[i]] -= a[i];
    }
}

void Model::solve_serial() {                  // simulate.cpp:558-581
    double p;
    for (int i = len - 1; i >= ncell; i--) {
        p = a[i] / d[i];
        d[parent[i]] -= p * b[i];
        rhs[parent[i]] -= p * rhs[i];
    }
    for (int i = 0; i < ncell; i++) rhs[i] /= d[i];
    for (int i = ncell; i < len; i++) {
        rhs[i] -= b[i] * rhs[parent[i]];
        rhs[i] /= d[i];
    }
}

// The reference also stores the capacitive current cfac * cm * x here (capac.cpp:54-66);
// no variable table of the reference or of the library exposes it, so it is left out.
void Model::update() {                        // simulate.cpp:759-770
    for (int i = 0; i < len; i++) v[i] += rhs[i];
}

void Model::nonvint() {                       // simulate.cpp:779-852
    for (auto* mm : state_ion_first) mm->state(v.data(), dt, t);
    for (auto* mm : state_rest) mm->state(v.data(), dt, t);
    log_data();
}

void Model::last_part() {                     // simulate.cpp:772-777
    t += 0.5 * dt;
    for (auto& vp : vecplay) vp.continuous(t);
    nonvint();
}

void Model::network_spike_send() {            // presyn.cpp:133-177
    int npre = (int)pre_node.size();
    for (int ipre = 0; ipre < npre; ipre++) {
        double pre_v = v[pre_node[ipre]];
        if (pre_v > pre_thr[ipre] && !pre_flag[ipre]) {
            Spike spk; spk.gid = pre_gid[ipre]; spk.deliver_time = t; spk.flag = NORMAL_EVENT;
            spk_vec[ipre] = spk;
            pre_flag[ipre] = 1;
            spk_flags[ipre] = NORMAL_EVENT;
            rec_spikes.emplace_back(t, pre_gid[ipre]);
            spk_output[ipre].push_back(t);
        } else if (pre_v <= pre_thr[ipre]) {
            pre_flag[ipre] = 0;
        }
    }
}

void Model::net_send_vecstim(uint32_t idx, double tt, int flag) {   // articell.cpp:18-35
    auto& ps = postsyns[vs_postsyn];
    if (flag == SELF_EVENT) {
        Spike spk; spk.syn_type = ps.type_id; spk.syn_id = (int)idx; spk.deliver_time = tt; spk.flag = flag;
        ps.buffer.push(spk);
    } else {
        Spike spk; spk.deliver_time = tt; spk.flag = flag;
        uint32_t slot = (uint32_t)pre_node.size() + idx;
        spk_vec[slot] = spk;
        spk_flags[slot] = flag;
    }
}

void Model::vecstim_element(int inode) {      // vecevent.cpp:140-170
    int i = vs_index[inode];
    if (i >= 0) {
        auto& vv = vs_times[inode];
        if (!vv.empty()) {
            int len2 = (int)vv.size();
            if (i < len2) { vs_etime[inode] = vv[i]; vs_index[inode] += 1; }
            else vs_index[inode] = -1;
        } else {
            vs_index[inode] = -1;
        }
    }
}

void Model::net_send_netstim(uint32_t idx, double tt, int flag) {   // articell.cpp:18-35
    auto& ps = postsyns[ns_postsyn];
    if (flag != NORMAL_EVENT) {
        Spike spk; spk.syn_type = ps.type_id; spk.syn_id = (int)idx; spk.deliver_time = tt; spk.flag = flag;
        ps.buffer.push(spk);
    } else {
        ns_spikes.emplace_back(tt, (int)idx);
        Spike spk; spk.deliver_time = tt; spk.flag = flag;
        int nvs = vs_postsyn >= 0 ? postsyns[vs_postsyn].mech->n : 0;
        uint32_t slot = (uint32_t)(pre_node.size() + nvs) + idx;
        spk_vec[slot] = spk;
        spk_flags[slot] = flag;
    }
}

void Model::netstim_init() {                  // netstim.cpp:211-246 (initialize_cpu)
    auto* ns = static_cast<NetStim*>(postsyns[ns_postsyn].mech);
    ns_spikes.clear();
    for (int i = 0; i < ns->n; i++) {
        double id1 = ns->C("id1")[i];
        ns->rng[i].setids(id1 < 0 ? (uint32_t)i : (uint32_t)id1, (uint32_t)ns->C("id2")[i], (uint32_t)ns->C("id3")[i]);
        ns->rng[i].setseq(0, 0);
        double& on = ns->C("on")[i];
        double& noise = ns->C("noise")[i];
        on = 0.0;
        ns->C("ispike")[i] = 0.0;
        if (noise < 0.0) noise = 0.0;
        if (noise > 1.0) noise = 1.0;
        double start = ns->C("start")[i], interval = ns->C("interval")[i];
        if (start >= 0.0 && ns->C("number")[i] > 0) {
            on = 1.0;
            double& event = ns->C("event")[i];
            event = start + ns->invl(i, interval) - interval * (1.0 - noise);
            if (event < 0.0) event = 0.0;
            net_send_netstim(i, event, NETSTIM_INIT_EVENT);
        }
    }
}

// The reference counts a send only where the next self event is scheduled, so the last
// spike of a sequence can wait in its slot until something else keeps the delivery loop
// going; here every processed event keeps the loop going, and that spike is gathered in
// the same step like any other.
bool Model::netstim_receive(int isyn, int flag) {   // netstim.cpp:247-290 (net_receive_cpu)
    auto* ns = static_cast<NetStim*>(postsyns[ns_postsyn].mech);
    double& on = ns->C("on")[isyn];
    bool sent = false;
    if (flag == NORMAL_EVENT) {                      // netstim.cpp:262-274
        const int w = static_cast<int>(postsyns[ns_postsyn].weight[isyn]);   // truncated, as there
        if (w > 0 && on == 0.0) {
            ns->init_sequence(isyn);
            ns->next_invl(isyn);
            double& event = ns->C("event")[isyn];
            event -= ns->C("interval")[isyn] * (1. - ns->C("noise")[isyn]);
            net_send_netstim(isyn, t + event, SELF_EVENT);
            sent = true;
        } else if (w < 0) {
            on = 0.0;
        }
    }
    if (flag == NETSTIM_INIT_EVENT && on == 1.0) {
        ns->init_sequence(isyn);
        net_send_netstim(isyn, t + 0.0, SELF_EVENT);
        sent = true;
    }
    if (flag == SELF_EVENT && on == 1.0) {
        ns->C("ispike")[isyn] += 1.0;
        net_send_netstim(isyn, t, NORMAL_EVENT);
        ns->next_invl(isyn);
        if (on == 1.0) net_send_netstim(isyn, t + ns->C("event")[isyn], SELF_EVENT);
        sent = true;
    }
    return sent;
}

void Model::network_spike_receive() {         // simulate.cpp:916-939
    bool hasSent = false;
    do {
        hasSent = false;
        for (auto& ps : postsyns) {           // get_spike_from_vec_common, postsyn.cpp:94-113
            int nn = ps.mech->n;
            for (int inode = 0; inode < nn; inode++) {
                uint32_t spk_idx = ps.spk_vec_idx[inode];
                if (spk_idx == kNoSource) continue;      // no netcon into this instance
                if (spk_flags[spk_idx] == NORMAL_EVENT) {
                    Spike spk = spk_vec[spk_idx];
                    spk.syn_id = inode;
                    spk.flag = spk_flags[spk_idx];
                    spk.deliver_time += ps.delay[inode];
                    ps.buffer.push(spk);
                }
            }
        }
        for (auto& f : spk_flags) if (f == NORMAL_EVENT) f = INVALID;   // clearValidSpkFlags
        for (size_t ip = 0; ip < postsyns.size(); ++ip) {
            auto& ps = postsyns[ip];
            // post_spike_receive_cpu(t + dt/2), postsyn.cpp:43-61
            double tt = t + dt / 2;
            ps.receive_count = 0;
            while (!ps.buffer.empty()) {
                Spike spk = ps.buffer.top();
                if (spk.deliver_time > tt) break;
                ps.buffer.pop();
                // the reference's receive list holds one entry per instance (postsyn.cpp:79-81)
                // and is written past its end when an instance receives several events in one
                // pass (a VecStim whose elements fall due together); the list grows here
                if (ps.receive_count == (int)ps.receive_idx.size()) {
                    ps.receive_idx.resize(2 * ps.receive_idx.size());
                    ps.receive_flag.resize(2 * ps.receive_flag.size(), -1);
                }
                ps.receive_idx[ps.receive_count] = (uint32_t)spk.syn_id;
                ps.receive_flag[ps.receive_count] = spk.flag;
                ps.receive_count++;
            }
            // net_receive_cpu(t)
            if (ps.artificial && ps.mech->name == "NetStim") {
                int send_count = 0;
                for (int i = 0; i < ps.receive_count; i++)
                    if (netstim_receive((int)ps.receive_idx[i], ps.receive_flag[i])) send_count++;
                hasSent |= send_count > 0;
            } else if (ps.artificial) {          // vecevent.cpp:172-199
                int send_count = 0;
                for (int i = 0; i < ps.receive_count; i++) {
                    int isyn = (int)ps.receive_idx[i];
                    if (ps.receive_flag[i] == SELF_EVENT) {
                        net_send_vecstim(isyn, t, NORMAL_EVENT);
                        vecstim_element(isyn);
                        if (vs_index[isyn] > 0) net_send_vecstim(isyn, vs_etime[isyn], SELF_EVENT);
                        send_count++;
                    }
                }
                hasSent |= send_count > 0;
            } else if (ps.mech->name == "ExpSyn") {
                auto* es = static_cast<ExpSyn*>(ps.mech);
                for (int i = 0; i < ps.receive_count; i++) {
                    int isyn = (int)ps.receive_idx[i];
                    es->receive(isyn, ps.weight[isyn]);
                }
            } else if (ps.mech->name == "Exp2Syn") {
                auto* es = static_cast<Exp2Syn*>(ps.mech);
                for (int i = 0; i < ps.receive_count; i++) {
                    int isyn = (int)ps.receive_idx[i];
                    es->receive(isyn, ps.weight[isyn]);
                }
            } else if (ps.mech->name == "syn_record") {
                auto* sr = static_cast<SynRecord*>(ps.mech);
                for (int i = 0; i < ps.receive_count; i++) {
                    int isyn = (int)ps.receive_idx[i];
                    sr->receive(isyn, ps.weight[isyn]);
                }
            }
        }
    } while (hasSent);
}

void Model::spike_deliver() {
    network_spike_send();
    network_spike_receive();
}

void Model::finitialize(double v_init) {      // simulate.cpp:106-141, 271-339
    t = 0;
    for (auto& vp : vecplay) { vp.reset(); vp.play(t); vp.continuous(t); }
    for (auto& ps : postsyns) while (!ps.buffer.empty()) ps.buffer.pop();
    cj = 1.0 / dt;
    for (int j = 0; j < len; j++) v[j] = v_init;
    gap_transfer();
    for (auto* mm : current_list) {
        if (mm->name == "NetStim") {
            netstim_init();
        } else if (mm->name == "VecStim") {           // vecevent.cpp:94-109
            for (int inode = 0; inode < mm->n; inode++) {
                vs_index[inode] = 0;
                vecstim_element(inode);
                if (vs_index[inode] > 0) net_send_vecstim(inode, vs_etime[inode], SELF_EVENT);
            }
        } else {
            mm->init(v.data());
        }
    }
    for (auto& r : rec_data) r.clear();
    log_data();
    // clearAllSpikes_cpu
    for (auto& s : spk_vec) s = Spike();
    for (auto& f : spk_flags) f = INVALID;
    spike_deliver();
    setup_tree_matrix();
}

void Model::fadvance() {                      // simulate.cpp:410-442
    spike_deliver();
    t += 0.5 * dt;
    for (auto& vp : vecplay) { vp.play(t); vp.continuous(t); }
    setup_tree_matrix();
    solve_serial();
    update();
    gap_transfer();
    last_part();
}

double* Model::var_ptr(const std::string& mech, const std::string& var, int idx) {
    if (mech == "global" || mech == "node") {
        std::vector<double>* arr = nullptr;
        if (var == "v") arr = &v; else if (var == "d") arr = &d; else if (var == "rhs") arr = &rhs;
        else if (var == "a") arr = &a; else if (var == "b") arr = &b; else if (var == "area") arr = &area;
        if (!arr || idx < 0 || idx >= len) return nullptr;
        return arr->data() + idx;
    }
    if (mech == "capacitance") {
        if (idx < 0 || idx >= len) return nullptr;
        if (var == "cm") return cm.data() + idx;
        return nullptr;
    }
    auto it = mechs.find(mech);
    if (it == mechs.end()) return nullptr;
    Mech* mm = it->second.get();
    if (mm->is_ion) {
        // ion variables are addressed by node index (eion.cuh:270-300)
        if (idx < 0 || idx >= len) return nullptr;
        int inst = static_cast<Ion*>(mm)->node2inst[idx];
        if (inst < 0) return nullptr;
        auto c = mm->col.find(var);
        if (c == mm->col.end()) return nullptr;
        return c->second.data() + inst;
    }
    auto g = mm->glob.find(var);
    if (g != mm->glob.end()) return &g->second;
    auto c = mm->col.find(var);
    if (c == mm->col.end() || idx < 0 || idx >= mm->n) return nullptr;
    return c->second.data() + idx;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI used by the tests and the CPU-baseline leg of the benchmark.
// ---------------------------------------------------------------------------
extern "C" {

void* hxo_create(double dt, double celsius) {
    auto* m = new Model();
    m->dt = dt;
    m->celsius = celsius;
    return m;
}

void hxo_destroy(void* h) { delete static_cast<Model*>(h); }

int hxo_set_nodes(void* h, int ncell, int nnode, const int* parent, const double* a, const double* b,
                  const double* area, const double* cm) {
    auto* m = static_cast<Model*>(h);
    if (ncell <= 0 || nnode < ncell) return -1;
    m->ncell = ncell; m->len = nnode;
    m->parent.assign(parent, parent + nnode);
    for (int i = ncell; i < nnode; ++i)
        if (parent[i] < 0 || parent[i] >= i) return -1;
    m->a.assign(a, a + nnode); m->b.assign(b, b + nnode); m->area.assign(area, area + nnode);
    m->cm.assign(cm, cm + nnode);
    m->v.assign(nnode, 0.0); m->d.assign(nnode, 0.0); m->rhs.assign(nnode, 0.0);
    return 0;
}

int hxo_insert(void* h, const char* mech, int n, const int* nodes) {
    auto* m = static_cast<Model*>(h);
    auto mm = make_mech(mech);
    if (!mm || n < 0) return -1;
    if (m->mechs.count(mech)) return -1;
    mm->m = m;
    mm->n = n;
    mm->node.assign(nodes, nodes + n);
    for (int i = 0; i < n; ++i) if (nodes[i] < 0 || nodes[i] >= m->len) return -1;
    mm->alloc();
    if (mm->is_ion) {
        auto* ion = static_cast<Ion*>(mm.get());
        ion->node2inst.assign(m->len, -1);
        for (int i = 0; i < n; ++i) ion->node2inst[nodes[i]] = i;
    }
    m->mechs[mech] = std::move(mm);
    return 0;
}

int hxo_set_param(void* h, const char* mech, const char* var, int n, const double* vals) {
    auto* m = static_cast<Model*>(h);
    if (std::string(mech) == "capacitance" && std::string(var) == "cm") {
        if (n != m->len) return -1;
        m->cm.assign(vals, vals + n);
        return 0;
    }
    auto it = m->mechs.find(mech);
    if (it == m->mechs.end()) return -1;
    auto* mm = it->second.get();
    auto c = mm->col.find(var);
    if (c == mm->col.end() || n != mm->n) return -1;
    c->second.assign(vals, vals + n);
    return 0;
}

int hxo_set_global(void* h, const char* mech, const char* var, double val) {
    auto* m = static_cast<Model*>(h);
    auto it = m->mechs.find(mech);
    if (it == m->mechs.end()) return -1;
    it->second->glob[var] = val;
    return 0;
}

int hxo_set_iontype(void* h, const char* ion, int n, const int* iontype) {
    auto* m = static_cast<Model*>(h);
    auto it = m->mechs.find(ion);
    if (it == m->mechs.end() || !it->second->is_ion || n != it->second->n) return -1;
    static_cast<Ion*>(it->second.get())->iontype.assign(iontype, iontype + n);
    return 0;
}

int hxo_add_presyn(void* h, int gid, int node, double thr) {
    auto* m = static_cast<Model*>(h);
    if (node < 0 || node >= m->len) return -1;
    m->pre_node.push_back(node); m->pre_gid.push_back(gid); m->pre_thr.push_back(thr);
    return (int)m->pre_node.size() - 1;
}

int hxo_set_vecstim(void* h, int inst, int n, const double* times) {
    auto* m = static_cast<Model*>(h);
    auto it = m->mechs.find("VecStim");
    if (it == m->mechs.end() || inst < 0 || inst >= it->second->n) return -1;
    if ((int)m->vs_times.size() != it->second->n) m->vs_times.assign(it->second->n, {});
    m->vs_times[inst].assign(times, times + n);
    return 0;
}

// VecEvent::play -> update_sequence (vecevent.cpp:280-309): a call with no element
// changes nothing; otherwise the instance's vector is replaced, and element() reads
// it from the instance's current index on (from the first after finitialize).
int hxo_vecstim_play(void* h, int inst, int n, const double* times) {
    auto* m = static_cast<Model*>(h);
    auto it = m->mechs.find("VecStim");
    if (it == m->mechs.end() || inst < 0 || inst >= it->second->n) return -1;
    if (n <= 0) return 0;
    return hxo_set_vecstim(h, inst, n, times);
}

static int finalize_model(Model* m) {
    // mechanism lists in CoreNEURON type order
    m->current_list.clear(); m->state_ion_first.clear(); m->state_rest.clear(); m->postsyns.clear();
    int type_id = 0;
    for (auto* nm : kMechOrder) {
        ++type_id;
        auto it = m->mechs.find(nm);
        if (it == m->mechs.end()) continue;
        Mech* mm = it->second.get();
        m->current_list.push_back(mm);
        if (mm->write_state_ion) m->state_ion_first.push_back(mm);
        if (!mm->is_ion && !mm->write_state_ion) m->state_rest.push_back(mm);
        std::string s = nm;
        if (s == "ExpSyn" || s == "Exp2Syn" || s == "VecStim" || s == "NetStim" || s == "syn_record") {
            Model::PostSynState ps;
            ps.mech = mm;
            ps.type_id = type_id;
            ps.spk_vec_idx.assign(mm->n, Model::kNoSource);
            ps.delay.assign(mm->n, 0.0);
            ps.weight.assign(mm->n, 0.0);
            ps.receive_idx.assign(mm->n + 1, 0);
            ps.receive_flag.assign(mm->n + 1, -1);
            ps.artificial = (s == "VecStim" || s == "NetStim");
            if (s == "VecStim") m->vs_postsyn = (int)m->postsyns.size();
            if (s == "NetStim") m->ns_postsyn = (int)m->postsyns.size();
            m->postsyns.push_back(std::move(ps));
        }
    }
    for (auto& kv : m->mechs) if (kv.second->is_ion) {
        auto* ion = static_cast<Ion*>(kv.second.get());
        if ((int)ion->iontype.size() != ion->n) ion->iontype.assign(ion->n, 0);
    }
    // every instance of an ion-using mechanism needs the ion at its node
    const std::pair<const char*, const char*> uses[] = {
        {"hh", "na_ion"}, {"hh", "k_ion"}, {"Ca_HVA", "ca_ion"}, {"CaDynamics_E2", "ca_ion"}};
    for (auto& u : uses) {
        auto it = m->mechs.find(u.first);
        if (it == m->mechs.end()) continue;
        for (int nd : it->second->node)
            if (ion_inst(m, u.second, nd) < 0) {
                std::fprintf(stderr, "oracle: %s instance at node %d has no %s\n", u.first, nd, u.second);
                return -1;
            }
    }
    for (auto* nm : kMechOrder) {
        auto it = m->mechs.find(nm);
        if (it != m->mechs.end()) it->second->bind();
    }
    int npre = (int)m->pre_node.size();
    int nvs = m->mechs.count("VecStim") ? m->mechs["VecStim"]->n : 0;
    int nns = m->mechs.count("NetStim") ? m->mechs["NetStim"]->n : 0;
    m->spk_vec.assign(npre + nvs + nns, Model::Spike());
    m->spk_flags.assign(npre + nvs + nns, Model::INVALID);
    m->pre_flag.assign(npre, 0);
    m->spk_output.assign(npre, {});
    if ((int)m->vs_times.size() != nvs) m->vs_times.resize(nvs);
    m->vs_index.assign(nvs, 0);
    m->vs_etime.assign(nvs, 0.0);
    m->finalized = true;
    return 0;
}

// Netcon into a synapse instance.  src_kind 0: real presyn index, 1: VecStim instance,
// 2: NetStim instance.
// The reference keeps one source per synapse instance (coredat_to_innerdat.cpp:356-364).
int hxo_add_netcon(void* h, int src_kind, int src, const char* target, int inst, double weight, double delay) {
    auto* m = static_cast<Model*>(h);
    if (!m->finalized && finalize_model(m) != 0) return -1;
    for (auto& ps : m->postsyns) {
        if (ps.mech->name != target) continue;
        if (inst < 0 || inst >= ps.mech->n) return -1;
        int npre = (int)m->pre_node.size();
        int nvs = m->mechs.count("VecStim") ? m->mechs["VecStim"]->n : 0;
        uint32_t slot = src_kind == 0 ? (uint32_t)src
                      : src_kind == 1 ? (uint32_t)(npre + src) : (uint32_t)(npre + nvs + src);
        if (slot >= m->spk_vec.size()) return -1;
        ps.spk_vec_idx[inst] = slot;
        ps.weight[inst] = weight;
        ps.delay[inst] = delay;
        return 0;
    }
    return -1;
}

int hxo_add_vecplay(void* h, const char* mech, const char* var, int idx, int n, const double* tv, const double* yv) {
    auto* m = static_cast<Model*>(h);
    double* p = m->var_ptr(mech, var, idx);
    if (!p || n <= 0) return -1;
    Model::VecPlayItem it;
    it.target = p; it.tvec.assign(tv, tv + n); it.yvec.assign(yv, yv + n); it.len = n;
    it.last_index = 0; it.next_idx = 0; it.done = false; it.next_time = tv[0];
    m->vecplay.push_back(std::move(it));
    return 0;
}

int hxo_add_gap(void* h, int src_node, int halfgap_inst) {
    auto* m = static_cast<Model*>(h);
    double* src = m->var_ptr("global", "v", src_node);
    double* dst = m->var_ptr("HalfGap", "vgap", halfgap_inst);
    if (!src || !dst) return -1;
    m->gaps.emplace_back(src, dst);
    return 0;
}

int hxo_add_monitor(void* h, const char* mech, const char* var, int idx) {
    auto* m = static_cast<Model*>(h);
    double* p = m->var_ptr(mech, var, idx);
    if (!p) return -1;
    m->rec_ptr.push_back(p);
    m->rec_data.emplace_back();
    return (int)m->rec_ptr.size() - 1;
}

int hxo_finalize(void* h) {
    auto* m = static_cast<Model*>(h);
    if (!m->finalized) return finalize_model(m);
    return 0;
}

int hxo_finitialize(void* h, double v_init) {
    auto* m = static_cast<Model*>(h);
    if (!m->finalized && finalize_model(m) != 0) return -1;
    for (auto* mm : m->current_list) mm->bind();   // picks up globals changed after finalize
    m->finitialize(v_init);
    return 0;
}

int hxo_fadvance(void* h) { static_cast<Model*>(h)->fadvance(); return 0; }

int hxo_run(void* h, double tstop) {          // simulate.cpp:343-371
    auto* m = static_cast<Model*>(h);
    int nstep = tstop / m->dt;
    m->t = 0.0;
    for (int iter = 0; iter < nstep; iter++) m->fadvance();
    return 0;
}

int hxo_continue_run(void* h, double runtime) {   // simulate.cpp:373-399
    auto* m = static_cast<Model*>(h);
    int nstep = runtime / m->dt;
    for (int iter = 0; iter < nstep; iter++) m->fadvance();
    return 0;
}

int hxo_nsteps(void* h, int nstep) {
    auto* m = static_cast<Model*>(h);
    for (int iter = 0; iter < nstep; iter++) m->fadvance();
    return 0;
}

double hxo_get_t(void* h) { return static_cast<Model*>(h)->t; }

int hxo_monitor_len(void* h, int handle) {
    auto* m = static_cast<Model*>(h);
    if (handle < 0 || handle >= (int)m->rec_data.size()) return -1;
    return (int)m->rec_data[handle].size();
}

int hxo_get_monitor(void* h, int handle, double* out, int cap) {
    auto* m = static_cast<Model*>(h);
    if (handle < 0 || handle >= (int)m->rec_data.size()) return -1;
    auto& r = m->rec_data[handle];
    int n = std::min<int>(cap, (int)r.size());
    std::memcpy(out, r.data(), sizeof(double) * n);
    return n;
}

int hxo_n_spikes(void* h) { return (int)static_cast<Model*>(h)->rec_spikes.size(); }

int hxo_get_spikes(void* h, double* t, int* gid, int cap) {
    auto* m = static_cast<Model*>(h);
    int n = std::min<int>(cap, (int)m->rec_spikes.size());
    for (int i = 0; i < n; ++i) { t[i] = m->rec_spikes[i].first; gid[i] = m->rec_spikes[i].second; }
    return n;
}

int hxo_get_var(void* h, const char* mech, const char* var, int idx, double* out) {
    double* p = static_cast<Model*>(h)->var_ptr(mech, var, idx);
    if (!p) return -1;
    *out = *p;
    return 0;
}

int hxo_set_var(void* h, const char* mech, const char* var, int idx, double val) {
    double* p = static_cast<Model*>(h)->var_ptr(mech, var, idx);
    if (!p) return -1;
    *p = val;
    return 0;
}

// Bulk read of one column (node arrays: len values; mechanism columns: n values).
int hxo_get_array(void* h, const char* mech, const char* var, double* out, int cap) {
    auto* m = static_cast<Model*>(h);
    std::string mn = mech, vn = var;
    if (mn == "global" || mn == "node") {
        double* p = m->var_ptr("global", var, 0);
        if (!p || cap < m->len) return -1;
        std::memcpy(out, p, sizeof(double) * m->len);
        return m->len;
    }
    auto it = m->mechs.find(mn);
    if (it == m->mechs.end()) return -1;
    auto c = it->second->col.find(vn);
    if (c == it->second->col.end() || cap < (int)c->second.size()) return -1;
    std::memcpy(out, c->second.data(), sizeof(double) * c->second.size());
    return (int)c->second.size();
}

// Stand-alone serial tree solve (simulate.cpp:558-581) on caller arrays; d and rhs are overwritten.
void hxo_solve_serial(int ncell, int len, const int* parent, const double* a, const double* b, double* d, double* rhs) {
    double p;
    for (int i = len - 1; i >= ncell; i--) {
        p = a[i] / d[i];
        d[parent[i]] -= p * b[i];
        rhs[parent[i]] -= p * rhs[i];
    }
    for (int i = 0; i < ncell; i++) rhs[i] /= d[i];
    for (int i = ncell; i < len; i++) {
        rhs[i] -= b[i] * rhs[parent[i]];
        rhs[i] /= d[i];
    }
}

// Adam over scalar parameters addressed by (mech, var, idx); tied groups share one entry.
// optimizer.cpp:351-393 with grads provided by the caller in `grads` (one per tied member).
int hxo_adam_step(double* w, const double* grads, const int* group_size, int nparam, double* mstate,
                  double* vstate, long long step, double lr, double inv_record_steps, double impedance,
                  double beta1, double beta2, double eps) {
    int off = 0;
    for (int idx = 0; idx < nparam; ++idx) {
        int bs = group_size[idx];
        double grad_sum = 0.0;
        for (int k = 0; k < bs; ++k) grad_sum += grads[off + k];
        double avg_grad = grad_sum / static_cast<double>(bs);
        double scaled_grad = avg_grad * impedance * inv_record_steps;
        double& m_ref = mstate[idx];
        double& v_ref = vstate[idx];
        m_ref = beta1 * m_ref + (1.0 - beta1) * scaled_grad;
        v_ref = beta2 * v_ref + (1.0 - beta2) * scaled_grad * scaled_grad;
        double beta1_pow = std::pow(beta1, static_cast<double>(step));
        double beta2_pow = std::pow(beta2, static_cast<double>(step));
        double m_hat = m_ref / (1.0 - beta1_pow);
        double v_hat = v_ref / (1.0 - beta2_pow);
        w[idx] = w[idx] - lr * m_hat / (std::sqrt(v_hat) + eps);
        off += bs;
    }
    return 0;
}

// Philox4x32-10 with key (key0, key1) (known-answer checks of the NetStim streams).
int hxo_philox4x32(const uint32_t* ctr, const uint32_t* key, uint32_t* out) {
    uint32_t x0 = ctr[0], x1 = ctr[1], x2 = ctr[2], x3 = ctr[3], k0 = key[0], k1 = key[1];
    for (int rnd = 0; rnd < 10; ++rnd) {
        if (rnd > 0) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint64_t a = (uint64_t)0xD2511F53u * x0, b = (uint64_t)0xCD9E8D57u * x2;
        uint32_t y0 = (uint32_t)(b >> 32) ^ x1 ^ k0, y1 = (uint32_t)b;
        uint32_t y2 = (uint32_t)(a >> 32) ^ x3 ^ k1, y3 = (uint32_t)a;
        x0 = y0; x1 = y1; x2 = y2; x3 = y3;
    }
    out[0] = x0; out[1] = x1; out[2] = x2; out[3] = x3;
    return 0;
}

// NetStim spikes emitted since finitialize, in emission order.
int hxo_netstim_spikes(void* h, double* t, int* inst, int cap) {
    auto* m = static_cast<Model*>(h);
    int n = (int)m->ns_spikes.size();
    for (int i = 0; i < n && i < cap; ++i) { t[i] = m->ns_spikes[i].first; inst[i] = m->ns_spikes[i].second; }
    return n;
}

}  // extern "C"
