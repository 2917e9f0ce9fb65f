// Reader of CoreNEURON model exports (format 1.8 and the older layout without
// the 1.8 additions): the library's set_data_path + load_model path.
//
// The files and the reference functions whose reading order this follows:
//   bbcore_mech.dat   read_mech         read_coredat.cpp:138-200
//   files.dat         read_filesdat     read_coredat.cpp:247-283
//   <id>_1.dat        read_phase1       read_coredat.cpp:300-397
//   <id>_2.dat        read_phase2       read_coredat.cpp:621-1141
//   <id>_gap.dat      gap_setup         read_coredat.cpp:574-619
//   globals.dat       read_global_dat   global_vars.cpp:12-88
// Integers and scalars are text lines ("%d ..."); every array is a line
// "chkpnt N" followed by the raw little-endian array.  N counts arrays: it
// starts at 0 in <id>_1.dat, runs on through <id>_2.dat and starts again at 0
// in <id>_gap.dat (the reference's chkpnt counter, read_coredat.cpp:19,218-234,585).
//
// What is read becomes the model builder's calls (hx_model_*), as
// coredat_to_innerdat.cpp:42-603 turns it into the reference's group data:
//  - mechanism columns from each instance's row of nrn_prop_param_size doubles,
//    at the offsets each mechanism's read_data_from_coredat uses
//    (mech_template.cuh:280-350 with array_dims prefix sums, hh_templated.cu:51-65,
//    pas.cpp:24-40, eion.cuh:81-86, expsyn.cpp:45-60, exp2syn.cpp:64-82,
//    netstim.cpp:56-76, iclamp.cpp:28-40, capac.cpp:22-32, CA_HVA.cu:57,
//    CaDynamics_E2.cu:60-63, hd_la.cu:53-55, HalfGap.cu:44-45);
//  - the ion style of each ion instance from its first dparam (eion.cuh:155);
//  - detectors of real cells from output_vindex / output_threshold, artificial
//    presyns decoded as -(type + index * user_mod_num) (read_coredat.cpp:906-960);
//  - netcons applied in presyn order, each presyn's netcons in file order, so
//    the last one into a synapse instance wins (determine_inputpresyn,
//    read_coredat.cpp:419-572; initSynapse, coredat_to_innerdat.cpp:231-365);
//    netcon weights at the running index of the reference's receive sizes
//    (ExpSyn 1, Exp2Syn 1, other point processes 0, no target 1;
//    read_coredat.cpp:1010-1035, expsyn.h:28, exp2syn_temp.cuh:70);
//  - VecStim trains from the bbcore_read arrays: iArray[i] times of instance
//    i, concatenated in dArray (vecevent.cpp:220-255);
//  - VecPlay and gap-junction targets through the legacy index
//    (legacy_index_utils.h:20-51, coredat_to_innerdat.cpp:366-541);
//  - celsius from globals.dat, and dt from it when the caller set none
//    (mechanism.cpp:26, SimRuntimeCore.cpp:41-48); the globals of hd_la by
//    their "<name>_hd_la" entries (hd_la.cu:65-73).
// The library's own node order and solver layout are built from the parent
// array, so the reference's permutations (permute_type) do not apply: instance
// and node indices are those of the files.
#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "heliox.h"

namespace hx {

namespace {

struct VarIdx { const char* var; int index; };

// Mechanisms the library runs, with the variables their file rows supply.
// `params` are loaded into the model; `targets` may also be named by VecPlay
// records and gap transfers.
struct MechTable {
    const char* name;
    std::vector<VarIdx> params;
    std::vector<VarIdx> targets;
    int receive;      // netcon weights per netcon into this mechanism
};

const std::vector<MechTable>& mech_tables() {
    static const std::vector<MechTable> t = {
        {"capacitance", {{"cm", 0}}, {}, 0},
        {"pas", {{"g_pas", 0}, {"e_pas", 1}}, {}, 0},
        {"hh", {{"gnabar", 0}, {"gkbar", 1}, {"gl", 2}, {"el", 3}}, {}, 0},
        {"na_ion", {{"erev", 0}, {"conci", 1}, {"conco", 2}}, {}, 0},
        {"k_ion", {{"erev", 0}, {"conci", 1}, {"conco", 2}}, {}, 0},
        {"ca_ion", {{"erev", 0}, {"conci", 1}, {"conco", 2}}, {}, 0},
        {"hd_la", {{"ghdbar", 0}, {"vhalfl", 1}, {"tau", 2}}, {}, 0},
        {"Ca_HVA", {{"gbar", 0}}, {}, 0},
        {"CaDynamics_E2", {{"gamma", 0}, {"decay", 1}, {"depth", 2}, {"minCai", 3}}, {}, 0},
        {"HalfGap", {{"g", 0}}, {{"vgap", 1}}, 0},
        {"IClamp", {{"delay", 0}, {"dur", 1}, {"amp", 2}}, {}, 0},
        {"ExpSyn", {{"tau", 0}, {"e", 1}}, {}, 1},
        {"Exp2Syn", {{"tau1", 0}, {"tau2", 1}, {"e", 2}}, {}, 1},
        {"NetStim", {{"interval", 0}, {"number", 1}, {"start", 2}, {"noise", 3}}, {}, 0},
        {"VecStim", {}, {}, 0},
    };
    return t;
}

const MechTable* find_table(const std::string& name) {
    for (const auto& m : mech_tables())
        if (name == m.name) return &m;
    return nullptr;
}

struct Error {
    std::string msg;
};

[[noreturn]] void raise(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void raise(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    throw Error{buf};
}

std::vector<int> parse_version(const std::string& v) {
    std::vector<int> parts;
    size_t i = 0;
    while (i < v.size()) {
        size_t j = v.find('.', i);
        if (j == std::string::npos) j = v.size();
        parts.push_back(std::atoi(v.substr(i, j - i).c_str()));
        i = j + 1;
    }
    return parts;
}

// version >= threshold, compared part by part (utils.cpp:18-33)
bool version_at_least(const std::string& v, const std::string& thr) {
    const auto a = parse_version(v), b = parse_version(thr);
    for (size_t i = 0; i < std::max(a.size(), b.size()); ++i) {
        const int x = i < a.size() ? a[i] : 0, y = i < b.size() ? b[i] : 0;
        if (x != y) return x > y;
    }
    return true;
}

// One data file: text lines and chkpnt-framed binary arrays.
class DataFile {
public:
    DataFile(const std::string& path, int* chkpnt) : path_(path), chkpnt_(chkpnt) {
        f_ = std::fopen(path.c_str(), "rb");
        if (!f_) raise("cannot open %s", path.c_str());
    }
    ~DataFile() { if (f_) std::fclose(f_); }
    DataFile(const DataFile&) = delete;
    DataFile& operator=(const DataFile&) = delete;

    std::string line() {
        char buf[1024];
        if (!std::fgets(buf, sizeof(buf), f_)) raise("%s: unexpected end of file", path_.c_str());
        return buf;
    }
    int read_int() {
        const std::string s = line();
        int v;
        if (std::sscanf(s.c_str(), "%d", &v) != 1) raise("%s: expected an integer line, got '%s'", path_.c_str(),
                                                           trim(s).c_str());
        return v;
    }
    template <class T>
    std::vector<T> array(long long n) {
        if (n < 0) raise("%s: negative array length %lld", path_.c_str(), n);
        const std::string s = line();
        int c;
        if (std::sscanf(s.c_str(), "chkpnt %d", &c) != 1)
            raise("%s: no chkpnt line before array %d (got '%s')", path_.c_str(), *chkpnt_, trim(s).c_str());
        if (c != *chkpnt_) raise("%s: chkpnt %d where %d was expected", path_.c_str(), c, *chkpnt_);
        ++*chkpnt_;
        std::vector<T> v(static_cast<size_t>(n));
        if (n && std::fread(v.data(), sizeof(T), v.size(), f_) != v.size())
            raise("%s: array %d is cut short", path_.c_str(), c);
        return v;
    }
    const std::string& path() const { return path_; }

    static std::string trim(std::string s) {
        while (!s.empty() && (s.back() == '\n' || s.back() == '\r')) s.pop_back();
        return s;
    }

private:
    std::string path_;
    FILE* f_ = nullptr;
    int* chkpnt_;
};

struct MechType {
    std::string name;
    int pnttype = 0, is_art = 0, is_ion = 0, dsize = 0, pdsize = 0;
    std::vector<int> dims;     // array_dims (format 1.8); empty: every variable is a scalar
    bool known = false;
};

struct MechData {
    int type = 0, n = 0;
    std::vector<int> nodes;
    std::vector<double> data;  // n rows of dsize
    std::vector<int> pdata;    // n rows of pdsize
};

struct VecPlayRec {
    int vtype, mtype, ix;
    std::vector<double> y, t;
};

struct Export {
    std::string version;
    std::vector<MechType> types;
    int group = 0;
    bool have_gaps = false;
    // phase 1
    std::vector<int> output_gid, netcon_srcgid;
    // phase 2
    int n_real_cell = 0, n_output = 0, n_real_output = 0, nnode = 0;
    std::vector<int> parent;
    std::vector<double> a, b, area;
    std::vector<MechData> mechs;   // file order
    std::vector<int> output_vindex;
    std::vector<double> output_threshold;
    std::vector<int> pnttype, pntindex;
    std::vector<double> weights, delay;
    std::map<int, std::pair<std::vector<int>, std::vector<double>>> bbcore;   // type -> (iArray, dArray)
    std::vector<VecPlayRec> vecplay;
    // gaps
    std::vector<int> src_sid, src_type, src_index, tar_sid, tar_type, tar_index;
    // globals
    std::map<std::string, std::vector<double>> globals;
};

void read_mech_file(const std::string& dir, Export& x) {
    const std::string path = dir + "/bbcore_mech.dat";
    FILE* f = std::fopen(path.c_str(), "r");
    if (!f) raise("cannot open %s", path.c_str());
    std::unique_ptr<FILE, int (*)(FILE*)> guard(f, std::fclose);
    char ver[256];
    int nmech = 0;
    if (std::fscanf(f, "%255s %d", ver, &nmech) != 2 || nmech < 2) raise("%s: bad header", path.c_str());
    const bool v18 = version_at_least(ver, "1.8");
    x.types.assign(nmech, MechType{});
    for (int i = 2; i < nmech; ++i) {
        char name[1000];
        MechType m;
        int type = -1;
        if (std::fscanf(f, "%999s %d %d %d %d %d %d", name, &type, &m.pnttype, &m.is_art, &m.is_ion, &m.dsize,
                        &m.pdsize) != 7)
            raise("%s: bad line for mechanism %d", path.c_str(), i);
        if (type != i) raise("%s: mechanism %s has type %d at line of type %d", path.c_str(), name, type, i);
        if (v18) {
            int nv = 0;
            if (std::fscanf(f, "%d", &nv) != 1 || nv < 0) raise("%s: %s: bad array_dims count", path.c_str(), name);
            m.dims.resize(nv);
            for (int k = 0; k < nv; ++k)
                if (std::fscanf(f, "%d", &m.dims[k]) != 1) raise("%s: %s: bad array_dims", path.c_str(), name);
        }
        if (m.is_ion) {
            double charge;
            if (std::fscanf(f, "%lf", &charge) != 1) raise("%s: %s: missing ion charge", path.c_str(), name);
        }
        m.name = name;
        m.known = true;
        x.types[i] = m;
    }
}

void read_files_dat(const std::string& dir, Export& x) {
    const std::string path = dir + "/files.dat";
    FILE* f = std::fopen(path.c_str(), "r");
    if (!f) raise("cannot open %s", path.c_str());
    std::unique_ptr<FILE, int (*)(FILE*)> guard(f, std::fclose);
    char ver[256];
    int n = 0;
    if (std::fscanf(f, "%255s %d", ver, &n) != 2) raise("%s: bad header", path.c_str());
    x.version = ver;
    if (n == -1) {
        x.have_gaps = true;
        if (std::fscanf(f, "%d", &n) != 1) raise("%s: bad file count", path.c_str());
    }
    // one group, as the reference reads (read_coredat.cpp:46)
    if (n != 1) raise("%s: %d groups; one group (one files.dat entry) is supported", path.c_str(), n);
    if (std::fscanf(f, "%d", &x.group) != 1) raise("%s: missing group id", path.c_str());
}

void read_phase1(const std::string& dir, Export& x, int* chk) {
    DataFile F(dir + "/" + std::to_string(x.group) + "_1.dat", chk);
    F.line();   // version
    const int npre = F.read_int();
    const int nnc = F.read_int();
    x.output_gid = F.array<int>(npre);
    x.netcon_srcgid = F.array<int>(nnc);
}

void read_phase2(const std::string& dir, Export& x, int* chk) {
    DataFile F(dir + "/" + std::to_string(x.group) + "_2.dat", chk);
    const std::string ver = DataFile::trim(F.line());
    const bool v18 = version_at_least(ver, "1.8");
    if (v18) x.n_real_cell = F.read_int();
    x.n_output = F.read_int();
    x.n_real_output = F.read_int();
    if (!v18) x.n_real_cell = x.n_real_output;
    x.nnode = F.read_int();
    const int ndiam = F.read_int();
    const int nmech = F.read_int();
    if (x.nnode <= 0 || x.n_real_cell < 0 || x.n_real_cell > x.nnode || nmech < 0)
        raise("%s: bad counts (cells %d, nodes %d, mechanisms %d)", F.path().c_str(), x.n_real_cell, x.nnode, nmech);
    x.mechs.resize(nmech);
    for (auto& m : x.mechs) {
        m.type = F.read_int();
        m.n = F.read_int();
        if (m.type < 2 || m.type >= static_cast<int>(x.types.size()) || !x.types[m.type].known)
            raise("%s: mechanism type %d is not in bbcore_mech.dat", F.path().c_str(), m.type);
        if (m.n < 0) raise("%s: negative instance count", F.path().c_str());
    }
    F.read_int();   // nidata
    F.read_int();   // nvdata
    const int nweight = F.read_int();
    x.parent = F.array<int>(x.nnode);
    x.a = F.array<double>(x.nnode);
    x.b = F.array<double>(x.nnode);
    x.area = F.array<double>(x.nnode);
    F.array<double>(x.nnode);                 // v
    if (ndiam) F.array<double>(x.nnode);      // diam
    for (auto& m : x.mechs) {
        const MechType& t = x.types[m.type];
        if (!t.is_art) m.nodes = F.array<int>(m.n);
        else m.nodes.assign(m.n, 0);
        m.data = F.array<double>(static_cast<long long>(m.n) * t.dsize);
        if (t.pdsize) m.pdata = F.array<int>(static_cast<long long>(m.n) * t.pdsize);
        if (v18 && t.pdsize > 0) {
            int sz = F.read_int();
            if (sz) F.array<int>(sz);          // pointer2type
            sz = F.read_int();
            if (sz) F.array<uint32_t>(sz);     // nmodlrandom
        }
    }
    const int npre = static_cast<int>(x.output_gid.size());
    const int nnc = static_cast<int>(x.netcon_srcgid.size());
    if (x.n_real_output < 0 || x.n_real_output > npre)
        raise("%s: %d real outputs but %d presyns", F.path().c_str(), x.n_real_output, npre);
    x.output_vindex = F.array<int>(npre);
    x.output_threshold = F.array<double>(x.n_real_output);
    x.pnttype = F.array<int>(nnc);
    x.pntindex = F.array<int>(nnc);
    x.weights = F.array<double>(nweight);
    x.delay = F.array<double>(nnc);
    F.read_int();   // number of point processes
    for (const auto& m : x.mechs) {
        if (x.types[m.type].name != "VecStim") continue;    // the only bbcore_read mechanism (read_coredat.cpp:191-196)
        const int type = F.read_int();
        const int icnt = F.read_int();
        const int dcnt = F.read_int();
        if (type != m.type) raise("%s: bbcore data of type %d where %d was expected", F.path().c_str(), type, m.type);
        auto& e = x.bbcore[type];
        if (icnt) e.first = F.array<int>(icnt);
        if (dcnt) e.second = F.array<double>(dcnt);
    }
    const int nvp = F.read_int();
    for (int i = 0; i < nvp; ++i) {
        VecPlayRec r;
        r.vtype = F.read_int();
        r.mtype = F.read_int();
        r.ix = F.read_int();
        const int sz = F.read_int();
        r.y = F.array<double>(sz);
        r.t = F.array<double>(sz);
        x.vecplay.push_back(std::move(r));
    }
    // what may follow (checkpoint restore: vecplay indices, patstim, presyn
    // flags, queued events) is not used by the reference either
}

void read_gap(const std::string& dir, Export& x) {
    int chk = 0;
    DataFile F(dir + "/" + std::to_string(x.group) + "_gap.dat", &chk);
    F.line();   // version
    const int sidt = F.read_int();
    if (sidt != static_cast<int>(sizeof(int))) raise("%s: sid size %d (4 expected)", F.path().c_str(), sidt);
    const int ntar = F.read_int();
    const int nsrc = F.read_int();
    if (nsrc) {
        x.src_sid = F.array<int>(nsrc);
        x.src_type = F.array<int>(nsrc);
        x.src_index = F.array<int>(nsrc);
    }
    if (ntar) {
        x.tar_sid = F.array<int>(ntar);
        x.tar_type = F.array<int>(ntar);
        x.tar_index = F.array<int>(ntar);
    }
}

void read_globals(const std::string& dir, Export& x) {
    const std::string path = dir + "/globals.dat";
    FILE* f = std::fopen(path.c_str(), "r");
    if (!f) raise("cannot open %s", path.c_str());
    std::unique_ptr<FILE, int (*)(FILE*)> guard(f, std::fclose);
    char line[512];
    if (!std::fgets(line, sizeof(line), f)) raise("%s: empty", path.c_str());   // version
    // name value lines, "name[n]" followed by n value lines, up to "0 0"
    while (true) {
        if (!std::fgets(line, sizeof(line), f)) raise("%s: no '0 0' line", path.c_str());
        char name[256];
        double val;
        int n;
        if (std::sscanf(line, "%255s %lf", name, &val) == 2) {
            if (std::strcmp(name, "0") == 0) break;
            x.globals.emplace(name, std::vector<double>{val});
        } else if (std::sscanf(line, "%255[^[][%d]", name, &n) == 2) {
            if (std::strcmp(name, "0") == 0) break;
            if (n < 0) raise("%s: bad array length for %s", path.c_str(), name);
            std::vector<double> v(n);
            for (int i = 0; i < n; ++i) {
                if (!std::fgets(line, sizeof(line), f) || std::sscanf(line, "%lf", &v[i]) != 1)
                    raise("%s: %s[%d] is cut short", path.c_str(), name, n);
            }
            x.globals.emplace(name, std::move(v));
        } else {
            raise("%s: cannot read line '%s'", path.c_str(), DataFile::trim(line).c_str());
        }
    }
    // the second part (secondorder, Random123_globalindex) is stored but not used by the reference
}

// legacy flat index -> (instance, variable, array element) (legacy_index_utils.h:20-40)
void legacy_index(int ix, const MechType& t, int& inst, int& var, int& elem) {
    std::vector<int> dims = t.dims;
    if (dims.empty()) dims.assign(std::max(t.dsize, 1), 1);
    int width = 0;
    for (int d : dims) width += d;
    if (width <= 0 || ix < 0) raise("%s: bad legacy index %d", t.name.c_str(), ix);
    const int colx = ix % width;
    inst = ix / width;
    var = 0;
    int prefix = 0;
    for (size_t k = 0; k + 1 < dims.size(); ++k) {
        if (colx >= prefix + dims[k]) {
            prefix += dims[k];
            var = static_cast<int>(k) + 1;
        } else {
            break;
        }
    }
    elem = colx - prefix;
}

// flat offset of variable `var` in an instance row
int var_offset(const MechType& t, int var) {
    if (t.dims.empty()) return var;
    if (var >= static_cast<int>(t.dims.size())) raise("%s: variable %d beyond its array_dims", t.name.c_str(), var);
    int off = 0;
    for (int k = 0; k < var; ++k) off += t.dims[k];
    return off;
}

const char* target_var(const MechTable& mt, int var) {
    for (const auto& p : mt.params)
        if (p.index == var) return p.var;
    for (const auto& p : mt.targets)
        if (p.index == var) return p.var;
    return nullptr;
}

void check(hx_sim* sim, int rc, const char* what) {
    if (rc < 0) raise("%s: %s", what, hx_last_error(sim));
}

void build(hx_sim* sim, const Export& x, int mod_num, bool take_dt) {
    // ---- globals
    auto g = x.globals.find("celsius");
    if (g == x.globals.end() || g->second.empty()) raise("globals.dat has no celsius");
    check(sim, hx_set_celsius(sim, g->second[0]), "celsius");
    if (take_dt) {
        auto d = x.globals.find("dt");
        if (d == x.globals.end() || d->second.empty()) raise("no dt was set and globals.dat has none");
        check(sim, hx_set_dt(sim, d->second[0]), "dt");
    }
    // ---- nodes
    const int nnode = x.nnode, ncell = x.n_real_cell;
    std::vector<int> parent = x.parent;
    for (int i = 0; i < ncell; ++i) parent[i] = -1;
    for (int i = ncell; i < nnode; ++i)
        if (parent[i] < 0 || parent[i] >= i)
            raise("node %d has parent %d: a node's parent must come before it", i, parent[i]);
    check(sim, hx_model_set_nodes(sim, ncell, nnode, parent.data(), x.a.data(), x.b.data(), x.area.data()), "nodes");

    // ---- mechanisms: unknown names first, so the error lists all of them
    std::string unknown;
    for (const auto& m : x.mechs) {
        const std::string& nm = x.types[m.type].name;
        if (!find_table(nm)) unknown += (unknown.empty() ? "" : ", ") + nm;
    }
    if (!unknown.empty()) raise("mechanisms not provided by this library: %s", unknown.c_str());
    std::vector<int> mech_of_type(x.types.size(), -1);
    for (size_t k = 0; k < x.mechs.size(); ++k) {
        if (mech_of_type[x.mechs[k].type] >= 0) raise("mechanism type %d is listed twice", x.mechs[k].type);
        mech_of_type[x.mechs[k].type] = static_cast<int>(k);
    }
    // ions first: the other mechanisms read them
    std::vector<int> order;
    for (int pass = 0; pass < 2; ++pass)
        for (size_t k = 0; k < x.mechs.size(); ++k)
            if ((x.types[x.mechs[k].type].is_ion != 0) == (pass == 0)) order.push_back(static_cast<int>(k));
    for (int k : order) {
        const MechData& m = x.mechs[k];
        const MechType& t = x.types[m.type];
        const MechTable& mt = *find_table(t.name);
        for (int nd : m.nodes)
            if (nd < 0 || nd >= nnode) raise("%s: node index %d out of range", t.name.c_str(), nd);
        auto column = [&](int var) {
            const int off = var_offset(t, var);
            if (off >= t.dsize) raise("%s: variable %d at offset %d beyond the row of %d", t.name.c_str(), var, off,
                                      t.dsize);
            std::vector<double> c(m.n);
            for (int i = 0; i < m.n; ++i) c[i] = m.data[static_cast<size_t>(i) * t.dsize + off];
            return c;
        };
        if (t.name == "capacitance") {
            std::vector<double> cm(nnode, 1.0);
            const auto c = column(0);
            for (int i = 0; i < m.n; ++i) cm[m.nodes[i]] = c[i];
            check(sim, hx_model_set_param(sim, "capacitance", "cm", nnode, cm.data()), "capacitance");
            continue;
        }
        check(sim, hx_model_insert(sim, t.name.c_str(), m.n, m.nodes.data()), t.name.c_str());
        for (const auto& p : mt.params) {
            const auto c = column(p.index);
            check(sim, hx_model_set_param(sim, t.name.c_str(), p.var, m.n, c.data()), p.var);
        }
        if (t.is_ion) {
            if (t.pdsize < 1) raise("%s: ion without its style dparam", t.name.c_str());
            std::vector<int> style(m.n);
            for (int i = 0; i < m.n; ++i) style[i] = m.pdata[static_cast<size_t>(i) * t.pdsize];
            check(sim, hx_model_set_iontype(sim, t.name.c_str(), m.n, style.data()), "ion style");
        }
        if (t.name == "hd_la") {
            static const char* hd[] = {"ehd", "kl", "vhalft", "a0t", "zetat", "gmt", "q10", "qtl"};
            for (const char* gname : hd) {
                auto it = x.globals.find(std::string(gname) + "_hd_la");
                if (it == x.globals.end() || it->second.empty()) raise("globals.dat has no %s_hd_la", gname);
                check(sim, hx_model_set_global(sim, "hd_la", gname, it->second[0]), gname);
            }
        }
    }

    // ---- presyns (read_coredat.cpp:906-960, coredat_to_innerdat.cpp:254-300)
    const int npre = static_cast<int>(x.output_gid.size());
    enum { DEAD = -1 };
    std::vector<int> src_kind(npre, DEAD), src_inst(npre, 0);
    for (int i = 0; i < npre; ++i) {
        int ix = x.output_vindex[i];
        if (ix == -1 && i < x.n_real_output) continue;      // real cell without a detector
        if (ix < 0) {
            ix = -ix;
            const int index = ix / mod_num;
            const int type = ix - index * mod_num;
            if (type < 2 || type >= static_cast<int>(x.types.size()) || mech_of_type[type] < 0)
                raise("presyn %d: artificial cell of type %d is not in the model (user_mod_num %d)", i, type, mod_num);
            const std::string& nm = x.types[type].name;
            if (nm != "VecStim" && nm != "NetStim") raise("presyn %d: %s cannot be an event source", i, nm.c_str());
            if (index < 0 || index >= x.mechs[mech_of_type[type]].n)
                raise("presyn %d: %s instance %d out of range", i, nm.c_str(), index);
            src_kind[i] = nm == "VecStim" ? 1 : 2;
            src_inst[i] = index;
        } else {
            if (i >= x.n_real_output) raise("presyn %d on node %d comes after the artificial presyns", i, ix);
            if (ix >= nnode) raise("presyn %d: node %d out of range", i, ix);
            if (x.output_gid[i] < 0) raise("presyn %d of a real cell has gid %d", i, x.output_gid[i]);
            const int det = hx_model_add_presyn(sim, x.output_gid[i], ix, x.output_threshold[i]);
            check(sim, det, "presyn");
            src_kind[i] = 0;
            src_inst[i] = det;
        }
    }

    // ---- netcons: gid -> presyn, then the winner per synapse instance
    std::map<int, int> gid2pre;
    for (int i = 0; i < npre; ++i) {
        const int gid = x.output_gid[i];
        if (gid == -1) continue;
        if (!gid2pre.emplace(gid, i).second) raise("gid %d names two presyns", gid);
    }
    const int nnc = static_cast<int>(x.netcon_srcgid.size());
    std::vector<int> weight_index(nnc);
    size_t iw = 0;
    for (int j = 0; j < nnc; ++j) {
        weight_index[j] = static_cast<int>(iw);
        const int type = x.pnttype[j];
        if (type > 0) {
            const MechTable* mt = type < static_cast<int>(x.types.size()) && x.types[type].known
                                      ? find_table(x.types[type].name) : nullptr;
            iw += mt ? mt->receive : 0;
        } else {
            iw += 1;
        }
    }
    if (iw != x.weights.size())
        raise("netcon weights: %zu in the file, %zu by the receive sizes (ExpSyn 1, Exp2Syn 1, others 0)",
              x.weights.size(), iw);
    std::vector<std::vector<int>> by_pre(npre);
    for (int j = 0; j < nnc; ++j) {
        auto it = gid2pre.find(x.netcon_srcgid[j]);
        if (it != gid2pre.end()) by_pre[it->second].push_back(j);
    }
    std::map<std::pair<int, int>, std::pair<int, int>> winner;   // (type, instance) -> (presyn, netcon)
    for (int p = 0; p < npre; ++p)
        for (int j : by_pre[p]) {
            if (x.pnttype[j] <= 0) continue;
            winner[{x.pnttype[j], x.pntindex[j]}] = {p, j};
        }
    for (const auto& w : winner) {
        const int type = w.first.first, inst = w.first.second;
        const int p = w.second.first, j = w.second.second;
        if (src_kind[p] == DEAD) continue;     // its source never fires
        if (type >= static_cast<int>(x.types.size()) || mech_of_type[type] < 0)
            raise("netcon %d into type %d, which the model does not hold", j, type);
        const std::string& nm = x.types[type].name;
        if (nm != "ExpSyn" && nm != "Exp2Syn") raise("netcon %d into %s: only ExpSyn and Exp2Syn take events", j,
                                                     nm.c_str());
        if (inst < 0 || inst >= x.mechs[mech_of_type[type]].n) raise("netcon %d: %s instance %d out of range", j,
                                                                     nm.c_str(), inst);
        check(sim, hx_model_add_netcon(sim, src_kind[p], src_inst[p], nm.c_str(), inst, x.weights[weight_index[j]],
                                       x.delay[j]), "netcon");
    }

    // ---- VecStim trains
    for (const auto& e : x.bbcore) {
        const auto& counts = e.second.first;
        const auto& times = e.second.second;
        const int n = x.mechs[mech_of_type[e.first]].n;
        size_t off = 0;
        for (size_t i = 0; i < counts.size(); ++i) {
            const int c = counts[i];
            if (c <= 0) continue;
            if (static_cast<int>(i) >= n) raise("VecStim train %zu beyond the %d instances", i, n);
            if (off + c > times.size()) raise("VecStim trains: %zu times listed, more counted", times.size());
            check(sim, hx_model_set_vecstim(sim, static_cast<int>(i), c, times.data() + off), "VecStim");
            off += c;
        }
    }

    // ---- VecPlay (coredat_to_innerdat.cpp:515-541)
    for (const auto& r : x.vecplay) {
        if (r.vtype != 4) raise("VecPlay record of type %d (only continuous play, type 4, is read)", r.vtype);
        if (r.mtype < 2 || r.mtype >= static_cast<int>(x.types.size()) || mech_of_type[r.mtype] < 0)
            raise("VecPlay into type %d, which the model does not hold", r.mtype);
        const MechType& t = x.types[r.mtype];
        int inst, var, elem;
        legacy_index(r.ix, t, inst, var, elem);
        const char* vn = target_var(*find_table(t.name), var);
        if (!vn || elem != 0) raise("VecPlay into %s variable %d[%d], which this library does not play", t.name.c_str(),
                                    var, elem);
        if (r.t.empty()) raise("VecPlay into %s.%s[%d] without points", t.name.c_str(), vn, inst);
        check(sim, hx_add_vecplay(sim, t.name.c_str(), vn, inst, static_cast<int>(r.t.size()), r.t.data(), r.y.data()),
              "VecPlay");
    }

    // ---- gap junctions (coredat_to_innerdat.cpp:418-513): v of a node into HalfGap.vgap
    if (x.have_gaps) {
        std::map<int, int> src_of_sid;
        for (size_t i = 0; i < x.src_sid.size(); ++i) src_of_sid[x.src_sid[i]] = static_cast<int>(i);
        for (size_t i = 0; i < x.tar_sid.size(); ++i) {
            auto it = src_of_sid.find(x.tar_sid[i]);
            if (it == src_of_sid.end()) raise("gap target %zu: sid %d has no source", i, x.tar_sid[i]);
            const int s = it->second;
            if (x.src_type[s] != -1) raise("gap source sid %d is type %d (only voltage, -1, is read)", x.src_sid[s],
                                           x.src_type[s]);
            const int node = x.src_index[s];
            if (node < 0 || node >= nnode) raise("gap source node %d out of range", node);
            const int tt = x.tar_type[i];
            if (tt < 2 || tt >= static_cast<int>(x.types.size()) || x.types[tt].name != "HalfGap" ||
                mech_of_type[tt] < 0)
                raise("gap target %zu is type %d (only HalfGap.vgap is read)", i, tt);
            int inst, var, elem;
            legacy_index(x.tar_index[i], x.types[tt], inst, var, elem);
            if (var != 1 || elem != 0) raise("gap target %zu is HalfGap variable %d (vgap, 1, expected)", i, var);
            if (inst >= x.mechs[mech_of_type[tt]].n) raise("gap target %zu: HalfGap instance %d out of range", i, inst);
            check(sim, hx_model_add_gap(sim, node, inst), "gap");
        }
    }
}

}  // namespace

// Reads the export in `dir` into the model builder of `sim`.  Returns 0, or -1
// with the reason in `err`.
int read_coredat(hx_sim* sim, const std::string& dir, int user_mod_num, bool take_dt, std::string& err) {
    try {
        if (user_mod_num <= 0) raise("user_mod_num must be positive");
        Export x;
        read_files_dat(dir, x);
        read_mech_file(dir, x);
        int chk = 0;
        read_phase1(dir, x, &chk);
        read_phase2(dir, x, &chk);
        if (x.have_gaps) read_gap(dir, x);
        read_globals(dir, x);
        build(sim, x, user_mod_num, take_dt);
    } catch (const Error& e) {
        err = e.msg;
        return -1;
    } catch (const std::exception& e) {
        err = std::string("reading the export: ") + e.what();
        return -1;
    }
    return 0;
}

}  // namespace hx
