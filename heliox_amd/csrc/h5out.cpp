// Monitor output to HDF5: <output_dir>/sim_out.h5 with one dataset per monitor at
// /group_0/<mech>/<var>/<idx>, double, one dimension, unlimited, chunks of 100
// samples, grown by each flush (the reference's layout, simulate.cpp:185-269, and
// its append-on-flush, variable_recorder.h:142-156 / variable_recorder.cu:54-70).
//
// The HDF5 C library is loaded with dlopen when the output is switched on, so the
// library itself has no link-time dependency on it; without it, switching the
// output on fails with a message and nothing else changes.  Version 1.10 or later
// is required (64-bit hid_t).
#include "h5out.h"

#include <dlfcn.h>

#include <cstdint>
#include <cstdlib>
#include <filesystem>
#include <stdexcept>
#include <string>

namespace hx {
namespace {

using hid_t = int64_t;
using herr_t = int;
using htri_t = int;
using hsize_t = unsigned long long;

constexpr hid_t kP_DEFAULT = 0;          // H5P_DEFAULT
constexpr hid_t kS_ALL = 0;              // H5S_ALL
constexpr hid_t kE_DEFAULT = 0;          // H5E_DEFAULT
constexpr unsigned kF_ACC_TRUNC = 0x0002u;
constexpr int kS_SELECT_SET = 0;
constexpr int kF_SCOPE_LOCAL = 0;
constexpr hsize_t kS_UNLIMITED = ~0ull;
constexpr hsize_t kChunk = 100;          // HighFive::Chunking({100}) in the reference

struct Api {
    void* so = nullptr;
    herr_t (*open)();
    herr_t (*get_libversion)(unsigned*, unsigned*, unsigned*);
    herr_t (*eset_auto2)(hid_t, void*, void*);
    hid_t (*fcreate)(const char*, unsigned, hid_t, hid_t);
    herr_t (*fclose)(hid_t);
    herr_t (*fflush)(hid_t, int);
    hid_t (*gcreate2)(hid_t, const char*, hid_t, hid_t, hid_t);
    herr_t (*gclose)(hid_t);
    htri_t (*lexists)(hid_t, const char*, hid_t);
    hid_t (*screate_simple)(int, const hsize_t*, const hsize_t*);
    herr_t (*sclose)(hid_t);
    hid_t (*pcreate)(hid_t);
    herr_t (*pset_chunk)(hid_t, int, const hsize_t*);
    herr_t (*pclose)(hid_t);
    hid_t (*dcreate2)(hid_t, const char*, hid_t, hid_t, hid_t, hid_t, hid_t);
    hid_t (*dopen2)(hid_t, const char*, hid_t);
    herr_t (*dclose)(hid_t);
    herr_t (*dset_extent)(hid_t, const hsize_t*);
    hid_t (*dget_space)(hid_t);
    int (*sget_simple_extent_dims)(hid_t, hsize_t*, hsize_t*);
    herr_t (*sselect_hyperslab)(hid_t, int, const hsize_t*, const hsize_t*, const hsize_t*, const hsize_t*);
    herr_t (*dwrite)(hid_t, hid_t, hid_t, hid_t, hid_t, const void*);
    hid_t* native_double = nullptr;      // H5T_NATIVE_DOUBLE_g
    hid_t* dataset_create = nullptr;     // H5P_CLS_DATASET_CREATE_ID_g
};

template <class F>
void bind(Api& a, F& f, const char* name) {
    f = reinterpret_cast<F>(dlsym(a.so, name));
    if (!f) throw std::runtime_error(std::string("libhdf5 lacks ") + name);
}

// The loaded library, once per process (dlopen keeps it loaded).
const Api& api() {
    static Api a;
    static std::string failure;
    static bool tried = false;
    if (tried) {
        if (!a.so) throw std::runtime_error(failure);
        return a;
    }
    tried = true;
    std::string tried_names;
    const char* env = std::getenv("HELIOX_HDF5_LIB");
    const char* names[] = {env, "libhdf5.so", "libhdf5.so.103", "/opt/conda/lib/libhdf5.so",
                           "/usr/lib/x86_64-linux-gnu/hdf5/serial/libhdf5.so"};
    for (const char* n : names) {
        if (!n || !*n) continue;
        a.so = dlopen(n, RTLD_NOW | RTLD_LOCAL);
        if (a.so) break;
        tried_names += std::string(tried_names.empty() ? "" : ", ") + n;
    }
    if (!a.so) {
        failure = "HDF5 output needs the HDF5 C library (1.10 or later); none found (tried " + tried_names +
                  "; HELIOX_HDF5_LIB names another)";
        throw std::runtime_error(failure);
    }
    try {
        bind(a, a.open, "H5open");
        bind(a, a.get_libversion, "H5get_libversion");
        bind(a, a.eset_auto2, "H5Eset_auto2");
        bind(a, a.fcreate, "H5Fcreate");
        bind(a, a.fclose, "H5Fclose");
        bind(a, a.fflush, "H5Fflush");
        bind(a, a.gcreate2, "H5Gcreate2");
        bind(a, a.gclose, "H5Gclose");
        bind(a, a.lexists, "H5Lexists");
        bind(a, a.screate_simple, "H5Screate_simple");
        bind(a, a.sclose, "H5Sclose");
        bind(a, a.pcreate, "H5Pcreate");
        bind(a, a.pset_chunk, "H5Pset_chunk");
        bind(a, a.pclose, "H5Pclose");
        bind(a, a.dcreate2, "H5Dcreate2");
        bind(a, a.dopen2, "H5Dopen2");
        bind(a, a.dclose, "H5Dclose");
        bind(a, a.dset_extent, "H5Dset_extent");
        bind(a, a.dget_space, "H5Dget_space");
        bind(a, a.sget_simple_extent_dims, "H5Sget_simple_extent_dims");
        bind(a, a.sselect_hyperslab, "H5Sselect_hyperslab");
        bind(a, a.dwrite, "H5Dwrite");
        bind(a, a.native_double, "H5T_NATIVE_DOUBLE_g");
        bind(a, a.dataset_create, "H5P_CLS_DATASET_CREATE_ID_g");
        if (a.open() < 0) throw std::runtime_error("H5open failed");
        unsigned maj = 0, min = 0, rel = 0;
        a.get_libversion(&maj, &min, &rel);
        if (maj < 1 || (maj == 1 && min < 10))
            throw std::runtime_error("HDF5 " + std::to_string(maj) + "." + std::to_string(min) +
                                     " is too old (1.10 or later has the 64-bit hid_t this writer uses)");
        a.eset_auto2(kE_DEFAULT, nullptr, nullptr);   // errors come back as return codes only
    } catch (const std::exception& e) {
        failure = e.what();
        dlclose(a.so);
        a.so = nullptr;
        throw;
    }
    return a;
}

void check(bool ok, const std::string& what) {
    if (!ok) throw std::runtime_error("HDF5: " + what + " failed");
}

}  // namespace

bool H5Recorder::available(std::string& why) {
    try {
        (void)api();
        return true;
    } catch (const std::exception& e) {
        why = e.what();
        return false;
    }
}

H5Recorder::~H5Recorder() { close(); }

void H5Recorder::close() {
    if (file_ < 0) return;
    const Api& a = api();
    for (auto& kv : dsets_) a.dclose(kv.second);
    dsets_.clear();
    a.fclose(file_);
    file_ = -1;
}

void H5Recorder::open(const std::string& dir) {
    close();
    const Api& a = api();
    std::error_code ec;
    std::filesystem::create_directories(dir, ec);
    if (ec) throw std::runtime_error("cannot create " + dir + ": " + ec.message());
    path_ = dir + "/sim_out.h5";
    file_ = a.fcreate(path_.c_str(), kF_ACC_TRUNC, kP_DEFAULT, kP_DEFAULT);
    check(file_ >= 0, "creating " + path_);
    ensure_group("/group_0");
}

void H5Recorder::ensure_group(const std::string& path) {
    const Api& a = api();
    const htri_t e = a.lexists(file_, path.c_str(), kP_DEFAULT);
    check(e >= 0, "looking up " + path);
    if (e > 0) return;
    const hid_t g = a.gcreate2(file_, path.c_str(), kP_DEFAULT, kP_DEFAULT, kP_DEFAULT);
    check(g >= 0, "creating group " + path);
    a.gclose(g);
}

int64_t H5Recorder::dataset(const std::string& mech, const std::string& var, int idx) {
    const std::string path = "/group_0/" + mech + "/" + var + "/" + std::to_string(idx);
    auto it = dsets_.find(path);
    if (it != dsets_.end()) return it->second;
    const Api& a = api();
    ensure_group("/group_0/" + mech);
    ensure_group("/group_0/" + mech + "/" + var);
    hid_t d = -1;
    const htri_t e = a.lexists(file_, path.c_str(), kP_DEFAULT);
    check(e >= 0, "looking up " + path);
    if (e > 0) {
        d = a.dopen2(file_, path.c_str(), kP_DEFAULT);
    } else {
        const hsize_t dims = 0, maxdims = kS_UNLIMITED;
        const hid_t space = a.screate_simple(1, &dims, &maxdims);
        check(space >= 0, "dataspace for " + path);
        const hid_t dcpl = a.pcreate(*a.dataset_create);
        check(dcpl >= 0 && a.pset_chunk(dcpl, 1, &kChunk) >= 0, "chunking for " + path);
        d = a.dcreate2(file_, path.c_str(), *a.native_double, space, kP_DEFAULT, dcpl, kP_DEFAULT);
        a.pclose(dcpl);
        a.sclose(space);
    }
    check(d >= 0, "dataset " + path);
    dsets_[path] = d;
    return d;
}

void H5Recorder::append(const std::string& mech, const std::string& var, int idx, const double* x, size_t n) {
    if (file_ < 0 || n == 0) return;
    const Api& a = api();
    const hid_t d = dataset(mech, var, idx);
    hid_t space = a.dget_space(d);
    hsize_t cur = 0;
    check(space >= 0 && a.sget_simple_extent_dims(space, &cur, nullptr) == 1, "reading the extent");
    a.sclose(space);
    const hsize_t grown = cur + n;
    check(a.dset_extent(d, &grown) >= 0, "growing a dataset");
    space = a.dget_space(d);
    const hsize_t count = n;
    const hid_t mem = a.screate_simple(1, &count, nullptr);
    const bool ok = space >= 0 && mem >= 0 &&
                    a.sselect_hyperslab(space, kS_SELECT_SET, &cur, nullptr, &count, nullptr) >= 0 &&
                    a.dwrite(d, *a.native_double, mem, space, kP_DEFAULT, x) >= 0;
    if (mem >= 0) a.sclose(mem);
    if (space >= 0) a.sclose(space);
    check(ok, "writing samples");
}

void H5Recorder::flush() {
    if (file_ >= 0) check(api().fflush(file_, kF_SCOPE_LOCAL) >= 0, "flushing " + path_);
}

}  // namespace hx
