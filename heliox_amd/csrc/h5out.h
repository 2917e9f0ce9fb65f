// Monitor samples written to <output_dir>/sim_out.h5 (the reference's recorder file,
// simulate.cpp:185-269, variable_recorder.h:142-156), through the HDF5 C library
// loaded at run time.
#pragma once
#include <cstddef>
#include <cstdint>
#include <map>
#include <string>

namespace hx {

class H5Recorder {
public:
    H5Recorder() = default;
    ~H5Recorder();
    H5Recorder(const H5Recorder&) = delete;
    H5Recorder& operator=(const H5Recorder&) = delete;

    // Whether the HDF5 library can be loaded; why it cannot otherwise.
    static bool available(std::string& why);
    // Creates (truncates) <dir>/sim_out.h5 with its /group_0.
    void open(const std::string& dir);
    bool is_open() const { return file_ >= 0; }
    const std::string& path() const { return path_; }
    // Appends n samples to /group_0/<mech>/<var>/<idx>, creating it on first use.
    void append(const std::string& mech, const std::string& var, int idx, const double* x, size_t n);
    void flush();
    void close();

private:
    void ensure_group(const std::string& path);
    int64_t dataset(const std::string& mech, const std::string& var, int idx);

    int64_t file_ = -1;
    std::string path_;
    std::map<std::string, int64_t> dsets_;
};

}  // namespace hx
