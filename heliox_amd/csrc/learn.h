// Learn gradient surface: learning-signal capture during a forward run and the
// LRDS replay of dv/dw over the captured signals (the reference's LearnRuntime,
// LearnRuntime.cpp:197-2457, kernels replay_dw_dx.cu:9-731).
//
// HBM layout:
//   * captured signals It, dIt/dv, dIt/dvpre are time-major (T, N) fp32, T =
//     ksteps + 1, row 0 zero: a capture writes one contiguous row per LR tick;
//   * dense block b (bn x bn x K_len, the caller's kernel K_b[i][j][tau]) is
//     kept twice, tau-major: kt1 = K_b[i][j][tau] at [tau][i][j] (base term) and
//     kt2 = K_b[j][k][tau] at [tau][k][j] (the correction GEMM's B operand,
//     contiguous in the output column j);
//   * the dv/dw history is a ring of K_len + 1 row-major N x N fp32 slices:
//     tick tau lives in slot tau % (K_len + 1), slot 0 starts as the zero slice
//     of tick 0, and the slot a tick writes is never in its own read window.
//     A second ring holds each slice's column-gathered copy G[i][c] =
//     D[i][pre(c)], written once per tick, so the correction's pre operand is a
//     contiguous read instead of a gather per (row, tap);
//     A per-slot fp32 scale carries the Frobenius clip's rescaling of the history
//     instead of rewriting K_len slices.
#pragma once
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

namespace hx {

constexpr int kLrMaxChannels = 3;     // pure_i, didv, didvpre
// Size of the per-device scratch array of the allocation-free replay (64 MiB).
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(64) << 20;

struct CaptureChannel {
    const int* begin = nullptr;       // N + 1: items of column c are [begin[c], begin[c+1])
    double* const* ptr = nullptr;     // item sources, grouped by column in input order
    const float* scale = nullptr;
    float* buf = nullptr;             // (T, N) time-major
};

struct CaptureArgs {
    int n_out = 0;
    double* const* out_ptr = nullptr;
    float* out_vs = nullptr;          // (nsample, n_out)
    int N = 0;
    int nch = 0;
    CaptureChannel ch[kLrMaxChannels];
};

struct ReplayBaseArgs {
    const float* kt1 = nullptr;
    const long long* koff = nullptr;  // per block offset into kt1 / kt2
    const long long* boff = nullptr;  // per block offset into base (sum of bn^2)
    const int* start = nullptr;
    const int* bn = nullptr;
    const float* it = nullptr;        // (T, N)
    int N = 0, it_t0 = 0, k_t0 = 0, tw = 0;
    float dt = 0.f;
    const float* gs = nullptr;        // device grad scale
    float* base = nullptr;
    float* slot_scale = nullptr;      // slot_scale[cur] is reset to 1
    int cur = 0;
};

struct ReplayCorrArgs {
    const float* hist = nullptr;
    const float* ghist = nullptr;     // column-gathered copies: ghist[h][i][c] = hist[h][i][pre(c)]
    long long slice = 0;              // N * N
    const float* slot_scale = nullptr;
    int R = 1;                        // ring slots
    const float* dv = nullptr;        // dIt/dv (T, N)
    const float* dp = nullptr;        // dIt/dvpre (T, N)
    const int* pre = nullptr;
    const float* kt2 = nullptr;
    const long long* koff = nullptr;
    const int* start = nullptr;
    const int* bn = nullptr;
    const float* base = nullptr;
    const long long* boff = nullptr;
    const int2* tiles = nullptr;      // (block, first column) of each column tile
    int N = 0, t_lr = 0, tw = 0, it_t0 = 0, k_t0 = 0;
    float dt = 0.f;
    float* out = nullptr;             // slot of this tick
    int sanitize = 0;                 // zero non-finite entries and write norm partials
    double* norm_part = nullptr;
    int* flag_part = nullptr;
};

void launch_lr_capture(const CaptureArgs& a, int sample, int lr, hipStream_t s);
void launch_rp_base(const ReplayBaseArgs& a, int nblk, int max_bn, hipStream_t s);
void launch_rp_corr(const ReplayCorrArgs& a, int ntiles, int tile_cols, hipStream_t s);
void launch_rp_pregather(const float* D, const int* pre, int N, float* G, hipStream_t s);
int rp_corr_row_tiles(int N);
void launch_rp_clip(const double* part, const int* flag, int n, float thr, float* gs, float* slot_scale, int R,
                    float* tick_scale, hipStream_t s);
void launch_rp_wtick(const float* cur, const float* slot_scale, int cur_slot, int N, const int* po, int n_out,
                     const float* dl, int clip_ran, const float* tick_scale, float* w_tick, float* dw_acc,
                     hipStream_t s);
void launch_rp_dx(const float* cur, const float* slot_scale, int cur_slot, int N, const int* pin, int n_in,
                  const float* w_tick, float eps, int t_idx, int ksteps, int clip_ran, const float* tick_scale,
                  float* dx, hipStream_t s);
void launch_rp_scale_into(const float* src, float scale, float* dst, long long n, hipStream_t s);
void launch_fill_f32(float* p, float v, long long n, hipStream_t s);
void launch_transpose_nt_tn(const float* src_nt, float* dst_tn, int N, int T, hipStream_t s);

// Host side of the learn surface, owned by a simulation handle.
class LearnRuntime {
public:
    explicit LearnRuntime(hipStream_t s) : stream_(s) {}
    ~LearnRuntime();
    LearnRuntime(const LearnRuntime&) = delete;
    LearnRuntime& operator=(const LearnRuntime&) = delete;

    std::string err;

    // LearnRuntime::set_dense_blocks_f32 / clear_dense_blocks (LearnRuntime.cpp:197-257)
    int set_dense_blocks(int nblk, const float* const* data, const int* bn, const int* k_len);
    void clear_dense_blocks();
    int k_len() const { return k_len_; }
    const std::vector<int>& block_sizes() const { return bn_; }

    // Capture session (LearnRuntime.cpp:1619-1984).  Channel c has its items'
    // sources, destination columns and scales; N = 0 captures outputs only.
    struct Channel {
        std::vector<double*> ptr;
        std::vector<int> dest;
        std::vector<float> scale;
    };
    // Where a capture's signals go: the cache that cached replays read, host
    // buffers given to end_capture (the _into variant), or a private set kept for
    // one streaming replay.  Only CACHE touches the cache.
    enum Sink { SINK_CACHE = 0, SINK_HOST, SINK_STREAM };
    // T <= 0 derives T = (nsample - 1) / k_mul + 1.
    void begin_capture(int nsample, const std::vector<double*>& out_ptr, int N, int T, int k_mul, bool percise,
                       const Channel* ch, int nch, Sink sink);
    bool capturing() const { return capturing_; }
    void sample();                                   // one record point
    void end_capture(float* out_vs_host, float* const* sig_host = nullptr);

    // Replay over the cached capture, host signals loaded by load_signals, or the
    // last streaming capture; the clip schedule follows the entry point.
    enum Source { SRC_CACHE = 0, SRC_HOST, SRC_STREAM };
    struct ReplayIn {
        const float* dl = nullptr;   // (ksteps, n_out)
        int ksteps = 0, n_out = 0, n_in = 0;
        const int* po = nullptr;
        const int* pin = nullptr;
        const int* pre = nullptr;    // N
        float* dw_out = nullptr;     // N
        float* dx_out = nullptr;     // (n_in, ksteps)
        double dt = 0, grad_scale = 1, eps = 1e-6, thr = 1e6;
        bool percise = false;
        int clip_strategy = 1, clip_every = 1;
        Source source = SRC_CACHE;
        bool cached_clip_rule = true;   // strategy 1 every tick, others every clip_every
    };
    int replay(const ReplayIn& in);
    int load_signals(const float* it_nt, const float* dv_nt, const float* dp_nt, int N, int T, bool percise);
    // The replay over host (N, T) signals with every device buffer carved from the
    // library's fixed scratch array (kNoAllocScratchBytes per device): no allocation.
    int replay_from_host_noalloc(const ReplayIn& in, const float* it_nt, const float* dv_nt, const float* dp_nt, int N,
                                 int T);
    int capture_N() const { return cap_N_; }
    int capture_T() const { return cap_T_; }
    bool capture_percise() const { return cap_percise_; }

    // kernel time of the last replay's correction GEMM launches, when timing is on
    bool timing = false;
    double corr_ms = 0;
    long long corr_launches = 0;

    struct Workspace {
        float *hist = nullptr, *ghist = nullptr, *slot_scale = nullptr, *gs = nullptr, *tick_scale = nullptr,
              *w_tick = nullptr, *dw_acc = nullptr, *dl = nullptr, *dx = nullptr, *dw_out = nullptr;
        int *po = nullptr, *pre = nullptr, *pin = nullptr, *flag_part = nullptr;
        double* norm_part = nullptr;
    };

private:
    int fail(const char* fmt, ...);
    void free_all(std::vector<void*>& v);
    int replay_on(const ReplayIn& in, const Workspace& ws, float* const* sig, int N);

    hipStream_t stream_;
    // dense blocks
    int k_len_ = 0, nblk_ = 0, max_bn_ = 0, tile_cols_ = 64;
    std::vector<int> bn_, start_;
    std::vector<long long> koff_, boff_;
    std::vector<int2> tiles_;
    std::vector<void*> blk_mem_;
    float *d_kt1_ = nullptr, *d_kt2_ = nullptr, *d_base_ = nullptr;
    long long *d_koff_ = nullptr, *d_boff_ = nullptr;
    int *d_start_ = nullptr, *d_bn_ = nullptr;
    int2* d_tiles_ = nullptr;
    // capture cache (T, N) per channel
    int cap_N_ = 0, cap_T_ = 0, cap_kmul_ = 0;
    bool cap_percise_ = false;
    std::vector<void*> cap_mem_;
    float* d_cap_[kLrMaxChannels] = {nullptr, nullptr, nullptr};
    // capture session
    bool capturing_ = false;
    int sample_ = 0, nsample_ = 0, kmul_ = 1, sess_T_ = 0;
    Sink sink_ = SINK_CACHE;
    std::vector<void*> sess_sig_mem_;   // HOST / STREAM signal buffers
    float* d_stream_[kLrMaxChannels] = {nullptr, nullptr, nullptr};
    int stream_N_ = 0, stream_T_ = 0;
    CaptureArgs cargs_{};
    std::vector<void*> sess_mem_;
    // host-loaded signals (T, N)
    int sig_N_ = 0, sig_T_ = 0;
    std::vector<void*> sig_mem_;
    float* d_sig_[kLrMaxChannels] = {nullptr, nullptr, nullptr};
    // replay workspace, kept while the problem shape is unchanged
    std::vector<void*> ws_mem_;
    std::vector<long long> ws_key_;
    Workspace ws_;
};

}  // namespace hx
