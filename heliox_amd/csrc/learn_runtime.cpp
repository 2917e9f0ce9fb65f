// Host side of the learn gradient surface: dense blocks, the capture session
// and the per-tick LRDS replay driver (LearnRuntime.cpp:197-257, 1619-2457).
//
// The replay loop issues, per LR tick, base -> correction GEMM -> [clip] ->
// w_tick -> [dx] on one stream with no host synchronisation: the Frobenius
// clip decision, the grad scale and the history rescale stay on the device
// (the reference copies the norm to the host every checked tick).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "learn.h"

namespace hx {
namespace {

struct HipFail : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define LRC(x)                                                                    \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) throw HipFail(std::string(#x) + ": " + hipGetErrorString(e_)); \
    } while (0)

template <class T>
T* lalloc(std::vector<void*>& owned, size_t n) {
    void* p = nullptr;
    LRC(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    owned.push_back(p);
    return static_cast<T*>(p);
}

template <class T>
T* lupload(std::vector<void*>& owned, const T* h, size_t n) {
    T* p = lalloc<T>(owned, n);
    if (n) LRC(hipMemcpy(p, h, n * sizeof(T), hipMemcpyHostToDevice));
    return p;
}

}  // namespace

LearnRuntime::~LearnRuntime() {
    free_all(blk_mem_);
    free_all(cap_mem_);
    free_all(sess_mem_);
    free_all(sig_mem_);
    free_all(ws_mem_);
}

void LearnRuntime::free_all(std::vector<void*>& v) {
    for (void* p : v) (void)hipFree(p);
    v.clear();
}

int LearnRuntime::fail(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    err = buf;
    return -1;
}

// LearnRuntime::clear_dense_blocks (LearnRuntime.cpp:246-257) also drops the
// capture cache and the replay workspace.
void LearnRuntime::clear_dense_blocks() {
    (void)hipStreamSynchronize(stream_);
    free_all(blk_mem_);
    free_all(cap_mem_);
    free_all(ws_mem_);
    free_all(sig_mem_);
    ws_key_.clear();
    k_len_ = nblk_ = max_bn_ = 0;
    bn_.clear();
    start_.clear();
    koff_.clear();
    boff_.clear();
    tiles_.clear();
    cap_N_ = cap_T_ = cap_kmul_ = 0;
    cap_percise_ = false;
    sig_N_ = sig_T_ = 0;
    for (int c = 0; c < kLrMaxChannels; ++c) d_cap_[c] = d_sig_[c] = nullptr;
}

// LearnRuntime::set_dense_blocks_f32 (LearnRuntime.cpp:197-244): every block is
// square with one common K_len; returns K_len.
int LearnRuntime::set_dense_blocks(int nblk, const float* const* data, const int* bn, const int* k_len) {
    clear_dense_blocks();
    if (nblk <= 0) return 0;
    int kl = -1;
    for (int b = 0; b < nblk; ++b) {
        if (!data || !data[b] || bn[b] <= 0 || k_len[b] <= 0) return fail("set_dense_blocks_f32: invalid block at %d", b);
        if (kl < 0) kl = k_len[b];
        else if (k_len[b] != kl)
            return fail("set_dense_blocks_f32: K_len mismatch in block %d (%d vs %d)", b, k_len[b], kl);
    }
    try {
        std::vector<float> kt1, kt2;
        int start = 0;
        long long koff = 0, boff = 0;
        for (int b = 0; b < nblk; ++b) {
            const int n = bn[b];
            const size_t plane = static_cast<size_t>(n) * n;
            bn_.push_back(n);
            start_.push_back(start);
            koff_.push_back(koff);
            boff_.push_back(boff);
            max_bn_ = std::max(max_bn_, n);
            kt1.resize(static_cast<size_t>(koff) + plane * kl);
            kt2.resize(static_cast<size_t>(koff) + plane * kl);
            // element K[i][j][tau] goes to kt1[tau][i][j] (base term) and, read as
            // K_b[j'][k][tau] with j' = i, k = j, to kt2[tau][k][j'] (GEMM B operand)
            const float* K = data[b];
            for (int i = 0; i < n; ++i)
                for (int j = 0; j < n; ++j)
                    for (int tau = 0; tau < kl; ++tau) {
                        const float v = K[(static_cast<size_t>(i) * n + j) * kl + tau];
                        kt1[koff + tau * plane + static_cast<size_t>(i) * n + j] = v;
                        kt2[koff + tau * plane + static_cast<size_t>(j) * n + i] = v;
                    }
            start += n;
            koff += static_cast<long long>(plane) * kl;
            boff += static_cast<long long>(plane);
        }
        k_len_ = kl;
        nblk_ = nblk;
        // column tile of the correction GEMM: 128 when a block is wider than 64
        tile_cols_ = max_bn_ > 64 ? 128 : 64;
        for (int b = 0; b < nblk; ++b)
            for (int j0 = 0; j0 < bn_[b]; j0 += tile_cols_) tiles_.push_back(make_int2(b, j0));
        d_kt1_ = lupload(blk_mem_, kt1.data(), kt1.size());
        d_kt2_ = lupload(blk_mem_, kt2.data(), kt2.size());
        d_koff_ = lupload(blk_mem_, koff_.data(), koff_.size());
        d_boff_ = lupload(blk_mem_, boff_.data(), boff_.size());
        d_start_ = lupload(blk_mem_, start_.data(), start_.size());
        d_bn_ = lupload(blk_mem_, bn_.data(), bn_.size());
        d_tiles_ = lupload(blk_mem_, tiles_.data(), tiles_.size());
        d_base_ = lalloc<float>(blk_mem_, static_cast<size_t>(boff));
    } catch (const std::exception& e) {
        clear_dense_blocks();
        return fail("set_dense_blocks_f32: %s", e.what());
    }
    return k_len_;
}

void LearnRuntime::begin_capture(int nsample, const std::vector<double*>& out_ptr, int N, int T, int k_mul,
                                 bool percise, const Channel* ch, int nch, Sink sink) {
    free_all(sess_mem_);
    free_all(sess_sig_mem_);
    for (int c = 0; c < kLrMaxChannels; ++c) d_stream_[c] = nullptr;
    stream_N_ = stream_T_ = 0;
    cargs_ = CaptureArgs{};
    cargs_.n_out = static_cast<int>(out_ptr.size());
    cargs_.out_ptr = lupload(sess_mem_, out_ptr.data(), out_ptr.size());
    cargs_.out_vs = lalloc<float>(sess_mem_, static_cast<size_t>(nsample) * out_ptr.size());
    cargs_.N = N;
    cargs_.nch = N > 0 ? nch : 0;
    nsample_ = nsample;
    sample_ = 0;
    kmul_ = k_mul;
    sink_ = sink;
    sess_T_ = 0;
    if (N > 0) {
        if (T <= 0) T = (nsample - 1) / k_mul + 1;
        sess_T_ = T;
        float* buf[kLrMaxChannels] = {nullptr, nullptr, nullptr};
        if (sink != SINK_CACHE) {
            for (int c = 0; c < nch; ++c) buf[c] = lalloc<float>(sess_sig_mem_, static_cast<size_t>(T) * N);
        } else {
            if (cap_N_ != N || cap_T_ != T || cap_kmul_ != k_mul || cap_percise_ != percise) {
                free_all(cap_mem_);
                for (int c = 0; c < kLrMaxChannels; ++c) d_cap_[c] = nullptr;
                for (int c = 0; c < nch; ++c) d_cap_[c] = lalloc<float>(cap_mem_, static_cast<size_t>(T) * N);
                cap_N_ = N;
                cap_T_ = T;
                cap_kmul_ = k_mul;
                cap_percise_ = percise;
            }
            for (int c = 0; c < nch; ++c) buf[c] = d_cap_[c];
        }
        for (int c = 0; c < nch; ++c) {
            // LR rows keep index 0 as zeros (LearnRuntime.cpp:1571-1574, 1938-1942)
            launch_fill_f32(buf[c], 0.f, static_cast<long long>(T) * N, stream_);
            // group the channel's items by destination column, keeping input order
            std::vector<int> begin(N + 1, 0);
            for (int d : ch[c].dest) begin[d + 1]++;
            for (int i = 0; i < N; ++i) begin[i + 1] += begin[i];
            std::vector<int> fill(begin.begin(), begin.end() - 1);
            std::vector<double*> ptr(ch[c].ptr.size());
            std::vector<float> scale(ch[c].ptr.size());
            for (size_t q = 0; q < ch[c].ptr.size(); ++q) {
                const int at = fill[ch[c].dest[q]]++;
                ptr[at] = ch[c].ptr[q];
                scale[at] = ch[c].scale[q];
            }
            cargs_.ch[c].begin = lupload(sess_mem_, begin.data(), begin.size());
            cargs_.ch[c].ptr = lupload(sess_mem_, ptr.data(), ptr.size());
            cargs_.ch[c].scale = lupload(sess_mem_, scale.data(), scale.size());
            cargs_.ch[c].buf = buf[c];
        }
    }
    capturing_ = true;
}

void LearnRuntime::sample() {
    if (!capturing_) return;
    if (sample_ >= nsample_) throw std::runtime_error("learn capture: more samples than steps");
    const int k = kmul_;
    const int lr = (cargs_.nch > 0 && sample_ > 0 && sample_ % k == 0 && sample_ / k < sess_T_) ? sample_ / k : 0;
    launch_lr_capture(cargs_, sample_, lr, stream_);
    ++sample_;
}

void LearnRuntime::end_capture(float* out_vs_host, float* const* sig_host) {
    capturing_ = false;
    LRC(hipStreamSynchronize(stream_));
    if (sample_ != nsample_) throw std::runtime_error("learn capture: sample count mismatch");
    if (out_vs_host && cargs_.n_out > 0)
        LRC(hipMemcpy(out_vs_host, cargs_.out_vs, sizeof(float) * static_cast<size_t>(nsample_) * cargs_.n_out,
                      hipMemcpyDeviceToHost));
    if (sink_ == SINK_HOST && sig_host) {
        const size_t n = static_cast<size_t>(sess_T_) * cargs_.N;
        for (int c = 0; c < kLrMaxChannels; ++c) {
            if (!sig_host[c]) continue;
            if (c < cargs_.nch)
                LRC(hipMemcpy(sig_host[c], cargs_.ch[c].buf, sizeof(float) * n, hipMemcpyDeviceToHost));
            else
                std::fill(sig_host[c], sig_host[c] + n, 0.f);
        }
    }
    if (sink_ == SINK_STREAM) {
        for (int c = 0; c < kLrMaxChannels; ++c) d_stream_[c] = c < cargs_.nch ? cargs_.ch[c].buf : nullptr;
        stream_N_ = cargs_.N;
        stream_T_ = sess_T_;
    } else {
        free_all(sess_sig_mem_);
    }
    free_all(sess_mem_);
}

// replay_compute_dw_dx_from_signals_into's signal upload (LearnRuntime.cpp:575-582):
// host (N, T) arrays are transposed on the device into the (T, N) layout.
int LearnRuntime::load_signals(const float* it_nt, const float* dv_nt, const float* dp_nt, int N, int T,
                               bool percise) {
    try {
        free_all(sig_mem_);
        for (int c = 0; c < kLrMaxChannels; ++c) d_sig_[c] = nullptr;
        const size_t n = static_cast<size_t>(N) * T;
        float* stage = lalloc<float>(sig_mem_, n);
        const float* src[3] = {it_nt, dv_nt, dp_nt};
        const int nch = percise ? 3 : 1;
        for (int c = 0; c < nch; ++c) {
            d_sig_[c] = lalloc<float>(sig_mem_, n);
            LRC(hipMemcpy(stage, src[c], n * sizeof(float), hipMemcpyHostToDevice));
            launch_transpose_nt_tn(stage, d_sig_[c], N, T, stream_);
            LRC(hipStreamSynchronize(stream_));
        }
        sig_N_ = N;
        sig_T_ = T;
    } catch (const std::exception& e) {
        return fail("replay_compute_dw_dx_from_signals_into: %s", e.what());
    }
    return 0;
}

int LearnRuntime::replay(const ReplayIn& in) {
    const int N = in.source == SRC_CACHE ? cap_N_ : in.source == SRC_HOST ? sig_N_ : stream_N_;
    const int T = in.source == SRC_CACHE ? cap_T_ : in.source == SRC_HOST ? sig_T_ : stream_T_;
    float* const* sig = in.source == SRC_CACHE ? d_cap_ : in.source == SRC_HOST ? d_sig_ : d_stream_;
    if (N <= 0 || T != in.ksteps + 1) return fail("replay: no signals of %d ticks", in.ksteps);
    const int K_len = k_len_;
    const int ks = in.ksteps;
    try {
        // workspace: history ring, base scratch, per-tick vectors, norm partials
        const int R = in.percise ? K_len + 1 : 1;
        const size_t slice = static_cast<size_t>(N) * N;
        const int ntiles = static_cast<int>(tiles_.size());
        const int nwg = ntiles * rp_corr_row_tiles(N);
        const std::vector<long long> key = {N, R, ks, in.n_out, in.n_in, nwg, in.percise ? 1 : 0};
        if (key != ws_key_) {
            free_all(ws_mem_);
            ws_key_.clear();
            ws_.hist = lalloc<float>(ws_mem_, slice * R);
            ws_.ghist = in.percise ? lalloc<float>(ws_mem_, slice * R) : nullptr;
            ws_.slot_scale = lalloc<float>(ws_mem_, R);
            ws_.gs = lalloc<float>(ws_mem_, 1);
            ws_.tick_scale = lalloc<float>(ws_mem_, 1);
            ws_.w_tick = lalloc<float>(ws_mem_, N);
            ws_.dw_acc = lalloc<float>(ws_mem_, N);
            ws_.dl = lalloc<float>(ws_mem_, static_cast<size_t>(ks) * in.n_out);
            ws_.po = lalloc<int>(ws_mem_, in.n_out);
            ws_.pre = lalloc<int>(ws_mem_, N);
            ws_.pin = lalloc<int>(ws_mem_, std::max(in.n_in, 1));
            ws_.dx = lalloc<float>(ws_mem_, static_cast<size_t>(std::max(in.n_in, 1)) * ks);
            ws_.norm_part = lalloc<double>(ws_mem_, nwg);
            ws_.flag_part = lalloc<int>(ws_mem_, nwg);
            ws_.dw_out = lalloc<float>(ws_mem_, N);
            ws_key_ = key;
        }
    } catch (const std::exception& e) {
        free_all(ws_mem_);
        ws_key_.clear();
        return fail("replay: %s", e.what());
    }
    return replay_on(in, ws_, sig, N);
}

// The replay proper over signals sig[c] ((T, N) on the device) with the buffers of ws;
// it allocates nothing (with timing off).
int LearnRuntime::replay_on(const ReplayIn& in, const Workspace& ws, float* const* sig, int N) {
    const int K_len = k_len_;
    const int ks = in.ksteps;
    const bool need_dx = in.n_in > 0;
    try {
        const int R = in.percise ? K_len + 1 : 1;
        const size_t slice = static_cast<size_t>(N) * N;
        const int ntiles = static_cast<int>(tiles_.size());
        const int nwg = ntiles * rp_corr_row_tiles(N);
        float* hist = ws.hist;
        float* ghist = ws.ghist;
        float* slot_scale = ws.slot_scale;
        float* gs = ws.gs;
        float* tick_scale = ws.tick_scale;
        float* w_tick = ws.w_tick;
        float* dw_acc = ws.dw_acc;
        float* dl = ws.dl;
        int* po = ws.po;
        int* pre = ws.pre;
        int* pin = ws.pin;
        float* dx = ws.dx;
        double* norm_part = ws.norm_part;
        int* flag_part = ws.flag_part;
        float* dw_out = ws.dw_out;
        LRC(hipMemcpyAsync(dl, in.dl, sizeof(float) * static_cast<size_t>(ks) * in.n_out, hipMemcpyHostToDevice,
                           stream_));
        LRC(hipMemcpyAsync(po, in.po, sizeof(int) * in.n_out, hipMemcpyHostToDevice, stream_));
        LRC(hipMemcpyAsync(pre, in.pre, sizeof(int) * N, hipMemcpyHostToDevice, stream_));
        if (need_dx) LRC(hipMemcpyAsync(pin, in.pin, sizeof(int) * in.n_in, hipMemcpyHostToDevice, stream_));

        launch_fill_f32(hist, 0.f, static_cast<long long>(slice), stream_);      // slot 0: tick 0
        if (in.percise) launch_fill_f32(ghist, 0.f, static_cast<long long>(slice), stream_);
        launch_fill_f32(slot_scale, 1.f, R, stream_);
        launch_fill_f32(gs, static_cast<float>(in.grad_scale), 1, stream_);
        launch_fill_f32(tick_scale, 1.f, 1, stream_);
        launch_fill_f32(dw_acc, 0.f, N, stream_);
        if (need_dx) launch_fill_f32(dx, 0.f, static_cast<long long>(in.n_in) * ks, stream_);

        const float dt = static_cast<float>(in.dt);
        const float eps = static_cast<float>(in.eps);
        const float thr = static_cast<float>(in.thr);
        corr_ms = 0;
        corr_launches = 0;
        std::vector<std::pair<hipEvent_t, hipEvent_t>> evs;

        for (int t_lr = 1; t_lr <= ks; ++t_lr) {
            const int tw = std::min(t_lr, K_len);
            const int it_t0 = t_lr - tw + 1;
            const int k_t0 = K_len - tw;
            const int cur = in.percise ? t_lr % R : 0;
            float* out = hist + static_cast<size_t>(cur) * slice;
            bool due = false;
            if (in.clip_strategy != 0) {
                if (in.cached_clip_rule) due = in.clip_strategy == 1 || (t_lr % in.clip_every) == 0;
                else due = in.clip_strategy == 1 && (t_lr % in.clip_every) == 0;
            }

            ReplayBaseArgs B{};
            B.kt1 = d_kt1_;
            B.koff = d_koff_;
            B.boff = d_boff_;
            B.start = d_start_;
            B.bn = d_bn_;
            B.it = sig[0];
            B.N = N;
            B.it_t0 = it_t0;
            B.k_t0 = k_t0;
            B.tw = tw;
            B.dt = dt;
            B.gs = gs;
            B.base = d_base_;
            B.slot_scale = slot_scale;
            B.cur = cur;
            launch_rp_base(B, nblk_, max_bn_, stream_);

            ReplayCorrArgs C{};
            C.hist = hist;
            C.ghist = ghist;
            C.slice = static_cast<long long>(slice);
            C.slot_scale = slot_scale;
            C.R = R;
            C.dv = sig[1];
            C.dp = sig[2];
            C.pre = pre;
            C.kt2 = d_kt2_;
            C.koff = d_koff_;
            C.start = d_start_;
            C.bn = d_bn_;
            C.base = d_base_;
            C.boff = d_boff_;
            C.tiles = d_tiles_;
            C.N = N;
            C.t_lr = t_lr;
            C.tw = in.percise ? tw : 0;
            C.it_t0 = it_t0;
            C.k_t0 = k_t0;
            C.dt = dt;
            C.out = out;
            C.sanitize = due ? 1 : 0;
            C.norm_part = norm_part;
            C.flag_part = flag_part;
            if (timing) {
                hipEvent_t a, b;
                LRC(hipEventCreate(&a));
                LRC(hipEventCreate(&b));
                LRC(hipEventRecord(a, stream_));
                launch_rp_corr(C, ntiles, tile_cols_, stream_);
                LRC(hipEventRecord(b, stream_));
                evs.push_back({a, b});
            } else {
                launch_rp_corr(C, ntiles, tile_cols_, stream_);
            }
            if (in.percise) launch_rp_pregather(out, pre, N, ghist + static_cast<size_t>(cur) * slice, stream_);
            if (due) launch_rp_clip(norm_part, flag_part, nwg, thr, gs, slot_scale, R, tick_scale, stream_);
            launch_rp_wtick(out, slot_scale, cur, N, po, in.n_out, dl + static_cast<size_t>(t_lr - 1) * in.n_out,
                            due ? 1 : 0, tick_scale, w_tick, dw_acc, stream_);
            if (need_dx)
                launch_rp_dx(out, slot_scale, cur, N, pin, in.n_in, w_tick, eps, t_lr - 1, ks, due ? 1 : 0,
                             tick_scale, dx, stream_);
        }
        // dw = dw_accum * (1 / ksteps) in fp32 (LearnRuntime.cpp:2281-2285)
        launch_rp_scale_into(dw_acc, 1.0f / static_cast<float>(ks), dw_out, N, stream_);
        LRC(hipStreamSynchronize(stream_));
        LRC(hipGetLastError());
        for (auto& pr : evs) {
            float ms = 0;
            LRC(hipEventElapsedTime(&ms, pr.first, pr.second));
            corr_ms += ms;
            corr_launches++;
            (void)hipEventDestroy(pr.first);
            (void)hipEventDestroy(pr.second);
        }
        LRC(hipMemcpy(in.dw_out, dw_out, sizeof(float) * N, hipMemcpyDeviceToHost));
        if (need_dx)
            LRC(hipMemcpy(in.dx_out, dx, sizeof(float) * static_cast<size_t>(in.n_in) * ks, hipMemcpyDeviceToHost));
    } catch (const std::exception& e) {
        return fail("replay: %s", e.what());
    }
    return 0;
}

// ---------------------------------------------------------------------------
// Replay without allocation: every device buffer of a host-signal replay is
// carved from one file-scope device array, `scratch`.  Each device holds its
// own copy; its address is looked up once per device with hipGetSymbolAddress
// (the array's name in host code is not a device address).  All calls on one
// device share it, so calls that overlap on one device race.
// ---------------------------------------------------------------------------
namespace {
constexpr int kScratchMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
std::mutex scratch_mu;
unsigned char* scratch_dev[kScratchMaxDevices] = {};

// 256-byte aligned sub-allocations of the scratch array, in a fixed order; with
// base == nullptr it only measures.
struct Carver {
    unsigned char* base;
    size_t used = 0;
    template <class T>
    T* take(size_t n) {
        used = (used + 255) & ~static_cast<size_t>(255);
        T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
        used += std::max<size_t>(n, 1) * sizeof(T);
        return p;
    }
};
}  // namespace

// Address of this device's scratch array (looked up on the first call on each device).
unsigned char* noalloc_scratch() {
    int dev = 0;
    LRC(hipGetDevice(&dev));
    if (dev < 0 || dev >= kScratchMaxDevices) throw HipFail("device index out of range for the scratch table");
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_dev[dev]) {
        void* p = nullptr;
        LRC(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        scratch_dev[dev] = static_cast<unsigned char*>(p);
    }
    return scratch_dev[dev];
}

int LearnRuntime::replay_from_host_noalloc(const ReplayIn& in, const float* it_nt, const float* dv_nt,
                                           const float* dp_nt, int N, int T) {
    if (N <= 0 || T != in.ksteps + 1) return fail("replay: no signals of %d ticks", in.ksteps);
    try {
        const int nch = in.percise ? 3 : 1;
        const int R = in.percise ? k_len_ + 1 : 1;
        const size_t slice = static_cast<size_t>(N) * N;
        const size_t sigsz = static_cast<size_t>(N) * T;
        const int nwg = static_cast<int>(tiles_.size()) * rp_corr_row_tiles(N);
        const int ks = in.ksteps;
        auto carve = [&](Carver& c, Workspace& w, float** sig, float** stage) {
            *stage = c.take<float>(sigsz);
            for (int ch = 0; ch < kLrMaxChannels; ++ch) sig[ch] = ch < nch ? c.take<float>(sigsz) : nullptr;
            w.hist = c.take<float>(slice * R);
            w.ghist = in.percise ? c.take<float>(slice * R) : nullptr;
            w.slot_scale = c.take<float>(R);
            w.gs = c.take<float>(1);
            w.tick_scale = c.take<float>(1);
            w.w_tick = c.take<float>(N);
            w.dw_acc = c.take<float>(N);
            w.dl = c.take<float>(static_cast<size_t>(ks) * in.n_out);
            w.po = c.take<int>(in.n_out);
            w.pre = c.take<int>(N);
            w.pin = c.take<int>(std::max(in.n_in, 1));
            w.dx = c.take<float>(static_cast<size_t>(std::max(in.n_in, 1)) * ks);
            w.norm_part = c.take<double>(nwg);
            w.flag_part = c.take<int>(nwg);
            w.dw_out = c.take<float>(N);
        };
        Workspace w;
        float* sig[kLrMaxChannels];
        float* stage = nullptr;
        Carver measure{nullptr};
        carve(measure, w, sig, &stage);
        if (measure.used > kNoAllocScratchBytes)
            return fail("replay needs %zu bytes of device scratch for N=%d, T=%d, K_len=%d%s; the allocation-free "
                        "entry point holds at most %zu bytes (use the allocating one)",
                        measure.used, N, T, k_len_, in.percise ? " (percise)" : "", kNoAllocScratchBytes);
        Carver c{noalloc_scratch()};
        carve(c, w, sig, &stage);
        // (N, T) host signals -> (T, N) on the device, as load_signals does
        const float* src[kLrMaxChannels] = {it_nt, dv_nt, dp_nt};
        for (int ch = 0; ch < nch; ++ch) {
            LRC(hipMemcpyAsync(stage, src[ch], sigsz * sizeof(float), hipMemcpyHostToDevice, stream_));
            launch_transpose_nt_tn(stage, sig[ch], N, T, stream_);
        }
        const bool was_timing = timing;
        timing = false;                 // the timing path creates events
        const int rc = replay_on(in, w, sig, N);
        timing = was_timing;
        return rc;
    } catch (const std::exception& e) {
        return fail("replay: %s", e.what());
    }
}

}  // namespace hx
