// Counter-based random streams for artificial cells (host and device).
//
// Philox4x32-10 is the published counter-based generator of Salmon, Moraes,
// Dror and Shaw, "Parallel random numbers: as easy as 1, 2, 3" (SC11): ten
// rounds of two 32x32->64 multiplications with the constants of the paper,
// the high halves xored with the other counter words and the key, the key
// bumped by the Weyl constants between rounds.  The reference uses it through
// its vendored Random123 headers (src/third_party/Random123/philox.h) and
// wraps it as a stream in src/utils/nrnran123.cpp:23-110; Stream123 below has
// that wrapper's behaviour: the counter's word 0 is the sequence number, words
// 1-3 the stream ids, key word 0 the global index (0 here), and each 128-bit
// output is handed out one 32-bit word at a time before the counter steps.
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace hx {

struct Philox4x32 {
    static constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u;   // round multipliers
    static constexpr uint32_t kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;   // key increments

    __host__ __device__ static void round(uint32_t c[4], const uint32_t k[2]) {
        const uint64_t p0 = static_cast<uint64_t>(kM0) * c[0];
        const uint64_t p1 = static_cast<uint64_t>(kM1) * c[2];
        const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
        const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
        const uint32_t out[4] = {hi1 ^ c[1] ^ k[0], lo1, hi0 ^ c[3] ^ k[1], lo0};
        for (int i = 0; i < 4; ++i) c[i] = out[i];
    }
    // ten rounds; the key is bumped before every round after the first
    __host__ __device__ static void block(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
        uint32_t c[4] = {ctr[0], ctr[1], ctr[2], ctr[3]};
        uint32_t k[2] = {key[0], key[1]};
        round(c, k);
        for (int r = 1; r < 10; ++r) {
            k[0] += kW0;
            k[1] += kW1;
            round(c, k);
        }
        for (int i = 0; i < 4; ++i) out[i] = c[i];
    }
};

// One stream (nrnran123.cpp: setids, setseq, ipick, dblpick, negexp).
struct Stream123 {
    uint32_t c[4] = {0, 0, 0, 0};
    uint32_t r[4] = {0, 0, 0, 0};
    int which = 0;
    uint32_t global_index = 0;

    __host__ __device__ void refill() {
        const uint32_t key[2] = {global_index, 0};
        Philox4x32::block(c, key, r);
    }
    __host__ __device__ void set_ids(uint32_t id1, uint32_t id2, uint32_t id3) {
        c[1] = id3;
        c[2] = id1;
        c[3] = id2;
    }
    __host__ __device__ void set_seq(uint32_t seq, int w) {
        which = (w < 0 || w > 3) ? 0 : w;
        c[0] = seq;
        refill();
    }
    __host__ __device__ void step_counter() {   // 128-bit increment, word 0 lowest
        for (int i = 0; i < 4; ++i)
            if (++c[i] != 0) break;
    }
    __host__ __device__ uint32_t pick() {
        const uint32_t v = r[which++];
        if (which > 3) {
            which = 0;
            step_counter();
            refill();
        }
        return v;
    }
    // uniform on (0, 1): (u + 1) / (2^32 + 1)
    __host__ __device__ double uniform() {
        constexpr double kShift = 1.0 / 4294967297.0;
        return (static_cast<double>(pick()) + 1.0) * kShift;
    }
    // exponential with mean 1
    __host__ __device__ double negexp() { return -log(uniform()); }
    // the state as kWords words (device copies of a stream)
    static constexpr int kWords = 10;
    __host__ __device__ void save(unsigned* w) const {
        for (int i = 0; i < 4; ++i) { w[i] = c[i]; w[4 + i] = r[i]; }
        w[8] = static_cast<unsigned>(which);
        w[9] = global_index;
    }
    __host__ __device__ void load(const unsigned* w) {
        for (int i = 0; i < 4; ++i) { c[i] = w[i]; r[i] = w[4 + i]; }
        which = static_cast<int>(w[8]);
        global_index = w[9];
    }
};

}  // namespace hx
