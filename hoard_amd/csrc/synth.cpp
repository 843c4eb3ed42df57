// Deterministic synthetic MoE layers (host only).  Counter-based splitmix64:
// word i of a tensor is mix(key ^ (i * 0xD1B54A32D192ED03)), so generation is
// order-free and parallel.  Block layouts are ggml's block_q{3,4,5,6}_K.
#include "hoard_synth.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

inline uint64_t word(uint64_t key, uint64_t i) { return mix64(key ^ (i * 0xD1B54A32D192ED03ull)); }

// uniform in (0, 1): 53 random bits, offset by half an ulp so 0 never occurs
inline double unit(uint64_t u) { return ((double)(u >> 11) + 0.5) * (1.0 / 9007199254740992.0); }

inline double normal(uint64_t key, uint64_t i) {
    const double u1 = unit(word(key, 2 * i)), u2 = unit(word(key, 2 * i + 1));
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

// fp32 -> IEEE binary16, round to nearest even
uint16_t to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) return (uint16_t)(sign | (uint32_t)std::nearbyint(std::fabs(f) * 16777216.0f));
    uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

constexpr int kQ3K = 11, kQ4K = 12, kQ5K = 13, kQ6K = 14;
constexpr uint64_t kSaltD = 0x5bd1e9955bd1e995ull;
constexpr uint64_t kSaltM = 0x27d4eb2f165667c5ull;

size_t block_bytes(int type) {
    switch (type) {
    case kQ3K: return 110;
    case kQ4K: return 144;
    case kQ5K: return 176;
    case kQ6K: return 210;
    default: return 0;
    }
}

void fill_range(int type, uint64_t key, uint8_t *dst, size_t b0, size_t b1, float dstd) {
    const size_t bb = block_bytes(type);
    for (size_t b = b0; b < b1; ++b) {
        uint8_t *blk = dst + b * bb;
        uint64_t w[26];
        // random bytes: 140 (Q4_K scales + nibbles), 172 (Q5_K scales, qh, qs),
        // 208 (Q6_K ql, qh, scales), 108 (Q3_K hmask, qs, scales)
        const int nrand = type == kQ4K ? 140 : type == kQ5K ? 172 : type == kQ6K ? 208 : 108;
        for (int i = 0; i < (nrand + 7) / 8; ++i) w[i] = word(key, b * 32 + (uint64_t)i);
        const uint8_t *rb = reinterpret_cast<const uint8_t *>(w);
        const uint16_t d = to_half((float)std::fabs(normal(key ^ kSaltD, b) * dstd));
        if (type == kQ4K || type == kQ5K) {
            const uint16_t dm = to_half((float)std::fabs(normal(key ^ kSaltM, b) * dstd));
            std::memcpy(blk, &d, 2);
            std::memcpy(blk + 2, &dm, 2);
            std::memcpy(blk + 4, rb, (size_t)nrand);
        } else {
            std::memcpy(blk, rb, (size_t)nrand);
            std::memcpy(blk + nrand, &d, 2);
        }
    }
}

template <class F>
void parallel_for(size_t n, size_t grain, F &&f) {
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (n < grain * 2 || nt == 1) {
        f(0, n);
        return;
    }
    nt = (unsigned)std::min<size_t>(nt, (n + grain - 1) / grain);
    std::vector<std::thread> ts;
    const size_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const size_t a = t * chunk, b = std::min(n, a + chunk);
        if (a >= b) break;
        ts.emplace_back([=, &f] { f(a, b); });
    }
    for (auto &t : ts) t.join();
}

}  // namespace

extern "C" {

uint64_t hoard_synth_key(uint32_t config, uint32_t seed, uint32_t layer, uint32_t tensor,
                         uint32_t expert) {
    uint64_t k = mix64(0x486f617264ull ^ config);
    k = mix64(k ^ seed);
    k = mix64(k ^ layer);
    k = mix64(k ^ tensor);
    return mix64(k ^ expert);
}

size_t hoard_synth_expert_bytes(int type, int rows, int cols) {
    return (size_t)rows * (size_t)(cols / 256) * block_bytes(type);
}

int hoard_synth_fill_blocks(int type, uint64_t key, void *dst, size_t nblocks, float dstd) {
    if (block_bytes(type) == 0 || !dst) return -1;
    uint8_t *p = static_cast<uint8_t *>(dst);
    parallel_for(nblocks, 4096, [&](size_t a, size_t b) { fill_range(type, key, p, a, b, dstd); });
    return 0;
}

void hoard_synth_fill_normal(uint64_t key, float *dst, size_t n, float std) {
    parallel_for(n, 1 << 16, [&](size_t a, size_t b) {
        for (size_t i = a; i < b; ++i) dst[i] = (float)(normal(key, i) * std);
    });
}

int hoard_synth_fill_experts(int type, uint32_t config, uint32_t seed, uint32_t layer,
                             uint32_t tensor, int n_expert, int rows, int cols, void *dst,
                             float dstd) {
    if (block_bytes(type) == 0 || !dst || cols % 256 || rows <= 0 || n_expert <= 0) return -1;
    const size_t nb = (size_t)rows * (cols / 256);
    const size_t stride = nb * block_bytes(type);
    uint8_t *p = static_cast<uint8_t *>(dst);
    parallel_for((size_t)n_expert, 1, [&](size_t a, size_t b) {
        for (size_t e = a; e < b; ++e)
            fill_range(type, hoard_synth_key(config, seed, layer, tensor, (uint32_t)e), p + e * stride,
                       0, nb, dstd);
    });
    return 0;
}

}  // extern "C"
