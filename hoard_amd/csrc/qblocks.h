// Device-side ggml K-quant super-block codecs for gfx950 (wave64).
//
// Formats (ggml-common.h, copied verbatim into the reference's expert slots,
// src/run_moe_stream.cpp:177-183):
//   block_q4_K 144 B: d fp16 | dmin fp16 | 12 B packed 6-bit scales+mins | 128 B nibbles
//   block_q6_K 210 B: ql[128] | qh[64] | int8 scales[16] | d fp16
//   block_q5_K 176 B: d fp16 | dmin fp16 | 12 B scales+mins as Q4_K | qh[32] | qs[128]
//   block_q3_K 110 B: hmask[32] | qs[64] (2-bit) | 12 B packed 6-bit scales | d fp16
//   block_q8_K 292 B: d f32 | int8 qs[256] | int16 bsums[16]   (activation side)
// Dot products are exact integer sums per super-block (v_dot4_i32_i8) scaled
// in fp32 exactly as the CPU path does: per block (d_w*d_x)*isum, and for
// Q4_K / Q5_K also (dmin_w*d_x)*msum, accumulated over blocks in block order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hoard {

constexpr int QK = 256;
constexpr int kTypeQ3K = 11;
constexpr int kTypeQ4K = 12;
constexpr int kTypeQ5K = 13;
constexpr int kTypeQ6K = 14;
constexpr int kQ3KBytes = 110;
constexpr int kQ4KBytes = 144;
constexpr int kQ5KBytes = 176;
constexpr int kQ6KBytes = 210;

// Bytes of one super-block of a supported type (0 for any other).
__host__ __device__ constexpr int kquant_block_bytes(int type) {
    return type == kTypeQ4K ? kQ4KBytes
                            : type == kTypeQ6K ? kQ6KBytes
                                               : type == kTypeQ5K ? kQ5KBytes : type == kTypeQ3K ? kQ3KBytes : 0;
}
// Types whose blocks carry a min term (value = d*sc*q - dmin*m).
__host__ __device__ constexpr bool kquant_has_min(int type) { return type == kTypeQ4K || type == kTypeQ5K; }

template <int T>
struct QType;
template <>
struct QType<kTypeQ4K> {
    static constexpr int bytes = kQ4KBytes;
    static constexpr bool has_min = true;
};
template <>
struct QType<kTypeQ6K> {
    static constexpr int bytes = kQ6KBytes;
    static constexpr bool has_min = false;
};
template <>
struct QType<kTypeQ5K> {
    static constexpr int bytes = kQ5KBytes;
    static constexpr bool has_min = true;
};
template <>
struct QType<kTypeQ3K> {
    static constexpr int bytes = kQ3KBytes;
    static constexpr bool has_min = false;
};

// Q8_K activation block as held in LDS (same field order as ggml's block_q8_K).
struct Q8Block {
    float d;
    int32_t qs[64];     // 256 int8, four per word
    int16_t bsums[16];  // sum of each group of 16 quants
};
static_assert(sizeof(Q8Block) == 292, "block_q8_K is 292 bytes");

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// 32-bit little-endian word at a 2-byte aligned LDS address.
__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3u);
    if (sh == 0) return w[0];
    return __builtin_amdgcn_alignbyte(w[1], w[0], sh);
}

// ggml's nearest_int (round to nearest even through the fp32 adder).
__device__ __forceinline__ int nearest_int(float f) {
    const float v = f + 12582912.0f;
    return (__float_as_int(v) & 0x007fffff) - 0x00400000;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Q4_K scale/min pair for sub-block s from the 12 packed bytes (three words).
__device__ __forceinline__ void q4k_scale_min(int s, uint32_t s0, uint32_t s1, uint32_t s2, int &sc,
                                              int &mn) {
    // bytes 0..3 = s0, 4..7 = s1, 8..11 = s2
    auto byte = [&](int i) -> int {
        const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
        return (int)((w >> (8 * (i & 3))) & 0xffu);
    };
    if (s < 4) {
        sc = byte(s) & 63;
        mn = byte(s + 4) & 63;
    } else {
        sc = (byte(s + 4) & 0x0f) | ((byte(s - 4) >> 6) << 4);
        mn = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
    }
}

// One Q4_K block (4-byte aligned in LDS) against one Q8_K block.
// t_main = (d*dx)*isum, t_min = (dmin*dx)*msum.
__device__ __forceinline__ void q4k_block_terms(const uint8_t *blk, const Q8Block &x, float &t_main,
                                                float &t_min) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(blk);
    const uint32_t dm = w[0];
    const uint32_t s0 = w[1], s1 = w[2], s2 = w[3];
    const uint32_t *qs = w + 4;
    int isum = 0, msum = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        int lo = 0, hi = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t q = qs[8 * c + t];
            lo = sdot4(q & 0x0f0f0f0fu, (uint32_t)x.qs[16 * c + t], lo);
            hi = sdot4((q >> 4) & 0x0f0f0f0fu, (uint32_t)x.qs[16 * c + 8 + t], hi);
        }
        int sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, s0, s1, s2, sc0, m0);
        q4k_scale_min(2 * c + 1, s0, s1, s2, sc1, m1);
        isum += sc0 * lo + sc1 * hi;
        msum += m0 * ((int)x.bsums[4 * c] + (int)x.bsums[4 * c + 1]) +
                m1 * ((int)x.bsums[4 * c + 2] + (int)x.bsums[4 * c + 3]);
    }
    const float d = half_bits_to_float(dm & 0xffffu) * x.d;
    const float dmin = half_bits_to_float(dm >> 16) * x.d;
    t_main = d * (float)isum;
    t_min = dmin * (float)msum;
}

// One Q6_K block (2-byte aligned in LDS) against one Q8_K block.
// value = d*sc[g]*(q-32); sum (q-32)*q8 over a group = sum q*q8 - 32*bsum.
__device__ __forceinline__ void q6k_block_terms(const uint8_t *blk, const Q8Block &x, float &t_main,
                                                float &t_min) {
    int isum = 0;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        uint32_t q[4][8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t wl = lds_u32(blk + 64 * n + 4 * t);
            const uint32_t wl2 = lds_u32(blk + 64 * n + 32 + 4 * t);
            const uint32_t wh = lds_u32(blk + 128 + 32 * n + 4 * t);
            q[0][t] = (wl & 0x0f0f0f0fu) | ((wh & 0x03030303u) << 4);
            q[1][t] = (wl2 & 0x0f0f0f0fu) | (((wh >> 2) & 0x03030303u) << 4);
            q[2][t] = ((wl >> 4) & 0x0f0f0f0fu) | (((wh >> 4) & 0x03030303u) << 4);
            q[3][t] = ((wl2 >> 4) & 0x0f0f0f0fu) | (((wh >> 6) & 0x03030303u) << 4);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                int s = 0;
#pragma unroll
                for (int t = 4 * a; t < 4 * a + 4; ++t)
                    s = sdot4(q[i][t], (uint32_t)x.qs[32 * n + 8 * i + t], s);
                const int g = 8 * n + 2 * i + a;
                const int sc = (int)(int8_t)blk[192 + g];
                isum += sc * (s - 32 * (int)x.bsums[g]);
            }
        }
    }
    const uint32_t dbits = (uint32_t)blk[208] | ((uint32_t)blk[209] << 8);
    t_main = (half_bits_to_float(dbits) * x.d) * (float)isum;
    t_min = 0.0f;
}

// One Q5_K block (4-byte aligned in LDS) against one Q8_K block: Q4_K's
// terms with the fifth bit of every quant from qh (bit 2c / 2c+1 of qh[l] for
// the low / high nibbles of chunk c).
__device__ __forceinline__ void q5k_block_terms(const uint8_t *blk, const Q8Block &x, float &t_main,
                                                float &t_min) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(blk);
    const uint32_t dm = w[0];
    const uint32_t s0 = w[1], s1 = w[2], s2 = w[3];
    const uint32_t *qh = w + 4;
    const uint32_t *qs = w + 12;
    int isum = 0, msum = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        int lo = 0, hi = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t q = qs[8 * c + t], h = qh[t];
            const uint32_t ql = (q & 0x0f0f0f0fu) | (((h >> (2 * c)) & 0x01010101u) << 4);
            const uint32_t qu = ((q >> 4) & 0x0f0f0f0fu) | (((h >> (2 * c + 1)) & 0x01010101u) << 4);
            lo = sdot4(ql, (uint32_t)x.qs[16 * c + t], lo);
            hi = sdot4(qu, (uint32_t)x.qs[16 * c + 8 + t], hi);
        }
        int sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, s0, s1, s2, sc0, m0);
        q4k_scale_min(2 * c + 1, s0, s1, s2, sc1, m1);
        isum += sc0 * lo + sc1 * hi;
        msum += m0 * ((int)x.bsums[4 * c] + (int)x.bsums[4 * c + 1]) +
                m1 * ((int)x.bsums[4 * c + 2] + (int)x.bsums[4 * c + 3]);
    }
    const float d = half_bits_to_float(dm & 0xffffu) * x.d;
    const float dmin = half_bits_to_float(dm >> 16) * x.d;
    t_main = d * (float)isum;
    t_min = dmin * (float)msum;
}

// Signed Q3_K scale g (stored as scale + 32 in 6 bits) from the 12 scale bytes
// held in words s0 (bytes 0..3), s1 (4..7), s2 (8..11).
__device__ __forceinline__ int q3k_scale(int g, uint32_t s0, uint32_t s1, uint32_t s2) {
    const uint32_t lw = (g & 4) ? s1 : s0;                   // byte g % 8
    const int lo = (int)((lw >> (8 * (g & 3) + ((g & 8) ? 4 : 0))) & 0x0fu);
    const int hi = (int)((s2 >> (8 * (g & 3) + 2 * (g >> 2))) & 3u);
    return (lo | (hi << 4)) - 32;
}

// One Q3_K block (2-byte aligned in LDS) against one Q8_K block.  Element
// 128n + 32j + l has q2 = bits 2j..2j+1 of qs[32n + l] and q3 = q2 - 4 unless
// bit 4n+j of hmask[l] is set; sum q3*q8 over a group of 16 is
// sum (q2 + 4*h)*q8 - 4*bsum.
__device__ __forceinline__ void q3k_block_terms(const uint8_t *blk, const Q8Block &x, float &t_main,
                                                float &t_min) {
    const uint32_t s0 = lds_u32(blk + 96), s1 = lds_u32(blk + 100), s2 = lds_u32(blk + 104);
    uint32_t hm[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) hm[t] = lds_u32(blk + 4 * t);
    int isum = 0;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        uint32_t qw[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) qw[t] = lds_u32(blk + 32 + 32 * n + 4 * t);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                int s = 0;
#pragma unroll
                for (int t = 4 * a; t < 4 * a + 4; ++t) {
                    const uint32_t v = ((qw[t] >> (2 * j)) & 0x03030303u) |
                                       (((hm[t] >> (4 * n + j)) & 0x01010101u) << 2);
                    s = sdot4(v, (uint32_t)x.qs[32 * n + 8 * j + t], s);
                }
                const int g = 8 * n + 2 * j + a;
                isum += q3k_scale(g, s0, s1, s2) * (s - 4 * (int)x.bsums[g]);
            }
        }
    }
    const uint32_t dbits = (uint32_t)blk[108] | ((uint32_t)blk[109] << 8);
    t_main = (half_bits_to_float(dbits) * x.d) * (float)isum;
    t_min = 0.0f;
}

template <int T>
__device__ __forceinline__ void block_terms(const uint8_t *blk, const Q8Block &x, float &t_main,
                                            float &t_min) {
    if constexpr (T == kTypeQ4K)
        q4k_block_terms(blk, x, t_main, t_min);
    else if constexpr (T == kTypeQ5K)
        q5k_block_terms(blk, x, t_main, t_min);
    else if constexpr (T == kTypeQ3K)
        q3k_block_terms(blk, x, t_main, t_min);
    else
        q6k_block_terms(blk, x, t_main, t_min);
}

// Row result from its per-block terms in block order, as the CPU path sums.
template <int T>
__device__ __forceinline__ float row_sum(const float *t_main, const float *t_min, int nb) {
    float acc = 0.0f, accm = 0.0f;
    for (int b = 0; b < nb; ++b) {
        acc = acc + t_main[b];
        if constexpr (QType<T>::has_min) accm = accm + t_min[b];
    }
    if constexpr (QType<T>::has_min)
        return acc - accm;
    else
        return acc;
}

// ---------------------------------------------------------------------------
// Wave-level Q8_K quantisation of one 256-element block (64 lanes x 4).
// Largest |x| wins, first index on ties, keeping its sign; iscale = -127/max;
// q = min(127, nearest_int(iscale*x)); d = 1/iscale; all-zero -> d = 0.
// `scale` multiplies x first (1.0f leaves it unchanged; rms-norm passes its
// factor so the product is rounded once, as a stored normed vector would be).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void wave_quantize_q8k(const float *x, Q8Block *out) {
    const int lane = threadIdx.x & 63;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = x[4 * lane + i];
    float amax = 0.0f;
    int idx = 0x7fffffff;
    float mval = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float a = fabsf(v[i]);
        if (a > amax) {
            amax = a;
            idx = 4 * lane + i;
            mval = v[i];
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float oa = __shfl_xor(amax, off);
        const int oi = __shfl_xor(idx, off);
        const float om = __shfl_xor(mval, off);
        if (oa > amax || (oa == amax && oi < idx)) {
            amax = oa;
            idx = oi;
            mval = om;
        }
    }
    if (amax == 0.0f) {
        out->qs[lane] = 0;
        if (lane < 16) out->bsums[lane] = 0;
        if (lane == 0) out->d = 0.0f;
        return;
    }
    const float iscale = -127.0f / mval;
    uint32_t packed = 0;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        int q = nearest_int(iscale * v[i]);
        q = q < 127 ? q : 127;
        s += q;
        packed |= ((uint32_t)(q & 0xff)) << (8 * i);
    }
    out->qs[lane] = (int32_t)packed;
    // groups of 16 elements = 4 consecutive lanes
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    if ((lane & 3) == 0) out->bsums[lane >> 2] = (int16_t)s;
    if (lane == 0) out->d = 1.0f / iscale;
}

}  // namespace hoard
