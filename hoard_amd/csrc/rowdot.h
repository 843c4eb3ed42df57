// Row dot products for K-quant rows staged in LDS, computed by an aligned
// group of 8 lanes per row.  Each lane takes 1/8 of every super-block with
// 16-byte LDS reads (the 8 lanes of a group read one contiguous 128-byte span,
// so a wave's reads are bank-conflict free), forms exact integer partial sums
// with v_dot4_i32_i8, and the group adds them with a 3-step DPP butterfly.
// The fp32 block terms are then accumulated over super-blocks in block order,
// exactly as the CPU path does, so the row value is bit-identical to it.
#pragma once

#include "qblocks.h"
#include "wave.h"

namespace hoard {

// Q8_K activation block as staged in LDS: quants first so every 16-byte read
// of them is 16-byte aligned (same fields as ggml's block_q8_K).
struct Q8L {
    int32_t qs[64];
    int16_t bsums[16];
    float d;
    int32_t pad[3];
};
static_assert(sizeof(Q8L) == 304, "Q8L is 19 x 16 bytes");

// Wave quantisation of 256 floats to Q8_K (ggml quantize_row_q8_K semantics:
// largest |x| with its sign, first index on ties; iscale = -127/max;
// q = min(127, nearest_int(iscale*x)); d = 1/iscale; all-zero block -> 0).
__device__ __forceinline__ float wave_quantize_q8l_regs(const float v[4], Q8L *out);
// Returns the block's scale d (in every lane).
__device__ __forceinline__ float wave_quantize_q8l(const float *x, Q8L *out) {
    const int lane = threadIdx.x & 63;
    const float4 v4 = *reinterpret_cast<const float4 *>(x + 4 * lane);
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    return wave_quantize_q8l_regs(v, out);
}

// One Q4_K row of nb super-blocks (16-byte aligned in LDS) dotted with x.
// t = lane & 7.  Lane t covers quant bytes [16t, 16t+16) of every block, i.e.
// 16 elements of sub-block 2*(t/2) (low nibbles) and of 2*(t/2)+1 (high).
__device__ __forceinline__ float g8_row_q4k(const uint8_t *row, const Q8L *x, int nb, int t) {
    const int c = t >> 1, h = t & 1;
    float acc = 0.0f, accm = 0.0f;
#pragma unroll
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + b * kQ4KBytes;
        const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
        const uint4 q = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * t);
        const Q8L &xb = x[b];
        const uint4 xl = *reinterpret_cast<const uint4 *>(&xb.qs[16 * c + 4 * h]);
        const uint4 xh = *reinterpret_cast<const uint4 *>(&xb.qs[16 * c + 8 + 4 * h]);
        int lo = 0, hi = 0;
        lo = sdot4(q.x & 0x0f0f0f0fu, xl.x, lo);
        lo = sdot4(q.y & 0x0f0f0f0fu, xl.y, lo);
        lo = sdot4(q.z & 0x0f0f0f0fu, xl.z, lo);
        lo = sdot4(q.w & 0x0f0f0f0fu, xl.w, lo);
        hi = sdot4((q.x >> 4) & 0x0f0f0f0fu, xh.x, hi);
        hi = sdot4((q.y >> 4) & 0x0f0f0f0fu, xh.y, hi);
        hi = sdot4((q.z >> 4) & 0x0f0f0f0fu, xh.z, hi);
        hi = sdot4((q.w >> 4) & 0x0f0f0f0fu, xh.w, hi);
        int sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, hd.y, hd.z, hd.w, sc0, m0);
        q4k_scale_min(2 * c + 1, hd.y, hd.z, hd.w, sc1, m1);
        int isum = sc0 * lo + sc1 * hi;
        int msum = h ? 0
                     : m0 * ((int)xb.bsums[4 * c] + (int)xb.bsums[4 * c + 1]) +
                           m1 * ((int)xb.bsums[4 * c + 2] + (int)xb.bsums[4 * c + 3]);
        isum = group8_sum(isum);
        msum = group8_sum(msum);
        const float d = half_bits_to_float(hd.x & 0xffffu) * xb.d;
        const float dm = half_bits_to_float(hd.x >> 16) * xb.d;
        acc = acc + d * (float)isum;
        accm = accm + dm * (float)msum;
    }
    return acc - accm;
}

// One Q5_K row of nb super-blocks (16-byte aligned in LDS) dotted with x:
// g8_row_q4k with the fifth bit of each quant from qh.  Lane t covers quant
// bytes [16t, 16t+16) (chunk t/2, positions l = 16(t&1) .. +15) and the qh
// bytes of the same positions, bits 2(t/2) and 2(t/2)+1.
__device__ __forceinline__ float g8_row_q5k(const uint8_t *row, const Q8L *x, int nb, int t) {
    const int c = t >> 1, h = t & 1;
    float acc = 0.0f, accm = 0.0f;
#pragma unroll
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + b * kQ5KBytes;
        const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
        const uint4 qh = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * h);
        const uint4 q = *reinterpret_cast<const uint4 *>(blk + 48 + 16 * t);
        const Q8L &xb = x[b];
        const uint4 xl = *reinterpret_cast<const uint4 *>(&xb.qs[16 * c + 4 * h]);
        const uint4 xh = *reinterpret_cast<const uint4 *>(&xb.qs[16 * c + 8 + 4 * h]);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w}, hw[4] = {qh.x, qh.y, qh.z, qh.w};
        const uint32_t xlw[4] = {xl.x, xl.y, xl.z, xl.w}, xhw[4] = {xh.x, xh.y, xh.z, xh.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            lo = sdot4((qw[k] & 0x0f0f0f0fu) | (((hw[k] >> (2 * c)) & 0x01010101u) << 4), xlw[k], lo);
            hi = sdot4(((qw[k] >> 4) & 0x0f0f0f0fu) | (((hw[k] >> (2 * c + 1)) & 0x01010101u) << 4), xhw[k], hi);
        }
        int sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, hd.y, hd.z, hd.w, sc0, m0);
        q4k_scale_min(2 * c + 1, hd.y, hd.z, hd.w, sc1, m1);
        int isum = sc0 * lo + sc1 * hi;
        int msum = h ? 0
                     : m0 * ((int)xb.bsums[4 * c] + (int)xb.bsums[4 * c + 1]) +
                           m1 * ((int)xb.bsums[4 * c + 2] + (int)xb.bsums[4 * c + 3]);
        isum = group8_sum(isum);
        msum = group8_sum(msum);
        const float d = half_bits_to_float(hd.x & 0xffffu) * xb.d;
        const float dm = half_bits_to_float(hd.x >> 16) * xb.d;
        acc = acc + d * (float)isum;
        accm = accm + dm * (float)msum;
    }
    return acc - accm;
}

// One Q6_K row of nb super-blocks (2-byte aligned in LDS) dotted with x.
// Lane t covers positions l in [8*(t&3), +8) of half t>>2 for all four
// 32-element quarters: 32 of the block's 256 elements.
__device__ __forceinline__ float g8_row_q6k(const uint8_t *row, const Q8L *x, int nb, int t) {
    const int n = t >> 2, lh = t & 3;
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + b * kQ6KBytes;
        const Q8L &xb = x[b];
        int s[4] = {0, 0, 0, 0}, z[4] = {0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t A = lds_u32(blk + 64 * n + 8 * lh + 4 * w);
            const uint32_t B = lds_u32(blk + 64 * n + 32 + 8 * lh + 4 * w);
            const uint32_t C = lds_u32(blk + 128 + 32 * n + 8 * lh + 4 * w);
            const uint32_t q[4] = {
                (A & 0x0f0f0f0fu) | ((C & 0x03030303u) << 4),
                (B & 0x0f0f0f0fu) | (((C >> 2) & 0x03030303u) << 4),
                ((A >> 4) & 0x0f0f0f0fu) | (((C >> 4) & 0x03030303u) << 4),
                ((B >> 4) & 0x0f0f0f0fu) | (((C >> 6) & 0x03030303u) << 4),
            };
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t xw = (uint32_t)xb.qs[32 * n + 8 * i + 2 * lh + w];
                s[i] = sdot4(q[i], xw, s[i]);
                z[i] = sdot4(0x01010101u, xw, z[i]);
            }
        }
        int isum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int g = 8 * n + 2 * i + (lh >> 1);
            isum += (int)(int8_t)blk[192 + g] * (s[i] - 32 * z[i]);
        }
        isum = group8_sum(isum);
        const uint32_t dbits = (uint32_t)blk[208] | ((uint32_t)blk[209] << 8);
        acc = acc + (half_bits_to_float(dbits) * xb.d) * (float)isum;
    }
    return acc;
}

// Q6_K rows whose start has the same 4-byte alignment (0 or 2) in every lane
// of the wave: 210-byte blocks alternate between the two, so each block takes
// one scalar branch to a body with a compile-time shift instead of per-lane
// alignment tests.
template <int SH>
__device__ __forceinline__ uint32_t lds_u32_c(const uint8_t *p) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(p - SH);
    if constexpr (SH == 0)
        return w[0];
    else
        return __builtin_amdgcn_alignbyte(w[1], w[0], SH);
}

template <int SH>
__device__ __forceinline__ int q6k_block_isum_g8(const uint8_t *blk, const Q8L &xb, int n, int lh) {
    int s[4] = {0, 0, 0, 0}, z[4] = {0, 0, 0, 0};
    uint32_t A[2], B[2], C[2];
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        A[w] = lds_u32_c<SH>(blk + 64 * n + 8 * lh + 4 * w);
        B[w] = lds_u32_c<SH>(blk + 64 * n + 32 + 8 * lh + 4 * w);
        C[w] = lds_u32_c<SH>(blk + 128 + 32 * n + 8 * lh + 4 * w);
    }
#pragma unroll
    for (int w = 0; w < 2; ++w) {
        const uint32_t q[4] = {
            (A[w] & 0x0f0f0f0fu) | ((C[w] & 0x03030303u) << 4),
            (B[w] & 0x0f0f0f0fu) | (((C[w] >> 2) & 0x03030303u) << 4),
            ((A[w] >> 4) & 0x0f0f0f0fu) | (((C[w] >> 4) & 0x03030303u) << 4),
            ((B[w] >> 4) & 0x0f0f0f0fu) | (((C[w] >> 6) & 0x03030303u) << 4),
        };
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t xw = (uint32_t)xb.qs[32 * n + 8 * i + 2 * lh + w];
            s[i] = sdot4(q[i], xw, s[i]);
            z[i] = sdot4(0x01010101u, xw, z[i]);
        }
    }
    int isum = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int g = 8 * n + 2 * i + (lh >> 1);
        isum += (int)(int8_t)blk[192 + g] * (s[i] - 32 * z[i]);
    }
    return isum;
}

template <int NB>
__device__ __forceinline__ float g8_row_q6k_u(const uint8_t *row, const Q8L *x, int t) {
    const int n = t >> 2, lh = t & 3;
    const uint32_t al = (uint32_t)__builtin_amdgcn_readfirstlane((int)(reinterpret_cast<uintptr_t>(row) & 3u));
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const uint8_t *blk = row + b * kQ6KBytes;
        int isum;
        if (((al + 2u * b) & 3u) == 0u)
            isum = q6k_block_isum_g8<0>(blk, x[b], n, lh);
        else
            isum = q6k_block_isum_g8<2>(blk, x[b], n, lh);
        isum = group8_sum(isum);
        const uint32_t dbits = (uint32_t)blk[208] | ((uint32_t)blk[209] << 8);
        acc = acc + (half_bits_to_float(dbits) * x[b].d) * (float)isum;
    }
    return acc;
}

// Row dot for a compile-time type and block count: the block loop unrolls
// fully, so every LDS read of the row is issued before the first dot product
// needs it, and a kernel instantiates only the bodies it uses.
template <int TYPE, int NB>
__device__ __forceinline__ float g8_row(const uint8_t *row, const Q8L *x, int t) {
    static_assert(TYPE == kTypeQ4K || TYPE == kTypeQ6K, "Q4_K or Q6_K rows");
    if constexpr (TYPE == kTypeQ4K)
        return g8_row_q4k(row, x, NB, t);
    else
        return g8_row_q6k(row, x, NB, t);
}

// ---------------------------------------------------------------------------
// One lane per super-block.  A row of NB <= G super-blocks is handled by an
// aligned group of G lanes, lane t taking block t whole: its integer sums are
// complete in-lane, and the fp32 block terms are then added in block order by
// a chain through the group's lanes (row_shr:1 makes lane i read lane i - 1).
// The activation block a lane needs is the same for every row, so it is held
// in registers across rows.

// Q8_K activation block held in registers by the lane that owns it.
struct Q8Reg {
    uint4 q[16];  // 256 int8 quants
    int bs[8];    // bsums[2s] + bsums[2s+1]: sum of the 32 quants of sub-block s
    float d;
};

__device__ __forceinline__ void load_q8reg(const Q8L &x, Q8Reg &r) {
    const uint4 *q = reinterpret_cast<const uint4 *>(x.qs);
#pragma unroll
    for (int i = 0; i < 16; ++i) r.q[i] = q[i];
    const uint4 b0 = *reinterpret_cast<const uint4 *>(&x.bsums[0]);
    const uint4 b1 = *reinterpret_cast<const uint4 *>(&x.bsums[8]);
    const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
    for (int s = 0; s < 8; ++s) r.bs[s] = (int)(int16_t)(w[s] & 0xffffu) + (int)(int16_t)(w[s] >> 16);
    r.d = x.d;
}

constexpr int kDppRowShr1 = 0x111;  // lane i reads lane i - 1 of its row

// Ordered fp32 sum over lanes 0..nb-1 of each aligned group: lane t holds v.
// Returns 0 + v0 + v1 + ... (left to right) in lane nb-1 of the group.
template <int NB>
__device__ __forceinline__ float group_chain_sum(float v, int t) {
    float acc = 0.0f + v;
#pragma unroll
    for (int s = 1; s < NB; ++s) {
        const float prev = dpp_f<kDppRowShr1>(acc);
        acc = t == s ? prev + v : acc;
    }
    return acc;
}

// Q4_K super-block (16-byte aligned) against the lane's activation block:
// the integer sums isum = sum_s sc_s * dot_s and msum = sum_s m_s * bsum_s.
__device__ __forceinline__ void q4k_block_sums(const uint8_t *blk, const Q8Reg &x, uint32_t &dm_bits, int &isum,
                                               int &msum) {
    const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
    uint4 q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * i);
    dm_bits = hd.x;
    const uint32_t sw[3] = {hd.y, hd.z, hd.w};
    auto byte = [&](int i) -> int { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    isum = 0;
    msum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // 64-element chunk j: sub-blocks 2j (low nibbles) and 2j+1 (high)
        const uint32_t qw[8] = {q[2 * j].x, q[2 * j].y, q[2 * j].z, q[2 * j].w,
                                q[2 * j + 1].x, q[2 * j + 1].y, q[2 * j + 1].z, q[2 * j + 1].w};
        const uint32_t xl[8] = {x.q[4 * j].x, x.q[4 * j].y, x.q[4 * j].z, x.q[4 * j].w,
                                x.q[4 * j + 1].x, x.q[4 * j + 1].y, x.q[4 * j + 1].z, x.q[4 * j + 1].w};
        const uint32_t xh[8] = {x.q[4 * j + 2].x, x.q[4 * j + 2].y, x.q[4 * j + 2].z, x.q[4 * j + 2].w,
                                x.q[4 * j + 3].x, x.q[4 * j + 3].y, x.q[4 * j + 3].z, x.q[4 * j + 3].w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            lo = sdot4(qw[k] & 0x0f0f0f0fu, xl[k], lo);
            hi = sdot4((qw[k] >> 4) & 0x0f0f0f0fu, xh[k], hi);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int s = 2 * j + h;
            int sc, mn;
            if (s < 4) {
                sc = byte(s) & 63;
                mn = byte(s + 4) & 63;
            } else {
                sc = (byte(s + 4) & 0x0f) | ((byte(s - 4) >> 6) << 4);
                mn = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
            }
            isum += sc * (h ? hi : lo);
            msum += mn * x.bs[s];
        }
    }
}

// One Q4_K row of NB super-blocks (16-byte aligned) dotted with the
// activation; valid in lane NB-1 of the lane's group.
template <int NB>
__device__ __forceinline__ float lpb_row_q4k(const uint8_t *row, const Q8Reg &x, int t) {
    float p = 0.0f, pm = 0.0f;
    if (t < NB) {
        uint32_t dm;
        int isum, msum;
        q4k_block_sums(row + t * kQ4KBytes, x, dm, isum, msum);
        const float d = half_bits_to_float(dm & 0xffffu) * x.d;
        const float dmin = half_bits_to_float(dm >> 16) * x.d;
        p = d * (float)isum;
        pm = dmin * (float)msum;
    }
    const float acc = group_chain_sum<NB>(p, t);
    const float accm = group_chain_sum<NB>(pm, t);
    return acc - accm;
}

// The same sums with the activation block read from memory (LDS) as it is
// used, for a lane that dots it with one row only: nothing is held across
// rows, which keeps the register count low.
// Split: the second half's loads are not hoisted above the first half's
// dots, which caps the registers the block holds at once (the batched gate/up
// kernel: 151 -> 93 VGPRs, a fourth wave per SIMD).
template <bool Split = false>
__device__ __forceinline__ void q4k_block_sums_mem(const uint8_t *blk, const Q8L &x, uint32_t &dm_bits, int &isum,
                                                   int &msum) {
    const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
    dm_bits = hd.x;
    const uint32_t sw[3] = {hd.y, hd.z, hd.w};
    auto byte = [&](int i) -> int { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    const uint4 *xq = reinterpret_cast<const uint4 *>(x.qs);
    isum = 0;
    msum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // 64-element chunk j: sub-blocks 2j (low nibbles) and 2j+1 (high)
        if (Split && j == 2) asm volatile("" ::: "memory");
        const uint4 q0 = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * j);
        const uint4 q1 = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * j);
        const uint4 x0 = xq[4 * j], x1 = xq[4 * j + 1], x2 = xq[4 * j + 2], x3 = xq[4 * j + 3];
        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            lo = sdot4(qw[k] & 0x0f0f0f0fu, xl[k], lo);
            hi = sdot4((qw[k] >> 4) & 0x0f0f0f0fu, xh[k], hi);
        }
        const uint32_t bw = *reinterpret_cast<const uint32_t *>(&x.bsums[4 * j]);
        const uint32_t bw1 = *reinterpret_cast<const uint32_t *>(&x.bsums[4 * j + 2]);
        const int bsl = (int)(int16_t)(bw & 0xffffu) + (int)(int16_t)(bw >> 16);
        const int bsh = (int)(int16_t)(bw1 & 0xffffu) + (int)(int16_t)(bw1 >> 16);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int s = 2 * j + h;
            int sc, mn;
            if (s < 4) {
                sc = byte(s) & 63;
                mn = byte(s + 4) & 63;
            } else {
                sc = (byte(s + 4) & 0x0f) | ((byte(s - 4) >> 6) << 4);
                mn = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
            }
            isum += sc * (h ? hi : lo);
            msum += mn * (h ? bsh : bsl);
        }
    }
}

// lpb_row_q4k with the lane's activation block xb read from memory.
template <int NB, bool Split = false>
__device__ __forceinline__ float lpb_row_q4k_mem(const uint8_t *row, const Q8L &xb, int t) {
    float p = 0.0f, pm = 0.0f;
    if (t < NB) {
        uint32_t dm;
        int isum, msum;
        q4k_block_sums_mem<Split>(row + t * kQ4KBytes, xb, dm, isum, msum);
        const float d = half_bits_to_float(dm & 0xffffu) * xb.d;
        const float dmin = half_bits_to_float(dm >> 16) * xb.d;
        p = d * (float)isum;
        pm = dmin * (float)msum;
    }
    const float acc = group_chain_sum<NB>(p, t);
    const float accm = group_chain_sum<NB>(pm, t);
    return acc - accm;
}

// Q5_K super-block (16-byte aligned: d/dmin and the Q4_K-packed scales in the
// first 16 bytes, qh[32], qs[128]) against an activation block in memory: the
// Q4_K sums with each quant's fifth bit taken from qh (bit 2j of qh[l] for
// the low nibbles of chunk j, bit 2j+1 for the high ones).
__device__ __forceinline__ void q5k_block_sums_mem(const uint8_t *blk, const Q8L &x, uint32_t &dm_bits, int &isum,
                                                   int &msum) {
    const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
    const uint4 h0 = *reinterpret_cast<const uint4 *>(blk + 16);
    const uint4 h1 = *reinterpret_cast<const uint4 *>(blk + 32);
    const uint32_t qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
    dm_bits = hd.x;
    const uint32_t sw[3] = {hd.y, hd.z, hd.w};
    auto byte = [&](int i) -> int { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    const uint4 *xq = reinterpret_cast<const uint4 *>(x.qs);
    isum = 0;
    msum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 q0 = *reinterpret_cast<const uint4 *>(blk + 48 + 32 * j);
        const uint4 q1 = *reinterpret_cast<const uint4 *>(blk + 64 + 32 * j);
        const uint4 x0 = xq[4 * j], x1 = xq[4 * j + 1], x2 = xq[4 * j + 2], x3 = xq[4 * j + 3];
        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
        int lo = 0, hi = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t ql = (qw[k] & 0x0f0f0f0fu) | (((qh[k] >> (2 * j)) & 0x01010101u) << 4);
            const uint32_t qu = ((qw[k] >> 4) & 0x0f0f0f0fu) | (((qh[k] >> (2 * j + 1)) & 0x01010101u) << 4);
            lo = sdot4(ql, xl[k], lo);
            hi = sdot4(qu, xh[k], hi);
        }
        const uint32_t bw = *reinterpret_cast<const uint32_t *>(&x.bsums[4 * j]);
        const uint32_t bw1 = *reinterpret_cast<const uint32_t *>(&x.bsums[4 * j + 2]);
        const int bsl = (int)(int16_t)(bw & 0xffffu) + (int)(int16_t)(bw >> 16);
        const int bsh = (int)(int16_t)(bw1 & 0xffffu) + (int)(int16_t)(bw1 >> 16);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int s = 2 * j + h;
            int sc, mn;
            if (s < 4) {
                sc = byte(s) & 63;
                mn = byte(s + 4) & 63;
            } else {
                sc = (byte(s + 4) & 0x0f) | ((byte(s - 4) >> 6) << 4);
                mn = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
            }
            isum += sc * (h ? hi : lo);
            msum += mn * (h ? bsh : bsl);
        }
    }
}

// One Q5_K row of NB super-blocks (16-byte aligned), one lane per block with
// the lane's activation block xb read from memory; valid in lane NB-1.
template <int NB>
__device__ __forceinline__ float lpb_row_q5k_mem(const uint8_t *row, const Q8L &xb, int t) {
    float p = 0.0f, pm = 0.0f;
    if (t < NB) {
        uint32_t dm;
        int isum, msum;
        q5k_block_sums_mem(row + t * kQ5KBytes, xb, dm, isum, msum);
        const float d = half_bits_to_float(dm & 0xffffu) * xb.d;
        const float dmin = half_bits_to_float(dm >> 16) * xb.d;
        p = d * (float)isum;
        pm = dmin * (float)msum;
    }
    const float acc = group_chain_sum<NB>(p, t);
    const float accm = group_chain_sum<NB>(pm, t);
    return acc - accm;
}

// Q3_K super-block (2-byte aligned: hmask[32], qs[64], 12 scale bytes, d)
// against an activation block in memory: isum = sum_g (sc_g - 32) *
// sum_{16} q3*q8, with q3 = q2 + 4*h - 4 and sum q3*q8 = sum (q2 + 4h)*q8 - 4*bsum.
// kRolled: the halves one after the other (fewer live registers, for kernels
// that keep it beside wait loops); otherwise both unrolled.
// The block's words come from the 4-byte aligned address at or below it
// (word i = alignbyte(w[i + 1], w[i], sh), no branch on the alignment), and
// that address is formed by pointer arithmetic, so a block in LDS is read with
// ds_read rather than through generic (flat) addresses.
template <bool kRolled>
__device__ __forceinline__ int q3k_block_isum_mem(const uint8_t *blk, const Q8L &x) {
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(blk - sh);
    auto word = [&](int i) -> uint32_t { return __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh); };
    const uint32_t s0 = word(24), s1 = word(25), s2 = word(26);  // scales at byte 96
    const uint4 *xq = reinterpret_cast<const uint4 *>(x.qs);
    int isum = 0;
    auto half = [&](int n) {  // elements 128n .. 128n + 127
        uint32_t qw[8], hm[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            qw[t] = word(8 + 8 * n + t);  // qs at byte 32
            hm[t] = word(t);              // hmask at byte 0
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // elements 128n + 32j + l: quant words 32n + 8j + t
            const uint4 x0 = xq[8 * n + 2 * j], x1 = xq[8 * n + 2 * j + 1];
            const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int a = 0; a < 2; ++a) {
                int sd = 0;
#pragma unroll
                for (int t = 4 * a; t < 4 * a + 4; ++t) {
                    const uint32_t v = ((qw[t] >> (2 * j)) & 0x03030303u) | (((hm[t] >> (4 * n + j)) & 0x01010101u) << 2);
                    sd = sdot4(v, xw[t], sd);
                }
                const int g = 8 * n + 2 * j + a;
                isum += q3k_scale(g, s0, s1, s2) * (sd - 4 * (int)x.bsums[g]);
            }
        }
    };
    if constexpr (kRolled) {
#pragma unroll 1
        for (int n = 0; n < 2; ++n) half(n);
    } else {
        half(0);
        half(1);
    }
    return isum;
}

// One Q3_K row of NB super-blocks, one lane per block with the lane's
// activation block xb read from memory; valid in lane NB-1.
template <int NB, bool kRolled = false>
__device__ __forceinline__ float lpb_row_q3k_mem(const uint8_t *row, const Q8L &xb, int t) {
    float p = 0.0f;
    if (t < NB) {
        const uint8_t *blk = row + t * kQ3KBytes;
        const int isum = q3k_block_isum_mem<kRolled>(blk, xb);
        const uint32_t dbits = (uint32_t)blk[108] | ((uint32_t)blk[109] << 8);
        p = (half_bits_to_float(dbits) * xb.d) * (float)isum;
    }
    return group_chain_sum<NB>(p, t);
}

// Wave max of non-negative IEEE floats held as their bit patterns (for such
// values the order of the patterns is the order of the values, so integer
// max needs no NaN handling): unsigned max inside each 16-lane row, then
// across rows through row_bcast:15 (rows 1, 3 take lane 15 / 47) and
// row_bcast:31 (rows 2, 3 take lane 31); lane 63 ends with the result.
__device__ __forceinline__ unsigned wave_max_bits(unsigned u) {
    u = max(u, (unsigned)dpp_i<kDppQuadXor1>((int)u));
    u = max(u, (unsigned)dpp_i<kDppQuadXor2>((int)u));
    u = max(u, (unsigned)dpp_i<kDppRowHalfMirror>((int)u));
    u = max(u, (unsigned)dpp_i<kDppRowMirror>((int)u));
    u = max(u, (unsigned)__builtin_amdgcn_update_dpp((int)u, (int)u, kDppRowBcast15, 0xa, 0xf, false));
    u = max(u, (unsigned)__builtin_amdgcn_update_dpp((int)u, (int)u, kDppRowBcast31, 0xc, 0xf, false));
    return (unsigned)__builtin_amdgcn_readlane((int)u, 63);
}

// Q8_K quantisation of 256 values held 4 per lane (lane l: elements 4l..4l+3).
// The scale comes from the first element (lowest index) of largest magnitude;
// NaN elements never set it.  Magnitudes are compared as bit patterns (NaN
// patterns cleared to 0 first), which orders them as the values would be, so
// the wave max is an integer max and the element that holds it is found with
// one compare per element, one ballot and one read of its lane.
__device__ __forceinline__ float wave_quantize_q8l_regs(const float v[4], Q8L *out) {
    const int lane = threadIdx.x & 63;
    unsigned b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned m = __float_as_uint(v[i]) & 0x7fffffffu;
        b[i] = m <= 0x7f800000u ? m : 0u;
    }
    const unsigned am = wave_max_bits(max(max(b[0], b[1]), max(b[2], b[3])));
    if (am == 0u) {  // all zero (or NaN): d = 0, q = 0
        out->qs[lane] = 0;
        if (lane < 16) out->bsums[lane] = 0;
        if (lane == 0) out->d = 0.0f;
        return 0.0f;
    }
    const bool h0 = b[0] == am, h1 = b[1] == am, h2 = b[2] == am, h3 = b[3] == am;
    const float c = h0 ? v[0] : (h1 ? v[1] : (h2 ? v[2] : v[3]));
    const int src = __ffsll((unsigned long long)__builtin_amdgcn_ballot_w64(h0 | h1 | h2 | h3)) - 1;
    const float mval = readlane_f(c, src);
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
    s = group4_sum(s);
    if ((lane & 3) == 0) out->bsums[lane >> 2] = (int16_t)s;
    const float d = 1.0f / iscale;
    if (lane == 0) out->d = d;
    return d;
}

}  // namespace hoard
