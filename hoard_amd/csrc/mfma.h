// int8 MFMA tiles for K-quant rows (v_mfma_i32_16x16x32_i8), shared by the
// batched kernels.
//
// Exactness: one MFMA covers one 32-element Q4_K sub-block (or, with half of A
// zeroed, one 16-element Q6_K group) of 16 rows against 16 token columns'
// Q8_K quants, so it yields exactly the integer sub-block sums the per-token
// path forms with dot4.  The sub-block scales, the min term and the fp32 block
// terms are then applied per (row, token) in the per-token path's order, so a
// token's result is bit-identical to a single-token call.
//
// MFMA lane layout (K = 32): lane l supplies A[l % 16][8 (l / 16) .. +7]
// (8 int8 of row l % 16) and B[8 (l / 16) .. +7][l % 16] (8 int8 of token
// column l % 16), and receives D[4 (l / 16) + i][l % 16], i = 0..3.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qblocks.h"
#include "rowdot.h"

namespace hoard {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_16x16x32(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

__device__ __forceinline__ long lo_nibbles(uint2 w) {
    return (long)(((unsigned long)(w.y & 0x0f0f0f0fu) << 32) | (w.x & 0x0f0f0f0fu));
}
__device__ __forceinline__ long hi_nibbles(uint2 w) {
    return (long)(((unsigned long)((w.y >> 4) & 0x0f0f0f0fu) << 32) | ((w.x >> 4) & 0x0f0f0f0fu));
}

// The 6-bit scales (sc) and mins (mn) of a Q4_K header, four per word: byte
// s of sc[0] / mn[0] belongs to sub-block s, byte s of sc[1] / mn[1] to s + 4.
__device__ __forceinline__ void q4k_scales_packed(const uint4 &hd, uint32_t sc[2], uint32_t mn[2]) {
    sc[0] = hd.y & 0x3f3f3f3fu;
    mn[0] = hd.z & 0x3f3f3f3fu;
    sc[1] = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
    mn[1] = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
}

__device__ __forceinline__ int byte_of(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); }

// 8 bytes at a 2-byte aligned LDS address.
__device__ __forceinline__ uint2 lds_u64_a2(const uint8_t *p) {
    // aligned base by pointer arithmetic, so that the compiler still sees an
    // LDS pointer and emits ds_read rather than flat loads
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(p - sh);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

// Operands of one super-block for one lane: its row's quants for the four
// 64-element chunks, the headers of the four rows whose results it receives,
// and its token's Q8_K quants, 16-element sums and scale.
struct Q4Ops {
    uint2 qa[4];
    uint4 hd[4];
    long xb[8];
    uint4 b0, b1;
    float xd;
};

// Rows of a tile of fewer than 16 rows repeat (row index & RM); the repeated
// rows' results are not used.
template <int RM>
__device__ __forceinline__ void q4_load(const uint8_t *W, size_t rb, const Q8L *xq, int b, Q4Ops &o) {
    const int lane = threadIdx.x & 63, r = lane & 15 & RM, q = lane >> 4;
    const uint8_t *blk_r = W + (size_t)r * rb + (size_t)b * kQ4KBytes;
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) o.qa[jc] = *reinterpret_cast<const uint2 *>(blk_r + 16 + 32 * jc + 8 * q);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o.hd[i] = *reinterpret_cast<const uint4 *>(W + (size_t)((4 * q + i) & RM) * rb + (size_t)b * kQ4KBytes);
    const Q8L &x = xq[b];
#pragma unroll
    for (int s = 0; s < 8; ++s) o.xb[s] = *reinterpret_cast<const long *>(&x.qs[8 * s + 2 * q]);
    o.b0 = *reinterpret_cast<const uint4 *>(&x.bsums[0]);
    o.b1 = *reinterpret_cast<const uint4 *>(&x.bsums[8]);
    o.xd = x.d;
}

__device__ __forceinline__ void q4_compute(const Q4Ops &o, float acc[4], float accm[4]) {
    const uint32_t bw[8] = {o.b0.x, o.b0.y, o.b0.z, o.b0.w, o.b1.x, o.b1.y, o.b1.z, o.b1.w};
    int bs[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) bs[s] = (int)(int16_t)(bw[s] & 0xffffu) + (int)(int16_t)(bw[s] >> 16);
    uint32_t sc[4][2], mn[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) q4k_scales_packed(o.hd[i], sc[i], mn[i]);
    int isum[4] = {0, 0, 0, 0}, msum[4] = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const long a = (s & 1) ? hi_nibbles(o.qa[s >> 1]) : lo_nibbles(o.qa[s >> 1]);
        const v4i d = mfma_16x16x32(a, o.xb[s]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            isum[i] += byte_of(sc[i][s >> 2], s & 3) * d[i];
            msum[i] += byte_of(mn[i][s >> 2], s & 3) * bs[s];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float dd = half_bits_to_float(o.hd[i].x & 0xffffu) * o.xd;
        const float dm = half_bits_to_float(o.hd[i].x >> 16) * o.xd;
        acc[i] = acc[i] + dd * (float)isum[i];
        accm[i] = accm[i] + dm * (float)msum[i];
    }
}

// One 16-row Q4_K tile (row r at W + r*rb, NBLK super-blocks; with RM = 7 an
// 8-row tile, rows 8-15 repeating rows 0-7) against the lane's token column.
// xq: the token's Q8_K blocks; a column without a token reads another
// column's token and its results are not used (the MFMA's output columns are
// independent), which keeps the loads free of divergent branches.  Returns,
// for rows 4(l/16)+i, acc_i - accm_i as the per-token path forms them.
template <int NBLK, int RM = 15>
__device__ __forceinline__ void tile_q4k(const uint8_t *W, size_t rb, const Q8L *xq, float out[4]) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
    for (int b = 0; b < NBLK; ++b) {
        Q4Ops o;
        q4_load<RM>(W, rb, xq, b, o);
        q4_compute(o, acc, accm);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = acc[i] - accm[i];
}

// A token's Q8_K operands of one super-block for one lane (see q4_load).
struct Q6X {
    long xb[8];
    uint4 b0, b1;
    float xd;
};

__device__ __forceinline__ void q6_load_x(const Q8L *xq, int b, Q6X &o) {
    const int q = (threadIdx.x & 63) >> 4;
    const Q8L &x = xq[b];
#pragma unroll
    for (int s = 0; s < 8; ++s) o.xb[s] = *reinterpret_cast<const long *>(&x.qs[8 * s + 2 * q]);
    o.b0 = *reinterpret_cast<const uint4 *>(&x.bsums[0]);
    o.b1 = *reinterpret_cast<const uint4 *>(&x.bsums[8]);
    o.xd = x.d;
}

// One 16-row Q6_K tile staged in LDS (row r at T + r*rb).  Element e of a
// super-block: half n = e/128, quarter qd = (e/32)%4, l = e%32; its 6-bit
// value is the (qd/2)-th nibble of ql[64n + 32(qd%2) + l] with bits
// 2qd..2qd+1 of qh[32n + l] on top, minus 32.  The -32 is applied through the
// token's 16-element sums (bsums), as the per-token path's zero-point term.
// One super-block b of a 16-row Q6_K tile staged in LDS (row r at T + r*rb)
// against the token column whose operands are x; adds its fp32 block term to
// acc in block order.
__device__ __forceinline__ void q6_tile_block(const uint8_t *T, size_t rb, int b, const Q6X &x, float acc[4]) {
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const bool first_half = q < 2;  // elements 0..15 of each 32-element range
    const uint8_t *blk_r = T + (size_t)r * rb + (size_t)b * kQ6KBytes;
    const uint32_t w[8] = {x.b0.x, x.b0.y, x.b0.z, x.b0.w, x.b1.x, x.b1.y, x.b1.z, x.b1.w};
    int bs[16];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        bs[2 * g] = (int)(int16_t)(w[g] & 0xffffu);
        bs[2 * g + 1] = (int)(int16_t)(w[g] >> 16);
    }
    int isum[4] = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 8; ++s) {  // 32-element range s: groups 2s and 2s+1
        const int n = s >> 2, qd = s & 3;
        const uint2 ql = lds_u64_a2(blk_r + 64 * n + 32 * (qd & 1) + 8 * q);
        const uint2 qh = lds_u64_a2(blk_r + 128 + 32 * n + 8 * q);
        const int nsh = 4 * (qd >> 1), hsh = 2 * qd;
        const uint32_t v0 = ((ql.x >> nsh) & 0x0f0f0f0fu) | (((qh.x >> hsh) & 0x03030303u) << 4);
        const uint32_t v1 = ((ql.y >> nsh) & 0x0f0f0f0fu) | (((qh.y >> hsh) & 0x03030303u) << 4);
        const long a = (long)(((unsigned long)v1 << 32) | v0);
        const v4i d0 = mfma_16x16x32(first_half ? a : 0, x.xb[s]);
        const v4i d1 = mfma_16x16x32(first_half ? 0 : a, x.xb[s]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint8_t *blk_i = T + (size_t)(4 * q + i) * rb + (size_t)b * kQ6KBytes;
            const int sc0 = (int)(int8_t)blk_i[192 + 2 * s], sc1 = (int)(int8_t)blk_i[193 + 2 * s];
            isum[i] += sc0 * (d0[i] - 32 * bs[2 * s]) + sc1 * (d1[i] - 32 * bs[2 * s + 1]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint8_t *blk_i = T + (size_t)(4 * q + i) * rb + (size_t)b * kQ6KBytes;
        const uint32_t dbits = (uint32_t)blk_i[208] | ((uint32_t)blk_i[209] << 8);
        acc[i] = acc[i] + (half_bits_to_float(dbits) * x.xd) * (float)isum[i];
    }
}

template <int NBLK>
__device__ __forceinline__ void tile_q6k(const uint8_t *T, size_t rb, const Q8L *xq, float out[4]) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
    for (int b = 0; b < NBLK; ++b) {
        Q6X cur;
        q6_load_x(xq, b, cur);
        q6_tile_block(T, rb, b, cur, acc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = acc[i];
}

// One super-block b of a 16-row Q4_K tile (row r at W + r*rb) against the
// token column whose operands are x (the fields q4_load fills); adds its fp32
// block terms to acc / accm in block order.
__device__ __forceinline__ void q4_tile_block(const uint8_t *W, size_t rb, int b, const Q6X &x, float acc[4],
                                              float accm[4]) {
    Q4Ops o;
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const uint8_t *blk_r = W + (size_t)r * rb + (size_t)b * kQ4KBytes;
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) o.qa[jc] = *reinterpret_cast<const uint2 *>(blk_r + 16 + 32 * jc + 8 * q);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o.hd[i] = *reinterpret_cast<const uint4 *>(W + (size_t)(4 * q + i) * rb + (size_t)b * kQ4KBytes);
#pragma unroll
    for (int s = 0; s < 8; ++s) o.xb[s] = x.xb[s];
    o.b0 = x.b0;
    o.b1 = x.b1;
    o.xd = x.xd;
    q4_compute(o, acc, accm);
}

}  // namespace hoard
