// Batched expert stage for M tokens (speculative verify / small prefill):
// tokens are grouped by expert so every selected expert's weights are read
// once per call, and the expert products run on int8 MFMA.
//
// Counterpart of ggml_mul_mat_id over the slot pool with per-token ids
// (src/run_specloop.cpp:126-139; all-resident form src/run_m1.cpp:97-108)
// followed by the weighted sum over the selected experts.
//
// Exactness: each v_mfma_i32_16x16x32_i8 covers one 32-element Q4_K
// sub-block (or, with half of A zeroed, one 16-element Q6_K group) of 16 rows
// against 16 tokens' Q8_K quants, so it yields exactly the integer sub-block
// sums the per-token path forms with dot4.  The sub-block scales, the min
// term and the fp32 block terms are then applied per (row, token) in the
// per-token path's order, so each token's output is bit-identical to a
// single-token call.
//
// MFMA lane layout (K = 32): lane l supplies A[l % 16][8 (l / 16) .. +7]
// (8 int8 of row l % 16) and B[8 (l / 16) .. +7][l % 16] (8 int8 of token
// column l % 16), and receives D[4 (l / 16) + i][l % 16], i = 0..3.
#include "kernels.h"
#include "qblocks.h"
#include "rowdot.h"

namespace hoard {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kTile = 16;                   // weight rows per MFMA tile
constexpr int kMaxTok = kBatchedMaxTokens;  // token columns per MFMA tile
constexpr int kMaxExperts = 1024;
static_assert(sizeof(Q8L) == kQ8LBytes, "Q8_K block size shared with the host");

__device__ __forceinline__ Q8L *q8(uint8_t *p) { return reinterpret_cast<Q8L *>(p); }

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

// Q4_K sub-block scale and min for sub-block s from a super-block header.
__device__ __forceinline__ void q4k_sm(const uint4 &hd, int s, int &sc, int &mn) {
    const uint32_t sw[3] = {hd.y, hd.z, hd.w};
    auto byte = [&](int i) -> int { return (int)((sw[i >> 2] >> (8 * (i & 3))) & 0xffu); };
    if (s < 4) {
        sc = byte(s) & 63;
        mn = byte(s + 4) & 63;
    } else {
        sc = (byte(s + 4) & 0x0f) | ((byte(s - 4) >> 6) << 4);
        mn = (byte(s + 4) >> 4) | ((byte(s) >> 6) << 4);
    }
}

// One 16-row Q4_K tile (row r at W + r*rb, NBLK super-blocks) against the
// lane's token column.  xq: the token's Q8_K blocks, or null for an empty
// column.  Returns, for rows 4(l/16)+i, acc_i - accm_i as the per-token path
// forms them.
template <int NBLK>
__device__ __forceinline__ void tile_q4k(const uint8_t *W, size_t rb, const Q8L *xq, float out[4]) {
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
    for (int b = 0; b < NBLK; ++b) {
        const uint8_t *blk_r = W + (size_t)r * rb + (size_t)b * kQ4KBytes;
        uint2 qa[4];
#pragma unroll
        for (int jc = 0; jc < 4; ++jc) qa[jc] = *reinterpret_cast<const uint2 *>(blk_r + 16 + 32 * jc + 8 * q);
        uint4 hd[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) hd[i] = *reinterpret_cast<const uint4 *>(W + (size_t)(4 * q + i) * rb + (size_t)b * kQ4KBytes);
        long xb[8];
        int bs[8];
        float xd = 0.0f;
        if (xq) {
            const Q8L &x = xq[b];
#pragma unroll
            for (int s = 0; s < 8; ++s) xb[s] = *reinterpret_cast<const long *>(&x.qs[8 * s + 2 * q]);
            const uint4 b0 = *reinterpret_cast<const uint4 *>(&x.bsums[0]);
            const uint4 b1 = *reinterpret_cast<const uint4 *>(&x.bsums[8]);
            const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
            for (int s = 0; s < 8; ++s) bs[s] = (int)(int16_t)(w[s] & 0xffffu) + (int)(int16_t)(w[s] >> 16);
            xd = x.d;
        } else {
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                xb[s] = 0;
                bs[s] = 0;
            }
        }
        int isum[4] = {0, 0, 0, 0}, msum[4] = {0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const long a = (s & 1) ? hi_nibbles(qa[s >> 1]) : lo_nibbles(qa[s >> 1]);
            const v4i d = mfma_16x16x32(a, xb[s]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int sc, mn;
                q4k_sm(hd[i], s, sc, mn);
                isum[i] += sc * d[i];
                msum[i] += mn * bs[s];
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float dd = half_bits_to_float(hd[i].x & 0xffffu) * xd;
            const float dm = half_bits_to_float(hd[i].x >> 16) * xd;
            acc[i] = acc[i] + dd * (float)isum[i];
            accm[i] = accm[i] + dm * (float)msum[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = acc[i] - accm[i];
}

// 8 bytes at a 2-byte aligned LDS address.
__device__ __forceinline__ uint2 lds_u64_a2(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3u);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
}

// One 16-row Q6_K tile staged in LDS (row r at T + r*rb).  Element e of a
// super-block: half n = e/128, quarter qd = (e/32)%4, l = e%32; its 6-bit
// value is the (qd/2)-th nibble of ql[64n + 32(qd%2) + l] with bits
// 2qd..2qd+1 of qh[32n + l] on top, minus 32.  The -32 is applied through the
// token's 16-element sums (bsums), as the per-token path's zero-point term.
template <int NBLK>
__device__ __forceinline__ void tile_q6k(const uint8_t *T, size_t rb, const Q8L *xq, float out[4]) {
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const bool first_half = q < 2;  // elements 0..15 of each 32-element range
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
    for (int b = 0; b < NBLK; ++b) {
        const uint8_t *blk_r = T + (size_t)r * rb + (size_t)b * kQ6KBytes;
        int bs[16];
        float xd = 0.0f;
        if (xq) {
            const uint4 b0 = *reinterpret_cast<const uint4 *>(&xq[b].bsums[0]);
            const uint4 b1 = *reinterpret_cast<const uint4 *>(&xq[b].bsums[8]);
            const uint32_t w[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                bs[2 * g] = (int)(int16_t)(w[g] & 0xffffu);
                bs[2 * g + 1] = (int)(int16_t)(w[g] >> 16);
            }
            xd = xq[b].d;
        } else {
#pragma unroll
            for (int g = 0; g < 16; ++g) bs[g] = 0;
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
            const long xb = xq ? *reinterpret_cast<const long *>(&xq[b].qs[8 * s + 2 * q]) : 0;
            const v4i d0 = mfma_16x16x32(first_half ? a : 0, xb);
            const v4i d1 = mfma_16x16x32(first_half ? 0 : a, xb);
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
            acc[i] = acc[i] + (half_bits_to_float(dbits) * xd) * (float)isum[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = acc[i];
}

// -- prep: Q8_K of every token's fx; grouping of (token, slot) by expert -----
__global__ __launch_bounds__(64) void prep_kernel(BatchedArgs a) {
    const int nb = a.n_embd / QK;
    if ((int)blockIdx.x < a.M * nb) {
        const int t = blockIdx.x / nb, b = blockIdx.x % nb;
        wave_quantize_q8l(a.fx + (size_t)t * a.n_embd + (size_t)b * QK, q8(a.q8x) + (size_t)t * nb + b);
        return;
    }
    // last workgroup: group the (token, slot) pairs by expert.  A token selects
    // an expert at most once, so a per-expert bitmask of tokens orders each
    // group by token; groups are numbered in ascending expert id.
    __shared__ unsigned mask[kMaxExperts];
    __shared__ int uidx[kMaxExperts];
    __shared__ int wave_total;
    const int lane = threadIdx.x, E = a.E, P = a.M * a.k;
    for (int e = lane; e < E; e += 64) mask[e] = 0u;
    __syncthreads();
    for (int p = lane; p < P; p += 64) {
        int e = a.sel[p];
        if (e < 0 || e >= E) e = 0;  // the router maps NaN logits to expert 0 with a NaN weight
        atomicOr(&mask[e], 1u << (p / a.k));
    }
    __syncthreads();
    // ascending prefix count of used experts: lane owns a contiguous run of experts
    const int per = (E + 63) / 64, e0 = lane * per;
    int cnt = 0;
    for (int e = e0; e < e0 + per && e < E; ++e) cnt += mask[e] ? 1 : 0;
    int incl = cnt;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    int u = incl - cnt;
    for (int e = e0; e < e0 + per && e < E; ++e) {
        const unsigned m = mask[e];
        a.hist[e] = (unsigned)__popc(m);
        if (m) {
            uidx[e] = u;
            a.uexp[u] = e;
            a.ucount[u] = __popc(m);
            ++u;
        }
    }
    if (lane == 63) wave_total = incl;
    __syncthreads();
    for (int p = lane; p < P; p += 64) {
        const int t = p / a.k, j = p % a.k;
        int e = a.sel[p];
        if (e < 0 || e >= E) e = 0;
        const int g = uidx[e], c = __popc(mask[e] & ((1u << t) - 1u));
        a.utok[g * kMaxTok + c] = t;
        a.uslot[g * kMaxTok + c] = j;
    }
    if (lane == 0) a.n_unique[0] = wave_total;
}

// -- gate/up: one 16-row tile of gate (wave 0) and up (wave 1) of one expert --
template <int NB>
__global__ __launch_bounds__(128) void gateup_mfma_kernel(BatchedArgs a) {
    const int u = blockIdx.y;
    if (u >= a.n_unique[0]) return;
    __shared__ float gu[2][kTile][kMaxTok];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = a.uexp[u], m = min(a.ucount[u], kMaxTok);
    const int row0 = blockIdx.x * kTile;
    const size_t rb = (size_t)NB * kQ4KBytes;
    const uint8_t *W = (wave ? a.up + (size_t)e * a.ustride : a.gate + (size_t)e * a.gstride) + (size_t)row0 * rb;
    const int c = lane & 15;
    const Q8L *xq = c < m ? q8(a.q8x) + (size_t)a.utok[u * kMaxTok + c] * NB : nullptr;
    float v[4];
    tile_q4k<NB>(W, rb, xq, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) gu[wave][4 * (lane >> 4) + i][c] = v[i];
    __syncthreads();
    for (int i = threadIdx.x; i < kTile * kMaxTok; i += blockDim.x) {
        const int r = i / kMaxTok, cc = i % kMaxTok;
        if (cc < m) {
            const float g = gu[0][r][cc], uu = gu[1][r][cc];
            a.hbuf[((size_t)u * kMaxTok + cc) * a.n_ff + row0 + r] = g / (1.0f + expf(-g)) * uu;
        }
    }
}

// -- Q8_K of h per (expert, token) ---------------------------------------------
__global__ __launch_bounds__(64) void quant_h_kernel(BatchedArgs a) {
    const int u = blockIdx.z, c = blockIdx.y, b = blockIdx.x;
    if (u >= a.n_unique[0] || c >= min(a.ucount[u], kMaxTok)) return;
    const int nbh = a.n_ff / QK;
    const size_t uc = (size_t)u * kMaxTok + c;
    wave_quantize_q8l(a.hbuf + uc * a.n_ff + (size_t)b * QK, q8(a.q8h) + uc * nbh + b);
}

// -- down: one 16-row tile of one expert; y to Y[token][slot] -------------------
template <int TD, int NBH>
__global__ __launch_bounds__(64) void down_mfma_kernel(BatchedArgs a) {
    const int u = blockIdx.y;
    if (u >= a.n_unique[0]) return;
    const int lane = threadIdx.x & 63, c = lane & 15;
    const int e = a.uexp[u], m = min(a.ucount[u], kMaxTok);
    const int row0 = blockIdx.x * kTile;
    const Q8L *xq = c < m ? q8(a.q8h) + ((size_t)u * kMaxTok + c) * NBH : nullptr;
    float v[4];
    if constexpr (TD == kTypeQ4K) {
        const size_t rb = (size_t)NBH * kQ4KBytes;
        tile_q4k<NBH>(a.down + (size_t)e * a.dstride + (size_t)row0 * rb, rb, xq, v);
    } else {
        // stage the tile's 16 rows (contiguous in the expert) in LDS: Q6_K rows
        // are only 2-byte aligned, which LDS reads handle with alignbyte
        constexpr size_t rb = (size_t)NBH * kQ6KBytes;
        constexpr int kBytes = (int)(kTile * rb);
        __shared__ __align__(16) uint8_t tile[kBytes + 16];
        const uint8_t *src = a.down + (size_t)e * a.dstride + (size_t)row0 * rb;
        for (int i = lane; i < kBytes / 16; i += 64)
            reinterpret_cast<uint4 *>(tile)[i] = reinterpret_cast<const uint4 *>(src)[i];
        for (int i = (kBytes / 16) * 16 + lane; i < kBytes; i += 64) tile[i] = src[i];
        __syncthreads();
        tile_q6k<NBH>(tile, rb, xq, v);
    }
    if (c < m) {
        const int t = a.utok[u * kMaxTok + c], j = a.uslot[u * kMaxTok + c];
        float *y = a.ybuf + ((size_t)t * a.k + j) * a.n_embd + row0;
#pragma unroll
        for (int i = 0; i < 4; ++i) y[4 * (lane >> 4) + i] = v[i];
    }
}

// -- combine: out[t][d] = (sum_j w[t][j] * y[t][j][d]) + res[t][d], j ascending --
__global__ __launch_bounds__(256) void combine_kernel(BatchedArgs a) {
    const int t = blockIdx.y;
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= a.n_embd) return;
    float acc = 0.0f;
    for (int j = 0; j < a.k; ++j)
        acc = acc + a.wsel[t * a.k + j] * a.ybuf[((size_t)t * a.k + j) * a.n_embd + d];
    a.out[(size_t)t * a.n_embd + d] = acc + a.res[(size_t)t * a.n_embd + d];
}

}  // namespace

bool batched_shape_compiled(int gu_type, int n_embd, int d_type, int n_ff) {
    return gu_type == kTypeQ4K && n_embd == 2048 && (n_ff == 768 || n_ff == 1024 || n_ff == 512) &&
           (d_type == kTypeQ4K || d_type == kTypeQ6K);
}

hipError_t launch_batched(const BatchedArgs &a, hipStream_t s) {
    if (a.M < 1 || a.M > kMaxTok || a.n_embd != 2048 || a.gu_type != kTypeQ4K) return hipErrorInvalidValue;
    const int nb = a.n_embd / QK, nbh = a.n_ff / QK;
    const int umax = a.E < a.M * a.k ? a.E : a.M * a.k;
    hipLaunchKernelGGL(prep_kernel, dim3(a.M * nb + 1), dim3(64), 0, s, a);
    hipLaunchKernelGGL(gateup_mfma_kernel<8>, dim3(a.n_ff / kTile, umax), dim3(128), 0, s, a);
    hipLaunchKernelGGL(quant_h_kernel, dim3(nbh, kMaxTok, umax), dim3(64), 0, s, a);
    const dim3 dg(a.n_embd / kTile, umax);
#define HOARD_DOWN(T, N)                                                              \
    if (a.d_type == T && nbh == N) {                                                  \
        hipLaunchKernelGGL((down_mfma_kernel<T, N>), dg, dim3(64), 0, s, a);          \
    } else
    HOARD_DOWN(kTypeQ6K, 3) HOARD_DOWN(kTypeQ6K, 2) HOARD_DOWN(kTypeQ6K, 4) HOARD_DOWN(kTypeQ4K, 4)
    HOARD_DOWN(kTypeQ4K, 3) HOARD_DOWN(kTypeQ4K, 2) { return hipErrorInvalidValue; }
#undef HOARD_DOWN
    hipLaunchKernelGGL(combine_kernel, dim3((a.n_embd + 255) / 256, a.M), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace hoard
