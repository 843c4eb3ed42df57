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
#include "lds_dma.h"
#include "qblocks.h"
#include "rowdot.h"
#include "router_tail.h"

namespace hoard {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kTile = 16;                   // weight rows per MFMA tile
constexpr int kMaxTok = kBatchedMaxTokens;  // token columns per MFMA tile
constexpr int kMfmaMinTokens = 12;          // smallest expert group computed on MFMA
constexpr int kXChunk = 4;                  // tokens of Q8_K x staged in LDS at a time
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

// The 6-bit scales (sc) and mins (mn) of a Q4_K header, four per word: byte
// s of sc[0] / mn[0] belongs to sub-block s, byte s of sc[1] / mn[1] to s + 4.
__device__ __forceinline__ void q4k_scales_packed(const uint4 &hd, uint32_t sc[2], uint32_t mn[2]) {
    sc[0] = hd.y & 0x3f3f3f3fu;
    mn[0] = hd.z & 0x3f3f3f3fu;
    sc[1] = (hd.w & 0x0f0f0f0fu) | ((hd.y >> 2) & 0x30303030u);
    mn[1] = ((hd.w >> 4) & 0x0f0f0f0fu) | ((hd.z >> 2) & 0x30303030u);
}

__device__ __forceinline__ int byte_of(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xffu); }

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

// 8 bytes at a 2-byte aligned LDS address.
__device__ __forceinline__ uint2 lds_u64_a2(const uint8_t *p) {
    // aligned base by pointer arithmetic, so that the compiler still sees an
    // LDS pointer and emits ds_read rather than flat loads
    const uint32_t sh = (uint32_t)(reinterpret_cast<uintptr_t>(p) & 3u);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(p - sh);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    return make_uint2(__builtin_amdgcn_alignbyte(w1, w0, sh), __builtin_amdgcn_alignbyte(w2, w1, sh));
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
template <int NBLK>
__device__ __forceinline__ void tile_q6k(const uint8_t *T, size_t rb, const Q8L *xq, float out[4]) {
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const bool first_half = q < 2;  // elements 0..15 of each 32-element range
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 1
    for (int b = 0; b < NBLK; ++b) {
        Q6X cur;
        q6_load_x(xq, b, cur);
        const uint8_t *blk_r = T + (size_t)r * rb + (size_t)b * kQ6KBytes;
        const uint32_t w[8] = {cur.b0.x, cur.b0.y, cur.b0.z, cur.b0.w, cur.b1.x, cur.b1.y, cur.b1.z, cur.b1.w};
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
            const v4i d0 = mfma_16x16x32(first_half ? a : 0, cur.xb[s]);
            const v4i d1 = mfma_16x16x32(first_half ? 0 : a, cur.xb[s]);
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
            acc[i] = acc[i] + (half_bits_to_float(dbits) * cur.xd) * (float)isum[i];
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = acc[i];
}

// -- route: router logits, softmax / top-k, Q8_K of fx, grouping by expert ----
// One launch replaces the router kernels and the grouping pass.  A workgroup
// (4 waves) takes kRouteRows router rows against kRouteTok tokens, a wave per
// token and a half-wave per row, with the single-token router's per-row
// accumulation order
// (lane l of 32 owns elements l, l+32, ...; ggml's f32 dot fold).  The last
// workgroup of a token group (device-scope counter) runs the tails of its
// tokens; the last token group's tail workgroup then groups the (token, slot)
// pairs by expert.  Waves with a spare slot quantise fx to Q8_K.
constexpr int kRouteRows = 2;
constexpr int kRouteTok = 4;
constexpr int kRouteN = 2048;  // n_embd of the batched path

// Group the (token, slot) pairs by expert (all threads of the workgroup call
// this).  A token selects an expert at most once, so a per-expert bitmask of
// tokens orders each group by token; groups are numbered in ascending expert
// id.
// With caller ids (ysrc, bad: the grouping workgroup's LDS copies) a pair that
// repeats an earlier id of its token, or whose token has an id out of range,
// joins no group.
__device__ __forceinline__ bool pair_computed(const BatchedArgs &a, const int *ysrc, const int *bad, int p) {
    return !ysrc || (ysrc[p] == p % a.k && !bad[p / a.k]);
}

__device__ void group_by_expert(const BatchedArgs &a, const int *ysrc = nullptr, const int *bad = nullptr) {
    __shared__ unsigned mask[kMaxExperts];
    __shared__ int uidx[kMaxExperts];
    __shared__ int wave_total;
    const int tid = threadIdx.x, nt = blockDim.x, E = a.n_ids, P = a.M * a.k;
    for (int e = tid; e < E; e += nt) mask[e] = 0u;
    __syncthreads();
    for (int p = tid; p < P; p += nt) {
        if (!pair_computed(a, ysrc, bad, p)) continue;
        int e = __hip_atomic_load(a.sel + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (e < 0 || e >= E) e = 0;  // out-of-range selections count as expert 0
        atomicOr(&mask[e], 1u << (p / a.k));
    }
    __syncthreads();
    if (tid < 64) {
        // ascending prefix count of used experts: lane owns a contiguous run of experts
        const int lane = tid, per = (E + 63) / 64, e0 = lane * per;
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
    }
    __syncthreads();
    for (int p = tid; p < P; p += nt) {
        if (!pair_computed(a, ysrc, bad, p)) continue;
        const int t = p / a.k, j = p % a.k;
        int e = __hip_atomic_load(a.sel + p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (e < 0 || e >= E) e = 0;
        const int g = uidx[e], c = __popc(mask[e] & ((1u << t) - 1u));
        a.utok[g * kMaxTok + c] = t;
        a.uslot[g * kMaxTok + c] = j;
    }
    if (tid == 0) a.n_unique[0] = wave_total;
}

__global__ __launch_bounds__(256) void route_kernel(BatchedArgs a) {
    constexpr int n = kRouteN, nb = kRouteN / QK;
    const int E = a.E;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l = lane & 31;
    const int tg = blockIdx.y;
    const int t = tg * kRouteTok + wave;  // this wave's token; its half-waves take one row each
    const int r0 = blockIdx.x * kRouteRows;
    const int nrows = min(kRouteRows, E - r0);
    // the workgroup's token rows and router rows go to LDS in one burst, so
    // that every load is in flight at once; the dot then reads them in the
    // per-lane order the accumulation needs
    __shared__ __align__(16) float xl[kRouteTok][kRouteN];
    __shared__ __align__(16) float wl[kRouteRows][kRouteN];
    if (t < a.M) dma_wave_copy(reinterpret_cast<uint8_t *>(xl[wave]), reinterpret_cast<const uint8_t *>(a.fx + (size_t)t * n),
                               n * (int)sizeof(float));
    {
        const int wbytes = nrows * n * (int)sizeof(float), per = wbytes / 4;  // a quarter per wave
        dma_wave_copy(reinterpret_cast<uint8_t *>(wl[0]) + wave * per,
                      reinterpret_cast<const uint8_t *>(a.router + (size_t)r0 * n) + wave * per, per);
    }
    lds_dma_wait();
    __syncthreads();
    const int row = r0 + (lane >> 5);
    if (t < a.M) {
        const float *x = xl[wave];
        const float *wr = wl[min(lane >> 5, nrows - 1)];
        float acc = 0.0f;
#pragma unroll 16
        for (int i = 0; i < n; i += 32) acc = fmaf(wr[i + l], x[i + l], acc);
        acc = acc + __shfl_xor(acc, 16);
        acc = acc + __shfl_xor(acc, 8);
        acc = acc + __shfl_xor(acc, 4);
        acc = acc + __shfl_xor(acc, 1);
        acc = acc + __shfl_xor(acc, 2);
        if (l == 0 && row < E)
            __hip_atomic_store(a.logits + (size_t)t * E + row, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Q8_K of fx: workgroup i of a token group quantises blocks i, i + gridDim.x, ...
        // of its tokens, so every block is formed whatever the expert count (grid width)
        for (int b = blockIdx.x; b < nb; b += gridDim.x) wave_quantize_q8l(x + b * QK, q8(a.q8x) + (size_t)t * nb + b);
    }
    // Completion protocol without cache-flushing fences: the logits and the
    // tails' sel / wsel are stored at device scope (through to memory, past
    // the per-XCD L2) and read back at device scope; each wave waits for its
    // stores to be acknowledged before its workgroup counts itself done.
    __shared__ int last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(&a.counters[tg], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    for (int tt = wave; tt < kRouteTok; tt += 4) {
        const int tok = tg * kRouteTok + tt;
        if (tok < a.M) router_tail<true>(a.logits, E, a.k, a.renorm, a.sel, a.wsel, tok);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_store(&a.counters[tg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = __hip_atomic_fetch_add(&a.counters[kBatchedCounters - 1], 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == gridDim.y - 1;
    }
    __syncthreads();
    if (!last) return;
    group_by_expert(a);
    if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[kBatchedCounters - 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// -- caller ids: Q8_K of fx (workgroups 0..M-1, a wave per block) and the
// grouping (workgroup M): each pair's first occurrence of its id within the
// token, tokens with an id out of range, then the groups as for routed ids.
// The counterpart of the verify step's mul_mat_id over the slot pool with the
// host's ids (src/run_specloop.cpp:116-139), where a token's padding repeats an
// id with weight 0.
__global__ __launch_bounds__(512) void prep_ids_kernel(BatchedArgs a) {
    constexpr int nb = kRouteN / QK;
    const int wave = threadIdx.x >> 6;
    if ((int)blockIdx.x < a.M) {
        const int t = blockIdx.x;
        for (int b = wave; b < nb; b += 8)
            wave_quantize_q8l(a.fx + (size_t)t * kRouteN + b * QK, q8(a.q8x) + (size_t)t * nb + b);
        return;
    }
    __shared__ int bad_s[kMaxTok];
    __shared__ int ysrc_s[kMaxTok * kMaxK];
    const int tid = threadIdx.x, P = a.M * a.k;
    if (tid < kMaxTok) bad_s[tid] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += blockDim.x) {
        const int t = p / a.k, j = p % a.k;
        const int e = a.sel[p];
        if (e < 0 || e >= a.n_ids) bad_s[t] = 1;
        int first = j;
        for (int i = j - 1; i >= 0; --i)
            if (a.sel[t * a.k + i] == e) first = i;
        ysrc_s[p] = first;
        a.ysrc[p] = first;  // for the combine launch
    }
    __syncthreads();
    if (tid < a.M) a.bad[tid] = bad_s[tid];
    group_by_expert(a, ysrc_s, bad_s);
}

// Expert groups are computed two ways.  A group of fewer than kMfmaMinTokens
// tokens runs token by token with the per-token row dot, whose cost grows with
// the group; a larger group runs on MFMA, whose cost is that of 16 token
// columns whatever the group's size.  Both give the per-token path's bits.
// Weight tiles are contiguous rows of the expert and are copied into LDS in
// one burst.

// A group's expert and size are read together with the group count (u < the
// grid's umax keeps them in bounds): one latency rather than two.  Testing them
// too keeps the compiler from moving their loads after the test (a group
// always has an expert >= 0 and a token).
__device__ __forceinline__ bool load_group(const BatchedArgs &a, int u, int &e, int &m) {
    const int nu = a.n_unique[0];
    e = a.uexp[u];
    m = min(a.ucount[u], kMaxTok);
    return (u < nu) & (e >= 0) & (m >= 1);
}

// Gather the Q8_K rows (nb blocks each) of tokens tok[c0 .. c0+mc) into LDS at
// xs, 16-byte granules spread over the workgroup's nw waves (issued, not
// waited for).
template <int NBX>
__device__ __forceinline__ void gather_tokens(uint8_t *xs, const uint8_t *q8base, const int *tok, int c0, int mc,
                                              int m, int wave, int nw) {
    constexpr int kTokGran = NBX * (int)sizeof(Q8L) / 16;
    int tk[kXChunk];  // uniform indices: scalar loads
#pragma unroll
    for (int i = 0; i < kXChunk; ++i) tk[i] = tok[min(c0 + i, m - 1)];
    const int lane = threadIdx.x & 63, ng = mc * kTokGran;
    for (int k = wave; 64 * k < ng; k += nw) {
        const int p = 64 * k + lane;
        if (p < ng) {
            const int t = p / kTokGran, o = p - t * kTokGran;
            int tt = tk[0];
#pragma unroll
            for (int i = 1; i < kXChunk; ++i) tt = t == i ? tk[i] : tt;
            dma_lanes(xs + 1024 * k, q8base + (size_t)tt * (NBX * sizeof(Q8L)) + 16 * o);
        }
    }
}

// -- gate/up: 8 rows of gate (wave 0) and up (wave 1) of one expert ----------
// Per-token dot: one 8-lane group per row, lane t holding the token's Q8_K
// block t.  MFMA: the 8 rows fill a 16-row tile twice.
template <int NB>
__global__ __launch_bounds__(128, 3) void gateup_kernel(BatchedArgs a) {
    static_assert(NB == 8, "one 8-lane group per row, one lane per super-block");
    constexpr int kRows = 8;
    constexpr int kRowBytes = NB * kQ4KBytes;
    constexpr int kTileBytes = kRows * kRowBytes;
    const int u = blockIdx.y;
    int e, m;
    if (!load_group(a, u, e, m)) return;
    __shared__ __align__(16) uint8_t wt[2][kTileBytes];
    __shared__ __align__(16) uint8_t xs[kXChunk * NB * sizeof(Q8L)];
    __shared__ float gu[2][kRows][kMaxTok];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, t8 = lane & 7, grp = lane >> 3;
    const int row0 = blockIdx.x * kRows;
    const int *tok = a.utok + u * kMaxTok;
    const uint8_t *W = (wave ? a.up + (size_t)e * a.ustride : a.gate + (size_t)e * a.gstride) + (size_t)row0 * kRowBytes;
    if (m >= kMfmaMinTokens) {
        dma_wave_copy(wt[wave], W, kTileBytes);
        const int c = lane & 15;
        const Q8L *xq = q8(a.q8x) + (size_t)tok[c < m ? c : 0] * NB;
        lds_dma_wait();
        float v[4];
        tile_q4k<NB, 7>(wt[wave], kRowBytes, xq, v);
        if (lane < 32) {
#pragma unroll
            for (int i = 0; i < 4; ++i) gu[wave][4 * (lane >> 4) + i][c] = v[i];
        }
    } else {
        // x goes into LDS with the tile, kXChunk tokens at a time: a vector
        // load issued during the compute would queue behind the tile copies
        // of the other workgroups on this CU
        const Q8L *xl = reinterpret_cast<const Q8L *>(xs);
        for (int c0 = 0; c0 < m; c0 += kXChunk) {
            const int mc = min(m - c0, kXChunk);
            if (c0 > 0) __syncthreads();  // both waves are done with the previous chunk
            gather_tokens<NB>(xs, a.q8x, tok, c0, mc, m, wave, 2);
            if (c0 == 0) dma_wave_copy(wt[wave], W, kTileBytes);
            lds_dma_wait();
            __syncthreads();
#pragma unroll 1
            for (int c = 0; c < mc; ++c) {
                const float v = lpb_row_q4k_mem<NB>(wt[wave] + grp * kRowBytes, xl[c * NB + t8], t8);
                if (t8 == NB - 1) gu[wave][grp][c0 + c] = v;
            }
        }
    }
    __syncthreads();
    const int r = threadIdx.x / kMaxTok, cc = threadIdx.x % kMaxTok;  // 128 threads: 8 rows x 16 columns
    if (cc < m) {
        const float g = gu[0][r][cc], uu = gu[1][r][cc];
        a.hbuf[((size_t)u * kMaxTok + cc) * a.n_ff + row0 + r] = g / (1.0f + expf(-g)) * uu;
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
// Q6_K rows are only 2-byte aligned, which LDS reads handle with alignbyte;
// the per-token Q6_K dot wants one alignment per wave, so each pass takes the
// rows of one parity (the row size is 2 mod 4).
template <int TD, int NBH>
__global__ __launch_bounds__(64, 4) void down_kernel(BatchedArgs a) {
    constexpr int kRowBytes = NBH * (TD == kTypeQ4K ? kQ4KBytes : kQ6KBytes);
    constexpr int kTileBytes = kTile * kRowBytes;
    const int u = blockIdx.y;
    int e, m;
    if (!load_group(a, u, e, m)) return;
    __shared__ __align__(16) uint8_t tile[kTileBytes];
    __shared__ __align__(16) uint8_t xs[kXChunk * NBH * sizeof(Q8L)];
    const int lane = threadIdx.x & 63, t8 = lane & 7, grp = lane >> 3;
    const int row0 = blockIdx.x * kTile;
    const int *tok = a.utok + u * kMaxTok, *slot = a.uslot + u * kMaxTok;
    const uint8_t *src = a.down + (size_t)e * a.dstride + (size_t)row0 * kRowBytes;
    if (m >= kMfmaMinTokens) {
        dma_wave_copy(tile, src, kTileBytes);
        const int c = lane & 15;
        const Q8L *xq = q8(a.q8h) + ((size_t)u * kMaxTok + (c < m ? c : 0)) * NBH;
        lds_dma_wait();
        float v[4];
        if constexpr (TD == kTypeQ4K)
            tile_q4k<NBH>(tile, kRowBytes, xq, v);
        else
            tile_q6k<NBH>(tile, kRowBytes, xq, v);
        if (c < m) {
            float *y = a.ybuf + ((size_t)tok[c] * a.k + slot[c]) * a.n_embd + row0;
#pragma unroll
            for (int i = 0; i < 4; ++i) y[4 * (lane >> 4) + i] = v[i];
        }
        return;
    }
    const Q8L *xl = reinterpret_cast<const Q8L *>(xs);
    for (int c0 = 0; c0 < m; c0 += kXChunk) {
        const int mc = min(m - c0, kXChunk);
        // the group's Q8_K h rows are contiguous, token-major
        dma_wave_copy(xs, a.q8h + ((size_t)u * kMaxTok + c0) * NBH * sizeof(Q8L), mc * NBH * (int)sizeof(Q8L));
        if (c0 == 0) dma_wave_copy(tile, src, kTileBytes);
        lds_dma_wait();
#pragma unroll 1
        for (int c = 0; c < mc; ++c) {
            float *y = a.ybuf + ((size_t)tok[c0 + c] * a.k + slot[c0 + c]) * a.n_embd + row0;
            if constexpr (TD == kTypeQ6K) {
#pragma unroll 1
                for (int p = 0; p < 2; ++p) {
                    const int row = 2 * grp + p;
                    const float v = g8_row_q6k_u<NBH>(tile + row * kRowBytes, xl + c * NBH, t8);
                    if (t8 == 0) y[row] = v;
                }
            } else {
#pragma unroll 1
                for (int p = 0; p < 2; ++p) {
                    const int row = 8 * p + grp;
                    const float v = lpb_row_q4k_mem<NBH>(tile + row * kRowBytes, xl[c * NBH + min(t8, NBH - 1)], t8);
                    if (t8 == NBH - 1) y[row] = v;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this chunk's LDS reads precede the next copy
    }
}

// -- combine: out[t][d] = (sum_j w[t][j] * y[t][j][d]) + res[t][d], j ascending --
__global__ __launch_bounds__(256) void combine_kernel(BatchedArgs a) {
    const int t = blockIdx.y;
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= a.n_embd) return;
    if (a.bad && a.bad[t]) {  // an id outside the pool or expert set: the token's row is poisoned
        a.out[(size_t)t * a.n_embd + d] = __builtin_nanf("");
        return;
    }
    float acc = 0.0f;
    for (int j = 0; j < a.k; ++j) {
        const int js = a.ysrc ? a.ysrc[t * a.k + j] : j;  // a repeated id takes its first output
        acc = acc + a.wsel[t * a.k + j] * a.ybuf[((size_t)t * a.k + js) * a.n_embd + d];
    }
    a.out[(size_t)t * a.n_embd + d] = acc + a.res[(size_t)t * a.n_embd + d];
}

}  // namespace

bool batched_shape_compiled(int gu_type, int n_embd, int d_type, int n_ff) {
    return gu_type == kTypeQ4K && n_embd == 2048 && (n_ff == 768 || n_ff == 1024 || n_ff == 512) &&
           (d_type == kTypeQ4K || d_type == kTypeQ6K);
}

namespace {

// The launches after the grouping: gate/up, Q8_K(h), down, combine.
hipError_t launch_groups(const BatchedArgs &a, hipStream_t s) {
    const int nbh = a.n_ff / QK;
    const int umax = a.n_ids < a.M * a.k ? a.n_ids : a.M * a.k;
    hipLaunchKernelGGL(gateup_kernel<8>, dim3(a.n_ff / 8, umax), dim3(128), 0, s, a);
    hipLaunchKernelGGL(quant_h_kernel, dim3(nbh, kMaxTok, umax), dim3(64), 0, s, a);
    const dim3 dg(a.n_embd / kTile, umax);
#define HOARD_DOWN(T, N)                                                  \
    if (a.d_type == T && nbh == N) {                                      \
        hipLaunchKernelGGL((down_kernel<T, N>), dg, dim3(64), 0, s, a);    \
    } else
    HOARD_DOWN(kTypeQ6K, 3) HOARD_DOWN(kTypeQ6K, 2) HOARD_DOWN(kTypeQ6K, 4) HOARD_DOWN(kTypeQ4K, 4)
    HOARD_DOWN(kTypeQ4K, 3) HOARD_DOWN(kTypeQ4K, 2) { return hipErrorInvalidValue; }
#undef HOARD_DOWN
    hipLaunchKernelGGL(combine_kernel, dim3((a.n_embd + 255) / 256, a.M), dim3(256), 0, s, a);
    return hipGetLastError();
}

bool args_ok(const BatchedArgs &a) {
    return a.M >= 1 && a.M <= kMaxTok && a.n_embd == kRouteN && a.gu_type == kTypeQ4K && a.k <= kMaxK &&
           a.n_ids >= 1 && a.n_ids <= kMaxExperts && a.E <= kMaxExperts;
}

}  // namespace

hipError_t launch_batched(const BatchedArgs &a, hipStream_t s) {
    if (!args_ok(a) || a.ysrc || a.n_ids != a.E || (a.M + kRouteTok - 1) / kRouteTok > kBatchedCounters - 1)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(route_kernel, dim3((a.E + kRouteRows - 1) / kRouteRows, (a.M + kRouteTok - 1) / kRouteTok),
                       dim3(256), 0, s, a);
    return launch_groups(a, s);
}

hipError_t launch_batched_ids(const BatchedArgs &a, hipStream_t s) {
    if (!args_ok(a) || !a.ysrc || !a.bad) return hipErrorInvalidValue;
    hipLaunchKernelGGL(prep_ids_kernel, dim3((unsigned)a.M + 1), dim3(512), 0, s, a);
    return launch_groups(a, s);
}

}  // namespace hoard
