// Expert products of a prefill-sized batch (more than 32 tokens): the
// counterpart of ggml_mul_mat_id over all T prompt tokens
// (src/run_m1.cpp:93-108) and of the verify step's mul_mat_id with per-token
// ids (src/run_specloop.cpp:126-139), followed by the weighted sum over the
// selected experts.
//
// batched.hip routes the tokens (or takes the caller's ids), forms Q8_K(fx)
// and sorts the (token, slot) pairs by (expert, token) into work units of at
// most kUnitTokens pairs of one expert.  Here, per unit:
//   gate/up  32 rows of gate and of up per workgroup (16 rows of one matrix per
//            wave) against the unit's tokens on v_mfma_i32_16x16x64_i8, 16
//            token columns per MFMA, the sub-block scales folded into the
//            weight operand; each weight super-block is loaded and folded once
//            and used for every token chunk of the unit; SwiGLU fused;
//   Q8_K(h)  per pair;
//   down     64 rows per workgroup, the tile staged in LDS in one burst;
//            y goes to its (token, slot) place;
// Q3_K gate/up rows (pf_gateup_q3_kernel) and Q4_K / Q5_K down rows run one
// MFMA per sub-block or scale group with the scales applied per (row, token)
// (mfma.h); Q4_K gate/up and Q6_K down rows fold the scales into the operand.
//   combine  per token, slots in order, plus the residual.
// Every expert's weights are read once per unit (once per call for a group of
// at most kUnitTokens tokens); each (row, token) value is formed from the
// per-token path's integer sub-block sums in its fp32 order (mfma.h), so every
// token's result is the single-token path's bit for bit.
#include "kernels.h"
#include "lds_dma.h"
#include "mfma.h"
#include "qblocks.h"
#include "rowdot.h"
#include "router_tail.h"

namespace hoard {

namespace {

constexpr int kWaveRows = 16;  // rows per wave: one MFMA tile
constexpr int kGuRows = 32;    // gate (and up) rows per workgroup: two 16-row tiles
constexpr int kDnRows = 64;    // down rows per workgroup
constexpr int kChunks = kUnitTokens / 16;  // 16-token MFMA chunks per unit
static_assert(kChunks == 4, "four token chunks per unit");

__device__ __forceinline__ const Q8L *q8c(const uint8_t *p) { return reinterpret_cast<const Q8L *>(p); }

// A work unit: expert e, its pairs [p0, p0 + n) in sorted order; one 16-byte
// record (a place past the last unit holds n = 0), so a workgroup knows its
// work after one memory latency.
struct Unit {
    int e, p0, n;
};
__device__ __forceinline__ bool load_unit(const BatchedArgs &a, int unit, Unit &w) {
    const int4 r = *reinterpret_cast<const int4 *>(a.units + 4 * unit);
    w.e = r.x;
    w.p0 = r.y;
    w.n = r.z;
    return w.n > 0;
}

__device__ __forceinline__ v4i mfma_16x16x64(v4i a, v4i b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// One Q4_K super-block of a 16-row tile, folded for v_mfma_i32_16x16x64_i8.
// Lane l supplies A[l % 16][16 g .. 16 g + 15] (g = l / 16) of each of the four
// MFMA steps (the lane layout checked by a probe: B[16 g ..][l % 16] alike,
// D[4 g + i][l % 16]).  Quant byte i of chunk q (32 bytes) holds element
// 64 q + i in its low nibble and 64 q + 32 + i in its high one (sub-blocks 2 q
// and 2 q + 1), and a step's K index is only a summation index: lane group g
// takes the whole of chunk g, as two 16-byte pieces p that each give two
// steps, step j = 2 p + h taking nibble half h of piece p, i.e. elements
// 64 g + 16 p + 32 h .. + 15 of sub-block 2 g + h.  Each quant byte is so
// loaded once (two 16-byte loads a lane), and the lane's B operand of step j
// is those 16 contiguous activation quants.  The sub-block scale sc (6 bits)
// is folded into A in two parts that keep every product an int8:
// hi = q * (sc >> 3) and lo = q * (sc & 7), each <= 105, with
// sc * q = 8 hi + lo; a nibble times a factor below 8 never carries into the
// next byte, so a whole word multiplies at once.  The min term
// sum_s m_s * (sum of sub-block s's activation quants) is a third MFMA with
// m_s broadcast over the step.  The three chains give exactly the per-token
// path's integer sums isum = 8 D_hi + D_lo and msum = D_min.  Each 16-bit half
// of a word of four nibbles multiplies at once (v_pk_mul_lo_u16, full rate,
// where a 32-bit multiply is quarter rate).
struct Q4Fold {
    v4i hi[4], lo[4];
    v4i mn[2];            // the min of sub-block 2 g + h in every byte (steps of nibble half h)
    float d[4], dmin[4];  // factors of the four rows whose results the lane receives
};

typedef unsigned short v2u16 __attribute__((ext_vector_type(2)));
// Bytes of w (each <= 15) times f (<= 7), byte by byte: no product carries.
__device__ __forceinline__ int nib_mul(uint32_t w, uint32_t f) {
    const v2u16 m = {(unsigned short)f, (unsigned short)f};
    return (int)__builtin_bit_cast(uint32_t, __builtin_bit_cast(v2u16, w) * m);
}

// Byte i of w in all four bytes (one v_perm_b32).
__device__ __forceinline__ int splat_byte_of(uint32_t w, int i) {
    return (int)__builtin_amdgcn_perm(w, w, 0x01010101u * (uint32_t)i);
}

// The lane's raw bytes of one super-block of a 16-row tile: its row's header
// and chunk g's 32 quant bytes; loaded one super-block ahead.  The fp16
// factors of the four rows whose results the lane receives come from those
// rows' lanes by a lane shuffle (four 4-byte gathers from global memory per
// super-block cost more than the shuffles).
struct Q4Raw {
    uint4 hd;
    uint4 qv[2];
};

__device__ __forceinline__ void q4_raw_load(const uint8_t *W, size_t rb, int b, Q4Raw &o) {
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const uint8_t *blk = W + (size_t)r * rb + (size_t)b * kQ4KBytes;
    o.hd = *reinterpret_cast<const uint4 *>(blk);
    o.qv[0] = *reinterpret_cast<const uint4 *>(blk + 16 + 32 * g);
    o.qv[1] = *reinterpret_cast<const uint4 *>(blk + 32 + 32 * g);
}

__device__ __forceinline__ void q4_fold(const Q4Raw &raw, Q4Fold &o) {
    const int g = (threadIdx.x & 63) >> 4;
    uint32_t sc[2], mn[2];
    q4k_scales_packed(raw.hd, sc, mn);
    // the scales and mins of sub-blocks 2 g (low nibbles) and 2 g + 1 (high)
    const int s0 = 2 * g;
    const uint32_t sc0 = (uint32_t)byte_of(sc[s0 >> 2], s0 & 3), sc1 = (uint32_t)byte_of(sc[s0 >> 2], (s0 & 3) + 1);
    const int mw = (int)mn[s0 >> 2];
    const int m0 = (int)__builtin_amdgcn_perm(mw, mw, 0x01010101u * (uint32_t)(s0 & 3));
    const int m1 = (int)__builtin_amdgcn_perm(mw, mw, 0x01010101u * (uint32_t)((s0 & 3) + 1));
    o.mn[0] = v4i{m0, m0, m0, m0};
    o.mn[1] = v4i{m1, m1, m1, m1};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 qv = raw.qv[j >> 1];
        const uint32_t nsh = 4u * (uint32_t)(j & 1), scs = (j & 1) ? sc1 : sc0;
        const uint32_t w[4] = {(qv.x >> nsh) & 0x0f0f0f0fu, (qv.y >> nsh) & 0x0f0f0f0fu, (qv.z >> nsh) & 0x0f0f0f0fu,
                               (qv.w >> nsh) & 0x0f0f0f0fu};
        const uint32_t h = scs >> 3, lw = scs & 7u;
        o.hi[j] = v4i{nib_mul(w[0], h), nib_mul(w[1], h), nib_mul(w[2], h), nib_mul(w[3], h)};
        o.lo[j] = v4i{nib_mul(w[0], lw), nib_mul(w[1], lw), nib_mul(w[2], lw), nib_mul(w[3], lw)};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t dm = (uint32_t)__shfl((int)raw.hd.x, 4 * g + i);
        o.d[i] = half_bits_to_float(dm & 0xffffu);
        o.dmin[i] = half_bits_to_float(dm >> 16);
    }
}

// One super-block of the folded tile against the lane's token column (its Q8_K
// block x): the integer sums from the three MFMA chains, then the per-token
// path's fp32 block terms added in order.  Step j's B operand: activation
// quants 64 g + 16 (j / 2) + 32 (j % 2) .. + 15.
template <class X>
__device__ __forceinline__ void q4_fold_step(const Q4Fold &w, const X &x, float acc[4], float accm[4]) {
    const int g = (threadIdx.x & 63) >> 4;
    v4i dh = {0, 0, 0, 0}, dl = {0, 0, 0, 0}, dn = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const v4i xv = *reinterpret_cast<const v4i *>(&x.qs[16 * g + 4 * (j >> 1) + 8 * (j & 1)]);
        dh = mfma_16x16x64(w.hi[j], xv, dh);
        dl = mfma_16x16x64(w.lo[j], xv, dl);
        dn = mfma_16x16x64(w.mn[j & 1], xv, dn);
    }
    const float xd = x.d;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int isum = 8 * dh[i] + dl[i];
        const float dd = w.d[i] * xd;
        const float dm = w.dmin[i] * xd;
        acc[i] = acc[i] + dd * (float)isum;
        accm[i] = accm[i] + dm * (float)dn[i];
    }
}

// -- gate/up + SwiGLU ------------------------------------------------------------
// grid (n_ff / 32, max units), block 256: wave w takes rows [32 x + 16 (w % 2), +16)
// of gate (w < 2) or up (w >= 2) of the unit's expert against every token of the
// unit.  Per super-block the workgroup copies the Q8_K blocks of the unit's
// token chunks into LDS (one buffer ahead) while each wave holds the next
// super-block of its rows in registers; the gate waves hand their values to the
// up waves through LDS, which form h and store it to hbuf[sorted pair][row].
// Three workgroups share a CU (43 KB of LDS each).  The kernel is compiled to
// the 128 registers of four waves a SIMD all the same: that schedule measured
// 1 % faster for the layer than the 146-register one at three waves (a fourth
// workgroup a CU, with the gate values over an x buffer, spilled and measured
// 12 % slower).
// The part of a Q8_K block the folded gate/up tiles read: the quants and the
// scale (granules 0-15 and 18 of the block; its 16-element sums are not read).
struct Q8S {
    int32_t qs[64];
    float d;
    int32_t pad[3];
};
static_assert(sizeof(Q8S) == 272 && offsetof(Q8L, d) == 288, "Q8S: 17 granules, d from granule 18 of Q8L");
constexpr int kXGran = (int)sizeof(Q8S) / 16;                          // 16-byte granules staged per token
constexpr int kXChunksPerBlock = (kUnitTokens * kXGran + 63) / 64;     // 1 KB copies per unit block

template <int NB>
__global__ __launch_bounds__(256, 4) void pf_gateup_kernel(BatchedArgs a) {
    __shared__ __align__(16) Q8S xs[2][kUnitTokens];  // the unit's Q8_K block b (two buffers)
    __shared__ float gx[2][kChunks][4][64];            // gate values: [row tile][chunk][row i][lane]
    Unit w;
    if (!load_unit(a, blockIdx.y, w)) return;
    const int wave = wave_index(), lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
    const int m = wave >> 1, rt = wave & 1;
    const int row0 = blockIdx.x * kGuRows + rt * kWaveRows;
    constexpr size_t rb = (size_t)NB * kQ4KBytes;
    const uint8_t *W = (m ? batched_up(a, w.e) : batched_gate(a, w.e)) + (size_t)row0 * rb;
    const int nch = (w.n + 15) >> 4;
    // this lane's granules of the x copy: chunks wave, wave + 4, ...; only the
    // unit's tokens are copied (the MFMA columns of the places past them read
    // whatever the buffer holds, and their results are not stored)
    constexpr int kXJ = (kXChunksPerBlock + 3) / 4;
    const int ngran = w.n * kXGran;
    // byte offsets into q8x (it holds at most 512 tokens' blocks): half the
    // registers of pointers
    uint32_t xoff[kXJ];
#pragma unroll
    for (int j = 0; j < kXJ; ++j) {
        const int p = 64 * (wave + 4 * j) + lane, tt = min(p / kXGran, kUnitTokens - 1), o = p % kXGran;
        xoff[j] = (uint32_t)a.ptok[w.p0 + min(tt, w.n - 1)] * (uint32_t)(NB * sizeof(Q8L)) + 16u * (o < 16 ? o : 18);
    }
    auto stage_x = [&](int b, int buf) {
#pragma unroll
        for (int j = 0; j < kXJ; ++j) {
            const int ck = wave + 4 * j;
            if (64 * ck < ngran && 64 * ck + lane < ngran)
                dma_lanes(reinterpret_cast<uint8_t *>(&xs[buf][0]) + 1024 * ck,
                          a.q8x + (xoff[j] + (uint32_t)(b * sizeof(Q8L))));
        }
    };
    float acc[kChunks][4], accm[kChunks][4];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ch][i] = accm[ch][i] = 0.0f;
    Q4Raw raw;
    q4_raw_load(W, rb, 0, raw);
    stage_x(0, 0);
#pragma unroll 1
    for (int b = 0; b < NB; ++b) {
        // Other waves read the x chunks this wave copied: the compiler does not
        // see the copies, so the wave waits for its own before the barrier (it
        // waits for the raw weight loads of block b there anyway).
        lds_dma_wait();
        __syncthreads();  // every wave's copies of x(b) landed, and x(b - 1) is read
        Q4Fold t;
        q4_fold(raw, t);
        // the fold is done before the next loads issue
        asm volatile("" ::"v"(t.hi[0]), "v"(t.hi[1]), "v"(t.hi[2]), "v"(t.hi[3]), "v"(t.lo[0]), "v"(t.lo[1]),
                     "v"(t.lo[2]), "v"(t.lo[3])
                     : "memory");
        // the next super-block's activation copies issue before its weight
        // loads (both are waited for at the next super-block; copies first
        // measured 3 % faster for the layer at 512 tokens)
        if (b + 1 < NB) {
            stage_x(b + 1, (b + 1) & 1);
            q4_raw_load(W, rb, b + 1, raw);
        }
        const Q8S *xb = xs[b & 1];
#pragma unroll
        for (int ch = 0; ch < kChunks; ++ch)
            if (ch < nch) q4_fold_step(t, xb[ch * 16 + c], acc[ch], accm[ch]);
    }
    if (m == 0) {
#pragma unroll
        for (int ch = 0; ch < kChunks; ++ch)
#pragma unroll
            for (int i = 0; i < 4; ++i) gx[rt][ch][i][lane] = acc[ch][i] - accm[ch][i];
    }
    __syncthreads();
    if (m == 0) return;
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
        const int idx = ch * 16 + c;
        if (ch < nch && idx < w.n) {
            float hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float g = gx[rt][ch][i][lane], uu = acc[ch][i] - accm[ch][i];
                hv[i] = g / (1.0f + expf(-g)) * uu;
            }
            *reinterpret_cast<float4 *>(a.hbuf + (size_t)(w.p0 + idx) * a.n_ff + row0 + 4 * q) =
                make_float4(hv[0], hv[1], hv[2], hv[3]);
        }
    }
}

// -- Q8_K of h per sorted pair --------------------------------------------------
// grid (pairs), block 64 * NBH: wave b quantises block b of the pair's h.
__global__ __launch_bounds__(256) void pf_quant_h_kernel(BatchedArgs a) {
    const int pos = blockIdx.x, b = wave_index();
    const int nbh = a.n_ff / QK;
    if (b >= nbh) return;
    const float d = wave_quantize_q8l(a.hbuf + (size_t)pos * a.n_ff + (size_t)b * QK,
                                      reinterpret_cast<Q8L *>(a.q8h) + (size_t)pos * nbh + b);
    // the scales again, four to a pair: the down kernels copy a unit's in one 16-byte load a lane
    if ((threadIdx.x & 63) == 0) a.q8hd[(size_t)pos * 4 + b] = d;
}

// -- down: 64 rows of the unit's expert, y to its (token, slot) place -----------
// grid (n_embd / 64, max units), block 256, for Q4_K down rows (OLMoE).  The
// 64-row tile is copied into LDS in one burst; wave w takes rows [16 w, +16) of it.
template <int NBH>
__global__ __launch_bounds__(256) void pf_down_q4_kernel(BatchedArgs a) {
    constexpr int kRowBytes = NBH * kQ4KBytes;
    constexpr int kTileBytes = kDnRows * kRowBytes;
    static_assert(kTileBytes % 16 == 0, "the tile copies in 16-byte units");
    __shared__ __align__(16) uint8_t tile[kTileBytes];
    Unit w;
    if (!load_unit(a, blockIdx.y, w)) return;
    const int wave = wave_index(), lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
    const int rt0 = blockIdx.x * kDnRows;
    // each wave copies its own 16 rows and waits for them alone
    constexpr int kWaveBytes = kWaveRows * kRowBytes;
    static_assert(kWaveBytes % 16 == 0, "a wave's rows copy in 16-byte units");
    uint8_t *T = tile + wave * kWaveBytes;
    dma_wave_copy_nt(T, batched_down(a, w.e) + (size_t)(rt0 + wave * kWaveRows) * kRowBytes, kWaveBytes);
    lds_dma_wait();
    const int nch = (w.n + 15) >> 4;
    const Q8L *q8h = reinterpret_cast<const Q8L *>(a.q8h);
    // (chunk, block) steps with the next step's activation operands loaded
    // while the current one computes
    auto xq_of = [&](int ch) { return q8h + (size_t)(w.p0 + min(ch * 16 + c, w.n - 1)) * NBH; };
    Q6X cur, nxt;
    q6_load_x(xq_of(0), 0, cur);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int steps = nch * NBH;
#pragma unroll 1
    for (int st = 0; st < steps; ++st) {
        const int ch = st / NBH, b = st - ch * NBH;
        if (st + 1 < steps) q6_load_x(xq_of((st + 1) / NBH), (st + 1) % NBH, nxt);
        q4_tile_block(T, kRowBytes, b, cur, acc, accm);
        if (b == NBH - 1) {
            const int idx = ch * 16 + c;
            if (idx < w.n) {
                const int pos = w.p0 + idx, t = a.ptok[pos], j = a.pslot[pos];
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = acc[i] - accm[i];
                *reinterpret_cast<float4 *>(a.ybuf + ((size_t)t * (a.k + a.sh) + j) * a.n_embd + rt0 + wave * kWaveRows +
                                            4 * q) = make_float4(v[0], v[1], v[2], v[3]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[i] = accm[i] = 0.0f;
        }
        cur = nxt;
    }
}

// -- down, Q6_K rows folded for v_mfma_i32_16x16x64_i8 --------------------------
// Lane l of a wave supplies A[l % 16][16 g .. + 15] (g = l / 16) of each 64-element
// chunk jc of a super-block: elements 64 jc + 16 g .. + 15 of row l % 16, whose
// 6-bit values are nibble (jc % 2) of ql bytes 64 (jc / 2) + 16 g .. + 15 with
// bits 4 (jc % 2) + 2 (g / 2) .. + 1 of qh bytes 128 + 32 (jc / 2) + 16 (g % 2) ..
// + 15 on top, and which share one group scale, sc = scales[4 jc + g].  The
// per-token path forms isum = sum_g sc_g * sum_{e in g} (q_e - 32) x_e.  Here
// w = sc * q (-8064 <= w <= 8001) is split as w = 64 hi + lo with lo = w & 63 in
// [0, 63] and hi = w >> 6 in [-126, 125], both int8, and the zero point comes from a third MFMA with
// sc broadcast over the lane's 16 elements (the token's group sums):
// isum = 64 D_hi + D_lo - 32 D_sc, exactly.  A super-block of the tile is
// folded once and used for every token chunk of the unit.
struct Q6Fold {
    v4i hi[4], lo[4];
    uint32_t sc;  // byte jc: the group scale of the lane's elements of chunk jc
    float d[4];   // factors of the four rows whose results the lane receives
};

// 16 bytes at a 2-byte aligned LDS address, as four words.
__device__ __forceinline__ uint4 lds_u128_a2(const uint8_t *p) {
    const uint2 a = lds_u64_a2(p), b = lds_u64_a2(p + 8);
    return make_uint4(a.x, a.y, b.x, b.y);
}

__device__ __forceinline__ void q6_fold(const uint8_t *T, size_t rb, int b, Q6Fold &o) {
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const uint8_t *blk = T + (size_t)r * rb + (size_t)b * kQ6KBytes;
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) {
        const uint4 ql = lds_u128_a2(blk + 64 * (jc >> 1) + 16 * g);
        const uint4 qh = lds_u128_a2(blk + 128 + 32 * (jc >> 1) + 16 * (g & 1));
        const int sc = (int)(int8_t)blk[192 + 4 * jc + g];
        const uint32_t nsh = 4u * (uint32_t)(jc & 1), hsh = 4u * (uint32_t)(jc & 1) + 2u * (uint32_t)(g >> 1);
        const uint32_t sc16 = ((uint32_t)sc & 0xffffu) * 0x00010001u;  // sc in both 16-bit halves
        const uint32_t qlw[4] = {ql.x, ql.y, ql.z, ql.w}, qhw[4] = {qh.x, qh.y, qh.z, qh.w};
        int hw[4], lw[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = ((qlw[k] >> nsh) & 0x0f0f0f0fu) | (((qhw[k] >> hsh) & 0x03030303u) << 4);
            // bytes 0, 2 and 1, 3 in 16-bit halves; w = sc * q in each half
            const uint32_t w02 = __builtin_amdgcn_perm(0u, q, 0x0c020c00u) ;
            const uint32_t w13 = __builtin_amdgcn_perm(0u, q, 0x0c030c01u);
            typedef short v2s __attribute__((ext_vector_type(2)));
            const v2s s2 = __builtin_bit_cast(v2s, sc16);
            const v2s a02 = __builtin_bit_cast(v2s, w02) * s2, a13 = __builtin_bit_cast(v2s, w13) * s2;
            // hi = w >> 6 (arithmetic: floor(w / 64)), lo = w & 63 = w - 64 hi
            const v2s h02 = a02 >> (v2s){6, 6}, h13 = a13 >> (v2s){6, 6};
            const v2s l02 = a02 & (v2s){63, 63}, l13 = a13 & (v2s){63, 63};
            // back to bytes: result byte 2i from the 02 half i, byte 2i + 1 from the 13 half i
            hw[k] = (int)__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, h13), __builtin_bit_cast(uint32_t, h02),
                                               0x06020400u);
            lw[k] = (int)__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, l13), __builtin_bit_cast(uint32_t, l02),
                                               0x06020400u);
        }
        o.hi[jc] = v4i{hw[0], hw[1], hw[2], hw[3]};
        o.lo[jc] = v4i{lw[0], lw[1], lw[2], lw[3]};
        if (jc == 0) o.sc = 0u;
        o.sc |= ((uint32_t)sc & 0xffu) << (8 * jc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint8_t *blk_i = T + (size_t)(4 * g + i) * rb + (size_t)b * kQ6KBytes;
        o.d[i] = half_bits_to_float((uint32_t)blk_i[208] | ((uint32_t)blk_i[209] << 8));
    }
}

// The lane's B operands of one token's Q8_K block: qs bytes 64 jc + 16 g .. + 15.
struct Q6XB {
    v4i x[4];
    float xd;
};
__device__ __forceinline__ void q6_load_xb(const Q8L &x, Q6XB &o) {
    const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) o.x[jc] = *reinterpret_cast<const v4i *>(&x.qs[16 * jc + 4 * g]);
    o.xd = x.d;
}
// The quants alone, the scale coming from elsewhere.
__device__ __forceinline__ void q6_load_xq(const Q8L &x, Q6XB &o) {
    const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) o.x[jc] = *reinterpret_cast<const v4i *>(&x.qs[16 * jc + 4 * g]);
}

__device__ __forceinline__ void q6_fold_step(const Q6Fold &w, const Q6XB &x, float acc[4]) {
    v4i dh = {0, 0, 0, 0}, dl = {0, 0, 0, 0}, ds = {0, 0, 0, 0};
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) {
        dh = mfma_16x16x64(w.hi[jc], x.x[jc], dh);
        dl = mfma_16x16x64(w.lo[jc], x.x[jc], dl);
        const int s4 = splat_byte_of(w.sc, jc);
        ds = mfma_16x16x64(v4i{s4, s4, s4, s4}, x.x[jc], ds);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int isum = 64 * dh[i] + dl[i] - 32 * ds[i];
        acc[i] = acc[i] + (w.d[i] * x.xd) * (float)isum;
    }
}

typedef short v2s16 __attribute__((ext_vector_type(2)));
typedef unsigned short v2u16b __attribute__((ext_vector_type(2)));

// Bytes 0, 2 and 1, 3 of w in the 16-bit halves of two words, and back.
__device__ __forceinline__ void bytes_to_halves(uint32_t w, uint32_t &w02, uint32_t &w13) {
    w02 = __builtin_amdgcn_perm(0u, w, 0x0c020c00u);
    w13 = __builtin_amdgcn_perm(0u, w, 0x0c030c01u);
}
__device__ __forceinline__ int halves_to_bytes(uint32_t w02, uint32_t w13) {
    return (int)__builtin_amdgcn_perm(w13, w02, 0x06020400u);
}

// Q3_K super-block b of a 16-row tile in LDS (row r at T + r*rb; 110-byte
// blocks, only 2-byte aligned), folded for v_mfma_i32_16x16x64_i8.  Lane group
// g of chunk jc supplies elements 64 jc + 16 g .. + 15 of its row: 32-element
// range 2 jc + g / 2 (half n = jc / 2, quarter j = 2 (jc & 1) + g / 2),
// positions l = 16 (g & 1) .. + 15, one 16-element scale group G = 4 jc + g.
// Its quants are q3 = q2 + 4 h - 4 (q2: bits 2 j .. 2 j + 1 of qs[32 n + l];
// h: bit 4 n + j of hmask[l]) and w = (sc_G - 32) * q3 lies in [-124, 128]; it
// is split as w = 64 hi + lo with lo = w & 63 and hi = w >> 6 in [-2, 2], both
// int8, so isum = 64 D_hi + D_lo is the per-token path's integer sum exactly.
struct Q3Fold {
    v4i hi[4], lo[4];
    float d[4];  // factors of the four rows whose results the lane receives
};

__device__ __forceinline__ void q3_fold(const uint8_t *T, size_t rb, int b, Q3Fold &o) {
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const uint8_t *blk = T + (size_t)r * rb + (size_t)b * kQ3KBytes;
    const uint4 hm = lds_u128_a2(blk + 16 * (g & 1));  // hmask[l], l = 16 (g & 1) .. + 15
    const uint2 s01 = lds_u64_a2(blk + 96);
    const uint32_t s2 = lds_u32(blk + 104);
    const uint32_t hmw[4] = {hm.x, hm.y, hm.z, hm.w};
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) {
        const int n = jc >> 1, j = 2 * (jc & 1) + (g >> 1);
        const uint4 qv = lds_u128_a2(blk + 32 + 32 * n + 16 * (g & 1));
        const int sc = q3k_scale(4 * jc + g, s01.x, s01.y, s2);
        const v2s16 scv = {(short)sc, (short)sc};
        const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
        int hw[4], lw[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = ((qw[k] >> (2 * j)) & 0x03030303u) | (((hmw[k] >> (4 * n + j)) & 0x01010101u) << 2);
            uint32_t q02, q13;
            bytes_to_halves(q, q02, q13);
            const v2s16 w02 = (__builtin_bit_cast(v2s16, q02) - (v2s16){4, 4}) * scv;
            const v2s16 w13 = (__builtin_bit_cast(v2s16, q13) - (v2s16){4, 4}) * scv;
            hw[k] = halves_to_bytes(__builtin_bit_cast(uint32_t, w02 >> (v2s16){6, 6}),
                                    __builtin_bit_cast(uint32_t, w13 >> (v2s16){6, 6}));
            lw[k] = halves_to_bytes(__builtin_bit_cast(uint32_t, w02 & (v2s16){63, 63}),
                                    __builtin_bit_cast(uint32_t, w13 & (v2s16){63, 63}));
        }
        o.hi[jc] = v4i{hw[0], hw[1], hw[2], hw[3]};
        o.lo[jc] = v4i{lw[0], lw[1], lw[2], lw[3]};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint8_t *blk_i = T + (size_t)(4 * g + i) * rb + (size_t)b * kQ3KBytes;
        o.d[i] = half_bits_to_float((uint32_t)blk_i[108] | ((uint32_t)blk_i[109] << 8));
    }
}

__device__ __forceinline__ void q3_fold_step(const Q3Fold &w, const Q6XB &x, float acc[4]) {
    v4i dh = {0, 0, 0, 0}, dl = {0, 0, 0, 0};
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) {
        dh = mfma_16x16x64(w.hi[jc], x.x[jc], dh);
        dl = mfma_16x16x64(w.lo[jc], x.x[jc], dl);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int isum = 64 * dh[i] + dl[i];
        acc[i] = acc[i] + (w.d[i] * x.xd) * (float)isum;
    }
}

// Q5_K super-block b of a 16-row tile in LDS (16-byte aligned 176-byte blocks:
// d, dmin, Q4_K-packed scales and mins, qh[32], qs[128]), folded as the Q4_K
// gate/up tile is: lane group g of chunk jc takes nibble g / 2 of qs bytes
// 32 jc + 16 (g & 1) .. + 15 with bit 2 jc + g / 2 of qh[l] on top (q5 in
// [0, 31]), sub-block s = 2 jc + g / 2.  w = sc_s * q5 <= 1953 is split as
// w = 64 hi + lo (lo = w & 63, hi = w >> 6 <= 30); the min term is a third MFMA
// with m_s broadcast over its sub-block: isum = 64 D_hi + D_lo, msum = D_min.
struct Q5Fold {
    v4i hi[4], lo[4];
    uint32_t mn;          // byte jc: the min of the lane's sub-block in chunk jc
    float d[4], dmin[4];  // factors of the four rows whose results the lane receives
};

__device__ __forceinline__ void q5_fold(const uint8_t *T, size_t rb, int b, Q5Fold &o) {
    const int lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
    const uint8_t *blk = T + (size_t)r * rb + (size_t)b * kQ5KBytes;
    const uint4 hd = *reinterpret_cast<const uint4 *>(blk);
    const uint4 qh = *reinterpret_cast<const uint4 *>(blk + 16 + 16 * (g & 1));  // qh[l], l = 16 (g & 1) .. + 15
    uint32_t sc[2], mn[2];
    q4k_scales_packed(hd, sc, mn);
    const uint32_t qhw[4] = {qh.x, qh.y, qh.z, qh.w};
    const uint32_t nsh = 4u * (uint32_t)(g >> 1), bsh = 8u * (uint32_t)(g >> 1);
    o.mn = 0u;
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) {
        const int s = 2 * jc + (g >> 1);
        const uint32_t sh = 16u * (uint32_t)(jc & 1) + bsh;  // byte 2 (jc & 1) + g / 2 of word jc / 2
        const uint32_t scs = (sc[jc >> 1] >> sh) & 0xffu, mns = (mn[jc >> 1] >> sh) & 0xffu;
        const v2u16b scv = {(unsigned short)scs, (unsigned short)scs};
        const uint4 qv = *reinterpret_cast<const uint4 *>(blk + 48 + 32 * jc + 16 * (g & 1));
        const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
        int hw[4], lw[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t q = ((qw[k] >> nsh) & 0x0f0f0f0fu) | (((qhw[k] >> s) & 0x01010101u) << 4);
            uint32_t q02, q13;
            bytes_to_halves(q, q02, q13);
            const v2u16b w02 = __builtin_bit_cast(v2u16b, q02) * scv, w13 = __builtin_bit_cast(v2u16b, q13) * scv;
            hw[k] = halves_to_bytes(__builtin_bit_cast(uint32_t, w02 >> (v2u16b){6, 6}),
                                    __builtin_bit_cast(uint32_t, w13 >> (v2u16b){6, 6}));
            lw[k] = halves_to_bytes(__builtin_bit_cast(uint32_t, w02 & (v2u16b){63, 63}),
                                    __builtin_bit_cast(uint32_t, w13 & (v2u16b){63, 63}));
        }
        o.hi[jc] = v4i{hw[0], hw[1], hw[2], hw[3]};
        o.lo[jc] = v4i{lw[0], lw[1], lw[2], lw[3]};
        o.mn |= mns << (8 * jc);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t dm = *reinterpret_cast<const uint32_t *>(T + (size_t)(4 * g + i) * rb + (size_t)b * kQ5KBytes);
        o.d[i] = half_bits_to_float(dm & 0xffffu);
        o.dmin[i] = half_bits_to_float(dm >> 16);
    }
}

__device__ __forceinline__ void q5_fold_step(const Q5Fold &w, const Q6XB &x, float acc[4], float accm[4]) {
    v4i dh = {0, 0, 0, 0}, dl = {0, 0, 0, 0}, dn = {0, 0, 0, 0};
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) {
        dh = mfma_16x16x64(w.hi[jc], x.x[jc], dh);
        dl = mfma_16x16x64(w.lo[jc], x.x[jc], dl);
        const int m4 = splat_byte_of(w.mn, jc);
        dn = mfma_16x16x64(v4i{m4, m4, m4, m4}, x.x[jc], dn);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int isum = 64 * dh[i] + dl[i];
        const float dd = w.d[i] * x.xd;
        const float dm = w.dmin[i] * x.xd;
        acc[i] = acc[i] + dd * (float)isum;
        accm[i] = accm[i] + dm * (float)dn[i];
    }
}

// -- gate/up + SwiGLU for Q3_K rows (OLMoE in its Q3_K_M form) --------------------
// grid (n_ff / 32, max units), block 256: wave w takes rows [32 x + 16 (w % 2), +16)
// of gate (w < 2) or up (w >= 2).  The 32 rows of each matrix are copied into
// LDS in one burst (110-byte blocks, 2-byte aligned, read with alignbyte); per
// super-block each wave folds its rows once (q3_fold) and runs them against
// every token chunk of the unit.  The gate waves hand their values to the up
// waves through LDS, which form h.
template <int NB>
__global__ __launch_bounds__(256, 2) void pf_gateup_q3_kernel(BatchedArgs a) {
    constexpr int kRowBytes = NB * kQ3KBytes;
    constexpr int kTileBytes = 2 * kWaveRows * kRowBytes;  // 32 rows of one matrix
    static_assert(kRowBytes % 16 == 0, "Q3_K rows of 8 blocks are 880 bytes: tiles start 16-byte aligned");
    __shared__ __align__(16) uint8_t tile[2][kTileBytes];
    __shared__ float gx[2][kChunks][4][64];  // gate values: [row tile][chunk][row i][lane]
    __shared__ float xds[4][kUnitTokens * NB];  // each wave's copy of the tokens' Q8_K block scales
    Unit w;
    if (!load_unit(a, blockIdx.y, w)) return;
    const int wave = wave_index(), lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
    const int m = wave >> 1, rt = wave & 1;
    const int row0 = blockIdx.x * 2 * kWaveRows;
    // the lane's token of each chunk, read once, while the tile lands
    int tok[kChunks];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) tok[ch] = a.ptok[w.p0 + min(ch * 16 + c, w.n - 1)];
    // each wave copies its own 16 rows and waits for them alone
    constexpr int kWaveBytes = kWaveRows * kRowBytes;
    uint8_t *T = tile[m] + rt * kWaveBytes;
    dma_wave_copy_nt(T, (m ? batched_up(a, w.e) : batched_gate(a, w.e)) + (size_t)(row0 + rt * kWaveRows) * kRowBytes,
                     kWaveBytes);
    // the block scales of the unit's token places, place-major, into the wave's
    // LDS copy (NB 4-byte copies a lane; the lane's place comes from the lane
    // that read its token): a 4-byte load of a scale with every chunk's quants
    // in the loop cost more
    static_assert(NB == 8, "eight blocks a token: a copy covers eight places");
    const Q8L *q8xs = reinterpret_cast<const Q8L *>(a.q8x);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int tk = __shfl(tok[j >> 1], 8 * (j & 1) + (lane >> 3));
        dma_lanes4(reinterpret_cast<uint8_t *>(&xds[wave][64 * j]),
                   reinterpret_cast<const uint8_t *>(&q8xs[(size_t)tk * NB + (lane & 7)].d));
    }
    lds_dma_wait();
    const int nch = (w.n + 15) >> 4;
    const Q8L *q8x = reinterpret_cast<const Q8L *>(a.q8x);
    auto x_of = [&](int ch, int b) -> const Q8L & { return q8x[(size_t)tok[ch] * NB + b]; };
    auto load_x = [&](int ch, int b, Q6XB &o) {
        q6_load_xq(x_of(ch, b), o);
        o.xd = xds[wave][(ch * 16 + c) * NB + b];
    };
    float acc[kChunks][4];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ch][i] = 0.0f;
#pragma unroll 1
    for (int b = 0; b < NB; ++b) {
        // every chunk's activation operands in flight before the fold, which covers them
        Q6XB xc[kChunks];
#pragma unroll
        for (int ch = 0; ch < kChunks; ++ch)
            if (ch < nch) load_x(ch, b, xc[ch]);
        Q3Fold f;
        q3_fold(T, kRowBytes, b, f);
#pragma unroll
        for (int ch = 0; ch < kChunks; ++ch)
            if (ch < nch) q3_fold_step(f, xc[ch], acc[ch]);
    }
    if (m == 0) {
#pragma unroll
        for (int ch = 0; ch < kChunks; ++ch)
#pragma unroll
            for (int i = 0; i < 4; ++i) gx[rt][ch][i][lane] = acc[ch][i];
    }
    __syncthreads();
    if (m == 0) return;
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
        const int idx = ch * 16 + c;
        if (ch < nch && idx < w.n) {
            float hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float g = gx[rt][ch][i][lane], uu = acc[ch][i];
                hv[i] = g / (1.0f + expf(-g)) * uu;
            }
            *reinterpret_cast<float4 *>(a.hbuf + (size_t)(w.p0 + idx) * a.n_ff + row0 + rt * kWaveRows + 4 * q) =
                make_float4(hv[0], hv[1], hv[2], hv[3]);
        }
    }
}

// grid (n_embd / 64, max units), block 256: as pf_down_q4_kernel for Q6_K rows,
// super-block major: each super-block of the wave's 16 rows is folded once,
// then run against every token chunk of the unit, the next chunk's activation
// operands in flight meanwhile.  Three workgroups per CU (166 VGPRs).
template <int NBH>
__global__ __launch_bounds__(256, 3) void pf_down_q6_kernel(BatchedArgs a) {
    constexpr int kRowBytes = NBH * kQ6KBytes;
    constexpr int kTileBytes = kDnRows * kRowBytes;
    static_assert(kTileBytes % 16 == 0, "the tile copies in 16-byte units");
    __shared__ __align__(16) uint8_t tile[kTileBytes];
    __shared__ int yrow[kUnitTokens];  // y row (token * slots + slot) of each of the unit's pairs
    __shared__ __align__(16) float xds[4][kUnitTokens][4];  // each wave's copy of the pairs' Q8_K(h) scales
    Unit w;
    if (!load_unit(a, blockIdx.y, w)) return;
    const int wave = wave_index(), lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
    const int rt0 = blockIdx.x * kDnRows;
    const int nch = (w.n + 15) >> 4;
    const Q8L *q8h = reinterpret_cast<const Q8L *>(a.q8h);
    auto x_of = [&](int ch, int b) -> const Q8L & {
        return q8h[(size_t)(w.p0 + min(ch * 16 + c, w.n - 1)) * NBH + b];
    };
    // the pairs' block scales come from the wave's LDS copy, copied with the
    // tile: a 4-byte load of a scale with every chunk's quants cost more
    auto load_x = [&](int ch, int b, Q6XB &o) {
        q6_load_xq(x_of(ch, b), o);
        o.xd = xds[wave][min(ch * 16 + c, kUnitTokens - 1)][b];
    };
    // Chunk ch of a super-block takes its activation operands from x[ch % 2]:
    // chunk 0's are loaded before the fold, each later chunk's while the one
    // before it computes.
    static_assert(kChunks == 4, "four chunks, two operand sets");
    Q6XB x0, x1;
    // the pairs' places, read while the tile lands
    const int tid = threadIdx.x;
    const int pt = tid < w.n ? a.ptok[w.p0 + tid] : 0, ps = tid < w.n ? a.pslot[w.p0 + tid] : 0;
    // each wave copies its own 16 rows and waits for them alone: no barrier
    // between the copies and the folds
    constexpr int kWaveBytes = kWaveRows * kRowBytes;
    static_assert(kWaveBytes % 16 == 0, "a wave's rows copy in 16-byte units");
    uint8_t *T = tile + wave * kWaveBytes;
    dma_lanes(reinterpret_cast<uint8_t *>(&xds[wave][0][0]),
              reinterpret_cast<const uint8_t *>(a.q8hd + (size_t)(w.p0 + min(lane, w.n - 1)) * 4));
    dma_wave_copy_nt(T, batched_down(a, w.e) + (size_t)(rt0 + wave * kWaveRows) * kRowBytes, kWaveBytes);
    lds_dma_wait();
    if (tid < w.n) yrow[tid] = pt * (a.k + a.sh) + ps;
    float acc[kChunks][4];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ch][i] = 0.0f;
#pragma unroll 1
    for (int b = 0; b < NBH; ++b) {
        load_x(0, b, x0);
        Q6Fold f;
        q6_fold(T, kRowBytes, b, f);
        if (nch > 1) load_x(1, b, x1);
        q6_fold_step(f, x0, acc[0]);
        if (nch > 1) {
            if (nch > 2) load_x(2, b, x0);
            q6_fold_step(f, x1, acc[1]);
            if (nch > 2) {
                if (nch > 3) load_x(3, b, x1);
                q6_fold_step(f, x0, acc[2]);
                if (nch > 3) q6_fold_step(f, x1, acc[3]);
            }
        }
    }
    __syncthreads();  // yrow is written
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
        const int idx = ch * 16 + c;
        if (ch < nch && idx < w.n) {
            *reinterpret_cast<float4 *>(a.ybuf + (size_t)yrow[idx] * a.n_embd + rt0 + wave * kWaveRows + 4 * q) =
                make_float4(acc[ch][0], acc[ch][1], acc[ch][2], acc[ch][3]);
        }
    }
}

// grid (n_embd / 64, max units), block 256: Q5_K down rows folded as the Q6_K
// ones are (each super-block of the wave's 16 rows folded once, then run against
// every token chunk of the unit); TS = Q6_K: the shared expert's Q6_K rows
// beside them (Qwen3.5), a unit of which takes the Q6_K fold.
template <int NBH, int TS>
__global__ __launch_bounds__(256, 2) void pf_down_q5_kernel(BatchedArgs a) {
    constexpr int kRowBytesD = NBH * kQ5KBytes, kRowBytesS = NBH * QType<TS>::bytes;
    constexpr int kTileBytes = kDnRows * (kRowBytesD > kRowBytesS ? kRowBytesD : kRowBytesS);
    static_assert(TS == kTypeQ5K || TS == kTypeQ6K, "the shared expert's down rows are Q5_K or Q6_K");
    __shared__ __align__(16) uint8_t tile[kTileBytes];
    __shared__ int yrow[kUnitTokens];  // y row (token * slots + slot) of each of the unit's pairs
    __shared__ __align__(16) float xds[4][kUnitTokens][4];  // each wave's copy of the pairs' Q8_K(h) scales
    Unit w;
    if (!load_unit(a, blockIdx.y, w)) return;
    const bool shx = TS != kTypeQ5K && a.sh && w.e == a.n_ids;  // the shared expert's Q6_K rows
    const int rbytes = shx ? kRowBytesS : kRowBytesD;
    const int wave = wave_index(), lane = threadIdx.x & 63, c = lane & 15, q = lane >> 4;
    const int rt0 = blockIdx.x * kDnRows;
    // the pairs' places, read while the tile lands
    const int tid = threadIdx.x;
    const int pt = tid < w.n ? a.ptok[w.p0 + tid] : 0, ps = tid < w.n ? a.pslot[w.p0 + tid] : 0;
    // each wave copies its own 16 rows and waits for them alone
    const int wbytes = kWaveRows * rbytes;  // a multiple of 16 for both row types
    uint8_t *T = tile + wave * wbytes;
    dma_lanes(reinterpret_cast<uint8_t *>(&xds[wave][0][0]),
              reinterpret_cast<const uint8_t *>(a.q8hd + (size_t)(w.p0 + min(lane, w.n - 1)) * 4));
    dma_wave_copy_nt(T, batched_down(a, w.e) + (size_t)(rt0 + wave * kWaveRows) * rbytes, wbytes);
    lds_dma_wait();
    if (tid < w.n) yrow[tid] = pt * (a.k + a.sh) + ps;
    const int nch = (w.n + 15) >> 4;
    const Q8L *q8h = reinterpret_cast<const Q8L *>(a.q8h);
    auto x_of = [&](int ch, int b) -> const Q8L & {
        return q8h[(size_t)(w.p0 + min(ch * 16 + c, w.n - 1)) * NBH + b];
    };
    // the quants from memory, the pairs' block scales from the wave's LDS copy
    auto load_x = [&](int ch, int b, Q6XB &o) {
        q6_load_xq(x_of(ch, b), o);
        o.xd = xds[wave][min(ch * 16 + c, kUnitTokens - 1)][b];
    };
    float acc[kChunks][4], accm[kChunks][4];
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[ch][i] = accm[ch][i] = 0.0f;
    if (shx) {
        if constexpr (TS == kTypeQ6K) {
#pragma unroll 1
            for (int b = 0; b < NBH; ++b) {
                Q6XB xc[kChunks];
#pragma unroll
                for (int ch = 0; ch < kChunks; ++ch)
                    if (ch < nch) load_x(ch, b, xc[ch]);
                Q6Fold f;
                q6_fold(T, kRowBytesS, b, f);
#pragma unroll
                for (int ch = 0; ch < kChunks; ++ch)
                    if (ch < nch) q6_fold_step(f, xc[ch], acc[ch]);
            }
        }
    } else {
#pragma unroll 1
        for (int b = 0; b < NBH; ++b) {
            Q6XB xc[kChunks];
#pragma unroll
            for (int ch = 0; ch < kChunks; ++ch)
                if (ch < nch) load_x(ch, b, xc[ch]);
            Q5Fold f;
            q5_fold(T, kRowBytesD, b, f);
#pragma unroll
            for (int ch = 0; ch < kChunks; ++ch)
                if (ch < nch) q5_fold_step(f, xc[ch], acc[ch], accm[ch]);
        }
    }
    __syncthreads();  // yrow is written
#pragma unroll
    for (int ch = 0; ch < kChunks; ++ch) {
        const int idx = ch * 16 + c;
        if (ch < nch && idx < w.n) {
            *reinterpret_cast<float4 *>(a.ybuf + (size_t)yrow[idx] * a.n_embd + rt0 + wave * kWaveRows + 4 * q) =
                make_float4(acc[ch][0] - accm[ch][0], acc[ch][1] - accm[ch][1], acc[ch][2] - accm[ch][2],
                            acc[ch][3] - accm[ch][3]);  // accm stays 0 for Q6_K rows
        }
    }
}

// -- combine: out[t][d] = (sum_j w[t][j] * y[t][j][d]) + res[t][d], j ascending --
__global__ __launch_bounds__(256) void pf_combine_kernel(BatchedArgs a) {
    // four consecutive elements a thread (n_embd is a multiple of 1024): at
    // hundreds of tokens the wider loads pay; at 16 tokens the one-element
    // form of the batched path keeps more workgroups in flight
    const int t = blockIdx.y;
    const int d = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (d >= a.n_embd) return;
    float4 *o = reinterpret_cast<float4 *>(a.out + (size_t)t * a.n_embd + d);
    if (a.bad && a.bad[t]) {  // an id outside the pool or expert set: the token's row is poisoned
        const float nan = __builtin_nanf("");
        *o = make_float4(nan, nan, nan, nan);
        return;
    }
    const int kk = a.k + a.sh;
    // every load is issued before the first is used: one memory latency, not k
    float w[kMaxK];
    float4 y[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        if (j < a.k) {
            const int js = a.ysrc ? a.ysrc[t * a.k + j] : j;  // a repeated id takes its first output
            w[j] = a.wsel[t * a.k + j];
            y[j] = *reinterpret_cast<const float4 *>(a.ybuf + ((size_t)t * kk + js) * a.n_embd + d);
        }
    }
    const float4 ysh = a.sh ? *reinterpret_cast<const float4 *>(a.ybuf + ((size_t)t * kk + a.k) * a.n_embd + d)
                            : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 r = *reinterpret_cast<const float4 *>(a.res + (size_t)t * a.n_embd + d);
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        if (j < a.k) {
            acc.x = acc.x + w[j] * y[j].x;
            acc.y = acc.y + w[j] * y[j].y;
            acc.z = acc.z + w[j] * y[j].z;
            acc.w = acc.w + w[j] * y[j].w;
        }
    }
    if (a.sh) {  // + sigmoid(gate logit) * shared expert output
        const float sg = 1.0f / (1.0f + expf(-a.sgl[t]));
        acc.x = acc.x + ysh.x * sg;
        acc.y = acc.y + ysh.y * sg;
        acc.z = acc.z + ysh.z * sg;
        acc.w = acc.w + ysh.w * sg;
    }
    *o = make_float4(acc.x + r.x, acc.y + r.y, acc.z + r.z, acc.w + r.w);
}

}  // namespace

hipError_t launch_prefill_groups(const BatchedArgs &a, hipStream_t s) {
    const int nbh = a.n_ff / QK;
    if (a.n_embd != 2048 || a.n_ff % kGuRows || a.n_embd % kDnRows || nbh > 4 || a.max_units < 1)
        return hipErrorInvalidValue;
    if (a.gu_type == kTypeQ4K)
        hipLaunchKernelGGL(pf_gateup_kernel<8>, dim3(a.n_ff / kGuRows, a.max_units), dim3(256), 0, s, a);
    else if (a.gu_type == kTypeQ3K)
        hipLaunchKernelGGL(pf_gateup_q3_kernel<8>, dim3(a.n_ff / kGuRows, a.max_units), dim3(256), 0, s, a);
    else
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(pf_quant_h_kernel, dim3(a.M * (a.k + a.sh)), dim3(64 * nbh), 0, s, a);
    const dim3 dg(a.n_embd / kDnRows, a.max_units);
    const int sd = a.sh ? a.sh_d_type : a.d_type;
// one kernel instance per (routed down type, super-blocks per row, shared down type)
#define HOARD_DOWN(T, N, TS, K)                                          \
    if (a.d_type == T && nbh == N && sd == TS) {                         \
        hipLaunchKernelGGL((K), dg, dim3(256), 0, s, a);                 \
    } else
    HOARD_DOWN(kTypeQ6K, 3, kTypeQ6K, pf_down_q6_kernel<3>)
    HOARD_DOWN(kTypeQ6K, 2, kTypeQ6K, pf_down_q6_kernel<2>)
    HOARD_DOWN(kTypeQ6K, 4, kTypeQ6K, pf_down_q6_kernel<4>)
    HOARD_DOWN(kTypeQ4K, 4, kTypeQ4K, pf_down_q4_kernel<4>)
    HOARD_DOWN(kTypeQ4K, 3, kTypeQ4K, pf_down_q4_kernel<3>)
    HOARD_DOWN(kTypeQ4K, 2, kTypeQ4K, pf_down_q4_kernel<2>)
    HOARD_DOWN(kTypeQ5K, 4, kTypeQ5K, (pf_down_q5_kernel<4, kTypeQ5K>))
    HOARD_DOWN(kTypeQ5K, 2, kTypeQ5K, (pf_down_q5_kernel<2, kTypeQ5K>))
    HOARD_DOWN(kTypeQ5K, 2, kTypeQ6K, (pf_down_q5_kernel<2, kTypeQ6K>)) {
        return hipErrorInvalidValue;
    }
#undef HOARD_DOWN
    hipLaunchKernelGGL(pf_combine_kernel, dim3((a.n_embd + 1023) / 1024, a.M), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace hoard
