// One-launch stacked decode with every selected expert's rows spread over all
// 256 workgroups (one per CU): the shape for many small experts, where the
// k routed experts plus a shared one do not map one expert to one XCD
// (Qwen3-Next: 512 experts, top-10 of ff 512, a gated shared expert).
//
// Replaces, for a whole token, the reference's per-layer loop of graph A's
// router tail (src/run_qwen35.cpp:554-580), graph B with the shared expert
// (:640-665) and the host combine (:675-676), with no host round trip.
//
// The U = k (+1 with a shared expert) expert units are laid end to end.
// Workgroup g = 32*xcd + rank (of 256) owns, per layer,
//   * router rows [RR*g, RR*g + RR) (RR = E/256);
//   * routed h rows [HR*g, HR*g + HR) of the k selected experts' h laid end
//     to end (HR = k*ff/256; a range may cross from one expert into the
//     next) and shared-expert h rows [HS*g, HS*g + HS);
//   * U blocks of 8 down rows, blocks U*g .. U*g + U-1 of the U*256 blocks
//     laid out unit by unit: rows of at most two units, so it needs the h
//     of at most two experts;
//   * the combine of output rows [64*rank, 64*rank + 64), which every XCD
//     forms for itself from the expert outputs y of all units.
// Exchanges, as {value, seq} words:
//   logits  all-to-all across XCDs, pushed into one mailbox per workgroup
//           (a line polled by many workgroups queues on the few memory
//           channels that hold it);
//   h       per unit, producers to the ~24 workgroups holding its down rows;
//   y       every row to the 8 workgroups (one per XCD) that combine it;
//   x       inside each XCD, through its L2.
// No buffer needs a second copy for the next layer: before any workgroup
// writes a word of layer l+1, the exchanges in between have made every
// reader of layer l's word read it.
//
// Top-k over E <= 512 probabilities: one per thread, keyed (probability bits,
// inverted index) so larger keys come first and ties go to the lower index;
// each wave finds its k best by a bitwise search for its k-th largest
// probability, and the k best of every wave (8k candidates) are ranked against
// each other.
#include "exchange.h"
#include "kernels.h"
#include "lds_dma.h"
#include "qblocks.h"
#include "rowdot.h"
#include "wave.h"

namespace hoard {

namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kGroups = 256;  // workgroups, one per CU
constexpr int kXcds = 8;
constexpr int kPerXcd = 32;
constexpr int kFlagStride = 32;   // ticket counters one 128-byte line apart

constexpr int align16(int v) { return (v + 15) & ~15; }

// Shape constants and LDS layout of one instantiation (byte offsets, 16-byte aligned).
template <int NB, int NBH, int K, int E, bool SH, int TD, int TS>
struct SpreadShape {
    static constexpr int kEmbd = NB * QK;
    static constexpr int kFF = NBH * QK;
    static constexpr int U = K + (SH ? 1 : 0);          // expert units: routed slots, then the shared expert
    static constexpr int HR = K * kFF / kGroups;        // routed h rows per workgroup
    static constexpr int HS = SH ? kFF / kGroups : 0;   // shared h rows per workgroup
    static constexpr int NH = U * kFF;                  // h words
    static constexpr int RR = E >= kGroups ? E / kGroups : 1;  // router rows per workgroup
    static constexpr int BLK = 8;                       // rows per down block
    static constexpr int NBLK = kEmbd / BLK;            // down blocks per unit
    static constexpr int NDR = U * BLK;                 // down rows per workgroup (U blocks)
    static constexpr int RC = kEmbd / kPerXcd;          // combined rows per workgroup
    static constexpr int RBG = NB * kQ4KBytes;          // gate/up row bytes
    static constexpr int RBD = NBH * QType<TD>::bytes;  // routed down row bytes
    static constexpr int RBDS = NBH * QType<TS>::bytes; // shared down row bytes
    static constexpr int RBDM = RBD > RBDS ? RBD : RBDS;
    static constexpr int NGU = 2 * HR;                  // routed gate/up rows dotted per workgroup
    static constexpr int kGuWaves = (NGU + 7) / 8;      // waves with gate/up rows (8 per wave)
    static constexpr bool kTwoCopyWaves = kGuWaves <= 5;  // wave 5 free to copy a second down segment
    static constexpr int kCand = 8 * K;                 // top-k candidates, k per wave
    static constexpr int kGatherH = 2 * kFF / 256;      // h words per gathering thread (waves 0-3, two units)

    static_assert(NB == 8, "one 8-lane group per gate/up row, one lane per super-block");
    static_assert((K * kFF) % kGroups == 0 && (!SH || kFF % kGroups == 0), "h rows split evenly");
    static_assert(E <= kThreads && (E % kGroups == 0 || kGroups % E == 0) && RR <= 2, "router rows per workgroup");
    static_assert(K <= 16 && K <= E && 4 * kCand <= kThreads, "top-k");
    static_assert(NBLK == kGroups && U <= NBLK, "U down blocks per workgroup, from at most two units");
    static_assert(NGU <= 48, "gate/up rows on waves 0-5");
    static_assert(HR <= 64 && 2 * HS <= 8, "h published by one wave; shared rows on one wave");
    static_assert(RC == 64 && U <= 16, "one combined row per lane of one wave");
    static_assert(2 * NBH <= 6, "Q8_K(h) of two units on waves 0-5");
    static_assert((BLK * RBD) % 16 == 0 && (BLK * RBDS) % 16 == 0, "down segments start 16-byte aligned");
    static_assert((TD == kTypeQ6K || TD == kTypeQ5K) && (TS == kTypeQ6K || TS == kTypeQ5K) && (SH || TS == TD),
                  "Q6_K or Q5_K down rows");

    static constexpr int oXS = 0;
    static constexpr int oWR = oXS + 4 * kEmbd;
    static constexpr int oSGR = oWR + 4 * RR * kEmbd;
    static constexpr int oSHGU = oSGR + (SH ? 4 * kEmbd : 0);
    static constexpr int oGU = align16(oSHGU + 2 * HS * RBG);
    static constexpr int oDN = align16(oGU + 2 * HR * RBG);
    static constexpr int oQ8X = align16(oDN + NDR * RBDM);
    static constexpr int oQ8H = oQ8X + (int)sizeof(Q8L) * NB;
    static constexpr int oHB = oQ8H + (int)sizeof(Q8L) * 2 * NBH;
    static constexpr int oLG = oHB + 4 * 2 * kFF;
    static constexpr int oCAND = oLG + 4 * kThreads;
    static constexpr int oGUV = oCAND + 8 * kCand;
    static constexpr int oYS = align16(oGUV + 4 * NGU);
    static constexpr int kBytes = align16(oYS + 4 * NDR);
};

// Copy nbytes (a multiple of 16) from src to LDS at dst as 1 KB chunks.  The
// chunks of consecutive calls form one stream numbered from `base`, dealt
// round-robin to nw waves; the calling wave is number wrel of them.  Lanes
// past the end copy nothing, so exactly [src, src + nbytes) is read.
// Returns the chunk number after this segment.
// NT: expert weights, copied with the non-temporal (streaming) cache policy.
template <bool NT = false>
__device__ __forceinline__ int dma_seg(uint8_t *dst, const uint8_t *src, int nbytes, int base, int wrel, int nw) {
    const int lane = threadIdx.x & 63;
    const int nch = (nbytes + 1023) >> 10;
    for (int c = ((wrel - base) % nw + nw) % nw; c < nch; c += nw)
        if (c * 1024 + 16 * lane < nbytes) {
            if constexpr (NT)
                dma_chunk_nt(dst + c * 1024, src + (size_t)c * 1024);
            else
                dma_chunk(dst + c * 1024, src + (size_t)c * 1024);
        }
    return base + nch;
}

// ggml's x86 f32 dot of one row held by a 32-lane half-wave against x*scale:
// lane l accumulates elements 32i + l with fma, i ascending, then the fold.
// Exact in lane 0 of the half-wave.
template <int N>
__device__ __forceinline__ float half_wave_dot(const float *w, const float *x, float scale) {
    const int l32 = threadIdx.x & 31;
    const float *wr = w + l32;
    const float *fr = x + l32;
    float acc = 0.0f;
    for (int i0 = 0; i0 < N; i0 += 32 * 16) {
        float wv[16], fv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            wv[j] = wr[i0 + 32 * j];
            fv[j] = fr[i0 + 32 * j] * scale;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) acc = fmaf(wv[j], fv[j], acc);
    }
    acc = acc + __shfl_xor(acc, 16);  // accumulators a and a+16
    return row16_ggml_fold(acc);
}

// One down row of type T (NBH super-blocks) against unit lu's Q8_K(h), by an
// 8-lane group (each lane an eighth of every super-block); valid in lane 0.
template <int T, int NBH>
__device__ __forceinline__ void down_row(const uint8_t *row, const Q8L *q8h, int lu, int t8, float *out) {
    if constexpr (T == kTypeQ6K) {
        const float y = g8_row_q6k_u<NBH>(row, q8h + lu * NBH, t8);
        if (t8 == 0) *out = y;
    } else {
        const float y = g8_row_q5k(row, q8h + lu * NBH, NBH, t8);
        if (t8 == 0) *out = y;
    }
}

template <int NB, int NBH, int K, int E, bool SH, int TD, int TS>
__global__ __launch_bounds__(kThreads) void spread_kernel(SpreadArgs a) {
    using S = SpreadShape<NB, NBH, K, E, SH, TD, TS>;
    constexpr int kEmbd = S::kEmbd, kFF = S::kFF, U = S::U, HR = S::HR, HS = S::HS, RR = S::RR;
    constexpr int BLK = S::BLK, NBLK = S::NBLK, NDR = S::NDR, RC = S::RC;
    constexpr int RBG = S::RBG, NGU = S::NGU, kCand = S::kCand;

    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red_mx[kWaves];
    __shared__ double red_ss[kWaves], red_sum[kWaves];
    __shared__ int sel_s[16];
    __shared__ float w_s[16];
    __shared__ float sg_s;
    __shared__ int fail_s, rank_s;
    __shared__ unsigned seq_s;
    __shared__ unsigned gu_done;  // waves 0-5 done with their gate/up rows, counted over layers

    const int tid = threadIdx.x, wave = wave_index(), lane = tid & 63;
    const int grp = tid >> 3, t8 = tid & 7;
    const unsigned xcc = xcc_id();
    if (tid == 0) {
        const unsigned t = __hip_atomic_fetch_add(a.tickets + xcc * kFlagStride, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        rank_s = (int)(t % kPerXcd);
        fail_s = 0;
        seq_s = seq_begin(a.seq);
        gu_done = 0;
    }
    __syncthreads();
    const int rank = rank_s;
    const unsigned seq0 = seq_s;
    const int g = (int)xcc * kPerXcd + rank;

    float *xs = reinterpret_cast<float *>(smem + S::oXS);
    const float *wr = reinterpret_cast<const float *>(smem + S::oWR);
    Q8L *q8x = reinterpret_cast<Q8L *>(smem + S::oQ8X);
    Q8L *q8h = reinterpret_cast<Q8L *>(smem + S::oQ8H);
    float *hb = reinterpret_cast<float *>(smem + S::oHB);
    float *lgv = reinterpret_cast<float *>(smem + S::oLG);
    uint64_t *cand = reinterpret_cast<uint64_t *>(smem + S::oCAND);
    float *guv = reinterpret_cast<float *>(smem + S::oGUV);
    float *ys = reinterpret_cast<float *>(smem + S::oYS);

    // routed h rows: unit u0 rows [r0, r0 + n0), then unit u0 + 1 rows [0, n1)
    const int h0 = g * HR, u0 = h0 / kFF, r0 = h0 % kFF;
    const int n0 = HR < kFF - r0 ? HR : kFF - r0, n1 = HR - n0;
    // down blocks: unit ua blocks [ba, ba + na), then unit ua + 1 blocks [0, nbb)
    const int q0 = g * U, ua = q0 / NBLK, ba = q0 % NBLK;
    const int na = U < NBLK - ba ? U : NBLK - ba, nbb = U - na;
    const int nunits = nbb ? 2 : 1;  // units whose h this workgroup needs
    const int RBa = ua < K ? S::RBD : S::RBDS, RBb = ua + 1 < K ? S::RBD : S::RBDS;  // row bytes of the two units
    const int rrow0 = g * RR;
    const bool has_router = rrow0 < E;

    // phase stamps: [layer][workgroup][phase], by thread 0
    auto stamp = [&](int l, int phase) {
        if (a.trace && tid == 0) a.trace[((size_t)(l - a.l0) * kGroups + g) * kTracePhases + phase] = wall_clock64();
    };

    // Router rows, the shared expert's gate row and gate/up rows of layer l:
    // none depends on the routing.
    auto prefetch = [&](int l, int w0, int nw) {
        if (wave < w0 || wave >= w0 + nw) return;
        const DecodeLayer &L = a.layers[l];
        const int wrel = wave - w0;
        int b = 0;
        if (has_router)
            b = dma_seg(smem + S::oWR, reinterpret_cast<const uint8_t *>(L.router + (size_t)rrow0 * kEmbd),
                        4 * RR * kEmbd, b, wrel, nw);
        if constexpr (SH) {
            b = dma_seg(smem + S::oSGR, reinterpret_cast<const uint8_t *>(L.sh_gate_inp), 4 * kEmbd, b, wrel, nw);
            b = dma_seg<true>(smem + S::oSHGU, L.sh_gate + (size_t)g * HS * RBG, HS * RBG, b, wrel, nw);
            b = dma_seg<true>(smem + S::oSHGU + HS * RBG, L.sh_up + (size_t)g * HS * RBG, HS * RBG, b, wrel, nw);
        }
    };

    prefetch(a.l0, 0, kWaves);
    double ss = 0.0;  // this thread's part of sum(x*x), for rms_norm
    for (int i = tid; i < kEmbd; i += kThreads) {
        const float v = a.x[i];
        xs[i] = v;
        ss += (double)(v * v);
    }

    for (int l = a.l0; l < a.l1; ++l) {
        const DecodeLayer &L = a.layers[l];
        const unsigned seq = seq0 + 4u * (unsigned)(l - a.l0);
        const bool last = l + 1 == a.l1;
        stamp(l, 0);

        // -- x of this layer, from this XCD's combine: waves 4-7 gather it (waves 0-3
        //    issued the prefetch of this layer's rows) --
        if (l > a.l0) {
            ss = 0.0;
            if (wave >= 4) {
                const int t4 = tid - 256;
                const uint64_t *xsrc = a.X + (size_t)xcc * kEmbd;
                uint64_t w[8];
                const bool got = poll(
                    [&]() {
                        bool r = true;
#pragma unroll
                        for (int c = 0; c < 8; ++c) w[c] = ld_l2(xsrc + t4 + 256 * c);
#pragma unroll
                        for (int c = 0; c < 8; ++c) r = r & (tag_seq(w[c]) == seq - 1u);
                        return r;
                    },
                    a.err, a.wait_ticks);
                if (!got) fail_s = 1;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const float v = tag_val(w[c]);
                    xs[t4 + 256 * c] = v;
                    ss += (double)(v * v);
                }
            }
        }
        lds_dma_wait();  // the prefetch this wave issued
        ss = wave_sum_d(ss);
        if (lane == 0) red_ss[wave] = ss;
        lds_barrier();
        stamp(l, 1);

        // rms_norm scale; fx = x*scale is formed where it is read
        float scale;
        {
            double tot = 0.0;
            for (int w = 0; w < kWaves; ++w) tot += red_ss[w];
            static_assert((kEmbd & (kEmbd - 1)) == 0, "n_embd a power of two: the mean is an exact multiply");
            const float mean = (float)(tot * (1.0 / (double)kEmbd));
            scale = 1.0f / sqrtf(mean + a.eps);
        }

        // -- router rows (wave 4), shared gate (wave 5), Q8_K(fx) (waves 4-7); logits gathered by waves 0-3 --
        if (wave == 4 && has_router) {
            const int row = lane >> 5;
            float r = 0.0f;
            if (row < RR && rrow0 + row < E) r = half_wave_dot<kEmbd>(wr + (size_t)row * kEmbd, xs, scale);
            // each half-wave's lane 0 holds its row; lanes 0-7 write row 0, lanes 8-15 row 1
            const float r0 = readlane_f(r, 0), r1 = readlane_f(r, 32);
            const int c = lane & 7, rr = lane >> 3;
            if (rr < RR && rrow0 + rr < E) st_dev64(a.LG + (size_t)c * E + rrow0 + rr, tag(rr ? r1 : r0, seq));
        }
        if constexpr (SH) {
            if (wave == 5 && lane < 32) {
                const float r = half_wave_dot<kEmbd>(reinterpret_cast<const float *>(smem + S::oSGR), xs, scale);
                if (lane == 0) sg_s = 1.0f / (1.0f + expf(-r));
            }
        }
        if (wave >= 4) {
            for (int b = wave - 4; b < NB; b += 4) {
                const float4 x4 = *reinterpret_cast<const float4 *>(xs + b * QK + 4 * lane);
                const float v[4] = {x4.x * scale, x4.y * scale, x4.z * scale, x4.w * scale};
                wave_quantize_q8l_regs(v, &q8x[b]);
            }
        } else if (wave == 0) {
            // one wave polls the XCD's copy: fewer requests on its few lines
            constexpr int kPer = (E + 63) / 64;
            const uint64_t *lsrc = a.LG + (size_t)xcc * E;
            uint64_t w[kPer];
            const bool got = poll(
                [&]() {
                    bool r = true;
#pragma unroll
                    for (int c = 0; c < kPer; ++c) w[c] = ld_dev64(lsrc + (lane + 64 * c < E ? lane + 64 * c : 0));
#pragma unroll
                    for (int c = 0; c < kPer; ++c) r = r & (tag_seq(w[c]) == seq);
                    return (bool)__all(r);
                },
                a.err, a.wait_ticks);
            if (!got) fail_s = 1;
            float m = -INFINITY;
#pragma unroll
            for (int c = 0; c < kThreads / 64; ++c) {
                const int i = lane + 64 * c;
                const float v = c < kPer && i < E ? tag_val(w[c < kPer ? c : 0]) : -INFINITY;
                lgv[i] = v;
                m = v > m ? v : m;
            }
            m = wave_max_f(m);
            if (lane == 0) red_mx[0] = red_mx[1] = red_mx[2] = red_mx[3] = m;
        }
        lds_barrier();
        stamp(l, 2);

        // -- softmax over all E (thread t: expert t), then the top-k --
        float pt;
        {
            float mx = red_mx[0];
#pragma unroll
            for (int w = 1; w < 4; ++w) mx = red_mx[w] > mx ? red_mx[w] : mx;
            const float et = tid < E ? expf(lgv[tid] - mx) : 0.0f;
            const double s = wave_sum_d((double)et);
            if (lane == 0) red_sum[wave] = s;
            lds_barrier();
            stamp(l, 3);
            double tot = 0.0;
            for (int w = 0; w < kWaves; ++w) tot += red_sum[w];
            pt = et * (float)(1.0 / tot);
        }
        {
            // key: probability bits over the inverted index (probabilities are >= +0, so
            // their bit patterns order as the values); absent experts rank last
            const uint64_t inv = (uint64_t)(0xFFFFu - (unsigned)tid);
            const uint64_t key = tid < E ? (((uint64_t)__float_as_uint(pt) << 16) | inv) : inv;
            // this wave's k best: the k-th largest probability bit pattern T by a
            // bitwise search (32-bit compares), every lane above T, and of the lanes
            // equal to T the lowest (lower lane = lower index) until there are k
            const uint32_t pb = tid < E ? __float_as_uint(pt) : 0u;
            uint32_t T = 0;
#pragma unroll
            for (int b = 31; b >= 0; --b) {
                const uint32_t tc = T | (1u << b);
                const uint64_t m = __builtin_amdgcn_ballot_w64(pb >= tc);
                // two 32-bit counts keep the test on the scalar unit
                const int cnt = __builtin_popcount((uint32_t)m) + __builtin_popcount((uint32_t)(m >> 32));
                if (cnt >= K) T = tc;
            }
            const uint64_t lt = (1ull << lane) - 1ull;
            const uint64_t eq = __builtin_amdgcn_ballot_w64(pb == T);
            const int need = K - (int)__popcll(__builtin_amdgcn_ballot_w64(pb > T));
            const bool in = pb > T || (pb == T && (int)__popcll(eq & lt) < need);  // exactly k lanes
            if (in) cand[wave * K + __popcll(__builtin_amdgcn_ballot_w64(in) & lt)] = key;
            stamp(l, 4);
        }
        lds_barrier();
        if (tid < 4 * kCand) {
            // rank among the candidates: four lanes per candidate, a quarter each
            constexpr int kSpan = kCand / 4;
            const int c = tid >> 2, q = tid & 3;
            const uint64_t kc = cand[c];
            int r2 = 0;
#pragma unroll
            for (int j = 0; j < kSpan; ++j) r2 += (int)(cand[q * kSpan + j] > kc);
            r2 = group4_sum(r2);
            if (q == 0 && r2 < K) {
                sel_s[r2] = (int)(0xFFFFu - (unsigned)(kc & 0xFFFFu));
                w_s[r2] = __uint_as_float((unsigned)(kc >> 16));
            }
        }
        lds_barrier();
        stamp(l, 5);

        // -- waves 0-5 stream this workgroup's routed gate/up rows into LDS --
        auto expert = [&](int u) {
            const int e = sel_s[u];
            return (e < 0 || e >= E) ? 0 : e;
        };
        if (wave < 6) {
            __builtin_amdgcn_s_waitcnt(0);  // ordinary loads first: the copies retire behind them
            const size_t e0 = (size_t)expert(u0), e1 = n1 ? (size_t)expert(u0 + 1) : 0;
            int b = 0;
            b = dma_seg<true>(smem + S::oGU, L.gate + e0 * L.gstride + (size_t)r0 * RBG, n0 * RBG, b, wave, 6);
            if (n1) b = dma_seg<true>(smem + S::oGU + n0 * RBG, L.gate + e1 * L.gstride, n1 * RBG, b, wave, 6);
            b = dma_seg<true>(smem + S::oGU + HR * RBG, L.up + e0 * L.ustride + (size_t)r0 * RBG, n0 * RBG, b, wave, 6);
            if (n1) b = dma_seg<true>(smem + S::oGU + (HR + n0) * RBG, L.up + e1 * L.ustride, n1 * RBG, b, wave, 6);
        } else if (wave == 7) {
            // renormalise the weights (read only by the combine): every lane forms the
            // same left-to-right sum; lane j normalises weight j
            float ws = 0.0f;
#pragma unroll
            for (int j = 0; j < K; ++j) ws = ws + w_s[j];
            float wj = lane < K ? w_s[lane] : 0.0f;
            if (a.renorm) {
                if (ws < 6.103515625e-5f) ws = 6.103515625e-5f;
                wj = wj / ws;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // every lane's reads precede the writes
            if (lane < K) w_s[lane] = wj;
            if constexpr (SH) {
                // the shared expert's gate/up rows (prefetched) while the routed rows
                // stream in: its h goes out a phase early
                const int sr = lane >> 3;  // rows: HS gate, then HS up
                float v = 0.0f;
                if (sr < 2 * HS) v = lpb_row_q4k_mem<NB>(smem + S::oSHGU + sr * RBG, q8x[t8], t8);
                // row sr's value is in lane 8*sr + 7
#pragma unroll
                for (int i = 0; i < HS; ++i) {
                    const float gv = readlane_f(v, 8 * i + 7), uv = readlane_f(v, 8 * (HS + i) + 7);
                    if (lane == i) st_dev64(a.H + K * kFF + g * HS + i, tag(gv / (1.0f + expf(-gv)) * uv, seq + 1u));
                }
            }
        }
        if (wave < 6) lds_dma_wait();
        lds_barrier();
        stamp(l, 6);

        // -- gate/up rows on the first kGuWaves waves; wave 6 (and wave 5 when it has
        //    no rows) streams the down rows; wave 7 publishes h once the row waves
        //    have counted themselves done (no barrier: the copying waves may still
        //    be issuing).  Rows of two experts are two segments in different pages:
        //    where a second wave is free each goes out from its own wave, so their
        //    address translations are not waited for one after the other. --
        const uint8_t *srcA = ua < K ? L.down + (size_t)expert(ua) * L.dstride : L.sh_down;
        const uint8_t *srcB = ua + 1 < K ? L.down + (size_t)expert(ua + 1) * L.dstride : L.sh_down;
        if (wave == 6) {
            const int b = dma_seg<true>(smem + S::oDN, srcA + (size_t)ba * BLK * RBa, na * BLK * RBa, 0, 0, 1);
            if (nbb && !S::kTwoCopyWaves) dma_seg<true>(smem + S::oDN + na * BLK * RBa, srcB, nbb * BLK * RBb, b, 0, 1);
        } else if (S::kTwoCopyWaves && wave == 5) {
            if (nbb) dma_seg<true>(smem + S::oDN + na * BLK * RBa, srcB, nbb * BLK * RBb, 0, 0, 1);
        } else if (wave < S::kGuWaves) {
            if (grp < NGU) {
                // one row per 8-lane group: the lane reads its activation block as it goes
                const float v = lpb_row_q4k_mem<NB>(smem + S::oGU + grp * RBG, q8x[t8], t8);
                if (t8 == NB - 1) guv[grp] = v;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's guv writes precede its count
            if (lane == 0) __hip_atomic_fetch_add(&gu_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        } else if (wave == 7) {
            const unsigned target = (unsigned)S::kGuWaves * (unsigned)(l - a.l0 + 1);
            const bool done = poll(
                [&]() { return __hip_atomic_load(&gu_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target; },
                a.err, a.wait_ticks);
            if (!done) fail_s = 1;
            if (lane < HR) {
                const float gv = guv[lane], uv = guv[HR + lane];
                st_dev64(a.H + h0 + lane, tag(gv / (1.0f + expf(-gv)) * uv, seq + 1u));
            }
        }
        stamp(l, 7);

        // -- h of the (at most two) units of this workgroup's down rows: waves 0-3 --
        if (wave < 4) {
            uint64_t w[S::kGatherH];
            const int lim = nunits * kFF;
            const bool got = poll(
                [&]() {
                    bool r = true;
#pragma unroll
                    for (int c = 0; c < S::kGatherH; ++c) {
                        const int i = tid + 256 * c;
                        w[c] = ld_dev64(a.H + ua * kFF + (i < lim ? i : lim - 1));
                    }
#pragma unroll
                    for (int c = 0; c < S::kGatherH; ++c) r = r & (tag_seq(w[c]) == seq + 1u);
                    return r;
                },
                a.err, a.wait_ticks);
            if (!got) fail_s = 1;
#pragma unroll
            for (int c = 0; c < S::kGatherH; ++c) {
                const int i = tid + 256 * c;
                if (i < lim) hb[i] = tag_val(w[c]);
            }
        }
        if (wave == 6 || (S::kTwoCopyWaves && wave == 5)) lds_dma_wait();
        lds_barrier();
        stamp(l, 8);

        // -- Q8_K(h) of those units, then the down rows --
        if (wave < nunits * NBH) wave_quantize_q8l(hb + wave * QK, &q8h[wave]);
        lds_barrier();
        stamp(l, 9);
        {
            // local row i = 8*block + r; a wave takes rows of one parity, so its rows
            // share their 4-byte alignment
            const int par = wave & 1;
            const int G = (wave >> 1) * 8 + (grp & 7);
#pragma unroll
            for (int pass = 0; pass < (NDR / 2 + 31) / 32; ++pass) {
                const int m = G + 32 * pass;
                if (m < NDR / 2) {
                    const int i = 2 * m + par;
                    const int lu = (q0 + i / BLK) / NBLK - ua;  // 0 or 1
                    const int ia = na * BLK;                    // rows of the first unit
                    const uint8_t *row = smem + S::oDN + (i < ia ? i * RBa : ia * RBa + (i - ia) * RBb);
                    if constexpr (TS == TD) {
                        down_row<TD, NBH>(row, q8h, lu, t8, &ys[i]);
                    } else {
                        if (ua + lu == K)
                            down_row<TS, NBH>(row, q8h, lu, t8, &ys[i]);
                        else
                            down_row<TD, NBH>(row, q8h, lu, t8, &ys[i]);
                    }
                }
            }
        }
        lds_barrier();
        stamp(l, 10);

        // -- y rows out (wave 7); next layer's rows in (waves 1-3); combine (wave 0) --
        if (wave == 7) {
#pragma unroll
            for (int i = lane; i < NDR; i += 64) {
                const int q = q0 + i / BLK;
                const int u = q / NBLK, d = (q % NBLK) * BLK + i % BLK;
                st_dev64(a.Y + (size_t)u * kEmbd + d, tag(ys[i], seq + 2u));
            }
        }
        if (!last) prefetch(l + 1, 1, 3);
        if (wave == 0) {
            // rows [64*rank, 64*rank + 64): units in order, then the shared expert and residual
            const int d = rank * RC + lane;
            uint64_t yw[U];
            const bool got = poll(
                [&]() {
#pragma unroll
                    for (int u = 0; u < U; ++u) yw[u] = ld_dev64(a.Y + (uint32_t)(u * kEmbd + d));
                    bool r = true;
#pragma unroll
                    for (int u = 0; u < U; ++u) r = r & (tag_seq(yw[u]) == seq + 2u);
                    return r;
                },
                a.err, a.wait_ticks);
            if (!got) fail_s = 1;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < K; ++j) acc = acc + w_s[j] * tag_val(yw[j]);
            float o;
            if constexpr (SH)
                o = (acc + tag_val(yw[K]) * sg_s) + xs[d];
            else
                o = acc + xs[d];
            if (last) {
                if (xcc == 0) a.x[d] = o;
            } else {
                st_l2(a.X + (size_t)xcc * kEmbd + d, tag(o, seq + 3u));
            }
        }
        stamp(l, 11);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (fail_s && xcc == 0 && tid < RC) a.x[rank * RC + tid] = __builtin_nanf("");  // the caller sees the failure
    if (tid == 0) seq_end(a.seq, seq0, 4u * (unsigned)(a.l1 - a.l0) + 4u, gridDim.x);
}

}  // namespace

// The shapes with an instantiated kernel: {n_embd/256, n_ff/256, k, E, shared expert,
// routed down type, shared down type}: Qwen3-Next, the Qwen3-30B shape, Qwen3.5.
#define HOARD_SPREAD_SHAPES(X)                   \
    X(8, 2, 10, 512, true, kTypeQ6K, kTypeQ6K)   \
    X(8, 3, 8, 128, false, kTypeQ6K, kTypeQ6K)   \
    X(8, 2, 8, 256, true, kTypeQ5K, kTypeQ6K)

using SpreadFn = void (*)(SpreadArgs);

static SpreadFn spread_fn(const SpreadArgs &a, size_t *lds) {
#define HOARD_PICK(P_NB, P_NBH, P_K, P_E, P_SH, P_TD, P_TS)                                     \
    if (a.n_embd == P_NB * QK && a.n_ff == P_NBH * QK && a.k == P_K && a.E == P_E &&                \
        (a.shared != 0) == P_SH && (a.d_type < 0 || a.d_type == P_TD) &&                            \
        (a.sh_d_type < 0 || !P_SH || a.sh_d_type == P_TS)) {                                        \
        *lds = SpreadShape<P_NB, P_NBH, P_K, P_E, P_SH, P_TD, P_TS>::kBytes;                        \
        return spread_kernel<P_NB, P_NBH, P_K, P_E, P_SH, P_TD, P_TS>;                              \
    }
    HOARD_SPREAD_SHAPES(HOARD_PICK)
#undef HOARD_PICK
    *lds = 0;
    return nullptr;
}

bool spread_shape_compiled(const SpreadArgs &a) {
    size_t lds;
    return spread_fn(a, &lds) != nullptr;
}

hipError_t launch_spread_decode(const SpreadArgs &a, hipStream_t s, bool cooperative) {
    size_t lds = 0;
    const SpreadFn fn = spread_fn(a, &lds);
    if (!fn || lds > kPersistentMaxLds) return hipErrorInvalidConfiguration;
    static SpreadFn attr_set[4] = {};
    int slot = 0;
    while (slot < 4 && attr_set[slot] && attr_set[slot] != fn) ++slot;
    if (slot == 4 || attr_set[slot] != fn) {
        hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        if (slot < 4) attr_set[slot] = fn;
    }
    SpreadArgs args = a;
    void *params[] = {&args};
    if (!cooperative) return hipLaunchKernel((const void *)fn, dim3(kGroups), dim3(kThreads), params, (unsigned)lds, s);
    return hipLaunchCooperativeKernel((const void *)fn, dim3(kGroups), dim3(kThreads), params, (unsigned)lds, s);
}

}  // namespace hoard
