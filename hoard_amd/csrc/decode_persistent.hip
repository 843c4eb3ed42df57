// Persistent stacked decode: every layer of one token in a single cooperative
// launch (router tail, grouped expert FFN, combine, rms_norm between layers).
//
// Replaces, for a whole token, the reference's per-layer loop of graph A's
// router tail (src/run_moe_stream.cpp:353-373), graph B (:424-445) and the
// host combine (:447), with no host round trip between layers.
//
// Mapping onto MI355X (256 CUs in 8 XCDs of 32, one workgroup per CU):
//   * expert slot j of the top-k runs on XCD j; its gate/up rows and down rows
//     are split over that XCD's 32 workgroups, so the h gather stays inside one
//     XCD's L2;
//   * every XCD computes the router (each workgroup E/32 rows, weights
//     prefetched into LDS during the previous layer) and the top-k redundantly,
//     so routing needs no cross-XCD traffic;
//   * only the expert outputs y_j cross XCDs: workgroup (j, r) publishes rows
//     [64r, 64r+64) of y_j with device-coherent stores and a flag, and the
//     workgroups of rank r on every XCD combine exactly those rows;
//   * weights stream straight into LDS with global_load_lds_dwordx4.
// Synchronisation uses per-workgroup flags holding a monotonically increasing
// sequence number (no atomics): XCD-local flags live in the XCD's L2 and are
// polled after invalidating L1; cross-XCD flags and y use device-scope
// (L2-bypassing) loads and stores.  Every wait is bounded by a wall-clock
// timeout that raises an error flag and poisons the output instead of hanging.
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
constexpr int kXcds = 8;
constexpr int kPerXcd = 32;
constexpr int kRankSlots = 128;              // experts the softmax / rank covers (E <= 128)
static_assert(kRankSlots == kThreads / 4, "four threads per expert in the rank");
constexpr int kFlagStride = 32;             // words: one 128-byte line per flag
constexpr int kDecodeK = 8;                     // experts per token: one per XCD
constexpr int kTopkWave = 2;                    // polls the logits, softmax, renorm
constexpr int kPublishWave = 7;                 // stores h and y

// Issue global_load_lds_dwordx4 for [src, src+nbytes) into LDS at dst, in
// 1 KB chunks (64 lanes x 16 B) spread over waves [w0, w0+nw).  Rounds the
// source down to 16 bytes (returned offset) and reads whole chunks, i.e. up to
// 1 KB + 15 bytes past the end, which device allocations keep as padding.
__device__ __forceinline__ int issue_lds_copy(uint8_t *dst, const uint8_t *src, size_t nbytes, int w0, int nw) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(src);
    const uintptr_t a0 = a & ~(uintptr_t)15;
    const int off = (int)(a - a0);
    const int nchunks = (int)((off + nbytes + 1023) >> 10);
    const int wave = threadIdx.x >> 6;
    if (wave >= w0 && wave < w0 + nw) {
        for (int c = wave - w0; c < nchunks; c += nw)
            dma_chunk(dst + c * 1024, reinterpret_cast<const uint8_t *>(a0) + (size_t)c * 1024);
    }
    return off;
}

__host__ __device__ __forceinline__ size_t chunk_region(size_t nbytes) { return ((nbytes + 15 + 1023) >> 10) << 10; }

struct Smem {
    // byte offsets into dynamic LDS
    int xs, w, gate, up, down, q8x, q8h, gu, ys, ps;
};

__host__ __device__ __forceinline__ Smem smem_layout(const PersistentArgs &a, size_t *total) {
    Smem s;
    size_t o = 0;
    auto take = [&](size_t n) {
        const int r = (int)o;
        o += (n + 15) & ~(size_t)15;
        return r;
    };
    s.xs = take(4 * (size_t)a.n_embd);
    s.w = take((size_t)(a.E / kPerXcd) * a.n_embd * 4);
    s.gate = take(chunk_region((size_t)a.rows_gu * a.max_rb_gu));
    s.up = take(chunk_region((size_t)a.rows_gu * a.max_rb_gu));
    s.down = take(chunk_region((size_t)a.rows_d * a.max_rb_d));
    s.q8x = take(sizeof(Q8L) * (a.n_embd / QK));
    s.q8h = take(sizeof(Q8L) * (a.n_ff / QK));
    s.gu = take(4 * 2 * (size_t)a.rows_gu);
    s.ys = take(4 * (size_t)a.rows_d);
    s.ps = take(4 * (size_t)kRankSlots);
    if (total) *total = o;
    return s;
}

// Raw workgroup barrier: LDS writes of every wave are done; global loads,
// stores and LDS DMA may stay in flight (the fence of __syncthreads would wait
// for them).  Waves exchange data only through LDS inside the layer loop, and
// every wave that issued LDS DMA waits for it itself before such a barrier.

// TGU/NB: gate and up type and super-blocks per row (n_embd / 256);
// TD/NBH: down type and super-blocks per row (n_ff / 256).  Compile-time
// shapes keep the code of one instantiation well inside the instruction cache.
template <int TGU, int NB, int TD, int NBH>
__global__ __launch_bounds__(kThreads) void decode_kernel(PersistentArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int sh_rank, sh_fail;
    __shared__ unsigned seq_s;
    __shared__ int sel_s[16];
    __shared__ float w_s[16];
    __shared__ unsigned gu_done;   // gate/up row waves done, counted over layers
    __shared__ double red_d[kWaves];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int grp = tid >> 3, t8 = tid & 7;  // 64 groups of 8 lanes
    const unsigned xcc = xcc_id();
    if (tid == 0) {
        const unsigned t = __hip_atomic_fetch_add(a.tickets + xcc * kFlagStride, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        sh_rank = (int)(t % kPerXcd);
        sh_fail = 0;
        gu_done = 0;
        seq_s = seq_begin(a.seq);
    }
    __syncthreads();
    const int rank = sh_rank;
    const unsigned seq0 = seq_s;
    const Smem S = smem_layout(a, nullptr);
    float *xs = reinterpret_cast<float *>(smem + S.xs);
    const float *wl = reinterpret_cast<const float *>(smem + S.w);
    Q8L *q8x = reinterpret_cast<Q8L *>(smem + S.q8x);
    Q8L *q8h = reinterpret_cast<Q8L *>(smem + S.q8h);
    float *gu = reinterpret_cast<float *>(smem + S.gu);
    float *ys = reinterpret_cast<float *>(smem + S.ys);
    float *ps = reinterpret_cast<float *>(smem + S.ps);

    const int n = a.n_embd, E = a.E, k = a.k;
    const int rw = E / kPerXcd;  // router rows per workgroup
    constexpr int nb = NB, nbh = NBH;
    constexpr int kEmbd = NB * QK;
    static_assert(TGU == kTypeQ4K || TGU == kTypeQ3K, "gate/up rows are Q4_K or Q3_K");
    static_assert(TD == kTypeQ6K || TD == kTypeQ5K || TD == kTypeQ4K, "down rows are Q6_K, Q5_K or Q4_K");
    static_assert(2 * (NBH * QK / kPerXcd) <= kThreads / 8, "one 8-lane group per gate/up row");
    const int R = a.rows_gu, RD = a.rows_d;
    const bool has_expert = (int)xcc < k;
    uint64_t *LGx = a.LG + (size_t)xcc * E;
    uint64_t *Hx = a.H + (size_t)xcc * a.n_ff;

    // phase stamps: [layer][xcc*32 + rank][phase]
    auto stamp = [&](int l, int phase) {
        if (a.trace && tid == 0)
            a.trace[((size_t)(l - a.l0) * (kXcds * kPerXcd) + xcc * kPerXcd + rank) * kTracePhases + phase] =
                wall_clock64();
    };
    auto prefetch_router = [&](int l, int w0, int nw) {
        const DecodeLayer &Lr = a.layers[l];
        issue_lds_copy(smem + S.w, reinterpret_cast<const uint8_t *>(Lr.router + (size_t)rank * rw * n),
                       (size_t)rw * n * 4, w0, nw);
    };

    // ---- prologue: router rows of the first layer, and x ----
    prefetch_router(a.l0, 0, kWaves);
    for (int i = tid; i < n; i += kThreads) xs[i] = a.x[i];

    bool ok = true;
    for (int l = a.l0; l < a.l1; ++l) {
        const DecodeLayer &L = a.layers[l];
        const unsigned seq = seq0 + 4u * (unsigned)(l - a.l0);
        const int cur = (l - a.l0) & 1;
        const bool last = l + 1 == a.l1;
        stamp(l, 0);
        // A wave's vmcnt counts its stores too and retires in order, so a wave that
        // polls must not have stores of its own in flight: each exchange below is
        // published by one set of waves and polled by another.
        if (wave >= kWaves / 2) __builtin_amdgcn_s_waitcnt(0);  // router rows these waves prefetched
        double ss = 0.0;  // this thread's part of sum(x*x), for rms_norm
        if (l == a.l0) {
            for (int i = tid; i < n; i += kThreads) {
                const float v = xs[i];
                ss += (double)(v * v);
            }
        } else if (wave >= kWaves / 2) {
            // x of this layer: the XCD's 32 workgroups published 64 rows each; gathered
            // by waves 4-7 (wave 0 has just stored its combined rows)
            const uint64_t *xsrc = a.X + ((size_t)cur * kXcds + xcc) * n;
            // all four of the thread's word pairs in one probe (one round trip
            // once the data is there), each a 16-byte load; pair c of thread t
            // is words 2 (t + 256 c) and the next, so a wave's load covers 1 KB
            static_assert(kEmbd == 8 * (kThreads / 2), "four word pairs per gathering thread");
            const int t = tid - kThreads / 2;
            uint64_t w[8];
            const bool got = poll(
                [&]() {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        ld_dev64x2(xsrc, (unsigned)kEmbd, (unsigned)(2 * (t + (kThreads / 2) * c)), w[2 * c], w[2 * c + 1]);
                    bool r = true;
#pragma unroll
                    for (int c = 0; c < 8; ++c) r = r & (tag_seq(w[c]) == seq - 1u);
                    return r;
                },
                a.err, a.wait_ticks);
            if (!got) sh_fail = 1;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float v0 = tag_val(w[2 * c]), v1 = tag_val(w[2 * c + 1]);
                *reinterpret_cast<float2 *>(xs + 2 * (t + (kThreads / 2) * c)) = make_float2(v0, v1);
                ss += (double)(v0 * v0);
                ss += (double)(v1 * v1);
            }
        }
        ss = wave_sum_d(ss);
        if (lane == 0) red_d[wave] = ss;
        lds_barrier();
        if (sh_fail) {
            ok = false;
            break;
        }
        stamp(l, 1);

        // -- P1: rms_norm scale, router rows (32 lanes each) --
        // fx = x * scale is formed where it is read (router, Q8_K(fx)): no
        // separate pass over x and no barrier for it
        float scale;
        {
            double tot = 0.0;
            for (int w = 0; w < kWaves; ++w) tot += red_d[w];
            static_assert((kEmbd & (kEmbd - 1)) == 0, "n_embd a power of two: the mean is an exact multiply");
            const float mean = (float)(tot * (1.0 / (double)kEmbd));
            scale = 1.0f / sqrtf(mean + a.eps);
        }
        {
            // lane l of a 32-lane half-wave holds accumulator l of ggml's x86 f32
            // dot (elements 32i + l, i ascending); rows 2w and 2w+1 on wave w
            const int row = 2 * wave + (lane >> 5), l32 = lane & 31;
            if (row < rw) {
                const float *wr = wl + (size_t)row * kEmbd + l32;
                const float *fr = xs + l32;
                float acc = 0.0f;
                for (int i0 = 0; i0 < kEmbd; i0 += 32 * 16) {
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
                const float r = row16_ggml_fold(acc);
                if (l32 == 0) st_l2(LGx + rank * rw + row, tag(r, seq));
            }
        }
        stamp(l, 2);
        stamp(l, 3);

        // -- P2: softmax (wave 2: waves 0-1 stored the logits), ranks (all threads) --
        if (wave == kTopkWave) {
            uint64_t w0 = 0, w1 = 0;
            const bool got = poll(
                [&]() {
                    if (lane < E) w0 = ld_l2(LGx + lane);
                    if (lane + 64 < E) w1 = ld_l2(LGx + lane + 64);
                    const bool r = (lane >= E || tag_seq(w0) == seq) && (lane + 64 >= E || tag_seq(w1) == seq);
                    return (bool)__all(r);
                },
                a.err, a.wait_ticks);
            if (!got && lane == 0) sh_fail = 1;
            float p0 = lane < E ? tag_val(w0) : -INFINITY;
            float p1 = lane + 64 < E ? tag_val(w1) : -INFINITY;
            const float mx = wave_max_f(p0 > p1 ? p0 : p1);
            double sum = 0.0;
            if (lane < E) {
                p0 = expf(p0 - mx);
                sum += (double)p0;
            }
            if (lane + 64 < E) {
                p1 = expf(p1 - mx);
                sum += (double)p1;
            }
            sum = wave_sum_d(sum);
            const float sc = (float)(1.0 / sum);
            // kRankSlots entries; absent experts hold -1, below every probability
            ps[lane] = lane < E ? p0 * sc : -1.0f;
            ps[lane + 64] = lane + 64 < E ? p1 * sc : -1.0f;
            if (lane < 16) sel_s[lane] = -1;
        }
        lds_barrier();
        {
            // rank of expert e = experts ahead of it in (probability desc, index asc)
            // order; four lanes split the kRankSlots comparisons and add their
            // counts.  Fixed trip counts: no branches, no scalar spills.
            const int e = tid >> 2, q = tid & 3;
            constexpr int kSpan = kRankSlots / 4;
            const float pe = ps[e];
            float4 pv[kSpan / 4];
#pragma unroll
            for (int c = 0; c < kSpan / 4; ++c) pv[c] = *reinterpret_cast<const float4 *>(ps + q * kSpan + 4 * c);
            int r = 0;
#pragma unroll
            for (int c = 0; c < kSpan / 4; ++c) {
                const int e4 = q * kSpan + 4 * c;
                r += (pv[c].x > pe) | ((pv[c].x == pe) & (e4 < e));
                r += (pv[c].y > pe) | ((pv[c].y == pe) & (e4 + 1 < e));
                r += (pv[c].z > pe) | ((pv[c].z == pe) & (e4 + 2 < e));
                r += (pv[c].w > pe) | ((pv[c].w == pe) & (e4 + 3 < e));
            }
            r = group4_sum(r);
            if (e < E && q == 0 && r < k) {
                sel_s[r] = e;
                w_s[r] = pe;
            }
        }
        lds_barrier();
        if (sh_fail) {
            ok = false;
            break;
        }
        stamp(l, 4);

        // -- P3: every wave streams its share of the gate/up rows into LDS (more
        // copies in flight at once than from four waves: 12.99 -> 12.83 us a
        // layer); wave 6 copies the down rows in P4 --
        int e = has_expert ? sel_s[xcc] : 0;
        if (e < 0 || e >= E) e = 0;  // only with NaN logits; their weights poison the output
        constexpr size_t rbg = (size_t)NB * QType<TGU>::bytes, rbu = rbg;
        constexpr size_t rbd = (size_t)NBH * QType<TD>::bytes;
        constexpr int kR = NBH * QK / kPerXcd, kRD = kEmbd / kPerXcd;  // rows per workgroup
        constexpr int kGuChunks = (int)((kR * rbg + 1023) / 1024);
        constexpr int kDownChunks = (int)((kRD * rbd + 1023) / 1024);
        static_assert(2 * kR <= kThreads / 8, "one 8-lane group per gate/up row");
        // sources are 16-byte aligned (checked on the host), so rows start at the staged offset 0
        const uint8_t *gsrc = L.gate + (size_t)e * L.gstride + (size_t)rank * kR * rbg;
        const uint8_t *usrc = L.up + (size_t)e * L.ustride + (size_t)rank * kR * rbu;
        const uint8_t *dsrc = L.down + (size_t)e * L.dstride + (size_t)rank * kRD * rbd;
        // Drain this wave's ordinary loads first: the compiler's waits for them
        // count outstanding operations, and the chunks issued below would
        // otherwise be counted in front of them.
        __builtin_amdgcn_s_waitcnt(0);
        if (has_expert) {
            for (int c = wave; c < kGuChunks; c += kWaves) {
                dma_chunk_nt(smem + S.gate + c * 1024, gsrc + (size_t)c * 1024);
                dma_chunk_nt(smem + S.up + c * 1024, usrc + (size_t)c * 1024);
            }
        }
        // Q8_K(fx) while the rows are in flight
        for (int b = wave; b < nb; b += kWaves) {
            const float4 x4 = *reinterpret_cast<const float4 *>(xs + b * QK + 4 * lane);
            const float v[4] = {x4.x * scale, x4.y * scale, x4.z * scale, x4.w * scale};
            wave_quantize_q8l_regs(v, &q8x[b]);
        }
        if (wave == 0) {
            // renormalise the weights (only the combine, on this wave, reads them): every
            // lane forms the same left-to-right sum; lane j normalises weight j
            int sv[kDecodeK];
            float wv[kDecodeK];
#pragma unroll
            for (int j = 0; j < kDecodeK; ++j) {
                sv[j] = sel_s[j];
                wv[j] = w_s[j];
            }
            float ws = 0.0f;
#pragma unroll
            for (int j = 0; j < kDecodeK; ++j)
                ws = ws + ((sv[j] < 0 || sv[j] >= E) ? __builtin_nanf("") : wv[j]);  // NaN logits only
            float wj = 0.0f;
#pragma unroll
            for (int j = 0; j < kDecodeK; ++j)
                if (lane == j) wj = (sv[j] < 0 || sv[j] >= E) ? __builtin_nanf("") : wv[j];
            if (a.renorm) {
                if (ws < 6.103515625e-5f) ws = 6.103515625e-5f;
                wj = wj / ws;
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the reads above precede the writes
            if (lane < k) w_s[lane] = wj;
        }
        stamp(l, 5);

        if (has_expert) {
            // -- P4: gate/up rows on every wave while the down rows still stream --
            __builtin_amdgcn_s_waitcnt(0);  // the gate/up chunks this wave issued
            lds_barrier();
            stamp(l, 6);
            // The down rows are needed only after the h exchange: fetched now, after
            // the gate/up rows, so that those did not share the bandwidth (issuing
            // them together with the gate/up rows measured 14.4 against 13.7 us a
            // layer for Qwen3-30B-A3B: the gate/up fetch is the critical path).  With
            // 2R <= 48 wave 6 has no gate/up row and copies them all, and wave 7
            // publishes h once the row waves have counted themselves done: no
            // barrier, so nothing waits for wave 6 to finish issuing its copies.
            // Otherwise waves 6-7 copy them besides their rows and a barrier
            // precedes the publish.
            constexpr bool kCounted = 2 * kR <= 48;
            constexpr int kGuWaves = (2 * kR + 7) / 8;
            auto gateup_rows = [&]() {
                // one 8-lane group per row; lane t reads Q8_K(x) block t as it goes
                const int pr = grp;
                if (pr < 2 * kR) {
                    const int mat = pr >= kR, row = pr - mat * kR;
                    const uint8_t *rp = mat ? smem + S.up + row * rbu : smem + S.gate + row * rbg;
                    float v;
                    if constexpr (TGU == kTypeQ3K)
                        v = lpb_row_q3k_mem<NB, true>(rp, q8x[t8 < NB ? t8 : 0], t8);
                    else
                        v = lpb_row_q4k_mem<NB>(rp, q8x[t8 < NB ? t8 : 0], t8);
                    if (t8 == NB - 1) gu[pr] = v;
                }
            };
            auto publish_h = [&]() {
                if (lane < R) {
                    const float g = gu[lane], uu = gu[R + lane];
                    st_l2(Hx + rank * R + lane, tag(g / (1.0f + expf(-g)) * uu, seq + 1u));
                }
            };
            if constexpr (kCounted) {
                if (wave == kWaves - 2) {
                    for (int c = 0; c < kDownChunks; ++c) dma_chunk_nt(smem + S.down + c * 1024, dsrc + (size_t)c * 1024);
                } else if (wave < kGuWaves) {
                    gateup_rows();
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's gu writes precede its count
                    if (lane == 0) __hip_atomic_fetch_add(&gu_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                } else if (wave == kPublishWave) {  // not a wave that polls h
                    const unsigned target = (unsigned)kGuWaves * (unsigned)(l - a.l0 + 1);
                    const bool done = poll(
                        [&]() {
                            return __hip_atomic_load(&gu_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= target;
                        },
                        a.err, a.wait_ticks);
                    if (!done) sh_fail = 1;
                    publish_h();
                }
            } else {
                if (wave >= kWaves - 2)
                    for (int c = wave - (kWaves - 2); c < kDownChunks; c += 2)
                        dma_chunk_nt(smem + S.down + c * 1024, dsrc + (size_t)c * 1024);
                gateup_rows();
                lds_barrier();
                if (wave == kPublishWave) publish_h();  // not a wave that polls h
            }
            stamp(l, 7);

            // -- P5: Q8_K(h) of the XCD's expert, down rows, publish y rows --
            if (wave < nbh) {
                uint64_t w[4];
                const bool got = poll(
                    [&]() {
                        // words 4 lane .. 4 lane + 3 of block `wave`, two 16-byte loads
                        ld_dev64x2(Hx, (unsigned)a.n_ff, (unsigned)(wave * QK + 4 * lane), w[0], w[1]);
                        ld_dev64x2(Hx, (unsigned)a.n_ff, (unsigned)(wave * QK + 4 * lane + 2), w[2], w[3]);
                        bool r = true;
#pragma unroll
                        for (int c = 0; c < 4; ++c) r = r && tag_seq(w[c]) == seq + 1u;
                        return (bool)__all(r);
                    },
                    a.err, a.wait_ticks);
                if (!got && lane == 0) sh_fail = 1;
                const float v[4] = {tag_val(w[0]), tag_val(w[1]), tag_val(w[2]), tag_val(w[3])};
                wave_quantize_q8l_regs(v, &q8h[wave]);
            }
            __builtin_amdgcn_s_waitcnt(0);  // down rows landed
            lds_barrier();
            if (sh_fail) {
                ok = false;
                break;
            }
            stamp(l, 8);
            if constexpr (TD == kTypeQ6K || TD == kTypeQ5K) {
                // 8 lanes per row; a wave takes rows of one parity so that its rows
                // share their 4-byte alignment when the row size is 2 mod 4
                const int row = 16 * (wave >> 1) + 2 * (grp & 7) + (wave & 1);
                if (row < RD) {
                    float y;
                    if constexpr (TD == kTypeQ6K)
                        y = g8_row_q6k_u<NBH>(smem + S.down + row * rbd, q8h, t8);
                    else
                        y = g8_row_q5k(smem + S.down + row * rbd, q8h, NBH, t8);
                    if (t8 == 0) ys[row] = y;
                }
            } else {
                Q8Reg hr;
                if (t8 < NBH) load_q8reg(q8h[t8], hr);
                const int row = grp;
                if (row < RD) {
                    const float y = lpb_row_q4k<NBH>(smem + S.down + row * rbd, hr, t8);
                    if (t8 == NBH - 1) ys[row] = y;
                }
            }
            lds_barrier();
            if (wave == kPublishWave) {  // wave 0 polls y next
                uint64_t *Y = a.Y + ((size_t)cur * kXcds + xcc) * n + rank * RD;
                for (int i = lane; i < RD; i += 64) st_dev64(Y + i, tag(ys[i], seq + 2u));
            }
            stamp(l, 9);
        }
        // next layer's router rows, from the waves that gather x next
        if (!last && wave >= kWaves / 2) prefetch_router(l + 1, kWaves / 2, kWaves / 2);

        // -- P6 (wave 0): combine rows [RD*rank, RD*rank+RD) over every expert slot --
        if (wave == 0) {
            for (int t = lane; t < RD; t += 64) {
                const int d = rank * RD + t;
                const float res = xs[d];
                // slots past k read slot 0 again: no branches around the loads
                uint64_t yw[8];
                const bool got = poll2(
                    [&](uint64_t(&w)[8]) {
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            w[j] = ld_dev64(a.Y + ((size_t)cur * kXcds + (j < k ? j : 0)) * n + d);
                    },
                    [&](const uint64_t(&w)[8]) {
                        bool r = true;
#pragma unroll
                        for (int j = 0; j < 8; ++j) r = r & ((j >= k) | (tag_seq(w[j]) == seq + 2u));
                        return r;
                    },
                    yw, a.err, a.wait_ticks);
                if (!got) sh_fail = 1;
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j < k) acc = acc + w_s[j] * tag_val(yw[j]);
                const float o = acc + res;
                if (last) {
                    if (xcc == 0) a.x[d] = o;
                } else {
                    st_l2(a.X + ((size_t)(cur ^ 1) * kXcds + xcc) * n + d, tag(o, seq + 3u));
                }
            }
        }
        stamp(l, 10);
        stamp(l, 11);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if ((!ok || sh_fail) && xcc == 0) {  // poison this workgroup's output rows so the caller sees the failure
        for (int t = tid; t < RD; t += kThreads) a.x[rank * RD + t] = __builtin_nanf("");
    }
    if (tid == 0) seq_end(a.seq, seq0, 4u * (unsigned)(a.l1 - a.l0) + 4u, gridDim.x);
}

}  // namespace

size_t persistent_lds_bytes(const PersistentArgs &a) {
    size_t total = 0;
    smem_layout(a, &total);
    return total;
}

// The shapes with an instantiated kernel: {gate/up type, n_embd, down type, n_ff}.
#define HOARD_PERSISTENT_SHAPES(X)      \
    X(kTypeQ4K, 2048, kTypeQ6K, 768)    \
    X(kTypeQ4K, 2048, kTypeQ4K, 1024)   \
    X(kTypeQ4K, 2048, kTypeQ6K, 512)    \
    X(kTypeQ4K, 2048, kTypeQ6K, 1024)   \
    X(kTypeQ3K, 2048, kTypeQ5K, 1024)

using KernelFn = void (*)(PersistentArgs);

static KernelFn persistent_kernel(int gu_type, int n_embd, int d_type, int n_ff) {
#define HOARD_PICK(TG, N, TD, F) \
    if (gu_type == TG && n_embd == N && d_type == TD && n_ff == F) return decode_kernel<TG, N / QK, TD, F / QK>;
    HOARD_PERSISTENT_SHAPES(HOARD_PICK)
#undef HOARD_PICK
    return nullptr;
}

bool persistent_shape_compiled(int gu_type, int n_embd, int d_type, int n_ff) {
    return persistent_kernel(gu_type, n_embd, d_type, n_ff) != nullptr;
}

hipError_t launch_persistent_decode(const PersistentArgs &a, hipStream_t s, bool cooperative) {
    const KernelFn fn = persistent_kernel(a.gu_type, a.n_embd, a.d_type, a.n_ff);
    if (!fn) return hipErrorInvalidConfiguration;
    const size_t lds = persistent_lds_bytes(a);
    if (lds > kPersistentMaxLds) return hipErrorInvalidConfiguration;
    static struct {
        KernelFn fn;
        size_t lds;
    } set_attr[8] = {};  // dynamic-LDS limit already applied per instantiation
    int slot = 0;
    while (slot < 8 && set_attr[slot].fn && set_attr[slot].fn != fn) ++slot;
    if (slot == 8 || set_attr[slot].fn != fn || set_attr[slot].lds != lds) {
        hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        if (slot < 8) set_attr[slot] = {fn, lds};
    }
    PersistentArgs args = a;
    void *params[] = {&args};
    if (!cooperative)
        return hipLaunchKernel((const void *)fn, dim3(kXcds * kPerXcd), dim3(kThreads), params, (unsigned)lds, s);
    return hipLaunchCooperativeKernel((const void *)fn, dim3(kXcds * kPerXcd), dim3(kThreads), params, (unsigned)lds, s);
}

}  // namespace hoard
