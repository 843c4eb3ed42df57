// Per-layer launches for one token: the path behind hoard_moe_route,
// hoard_moe_ffn_combine and hoard_moe_layer, i.e. the reference's per-layer
// contract where attention and graph A's other nodes run between MoE layers.
//
//   route   router rows -> softmax -> top-k -> renorm
//           (src/run_moe_stream.cpp:353-356, :371-373; src/run_qwen35.cpp:556-559)
//   gateup  gate/up rows of every selected expert (and the shared one) with
//           SwiGLU fused (:431-434; src/run_qwen35.cpp:650-652, :659-663)
//   down    down rows of every selected expert for 8 output rows, fused with
//           the weighted combine, shared expert and residual (:435-447;
//           src/run_qwen35.cpp:653, :664-676)
//
// Each kernel copies its weight rows into LDS with global_load_lds_dwordx4 and
// forms the activation's Q8_K blocks while they are in flight; the row dots
// and every fp32 order are those of the one-launch decode, so the three
// launches give its bits.  The route kernel's last workgroup runs the tail:
// the logits are stored and read at device scope (past the per-XCD L2) and
// each workgroup counts itself done after its stores are acknowledged, with
// no cache-flushing fence.
#include "exchange.h"
#include "kernels.h"
#include "lds_dma.h"
#include "qblocks.h"
#include "router_tail.h"
#include "rowdot.h"
#include "wave.h"

namespace hoard {

namespace {

constexpr int kRouteRows = 4;  // router rows per workgroup: 2 waves x 2 half-waves
constexpr int kGuRows = 16;    // gate rows (and up rows) per workgroup
constexpr int kDownRows = 8;   // output rows per workgroup

// Copy nbytes (a multiple of 16) to LDS from the calling wave alone; lanes
// past the end copy nothing.
__device__ __forceinline__ void wave_copy(uint8_t *dst, const uint8_t *src, int nbytes) {
    const int lane = threadIdx.x & 63;
    for (int c = 0; c * 1024 < nbytes; ++c)
        if (c * 1024 + 16 * lane < nbytes) dma_chunk(dst + c * 1024, src + (size_t)c * 1024);
}
// The same for expert weights, streamed (non-temporal cache policy).
__device__ __forceinline__ void wave_copy_nt(uint8_t *dst, const uint8_t *src, int nbytes) {
    const int lane = threadIdx.x & 63;
    for (int c = 0; c * 1024 < nbytes; ++c)
        if (c * 1024 + 16 * lane < nbytes) dma_chunk_nt(dst + c * 1024, src + (size_t)c * 1024);
}

// -- route --------------------------------------------------------------------
// grid = ceil(E / 4), block = 128.  xin is fx, or (xin_is_residual) x, whose
// rms_norm every workgroup forms for itself; workgroup 0 then writes fx.
template <int N>
__global__ __launch_bounds__(128) void layer_route_kernel(RouterArgs a) {
    __shared__ __align__(16) float xl[N];
    __shared__ __align__(16) float wl[kRouteRows][N];
    __shared__ double red[2];
    __shared__ int last;
    const int E = a.E;
    const int wave = wave_index(), lane = threadIdx.x & 63, l = lane & 31;
    const int r0 = blockIdx.x * kRouteRows;
    const int nrows = min(kRouteRows, E - r0);
    // both copies in flight at once: x on wave 0, the rows split over the waves
    if (wave == 0) wave_copy(reinterpret_cast<uint8_t *>(xl), reinterpret_cast<const uint8_t *>(a.xin), N * 4);
    {
        const int bytes = nrows * N * 4, half = (bytes / 2 + 1023) & ~1023;
        const int off = wave * half, len = min(half, bytes - off);
        if (len > 0)
            wave_copy(reinterpret_cast<uint8_t *>(wl[0]) + off, reinterpret_cast<const uint8_t *>(a.w + (size_t)r0 * N) + off,
                      len);
    }
    lds_dma_wait();
    __syncthreads();
    float scale = 1.0f;
    if (a.xin_is_residual) {
        // rms_norm: mean of x*x in double, scale = 1/sqrtf(mean + eps)
        double ss = 0.0;
        for (int i = threadIdx.x; i < N; i += 128) {
            const float v = xl[i];
            ss += (double)(v * v);
        }
        ss = wave_sum_d(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        const float mean = (float)((red[0] + red[1]) * (1.0 / (double)N));
        scale = 1.0f / sqrtf(mean + a.eps);
        if (blockIdx.x == 0)
            for (int i = threadIdx.x; i < N; i += 128) a.fx_out[i] = xl[i] * scale;
    }
    const int rr = 2 * wave + (lane >> 5);
    if (rr < nrows) {
        // ggml's x86 f32 dot: lane l accumulates elements 32i + l, i ascending
        const float *wr = wl[rr] + l;
        const float *xr = xl + l;
        float acc = 0.0f;
#pragma unroll 16
        for (int i = 0; i < N; i += 32) acc = fmaf(wr[i], xr[i] * scale, acc);
        acc = acc + __shfl_xor(acc, 16);
        acc = row16_ggml_fold(acc);
        if (l == 0) __hip_atomic_store(a.logits + r0 + rr, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the logits are acknowledged
    __syncthreads();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(&a.counters[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    if (wave == 0) router_tail<true>(a.logits, E, a.k, a.renorm, a.sel, a.wsel, 0);
    if (threadIdx.x == 0) __hip_atomic_store(&a.counters[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// -- gate/up + SwiGLU ---------------------------------------------------------
// grid = (n_ff / 16, k + shared), block = 512.  Rows of NB super-blocks of type
// TG (Q4_K or Q3_K), the same for the routed and the shared expert.
// Waves 0-3 copy the rows, waves 4-7 form Q8_K(fx) meanwhile: the compiler
// cannot see the copies, so a wave that issued them would wait for them at
// its first use of a loaded value.
template <int NB, int TG>
__global__ __launch_bounds__(512) void layer_gateup_kernel(GateUpArgs a) {
    constexpr int kRowBytes = NB * QType<TG>::bytes;
    static_assert(kRowBytes % 16 == 0, "rows stay 16-byte aligned");
    __shared__ __align__(16) uint8_t wt[2][kGuRows * kRowBytes];
    __shared__ __align__(16) Q8L q8[NB];
    __shared__ float gu[2 * kGuRows];
    const int j = blockIdx.y;
    const bool shared = j >= a.k;
    const MatDesc &G = shared ? a.sh_gate : a.gate;
    const MatDesc &U = shared ? a.sh_up : a.up;
    const int r0 = blockIdx.x * kGuRows;
    if (r0 >= G.rows) return;
    const int wave = wave_index(), lane = threadIdx.x & 63;
    float *hout = a.h + (size_t)j * a.hstride + r0;
    const uint8_t *gsrc = G.base, *usrc = U.base;
    if (!shared) {
        const int id = a.ids[j];
        if (id < 0 || id >= G.n_ids) {  // invalid id: poison this expert's rows
            if (threadIdx.x < kGuRows) hout[threadIdx.x] = __builtin_nanf("");
            return;
        }
        gsrc += (size_t)id * G.stride;
        usrc += (size_t)id * U.stride;
    }
    gsrc += (size_t)r0 * kRowBytes;
    usrc += (size_t)r0 * kRowBytes;
    if (wave < 4) {
        // gate rows on waves 0-1, up rows on waves 2-3
        constexpr int half = (kGuRows * kRowBytes / 2 + 1023) & ~1023;
        const int m = wave >> 1, off = (wave & 1) * half;
        const int len = min(half, kGuRows * kRowBytes - off);
        wave_copy_nt(wt[m] + off, (m ? usrc : gsrc) + off, len);
        lds_dma_wait();
    } else {
        for (int b = wave - 4; b < NB; b += 4) wave_quantize_q8l(a.fx + b * QK, &q8[b]);
    }
    if (shared && blockIdx.x == 0 && wave == 7 && lane < 32) {
        // sigmoid gate of the shared expert: an f32 row in the router's order
        const float *wr = a.sh_gate_inp + lane;
        const float *xr = a.fx + lane;
        float acc = 0.0f;
#pragma unroll 16
        for (int i = 0; i < NB * QK; i += 32) acc = fmaf(wr[i], xr[i], acc);
        acc = acc + __shfl_xor(acc, 16);
        acc = row16_ggml_fold(acc);
        if (lane == 0) a.sgate[0] = 1.0f / (1.0f + expf(-acc));
    }
    __syncthreads();
    if ((threadIdx.x >> 3) < 2 * kGuRows) {
        // one 8-lane group per row, lane t taking super-block t
        const int grp = threadIdx.x >> 3, t8 = threadIdx.x & 7;
        const int m = grp >= kGuRows, row = grp - m * kGuRows;
        float v;
        if constexpr (TG == kTypeQ3K)
            v = lpb_row_q3k_mem<NB>(wt[m] + row * kRowBytes, q8[t8 < NB ? t8 : 0], t8);
        else
            v = lpb_row_q4k_mem<NB>(wt[m] + row * kRowBytes, q8[t8], t8);
        if (t8 == NB - 1) gu[grp] = v;
    }
    __syncthreads();
    if (threadIdx.x < kGuRows) {
        const float g = gu[threadIdx.x], u = gu[kGuRows + threadIdx.x];
        hout[threadIdx.x] = g / (1.0f + expf(-g)) * u;
    }
}

// -- down + combine -----------------------------------------------------------
// Rows [0, n) of type T with NB super-blocks, row r at base + r * row bytes,
// dotted with unit (u0 + r / 8)'s Q8_K(h); results to ys[u0 * 8 + r].  NT
// threads of the workgroup take part.
template <int T, int NB, int NT>
__device__ __forceinline__ void down_rows(const uint8_t *base, int n, int u0, const Q8L *q8h, float *ys) {
    static_assert(NT % 128 == 0, "whole wave pairs");
    constexpr int kRowBytes = NB * QType<T>::bytes;
    const int wave = wave_index(), grp = threadIdx.x >> 3, t8 = threadIdx.x & 7;
    if constexpr (T == kTypeQ6K) {
        // 8 lanes per row; a wave takes rows of one parity so that its 2-byte
        // aligned rows share their 4-byte alignment
        const int par = wave & 1, G = (wave >> 1) * 8 + (grp & 7);
        for (int m = G; m < n / 2; m += NT / 16) {
            const int r = 2 * m + par, u = u0 + r / kDownRows;
            const float y = g8_row_q6k_u<NB>(base + r * kRowBytes, q8h + u * NB, t8);
            if (t8 == 0) ys[u0 * kDownRows + r] = y;
        }
    } else {
        // one 8-lane group per row, lane t taking super-block t
        for (int r = grp; r < n; r += NT / 8) {
            const int u = u0 + r / kDownRows;
            const Q8L &xb = q8h[u * NB + (t8 < NB ? t8 : 0)];
            float y;
            if constexpr (T == kTypeQ5K) {
                y = g8_row_q5k(base + r * kRowBytes, q8h + u * NB, NB, t8);  // 8 lanes per super-block
                if (t8 == 0) ys[u0 * kDownRows + r] = y;
            } else {
                y = lpb_row_q4k_mem<NB>(base + r * kRowBytes, xb, t8);
                if (t8 == NB - 1) ys[u0 * kDownRows + r] = y;
            }
        }
    }
}

// grid = n_embd / 8, block = 1024.  Down rows of type TD with NBH super-blocks;
// the shared expert (when present) has rows of type TS and the same width.
// Waves 0-7 copy the rows (expert u from wave u % 8: segments in different
// pages do not wait for each other's address translation), waves 8-15 form
// Q8_K(h) of every unit meanwhile.
template <int TD, int NBH, int TS>
__global__ __launch_bounds__(1024) void layer_down_kernel(DownArgs a) {
    constexpr int kRowBytes = NBH * QType<TD>::bytes;
    constexpr int kSegBytes = kDownRows * kRowBytes;  // 8 rows of one expert
    constexpr int kSegBytesS = kDownRows * NBH * QType<TS>::bytes;
    static_assert(kSegBytes % 16 == 0 && kSegBytesS % 16 == 0, "segments stay 16-byte aligned");
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float ys[17 * kDownRows];
    __shared__ int bad;
    const int k = a.k;
    const bool has_sh = a.sh_down.base != nullptr;
    const int nu = k + (has_sh ? 1 : 0);
    uint8_t *wd = smem;
    Q8L *q8h = reinterpret_cast<Q8L *>(smem + k * kSegBytes + (has_sh ? kSegBytesS : 0));
    const int wave = wave_index();
    const int d0 = blockIdx.x * kDownRows;
    if (threadIdx.x == 0) bad = 0;
    __syncthreads();
    if (wave < 8) {
        for (int u = wave; u < nu; u += 8) {
            if (u < k) {
                const int id = a.ids[u];
                if (id < 0 || id >= a.down.n_ids) {
                    bad = 1;
                    continue;
                }
                wave_copy_nt(wd + u * kSegBytes, a.down.base + (size_t)id * a.down.stride + (size_t)d0 * kRowBytes,
                          kSegBytes);
            } else {
                wave_copy_nt(wd + k * kSegBytes, a.sh_down.base + (size_t)d0 * (kSegBytesS / kDownRows), kSegBytesS);
            }
        }
    } else {
        for (int q = wave - 8; q < nu * NBH; q += 8) {
            const int u = q / NBH, b = q - u * NBH;
            wave_quantize_q8l(a.h + (size_t)u * a.hstride + b * QK, &q8h[q]);
        }
    }
    lds_dma_wait();
    __syncthreads();
    if (bad) {
        if (threadIdx.x < kDownRows) a.out[d0 + threadIdx.x] = __builtin_nanf("");
        return;
    }
    if constexpr (TS == TD) {
        down_rows<TD, NBH, 1024>(wd, nu * kDownRows, 0, q8h, ys);  // the shared segment follows the routed ones
    } else {
        down_rows<TD, NBH, 1024>(wd, k * kDownRows, 0, q8h, ys);
        if (has_sh) down_rows<TS, NBH, 1024>(wd + k * kSegBytes, kDownRows, k, q8h, ys);
    }
    __syncthreads();
    if (threadIdx.x < kDownRows) {
        const int r = threadIdx.x, d = d0 + r;
        float acc = 0.0f;
        for (int j = 0; j < k; ++j) acc = acc + a.w[j] * ys[j * kDownRows + r];
        a.out[d] = has_sh ? (acc + ys[k * kDownRows + r] * a.sgate[0]) + a.res[d] : acc + a.res[d];
    }
}

// -- one launch per layer ---------------------------------------------------------
// Workgroups take a ticket when they start, from a counter of their XCD; each
// XCD's tickets give its share of the roles in order: router workgroups, then
// gate/up ones, then down ones (the launch deals the workgroups round-robin to
// the 8 XCDs, so every XCD holds an eighth of each role).  A workgroup waits
// only for roles with lower tickets on its own XCD, which started before it,
// or for roles that come first on every XCD, which need nothing from later
// ones; so every wait ends whatever the number of workgroups resident at once.
// Router workgroups store their logits as tagged words {value, launch
// epoch}, one copy per XCD; every gate/up and down workgroup polls its XCD's
// copy of all of them and forms the top-k itself (the same code on the same
// words, so the same experts and weights), and the first down workgroup of
// XCD 0 writes the caller's sel / wsel from its selection.
// h is formed in 256-row blocks (one Q8_K block each), and a XCD holds whole
// blocks: the 16 gate/up workgroups of a block store their h as tagged words
// into its L2, and the block's last workgroup (the latest ticket of the
// block) waits for them, quantises the block once and publishes it past the
// L2 with a flag in every XCD's line, which the down workgroups poll
// before they read the blocks.  The ticket
// counters grow across launches, so launch e = ticket / workgroups per XCD
// and every tag is e + 1: words of earlier launches never match.
constexpr int kFRouteRows = 4;  // router rows per router workgroup
constexpr int kFGuRows = 16;    // gate rows (and up rows) per gate/up workgroup
constexpr int kFDownRows = 8;   // output rows per down workgroup
constexpr int kFXcds = 8;
constexpr int kFBlockGroups = QK / kFGuRows;         // gate/up workgroups of one 256-row block of h
constexpr int kQ8Words = kFusedQ8Words;              // a Q8_K block in 32-bit words
static_assert(kQ8Words * 4 == (int)sizeof(Q8L), "Q8L layout");
constexpr int kFQ8FlagStride = 128;                   // words per XCD line of block flags (>= blocks)
// counter words (16 to a 128-byte line)
constexpr int kFCtrTicket = 0;               // line x: tickets of XCD x
static_assert(kFCtrTicket + 16 * kFXcds <= kFusedCounterWords, "counter lines");

__device__ __forceinline__ unsigned long long ctr_add(unsigned long long *p) {
    return __hip_atomic_fetch_add(p, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// rms_norm scale of x (every thread takes part): mean of x*x in double,
// 1/sqrtf(mean + eps), as the route kernel forms it.
__device__ __forceinline__ float rms_scale(const float *x, int n, float eps, double *red) {
    const int wave = wave_index(), lane = threadIdx.x & 63;
    double ss = 0.0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = x[i];
        ss += (double)(v * v);
    }
    ss = wave_sum_d(ss);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) tot += red[w];
    const float mean = (float)(tot * (1.0 / (double)n));
    return 1.0f / sqrtf(mean + eps);
}

// Workgroups of each role per XCD; ns = gate/up units (the routed slots and
// the shared expert).
struct FusedRoles {
    int route, gu, down;
};
__host__ __device__ __forceinline__ FusedRoles fused_roles(int E, int ns, int n_ff, int n_embd) {
    const int r = (E + kFRouteRows - 1) / kFRouteRows, nq = ns * (n_ff / QK), d = n_embd / kFDownRows;
    // gate/up: whole blocks per XCD (blocks q = x, x + 8, ... on XCD x)
    return {(r + kFXcds - 1) / kFXcds, kFBlockGroups * ((nq + kFXcds - 1) / kFXcds), (d + kFXcds - 1) / kFXcds};
}
__host__ __device__ __forceinline__ int fused_units(const FusedLayerArgs &a) {
    return a.k + (a.sh_gate.base ? 1 : 0);
}

// Gate/up rows of type TG (Q4_K or Q3_K, 8 super-blocks); down rows of type TD
// with NBH super-blocks; SH: a shared expert, whose down rows have type TS and
// the same width.
template <int TG, int TD, int NBH, int TS, bool SH>
__global__ __launch_bounds__(512) void fused_layer_kernel(FusedLayerArgs a) {
    constexpr int N = 2048, NB = N / QK;
    constexpr int kGuRowBytes = NB * QType<TG>::bytes;
    constexpr int kDnRowBytes = NBH * QType<TD>::bytes;
    constexpr int kSegBytes = kFDownRows * kDnRowBytes;                 // 8 rows of one expert
    constexpr int kSegBytesS = kFDownRows * NBH * QType<TS>::bytes;     // 8 rows of the shared expert
    static_assert(kGuRowBytes % 16 == 0 && kSegBytes % 16 == 0 && kSegBytesS % 16 == 0, "16-byte copies");
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ unsigned long long tk_s;
    __shared__ int flag_s;
    __shared__ double red[8];
    __shared__ int sel_s[16];
    __shared__ float w_s[16];
    __shared__ __align__(16) float ps[128];
    __shared__ float lg_s[1024];  // this launch's logits, gathered from the XCD's tagged copy
    const int tid = threadIdx.x, wave = wave_index(), lane = tid & 63;
    const int E = a.E, k = a.k, nff = a.gate.rows;
    // The selection in the gate/up and down roles.  select_a (wave 0) waits
    // until every logit of this launch is stored; with E <= 128 it forms the
    // softmax into ps, as router_tail does (the same loads, reductions and
    // scale), and select_b (every thread) ranks it: expert e's rank is the
    // number of experts of larger probability or of equal probability and a
    // lower index, the order of router_tail's repeated maxima, and ranks below
    // k fill sel_s / w_s (a bitwise search for the k-th probability on wave
    // 0 alone measured 0.6 us a layer slower).  With E > 128 wave 0 runs
    // router_tail itself (a rank over more experts, in two steps or through a
    // threshold, measured no faster on 512 threads).  A wait that ran out
    // raises flag_s instead.  With E <= 128, w_s holds the raw top-k
    // probabilities until select_renorm.
    const bool rank_sel = E <= 128;
    auto select_a = [&](unsigned long long epoch) {
        // every logit of this launch, from this XCD's copy: lanes take experts
        // lane, lane + 64, ...; a probe that finds a word of an earlier launch
        // probes again at once (a sleep between probes measured slower)
        const unsigned tg = (unsigned)epoch;
        const uint64_t *src = a.lgw + (size_t)xcc_id() * E;
        const int per = (E + 63) >> 6;
        const bool got = poll(
            [&]() {
                bool r = true;
                for (int t = 0; t < per; ++t) {
                    const int e = lane + 64 * t;
                    if (e < E) {
                        const uint64_t w = ld_dev64(src + e);
                        r = r & (tag_seq(w) == tg);
                        lg_s[e] = tag_val(w);
                    }
                }
                return (bool)__all(r);
            },
            a.err, a.wait_ticks);
        if (!got) {
            if (lane == 0) flag_s = 1;
            return;
        }
        // no expert, weight NaN, unless ranked: what router_tail gives for
        // probabilities that are NaN (all of them are when any logit is not finite)
        if (lane < kMaxK) {
            sel_s[lane] = 0x7fffffff;
            w_s[lane] = __builtin_nanf("");
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // lg_s written by this wave
        if (!rank_sel) {
            router_tail<false, false>(lg_s, E, k, a.renorm, sel_s, w_s, 0);
            return;
        }
        float p0 = lane < E ? lg_s[lane] : -INFINITY;
        float p1 = lane + 64 < E ? lg_s[lane + 64] : -INFINITY;
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
        ps[lane] = lane < E ? p0 * sc : -1.0f;  // absent experts below every probability
        ps[lane + 64] = lane + 64 < E ? p1 * sc : -1.0f;
    };
    auto select_b = [&]() {
        if (!rank_sel || flag_s) return;
        const int e = tid >> 2, q = tid & 3;  // four threads per expert, 32 comparisons each
        const float pe = ps[e];
        int r = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const float4 v = *reinterpret_cast<const float4 *>(ps + 32 * q + 4 * c);
            const int e4 = 32 * q + 4 * c;
            r += (v.x > pe) | ((v.x == pe) & (e4 < e));
            r += (v.y > pe) | ((v.y == pe) & (e4 + 1 < e));
            r += (v.z > pe) | ((v.z == pe) & (e4 + 2 < e));
            r += (v.w > pe) | ((v.w == pe) & (e4 + 3 < e));
        }
        r = group4_sum(r);
        if (e < E && q == 0 && r < k && pe == pe) {
            sel_s[r] = e;
            w_s[r] = pe;
        }
    };
    // (wave 0, after the rank is visible) router_tail's renorm of the weights
    auto select_renorm = [&]() {
        if (!rank_sel || !a.renorm) return;
        float ws = 0.0f, wj = 0.0f;
        for (int j = 0; j < k; ++j) {
            const float v = w_s[j];
            ws = ws + v;
            if (j == lane) wj = v;
        }
        if (ws < 6.103515625e-5f) ws = 6.103515625e-5f;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // every lane has read w_s
        if (lane < k) w_s[lane] = wj / ws;
    };
    const unsigned xcc = xcc_id();
    constexpr bool has_sh = SH;
    const int ns = k + (SH ? 1 : 0);  // gate/up and down units: the k slots, then the shared expert
    const FusedRoles R = fused_roles(E, ns, nff, N);
    const unsigned long long Gx = (unsigned long long)(R.route + R.gu + R.down);
    if (tid == 0) {
        tk_s = ctr_add(a.ctr + kFCtrTicket + 16 * xcc);
        flag_s = 0;
    }
    __syncthreads();
    const unsigned long long ep = tk_s / Gx;
    const int lt = (int)(tk_s - ep * Gx);  // role slot within this XCD's share
    const int nq = ns * NBH;  // 256-row blocks of h over the units
    // phase stamps: [xcc * Gx + lt][id, start, e1, e2, e3, end]
    unsigned long long *st = a.trace ? a.trace + ((size_t)xcc * Gx + lt) * kFusedStamps : nullptr;
    auto stamp = [&](int i) {
        if (st && tid == 0) st[i] = wall_clock64();
    };
    if (st && tid == 0) st[0] = (unsigned long long)xcc * 65536ull + (unsigned long long)lt;
    stamp(1);

    if (lt < R.route) {
        // -- router rows [4 i, +4): a half-wave per row in ggml's x86 f32 order --
        // the rows (waves 0-3, one each) and x (wave 4) go to LDS in one burst,
        // so every load is in flight at once
        const int i = (int)xcc * R.route + lt;
        const int nrows = min(kFRouteRows, E - i * kFRouteRows);
        float *wl = reinterpret_cast<float *>(smem);  // [4][N]
        float *xl = wl + kFRouteRows * N;             // [N]
        if (wave < nrows)
            wave_copy(reinterpret_cast<uint8_t *>(wl + wave * N),
                      reinterpret_cast<const uint8_t *>(a.router + (size_t)(i * kFRouteRows + wave) * N), N * 4);
        else if (wave == kFRouteRows)
            wave_copy(reinterpret_cast<uint8_t *>(xl), reinterpret_cast<const uint8_t *>(a.xin), N * 4);
        const float scale = a.rms ? rms_scale(a.xin, N, a.eps, red) : 1.0f;
        lds_dma_wait();
        __syncthreads();
        const int rr = tid >> 5, row = i * kFRouteRows + rr, l = tid & 31;
        if (rr < nrows) {
            const float *wr = wl + rr * N + l;
            const float *xr = xl + l;
            float acc = 0.0f;
#pragma unroll 16
            for (int c = 0; c < N; c += 32) acc = fmaf(wr[c], xr[c] * scale, acc);
            acc = acc + __shfl_xor(acc, 16);
            acc = row16_ggml_fold(acc);
            // the logit is exact in the half-wave's first lane; lanes 0..7 of the
            // half-wave store the copies of the 8 XCDs
            const float lv = __shfl(acc, lane & 32);
            if (l < kFXcds) st_dev64(a.lgw + (size_t)l * E + row, tag(lv, (unsigned)(ep + 1ull)));
        }
        stamp(2);
        stamp(3);
        stamp(4);
        stamp(5);
        return;
    }

    if (lt < R.route + R.gu) {
        // -- gate/up rows [16 r, +16) of super-block b of unit j, SwiGLU --
        // A XCD holds whole 256-row blocks: its share is blocks q = x, x + 8, ...
        // (the shared expert's first), 16 workgroups each, so a block's h stays in
        // this XCD's L2 and its last workgroup (r = 15, the latest ticket of the
        // block) quantises it once for every down workgroup.
        const int g = lt - R.route, r = g % kFBlockGroups, q = (g / kFBlockGroups) * kFXcds + (int)xcc;
        if (q >= nq) return;  // padding of the XCD shares
        const bool shared = has_sh && q < NBH;
        const int j = shared ? k : (q - (has_sh ? NBH : 0)) / NBH;
        const int b = shared ? q : (q - (has_sh ? NBH : 0)) % NBH;
        const int r0 = b * QK + r * kFGuRows;
        uint8_t *wt = smem;  // [2][16 rows]
        Q8L *q8 = reinterpret_cast<Q8L *>(smem + 2 * kFGuRows * kGuRowBytes);
        float *gu = reinterpret_cast<float *>(q8 + NB);
        Q8L *q8b = reinterpret_cast<Q8L *>(gu + 2 * kFGuRows);  // the block's Q8_K(h) (quantiser)
        // gate rows on waves 0-1, up rows on waves 2-3
        auto copy_rows = [&](const MatDesc &G, const MatDesc &U, int id) {
            constexpr int half = (kFGuRows * kGuRowBytes / 2 + 1023) & ~1023;
            const int m = wave >> 1, off = (wave & 1) * half;
            const int len = min(half, kFGuRows * kGuRowBytes - off);
            const uint8_t *src =
                (m ? U.base + (size_t)id * U.stride : G.base + (size_t)id * G.stride) + (size_t)r0 * kGuRowBytes;
            wave_copy_nt(wt + m * kFGuRows * kGuRowBytes + off, src + off, len);
        };
        if (shared && wave < 4) copy_rows(a.sh_gate, a.sh_up, 0);
        const float scale = a.rms ? rms_scale(a.xin, N, a.eps, red) : 1.0f;
        if (wave >= 4) {
            // Q8_K of fx while the selection is awaited and the rows are copied
            for (int bb = wave - 4; bb < NB; bb += 4) {
                const float4 x4 = *reinterpret_cast<const float4 *>(a.xin + bb * QK + 4 * lane);
                const float v[4] = {x4.x * scale, x4.y * scale, x4.z * scale, x4.w * scale};
                wave_quantize_q8l_regs(v, &q8[bb]);
            }
        } else if (wave == 0 && !shared) {
            select_a(ep + 1ull);
        } else if (wave == 0 && r0 == 0 && lane < 32) {
            // the shared expert's sigmoid gate: its f32 row against fx in the
            // router's order, for the down workgroups (a tagged word)
            const float *wr = a.sh_gate_inp + lane;
            const float *xr = a.xin + lane;
            float acc = 0.0f;
#pragma unroll 16
            for (int c = 0; c < N; c += 32) acc = fmaf(wr[c], xr[c] * scale, acc);
            acc = acc + __shfl_xor(acc, 16);
            acc = row16_ggml_fold(acc);
            if (lane == 0) st_dev64(a.sgt, tag(1.0f / (1.0f + expf(-acc)), (unsigned)(ep + 1ull)));
        }
        __syncthreads();
        if (!shared) select_b();
        __syncthreads();
        stamp(2);
        const int id = shared ? 0 : sel_s[j];
        const bool bad = !shared && (flag_s || id < 0 || id >= a.gate.n_ids);
        if (!shared && !bad && wave < 4) copy_rows(a.gate, a.up, id);
        if (wave < 4) lds_dma_wait();
        __syncthreads();
        stamp(3);
        if (!bad && (tid >> 3) < 2 * kFGuRows) {
            const int grp = tid >> 3, t8 = tid & 7;
            const int m = grp >= kFGuRows, row = grp - m * kFGuRows;
            const uint8_t *wr = wt + (m * kFGuRows + row) * kGuRowBytes;
            float v;
            if constexpr (TG == kTypeQ3K)
                v = lpb_row_q3k_mem<NB>(wr, q8[t8], t8);
            else
                v = lpb_row_q4k_mem<NB>(wr, q8[t8], t8);
            if (t8 == NB - 1) gu[grp] = v;
        }
        __syncthreads();
        uint64_t *hb = a.ht + (size_t)j * nff + b * QK;  // the block's tagged h, in this XCD's L2
        const unsigned tg = (unsigned)(ep + 1ull);
        if (tid < kFGuRows) {
            const float gv = gu[tid], uv = gu[kFGuRows + tid];
            const float hv = bad ? __builtin_nanf("") : gv / (1.0f + expf(-gv)) * uv;
            st_l2(hb + r * kFGuRows + tid, tag(hv, tg));
        }
        stamp(4);
        if (r != kFBlockGroups - 1) {
            stamp(5);
            return;
        }
        // -- the block's quantiser: all 256 h of the block (4 a lane), Q8_K once,
        // published as tagged words for the down workgroups of every XCD --
        if (wave == 1) {  // not the wave that stored h: its poll does not wait for those stores
            uint64_t w[4];
            const bool got = poll(
                [&]() {
                    ld_dev64x2(hb, QK, 4 * lane, w[0], w[1]);
                    ld_dev64x2(hb, QK, 4 * lane + 2, w[2], w[3]);
                    bool ok4 = true;
#pragma unroll
                    for (int c = 0; c < 4; ++c) ok4 = ok4 & (tag_seq(w[c]) == tg);
                    return (bool)__all(ok4);
                },
                a.err, a.wait_ticks);
            const float v[4] = {tag_val(w[0]), tag_val(w[1]), tag_val(w[2]), tag_val(w[3])};
            wave_quantize_q8l_regs(v, q8b);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the block is in LDS
            if (got) {
                // the block's words past the L2, then (once they are acknowledged)
                // its flag in every XCD's line, which the down workgroups poll
                const uint32_t *qw = reinterpret_cast<const uint32_t *>(q8b);
                uint32_t *dst = a.q8d + (size_t)q * kQ8Words;
                st_dev_u32(dst + lane, qw[lane]);
                if (lane < kQ8Words - 64) st_dev_u32(dst + 64 + lane, qw[64 + lane]);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                if (lane < kFXcds) st_dev64(a.q8f + (size_t)lane * kFQ8FlagStride + q, tag(0.0f, tg));
            }
        }
        __syncthreads();  // the stamp below marks the block published
        stamp(5);
        return;
    }

    // -- down rows [8 i, +8) of every selected expert (and the shared one), then the combine --
    const int i = (int)xcc * R.down + (lt - R.route - R.gu);
    if (i * kFDownRows >= N) return;  // padding of the XCD shares
    const int d0 = i * kFDownRows;
    uint8_t *wd = smem;  // [k][8 rows], then the shared expert's 8 rows
    Q8L *q8h = reinterpret_cast<Q8L *>(smem + k * kSegBytes + (has_sh ? kSegBytesS : 0));
    float *ys = reinterpret_cast<float *>(q8h + ns * NBH);
    // the shared expert's rows need no selection: copied at once (not by wave
    // 0, whose probes would queue behind the copy)
    if (has_sh && wave == 7)
        wave_copy_nt(wd + k * kSegBytes, a.sh_down.base + (size_t)d0 * (kSegBytesS / kFDownRows), kSegBytesS);
    if (wave == 0) select_a(ep + 1ull);
    __syncthreads();
    select_b();
    __syncthreads();
    if (wave == 0) select_renorm();
    stamp(2);
    // the first down workgroup of XCD 0 also gives the caller sel / wsel (a
    // selection that could not be gathered reads as no expert, weight NaN)
    const bool caller_sel = xcc == 0 && lt == R.route + R.gu;
    int bad = flag_s;
    for (int u = wave; u < k; u += 8) {
        // expert u's 8 rows from wave u: copies in different pages do not wait on each other
        const int id = sel_s[u];
        if (id < 0 || id >= a.down.n_ids) {
            bad = 1;
            continue;
        }
        if (!flag_s)
            wave_copy_nt(wd + u * kSegBytes, a.down.base + (size_t)id * a.down.stride + (size_t)d0 * kDnRowBytes,
                         kSegBytes);
    }
    if (caller_sel && wave == 0 && lane < k) {
        // the renormed weights: lane j wrote w_s[j] itself in select_renorm
        // (or router_tail's lane j did)
        a.sel[lane] = flag_s ? 0x7fffffff : sel_s[lane];
        a.wsel[lane] = flag_s ? __builtin_nanf("") : w_s[lane];
    }
    // every unit's Q8_K(h), published once per block by its quantiser: wave 0
    // polls this XCD's line of block flags (no sleep between probes), then every
    // thread moves 16-byte pieces of the blocks into LDS, read past the L2
    const unsigned tg = (unsigned)(ep + 1ull);
    float sgate = 0.0f;
    if (!flag_s && wave == 0) {
        const uint64_t *fl = a.q8f + (size_t)xcc * kFQ8FlagStride;
        const bool got = poll(
            [&]() {
                bool r = true;
                for (int qq = lane; qq < nq; qq += 64) r = r & (tag_seq(ld_dev64(fl + qq)) == tg);
                if (has_sh && lane == 0) r = r & (tag_seq(ld_dev64(a.sgt)) == tg);
                return (bool)__all(r);
            },
            a.err, a.wait_ticks);
        if (!got && lane == 0) flag_s = 1;
    }
    __syncthreads();
    if (!flag_s) {
        // block q (publication order, the shared expert's first) goes to its place
        // in unit order (routed slots, then the shared expert)
        constexpr int kPieces = kQ8Words / 4;  // 16-byte pieces of a block
        for (int c = tid; c < nq * kPieces; c += 512) {
            const int qq = c / kPieces, pc = c - qq * kPieces;
            const int pos = has_sh ? (qq < NBH ? k * NBH + qq : qq - NBH) : qq;
            const float4 f = ld_dev_f4(reinterpret_cast<const float *>(a.q8d), (unsigned)(nq * kQ8Words * 4),
                                       (unsigned)((qq * kQ8Words + 4 * pc) * 4));
            *reinterpret_cast<float4 *>(reinterpret_cast<uint32_t *>(q8h + pos) + 4 * pc) = f;
        }
        if (has_sh) sgate = tag_val(ld_dev64(a.sgt));
    }
    if (bad) atomicOr(&flag_s, 1);
    __syncthreads();
    if (flag_s) {
        if (tid < kFDownRows) a.out[d0 + tid] = __builtin_nanf("");
        return;
    }
    stamp(3);
    stamp(4);
    if constexpr (TS == TD) {
        down_rows<TD, NBH, 512>(wd, ns * kFDownRows, 0, q8h, ys);  // the shared segment follows the routed ones
    } else {
        down_rows<TD, NBH, 512>(wd, k * kFDownRows, 0, q8h, ys);
        if (has_sh) down_rows<TS, NBH, 512>(wd + k * kSegBytes, kFDownRows, k, q8h, ys);
    }
    __syncthreads();
    if (tid < kFDownRows) {
        const int rr = tid, d = d0 + rr;
        float acc = 0.0f;
        for (int jj = 0; jj < k; ++jj) acc = acc + w_s[jj] * ys[jj * kFDownRows + rr];
        if (has_sh) {
            a.out[d] = (acc + ys[k * kFDownRows + rr] * sgate) + a.res[d];
        } else {
            a.out[d] = acc + a.res[d];
        }
    }
    stamp(5);
}

}  // namespace

// Instantiated shapes: router n_embd 2048; gate/up Q4_K or Q3_K with 8
// super-blocks per row; down Q6_K with 2-4, Q5_K with 2 or 4, or Q4_K with 4
// super-blocks per row.
bool layer_route_ok(const RouterArgs &a) { return a.n == 2048 && a.E <= 1024 && a.M == 1; }

hipError_t launch_layer_route(const RouterArgs &a, hipStream_t s) {
    if (!layer_route_ok(a)) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(layer_route_kernel<2048>, dim3((unsigned)((a.E + kRouteRows - 1) / kRouteRows)), dim3(128), 0, s,
                       a);
    return hipGetLastError();
}

bool layer_ffn_ok(const GateUpArgs &g, const DownArgs &d) {
    const bool gu_type = (g.gate.type == kTypeQ4K || g.gate.type == kTypeQ3K) && g.up.type == g.gate.type;
    if (g.n_embd != 2048 || !gu_type || g.gate.rows % kGuRows) return false;
    if (d.k > 16 || d.n_embd % kDownRows) return false;
    const int nbh = d.down.cols / QK;
    const bool q6 = d.down.type == kTypeQ6K && nbh >= 2 && nbh <= 4;
    const bool q4 = d.down.type == kTypeQ4K && nbh == 4;
    const bool q5 = d.down.type == kTypeQ5K && (nbh == 2 || nbh == 4);
    if (!q6 && !q4 && !q5) return false;
    if (g.sh_gate.base) {
        if (g.sh_gate.type != g.gate.type || g.sh_up.type != g.gate.type || g.sh_gate.rows != g.gate.rows) return false;
        if (!d.sh_down.base || d.sh_down.cols != d.down.cols) return false;
        // a Q5_K routed down may have a Q6_K shared one; otherwise the types agree
        if (d.sh_down.type != d.down.type && !(d.down.type == kTypeQ5K && d.sh_down.type == kTypeQ6K && nbh == 2))
            return false;
    }
    // every copy source 16-byte aligned
    uintptr_t al = reinterpret_cast<uintptr_t>(g.gate.base) | reinterpret_cast<uintptr_t>(g.up.base) |
                   reinterpret_cast<uintptr_t>(d.down.base) | g.gate.stride | g.up.stride | d.down.stride |
                   reinterpret_cast<uintptr_t>(g.fx) | reinterpret_cast<uintptr_t>(d.h) | (uintptr_t)(d.hstride * 4);
    if (g.sh_gate.base)
        al |= reinterpret_cast<uintptr_t>(g.sh_gate.base) | reinterpret_cast<uintptr_t>(g.sh_up.base) |
              reinterpret_cast<uintptr_t>(d.sh_down.base);
    return (al & 15) == 0;
}

hipError_t launch_layer_gateup(const GateUpArgs &g, hipStream_t s) {
    const dim3 gg((unsigned)(g.gate.rows / kGuRows), (unsigned)(g.k + (g.sh_gate.base ? 1 : 0)));
    if (g.gate.type == kTypeQ3K)
        hipLaunchKernelGGL((layer_gateup_kernel<8, kTypeQ3K>), gg, dim3(512), 0, s, g);
    else
        hipLaunchKernelGGL((layer_gateup_kernel<8, kTypeQ4K>), gg, dim3(512), 0, s, g);
    return hipGetLastError();
}

hipError_t launch_layer_down(const DownArgs &d, hipStream_t s) {
    const bool has_sh = d.sh_down.base != nullptr;
    const int nu = d.k + (has_sh ? 1 : 0);
    const int nbh = d.down.cols / QK;
    const int ts = has_sh ? d.sh_down.type : d.down.type;
    const size_t seg = (size_t)kDownRows * nbh * block_bytes(d.down.type);
    const size_t seg_s = has_sh ? (size_t)kDownRows * nbh * block_bytes(ts) : 0;
    const size_t lds = d.k * seg + seg_s + (size_t)nu * nbh * sizeof(Q8L);
    if (lds > 65536) return hipErrorInvalidConfiguration;
    const dim3 dg((unsigned)(d.n_embd / kDownRows));
#define HOARD_DOWN(TD, NBH, TS)                                                                 \
    if (d.down.type == TD && nbh == NBH && ts == TS) {                                          \
        hipLaunchKernelGGL((layer_down_kernel<TD, NBH, TS>), dg, dim3(1024), lds, s, d);        \
        return hipGetLastError();                                                               \
    }
    HOARD_DOWN(kTypeQ6K, 2, kTypeQ6K)
    HOARD_DOWN(kTypeQ6K, 3, kTypeQ6K)
    HOARD_DOWN(kTypeQ6K, 4, kTypeQ6K)
    HOARD_DOWN(kTypeQ4K, 4, kTypeQ4K)
    HOARD_DOWN(kTypeQ5K, 2, kTypeQ5K)
    HOARD_DOWN(kTypeQ5K, 4, kTypeQ5K)
    HOARD_DOWN(kTypeQ5K, 2, kTypeQ6K)
#undef HOARD_DOWN
    return hipErrorInvalidConfiguration;
}

}  // namespace hoard

namespace hoard {

namespace {

size_t fused_lds_bytes(const FusedLayerArgs &a) {
    const int nbh = a.down.cols / QK, ns = fused_units(a);
    const size_t gu = 2 * kFGuRows * (size_t)(8 * block_bytes(a.gate.type)) + 8 * sizeof(Q8L) +
                      2 * kFGuRows * sizeof(float) + sizeof(Q8L);
    const size_t seg_s = a.sh_gate.base ? (size_t)kFDownRows * nbh * block_bytes(a.sh_down.type) : 0;
    const size_t dn = (size_t)a.k * kFDownRows * nbh * block_bytes(a.down.type) + seg_s +
                      (size_t)ns * nbh * sizeof(Q8L) + (size_t)ns * kFDownRows * sizeof(float);
    const size_t rt = (size_t)(kFRouteRows + 1) * a.n_embd * sizeof(float);  // router rows and x
    const size_t m = gu > dn ? gu : dn;
    return m > rt ? m : rt;
}

}  // namespace

// The shapes of the fused launch: n_embd 2048, at most 1024 experts; gate/up
// Q4_K or Q3_K with n_ff a multiple of 256; down Q6_K with 2-4 super-blocks,
// Q5_K with 2 or 4, or Q4_K with 4 per row; a shared expert of the same gate/up
// type and width, whose down rows have the routed type (or Q6_K beside Q5_K
// with 2), at most 16 units in all; 16-byte aligned tensors and activations.
bool fused_layer_ok(const FusedLayerArgs &a) {
    const bool gu_type = (a.gate.type == kTypeQ4K || a.gate.type == kTypeQ3K) && a.up.type == a.gate.type;
    if (a.n_embd != 2048 || !gu_type || a.gate.rows % QK || a.gate.rows != a.up.rows || a.k < 1 ||
        fused_units(a) > 16 || a.E < a.k || a.E > 1024)
        return false;
    const int nbh = a.down.cols / QK;
    const bool q6 = a.down.type == kTypeQ6K && nbh >= 2 && nbh <= 4;
    const bool q4 = a.down.type == kTypeQ4K && nbh == 4;
    const bool q5 = a.down.type == kTypeQ5K && (nbh == 2 || nbh == 4);
    if (!q6 && !q4 && !q5) return false;
    uintptr_t al = reinterpret_cast<uintptr_t>(a.gate.base) | reinterpret_cast<uintptr_t>(a.up.base) |
                   reinterpret_cast<uintptr_t>(a.down.base) | a.gate.stride | a.up.stride | a.down.stride |
                   reinterpret_cast<uintptr_t>(a.xin);
    if (!a.ht || !a.q8d || !a.q8f || !a.sgt || fused_units(a) * (a.gate.rows / QK) > kFQ8FlagStride) return false;
    if (a.sh_gate.base) {
        if (a.sh_gate.type != a.gate.type || a.sh_up.type != a.gate.type || a.sh_gate.rows != a.gate.rows ||
            a.sh_up.rows != a.gate.rows || !a.sh_up.base || !a.sh_down.base || !a.sh_gate_inp ||
            a.sh_down.cols != a.down.cols)
            return false;
        if (a.sh_down.type != a.down.type && !(a.down.type == kTypeQ5K && a.sh_down.type == kTypeQ6K && nbh == 2))
            return false;
        al |= reinterpret_cast<uintptr_t>(a.sh_gate.base) | reinterpret_cast<uintptr_t>(a.sh_up.base) |
              reinterpret_cast<uintptr_t>(a.sh_down.base);
    }
    return (al & 15) == 0 && fused_lds_bytes(a) <= 65536;
}

int fused_layer_groups(const FusedLayerArgs &a) {
    const FusedRoles R = fused_roles(a.E, fused_units(a), a.gate.rows, a.n_embd);
    return kFXcds * (R.route + R.gu + R.down);
}

hipError_t launch_fused_layer(const FusedLayerArgs &a, hipStream_t s) {
    if (!fused_layer_ok(a)) return hipErrorInvalidConfiguration;
    const int nbh = a.down.cols / QK;
    const int ts = a.sh_gate.base ? a.sh_down.type : a.down.type;
    const unsigned G = (unsigned)fused_layer_groups(a);
    const size_t lds = fused_lds_bytes(a);
    const bool sh = a.sh_gate.base != nullptr;
#define HOARD_FUSED(TG, TD, NBH, TS, SH)                                                                  \
    if (a.gate.type == TG && a.down.type == TD && nbh == NBH && ts == TS && sh == SH) {                   \
        hipLaunchKernelGGL((fused_layer_kernel<TG, TD, NBH, TS, SH>), dim3(G), dim3(512), lds, s, a);    \
        return hipGetLastError();                                                                         \
    }
    HOARD_FUSED(kTypeQ4K, kTypeQ6K, 2, kTypeQ6K, false)
    HOARD_FUSED(kTypeQ4K, kTypeQ6K, 3, kTypeQ6K, false)
    HOARD_FUSED(kTypeQ4K, kTypeQ6K, 4, kTypeQ6K, false)
    HOARD_FUSED(kTypeQ4K, kTypeQ4K, 4, kTypeQ4K, false)
    HOARD_FUSED(kTypeQ4K, kTypeQ5K, 2, kTypeQ5K, false)
    HOARD_FUSED(kTypeQ4K, kTypeQ5K, 4, kTypeQ5K, false)
    HOARD_FUSED(kTypeQ3K, kTypeQ5K, 4, kTypeQ5K, false)
    HOARD_FUSED(kTypeQ3K, kTypeQ4K, 4, kTypeQ4K, false)
    HOARD_FUSED(kTypeQ4K, kTypeQ6K, 2, kTypeQ6K, true)
    HOARD_FUSED(kTypeQ4K, kTypeQ5K, 2, kTypeQ6K, true)
#undef HOARD_FUSED
    return hipErrorInvalidConfiguration;
}

}  // namespace hoard
