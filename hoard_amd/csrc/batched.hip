// Batched expert stage for M tokens (speculative verify / small prefill):
// tokens are grouped by expert so every selected expert's weights are read
// once per call, and the expert products run on int8 MFMA.
//
// Counterpart of ggml_mul_mat_id over the slot pool with per-token ids
// (src/run_specloop.cpp:126-139; all-resident form src/run_m1.cpp:97-108)
// followed by the weighted sum over the selected experts.
//
// The MFMA tiles and why they give the per-token path's bits are in mfma.h.
// Batches of more than 32 tokens take the sorted-pair path of prefill.hip after
// the routing and grouping here.
#include "kernels.h"
#include "lds_dma.h"
#include "mfma.h"
#include "qblocks.h"
#include "rowdot.h"
#include "router_tail.h"

namespace hoard {

namespace {

constexpr int kTile = 16;                   // weight rows per MFMA tile
constexpr int kMaxTok = kBatchedMaxTokens;  // token places per expert group
constexpr int kCols = 16;                   // token columns per MFMA tile
constexpr int kMfmaMinTokens = 12;          // smallest expert group computed on MFMA
constexpr int kXChunk = 1;                  // tokens of Q8_K x staged in LDS at a time
constexpr int kMaxExperts = 1024;
static_assert(sizeof(Q8L) == kQ8LBytes, "Q8_K block size shared with the host");

__device__ __forceinline__ Q8L *q8(uint8_t *p) { return reinterpret_cast<Q8L *>(p); }

// -- route: router logits, softmax / top-k, Q8_K of fx, grouping by expert ----
// One launch replaces the router kernels and the grouping pass.  A workgroup
// (4 waves) takes R router rows against kRouteTok tokens, a wave per token and
// a half-wave per row at a time, with the single-token router's per-row
// accumulation order (lane l of 32 owns elements l, l+32, ...; ggml's f32 dot
// fold).  Up to 8 tokens two rows per workgroup, above that four (fewer
// copies of the tokens' fx): measured per layer, four rows against two took
// 0.5 us off at 16 tokens and 2.8 at 32 (Qwen3-30B shape), 3.3 and 7.5 with
// 512 experts (Qwen3-Next), and added 1.2 us at 4 tokens; eight rows were
// slower than four everywhere.  A remainder of one row (a shared expert's
// gate row after a multiple of R routed rows) goes to the last workgroup of
// the row range as an extra pass instead of a workgroup of its own: with 512
// experts and four token groups the extra workgroups would not fit the two a
// CU that the LDS allows, and a second round of workgroups would follow the
// first.  The last
// workgroup of a token group (device-scope counter) runs the tails of its
// tokens; the last token group's tail workgroup then groups the (token, slot)
// pairs by expert.  Waves with a spare slot quantise fx to Q8_K.
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

// LDS of the grouping passes; the route kernel lays it over its staging
// buffers, which are free by then.
struct GroupLds {
    unsigned mask[kMaxExperts];  // tokens (of a chunk) selecting each expert
    int uidx[kMaxExperts];       // group of each expert
    unsigned cnt[kMaxExperts];   // pairs per expert
    int base[kMaxExperts];       // next sorted position of each expert
    int total;
};

__device__ void group_by_expert(const BatchedArgs &a, GroupLds &g, const int *ysrc = nullptr,
                                const int *bad = nullptr) {
    unsigned *mask = g.mask;
    int *uidx = g.uidx;
    int &wave_total = g.total;
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
    if (a.sh) {
        // the shared expert: group n_unique (after the routed groups), every
        // token, slot k
        const int g = wave_total;
        for (int t = tid; t < a.M; t += nt) {
            a.utok[g * kMaxTok + t] = t;
            a.uslot[g * kMaxTok + t] = a.k;
        }
        if (tid == 0) {
            a.uexp[g] = a.n_ids;
            a.ucount[g] = a.M;
        }
    }
    if (tid == 0) a.n_unique[0] = wave_total;
    // the grid's group places past the used ones hold no expert, so a
    // workgroup learns from its place alone whether it has work
    const int umax = min(E, P) + a.sh;
    for (int g = wave_total + a.sh + tid; g < umax; g += nt) a.uexp[g] = -1;
}

// Groups and units in ascending expert order from the per-expert pair counts
// g.cnt (wave 0 of the grouping workgroup): uexp / ucount / goff / hist, the
// unit records {expert, first sorted pair, pairs} (every place past the last
// unit zeroed), n_unique / n_units, and g.base[e], the first sorted place of
// expert e.
__device__ void group_units(const BatchedArgs &a, GroupLds &g) {
    const int tid = threadIdx.x, E = a.n_ids + a.sh;
    {
        // groups and units in ascending expert order: lane owns a contiguous run of experts
        const int lane = tid, per = (E + 63) / 64, e0 = lane * per;
        int cg = 0, cu = 0, cp = 0;
        for (int e = e0; e < e0 + per && e < E; ++e) {
            const int c = (int)g.cnt[e];
            cg += c ? 1 : 0;
            cu += (c + kUnitTokens - 1) / kUnitTokens;
            cp += c;
        }
        int ig = cg, iu = cu, ip = cp;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int og = __shfl_up(ig, off), ou = __shfl_up(iu, off), op = __shfl_up(ip, off);
            if (lane >= off) {
                ig += og;
                iu += ou;
                ip += op;
            }
        }
        int gi = ig - cg, ui = iu - cu, pi = ip - cp;
        for (int e = e0; e < e0 + per && e < E; ++e) {
            const int c = (int)g.cnt[e];
            a.hist[e] = (unsigned)c;
            g.base[e] = pi;
            if (c) {
                a.uexp[gi] = e;
                a.ucount[gi] = c;
                a.goff[gi] = pi;
                for (int s0 = 0; s0 < c; s0 += kUnitTokens, ++ui)
                    *reinterpret_cast<int4 *>(a.units + 4 * ui) = make_int4(e, pi + s0, min(kUnitTokens, c - s0), 0);
                ++gi;
            }
            pi += c;
        }
        if (lane == 63) {
            a.n_unique[0] = ig - a.sh;  // routed experts used
            a.n_units[0] = iu;
            g.total = ip;  // pairs in all groups
        }
        // the grid's unit places past the last unit hold no pairs, so a workgroup
        // learns from its own place alone whether it has work
        for (int x = __shfl(iu, 63) + lane; x < a.max_units; x += 64)
            *reinterpret_cast<int4 *>(a.units + 4 * x) = make_int4(0, 0, 0, 0);
    }
}

// Grouping of a prefill-sized batch (all threads of one workgroup): the
// computed (token, slot) pairs sorted by (expert, token) into ptok / pslot, the
// groups (used experts in ascending order: uexp, ucount, goff) and the work
// units (at most kUnitTokens pairs of one group each).  pe[p] (in LDS) is the
// expert of pair p, or -1 for a pair that joins no group.  The order within an
// expert comes from chunks of at most 32 tokens taken in token order: a pair's
// place is its expert's running base plus the tokens of its chunk before it
// that select the same expert (a token joins a group at most once).
__device__ void group_large(const BatchedArgs &a, GroupLds &g, const int *pe, int *sorted) {
    const int tid = threadIdx.x, nt = blockDim.x, E = a.n_ids + a.sh, k = a.k + a.sh, P = a.M * k;
    for (int e = tid; e < E; e += nt) g.cnt[e] = 0u;
    __syncthreads();
    for (int p = tid; p < P; p += nt)
        if (pe[p] >= 0) atomicAdd(&g.cnt[pe[p]], 1u);
    __syncthreads();
    if (tid < 64) group_units(a, g);
    __syncthreads();
    const int tpc = min(32, max(1, nt / k));  // tokens per chunk: one mask bit each
    for (int t0 = 0; t0 < a.M; t0 += tpc) {
        for (int e = tid; e < E; e += nt) g.mask[e] = 0u;
        __syncthreads();
        const int pend = min(P, (t0 + tpc) * k);
        for (int p = t0 * k + tid; p < pend; p += nt)
            if (pe[p] >= 0) atomicOr(&g.mask[pe[p]], 1u << (p / k - t0));
        __syncthreads();
        for (int p = t0 * k + tid; p < pend; p += nt) {
            const int e = pe[p];
            if (e < 0) continue;
            const int t = p / k;
            const int pos = g.base[e] + __popc(g.mask[e] & ((1u << (t - t0)) - 1u));
            sorted[pos] = t | (p - t * k) << 16;
        }
        __syncthreads();
        for (int e = tid; e < E; e += nt) g.base[e] += __popc(g.mask[e]);
        __syncthreads();
    }
}

template <int R>
__global__ __launch_bounds__(256) void route_kernel(BatchedArgs a) {
    constexpr int n = kRouteN, nb = kRouteN / QK;
    const int E = a.E;
    const int wave = wave_index(), lane = threadIdx.x & 63, l = lane & 31;
    const int tg = blockIdx.y;
    const int t = tg * kRouteTok + wave;  // this wave's token; its half-waves take one row each
    // rows 0..E-1 are the router's; row E (with a shared expert) is its gate row
    const int r0 = blockIdx.x * R;
    const int nrows = blockIdx.x == gridDim.x - 1 ? E + a.sh - r0 : R;  // R + 1 with a one-row remainder
    // the workgroup's token rows and router rows go to LDS in one burst, so
    // that every load is in flight at once; the dot then reads them in the
    // per-lane order the accumulation needs
    __shared__ __align__(16) float xl[kRouteTok][kRouteN];
    __shared__ __align__(16) float wl[R + 1][kRouteN];
    if (t < a.M) dma_wave_copy(reinterpret_cast<uint8_t *>(xl[wave]), reinterpret_cast<const uint8_t *>(a.fx + (size_t)t * n),
                               n * (int)sizeof(float));
    {
        // the rows' 1 KB pieces, dealt to the four waves in turn
        constexpr int kPieces = n * (int)sizeof(float) / 1024;
        for (int c = wave; c < nrows * kPieces; c += 4) {
            const int rr = c / kPieces, o = (c % kPieces) * 1024;
            const float *src = r0 + rr < E ? a.router + (size_t)(r0 + rr) * n : a.sh_gate_inp;
            dma_chunk(reinterpret_cast<uint8_t *>(wl[rr]) + o, reinterpret_cast<const uint8_t *>(src) + o);
        }
    }
    lds_dma_wait();
    __syncthreads();
    if (t < a.M) {
        const float *x = xl[wave];
        // half-wave h takes rows rp + h, rp = 0, 2, ...; the R / 2 rows of a lane
        // accumulate side by side, so their FMA chains overlap
        static_assert(R % 2 == 0, "two rows a pass, one a half-wave");
        constexpr int kP = R / 2;
        const float *wr[kP];
        float acc[kP];
#pragma unroll
        for (int j = 0; j < kP; ++j) {
            wr[j] = wl[min(2 * j + (lane >> 5), nrows - 1)];
            acc[j] = 0.0f;
        }
#pragma unroll 8
        for (int i = 0; i < n; i += 32) {
            const float xv = x[i + l];
#pragma unroll
            for (int j = 0; j < kP; ++j) acc[j] = fmaf(wr[j][i + l], xv, acc[j]);
        }
        // the remainder row, on both half-waves (the second one's result is
        // past the rows and not stored)
        float acc_r = 0.0f;
        if (nrows > R) {
            const float *w = wl[R];
#pragma unroll 8
            for (int i = 0; i < n; i += 32) acc_r = fmaf(w[i + l], x[i + l], acc_r);
        }
#pragma unroll
        for (int j = 0; j <= kP; ++j) {
            if (j == kP && nrows <= R) break;
            float v = j < kP ? acc[j] : acc_r;
            v = v + __shfl_xor(v, 16);
            v = v + __shfl_xor(v, 8);
            v = v + __shfl_xor(v, 4);
            v = v + __shfl_xor(v, 1);
            v = v + __shfl_xor(v, 2);
            const int row = r0 + 2 * j + (lane >> 5);
            if (l == 0 && row < E)
                __hip_atomic_store(a.logits + (size_t)t * E + row, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else if (l == 0 && row == E && a.sh)
                a.sgl[t] = v;
        }
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
    // the staging buffers are free: the grouping's LDS goes over them
    static_assert(sizeof(GroupLds) <= sizeof(xl), "grouping LDS fits the token staging");
    GroupLds &g = *reinterpret_cast<GroupLds *>(&xl[0][0]);
    group_by_expert(a, g);
    if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[kBatchedCounters - 1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// -- prefill-sized routing: tiled router GEMM, then tails, then the grouping -----
// Logits of 16 experts x TT tokens per workgroup of 512 threads (TT = 16, or 8
// where 16-token tiles would leave CUs idle).  Thread (group q = tid / 32, lane
// l = tid % 32) holds accumulator l of ggml's x86 f32 dot (elements 32 i + l,
// i ascending) for 4 experts x TT / 4 tokens: the rows and tokens pass through
// LDS 512 elements at a time, 8 (6) reads for every 16 (8) dots.  The 32
// accumulators of a dot sit in the 32 lanes of a half-wave, which fold them in
// ggml's order, so every logit is the single-token router's.
// One workgroup per CU: eight waves (two per SIMD) took 4 us less per launch
// than four waves with 4 x 8 dots each, sixteen waves with 2 x 4 each 1 us
// more than eight.  Each K step costs a wait and a barrier besides its dots:
// 512-element steps (4 of them) took 3.5 us less per launch than 256-element
// ones (8), and 1024-element ones without a second buffer 1.6 us more than
// 512 at M = 512 (four waves).  8-token tiles where 16-token ones would fill
// at most half the CUs: 2.5 us less per layer at 128 tokens of 128 experts
// (2.2 more at 512, where 16-token tiles fill the CUs once).
constexpr int kTileE = 16;

// K steps in LDS: the current one and the next in flight (four buffers, three
// steps in flight, measured the same: once one step is prefetched the dots and
// the per-step barrier set the pace).  kTileK = 512: 128 KB of LDS, one
// workgroup per CU; 256: 64 KB, two a CU, for grids of more tiles than CUs
// (512 experts at 128 and 512 tokens: 49.5 against 2 x 12 us per launch).
constexpr int kGemmBufs = 2;
template <int kTileK, int kTileT>
__global__ __launch_bounds__(512) void route_gemm_kernel(BatchedArgs a) {
    constexpr int kTQ = kTileT / 4;  // tokens per thread group
    static_assert((kTileE + kTileT) % 8 == 0, "every wave copies as many rows");
    __shared__ __align__(16) float wl[kGemmBufs][kTileE][kTileK];
    __shared__ __align__(16) float xl[kGemmBufs][kTileT][kTileK];
    constexpr int n = kRouteN, kSteps = n / kTileK;
    static_assert(kSteps >= kGemmBufs, "the ring is filled before the first step");
    constexpr int kRowsPerWave = (kTileE + kTileT) / 8 * (kTileK / 256);  // 1 KB copies each wave issues per step
    const int tid = threadIdx.x, q = tid >> 5, l = tid & 31, wave = wave_index(), lane = tid & 63;
    const int e0 = blockIdx.x * kTileE, t0 = blockIdx.y * kTileT;
    const int re = (q & 3) * 4, rt = (q >> 2) * kTQ;  // this group's 4 experts and kTQ tokens within the tile
    float acc[4][kTQ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kTQ; ++j) acc[i][j] = 0.0f;
    // 16 + TT rows of 1 KB per step: expert rows then token rows, one wave per 8 rows;
    // rows past the end repeat the last one (their results are not stored).  The
    // next steps' rows are in flight while the current one is dotted.  A shared
    // expert's gate row is not a row here: the tails kernel forms its logit,
    // which keeps 512 (256) routed experts at a whole number of rounds of tiles.
    const int er = a.E;
    auto issue = [&](int k0, int buf) {
        for (int r = wave; r < kTileE + kTileT; r += 8) {
            const int row = min(e0 + r, er - 1);
            const float *src = r < kTileE ? a.router + (size_t)row * n
                                          : a.fx + (size_t)min(t0 + r - kTileE, a.M - 1) * n;
            float *dst = r < kTileE ? wl[buf][r] : xl[buf][r - kTileE];
#pragma unroll
            for (int ck = 0; ck < kTileK / 256; ++ck)
                dma_chunk(reinterpret_cast<uint8_t *>(dst + 256 * ck), reinterpret_cast<const uint8_t *>(src + k0 + 256 * ck));
        }
    };
#pragma unroll
    for (int b = 0; b < kGemmBufs - 1; ++b) issue(b * kTileK, b);
#pragma unroll 1
    for (int st = 0; st < kSteps; ++st) {
        const int buf = st % kGemmBufs;
        const int nx = st + kGemmBufs - 1;
        if (nx < kSteps) issue(nx * kTileK, nx % kGemmBufs);
        // this step's copies landed: the wave's newer copies (up to kGemmBufs - 1 steps) may still fly
        const int newer = min(kSteps - 1 - st, kGemmBufs - 1);
        if (newer == 3)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * kRowsPerWave) : "memory");
        else if (newer == 2)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * kRowsPerWave) : "memory");
        else if (newer == 1)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kRowsPerWave) : "memory");
        else
            lds_dma_wait();
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kTileK / 32; ++i) {
            float wv[4], xv[kTQ];
#pragma unroll
            for (int r = 0; r < 4; ++r) wv[r] = wl[buf][re + r][32 * i + l];
#pragma unroll
            for (int t = 0; t < kTQ; ++t) xv[t] = xl[buf][rt + t][32 * i + l];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int t = 0; t < kTQ; ++t) acc[r][t] = fmaf(wv[r], xv[t], acc[r][t]);
        }
        __syncthreads();  // every wave is done with this buffer before it is refilled
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int t = 0; t < kTQ; ++t) {
            float v = acc[r][t];
            v = v + __shfl_xor(v, 16);  // accumulators l and l + 16
            v = row16_ggml_fold(v);
            const int e = e0 + re + r, tok = t0 + rt + t;
            if (l == 0 && e < a.E && tok < a.M) a.logits[(size_t)tok * a.E + e] = v;
        }
    (void)lane;
}

// w . x over kRouteN elements in the router's order (lane l of 32 owns
// elements l, l + 32, ...; ggml's f32 dot fold), from memory; every lane of
// the wave returns it.
__device__ __forceinline__ float router_order_dot(const float *w, const float *x) {
    const int l = threadIdx.x & 31;
    float acc = 0.0f;
#pragma unroll 16
    for (int i = 0; i < kRouteN; i += 32) acc = fmaf(w[i + l], x[i + l], acc);
    acc = acc + __shfl_xor(acc, 16);
    acc = acc + __shfl_xor(acc, 8);
    acc = acc + __shfl_xor(acc, 4);
    acc = acc + __shfl_xor(acc, 1);
    acc = acc + __shfl_xor(acc, 2);
    return acc;
}

// One token per workgroup of 640 threads: wave 0 runs the router tail
// (softmax, top-k, renorm) on the token's logits, wave b + 1 forms Q8_K of
// block b of its fx, and wave 9 the shared expert's gate logit.
// The pair's expert for the grouping: its id clamped into range (an id out of
// range counts as expert 0), or -1 where an earlier slot of the token holds the
// same clamped id, so that a token joins a group once.  ids: the token's k ids
// in lanes 0..k-1 of the calling wave.
__device__ __forceinline__ int pair_expert(int id, int j, int k, int n_ids) {
    const int e = (id < 0 || id >= n_ids) ? 0 : id;
    bool first = true;
    for (int i = 0; i < k; ++i) {
        const int o = __shfl(e, i);
        first = first && !(i < j && o == e);
    }
    return first ? e : -1;
}

// One token per workgroup of 64 (nb + 1) threads: wave 0 runs the router tail
// (softmax, top-k, renorm) on the token's logits and writes the pairs' experts
// for the grouping from the selection it holds; wave b + 1 forms Q8_K of block
// b of its fx.
__global__ __launch_bounds__(640) void route_tails_kernel(BatchedArgs a) {
    constexpr int nb = kRouteN / QK;
    static_assert(64 * (nb + 2) == 640, "a tail wave, a wave per fx block and a shared-gate wave");
    const int t = blockIdx.x, wave = wave_index(), lane = threadIdx.x & 63;
    if (wave == 0) {
        const int id = router_tail<false>(a.logits, a.E, a.k, a.renorm, a.sel, a.wsel, t);
        const int e = pair_expert(lane < a.k ? id : 0, lane, a.k, a.n_ids);
        const int kk = a.k + a.sh;  // pair (t, k): the shared expert, id n_ids
        if (lane < kk) a.pexp[(size_t)t * kk + lane] = lane < a.k ? e : a.n_ids;
    } else if (wave <= nb) {
        const int b = wave - 1;
        wave_quantize_q8l(a.fx + (size_t)t * kRouteN + b * QK, q8(a.q8x) + (size_t)t * nb + b);
    } else if (a.sh) {
        const float v = router_order_dot(a.sh_gate_inp, a.fx + (size_t)t * kRouteN);
        if (lane == 0) a.sgl[t] = v;
    }
}

// Caller ids of a prefill-sized batch, one token per workgroup of 512 threads:
// wave b forms Q8_K of block b; wave 0 finds each slot's first occurrence of its
// id within the token (ysrc) and whether the token has an id out of range
// (bad), and writes the pairs' experts for the grouping (none for a bad token
// or a repeated id).
__global__ __launch_bounds__(512) void prep_ids_large_kernel(BatchedArgs a) {
    constexpr int nb = kRouteN / QK;
    const int t = blockIdx.x, wave = wave_index(), lane = threadIdx.x & 63, k = a.k;
    if (wave == 0) {
        const int id = lane < k ? a.sel[(size_t)t * k + lane] : 0;
        const bool bad = __any(lane < k && (id < 0 || id >= a.n_ids));
        int first = lane;
        for (int i = k - 1; i >= 0; --i) {
            const int o = __shfl(id, i);
            if (i < lane && o == id) first = i;
        }
        const int kk = k + a.sh;  // pair (t, k): the shared expert, id n_ids
        if (lane < k) {
            a.ysrc[(size_t)t * k + lane] = first;
            a.pexp[(size_t)t * kk + lane] = (bad || first != lane) ? -1 : id;
        } else if (lane < kk) {
            a.pexp[(size_t)t * kk + lane] = a.n_ids;
        }
        if (lane == 0) a.bad[t] = bad ? 1 : 0;
    }
    if (wave < nb) wave_quantize_q8l(a.fx + (size_t)t * kRouteN + wave * QK, q8(a.q8x) + (size_t)t * nb + wave);
    if (a.sh && wave == 1) {
        const float v = router_order_dot(a.sh_gate_inp, a.fx + (size_t)t * kRouteN);
        if (lane == 0) a.sgl[t] = v;
    }
}

// The grouping of a prefill-sized batch, in one workgroup: the pairs' experts
// are copied into LDS first, so every pass reads them from there.
// The same order with every chunk's masks formed in one pass (when the
// chunks' masks of all experts fit kGroupChunkWords): chunk c (tokens
// [32 c, 32 c + 32)) of expert e has mask cm[c E + e] and starts at cb[c E + e]
// within the expert's run, so a pair's place is its expert's first place, its
// chunk's start and the tokens of its chunk before it that select the expert.
// Three barriers in all, where the chunk loop takes four per chunk.
constexpr int kGroupChunkWords = 8448;  // 16 chunks of 32 tokens x 528 experts
__device__ void group_large_chunks(const BatchedArgs &a, GroupLds &g, const int *pe, unsigned *cm, int *cb,
                                   int *sorted) {
    const int tid = threadIdx.x, nt = blockDim.x, E = a.n_ids + a.sh, k = a.k + a.sh, P = a.M * k;
    const int nch = (a.M + 31) >> 5;
    for (int e = tid; e < E; e += nt) g.cnt[e] = 0u;
    for (int i = tid; i < nch * E; i += nt) cm[i] = 0u;
    __syncthreads();
    for (int p = tid; p < P; p += nt) {
        const int e = pe[p];
        if (e < 0) continue;
        const int t = p / k;
        atomicAdd(&g.cnt[e], 1u);
        atomicOr(&cm[(t >> 5) * E + e], 1u << (t & 31));
    }
    __syncthreads();
    if (tid < 64) {
        group_units(a, g);
    } else {
        for (int e = tid - 64; e < E; e += nt - 64) {
            int run = 0;
            for (int c = 0; c < nch; ++c) {
                cb[c * E + e] = run;
                run += __popc(cm[c * E + e]);
            }
        }
    }
    __syncthreads();
    for (int p = tid; p < P; p += nt) {
        const int e = pe[p];
        if (e < 0) continue;
        const int t = p / k, c = t >> 5;
        const int pos = g.base[e] + cb[c * E + e] + __popc(cm[c * E + e] & ((1u << (t & 31)) - 1u));
        sorted[pos] = t | (p - t * k) << 16;
    }
}

// The pairs are sorted into LDS (token | slot << 16 at each sorted place) and
// copied out in order: scattered 4-byte stores from one CU took 3 us at 4,096
// pairs, the copy a fraction of that.
__global__ __launch_bounds__(1024) void group_kernel(BatchedArgs a) {
    __shared__ GroupLds g;
    __shared__ int pe[kBatchedMaxTokensLarge * kMaxK];
    __shared__ int sorted[kBatchedMaxTokensLarge * kMaxK];
    __shared__ unsigned cm[kGroupChunkWords];
    __shared__ int cb[kGroupChunkWords];
    const int P = a.M * (a.k + a.sh);
    for (int p = threadIdx.x; p < P; p += blockDim.x) pe[p] = a.pexp[p];
    __syncthreads();
    if (((a.M + 31) >> 5) * (a.n_ids + a.sh) <= kGroupChunkWords)
        group_large_chunks(a, g, pe, cm, cb, sorted);
    else
        group_large(a, g, pe, sorted);
    __syncthreads();
    for (int i = threadIdx.x; i < g.total; i += blockDim.x) {
        const int v = sorted[i];
        a.ptok[i] = v & 0xffff;
        a.pslot[i] = v >> 16;
    }
}

// -- caller ids: Q8_K of fx (workgroups 0..M-1, a wave per block) and the
// grouping (workgroup M): each pair's first occurrence of its id within the
// token, tokens with an id out of range, then the groups as for routed ids.
// The counterpart of the verify step's mul_mat_id over the slot pool with the
// host's ids (src/run_specloop.cpp:116-139), where a token's padding repeats an
// id with weight 0.
__global__ __launch_bounds__(512) void prep_ids_kernel(BatchedArgs a) {
    constexpr int nb = kRouteN / QK;
    const int wave = wave_index();
    if ((int)blockIdx.x < a.M) {
        const int t = blockIdx.x;
        for (int b = wave; b < nb; b += 8)
            wave_quantize_q8l(a.fx + (size_t)t * kRouteN + b * QK, q8(a.q8x) + (size_t)t * nb + b);
        if (a.sh && wave == 0) {
            const float v = router_order_dot(a.sh_gate_inp, a.fx + (size_t)t * kRouteN);
            if ((threadIdx.x & 63) == 0) a.sgl[t] = v;
        }
        return;
    }
    __shared__ int bad_s[kMaxTok];
    __shared__ int ysrc_s[kMaxTok * kMaxK];
    __shared__ GroupLds g;
    const int tid = threadIdx.x, P = a.M * a.k;
    for (int t = tid; t < a.M; t += blockDim.x) bad_s[t] = 0;
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
    for (int t = tid; t < a.M; t += blockDim.x) a.bad[t] = bad_s[t];
    group_by_expert(a, g, ysrc_s, bad_s);
}

// Expert groups are computed two ways.  A group of fewer than kMfmaMinTokens
// tokens runs token by token with the per-token row dot, whose cost grows with
// the group; a larger group runs on MFMA, whose cost is that of 16 token
// columns whatever the group's size (two passes over the LDS tile above 16
// tokens).  Both give the per-token path's bits.
// Weight tiles are contiguous rows of the expert and are copied into LDS in
// one burst.

// A group's expert and size, read together (u < the grid's umax keeps them in
// bounds; the grouping leaves expert -1 at every place past the used groups):
// one latency.  Testing both keeps the compiler from moving their loads after
// the test (a group always has an expert >= 0 and a token).
__device__ __forceinline__ bool load_group(const BatchedArgs &a, int u, int &e, int &m) {
    e = a.uexp[u];
    m = min(a.ucount[u], kMaxTok);
    return (e >= 0) & (m >= 1);
}

// Gather the Q8_K row (nb blocks) of token tt into LDS at xs, 16-byte granules
// spread over the workgroup's nw waves (issued, not waited for).
template <int NBX>
__device__ __forceinline__ void gather_token(uint8_t *xs, const uint8_t *q8base, int tt, int wave, int nw) {
    constexpr int kTokGran = NBX * (int)sizeof(Q8L) / 16;
    const int lane = threadIdx.x & 63;
    for (int k = wave; 64 * k < kTokGran; k += nw) {
        const int p = 64 * k + lane;
        if (p < kTokGran) dma_lanes(xs + 1024 * k, q8base + (size_t)tt * (NBX * sizeof(Q8L)) + 16 * p);
    }
}

// -- gate/up: 8 rows of gate (wave 0) and up (wave 1) of one expert ----------
// Per-token dot: one 8-lane group per row, lane t holding the token's Q8_K
// block t.  MFMA (Q4_K groups of kMfmaMinTokens or more): the 8 rows fill a
// 16-row tile twice.  Q3_K groups of any size run token by token.
template <int TGU, int NB>
__global__ __launch_bounds__(128, 3) void gateup_kernel(BatchedArgs a) {
    static_assert(NB == 8, "one 8-lane group per row, one lane per super-block");
    static_assert(TGU == kTypeQ4K || TGU == kTypeQ3K, "gate/up rows are Q4_K or Q3_K");
    constexpr int kRows = 8;
    constexpr int kRowBytes = NB * QType<TGU>::bytes;
    constexpr int kTileBytes = kRows * kRowBytes;
    static_assert(kTileBytes % 16 == 0, "the tile copies in 16-byte units");
    const int u = blockIdx.y;
    const int *tok = a.utok + u * kMaxTok;
    // the group's first four tokens are read with its size and expert (the
    // group's places are in the buffer whatever they turn out to be): one
    // latency, not two
    static_assert(kMaxTok % 4 == 0, "a group's token places are 16-byte aligned");
    const int4 tok4 = *reinterpret_cast<const int4 *>(tok);
    int e, m;
    const bool has = load_group(a, u, e, m);
    asm volatile("" ::"s"(tok4.x), "s"(tok4.y), "s"(tok4.z), "s"(tok4.w));  // loaded before the test, not after
    if (!has) return;
    __shared__ __align__(16) uint8_t wt[2][kTileBytes];
    __shared__ __align__(16) uint8_t xs[kXChunk * NB * sizeof(Q8L)];
    __shared__ float gu[2][kRows][kCols];  // gate and up values of 16 token columns
    const int wave = wave_index(), lane = threadIdx.x & 63, t8 = lane & 7, grp = lane >> 3;
    const int row0 = blockIdx.x * kRows;
    const uint8_t *W = (wave ? batched_up(a, e) : batched_gate(a, e)) + (size_t)row0 * kRowBytes;
    // h = silu(gate) * up of columns c0 .. c0 + 15 from gu (128 threads: 8 rows x 16 columns)
    auto store_h = [&](int c0) {
        __syncthreads();
        const int r = threadIdx.x / kCols, cc = threadIdx.x % kCols;
        if (c0 + cc < m) {
            const float g = gu[0][r][cc], uu = gu[1][r][cc];
            a.hbuf[((size_t)u * kMaxTok + c0 + cc) * a.n_ff + row0 + r] = g / (1.0f + expf(-g)) * uu;
        }
    };
    if (TGU == kTypeQ4K && m >= kMfmaMinTokens) {
        dma_wave_copy_nt(wt[wave], W, kTileBytes);
        lds_dma_wait();
        // 16 token columns at a time over the LDS tile
        for (int c0 = 0; c0 < m; c0 += kCols) {
            if (c0 > 0) __syncthreads();  // the previous columns' h is formed
            const int c = c0 + (lane & 15);
            const Q8L *xq = q8(a.q8x) + (size_t)tok[c < m ? c : 0] * NB;
            float v[4];
            tile_q4k<NB, 7>(wt[wave], kRowBytes, xq, v);
            if (lane < 32) {
#pragma unroll
                for (int i = 0; i < 4; ++i) gu[wave][4 * (lane >> 4) + i][lane & 15] = v[i];
            }
            store_h(c0);
        }
        return;
    }
    // token by token: x goes into LDS with the tile, kXChunk tokens at a time (a
    // vector load issued during the compute would queue behind the tile copies
    // of the other workgroups on this CU); h is stored every 16 token columns
    const Q8L *xl = reinterpret_cast<const Q8L *>(xs);
    for (int c0 = 0; c0 < m; c0 += kXChunk) {
        const int mc = min(m - c0, kXChunk);
        if (c0 > 0) __syncthreads();  // both waves are done with the previous chunk
        static_assert(kXChunk == 1, "one token a copy");
        const int tt = c0 == 0 ? tok4.x : c0 == 1 ? tok4.y : c0 == 2 ? tok4.z : c0 == 3 ? tok4.w : tok[c0];
        gather_token<NB>(xs, a.q8x, tt, wave, 2);
        if (c0 == 0) dma_wave_copy_nt(wt[wave], W, kTileBytes);
        lds_dma_wait();
        __syncthreads();
#pragma unroll 1
        for (int c = 0; c < mc; ++c) {
            const uint8_t *rp = wt[wave] + grp * kRowBytes;
            float v;
            if constexpr (TGU == kTypeQ3K)
                v = lpb_row_q3k_mem<NB, true>(rp, xl[c * NB + t8], t8);
            else
                v = lpb_row_q4k_mem<NB, true>(rp, xl[c * NB + t8], t8);
            if (t8 == NB - 1) gu[wave][grp][(c0 + c) % kCols] = v;
        }
        static_assert(kCols % kXChunk == 0, "a chunk of tokens stays within 16 columns");
        if ((c0 + mc) % kCols == 0 && c0 + mc < m) store_h(c0 + mc - kCols);  // a full 16 columns, more to come
    }
    store_h((m - 1) / kCols * kCols);
}

// -- Q8_K of h per (expert, token) ---------------------------------------------
// One workgroup per (group, token), a wave per 256-element block of h.
__global__ __launch_bounds__(256) void quant_h_kernel(BatchedArgs a) {
    const int u = blockIdx.y, c = blockIdx.x, b = wave_index();
    const int nbh = a.n_ff / QK;
    const size_t uc = (size_t)u * kMaxTok + c;
    // h is loaded with the group count and size, not after them (its place
    // does not depend on them; a place past the groups is in the buffer and
    // its values are dropped), all three as vector loads in flight together
    // (u < the grid's umax and b < nbh keep them in bounds)
    const int nu = __hip_atomic_load(a.n_unique, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + a.sh;
    const int cnt = __hip_atomic_load(a.ucount + u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const float4 v4 = *reinterpret_cast<const float4 *>(a.hbuf + uc * a.n_ff + (size_t)b * QK + 4 * (threadIdx.x & 63));
    asm volatile("" ::"v"(v4.x), "v"(v4.y), "v"(v4.z), "v"(v4.w));  // the load is not moved past the test
    if (u >= nu || c >= min(cnt, kMaxTok)) return;
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    wave_quantize_q8l_regs(v, q8(a.q8h) + uc * nbh + b);
}

// -- down: one 16-row tile of one expert; y to Y[token][slot] -------------------
// Q6_K rows are only 2-byte aligned, which LDS reads handle with alignbyte;
// the per-token Q6_K dot wants one alignment per wave, so each pass takes the
// rows of one parity (the row size is 2 mod 4).
template <int TD, int NBH>
__device__ __forceinline__ void down_group(const BatchedArgs &a, int u, int e, int m, uint8_t *tile, uint8_t *xs) {
    constexpr int kRowBytes = NBH * QType<TD>::bytes;
    constexpr int kTileBytes = kTile * kRowBytes;
    const int lane = threadIdx.x & 63, t8 = lane & 7, grp = lane >> 3;
    const int row0 = blockIdx.x * kTile;
    const int *tok = a.utok + u * kMaxTok, *slot = a.uslot + u * kMaxTok;
    const uint8_t *src = batched_down(a, e) + (size_t)row0 * kRowBytes;
    const int kk = a.k + a.sh;  // output slots per token
    if (TD != kTypeQ5K && m >= kMfmaMinTokens) {  // Q5_K groups of any size run token by token
        dma_wave_copy_nt(tile, src, kTileBytes);
        lds_dma_wait();
        // 16 token columns at a time over the LDS tile
        for (int c0 = 0; c0 < m; c0 += kCols) {
            const int c = c0 + (lane & 15);
            const Q8L *xq = q8(a.q8h) + ((size_t)u * kMaxTok + (c < m ? c : 0)) * NBH;
            float v[4];
            if constexpr (TD == kTypeQ4K)
                tile_q4k<NBH>(tile, kRowBytes, xq, v);
            else if constexpr (TD == kTypeQ6K)
                tile_q6k<NBH>(tile, kRowBytes, xq, v);
            if (c < m) {
                float *y = a.ybuf + ((size_t)tok[c] * kk + slot[c]) * a.n_embd + row0;
#pragma unroll
                for (int i = 0; i < 4; ++i) y[4 * (lane >> 4) + i] = v[i];
            }
        }
        return;
    }
    const Q8L *xl = reinterpret_cast<const Q8L *>(xs);
    for (int c0 = 0; c0 < m; c0 += kXChunk) {
        const int mc = min(m - c0, kXChunk);
        // the group's Q8_K h rows are contiguous, token-major
        dma_wave_copy(xs, a.q8h + ((size_t)u * kMaxTok + c0) * NBH * sizeof(Q8L), mc * NBH * (int)sizeof(Q8L));
        if (c0 == 0) dma_wave_copy_nt(tile, src, kTileBytes);
        lds_dma_wait();
#pragma unroll 1
        for (int c = 0; c < mc; ++c) {
            float *y = a.ybuf + ((size_t)tok[c0 + c] * kk + slot[c0 + c]) * a.n_embd + row0;
            if constexpr (TD == kTypeQ6K) {
#pragma unroll 1
                for (int p = 0; p < 2; ++p) {
                    const int row = 2 * grp + p;
                    const float v = g8_row_q6k_u<NBH>(tile + row * kRowBytes, xl + c * NBH, t8);
                    if (t8 == 0) y[row] = v;
                }
            } else if constexpr (TD == kTypeQ5K) {
#pragma unroll 1
                for (int p = 0; p < 2; ++p) {  // the single-token down kernel's Q5_K row dot
                    const int row = 8 * p + grp;
                    const float v = g8_row_q5k(tile + row * kRowBytes, xl + c * NBH, NBH, t8);
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

// TD: the routed experts' down type; TS: the shared expert's (Q6_K beside
// Q5_K routed rows, as Qwen3.5 has them), run by the same launch.
template <int TD, int NBH, int TS = TD>
__global__ __launch_bounds__(64, 4) void down_kernel(BatchedArgs a) {
    constexpr int kTileBytes = kTile * NBH * (QType<TD>::bytes > QType<TS>::bytes ? QType<TD>::bytes : QType<TS>::bytes);
    const int u = blockIdx.y;
    int e, m;
    if (!load_group(a, u, e, m)) return;
    __shared__ __align__(16) uint8_t tile[kTileBytes];
    __shared__ __align__(16) uint8_t xs[kXChunk * NBH * sizeof(Q8L)];
    if (TS != TD && a.sh && e == a.n_ids)
        down_group<TS, NBH>(a, u, e, m, tile, xs);
    else
        down_group<TD, NBH>(a, u, e, m, tile, xs);
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
    const int kk = a.k + a.sh;
    // every load is issued before the first is used: one memory latency, not k
    float w[kMaxK], y[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        if (j < a.k) {
            const int js = a.ysrc ? a.ysrc[t * a.k + j] : j;  // a repeated id takes its first output
            w[j] = a.wsel[t * a.k + j];
            y[j] = a.ybuf[((size_t)t * kk + js) * a.n_embd + d];
        }
    }
    const float ysh = a.sh ? a.ybuf[((size_t)t * kk + a.k) * a.n_embd + d] : 0.0f;
    const float r = a.res[(size_t)t * a.n_embd + d];
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
        if (j < a.k) acc = acc + w[j] * y[j];
    if (a.sh) {  // + sigmoid(gate logit) * shared expert output
        const float sg = 1.0f / (1.0f + expf(-a.sgl[t]));
        acc = acc + ysh * sg;
    }
    a.out[(size_t)t * a.n_embd + d] = acc + r;
}

}  // namespace

bool batched_shape_compiled(int gu_type, int n_embd, int d_type, int n_ff) {
    return (gu_type == kTypeQ4K || gu_type == kTypeQ3K) && n_embd == 2048 &&
           (n_ff == 768 || n_ff == 1024 || n_ff == 512) &&
           (d_type == kTypeQ4K || d_type == kTypeQ6K || (d_type == kTypeQ5K && n_ff != 768));
}

namespace {

// The launches after the grouping: gate/up, Q8_K(h), down, combine.
hipError_t launch_groups(const BatchedArgs &a, hipStream_t s) {
    const int nbh = a.n_ff / QK;
    const int umax = (a.n_ids < a.M * a.k ? a.n_ids : a.M * a.k) + a.sh;
    if (a.gu_type == kTypeQ3K)
        hipLaunchKernelGGL((gateup_kernel<kTypeQ3K, 8>), dim3(a.n_ff / 8, umax), dim3(128), 0, s, a);
    else
        hipLaunchKernelGGL((gateup_kernel<kTypeQ4K, 8>), dim3(a.n_ff / 8, umax), dim3(128), 0, s, a);
    // a group holds at most M (<= kMaxTok) tokens
    hipLaunchKernelGGL(quant_h_kernel, dim3(a.M, umax), dim3(64 * nbh), 0, s, a);
    const dim3 dg(a.n_embd / kTile, umax);
#define HOARD_DOWN(T, N, TS)                                                    \
    if (a.d_type == T && nbh == N && sd == TS) {                                \
        hipLaunchKernelGGL((down_kernel<T, N, TS>), dg, dim3(64), 0, s, a);     \
    } else
    const int sd = a.sh ? a.sh_d_type : a.d_type;
    HOARD_DOWN(kTypeQ6K, 3, kTypeQ6K) HOARD_DOWN(kTypeQ6K, 2, kTypeQ6K) HOARD_DOWN(kTypeQ6K, 4, kTypeQ6K)
    HOARD_DOWN(kTypeQ4K, 4, kTypeQ4K) HOARD_DOWN(kTypeQ4K, 3, kTypeQ4K) HOARD_DOWN(kTypeQ4K, 2, kTypeQ4K)
    HOARD_DOWN(kTypeQ5K, 2, kTypeQ5K) HOARD_DOWN(kTypeQ5K, 4, kTypeQ5K) HOARD_DOWN(kTypeQ5K, 2, kTypeQ6K) {
        return hipErrorInvalidValue;
    }
#undef HOARD_DOWN
    hipLaunchKernelGGL(combine_kernel, dim3((a.n_embd + 255) / 256, a.M), dim3(256), 0, s, a);
    return hipGetLastError();
}

bool args_ok(const BatchedArgs &a) {
    return a.M >= 1 && a.M <= kBatchedMaxTokensLarge && a.n_embd == kRouteN &&
           (a.gu_type == kTypeQ4K || a.gu_type == kTypeQ3K) &&
           a.k + a.sh <= kMaxK && a.n_ids >= 1 && a.n_ids + a.sh <= kMaxExperts && a.E + a.sh <= kMaxExperts &&
           (!a.sh || (a.sh == 1 && a.sh_gate && a.sh_up && a.sh_down && a.sh_gate_inp && a.sgl)) &&
           (a.M <= kMaxTok || (a.goff && a.ptok && a.pslot && a.pexp && a.units && a.n_units && a.max_units >= 1));
}

}  // namespace

// Batches of up to 32 tokens group by expert with 32 token places per group;
// larger ones sort the pairs and run the prefill units (prefill.hip).
hipError_t launch_batched(const BatchedArgs &a, hipStream_t s) {
    if (!args_ok(a) || a.ysrc || a.n_ids != a.E || (a.M + kRouteTok - 1) / kRouteTok > kBatchedCounters - 1)
        return hipErrorInvalidValue;
    if (a.M > kMaxTok) {
        const unsigned et = (a.E + kTileE - 1) / kTileE;
        const dim3 rg(et, (a.M + 15) / 16);
        if (rg.x * rg.y > 256)  // more tiles than CUs: two workgroups a CU
            hipLaunchKernelGGL((route_gemm_kernel<256, 16>), rg, dim3(512), 0, s, a);
        else if (rg.x * rg.y > 128)
            hipLaunchKernelGGL((route_gemm_kernel<512, 16>), rg, dim3(512), 0, s, a);
        else  // at most half the CUs with 16-token tiles: 8-token ones, at most one a CU
            hipLaunchKernelGGL((route_gemm_kernel<512, 8>), dim3(et, (a.M + 7) / 8), dim3(512), 0, s, a);
        hipLaunchKernelGGL(route_tails_kernel, dim3(a.M), dim3(640), 0, s, a);
        hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, s, a);
        return launch_prefill_groups(a, s);
    }
    // row workgroups: a remainder of one row joins the last workgroup
    const int nr = a.E + a.sh, ntg = (a.M + kRouteTok - 1) / kRouteTok;
    auto row_groups = [nr](int R) { return nr > R && nr % R == 1 ? nr / R : (nr + R - 1) / R; };
    if (a.M > 8)
        hipLaunchKernelGGL(route_kernel<4>, dim3(row_groups(4), ntg), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(route_kernel<2>, dim3(row_groups(2), ntg), dim3(256), 0, s, a);
    return launch_groups(a, s);
}

hipError_t launch_batched_ids(const BatchedArgs &a, hipStream_t s) {
    if (!args_ok(a) || !a.ysrc || !a.bad) return hipErrorInvalidValue;
    if (a.M > kMaxTok) {
        hipLaunchKernelGGL(prep_ids_large_kernel, dim3(a.M), dim3(512), 0, s, a);
        hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, s, a);
        return launch_prefill_groups(a, s);
    }
    hipLaunchKernelGGL(prep_ids_kernel, dim3((unsigned)a.M + 1), dim3(512), 0, s, a);
    return launch_groups(a, s);
}

}  // namespace hoard
