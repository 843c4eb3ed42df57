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
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l = lane & 31;
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
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
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
        wave_copy(wt[m] + off, (m ? usrc : gsrc) + off, len);
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
// dotted with unit (u0 + r / 8)'s Q8_K(h); results to ys[u0 * 8 + r].
template <int T, int NB>
__device__ __forceinline__ void down_rows(const uint8_t *base, int n, int u0, const Q8L *q8h, float *ys) {
    constexpr int kRowBytes = NB * QType<T>::bytes;
    const int wave = threadIdx.x >> 6, grp = threadIdx.x >> 3, t8 = threadIdx.x & 7;
    if constexpr (T == kTypeQ6K) {
        // 8 lanes per row; a wave takes rows of one parity so that its 2-byte
        // aligned rows share their 4-byte alignment
        const int par = wave & 1, G = (wave >> 1) * 8 + (grp & 7);
        for (int m = G; m < n / 2; m += 64) {
            const int r = 2 * m + par, u = u0 + r / kDownRows;
            const float y = g8_row_q6k_u<NB>(base + r * kRowBytes, q8h + u * NB, t8);
            if (t8 == 0) ys[u0 * kDownRows + r] = y;
        }
    } else {
        // one 8-lane group per row, lane t taking super-block t
        for (int r = grp; r < n; r += 128) {
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
    const int wave = threadIdx.x >> 6;
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
                wave_copy(wd + u * kSegBytes, a.down.base + (size_t)id * a.down.stride + (size_t)d0 * kRowBytes,
                          kSegBytes);
            } else {
                wave_copy(wd + k * kSegBytes, a.sh_down.base + (size_t)d0 * (kSegBytesS / kDownRows), kSegBytesS);
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
        down_rows<TD, NBH>(wd, nu * kDownRows, 0, q8h, ys);  // the shared segment follows the routed ones
    } else {
        down_rows<TD, NBH>(wd, k * kDownRows, 0, q8h, ys);
        if (has_sh) down_rows<TS, NBH>(wd + k * kSegBytes, kDownRows, k, q8h, ys);
    }
    __syncthreads();
    if (threadIdx.x < kDownRows) {
        const int r = threadIdx.x, d = d0 + r;
        float acc = 0.0f;
        for (int j = 0; j < k; ++j) acc = acc + a.w[j] * ys[j * kDownRows + r];
        a.out[d] = has_sh ? (acc + ys[k * kDownRows + r] * a.sgate[0]) + a.res[d] : acc + a.res[d];
    }
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
