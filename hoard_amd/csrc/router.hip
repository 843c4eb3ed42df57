// Fused router tail (kernel family 1): f32 router GEMV, softmax over all
// experts, top-k, gather and optional renorm, in one launch.
//
// Replaces ggml_mul_mat(ffn_gate_inp, fx) + ggml_soft_max + ggml_top_k +
// ggml_get_rows (src/run_moe_stream.cpp:353-356, src/run_qwen35.cpp:556-559)
// and the host renorm (src/run_moe_stream.cpp:371-373).
//
// Layout: one 64-lane wave per workgroup computes two router rows; lane l of a
// row owns elements l, l+32, l+64, ... and keeps one fused multiply-add chain,
// the same 32 accumulators ggml's x86 f32 dot keeps (4 vectors x 8 lanes), and
// folds them in that dot's order (16, 8, 4 lanes apart, then pairs), so the
// logits are the CPU path's bit for bit.  The last workgroup to finish a token
// (device-scope counter) runs softmax / top-k on one wave.
#include "kernels.h"
#include "qblocks.h"
#include "router_tail.h"

namespace hoard {

namespace {

constexpr int kMaxRouterTokens = 16;    // tokens per call of the multi-token logits kernel

__global__ __launch_bounds__(64) void router_kernel(RouterArgs a) {
    const int lane = threadIdx.x;
    const int half = lane >> 5, l = lane & 31;
    const int tok = blockIdx.y;
    const int n = a.n, E = a.E;
    const float *x = a.xin + (size_t)tok * n;
    const int row = blockIdx.x * 2 + half;

    float scale = 1.0f;
    if (a.xin_is_residual) {
        // rms_norm: mean of x*x accumulated in double, scale = 1/sqrtf(mean + eps)
        double ss = 0.0;
        for (int i = lane; i < n; i += 64) {
            const float v = x[i];
            ss += (double)(v * v);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
        const float mean = (float)(ss / (double)n);
        scale = 1.0f / sqrtf(mean + a.eps);
        if (blockIdx.x == 0) {
            float *fo = a.fx_out + (size_t)tok * n;
            for (int i = lane; i < n; i += 64) fo[i] = x[i] * scale;
        }
    }

    if (row < E) {
        const float *wr = a.w + (size_t)row * n;
        float acc = 0.0f;
        if (a.xin_is_residual) {
#pragma unroll 8
            for (int i = 0; i < n; i += 32) acc = fmaf(wr[i + l], x[i + l] * scale, acc);
        } else {
#pragma unroll 8
            for (int i = 0; i < n; i += 32) acc = fmaf(wr[i + l], x[i + l], acc);
        }
        acc = acc + __shfl_xor(acc, 16);
        acc = acc + __shfl_xor(acc, 8);
        acc = acc + __shfl_xor(acc, 4);
        acc = acc + __shfl_xor(acc, 1);
        acc = acc + __shfl_xor(acc, 2);
        if (l == 0) a.logits[(size_t)tok * E + row] = acc;
    }

    // ---- the last workgroup of this token runs the tail ----
    __shared__ int is_last;
    __threadfence();
    if (lane == 0) is_last = atomicAdd(&a.counters[tok], 1u) == gridDim.x - 1;
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    router_tail(a.logits, a.E, a.k, a.renorm, a.sel, a.wsel, tok);
    if (lane == 0) a.counters[tok] = 0u;
}

// Logits for M > 1 tokens (xin = fx): a workgroup of 4 waves takes 8 rows
// (32 lanes per row) against 4 tokens staged in LDS, so the router weight is
// read M/4 times per call instead of M times.  Per token the accumulation
// order is the single-token kernel's.
constexpr int kRowsPerWg = 8;
constexpr int kTokPerWg = 4;

__global__ __launch_bounds__(256) void router_rows_m_kernel(RouterArgs a) {
    extern __shared__ float xs[];  // [kTokPerWg][n]
    const int n = a.n, E = a.E;
    const int t0 = blockIdx.y * kTokPerWg;
    const int nt = min(kTokPerWg, a.M - t0);
    const float4 *src = reinterpret_cast<const float4 *>(a.xin + (size_t)t0 * n);
    for (int i = threadIdx.x; i < nt * n / 4; i += blockDim.x) reinterpret_cast<float4 *>(xs)[i] = src[i];
    __syncthreads();
    const int wave = wave_index(), lane = threadIdx.x & 63, l = lane & 31;
    const int row = blockIdx.x * kRowsPerWg + wave * 2 + (lane >> 5);
    if (row >= E) return;
    const float *wr = a.w + (size_t)row * n;
    float acc[kTokPerWg] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i0 = 0; i0 < n; i0 += 32 * 16) {
        float w[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = i0 + 32 * i < n ? wr[i0 + 32 * i + l] : 0.0f;
#pragma unroll
        for (int t = 0; t < kTokPerWg; ++t) {
            if (t < nt) {
                const float *x = xs + t * n + i0 + l;
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (i0 + 32 * i < n) acc[t] = fmaf(w[i], x[32 * i], acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kTokPerWg; ++t) {
        if (t < nt) {
            float v = acc[t];
            v = v + __shfl_xor(v, 16);
            v = v + __shfl_xor(v, 8);
            v = v + __shfl_xor(v, 4);
            v = v + __shfl_xor(v, 1);
            v = v + __shfl_xor(v, 2);
            if (l == 0) a.logits[(size_t)(t0 + t) * E + row] = v;
        }
    }
}

// Softmax, top-k and renorm of one token per workgroup (M > 1).
__global__ __launch_bounds__(64) void router_tail_kernel(RouterArgs a) {
    router_tail(a.logits, a.E, a.k, a.renorm, a.sel, a.wsel, blockIdx.x);
}

}  // namespace

hipError_t launch_router(const RouterArgs &a, hipStream_t s) {
    if (a.M > 1 && !a.xin_is_residual && a.M <= kMaxRouterTokens) {
        const dim3 grid((unsigned)((a.E + kRowsPerWg - 1) / kRowsPerWg), (unsigned)((a.M + kTokPerWg - 1) / kTokPerWg));
        const size_t lds = sizeof(float) * kTokPerWg * (size_t)a.n;
        if (lds > 65536) return hipErrorInvalidValue;
        hipLaunchKernelGGL(router_rows_m_kernel, grid, dim3(256), lds, s, a);
        hipLaunchKernelGGL(router_tail_kernel, dim3((unsigned)a.M), dim3(64), 0, s, a);
        return hipGetLastError();
    }
    dim3 grid((unsigned)((a.E + 1) / 2), (unsigned)a.M);
    hipLaunchKernelGGL(router_kernel, grid, dim3(64), 0, s, a);
    return hipGetLastError();
}

}  // namespace hoard
