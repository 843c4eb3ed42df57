// Router tail for one token on one wave: softmax over all experts, top-k
// (larger probability first, lower index on ties) and the optional renorm.
// Counterpart of ggml_soft_max + ggml_top_k + ggml_get_rows
// (src/run_moe_stream.cpp:354-356) and the host renorm (:371-373).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "wave.h"

namespace hoard {

constexpr int kMaxExpertsPerLane = 16;  // E <= 1024
constexpr int kMaxK = 16;

// The softmax of one token's logits lg[0, E) on one wave: p[t] holds expert
// lane + 64 t (experts past E hold -infinity).  The tail below and every
// other selection of these probabilities form them here, so they agree bit
// for bit.
template <bool AGENT, int NT>
__device__ inline void softmax_nt(const float *lg, int E, float (&p)[NT]) {
    const int lane = threadIdx.x & 63;
    const int nt = NT;
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int e = lane + 64 * t;
        float v = -INFINITY;
        if (t < nt && e < E) {
            if constexpr (AGENT)
                v = __hip_atomic_load(lg + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else
                v = lg[e];
        }
        p[t] = v;
        mx = p[t] > mx ? p[t] : mx;
    }
    mx = wave_max_f(mx);
    // softmax: exp(l - max), sum in double, scale by (float)(1/sum)
    double sum = 0.0;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int e = lane + 64 * t;
        if (t < nt && e < E) {
            p[t] = expf(p[t] - mx);
            sum += (double)p[t];
        }
    }
    sum = wave_sum_d(sum);
    const float sc = (float)(1.0 / sum);
#pragma unroll
    for (int t = 0; t < NT; ++t) p[t] = p[t] * sc;
}

// Wave-uniform results: the reductions are DPP butterflies (wave.h).  The max
// and the top-k argmax are order-independent; the double-precision sum of
// the probabilities is exact unless they span more than 2^29 in magnitude,
// and its float reciprocal absorbs the remaining rounding differences.
// AGENT: the logits come from other workgroups of the same launch and are read
// at device (agent) scope, which bypasses the per-XCD L2, instead of behind a
// cache-flushing fence.  STORE_AGENT: sel / wsel go to other workgroups and
// are written at device scope; otherwise plain stores (global memory of this
// workgroup's own use, or LDS).
// NT: experts per lane the body is compiled for (E <= 64 NT, E <= 1024).
template <bool AGENT, int NT, bool STORE_AGENT = AGENT>
__device__ inline int router_tail_nt(const float *logits, int E, int k, int renorm, int32_t *sel, float *wsel,
                                     int tok) {
    const int lane = threadIdx.x & 63;
    float p[NT];
    softmax_nt<AGENT, NT>(logits + (size_t)tok * E, E, p);

    // top-k: repeated wave max, larger probability first, lower index on ties.
    // A taken or absent expert holds -1 (probabilities are >= 0); the lowest
    // index holding the max comes from the ballots of the slots, low slot
    // (lower experts) first.
#pragma unroll
    for (int t = 0; t < NT; ++t)
        if (!(lane + 64 * t < E)) p[t] = -1.0f;
    int my_sel = 0;
    float my_w = 0.0f, ws = 0.0f;
    for (int j = 0; j < k; ++j) {
        float lm = p[0];
#pragma unroll
        for (int t = 1; t < NT; ++t) lm = p[t] > lm ? p[t] : lm;
        const float bv = wave_max_f(lm);
        int be = 0x7fffffff;
#pragma unroll
        for (int t = NT - 1; t >= 0; --t) {
            const uint64_t b = __ballot(p[t] == bv);
            if (b) be = 64 * t + (int)__builtin_ctzll(b);
        }
        if (be != 0x7fffffff && (be & 63) == lane) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
                if (t == (be >> 6)) p[t] = -1.0f;
        }
        if (lane == j) {
            my_sel = be;
            my_w = bv;
        }
        ws = ws + bv;  // the top-k weights summed in selection order
    }
    if (renorm) {
        if (ws < 6.103515625e-5f) ws = 6.103515625e-5f;
        my_w = my_w / ws;
    }
    if (lane < k) {
        if constexpr (STORE_AGENT) {
            __hip_atomic_store(sel + (size_t)tok * k + lane, my_sel, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(wsel + (size_t)tok * k + lane, my_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            sel[(size_t)tok * k + lane] = my_sel;
            wsel[(size_t)tok * k + lane] = my_w;
        }
    }
    return my_sel;
}

// Returns the selection of slot `lane` in lane `lane` (lanes < k).
template <bool AGENT = false, bool STORE_AGENT = AGENT>
__device__ inline int router_tail(const float *logits, int E, int k, int renorm, int32_t *sel, float *wsel, int tok) {
    if (E <= 64)
        return router_tail_nt<AGENT, 1, STORE_AGENT>(logits, E, k, renorm, sel, wsel, tok);
    else if (E <= 128)
        return router_tail_nt<AGENT, 2, STORE_AGENT>(logits, E, k, renorm, sel, wsel, tok);
    else if (E <= 256)
        return router_tail_nt<AGENT, 4, STORE_AGENT>(logits, E, k, renorm, sel, wsel, tok);
    else if (E <= 512)
        return router_tail_nt<AGENT, 8, STORE_AGENT>(logits, E, k, renorm, sel, wsel, tok);
    else
        return router_tail_nt<AGENT, kMaxExpertsPerLane, STORE_AGENT>(logits, E, k, renorm, sel, wsel, tok);
}

}  // namespace hoard
