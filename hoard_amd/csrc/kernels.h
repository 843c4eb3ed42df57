// Internal launch interface between the C++ orchestrator (moe.cpp) and the
// HIP kernels.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace hoard {

// Router tail for M tokens (grid.y = token).  When `xin_is_residual`, fx is
// rms_norm(xin, eps) and is also written to fx_out; otherwise xin is fx.
struct RouterArgs {
    const float *xin;      // [M][n]
    float *fx_out;         // [M][n] (rms-norm mode only)
    float eps;
    int xin_is_residual;
    const float *w;        // [E][n]
    int n, E, k, renorm, M;
    float *logits;         // scratch [M][E]
    unsigned *counters;    // [M], zero on entry, left zero on exit
    int32_t *sel;          // [M][k]
    float *wsel;           // [M][k]
};
hipError_t launch_router(const RouterArgs &a, hipStream_t s);

// Expert "matrix" descriptor: matrix of expert id at base + id*stride.
struct MatDesc {
    const uint8_t *base;
    size_t stride;    // bytes per expert (0 for a single fixed matrix)
    int type;         // ggml type id
    int rows, cols;
    int n_ids;        // number of valid ids (experts or slots); ids outside -> poison
};

// g/u GEMVs + SwiGLU for k routed experts (ids[j]) and optionally one fixed
// shared expert, one token.  h[j*hstride + r] = silu(g_r) * u_r.
struct GateUpArgs {
    const float *fx;        // [n_embd]
    const int32_t *ids;     // [k]
    MatDesc gate, up;       // routed
    MatDesc sh_gate, sh_up; // shared (base == nullptr: none)
    const float *sh_gate_inp; // [n_embd] f32 gate row of the shared expert
    float *sgate;           // [1] out: sigmoid(sh_gate_inp . fx)
    int n_embd, k;
    float *h;               // [(k+1)][hstride]
    int hstride;
};
hipError_t launch_gateup(const GateUpArgs &a, hipStream_t s);

// Down GEMVs over all selected experts for a slice of output rows, fused with
// the weighted combine: out[d] = ((sum_j w_j*y_j[d]) + sgate*ysh[d]) + res[d].
struct DownArgs {
    const float *h;         // [(k+1)][hstride]
    int hstride;
    const int32_t *ids;     // [k]
    const float *w;         // [k]
    MatDesc down, sh_down;  // sh_down.base == nullptr: none
    const float *sgate;     // [1] (when shared)
    int n_embd, k;
    const float *res;
    float *out;
};
hipError_t launch_down_combine(const DownArgs &a, hipStream_t s);

size_t block_bytes(int type);

}  // namespace hoard
