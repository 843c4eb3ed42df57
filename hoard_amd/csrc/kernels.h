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

// Batched expert stage for M tokens: grouping by expert, int8-MFMA
// gate/up (+SwiGLU) and down tiles, ordered combine.
struct BatchedArgs {
    int M, n_embd, n_ff, E, k;
    int gu_type, d_type;
    const float *fx;        // [M][n_embd] normalised inputs
    const float *res;       // [M][n_embd]
    float *out;             // [M][n_embd] (may alias res)
    const float *router;    // [E][n_embd] f32 router weight
    int renorm;             // renormalise the top-k weights
    float *logits;          // [M][E] scratch
    unsigned *counters;     // [kBatchedCounters], zero on entry, left zero on exit
    int32_t *sel;           // [M][k] selected experts (written by the call)
    float *wsel;            // [M][k] their weights
    const uint8_t *gate, *up, *down;
    size_t gstride, ustride, dstride;
    uint8_t *q8x;           // Q8_K(fx): [M][n_embd/256] blocks of 304 bytes
    uint8_t *q8h;           // Q8_K(h):  [umax][kBatchedMaxTokens][n_ff/256] blocks
    float *hbuf;            // [umax][kBatchedMaxTokens][n_ff]
    float *ybuf;            // [M][k + sh][n_embd]: slot k holds the shared expert's output
    int *n_unique;          // [1]
    int *slot_of;           // [E] scratch
    int *uexp, *ucount;     // [umax] expert of each group, tokens in it
    int *utok, *uslot;      // [umax][kBatchedMaxTokens] token and slot of each member
    unsigned *hist;         // [n_ids] tokens per expert (or slot) in the call
    int n_ids;              // id space the groups are formed over: E, or the slots of a pool
    int *ysrc;              // [M][k] caller ids only: the slot j' <= j whose output pair (t, j) takes
                            // (its first occurrence of the same id), else null
    int *bad;               // [M] caller ids only: 1 for a token with an id outside [0, n_ids), else null
    // prefill-sized batches (M > kBatchedMaxTokens): the pairs sorted by (expert, token)
    // and cut into work units of at most kUnitTokens pairs of one expert
    int *goff;              // [umax] first sorted position of each group
    int *ptok, *pslot;      // [M*k] token and slot of each sorted pair
    int *pexp;              // [M*k] expert of each pair for the grouping, -1 for one that joins none
    int *units;             // [max_units][4] expert, first sorted pair, pairs (0: no unit), unused
    float *q8hd;            // [pairs][4] the scales d of each sorted pair's Q8_K(h) blocks (prefill)
    int *n_units;           // [1]
    int max_units;
    // The gated shared expert (sh = 1): every token's pair (t, k) with the
    // expert id n_ids, whose weights are these tensors (n_ff rows, the routed
    // experts' types), and out = (sum_j w_j y_j + sigmoid(sgl[t]) * y_k) + res.
    int sh;                       // 1 with a shared expert, else 0
    int sh_d_type;                // its down type: d_type, or Q6_K beside Q5_K routed rows
    const uint8_t *sh_gate, *sh_up, *sh_down;
    const float *sh_gate_inp;     // [n_embd] f32 gate row of the shared expert
    float *sgl;                   // [M] sh_gate_inp . fx[t] (the logit, before the sigmoid)
};
// Expert e's matrices in a batched call; e == n_ids is the shared expert.
__device__ __forceinline__ const uint8_t *batched_gate(const BatchedArgs &a, int e) {
    return a.sh && e == a.n_ids ? a.sh_gate : a.gate + (size_t)e * a.gstride;
}
__device__ __forceinline__ const uint8_t *batched_up(const BatchedArgs &a, int e) {
    return a.sh && e == a.n_ids ? a.sh_up : a.up + (size_t)e * a.ustride;
}
__device__ __forceinline__ const uint8_t *batched_down(const BatchedArgs &a, int e) {
    return a.sh && e == a.n_ids ? a.sh_down : a.down + (size_t)e * a.dstride;
}
constexpr int kBatchedMaxTokens = 32;         // the verify-sized path: per-token dots or MFMA per group
constexpr int kBatchedMaxTokensLarge = 512;   // the prefill-sized path: sorted pairs, MFMA units
constexpr int kUnitTokens = 64;               // pairs of one expert per prefill work unit
constexpr int kBatchedCounters = 160;         // route completion counters: one per 4 tokens, and the tails'
constexpr size_t kQ8LBytes = 304;
hipError_t launch_batched(const BatchedArgs &a, hipStream_t s);
// The same expert products and combine for the caller's ids (a.sel) and weights (a.wsel).
hipError_t launch_batched_ids(const BatchedArgs &a, hipStream_t s);
bool batched_shape_compiled(int gu_type, int n_embd, int d_type, int n_ff);
// The allocation-free batched entry point's fixed scratch (noalloc.hip): the
// route counters lead it, zeroed at set-up; the rest is laid out per call.
constexpr int kNoAllocMaxTokens = 16;
constexpr size_t kNoAllocCounterBytes = 1024;
hipError_t noalloc_setup(int device);
uint8_t *noalloc_scratch(int device);
size_t noalloc_scratch_bytes();
// The expert products and combine of a prefill-sized batch after its grouping
// (prefill.hip): gate/up + SwiGLU, Q8_K(h), down, ordered combine.
hipError_t launch_prefill_groups(const BatchedArgs &a, hipStream_t s);
// Upper bound of the prefill work units for M*k pairs over n_ids groups.
inline int prefill_max_units(int M, int k, int n_ids) {
    const int P = M * k, umax = n_ids < P ? n_ids : P;
    return umax + (P + kUnitTokens - 1) / kUnitTokens;
}

// Persistent stacked decode (one cooperative launch per token).
struct DecodeLayer {
    const float *router;
    const uint8_t *gate, *up, *down;
    size_t gstride, ustride, dstride;
    int gate_type, up_type, down_type;
    // shared expert (spread kernel only; null without one)
    const uint8_t *sh_gate, *sh_up, *sh_down;
    const float *sh_gate_inp;
};
struct PersistentArgs {
    const DecodeLayer *layers;  // device array, indexed by layer
    int l0, l1;
    float *x;                   // [n_embd] in/out
    float eps;
    int n_embd, E, k, n_ff, renorm;
    int rows_gu, rows_d;        // n_ff/32 and n_embd/32 rows per workgroup
    int max_rb_gu, max_rb_d;    // largest gate/up and down row bytes over the layers
    int gu_type, d_type;        // gate/up and down types, the same in every layer of [l0, l1)
    // exchanged values carry their sequence number: {float bits, seq} per 64-bit word
    uint64_t *X;                // [2][8][n_embd]  per-XCD copies of x
    uint64_t *LG;               // [8][E]          per-XCD router logits
    uint64_t *H;                // [8][n_ff]       per-XCD h
    uint64_t *Y;                // [2][8][n_embd]  expert outputs by slot
    unsigned *tickets;          // [8] counters, 128 B apart
    int *err;
    unsigned *seq;              // [2] device-side sequence base and finished-workgroup count
    long long wait_ticks;       // bound of every cross-workgroup wait (100 MHz ticks)
    unsigned long long *trace;  // optional [layer][256 workgroups][kTracePhases] wall-clock stamps
};
constexpr int kTracePhases = 12;
constexpr size_t kPersistentMaxLds = 163840 - 1024;
size_t persistent_lds_bytes(const PersistentArgs &a);
// cooperative: launched with the runtime's co-residency guarantee (every
// workgroup resident at once); otherwise as a plain launch, which costs about
// 18 us less but relies on the device holding no other work (the kernels'
// waits are bounded, so a workgroup left waiting ends with the error flag).
hipError_t launch_persistent_decode(const PersistentArgs &a, hipStream_t s, bool cooperative = true);
bool persistent_shape_compiled(int gu_type, int n_embd, int d_type, int n_ff);

// One-launch decode with each selected expert's rows spread over all 256
// workgroups (decode_spread.hip): k routed experts plus an optional shared one,
// gate/up Q4_K and down Q6_K in every layer of the range.
struct SpreadArgs {
    const DecodeLayer *layers;  // device array, indexed by layer
    int l0, l1;
    float *x;                   // [n_embd] in/out
    float eps;
    int renorm;
    int n_embd, n_ff, E, k, shared;  // select the instantiation (shared: n_ff_shexp == n_ff)
    int d_type, sh_d_type;           // down types of the routed and shared experts (-1: any)
    // exchanged values carry their sequence number: {float bits, seq} per 64-bit word
    uint64_t *LG;               // [256][E]             router logits, one mailbox per workgroup
    uint64_t *H;                // [(k+shared)*n_ff]    h of the routed experts, then the shared one
    uint64_t *Y;                // [k+shared][n_embd]   expert outputs
    uint64_t *X;                // [8][n_embd]          x between layers, one copy per XCD
    unsigned *tickets;          // [8] counters, 128 B apart
    int *err;
    unsigned *seq;              // [2] device-side sequence base and finished-workgroup count
    long long wait_ticks;       // bound of every cross-workgroup wait (100 MHz ticks)
    unsigned long long *trace;  // optional [layer][256 workgroups][kTracePhases] wall-clock stamps
};
bool spread_shape_compiled(const SpreadArgs &a);
hipError_t launch_spread_decode(const SpreadArgs &a, hipStream_t s, bool cooperative = true);

// One launch for a whole layer of one token (layer.hip): router, gate/up and
// down workgroups in the order they start, each waiting only on workgroups
// that started before it, so no workgroup needs another to become resident.
struct FusedLayerArgs {
    const float *xin;          // [n_embd]: fx, or (rms) x whose rms_norm is fx
    int rms;
    float eps;
    const float *res;          // [n_embd] residual (may alias out)
    float *out;                // [n_embd]
    int32_t *sel;              // [k] selected experts (written)
    float *wsel;               // [k] their weights (written)
    const float *router;       // [E][n_embd]
    MatDesc gate, up, down;    // routed experts (stride per expert)
    MatDesc sh_gate, sh_up, sh_down;  // the shared expert (sh_gate.base == nullptr: none)
    const float *sh_gate_inp;  // [n_embd] f32 gate row of the shared expert
    uint64_t *sgt;             // [1] sigmoid(sh_gate_inp . fx) as a tagged word {value, launch epoch}
    int n_embd, E, k, renorm;
    uint64_t *lgw;             // [8][E] logits as tagged words {value, launch epoch}, one copy per XCD
    uint64_t *ht;              // [k (+1 shared)][n_ff] h as tagged words (each block in its XCD's L2)
    uint32_t *q8d;             // [units * n_ff / 256][kFusedQ8Words] Q8_K(h) blocks
    uint64_t *q8f;             // [8][128] block flags as tagged words, one line per XCD
    unsigned long long *ctr;   // kFusedCounterWords zeroed words: tickets, completion counts and flags
    int *err;                  // raised by a wait that runs out
    long long wait_ticks;
    unsigned long long *trace; // optional [workgroup][kFusedStamps] wall-clock stamps, by ticket order per XCD
};
constexpr int kFusedQ8Words = 76;  // a Q8_K block (256 int8, 16 int16 sums, d, padding) in 32-bit words
constexpr int kFusedStamps = 6;  // xcd * 65536 + role slot, start, 3 role events, end
constexpr int kFusedCounterWords = 16 * (8 + 16 + 8);
bool fused_layer_ok(const FusedLayerArgs &a);
int fused_layer_groups(const FusedLayerArgs &a);  // workgroups of one launch
hipError_t launch_fused_layer(const FusedLayerArgs &a, hipStream_t s);

// Per-layer launches for the instantiated shapes (layer.hip); the *_ok tests
// say whether they take the arguments, else the kernels above run.
bool layer_route_ok(const RouterArgs &a);
hipError_t launch_layer_route(const RouterArgs &a, hipStream_t s);
bool layer_ffn_ok(const GateUpArgs &g, const DownArgs &d);
hipError_t launch_layer_gateup(const GateUpArgs &g, hipStream_t s);
hipError_t launch_layer_down(const DownArgs &d, hipStream_t s);

size_t block_bytes(int type);

}  // namespace hoard
