/*
 * hoard_moe.h -- C ABI of the MI355X MoE expert stage.
 *
 * Drop-in for the per-layer expert stage of bgallon-dev/hoard: the router tail
 * of "graph A", the VRAM expert-slot pool, "graph B" (expert FFN over the
 * selected experts) and the host weighted combine.  Every call is extern "C",
 * returns 0 on success or a negative HOARD_ERR_* code (hoard_last_error()
 * then describes it), throws nothing across the boundary and takes the
 * hipStream_t to run on as a void*.  A handle is not thread-safe: use one
 * handle per host thread, as the reference keeps all ggml/device calls on one
 * thread (src/run_moe_stream.cpp:415).
 *
 * Weights cross the boundary as raw GGUF-layout bytes (expert e of a
 * [n_expert] tensor at e*stride, src/run_moe_stream.cpp:177-179); activations
 * are fp32 device pointers.
 */
#ifndef HOARD_MOE_H
#define HOARD_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define HOARD_OK 0
#define HOARD_ERR_INVALID (-1)     /* bad argument or shape */
#define HOARD_ERR_UNSUPPORTED (-2) /* valid but not implemented (e.g. quant type) */
#define HOARD_ERR_HIP (-3)         /* HIP runtime error */
#define HOARD_ERR_OOM (-4)         /* device or pinned host allocation failed */
#define HOARD_ERR_STATE (-5)       /* call not valid in the handle's state */
#define HOARD_ERR_IO (-6)          /* reading the model file failed */

/* ggml type ids accepted for expert tensors (ggml.h enum ggml_type). */
#define HOARD_TYPE_F32 0
#define HOARD_TYPE_Q3_K 11
#define HOARD_TYPE_Q4_K 12
#define HOARD_TYPE_Q5_K 13
#define HOARD_TYPE_Q6_K 14

typedef struct hoard_moe hoard_moe;

/* Stage shape.  Replaces the hparams the reference reads from GGUF in
   load_model (src/run_moe_stream.cpp:128-150, src/run_qwen35.cpp:161-172)
   plus the pool size K (src/run_moe_stream.cpp:232). */
typedef struct hoard_moe_cfg {
    int32_t n_embd;     /* hidden size, multiple of 256 */
    int32_t n_expert;   /* routed experts per layer, <= 1024 */
    int32_t n_used;     /* experts per token (top-k), 1..16 */
    int32_t n_ff;       /* routed expert intermediate, multiple of 256 */
    int32_t n_ff_shexp; /* shared expert intermediate (multiple of 256), 0 = none */
    int32_t n_layer;
    int32_t renorm;     /* norm_topk_prob: 1 renormalises the top-k weights (wnorm, :150) */
    int32_t pool_k;     /* 0: every expert resident in HBM; >0: K HBM slots per layer
                           filled from pinned host memory (the reference's Slots, :193-203) */
    int32_t max_tokens; /* largest M accepted by hoard_moe_forward_batched (>= 1) */
} hoard_moe_cfg;

/* One layer's weights, host pointers to GGUF-layout bytes.  Types are per layer
   (mixed quantisation across layers, src/run_moe_stream.cpp:177-179). */
typedef struct hoard_layer_weights {
    const float *router;  /* ffn_gate_inp [n_expert][n_embd] f32 */
    int32_t gate_type, up_type, down_type;
    const void *gate;     /* ffn_gate_exps: n_expert x (n_ff rows of n_embd) */
    const void *up;       /* ffn_up_exps:   n_expert x (n_ff rows of n_embd) */
    const void *down;     /* ffn_down_exps: n_expert x (n_embd rows of n_ff) */
    int32_t sh_gate_type, sh_up_type, sh_down_type;
    const void *sh_gate;  /* ffn_gate_shexp (n_ff_shexp rows of n_embd), or NULL */
    const void *sh_up;    /* ffn_up_shexp */
    const void *sh_down;  /* ffn_down_shexp (n_embd rows of n_ff_shexp) */
    const float *sh_gate_inp; /* ffn_gate_inp_shexp [n_embd] f32 */
} hoard_layer_weights;

typedef struct hoard_moe_stats {
    uint64_t reqs;       /* expert requests seen by the pool (reference `reqs`, :264) */
    uint64_t hits;       /* requests served from an HBM slot (`vram_hit`) */
    uint64_t misses;     /* requests that needed an upload (`copies`) */
    uint64_t bytes_h2d;  /* bytes uploaded host -> HBM */
    uint64_t tokens;     /* tokens routed through hoard_moe_forward_batched */
    uint64_t expert_hist[1024]; /* per-expert token count of the last batched call */
    int32_t last_unique; /* unique experts in the last batched call */
} hoard_moe_stats;

/* Text of the last error on this host thread ("" if none). */
const char *hoard_last_error(void);

/* Creates a handle and allocates the device state for cfg: resident expert
   tensors (pool_k == 0) or K slots per layer plus pinned host masters
   (pool_k > 0), the router weights and per-call scratch.  Replaces the
   Slots / KV / weight-buffer set-up of src/run_moe_stream.cpp:237-254. */
int hoard_moe_create(const hoard_moe_cfg *cfg, hoard_moe **out);
void hoard_moe_destroy(hoard_moe *h);

/* Copies one layer's weights in (synchronously).  Replaces load_model's
   upload of ffn_gate_inp and the expert byte ranges recorded at
   src/run_moe_stream.cpp:171-184 (and ggml_backend_tensor_set of the shared
   expert tensors, src/run_qwen35.cpp:219, 250-253). */
int hoard_moe_set_layer_weights(hoard_moe *h, int layer, const hoard_layer_weights *w);

/* Router tail for one token: logits = ffn_gate_inp . fx (f32), softmax over
   all experts, top-k (descending, ties -> lower index), gather, optional
   renorm with the 6.103515625e-5 clamp.  Replaces ggml_mul_mat, ggml_soft_max,
   ggml_top_k, ggml_get_rows at src/run_moe_stream.cpp:353-356 and the host
   renorm at :371-373.  sel_dev: int32[n_used], w_dev: f32[n_used]. */
int hoard_moe_route(hoard_moe *h, int layer, const float *fx_dev, int32_t *sel_dev, float *w_dev,
                    void *stream);

/* Graph B plus the combine for one token: for j in 0..n_used-1 the expert
   FFN y_j = down(silu(gate x) * up x) of expert ids_dev[j] (an expert id when
   pool_k == 0, a slot index from hoard_moe_pool_ensure when pool_k > 0), then
   out[d] = (sum_j w_j*y_j[d]) + shex[d] + res[d], shex being the
   sigmoid-gated shared expert when n_ff_shexp > 0.  Replaces graph B at
   src/run_moe_stream.cpp:424-445 (src/run_qwen35.cpp:640-666) and the host
   combine at :447 (:675-676).  out_dev may alias res_dev. */
int hoard_moe_ffn_combine(hoard_moe *h, int layer, const float *fx_dev, const int32_t *ids_dev,
                          const float *w_dev, const float *res_dev, float *out_dev, void *stream);

/* Route + FFN + combine for one token with nothing leaving the device when
   pool_k == 0 (with a slot pool the selection is read back to ensure the
   slots, see hoard_moe_pool_ensure).  sel_dev / w_dev receive the selection
   when non-NULL. */
int hoard_moe_layer(hoard_moe *h, int layer, const float *fx_dev, const float *res_dev,
                    float *out_dev, int32_t *sel_dev, float *w_dev, void *stream);

/* Stacked decode over layers [layer_begin, layer_end) for one token, in place
   on x_dev: per layer fx = rms_norm(x, eps), x = layer(fx, x).
   The reference round-trips to the host twice per layer
   (src/run_moe_stream.cpp:362-370, 441-447); here the chain stays on device. */
int hoard_moe_decode(hoard_moe *h, int layer_begin, int layer_end, float *x_dev, float eps,
                     void *stream);

/* Batched expert stage for M tokens (1 <= M <= min(max_tokens, 512)), every
   token routed independently: the counterpart of ggml_mul_mat_id over the
   experts with per-token ids and the weighted sum over them
   (src/run_specloop.cpp:126-139, src/run_m1.cpp:97-108).  The (token, slot)
   pairs are grouped by expert so each selected expert's weights are read once
   per call (per 64 pairs above 32 tokens, where the pairs are sorted by
   expert into 64-pair units), and the expert products run on per-token int8
   dots or int8 MFMA; each token's result is the single-token
   hoard_moe_layer's bit for bit.  M > 512 returns HOARD_ERR_INVALID.  fx_dev, res_dev, out_dev:
   [M][n_embd], 16-byte aligned (out may alias res); sel_dev / w_dev ([M][n_used]) receive the
   routing when non-NULL.  The call's per-expert token histogram and unique
   expert count are reported by hoard_moe_get_stats.  Needs pool_k == 0.  A
   shared expert (n_ff_shexp > 0) must have the routed experts' n_ff and types
   (or a Q6_K down beside Q5_K routed down rows, n_ff 512) and n_used <= 15: it
   runs as one more expert taken by every token, gated by
   sigmoid(ffn_gate_inp_shexp . fx) as in hoard_moe_layer.  Expert types: Q4_K
   or Q3_K gate/up (both the same) with Q4_K, Q5_K or Q6_K down rows, n_ff of
   512, 768 (not with Q5_K) or 1024, n_embd 2048. */
int hoard_moe_forward_batched(hoard_moe *h, int layer, int M, const float *fx_dev, const float *res_dev,
                              float *out_dev, int32_t *sel_dev, float *w_dev, void *stream);

/* hoard_moe_forward_batched with nothing allocated by the call, for callers
   that cannot allocate device memory (code under HIP graph capture, tight
   serving loops, harnesses that forbid hipMalloc).  No counterpart in the
   reference.  The per-call scratch lives in one fixed device array per GPU,
   32 MiB, looked up when a handle is created and held until the process ends;
   1 <= M <= min(max_tokens, 16), and a shape whose scratch for M tokens exceeds
   the array is refused with HOARD_ERR_INVALID (the Qwen3-30B shape needs about
   17 MiB at M = 16, the Qwen3-Next shape about 16.5 MiB).  Results are hoard_moe_forward_batched's bit for bit.  Every
   call on a GPU shares that GPU's array: calls that overlap on one GPU (any
   handle, any stream) race.  The call's histogram and unique-expert count are
   copied into the handle's own memory on `stream` (allocated by
   hoard_moe_create), so hoard_moe_get_stats reports them whatever later calls
   on the GPU leave in the array. */
int hoard_moe_forward_batched_noalloc(hoard_moe *h, int layer, int M, const float *fx_dev, const float *res_dev,
                                      float *out_dev, int32_t *sel_dev, float *w_dev, void *stream);

/* The batched expert products and combine for the caller's selection, the
   counterpart of the verify step's mul_mat_id over the slot pool with the host's
   ids and weights and the sum over views (src/run_specloop.cpp:116-139):
   ids_dev[M][n_used] are expert ids, or slot indices from
   hoard_moe_pool_ensure_batched when pool_k > 0; w_dev[M][n_used] are used as
   given (no renormalisation).  out[t] = res[t] + sum_j w[t][j] y(ids[t][j]), j
   ascending.  A token may repeat an id (the verify loop pads with a repeated id
   of weight 0); a token with an id outside the pool or expert set gets a NaN
   row.  A shared expert adds its gated output as in hoard_moe_ffn_combine
   (with hoard_moe_forward_batched's limits on it).  1 <= M <= min(max_tokens,
   512).  Each token's result equals hoard_moe_ffn_combine's for that token. */
int hoard_moe_ffn_combine_batched(hoard_moe *h, int layer, int M, const float *fx_dev, const int32_t *ids_dev,
                                  const float *w_dev, const float *res_dev, float *out_dev, void *stream);

/* Slot-pool step for a batch (pool_k > 0): the n ids sel_host[] of up to
   min(max_tokens, 512) tokens (token-major, n_used per token, so
   1 <= n <= min(max_tokens, 512) * n_used: the batch hoard_moe_ffn_combine_batched
   takes), taken one after the other as the verify loop's ensure does
   (src/run_specloop.cpp:59-67; no hits-first pass), uploads as
   hoard_moe_pool_ensure.  The distinct experts must fit the K slots.
   slot_host / slot_dev (either optional) receive n slots. */
int hoard_moe_pool_ensure_batched(hoard_moe *h, int layer, int n, const int32_t *sel_host, int32_t *slot_host,
                                  int32_t *slot_dev, void *stream, void *copy_stream);

/* Per-kernel timing, the device counterpart of the reference's phase timers
   (tA/tFetch/tB, src/run_moe_stream.cpp:291,311,377,422,448): while enabled,
   every kernel launch is bracketed by a pair of hipEvents on its stream.
   hoard_moe_profile_read synchronises on the last event, returns the launch
   counts and summed durations per kernel kind, and clears them. */
#define HOARD_KERNEL_ROUTER 0
#define HOARD_KERNEL_GATEUP 1
#define HOARD_KERNEL_DOWN 2
#define HOARD_KERNEL_DECODE 3
#define HOARD_KERNEL_BATCHED 4 /* the batched path's grouping, MFMA and combine launches together */
#define HOARD_KERNEL_LAYER 5   /* the one-launch layer (router, gate/up, down and combine) */
#define HOARD_KERNEL_KINDS 8
typedef struct hoard_moe_kernel_times {
    uint64_t launches[HOARD_KERNEL_KINDS];
    double total_ms[HOARD_KERNEL_KINDS];
} hoard_moe_kernel_times;

int hoard_moe_profile(hoard_moe *h, int enable);

/* Phase trace of the one-launch decode, the counterpart of the reference's
   DECODE BREAKDOWN (src/run_moe_stream.cpp:551-554): while enabled, every
   workgroup stamps the 100 MHz device wall clock at 12 phase boundaries of every
   layer.  hoard_moe_phase_trace_read synchronises and copies the stamps of the
   last traced call as [layer][256 workgroups (xcd*32 + rank)][12]. */
int hoard_moe_phase_trace(hoard_moe *h, int enable);
int hoard_moe_phase_trace_read(hoard_moe *h, uint64_t *out, size_t max_words, int *n_layers);
/* The same tracing for the one-launch layer (HOARD_OPT_LAYER_FUSED): the stamps
   of the last traced launch, 6 words per workgroup in XCD-major ticket order:
   xcd * 65536 + role slot, then the 100 MHz wall clock at its start, three
   role events and its end.  Role slots count router, gate/up and down
   workgroups in that order; the events are the logits stored (router, all
   three), the selection formed / rows landed / h stored (gate/up, whose end
   is the block's Q8_K(h) published for the last workgroup of each 256-row
   block), and the selection formed / every Q8_K(h) block read and rows
   landed (twice) (down). */
int hoard_moe_fused_trace_read(hoard_moe *h, uint64_t *out, size_t max_words, size_t *n_words);

/* Options.  HOARD_OPT_PERSISTENT_DECODE selects how hoard_moe_decode runs:
   0 = one launch per kernel per layer, 1 = one cooperative launch per run of
   layers with the same quant types when the shape and device admit it and the
   run holds at least 3 layers (default; shorter runs are faster layer by
   layer, and a range whose types change is split into such runs), 2 = require
   one launch for the whole range.
   HOARD_OPT_PERSISTENT_AVAILABLE (read-only) reports whether they admit it. */
#define HOARD_OPT_PERSISTENT_DECODE 1
#define HOARD_OPT_PERSISTENT_AVAILABLE 2
/* HOARD_OPT_POOL_NAIVE: 1 = the reference's "naive" mode (every selected
   expert is uploaded into slot j on every call, :417), 0 = LRU (default). */
#define HOARD_OPT_POOL_NAIVE 3
/* HOARD_OPT_DECODE_KERNEL picks the one-launch decode kernel: 0 = auto (the
   expert-per-XCD kernel where it applies, else the rows-spread one), 1 = the
   expert-per-XCD kernel (k = 8 routed experts of E <= 128, one per XCD, no
   shared expert), 2 = the rows-spread kernel (each selected expert's rows, and
   a shared expert's, spread over all 256 CUs; Qwen3-Next-shaped layers).
   HOARD_OPT_DECODE_KERNELS_AVAILABLE (read-only) is a mask: bit 0 the first,
   bit 1 the second. */
#define HOARD_OPT_DECODE_KERNEL 4
#define HOARD_OPT_DECODE_KERNELS_AVAILABLE 5
/* HOARD_OPT_LAYER_KERNELS: 1 (default) = the per-layer entry points (route,
   ffn_combine, layer, and decode when it runs layer by layer) use kernels
   compiled for the shape (n_embd 2048, Q4_K gate/up, Q6_K or Q4_K down, 16-byte
   aligned tensors) where it matches; 0 = always the shape-generic kernels.
   Both give the same bits. */
#define HOARD_OPT_LAYER_KERNELS 6
/* HOARD_OPT_DECODE_LAUNCH: how the one-launch decode is launched.  0 (default)
   = cooperatively: the runtime guarantees every workgroup is resident at once.
   1 = as a plain launch, about 18 us less per call (Qwen3-30B shape: 13.9 ->
   13.5 us per layer), for callers that own the device: it relies on no other
   work holding compute units while it runs.  Its cross-workgroup waits are
   bounded either way: a workgroup left waiting sets the error flag, the
   output is NaN and hoard_moe_sync_check reports HOARD_ERR_HIP.
   The plain launch can be captured into a HIP graph: its sequence tags live
   in device memory and advance at the end of every launch, replays included.
   Under capture with the cooperative launch, automatic mode records the
   per-layer kernels instead and forced mode returns HOARD_ERR_UNSUPPORTED. */
#define HOARD_OPT_DECODE_LAUNCH 7
/* HOARD_OPT_WAIT_LIMIT_US: bound of every cross-workgroup wait of the
   one-launch decode, in microseconds (default 200000).  A wait that runs past
   it gives up as described above; 0 makes the first wait that is not met at
   once give up, which forces that failure path from the host. */
#define HOARD_OPT_WAIT_LIMIT_US 8
/* HOARD_OPT_FAIL_UPLOAD: test hook of the slot pool.  n > 0 makes the n-th
   slot upload from now fail before it is issued, as a refused hipMemcpyAsync
   would: the pool call returns HOARD_ERR_HIP and the layer's slot residency is
   forgotten (its next call uploads every selected expert again).  0 = off. */
#define HOARD_OPT_FAIL_UPLOAD 9
/* HOARD_OPT_LAYER_FUSED: 1 (default) = hoard_moe_layer, and hoard_moe_decode
   when it runs layer by layer, take one launch per layer where the shape
   admits it (every expert resident, no shared expert, the shapes of
   HOARD_OPT_LAYER_KERNELS with Q4_K gate/up): router, gate/up and down
   workgroups run in the order they start, each waiting only on workgroups that
   started before it, so the launch needs no co-residency and can be captured.
   Its waits are bounded as HOARD_OPT_WAIT_LIMIT_US says, reported by
   hoard_moe_sync_check.  0 = the three launches per layer.  Both give the same
   bits. */
#define HOARD_OPT_LAYER_FUSED 10
int hoard_moe_set_option(hoard_moe *h, int option, int value);
int hoard_moe_get_option(hoard_moe *h, int option, int *value);

/* Expert slot pool (pool_k > 0), the reference's Slots
   (src/run_moe_stream.cpp:193-203): K HBM slots per layer, filled from the
   full expert set kept in pinned host memory.

   hoard_moe_pool_ensure makes the n_used experts sel_host[] of `layer`
   resident, as the fetch step at :379-420 does: hits are classified first
   and move to the front of the layer's LRU list (:385-387), then each miss
   takes the least recently used slot, evicts its expert and is uploaded with
   hipMemcpyAsync (:416-419; to_vram, :279-284), the misses dealt round-robin
   to copy_stream and two upload streams of the handle's own.  Each upload
   stream first waits for the last FFN that read this layer's slots, and
   `stream` is made to wait for the uploads, so an FFN launched on `stream` afterwards reads
   them; with copy_stream distinct from `stream` the uploads of layer l+1 overlap
   the FFN of layer l.  The slots go to slot_host and/or slot_dev (int32[n_used]),
   to be passed as ids to hoard_moe_ffn_combine.  hoard_moe_layer and
   hoard_moe_decode on a pool handle read the device-routed selection back
   (a synchronisation, as the reference's D2H at :367) and call the same step. */
int hoard_moe_pool_ensure(hoard_moe *h, int layer, const int32_t *sel_host, int32_t *slot_host,
                          int32_t *slot_dev, void *stream, void *copy_stream);

/* Counters since creation or the last reset: pool requests, hits, misses and
   bytes uploaded (the reference's reqs / vram_hit / copies, :264), and the
   batched path's token histogram. */
int hoard_moe_get_stats(hoard_moe *h, hoard_moe_stats *out);
int hoard_moe_reset_stats(hoard_moe *h);

/* Host replay of the slot pool's LRU bookkeeping, with no device: the same
   placement decisions hoard_moe_pool_ensure makes, for trace studies (the
   reference's simulators, bench/profiler.py:65-91).  naive = 1 reproduces the
   reference's "naive" mode (:417): request j goes to slot j, always a miss;
   naive = 2 takes the ids one after the other as hoard_moe_pool_ensure_batched
   does (src/run_specloop.cpp:59-67), any number of them per call.
   slot_out[n] receives the slots, miss_out[n] (optional) 1 per miss. */
typedef struct hoard_slot_lru hoard_slot_lru;
int hoard_slot_lru_create(int n_layer, int n_expert, int k, int naive, hoard_slot_lru **out);
int hoard_slot_lru_access(hoard_slot_lru *p, int layer, const int32_t *sel, int n, int32_t *slot_out,
                          uint8_t *miss_out);
void hoard_slot_lru_destroy(hoard_slot_lru *p);

/* Synchronises the device and reports a cross-workgroup wait that timed out
   in the one-launch decode (its output rows are then NaN). */
int hoard_moe_sync_check(hoard_moe *h);
int hoard_moe_profile_read(hoard_moe *h, hoard_moe_kernel_times *out);

#ifdef __cplusplus
}
#endif
#endif
