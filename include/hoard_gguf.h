/* hoard_gguf.h -- the MoE expert stage's weights straight from a GGUF file.
 *
 * Replaces the hparams and tensor discovery of the reference's load_model
 * (src/run_moe_stream.cpp:119-186; the shared expert and the bf16 -> f32
 * upconversion of src/run_qwen35.cpp:187-253): the file is memory-mapped, its
 * metadata fills a hoard_moe_cfg, and each layer's router, routed experts
 * (expert e at e * stride, stride = tensor bytes / n_expert, :177-179) and
 * shared expert become a hoard_layer_weights whose pointers are into the
 * mapping, ready for hoard_moe_set_layer_weights.  Routers and the shared
 * gate row stored as f16 or bf16 are converted to f32 into buffers the handle
 * owns.  Host only; no device calls.
 *
 * Every call returns HOARD_OK or a negative HOARD_ERR_* (hoard_moe.h) with
 * hoard_last_error() set; nothing aborts.
 */
#ifndef HOARD_GGUF_H
#define HOARD_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "hoard_moe.h"
#include "hoard_store.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hoard_gguf hoard_gguf;

/* Map and parse a GGUF file (versions 2 and 3): header, metadata, tensor
   infos.  gguf_init_from_file + the reads of src/run_moe_stream.cpp:122-145. */
int hoard_gguf_open(const char *path, hoard_gguf **out);
void hoard_gguf_close(hoard_gguf *g);

/* general.architecture ("" when absent); the pointer lives as long as g. */
const char *hoard_gguf_arch(const hoard_gguf *g);

/* The stage's shape from `{arch}.block_count`, `embedding_length`,
   `expert_feed_forward_length` (else `feed_forward_length`), `expert_count`,
   `expert_used_count` and `expert_shared_feed_forward_length`; renorm = 1
   unless the architecture is "olmoe" (:150).  pool_k = 0, max_tokens = 1. */
int hoard_gguf_moe_cfg(const hoard_gguf *g, hoard_moe_cfg *cfg);

/* `{arch}.attention.layer_norm_rms_epsilon` (default 1e-5, :138). */
float hoard_gguf_rms_eps(const hoard_gguf *g);

/* Layer `layer`'s blk.N.ffn_gate_inp, ffn_{gate,up,down}_exps and, when the
   file has them, ffn_{gate,up,down}_shexp and ffn_gate_inp_shexp, checked
   against the shape hoard_gguf_moe_cfg reports. */
int hoard_gguf_layer_weights(hoard_gguf *g, int layer, hoard_layer_weights *w);

/* A tensor by name: ggml type, up to 4 dims (ne[0] fastest), bytes and a
   pointer into the mapping.  HOARD_ERR_INVALID when absent. */
int hoard_gguf_tensor(const hoard_gguf *g, const char *name, int32_t *type, int64_t ne[4], size_t *nbytes,
                      const void **data);

/* Where each layer's gate, up and down expert tensors lie in the file, for
   hoard_store_open: layers[0..n_layer) with n_layer from hoard_gguf_moe_cfg
   (the offsets and strides load_model records, src/run_moe_stream.cpp:171-179). */
int hoard_gguf_store_layers(const hoard_gguf *g, hoard_store_layer *layers, int n_layer);

#ifdef __cplusplus
}
#endif

#endif /* HOARD_GGUF_H */
