/*
 * hoard_synth.h -- deterministic synthetic MoE layers (host only, no GPU).
 *
 * The reference runs on real GGUF weights; the measured workloads here are
 * synthetic layers of the same shapes.  Every byte is a pure function of
 * (config, seed, layer, tensor, expert, index) through a counter-based
 * splitmix64 hash, so any process -- bench, tests, oracle checks -- can
 * regenerate any expert on its own, in any order, on any number of threads.
 *
 *   Q4_K block: 12 scale bytes and 128 nibble bytes uniform random (every byte
 *               pattern decodes to valid 6-bit scales/mins), d and dmin =
 *               fp16(|N(0, dstd)|).
 *   Q6_K block: ql, qh and the 16 int8 scales uniform random,
 *               d = fp16(|N(0, dstd)|).
 *   f32 tensors: N(0, std) by Box-Muller over the same hash.
 */
#ifndef HOARD_SYNTH_H
#define HOARD_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* tensor ids used in key derivation */
#define HOARD_SYNTH_ROUTER 0
#define HOARD_SYNTH_GATE 1
#define HOARD_SYNTH_UP 2
#define HOARD_SYNTH_DOWN 3
#define HOARD_SYNTH_SH_GATE 4
#define HOARD_SYNTH_SH_UP 5
#define HOARD_SYNTH_SH_DOWN 6
#define HOARD_SYNTH_SH_GATE_INP 7
#define HOARD_SYNTH_HIDDEN 8

uint64_t hoard_synth_key(uint32_t config, uint32_t seed, uint32_t layer, uint32_t tensor,
                         uint32_t expert);

/* nblocks super-blocks of ggml type `type` (Q4_K or Q6_K) into dst. */
int hoard_synth_fill_blocks(int type, uint64_t key, void *dst, size_t nblocks, float dstd);

/* n floats ~ N(0, std). */
void hoard_synth_fill_normal(uint64_t key, float *dst, size_t n, float std);

/* Every expert of one [n_expert] tensor: expert e is filled with
   key hoard_synth_key(config, seed, layer, tensor, e) and lands at
   dst + e*stride, stride = rows * (cols/256) * block bytes.  Multi-threaded. */
int hoard_synth_fill_experts(int type, uint32_t config, uint32_t seed, uint32_t layer,
                             uint32_t tensor, int n_expert, int rows, int cols, void *dst,
                             float dstd);

/* bytes of one expert matrix of `rows` rows of `cols` columns. */
size_t hoard_synth_expert_bytes(int type, int rows, int cols);

#ifdef __cplusplus
}
#endif
#endif
