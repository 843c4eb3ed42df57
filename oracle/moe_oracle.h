/*
 * moe_oracle.h -- CPU restatement of the reference's MoE expert stage.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load this library, and only as the checker or
 * as the timed CPU baseline.  The product (hoard_amd/) never links or calls it.
 *
 * The reference (bgallon-dev/hoard) keeps every piece of arithmetic of this
 * stage inside ggml (llama.cpp build b9660), which is neither vendored in the
 * reference tree nor present offline.  This file restates ggml-CPU's published
 * algorithm for exactly the ops the reference calls on the path:
 *
 *   router tail  src/run_moe_stream.cpp:353-356, 371-373  (src/run_qwen35.cpp:556-559, 578-580)
 *   graph B      src/run_moe_stream.cpp:431-438            (src/run_qwen35.cpp:649-666)
 *   combine      src/run_moe_stream.cpp:447                (src/run_qwen35.cpp:675-676)
 *   batched      src/run_specloop.cpp:116-140, src/run_m1.cpp:93-108
 *
 * and the ggml block formats the expert bytes are copied in verbatim
 * (src/run_moe_stream.cpp:177-183): block_q4_K (144 B), block_q6_K (210 B),
 * block_q5_K (176 B) and block_q3_K (110 B) -- the expert types of the
 * reference's model table (notes/FEASIBILITY.md:73-77) -- and the activation
 * format block_q8_K (ggml-cpu's vec_dot_type for all four).
 *
 * Pinning (see tests/test_oracle_*.py): block codecs by an independent
 * encoder written from the layout (decode(encode(v)) == v) and hand-built
 * known-answer blocks; Q8_K by closed-form special cases; the integer dot
 * products by an fp64 brute force over dequantised operands; router by an
 * fp64 softmax, brute-force top-k and the renorm clamp constant.  The fp32
 * summation order of ggml's SIMD kernels is not pinnable offline (ggml is
 * absent); the orders chosen here are stated at each function.
 */
#ifndef HOARD_MOE_ORACLE_H
#define HOARD_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_QK_K = 256 };
enum { ORC_TYPE_F32 = 0, ORC_TYPE_Q3_K = 11, ORC_TYPE_Q4_K = 12, ORC_TYPE_Q5_K = 13,
       ORC_TYPE_Q6_K = 14 };  /* ggml type ids */
enum { ORC_Q3_K_BYTES = 110, ORC_Q4_K_BYTES = 144, ORC_Q5_K_BYTES = 176, ORC_Q6_K_BYTES = 210,
       ORC_Q8_K_BYTES = 292 };

/* ggml block_q8_K: fp32 d, 256 int8 quants, 16 int16 group sums. */
typedef struct {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} orc_block_q8_K;

/* --- scalar helpers ----------------------------------------------------- */
float orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);
int orc_nearest_int(float f);

/* --- block codecs (one 256-element super-block) ------------------------- */
size_t orc_type_block_bytes(int type);
void orc_dequant_q4_K(const uint8_t *blk, float *y);
void orc_dequant_q6_K(const uint8_t *blk, float *y);
void orc_dequant_q3_K(const uint8_t *blk, float *y);
void orc_dequant_q5_K(const uint8_t *blk, float *y);
void orc_dequant_row(int type, const uint8_t *row, int n, float *y);
void orc_quantize_q8_K(const float *x, int n, orc_block_q8_K *y);
size_t orc_sizeof_q8_K(void);

/* --- dot products ------------------------------------------------------- */
float orc_vec_dot_f32(int n, const float *x, const float *y);
float orc_vec_dot_q4_K_q8_K(int n, const uint8_t *row, const orc_block_q8_K *y);
float orc_vec_dot_q6_K_q8_K(int n, const uint8_t *row, const orc_block_q8_K *y);
float orc_vec_dot_q3_K_q8_K(int n, const uint8_t *row, const orc_block_q8_K *y);
float orc_vec_dot_q5_K_q8_K(int n, const uint8_t *row, const orc_block_q8_K *y);
/* the row dot of any supported type */
float orc_vec_dot_q_q8_K(int type, int n, const uint8_t *row, const orc_block_q8_K *y);

/* out[r] = row_r(W) . x for a quantised W of nrows x ncols, x quantised to Q8_K first. */
void orc_mul_mat_q(int type, const uint8_t *w, int nrows, int ncols, const float *x, float *out);
/* same, with x already in Q8_K */
void orc_mul_mat_q8(int type, const uint8_t *w, int nrows, int ncols, const orc_block_q8_K *qx,
                    float *out);

/* --- elementwise -------------------------------------------------------- */
float orc_silu(float x);
float orc_sigmoid(float x);

/* --- router tail (a1-a5) ------------------------------------------------ */
/* logits, softmax over all experts, top-k (ties -> lower index), gather, renorm.
   probs_out may be NULL. */
void orc_route(int n_embd, int n_expert, int n_used, int renorm, const float *w_router,
               const float *fx, int32_t *sel, float *wsel, float *probs_out);

/* --- one layer ---------------------------------------------------------- */
typedef struct {
    int n_embd, n_expert, n_used, n_ff, n_ff_shexp, renorm;
    int gate_type, up_type, down_type;          /* routed experts */
    int sh_gate_type, sh_up_type, sh_down_type; /* shared expert */
} orc_layer_cfg;

typedef struct {
    const float *router;   /* [n_expert][n_embd] f32 */
    const uint8_t *gate;   /* [n_expert] x [n_ff rows of n_embd] */
    const uint8_t *up;
    const uint8_t *down;   /* [n_expert] x [n_embd rows of n_ff] */
    const uint8_t *sh_gate, *sh_up, *sh_down; /* shared expert, or NULL */
    const float *sh_gate_inp;                 /* [n_embd] f32, or NULL */
} orc_layer_weights;

size_t orc_expert_stride(int type, int rows, int cols);

/* One expert FFN: y[n_embd] = down . (silu(gate . x) * (up . x)), each GEMV
   with its activation quantised to Q8_K.  h_out (n_ff) may be NULL. */
void orc_expert_ffn(int n_embd, int n_ff, int gate_type, int up_type, int down_type,
                    const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                    const orc_block_q8_K *qx, float *y, float *h_out);

/* Full stage for one token: route, expert FFN, shared expert, combine.
   out[d] = (sum_j w_j*y_j[d]) + shex[d] + res[d]; sel/wsel returned. */
void orc_moe_layer(const orc_layer_cfg *cfg, const orc_layer_weights *w, const float *fx,
                   const float *res, float *out, int32_t *sel, float *wsel);

/* Same stage with the selection and weights given (the reference's graph B +
   host combine on externally supplied sel/wsel). */
void orc_moe_ffn_combine(const orc_layer_cfg *cfg, const orc_layer_weights *w, const float *fx,
                         const int32_t *sel, const float *wsel, const float *res, float *out);

/* Batched form (run_specloop / mul_mat_id): m tokens, row-major [m][n_embd]. */
void orc_moe_layer_batched(const orc_layer_cfg *cfg, const orc_layer_weights *w, int m,
                           const float *fx, const float *res, float *out, int32_t *sel,
                           float *wsel);

/* RMS norm used to chain stacked layers: y = x / sqrt(mean(x^2) + eps). */
void orc_rms_norm(int n, const float *x, float eps, float *y);

/* OpenMP thread count actually used by the parallel entry points (1 if built without). */
int orc_num_threads(void);
void orc_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
