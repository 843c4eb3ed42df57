/*
 * moe_oracle.c -- CPU restatement of the reference's MoE expert stage.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the timed CPU baseline); the
 * product never links it.  Every function states the reference call site it
 * follows and, for ggml internals (absent offline, llama.cpp b9660), the
 * published ggml semantics it restates.  Built with -ffp-contract=off so each
 * fp32 operation below rounds exactly where it is written.
 *
 * Parity status per function (pins live in tests/test_oracle_*.py):
 *   orc_fp16_to_fp32 / orc_fp32_to_fp16  pinned: exhaustive / numpy float16
 *   orc_dequant_q{3,4,5,6}_K             pinned: independent encoder + known-answer blocks
 *   orc_quantize_q8_K                    pinned: closed-form special cases + bounds
 *   orc_vec_dot_q{3,4,5,6}_K_q8_K        pinned: fp64 brute force over dequantised operands
 *   orc_vec_dot_f32                      pinned: fp64 within bound (the value only)
 *   orc_route                            pinned: fp64 softmax, brute-force top-k, clamp
 *   orc_expert_ffn / orc_moe_*           pinned: fp64 composition of the pinned parts
 *   fp32 summation ORDER of ggml's SIMD kernels: parity unpinned (ggml absent);
 *   the order used is stated at each function.  The router dot's order in
 *   particular is a choice, not a pin: it is the tree of ggml-cpu's AVX2 build;
 *   the AVX-512 build of the same ggml (which an AVX-512 host loads) steps 64
 *   elements as 4 vectors of 16 lanes and reduces another tree, so its logits
 *   may differ in the last bits from these.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32 (ggml stores d/dmin as IEEE binary16; F16C converts exactly,
   fp32 -> fp16 rounds to nearest even).                                     */
/* ------------------------------------------------------------------------ */
float orc_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    float f;
    if (ex == 0) {
        /* zero or subnormal: man * 2^-24, exact in fp32 */
        f = (float)man * 5.9604644775390625e-08f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);      /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);     /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                       /* below 2^-14 */
        float v = fabsf(f) * 16777216.0f;                         /* exact scaling by 2^24 */
        return (uint16_t)(sign | (uint32_t)rintf(v));             /* RNE; 1024 == min normal */
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* ggml's nearest_int: add 1.5*2^23 so the fp32 adder rounds to nearest even,
   then read the integer from the mantissa (valid for |f| <= 4194303). */
int orc_nearest_int(float f) {
    float v = f + 12582912.0f;
    int32_t i;
    memcpy(&i, &v, 4);
    return (i & 0x007fffff) - 0x00400000;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

size_t orc_type_block_bytes(int type) {
    switch (type) {
    case ORC_TYPE_Q3_K: return ORC_Q3_K_BYTES;
    case ORC_TYPE_Q4_K: return ORC_Q4_K_BYTES;
    case ORC_TYPE_Q5_K: return ORC_Q5_K_BYTES;
    case ORC_TYPE_Q6_K: return ORC_Q6_K_BYTES;
    default: return 0;
    }
}

size_t orc_sizeof_q8_K(void) { return sizeof(orc_block_q8_K); }

size_t orc_expert_stride(int type, int rows, int cols) {
    return (size_t)rows * (size_t)(cols / ORC_QK_K) * orc_type_block_bytes(type);
}

/* ------------------------------------------------------------------------ */
/* block_q4_K: [0..1] d fp16, [2..3] dmin fp16, [4..15] 8 six-bit scales and
   8 six-bit mins packed in 12 bytes, [16..143] 256 nibbles.  Sub-block s of
   32 elements: chunk c = s/2 covers qs[32c..32c+31]; even s takes the low
   nibbles, odd s the high nibbles.  value = d*sc[s]*q - dmin*m[s].          */
/* ------------------------------------------------------------------------ */
static void q4k_scale_min(int s, const uint8_t *sb, int *sc, int *mn) {
    /* sub-blocks 0..3: low 6 bits of bytes 0..3 (scale) and 4..7 (min).
       sub-blocks 4..7: low/high nibble of bytes 8..11 give the low 4 bits
       of scale/min, the top 2 bits of bytes 0..3 / 4..7 give bits 4..5.   */
    if (s < 4) {
        *sc = sb[s] & 63;
        *mn = sb[s + 4] & 63;
    } else {
        *sc = (sb[s + 4] & 0x0f) | ((sb[s - 4] >> 6) << 4);
        *mn = (sb[s + 4] >> 4) | ((sb[s] >> 6) << 4);
    }
}

/* ggml dequantize_row_q4_K, one block. */
void orc_dequant_q4_K(const uint8_t *blk, float *y) {
    const float d = orc_fp16_to_fp32(rd16(blk));
    const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
    const uint8_t *sb = blk + 4;
    const uint8_t *qs = blk + 16;
    for (int c = 0; c < 4; ++c) {
        int sc0, m0, sc1, m1;
        q4k_scale_min(2 * c, sb, &sc0, &m0);
        q4k_scale_min(2 * c + 1, sb, &sc1, &m1);
        const float d0 = d * (float)sc0, mm0 = dmin * (float)m0;
        const float d1 = d * (float)sc1, mm1 = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) {
            y[64 * c + l] = d0 * (float)(qs[32 * c + l] & 0x0f) - mm0;
            y[64 * c + 32 + l] = d1 * (float)(qs[32 * c + l] >> 4) - mm1;
        }
    }
}

/* block_q6_K: [0..127] ql (low 4 bits), [128..191] qh (high 2 bits),
   [192..207] 16 int8 scales (one per 16 elements), [208..209] d fp16.
   Half n (128 elements) uses ql[64n..], qh[32n..], scales[8n..]; element
   128n+32*i+l (i=0..3, l=0..31) takes the low (i even) or high (i odd)
   nibble of ql[64n + 32*(i&1) + l] and bits 2i..2i+1 of qh[32n + l].
   value = d * scale[element/16] * (q - 32).                                 */
static void q6k_unpack(const uint8_t *blk, int *q /* 256 values 0..63 */) {
    const uint8_t *ql = blk, *qh = blk + 128;
    for (int n = 0; n < 2; ++n) {
        for (int l = 0; l < 32; ++l) {
            const int h = qh[32 * n + l];
            q[128 * n + l] = (ql[64 * n + l] & 0x0f) | (((h >> 0) & 3) << 4);
            q[128 * n + 32 + l] = (ql[64 * n + 32 + l] & 0x0f) | (((h >> 2) & 3) << 4);
            q[128 * n + 64 + l] = (ql[64 * n + l] >> 4) | (((h >> 4) & 3) << 4);
            q[128 * n + 96 + l] = (ql[64 * n + 32 + l] >> 4) | (((h >> 6) & 3) << 4);
        }
    }
}

/* ggml dequantize_row_q6_K, one block: y = d * sc * (q - 32). */
void orc_dequant_q6_K(const uint8_t *blk, float *y) {
    const float d = orc_fp16_to_fp32(rd16(blk + 208));
    const int8_t *sc = (const int8_t *)(blk + 192);
    int q[256];
    q6k_unpack(blk, q);
    for (int k = 0; k < 256; ++k) y[k] = d * (float)sc[k / 16] * (float)(q[k] - 32);
}

/* block_q5_K: [0..1] d fp16, [2..3] dmin fp16, [4..15] scales/mins packed as
   in block_q4_K, [16..47] qh (fifth bits), [48..175] qs (low nibbles).
   Chunk c (elements 64c..64c+63): element 64c+l takes the low nibble of
   qs[32c+l] and bit 2c of qh[l]; element 64c+32+l the high nibble and bit
   2c+1.  value = d*sc[s]*q - dmin*m[s], q in 0..31, s = element/32.         */
static void q5k_unpack(const uint8_t *blk, int *q /* 256 values 0..31 */) {
    const uint8_t *qh = blk + 16, *qs = blk + 48;
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l) {
            q[64 * c + l] = (qs[32 * c + l] & 0x0f) | (((qh[l] >> (2 * c)) & 1) << 4);
            q[64 * c + 32 + l] = (qs[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4);
        }
}

/* ggml dequantize_row_q5_K, one block. */
void orc_dequant_q5_K(const uint8_t *blk, float *y) {
    const float d = orc_fp16_to_fp32(rd16(blk));
    const float dmin = orc_fp16_to_fp32(rd16(blk + 2));
    int q[256];
    q5k_unpack(blk, q);
    for (int s = 0; s < 8; ++s) {
        int sc, m;
        q4k_scale_min(s, blk + 4, &sc, &m);
        const float ds = d * (float)sc, ms = dmin * (float)m;
        for (int l = 0; l < 32; ++l) y[32 * s + l] = ds * (float)q[32 * s + l] - ms;
    }
}

/* block_q3_K: [0..31] hmask, [32..95] qs (2-bit pairs), [96..107] sixteen
   6-bit scales, [108..109] d fp16.  Scale g (one per 16 elements): low 4 bits
   are the low nibble of byte g (g < 8) or the high nibble of byte g-8, the top
   2 bits are bits 2*(g/4)..+1 of byte 8 + g%4; the signed scale is that minus
   32.  Half n (128 elements), pass j = 0..3: element 128n+32j+l (l < 32) takes
   bits 2j..2j+1 of qs[32n+l] and hmask bit 4n+j of hmask[l]; q3 = q2 - 4 when
   that bit is clear.  value = d * (sc[g] - 32) * q3, q3 in -4..3.           */
static int q3k_scale(const uint8_t *sb, int g) {
    const int lo = g < 8 ? (sb[g] & 0x0f) : (sb[g - 8] >> 4);
    const int hi = (sb[8 + (g & 3)] >> (2 * (g >> 2))) & 3;
    return (lo | (hi << 4)) - 32;
}

static void q3k_unpack(const uint8_t *blk, int *q /* 256 values -4..3 */) {
    const uint8_t *hm = blk, *qs = blk + 32;
    for (int n = 0; n < 2; ++n)
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 32; ++l) {
                const int q2 = (qs[32 * n + l] >> (2 * j)) & 3;
                const int h = (hm[l] >> (4 * n + j)) & 1;
                q[128 * n + 32 * j + l] = q2 - (h ? 0 : 4);
            }
}

/* ggml dequantize_row_q3_K, one block: y = (d * sc) * q3. */
void orc_dequant_q3_K(const uint8_t *blk, float *y) {
    const float d = orc_fp16_to_fp32(rd16(blk + 108));
    int q[256];
    q3k_unpack(blk, q);
    for (int k = 0; k < 256; ++k) y[k] = (d * (float)q3k_scale(blk + 96, k / 16)) * (float)q[k];
}

void orc_dequant_row(int type, const uint8_t *row, int n, float *y) {
    const size_t bb = orc_type_block_bytes(type);
    for (int i = 0; i < n / ORC_QK_K; ++i) {
        const uint8_t *b = row + i * bb;
        float *o = y + i * ORC_QK_K;
        switch (type) {
        case ORC_TYPE_Q3_K: orc_dequant_q3_K(b, o); break;
        case ORC_TYPE_Q4_K: orc_dequant_q4_K(b, o); break;
        case ORC_TYPE_Q5_K: orc_dequant_q5_K(b, o); break;
        default: orc_dequant_q6_K(b, o); break;
        }
    }
}

/* ggml quantize_row_q8_K_ref: per 256-block take the element of largest |x|
   (first one on ties) WITH its sign, iscale = -127/max, q = min(127,
   nearest_int(iscale*x)), d = 1/iscale (negative when max > 0), bsums over
   groups of 16.  An all-zero block gives d = 0 and q = 0. */
void orc_quantize_q8_K(const float *x, int n, orc_block_q8_K *y) {
    for (int i = 0; i < n / ORC_QK_K; ++i, x += ORC_QK_K) {
        float amax = 0.0f, mx = 0.0f;
        for (int j = 0; j < ORC_QK_K; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                mx = x[j];
            }
        }
        if (amax == 0.0f) {
            memset(&y[i], 0, sizeof(y[i]));
            continue;
        }
        const float iscale = -127.0f / mx;
        for (int j = 0; j < ORC_QK_K; ++j) {
            int v = orc_nearest_int(iscale * x[j]);
            y[i].qs[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += y[i].qs[16 * g + l];
            y[i].bsums[g] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}

/* ------------------------------------------------------------------------ */
/* Dot products                                                              */
/* ------------------------------------------------------------------------ */

/* ggml_vec_dot_f32 as built for x86 AVX2+FMA (GGML_F32_STEP 32, 4 vectors of
   8 lanes): 32 fused multiply-add chains over stride-32 elements, then
   GGML_F32x8_REDUCE (v0+=v2, v1+=v3; v0+=v1; low128+high128; two hadds). */
float orc_vec_dot_f32(int n, const float *x, const float *y) {
    float a[32];
    for (int k = 0; k < 32; ++k) a[k] = 0.0f;
    const int np = n & ~31;
    for (int i = 0; i < np; i += 32)
        for (int k = 0; k < 32; ++k) a[k] = fmaf(x[i + k], y[i + k], a[k]);
    for (int k = 0; k < 8; ++k) {
        a[k] = a[k] + a[16 + k];
        a[8 + k] = a[8 + k] + a[24 + k];
    }
    for (int k = 0; k < 8; ++k) a[k] = a[k] + a[8 + k];
    float t[4];
    for (int k = 0; k < 4; ++k) t[k] = a[k] + a[4 + k];
    float s = (t[0] + t[1]) + (t[2] + t[3]);
    for (int i = np; i < n; ++i) s += x[i] * y[i];
    return s;
}

/* ggml vec_dot_q4_K_q8_K: per block an exact integer sum
   isum = sum_s sc[s] * sum_{32} q4*q8 and msum = sum_s m[s]*(bsum pair),
   then fp32: acc += (d*dx)*isum, accm += (dmin*dx)*msum; result acc - accm.
   (ggml's generic kernel spreads acc over 8 lanes; fp32 order unpinned.)   */
float orc_vec_dot_q4_K_q8_K(int n, const uint8_t *row, const orc_block_q8_K *y) {
    float acc = 0.0f, accm = 0.0f;
    for (int i = 0; i < n / ORC_QK_K; ++i) {
        const uint8_t *b = row + (size_t)i * ORC_Q4_K_BYTES;
        const uint8_t *qs = b + 16;
        const int8_t *q8 = y[i].qs;
        int32_t isum = 0, msum = 0;
        for (int c = 0; c < 4; ++c) {
            int sc0, m0, sc1, m1;
            q4k_scale_min(2 * c, b + 4, &sc0, &m0);
            q4k_scale_min(2 * c + 1, b + 4, &sc1, &m1);
            int32_t s0 = 0, s1 = 0;
            for (int l = 0; l < 32; ++l) {
                s0 += (int32_t)(qs[32 * c + l] & 0x0f) * q8[64 * c + l];
                s1 += (int32_t)(qs[32 * c + l] >> 4) * q8[64 * c + 32 + l];
            }
            isum += sc0 * s0 + sc1 * s1;
            msum += m0 * (y[i].bsums[4 * c] + y[i].bsums[4 * c + 1]) +
                    m1 * (y[i].bsums[4 * c + 2] + y[i].bsums[4 * c + 3]);
        }
        const float d = orc_fp16_to_fp32(rd16(b)) * y[i].d;
        const float dm = orc_fp16_to_fp32(rd16(b + 2)) * y[i].d;
        acc = acc + d * (float)isum;
        accm = accm + dm * (float)msum;
    }
    return acc - accm;
}

/* ggml vec_dot_q6_K_q8_K: per block isum = sum_g sc[g] * sum_{16} (q-32)*q8,
   then acc += (d*dx)*isum in fp32. */
float orc_vec_dot_q6_K_q8_K(int n, const uint8_t *row, const orc_block_q8_K *y) {
    float acc = 0.0f;
    int q[256];
    for (int i = 0; i < n / ORC_QK_K; ++i) {
        const uint8_t *b = row + (size_t)i * ORC_Q6_K_BYTES;
        const int8_t *sc = (const int8_t *)(b + 192);
        const int8_t *q8 = y[i].qs;
        q6k_unpack(b, q);
        int32_t isum = 0;
        for (int g = 0; g < 16; ++g) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += (q[16 * g + l] - 32) * q8[16 * g + l];
            isum += sc[g] * s;
        }
        const float d = orc_fp16_to_fp32(rd16(b + 208)) * y[i].d;
        acc = acc + d * (float)isum;
    }
    return acc;
}

/* ggml vec_dot_q5_K_q8_K: as Q4_K with the fifth bit from qh: per block
   isum = sum_s sc[s] * sum_{32} q5*q8, msum = sum_s m[s]*(bsum pair);
   acc += (d*dx)*isum, accm += (dmin*dx)*msum; result acc - accm. */
float orc_vec_dot_q5_K_q8_K(int n, const uint8_t *row, const orc_block_q8_K *y) {
    float acc = 0.0f, accm = 0.0f;
    int q[256];
    for (int i = 0; i < n / ORC_QK_K; ++i) {
        const uint8_t *b = row + (size_t)i * ORC_Q5_K_BYTES;
        const int8_t *q8 = y[i].qs;
        q5k_unpack(b, q);
        int32_t isum = 0, msum = 0;
        for (int s = 0; s < 8; ++s) {
            int sc, m;
            q4k_scale_min(s, b + 4, &sc, &m);
            int32_t t = 0;
            for (int l = 0; l < 32; ++l) t += q[32 * s + l] * q8[32 * s + l];
            isum += sc * t;
            msum += m * (y[i].bsums[2 * s] + y[i].bsums[2 * s + 1]);
        }
        const float d = orc_fp16_to_fp32(rd16(b)) * y[i].d;
        const float dm = orc_fp16_to_fp32(rd16(b + 2)) * y[i].d;
        acc = acc + d * (float)isum;
        accm = accm + dm * (float)msum;
    }
    return acc - accm;
}

/* ggml vec_dot_q3_K_q8_K: per block isum = sum_g (sc[g]-32) * sum_{16} q3*q8,
   then acc += (d*dx)*isum in fp32. */
float orc_vec_dot_q3_K_q8_K(int n, const uint8_t *row, const orc_block_q8_K *y) {
    float acc = 0.0f;
    int q[256];
    for (int i = 0; i < n / ORC_QK_K; ++i) {
        const uint8_t *b = row + (size_t)i * ORC_Q3_K_BYTES;
        const int8_t *q8 = y[i].qs;
        q3k_unpack(b, q);
        int32_t isum = 0;
        for (int g = 0; g < 16; ++g) {
            int32_t s = 0;
            for (int l = 0; l < 16; ++l) s += q[16 * g + l] * q8[16 * g + l];
            isum += q3k_scale(b + 96, g) * s;
        }
        const float d = orc_fp16_to_fp32(rd16(b + 108)) * y[i].d;
        acc = acc + d * (float)isum;
    }
    return acc;
}

float orc_vec_dot_q_q8_K(int type, int n, const uint8_t *row, const orc_block_q8_K *y) {
    switch (type) {
    case ORC_TYPE_Q3_K: return orc_vec_dot_q3_K_q8_K(n, row, y);
    case ORC_TYPE_Q4_K: return orc_vec_dot_q4_K_q8_K(n, row, y);
    case ORC_TYPE_Q5_K: return orc_vec_dot_q5_K_q8_K(n, row, y);
    default: return orc_vec_dot_q6_K_q8_K(n, row, y);
    }
}

void orc_mul_mat_q8(int type, const uint8_t *w, int nrows, int ncols, const orc_block_q8_K *qx,
                    float *out) {
    const size_t row_bytes = (size_t)(ncols / ORC_QK_K) * orc_type_block_bytes(type);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) if (nrows >= 64)
#endif
    for (int r = 0; r < nrows; ++r) {
        const uint8_t *row = w + (size_t)r * row_bytes;
        out[r] = orc_vec_dot_q_q8_K(type, ncols, row, qx);
    }
}

void orc_mul_mat_q(int type, const uint8_t *w, int nrows, int ncols, const float *x, float *out) {
    orc_block_q8_K *qx = (orc_block_q8_K *)malloc(sizeof(orc_block_q8_K) * (ncols / ORC_QK_K));
    orc_quantize_q8_K(x, ncols, qx);
    orc_mul_mat_q8(type, w, nrows, ncols, qx, out);
    free(qx);
}

/* ------------------------------------------------------------------------ */
/* Elementwise (ggml_silu_f32, ggml sigmoid)                                 */
/* ------------------------------------------------------------------------ */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* ------------------------------------------------------------------------ */
/* Router tail: src/run_moe_stream.cpp:353-356 (mul_mat, soft_max, top_k,
   get_rows) and :371-373 (host renorm with the 6.103515625e-5 clamp).      */
/* ------------------------------------------------------------------------ */
void orc_route(int n_embd, int n_expert, int n_used, int renorm, const float *w_router,
               const float *fx, int32_t *sel, float *wsel, float *probs_out) {
    float *p = (float *)malloc(sizeof(float) * n_expert);
    /* logits: ggml_mul_mat(ffn_gate_inp, fx) -> one ggml_vec_dot_f32 per expert row */
    for (int e = 0; e < n_expert; ++e) p[e] = orc_vec_dot_f32(n_embd, w_router + (size_t)e * n_embd, fx);
    /* ggml_soft_max: max, exp(x - max) summed in double, scale by (float)(1/sum) */
    float mx = -INFINITY;
    for (int e = 0; e < n_expert; ++e) mx = p[e] > mx ? p[e] : mx;
    double sum = 0.0;
    for (int e = 0; e < n_expert; ++e) {
        const float v = expf(p[e] - mx);
        sum += (double)v;
        p[e] = v;
    }
    const float scale = (float)(1.0 / sum);
    for (int e = 0; e < n_expert; ++e) p[e] *= scale;
    /* ggml_top_k: the n_used largest probabilities, descending; ties -> lower index */
    char *taken = (char *)calloc((size_t)n_expert, 1);
    for (int j = 0; j < n_used; ++j) {
        int best = -1;
        for (int e = 0; e < n_expert; ++e) {
            if (taken[e]) continue;
            if (best < 0 || p[e] > p[best]) best = e;
        }
        taken[best] = 1;
        sel[j] = best;
        wsel[j] = p[best]; /* ggml_get_rows(probs, sel) */
    }
    free(taken);
    if (renorm) {
        float ws = 0.0f;
        for (int j = 0; j < n_used; ++j) ws += wsel[j];
        if (ws < 6.103515625e-5f) ws = 6.103515625e-5f;
        for (int j = 0; j < n_used; ++j) wsel[j] /= ws;
    }
    if (probs_out) memcpy(probs_out, p, sizeof(float) * n_expert);
    free(p);
}

/* ------------------------------------------------------------------------ */
/* Graph B: src/run_moe_stream.cpp:432-435 per expert:
     g = mul_mat(gate, x); u = mul_mat(up, x); h = mul(silu(g), u); y = mul_mat(down, h)
   ggml-cpu quantises the f32 activation of every Q4_K/Q6_K mul_mat to Q8_K. */
/* ------------------------------------------------------------------------ */
void orc_expert_ffn(int n_embd, int n_ff, int gate_type, int up_type, int down_type,
                    const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                    const orc_block_q8_K *qx, float *y, float *h_out) {
    float *g = (float *)malloc(sizeof(float) * n_ff);
    float *u = (float *)malloc(sizeof(float) * n_ff);
    orc_block_q8_K *qh = (orc_block_q8_K *)malloc(sizeof(orc_block_q8_K) * (n_ff / ORC_QK_K));
    orc_mul_mat_q8(gate_type, gate, n_ff, n_embd, qx, g);
    orc_mul_mat_q8(up_type, up, n_ff, n_embd, qx, u);
    for (int r = 0; r < n_ff; ++r) g[r] = orc_silu(g[r]) * u[r];
    if (h_out) memcpy(h_out, g, sizeof(float) * n_ff);
    orc_quantize_q8_K(g, n_ff, qh);
    orc_mul_mat_q8(down_type, down, n_embd, n_ff, qh, y);
    free(g);
    free(u);
    free(qh);
}

/* Graph B over sel plus the host combine, src/run_moe_stream.cpp:424-447 and
   the gated shared expert of src/run_qwen35.cpp:658-666, 675-676:
     out[d] = ((sum_{j ascending} w_j*y_j[d]) + shex[d]) + res[d]
     shex = sigmoid(gate_inp_shexp . x) * down_sh(silu(gate_sh x) * up_sh x)  */
void orc_moe_ffn_combine(const orc_layer_cfg *cfg, const orc_layer_weights *w, const float *fx,
                         const int32_t *sel, const float *wsel, const float *res, float *out) {
    const int ne = cfg->n_embd, nf = cfg->n_ff, k = cfg->n_used;
    const size_t gs = orc_expert_stride(cfg->gate_type, nf, ne);
    const size_t us = orc_expert_stride(cfg->up_type, nf, ne);
    const size_t ds = orc_expert_stride(cfg->down_type, ne, nf);
    orc_block_q8_K *qx = (orc_block_q8_K *)malloc(sizeof(orc_block_q8_K) * (ne / ORC_QK_K));
    orc_quantize_q8_K(fx, ne, qx);
    float *eout = (float *)malloc(sizeof(float) * (size_t)ne * k);
    for (int j = 0; j < k; ++j) {
        const size_t e = (size_t)sel[j];
        orc_expert_ffn(ne, nf, cfg->gate_type, cfg->up_type, cfg->down_type, w->gate + e * gs,
                       w->up + e * us, w->down + e * ds, qx, eout + (size_t)j * ne, NULL);
    }
    float *shex = NULL;
    if (cfg->n_ff_shexp > 0) {
        shex = (float *)malloc(sizeof(float) * ne);
        orc_expert_ffn(ne, cfg->n_ff_shexp, cfg->sh_gate_type, cfg->sh_up_type, cfg->sh_down_type,
                       w->sh_gate, w->sh_up, w->sh_down, qx, shex, NULL);
        const float sg = orc_sigmoid(orc_vec_dot_f32(ne, w->sh_gate_inp, fx));
        for (int d = 0; d < ne; ++d) shex[d] = shex[d] * sg;
    }
    for (int d = 0; d < ne; ++d) {
        float acc = 0.0f;
        for (int j = 0; j < k; ++j) acc += wsel[j] * eout[(size_t)j * ne + d];
        out[d] = shex ? (acc + shex[d]) + res[d] : acc + res[d];
    }
    free(shex);
    free(eout);
    free(qx);
}

void orc_moe_layer(const orc_layer_cfg *cfg, const orc_layer_weights *w, const float *fx,
                   const float *res, float *out, int32_t *sel, float *wsel) {
    orc_route(cfg->n_embd, cfg->n_expert, cfg->n_used, cfg->renorm, w->router, fx, sel, wsel, NULL);
    orc_moe_ffn_combine(cfg, w, fx, sel, wsel, res, out);
}

/* ggml_mul_mat_id over m tokens (src/run_specloop.cpp:126-139): each token's
   activation row is quantised on its own and each (token, expert) product is
   the same vec_dot as the single-token path, so the batch is the per-token
   stage applied to every row. */
void orc_moe_layer_batched(const orc_layer_cfg *cfg, const orc_layer_weights *w, int m,
                           const float *fx, const float *res, float *out, int32_t *sel,
                           float *wsel) {
    const int ne = cfg->n_embd, k = cfg->n_used;
    for (int t = 0; t < m; ++t)
        orc_moe_layer(cfg, w, fx + (size_t)t * ne, res + (size_t)t * ne, out + (size_t)t * ne,
                      sel + (size_t)t * k, wsel + (size_t)t * k);
}

/* ggml_rms_norm: mean of x*x accumulated in double, scale = 1/sqrtf(mean+eps). */
void orc_rms_norm(int n, const float *x, float eps, float *y) {
    double sum = 0.0;
    for (int i = 0; i < n; ++i) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = 0; i < n; ++i) y[i] = x[i] * scale;
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
