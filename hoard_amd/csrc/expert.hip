// Grouped dequant-GEMV over the selected experts (kernel family 2) and the
// fused weighted combine (family 4), one token.
//
// Replaces graph B of src/run_moe_stream.cpp:431-438 (per expert:
// mul_mat(gate), mul_mat(up), mul(silu(g), u), mul_mat(down), concat) plus the
// shared expert of src/run_qwen35.cpp:658-666, and the host combine at
// src/run_moe_stream.cpp:447 / src/run_qwen35.cpp:675-676.
//
// Both kernels stage the weight bytes they own into LDS with 16-byte loads of
// the contiguous GGUF byte stream (a run of whole rows of one expert matrix is
// contiguous), quantise their activation to Q8_K in LDS exactly as the CPU path
// does, then give each lane one (matrix, row, super-block) integer dot.  The
// per-block fp32 terms go back through LDS and one lane per row adds them in
// block order, so g, u and y match the CPU restatement bit for bit given the
// same activation.
#include "kernels.h"
#include "qblocks.h"
#include "wave.h"

namespace hoard {

namespace {

constexpr int kThreads = 256;
constexpr int kGateUpRows = 16;

__device__ __forceinline__ int block_bytes_dev(int type) { return kquant_block_bytes(type); }

template <class P>
__device__ __forceinline__ void *align16(P *p) {
    return reinterpret_cast<void *>((reinterpret_cast<uintptr_t>(p) + 15) & ~(uintptr_t)15);
}

// LDS bytes reserved for a staged run of `nbytes` starting at any address.
__host__ __device__ __forceinline__ size_t stage_region(size_t nbytes) {
    return (nbytes + 32 + 15) & ~(size_t)15;
}

// Copy [src, src+nbytes) into LDS starting at dst + (src & 15) with aligned
// 16-byte loads; returns that offset.  Reads up to 15 bytes past the end,
// which device allocations keep as padding.
__device__ __forceinline__ int stage_issue(uint8_t *dst, const uint8_t *src, size_t nbytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(src);
    const uintptr_t a0 = a & ~(uintptr_t)15;
    const int n16 = (int)((a + nbytes + 15 - a0) >> 4);
    const uint4 *s = reinterpret_cast<const uint4 *>(a0);
    uint4 *d = reinterpret_cast<uint4 *>(dst);
#pragma unroll 8
    for (int i = threadIdx.x; i < n16; i += kThreads) d[i] = s[i];
    return (int)(a - a0);
}

__device__ __forceinline__ size_t row_bytes(int type, int cols) {
    return (size_t)(cols / QK) * (size_t)kquant_block_bytes(type);
}

__device__ __forceinline__ void terms_dyn(int type, const uint8_t *blk, const Q8Block &x, float &tm,
                                          float &tn) {
    switch (type) {
    case kTypeQ4K: q4k_block_terms(blk, x, tm, tn); break;
    case kTypeQ5K: q5k_block_terms(blk, x, tm, tn); break;
    case kTypeQ3K: q3k_block_terms(blk, x, tm, tn); break;
    default: q6k_block_terms(blk, x, tm, tn); break;
    }
}

__device__ __forceinline__ float row_sum_dyn(int type, const float2 *t, int nb) {
    float acc = 0.0f, accm = 0.0f;
    for (int b = 0; b < nb; ++b) {
        acc = acc + t[b].x;
        accm = accm + t[b].y;
    }
    return kquant_has_min(type) ? acc - accm : acc;
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// gate/up + SwiGLU.  grid = (rows_max / R, k + has_shared); block = 256; R
// rows of gate and of up per workgroup (fewer for wide rows, so they fit LDS).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void gateup_kernel(GateUpArgs a, int R) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int j = blockIdx.y;
    const bool shared = j >= a.k;
    const MatDesc G = shared ? a.sh_gate : a.gate;
    const MatDesc U = shared ? a.sh_up : a.up;
    const int rows = G.rows;
    const int r0 = blockIdx.x * R;
    if (r0 >= rows) return;
    const int nb = a.n_embd / QK;
    float *hout = a.h + (size_t)j * a.hstride + r0;

    if (shared && blockIdx.x == 0 && threadIdx.x < 32) {
        // sigmoid gate of the shared expert: f32 dot in the router's lane order
        const int l = threadIdx.x;
        float acc = 0.0f;
        for (int i = 0; i < a.n_embd; i += 32) acc = fmaf(a.sh_gate_inp[i + l], a.fx[i + l], acc);
        acc = acc + __shfl_xor(acc, 16);
        acc = acc + __shfl_xor(acc, 8);
        acc = acc + __shfl_xor(acc, 4);
        acc = acc + __shfl_xor(acc, 1);
        acc = acc + __shfl_xor(acc, 2);
        if (l == 0) a.sgate[0] = 1.0f / (1.0f + expf(-acc));
    }

    const uint8_t *gsrc, *usrc;
    if (shared) {
        gsrc = G.base;
        usrc = U.base;
    } else {
        const int id = a.ids[j];
        if (id < 0 || id >= G.n_ids) {  // invalid id: poison this expert's rows
            if (threadIdx.x < R) hout[threadIdx.x] = __builtin_nanf("");
            return;
        }
        gsrc = G.base + (size_t)id * G.stride;
        usrc = U.base + (size_t)id * U.stride;
    }
    const size_t rbg = row_bytes(G.type, a.n_embd), rbu = row_bytes(U.type, a.n_embd);
    gsrc += (size_t)r0 * rbg;
    usrc += (size_t)r0 * rbu;

    uint8_t *lds_g = smem;
    uint8_t *lds_u = lds_g + stage_region(R * rbg);
    Q8Block *qx = reinterpret_cast<Q8Block *>(lds_u + stage_region(R * rbu));
    float2 *terms = reinterpret_cast<float2 *>(align16(qx + nb));

    const int og = stage_issue(lds_g, gsrc, R * rbg);
    const int ou = stage_issue(lds_u, usrc, R * rbu);

    const int wave = wave_index();
    for (int b = wave; b < nb; b += kThreads / 64) wave_quantize_q8k(a.fx + b * QK, &qx[b]);
    __syncthreads();

    const int per_mat = R * nb;
    for (int u = threadIdx.x; u < 2 * per_mat; u += kThreads) {
        const int mat = u / per_mat, rem = u - mat * per_mat;
        const int row = rem / nb, b = rem - row * nb;
        float tm, tn;
        if (mat == 0)
            terms_dyn(G.type, lds_g + og + row * rbg + b * block_bytes_dev(G.type), qx[b], tm, tn);
        else
            terms_dyn(U.type, lds_u + ou + row * rbu + b * block_bytes_dev(U.type), qx[b], tm, tn);
        terms[u] = make_float2(tm, tn);
    }
    __syncthreads();

    if (threadIdx.x < R) {
        const int r = threadIdx.x;
        const float g = row_sum_dyn(G.type, terms + r * nb, nb);
        const float uu = row_sum_dyn(U.type, terms + per_mat + r * nb, nb);
        hout[r] = silu(g) * uu;
    }
}

// ---------------------------------------------------------------------------
// down + combine.  grid = n_embd / rd; block = 256.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void down_combine_kernel(DownArgs a, int rd) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int d0 = blockIdx.x * rd;
    const int k = a.k;
    const bool has_sh = a.sh_down.base != nullptr;
    const int nseg = k + (has_sh ? 1 : 0);
    const int nbh = a.down.cols / QK;
    const int nbs = has_sh ? a.sh_down.cols / QK : 0;
    const size_t rbd = row_bytes(a.down.type, a.down.cols);
    const size_t rbs = has_sh ? row_bytes(a.sh_down.type, a.sh_down.cols) : 0;
    const size_t reg_d = stage_region(rd * rbd), reg_s = has_sh ? stage_region(rd * rbs) : 0;

    uint8_t *lds_w = smem;
    Q8Block *qh = reinterpret_cast<Q8Block *>(lds_w + k * reg_d + reg_s);
    const int nq = k * nbh + nbs;
    float2 *terms = reinterpret_cast<float2 *>(align16(qh + nq));
    __shared__ int offs[17];
    __shared__ int bad;
    __shared__ float wj[16];

    if (threadIdx.x == 0) bad = 0;
    if (threadIdx.x < k) wj[threadIdx.x] = a.w[threadIdx.x];
    __syncthreads();
    for (int s = 0; s < nseg; ++s) {
        const uint8_t *src;
        size_t nbytes;
        uint8_t *dst;
        if (s < k) {
            const int id = a.ids[s];
            if (id < 0 || id >= a.down.n_ids) {
                if (threadIdx.x == 0) bad = 1;
                continue;
            }
            src = a.down.base + (size_t)id * a.down.stride + (size_t)d0 * rbd;
            nbytes = rd * rbd;
            dst = lds_w + s * reg_d;
        } else {
            src = a.sh_down.base + (size_t)d0 * rbs;
            nbytes = rd * rbs;
            dst = lds_w + k * reg_d;
        }
        const int o = stage_issue(dst, src, nbytes);
        if (threadIdx.x == 0) offs[s] = o;
    }

    const int wave = wave_index();
    for (int q = wave; q < nq; q += kThreads / 64) {
        const int j = q < k * nbh ? q / nbh : k;
        const int b = q < k * nbh ? q - j * nbh : q - k * nbh;
        wave_quantize_q8k(a.h + (size_t)j * a.hstride + b * QK, &qh[q]);
    }
    __syncthreads();
    if (bad) {
        if (threadIdx.x < rd) a.out[d0 + threadIdx.x] = __builtin_nanf("");
        return;
    }

    const int routed_units = k * rd * nbh;
    const int units = routed_units + rd * nbs;
    for (int u = threadIdx.x; u < units; u += kThreads) {
        float tm, tn;
        if (u < routed_units) {
            const int j = u / (rd * nbh), rem = u - j * rd * nbh;
            const int row = rem / nbh, b = rem - row * nbh;
            terms_dyn(a.down.type,
                      lds_w + j * reg_d + offs[j] + row * rbd + b * block_bytes_dev(a.down.type),
                      qh[j * nbh + b], tm, tn);
        } else {
            const int v = u - routed_units;
            const int row = v / nbs, b = v - row * nbs;
            terms_dyn(a.sh_down.type,
                      lds_w + k * reg_d + offs[k] + row * rbs + b * block_bytes_dev(a.sh_down.type),
                      qh[k * nbh + b], tm, tn);
        }
        terms[u] = make_float2(tm, tn);
    }
    __syncthreads();

    if (threadIdx.x < rd) {
        const int r = threadIdx.x;
        float acc = 0.0f;
        for (int j = 0; j < k; ++j) {
            const float y = row_sum_dyn(a.down.type, terms + (j * rd + r) * nbh, nbh);
            acc = acc + wj[j] * y;
        }
        const int d = d0 + r;
        float o;
        if (has_sh) {
            const float ysh = row_sum_dyn(a.sh_down.type, terms + routed_units + r * nbs, nbs);
            o = (acc + ysh * a.sgate[0]) + a.res[d];
        } else {
            o = acc + a.res[d];
        }
        a.out[d] = o;
    }
}

}  // namespace

size_t block_bytes(int type) { return (size_t)kquant_block_bytes(type); }

static size_t host_row_bytes(int type, int cols) { return (size_t)(cols / QK) * block_bytes(type); }

hipError_t launch_gateup(const GateUpArgs &a, hipStream_t s) {
    const int nb = a.n_embd / QK;
    int rows_max = a.gate.rows;
    if (a.sh_gate.base) rows_max = rows_max > a.sh_gate.rows ? rows_max : a.sh_gate.rows;
    // the most rows per workgroup (16 down to 1) whose staged tiles fit 64 KiB of LDS
    for (int R = kGateUpRows; R >= 1; R >>= 1) {
        size_t need = stage_region(R * host_row_bytes(a.gate.type, a.n_embd)) +
                      stage_region(R * host_row_bytes(a.up.type, a.n_embd));
        if (a.sh_gate.base) {
            const size_t ns = stage_region(R * host_row_bytes(a.sh_gate.type, a.n_embd)) +
                              stage_region(R * host_row_bytes(a.sh_up.type, a.n_embd));
            need = need > ns ? need : ns;
        }
        const size_t lds = need + nb * sizeof(Q8Block) + 16 + 2 * (size_t)R * nb * sizeof(float2);
        if (lds > 65536 || rows_max % R) continue;
        dim3 grid((unsigned)(rows_max / R), (unsigned)(a.k + (a.sh_gate.base ? 1 : 0)));
        hipLaunchKernelGGL(gateup_kernel, grid, dim3(kThreads), lds, s, a, R);
        return hipGetLastError();
    }
    return hipErrorInvalidConfiguration;
}

hipError_t launch_down_combine(const DownArgs &a, hipStream_t s) {
    const bool has_sh = a.sh_down.base != nullptr;
    const int nbh = a.down.cols / QK, nbs = has_sh ? a.sh_down.cols / QK : 0;
    for (int rd = 8; rd >= 1; rd >>= 1) {
        if (a.n_embd % rd) continue;
        const size_t reg_d = stage_region(rd * host_row_bytes(a.down.type, a.down.cols));
        const size_t reg_s = has_sh ? stage_region(rd * host_row_bytes(a.sh_down.type, a.sh_down.cols)) : 0;
        const int nq = a.k * nbh + nbs;
        const size_t lds = a.k * reg_d + reg_s + nq * sizeof(Q8Block) + 16 +
                           (size_t)(a.k * rd * nbh + rd * nbs) * sizeof(float2);
        if (lds > 65536) continue;
        hipLaunchKernelGGL(down_combine_kernel, dim3((unsigned)(a.n_embd / rd)), dim3(kThreads), lds, s,
                           a, rd);
        return hipGetLastError();
    }
    return hipErrorInvalidConfiguration;
}

}  // namespace hoard
