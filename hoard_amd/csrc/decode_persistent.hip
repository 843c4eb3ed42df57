// Persistent stacked decode: every layer of one token in a single cooperative
// launch (router tail, grouped expert FFN, combine, rms_norm between layers).
//
// Replaces, for a whole token, the reference's per-layer loop of graph A's
// router tail (src/run_moe_stream.cpp:353-373), graph B (:424-445) and the
// host combine (:447), with no host round trip between layers.
//
// Mapping onto MI355X (256 CUs in 8 XCDs of 32, one workgroup per CU):
//   * expert slot j of the top-k runs on XCD j; its gate/up rows and down rows
//     are split over that XCD's 32 workgroups, so the h gather stays inside one
//     XCD's L2;
//   * every XCD computes the router (each workgroup E/32 rows, weights
//     prefetched into LDS during the previous layer) and the top-k redundantly,
//     so routing needs no cross-XCD traffic;
//   * only the expert outputs y_j cross XCDs: workgroup (j, r) publishes rows
//     [64r, 64r+64) of y_j with device-coherent stores and a flag, and the
//     workgroups of rank r on every XCD combine exactly those rows;
//   * weights stream straight into LDS with global_load_lds_dwordx4.
// Synchronisation uses per-workgroup flags holding a monotonically increasing
// sequence number (no atomics): XCD-local flags live in the XCD's L2 and are
// polled after invalidating L1; cross-XCD flags and y use device-scope
// (L2-bypassing) loads and stores.  Every wait is bounded by a wall-clock
// timeout that raises an error flag and poisons the output instead of hanging.
#include "kernels.h"
#include "qblocks.h"
#include "rowdot.h"
#include "wave.h"

namespace hoard {

namespace {

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kXcds = 8;
constexpr int kPerXcd = 32;
constexpr int kFlagStride = 32;             // words: one 128-byte line per flag
constexpr long long kTimeoutTicks = 20000000;  // 200 ms at the 100 MHz wall clock

__device__ __forceinline__ unsigned xcc_id() {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 7u;
}


__device__ __forceinline__ unsigned ld_dev_u32(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev_f32(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u32(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_f32(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool reached(unsigned v, unsigned target) { return (int)(v - target) >= 0; }

// Issue global_load_lds_dwordx4 for [src, src+nbytes) into LDS at dst, in
// 1 KB chunks (64 lanes x 16 B) spread over waves [w0, w0+nw).  Rounds the
// source down to 16 bytes (returned offset) and reads whole chunks, i.e. up to
// 1 KB + 15 bytes past the end, which device allocations keep as padding.
__device__ __forceinline__ int issue_lds_copy(uint8_t *dst, const uint8_t *src, size_t nbytes, int w0, int nw) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(src);
    const uintptr_t a0 = a & ~(uintptr_t)15;
    const int off = (int)(a - a0);
    const int nchunks = (int)((off + nbytes + 1023) >> 10);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (wave >= w0 && wave < w0 + nw) {
        for (int c = wave - w0; c < nchunks; c += nw)
            __builtin_amdgcn_global_load_lds((const void *)(a0 + (size_t)c * 1024 + lane * 16),
                                             (lds_void *)(dst + c * 1024), 16, 0, 0);
    }
    return off;
}

__host__ __device__ __forceinline__ size_t chunk_region(size_t nbytes) { return ((nbytes + 15 + 1023) >> 10) << 10; }

__device__ __forceinline__ size_t row_bytes_dev(int type, int cols) {
    return (size_t)(cols / QK) * (type == kTypeQ4K ? kQ4KBytes : kQ6KBytes);
}

struct Smem {
    // byte offsets into dynamic LDS
    int xs, fxs, w, gate, up, down, q8x, q8h, gu, ys, ps;
};

__host__ __device__ __forceinline__ Smem smem_layout(const PersistentArgs &a, size_t *total) {
    Smem s;
    size_t o = 0;
    auto take = [&](size_t n) {
        const int r = (int)o;
        o += (n + 15) & ~(size_t)15;
        return r;
    };
    s.xs = take(4 * (size_t)a.n_embd);
    s.fxs = take(4 * (size_t)a.n_embd);
    s.w = take((size_t)(a.E / kPerXcd) * a.n_embd * 4);
    s.gate = take(chunk_region((size_t)a.rows_gu * a.max_rb_gu));
    s.up = take(chunk_region((size_t)a.rows_gu * a.max_rb_gu));
    s.down = take(chunk_region((size_t)a.rows_d * a.max_rb_d));
    s.q8x = take(sizeof(Q8L) * (a.n_embd / QK));
    s.q8h = take(sizeof(Q8L) * (a.n_ff / QK));
    s.gu = take(4 * 2 * (size_t)a.rows_gu);
    s.ys = take(4 * (size_t)a.rows_d);
    s.ps = take(4 * (size_t)a.E);
    if (total) *total = o;
    return s;
}

// Raw workgroup barrier: LDS writes of every wave are done, global and LDS-DMA
// loads may stay in flight (a __syncthreads fence would wait for those too).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// {value, seq} words: the value travels with the sequence number of the step that
// produced it, so a consumer polls the data itself instead of a separate flag.
__device__ __forceinline__ uint64_t tag(float v, unsigned seq) {
    return ((uint64_t)seq << 32) | (uint64_t)__float_as_uint(v);
}
__device__ __forceinline__ unsigned tag_seq(uint64_t w) { return (unsigned)(w >> 32); }
__device__ __forceinline__ float tag_val(uint64_t w) { return __uint_as_float((unsigned)w); }
// XCD-local words: plain 8-byte stores, which write through the CU's L1 into
// the XCD's L2.  Readers use device-scope (sc1) loads: they skip L1 and are
// served by this XCD's L2 for lines its own CUs wrote.  No L1 invalidate is
// used anywhere: a buffer_inv issued while another wave of the same CU still
// has stores in flight lost those stores on gfx950.  One aligned 8-byte access
// is a single memory transaction, so a value and its sequence number are
// always read together.
__device__ __forceinline__ void st_l2(uint64_t *p, uint64_t w) { *p = w; }
__device__ __forceinline__ uint64_t ld_l2(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Device-wide words (L2-bypassing).
__device__ __forceinline__ void st_dev64(uint64_t *p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev64(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded poll: true once ready() holds; false on timeout or a raised error.
template <class F>
__device__ __forceinline__ bool poll(F ready, int *err) {
    const long long t0 = wall_clock64();
    for (int it = 0;; ++it) {
        if (ready()) return true;
        if ((it & 31) == 31) {
            if (ld_dev_u32((const unsigned *)err) != 0u) return false;
            if (wall_clock64() - t0 > kTimeoutTicks) {
                st_dev_u32((unsigned *)err, 1u);
                return false;
            }
        }
    }
}

__global__ __launch_bounds__(kThreads) void decode_kernel(PersistentArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int sh_rank, sh_fail;
    __shared__ int sel_s[16];
    __shared__ float w_s[16];
    __shared__ double red_d[kWaves];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int grp = tid >> 3, t8 = tid & 7;  // 64 groups of 8 lanes
    const unsigned xcc = xcc_id();
    if (tid == 0) {
        const unsigned t = __hip_atomic_fetch_add(a.tickets + xcc * kFlagStride, 1u, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        sh_rank = (int)(t % kPerXcd);
        sh_fail = 0;
    }
    __syncthreads();
    const int rank = sh_rank;
    const Smem S = smem_layout(a, nullptr);
    float *xs = reinterpret_cast<float *>(smem + S.xs);
    float *fxs = reinterpret_cast<float *>(smem + S.fxs);
    const float *wl = reinterpret_cast<const float *>(smem + S.w);
    Q8L *q8x = reinterpret_cast<Q8L *>(smem + S.q8x);
    Q8L *q8h = reinterpret_cast<Q8L *>(smem + S.q8h);
    float *gu = reinterpret_cast<float *>(smem + S.gu);
    float *ys = reinterpret_cast<float *>(smem + S.ys);
    float *ps = reinterpret_cast<float *>(smem + S.ps);

    const int n = a.n_embd, E = a.E, k = a.k;
    const int rw = E / kPerXcd;  // router rows per workgroup
    const int nb = n / QK, nbh = a.n_ff / QK;
    const int R = a.rows_gu, RD = a.rows_d;
    const bool has_expert = (int)xcc < k;
    uint64_t *LGx = a.LG + (size_t)xcc * E;
    uint64_t *Hx = a.H + (size_t)xcc * a.n_ff;

    // phase stamps: [layer][xcc*32 + rank][phase]
    auto stamp = [&](int l, int phase) {
        if (a.trace && tid == 0)
            a.trace[((size_t)(l - a.l0) * (kXcds * kPerXcd) + xcc * kPerXcd + rank) * kTracePhases + phase] =
                wall_clock64();
    };
    auto prefetch_router = [&](int l, int w0, int nw) {
        const DecodeLayer &Lr = a.layers[l];
        issue_lds_copy(smem + S.w, reinterpret_cast<const uint8_t *>(Lr.router + (size_t)rank * rw * n),
                       (size_t)rw * n * 4, w0, nw);
    };

    // ---- prologue: router rows of the first layer, and x ----
    prefetch_router(a.l0, 0, kWaves);
    for (int i = tid; i < n; i += kThreads) xs[i] = a.x[i];

    bool ok = true;
    for (int l = a.l0; l < a.l1; ++l) {
        const DecodeLayer &L = a.layers[l];
        const unsigned seq = a.seq0 + 4u * (unsigned)(l - a.l0);
        const int cur = (l - a.l0) & 1;
        const bool last = l + 1 == a.l1;
        stamp(l, 0);
        __builtin_amdgcn_s_waitcnt(0);  // router rows in flight since the previous layer
        if (l > a.l0) {
            // x of this layer: the XCD's 32 workgroups published 64 rows each
            const uint64_t *xsrc = a.X + ((size_t)cur * kXcds + xcc) * n;
            for (int i0 = 4 * tid; i0 < n; i0 += 4 * kThreads) {
                uint64_t w[4];
                const bool got = poll(
                    [&]() {
                        bool r = true;
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            w[c] = ld_l2(xsrc + i0 + c);
                            r = r && tag_seq(w[c]) == seq - 1u;
                        }
                        return r;
                    },
                    a.err);
                if (!got) sh_fail = 1;
                *reinterpret_cast<float4 *>(xs + i0) = make_float4(tag_val(w[0]), tag_val(w[1]), tag_val(w[2]), tag_val(w[3]));
            }
        }
        __syncthreads();
        if (sh_fail) {
            ok = false;
            break;
        }
        stamp(l, 1);

        // -- P1: rms_norm scale, fx, router rows (8 lanes each), Q8_K(fx) --
        {
            double ss = 0.0;
            for (int i = tid; i < n; i += kThreads) {
                const float v = xs[i];
                ss += (double)(v * v);
            }
            ss = wave_sum_d(ss);
            if (lane == 0) red_d[wave] = ss;
        }
        __syncthreads();
        {
            double tot = 0.0;
            for (int w = 0; w < kWaves; ++w) tot += red_d[w];
            const float mean = (float)(tot / (double)n);
            const float scale = 1.0f / sqrtf(mean + a.eps);
            for (int i = tid; i < n; i += kThreads) fxs[i] = xs[i] * scale;
        }
        __syncthreads();
        if (wave == 0) {
            const int row = lane >> 3, m = lane & 7;
            if (row < rw) {
                const float *wr = wl + (size_t)row * n + 4 * m;
                const float *fr = fxs + 4 * m;
                float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll 8
                for (int i = 0; i < n; i += 32) {
                    const float4 wv = *reinterpret_cast<const float4 *>(wr + i);
                    const float4 fv = *reinterpret_cast<const float4 *>(fr + i);
                    a0 = fmaf(wv.x, fv.x, a0);
                    a1 = fmaf(wv.y, fv.y, a1);
                    a2 = fmaf(wv.z, fv.z, a2);
                    a3 = fmaf(wv.w, fv.w, a3);
                }
                const float r = group8_ggml_fold(a0, a1, a2, a3);
                if (m == 0) st_l2(LGx + rank * rw + row, tag(r, seq));
            }
        }
        for (int b = wave; b < nb; b += kWaves) wave_quantize_q8l(fxs + b * QK, &q8x[b]);
        stamp(l, 2);
        stamp(l, 3);

        // -- P2 (wave 0): softmax over all experts, top-k by rank, renorm --
        if (wave == 0) {
            uint64_t w0 = 0, w1 = 0;
            const bool got = poll(
                [&]() {
                    if (lane < E) w0 = ld_l2(LGx + lane);
                    if (lane + 64 < E) w1 = ld_l2(LGx + lane + 64);
                    const bool r = (lane >= E || tag_seq(w0) == seq) && (lane + 64 >= E || tag_seq(w1) == seq);
                    return (bool)__all(r);
                },
                a.err);
            if (!got && lane == 0) sh_fail = 1;
            float p0 = lane < E ? tag_val(w0) : -INFINITY;
            float p1 = lane + 64 < E ? tag_val(w1) : -INFINITY;
            const float mx = wave_max_f(p0 > p1 ? p0 : p1);
            double sum = 0.0;
            if (lane < E) {
                p0 = expf(p0 - mx);
                sum += (double)p0;
            }
            if (lane + 64 < E) {
                p1 = expf(p1 - mx);
                sum += (double)p1;
            }
            sum = wave_sum_d(sum);
            const float sc = (float)(1.0 / sum);
            p0 = p0 * sc;
            p1 = p1 * sc;
            if (lane < E) ps[lane] = p0;
            if (lane + 64 < E) ps[lane + 64] = p1;
            if (lane < 16) sel_s[lane] = -1;
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are visible to it
            __builtin_amdgcn_wave_barrier();
            // rank = experts ahead in (probability desc, index asc) order
            int r0 = 0, r1 = 0;
            for (int e4 = 0; e4 < E; e4 += 4) {
                const float4 pv = *reinterpret_cast<const float4 *>(ps + e4);
                const float pe[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int e2 = e4 + c;
                    r0 += (pe[c] > p0 || (pe[c] == p0 && e2 < lane)) ? 1 : 0;
                    r1 += (pe[c] > p1 || (pe[c] == p1 && e2 < lane + 64)) ? 1 : 0;
                }
            }
            if (lane < E && r0 < k) {
                sel_s[r0] = lane;
                w_s[r0] = p0;
            }
            if (lane + 64 < E && r1 < k) {
                sel_s[r1] = lane + 64;
                w_s[r1] = p1;
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __builtin_amdgcn_wave_barrier();
            if (lane == 0) {
                float ws = 0.0f;
                for (int j = 0; j < k; ++j) {
                    if (sel_s[j] < 0 || sel_s[j] >= E) {  // only reachable with NaN logits
                        sel_s[j] = 0;
                        w_s[j] = __builtin_nanf("");
                    }
                    ws = ws + w_s[j];
                }
                if (a.renorm) {
                    if (ws < 6.103515625e-5f) ws = 6.103515625e-5f;
                    for (int j = 0; j < k; ++j) w_s[j] = w_s[j] / ws;
                }
            }
        }
        __syncthreads();
        if (sh_fail) {
            ok = false;
            break;
        }
        stamp(l, 4);

        // -- P3: waves 0-3 stream gate/up rows, waves 4-7 stream down rows --
        const int e = has_expert ? sel_s[xcc] : 0;
        const size_t rbg = row_bytes_dev(L.gate_type, n), rbu = row_bytes_dev(L.up_type, n);
        const size_t rbd = row_bytes_dev(L.down_type, a.n_ff);
        const uint8_t *gsrc = L.gate + (size_t)e * L.gstride + (size_t)rank * R * rbg;
        const uint8_t *usrc = L.up + (size_t)e * L.ustride + (size_t)rank * R * rbu;
        const uint8_t *dsrc = L.down + (size_t)e * L.dstride + (size_t)rank * RD * rbd;
        const int og = (int)(reinterpret_cast<uintptr_t>(gsrc) & 15);
        const int ou = (int)(reinterpret_cast<uintptr_t>(usrc) & 15);
        const int od = (int)(reinterpret_cast<uintptr_t>(dsrc) & 15);
        if (has_expert) {
            issue_lds_copy(smem + S.gate, gsrc, (size_t)R * rbg, 0, kWaves / 2);
            issue_lds_copy(smem + S.up, usrc, (size_t)R * rbu, 0, kWaves / 2);
            issue_lds_copy(smem + S.down, dsrc, (size_t)RD * rbd, kWaves / 2, kWaves / 2);
        }
        stamp(l, 5);

        if (has_expert) {
            // -- P4: gate/up rows on waves 0-3 while the down rows still stream --
            if (wave < kWaves / 2) __builtin_amdgcn_s_waitcnt(0);
            lds_barrier();
            stamp(l, 6);
            if (wave < kWaves / 2) {
                for (int pr = grp; pr < 2 * R; pr += kThreads / 16) {
                    const int mat = pr >= R, row = pr - mat * R;
                    const float v = mat ? g8_row(L.up_type, smem + S.up + ou + row * rbu, q8x, nb, t8)
                                        : g8_row(L.gate_type, smem + S.gate + og + row * rbg, q8x, nb, t8);
                    if (t8 == 0) gu[pr] = v;
                }
            } else {
                __builtin_amdgcn_s_waitcnt(0);  // down rows landed
            }
            __syncthreads();
            if (tid < R) {
                const float g = gu[tid], uu = gu[R + tid];
                st_l2(Hx + rank * R + tid, tag(g / (1.0f + expf(-g)) * uu, seq + 1u));
            }
            stamp(l, 7);

            // -- P5: Q8_K(h) of the XCD's expert, down rows, publish y rows --
            if (wave < nbh) {
                uint64_t w[4];
                const uint64_t *hsrc = Hx + wave * QK + 4 * lane;
                const bool got = poll(
                    [&]() {
                        bool r = true;
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            w[c] = ld_l2(hsrc + c);
                            r = r && tag_seq(w[c]) == seq + 1u;
                        }
                        return (bool)__all(r);
                    },
                    a.err);
                if (!got && lane == 0) sh_fail = 1;
                const float v[4] = {tag_val(w[0]), tag_val(w[1]), tag_val(w[2]), tag_val(w[3])};
                wave_quantize_q8l_regs(v, &q8h[wave]);
            }
            __syncthreads();
            if (sh_fail) {
                ok = false;
                break;
            }
            stamp(l, 8);
            for (int row = grp; row < RD; row += kThreads / 8) {
                const float y = g8_row(L.down_type, smem + S.down + od + row * rbd, q8h, nbh, t8);
                if (t8 == 0) ys[row] = y;
            }
            __syncthreads();
            if (wave == 0) {
                uint64_t *Y = a.Y + ((size_t)cur * kXcds + xcc) * n + rank * RD;
                for (int i = lane; i < RD; i += 64) st_dev64(Y + i, tag(ys[i], seq + 2u));
            }
            stamp(l, 9);
        }
        // next layer's router rows, from waves that touch no other memory before then
        if (!last && wave >= kWaves / 2) prefetch_router(l + 1, kWaves / 2, kWaves / 2);

        // -- P6 (wave 0): combine rows [RD*rank, RD*rank+RD) over every expert slot --
        if (wave == 0) {
            for (int t = lane; t < RD; t += 64) {
                const int d = rank * RD + t;
                const float res = xs[d];
                uint64_t yw[8];
                const bool got = poll(
                    [&]() {
                        bool r = true;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            if (j < k) {
                                yw[j] = ld_dev64(a.Y + ((size_t)cur * kXcds + j) * n + d);
                                r = r && tag_seq(yw[j]) == seq + 2u;
                            }
                        }
                        return r;
                    },
                    a.err);
                if (!got) sh_fail = 1;
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j < k) acc = acc + w_s[j] * tag_val(yw[j]);
                const float o = acc + res;
                if (last) {
                    if (xcc == 0) a.x[d] = o;
                } else {
                    st_l2(a.X + ((size_t)(cur ^ 1) * kXcds + xcc) * n + d, tag(o, seq + 3u));
                }
            }
        }
        stamp(l, 10);
        stamp(l, 11);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if ((!ok || sh_fail) && xcc == 0) {  // poison this workgroup's output rows so the caller sees the failure
        for (int t = tid; t < RD; t += kThreads) a.x[rank * RD + t] = __builtin_nanf("");
    }
}

}  // namespace

size_t persistent_lds_bytes(const PersistentArgs &a) {
    size_t total = 0;
    smem_layout(a, &total);
    return total;
}

hipError_t launch_persistent_decode(const PersistentArgs &a, hipStream_t s) {
    const size_t lds = persistent_lds_bytes(a);
    if (lds > kPersistentMaxLds) return hipErrorInvalidConfiguration;
    static int attr_bytes = -1;
    if (attr_bytes != (int)lds) {
        hipError_t e = hipFuncSetAttribute((const void *)decode_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_bytes = (int)lds;
    }
    PersistentArgs args = a;
    void *params[] = {&args};
    return hipLaunchCooperativeKernel((const void *)decode_kernel, dim3(kXcds * kPerXcd), dim3(kThreads), params,
                                      (unsigned)lds, s);
}

}  // namespace hoard
