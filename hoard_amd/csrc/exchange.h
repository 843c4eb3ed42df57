// Cross-workgroup exchange words for the persistent decode kernels.
//
// A value travels with the sequence number of the step that produced it in
// one aligned 8-byte word {float bits, seq}, so a consumer polls the data
// itself instead of a separate flag, and words left over from earlier steps
// or launches never match.  Every wait is bounded: on a wall-clock timeout
// the waiter raises a device-wide error flag, and every other wait returns
// once it sees the flag.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hoard {

constexpr long long kTimeoutTicks = 20000000;  // default bound of a wait: 200 ms at the 100 MHz wall clock

__device__ __forceinline__ unsigned xcc_id() {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 7u;
}

__device__ __forceinline__ unsigned ld_dev_u32(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_dev_u32(unsigned *p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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
// Device-wide words: the store writes past the XCD's L2, the load skips it,
// so the pair works between any two CUs of the device.
__device__ __forceinline__ void st_dev64(uint64_t *p, uint64_t w) {
    __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_dev64(const uint64_t *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Four consecutive words at base + off_bytes (16-byte aligned), read past the
// L2 like ld_dev64 (cache policy sc1) in one 16-byte buffer load, where four
// 4-byte loads of lanes 16 bytes apart would each touch every line of the
// span.  base must be the same in every lane (the buffer descriptor lives in
// scalar registers); offsets at or past span_bytes read as zero.
__device__ __forceinline__ float4 ld_dev_f4(const float *base, unsigned span_bytes, unsigned off_bytes) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, (int)span_bytes, 0x00020000);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off_bytes, 0, 16 /* sc1 */);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
}

// Two consecutive tagged words base[i], base[i + 1] (i even, base 16-byte
// aligned), read as ld_l2 / ld_dev64 read one (cache policy sc1) in one
// 16-byte load; each aligned 8-byte word comes whole from the one transfer.
// base must be the same in every lane; words at or past span_words read as 0.
__device__ __forceinline__ void ld_dev64x2(const uint64_t *base, unsigned span_words, unsigned i, uint64_t &w0,
                                           uint64_t &w1) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t *>(base), 0, (int)(span_words * 8u), 0x00020000);
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(i * 8u), 0, 16 /* sc1 */);
    w0 = ((uint64_t)v[1] << 32) | v[0];
    w1 = ((uint64_t)v[3] << 32) | v[2];
}

// Sequence base of a one-launch decode, kept in device memory so that a
// launch needs no host-side state and a launch replayed from a captured
// graph tags its words afresh: seq[0] holds the base of the next launch,
// seq[1] counts finished workgroups.  Every workgroup reads the base when it
// starts; the last of a launch's `groups` workgroups to finish moves it past
// every tag the launch used.  The next launch on the stream starts after this
// one has ended, so it reads the moved base.
__device__ __forceinline__ unsigned seq_begin(const unsigned *seq) { return ld_dev_u32(seq); }
__device__ __forceinline__ void seq_end(unsigned *seq, unsigned base, unsigned used, unsigned groups) {
    const unsigned done = __hip_atomic_fetch_add(seq + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    if (done % groups == 0u) st_dev_u32(seq, base + used);
}

// Bounded poll: true once ready() holds; false on timeout (`limit` ticks of
// the 100 MHz wall clock) or a raised error.  The flag and the clock are
// checked every 32 probes; a limit of 0 gives up at the first probe that finds
// the data missing (the host forces the failure path that way).
template <class F>
__device__ __forceinline__ bool poll(F ready, int *err, long long limit) {
    const long long t0 = wall_clock64();
    for (int it = 0;; ++it) {
        if (ready()) return true;
        if ((it & 31) == 31 || limit == 0) {
            if (ld_dev_u32((const unsigned *)err) != 0u) return false;
            if (wall_clock64() - t0 >= limit) {
                st_dev_u32((unsigned *)err, 1u);
                return false;
            }
        }
    }
}

// Bounded poll with two probes in flight: probe(buf) issues N loads into buf
// and landed(buf) checks them; the next probe is issued before the previous
// one is checked, so a probe starts every half round trip.  The probes
// alternate between two buffers (a copy out of the one in flight would wait
// for it); the probe's loads must not sit behind branches, or the compiler
// waits for both.  On success the landed probe is copied to out.
template <int N, class P, class C>
__device__ __forceinline__ bool poll2(P probe, C landed, uint64_t (&out)[N], int *err, long long limit) {
    uint64_t pa[N], pb[N];
    probe(pa);
    return poll(
        [&]() {
            probe(pb);
            if (landed(pa)) {
#pragma unroll
                for (int i = 0; i < N; ++i) out[i] = pa[i];
                return true;
            }
            probe(pa);
            if (landed(pb)) {
#pragma unroll
                for (int i = 0; i < N; ++i) out[i] = pb[i];
                return true;
            }
            return false;
        },
        err, limit);
}

}  // namespace hoard
