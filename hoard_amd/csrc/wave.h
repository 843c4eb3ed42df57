// Wave64 cross-lane primitives on DPP (data-parallel primitives: VALU lane
// permutes with a few cycles of latency) instead of ds_bpermute (an LDS round
// trip per step).  Reductions run as butterflies inside each 16-lane row
// (quad_perm, row_half_mirror, row_mirror); rows are combined through
// v_readlane into wave-uniform values.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hoard {

// DPP controls (gfx9 encoding)
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm:[1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm:[2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowRor4 = 0x124;   // lane i reads lane (i - 4) mod 16 of its row
constexpr int kDppRowRor8 = 0x128;
constexpr int kDppRowRor12 = 0x12C;  // lane i reads lane i + 4
constexpr int kDppRowRor14 = 0x12E;  // lane i reads lane i + 2
constexpr int kDppRowRor15 = 0x12F;  // lane i reads lane i + 1
constexpr int kDppRowBcast15 = 0x142;  // lane 15 of each row to the next row (row_mask picks rows)
constexpr int kDppRowBcast31 = 0x143;  // lane 31 to rows 2 and 3

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = dpp_i<CTRL>((int)(b & 0xffffffffll)), hi = dpp_i<CTRL>((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// The wave's index within its workgroup, in a scalar register: addresses
// formed from it (LDS staging bases, row pointers) stay scalar instead of
// being formed per lane.
__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }
__device__ __forceinline__ int readlane_i(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double readlane_d(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// Sum over each aligned group of 8 lanes; every lane of the group gets it.
__device__ __forceinline__ int group8_sum(int v) {
    v += dpp_i<kDppQuadXor1>(v);
    v += dpp_i<kDppQuadXor2>(v);
    v += dpp_i<kDppRowHalfMirror>(v);
    return v;
}
// Sum over each aligned group of 4 lanes.
__device__ __forceinline__ int group4_sum(int v) {
    v += dpp_i<kDppQuadXor1>(v);
    v += dpp_i<kDppQuadXor2>(v);
    return v;
}

// Row (16-lane) butterflies; every lane of a row ends with the row result.
__device__ __forceinline__ double row16_sum_d(double v) {
    v = v + dpp_d<kDppQuadXor1>(v);
    v = v + dpp_d<kDppQuadXor2>(v);
    v = v + dpp_d<kDppRowHalfMirror>(v);
    v = v + dpp_d<kDppRowMirror>(v);
    return v;
}
// v_max_f32 (fmaxf) per step, one instruction where a compare and a select
// were two on the dependent chain; a NaN lane never wins unless every lane is
// NaN (the callers sanitise or only meet all-NaN inputs).
__device__ __forceinline__ float row16_max_f(float v) {
    v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
    v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
    v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
    v = fmaxf(v, dpp_f<kDppRowMirror>(v));
    return v;
}

// Wave-uniform results (rows combined in lane order 0, 16, 32, 48).
__device__ __forceinline__ double wave_sum_d(double v) {
    v = row16_sum_d(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
__device__ __forceinline__ float wave_max_f(float v) {
    v = row16_max_f(v);
    const float a = readlane_f(v, 0), b = readlane_f(v, 16), c = readlane_f(v, 32), d = readlane_f(v, 48);
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Wave-uniform argmax of (value, index): larger value first, lower index on
// ties; lanes without a candidate pass idx = INT_MAX.  NaN never wins.
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
    if (bi == 0x7fffffff) return ai != 0x7fffffff;
    if (ai == 0x7fffffff) return false;
    return av > bv || (av == bv && ai < bi);
}
template <int CTRL>
__device__ __forceinline__ void argmax_step(float &v, int &i) {
    const float ov = dpp_f<CTRL>(v);
    const int oi = dpp_i<CTRL>(i);
    if (better(ov, oi, v, i)) {
        v = ov;
        i = oi;
    }
}
__device__ __forceinline__ void wave_argmax(float &v, int &i) {
    argmax_step<kDppQuadXor1>(v, i);
    argmax_step<kDppQuadXor2>(v, i);
    argmax_step<kDppRowHalfMirror>(v, i);
    argmax_step<kDppRowMirror>(v, i);
    float bv = readlane_f(v, 0);
    int bi = readlane_i(i, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) {
        const float ov = readlane_f(v, r);
        const int oi = readlane_i(i, r);
        if (better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    v = bv;
    i = bi;
}

// ggml's x86 f32 dot fold for one row held by 16 lanes, lane l owning the
// partial sums of accumulators l and l+16 (already added in-lane as the first
// fold step): then +8 lanes, +4 lanes, pairs, halves.  Exact in lane 0 of the
// row; other lanes hold partial garbage.
__device__ __forceinline__ float row16_ggml_fold(float a) {
    a = a + dpp_f<kDppRowRor8>(a);
    a = a + dpp_f<kDppRowRor4>(a);
    a = a + dpp_f<kDppQuadXor1>(a);
    a = a + dpp_f<kDppQuadXor2>(a);
    return a;
}

// The same fold for a row held by 8 lanes, lane m owning accumulators
// 4m..4m+3 (elements 32i + 4m + c): +16 accumulators is 4 lanes up, +8 is 2,
// +4 is 1; lane 0 of the group then adds its four in the (0+1)+(2+3) order.
// row_ror:n makes lane i read lane (i - n) mod 16, so reading lane i + j is
// row_ror:(16 - j).  Exact in lane 0 of each aligned 8-lane group.
__device__ __forceinline__ float group8_ggml_fold(float a0, float a1, float a2, float a3) {
    a0 = a0 + dpp_f<kDppRowRor12>(a0);
    a1 = a1 + dpp_f<kDppRowRor12>(a1);
    a2 = a2 + dpp_f<kDppRowRor12>(a2);
    a3 = a3 + dpp_f<kDppRowRor12>(a3);
    a0 = a0 + dpp_f<kDppRowRor14>(a0);
    a1 = a1 + dpp_f<kDppRowRor14>(a1);
    a2 = a2 + dpp_f<kDppRowRor14>(a2);
    a3 = a3 + dpp_f<kDppRowRor14>(a3);
    a0 = a0 + dpp_f<kDppRowRor15>(a0);
    a1 = a1 + dpp_f<kDppRowRor15>(a1);
    a2 = a2 + dpp_f<kDppRowRor15>(a2);
    a3 = a3 + dpp_f<kDppRowRor15>(a3);
    return (a0 + a1) + (a2 + a3);
}

}  // namespace hoard
