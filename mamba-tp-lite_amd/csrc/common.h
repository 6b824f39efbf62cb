// Shared device helpers and host-side error plumbing for libmtl (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <string>

#include "mtl.h"

namespace mtl {

// ---------------------------------------------------------------- host side
void set_error(const std::string& msg);
void clear_error();

#define MTL_REQUIRE(cond, msg)                                               \
    do {                                                                     \
        if (!(cond)) {                                                       \
            ::mtl::set_error(std::string(__func__) + ": " + (msg));          \
            return MTL_EINVAL;                                               \
        }                                                                    \
    } while (0)

// Checks the launch that was just enqueued.
int check_launch(const char* what);

inline hipStream_t as_stream(mtl_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------- device side
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// bf16 <-> fp32 (round to nearest even, NaN kept quiet)
// fp32 -> bf16 is gfx950's v_cvt_pk_bf16_f32 (round to nearest even; a pair
// per instruction where two values convert together).
__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
    typedef float F2 __attribute__((ext_vector_type(2)));
    typedef __bf16 B2 __attribute__((ext_vector_type(2)));
    const F2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, B2));
}

template <typename T> struct Act;
template <> struct Act<float> {
    __device__ __forceinline__ static float load(const float* p) { return *p; }
    __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
};
template <> struct Act<uint16_t> {  // bf16 storage
    __device__ __forceinline__ static float load(const uint16_t* p) { return bf16_to_f32(*p); }
    __device__ __forceinline__ static void store(uint16_t* p, float v) { *p = f32_to_bf16(v); }
};

// exp(x) through the hardware base-2 exponential.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

// softplus in log2 units: softplus(x) * log2(e) from xl = x * log2(e), as
//   max(xl, 0) + log2(1 + e),  e = 2^-|xl|  (= log2(1 + 2^xl) for either sign).
// 1 + e rounds; its rounding error d = e - ((1 + e) - 1) is exact and is put
// back as d * log2(e) (the first-order term of log2(1 + d / (1 + e)); the
// neglected factor 1 / (1 + e) changes the result by < 2^-24 relative).
// Measured on gfx950 against float64 over x in [-30, 30]: relative error
// under 7e-7 for x in [-8, -2], where the dt of a Mamba layer lives, and
// under 2e-6 everywhere the result is a normal float.  Above x = 20 torch's
// softplus returns x; here x + log1p(e^-x) has rounded to x from x = 16 on.
// A NaN input gives NaN, as torch's does.
// A scan that keeps dt in these units takes exp(dt * A) as exp2(dt_l2 * A).
__device__ __forceinline__ float softplus_l2_f(float xl) {
    const float e = __builtin_amdgcn_exp2f(-fabsf(xl));
    const float u = 1.f + e;
    const float d = e - (u - 1.f);
    return fmaxf(xl, 0.f) + fmaf(d, kLog2e, __builtin_amdgcn_logf(u));
}

// torch softplus (beta 1, threshold 20), through softplus_l2_f.
__device__ __forceinline__ float softplus_f(float x) {
    return softplus_l2_f(x * kLog2e) * kLn2;
}

// x * sigmoid(x)
__device__ __forceinline__ float silu_f(float x) {
    return x * __builtin_amdgcn_rcpf(1.f + fast_exp(-x));
}

// Reductions over a 16-lane DPP row or a whole 64-lane wavefront, in DPP
// lane moves instead of LDS permutes.  Within a row: butterfly over
// quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror --
// each step combines two values that the partner lane combines in the other
// order, so (with + and max commutative) every lane ends with the same bits.
// Across rows: lanes 0, 16, 32, 48 are read out and combined as
// (r0 + r1) + (r2 + r3).  Callers keep whole rows (whole wavefronts for the
// 64-wide forms) active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_read(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRowMirror = 0x140, kDppHalfMirror = 0x141;
constexpr int kDppWaveShr1 = 0x138;   // lane i takes lane i - 1 (gfx9 wave_shr:1); lane 0 keeps its old value

template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(WIDTH == 16 || WIDTH == 64, "16 or 64 lanes");
    v += dpp_mov<kDppXor1>(v);
    v += dpp_mov<kDppXor2>(v);
    v += dpp_mov<kDppHalfMirror>(v);
    v += dpp_mov<kDppRowMirror>(v);
    if constexpr (WIDTH == 64) v = (lane_read(v, 0) + lane_read(v, 16)) + (lane_read(v, 32) + lane_read(v, 48));
    return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
    static_assert(WIDTH == 16 || WIDTH == 64, "16 or 64 lanes");
    v = fmaxf(v, dpp_mov<kDppXor1>(v));
    v = fmaxf(v, dpp_mov<kDppXor2>(v));
    v = fmaxf(v, dpp_mov<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_mov<kDppRowMirror>(v));
    if constexpr (WIDTH == 64) v = fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
    return v;
}

// Max over a 16- or 64-lane group of unsigned words (same lane moves as
// group_max).  On the bit patterns of |x| (sign cleared) this is a float max
// that returns NaN when any input is NaN -- fmaxf would drop it.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ uint32_t lane_read_u(uint32_t v, int lane) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}
template <int WIDTH>
__device__ __forceinline__ uint32_t group_umax(uint32_t v) {
    static_assert(WIDTH == 16 || WIDTH == 64, "16 or 64 lanes");
    v = max(v, dpp_mov_u<kDppXor1>(v));
    v = max(v, dpp_mov_u<kDppXor2>(v));
    v = max(v, dpp_mov_u<kDppHalfMirror>(v));
    v = max(v, dpp_mov_u<kDppRowMirror>(v));
    if constexpr (WIDTH == 64)
        v = max(max(lane_read_u(v, 0), lane_read_u(v, 16)), max(lane_read_u(v, 32), lane_read_u(v, 48)));
    return v;
}
__device__ __forceinline__ uint32_t abs_bits(float x) { return __float_as_uint(x) & 0x7fffffffu; }

// Fixed-count register blocking: kernels that hold RUNS values per lane are
// instantiated for these counts; a size needing `need` runs uses the
// smallest instantiated count >= need (the extra runs are masked).
constexpr int kMaxRuns = 16;
inline int round_runs(int need) {
    for (int p : {1, 2, 3, 4, 6, 8, 12})
        if (p >= need) return p;
    return kMaxRuns;
}
#define MTL_DISPATCH_RUNS(NAME, VALUE, ...)                          \
    switch (VALUE) {                                                 \
        case 1: { constexpr int NAME = 1; __VA_ARGS__; } break;      \
        case 2: { constexpr int NAME = 2; __VA_ARGS__; } break;      \
        case 3: { constexpr int NAME = 3; __VA_ARGS__; } break;      \
        case 4: { constexpr int NAME = 4; __VA_ARGS__; } break;      \
        case 6: { constexpr int NAME = 6; __VA_ARGS__; } break;      \
        case 8: { constexpr int NAME = 8; __VA_ARGS__; } break;      \
        case 12: { constexpr int NAME = 12; __VA_ARGS__; } break;    \
        default: { constexpr int NAME = 16; __VA_ARGS__; } break;    \
    }

}  // namespace mtl
