// Shared device helpers and host-side error plumbing for libmtl (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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
__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(uint32_t(v) << 16); }
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return uint16_t(u >> 16);
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

// torch softplus (beta 1, threshold 20): x above 20, else log1p(exp(x)).
// For e = exp(x) < 1/32 log1p(e) is the alternating series to e^4 (relative
// truncation error < e^4/5 < 2e-7); above it log2(1 + e) * ln2, where
// 1 + e >= 1.03 keeps the hardware log's error relative to the result small.
__device__ __forceinline__ float softplus_f(float x) {
    const float e = fast_exp(fminf(x, 20.f));
    const float series = e * (1.f - e * (0.5f - e * (0.33333334f - e * 0.25f)));
    const float viaLog = __builtin_amdgcn_logf(1.f + e) * kLn2;
    const float r = e < 0.03125f ? series : viaLog;
    return x > 20.f ? x : r;
}

// x * sigmoid(x)
__device__ __forceinline__ float silu_f(float x) {
    return x * __builtin_amdgcn_rcpf(1.f + fast_exp(-x));
}

// Butterfly reductions inside a wavefront (64 lanes) or a power-of-two
// group of lanes; __shfl_xor lowers to ds_swizzle / DPP on gfx950.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, WIDTH);
    return v;
}
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WIDTH));
    return v;
}

}  // namespace mtl
