// AllReduce payload quantizers, run locally on one GPU (gfx950).
//
// int8 per token replaces mamba-tp-lite tp_utils.py:103-131 (_int8_gather,
// per_token=True): per row scale = max(amax, 1e-8) / 127, codes =
// clamp(round_half_even(x / scale), +-127), payload = [scales || codes],
// then the rank-ordered dequantize-sum out = (0 + q0*s0) + q1*s1 + ...
// fp16 replaces tp_utils.py:31-42: cast each partial to fp16, sum in fp16,
// cast back.
//
// Bit-exactness: the division is IEEE binary32 (hipcc's default correctly
// rounded fp32 divide; this file must never be built with fast-math), rint
// is round-half-to-even, and the dequantize-sum runs with FP contraction off
// so every q*s and every + rounds once, as torch's separate CPU ops do.
// amax is a max of absolute values: order-independent, hence exact.  It is
// taken on the bit patterns of |x| as unsigned words, so a NaN in the row
// makes amax NaN, as torch's amax does (tp_utils.py:111); the clamp at 1e-8
// keeps the NaN (torch.clamp does), the row's scale is NaN and its outputs
// are NaN.  An infinite element makes the row's scale inf: its finite
// elements quantize to 0, its own quotient inf / inf is NaN, and every
// output of the row is 0 * inf = NaN, as in the reference.  The clamp of the
// codes keeps a NaN quotient NaN (torch.clamp does), and a NaN code is
// written as byte 0: the reference's float -> int8 conversion of NaN has no
// defined value, and 0 is what x86 and GPU conversions give for it.

#include "common.h"

namespace mtl {
namespace {

// Payloads and outputs are written with nontemporal stores: they are
// written once and read by a later kernel (or the wire), and streaming them
// past the caches took two [32768, 768] partials from 64.8 to 57.2 us (int8)
// and from 73.0 to 56.3 us (fp16).
constexpr int kMaxParts = 8;

// clamp(round_half_even(x / s), -127, 127), a NaN quotient kept NaN
__device__ __forceinline__ float int8_code(float x, float s) {
    const float r = rintf(x / s);
    return r < -127.f ? -127.f : (r > 127.f ? 127.f : r);
}
// the payload byte of a code; a NaN code is written as 0
__device__ __forceinline__ uint32_t int8_byte(float q) {
    return q == q ? (uint32_t)(uint8_t)(int8_t)(int)q : 0u;
}
constexpr int kQThreads = 256;          // 4 wavefronts, one row each
constexpr int kRowsPerBlock = kQThreads / 64;
constexpr int kMaxColsPerLane = 32;     // cols <= 2048 keeps the row in registers

struct PartPtrs {
    const float* p[kMaxParts];
    uint8_t* pay[kMaxParts];
    uint16_t* pay16[kMaxParts];
};

template <int PER_LANE>
__global__ void __launch_bounds__(kQThreads)
quant_int8_tok_kernel(PartPtrs pp, int nparts, int64_t rows, int cols, float* __restrict__ out) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;  // uniform over the wavefront
    const int64_t base = row * cols;

    float acc[PER_LANE];
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) acc[j] = 0.f;

    for (int r = 0; r < nparts; ++r) {
        const float* src = pp.p[r] + base;
        float v[PER_LANE];
        uint32_t abits = 0;
#pragma unroll
        for (int j = 0; j < PER_LANE; ++j) {
            const int col = lane + 64 * j;
            v[j] = col < cols ? src[col] : 0.f;
            abits = max(abits, abs_bits(v[j]));
        }
        const float amax = __uint_as_float(group_umax<64>(abits));
        const float scale = (amax < 1e-8f ? 1e-8f : amax) / 127.0f;
        uint8_t* pay = pp.pay[r];
        if (pay && lane == 0) reinterpret_cast<float*>(pay)[row] = scale;  // 4*rows scale bytes first
#pragma unroll
        for (int j = 0; j < PER_LANE; ++j) {
            const int col = lane + 64 * j;
            const float q = int8_code(v[j], scale);
            if (col < cols) {
                if (pay) __builtin_nontemporal_store((uint8_t)int8_byte(q), pay + 4 * rows + base + col);
                acc[j] = acc[j] + q * scale;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) {
        const int col = lane + 64 * j;
        if (col < cols) __builtin_nontemporal_store(acc[j], out + base + col);
    }
}

// The same arithmetic with four adjacent columns per lane (cols % 4 == 0,
// 16-byte aligned rows): float4 loads, the four codes of a lane packed into
// one 4-byte store (a wavefront writes whole 256-byte runs of the payload,
// where one byte per lane wrote partial lines), float4 output stores.
template <int PER4>
__global__ void __launch_bounds__(kQThreads)
quant_int8_tok_vec_kernel(PartPtrs pp, int nparts, int64_t rows, int cols, float* __restrict__ out) {
#pragma clang fp contract(off)
    typedef float F4 __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;  // uniform over the wavefront
    const int64_t base = row * cols;
    const int cols4 = cols >> 2;

    float acc[PER4][4];
#pragma unroll
    for (int j = 0; j < PER4; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[j][k] = 0.f;

    for (int r = 0; r < nparts; ++r) {
        const F4* src = reinterpret_cast<const F4*>(pp.p[r] + base);
        F4 v[PER4];
        uint32_t abits = 0;
#pragma unroll
        for (int j = 0; j < PER4; ++j) {
            const int c4 = lane + 64 * j;
            v[j] = c4 < cols4 ? src[c4] : F4{0.f, 0.f, 0.f, 0.f};
            abits = max(abits, max(max(abs_bits(v[j].x), abs_bits(v[j].y)), max(abs_bits(v[j].z), abs_bits(v[j].w))));
        }
        const float amax = __uint_as_float(group_umax<64>(abits));
        const float scale = (amax < 1e-8f ? 1e-8f : amax) / 127.0f;
        uint8_t* pay = pp.pay[r];
        if (pay && lane == 0) reinterpret_cast<float*>(pay)[row] = scale;  // 4*rows scale bytes first
#pragma unroll
        for (int j = 0; j < PER4; ++j) {
            const int c4 = lane + 64 * j;
            if (c4 < cols4) {
                float q[4];
                uint32_t packed = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    q[k] = int8_code(v[j][k], scale);
                    packed |= int8_byte(q[k]) << (8 * k);
                    acc[j][k] = acc[j][k] + q[k] * scale;
                }
                if (pay) __builtin_nontemporal_store(packed, reinterpret_cast<uint32_t*>(pay + 4 * rows + base) + c4);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < PER4; ++j) {
        const int c4 = lane + 64 * j;
        if (c4 < cols4)
            __builtin_nontemporal_store(F4{acc[j][0], acc[j][1], acc[j][2], acc[j][3]},
                                        reinterpret_cast<F4*>(out + base) + c4);
    }
}

// Rows wider than the register tile: the row is re-read from HBM (L2) for
// every pass instead of held in registers.
__global__ void __launch_bounds__(kQThreads)
quant_int8_tok_wide_kernel(PartPtrs pp, int nparts, int64_t rows, int cols, float* __restrict__ out) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t base = row * cols;
    for (int r = 0; r < nparts; ++r) {
        const float* src = pp.p[r] + base;
        uint32_t abits = 0;
        for (int col = lane; col < cols; col += 64) abits = max(abits, abs_bits(src[col]));
        const float amax = __uint_as_float(group_umax<64>(abits));
        const float scale = (amax < 1e-8f ? 1e-8f : amax) / 127.0f;
        uint8_t* pay = pp.pay[r];
        if (pay && lane == 0) reinterpret_cast<float*>(pay)[row] = scale;
        for (int col = lane; col < cols; col += 64) {
            const float q = int8_code(src[col], scale);
            if (pay) pay[4 * rows + base + col] = (uint8_t)int8_byte(q);
            const float prev = r == 0 ? 0.f : out[base + col];
            out[base + col] = prev + q * scale;
        }
    }
}

__global__ void __launch_bounds__(256)
fp16_sum_kernel(PartPtrs pp, int nparts, int64_t n, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    _Float16 acc = (_Float16)pp.p[0][i];
    if (pp.pay16[0]) reinterpret_cast<_Float16*>(pp.pay16[0])[i] = acc;
    for (int r = 1; r < nparts; ++r) {
        const _Float16 lo = (_Float16)pp.p[r][i];
        if (pp.pay16[r]) reinterpret_cast<_Float16*>(pp.pay16[r])[i] = lo;
        acc = (_Float16)((float)acc + (float)lo);
    }
    out[i] = (float)acc;
}

// Four elements per thread: float4 loads of every part issued first, 8-byte
// fp16 payload stores, float4 output.  Same roundings as fp16_sum_kernel.
template <int P>
__global__ void __launch_bounds__(256) fp16_sum_vec_kernel(PartPtrs pp, int64_t n4, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    float4 v[P];
#pragma unroll
    for (int r = 0; r < P; ++r) v[r] = reinterpret_cast<const float4*>(pp.p[r])[i];
    _Float16 acc[4];
#pragma unroll
    for (int r = 0; r < P; ++r) {
        const _Float16 lo[4] = {(_Float16)v[r].x, (_Float16)v[r].y, (_Float16)v[r].z, (_Float16)v[r].w};
        if (pp.pay16[r]) {
            typedef _Float16 half4 __attribute__((ext_vector_type(4)));
            half4 h = {lo[0], lo[1], lo[2], lo[3]};
            __builtin_nontemporal_store(h, reinterpret_cast<half4*>(pp.pay16[r]) + i);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = r == 0 ? lo[q] : (_Float16)((float)acc[q] + (float)lo[q]);
    }
    typedef float F4 __attribute__((ext_vector_type(4)));
    const F4 o = {(float)acc[0], (float)acc[1], (float)acc[2], (float)acc[3]};
    __builtin_nontemporal_store(o, reinterpret_cast<F4*>(out) + i);
}

}  // namespace
}  // namespace mtl

extern "C" int mtl_quant_dequant_sum_int8_tok(const float* const* parts, int32_t nparts, int64_t rows, int64_t cols,
                                              uint8_t* const* payloads, float* out, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(parts != nullptr, "null parts array");
    MTL_REQUIRE(nparts >= 1 && nparts <= kMaxParts, "nparts must be in [1, 8]");
    MTL_REQUIRE(rows >= 0 && cols >= 0 && cols < (int64_t(1) << 31), "size out of range");
    MTL_REQUIRE((rows + kRowsPerBlock - 1) / kRowsPerBlock < (int64_t(1) << 31), "too many rows");
    if (rows == 0 || cols == 0) return MTL_OK;
    MTL_REQUIRE(out != nullptr, "null out");
    PartPtrs pp{};
    for (int r = 0; r < nparts; ++r) {
        MTL_REQUIRE(parts[r] != nullptr, "null part pointer");
        pp.p[r] = parts[r];
        pp.pay[r] = payloads ? payloads[r] : nullptr;
    }
    hipStream_t st = as_stream(stream);
    dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const int c = (int)cols;
    const int per_lane = (c + 63) / 64;
    bool vec = c % 4 == 0 && (uintptr_t)out % 16 == 0;
    for (int r = 0; r < nparts; ++r)
        vec = vec && (uintptr_t)pp.p[r] % 16 == 0 && (uintptr_t)pp.pay[r] % 4 == 0;
    const int per4 = (c / 4 + 63) / 64;
    if (vec && per4 <= 8) {
        switch (per4) {
#define MTL_Q8V_CASE(P4) \
    case P4: hipLaunchKernelGGL((quant_int8_tok_vec_kernel<P4>), grid, dim3(kQThreads), 0, st, pp, nparts, rows, c, out); break;
            MTL_Q8V_CASE(1) MTL_Q8V_CASE(2) MTL_Q8V_CASE(3) MTL_Q8V_CASE(4)
            MTL_Q8V_CASE(5) MTL_Q8V_CASE(6) MTL_Q8V_CASE(7) MTL_Q8V_CASE(8)
#undef MTL_Q8V_CASE
        }
    } else if (per_lane <= 4) hipLaunchKernelGGL((quant_int8_tok_kernel<4>), grid, dim3(kQThreads), 0, st, pp, nparts, rows, c, out);
    else if (per_lane <= 8) hipLaunchKernelGGL((quant_int8_tok_kernel<8>), grid, dim3(kQThreads), 0, st, pp, nparts, rows, c, out);
    else if (per_lane <= 16) hipLaunchKernelGGL((quant_int8_tok_kernel<16>), grid, dim3(kQThreads), 0, st, pp, nparts, rows, c, out);
    else if (per_lane <= kMaxColsPerLane) hipLaunchKernelGGL((quant_int8_tok_kernel<kMaxColsPerLane>), grid, dim3(kQThreads), 0, st, pp, nparts, rows, c, out);
    else hipLaunchKernelGGL(quant_int8_tok_wide_kernel, grid, dim3(kQThreads), 0, st, pp, nparts, rows, c, out);
    return check_launch("quant_dequant_sum_int8_tok");
}

extern "C" int mtl_quant_dequant_sum_fp16(const float* const* parts, int32_t nparts, int64_t n,
                                          uint16_t* const* payloads, float* out, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(parts != nullptr, "null parts array");
    MTL_REQUIRE(nparts >= 1 && nparts <= kMaxParts, "nparts must be in [1, 8]");
    MTL_REQUIRE(n >= 0 && (n + 255) / 256 < (int64_t(1) << 31), "size out of range");
    if (n == 0) return MTL_OK;
    MTL_REQUIRE(out != nullptr, "null out");
    PartPtrs pp{};
    for (int r = 0; r < nparts; ++r) {
        MTL_REQUIRE(parts[r] != nullptr, "null part pointer");
        pp.p[r] = parts[r];
        pp.pay16[r] = payloads ? payloads[r] : nullptr;
    }
    bool vec = n % 4 == 0 && (uintptr_t)out % 16 == 0;
    for (int r = 0; r < nparts; ++r)
        vec = vec && (uintptr_t)pp.p[r] % 16 == 0 && (uintptr_t)pp.pay16[r] % 8 == 0;
    hipStream_t st = as_stream(stream);
    if (vec) {
        const int64_t n4 = n / 4;
        const dim3 grid((unsigned)((n4 + 255) / 256));
        switch (nparts) {
#define MTL_FP16_CASE(PP) \
    case PP: hipLaunchKernelGGL((fp16_sum_vec_kernel<PP>), grid, dim3(256), 0, st, pp, n4, out); break;
            MTL_FP16_CASE(1) MTL_FP16_CASE(2) MTL_FP16_CASE(3) MTL_FP16_CASE(4)
            MTL_FP16_CASE(5) MTL_FP16_CASE(6) MTL_FP16_CASE(7) MTL_FP16_CASE(8)
#undef MTL_FP16_CASE
        }
    } else {
        hipLaunchKernelGGL(fp16_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, pp, nparts, n, out);
    }
    return check_launch("quant_dequant_sum_fp16");
}
