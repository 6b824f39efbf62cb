// Causal depthwise conv1d (+ SiLU) for gfx950: prefill and single-token step.
//
// Prefill replaces model.py:201-212 (left-pad with the carried conv history
// or zeros, F.conv1d(groups=D) + bias, [..., :l], F.silu, and the final
// conv state = last K-1 padded inputs); the step replaces model.py:264-277
// (conv_in = cat(conv_state, x), sum(conv_in * w) + bias, in-place history
// shift, F.silu).
//
// Prefill mapping: a thread owns one channel and a run of kTC consecutive
// timesteps and slides a K-wide window along l, so each input element is
// read once from HBM (plus a K-1 halo per run).  For the token-major
// layout of the mixer (x a strided view of in_proj's output, stride 1 along
// d) consecutive lanes read consecutive channels: fully coalesced.

#include "common.h"

namespace mtl {
namespace {

constexpr int kConvThreads = 256;
constexpr int kTC = 32;      // timesteps per thread
constexpr int kMaxK = 8;

struct ConvArgs {
    const void* x; void* out; const float* w; const float* bias;
    const void* st_in; void* st_out;
    int64_t x_sb, x_sd, x_sl, o_sb, o_sd, o_sl;
    int L, D, K, silu;
};

template <typename T, int K>
__global__ void __launch_bounds__(kConvThreads) conv_fwd_kernel(const ConvArgs a) {
    const int c = blockIdx.x * kConvThreads + threadIdx.x;
    const int b = blockIdx.z;
    const int t0 = blockIdx.y * kTC;
    if (c >= a.D || t0 >= a.L) return;

    const T* __restrict__ xp = static_cast<const T*>(a.x) + b * a.x_sb + (int64_t)c * a.x_sd;
    T* __restrict__ op = static_cast<T*>(a.out) + b * a.o_sb + (int64_t)c * a.o_sd;
    const T* __restrict__ sin = a.st_in ? static_cast<const T*>(a.st_in) + ((int64_t)b * a.D + c) * (K - 1)
                                        : nullptr;

    float w[K];
#pragma unroll
    for (int k = 0; k < K; ++k) w[k] = a.w[(int64_t)c * K + k];
    const float bias = a.bias ? a.bias[c] : 0.f;

    // padded input xp_pad[i] = state[i] for i < K-1, x[i-(K-1)] otherwise;
    // out[t] needs xp_pad[t .. t+K-1].  win[k] holds xp_pad[t + k].
    auto padded = [&](int i) -> float {
        if (i >= K - 1) return Act<T>::load(xp + (int64_t)(i - (K - 1)) * a.x_sl);
        return sin ? Act<T>::load(sin + i) : 0.f;
    };
    float win[K];
#pragma unroll
    for (int k = 0; k < K - 1; ++k) win[k] = padded(t0 + k);

    const int t1 = min(t0 + kTC, a.L);
    for (int t = t0; t < t1; ++t) {
        win[K - 1] = Act<T>::load(xp + (int64_t)t * a.x_sl);
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) acc = fmaf(w[k], win[k], acc);
        acc += bias;
        if (a.silu) acc = silu_f(acc);
        Act<T>::store(op + (int64_t)t * a.o_sl, acc);
#pragma unroll
        for (int k = 0; k < K - 1; ++k) win[k] = win[k + 1];
    }

    // final conv state: padded positions L .. L+K-2, written by the run that
    // holds the last timestep
    if (a.st_out && t1 == a.L) {
        T* so = static_cast<T*>(a.st_out) + ((int64_t)b * a.D + c) * (K - 1);
#pragma unroll
        for (int k = 0; k < K - 1; ++k) Act<T>::store(so + k, padded(a.L + k));
    }
}

// State-only kernel for l == 0: the history passes through unchanged.
template <typename T>
__global__ void conv_state_copy_kernel(const T* __restrict__ in, T* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = in ? in[i] : T(0);
}

template <typename T, int K>
__global__ void __launch_bounds__(256) conv_step_kernel(T* __restrict__ state, const T* __restrict__ x,
                                                        int64_t x_sb, const float* __restrict__ w,
                                                        const float* __restrict__ bias, T* __restrict__ out,
                                                        int64_t o_sb, int D, int silu) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int b = blockIdx.y;
    if (c >= D) return;
    T* s = state + ((int64_t)b * D + c) * (K - 1);
    float win[K];
#pragma unroll
    for (int k = 0; k < K - 1; ++k) win[k] = Act<T>::load(s + k);
    win[K - 1] = Act<T>::load(x + b * x_sb + c);
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k) acc = fmaf(win[k], w[(int64_t)c * K + k], acc);
    if (bias) acc += bias[c];
    // in-place history shift: conv_state <- conv_in[..., 1:]
#pragma unroll
    for (int k = 0; k < K - 1; ++k) Act<T>::store(s + k, win[k + 1]);
    Act<T>::store(out + b * o_sb + c, silu ? silu_f(acc) : acc);
}

template <typename T>
int launch_conv(const ConvArgs& a, int64_t batch, hipStream_t st) {
    dim3 block(kConvThreads);
    dim3 grid((unsigned)((a.D + kConvThreads - 1) / kConvThreads), (unsigned)((a.L + kTC - 1) / kTC),
              (unsigned)batch);
    switch (a.K) {
#define MTL_CONV_CASE(KK) \
    case KK: hipLaunchKernelGGL((conv_fwd_kernel<T, KK>), grid, block, 0, st, a); break;
        MTL_CONV_CASE(2) MTL_CONV_CASE(3) MTL_CONV_CASE(4) MTL_CONV_CASE(5)
        MTL_CONV_CASE(6) MTL_CONV_CASE(7) MTL_CONV_CASE(8)
#undef MTL_CONV_CASE
        default: set_error("conv width unsupported"); return MTL_EINVAL;
    }
    return check_launch("causal_conv1d_fwd");
}

template <typename T>
int launch_conv_step(void* state, const void* x, int64_t x_sb, const float* w, const float* bias, void* out,
                     int64_t o_sb, int64_t batch, int D, int K, int silu, hipStream_t st) {
    dim3 block(256);
    dim3 grid((unsigned)((D + 255) / 256), (unsigned)batch);
    T* s = static_cast<T*>(state);
    const T* xx = static_cast<const T*>(x);
    T* o = static_cast<T*>(out);
    switch (K) {
#define MTL_STEP_CASE(KK) \
    case KK: hipLaunchKernelGGL((conv_step_kernel<T, KK>), grid, block, 0, st, s, xx, x_sb, w, bias, o, o_sb, D, silu); break;
        MTL_STEP_CASE(2) MTL_STEP_CASE(3) MTL_STEP_CASE(4) MTL_STEP_CASE(5)
        MTL_STEP_CASE(6) MTL_STEP_CASE(7) MTL_STEP_CASE(8)
#undef MTL_STEP_CASE
        default: set_error("conv width unsupported"); return MTL_EINVAL;
    }
    return check_launch("conv_step");
}

}  // namespace
}  // namespace mtl

extern "C" int mtl_causal_conv1d_fwd(const mtl_conv_params* p, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(p != nullptr, "null params");
    MTL_REQUIRE(p->batch >= 0 && p->seqlen >= 0 && p->dim >= 0, "negative size");
    MTL_REQUIRE(p->width >= 2 && p->width <= kMaxK, "width (d_conv) must be in [2, 8]");
    MTL_REQUIRE(p->batch <= 65535, "batch must be <= 65535");
    MTL_REQUIRE(p->seqlen < (int64_t(1) << 31) && p->dim < (int64_t(1) << 31), "size overflows int32");
    MTL_REQUIRE((p->seqlen + kTC - 1) / kTC <= 65535, "seqlen too long for one launch");
    MTL_REQUIRE(p->dtype == MTL_F32 || p->dtype == MTL_BF16, "dtype must be MTL_F32 or MTL_BF16");
    MTL_REQUIRE(p->conv_state_in == nullptr || p->conv_state_in != p->conv_state_out,
                "conv_state_out must not alias conv_state_in");
    if (p->batch == 0 || p->dim == 0) return MTL_OK;
    hipStream_t st = as_stream(stream);
    if (p->seqlen == 0) {
        if (!p->conv_state_out) return MTL_OK;
        const int64_t n = p->batch * p->dim * (p->width - 1);
        const unsigned blocks = (unsigned)((n + 255) / 256);
        if (p->dtype == MTL_F32)
            hipLaunchKernelGGL((conv_state_copy_kernel<float>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const float*>(p->conv_state_in), static_cast<float*>(p->conv_state_out), n);
        else
            hipLaunchKernelGGL((conv_state_copy_kernel<uint16_t>), dim3(blocks), dim3(256), 0, st,
                               static_cast<const uint16_t*>(p->conv_state_in),
                               static_cast<uint16_t*>(p->conv_state_out), n);
        return check_launch("causal_conv1d_fwd(state copy)");
    }
    MTL_REQUIRE(p->x && p->out && p->w, "null required pointer");
    ConvArgs a;
    a.x = p->x; a.out = p->out; a.w = p->w; a.bias = p->bias;
    a.st_in = p->conv_state_in; a.st_out = p->conv_state_out;
    a.x_sb = p->x_sb; a.x_sd = p->x_sd; a.x_sl = p->x_sl;
    a.o_sb = p->out_sb; a.o_sd = p->out_sd; a.o_sl = p->out_sl;
    a.L = (int)p->seqlen; a.D = (int)p->dim; a.K = p->width; a.silu = p->silu;
    return p->dtype == MTL_F32 ? launch_conv<float>(a, p->batch, st) : launch_conv<uint16_t>(a, p->batch, st);
}

extern "C" int mtl_conv_step(void* conv_state, const void* x, int64_t x_sb, const float* w, const float* bias,
                             void* out, int64_t out_sb, int64_t batch, int64_t dim, int32_t width,
                             int32_t dtype, int32_t silu, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch >= 0 && dim >= 0, "negative size");
    MTL_REQUIRE(width >= 2 && width <= kMaxK, "width (d_conv) must be in [2, 8]");
    MTL_REQUIRE(batch <= 65535 && dim < (int64_t(1) << 31), "size out of range");
    MTL_REQUIRE(dtype == MTL_F32 || dtype == MTL_BF16, "dtype must be MTL_F32 or MTL_BF16");
    if (batch == 0 || dim == 0) return MTL_OK;
    MTL_REQUIRE(conv_state && x && w && out, "null required pointer");
    hipStream_t st = as_stream(stream);
    return dtype == MTL_F32
               ? launch_conv_step<float>(conv_state, x, x_sb, w, bias, out, out_sb, batch, (int)dim, width, silu, st)
               : launch_conv_step<uint16_t>(conv_state, x, x_sb, w, bias, out, out_sb, batch, (int)dim, width, silu,
                                            st);
}
