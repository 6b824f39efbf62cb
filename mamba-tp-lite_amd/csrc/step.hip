// Single-token selective state update and residual+RMSNorm for gfx950.
//
// mtl_selective_state_update replaces model.py:280-292 (after x_proj):
//   dt = softplus(dt_low . W_dt[d] + b_dt[d]); dA = exp(dt*A);
//   h <- h*dA + (dt*B)*x (in place, the graph-stable cache buffer, 289);
//   y = sum_n h*C + D*x; y *= silu(z).
// Sixteen lanes serve one channel: lane n owns state n and a 1/16 slice of
// the dt_proj dot product; both the dot product and y are 16-lane butterfly
// sums, so a single wavefront updates four channels with no LDS traffic.
//
// mtl_add_rmsnorm replaces the residual add of MambaBlock (model.py:306,
// 311) fused with the following RMSNorm (model.py:130-135).

#include "common.h"

namespace mtl {
namespace {

constexpr int kLanesPerChannel = 16;
constexpr int kStepThreads = 256;
constexpr int kChPerBlock = kStepThreads / kLanesPerChannel;

template <typename T>
__global__ void __launch_bounds__(kStepThreads)
ssm_step_kernel(float* __restrict__ state, const T* __restrict__ x, int64_t x_sb, const T* __restrict__ z,
                int64_t z_sb, const T* __restrict__ xdbl, int64_t xdbl_sb, const float* __restrict__ Wdt,
                const float* __restrict__ bdt, const float* __restrict__ A, const float* __restrict__ Dv,
                T* __restrict__ y, int64_t y_sb, int D, int N, int R, int a_is_log) {
    const int g = threadIdx.x / kLanesPerChannel;
    const int n = threadIdx.x % kLanesPerChannel;
    const int c = blockIdx.x * kChPerBlock + g;
    const int b = blockIdx.y;
    if (c >= D) return;  // uniform over the 16-lane group

    const T* xd = xdbl + b * xdbl_sb;
    float acc = 0.f;
    for (int r = n; r < R; r += kLanesPerChannel)
        acc = fmaf(Wdt[(int64_t)c * R + r], Act<T>::load(xd + r), acc);
    acc = group_sum<kLanesPerChannel>(acc);
    const float dt = softplus_f(acc + bdt[c]);
    const float xv = Act<T>::load(x + b * x_sb + c);

    float yv = 0.f;
    if (n < N) {
        float av = A[(int64_t)c * N + n];
        if (a_is_log) av = -expf(av);
        const float dA = __builtin_amdgcn_exp2f(dt * (av * kLog2e));
        const float Bn = Act<T>::load(xd + R + n);
        const float Cn = Act<T>::load(xd + R + N + n);
        float* sp = state + ((int64_t)b * D + c) * N + n;
        const float hv = fmaf(*sp, dA, (dt * Bn) * xv);
        *sp = hv;
        yv = hv * Cn;
    }
    yv = group_sum<kLanesPerChannel>(yv);
    if (n == 0) {
        if (Dv) yv += xv * Dv[c];
        if (z) yv *= silu_f(Act<T>::load(z + b * z_sb + c));
        Act<T>::store(y + b * y_sb + c, yv);
    }
}

constexpr int kNormThreads = 256;

__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ y, float* x_out,
                   const float* __restrict__ w, float* __restrict__ normed, int cols, float eps) {
    __shared__ float s_part[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const float* xr = x + row * cols;
    const float* yr = y ? y + row * cols : nullptr;
    float* xo = x_out ? x_out + row * cols : nullptr;
    float ss = 0.f;
    for (int i = threadIdx.x; i < cols; i += kNormThreads) {
        float v = xr[i];
        if (yr) v += yr[i];
        ss = fmaf(v, v, ss);
    }
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot += s_part[i];
    const float r = rsqrtf(tot / (float)cols + eps);
    for (int i = threadIdx.x; i < cols; i += kNormThreads) {
        float v = xr[i];
        if (yr) v += yr[i];
        if (xo) xo[i] = v;
        normed[row * cols + i] = w[i] * (v * r);
    }
}

}  // namespace
}  // namespace mtl

extern "C" int mtl_selective_state_update(float* ssm_state, const void* x, int64_t x_sb, const void* z, int64_t z_sb,
                                          const void* x_dbl, int64_t xdbl_sb, const float* W_dt, const float* b_dt,
                                          const float* A, const float* Dvec, void* y, int64_t y_sb, int64_t batch,
                                          int64_t dim, int64_t dstate, int64_t dt_rank, int32_t dtype,
                                          int32_t a_is_log, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch >= 0 && dim >= 0 && dt_rank >= 0, "negative size");
    MTL_REQUIRE(dstate >= 1 && dstate <= kLanesPerChannel, "dstate must be in [1, 16]");
    MTL_REQUIRE(batch <= 65535 && dim < (int64_t(1) << 31) && dt_rank < (int64_t(1) << 31), "size out of range");
    MTL_REQUIRE(dtype == MTL_F32 || dtype == MTL_BF16, "dtype must be MTL_F32 or MTL_BF16");
    if (batch == 0 || dim == 0) return MTL_OK;
    MTL_REQUIRE(ssm_state && x && x_dbl && W_dt && b_dt && A && y, "null required pointer");
    hipStream_t st = as_stream(stream);
    dim3 grid((unsigned)((dim + kChPerBlock - 1) / kChPerBlock), (unsigned)batch);
    if (dtype == MTL_F32)
        hipLaunchKernelGGL((ssm_step_kernel<float>), grid, dim3(kStepThreads), 0, st, ssm_state,
                           static_cast<const float*>(x), x_sb, static_cast<const float*>(z), z_sb,
                           static_cast<const float*>(x_dbl), xdbl_sb, W_dt, b_dt, A, Dvec, static_cast<float*>(y),
                           y_sb, (int)dim, (int)dstate, (int)dt_rank, a_is_log);
    else
        hipLaunchKernelGGL((ssm_step_kernel<uint16_t>), grid, dim3(kStepThreads), 0, st, ssm_state,
                           static_cast<const uint16_t*>(x), x_sb, static_cast<const uint16_t*>(z), z_sb,
                           static_cast<const uint16_t*>(x_dbl), xdbl_sb, W_dt, b_dt, A, Dvec,
                           static_cast<uint16_t*>(y), y_sb, (int)dim, (int)dstate, (int)dt_rank, a_is_log);
    return check_launch("selective_state_update");
}

extern "C" int mtl_add_rmsnorm(const float* x, const float* y, float* x_out, const float* w, float* normed,
                               int64_t rows, int64_t cols, float eps, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(rows >= 0 && cols >= 1 && cols < (int64_t(1) << 31), "size out of range");
    MTL_REQUIRE(rows < (int64_t(1) << 31), "too many rows");
    if (rows == 0) return MTL_OK;
    MTL_REQUIRE(x && w && normed, "null required pointer");
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, as_stream(stream), x, y,
                       x_out, w, normed, (int)cols, eps);
    return check_launch("add_rmsnorm");
}
