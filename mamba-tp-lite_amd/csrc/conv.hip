// Causal depthwise conv1d (+ SiLU) for gfx950: prefill and single-token step.
//
// Prefill replaces model.py:201-212 (left-pad with the carried conv history
// or zeros, F.conv1d(groups=D) + bias, [..., :l], F.silu, and the final
// conv state = last K-1 padded inputs); the step replaces model.py:264-277
// (conv_in = cat(conv_state, x), sum(conv_in * w) + bias, in-place history
// shift, F.silu).
//
// Prefill mapping: a thread owns 4 adjacent channels (one vector) and a run
// of kTC consecutive timesteps; it loads the kTC + K - 1 inputs of its
// window up front and forms the outputs from registers, so each input
// element is read once from HBM (plus a K-1 halo per run, which the
// neighbouring run has just pulled into L2).  For the token-major layout of
// the mixer (x a strided view of in_proj's output, stride 1 along d)
// consecutive lanes read consecutive vectors: fully coalesced.  Layouts
// without unit channel stride use one channel per thread.

#include <mutex>

#include "common.h"

namespace mtl {
namespace {

constexpr int kConvThreads = 256;
constexpr int kTC = 16;      // timesteps per thread
constexpr int kMaxK = 8;

struct ConvArgs {
    const void* x; void* out; const float* w; const float* bias;
    const void* st_in; void* st_out;
    int64_t x_sb, x_sd, x_sl, o_sb, o_sd, o_sl;
    int L, D, K, silu;
};

// VC adjacent channels as one vector (VC > 1 needs unit channel stride and
// VC-aligned rows), TC timesteps per thread.
template <typename T, int VC> struct Vec;
template <> struct Vec<float, 1> {
    __device__ __forceinline__ static void load(const float* p, float* v) { v[0] = *p; }
    __device__ __forceinline__ static void store(float* p, const float* v) { *p = v[0]; }
};
template <> struct Vec<uint16_t, 1> {
    __device__ __forceinline__ static void load(const uint16_t* p, float* v) { v[0] = bf16_to_f32(*p); }
    __device__ __forceinline__ static void store(uint16_t* p, const float* v) { *p = f32_to_bf16(v[0]); }
};
// The vector stores are nontemporal: the conv output is written once and
// read back by later kernels, and streaming it past the caches took the bf16
// [32, 2048, 2048] conv from 105.7 to 80.7 us (loads stay cached: the next
// run re-reads a K-1 halo, and nontemporal loads made that 107 us).
template <> struct Vec<float, 4> {
    __device__ __forceinline__ static void load(const float* p, float* v) {
        const float4 x = *reinterpret_cast<const float4*>(p);
        v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
    }
    __device__ __forceinline__ static void store(float* p, const float* v) {
        typedef float F4 __attribute__((ext_vector_type(4)));
        const F4 x = {v[0], v[1], v[2], v[3]};
        __builtin_nontemporal_store(x, reinterpret_cast<F4*>(p));
    }
};
template <> struct Vec<uint16_t, 4> {
    __device__ __forceinline__ static void load(const uint16_t* p, float* v) {
        const uint2 x = *reinterpret_cast<const uint2*>(p);
        v[0] = __uint_as_float(x.x << 16); v[1] = __uint_as_float(x.x & 0xffff0000u);
        v[2] = __uint_as_float(x.y << 16); v[3] = __uint_as_float(x.y & 0xffff0000u);
    }
    __device__ __forceinline__ static void store(uint16_t* p, const float* v) {
        uint2 x;
        x.x = f32x2_to_bf16x2(v[0], v[1]);
        x.y = f32x2_to_bf16x2(v[2], v[3]);
        typedef unsigned U2 __attribute__((ext_vector_type(2)));
        const U2 y = {x.x, x.y};
        __builtin_nontemporal_store(y, reinterpret_cast<U2*>(p));
    }
};

// A thread owns VC channels x TC timesteps.  The TC + K - 1 padded inputs
// it needs are loaded up front (clamped addresses; positions before the
// sequence come from the carried history or are zero), then the TC outputs
// are formed from registers.
// CWV channel vectors x (kConvThreads / CWV) consecutive time tiles per
// workgroup (each wavefront one time tile when CWV = 64).
template <typename T, int K, int VC, int TC, int CWV>
__global__ void __launch_bounds__(kConvThreads) conv_fwd_kernel(const ConvArgs a) {
    constexpr int W = TC + K - 1;
    constexpr int TW = kConvThreads / CWV;      // time tiles per workgroup
    // XCD-aware tile order: tiles are numbered (batch row, time tile, channel
    // group), channel group fastest, and workgroups are dealt to the 8 XCDs
    // round robin, so workgroup w takes tile (w % 8) * (tiles / 8) + w / 8.
    // An XCD then walks consecutive time tiles of a row: the K-1 halo a tile
    // re-reads was pulled into the same L2 by the tile before it.
    const int ncg = gridDim.x, ntt = gridDim.y;
    int wl = (blockIdx.z * ntt + blockIdx.y) * ncg + blockIdx.x;
    const int wt = ncg * ntt * gridDim.z;
    if (wt % 8 == 0) wl = (wl % 8) * (wt / 8) + wl / 8;
    const int cg = wl % ncg, tt_i = (wl / ncg) % ntt;
    const int cw = threadIdx.x % CWV, tw = threadIdx.x / CWV;
    const int c0 = (cg * CWV + cw) * VC;
    const int b = wl / (ncg * ntt);
    const int t0 = (tt_i * TW + tw) * TC;
    if (c0 >= a.D || t0 >= a.L) return;

    const T* __restrict__ xp = static_cast<const T*>(a.x) + b * a.x_sb + (int64_t)c0 * a.x_sd;
    T* __restrict__ op = static_cast<T*>(a.out) + b * a.o_sb + (int64_t)c0 * a.o_sd;

    // v[j] = padded input at position t0 + j, i.e. x[t0 + j - (K-1)]
    float v[W][VC];
#pragma unroll
    for (int j = 0; j < W; ++j) {
        const int t = min(max(t0 + j - (K - 1), 0), a.L - 1);
        Vec<T, VC>::load(xp + (int64_t)t * a.x_sl, v[j]);
    }
    float w[K][VC], bias[VC];
#pragma unroll
    for (int ci = 0; ci < VC; ++ci) {
#pragma unroll
        for (int k = 0; k < K; ++k) w[k][ci] = a.w[(int64_t)(c0 + ci) * K + k];
        bias[ci] = a.bias ? a.bias[c0 + ci] : 0.f;
    }
    // padded positions below K-1 are the carried history or zeros; with runs
    // shorter than K-1 they reach past the first run (uniform per wavefront)
    if (t0 < K - 1) {
        const T* __restrict__ sin = a.st_in ? static_cast<const T*>(a.st_in) : nullptr;
#pragma unroll
        for (int j = 0; j < K - 1; ++j) {
            const int p = t0 + j;
            if (p < K - 1)
#pragma unroll
                for (int ci = 0; ci < VC; ++ci)
                    v[j][ci] = sin ? Act<T>::load(sin + ((int64_t)b * a.D + c0 + ci) * (K - 1) + p) : 0.f;
        }
    }

#pragma unroll
    for (int tt = 0; tt < TC; ++tt) {
        if (t0 + tt >= a.L) break;  // uniform per wavefront
        float o[VC];
#pragma unroll
        for (int ci = 0; ci < VC; ++ci) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < K; ++k) acc = fmaf(w[k][ci], v[tt + k][ci], acc);
            acc += bias[ci];
            o[ci] = a.silu ? silu_f(acc) : acc;
        }
        Vec<T, VC>::store(op + (int64_t)(t0 + tt) * a.o_sl, o);
    }

    // final conv state = padded positions L .. L+K-2, held by the block with the last timestep
    if (a.st_out && t0 + TC >= a.L) {
        T* so = static_cast<T*>(a.st_out) + ((int64_t)b * a.D + c0) * (K - 1);
        const int j0 = a.L - t0;  // v index of padded position L
#pragma unroll
        for (int j = 0; j < W; ++j) {
            const int k = j - j0;
            if (k >= 0 && k < K - 1)
#pragma unroll
                for (int ci = 0; ci < VC; ++ci) Act<T>::store(so + (int64_t)ci * (K - 1) + k, v[j][ci]);
        }
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

// Channel vectors per workgroup: fp32 rows take 64 (four time tiles per
// workgroup, one per wavefront), bf16 rows 256 (one time tile).  Measured,
// outputs bit-identical either way: fp32 [32, 4096, 1024] 206.0 -> 186.6 us,
// [1, 1536, 64] 3.93 -> 3.48 us, [32, 1536, 1024] equal; bf16 [32, 2048,
// 2048] 79.5 us with 256 against 82.6 us with 64 (a workgroup then reads a
// whole 4 KB token row).
template <typename T, int VC, int TC>
int launch_conv_vc(const ConvArgs& a, int64_t batch, hipStream_t st) {
    constexpr int CWV = sizeof(T) == 4 ? 64 : kConvThreads, TW = kConvThreads / CWV;
    const int64_t ncg = (a.D / VC + CWV - 1) / CWV, ntb = ((a.L + TC - 1) / TC + TW - 1) / TW;
    MTL_REQUIRE(ncg * ntb * batch < (int64_t(1) << 31), "batch * channel groups * time tiles overflows int32");
    dim3 block(kConvThreads);
    dim3 grid((unsigned)ncg, (unsigned)ntb, (unsigned)batch);
    switch (a.K) {
#define MTL_CONV_CASE(KK) \
    case KK: hipLaunchKernelGGL((conv_fwd_kernel<T, KK, VC, TC, CWV>), grid, block, 0, st, a); break;
        MTL_CONV_CASE(1) MTL_CONV_CASE(2) MTL_CONV_CASE(3) MTL_CONV_CASE(4) MTL_CONV_CASE(5)
        MTL_CONV_CASE(6) MTL_CONV_CASE(7) MTL_CONV_CASE(8)
#undef MTL_CONV_CASE
        default: set_error("conv width unsupported"); return MTL_EINVAL;
    }
    return check_launch("causal_conv1d_fwd");
}

// 4-channel vectors when channels are unit-stride and every row start is
// vector-aligned; one channel per thread otherwise.
template <typename T>
int launch_conv(const ConvArgs& a, int64_t batch, hipStream_t st) {
    constexpr int kVC = 4;
    const uintptr_t al = kVC * sizeof(T);
    const bool vec = a.x_sd == 1 && a.o_sd == 1 && a.D % kVC == 0 && (uintptr_t)a.x % al == 0 &&
                     (uintptr_t)a.out % al == 0 && (a.x_sl * (int64_t)sizeof(T)) % al == 0 &&
                     (a.o_sl * (int64_t)sizeof(T)) % al == 0 &&
                     (batch == 1 || ((a.x_sb * (int64_t)sizeof(T)) % al == 0 && (a.o_sb * (int64_t)sizeof(T)) % al == 0));
    // Short sequences: with 16-step runs a 64-token prompt at D = 1536 is 8
    // workgroups, each thread forming 16 outputs in turn; 4-step runs give
    // 4x the workgroups and a quarter of the serial work per thread.
    const int64_t groups = (a.D / (vec ? kVC : 1) + kConvThreads - 1) / kConvThreads;
    if (groups * ((a.L + kTC - 1) / kTC) * batch < 256)
        return vec ? launch_conv_vc<T, kVC, 4>(a, batch, st) : launch_conv_vc<T, 1, 4>(a, batch, st);
    return vec ? launch_conv_vc<T, kVC, kTC>(a, batch, st) : launch_conv_vc<T, 1, kTC>(a, batch, st);
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
        MTL_STEP_CASE(1) MTL_STEP_CASE(2) MTL_STEP_CASE(3) MTL_STEP_CASE(4) MTL_STEP_CASE(5)
        MTL_STEP_CASE(6) MTL_STEP_CASE(7) MTL_STEP_CASE(8)
#undef MTL_STEP_CASE
        default: set_error("conv width unsupported"); return MTL_EINVAL;
    }
    return check_launch("conv_step");
}

// Batched single-token conv step fused with the x_proj split-K partials
// (model.py:264-279 for b rows at once): a workgroup owns kXpCB channels of
// 8 TB rows (blockIdx.y: rows [8 TB y, 8 TB (y + 1)) of b <= 32).  Phase 1: conv step (history shifted in place) + SiLU for
// its (channel, row) pairs, xc to global memory and to LDS.  Phase 2: the
// block's partial x_dbl[b][j] = sum over its channels of xc[b][c] W_xT[c][j],
// from LDS, a TB x (J/32) register tile per thread (rows b0.., columns jg +
// 32 q).  Partials land in xpart[block][b][j]; the caller sums them in block
// order.
constexpr int kXpCB = 32;                 // channels per workgroup
constexpr int kXpMaxJQ = 9;               // J <= 288 = 256 + 32
#ifndef MTL_XP_ROW_TB
#define MTL_XP_ROW_TB 2
#endif
constexpr int kXpRowTB = MTL_XP_ROW_TB;   // above 8 rows: 8 kXpRowTB rows per workgroup

template <int K, int TB, int JQ>
__global__ void __launch_bounds__(256) conv_step_xproj_kernel(float* __restrict__ state, const float* __restrict__ x,
                                                              int64_t x_sb, const float* __restrict__ w,
                                                              const float* __restrict__ bias, float* __restrict__ out,
                                                              int64_t o_sb, const float* __restrict__ WxT,
                                                              float* __restrict__ xpart, int batch, int D, int J) {
    constexpr int BMAX = 8 * TB;                     // rows covered: 8 row groups of TB
    __shared__ float s_xc[BMAX][kXpCB + 1];          // local rows
    const int b0 = blockIdx.y * BMAX;
    __shared__ float s_w[kXpCB][kXpMaxJQ * 32];       // rows c >= nch are never read (see phase 2)
    const int tid = threadIdx.x;
    const int c0 = blockIdx.x * kXpCB;
    const int nch = min(kXpCB, D - c0);

    // every load first, with clamped addresses: the block's x_proj columns
    // (8 threads per channel row, element j = tid % 8 + 8 k), then the conv
    // operands of pair tid + 256 q (channel fastest)
    constexpr int kWLoads = kXpMaxJQ * 32 / 8;
    const int wc = tid >> 3, wj = tid & 7;
    const float* wrow = WxT + (int64_t)(c0 + min(wc, nch - 1)) * J;
    float wl[kWLoads];
#pragma unroll
    for (int k = 0; k < kWLoads; ++k) wl[k] = wrow[min(wj + 8 * k, J - 1)];
    constexpr int kPairs = kXpCB * BMAX;     // = 256 TB
    float win[TB][K], wk[TB][K], bs[TB];
#pragma unroll
    for (int q = 0; q < TB; ++q) {
        const int ch = c0 + min(tid % kXpCB, nch - 1), bi = min(b0 + tid / kXpCB + 8 * q, batch - 1);
        const float* s = state + ((int64_t)bi * D + ch) * (K - 1);
#pragma unroll
        for (int k = 0; k < K - 1; ++k) win[q][k] = s[k];
        win[q][K - 1] = x[bi * x_sb + ch];
#pragma unroll
        for (int k = 0; k < K; ++k) wk[q][k] = w[(int64_t)ch * K + k];
        bs[q] = bias ? bias[ch] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < kWLoads; ++k)
        if (wj + 8 * k < J) s_w[wc][wj + 8 * k] = wl[k];
    // phase 1: conv step + SiLU
    static_assert(kPairs == 256 * TB, "one pair per thread per row group");
#pragma unroll
    for (int q = 0; q < TB; ++q) {
        const int c = tid % kXpCB, bl = tid / kXpCB + 8 * q, bi = b0 + bl;
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) acc = fmaf(win[q][k], wk[q][k], acc);
        acc += bs[q];
        const bool ok = c < nch && bi < batch;
        const float xcv = ok ? silu_f(acc) : 0.f;
        if (ok) {
            const int ch = c0 + c;
            float* s = state + ((int64_t)bi * D + ch) * (K - 1);
#pragma unroll
            for (int k = 0; k < K - 1; ++k) s[k] = win[q][k + 1];
            out[bi * o_sb + ch] = xcv;
        }
        s_xc[bl][c] = xcv;
    }
    __syncthreads();

    // phase 2: thread = (row group rg of TB rows, column lane jg)
    // JQ = column runs (J <= 32 JQ); columns past J read unwritten LDS and
    // are never stored, so the loop has no branches
    const int rg = tid / 32, jg = tid % 32;
    float acc[TB][JQ];
#pragma unroll
    for (int i = 0; i < TB; ++i)
#pragma unroll
        for (int q = 0; q < JQ; ++q) acc[i][q] = 0.f;
    for (int c = 0; c < nch; ++c) {
        float xv[TB], wv[JQ];
#pragma unroll
        for (int i = 0; i < TB; ++i) xv[i] = s_xc[rg * TB + i][c];
#pragma unroll
        for (int q = 0; q < JQ; ++q) wv[q] = s_w[c][jg + 32 * q];
#pragma unroll
        for (int q = 0; q < JQ; ++q)
#pragma unroll
            for (int i = 0; i < TB; ++i) acc[i][q] = fmaf(xv[i], wv[q], acc[i][q]);
    }
#pragma unroll
    for (int i = 0; i < TB; ++i) {
        const int bi = b0 + rg * TB + i;
        if (bi >= batch) continue;
#pragma unroll
        for (int q = 0; q < JQ; ++q) {
            const int j = jg + 32 * q;
            if (j < J) xpart[((int64_t)blockIdx.x * batch + bi) * J + j] = acc[i][q];
        }
    }
}

}  // namespace
}  // namespace mtl

extern "C" int mtl_causal_conv1d_fwd(const mtl_conv_params* p, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(p != nullptr, "null params");
    MTL_REQUIRE(p->batch >= 0 && p->seqlen >= 0 && p->dim >= 0, "negative size");
    MTL_REQUIRE(p->width >= 1 && p->width <= kMaxK, "width (d_conv) must be in [1, 8]");
    MTL_REQUIRE(p->batch <= 65535, "batch must be <= 65535");
    MTL_REQUIRE(p->seqlen < (int64_t(1) << 31) && p->dim < (int64_t(1) << 31), "size overflows int32");
    MTL_REQUIRE((p->seqlen + kTC - 1) / kTC <= 65535, "seqlen too long for one launch");
    MTL_REQUIRE(p->dtype == MTL_F32 || p->dtype == MTL_BF16, "dtype must be MTL_F32 or MTL_BF16");
    MTL_REQUIRE(p->conv_state_in == nullptr || p->conv_state_in != p->conv_state_out,
                "conv_state_out must not alias conv_state_in");
    if (p->batch == 0 || p->dim == 0) return MTL_OK;
    hipStream_t st = as_stream(stream);
    if (p->seqlen == 0) {
        const int64_t n = p->batch * p->dim * (p->width - 1);
        if (!p->conv_state_out || n == 0) return MTL_OK;
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
    MTL_REQUIRE(width >= 1 && width <= kMaxK, "width (d_conv) must be in [1, 8]");
    MTL_REQUIRE(batch <= 65535 && dim < (int64_t(1) << 31), "size out of range");
    MTL_REQUIRE(dtype == MTL_F32 || dtype == MTL_BF16, "dtype must be MTL_F32 or MTL_BF16");
    if (batch == 0 || dim == 0) return MTL_OK;
    MTL_REQUIRE((conv_state || width == 1) && x && w && out, "null required pointer");
    hipStream_t st = as_stream(stream);
    return dtype == MTL_F32
               ? launch_conv_step<float>(conv_state, x, x_sb, w, bias, out, out_sb, batch, (int)dim, width, silu, st)
               : launch_conv_step<uint16_t>(conv_state, x, x_sb, w, bias, out, out_sb, batch, (int)dim, width, silu,
                                            st);
}

namespace mtl {
namespace {

// Launches conv_step_xproj_kernel (sizes already checked).
int launch_conv_step_xproj(float* conv_state, const float* x, int64_t x_sb, const float* w, const float* bias,
                           float* out, int64_t out_sb, const float* W_xT, float* xpart, int64_t batch, int64_t dim,
                           int32_t width, int32_t xdbl_cols, hipStream_t st) {
    const int D = (int)dim, J = xdbl_cols, B = (int)batch;
    // rows per workgroup: 8 TB; above 8 rows the rows are split over
    // workgroups of 16 (kXpRowSplit) so that the grid covers every CU
    const int tb = B <= 8 ? 1 : kXpRowTB;
    const dim3 grid((unsigned)((dim + kXpCB - 1) / kXpCB), (unsigned)((B + 8 * tb - 1) / (8 * tb)));
#define MTL_XP_LAUNCH(KK, TBV, JQV) hipLaunchKernelGGL((conv_step_xproj_kernel<KK, TBV, JQV>), grid, dim3(256), 0, \
        st, conv_state, x, x_sb, w, bias, out, out_sb, W_xT, xpart, B, D, J)
#define MTL_XP_J(KK, TBV)                                                \
    if (J <= 64) MTL_XP_LAUNCH(KK, TBV, 2);                              \
    else if (J <= 96) MTL_XP_LAUNCH(KK, TBV, 3);                         \
    else if (J <= 160) MTL_XP_LAUNCH(KK, TBV, 5);                        \
    else MTL_XP_LAUNCH(KK, TBV, 9);
#define MTL_XP_K(KK)                                                     \
    case KK:                                                             \
        if (tb == 1) { MTL_XP_J(KK, 1) }                                 \
        else { MTL_XP_J(KK, kXpRowTB) }                                  \
        break;
    switch (width) {
        MTL_XP_K(1) MTL_XP_K(2) MTL_XP_K(3) MTL_XP_K(4) MTL_XP_K(5) MTL_XP_K(6) MTL_XP_K(7) MTL_XP_K(8)
        default: break;
    }
#undef MTL_XP_K
#undef MTL_XP_J
#undef MTL_XP_LAUNCH
    return check_launch("conv_step_xproj");
}

}  // namespace

// ---- scratch of the allocation-free batched step (mtl_conv_step_xproj_noalloc)
// The x_proj partials live in this array instead of a caller buffer.  In host
// code its name is only a stand-in: the device address comes from
// hipGetSymbolAddress, once per device (each GPU holds its own copy of the
// array for the life of the process), and only that address is ever handed
// to a kernel.
constexpr int64_t kXpScratchFloats = int64_t(1) << 20;     // 4 MiB: nblk * batch * xdbl_cols <= 2^20
static __device__ __align__(256) float scratch[kXpScratchFloats];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the device that `stream` belongs to (looked
// up on the first call on each device).  The lookup needs that device to be
// the current one, so when the calling thread has another device current it
// is switched for the lookup and switched back.
int scratch_for_stream(hipStream_t stream, float** out) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) {
        set_error(std::string("hipGetDevice: ") + hipGetErrorString(e));
        return MTL_EHIP;
    }
    int dev = cur;
    if (stream != nullptr) {
        hipDevice_t sd = -1;
        e = hipStreamGetDevice(stream, &sd);
        if (e != hipSuccess) {
            set_error(std::string("hipStreamGetDevice: ") + hipGetErrorString(e));
            return MTL_EHIP;
        }
        dev = static_cast<int>(sd);
    }
    if (dev < 0 || dev >= kMaxScratchDevices) {
        set_error("device index beyond the scratch table");
        return MTL_EUNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) {
            set_error(std::string("hipSetDevice: ") + hipGetErrorString(e));
            return MTL_EHIP;
        }
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        const hipError_t back = dev != cur ? hipSetDevice(cur) : hipSuccess;
        if (e != hipSuccess || p == nullptr) {
            set_error(std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
            return MTL_EHIP;
        }
        if (back != hipSuccess) {
            set_error(std::string("hipSetDevice (restoring the caller's device): ") + hipGetErrorString(back));
            return MTL_EHIP;
        }
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return MTL_OK;
}

}  // namespace
}  // namespace mtl

extern "C" int mtl_conv_step_xproj(float* conv_state, const float* x, int64_t x_sb, const float* w, const float* bias,
                                   float* out, int64_t out_sb, const float* W_xT, float* xpart, int64_t batch,
                                   int64_t dim, int32_t width, int32_t xdbl_cols, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch >= 1 && batch <= 32, "batch must be in [1, 32]");
    MTL_REQUIRE(dim >= 1 && dim < (int64_t(1) << 31), "dim out of range");
    MTL_REQUIRE(width >= 1 && width <= kMaxK, "width (d_conv) must be in [1, 8]");
    MTL_REQUIRE(xdbl_cols >= 1 && xdbl_cols <= kXpMaxJQ * 32, "xdbl_cols must be in [1, 288]");
    MTL_REQUIRE((conv_state || width == 1) && x && w && out && W_xT && xpart, "null required pointer");
    return launch_conv_step_xproj(conv_state, x, x_sb, w, bias, out, out_sb, W_xT, xpart, batch, dim, width,
                                  xdbl_cols, as_stream(stream));
}

extern "C" int mtl_conv_step_xproj_noalloc(float* conv_state, const float* x, int64_t x_sb, const float* w,
                                           const float* bias, float* out, int64_t out_sb, const float* W_xT,
                                           float* x_dbl, int64_t batch, int64_t dim, int32_t width,
                                           int32_t xdbl_cols, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch >= 1 && batch <= 32, "batch must be in [1, 32]");
    MTL_REQUIRE(dim >= 1 && dim < (int64_t(1) << 31), "dim out of range");
    MTL_REQUIRE(width >= 1 && width <= kMaxK, "width (d_conv) must be in [1, 8]");
    MTL_REQUIRE(xdbl_cols >= 1 && xdbl_cols <= kXpMaxJQ * 32, "xdbl_cols must be in [1, 288]");
    const int64_t nblk = (dim + kXpCB - 1) / kXpCB;
    MTL_REQUIRE(nblk * batch * xdbl_cols <= kXpScratchFloats,
                "ceil(dim / 32) * batch * xdbl_cols exceeds the 2^20-float scratch; use mtl_conv_step_xproj with "
                "a caller buffer");
    MTL_REQUIRE((conv_state || width == 1) && x && w && out && W_xT && x_dbl, "null required pointer");
    hipStream_t st = as_stream(stream);
    float* part = nullptr;
    const int rc = scratch_for_stream(st, &part);
    if (rc != MTL_OK) return rc;
    // every [block, row, column] of the partials is written before it is read:
    // nothing in the scratch needs clearing between calls
    const int r1 = launch_conv_step_xproj(conv_state, x, x_sb, w, bias, out, out_sb, W_xT, part, batch, dim, width,
                                          xdbl_cols, st);
    if (r1 != MTL_OK) return r1;
    return mtl_sum_parts(part, (int32_t)nblk, batch * xdbl_cols, x_dbl, stream);
}
