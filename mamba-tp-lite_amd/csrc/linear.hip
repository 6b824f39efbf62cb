// Skinny fp32 GEMM on the matrix cores for the projections of a batched
// decode step (gfx950).
//
//   Y[m, n] = sum_k X[m, k] * W[n, k]  (+ bias[n]),   m < M <= 32
//
// is nn.Linear on a [b, K] activation with b <= 32 tokens: in_proj
// (model.py:261), out_proj (model.py:293) and the tied lm_head
// (model.py:326, 353) of MambaMixer.step / MambaLM.step.  At these shapes the
// product streams the weight once and does 2*M flops per weight element, so
// it is bound by HBM; a GEMM library tiles it for large M and leaves much of
// the weight stream idle (fp32 M=32 at the mamba-1.4b width: in_proj 3.8,
// out_proj 2.0 TB/s).
//
// Mapping: one workgroup per n-tile of 16*RB weight rows; optionally KS
// workgroups per n-tile split K and write KS partial outputs that the
// consumer adds in split order.  K is walked in stages of kKC columns:
//   * all 256 threads load the stage's W tile [16 RB x kKC] and X tile
//     [16 MB x kKC] with float4 loads in row order (every 32 lanes read one
//     512-byte run of a row) into registers, two stages ahead, and write them
//     to a double-buffered LDS tile (rows padded by 4 floats);
//   * wavefront w multiplies the stage's k-blocks 2w and 2w+1 (16 columns
//     each) on the matrix cores: per block a lane l = r + 16 kk (r < 16,
//     kk < 4) reads W[16 rb + r][k + 4 kk .. + 3] and X[16 mb + r][same k]
//     from LDS and feeds four v_mfma_f32_16x16x4_f32, the q-th taking
//     component q of both as its A and B operand, so the 16 columns enter in
//     the order (kk, q) on both sides and each MFMA adds
//     sum_kk W[n][k + 4 kk + q] X[m][k + 4 kk + q] into D[n][m];
//   * one barrier per stage.
// The four wavefronts' accumulators are added in wavefront order through LDS
// at the end, so the result is deterministic.  Reading the weight rows in
// 512-byte runs instead of the MFMA operand layout's 64-byte pieces per row
// took the mamba-1.4b in_proj (M=32) from 19.5 to 13.3 us (time measured on
// the bytes alone).

#include "common.h"

namespace mtl {
namespace {

typedef float F4v __attribute__((ext_vector_type(4)));

struct LinArgs {
    const float* x;        // [M, K], row stride x_rs
    const float* W;        // [N, K] contiguous
    const float* bias;     // [N] or null
    float* y;              // [M, N] (row stride y_rs); split s at y + s * y_ks
    int64_t x_rs, y_rs, y_ks;
    int M, N, K, KS;
};

constexpr int kLinThreads = 256;
constexpr int kLinWaves = kLinThreads / 64;
constexpr int kKC = 128;                          // K columns per stage
constexpr int kKP = kKC + 4;                      // padded LDS row: b128 reads of 16 rows hit distinct banks
constexpr int kC4 = kKC / 4;                      // float4 per stage row

__device__ __forceinline__ F4v ld4(const float* p) { return *reinterpret_cast<const F4v*>(p); }

template <int RB, int MB>
__global__ void __launch_bounds__(kLinThreads) linear_skinny_kernel(const LinArgs a) {
    constexpr int WR = 16 * RB, XR = 16 * MB;          // tile rows
    constexpr int WL = WR * kC4 / kLinThreads;          // float4 loads per thread per stage
    constexpr int XL = XR * kC4 / kLinThreads;
    static_assert(WL >= 1 && XL >= 1, "tile shape");
    __shared__ __align__(16) float s_w[2][WR][kKP];
    __shared__ __align__(16) float s_x[2][XR][kKP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, kk = lane >> 4;
    const int n0 = blockIdx.x * WR;
    const int ks = blockIdx.y;
    const int kper = a.K / a.KS;                        // a multiple of kKC (host-checked)
    const int kbeg = ks * kper;
    const int ns = kper / kKC;

    // loader slots: float4 e = tid + 256 i of a stage tile is (row e / kC4, column 4 (e % kC4))
    const float* wsrc[WL];
    int wdst[WL];
#pragma unroll
    for (int i = 0; i < WL; ++i) {
        const int e = tid + kLinThreads * i, row = e / kC4, c = 4 * (e % kC4);
        wsrc[i] = a.W + (int64_t)min(n0 + row, a.N - 1) * a.K + kbeg + c;
        wdst[i] = row * kKP + c;
    }
    const float* xsrc[XL];
    int xdst[XL];
#pragma unroll
    for (int i = 0; i < XL; ++i) {
        const int e = tid + kLinThreads * i, row = e / kC4, c = 4 * (e % kC4);
        xsrc[i] = a.x + (int64_t)min(row, a.M - 1) * a.x_rs + kbeg + c;
        xdst[i] = row * kKP + c;
    }
    struct Set { F4v w[WL], x[XL]; };
    auto load = [&](Set& st, int s) __attribute__((always_inline)) {
        const int off = min(s, ns - 1) * kKC;           // past the end: the last stage again, never used
#pragma unroll
        for (int i = 0; i < WL; ++i) st.w[i] = ld4(wsrc[i] + off);
#pragma unroll
        for (int i = 0; i < XL; ++i) st.x[i] = ld4(xsrc[i] + off);
    };
    auto store = [&](const Set& st, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < WL; ++i) *reinterpret_cast<F4v*>(&s_w[buf][0][0] + wdst[i]) = st.w[i];
#pragma unroll
        for (int i = 0; i < XL; ++i) *reinterpret_cast<F4v*>(&s_x[buf][0][0] + xdst[i]) = st.x[i];
    };

    F4v acc[RB][MB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = F4v{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int k = 32 * wave + 16 * kb + 4 * kk;
            F4v wv[RB], xv[MB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) wv[rb] = ld4(&s_w[buf][16 * rb + r][k]);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) xv[mb] = ld4(&s_x[buf][16 * mb + r][k]);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb)
                        acc[rb][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[rb][q], xv[mb][q], acc[rb][mb], 0, 0, 0);
        }
    };

    // stage s is in LDS buffer s % 2; register sets A and B hold the stages
    // one and two ahead of the one being multiplied
    Set A, B;
    load(A, 0);
    load(B, 1);
    store(A, 0);
    load(A, 2);
    __syncthreads();
    // one stage: multiply s from LDS, move stage s + 1 from its registers
    // into the other buffer, refill those registers with stage s + 3
    auto stage = [&](int s, Set& nxt) __attribute__((always_inline)) {
        mma(s & 1);
        store(nxt, (s + 1) & 1);
        load(nxt, s + 3);
        __syncthreads();
    };
    int s = 0;
    for (; s + 2 <= ns; s += 2) {
        stage(s, B);       // B holds s + 1, then s + 3
        stage(s + 1, A);   // A holds s + 2, then s + 4
    }
    if (s < ns) mma(s & 1);

    // D[i][j] of an MFMA tile sits in lane j + 16 (i / 4), register i % 4:
    // n = n0 + 16 rb + 4 (lane / 16) + reg, m = 16 mb + lane % 16.  The
    // reduction reuses the W buffers (every wavefront is past its last read).
    __syncthreads();
    F4v* s_acc = reinterpret_cast<F4v*>(&s_w[0][0][0]);
    static_assert(sizeof(s_w) >= sizeof(F4v) * kLinWaves * RB * MB * 64, "reduction space");
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) s_acc[(wave * RB * MB + rb * MB + mb) * 64 + lane] = acc[rb][mb];
    __syncthreads();
    for (int t = tid; t < RB * MB * 64; t += kLinThreads) {
        const int tile = t >> 6, ln = t & 63;
        const int rb = tile / MB, mb = tile - rb * MB;
        F4v sum = s_acc[tile * 64 + ln];
#pragma unroll
        for (int w = 1; w < kLinWaves; ++w) sum += s_acc[(w * RB * MB + tile) * 64 + ln];
        const int m = 16 * mb + (ln & 15);
        const int n = n0 + 16 * rb + 4 * (ln >> 4);
        if (m < a.M && n < a.N) {
            if (a.bias && ks == 0) sum += ld4(a.bias + n);
            *reinterpret_cast<F4v*>(a.y + ks * a.y_ks + (int64_t)m * a.y_rs + n) = sum;
        }
    }
}

template <int RB, int MB>
void launch_linear(const LinArgs& a, hipStream_t st) {
    dim3 grid((unsigned)((a.N + 16 * RB - 1) / (16 * RB)), (unsigned)a.KS);
    hipLaunchKernelGGL((linear_skinny_kernel<RB, MB>), grid, dim3(kLinThreads), 0, st, a);
}

}  // namespace
}  // namespace mtl

using namespace mtl;

extern "C" int mtl_linear_skinny(const float* x, int64_t x_rs, const float* W, const float* bias, float* y,
                                 int64_t y_rs, int64_t y_ks, int64_t M, int64_t N, int64_t K, int32_t ksplit,
                                 int32_t rows_per_block, mtl_stream_t stream) {
    clear_error();
    MTL_REQUIRE(x && W && y, "null pointer");
    MTL_REQUIRE(M >= 1 && M <= 32, "M (rows of x) must be in [1, 32]");
    MTL_REQUIRE(N >= 1 && N % 4 == 0 && N < (int64_t(1) << 31), "N must be a positive multiple of 4");
    MTL_REQUIRE(ksplit >= 1 && ksplit <= 64, "ksplit must be in [1, 64]");
    MTL_REQUIRE(K >= 1 && K % (int64_t(kKC) * ksplit) == 0 && K < (int64_t(1) << 31),
                "K must be a positive multiple of 128 * ksplit");
    MTL_REQUIRE(rows_per_block == 16 || rows_per_block == 32, "rows_per_block must be 16 or 32");
    MTL_REQUIRE(x_rs >= K && x_rs % 4 == 0 && y_rs >= N && y_rs % 4 == 0, "row strides must cover a row and be multiples of 4");
    MTL_REQUIRE(ksplit == 1 || y_ks >= (M - 1) * y_rs + N, "split outputs must not overlap");
    MTL_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(y) |
                 reinterpret_cast<uintptr_t>(bias)) % 16 == 0, "x, W, y and bias must be 16-byte aligned");
    MTL_REQUIRE(y_ks % 4 == 0, "y_ks must be a multiple of 4");
    LinArgs a{x, W, bias, y, x_rs, y_rs, y_ks, (int)M, (int)N, (int)K, (int)ksplit};
    hipStream_t st = as_stream(stream);
    const bool two_m = M > 16;
    if (rows_per_block == 32) {
        if (two_m) launch_linear<2, 2>(a, st); else launch_linear<2, 1>(a, st);
    } else {
        if (two_m) launch_linear<1, 2>(a, st); else launch_linear<1, 1>(a, st);
    }
    return check_launch("linear_skinny_kernel");
}
