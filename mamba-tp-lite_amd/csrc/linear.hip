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
// the weight stream idle (fp32 M=32, weights cold in HBM, mamba-1.4b width:
// in_proj 3.6-3.8, out_proj 2.0 TB/s).
//
// Mapping: one workgroup per n-tile of 16*RB weight rows; optionally KS
// workgroups per n-tile split K and write KS partial outputs that the
// consumer adds in split order.  Each of the four wavefronts owns a
// contiguous quarter of the workgroup's K range and walks it in stages of
// 32 columns:
//   * a stage is the wavefront's W rows [16 RB x 32] and X rows [16 MB x 32],
//     copied from global memory straight into a ring of D stage slots of
//     its own in LDS by global_load_lds_dwordx4 (no register staging, so the
//     ring depth costs LDS, not VGPRs).  One such instruction moves 8 rows x
//     128 bytes (8 lanes per row); lane p of a row fetches 16-byte chunk
//     p ^ (row & 7), so chunk c of a row sits at position c ^ (row & 7);
//   * it multiplies a stage as two 16-column blocks: lane l = r + 16 kk
//     (r < 16, kk < 4) reads chunk 4 kb + kk of W row 16 rb + r and of X row
//     16 mb + r (the swizzle puts 8 consecutive rows of one chunk in
//     distinct banks) and feeds four v_mfma_f32_16x16x4_f32, the q-th taking
//     component q of both as its A and B operand, so the 16 columns enter
//     in the order (kk, q) on both sides and each MFMA adds
//     sum_kk W[n][k + 4 kk + q] X[m][k + 4 kk + q] into D[n][m];
//   * the copies count on the vector-memory counter, and the compiler does
//     not track their LDS writes: the loop waits with explicit
//     s_waitcnt vmcnt(n), n = the copies still allowed in flight, before it
//     reads a stage, and lgkmcnt(0) (its reads of the slot done) before it
//     refills a slot.  Only the wavefront reads what it copied, so the K
//     loop has no barrier.
// The four wavefronts' accumulators are added in wavefront order through LDS
// at the end, so the result is deterministic.  Measured on the mamba-1.4b
// in_proj at M = 32 with the weights cold in HBM: hipBLASLt 17.8-18.7 us;
// register-staged per-wavefront LDS stages 19.2-21.7 us; this form 15.6-15.8
// us (out_proj 16.7 / 12.6 / 10.0 us).

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
constexpr int kKW = 32;                           // K columns per wavefront per stage
constexpr int kKC = kLinWaves * kKW;              // K granule of a workgroup (128)

__device__ __forceinline__ F4v ld4(const float* p) { return *reinterpret_cast<const F4v*>(p); }

#define MTL_WAIT_VMCNT(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")

template <int RB, int MB, int D>
__global__ void __launch_bounds__(kLinThreads) linear_skinny_kernel(const LinArgs a) {
    constexpr int WR = 16 * RB, XR = 16 * MB, SROWS = WR + XR;   // rows of a stage: W then X
    constexpr int NI = SROWS / 8;                                 // copies per stage (8 rows each)
    static_assert(D >= 2 && D <= 3, "ring depth");
    static_assert((D - 1) * NI <= 63, "vmcnt range");
    __shared__ __align__(16) float ring[kLinWaves][D][SROWS * kKW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, kk = lane >> 4;
    const int n0 = blockIdx.x * WR;
    const int ks = blockIdx.y;
    const int kper = a.K / a.KS;                       // a multiple of kKC (host-checked)
    const int ns = kper / kKC;                         // stages per wavefront, >= D - 1 (host-checked)
    const int kbeg = ks * kper + wave * (kper / kLinWaves);

    // copy lane: row 8 i + lane / 8 of the stage, fetching chunk (lane % 8) ^ (row & 7)
    const int crow = lane >> 3, cch = (lane & 7) ^ crow;
    const float* src[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = 8 * i + crow;
        src[i] = row < WR ? a.W + (int64_t)min(n0 + row, a.N - 1) * a.K + kbeg + 4 * cch
                          : a.x + (int64_t)min(row - WR, a.M - 1) * a.x_rs + kbeg + 4 * cch;
    }
    auto issue = [&](int s) __attribute__((always_inline)) {
        float* dst = &ring[wave][s % D][0];
        // the builtin exists for the device pass only; the host pass still
        // has to see the kernel to emit its launch stub
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
        for (int i = 0; i < NI; ++i)
            __builtin_amdgcn_global_load_lds(src[i] + s * kKW, dst + i * 256, 16, 0, 0);
#else
        (void)dst;
#endif
    };

    F4v acc[RB][MB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = F4v{0.f, 0.f, 0.f, 0.f};
    auto mma = [&](int s) __attribute__((always_inline)) {
        const float* st = &ring[wave][s % D][0];
#pragma unroll
        for (int kb = 0; kb < kKW / 16; ++kb) {
            const int c = 4 * kb + kk;
            F4v wv[RB], xv[MB];
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const int row = 16 * rb + r;
                wv[rb] = ld4(st + (row * 8 + (c ^ (row & 7))) * 4);
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int row = WR + 16 * mb + r;
                xv[mb] = ld4(st + (row * 8 + (c ^ (row & 7))) * 4);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int mb = 0; mb < MB; ++mb)
                        acc[rb][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[rb][q], xv[mb][q], acc[rb][mb], 0, 0, 0);
        }
    };

    // D - 1 stages in flight ahead of the one being multiplied
#pragma unroll
    for (int s = 0; s < D - 1; ++s) issue(s);
    int s = 0;
    for (; s < ns - (D - 1); ++s) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // reads of slot (s - 1) % D are done
        issue(s + D - 1);
        MTL_WAIT_VMCNT((D - 1) * NI);                          // stage s has landed
        mma(s);
    }
    // the last D - 1 stages are already in flight
    MTL_WAIT_VMCNT((D - 2) * NI);
    mma(s);
    if constexpr (D == 3) {
        MTL_WAIT_VMCNT(0);
        mma(s + 1);
    }

    // D[i][j] of an MFMA tile sits in lane j + 16 (i / 4), register i % 4:
    // n = n0 + 16 rb + 4 (lane / 16) + reg, m = 16 mb + lane % 16.  The
    // reduction reuses the ring once every wavefront is past its reads.
    __syncthreads();
    F4v* s_acc = reinterpret_cast<F4v*>(&ring[0][0][0]);
    static_assert(sizeof(ring) >= sizeof(F4v) * kLinWaves * RB * MB * 64, "reduction space");
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
    if (a.K / a.KS >= 2 * kKC)
        hipLaunchKernelGGL((linear_skinny_kernel<RB, MB, 3>), grid, dim3(kLinThreads), 0, st, a);
    else
        hipLaunchKernelGGL((linear_skinny_kernel<RB, MB, 2>), grid, dim3(kLinThreads), 0, st, a);
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
