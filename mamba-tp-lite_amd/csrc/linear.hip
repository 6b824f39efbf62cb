// Skinny fp32 GEMM on the matrix cores for the projections of a batched
// decode step and of a short prefill (gfx950).
//
//   Y[m, n] = sum_k X[m, k] * W[n, k]  (+ bias[n]),   m < M <= 64
//
// is nn.Linear on a [b, K] activation with b <= 32 tokens: in_proj
// (model.py:261), out_proj (model.py:293) and the tied lm_head
// (model.py:326, 353) of MambaMixer.step / MambaLM.step; and on the [b l, K]
// activations of a prefill of b l <= 64 tokens (model.py:197, 214, 240,
// 339).  At these shapes the
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

// The tile product of one workgroup: W rows [n0, n0 + 16 RB) against the M
// rows of x over the K range of split ks.  On return every wavefront's
// accumulators sit in s_acc = the ring's first RB MB 4 KB (after a barrier),
// and tile_sum() adds them in wavefront order.  A kernel that calls it keeps
// all of its LDS in the ring array (see in_conv_xproj_kernel).
template <int RB, int MB, int D>
__device__ __forceinline__ void skinny_tile(const LinArgs& a, float* ring, int n0, int ks) {
    constexpr int WR = 16 * RB, XR = 16 * MB, SROWS = WR + XR;   // rows of a stage: W then X
    constexpr int NI = SROWS / 8;                                 // copies per stage (8 rows each)
    constexpr int SLOT = SROWS * kKW;                             // floats per ring slot
    static_assert(D >= 2 && D <= 3, "ring depth");
    static_assert((D - 1) * NI <= 63, "vmcnt range");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, kk = lane >> 4;
    const int kper = a.K / a.KS;                       // a multiple of kKC (host-checked)
    const int ns = kper / kKC;                         // stages per wavefront, >= D - 1 (host-checked)
    const int kbeg = ks * kper + wave * (kper / kLinWaves);
    float* myring = ring + wave * D * SLOT;

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
        float* dst = myring + (s % D) * SLOT;
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
        const float* st = myring + (s % D) * SLOT;
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

    // the reduction space reuses the ring once every wavefront is past its reads
    __syncthreads();
    F4v* s_acc = reinterpret_cast<F4v*>(ring);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) s_acc[(wave * RB * MB + rb * MB + mb) * 64 + lane] = acc[rb][mb];
    __syncthreads();
}

// Pair t < 64 RB MB of the tile: D[i][j] of an MFMA tile sits in lane
// j + 16 (i / 4), register i % 4, so pair (tile, ln) holds outputs
// n = n0 + 16 rb + 4 (ln / 16) + 0..3 of row m = 16 mb + ln % 16.
template <int RB, int MB>
__device__ __forceinline__ F4v tile_sum(const float* ring, int t, int& m, int& nl) {
    const F4v* s_acc = reinterpret_cast<const F4v*>(ring);
    const int tile = t >> 6, ln = t & 63;
    const int rb = tile / MB, mb = tile - rb * MB;
    F4v sum = s_acc[tile * 64 + ln];
#pragma unroll
    for (int w = 1; w < kLinWaves; ++w) sum += s_acc[(w * RB * MB + tile) * 64 + ln];
    m = 16 * mb + (ln & 15);
    nl = 16 * rb + 4 * (ln >> 4);
    return sum;
}

template <int RB, int MB, int D>
constexpr int ring_floats() { return kLinWaves * D * (16 * RB + 16 * MB) * kKW; }

// blockIdx.z: the chunk of 16 MB rows of x (and y) this workgroup takes;
// one chunk (z = 0, all M <= 16 MB rows) unless M is larger.  A chunk's
// workgroups are those of the z = 0 launch with x and y moved down, so the
// n-tiles of every chunk share the tile order and land on the same XCD as
// their z = 0 twins when the tiles per chunk are a multiple of 8.
template <int RB, int MB, int D>
__global__ void __launch_bounds__(kLinThreads) linear_skinny_kernel(const LinArgs a) {
    __shared__ __align__(16) float ring[ring_floats<RB, MB, D>()];
    static_assert(sizeof(ring) >= sizeof(F4v) * kLinWaves * RB * MB * 64, "reduction space");
    const int n0 = blockIdx.x * 16 * RB, ks = blockIdx.y;
    const int r0 = blockIdx.z * 16 * MB;
    LinArgs c = a;
    c.x += (int64_t)r0 * a.x_rs;
    c.y += (int64_t)r0 * a.y_rs;
    c.M = min(16 * MB, a.M - r0);
    skinny_tile<RB, MB, D>(c, ring, n0, ks);
    for (int t = threadIdx.x; t < RB * MB * 64; t += kLinThreads) {
        int m, nl;
        F4v sum = tile_sum<RB, MB>(ring, t, m, nl);
        const int n = n0 + nl;
        if (m < c.M && n < c.N) {
            if (c.bias && ks == 0) sum += ld4(c.bias + n);
            *reinterpret_cast<F4v*>(c.y + ks * c.y_ks + (int64_t)m * c.y_rs + n) = sum;
        }
    }
}

template <int RB, int MB>
void launch_linear(const LinArgs& a, hipStream_t st) {
    dim3 grid((unsigned)((a.N + 16 * RB - 1) / (16 * RB)), (unsigned)a.KS, (unsigned)((a.M + 16 * MB - 1) / (16 * MB)));
    // 64 rows of x: a 2-stage ring (80 KB of LDS at 16 W rows, 96 KB at 32)
    if constexpr (MB > 2)
        hipLaunchKernelGGL((linear_skinny_kernel<RB, MB, 2>), grid, dim3(kLinThreads), 0, st, a);
    else if (a.K / a.KS >= 2 * kKC)
        hipLaunchKernelGGL((linear_skinny_kernel<RB, MB, 3>), grid, dim3(kLinThreads), 0, st, a);
    else
        hipLaunchKernelGGL((linear_skinny_kernel<RB, MB, 2>), grid, dim3(kLinThreads), 0, st, a);
}

// ------------------------------------------------------- out_proj + residual add + the next norm's inputs
// A batched step's out_proj split over K (model.py:293), the block's residual
// add (model.py:311) and what the next block's RMSNorm (model.py:130-135)
// needs from its input, without the add + norm launch between the blocks.
// Every workgroup writes its split's partial tile, then counts its arrival on
// its n-tile's counter; the last of the KS arrivals adds the KS partials in
// split order, then the residual, exactly as mtl_add_rmsnorm_parts does:
//   h[m][n] += ((part0 + part1) + part2) + ...,
// stores h, xn[m][n] = h[m][n] * w[n] (the next in_proj's operand) and, per
// row, the sum of h^2 over the tile's 16 RB columns into sq[tile][m] (the
// columns added in order).  The next in_proj adds the sq row of every tile
// and scales its dot products by rsqrt(mean h^2 + eps).
// The partials move between workgroups (and XCDs) as agent-scope atomic
// stores and loads (sc1: coherent at agent scope once complete, never served
// from a stale L2 line); each wavefront waits for its stores (vmcnt(0))
// before the workgroup counts its arrival, and the last arrival issues its
// loads only after its count returned.  That is the release/acquire pair for
// data that is itself written and read atomically: the L2 write-back of a
// release fence exists for plain stores, the L2 invalidate of an acquire
// fence for plain loads, and neither is needed here.  They cost: a release
// fence per wavefront and an acquire fence per wavefront of the last arrival
// took the launch from 10.9 to 27.8 us at the mamba-1.4b width, 32 rows; a
// release on the count and an acquire in the last arrival only (one each per
// workgroup) still added 8.6 us per layer to the 8-row step (2494 -> 2906 us).  h and w come from earlier launches, so
// every workgroup loads its pairs' h and w before it counts.  Counters start
// at zero and each is taken by exactly KS workgroups of one launch; nothing
// is reset, so a call needs its own zeroed counters.
struct ResidArgs {
    float* h;          // [M, N] residual rows, in place
    const float* w;    // [N] next RMSNorm's weight
    float* xn;         // [M, N]
    float* sq;         // [N / (16 RB), M]
    unsigned* cnt;     // [N / (16 RB)], zero on entry
};

constexpr int kResidMaxSplit = 4;

__device__ __forceinline__ void store_coherent(float* p, F4v v) {
#pragma unroll
    for (int q = 0; q < 4; ++q) __hip_atomic_store(p + q, v[q], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ F4v load_coherent(const float* p) {
    F4v v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = __hip_atomic_load(p + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return v;
}

template <int RB, int MB, int D>
__global__ void __launch_bounds__(kLinThreads) linear_resid_kernel(const LinArgs a, const ResidArgs r) {
    constexpr int WR = 16 * RB, NPAIR = RB * MB * 64;
    __shared__ __align__(16) float ring[ring_floats<RB, MB, D>()];
    static_assert(sizeof(ring) >= sizeof(float) * (16 * MB * 4 * RB + 4), "epilogue space");
    const int n0 = blockIdx.x * WR, ks = blockIdx.y, tid = threadIdx.x;
    // this thread's pair: 4 columns n0 + nl .. n0 + nl + 3 of row m (the
    // layout tile_sum hands out); its bias, h and w do not depend on the
    // product, so their loads are issued ahead of the product's copies and
    // the first stage's wait covers them
    const bool has_pair = tid < NPAIR;
    int m, nl;
    {
        const int tile = tid >> 6, ln = tid & 63;
        m = 16 * (tile % MB) + (ln & 15);
        nl = 16 * (tile / MB) + 4 * (ln >> 4);
    }
    F4v bv = {0.f, 0.f, 0.f, 0.f}, hv = bv, wv = bv;
    if (has_pair) {
        if (a.bias && ks == 0) bv = ld4(a.bias + n0 + nl);
        hv = ld4(r.h + (int64_t)min(m, a.M - 1) * a.N + n0 + nl);
        wv = ld4(r.w + n0 + nl);
    }
    skinny_tile<RB, MB, D>(a, ring, n0, ks);
    asm volatile("" : "+v"(bv), "+v"(hv), "+v"(wv));   // consumed after the product only
    F4v own = {0.f, 0.f, 0.f, 0.f};
    if (has_pair) {
        int mt, nt;
        own = tile_sum<RB, MB>(ring, tid, mt, nt);
        if (a.bias && ks == 0) own += bv;
        if (m < a.M) store_coherent(a.y + ks * a.y_ks + (int64_t)m * a.y_rs + n0 + nl, own);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wavefront's partial stores are done
    __syncthreads();                                     // every wavefront's; s_acc reads done
    int* s_last = reinterpret_cast<int*>(ring);
    if (tid == 0)
        *s_last = __hip_atomic_fetch_add(r.cnt + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  (unsigned)(a.KS - 1);
    __syncthreads();
    if (!*s_last) return;                                // uniform

    float* s_sq = ring + 4;                              // [16 MB][4 RB]: row m's squares, by column group
    if (has_pair && m < a.M) {
        const float* pp = a.y + (int64_t)m * a.y_rs + n0 + nl;
        F4v pv[kResidMaxSplit];                          // one batch of loads, no branches
#pragma unroll
        for (int p = 0; p < kResidMaxSplit; ++p) pv[p] = load_coherent(pp + min(p, a.KS - 1) * a.y_ks);
        F4v t = ks == 0 ? own : pv[0];
#pragma unroll
        for (int p = 1; p < kResidMaxSplit; ++p)
            if (p < a.KS) t += p == ks ? own : pv[p];
        hv += t;
        const int64_t o = (int64_t)m * a.N + n0 + nl;
        *reinterpret_cast<F4v*>(r.h + o) = hv;
        *reinterpret_cast<F4v*>(r.xn + o) = hv * wv;
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) s = fmaf(hv[q], hv[q], s);
        s_sq[m * 4 * RB + (nl >> 2)] = s;
    }
    __syncthreads();
    if (tid < a.M && tid < 16 * MB) {
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < 4 * RB; ++j) s += s_sq[tid * 4 * RB + j];
        r.sq[(int64_t)blockIdx.x * a.M + tid] = s;
    }
}

template <int RB, int MB>
void launch_resid(const LinArgs& a, const ResidArgs& r, hipStream_t st) {
    dim3 grid((unsigned)(a.N / (16 * RB)), (unsigned)a.KS);
    if (a.K / a.KS >= 2 * kKC)
        hipLaunchKernelGGL((linear_resid_kernel<RB, MB, 3>), grid, dim3(kLinThreads), 0, st, a, r);
    else
        hipLaunchKernelGGL((linear_resid_kernel<RB, MB, 2>), grid, dim3(kLinThreads), 0, st, a, r);
}

// ------------------------------------------------------- in_proj + conv step + x_proj partials
// The batched step's in_proj (model.py:261), conv step + SiLU (264-277) and
// x_proj (279) as one launch.  in_proj's output rows [0, D) are the x half
// and [D, 2D) the z half; a workgroup's tile of CB = 16 RB rows lies in one
// half (D % CB == 0).  A z tile stores z.  An x tile keeps its outputs
// x[m][c] (c = its CB channels, m = the b rows) and, as the epilogue:
//   * the conv step of each (row, channel): window = the K - 1 history
//     values of conv_state then x, xc = SiLU(window . conv_w[c] + conv_b[c]),
//     history shifted by one in place; xc to global memory;
//   * the x_proj partial of its channels on the matrix cores:
//     xpart[tile][m][j] = sum over its channels c of xc[m][c] W_xT[c][j],
//     as 16 x 16 blocks of (m, j) with K = the channels in steps of 4.  The
//     caller adds the D / CB partials in tile order.
// The tile's W_xT rows are one contiguous block of CB J floats; the
// workgroup copies it into LDS past the ring with global_load_lds before the
// GEMM (the GEMM's last vmcnt(0) and barrier cover it).  The conv operands
// are loaded after the GEMM: loaded before it (into registers), their
// scattered history rows delayed the first stages by more than the memory
// round trip they save (1.4b width, 32 tokens: 24.5 against 21.7 us).
// With sq set, x holds h * w (the block's RMSNorm weight applied to the
// residual rows h, as linear_resid_kernel leaves them) and sq [nsq, b] the
// per-tile sums of h^2 of each row: the tile's in_proj outputs are scaled by
// rsqrt(sum / d_model + eps) before the bias, which is in_proj applied to
// RMSNorm(h) (model.py:130-135), the norm taken on the dot products.
struct InConvArgs {
    float* state;            // [b, D, K - 1], in place
    const float* conv_w;     // [D, K]
    const float* conv_b;     // [D] or null
    const float* WxT;        // [D, J]
    float* xc;               // [b, D]
    float* z;                // [b, D] rows at stride z_rs
    float* xpart;            // [D / CB, b, J]
    const float* sq;         // [nsq, b] or null
    int64_t z_rs;
    int D, J, nsq;
    float eps;
};

constexpr int kIcMaxJ = 288;
constexpr int kSqPerThread = 16;                 // nsq <= 8 kSqPerThread

template <int RB, int MB, int D, int K, int NBJ>
__global__ void __launch_bounds__(kLinThreads) in_conv_xproj_kernel(const LinArgs a, const InConvArgs c) {
    constexpr int CB = 16 * RB, XR = 16 * MB;           // channels of a tile, rows of x
    constexpr int RING = ring_floats<RB, MB, D>();
    constexpr int WXF = (CB * 16 * NBJ + 255) / 256 * 256;   // W_xT tile space, whole 1 KB copies
    // All of the kernel's LDS is one array: with a second LDS array the
    // compiler can no longer tell the ring reads from the copies' LDS writes
    // and drains vmcnt to zero before every stage (1.4b width: 28.9 us
    // against 17 us for the plain product).
    __shared__ __align__(16) float lds[RING + WXF];
    float* ring = lds;
    float* s_wx = lds + RING;                          // [CB][J]
    constexpr int kAcc = kLinWaves * RB * MB * 64 * 4;  // floats of the reduction space
    static_assert(kAcc + XR * (CB + 1) + 8 * 32 <= RING, "epilogue space");
    static_assert(XR <= 32, "row scales for at most 32 rows");
    float (*s_xc)[CB + 1] = reinterpret_cast<float (*)[CB + 1]>(ring + kAcc);
    float* s_rs = ring + kAcc + XR * (CB + 1);          // [8][32] group sums of sq

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * CB;
    const bool xtile = n0 < c.D;                       // uniform
    const int J = c.J;

    if (xtile) {
        // the tile's W_xT block, 1 KB per copy, copies dealt to the wavefronts;
        // lanes past the block re-read its last 16 bytes into the padding
        const int nf = CB * J;                         // a multiple of 4
        const float* src = c.WxT + (int64_t)n0 * J;
        for (int ch = wave; ch * 256 < nf; ch += kLinWaves) {
            const int f = min(ch * 256 + 4 * lane, nf - 4);
#if defined(__HIP_DEVICE_COMPILE__)
            __builtin_amdgcn_global_load_lds(src + f, s_wx + ch * 256, 16, 0, 0);
#else
            (void)f;
#endif
        }
    }

    // Row m's scale rsqrt(mean h^2 + eps) (normed input only): thread (row
    // tid % 32, group g = tid / 32) adds tiles g, g + 8, ... in order, then
    // the 8 group sums are added in group order.  The sq loads are issued
    // ahead of the product's copies, so the first stage's wait covers them
    // (loads return in order) and no round trip follows the product.
    const int sm = min(tid & 31, a.M - 1), sg = tid >> 5;
    float sv[kSqPerThread];
    if (c.sq) {
#pragma unroll
        for (int i = 0; i < kSqPerThread; ++i) sv[i] = c.sq[(int64_t)min(sg + 8 * i, c.nsq - 1) * a.M + sm];
    }

    skinny_tile<RB, MB, D>(a, ring, n0, 0);

    // every thread calls it (normed input only)
    auto row_scale = [&](int m) __attribute__((always_inline)) {
        // opaque from here on: no part of the sum may move ahead of the product
#pragma unroll
        for (int i = 0; i < kSqPerThread; ++i) asm volatile("" : "+v"(sv[i]));
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < kSqPerThread; ++i)
            if (sg + 8 * i < c.nsq) s += sv[i];
        s_rs[sg * 32 + (tid & 31)] = s;
        __syncthreads();
        float tot = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) tot += s_rs[g * 32 + min(m, 31)];
        return rsqrtf(tot / (float)a.K + c.eps);
    };

    const int t = tid;                                 // this thread's output pair, if t < 64 RB MB
    const bool has_pair = t < RB * MB * 64;
    if (!xtile) {
        int m = 0, nl = 0;
        F4v v = {0.f, 0.f, 0.f, 0.f};
        if (has_pair) v = tile_sum<RB, MB>(ring, t, m, nl);
        if (c.sq) v *= row_scale(m);
        if (has_pair && m < a.M) {
            if (a.bias) v += ld4(a.bias + n0 + nl);
            *reinterpret_cast<F4v*>(c.z + m * c.z_rs + (n0 + nl - c.D)) = v;
        }
        return;
    }

    // the pair's conv results, stored after the x_proj phase: global stores
    // issued before its LDS reads would be waited for there (the compiler
    // orders LDS reads after every earlier vector-memory operation once the
    // kernel has copied into LDS)
    int m = 0, nl = 0, ch = 0;
    F4v xcv = {0.f, 0.f, 0.f, 0.f}, nh[K - 1];
    F4v v = {0.f, 0.f, 0.f, 0.f}, hist[K - 1], cw[K], cb = {0.f, 0.f, 0.f, 0.f};
    if (has_pair) {
        v = tile_sum<RB, MB>(ring, t, m, nl);
        ch = n0 + nl;
        const int mm = min(m, a.M - 1);
        const F4v* sp = reinterpret_cast<const F4v*>(c.state + ((int64_t)mm * c.D + ch) * (K - 1));
#pragma unroll
        for (int k = 0; k < K - 1; ++k) hist[k] = sp[k];
        const F4v* wp = reinterpret_cast<const F4v*>(c.conv_w + (int64_t)ch * K);
#pragma unroll
        for (int k = 0; k < K; ++k) cw[k] = wp[k];
        if (c.conv_b) cb = ld4(c.conv_b + ch);
    }
    if (c.sq) v *= row_scale(m);
    if (has_pair) {
        if (a.bias) v += ld4(a.bias + n0 + nl);
        // channel q of the four: history tap k is float q (K - 1) + k of the
        // pair's history block, conv weight k float q K + k of its weight block
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float win[K];
#pragma unroll
            for (int k = 0; k < K - 1; ++k) win[k] = hist[(q * (K - 1) + k) / 4][(q * (K - 1) + k) % 4];
            win[K - 1] = v[q];
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < K; ++k) acc = fmaf(win[k], cw[(q * K + k) / 4][(q * K + k) % 4], acc);
            acc += cb[q];
            xcv[q] = silu_f(acc);
#pragma unroll
            for (int k = 0; k < K - 1; ++k) nh[(q * (K - 1) + k) / 4][(q * (K - 1) + k) % 4] = win[k + 1];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) s_xc[m][nl + q] = m < a.M ? xcv[q] : 0.f;
    }
    __syncthreads();

    // x_proj partial on the matrix cores: wavefront w takes column blocks
    // jb = w + 4 i (i < JPW); lane l = r + 16 kk feeds A = xc[16 mb + r][4 s + kk]
    // (read once, shared by the blocks) and B = W_xT[4 s + kk][16 jb + r]
    // (columns past J clamped, never stored); D[i][j] lands in lane
    // j + 16 (i / 4), register i % 4.  The JPW MB accumulators are
    // independent chains, interleaved step by step.
    constexpr int JPW = (NBJ + kLinWaves - 1) / kLinWaves;
    const int r = lane & 15, kk = lane >> 4;
    float av[CB / 4][MB];
#pragma unroll
    for (int s4 = 0; s4 < CB / 4; ++s4)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) av[s4][mb] = s_xc[16 * mb + r][4 * s4 + kk];
    F4v acc[JPW][MB];
#pragma unroll
    for (int i = 0; i < JPW; ++i)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) acc[i][mb] = F4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < CB / 4; ++s4) {
#pragma unroll
        for (int i = 0; i < JPW; ++i) {
            const int jr = min(16 * (wave + kLinWaves * i) + r, J - 1);
            const float bv = s_wx[(4 * s4 + kk) * J + jr];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                acc[i][mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s4][mb], bv, acc[i][mb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < JPW; ++i) {
        const int j = 16 * (wave + kLinWaves * i) + r;
        if (j < J) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int mo = 16 * mb + 4 * kk + q;
                    if (mo < a.M) c.xpart[((int64_t)blockIdx.x * a.M + mo) * J + j] = acc[i][mb][q];
                }
        }
    }
    if (has_pair && m < a.M) {
        F4v* spo = reinterpret_cast<F4v*>(c.state + ((int64_t)m * c.D + ch) * (K - 1));
#pragma unroll
        for (int k = 0; k < K - 1; ++k) spo[k] = nh[k];
        *reinterpret_cast<F4v*>(c.xc + (int64_t)m * c.D + ch) = xcv;
    }
}

// ------------------------------------------------------- a short prefill's in_proj + causal conv
// MambaMixer.prefill's in_proj (model.py:197) for b l <= 64 tokens with, as
// the x tiles' epilogue, the causal depthwise conv + SiLU and the final conv
// state (198-212).  Row m of x is token t = m % l of batch row m / l, so a
// tile holds every token of its 16 RB channels: its in_proj outputs (with
// the in_proj bias) go to LDS, and pair (m, channel) takes the window of the
// K - 1 tokens before t (from the tile, or, before the first token, from the
// incoming history, or zeros) and t itself:
//   u[m][c] = SiLU(sum_k window[k] conv_w[c][k] + conv_b[c])   (k in order,
//   then the bias, as conv_fwd_kernel sums them), and the final history
//   state_out[b][c][j] = the input at token l - (K - 1) + j (from the
//   incoming history where that is before the first token).
// z tiles store z.  Thread t's pairs all have channel t % (16 RB), so its
// conv weights and bias are loaded once, with the history taps its pairs
// need, before the product.
struct PrefillConvArgs {
    const float* state_in;   // [b, D, K - 1] or null (zeros)
    float* state_out;        // [b, D, K - 1], not aliasing state_in
    const float* conv_w;     // [D, K]
    const float* conv_b;     // [D] or null
    float* u;                // [b l, D]
    float* z;                // [b l, D]
    int D, L;                // L = tokens per batch row
};

template <int RB, int K>
__global__ void __launch_bounds__(kLinThreads) in_conv_prefill_kernel(const LinArgs a, const PrefillConvArgs c) {
    constexpr int MB = 4, DEPTH = 2;
    constexpr int CB = 16 * RB, XR = 16 * MB;
    constexpr int RING = ring_floats<RB, MB, DEPTH>();
    __shared__ __align__(16) float ring[RING];
    constexpr int kAcc = kLinWaves * RB * MB * 64 * 4;
    static_assert(kAcc + XR * (CB + 1) <= RING, "epilogue space");
    static_assert(kLinThreads % CB == 0, "a thread's pairs share one channel");
    float (*s_x)[CB + 1] = reinterpret_cast<float (*)[CB + 1]>(ring + kAcc);
    const int tid = threadIdx.x;
    const int n0 = blockIdx.x * CB;
    const bool xtile = n0 < c.D;                       // uniform

    // the thread's conv operands, requested ahead of the product: its
    // channel's weights and bias, and the incoming history taps of its pairs
    // that fall before their sequence's first token
    constexpr int IT = XR * CB / kLinThreads;          // pairs per thread
    const int cl = tid % CB, ch = n0 + cl;
    const float* hin = c.state_in;
    float w[K], cb = 0.f, hv[IT][K - 1];
    if (xtile) {
#pragma unroll
        for (int k = 0; k < K; ++k) w[k] = c.conv_w[(int64_t)ch * K + k];
        cb = c.conv_b ? c.conv_b[ch] : 0.f;
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const int m = (tid + i * kLinThreads) / CB;
            const int bi = m / c.L, tt = m - bi * c.L;
#pragma unroll
            for (int k = 0; k < K - 1; ++k) {
                const int tau = tt - (K - 1) + k;
                hv[i][k] = (hin && m < a.M && tau < 0) ? hin[((int64_t)bi * c.D + ch) * (K - 1) + tau + K - 1] : 0.f;
            }
        }
    }

    skinny_tile<RB, MB, DEPTH>(a, ring, n0, 0);

    for (int t = tid; t < RB * MB * 64; t += kLinThreads) {
        int m, nl;
        F4v v = tile_sum<RB, MB>(ring, t, m, nl);
        if (a.bias) v += ld4(a.bias + n0 + nl);
        if (!xtile) {
            if (m < a.M) *reinterpret_cast<F4v*>(c.z + (int64_t)m * c.D + (n0 + nl - c.D)) = v;
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) s_x[m][nl + q] = v[q];
        }
    }
    if (!xtile) return;
    __syncthreads();

#pragma unroll
    for (int i = 0; i < IT; ++i) {
        const int m = (tid + i * kLinThreads) / CB;
        if (m >= a.M) break;
        const int tt = m % c.L;
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int tau = tt - (K - 1) + k;
            const float xv = tau >= 0 ? s_x[m - (K - 1) + k][cl] : hv[i][k < K - 1 ? k : K - 2];
            acc = fmaf(w[k], xv, acc);
        }
        acc += cb;
        c.u[(int64_t)m * c.D + ch] = silu_f(acc);
    }
    const int nb = a.M / c.L;
    for (int p = tid; p < nb * CB * (K - 1); p += kLinThreads) {
        const int j = p % (K - 1), rest = p / (K - 1);
        const int cj = rest % CB, bi = rest / CB, chj = n0 + cj;
        const int tau = c.L - (K - 1) + j;
        const float v = tau >= 0 ? s_x[bi * c.L + tau][cj]
                                 : (hin ? hin[((int64_t)bi * c.D + chj) * (K - 1) + tau + K - 1] : 0.f);
        c.state_out[((int64_t)bi * c.D + chj) * (K - 1) + j] = v;
    }
}

template <int RB, int MB, int K, int NBJ>
void launch_in_conv(const LinArgs& a, const InConvArgs& c, hipStream_t st) {
    hipLaunchKernelGGL((in_conv_xproj_kernel<RB, MB, 3, K, NBJ>), dim3((unsigned)(a.N / (16 * RB))),
                       dim3(kLinThreads), 0, st, a, c);
}

// NBJ = 16-column blocks of x_proj's output: the smallest of 2, 6, 10, 18 that covers J
template <int RB, int MB, int K>
void dispatch_in_conv_j(int J, const LinArgs& a, const InConvArgs& c, hipStream_t st) {
    if (J <= 32) launch_in_conv<RB, MB, K, 2>(a, c, st);
    else if (J <= 96) launch_in_conv<RB, MB, K, 6>(a, c, st);
    else if (J <= 160) launch_in_conv<RB, MB, K, 10>(a, c, st);
    else launch_in_conv<RB, MB, K, 18>(a, c, st);
}

template <int RB, int MB>
void dispatch_in_conv(int K, const LinArgs& a, const InConvArgs& c, hipStream_t st) {
    if (K == 2) dispatch_in_conv_j<RB, MB, 2>(c.J, a, c, st);
    else if (K == 3) dispatch_in_conv_j<RB, MB, 3>(c.J, a, c, st);
    else dispatch_in_conv_j<RB, MB, 4>(c.J, a, c, st);
}

}  // namespace
}  // namespace mtl

using namespace mtl;

extern "C" int mtl_linear_skinny(const float* x, int64_t x_rs, const float* W, const float* bias, float* y,
                                 int64_t y_rs, int64_t y_ks, int64_t M, int64_t N, int64_t K, int32_t ksplit,
                                 int32_t rows_per_block, mtl_stream_t stream) {
    clear_error();
    MTL_REQUIRE(x && W && y, "null pointer");
    MTL_REQUIRE(M >= 1 && M <= 64 * 65535, "M (rows of x) must be in [1, 4194240]");
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
    // 16-row MFMA blocks of x: 1, 2 or 4
    if (rows_per_block == 32) {
        if (M > 32) launch_linear<2, 4>(a, st);
        else if (M > 16) launch_linear<2, 2>(a, st);
        else launch_linear<2, 1>(a, st);
    } else {
        if (M > 32) launch_linear<1, 4>(a, st);
        else if (M > 16) launch_linear<1, 2>(a, st);
        else launch_linear<1, 1>(a, st);
    }
    return check_launch("linear_skinny_kernel");
}

extern "C" int mtl_in_proj_conv_prefill(const float* x, int64_t x_rs, const float* W_in, const float* b_in,
                                        const float* conv_w, const float* conv_b, int32_t d_conv,
                                        const float* conv_state_in, float* conv_state_out, float* u, float* z,
                                        int64_t batch, int64_t seqlen, int64_t d_model, int64_t d_inner,
                                        mtl_stream_t stream) {
    clear_error();
    MTL_REQUIRE(x && W_in && conv_w && conv_state_out && u && z, "null required pointer");
    MTL_REQUIRE(batch >= 1 && seqlen >= 1 && batch * seqlen <= 64, "batch * seqlen must be in [1, 64]");
    MTL_REQUIRE(d_model >= kKC && d_model % kKC == 0 && d_model < (int64_t(1) << 30),
                "d_model must be a positive multiple of 128");
    MTL_REQUIRE(d_inner >= 16 && d_inner % 16 == 0 && d_inner < (int64_t(1) << 29), "d_inner must be a multiple of 16");
    MTL_REQUIRE(d_conv >= 2 && d_conv <= 4, "d_conv must be 2, 3 or 4");
    MTL_REQUIRE(x_rs >= d_model && x_rs % 4 == 0, "x row stride must cover a row and be a multiple of 4");
    MTL_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W_in) | reinterpret_cast<uintptr_t>(b_in) |
                 reinterpret_cast<uintptr_t>(z)) % 16 == 0, "x, W_in, b_in and z must be 16-byte aligned");
    MTL_REQUIRE(conv_state_in != conv_state_out, "conv_state_out must not alias conv_state_in");
    const int64_t M = batch * seqlen;
    LinArgs a{x, W_in, b_in, nullptr, x_rs, 0, 0, (int)M, (int)(2 * d_inner), (int)d_model, 1};
    const PrefillConvArgs c{conv_state_in, conv_state_out, conv_w, conv_b, u, z, (int)d_inner, (int)seqlen};
    const dim3 grid((unsigned)(2 * d_inner / 16));
    hipStream_t st = as_stream(stream);
    if (d_conv == 2) hipLaunchKernelGGL((in_conv_prefill_kernel<1, 2>), grid, dim3(kLinThreads), 0, st, a, c);
    else if (d_conv == 3) hipLaunchKernelGGL((in_conv_prefill_kernel<1, 3>), grid, dim3(kLinThreads), 0, st, a, c);
    else hipLaunchKernelGGL((in_conv_prefill_kernel<1, 4>), grid, dim3(kLinThreads), 0, st, a, c);
    return check_launch("in_conv_prefill_kernel");
}

extern "C" int mtl_linear_skinny_residual(const float* x, int64_t x_rs, const float* W, const float* bias,
                                          float* parts, int64_t M, int64_t N, int64_t K, int32_t ksplit,
                                          int32_t rows_per_block, float* h, const float* w_next, float* x_next,
                                          float* sq, uint32_t* counters, mtl_stream_t stream) {
    clear_error();
    MTL_REQUIRE(x && W && parts && h && w_next && x_next && sq && counters, "null required pointer");
    MTL_REQUIRE(M >= 1 && M <= 32, "M (rows of x) must be in [1, 32]");
    MTL_REQUIRE(rows_per_block == 16 || rows_per_block == 32, "rows_per_block must be 16 or 32");
    MTL_REQUIRE(N >= rows_per_block && N % rows_per_block == 0 && N < (int64_t(1) << 30),
                "N must be a positive multiple of rows_per_block");
    MTL_REQUIRE(ksplit >= 1 && ksplit <= kResidMaxSplit, "ksplit must be in [1, 4]");
    MTL_REQUIRE(K >= 1 && K % (int64_t(kKC) * ksplit) == 0 && K < (int64_t(1) << 31),
                "K must be a positive multiple of 128 * ksplit");
    MTL_REQUIRE(x_rs >= K && x_rs % 4 == 0, "x row stride must cover a row and be a multiple of 4");
    MTL_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(bias) |
                 reinterpret_cast<uintptr_t>(parts) | reinterpret_cast<uintptr_t>(h) |
                 reinterpret_cast<uintptr_t>(w_next) | reinterpret_cast<uintptr_t>(x_next)) % 16 == 0,
                "x, W, bias, parts, h, w_next and x_next must be 16-byte aligned");
    MTL_REQUIRE(x_next != h, "x_next must not alias h");
    LinArgs a{x, W, bias, parts, x_rs, N, M * N, (int)M, (int)N, (int)K, (int)ksplit};
    const ResidArgs r{h, w_next, x_next, sq, counters};
    hipStream_t st = as_stream(stream);
    if (rows_per_block == 32) {
        if (M > 16) launch_resid<2, 2>(a, r, st); else launch_resid<2, 1>(a, r, st);
    } else {
        if (M > 16) launch_resid<1, 2>(a, r, st); else launch_resid<1, 1>(a, r, st);
    }
    return check_launch("linear_resid_kernel");
}

static int in_proj_conv_xproj(const float* x, int64_t x_rs, const float* W_in, const float* b_in, float* conv_state,
                              const float* conv_w, const float* conv_b, int32_t d_conv, const float* W_xT, int32_t J,
                              float* xc, float* z, int64_t z_rs, float* xpart, int64_t batch, int64_t d_model,
                              int64_t d_inner, int32_t channels_per_part, const float* sq, int32_t sq_tiles, float eps,
                              mtl_stream_t stream) {
    MTL_REQUIRE(x && W_in && conv_state && conv_w && W_xT && xc && z && xpart, "null required pointer");
    MTL_REQUIRE(batch >= 1 && batch <= 32, "batch must be in [1, 32]");
    MTL_REQUIRE(d_model >= 2 * kKC && d_model % kKC == 0 && d_model < (int64_t(1) << 30),
                "d_model must be a multiple of 128, at least 256");
    MTL_REQUIRE(channels_per_part == 16 || channels_per_part == 32, "channels_per_part must be 16 or 32");
    MTL_REQUIRE(d_inner >= channels_per_part && d_inner % channels_per_part == 0 && d_inner < (int64_t(1) << 29),
                "d_inner must be a positive multiple of channels_per_part");
    MTL_REQUIRE(d_conv >= 2 && d_conv <= 4, "d_conv must be 2, 3 or 4");
    MTL_REQUIRE(J >= 1 && J <= kIcMaxJ, "J (x_proj rows) must be in [1, 288]");
    MTL_REQUIRE(x_rs >= d_model && x_rs % 4 == 0 && z_rs >= d_inner && z_rs % 4 == 0,
                "row strides must cover a row and be multiples of 4");
    MTL_REQUIRE((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(W_in) | reinterpret_cast<uintptr_t>(b_in) |
                 reinterpret_cast<uintptr_t>(conv_state) | reinterpret_cast<uintptr_t>(conv_w) |
                 reinterpret_cast<uintptr_t>(conv_b) | reinterpret_cast<uintptr_t>(xc) |
                 reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(W_xT)) % 16 == 0,
                "x, W_in, b_in, conv_state, conv_w, conv_b, W_xT, xc and z must be 16-byte aligned");
    LinArgs a{x, W_in, b_in, nullptr, x_rs, 0, 0, (int)batch, (int)(2 * d_inner), (int)d_model, 1};
    InConvArgs c{conv_state, conv_w, conv_b, W_xT, xc, z, xpart, sq, z_rs, (int)d_inner, (int)J, (int)sq_tiles, eps};
    hipStream_t st = as_stream(stream);
    const bool two_m = batch > 16;
    if (channels_per_part == 32) {
        if (two_m) dispatch_in_conv<2, 2>(d_conv, a, c, st); else dispatch_in_conv<2, 1>(d_conv, a, c, st);
    } else {
        if (two_m) dispatch_in_conv<1, 2>(d_conv, a, c, st); else dispatch_in_conv<1, 1>(d_conv, a, c, st);
    }
    return check_launch("in_conv_xproj_kernel");
}

extern "C" int mtl_in_proj_conv_xproj(const float* x, int64_t x_rs, const float* W_in, const float* b_in,
                                      float* conv_state, const float* conv_w, const float* conv_b, int32_t d_conv,
                                      const float* W_xT, int32_t J, float* xc, float* z, int64_t z_rs, float* xpart,
                                      int64_t batch, int64_t d_model, int64_t d_inner, int32_t channels_per_part,
                                      mtl_stream_t stream) {
    clear_error();
    return in_proj_conv_xproj(x, x_rs, W_in, b_in, conv_state, conv_w, conv_b, d_conv, W_xT, J, xc, z, z_rs, xpart,
                              batch, d_model, d_inner, channels_per_part, nullptr, 0, 0.f, stream);
}

extern "C" int mtl_in_proj_conv_xproj_normed(const float* x, int64_t x_rs, const float* W_in, const float* b_in,
                                             float* conv_state, const float* conv_w, const float* conv_b,
                                             int32_t d_conv, const float* W_xT, int32_t J, float* xc, float* z,
                                             int64_t z_rs, float* xpart, int64_t batch, int64_t d_model,
                                             int64_t d_inner, int32_t channels_per_part, const float* sq,
                                             int32_t sq_tiles, float eps, mtl_stream_t stream) {
    clear_error();
    MTL_REQUIRE(sq, "null sq");
    MTL_REQUIRE(sq_tiles >= 1 && sq_tiles <= 8 * kSqPerThread, "sq_tiles must be in [1, 128]");
    MTL_REQUIRE(eps >= 0.f, "eps must be >= 0");
    return in_proj_conv_xproj(x, x_rs, W_in, b_in, conv_state, conv_w, conv_b, d_conv, W_xT, J, xc, z, z_rs, xpart,
                              batch, d_model, d_inner, channels_per_part, sq, sq_tiles, eps, stream);
}
