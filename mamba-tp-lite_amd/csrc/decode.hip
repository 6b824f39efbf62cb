// Fused single-token decode step for small batch (b in {1, 2, 4}), fp32, gfx950.
//
// One Mamba block step (reference model.py:308-311 around MambaMixer.step,
// model.py:249-294) in three or four kernels instead of one per ATen op:
//
//   decode_in    residual rows (or the embedding rows for the first layer,
//                model.py:348) -> RMSNorm (model.py:130-135) -> the in_proj
//                rows of this workgroup's channel block (model.py:261) ->
//                conv step with the in-place history shift + SiLU (264-277)
//                -> SiLU(z) (292) -> optionally the x_proj split-K partial
//                sums over the block (279)
//   decode_gemv  out = W v (+ residual): the x_proj rows (279) when x_proj
//                runs as its own kernel, and the out_proj rows (293) with the
//                residual add (311)
//   decode_ssm   x_dbl = the x_proj partials summed in block order ->
//                dt_proj + softplus (281-282) -> state update in place
//                (284-289) -> y = C.h + D x, * SiLU(z) (290-292)
//
// A decode step is latency-bound: every kernel moves a few MB and each
// dependent memory round trip costs about a microsecond.  So each kernel
// issues every load that does not depend on another load first -- weight
// rows as float4 runs (lane l holds float4s l, l+64, ...), conv history,
// norm weights, the activation rows -- with fixed, unrolled counts and
// clamped addresses (masks are applied where values are consumed), so the
// loads go out back to back and the kernel waits for memory once.
// Reductions use DPP lane moves.  No atomics: split-K partials are summed in
// a fixed order, so a step is deterministic and a graph replay equals eager
// execution bit for bit.

#include "common.h"

namespace mtl {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxPL = kMaxRuns;                   // float4 runs per lane: rows of up to 4096 floats
static_assert(kWaves == 4, "the block reductions below add 4 wavefront sums");

template <int B>
__device__ __forceinline__ void wave_sum(float* v) {
#pragma unroll
    for (int i = 0; i < B; ++i) v[i] = group_sum<64>(v[i]);
}

// Weight rows are read once per token and are larger than the caches (516 MB
// at the 130m shape), so they are loaded nontemporally: 130m batch 1 went
// from 338.5 to 320.3 us per token and 1.4b batch 1 from 1517 to 1468 us.
__device__ __forceinline__ float4 ntload4(const float4* p) {
    typedef float F4 __attribute__((ext_vector_type(4)));
    const F4 v = __builtin_nontemporal_load(reinterpret_cast<const F4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float dot4(const float4 w, const float4 x, float acc) {
    return fmaf(w.x, x.x, fmaf(w.y, x.y, fmaf(w.z, x.z, fmaf(w.w, x.w, acc))));
}

// ---------------------------------------------------------------- decode_in
struct InArgs {
    const float* x;          // [b, M] residual stream (null for the first layer)
    const float* emb;        // [V, M] embedding table (first layer)
    const int64_t* ids;      // [b] token ids (first layer)
    int V;                   // rows of emb
    float* resid_out;        // [b, M] residual copy written by block 0 (first layer), else null
    const float* norm_w;     // [M]
    const float* W_in;       // [2D, M]
    const float* b_in;       // [2D] or null
    float* conv_state;       // [b, D, K-1], in place
    const float* conv_w;     // [D, K]
    const float* conv_b;     // [D] or null
    const float* W_xT;       // [D, J] x_proj transposed, or null (x_proj in its own kernel)
    float* xc;               // [b, D]
    float* gz;               // [b, D]
    float* xpart;            // [nblk, b, J] or null
    int M, D, K, J;
    float eps;
};

// channels per decode_in workgroup: 8 (2 in_proj rows per wavefront), or 4
// (one row per wavefront, twice the workgroups on the weight stream)
constexpr int kMaxConv = 8;                        // d_conv <= 8

// PL = float4 runs per lane (M <= 256 * PL; lanes past M/4 in the last run
// are masked).  Every wavefront: 2 in_proj rows.  Every thread: PL elements
// of each activation row and of the norm weights.
//
// The grid is two sets of nblk workgroups over the same channel blocks: the
// first takes the x rows of in_proj (then the conv step and the x_proj
// partials), the second the z rows (then SiLU(z)).  Halving the rows per
// workgroup puts the weight stream on twice as many CUs, so more of it is in
// flight at once.
template <int B, int PL, int CB>
__global__ void __launch_bounds__(kThreads) decode_in_kernel(const InArgs a) {
    constexpr int G = CB / kWaves;                // in_proj rows per wavefront
    static_assert(G >= 1 && G * kWaves == CB, "channels per workgroup");
    extern __shared__ __align__(16) float s_xw[];  // [B][M]: norm_w * x (the rms scale is applied to the dots)
    __shared__ float s_pre[CB][B];
    __shared__ float s_xc[CB][B];
    __shared__ float s_red[B][kWaves];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int M = a.M, D = a.D, J = a.J, K = a.K;
    const int K4 = M >> 2;
    const int nblk = (D + CB - 1) / CB;
    const bool zblk = (int)blockIdx.x >= nblk;     // uniform: this workgroup takes the z rows
    const int blk = zblk ? (int)blockIdx.x - nblk : (int)blockIdx.x;
    const int c0 = blk * CB;
    const int nch = min(CB, D - c0);

    // ---- 0. every independent load, in one batch
    const float* rows[G];
    int rloc[G];
    float bin[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int ch = wave * G + g;               // local row = channel of the block
        const bool ok = ch < nch;
        const int64_t row = (zblk ? (int64_t)D : 0) + c0 + (ok ? ch : 0);
        rows[g] = a.W_in + row * M;
        rloc[g] = ok ? ch : -1;
        bin[g] = a.b_in ? a.b_in[row] : 0.f;
    }
    float4 w[G][PL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int p = 0; p < PL; ++p)
            w[g][p] = ntload4(reinterpret_cast<const float4*>(rows[g]) + min(p * 64 + lane, K4 - 1));

    // conv operands of (channel, batch) pair tid (clamped to a valid pair)
    const int npair = nch * B;
    const int pt = min(tid, npair - 1);
    const int cv_ch = pt % nch, cv_b = pt / nch, cv_c = c0 + cv_ch;
    float* stp = a.conv_state + ((int64_t)cv_b * D + cv_c) * (K - 1);
    float cst[kMaxConv - 1], cw[kMaxConv];
#pragma unroll
    for (int k = 0; k < kMaxConv - 1; ++k) cst[k] = stp[min(k, K - 2)];
#pragma unroll
    for (int k = 0; k < kMaxConv; ++k) cw[k] = a.conv_w[(int64_t)cv_c * K + min(k, K - 1)];
    const float cbias = a.conv_b ? a.conv_b[cv_c] : 0.f;

    // x_proj columns of (j, batch) pair tid over the block's channels
    float wx[CB];
    const int xt = min(tid, J * B - 1);
    const int xp_j = xt % J, xp_b = xt / J;
    if (a.W_xT) {
#pragma unroll
        for (int ch = 0; ch < CB; ++ch) wx[ch] = a.W_xT[(int64_t)(c0 + min(ch, nch - 1)) * J + xp_j];
    }

    // activation rows and norm weights: element e = tid + 256 q
    // A token id outside [0, V) reads row 0 instead and turns that batch
    // row's residual into NaN, so its logits come out NaN (no device trap,
    // no read outside the table).
    const float* rows_in[B];
    bool id_ok[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) {
        if (a.x) {
            rows_in[bi] = a.x + (int64_t)bi * M;
            id_ok[bi] = true;
        } else {
            const int64_t id = a.ids[bi];
            id_ok[bi] = id >= 0 && id < a.V;
            rows_in[bi] = a.emb + (id_ok[bi] ? id : 0) * (int64_t)M;
        }
    }
    float xv[B][PL], nw[PL];
#pragma unroll
    for (int q = 0; q < PL; ++q) {
        const int e = min(tid + q * kThreads, M - 1);
        nw[q] = a.norm_w[e];
#pragma unroll
        for (int bi = 0; bi < B; ++bi) xv[bi][q] = rows_in[bi][e];
    }
#pragma unroll
    for (int bi = 0; bi < B; ++bi)
#pragma unroll
        for (int q = 0; q < PL; ++q) xv[bi][q] = id_ok[bi] ? xv[bi][q] : __builtin_nanf("");

    // ---- 1. sum of squares; norm_w * x into LDS
    float ss[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) ss[bi] = 0.f;
#pragma unroll
    for (int q = 0; q < PL; ++q) {
        const int e = tid + q * kThreads;
        if (e < M) {
#pragma unroll
            for (int bi = 0; bi < B; ++bi) {
                ss[bi] = fmaf(xv[bi][q], xv[bi][q], ss[bi]);
                s_xw[bi * M + e] = nw[q] * xv[bi][q];
                if (a.resid_out && blockIdx.x == 0) a.resid_out[(int64_t)bi * M + e] = xv[bi][q];
            }
        }
    }
    wave_sum<B>(ss);
    if (lane == 0)
#pragma unroll
        for (int bi = 0; bi < B; ++bi) s_red[bi][wave] = ss[bi];
    __syncthreads();

    // ---- 2. in_proj rows: <W row, norm_w * x> * rsqrt(mean(x^2) + eps)
    float r[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi)
        r[bi] = rsqrtf(((s_red[bi][0] + s_red[bi][1]) + (s_red[bi][2] + s_red[bi][3])) / (float)M + a.eps);
    const bool tail_ok = (PL - 1) * 64 + lane < K4;
    float acc[G][B];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int bi = 0; bi < B; ++bi) acc[g][bi] = 0.f;
#pragma unroll
    for (int p = 0; p < PL; ++p) {
        const bool ok = p < PL - 1 || tail_ok;
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            const float4 x4 = reinterpret_cast<const float4*>(s_xw + (size_t)bi * M)[min(p * 64 + lane, K4 - 1)];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float t = dot4(w[g][p], x4, acc[g][bi]);
                acc[g][bi] = ok ? t : acc[g][bi];
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) wave_sum<B>(acc[g]);
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (rloc[g] < 0) continue;   // rows past d_inner
#pragma unroll
            for (int bi = 0; bi < B; ++bi) s_pre[rloc[g]][bi] = fmaf(acc[g][bi], r[bi], bin[g]);
        }
    }
    __syncthreads();

    // ---- 3. z blocks: SiLU(z); x blocks: conv step (history shifted in place) + SiLU
    if (zblk) {
        if (tid < npair) a.gz[(int64_t)cv_b * D + cv_c] = silu_f(s_pre[cv_ch][cv_b]);
        return;
    }
    if (tid < npair) {
        const float xin = s_pre[cv_ch][cv_b];
        float cacc = 0.f;
#pragma unroll
        for (int k = 0; k < kMaxConv - 1; ++k)
            if (k < K - 1) cacc = fmaf(cst[k], cw[k], cacc);
#pragma unroll
        for (int k = 0; k < kMaxConv; ++k)
            if (k == K - 1) cacc = fmaf(xin, cw[k], cacc);
        cacc += cbias;
#pragma unroll
        for (int k = 0; k < kMaxConv - 2; ++k)
            if (k < K - 2) stp[k] = cst[k + 1];
        stp[K - 2] = xin;
        const float xcv = silu_f(cacc);
        s_xc[cv_ch][cv_b] = xcv;
        a.xc[(int64_t)cv_b * D + cv_c] = xcv;
    }
    if (!a.W_xT) return;
    __syncthreads();

    // ---- 4. x_proj partial sums over this block's channels
    if (tid < J * B) {
        float xacc = 0.f;
#pragma unroll
        for (int ch = 0; ch < CB; ++ch) xacc = ch < nch ? fmaf(wx[ch], s_xc[ch][xp_b], xacc) : xacc;
        a.xpart[((int64_t)blk * B + xp_b) * J + xp_j] = xacc;
    }
    for (int t = tid + kThreads; t < J * B; t += kThreads) {   // pairs beyond the first 256
        const int j = t % J, bi = t / J;
        float xacc = 0.f;
        for (int ch = 0; ch < nch; ++ch) xacc = fmaf(a.W_xT[(int64_t)(c0 + ch) * J + j], s_xc[ch][bi], xacc);
        a.xpart[((int64_t)blk * B + bi) * J + j] = xacc;
    }
}

// ---------------------------------------------------------------- decode_gemv
struct GemvArgs {
    const float* v;          // [b, K]
    const float* W;          // [Mrows, K]
    const float* bias;       // [Mrows] or null
    const float* x_in;       // [b, Mrows] residual or null
    float* out;              // [b, Mrows]
    int Mrows, K;
    const float* norm_w;     // [K]: v is RMS-normalized with these weights first (NORM kernels)
    float eps;
    int ld;                  // row stride of W and v (the split kernel's parts: K = ld / parts)
    int64_t out_ps;          // split kernel: part p writes out + p * out_ps
};

// one wavefront per output row, 4 rows per workgroup; K <= 256 * PL.
// NORM: out = (W . (norm_w * v)) * rsqrt(mean(v^2) + eps) + bias -- the final
// RMSNorm folded into the lm_head rows (every workgroup recomputes the rms of
// the few-kB vector instead of waiting for a separate norm kernel)
// Batch 1 and 2 without the norm: one wavefront per workgroup and per row,
// v read straight from global memory (a few KB per batch row, in L2 after
// the first workgroups), so a row needs no LDS stage and no barrier.  Four
// times the workgroups of the form below on the same weight stream: the
// mamba-1.4b decode step went 1410-1415 -> 1401-1406 us/token at batch 1 and
// 1712 -> 1664 us/step at batch 2, the 130m one 322.5-324 -> 320.5-321.5
// and 414 -> 403 (same dot-product order, the same bits).
template <int B, int PL>
__global__ void __launch_bounds__(64) decode_gemv_row_kernel(const GemvArgs a) {
    const int lane = threadIdx.x;
    const int K = a.K, K4 = K >> 2;
    const int m = blockIdx.x;
    const float4* row = reinterpret_cast<const float4*>(a.W + (int64_t)m * K);
    float4 w[PL];
#pragma unroll
    for (int p = 0; p < PL; ++p) w[p] = ntload4(row + min(p * 64 + lane, K4 - 1));
    const float bias = a.bias ? a.bias[m] : 0.f;
    float xin[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) xin[bi] = a.x_in ? a.x_in[(int64_t)bi * a.Mrows + m] : 0.f;
    const bool tail_ok = (PL - 1) * 64 + lane < K4;
    float acc[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) acc[bi] = 0.f;
#pragma unroll
    for (int p = 0; p < PL; ++p)
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            const float4* v4 = reinterpret_cast<const float4*>(a.v + (int64_t)bi * K);
            const float t = dot4(w[p], v4[min(p * 64 + lane, K4 - 1)], acc[bi]);
            acc[bi] = p < PL - 1 || tail_ok ? t : acc[bi];
        }
    wave_sum<B>(acc);
    if (lane == 0)
#pragma unroll
        for (int bi = 0; bi < B; ++bi)
            a.out[(int64_t)bi * a.Mrows + m] = a.x_in ? xin[bi] + (acc[bi] + bias) : acc[bi] + bias;
}

template <int B, int PL, bool NORM = false>
__global__ void __launch_bounds__(kThreads) decode_gemv_kernel(const GemvArgs a) {
    extern __shared__ __align__(16) float s_v[];      // [B][K]
    __shared__ float s_red[B][kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K, K4 = K >> 2;
    const int m = min((int)blockIdx.x * kWaves + wave, a.Mrows - 1);
    const float4* row = reinterpret_cast<const float4*>(a.W + (int64_t)m * K);
    float4 w[PL];
#pragma unroll
    for (int p = 0; p < PL; ++p) w[p] = ntload4(row + min(p * 64 + lane, K4 - 1));
    const float bias = a.bias ? a.bias[m] : 0.f;
    float xin[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) xin[bi] = a.x_in ? a.x_in[(int64_t)bi * a.Mrows + m] : 0.f;
    float vv[B][PL], nw[PL];
#pragma unroll
    for (int q = 0; q < PL; ++q) {
        if constexpr (NORM) nw[q] = a.norm_w[min(tid + q * kThreads, K - 1)];
#pragma unroll
        for (int bi = 0; bi < B; ++bi) vv[bi][q] = a.v[(int64_t)bi * K + min(tid + q * kThreads, K - 1)];
    }
    if constexpr (NORM) {
        float ss[B];
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            ss[bi] = 0.f;
#pragma unroll
            for (int q = 0; q < PL; ++q) ss[bi] = tid + q * kThreads < K ? fmaf(vv[bi][q], vv[bi][q], ss[bi]) : ss[bi];
        }
        wave_sum<B>(ss);
        if (lane == 0)
#pragma unroll
            for (int bi = 0; bi < B; ++bi) s_red[bi][wave] = ss[bi];
    }
#pragma unroll
    for (int q = 0; q < PL; ++q)
        if (tid + q * kThreads < K)
#pragma unroll
            for (int bi = 0; bi < B; ++bi) s_v[bi * K + tid + q * kThreads] = NORM ? nw[q] * vv[bi][q] : vv[bi][q];
    __syncthreads();
    if ((int)blockIdx.x * kWaves + wave >= a.Mrows) return;   // whole wavefront
    float rs[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi)
        rs[bi] = NORM ? rsqrtf(((s_red[bi][0] + s_red[bi][1]) + (s_red[bi][2] + s_red[bi][3])) / (float)K + a.eps) : 1.f;

    const bool tail_ok = (PL - 1) * 64 + lane < K4;
    float acc[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) acc[bi] = 0.f;
#pragma unroll
    for (int p = 0; p < PL; ++p) {
        const bool ok = p < PL - 1 || tail_ok;
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            const float4 x4 = reinterpret_cast<const float4*>(s_v + (size_t)bi * K)[min(p * 64 + lane, K4 - 1)];
            const float t = dot4(w[p], x4, acc[bi]);
            acc[bi] = ok ? t : acc[bi];
        }
    }
    wave_sum<B>(acc);
    if (lane == 0) {
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            const float o = NORM ? fmaf(acc[bi], rs[bi], bias) : acc[bi] + bias;
            a.out[(int64_t)bi * a.Mrows + m] = a.x_in ? xin[bi] + o : o;
        }
    }
}

// Few long rows (x_proj at d_inner 4096: 160 rows): one workgroup per row
// and column part (blockIdx.y: columns [p K, (p + 1) K) of rows of length
// ld), the 4 wavefronts take quarters of it (PLW float4 runs per lane each,
// K <= 1024 PLW) and their sums are added in wavefront order; part p writes
// its partial product to out + p * out_ps (bias and x_in in part 0).  The
// products are the LDS-staged form's, in the same order, so the bits are
// unchanged (1.4b b=1 x_proj: one barrier instead of three).
template <int B, int PLW>
__global__ void __launch_bounds__(kThreads) decode_gemv_split_kernel(const GemvArgs a) {
    __shared__ float s_sum[kWaves][B];                // the wavefront sums
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int K = a.K, K4 = K >> 2;
    const int m = blockIdx.x, part = blockIdx.y;
    const int64_t k0 = (int64_t)part * K;
    const float4* row = reinterpret_cast<const float4*>(a.W + (int64_t)m * a.ld + k0);
    float4 w[PLW];
#pragma unroll
    for (int p = 0; p < PLW; ++p) w[p] = ntload4(row + min((wave * PLW + p) * 64 + lane, K4 - 1));
    const float bias = a.bias && part == 0 ? a.bias[m] : 0.f;
    const bool add_x = a.x_in && part == 0;
    float xin[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) xin[bi] = add_x ? a.x_in[(int64_t)bi * a.Mrows + m] : 0.f;
    // v straight from global memory (a few KB, in L2 after the first
    // workgroups): each lane reads the float4 runs it multiplies, so there
    // is no LDS stage and no barrier before the products
    float4 xv[B][PLW];
#pragma unroll
    for (int p = 0; p < PLW; ++p)
#pragma unroll
        for (int bi = 0; bi < B; ++bi)
            xv[bi][p] = reinterpret_cast<const float4*>(a.v + (int64_t)bi * a.ld + k0)
                [min((wave * PLW + p) * 64 + lane, K4 - 1)];

    float acc[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) acc[bi] = 0.f;
#pragma unroll
    for (int p = 0; p < PLW; ++p) {
        const bool ok = (wave * PLW + p) * 64 + lane < K4;
#pragma unroll
        for (int bi = 0; bi < B; ++bi) {
            const float t = dot4(w[p], xv[bi][p], acc[bi]);
            acc[bi] = ok ? t : acc[bi];
        }
    }
    wave_sum<B>(acc);
    if (lane == 0)
#pragma unroll
        for (int bi = 0; bi < B; ++bi) s_sum[wave][bi] = acc[bi];
    __syncthreads();
    if (tid < B) {
        const float o = ((s_sum[0][tid] + s_sum[1][tid]) + (s_sum[2][tid] + s_sum[3][tid])) + bias;
        a.out[part * a.out_ps + (int64_t)tid * a.Mrows + m] = add_x ? xin[tid] + o : o;
    }
}

// ---------------------------------------------------------------- decode_ssm
struct SsmArgs {
    const float* xpart;      // [nblk, b, J]
    int nblk;
    const float* xc;         // [b, D]
    const float* gz;         // [b, D]
    const float* W_dt;       // [D, R]
    const float* b_dt;       // [D]
    const float* A_log;      // [D, N]
    const float* Dv;         // [D] or null
    float* ssm_state;        // [b, D, N], in place
    float* y;                // [b, D]
    int D, N, R, J;
};

constexpr int kSsmChannels = kThreads / 16;   // one 16-lane DPP row per channel
constexpr int kPartBatch = 64;                // partial loads in flight per thread

// RQ = dt_proj columns per lane (R <= 16 * RQ)
template <int B, int RQ>
__global__ void __launch_bounds__(kThreads) decode_ssm_kernel(const SsmArgs a) {
    extern __shared__ __align__(16) float s_xd[];     // [B][J] sums, then [Q][B*J] range sums
    const int tid = threadIdx.x;
    const int J = a.J, R = a.R, N = a.N, D = a.D;

    // ---- 0. per-channel operands (independent of x_dbl): lane n of the
    //      16-lane row owns state n and dt_proj columns n, n+16, ...
    const int g = tid >> 4, n = tid & 15;
    const int cc = min((int)blockIdx.x * kSsmChannels + g, D - 1);
    const int nn = min(n, N - 1);
    float wdt[RQ];
#pragma unroll
    for (int q = 0; q < RQ; ++q) wdt[q] = a.W_dt[(int64_t)cc * R + min(n + 16 * q, R - 1)];
    const float alog = a.A_log[(int64_t)cc * N + nn];
    const float bdt = a.b_dt[cc];
    const float Dc = a.Dv ? a.Dv[cc] : 0.f;
    float hst[B], xvs[B], gzs[B];
#pragma unroll
    for (int bi = 0; bi < B; ++bi) {
        hst[bi] = a.ssm_state[((int64_t)bi * D + cc) * N + nn];
        xvs[bi] = a.xc[(int64_t)bi * D + cc];
        gzs[bi] = a.gz[(int64_t)bi * D + cc];
    }

    // ---- 1. x_dbl = sum of the x_proj partials in block order.  Q threads
    //      per (j, b) pair each sum a contiguous range of at most kPartBatch
    //      blocks (one batch of loads); the Q range sums are then added in
    //      order.
    const int pairs = J * B;
    const int Q = max(1, min(kThreads / pairs, 8));
    const int per = (a.nblk + Q - 1) / Q;             // <= kPartBatch (checked on the host)
    float* s_q = s_xd + pairs;
    const int64_t stride = (int64_t)B * J;
    for (int t = tid; t < pairs * Q; t += kThreads) {
        const int pr = t % pairs, q = t / pairs;
        const int k0 = q * per, nk = min(a.nblk - k0, per);
        const float* p = a.xpart + pr;
        float v[kPartBatch];
#pragma unroll
        for (int u = 0; u < kPartBatch; ++u) v[u] = p[(int64_t)min(k0 + u, a.nblk - 1) * stride];
        float s = 0.f;
#pragma unroll
        for (int u = 0; u < kPartBatch; ++u) s += u < nk ? v[u] : 0.f;
        s_q[q * pairs + pr] = s;
    }
    __syncthreads();
    for (int pr = tid; pr < pairs; pr += kThreads) {
        float s = s_q[pr];
        for (int q = 1; q < Q; ++q) s += s_q[q * pairs + pr];
        s_xd[pr] = s;
    }
    __syncthreads();

    // ---- 2. per channel: dt, state update, y
    const int c = blockIdx.x * kSsmChannels + g;
    if (c >= D) return;  // whole 16-lane row
    const float av = -expf(alog);
#pragma unroll
    for (int bi = 0; bi < B; ++bi) {
        const float* xd = s_xd + bi * J;
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < RQ; ++q) {
            const float t = fmaf(wdt[q], xd[min(n + 16 * q, R - 1)], acc);
            acc = n + 16 * q < R ? t : acc;
        }
        acc = group_sum<16>(acc);
        const float dt = softplus_f(acc + bdt);
        const float xv = xvs[bi];
        float yv = 0.f;
        if (n < N) {
            const float dA = __builtin_amdgcn_exp2f(dt * (av * kLog2e));
            const float hv = fmaf(hst[bi], dA, (dt * xd[R + n]) * xv);
            a.ssm_state[((int64_t)bi * D + c) * N + n] = hv;
            yv = hv * xd[R + N + n];
        }
        yv = group_sum<16>(yv);
        if (n == 0) a.y[(int64_t)bi * D + c] = (yv + xv * Dc) * gzs[bi];
    }
}

#define MTL_DISPATCH_B(BV, ...)                                    \
    switch (BV) {                                                  \
        case 1: { constexpr int B = 1; __VA_ARGS__; } break;       \
        case 2: { constexpr int B = 2; __VA_ARGS__; } break;       \
        default: { constexpr int B = 4; __VA_ARGS__; } break;      \
    }
}  // namespace
}  // namespace mtl

extern "C" int mtl_decode_in(const float* x, const float* emb, const int64_t* ids, int32_t vocab, float* resid_out,
                             const float* norm_w, float eps, const float* W_in, const float* b_in, float* conv_state,
                             const float* conv_w, const float* conv_b, const float* W_xT, float* xc, float* gz,
                             float* xpart, int32_t batch, int32_t d_model, int32_t d_inner, int32_t d_conv,
                             int32_t xdbl_cols, int32_t channels_per_block, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch == 1 || batch == 2 || batch == 4, "batch must be 1, 2 or 4");
    MTL_REQUIRE(d_model >= 4 && d_model % 4 == 0 && d_model <= 256 * kMaxPL,
                "d_model must be a multiple of 4 in [4, 4096]");
    MTL_REQUIRE(d_inner >= 1 && d_conv >= 2 && d_conv <= kMaxConv && xdbl_cols >= 1, "bad sizes");
    MTL_REQUIRE(channels_per_block == 8 || channels_per_block == 4, "channels_per_block must be 8 or 4");
    MTL_REQUIRE((x != nullptr) != (emb != nullptr && ids != nullptr), "give either x or (emb, ids)");
    MTL_REQUIRE(x != nullptr || vocab >= 1, "vocab must be >= 1 with (emb, ids)");
    MTL_REQUIRE(norm_w && W_in && conv_state && conv_w && xc && gz, "null required pointer");
    MTL_REQUIRE((W_xT == nullptr) == (xpart == nullptr), "W_xT and xpart go together");
    MTL_REQUIRE(((uintptr_t)W_in % 16) == 0, "W_in must be 16-byte aligned");
    const size_t smem = sizeof(float) * (size_t)batch * d_model;
    MTL_REQUIRE(smem <= 60 * 1024, "batch * d_model too large for the decode LDS tile");
    InArgs a{x, emb, ids, vocab, resid_out, norm_w, W_in, b_in, conv_state, conv_w, conv_b, W_xT, xc, gz, xpart,
             d_model, d_inner, d_conv, xdbl_cols, eps};
    const int cb = channels_per_block;
    const dim3 grid((unsigned)(2 * ((d_inner + cb - 1) / cb)));   // x-row blocks, then z-row blocks
    hipStream_t st = as_stream(stream);
    const int plv = round_runs((d_model / 4 + 63) / 64);
    if (cb == 8) {
        MTL_DISPATCH_B(batch, MTL_DISPATCH_RUNS(PL, plv, hipLaunchKernelGGL((decode_in_kernel<B, PL, 8>), grid,
                                                                      dim3(kThreads), smem, st, a)));
    } else {
        MTL_DISPATCH_B(batch, MTL_DISPATCH_RUNS(PL, plv, hipLaunchKernelGGL((decode_in_kernel<B, PL, 4>), grid,
                                                                      dim3(kThreads), smem, st, a)));
    }
    return check_launch("decode_in");
}

extern "C" int mtl_decode_gemv(const float* v, const float* W, const float* bias, const float* x_in, float* out,
                               int32_t batch, int32_t rows, int32_t cols, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch == 1 || batch == 2 || batch == 4, "batch must be 1, 2 or 4");
    MTL_REQUIRE(cols >= 4 && cols % 4 == 0 && cols <= 256 * kMaxPL && rows >= 1,
                "cols must be a multiple of 4 in [4, 4096]");
    MTL_REQUIRE(v && W && out, "null required pointer");
    MTL_REQUIRE(((uintptr_t)W % 16) == 0 && ((uintptr_t)v % 16) == 0, "W and v must be 16-byte aligned");
    MTL_REQUIRE(x_in == nullptr || x_in != out, "out must not alias x_in");
    const size_t smem = sizeof(float) * (size_t)batch * cols;
    MTL_REQUIRE(smem <= 64 * 1024, "batch * cols too large for the decode LDS tile");
    GemvArgs a{v, W, bias, x_in, out, rows, cols, nullptr, 0.f, cols, 0};
    hipStream_t st = as_stream(stream);
    const int runs = (cols / 4 + 63) / 64;
    if (rows < 128 * kWaves && runs >= 2 * kWaves) {
        // few long rows: a workgroup per row, split four ways
        const int plw = round_runs((runs + kWaves - 1) / kWaves);
        MTL_REQUIRE(plw * kWaves <= kMaxPL, "internal: split GEMV run count");
        MTL_DISPATCH_B(batch, MTL_DISPATCH_RUNS(PLW, plw,
            if constexpr (PLW * kWaves <= kMaxPL) hipLaunchKernelGGL((decode_gemv_split_kernel<B, PLW>),
                dim3((unsigned)rows), dim3(kThreads), 0, st, a)));
    } else if (batch <= 2) {
        if (batch == 1) {
            MTL_DISPATCH_RUNS(PL, round_runs(runs), hipLaunchKernelGGL((decode_gemv_row_kernel<1, PL>),
                                                                       dim3((unsigned)rows), dim3(64), 0, st, a));
        } else {
            MTL_DISPATCH_RUNS(PL, round_runs(runs), hipLaunchKernelGGL((decode_gemv_row_kernel<2, PL>),
                                                                       dim3((unsigned)rows), dim3(64), 0, st, a));
        }
    } else {
        const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
        MTL_DISPATCH_B(batch, MTL_DISPATCH_RUNS(PL, round_runs(runs), hipLaunchKernelGGL((decode_gemv_kernel<B, PL>),
                                                                  grid, dim3(kThreads), smem, st, a)));
    }
    return check_launch("decode_gemv");
}

extern "C" int mtl_decode_gemv_parts(const float* v, const float* W, float* out_parts, int32_t batch, int32_t rows,
                                     int32_t cols, int32_t nparts, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch == 1 || batch == 2 || batch == 4, "batch must be 1, 2 or 4");
    MTL_REQUIRE(nparts >= 1 && nparts <= 64 && rows >= 1, "nparts must be in [1, 64]");
    MTL_REQUIRE(cols >= 4 && cols % (4 * nparts) == 0, "cols must be a multiple of 4 * nparts");
    const int K = cols / nparts;
    const int runs = (K / 4 + 63) / 64;
    const int plw = round_runs((runs + kWaves - 1) / kWaves);
    MTL_REQUIRE(plw * kWaves <= kMaxPL, "cols / nparts must be at most 4096");
    MTL_REQUIRE(v && W && out_parts, "null required pointer");
    MTL_REQUIRE(((uintptr_t)W % 16) == 0 && ((uintptr_t)v % 16) == 0, "W and v must be 16-byte aligned");
    GemvArgs a{v, W, nullptr, nullptr, out_parts, rows, K, nullptr, 0.f, cols, (int64_t)batch * rows};
    hipStream_t st = as_stream(stream);
    MTL_DISPATCH_B(batch, MTL_DISPATCH_RUNS(PLW, plw,
        if constexpr (PLW * kWaves <= kMaxPL) hipLaunchKernelGGL((decode_gemv_split_kernel<B, PLW>),
            dim3((unsigned)rows, (unsigned)nparts), dim3(kThreads), 0, st, a)));
    return check_launch("decode_gemv_parts");
}

extern "C" int mtl_decode_norm_gemv(const float* v, const float* norm_w, float eps, const float* W, const float* bias,
                                    float* out, int32_t batch, int32_t rows, int32_t cols, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch == 1 || batch == 2 || batch == 4, "batch must be 1, 2 or 4");
    MTL_REQUIRE(cols >= 4 && cols % 4 == 0 && cols <= 256 * kMaxPL && rows >= 1,
                "cols must be a multiple of 4 in [4, 4096]");
    MTL_REQUIRE(v && norm_w && W && out, "null required pointer");
    MTL_REQUIRE(((uintptr_t)W % 16) == 0, "W must be 16-byte aligned");
    MTL_REQUIRE(v != out, "out must not alias v");
    const size_t smem = sizeof(float) * (size_t)batch * cols;
    MTL_REQUIRE(smem <= 64 * 1024, "batch * cols too large for the decode LDS tile");
    GemvArgs a{v, W, bias, nullptr, out, rows, cols, norm_w, eps, cols, 0};
    hipStream_t st = as_stream(stream);
    const int runs = (cols / 4 + 63) / 64;
    const dim3 grid((unsigned)((rows + kWaves - 1) / kWaves));
    MTL_DISPATCH_B(batch, MTL_DISPATCH_RUNS(PL, round_runs(runs), hipLaunchKernelGGL((decode_gemv_kernel<B, PL, true>),
                                                              grid, dim3(kThreads), smem, st, a)));
    return check_launch("decode_norm_gemv");
}

extern "C" int mtl_decode_ssm(const float* xpart, int32_t nblk, const float* xc, const float* gz, const float* W_dt,
                              const float* b_dt, const float* A_log, const float* Dv, float* ssm_state, float* y,
                              int32_t batch, int32_t d_inner, int32_t d_state, int32_t dt_rank, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(batch == 1 || batch == 2 || batch == 4, "batch must be 1, 2 or 4");
    MTL_REQUIRE(d_state >= 1 && d_state <= 16, "d_state must be in [1, 16]");
    MTL_REQUIRE(d_inner >= 1 && dt_rank >= 1 && dt_rank <= 256 && nblk >= 1, "bad sizes (dt_rank <= 256)");
    MTL_REQUIRE(xpart && xc && gz && W_dt && b_dt && A_log && ssm_state && y, "null required pointer");
    const int J = dt_rank + 2 * d_state;
    const int pairs = J * batch;
    const int Q = std::max(1, std::min(kThreads / pairs, 8));
    const size_t smem = sizeof(float) * (size_t)pairs * (1 + Q);
    MTL_REQUIRE(smem <= 64 * 1024, "x_dbl too wide");
    MTL_REQUIRE((nblk + Q - 1) / Q <= kPartBatch, "too many x_proj partial blocks for this batch and width");
    SsmArgs a{xpart, nblk, xc, gz, W_dt, b_dt, A_log, Dv, ssm_state, y, d_inner, d_state, dt_rank, J};
    const dim3 grid((unsigned)((d_inner + kSsmChannels - 1) / kSsmChannels));
    hipStream_t st = as_stream(stream);
    const int rqv = round_runs((dt_rank + 15) / 16);
    MTL_DISPATCH_B(batch, MTL_DISPATCH_RUNS(RQ, rqv, hipLaunchKernelGGL((decode_ssm_kernel<B, RQ>), grid, dim3(kThreads),
                                                                  smem, st, a)));
    return check_launch("decode_ssm");
}
