// Single-token selective state update and residual+RMSNorm for gfx950.
//
// mtl_selective_state_update replaces model.py:280-292 (after x_proj):
//   dt = softplus(dt_low . W_dt[d] + b_dt[d]); dA = exp(dt*A);
//   h <- h*dA + (dt*B)*x (in place, the graph-stable cache buffer, 289);
//   y = sum_n h*C + D*x; y *= silu(z).
// Sixteen lanes serve one channel: lane n owns state n and a 1/16 slice of
// the dt_proj dot product; both the dot product and y are 16-lane DPP
// butterfly sums, so a single wavefront updates four channels with no LDS
// traffic.  A workgroup serves 16 channels of up to 8 batch rows.
//
// mtl_add_rmsnorm replaces the residual add of MambaBlock (model.py:306,
// 311) fused with the following RMSNorm (model.py:130-135).

#include <type_traits>

#include "common.h"

namespace mtl {
namespace {

constexpr int kLanesPerChannel = 16;
constexpr int kStepThreads = 256;
constexpr int kChPerBlock = kStepThreads / kLanesPerChannel;

// RQ = dt_proj columns per lane (R <= 16 RQ); BB = batch rows per workgroup,
// so W_dt, A, D and the biases are read once per BB rows.  The BB rows of
// x_dbl and the block's x, z are staged in LDS by all threads; every other
// operand is loaded up front with clamped addresses.
template <typename T, int RQ, int BB>
__global__ void __launch_bounds__(kStepThreads)
ssm_step_kernel(float* __restrict__ state, const T* __restrict__ x, int64_t x_sb, const T* __restrict__ z,
                int64_t z_sb, const T* __restrict__ xdbl, int64_t xdbl_sb, const float* __restrict__ Wdt,
                const float* __restrict__ bdt, const float* __restrict__ A, const float* __restrict__ Dv,
                T* __restrict__ y, int64_t y_sb, int D, int N, int R, int batch, int a_is_log) {
    constexpr int kJMax = 16 * RQ + 2 * kLanesPerChannel;          // R + 2N <= 16 RQ + 32
    constexpr int kStage = (BB * kJMax + kStepThreads - 1) / kStepThreads;
    __shared__ float s_xd[BB * kJMax];
    __shared__ float s_x[BB][kChPerBlock], s_z[BB][kChPerBlock];
    const int tid = threadIdx.x;
    const int g = tid / kLanesPerChannel;
    const int n = tid % kLanesPerChannel;
    const int c = blockIdx.x * kChPerBlock + g;
    const int cc = min(c, D - 1), nn = min(n, N - 1);
    const int b0 = blockIdx.y * BB;
    const int J = R + 2 * N;

    float wdt[RQ];
#pragma unroll
    for (int q = 0; q < RQ; ++q) wdt[q] = Wdt[(int64_t)cc * R + min(n + 16 * q, R - 1)];
    float av = A[(int64_t)cc * N + nn];
    const float bd = bdt[cc];
    const float Dc = Dv ? Dv[cc] : 0.f;
    float hs[BB];
#pragma unroll
    for (int i = 0; i < BB; ++i) hs[i] = state[((int64_t)min(b0 + i, batch - 1) * D + cc) * N + nn];
    // staging: x_dbl rows (element e = i*J + j of the block), and x, z of the block's channels
    float st[kStage];
#pragma unroll
    for (int q = 0; q < kStage; ++q) {
        const int e = min(tid + q * kStepThreads, BB * J - 1);
        const int i = e / J, j = e - i * J;
        st[q] = Act<T>::load(xdbl + (int64_t)min(b0 + i, batch - 1) * xdbl_sb + j);
    }
    const bool xz_t = tid < BB * kChPerBlock;
    const int xi = min(tid / kChPerBlock, BB - 1), xch = tid % kChPerBlock;
    const int64_t xb = min(b0 + xi, batch - 1);
    const int xc_ = min((int)blockIdx.x * kChPerBlock + xch, D - 1);
    const float xs = Act<T>::load(x + xb * x_sb + xc_);
    const float zs = z ? Act<T>::load(z + xb * z_sb + xc_) : 0.f;
#pragma unroll
    for (int q = 0; q < kStage; ++q)
        if (tid + q * kStepThreads < BB * J) s_xd[tid + q * kStepThreads] = st[q];
    if (xz_t) {
        s_x[xi][xch] = xs;
        s_z[xi][xch] = zs;
    }
    __syncthreads();
    if (c >= D) return;  // whole 16-lane row
    if (a_is_log) av = -expf(av);

#pragma unroll
    for (int i = 0; i < BB; ++i) {
        const int64_t b = b0 + i;
        if (b >= batch) break;  // uniform over the workgroup
        const float* xd = s_xd + i * J;
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < RQ; ++q) {
            const float t = fmaf(wdt[q], xd[min(n + 16 * q, R - 1)], acc);
            acc = n + 16 * q < R ? t : acc;
        }
        acc = group_sum<kLanesPerChannel>(acc);
        const float dt = softplus_f(acc + bd);
        const float xv = s_x[i][g];
        float yv = 0.f;
        if (n < N) {
            const float dA = __builtin_amdgcn_exp2f(dt * (av * kLog2e));
            const float hv = fmaf(hs[i], dA, (dt * xd[R + n]) * xv);
            state[(b * D + c) * N + n] = hv;
            yv = hv * xd[R + N + n];
        }
        yv = group_sum<kLanesPerChannel>(yv);
        if (n == 0) {
            if (Dv) yv += xv * Dc;
            if (z) yv *= silu_f(s_z[i][g]);
            Act<T>::store(y + b * y_sb + c, yv);
        }
    }
}

// More than 32 parts: the parts are split into 4 contiguous quarters of
// ceil(P/4); wavefront q of a block sums quarter q of 64 outputs in part
// order, and the (non-empty) quarter sums are added left to right.
template <int PQ>
__global__ void __launch_bounds__(256) sum_parts4_kernel(const float* __restrict__ parts, int nparts, int64_t n,
                                                         float* __restrict__ out) {
    __shared__ float s_q[4][64];
    const int oq = threadIdx.x & 63, q = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * 64 + oq;
    const int64_t ii = min(i, n - 1);
    const int per = (nparts + 3) / 4, p0 = q * per, np = min(per, nparts - p0);
    float v[PQ];
#pragma unroll
    for (int u = 0; u < PQ; ++u) v[u] = parts[(int64_t)max(min(p0 + u, nparts - 1), 0) * n + ii];
    float acc = v[0];
#pragma unroll
    for (int u = 1; u < PQ; ++u) acc = u < np ? acc + v[u] : acc;
    s_q[q][oq] = acc;
    __syncthreads();
    if (q == 0 && i < n) {
        float r = s_q[0][oq];
#pragma unroll
        for (int k = 1; k < 4; ++k) r = k * per < nparts ? r + s_q[k][oq] : r;
        out[i] = r;
    }
}

// The same four-quarter order for any part count: each quarter's parts are
// summed by a runtime-count loop (a load round trip per part), for more than
// 512 parts.  Up to 512, sum_parts4_kernel loads a quarter in one batch: the
// 256 x_proj blocks of a mamba-1.4b-width step at up to 16 rows (16-channel
// blocks) took 16.8 us here at 8 rows.
__global__ void __launch_bounds__(256) sum_parts4_any_kernel(const float* __restrict__ parts, int nparts, int64_t n,
                                                             float* __restrict__ out) {
    __shared__ float s_q[4][64];
    const int oq = threadIdx.x & 63, q = threadIdx.x >> 6;
    const int64_t i = (int64_t)blockIdx.x * 64 + oq;
    const int64_t ii = min(i, n - 1);
    const int per = (nparts + 3) / 4, p0 = q * per, np = min(per, nparts - p0);
    float acc = 0.f;
    if (np > 0) {
        acc = parts[(int64_t)p0 * n + ii];
        for (int u = 1; u < np; ++u) acc += parts[(int64_t)(p0 + u) * n + ii];
    }
    s_q[q][oq] = acc;
    __syncthreads();
    if (q == 0 && i < n) {
        float r = s_q[0][oq];
#pragma unroll
        for (int k = 1; k < 4; ++k) r = k * per < nparts ? r + s_q[k][oq] : r;
        out[i] = r;
    }
}

// out[i] = parts[0][i] + parts[1][i] + ... in part order (split-K partials)
template <int P>
__global__ void __launch_bounds__(256) sum_parts_kernel(const float* __restrict__ parts, int nparts, int64_t n,
                                                        float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t ii = min(i, n - 1);
    float v[P];
#pragma unroll
    for (int p = 0; p < P; ++p) v[p] = parts[(int64_t)min(p, nparts - 1) * n + ii];
    float s = v[0];
#pragma unroll
    for (int p = 1; p < P; ++p) s = p < nparts ? s + v[p] : s;
    if (i < n) out[i] = s;
}

// x_proj's split-K parts of a short prefill summed, with dt_proj applied to
// the sum (model.py:214-216 without the bias, which the scan adds):
//   x_dbl[r][j] = parts[0][r][j] + parts[1][r][j] + ... (part order, as
//                 sum_parts_kernel adds them),
//   dt[r][c]    = sum_{k < R} x_dbl[r][k] W_dt[c][k]   (k in order).
// One workgroup per 64 channels x 4 rows.  It sums the dt_low columns of its
// rows into LDS (workgroups of the first channel tile sum all J columns and
// write x_dbl) and copies its 64 W_dt rows -- one contiguous block of 64 R
// floats -- into LDS transposed; then wavefront w takes row w and lane l
// channel l: a W_dt read per k that is conflict-free across the lanes and a
// broadcast read of dt_low.  The loads are issued before their first use
// (W_dt's first batch, then up to PMAX parts per element for 2 elements per
// thread), so the workgroup waits for memory once.  Two launches (the sum
// and a library GEMM of K = R) become one.
constexpr int kXdCh = 64, kXdRows = 4, kXdMaxR = 160, kXdMaxParts = 16;
template <int PMAX>
__global__ void __launch_bounds__(256) xproj_sum_dt_kernel(const float* __restrict__ parts, int nparts, int rows,
                                                           int J, int R, const float* __restrict__ Wdt, int D,
                                                           float* __restrict__ xdbl, float* __restrict__ dt) {
    __shared__ float s_lo[kXdRows][kXdMaxR + 1];
    __shared__ float s_w[kXdMaxR][kXdCh + 1];
    const int tid = threadIdx.x;
    const int c0 = blockIdx.x * kXdCh, r0 = blockIdx.y * kXdRows;
    const int64_t n = (int64_t)rows * J;
    // the rows' x_dbl columns: all J in the first channel tile, else the R of dt_low
    const int cols = (blockIdx.x == 0 && xdbl) ? J : R;
    const int ne = kXdRows * cols;
    const int nch = min(kXdCh, D - c0);
    const int nw = nch * R;
    const float* wb = Wdt + (int64_t)c0 * R;
    constexpr int QE = 2, QW = 16;
    // W_dt in batches of QW per thread (one batch covers R <= 64); the first
    // batch's loads go out ahead of the parts' loads
    float w[QW];
    auto load_w = [&](int e0) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < QW; ++q) w[q] = wb[min(e0 + tid + q * 256, nw - 1)];
    };
    auto store_w = [&](int e0) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < QW; ++q) {
            const int e = e0 + tid + q * 256;
            if (e < nw) {
                const int c = e / R, k = e - c * R;
                s_w[k][c] = w[q];
            }
        }
    };
    load_w(0);
    for (int e0 = 0; e0 < ne; e0 += QE * 256) {
        float v[QE][PMAX];
        int64_t idx[QE];
#pragma unroll
        for (int q = 0; q < QE; ++q) {
            const int e = min(e0 + tid + q * 256, ne - 1);
            const bool live = e0 + tid + q * 256 < ne;
            const int rl = e / cols, j = e - rl * cols;
            idx[q] = (int64_t)min(r0 + rl, rows - 1) * J + j;
            // lanes past the elements and parts past nparts request nothing
#pragma unroll
            for (int p = 0; p < PMAX; ++p) v[q][p] = (live && p < nparts) ? parts[p * n + idx[q]] : 0.f;
        }
#pragma unroll
        for (int q = 0; q < QE; ++q) {
            const int e = e0 + tid + q * 256;
            float acc = v[q][0];
#pragma unroll
            for (int p = 1; p < PMAX; ++p) acc = p < nparts ? acc + v[q][p] : acc;
            if (e < ne) {
                const int rl = e / cols, j = e - rl * cols;
                if (j < R) s_lo[rl][j] = acc;
                if (cols == J && r0 + rl < rows) xdbl[idx[q]] = acc;
            }
        }
    }
    store_w(0);
    for (int e0 = QW * 256; e0 < nw; e0 += QW * 256) {
        load_w(e0);
        store_w(e0);
    }
    __syncthreads();
    // dt: k in order; LDS reads 8 k at a time ahead of their fmas
    const int c = tid & (kXdCh - 1), rl = tid >> 6;
    float acc = 0.f;
    int k = 0;
    for (; k + 8 <= R; k += 8) {
        float a[8], b[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            a[u] = s_lo[rl][k + u];
            b[u] = s_w[k + u][c];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = fmaf(a[u], b[u], acc);
    }
    for (; k < R; ++k) acc = fmaf(s_lo[rl][k], s_w[k][c], acc);
    if (c < nch && r0 + rl < rows) dt[(int64_t)(r0 + rl) * D + c0 + c] = acc;
}

constexpr int kNormThreads = 256;

// One workgroup per row.  RUNS elements per thread (cols <= 256 RUNS),
// loaded up front with clamped addresses.
// y: NP parts (NP = 0: none) at stride yps, added to each other in part order
// and then to x -- the split-K partial products of the out_proj before the
// residual add
template <int RUNS, int NP>
__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ y, int64_t yps, float* x_out,
                   const float* __restrict__ w, float* __restrict__ normed, int cols, float eps) {
    __shared__ float s_part[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* xr = x + row * cols;
    float v[RUNS], wv[RUNS];
#pragma unroll
    for (int q = 0; q < RUNS; ++q) {
        const int i = min(tid + q * kNormThreads, cols - 1);
        v[q] = xr[i];
        wv[q] = w[i];
    }
    if constexpr (NP > 0) {
        float yv[NP][RUNS];
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
            for (int q = 0; q < RUNS; ++q) yv[p][q] = y[p * yps + row * cols + min(tid + q * kNormThreads, cols - 1)];
#pragma unroll
        for (int q = 0; q < RUNS; ++q) {
            float t = yv[0][q];
#pragma unroll
            for (int p = 1; p < NP; ++p) t += yv[p][q];
            v[q] += t;
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < RUNS; ++q)
        if (tid + q * kNormThreads < cols) ss = fmaf(v[q], v[q], ss);
    ss = group_sum<64>(ss);
    if ((tid & 63) == 0) s_part[tid >> 6] = ss;
    __syncthreads();
    const float tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float r = rsqrtf(tot / (float)cols + eps);
#pragma unroll
    for (int q = 0; q < RUNS; ++q) {
        const int i = tid + q * kNormThreads;
        if (i < cols) {
            if (x_out) x_out[row * cols + i] = v[q];
            normed[row * cols + i] = wv[q] * (v[q] * r);
        }
    }
}

// rows longer than 256 * kMaxRuns
__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_long_kernel(const float* __restrict__ x, const float* __restrict__ y, int np, int64_t yps, float* x_out,
                        const float* __restrict__ w, float* __restrict__ normed, int cols, float eps) {
    __shared__ float s_part[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const float* xr = x + row * cols;
    const float* yr = np > 0 ? y + row * cols : nullptr;
    auto ysum = [&](int i) {
        float t = yr[i];
        for (int p = 1; p < np; ++p) t += yr[p * yps + i];
        return t;
    };
    float ss = 0.f;
    for (int i = threadIdx.x; i < cols; i += kNormThreads) {
        float v = xr[i];
        if (yr) v += ysum(i);
        ss = fmaf(v, v, ss);
    }
    ss = group_sum<64>(ss);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = (s_part[0] + s_part[1]) + (s_part[2] + s_part[3]);
    const float r = rsqrtf(tot / (float)cols + eps);
    for (int i = threadIdx.x; i < cols; i += kNormThreads) {
        float v = xr[i];
        if (yr) v += ysum(i);
        if (x_out) x_out[row * cols + i] = v;
        normed[row * cols + i] = w[i] * (v * r);
    }
}

#define MTL_DISPATCH_BB(BBV, ...)                                  \
    switch (BBV) {                                                 \
        case 1: { constexpr int BB = 1; __VA_ARGS__; } break;      \
        case 2: { constexpr int BB = 2; __VA_ARGS__; } break;      \
        case 4: { constexpr int BB = 4; __VA_ARGS__; } break;      \
        default: { constexpr int BB = 8; __VA_ARGS__; } break;     \
    }

// Batched form for many rows (fp32, 16 states, dt_rank a multiple of 16):
// one workgroup per 16 channels x 16 MB batch rows (MB = 1; 32-row tiles
// measured the same at batch 32 and slower at 16).
//  * dt_low . W_dt for the tile on the matrix cores: A = W_dt rows (16
//    channels), B = the rows' dt_low (MB 16-row blocks), K = dt_rank in
//    16-column blocks dealt to the four wavefronts; lane r + 16 kk loads a
//    float4 of columns k + 4 kk and feeds four v_mfma_f32_16x16x4_f32, the
//    q-th taking component q on both sides.  The wavefronts' tiles are added
//    in wavefront order through LDS (deterministic).
//  * Then thread t owns the (row, channel) pairs (16 u + t / 16, t % 16),
//    u < MB, with all 16 states in registers: the state moves
//    as four float4 per pair (a row's 16 channels are 1 KB contiguous), y is
//    a sum over registers, and B, C of the row and A of the channel come from
//    LDS broadcasts -- no cross-lane reduction per row as in the 16-lanes-per-
//    channel form above, whose dt dot, state stores and y butterflies measured
//    1.6, 1.1 and 0.2 us of its 9.2 us at batch 32, d_inner 4096 (this form:
//    6.7 us; batch 16: 6.4 -> 4.3 us).
constexpr int kRowsCh = 16;
#ifndef MTL_ROWS_MIN_BATCH
#define MTL_ROWS_MIN_BATCH 16
#endif
constexpr int64_t kRowsMinBatch = MTL_ROWS_MIN_BATCH;   // the rows form from this batch on
#ifndef MTL_ROWS_TILE
#define MTL_ROWS_TILE 16
#endif
constexpr int kRowsTile = MTL_ROWS_TILE;                  // batch rows per workgroup (16 or 32)
typedef float F4s __attribute__((ext_vector_type(4)));

template <int KBW, int MB>   // KBW: 16-column blocks of dt_rank per wavefront (dt_rank <= 64 KBW); MB: 16-row blocks
__global__ void __launch_bounds__(kStepThreads)
ssm_step_rows_kernel(float* __restrict__ state, const float* __restrict__ x, int64_t x_sb,
                     const float* __restrict__ z, int64_t z_sb, const float* __restrict__ xdbl, int64_t xdbl_sb,
                     const float* __restrict__ Wdt, const float* __restrict__ bdt, const float* __restrict__ A,
                     const float* __restrict__ Dv, float* __restrict__ y, int64_t y_sb, int D, int R, int batch,
                     int a_is_log) {
    constexpr int N = 16, TR = 16 * MB;               // rows per workgroup
    __shared__ __align__(16) F4s s_dt[kStepThreads / 64][MB][64];
    __shared__ __align__(16) float s_bc[TR][2 * N];
    __shared__ __align__(16) float s_a[kRowsCh][N];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c0 = blockIdx.x * kRowsCh, b0 = blockIdx.y * TR;

    // ---- every independent load first
    const int r16 = lane & 15, kk = lane >> 4;
    const int nkb = R / 16;
    const float* wrow = Wdt + (int64_t)min(c0 + r16, D - 1) * R + 4 * kk;
    const float* xr[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) xr[mb] = xdbl + (int64_t)min(b0 + 16 * mb + r16, batch - 1) * xdbl_sb + 4 * kk;
    F4s wv[KBW], xo[KBW][MB];
#pragma unroll
    for (int j = 0; j < KBW; ++j) {
        const int kc = min(wave + 4 * j, nkb - 1) * 16;
        wv[j] = *reinterpret_cast<const F4s*>(wrow + kc);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) xo[j][mb] = *reinterpret_cast<const F4s*>(xr[mb] + kc);
    }
    // pairs (row, channel): u-th = (16 u + tid / 16, tid % 16)
    const int pc = tid & 15, pr = tid >> 4;
    const int cg = min(c0 + pc, D - 1);
    int64_t brow[MB];
    float hs[MB][N], xv[MB], zv[MB];
#pragma unroll
    for (int u = 0; u < MB; ++u) {
        brow[u] = min(b0 + pr + 16 * u, batch - 1);
        const F4s* sp = reinterpret_cast<const F4s*>(state + (brow[u] * D + cg) * N);
#pragma unroll
        for (int q = 0; q < N / 4; ++q) {
            const F4s v = sp[q];
            hs[u][4 * q] = v.x; hs[u][4 * q + 1] = v.y; hs[u][4 * q + 2] = v.z; hs[u][4 * q + 3] = v.w;
        }
        xv[u] = x[brow[u] * x_sb + cg];
        zv[u] = z ? z[brow[u] * z_sb + cg] : 0.f;
    }
    const float bd = bdt[cg];
    const float Dc = Dv ? Dv[cg] : 0.f;
    // A of (channel tid / 16, state tid % 16), in log2 units
    float av = A[(int64_t)min(c0 + (tid >> 4), D - 1) * N + (tid & 15)];
    // B | C of row tid / 8, columns 4 (tid % 8) .. + 3
    const int bcr = tid >> 3, bcj = 4 * (tid & 7);
    const F4s bc = *reinterpret_cast<const F4s*>(xdbl + (int64_t)min(b0 + min(bcr, TR - 1), batch - 1) * xdbl_sb + R +
                                                 bcj);

    // ---- dt_raw tile on the matrix cores
    F4s acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = F4s{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KBW; ++j) {
        if (wave + 4 * j < nkb) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[j][q], xo[j][mb][q], acc[mb], 0, 0, 0);
        }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) s_dt[wave][mb][lane] = acc[mb];
    if (a_is_log) av = -expf(av);
    s_a[tid >> 4][tid & 15] = av * kLog2e;
    if (bcr < TR) *reinterpret_cast<F4s*>(&s_bc[bcr][bcj]) = bc;
    __syncthreads();

    // ---- per pair: dt, the 16 state updates, y
#pragma unroll
    for (int u = 0; u < MB; ++u) {
        const int r = pr + 16 * u;
        // D[i][j] of block u sits in lane j + 16 (i / 4), register i % 4 (i = channel, j = row)
        const int dl = (r & 15) + 16 * (pc >> 2), dr = pc & 3;
        float raw = s_dt[0][u][dl][dr];
#pragma unroll
        for (int w = 1; w < kStepThreads / 64; ++w) raw += s_dt[w][u][dl][dr];
        const float dt = softplus_f(raw + bd);
        const float dtx = dt * xv[u];
        float yv = 0.f;
#pragma unroll
        for (int n = 0; n < N; ++n) {
            const float dA = __builtin_amdgcn_exp2f(dt * s_a[pc][n]);
            hs[u][n] = fmaf(hs[u][n], dA, dtx * s_bc[r][n]);
            yv = fmaf(hs[u][n], s_bc[r][N + n], yv);
        }
        if (b0 + r < batch && c0 + pc < D) {
            F4s* sp = reinterpret_cast<F4s*>(state + ((int64_t)(b0 + r) * D + c0 + pc) * N);
#pragma unroll
            for (int q = 0; q < N / 4; ++q)
                sp[q] = F4s{hs[u][4 * q], hs[u][4 * q + 1], hs[u][4 * q + 2], hs[u][4 * q + 3]};
            yv = fmaf(xv[u], Dc, yv);
            if (z) yv *= silu_f(zv[u]);
            y[(int64_t)(b0 + r) * y_sb + c0 + pc] = yv;
        }
    }
}

template <typename T>
void launch_ssm_step(float* state, const void* x, int64_t x_sb, const void* z, int64_t z_sb, const void* xdbl,
                     int64_t xdbl_sb, const float* Wdt, const float* bdt, const float* A, const float* Dv, void* y,
                     int64_t y_sb, int64_t batch, int D, int N, int R, int a_is_log, hipStream_t st) {
    if constexpr (std::is_same<T, float>::value) {
        const bool aligned = ((uintptr_t)state | (uintptr_t)xdbl | (uintptr_t)Wdt) % 16 == 0 && xdbl_sb % 4 == 0;
        if (batch >= kRowsMinBatch && N == 16 && R % 16 == 0 && R <= 256 && aligned) {
            const int tr = kRowsTile;
            dim3 grid((unsigned)((D + kRowsCh - 1) / kRowsCh), (unsigned)((batch + tr - 1) / tr));
            const int kbw = (R / 16 + 3) / 4;
#define MTL_ROWS(KB) hipLaunchKernelGGL((ssm_step_rows_kernel<KB, kRowsTile / 16>), grid, dim3(kStepThreads), 0, st, state, \
        static_cast<const float*>(x), x_sb, static_cast<const float*>(z), z_sb, static_cast<const float*>(xdbl),      \
        xdbl_sb, Wdt, bdt, A, Dv, static_cast<float*>(y), y_sb, D, R, (int)batch, a_is_log)
            if (kbw <= 1) MTL_ROWS(1);
            else if (kbw == 2) MTL_ROWS(2);
            else if (kbw == 3) MTL_ROWS(3);
            else MTL_ROWS(4);
#undef MTL_ROWS
            return;
        }
    }
    const int bb = batch >= 8 ? 8 : batch >= 4 ? 4 : batch >= 2 ? 2 : 1;
    const int rq = round_runs((R + 15) / 16);
    dim3 grid((unsigned)((D + kChPerBlock - 1) / kChPerBlock), (unsigned)((batch + bb - 1) / bb));
    MTL_DISPATCH_BB(bb, MTL_DISPATCH_RUNS(RQ, rq, hipLaunchKernelGGL((ssm_step_kernel<T, RQ, BB>), grid,
        dim3(kStepThreads), 0, st, state, static_cast<const T*>(x), x_sb, static_cast<const T*>(z), z_sb,
        static_cast<const T*>(xdbl), xdbl_sb, Wdt, bdt, A, Dv, static_cast<T*>(y), y_sb, D, N, R, (int)batch,
        a_is_log)));
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
    MTL_REQUIRE(dt_rank >= 1 && dt_rank <= 16 * kMaxRuns, "dt_rank must be in [1, 256]");
    hipStream_t st = as_stream(stream);
    if (dtype == MTL_F32)
        launch_ssm_step<float>(ssm_state, x, x_sb, z, z_sb, x_dbl, xdbl_sb, W_dt, b_dt, A, Dvec, y, y_sb, batch,
                               (int)dim, (int)dstate, (int)dt_rank, a_is_log, st);
    else
        launch_ssm_step<uint16_t>(ssm_state, x, x_sb, z, z_sb, x_dbl, xdbl_sb, W_dt, b_dt, A, Dvec, y, y_sb, batch,
                                  (int)dim, (int)dstate, (int)dt_rank, a_is_log, st);
    return check_launch("selective_state_update");
}

namespace mtl {
namespace {
int add_rmsnorm_launch(const float* x, const float* y, int32_t nparts, int64_t yps, float* x_out, const float* w,
                       float* normed, int64_t rows, int64_t cols, float eps, hipStream_t st) {
    const int runs = (int)((cols + kNormThreads - 1) / kNormThreads);
    const int np = y ? nparts : 0;
    if (runs > kMaxRuns || (np != 0 && np != 1 && np != 2 && np != 4)) {
        hipLaunchKernelGGL(add_rmsnorm_long_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, st, x, y, np, yps,
                           x_out, w, normed, (int)cols, eps);
    } else {
#define MTL_NORM_NP(NPV)                                                                                             \
    MTL_DISPATCH_RUNS(RUNS, round_runs(runs), hipLaunchKernelGGL((add_rmsnorm_kernel<RUNS, NPV>), dim3((unsigned)rows), \
                                                                 dim3(kNormThreads), 0, st, x, y, yps, x_out, w,       \
                                                                 normed, (int)cols, eps))
        if (np == 0) { MTL_NORM_NP(0); }
        else if (np == 1) { MTL_NORM_NP(1); }
        else if (np == 2) { MTL_NORM_NP(2); }
        else { MTL_NORM_NP(4); }
#undef MTL_NORM_NP
    }
    return check_launch("add_rmsnorm");
}
}  // namespace
}  // namespace mtl

extern "C" int mtl_add_rmsnorm(const float* x, const float* y, float* x_out, const float* w, float* normed,
                               int64_t rows, int64_t cols, float eps, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(rows >= 0 && cols >= 1 && cols < (int64_t(1) << 31), "size out of range");
    MTL_REQUIRE(rows < (int64_t(1) << 31), "too many rows");
    if (rows == 0) return MTL_OK;
    MTL_REQUIRE(x && w && normed, "null required pointer");
    return add_rmsnorm_launch(x, y, 1, 0, x_out, w, normed, rows, cols, eps, as_stream(stream));
}

extern "C" int mtl_add_rmsnorm_parts(const float* x, const float* y_parts, int32_t nparts, float* x_out,
                                     const float* w, float* normed, int64_t rows, int64_t cols, float eps,
                                     mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(rows >= 0 && cols >= 1 && cols < (int64_t(1) << 31), "size out of range");
    MTL_REQUIRE(rows < (int64_t(1) << 31), "too many rows");
    MTL_REQUIRE(nparts >= 1 && nparts <= 64, "nparts must be in [1, 64]");
    if (rows == 0) return MTL_OK;
    MTL_REQUIRE(x && y_parts && w && normed, "null required pointer");
    return add_rmsnorm_launch(x, y_parts, nparts, rows * cols, x_out, w, normed, rows, cols, eps, as_stream(stream));
}

extern "C" int mtl_xproj_sum_dt(const float* parts, int32_t nparts, int64_t rows, int32_t J, const float* W_dt,
                                int32_t R, int64_t D, float* x_dbl, float* dt, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(nparts >= 1 && nparts <= kXdMaxParts, "nparts must be in [1, 16]");
    MTL_REQUIRE(rows >= 0 && rows < (int64_t(1) << 24), "rows out of range");
    MTL_REQUIRE(R >= 1 && R <= kXdMaxR && J >= R, "dt_rank must be in [1, 160] and at most J");
    MTL_REQUIRE(D >= 1 && D < (int64_t(1) << 24), "d_inner out of range");
    MTL_REQUIRE((int64_t)rows * J * nparts < (int64_t(1) << 31), "parts too large");
    if (rows == 0) return MTL_OK;
    MTL_REQUIRE(parts && W_dt && dt, "null required pointer");
    MTL_REQUIRE(nparts > 1 || x_dbl == nullptr || x_dbl != parts, "x_dbl must not alias parts");
    const dim3 grid((unsigned)((D + kXdCh - 1) / kXdCh), (unsigned)((rows + kXdRows - 1) / kXdRows));
    hipStream_t st = as_stream(stream);
    if (nparts <= 4)
        hipLaunchKernelGGL((xproj_sum_dt_kernel<4>), grid, dim3(256), 0, st, parts, nparts, (int)rows, J, R, W_dt,
                           (int)D, x_dbl, dt);
    else if (nparts <= 8)
        hipLaunchKernelGGL((xproj_sum_dt_kernel<8>), grid, dim3(256), 0, st, parts, nparts, (int)rows, J, R, W_dt,
                           (int)D, x_dbl, dt);
    else if (nparts <= 12)
        hipLaunchKernelGGL((xproj_sum_dt_kernel<12>), grid, dim3(256), 0, st, parts, nparts, (int)rows, J, R, W_dt,
                           (int)D, x_dbl, dt);
    else
        hipLaunchKernelGGL((xproj_sum_dt_kernel<16>), grid, dim3(256), 0, st, parts, nparts, (int)rows, J, R, W_dt,
                           (int)D, x_dbl, dt);
    return check_launch("xproj_sum_dt");
}

extern "C" int mtl_sum_parts(const float* parts, int32_t nparts, int64_t n, float* out, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(nparts >= 1 && n >= 0, "nparts must be >= 1");
    if (n == 0) return MTL_OK;
    MTL_REQUIRE(parts && out, "null required pointer");
    MTL_REQUIRE(n < (int64_t(1) << 31), "n too large");
    const dim3 grid((unsigned)((n + 255) / 256)), grid4((unsigned)((n + 63) / 64));
    hipStream_t st = as_stream(stream);
    if (nparts <= 8) hipLaunchKernelGGL((sum_parts_kernel<8>), grid, dim3(256), 0, st, parts, nparts, n, out);
    else if (nparts <= 16) hipLaunchKernelGGL((sum_parts_kernel<16>), grid, dim3(256), 0, st, parts, nparts, n, out);
    else if (nparts <= 32) hipLaunchKernelGGL((sum_parts_kernel<32>), grid, dim3(256), 0, st, parts, nparts, n, out);
    else if (nparts <= 64) hipLaunchKernelGGL((sum_parts4_kernel<16>), grid4, dim3(256), 0, st, parts, nparts, n, out);
    else if (nparts <= 128) hipLaunchKernelGGL((sum_parts4_kernel<32>), grid4, dim3(256), 0, st, parts, nparts, n, out);
    else if (nparts <= 256) hipLaunchKernelGGL((sum_parts4_kernel<64>), grid4, dim3(256), 0, st, parts, nparts, n, out);
    else if (nparts <= 512) hipLaunchKernelGGL((sum_parts4_kernel<128>), grid4, dim3(256), 0, st, parts, nparts, n, out);
    else hipLaunchKernelGGL(sum_parts4_any_kernel, grid4, dim3(256), 0, st, parts, nparts, n, out);
    return check_launch("sum_parts");
}
