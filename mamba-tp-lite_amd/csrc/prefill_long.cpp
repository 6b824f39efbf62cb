// A prompt's whole layer stack in one C call past the short-prompt limit
// (MambaLM.prefill, reference model.py:328-341 over MambaBlock.prefill
// 303-306 and MambaMixer.prefill 184-241), fp32.
//
// An eager prefill of 65 to ~1000 tokens at the mamba-130m width spends more
// time launching its ~8 ops per layer from Python than the GPU spends on
// them (130m, 256 tokens: 3.9 ms per prompt eager against 1.66 ms replayed as
// a HIP graph).  This call launches the same sequence from C++:
//   residual add + RMSNorm (mtl_add_rmsnorm; the first layer's norm alone)
//   -> in_proj GEMM (+ bias)                        xz [rows, 2D]
//   -> causal conv + SiLU over the x half, the final history
//      (mtl_causal_conv1d_fwd)                      u  [rows, D]
//   -> x_proj GEMM                                  x_dbl [rows, R + 2N]
//   -> dt_proj GEMM on x_dbl's first R columns      dt [rows, D]
//   -> the selective scan (dt bias + softplus, D skip, SiLU(z) gate fused;
//      B, C and z read in place from x_dbl and xz)  y  [rows, D]
//   -> out_proj GEMM (+ bias)                       out [rows, M]
// and after the last layer the residual add + norm_f.
//
// Up to skinny_rows token rows (and where every operand fits them) the
// projections run on the library's matrix-core skinny GEMM instead, in
// 64-row chunks (mtl_linear_skinny): in_proj with its bias; x_proj as split-K
// parts whose ordered sum also applies dt_proj (mtl_xproj_sum_dt); out_proj
// as 4 split-K parts that the residual add + norm sums (mtl_add_rmsnorm_parts)
// -- the short prompt's launches with the conv as its own kernel, because a
// conv over more than 64 rows crosses the in_proj tiles.  The parts live in
// blas_ws, which the skinny form does not otherwise use.
//
// The GEMMs are hipBLASLt matmuls, fp32 in and out, fp32 compute.  For each
// shape the heuristic's first algorithm is looked up once per device and
// kept (descriptors and algorithm), so a call costs the launches only; the
// workspace is the caller's, so the call allocates no device memory and can
// be captured into a HIP graph once each shape has been run eagerly (the
// handle and the algorithm lookups happen on first use).  A GEMM
//   Y [rows, n] (row stride ldy) = X [rows, k] (row stride ldx) . W [n, k]^T
// is the column-major product Y^T = W^T X^T: A = W as a k x n column-major
// matrix taken transposed, B = X^T as k x rows, D = Y^T as n x rows.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "common.h"

namespace {

struct GemmPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
    hipblasLtMatmulAlgo_t algo{};
};

// (device, n, rows, k, ldw, ldx, ldy, bias, workspace bytes)
using GemmKey = std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, bool, size_t>;

std::mutex g_mu;                                  // guards the handles, the plans and every call's launches
std::map<int, hipblasLtHandle_t> g_handles;
std::map<GemmKey, GemmPlan> g_plans;

#define MTL_BLAS(expr, what)                                                                            \
    do {                                                                                                \
        const hipblasStatus_t s_ = (expr);                                                              \
        if (s_ != HIPBLAS_STATUS_SUCCESS) {                                                             \
            mtl::set_error(std::string("hipBLASLt ") + (what) + " failed: status " + std::to_string((int)s_)); \
            return MTL_EHIP;                                                                            \
        }                                                                                               \
    } while (0)

int get_plan(int dev, int64_t n, int64_t rows, int64_t k, int64_t ldw, int64_t ldx, int64_t ldy, bool bias,
             size_t ws_bytes, const GemmPlan** out) {
    const GemmKey key{dev, n, rows, k, ldw, ldx, ldy, bias, ws_bytes};
    auto it = g_plans.find(key);
    if (it != g_plans.end()) {
        *out = &it->second;
        return MTL_OK;
    }
    auto h = g_handles.find(dev);
    if (h == g_handles.end()) {
        hipblasLtHandle_t handle;
        MTL_BLAS(hipblasLtCreate(&handle), "handle creation");
        h = g_handles.emplace(dev, handle).first;
    }
    GemmPlan p;
    MTL_BLAS(hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F), "matmul descriptor");
    const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
    MTL_BLAS(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)), "transA");
    MTL_BLAS(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)), "transB");
    if (bias) {
        const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
        const int32_t bt = HIP_R_32F;
        MTL_BLAS(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)),
                 "bias epilogue");
        MTL_BLAS(hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)),
                 "bias type");
    }
    MTL_BLAS(hipblasLtMatrixLayoutCreate(&p.a, HIP_R_32F, k, n, ldw), "A layout");
    MTL_BLAS(hipblasLtMatrixLayoutCreate(&p.b, HIP_R_32F, k, rows, ldx), "B layout");
    MTL_BLAS(hipblasLtMatrixLayoutCreate(&p.d, HIP_R_32F, n, rows, ldy), "D layout");
    hipblasLtMatmulPreference_t pref;
    MTL_BLAS(hipblasLtMatmulPreferenceCreate(&pref), "preference");
    const uint64_t ws = ws_bytes;
    MTL_BLAS(hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)),
             "workspace preference");
    hipblasLtMatmulHeuristicResult_t res[1];
    int found = 0;
    const hipblasStatus_t hs =
        hipblasLtMatmulAlgoGetHeuristic(h->second, p.desc, p.a, p.b, p.d, p.d, pref, 1, res, &found);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (hs != HIPBLAS_STATUS_SUCCESS || found < 1) {
        mtl::set_error("hipBLASLt has no algorithm for the GEMM " + std::to_string(n) + " x " +
                       std::to_string(rows) + " x " + std::to_string(k));
        return MTL_EHIP;
    }
    p.algo = res[0].algo;
    *out = &g_plans.emplace(key, p).first->second;
    return MTL_OK;
}

// Y [rows, n] (row stride ldy) = X [rows, k] (row stride ldx) . W [n, k]^T (row stride ldw) (+ bias [n])
int gemm(int dev, const float* W, int64_t ldw, const float* X, int64_t ldx, float* Y, int64_t ldy, const float* bias,
         int64_t n, int64_t rows, int64_t k, void* ws, size_t ws_bytes, hipStream_t st) {
    const GemmPlan* p = nullptr;
    int rc = get_plan(dev, n, rows, k, ldw, ldx, ldy, bias != nullptr, ws_bytes, &p);
    if (rc) return rc;
    if (bias)
        MTL_BLAS(hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias)),
                 "bias pointer");
    const float one = 1.f, zero = 0.f;
    MTL_BLAS(hipblasLtMatmul(g_handles[dev], p->desc, &one, W, p->a, X, p->b, &zero, Y, p->d, Y, p->d, &p->algo, ws,
                             ws_bytes, st),
             "matmul");
    return MTL_OK;
}

// the largest split of K into whole 128-column granules, at most `most` parts
int32_t split_of(int64_t K, int32_t most) {
    const int64_t g = K / 128;
    int32_t best = 1;
    for (int32_t p = 1; p <= most && p <= g; ++p)
        if (g % p == 0) best = p;
    return best;
}

// rows_per_block of mtl_linear_skinny for M rows (the Python layer's rule):
// 32-row weight tiles only at 17..32 rows of x where every CU still gets one
int32_t rows_per_block_of(int64_t M, int64_t N, int32_t ksplit) {
    return (M > 16 && M <= 32 && (N + 31) / 32 * ksplit >= 256) ? 32 : 16;
}

}  // namespace

extern "C" int mtl_prefill_long(const mtl_prefill_long_args* a, const mtl_prefill_layer* layers,
                                mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(a && layers, "null args or layers");
    const int64_t b = a->batch, l = a->seqlen, M = a->d_model, D = a->d_inner, N = a->d_state, R = a->dt_rank;
    const int64_t rows = b * l, J = R + 2 * N;
    const int32_t K = a->d_conv;
    MTL_REQUIRE(b >= 1 && l >= 1 && rows <= (int64_t(1) << 20), "batch * seqlen must be in [1, 2^20]");
    MTL_REQUIRE(b <= 65535, "batch must be <= 65535");   // the conv and scan grids' row limit
    MTL_REQUIRE(l <= 65535 * 16, "seqlen must be <= 1048560");   // the conv grid's time tiles of 16 steps
    MTL_REQUIRE(a->n_layers >= 1, "n_layers must be >= 1");
    MTL_REQUIRE(M >= 1 && M <= (int64_t(1) << 16) && D >= 1 && D <= (int64_t(1) << 16),
                "d_model and d_inner must be in [1, 65536]");
    MTL_REQUIRE(N >= 1 && N <= 32 && R >= 1 && R <= D, "d_state must be in [1, 32] and dt_rank in [1, d_inner]");
    MTL_REQUIRE(K >= 1 && K <= 8, "d_conv must be in [1, 8]");
    MTL_REQUIRE(a->h && a->xn && a->xz && a->u && a->x_dbl && a->dt && a->y && a->out && a->norm_f &&
                a->normed_out && a->blas_ws, "null workspace pointer");
    MTL_REQUIRE(a->blas_ws_bytes >= 0, "negative blas_ws_bytes");
    // every layer is checked before the first launch, so a bad layer leaves
    // nothing half written
    for (int32_t i = 0; i < a->n_layers; ++i) {
        const mtl_prefill_layer& L = layers[i];
        MTL_REQUIRE(L.norm_w && L.W_in && L.conv_w && L.W_x && L.W_dt && L.A_log && L.W_out && L.h_out &&
                    (K == 1 || L.conv_state_out), "layer " + std::to_string(i) + ": null required pointer");
        MTL_REQUIRE(K == 1 || L.conv_state_in != L.conv_state_out,
                    "layer " + std::to_string(i) + ": conv_state_out must not alias conv_state_in");
    }
    // the skinny form: sizes and alignments the skinny GEMMs and the fused
    // x_proj sum + dt_proj take, on every layer, and room for the parts
    constexpr int32_t kOutSplit = 4;
    const int32_t xs = split_of(D, 16);
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    bool skinny = a->skinny_rows > 0 && rows <= a->skinny_rows && M % 128 == 0 && D % (128 * kOutSplit) == 0 &&
                  J % 4 == 0 && R <= 160 && al16(a->xn) && al16(a->u) && al16(a->y) && al16(a->xz) &&
                  al16(a->blas_ws) && (int64_t)xs * J * rows < (int64_t(1) << 31) &&
                  (int64_t)(xs * J + kOutSplit * M) * rows * (int64_t)sizeof(float) <= a->blas_ws_bytes;
    for (int32_t i = 0; skinny && i < a->n_layers; ++i) {
        const mtl_prefill_layer& L = layers[i];
        skinny = al16(L.W_in) && al16(L.b_in) && al16(L.W_x) && al16(L.W_out) && al16(L.b_out);
    }
    float* x_parts = static_cast<float*>(a->blas_ws);                 // [xs, rows, J]
    float* y_parts = x_parts + (int64_t)xs * rows * J;                 // [4, rows, M]
    hipStream_t st = as_stream(stream);
    int dev = 0;
    if (hipStreamGetDevice(st, &dev) != hipSuccess) {
        set_error("hipStreamGetDevice failed");
        return MTL_EHIP;
    }
    std::lock_guard<std::mutex> lock(g_mu);
    void* ws = a->blas_ws;
    const size_t wsb = (size_t)a->blas_ws_bytes;
    int rc = mtl_add_rmsnorm(a->h, nullptr, nullptr, layers[0].norm_w, a->xn, rows, M, layers[0].eps, stream);
    if (rc) return rc;
    for (int32_t i = 0; i < a->n_layers; ++i) {
        const mtl_prefill_layer& L = layers[i];
        if (skinny)
            rc = mtl_linear_skinny(a->xn, M, L.W_in, L.b_in, a->xz, 2 * D, 0, rows, 2 * D, M, 1,
                                   rows_per_block_of(rows, 2 * D, 1), stream);
        else
            rc = gemm(dev, L.W_in, M, a->xn, M, a->xz, 2 * D, L.b_in, 2 * D, rows, M, ws, wsb, st);
        if (rc) return rc;
        // [b, D, l] views of the [b l, 2D] and [b l, D] buffers
        mtl_conv_params c{};
        c.x = a->xz;   c.x_sb = l * 2 * D; c.x_sd = 1; c.x_sl = 2 * D;
        c.out = a->u;  c.out_sb = l * D;   c.out_sd = 1; c.out_sl = D;
        c.w = L.conv_w; c.bias = L.conv_b;
        c.conv_state_in = K > 1 ? L.conv_state_in : nullptr;
        c.conv_state_out = K > 1 ? L.conv_state_out : nullptr;
        c.batch = b; c.seqlen = l; c.dim = D; c.width = K; c.dtype = MTL_F32; c.silu = 1;
        rc = mtl_causal_conv1d_fwd(&c, stream);
        if (rc) return rc;
        const float* x_dbl = a->x_dbl;
        if (skinny) {
            rc = mtl_linear_skinny(a->u, D, L.W_x, nullptr, x_parts, J, rows * J, rows, J, D, xs,
                                   rows_per_block_of(rows, J, xs), stream);
            if (rc) return rc;
            rc = mtl_xproj_sum_dt(x_parts, xs, rows, (int32_t)J, L.W_dt, (int32_t)R, D, xs > 1 ? a->x_dbl : nullptr,
                                  a->dt, stream);
            if (rc) return rc;
            if (xs == 1) x_dbl = x_parts;
        } else {
            rc = gemm(dev, L.W_x, D, a->u, D, a->x_dbl, J, nullptr, J, rows, D, ws, wsb, st);
            if (rc) return rc;
            rc = gemm(dev, L.W_dt, R, a->x_dbl, J, a->dt, D, nullptr, D, rows, R, ws, wsb, st);
            if (rc) return rc;
        }
        mtl_scan_params p{};
        p.u = a->u;          p.u_sb = l * D;       p.u_sd = 1; p.u_sl = D;
        p.delta = a->dt;     p.delta_sb = l * D;   p.delta_sd = 1; p.delta_sl = D;
        p.z = a->xz + D;     p.z_sb = l * 2 * D;   p.z_sd = 1; p.z_sl = 2 * D;
        p.B = x_dbl + R;     p.B_sb = l * J;       p.B_sn = 1; p.B_sl = J;
        p.C = x_dbl + R + N; p.C_sb = l * J;       p.C_sn = 1; p.C_sl = J;
        p.y = a->y;          p.y_sb = l * D;       p.y_sd = 1; p.y_sl = D;
        p.A = L.A_log; p.D = L.Dv; p.delta_bias = L.dt_bias; p.h0 = L.h0; p.h_out = L.h_out;
        p.batch = b; p.seqlen = l; p.dim = D; p.dstate = N;
        p.dtype = MTL_F32; p.delta_softplus = 1; p.a_is_log = 1; p.algo = 0;
        rc = mtl_selective_scan_fwd(&p, stream);
        if (rc) return rc;
        const bool last = i + 1 == a->n_layers;
        const float* w_next = last ? a->norm_f : layers[i + 1].norm_w;
        float* normed = last ? a->normed_out : a->xn;
        const float eps = last ? a->eps_f : layers[i + 1].eps;
        if (skinny) {
            rc = mtl_linear_skinny(a->y, D, L.W_out, L.b_out, y_parts, M, rows * M, rows, M, D, kOutSplit,
                                   rows_per_block_of(rows, M, kOutSplit), stream);
            if (rc) return rc;
            rc = mtl_add_rmsnorm_parts(a->h, y_parts, kOutSplit, a->h, w_next, normed, rows, M, eps, stream);
        } else {
            rc = gemm(dev, L.W_out, D, a->y, D, a->out, M, L.b_out, M, rows, D, ws, wsb, st);
            if (rc) return rc;
            rc = mtl_add_rmsnorm(a->h, a->out, a->h, w_next, normed, rows, M, eps, stream);
        }
        if (rc) return rc;
    }
    return MTL_OK;
}
