// One fused decode step of the whole layer stack in one C call
// (MambaLM.step, reference model.py:343-353 over MambaBlock.step 308-311 and
// MambaMixer.step 249-294), fp32, batch 1, 2 or 4.
//
// The kernels are the fused-step ones the Python layer launches per layer, in
// the same order with the same arguments, so the logits and the updated
// caches are the same bits; what goes away is launching 3-4 ops per layer
// from Python, which bounds an eager step (130m batch 1: 744 us eager against
// 320 us replayed as a HIP graph).  Per layer:
//   mtl_decode_in: residual in (embedding gather for the first layer),
//     RMSNorm, in_proj rows, conv step + SiLU (history updated in place),
//     SiLU(z), and with W_xT the x_proj partials of each channel block
//   [mtl_decode_gemv_parts: x_proj as column parts, when there is no W_xT]
//   mtl_decode_ssm: partials summed, dt_proj + bias + softplus, the state
//     update in place, C h + D x, SiLU(z) gate
//   mtl_decode_gemv: out_proj + the residual add
// then mtl_decode_norm_gemv: norm_f and the tied lm_head.
#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

extern "C" int mtl_decode_step(const mtl_decode_step_args* a, const mtl_decode_layer* layers, mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(a && layers, "null args or layers");
    const int32_t b = a->batch, M = a->d_model, D = a->d_inner, N = a->d_state, R = a->dt_rank, K = a->d_conv;
    const int32_t J = R + 2 * N, cpb = a->channels_per_block;
    const bool split_k = a->split_k != 0;
    MTL_REQUIRE(b == 1 || b == 2 || b == 4, "batch must be 1, 2 or 4");
    MTL_REQUIRE(a->n_layers >= 1, "n_layers must be >= 1");
    MTL_REQUIRE(a->vocab >= 1, "vocab must be >= 1");
    MTL_REQUIRE(cpb == 4 || cpb == 8, "channels_per_block must be 8 or 4");
    MTL_REQUIRE(split_k || a->xproj_parts >= 1, "xproj_parts must be >= 1 without W_xT");
    // the sizes the per-layer entry points take, checked here so that a bad
    // size fails before the first layer's conv history is updated
    MTL_REQUIRE(M >= 4 && M % 4 == 0 && M <= 4096, "d_model must be a multiple of 4, at most 4096");
    MTL_REQUIRE(D >= 4 && D % 4 == 0 && D <= 4096, "d_inner must be a multiple of 4, at most 4096");
    MTL_REQUIRE(N >= 1 && N <= 16 && R >= 1 && R <= 256, "d_state must be in [1, 16] and dt_rank in [1, 256]");
    MTL_REQUIRE(K >= 2 && K <= 8, "d_conv must be in [2, 8]");
    MTL_REQUIRE(a->ids && a->emb && a->norm_f && a->logits && a->xc && a->gz && a->y && a->x0 && a->x1 &&
                a->resid && a->xpart, "null workspace pointer");
    // the LDS tiles of decode_in (b d_model), of the out_proj GEMV (b d_inner)
    // and of the norm + lm_head GEMV (b d_model)
    MTL_REQUIRE((size_t)b * M * sizeof(float) <= 60 * 1024, "batch * d_model too large for the decode LDS tile");
    MTL_REQUIRE((size_t)b * D * sizeof(float) <= 64 * 1024, "batch * d_inner too large for the decode LDS tile");
    const int32_t nblk = split_k ? (D + cpb - 1) / cpb : a->xproj_parts;
    if (!split_k) {
        // mtl_decode_gemv_parts: d_inner in xproj_parts column parts of whole
        // float4 runs, each at most 4096 columns
        MTL_REQUIRE(a->xproj_parts <= 64, "xproj_parts must be in [1, 64]");
        MTL_REQUIRE(D % (4 * a->xproj_parts) == 0, "d_inner must be a multiple of 4 * xproj_parts");
    }
    {
        // mtl_decode_ssm: Q threads per (j, batch) pair sum at most 64 partials each
        const int32_t pairs = J * b;
        const int32_t Q = std::max(1, std::min(256 / pairs, 8));
        MTL_REQUIRE((nblk + Q - 1) / Q <= 64,
                    "too many x_proj partial blocks for this batch and width (use split_k = 0)");
        MTL_REQUIRE((size_t)pairs * (1 + Q) * sizeof(float) <= 64 * 1024, "x_dbl too wide");
    }
    // the GEMVs' vector operands (xc for x_proj, y for out_proj, the
    // residual for the lm_head) and their weights are read as float4 runs
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    MTL_REQUIRE(al16(a->xc) && al16(a->y) && al16(a->emb), "xc, y and emb must be 16-byte aligned");
    // out_proj writes x0 / x1 while reading the residual in the other one
    MTL_REQUIRE(a->x0 != a->x1 && a->x0 != a->resid && a->x1 != a->resid, "x0, x1 and resid must be distinct");
    // every layer is checked before the first launch, so a bad layer leaves
    // no conv history or SSM state half stepped
    for (int32_t i = 0; i < a->n_layers; ++i) {
        const mtl_decode_layer& L = layers[i];
        const std::string at = "layer " + std::to_string(i) + ": ";
        MTL_REQUIRE(L.norm_w && L.W_in && L.conv_w && L.W_dt && L.dt_bias && L.A_log && L.W_out && L.conv_state &&
                    L.ssm_state &&
                    (split_k ? L.W_xT != nullptr : L.W_x != nullptr),
                    at + "null required pointer");
        MTL_REQUIRE(al16(L.W_in) && al16(L.W_out) && (split_k || al16(L.W_x)),
                    at + "W_in, W_out and W_x must be 16-byte aligned");
    }
    const float* x_cur = nullptr;
    int rc;
    for (int32_t i = 0; i < a->n_layers; ++i) {
        const mtl_decode_layer& L = layers[i];
        const bool first = i == 0;
        rc = mtl_decode_in(first ? nullptr : x_cur, first ? a->emb : nullptr, first ? a->ids : nullptr,
                           first ? a->vocab : 0, first ? a->resid : nullptr, L.norm_w, L.eps, L.W_in, L.b_in,
                           L.conv_state, L.conv_w, L.conv_b, split_k ? L.W_xT : nullptr, a->xc, a->gz,
                           split_k ? a->xpart : nullptr, b, M, D, K, split_k ? J : 1, cpb, stream);
        if (rc) return rc;
        if (!split_k) {
            rc = mtl_decode_gemv_parts(a->xc, L.W_x, a->xpart, b, J, D, a->xproj_parts, stream);
            if (rc) return rc;
        }
        rc = mtl_decode_ssm(a->xpart, nblk, a->xc, a->gz, L.W_dt, L.dt_bias, L.A_log, L.Dv, L.ssm_state, a->y, b, D,
                            N, R, stream);
        if (rc) return rc;
        float* x_next = (i % 2 == 0) ? a->x0 : a->x1;
        rc = mtl_decode_gemv(a->y, L.W_out, L.b_out, first ? a->resid : x_cur, x_next, b, M, D, stream);
        if (rc) return rc;
        x_cur = x_next;
    }
    return mtl_decode_norm_gemv(x_cur, a->norm_f, a->eps_f, a->emb, nullptr, a->logits, b, a->vocab, M, stream);
}

// A batched step of the whole layer stack in one C call, for the row counts
// the fused kernels above do not take (MambaLM.step at b <= 32, reference
// model.py:343-353 over MambaBlock.step 308-311 and MambaMixer.step 249-294),
// fp32.  The launches are the per-op ones the Python layer makes at these
// sizes, with the same tile choices, so the results are the same bits; what
// goes away is launching ~5 ops per layer from Python.  Per layer:
//   in_proj + conv step (history updated in place) + the x_proj partials of
//     each channel block (mtl_in_proj_conv_xproj; folded, from layer 1 on,
//     its _normed form, which applies the norm to the dot products from the
//     previous out_proj's h * w and per-tile sums of h^2)
//   -> the partials summed in block order (mtl_sum_parts)
//   -> the SSM update in place, y (mtl_selective_state_update)
//   -> out_proj as 4 split-K parts: folded and not the last layer, with the
//      residual add and the next norm's inputs (mtl_linear_skinny_residual);
//      otherwise mtl_linear_skinny, then the residual add + the next RMSNorm
//      (mtl_add_rmsnorm_parts), norm_f after the last layer.
namespace {

constexpr int32_t kStepOutSplit = 4;   // out_proj split-K parts

// the tile rules of the Python layer's wrappers (ops.in_proj_conv_xproj,
// ops.linear_skinny, ops.residual_rows_per_block)
int32_t step_channels_per_part(int32_t b, int32_t D) { return (b > 16 && D % 32 == 0 && 2 * D / 32 >= 256) ? 32 : 16; }
int32_t step_out_rows_per_block(int32_t b, int32_t M) {
    return (b > 16 && b <= 32 && (M + 31) / 32 * kStepOutSplit >= 256) ? 32 : 16;
}
int32_t step_resid_rows_per_block(int32_t b, int32_t M) {
    return (b > 16 && b <= 32 && M % 32 == 0 && M / 32 * kStepOutSplit >= 256) ? 32 : 16;
}

}  // namespace

extern "C" int mtl_decode_step_batched(const mtl_decode_step_batched_args* a, const mtl_decode_layer* layers,
                                       mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(a && layers, "null args or layers");
    const int32_t b = a->batch, M = a->d_model, D = a->d_inner, N = a->d_state, R = a->dt_rank, K = a->d_conv;
    const int32_t J = R + 2 * N, nl = a->n_layers;
    const bool fold = a->fold != 0;
    MTL_REQUIRE(b >= 1 && b <= 32, "batch must be in [1, 32]");
    MTL_REQUIRE(nl >= 1, "n_layers must be >= 1");
    MTL_REQUIRE(M >= 256 && M % 128 == 0 && M <= 65536, "d_model must be a multiple of 128 in [256, 65536]");
    MTL_REQUIRE(D >= 512 && D % 512 == 0 && D <= 65536, "d_inner must be a multiple of 512 in [512, 65536]");
    MTL_REQUIRE(N >= 1 && N <= 16 && R >= 1 && R <= 256, "d_state must be in [1, 16] and dt_rank in [1, 256]");
    MTL_REQUIRE(J <= 288, "dt_rank + 2 d_state must be at most 288");
    MTL_REQUIRE(K >= 2 && K <= 4, "d_conv must be 2, 3 or 4");
    const int32_t cpp = step_channels_per_part(b, D);
    const int32_t rpb_o = step_out_rows_per_block(b, M), rpb_r = step_resid_rows_per_block(b, M);
    const int32_t tiles = M / rpb_r;
    MTL_REQUIRE(!fold || tiles <= 128, "fold: d_model / rows_per_block must be at most 128");
    MTL_REQUIRE(a->h && a->inp && a->xc && a->z && a->y && a->xpart && a->x_dbl && a->parts && a->norm_f &&
                a->normed_out, "null workspace pointer");
    MTL_REQUIRE(!fold || (a->xn && a->sq && a->counters), "fold needs xn, sq and counters");
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    MTL_REQUIRE(al16(a->h) && al16(a->inp) && al16(a->xc) && al16(a->z) && al16(a->y) && al16(a->parts) &&
                (!fold || al16(a->xn)), "workspace h, inp, xn, xc, z, y and parts must be 16-byte aligned");
    MTL_REQUIRE(!fold || (a->xn != a->h && a->xn != a->inp), "xn must not alias h or inp");
    // h carries the residual stream through every layer and out of the call
    MTL_REQUIRE(a->inp != a->h && a->normed_out != a->h && a->normed_out != a->parts,
                "inp and normed_out must not alias h (normed_out not parts either)");
    // every layer is checked before the first launch, so a bad layer leaves
    // no conv history or SSM state half stepped
    for (int32_t i = 0; i < nl; ++i) {
        const mtl_decode_layer& L = layers[i];
        const std::string at = "layer " + std::to_string(i) + ": ";
        MTL_REQUIRE(L.norm_w && L.W_in && L.conv_w && L.W_xT && L.W_dt && L.dt_bias && L.A_log && L.W_out &&
                    L.conv_state && L.ssm_state, at + "null required pointer (W_xT included)");
        MTL_REQUIRE(al16(L.W_in) && al16(L.b_in) && al16(L.conv_state) && al16(L.conv_w) && al16(L.conv_b) &&
                    al16(L.W_xT) && al16(L.W_out) && al16(L.b_out) && (!fold || al16(L.norm_w)),
                    at + "W_in, b_in, conv_state, conv_w, conv_b, W_xT, W_out, b_out and (folded) norm_w must be "
                         "16-byte aligned");
        MTL_REQUIRE(L.eps >= 0.f, at + "eps must be >= 0 (not NaN)");
    }
    const int64_t bJ = (int64_t)b * J, bM = (int64_t)b * M;
    int rc = mtl_add_rmsnorm(a->h, nullptr, nullptr, layers[0].norm_w, a->inp, b, M, layers[0].eps, stream);
    if (rc) return rc;
    for (int32_t i = 0; i < nl; ++i) {
        const mtl_decode_layer& L = layers[i];
        const bool last = i + 1 == nl;
        if (fold && i > 0)
            rc = mtl_in_proj_conv_xproj_normed(a->xn, M, L.W_in, L.b_in, L.conv_state, L.conv_w, L.conv_b, K, L.W_xT,
                                               J, a->xc, a->z, D, a->xpart, b, M, D, cpp, a->sq, tiles, L.eps, stream);
        else
            rc = mtl_in_proj_conv_xproj(a->inp, M, L.W_in, L.b_in, L.conv_state, L.conv_w, L.conv_b, K, L.W_xT, J,
                                        a->xc, a->z, D, a->xpart, b, M, D, cpp, stream);
        if (rc) return rc;
        rc = mtl_sum_parts(a->xpart, D / cpp, bJ, a->x_dbl, stream);
        if (rc) return rc;
        rc = mtl_selective_state_update(L.ssm_state, a->xc, D, a->z, D, a->x_dbl, J, L.W_dt, L.dt_bias, L.A_log, L.Dv,
                                        a->y, D, b, D, N, R, MTL_F32, 1, stream);
        if (rc) return rc;
        if (fold && !last) {
            rc = mtl_linear_skinny_residual(a->y, D, L.W_out, L.b_out, a->parts, b, M, D, kStepOutSplit, rpb_r, a->h,
                                            layers[i + 1].norm_w, a->xn, a->sq,
                                            a->counters + (int64_t)i * tiles, stream);
            if (rc) return rc;
            continue;
        }
        rc = mtl_linear_skinny(a->y, D, L.W_out, L.b_out, a->parts, M, bM, b, M, D, kStepOutSplit, rpb_o, stream);
        if (rc) return rc;
        rc = mtl_add_rmsnorm_parts(a->h, a->parts, kStepOutSplit, a->h, last ? a->norm_f : layers[i + 1].norm_w,
                                   last ? a->normed_out : a->inp, b, M, last ? a->eps_f : layers[i + 1].eps, stream);
        if (rc) return rc;
    }
    return MTL_OK;
}
