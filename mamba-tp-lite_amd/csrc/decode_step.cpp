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
