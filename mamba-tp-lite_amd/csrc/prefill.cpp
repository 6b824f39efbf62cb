// A short prompt's whole layer stack in one C call (MambaLM.prefill,
// reference model.py:328-341 over MambaBlock.prefill 303-306 and
// MambaMixer.prefill 184-241), for b l <= 64 token rows, fp32.
//
// The kernels are the ones the Python layer launches one by one for such a
// prompt, in the same order and with the same tile choices, so the results
// are the same bits; what goes away is the host time of launching about
// seven ops per layer from Python (an eager 64-token 130m prefill spent
// ~107 us of host time per layer against ~35 us of GPU time).  Per layer:
//   residual add of the previous layer's out_proj parts + RMSNorm
//   -> in_proj with the causal conv + SiLU and the final conv history
//      (mtl_in_proj_conv_prefill)
//   -> x_proj split over K (mtl_linear_skinny) -> the parts summed with
//      dt_proj applied (mtl_xproj_sum_dt)
//   -> the selective scan (dt bias + softplus, D skip, SiLU(z) gate fused)
//   -> out_proj as split-K parts (mtl_linear_skinny), added by the next
//      residual add; after the last layer that add feeds norm_f.
#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace {

// mtl_linear_skinny's tile choice in the Python layer (ops.linear_skinny):
// 32-row tiles for 17..32 rows of x when they still give every CU a
// workgroup, 16 otherwise
int skinny_rows_per_block(int64_t M, int64_t N, int32_t ksplit) {
    return (M > 16 && M <= 32 && (N + 31) / 32 * ksplit >= 256) ? 32 : 16;
}

// the largest split of K into whole 128-column granules, at most 16 parts
int32_t skinny_split(int64_t K) {
    const int64_t g = K / 128;
    int32_t best = 1;
    for (int32_t p = 1; p <= 16 && p <= g; ++p)
        if (g % p == 0) best = p;
    return best;
}

}  // namespace

extern "C" int mtl_prefill_short(const mtl_prefill_short_args* a, const mtl_prefill_layer* layers,
                                 mtl_stream_t stream) {
    using namespace mtl;
    clear_error();
    MTL_REQUIRE(a && layers, "null args or layers");
    const int64_t b = a->batch, l = a->seqlen, M = a->d_model, D = a->d_inner, N = a->d_state, R = a->dt_rank;
    const int64_t rows = b * l, J = R + 2 * N;
    MTL_REQUIRE(b >= 1 && l >= 1 && rows <= 64, "batch * seqlen must be in [1, 64]");
    MTL_REQUIRE(a->n_layers >= 1, "n_layers must be >= 1");
    MTL_REQUIRE(M >= 256 && M % 128 == 0, "d_model must be a multiple of 128, at least 256");
    MTL_REQUIRE(D >= 512 && D % 512 == 0, "d_inner must be a multiple of 512");
    MTL_REQUIRE(N >= 1 && N <= 16 && R >= 1 && R <= 160, "d_state must be in [1, 16] and dt_rank in [1, 160]");
    MTL_REQUIRE(J % 4 == 0, "dt_rank + 2 d_state must be a multiple of 4");
    MTL_REQUIRE(a->d_conv >= 2 && a->d_conv <= 4, "d_conv must be 2, 3 or 4");
    MTL_REQUIRE(a->h && a->xn && a->u && a->z && a->dt && a->y && a->x_parts && a->x_dbl && a->y_parts &&
                a->norm_f && a->normed_out, "null workspace pointer");
    // the 16-byte alignment the skinny GEMMs and the fused in_proj take of
    // their operands (mtl_linear_skinny, mtl_in_proj_conv_prefill)
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    MTL_REQUIRE(al16(a->xn) && al16(a->u) && al16(a->z) && al16(a->y) && al16(a->x_parts) && al16(a->y_parts),
                "workspace xn, u, z, y, x_parts and y_parts must be 16-byte aligned");
    // every layer is checked before the first launch, so a bad layer leaves
    // nothing half written: pointers, aliasing and alignment are the checks
    // that differ from layer to layer (the sizes are common to all layers)
    for (int32_t i = 0; i < a->n_layers; ++i) {
        const mtl_prefill_layer& L = layers[i];
        MTL_REQUIRE(L.norm_w && L.W_in && L.conv_w && L.W_x && L.W_dt && L.A_log && L.W_out && L.conv_state_out &&
                    L.h_out, "layer " + std::to_string(i) + ": null required pointer");
        // h_out may be h0 (each state is read and written by one thread); the
        // conv history is read and written in different runs
        MTL_REQUIRE(L.conv_state_in != L.conv_state_out,
                    "layer " + std::to_string(i) + ": conv_state_out must not alias conv_state_in");
        MTL_REQUIRE(al16(L.W_in) && al16(L.b_in) && al16(L.W_x) && al16(L.W_out) && al16(L.b_out),
                    "layer " + std::to_string(i) + ": W_in, b_in, W_x, W_out and b_out must be 16-byte aligned");
    }
    const int32_t xs = skinny_split(D), os = 4;
    const int rpb_x = skinny_rows_per_block(rows, J, xs), rpb_o = skinny_rows_per_block(rows, M, os);
    int rc = mtl_add_rmsnorm(a->h, nullptr, nullptr, layers[0].norm_w, a->xn, rows, M, layers[0].eps, stream);
    if (rc) return rc;
    for (int32_t i = 0; i < a->n_layers; ++i) {
        const mtl_prefill_layer& L = layers[i];
        rc = mtl_in_proj_conv_prefill(a->xn, M, L.W_in, L.b_in, L.conv_w, L.conv_b, a->d_conv, L.conv_state_in,
                                      L.conv_state_out, a->u, a->z, b, l, M, D, stream);
        if (rc) return rc;
        rc = mtl_linear_skinny(a->u, D, L.W_x, nullptr, a->x_parts, J, rows * J, rows, J, D, xs, rpb_x, stream);
        if (rc) return rc;
        float* x_dbl = xs > 1 ? a->x_dbl : a->x_parts;
        rc = mtl_xproj_sum_dt(a->x_parts, xs, rows, (int32_t)J, L.W_dt, (int32_t)R, D, xs > 1 ? a->x_dbl : nullptr,
                              a->dt, stream);
        if (rc) return rc;
        // [b, D, l] views of the [b l, D] buffers; B and C are columns of x_dbl [b l, J]
        mtl_scan_params p{};
        p.u = a->u;       p.u_sb = l * D;     p.u_sd = 1; p.u_sl = D;
        p.delta = a->dt;  p.delta_sb = l * D; p.delta_sd = 1; p.delta_sl = D;
        p.z = a->z;       p.z_sb = l * D;     p.z_sd = 1; p.z_sl = D;
        p.B = x_dbl + R;  p.B_sb = l * J;     p.B_sn = 1; p.B_sl = J;
        p.C = x_dbl + R + N; p.C_sb = l * J;  p.C_sn = 1; p.C_sl = J;
        p.y = a->y;       p.y_sb = l * D;     p.y_sd = 1; p.y_sl = D;
        p.A = L.A_log; p.D = L.Dv; p.delta_bias = L.dt_bias; p.h0 = L.h0; p.h_out = L.h_out;
        p.batch = b; p.seqlen = l; p.dim = D; p.dstate = N;
        p.dtype = MTL_F32; p.delta_softplus = 1; p.a_is_log = 1; p.algo = 0;
        rc = mtl_selective_scan_fwd(&p, stream);
        if (rc) return rc;
        rc = mtl_linear_skinny(a->y, D, L.W_out, L.b_out, a->y_parts, M, rows * M, rows, M, D, os, rpb_o, stream);
        if (rc) return rc;
        const bool last = i + 1 == a->n_layers;
        rc = mtl_add_rmsnorm_parts(a->h, a->y_parts, os, a->h, last ? a->norm_f : layers[i + 1].norm_w,
                                   last ? a->normed_out : a->xn, rows, M, last ? a->eps_f : layers[i + 1].eps,
                                   stream);
        if (rc) return rc;
    }
    return MTL_OK;
}
