/*
 * mtl.h -- C ABI of the MI355X (gfx950) Mamba mixer hot-path library
 * (libmtl.so, built from mamba-tp-lite_amd/csrc).
 *
 * The reference (mamba-tp-lite) has no FFI: its operator surface is the
 * Python method set of mamba_lite/model.py and mamba_lite/tp_utils.py.  Each
 * entry point below replaces the named span of that Python code; the Python
 * package mamba_lite (mamba-tp-lite_amd/mamba_lite) binds them with ctypes.
 *
 * Conventions
 *   - Every buffer is device memory owned by the caller.  No entry point
 *     allocates, frees, synchronizes or reads host memory behind a device
 *     pointer, so every call can be captured into a hipGraph.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = legacy default).
 *   - Return 0 on success, a nonzero MTL_E* code otherwise; the message is in
 *     mtl_last_error() (thread-local).  No C++ exception crosses the ABI.
 *   - Strides are in ELEMENTS of the tensor they describe.
 *   - Activations are fp32 or bf16 (`dtype`); weights, A, D, biases and the
 *     SSM state are always fp32.
 *   - Calls are re-entrant; calls on one stream are ordered.  Two keep device
 *     state between calls: mtl_decode_step_persist in the caller's workspace
 *     and mtl_conv_step_xproj_noalloc in a per-GPU array of the library.
 */
#ifndef MTL_H
#define MTL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum mtl_status { MTL_OK = 0, MTL_EINVAL = 1, MTL_EHIP = 2, MTL_EUNSUPPORTED = 3 };
enum mtl_dtype { MTL_F32 = 0, MTL_BF16 = 1 };

typedef void* mtl_stream_t; /* hipStream_t */

/* Thread-local text of the last failure ("" if none). */
const char* mtl_last_error(void);
/* ABI version, bumped on any signature change or new entry point the Python layer binds. */
int mtl_abi_version(void);

/* ------------------------------------------------------------------------
 * Selective scan, prefill.
 * Replaces model.py:216-238 (dt bias + softplus, dA = exp(dt*A),
 * dBx = dt*B*x, the per-token recurrence loop 231-236, y = C.h, the D skip
 * 237 and the silu(z) gate 238) and returns the final state (model.py:241).
 * Also the same span of the TP shard, tp_model.py:110-129.
 *
 *   dt[b,d,t] = delta[b,d,t] + delta_bias[d]     (delta_bias may be NULL)
 *   dt        = softplus(dt)                      (if delta_softplus)
 *   h[b,d,:]  = h0[b,d,:] or 0
 *   for t:  h[n] = exp(dt*A[d,n]) * h[n] + dt * B[b,n,t] * u[b,d,t]
 *           y[b,d,t] = sum_n C[b,n,t] h[n]  (+ D[d]*u)  (* silu(z))
 *   h_out[b,d,:] = h                               (fp32, contiguous [b,D,N])
 *
 * A is the negated continuous-time matrix [D,N] (A = -exp(A_log)); with
 * a_is_log != 0 the pointer holds A_log and the kernel forms -exp(A_log).
 * u, delta, z, y: 3-D [b, D, l] with strides (sb, sd, sl) -- either
 * channel-major (sl == 1) or token-major (sd == 1) is fast, any other
 * stride pattern is rejected.  B, C: [b, N, l] with strides (sb, sn, sl).
 * h0 (nullable) and h_out (nullable): contiguous fp32 [b, D, N]; h_out may
 * be h0 (a state is read before it is overwritten, by the same thread).
 * Two kernels compute this.  The tiled one (algo 1) walks the steps of a
 * sequence in turn with the state in registers: its time is the sequence
 * length times one step's latency, which is the right trade when the grid
 * (batch * ceil(D / 64) workgroups) fills the GPU.  The chunked one (algo 2)
 * gives each (batch row, channel) a wavefront whose 64 lanes hold 64 steps
 * and scans them in parallel, carrying (prod dA, h) from chunk to chunk:
 * more arithmetic per step, but a latency of l / 64 chunks.  algo 0 takes
 * the chunked kernel when batch * ceil(D / 64) < 160 and l > 32.  Both are
 * deterministic and agree within fp32 rounding.
 * Limits: 1 <= N <= 32, l >= 0; B/C strides non-negative with
 * ((N-1)*sn + 31*sl + 1) elements under 4 GiB; token-major step strides
 * non-negative with (7*sl + D) elements under 2 GiB (the kernel addresses
 * these spans with 32-bit offsets from a uniform base).
 * ---------------------------------------------------------------------- */
typedef struct {
    const void* u;     int64_t u_sb, u_sd, u_sl;
    const void* delta; int64_t delta_sb, delta_sd, delta_sl;
    const void* z;     int64_t z_sb, z_sd, z_sl;        /* nullable */
    const void* B;     int64_t B_sb, B_sn, B_sl;
    const void* C;     int64_t C_sb, C_sn, C_sl;
    void* y;           int64_t y_sb, y_sd, y_sl;
    const float* A;            /* [D, N] contiguous */
    const float* D;            /* [D] nullable */
    const float* delta_bias;   /* [D] nullable */
    const float* h0;           /* [b, D, N] nullable */
    float* h_out;              /* [b, D, N] nullable */
    int64_t batch, seqlen, dim, dstate;
    int32_t dtype;             /* mtl_dtype of u, delta, z, B, C, y */
    int32_t delta_softplus;
    int32_t a_is_log;
    int32_t algo;              /* 0: choose by grid size; 1: tiled (steps in turn); 2: chunked over lanes */
} mtl_scan_params;

int mtl_selective_scan_fwd(const mtl_scan_params* p, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Causal depthwise conv1d (+ optional SiLU), prefill.
 * Replaces model.py:201-212 (left-pad with cache.conv_state or zeros,
 * F.conv1d(groups=D) + bias, [..., :l], F.silu, final_conv_state =
 * x_padded[..., -(K-1):]); tp_model.py:95-103 on a channel shard.
 *
 *   xp = concat(conv_state_in or 0 [b,D,K-1], x [b,D,l]) along l
 *   out[b,d,t] = act( sum_k w[d,k] * xp[b,d,t+k] + bias[d] )
 *   conv_state_out[b,d,:] = xp[b,d, l : l+K-1]       (pre-activation inputs)
 *
 * x, out: [b, D, l] strided (sb, sd, sl); w: [D, K] fp32 contiguous;
 * bias: [D] fp32 nullable; conv_state_in/out: contiguous [b, D, K-1] in the
 * activation dtype, nullable, must not alias each other.  1 <= K <= 8
 * (K = 1 carries no history: the states are empty and may be NULL).
 * ---------------------------------------------------------------------- */
typedef struct {
    const void* x;   int64_t x_sb, x_sd, x_sl;
    void* out;       int64_t out_sb, out_sd, out_sl;
    const float* w;
    const float* bias;
    const void* conv_state_in;
    void* conv_state_out;
    int64_t batch, seqlen, dim;
    int32_t width;    /* K = d_conv */
    int32_t dtype;    /* mtl_dtype of x, out, conv states */
    int32_t silu;
    int32_t reserved;
} mtl_conv_params;

int mtl_causal_conv1d_fwd(const mtl_conv_params* p, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Single-token conv step, in place.
 * Replaces model.py:264-277 (conv_in = cat(conv_state, x), sum(conv_in*w)
 * + bias, conv_state.copy_(conv_in[..., 1:]), F.silu); tp_model.py:145-157.
 *
 * conv_state: [b, D, K-1] contiguous (activation dtype), updated in place.
 * x: [b, D] with batch stride x_sb (channel stride 1); out: [b, D] with
 * batch stride out_sb.  w: [D, K] fp32; bias: [D] fp32 nullable.
 * 1 <= K <= 8; with K = 1 conv_state is empty and may be NULL.  (The
 * reference's step takes x unchanged when d_conv == 1, model.py:275-276:
 * its caller passes a unit weight and no bias for that.)
 * ---------------------------------------------------------------------- */
int mtl_conv_step(void* conv_state, const void* x, int64_t x_sb, const float* w, const float* bias,
                  void* out, int64_t out_sb, int64_t batch, int64_t dim, int32_t width,
                  int32_t dtype, int32_t silu, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Batched single-token conv step fused with the x_proj split-K partials,
 * fp32, 1 <= batch <= 32.  Replaces model.py:264-279 for the batch at once:
 * the conv step of mtl_conv_step (history shifted in place, SiLU) into out
 * [b, D] (batch stride out_sb), and
 *   xpart[k, b, j] = sum_{c in block k} out[b, c] * W_xT[c, j]
 * for blocks of 32 channels (nblk = ceil(D / 32)); mtl_sum_parts over the
 * nblk blocks gives x_dbl [b, J] (J = xdbl_cols = R + 2N <= 288).
 * x: [b, D] (batch stride x_sb, channel stride 1); W_xT: x_proj weight
 * transposed, contiguous [D, J]; xpart: contiguous [nblk, b, J].
 * ---------------------------------------------------------------------- */
int mtl_conv_step_xproj(float* conv_state, const float* x, int64_t x_sb, const float* w, const float* bias,
                        float* out, int64_t out_sb, const float* W_xT, float* xpart, int64_t batch, int64_t dim,
                        int32_t width, int32_t xdbl_cols, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Allocation-free form of mtl_conv_step_xproj + mtl_sum_parts.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same conv step into out [b, D] and
 * conv_state as mtl_conv_step_xproj, and x_dbl [b, J] (contiguous) =
 * the ordered sum of the block partials, exactly as mtl_sum_parts gives
 * it -- but the partials live in a fixed device array inside the library
 * (2^20 floats = 4 MiB per GPU, held until the process ends) instead of a
 * caller buffer.  Rejects ceil(D / 32) * b * J > 2^20 with MTL_EINVAL.
 * The array used is the one of the device `stream` belongs to (the current
 * device for the null stream), whichever device the calling thread has
 * current.  Allocates and frees nothing.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (different streams, threads or
 * processes sharing a context) race and must be serialized by the caller.
 * ---------------------------------------------------------------------- */
int mtl_conv_step_xproj_noalloc(float* conv_state, const float* x, int64_t x_sb, const float* w, const float* bias,
                                float* out, int64_t out_sb, const float* W_xT, float* x_dbl, int64_t batch,
                                int64_t dim, int32_t width, int32_t xdbl_cols, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Single-token selective state update, in place.
 * Replaces model.py:280-292 after x_proj (dt = softplus(F.linear(dt_low,
 * W_dt, b_dt)), dA = exp(dt*A), dBx = dt*B*x, ssm_state.copy_(h*dA + dBx),
 * y = einsum(h_new, C) + x*D, y *= silu(z)); tp_model.py:161-173.
 *
 * ssm_state: fp32 [b, D, N] contiguous, updated in place.
 * x, z, y: [b, D] with batch strides (channel stride 1).  x_dbl: [b, R+2N]
 * with batch stride xdbl_sb holding [dt_low | B | C] (model.py:280).
 * W_dt: [D, R] fp32; b_dt: [D] fp32; A: [D, N] (a_is_log as in the scan);
 * Dvec: [D] nullable.  1 <= N <= 16.
 * ---------------------------------------------------------------------- */
int mtl_selective_state_update(float* ssm_state, const void* x, int64_t x_sb, const void* z, int64_t z_sb,
                               const void* x_dbl, int64_t xdbl_sb, const float* W_dt, const float* b_dt,
                               const float* A, const float* Dvec, void* y, int64_t y_sb,
                               int64_t batch, int64_t dim, int64_t dstate, int64_t dt_rank,
                               int32_t dtype, int32_t a_is_log, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Residual add + RMSNorm (fp32).
 * Replaces MambaBlock's residual (model.py:306, 311) fused with the next
 * RMSNorm (model.py:130-135): x_out = x + y (if y != NULL), then
 * normed = w * (x_out * rsqrt(mean(x_out^2) + eps)).  x_out may alias x.
 * All [rows, cols] contiguous fp32.
 * ---------------------------------------------------------------------- */
int mtl_add_rmsnorm(const float* x, const float* y, float* x_out, const float* w, float* normed,
                    int64_t rows, int64_t cols, float eps, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * mtl_add_rmsnorm with y given as nparts split-K partial products
 * y_parts [nparts, rows, cols] (contiguous): y = ((p0 + p1) + ...) in part
 * order, then x_out = x + y and normed as above -- the residual add of
 * model.py:311 after an out_proj computed by mtl_linear_skinny with
 * ksplit = nparts, without a separate reduction launch.  1 <= nparts <= 64.
 * ---------------------------------------------------------------------- */
int mtl_add_rmsnorm_parts(const float* x, const float* y_parts, int32_t nparts, float* x_out, const float* w,
                          float* normed, int64_t rows, int64_t cols, float eps, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Sum of split-K partial products in a fixed order: for nparts <= 32
 *   out[i] = ((parts[0*n + i] + parts[1*n + i]) + ...) + parts[(nparts-1)*n + i];
 * above 32 the parts form 4 contiguous quarters of ceil(nparts/4), each
 * summed in that order, and the non-empty quarter sums are added left to
 * right.
 * The x_proj of the batched step (model.py:279, x_dbl = x_proj(x)) runs as
 * nparts GEMMs over channel chunks on hipBLASLt; this adds their outputs.
 * parts: contiguous fp32 [nparts, n]; out: fp32 [n].  nparts >= 1 (with
 * nparts * n elements addressable by int64).
 * ---------------------------------------------------------------------- */
int mtl_sum_parts(const float* parts, int32_t nparts, int64_t n, float* out, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * x_proj's split-K parts summed, and dt_proj on the sum, in one launch
 * (model.py:214-216 of MambaMixer.prefill, dt_proj without its bias, which
 * the scan adds):
 *   x_dbl[r][j] = ((parts[0][r][j] + parts[1][r][j]) + ...)   (part order,
 *                 as mtl_sum_parts for nparts <= 32),
 *   dt[r][c]    = sum over k < R, in order, of x_dbl[r][k] W_dt[c][k].
 * parts: contiguous [nparts, rows, J] (x_proj of rows tokens by
 * mtl_linear_skinny with ksplit = nparts); W_dt: contiguous [D, R], R <=
 * min(J, 160); x_dbl: [rows, J] contiguous, or NULL to skip writing it
 * (with nparts = 1 the caller reads parts itself); dt: [rows, D]
 * contiguous.  1 <= nparts <= 16.  Deterministic.
 * ---------------------------------------------------------------------- */
int mtl_xproj_sum_dt(const float* parts, int32_t nparts, int64_t rows, int32_t J, const float* W_dt, int32_t R,
                     int64_t D, float* x_dbl, float* dt, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Per-token int8 quantize -> dequantize-sum of an AllReduce payload,
 * local (the collective replaced by nparts partials resident on one GPU).
 * Replaces tp_utils.py:103-131 (_int8_gather, per_token=True, reached via
 * all_reduce_sum_int8_gather_tok 145-149).  For each part r (rank order):
 *   s_r[i] = max(max_j |part_r[i,j]|, 1e-8f) / 127.0f        (IEEE fp32 div)
 *   q_r[i,j] = clamp(rint(part_r[i,j] / s_r[i]), -127, 127)  (half-even)
 *   payload_r = [s_r as 4*rows LE bytes || q_r row-major int8]  (nullable)
 *   out = ((0 + q_0*s_0) + q_1*s_1) + ...  (fp32, no FMA contraction)
 * parts: host array of nparts device pointers to contiguous fp32
 * [rows, cols]; payloads: host array of nparts device pointers (each
 * rows*(cols+4) bytes) or NULL.  1 <= nparts <= 8.  Codes and scales are
 * bit-identical to the reference's torch CPU arithmetic.
 * ---------------------------------------------------------------------- */
int mtl_quant_dequant_sum_int8_tok(const float* const* parts, int32_t nparts, int64_t rows, int64_t cols,
                                   uint8_t* const* payloads, float* out, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * fp16 cast -> sum -> cast back, local.  Replaces tp_utils.py:31-42
 * (all_reduce_sum_fp16): low_r = fp16_rne(part_r); acc = low_0;
 * acc = fp16_rne(acc + low_r) for r = 1.. (rank order); out = fp32(acc).
 * payloads: host array of nparts device pointers to n fp16 values each
 * (the materialized wire payload) or NULL.  1 <= nparts <= 8.
 * ---------------------------------------------------------------------- */
int mtl_quant_dequant_sum_fp16(const float* const* parts, int32_t nparts, int64_t n,
                               uint16_t* const* payloads, float* out, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Skinny fp32 GEMM on the matrix cores for the projections of a batched
 * decode step: y = x W^T (+ bias), nn.Linear on [b, K] with b <= 32 tokens --
 * in_proj (model.py:261), out_proj (model.py:293) and the tied lm_head
 * (model.py:326, 353) in MambaMixer.step / MambaLM.step -- and of a prefill
 * of at most 64 tokens (model.py:197, 214, 240, 339).
 *   x: [M, K], row stride x_rs (>= K, multiple of 4), M >= 1: up to 64 rows
 *      per launch chunk (a prefill's longer row counts run as 64-row chunks);
 *   W: [N, K] contiguous, N a multiple of 4; bias: [N] or NULL;
 *   y: [M, N] with row stride y_rs (>= N, multiple of 4).
 * K must be a multiple of 128 * ksplit.  With ksplit > 1 the K range is cut
 * into ksplit equal parts and part s writes its partial product to
 * y + s * y_ks (bias in part 0 only); the caller adds the parts in order
 * (mtl_sum_parts, or mtl_add_rmsnorm_parts for out_proj).  rows_per_block
 * (16 or 32) is the weight rows per workgroup.  Every pointer 16-byte
 * aligned.  Deterministic (fixed summation order).
 * ---------------------------------------------------------------------- */
int mtl_linear_skinny(const float* x, int64_t x_rs, const float* W, const float* bias, float* y, int64_t y_rs,
                      int64_t y_ks, int64_t M, int64_t N, int64_t K, int32_t ksplit, int32_t rows_per_block,
                      mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * A short prefill's in_proj with the causal conv + SiLU in one launch
 * (MambaMixer.prefill, model.py:197-212), fp32, batch * seqlen <= 64 token
 * rows.  x: [batch * seqlen, d_model] (row m = token m % seqlen of batch row
 * m / seqlen; row stride x_rs); W_in: [2 d_inner, d_model] contiguous; b_in:
 * [2 d_inner] or NULL; conv_w: [d_inner, d_conv]; conv_b: [d_inner] or NULL;
 * conv_state_in: [batch, d_inner, d_conv - 1] incoming history, or NULL for
 * zeros.  Writes u [batch * seqlen, d_inner] = SiLU(causal depthwise conv of
 * the x half + conv_b), z [batch * seqlen, d_inner] = the z half, and
 * conv_state_out [batch, d_inner, d_conv - 1] = the last d_conv - 1 conv
 * inputs (model.py:212), which must not alias conv_state_in.  The conv sums
 * its taps in order and adds the bias last, as mtl_causal_conv1d_fwd does,
 * and the in_proj product is mtl_linear_skinny's, so u, z and the state
 * equal those two launches' bit for bit.  d_model a multiple of 128;
 * d_inner a multiple of 16; d_conv 2, 3 or 4; x, W_in, b_in, z 16-byte
 * aligned.  Deterministic.
 * ---------------------------------------------------------------------- */
/* ------------------------------------------------------------------------
 * A batched step's in_proj, conv step and x_proj partials in one launch:
 * model.py:261 (xz = in_proj(x)), 264-277 (conv step + SiLU of the x half,
 * the history shifted in place) and 279 (x_dbl = x_proj(xc)) for b <= 32
 * tokens, fp32.  The in_proj product runs on the matrix cores like
 * mtl_linear_skinny (same operand rules, K = d_model); a workgroup that owns
 * channels [c0, c0 + channels_per_part) of the x half then does their conv
 * step and writes
 *   xpart[c0 / channels_per_part][m][j] = sum over its channels c, in order,
 *                                          of xc[m][c] W_xT[c][j],
 * which the caller adds in block order (mtl_sum_parts) to get x_dbl.
 *   x: [b, d_model] (row stride x_rs); W_in: [2 d_inner, d_model]
 *   contiguous; b_in: [2 d_inner] or NULL; conv_state: [b, d_inner,
 *   d_conv - 1] contiguous, in place; conv_w: [d_inner, d_conv]; conv_b:
 *   [d_inner] or NULL; W_xT: [d_inner, J] (x_proj weight transposed);
 *   xc: [b, d_inner] contiguous; z: [b, d_inner], row stride z_rs; xpart:
 *   [d_inner / channels_per_part, b, J].
 * 1 <= b <= 32; d_model a multiple of 128, at least 256; channels_per_part
 * 16 or 32, dividing d_inner; d_conv 2, 3 or 4; J <= 288.  x, W_in, b_in,
 * conv_state, conv_w, conv_b, xc and z 16-byte aligned.  Deterministic.
 * Replaces mtl_linear_skinny (in_proj) + mtl_conv_step_xproj in the step.
 * ---------------------------------------------------------------------- */
int mtl_in_proj_conv_prefill(const float* x, int64_t x_rs, const float* W_in, const float* b_in, const float* conv_w,
                             const float* conv_b, int32_t d_conv, const float* conv_state_in, float* conv_state_out,
                             float* u, float* z, int64_t batch, int64_t seqlen, int64_t d_model, int64_t d_inner,
                             mtl_stream_t stream);
/* ------------------------------------------------------------------------
 * A short prompt's whole layer stack in one call: MambaLM.prefill
 * (model.py:328-341) over MambaBlock.prefill (303-306) and
 * MambaMixer.prefill (184-241), fp32, batch * seqlen <= 64 token rows, with
 * the kernels the per-op entry points above launch, in the same order:
 *   xn = RMSNorm_0(h);  per layer i:
 *     mtl_in_proj_conv_prefill(xn) -> u, z, conv_state_out
 *     mtl_linear_skinny(u, W_x, ksplit = the largest split of d_inner / 128
 *       into at most 16 parts) -> x_parts
 *     mtl_xproj_sum_dt(x_parts, W_dt) -> x_dbl, dt
 *     mtl_selective_scan_fwd(u, dt + dt_bias (softplus), A = -exp(A_log),
 *       B, C = columns of x_dbl, D, z, h0) -> y, h_out
 *     mtl_linear_skinny(y, W_out, b_out, ksplit = 4) -> y_parts
 *     h += the y_parts in order, xn = RMSNorm_{i+1}(h) (norm_f after the
 *       last layer, into normed_out)    (mtl_add_rmsnorm_parts)
 * h: [b seqlen, d_model], the embedded tokens in, the final residual out.
 * Workspace (all contiguous fp32): xn [rows, d_model]; u, z, dt, y [rows,
 * d_inner]; x_parts [16, rows, J]; x_dbl [rows, J] (J = dt_rank +
 * 2 d_state); y_parts [4, rows, d_model]; normed_out [rows, d_model].
 * layers[i]: the layer's weights (as the per-op entry points take them) and
 * its cache: conv_state_in / h0 (NULL: zeros) and conv_state_out / h_out
 * ([b, d_inner, d_conv - 1] and [b, d_inner, d_state]; conv_state_out must
 * not alias conv_state_in, h_out may alias h0).  d_model a multiple of 128
 * (at least 256), d_inner a multiple of 512, d_state <= 16, dt_rank <= 160,
 * dt_rank + 2 d_state a multiple of 4, d_conv 2..4.  Every layer is checked
 * before the first launch.  The bits equal those of the per-op launches.
 * ---------------------------------------------------------------------- */
typedef struct {
    const float* norm_w;       /* [d_model] the block's RMSNorm */
    float eps;
    int32_t reserved;
    const float* W_in;         /* [2 d_inner, d_model] */
    const float* b_in;         /* [2 d_inner] or NULL */
    const float* conv_w;       /* [d_inner, d_conv] */
    const float* conv_b;       /* [d_inner] or NULL */
    const float* W_x;          /* [J, d_inner] */
    const float* W_dt;         /* [d_inner, dt_rank] */
    const float* dt_bias;      /* [d_inner] */
    const float* A_log;        /* [d_inner, d_state] */
    const float* Dv;           /* [d_inner] or NULL */
    const float* W_out;        /* [d_model, d_inner] */
    const float* b_out;        /* [d_model] or NULL */
    const float* conv_state_in;
    float* conv_state_out;
    const float* h0;
    float* h_out;
} mtl_prefill_layer;

typedef struct {
    float* h;
    float* xn;
    float* u;
    float* z;
    float* dt;
    float* y;
    float* x_parts;
    float* x_dbl;
    float* y_parts;
    const float* norm_f;
    float* normed_out;
    float eps_f;
    int32_t d_conv;
    int32_t n_layers;
    int32_t reserved;
    int64_t batch, seqlen, d_model, d_inner, d_state, dt_rank;
} mtl_prefill_short_args;

int mtl_prefill_short(const mtl_prefill_short_args* args, const mtl_prefill_layer* layers, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * A prompt's whole layer stack in one call past the short-prompt limit:
 * MambaLM.prefill (model.py:328-341) over MambaBlock.prefill (303-306) and
 * MambaMixer.prefill (184-241), fp32, any number of token rows, with the
 * per-op path's kernels launched from C++ (the projections as hipBLASLt
 * GEMMs):
 *   xn = RMSNorm_0(h);  per layer i:
 *     xz = xn W_in^T + b_in;  u = SiLU(causal conv of xz's x half), the final
 *     history into conv_state_out (mtl_causal_conv1d_fwd);
 *     x_dbl = u W_x^T;  dt = x_dbl[:, :R] W_dt^T;
 *     y = selective scan (dt_bias + softplus, D skip, gate SiLU(xz's z half);
 *         h0 -> h_out, which may alias) (mtl_selective_scan_fwd);
 *     h += y W_out^T + b_out;  xn = RMSNorm_{i+1}(h)  (norm_f into normed_out
 *     after the last layer) (mtl_add_rmsnorm).
 * h: [b l, d_model] (row m = token m % seqlen of batch row m / seqlen), the
 * embedded tokens in, the final residual stream out.  The layers are
 * mtl_prefill_layer entries as mtl_prefill_short takes them (conv_w [D, K],
 * W_in [2D, M], W_x [R + 2N, D], W_dt [D, R], W_out [M, D], all contiguous;
 * conv_state_in may be NULL for zeros; with d_conv 1 the conv states are not
 * used).  Workspace (contiguous fp32): xn, out [b l, M]; xz [b l, 2D]; u, dt,
 * y [b l, D]; x_dbl [b l, R + 2N]; blas_ws: blas_ws_bytes of GEMM workspace.
 * The GEMM algorithm of each shape is hipBLASLt's first heuristic pick,
 * looked up on the shape's first call on a device and kept; the handle is
 * created on the first call on a device.  After that a call allocates no
 * device memory and may be captured into a HIP graph.  Calls on one process
 * are serialized inside the library.  b l <= 2^20 with b <= 65535 and
 * l <= 1048560, d_state <= 32, 1 <= d_conv <= 8.
 * With b l <= skinny_rows (0: never) the projections run on mtl_linear_skinny
 * instead (in 64-row chunks; x_proj as split-K parts summed by
 * mtl_xproj_sum_dt, which also applies dt_proj; out_proj as 4 parts summed by
 * mtl_add_rmsnorm_parts), where every operand fits it: d_model a multiple of
 * 128, d_inner of 512, R + 2N of 4, dt_rank <= 160, xn, xz, u, y, blas_ws and
 * every layer's W_in, b_in, W_x, W_out, b_out 16-byte aligned, and blas_ws
 * holding (xs (R + 2N) + 4 d_model) b l floats for the parts (xs: the x_proj
 * split, at most 16), xs (R + 2N) b l below 2^31; otherwise the hipBLASLt
 * form runs.
 * ---------------------------------------------------------------------- */
typedef struct {
    float* h;
    float* xn;
    float* xz;
    float* u;
    float* x_dbl;
    float* dt;
    float* y;
    float* out;
    void* blas_ws;
    int64_t blas_ws_bytes;
    const float* norm_f;
    float* normed_out;
    float eps_f;
    int32_t d_conv;
    int32_t n_layers;
    int32_t skinny_rows;       /* the projections on mtl_linear_skinny up to this many b l rows; 0: never */
    int64_t batch, seqlen, d_model, d_inner, d_state, dt_rank;
} mtl_prefill_long_args;

int mtl_prefill_long(const mtl_prefill_long_args* args, const mtl_prefill_layer* layers, mtl_stream_t stream);

int mtl_in_proj_conv_xproj(const float* x, int64_t x_rs, const float* W_in, const float* b_in, float* conv_state,
                           const float* conv_w, const float* conv_b, int32_t d_conv, const float* W_xT, int32_t J,
                           float* xc, float* z, int64_t z_rs, float* xpart, int64_t batch, int64_t d_model,
                           int64_t d_inner, int32_t channels_per_part, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * A batched step's out_proj with the block's residual add and the next
 * block's RMSNorm inputs, so no add + norm launch runs between two blocks:
 * model.py:293 (out = out_proj(y)), 311 (x + mixer(...)) and the input side
 * of 130-135 (the next block's norm).  The product is mtl_linear_skinny's
 * with ksplit parts written to parts [ksplit, M, N] (bias in part 0); the
 * last workgroup of each n-tile to finish then adds the parts in order and
 * the residual, exactly as mtl_add_rmsnorm_parts does:
 *   h[m][n] += ((parts[0][m][n] + parts[1][m][n]) + ...)      (in place)
 * and writes x_next[m][n] = h[m][n] * w_next[n] and, per n-tile t of
 * rows_per_block columns, sq[t][m] = the sum over its columns, in order, of
 * h[m][n]^2.  mtl_in_proj_conv_xproj_normed takes x_next and sq as the next
 * block's input.  counters [N / rows_per_block] must be zero on entry (each
 * counts its tile's ksplit workgroups; none is reset), so every call needs
 * zeroed counters of its own.
 *   x: [M, K] (row stride x_rs), 1 <= M <= 32; W: [N, K] contiguous; bias:
 *   [N] or NULL; h, x_next: [M, N] contiguous, not aliasing; w_next: [N];
 *   sq: [N / rows_per_block, M].
 * N a multiple of rows_per_block (16 or 32); 1 <= ksplit <= 4; K a multiple
 * of 128 * ksplit.
 * x, W, bias, parts, h, w_next, x_next 16-byte aligned.  Deterministic.
 * ---------------------------------------------------------------------- */
int mtl_linear_skinny_residual(const float* x, int64_t x_rs, const float* W, const float* bias, float* parts,
                               int64_t M, int64_t N, int64_t K, int32_t ksplit, int32_t rows_per_block, float* h,
                               const float* w_next, float* x_next, float* sq, uint32_t* counters,
                               mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * mtl_in_proj_conv_xproj on a block input left by
 * mtl_linear_skinny_residual: x = h * w (the block norm's weight applied to
 * the residual rows h) and sq [sq_tiles, batch] the per-tile sums of h^2;
 * the in_proj outputs are scaled by rsqrt(sum over tiles / d_model + eps)
 * before b_in, which is in_proj(RMSNorm(h)) (model.py:130-135, 261) with the
 * norm applied to the dot products.  1 <= sq_tiles <= 128; other arguments
 * and rules as mtl_in_proj_conv_xproj.  Deterministic.
 * ---------------------------------------------------------------------- */
int mtl_in_proj_conv_xproj_normed(const float* x, int64_t x_rs, const float* W_in, const float* b_in,
                                  float* conv_state, const float* conv_w, const float* conv_b, int32_t d_conv,
                                  const float* W_xT, int32_t J, float* xc, float* z, int64_t z_rs, float* xpart,
                                  int64_t batch, int64_t d_model, int64_t d_inner, int32_t channels_per_part,
                                  const float* sq, int32_t sq_tiles, float eps, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused single-token decode step, fp32, batch 1, 2 or 4.
 * Together these replace one MambaBlock.step (model.py:308-311) around
 * MambaMixer.step (model.py:249-294): 3 launches per layer (4 when x_proj
 * runs as its own row GEMV) instead of one per ATen op, every weight byte
 * read once.  Deterministic: no atomics, fixed summation orders.
 *
 * mtl_decode_in: x [b, M] (or, for the first layer, emb [vocab, M] + ids
 *   [b], with resid_out [b, M] receiving the gathered rows, model.py:348; an
 *   id outside [0, vocab) makes that batch row NaN instead of reading
 *   outside the table, where the reference's nn.Embedding raises) ->
 *   RMSNorm (norm_w, eps; model.py:130-135) -> in_proj rows W_in [2D, M]
 *   (+ b_in) of channel blocks of `channels_per_block` (8 or 4: one
 *   workgroup per block of the x rows and one per block of the z rows, 2 or
 *   1 in_proj rows per wavefront; model.py:261) ->
 *   conv step with the in-place history shift of conv_state [b, D, K-1]
 *   (conv_w [D, K], conv_b; model.py:264-274) -> xc = SiLU(conv)
 *   (model.py:277), gz = SiLU(z) [b, D] -> if W_xT (x_proj transposed
 *   [D, J], J = R + 2N) is given, the split-K partial x_proj sums of each
 *   block into xpart [nblk, b, J] (model.py:279), nblk = ceil(D / cpb).
 * mtl_decode_gemv: out [b, rows] = W [rows, cols] . v [b, cols] (+ bias)
 *   (+ x_in, the residual add of model.py:311): the out_proj rows
 *   (model.py:293) and, in the 4-launch form, the x_proj rows (279).
 * mtl_decode_gemv_parts: out_parts [nparts, b, rows], part p = the product
 *   of columns [p cols/nparts, (p+1) cols/nparts) of W [rows, cols] and v
 *   [b, cols] (cols/nparts a multiple of 4, at most 4096): the x_proj rows
 *   (model.py:279) of a width whose block partials do not fit decode_in, as
 *   split-K parts that mtl_decode_ssm adds in part order (nblk = nparts).
 * mtl_decode_norm_gemv: out [b, rows] = W [rows, cols] . RMSNorm(v) (+ bias)
 *   with RMSNorm(v) = norm_w * v * rsqrt(mean(v^2) + eps): the final norm_f
 *   and the tied lm_head of MambaLM.step (model.py:351-352, RMSNorm at
 *   model.py:130-135, lm_head at 325-326) in one launch.  The rms scale is
 *   applied to each row's dot product.
 * mtl_decode_ssm: x_dbl [b, J] = sum over nblk of xpart (block order) ->
 *   dt = softplus(W_dt [D, R] . dt_low + b_dt) (model.py:281-282) ->
 *   ssm_state [b, D, N] updated in place with A = -exp(A_log) (284-289) ->
 *   y [b, D] = (C . h + D x) * gz (model.py:290-292).  N <= 16.
 * All pointers are device memory; W_in, W and v must be 16-byte aligned.
 * ---------------------------------------------------------------------- */
int mtl_decode_in(const float* x, const float* emb, const int64_t* ids, int32_t vocab, float* resid_out, const float* norm_w,
                  float eps, const float* W_in, const float* b_in, float* conv_state, const float* conv_w,
                  const float* conv_b, const float* W_xT, float* xc, float* gz, float* xpart, int32_t batch,
                  int32_t d_model, int32_t d_inner, int32_t d_conv, int32_t xdbl_cols, int32_t channels_per_block,
                  mtl_stream_t stream);
int mtl_decode_gemv(const float* v, const float* W, const float* bias, const float* x_in, float* out, int32_t batch,
                    int32_t rows, int32_t cols, mtl_stream_t stream);
int mtl_decode_gemv_parts(const float* v, const float* W, float* out_parts, int32_t batch, int32_t rows, int32_t cols,
                          int32_t nparts, mtl_stream_t stream);
int mtl_decode_norm_gemv(const float* v, const float* norm_w, float eps, const float* W, const float* bias, float* out,
                         int32_t batch, int32_t rows, int32_t cols, mtl_stream_t stream);
int mtl_decode_ssm(const float* xpart, int32_t nblk, const float* xc, const float* gz, const float* W_dt,
                   const float* b_dt, const float* A_log, const float* Dv, float* ssm_state, float* y,
                   int32_t batch, int32_t d_inner, int32_t d_state, int32_t dt_rank, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * mtl_decode_step: one fused decode step of the whole layer stack in one
 * call -- MambaLM.step (model.py:343-353) over MambaBlock.step (308-311)
 * and MambaMixer.step (249-294) -- fp32, batch 1, 2 or 4: per layer
 * mtl_decode_in, [mtl_decode_gemv_parts], mtl_decode_ssm, mtl_decode_gemv,
 * then mtl_decode_norm_gemv into logits [b, vocab].  The same launches with
 * the same arguments as calling those entry points one by one, so the same
 * bits.  With split_k, decode_in forms the x_proj partials from W_xT
 * ([d_inner, J], x_proj transposed) in blocks of channels_per_block, and
 * xpart holds ceil(d_inner / channels_per_block) of them; without it, x_proj
 * (W_x [J, d_inner]) runs as xproj_parts column parts.  Each layer's
 * conv_state [b, d_inner, d_conv - 1] and ssm_state [b, d_inner, d_state]
 * are updated in place.  Workspace: xc, gz, y [b, d_inner]; x0, x1, resid
 * [b, d_model]; xpart [parts, b, J].  d_model and d_inner multiples of 4 up
 * to 4096, d_state <= 16, dt_rank <= 256, d_conv 2..8.  Every layer's
 * pointers and these sizes are checked before the first launch.
 * ---------------------------------------------------------------------- */
typedef struct {
    const float* norm_w;       /* [d_model] the block's RMSNorm */
    float eps;
    int32_t reserved;
    const float* W_in;         /* [2 d_inner, d_model] */
    const float* b_in;         /* [2 d_inner] or NULL */
    const float* conv_w;       /* [d_inner, d_conv] */
    const float* conv_b;       /* [d_inner] or NULL */
    const float* W_xT;         /* [d_inner, J] (split_k) or NULL */
    const float* W_x;          /* [J, d_inner] (without split_k) or NULL */
    const float* W_dt;         /* [d_inner, dt_rank] */
    const float* dt_bias;      /* [d_inner] */
    const float* A_log;        /* [d_inner, d_state] */
    const float* Dv;           /* [d_inner] or NULL */
    const float* W_out;        /* [d_model, d_inner] */
    const float* b_out;        /* [d_model] or NULL */
    float* conv_state;
    float* ssm_state;
} mtl_decode_layer;

typedef struct {
    const int64_t* ids;        /* [b] token ids */
    const float* emb;          /* [vocab, d_model], also the tied lm_head */
    const float* norm_f;       /* [d_model] */
    float* logits;             /* [b, vocab] */
    float* xc;
    float* gz;
    float* y;
    float* x0;
    float* x1;
    float* resid;
    float* xpart;
    float eps_f;
    int32_t vocab;
    int32_t n_layers;
    int32_t batch;
    int32_t d_model, d_inner, d_state, dt_rank, d_conv, channels_per_block, split_k, xproj_parts;
} mtl_decode_step_args;

int mtl_decode_step(const mtl_decode_step_args* args, const mtl_decode_layer* layers, mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * mtl_decode_step_batched: a batched decode step of the whole layer stack in
 * one call -- MambaLM.step (model.py:343-353) over MambaBlock.step (308-311)
 * and MambaMixer.step (249-294) -- fp32, 1..32 rows, up to the lm_head's
 * input.  Per layer: mtl_in_proj_conv_xproj (with fold, from layer 1 on,
 * mtl_in_proj_conv_xproj_normed), mtl_sum_parts, mtl_selective_state_update,
 * then out_proj as 4 split-K parts: with fold and before the last layer
 * mtl_linear_skinny_residual, otherwise mtl_linear_skinny followed by
 * mtl_add_rmsnorm_parts (the residual add and the next RMSNorm; norm_f after
 * the last layer).  The tile choices are those of the Python layer's per-op
 * step, so the results are the same bits as calling those entry points one
 * by one.
 *   h           [b, d_model] in: the embedding rows of the step's tokens;
 *               out: the residual stream after the last layer
 *   normed_out  [b, d_model] out: norm_f of it, the tied lm_head's input
 *   workspace   inp, xn [b, d_model]; xc, z, y [b, d_inner]; xpart
 *               [d_inner / 16, b, J]; x_dbl [b, J]; parts [4, b, d_model];
 *               with fold also sq [d_model / 16, b] and counters
 *               [n_layers - 1, d_model / 16], zero-filled before each call
 *               (a call needs its own zeroed counters); xn, sq and counters
 *               may be NULL without fold
 *   layers      mtl_decode_layer with W_xT ([d_inner, J], x_proj transposed)
 *               and conv_w [d_inner, d_conv]; W_x is not read.  Each layer's
 *               conv_state [b, d_inner, d_conv - 1] and ssm_state
 *               [b, d_inner, d_state] are updated in place.
 * d_model a multiple of 128 (at least 256), d_inner a multiple of 512,
 * d_state <= 16, dt_rank <= 256 with dt_rank + 2 d_state <= 288, d_conv
 * 2..4.  Every layer's pointers, its eps (>= 0, not NaN), the sizes and the
 * alignments the entry points take are checked before the first launch.
 * ---------------------------------------------------------------------- */
typedef struct {
    float* h;
    float* normed_out;
    const float* norm_f;       /* [d_model] */
    float* inp;
    float* xn;
    float* xc;
    float* z;
    float* y;
    float* xpart;
    float* x_dbl;
    float* parts;
    float* sq;
    uint32_t* counters;
    float eps_f;
    int32_t n_layers;
    int32_t batch;
    int32_t d_model, d_inner, d_state, dt_rank, d_conv;
    int32_t fold;              /* 1: residual add + norm folded into the projections */
    int32_t reserved;
} mtl_decode_step_batched_args;

int mtl_decode_step_batched(const mtl_decode_step_batched_args* args, const mtl_decode_layer* layers,
                            mtl_stream_t stream);

/* ------------------------------------------------------------------------
 * mtl_decode_step_persist: the same step -- MambaLM.step (model.py:343-353)
 * over MambaBlock.step (308-311) and MambaMixer.step (249-294) -- for batch
 * 1 as ONE persistent launch over every layer, then the norm_f + tied
 * lm_head GEMV of mtl_decode_norm_gemv into logits [1, vocab].  Its
 * workgroups stay resident and exchange the x_proj partials, y and the new
 * residual through the workspace three times per layer instead of ending
 * three kernels per layer.
 *   args     as mtl_decode_step (batch 1; x0 receives the final residual;
 *            xc, gz, y, x1, resid, xpart, channels_per_block, split_k and
 *            xproj_parts are not used).
 *   layers   host array [n_layers]: validated here; each layer's
 *            conv_state [1, D, K-1] and ssm_state [1, D, N] are updated in
 *            place.  W_xT ([d_inner, J], x_proj transposed) is required.
 *   layers_dev  a device copy of the same array (its weight pointers are
 *            read by the kernel; its cache fields are not).
 *   workspace   device memory of mtl_decode_persist_workspace_bytes(),
 *            256-byte aligned, zero-filled before its first use and then
 *            left to the library: it carries an epoch from call to call
 *            (word 0) and an error word (word 1, nonzero after a wait timed
 *            out; the logits of that call are then NaN and its layer caches
 *            partly advanced).  After a nonzero error word the workspace
 *            must be zero-filled again before the next call: a workgroup of
 *            the failed launch that started late may have left slots tagged
 *            for the next one.  Calls that share a workspace must be ordered
 *            (one stream); concurrent calls race.
 *   blocking 0 picks the register blocking (workgroups per launch) itself;
 *            1 and 2 force 6 or 3 channels per compute wavefront pair.
 * Shapes: d_model a multiple of 4 up to 1024, d_inner a multiple of 4 up to
 * 2 d_model, d_state <= 16, dt_rank <= 64 with dt_rank + 2 d_state <= 128,
 * d_conv 2..4, n_layers <= 64.  All workgroups must be co-resident: the grid
 * is at most the device's CU count (checked) and the GPU must not be shared
 * with other long kernels meanwhile (a wait then times out, see above).
 * ---------------------------------------------------------------------- */
size_t mtl_decode_persist_workspace_bytes(int32_t d_model, int32_t d_inner, int32_t d_state, int32_t dt_rank);
/* Workgroups mtl_decode_step_persist launches for this shape and blocking on
 * a device of 256 or more CUs, or 0 when it does not take the shape. */
int32_t mtl_decode_persist_grid(int32_t d_model, int32_t d_inner, int32_t d_state, int32_t dt_rank, int32_t d_conv,
                                int32_t n_layers, int32_t blocking);
int mtl_decode_step_persist(const mtl_decode_step_args* args, const mtl_decode_layer* layers,
                            const mtl_decode_layer* layers_dev, void* workspace, size_t workspace_bytes,
                            int32_t blocking, mtl_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MTL_H */
