"""numpy restatement of the reference Mamba mixer math (test infrastructure).

Every function names the reference lines it follows (paths relative to the
mamba-tp-lite repository).  `dtype=np.float32` keeps the reference's op
order and intermediate roundings (materialize dA / dB / dBx, then a
sequential loop over tokens); `dtype=np.float64` is the brute-force variant
used as the high-precision target.

Layout conventions (same as the reference):
  x, z, u, delta, dt : [b, D, l]   (channel-major, as after model.py:199)
  B, C               : [b, l, N]   (token-major, as split from x_dbl at model.py:215)
  A                  : [D, N]      (already negated: A = -exp(A_log), model.py:220)
  conv_w             : [D, K]      (nn.Conv1d weight [D,1,K] squeezed, model.py:267)
  ssm_state          : [b, D, N];  conv_state: [b, D, K-1]  (model.py:100-101)

Parity: pinned in tests/test_oracle.py by pins.py (closed-form scan,
np.convolve conv, geometric series), by the l=1 prefill == step identity,
by chunked-prefill continuation and by float32-vs-float64 agreement.
"""
from __future__ import annotations

import numpy as np


# ---------------------------------------------------------------------------
# elementwise helpers
# ---------------------------------------------------------------------------
def softplus(x: np.ndarray) -> np.ndarray:
    """torch.nn.functional.softplus(beta=1, threshold=20): identity above 20,
    log1p(exp(x)) otherwise (used at model.py:218 and model.py:282)."""
    x = np.asarray(x)
    with np.errstate(over="ignore"):
        return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20)))).astype(x.dtype)


def silu(x: np.ndarray) -> np.ndarray:
    """F.silu = x * sigmoid(x) (model.py:209, 238, 277, 292)."""
    x = np.asarray(x)
    with np.errstate(over="ignore"):
        return (x / (1 + np.exp(-x))).astype(x.dtype)


def inv_softplus(y: np.ndarray) -> np.ndarray:
    """y + log(-expm1(-y)): the dt_bias init of HF Mamba
    (transformers modeling_mamba.py:354-355); used only to build inputs."""
    y = np.asarray(y, dtype=np.float64)
    return y + np.log(-np.expm1(-y))


# ---------------------------------------------------------------------------
# conv1d (model.py:198-212 prefill, model.py:264-277 step)
# ---------------------------------------------------------------------------
def causal_conv1d(x, w, bias=None, conv_state=None, dtype=np.float32):
    """Depthwise causal conv over l with K taps, left-padded by the incoming
    conv history (or zeros), model.py:202-208; returns the PRE-activation
    output [b,D,l] and the final conv state = last K-1 padded inputs
    (model.py:210-212)."""
    x = np.asarray(x, dtype=dtype)
    w = np.asarray(w, dtype=dtype)
    b, D, l = x.shape
    K = w.shape[1]
    if conv_state is not None:
        xp = np.concatenate([np.asarray(conv_state, dtype=dtype), x], axis=-1)  # model.py:203
    else:
        xp = np.concatenate([np.zeros((b, D, K - 1), dtype=dtype), x], axis=-1)  # model.py:205
    out = np.zeros((b, D, l), dtype=dtype)
    # F.conv1d is a cross-correlation: out[t] = sum_k w[k] * xp[t + k]
    for k in range(K):
        out = out + w[None, :, k:k + 1] * xp[:, :, k:k + l]
    if bias is not None:
        out = out + np.asarray(bias, dtype=dtype)[None, :, None]
    final_state = xp[:, :, xp.shape[-1] - (K - 1):].copy() if K > 1 else np.zeros((b, D, 0), dtype)
    return out.astype(dtype), final_state.astype(dtype)


def conv_step(conv_state, x_t, w, bias=None, dtype=np.float32):
    """Single-token conv (model.py:265-277): conv_in = cat(state, x),
    sum(conv_in * w) + bias, state <- conv_in[..., 1:] (returned, the caller
    decides whether to write in place).  Returns (pre-activation [b,D], new_state)."""
    conv_in = np.concatenate([np.asarray(conv_state, dtype), np.asarray(x_t, dtype)[..., None]], axis=-1)
    out = (conv_in * np.asarray(w, dtype)[None]).sum(axis=-1)
    if bias is not None:
        out = out + np.asarray(bias, dtype)
    return out.astype(dtype), conv_in[..., 1:].copy()


# ---------------------------------------------------------------------------
# selective scan (model.py:216-238)
# ---------------------------------------------------------------------------
def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, h0=None,
                   delta_softplus=True, dtype=np.float32):
    """Materialize-then-loop selective scan, model.py:216-238.

    u, delta, z: [b,D,l]; A: [D,N]; B, C: [b,l,N]; D: [D]; delta_bias: [D];
    h0: [b,D,N] or None (model.py:226-230).  Returns (y [b,D,l], h_last [b,D,N]).
    delta -> (+delta_bias) -> softplus as model.py:217-218; dA = exp(dt*A)
    (222); dB = dt*B (223); dBx = dB*x (224); h_t = dA_t*h + dBx_t (233);
    y_t = sum_n h_t[n] C_t[n] (234); y += x*D (237); y *= silu(z) (238).
    """
    u = np.asarray(u, dtype)
    dt = np.asarray(delta, dtype)
    if delta_bias is not None:
        dt = dt + np.asarray(delta_bias, dtype)[None, :, None]
    if delta_softplus:
        dt = softplus(dt)
    A = np.asarray(A, dtype)
    B = np.asarray(B, dtype)
    C = np.asarray(C, dtype)
    b, Dm, l = u.shape
    N = A.shape[1]
    dA = np.exp(dt[..., None] * A[None, :, None, :])          # [b,D,l,N]
    dB = dt[..., None] * B[:, None, :, :]                    # [b,D,l,N]
    dBx = dB * u[..., None]                                  # [b,D,l,N]
    h = np.zeros((b, Dm, N), dtype) if h0 is None else np.asarray(h0, dtype).copy()
    ys = np.empty((b, l, Dm), dtype)
    for t in range(l):
        h = dA[:, :, t] * h + dBx[:, :, t]
        ys[:, t] = np.einsum("bdn,bn->bd", h, C[:, t])
    y = ys.transpose(0, 2, 1)                                # [b,D,l]
    if D is not None:
        y = y + u * np.asarray(D, dtype)[None, :, None]
    if z is not None:
        y = y * silu(np.asarray(z, dtype))
    return y.astype(dtype), h.astype(dtype)


def selective_scan_bnl(u, delta, A, B, C, D=None, z=None, delta_bias=None, h0=None,
                       delta_softplus=True, dtype=np.float32):
    """Same scan with B, C given channel-major as [b,N,l] (the isolated-op
    layout of the selective-scan benchmark)."""
    return selective_scan(u, delta, A, np.swapaxes(B, 1, 2), np.swapaxes(C, 1, 2), D, z,
                          delta_bias, h0, delta_softplus, dtype)


def selective_state_update(ssm_state, x, dt_low, W_dt, b_dt, A, B, C, D, z, dtype=np.float32):
    """Single-token SSM update, model.py:279-292 (after x_proj):
    dt = softplus(dt_low @ W_dt^T + b_dt) (281-282); dA = exp(dt*A) (285);
    dBx = (dt*B)*x (286-287); h <- h*dA + dBx (289, the state written back);
    y = sum_n h_new*C + x*D, then *silu(z) (290-292).
    Shapes: ssm_state [b,D,N], x,z [b,D], dt_low [b,R], W_dt [D,R], B,C [b,N].
    Returns (y [b,D], new_state [b,D,N])."""
    x = np.asarray(x, dtype)
    dt = np.asarray(dt_low, dtype) @ np.asarray(W_dt, dtype).T + np.asarray(b_dt, dtype)
    dt = softplus(dt)
    A = np.asarray(A, dtype)
    dA = np.exp(dt[..., None] * A[None])
    dB = dt[..., None] * np.asarray(B, dtype)[:, None, :]
    dBx = dB * x[..., None]
    h = (np.asarray(ssm_state, dtype) * dA + dBx).astype(dtype)
    y = np.einsum("bdn,bn->bd", h, np.asarray(C, dtype))
    y = y + x * np.asarray(D, dtype)
    y = y * silu(np.asarray(z, dtype))
    return y.astype(dtype), h


# ---------------------------------------------------------------------------
# mixer / block / LM (model.py:124-135, 184-294, 297-365)
# ---------------------------------------------------------------------------
def rmsnorm(x, weight, eps=1e-5, dtype=np.float32):
    """RMSNorm in fp32, model.py:130-135: w * (x * rsqrt(mean(x^2) + eps))."""
    x = np.asarray(x, dtype)
    var = np.mean(x * x, axis=-1, keepdims=True)
    return (np.asarray(weight, dtype) * (x / np.sqrt(var + dtype(eps)))).astype(dtype)


def _linear(x, w, b=None):
    y = x @ w.T
    return y + b if b is not None else y


def mixer_prefill(p, x, conv_state=None, ssm_state=None, dtype=np.float32, act=None):
    """MambaMixer.prefill, model.py:184-241.  p holds numpy weights:
    in_proj_w [2D,M] (+in_proj_b), conv_w [D,K], conv_b [D], x_proj_w [R+2N,D],
    dt_proj_w [D,R], dt_proj_b [D], A_log [D,N], D [D], out_proj_w [M,D]
    (+out_proj_b).  x: [b,l,M].  Returns (out [b,l,M], conv_state, ssm_state).

    act, if given, is applied to each activation tensor as an op stores it,
    modelling a model whose activations are held in a narrower type (e.g. a
    round to bfloat16) while the scan state keeps `dtype`: the in_proj output
    (model.py:197), SiLU of the conv (206-209; conv and SiLU as one op), the
    x_proj output (214), the dt_proj output (216), the gated scan output
    (233-238; the scan as one op) and out_proj's output (239).  Each op
    computes in `dtype` from its rounded inputs."""
    P = {k: (np.asarray(v, dtype) if v is not None else None) for k, v in p.items()}
    x = np.asarray(x, dtype)
    store = (lambda t: np.asarray(act(t), dtype)) if act is not None else (lambda t: t)
    Dm = P["D"].shape[0]
    N = P["A_log"].shape[1]
    R = P["dt_proj_w"].shape[1]
    xz = store(_linear(x, P["in_proj_w"], P.get("in_proj_b")))         # model.py:197
    xs, z = xz[..., :Dm], xz[..., Dm:]                                  # model.py:198
    xs = np.ascontiguousarray(xs.transpose(0, 2, 1))                     # model.py:199
    conv, fstate = causal_conv1d(xs, P["conv_w"], P.get("conv_b"), conv_state, dtype)
    xs = store(silu(conv))                                              # model.py:209
    x_dbl = store(_linear(xs.transpose(0, 2, 1), P["x_proj_w"]))         # model.py:214
    dt, B, C = x_dbl[..., :R], x_dbl[..., R:R + N], x_dbl[..., R + N:]   # model.py:215
    dt = store(P["dt_proj_w"] @ dt.transpose(0, 2, 1))                   # model.py:216
    A = -np.exp(P["A_log"])                                             # model.py:220
    y, h = selective_scan(xs, dt, A, B, C, P["D"], z.transpose(0, 2, 1),
                          delta_bias=P["dt_proj_b"], h0=ssm_state, delta_softplus=True, dtype=dtype)
    y = store(y)
    out = store(_linear(y.transpose(0, 2, 1), P["out_proj_w"], P.get("out_proj_b")))  # model.py:239
    return out.astype(dtype), fstate, h


def mixer_step(p, x_t, conv_state, ssm_state, dtype=np.float32):
    """MambaMixer.step, model.py:249-294.  x_t: [b,M].  Updates conv_state and
    ssm_state IN PLACE (model.py:274, 289) and returns out [b,M]."""
    P = {k: (np.asarray(v, dtype) if v is not None else None) for k, v in p.items()}
    Dm = P["D"].shape[0]
    N = P["A_log"].shape[1]
    R = P["dt_proj_w"].shape[1]
    xz = _linear(np.asarray(x_t, dtype), P["in_proj_w"], P.get("in_proj_b"))  # model.py:261
    xs, z = xz[..., :Dm], xz[..., Dm:]
    if P["conv_w"].shape[1] > 1:
        conv, new_cs = conv_step(conv_state, xs, P["conv_w"], P.get("conv_b"), dtype)
        conv_state[...] = new_cs                                        # model.py:274
    else:
        # d_conv == 1: the step takes x as is, with neither the 1-tap weight
        # nor the conv bias (model.py:275-276), unlike prefill (206-208)
        conv = xs
    xs = silu(conv)                                                     # model.py:277
    x_dbl = _linear(xs, P["x_proj_w"])                                  # model.py:279
    dt_low, B, C = x_dbl[..., :R], x_dbl[..., R:R + N], x_dbl[..., R + N:]
    A = -np.exp(P["A_log"])
    y, h = selective_state_update(ssm_state, xs, dt_low, P["dt_proj_w"], P["dt_proj_b"],
                                  A, B, C, P["D"], z, dtype)
    ssm_state[...] = h                                                  # model.py:289
    out = _linear(y, P["out_proj_w"], P.get("out_proj_b"))              # model.py:293
    return out.astype(dtype)


def lm_prefill(weights, ids, cache=None, eps=1e-5, dtype=np.float32):
    """MambaLM.prefill, model.py:328-341 (+ MambaBlock.prefill 303-306).
    weights: {"embedding": [V,M], "norm_f": [M], "layers": [{"norm": [M], **mixer}]}.
    cache: list of (conv_state, ssm_state) or None.  Returns (logits, new cache)."""
    E = np.asarray(weights["embedding"], dtype)
    x = E[np.asarray(ids)]
    new_cache = []
    for i, lw in enumerate(weights["layers"]):
        cs, hs = (cache[i] if cache is not None else (None, None))
        y, c2, h2 = mixer_prefill(lw, rmsnorm(x, lw["norm"], eps, dtype), cs, hs, dtype)
        x = x + y
        new_cache.append((c2, h2))
    x = rmsnorm(x, weights["norm_f"], eps, dtype)
    return (x @ E.T).astype(dtype), new_cache


def lm_step(weights, ids, cache, eps=1e-5, dtype=np.float32):
    """MambaLM.step, model.py:343-353: ids [b,1]; cache updated in place.
    Returns logits [b,1,V]."""
    E = np.asarray(weights["embedding"], dtype)
    x = E[np.asarray(ids)[:, 0]]
    for i, lw in enumerate(weights["layers"]):
        cs, hs = cache[i]
        x = x + mixer_step(lw, rmsnorm(x, lw["norm"], eps, dtype), cs, hs, dtype)
    x = rmsnorm(x, weights["norm_f"], eps, dtype)
    return (x @ E.T).astype(dtype)[:, None, :]
