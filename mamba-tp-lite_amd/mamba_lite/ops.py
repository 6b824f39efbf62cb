"""torch-facing wrappers of the libmtl HIP kernels.

Each function validates shapes, dtypes, devices and strides on the host
(so a kernel never sees operands that disagree with its grid), then calls
the C ABI on torch's current stream.  Inputs must be GPU tensors: there is
no CPU path, a CPU tensor raises.

Shape conventions follow the reference mixer (mamba_lite/model.py):
  u, delta, z, y : [b, D, l]  (any view whose l-stride or D-stride is 1)
  B, C           : [b, N, l]  (strided views of x_dbl are fine)
  A / A_log      : [D, N];  D, delta_bias : [D];  ssm state [b, D, N] fp32
"""
from __future__ import annotations

import contextlib
import ctypes

import torch

from . import _lib

_ACT_DTYPES = {torch.float32: _lib.MTL_F32, torch.bfloat16: _lib.MTL_BF16}


# These helpers run on every launch; at small sizes host time decides the
# speed of a call, so they compare device indices rather than building
# torch.device objects, and hand ctypes plain ints.
_NO_GUARD = contextlib.nullcontext()
_current_device = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _dev_guard(t: torch.Tensor):
    if not t.is_cuda:
        raise RuntimeError(f"mamba_lite kernels need GPU tensors, got a tensor on {t.device} "
                           "(there is no CPU fallback)")
    idx = t.get_device()
    if idx != _current_device():
        return torch.cuda.device(idx)
    return _NO_GUARD


# torch's current stream of a device as a raw handle: the private accessor
# skips building a torch.cuda.Stream object per call (about 4.5 us of host time
# per kernel launch, which decides small prefills); the public route is the
# fallback where a torch build lacks it.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _act_code(*ts) -> int:
    dt = None
    for t in ts:
        if t is None:
            continue
        if dt is None:
            dt = t.dtype
        elif t.dtype != dt:
            dt = False
            break
    if dt is None or dt is False:
        dts = {t.dtype for t in ts if t is not None}
        raise TypeError(f"activations must share one dtype, got {sorted(map(str, dts))}")
    code = _ACT_DTYPES.get(dt)
    if code is None:
        raise TypeError(f"activation dtype must be float32 or bfloat16, got {dt}")
    return code


def _same_device(ref: torch.Tensor, *ts):
    dev = ref.get_device()
    for t in ts:
        if t is not None and t.get_device() != dev:
            raise RuntimeError(f"all operands must be on {ref.device}, got {t.device}")


def _f32_vec(t, n, name):
    if t is None:
        return None
    if t.dtype != torch.float32 or t.dim() != 1 or t.shape[0] != n or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 vector of length {n}, got "
                         f"{tuple(t.shape)} {t.dtype}")
    return t


def _f32_mat(t, shape, name):
    if t.dtype != torch.float32 or t.shape != shape or not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous float32 {tuple(shape)}, got {tuple(t.shape)} {t.dtype}"
                         f"{'' if t.is_contiguous() else ' (non-contiguous)'}")
    return t


def _bdl_layout_ok(*ts):
    """True if every [b,D,l] operand is channel-major (l-stride 1) or every one
    is token-major (D-stride 1)."""
    cm = tm = True
    for t in ts:
        if t is not None:
            st = t.stride()
            cm = cm and st[2] == 1
            tm = tm and st[1] == 1
    return cm or tm


# --------------------------------------------------------------------------- selective scan
SCAN_ALGOS = {"auto": 0, "tiled": 1, "chunked": 2}


def selective_scan(u, delta, A, B, C, D=None, z=None, delta_bias=None, h0=None, delta_softplus=True,
                   a_is_log=False, y=None, h_out=None, return_last_state=True, algo="auto"):
    """Fused selective scan (mtl_selective_scan_fwd); see include/mtl.h.

    Returns (y [b,D,l] in the activation dtype, h_last [b,D,N] fp32) -- the
    pair MambaMixer.prefill gets from its scan loop (model.py:226-241).
    `y` / `h_out` may be preallocated (y with the same layout rules as u)."""
    if u.dim() != 3:
        raise ValueError(f"u must be [b, D, l], got {tuple(u.shape)}")
    b, Dm, L = u.shape
    if A.dim() != 2 or A.shape[0] != Dm:
        raise ValueError(f"A must be [D={Dm}, N], got {tuple(A.shape)}")
    N = A.shape[1]
    _f32_mat(A, (Dm, N), "A")
    for name, t in (("delta", delta), ("z", z)):
        if t is not None and tuple(t.shape) != (b, Dm, L):
            raise ValueError(f"{name} must be {(b, Dm, L)}, got {tuple(t.shape)}")
    for name, t in (("B", B), ("C", C)):
        if tuple(t.shape) != (b, N, L):
            raise ValueError(f"{name} must be {(b, N, L)}, got {tuple(t.shape)}")
    _f32_vec(D, Dm, "D")
    _f32_vec(delta_bias, Dm, "delta_bias")
    if h0 is not None:
        _f32_mat(h0, (b, Dm, N), "h0")
    code = _act_code(u, delta, z, B, C)
    _same_device(u, delta, z, B, C, A, D, delta_bias, h0, y, h_out)
    if not _bdl_layout_ok(u, delta, z, y):
        u, delta = u.contiguous(), delta.contiguous()
        z = z.contiguous() if z is not None else None
    if y is None:
        if u.stride(1) == 1 and L > 1:
            y = torch.empty(b, L, Dm, device=u.device, dtype=u.dtype).transpose(1, 2)
        else:
            y = torch.empty(b, Dm, L, device=u.device, dtype=u.dtype)
    elif tuple(y.shape) != (b, Dm, L) or y.dtype != u.dtype:
        raise ValueError(f"y must be {(b, Dm, L)} {u.dtype}, got {tuple(y.shape)} {y.dtype}")
    if not _bdl_layout_ok(u, delta, z, y):
        raise ValueError("u, delta, z and y must all have l-stride 1 or all have D-stride 1")
    if h_out is None and return_last_state:
        h_out = torch.empty(b, Dm, N, device=u.device, dtype=torch.float32)
    elif h_out is not None:
        _f32_mat(h_out, (b, Dm, N), "h_out")

    p = _lib.ScanParams()
    p.u, (p.u_sb, p.u_sd, p.u_sl) = u.data_ptr(), u.stride()
    p.delta, (p.delta_sb, p.delta_sd, p.delta_sl) = delta.data_ptr(), delta.stride()
    if z is not None:
        p.z, (p.z_sb, p.z_sd, p.z_sl) = z.data_ptr(), z.stride()
    p.B, (p.B_sb, p.B_sn, p.B_sl) = B.data_ptr(), B.stride()
    p.C, (p.C_sb, p.C_sn, p.C_sl) = C.data_ptr(), C.stride()
    p.y, (p.y_sb, p.y_sd, p.y_sl) = y.data_ptr(), y.stride()
    p.A = A.data_ptr()
    p.D = D.data_ptr() if D is not None else None
    p.delta_bias = delta_bias.data_ptr() if delta_bias is not None else None
    p.h0 = h0.data_ptr() if h0 is not None else None
    p.h_out = h_out.data_ptr() if h_out is not None else None
    p.batch, p.seqlen, p.dim, p.dstate = b, L, Dm, N
    p.dtype, p.delta_softplus, p.a_is_log = code, int(bool(delta_softplus)), int(bool(a_is_log))
    p.algo = SCAN_ALGOS[algo]
    with _dev_guard(u):
        _lib.check(_lib.load().mtl_selective_scan_fwd(ctypes.byref(p), _stream(u)), "selective_scan_fwd")
    return y, h_out


# --------------------------------------------------------------------------- conv
def causal_conv1d(x, weight, bias=None, conv_state=None, silu=True, out=None, final_state=None,
                  return_final_state=True):
    """Fused causal depthwise conv (+SiLU) over x [b,D,l] (mtl_causal_conv1d_fwd).
    weight: [D,K] or [D,1,K] fp32; conv_state: [b,D,K-1] incoming history.
    Returns (out [b,D,l], final conv state [b,D,K-1]) as model.py:206-212."""
    if x.dim() != 3:
        raise ValueError(f"x must be [b, D, l], got {tuple(x.shape)}")
    b, Dm, L = x.shape
    w = weight.reshape(weight.shape[0], weight.shape[-1]) if weight.dim() == 3 else weight
    if w.shape[0] != Dm:
        raise ValueError(f"weight must be [D={Dm}, K], got {tuple(weight.shape)}")
    K = w.shape[1]
    _f32_mat(w, (Dm, K), "weight")
    _f32_vec(bias, Dm, "bias")
    code = _act_code(x, out, conv_state, final_state)
    _same_device(x, w, bias, conv_state, out, final_state)
    if conv_state is not None and (tuple(conv_state.shape) != (b, Dm, K - 1) or not conv_state.is_contiguous()):
        raise ValueError(f"conv_state must be contiguous {(b, Dm, K - 1)}, got {tuple(conv_state.shape)}")
    if out is None:
        if x.stride(1) == 1 and L > 1:
            out = torch.empty(b, L, Dm, device=x.device, dtype=x.dtype).transpose(1, 2)
        else:
            out = torch.empty(b, Dm, L, device=x.device, dtype=x.dtype)
    elif tuple(out.shape) != (b, Dm, L):
        raise ValueError(f"out must be {(b, Dm, L)}, got {tuple(out.shape)}")
    if final_state is None and return_final_state:
        final_state = torch.empty(b, Dm, K - 1, device=x.device, dtype=x.dtype)
    elif final_state is not None and (tuple(final_state.shape) != (b, Dm, K - 1) or not final_state.is_contiguous()):
        raise ValueError(f"final_state must be contiguous {(b, Dm, K - 1)}")
    if final_state is not None and conv_state is not None and final_state.numel() > 0 and \
            final_state.data_ptr() == conv_state.data_ptr():
        raise ValueError("final_state must not alias conv_state")

    p = _lib.ConvParams()
    p.x, (p.x_sb, p.x_sd, p.x_sl) = x.data_ptr(), x.stride()
    p.out, (p.out_sb, p.out_sd, p.out_sl) = out.data_ptr(), out.stride()
    p.w = w.data_ptr()
    p.bias = bias.data_ptr() if bias is not None else None
    # K = 1 carries no history: its empty states go over as NULL
    p.conv_state_in = conv_state.data_ptr() if conv_state is not None and conv_state.numel() else None
    p.conv_state_out = final_state.data_ptr() if final_state is not None and final_state.numel() else None
    p.batch, p.seqlen, p.dim, p.width = b, L, Dm, K
    p.dtype, p.silu = code, int(bool(silu))
    with _dev_guard(x):
        _lib.check(_lib.load().mtl_causal_conv1d_fwd(ctypes.byref(p), _stream(x)), "causal_conv1d_fwd")
    return out, final_state


def conv_step(conv_state, x, weight, bias=None, silu=True, out=None):
    """In-place single-token conv (mtl_conv_step).  conv_state: [b,D,K-1]
    contiguous, updated in place; x: [b,D] with channel stride 1."""
    b, Dm = x.shape
    w = weight.reshape(weight.shape[0], weight.shape[-1]) if weight.dim() == 3 else weight
    K = w.shape[1]
    _f32_mat(w, (Dm, K), "weight")
    _f32_vec(bias, Dm, "bias")
    if tuple(conv_state.shape) != (b, Dm, K - 1) or not conv_state.is_contiguous():
        raise ValueError(f"conv_state must be contiguous {(b, Dm, K - 1)}, got {tuple(conv_state.shape)}")
    if x.stride(1) != 1:
        raise ValueError("x must have channel stride 1")
    if out is None:
        out = torch.empty(b, Dm, device=x.device, dtype=x.dtype)
    elif tuple(out.shape) != (b, Dm) or out.stride(1) != 1:
        raise ValueError(f"out must be {(b, Dm)} with channel stride 1")
    code = _act_code(x, conv_state, out)
    _same_device(x, conv_state, w, bias, out)
    with _dev_guard(x):
        _lib.check(_lib.load().mtl_conv_step(_ptr(conv_state), _ptr(x), x.stride(0), _ptr(w), _ptr(bias), _ptr(out),
                                             out.stride(0), b, Dm, K, code, int(bool(silu)), _stream(x)),
                   "conv_step")
    return out


XPROJ_BLOCK = 32   # channels per x_proj partial block of conv_step_xproj


def conv_step_xproj(conv_state, x, weight, bias, W_xT, out=None, xpart=None):
    """mtl_conv_step_xproj: in-place conv step + SiLU of x [b, D] (fp32,
    channel stride 1, b <= 32) into out [b, D], and the x_proj partials of
    each 32-channel block into xpart [ceil(D/32), b, J] (W_xT: [D, J]).
    Returns (out, xpart); ops.sum_parts(xpart) is x_dbl."""
    b, Dm = x.shape
    w = weight.reshape(weight.shape[0], weight.shape[-1]) if weight.dim() == 3 else weight
    K = w.shape[1]
    _f32_mat(w, (Dm, K), "weight")
    _f32_vec(bias, Dm, "bias")
    J = W_xT.shape[1]
    _f32_mat(W_xT, (Dm, J), "W_xT")
    _f32_mat(conv_state, (b, Dm, K - 1), "conv_state")
    if x.dtype != torch.float32 or x.stride(1) != 1:
        raise ValueError("x must be float32 with channel stride 1")
    nblk = -(-Dm // XPROJ_BLOCK)
    if out is None:
        out = torch.empty(b, Dm, device=x.device, dtype=torch.float32)
    elif tuple(out.shape) != (b, Dm) or out.dtype != torch.float32 or out.stride(1) != 1:
        raise ValueError(f"out must be float32 {(b, Dm)} with channel stride 1")
    if xpart is None:
        xpart = torch.empty(nblk, b, J, device=x.device, dtype=torch.float32)
    else:
        _f32_mat(xpart, (nblk, b, J), "xpart")
    _same_device(x, conv_state, w, bias, W_xT, out, xpart)
    with _dev_guard(x):
        _lib.check(_lib.load().mtl_conv_step_xproj(_ptr(conv_state), _ptr(x), x.stride(0), _ptr(w), _ptr(bias),
                                                   _ptr(out), out.stride(0), _ptr(W_xT), _ptr(xpart), b, Dm, K, J,
                                                   _stream(x)), "conv_step_xproj")
    return out, xpart


def in_proj_conv_prefill_ok(x2, W_in, d_conv) -> bool:
    """Whether mtl_in_proj_conv_prefill takes this prefill: fp32 on the GPU,
    1..64 token rows, d_model a multiple of 128, d_inner a multiple of 16,
    d_conv 2..4, 16-byte aligned rows."""
    if x2.dim() != 2 or W_in.dim() != 2 or x2.dtype != torch.float32 or W_in.dtype != torch.float32:
        return False
    M, K = x2.shape
    D = W_in.shape[0] // 2
    return (x2.is_cuda and 1 <= M <= SKINNY_MAX_ROWS and K % 128 == 0 and W_in.shape == (2 * D, K) and D % 16 == 0
            and 2 <= d_conv <= 4 and x2.stride(1) == 1 and x2.stride(0) % 4 == 0 and W_in.is_contiguous()
            and x2.data_ptr() % 16 == 0 and W_in.data_ptr() % 16 == 0)


def in_proj_conv_prefill(x2, W_in, b_in, conv_w, conv_b, conv_state_in, conv_state_out, batch, seqlen):
    """mtl_in_proj_conv_prefill: x2 [b l, d_model] -> (u [b l, D] =
    SiLU(causal conv of the x half), z [b l, D]); conv_state_out [b, D, K-1]
    receives the final history (conv_state_in [b, D, K-1] or None: zeros)."""
    M, K = x2.shape
    D = W_in.shape[0] // 2
    Kc = conv_w.shape[-1]
    if not in_proj_conv_prefill_ok(x2, W_in, Kc) or M != batch * seqlen:
        raise ValueError("in_proj_conv_prefill: fp32 x [b l <= 64, K%128==0], W_in [2D, K] (D%16==0), d_conv 2..4")
    _f32_mat(conv_w, (D, Kc), "conv_w")
    _f32_vec(b_in, 2 * D, "b_in")
    _f32_vec(conv_b, D, "conv_b")
    for name, t in (("conv_state_in", conv_state_in), ("conv_state_out", conv_state_out)):
        if t is not None and (tuple(t.shape) != (batch, D, Kc - 1) or t.dtype != torch.float32
                              or not t.is_contiguous()):
            raise ValueError(f"{name} must be contiguous float32 {(batch, D, Kc - 1)}")
    if conv_state_out is None:
        raise ValueError("conv_state_out is required")
    u = torch.empty(M, D, device=x2.device, dtype=torch.float32)
    z = torch.empty(M, D, device=x2.device, dtype=torch.float32)
    _same_device(x2, W_in, b_in, conv_w, conv_b, conv_state_in, conv_state_out)
    with _dev_guard(x2):
        _lib.check(_lib.load().mtl_in_proj_conv_prefill(_ptr(x2), x2.stride(0), _ptr(W_in), _ptr(b_in), _ptr(conv_w),
                                                        _ptr(conv_b), Kc, _ptr(conv_state_in), _ptr(conv_state_out),
                                                        _ptr(u), _ptr(z), batch, seqlen, K, D, _stream(x2)),
                   "in_proj_conv_prefill")
    return u, z


def aligned16(*ts) -> bool:
    """Whether every tensor given (None skipped) starts on a 16-byte boundary,
    as the library's 16-byte loads of weights, biases and histories need."""
    return all(t is None or t.data_ptr() % 16 == 0 for t in ts)


def in_proj_conv_xproj_ok(x, W_in, conv_state, d_conv, J, b_in=None, conv_w=None, conv_b=None) -> bool:
    """Whether mtl_in_proj_conv_xproj takes this batched step: fp32 on the
    GPU, 1..32 rows, d_model a multiple of 128 (at least 256), d_conv 2..4,
    J <= 288, d_inner a multiple of 16, x, W_in, the conv history and the
    given b_in, conv_w and conv_b 16-byte aligned."""
    if x.dim() != 2 or W_in.dim() != 2 or x.dtype != torch.float32 or W_in.dtype != torch.float32:
        return False
    b, M = x.shape
    D = W_in.shape[0] // 2
    return (x.is_cuda and 1 <= b <= IN_CONV_MAX_ROWS and M >= 256 and M % 128 == 0 and W_in.shape == (2 * D, M)
            and D % 16 == 0 and 2 <= d_conv <= 4 and 1 <= J <= 288 and x.stride(1) == 1 and x.stride(0) % 4 == 0
            and W_in.is_contiguous() and x.data_ptr() % 16 == 0 and W_in.data_ptr() % 16 == 0
            and conv_state.dtype == torch.float32 and conv_state.is_contiguous()
            and tuple(conv_state.shape) == (b, D, d_conv - 1) and aligned16(conv_state, b_in, conv_w, conv_b))


def in_proj_conv_xproj(x, W_in, b_in, conv_state, conv_w, conv_b, W_xT, channels_per_part=None, sq=None, eps=0.0):
    """mtl_in_proj_conv_xproj: a batched step's in_proj (x [b, d_model] .
    W_in [2D, d_model]^T + b_in), the conv step + SiLU of its x half (conv
    history [b, D, K-1] updated in place) and the x_proj partials of each
    channel block, in one launch.  Returns (xc [b, D], z [b, D], xpart
    [D / channels_per_part, b, J]); ops.sum_parts(xpart) is x_dbl.
    With sq [tiles, b] (mtl_in_proj_conv_xproj_normed): x is h * w and sq
    the per-tile sums of h^2 that linear_skinny_residual left, and the
    in_proj input is RMSNorm(h) with this eps."""
    b, M = x.shape
    D = W_in.shape[0] // 2
    w = conv_w.reshape(conv_w.shape[0], conv_w.shape[-1]) if conv_w.dim() == 3 else conv_w
    K = w.shape[1]
    J = W_xT.shape[1]
    if not in_proj_conv_xproj_ok(x, W_in, conv_state, K, J, b_in, w, conv_b):
        raise ValueError("in_proj_conv_xproj: fp32 x [b<=32, d_model%128==0, >=256], contiguous W_in [2D, d_model] "
                         "(D%16==0), conv_state [b, D, K-1] with K in 2..4, J <= 288; x, W_in, b_in, conv_state, "
                         "conv_w and conv_b 16-byte aligned")
    _f32_mat(w, (D, K), "conv_w")
    _f32_vec(conv_b, D, "conv_b")
    _f32_vec(b_in, 2 * D, "b_in")
    _f32_mat(W_xT, (D, J), "W_xT")
    if channels_per_part is None:
        # 32-channel tiles where they still give every CU a workgroup (the
        # same rule as linear_skinny's rows_per_block)
        channels_per_part = 32 if b > 16 and D % 32 == 0 and 2 * D // 32 >= 256 else 16
    xc = torch.empty(b, D, device=x.device, dtype=torch.float32)
    z = torch.empty(b, D, device=x.device, dtype=torch.float32)
    xpart = torch.empty(D // channels_per_part, b, J, device=x.device, dtype=torch.float32)
    _same_device(x, W_in, b_in, conv_state, w, conv_b, W_xT, sq)
    lib = _lib.load()
    with _dev_guard(x):
        if sq is None:
            _lib.check(lib.mtl_in_proj_conv_xproj(_ptr(x), x.stride(0), _ptr(W_in), _ptr(b_in), _ptr(conv_state),
                                                  _ptr(w), _ptr(conv_b), K, _ptr(W_xT), J, _ptr(xc), _ptr(z),
                                                  z.stride(0), _ptr(xpart), b, M, D, channels_per_part,
                                                  _stream(x)), "in_proj_conv_xproj")
        else:
            _f32c(sq, "sq")
            if sq.dim() != 2 or sq.shape[1] != b:
                raise ValueError(f"in_proj_conv_xproj: sq must be [tiles, {b}], got {tuple(sq.shape)}")
            _lib.check(lib.mtl_in_proj_conv_xproj_normed(_ptr(x), x.stride(0), _ptr(W_in), _ptr(b_in),
                                                         _ptr(conv_state), _ptr(w), _ptr(conv_b), K, _ptr(W_xT), J,
                                                         _ptr(xc), _ptr(z), z.stride(0), _ptr(xpart), b, M, D,
                                                         channels_per_part, _ptr(sq), sq.shape[0], float(eps),
                                                         _stream(x)), "in_proj_conv_xproj_normed")
    return xc, z, xpart


# --------------------------------------------------------------------------- step
def selective_state_update(ssm_state, x, z, x_dbl, W_dt, b_dt, A, D=None, a_is_log=False, out=None):
    """In-place single-token SSM update (mtl_selective_state_update).
    ssm_state: fp32 [b,D,N] contiguous; x, z: [b,D]; x_dbl: [b, R+2N] holding
    [dt_low | B | C]; W_dt: [D,R]; b_dt: [D]; A or A_log: [D,N].  Returns y [b,D]."""
    b, Dm = x.shape
    N = A.shape[1]
    R = W_dt.shape[1]
    _f32_mat(ssm_state, (b, Dm, N), "ssm_state")
    _f32_mat(W_dt, (Dm, R), "W_dt")
    _f32_mat(A, (Dm, N), "A")
    _f32_vec(b_dt, Dm, "b_dt")
    _f32_vec(D, Dm, "D")
    if N > STEP_MAX_D_STATE or R > STEP_MAX_DT_RANK:
        raise ValueError(f"selective_state_update supports d_state <= {STEP_MAX_D_STATE} and dt_rank <= "
                         f"{STEP_MAX_DT_RANK}")
    if tuple(x_dbl.shape) != (b, R + 2 * N) or x_dbl.stride(1) != 1:
        raise ValueError(f"x_dbl must be {(b, R + 2 * N)} with unit column stride, got {tuple(x_dbl.shape)}")
    for name, t in (("x", x), ("z", z)):
        if t is not None and (tuple(t.shape) != (b, Dm) or t.stride(1) != 1):
            raise ValueError(f"{name} must be {(b, Dm)} with channel stride 1")
    if out is None:
        out = torch.empty(b, Dm, device=x.device, dtype=x.dtype)
    elif tuple(out.shape) != (b, Dm) or out.stride(1) != 1:
        raise ValueError(f"out must be {(b, Dm)} with channel stride 1")
    code = _act_code(x, z, x_dbl, out)
    _same_device(x, ssm_state, z, x_dbl, W_dt, b_dt, A, D, out)
    with _dev_guard(x):
        _lib.check(_lib.load().mtl_selective_state_update(
            _ptr(ssm_state), _ptr(x), x.stride(0), _ptr(z), z.stride(0) if z is not None else 0,
            _ptr(x_dbl), x_dbl.stride(0), _ptr(W_dt), _ptr(b_dt), _ptr(A), _ptr(D), _ptr(out), out.stride(0),
            b, Dm, N, R, code, int(bool(a_is_log)), _stream(x)), "selective_state_update")
    return out


# --------------------------------------------------------------------------- norm
def add_rmsnorm(x, weight, eps, y=None, x_out=None, out=None, y_parts=None):
    """normed = weight * rmsnorm(x + y) (fp32, rows = all leading dims);
    x_out (may alias x) receives x + y.  y_parts [P, *x.shape] instead of y:
    y = the sum of the P parts in order (split-K partial products)."""
    if y_parts is not None:
        if y is not None:
            raise ValueError("give y or y_parts, not both")
        if (y_parts.dtype != torch.float32 or not y_parts.is_contiguous() or y_parts.dim() != x.dim() + 1
                or tuple(y_parts.shape[1:]) != tuple(x.shape)):
            raise ValueError(f"y_parts must be contiguous float32 [P, {', '.join(map(str, x.shape))}]")
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("x must be contiguous float32")
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    _f32_vec(weight, cols, "weight")
    for name, t in (("y", y), ("x_out", x_out)):
        if t is not None and (t.shape != x.shape or t.dtype != torch.float32 or not t.is_contiguous()):
            raise ValueError(f"{name} must be contiguous float32 {tuple(x.shape)}")
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be contiguous float32 like x")
    _same_device(x, weight, y, x_out, out, y_parts)
    with _dev_guard(x):
        if y_parts is not None:
            _lib.check(_lib.load().mtl_add_rmsnorm_parts(_ptr(x), _ptr(y_parts), y_parts.shape[0], _ptr(x_out),
                                                         _ptr(weight), _ptr(out), rows, cols, float(eps), _stream(x)),
                       "add_rmsnorm")
        else:
            _lib.check(_lib.load().mtl_add_rmsnorm(_ptr(x), _ptr(y), _ptr(x_out), _ptr(weight), _ptr(out), rows, cols,
                                                   float(eps), _stream(x)), "add_rmsnorm")
    return out


# --------------------------------------------------------------------------- payload quantizers
def sum_parts(parts, out=None):
    """mtl_sum_parts: parts [P, ...] fp32 contiguous -> out [...] =
    parts[0] + parts[1] + ... in part order."""
    _f32c(parts, "parts")
    if parts.dim() < 2:
        raise ValueError("parts must be [P, ...]")
    if out is None:
        out = torch.empty(parts.shape[1:], device=parts.device, dtype=torch.float32)
    _f32c(out, "out")
    if tuple(out.shape) != tuple(parts.shape[1:]):
        raise ValueError("out must have the shape of one part")
    with _dev_guard(parts):
        _lib.check(_lib.load().mtl_sum_parts(_ptr(parts), parts.shape[0], out.numel(), _ptr(out), _stream(parts)),
                   "sum_parts")
    return out


XPROJ_SUM_DT_MAX_R = 160


def xproj_sum_dt(parts, W_dt, x_dbl=None, write_x_dbl=True):
    """mtl_xproj_sum_dt: parts [P, rows, J] (x_proj split over K) ->
    (x_dbl [rows, J] = the parts summed in order, dt [rows, D] = x_dbl[:, :R]
    . W_dt^T), one launch.  With P = 1 and write_x_dbl False, x_dbl is
    parts[0] itself."""
    _f32c(parts, "parts")
    _f32c(W_dt, "W_dt")
    if parts.dim() != 3 or W_dt.dim() != 2:
        raise ValueError("xproj_sum_dt: parts [P, rows, J] and W_dt [D, R] expected")
    P, rows, J = parts.shape
    D, R = W_dt.shape
    if not 1 <= R <= min(J, XPROJ_SUM_DT_MAX_R):
        raise ValueError(f"xproj_sum_dt: dt_rank must be in [1, min(J, {XPROJ_SUM_DT_MAX_R})]")
    if not write_x_dbl and P != 1:
        raise ValueError("xproj_sum_dt: x_dbl is written unless there is one part")
    if write_x_dbl:
        if x_dbl is None:
            x_dbl = torch.empty(rows, J, device=parts.device, dtype=torch.float32)
        _f32c(x_dbl, "x_dbl")
        if tuple(x_dbl.shape) != (rows, J):
            raise ValueError(f"xproj_sum_dt: x_dbl must be {(rows, J)}")
    dt = torch.empty(rows, D, device=parts.device, dtype=torch.float32)
    _same_device(parts, W_dt, x_dbl)
    with _dev_guard(parts):
        _lib.check(_lib.load().mtl_xproj_sum_dt(_ptr(parts), P, rows, J, _ptr(W_dt), R, D,
                                                _ptr(x_dbl) if write_x_dbl else None, _ptr(dt), _stream(parts)),
                   "xproj_sum_dt")
    return (x_dbl if write_x_dbl else parts[0]), dt


def prefill_short_ok(rows, d_model, d_inner, d_state, dt_rank, d_conv) -> bool:
    """Whether mtl_prefill_short takes a prompt of `rows` = b l tokens of this
    layer shape."""
    return (1 <= rows <= SKINNY_MAX_ROWS and d_model >= 256 and d_model % 128 == 0 and d_inner >= 512
            and d_inner % 512 == 0 and 1 <= d_state <= 16 and 1 <= dt_rank <= XPROJ_SUM_DT_MAX_R
            and (dt_rank + 2 * d_state) % 4 == 0 and 2 <= d_conv <= 4)


def prefill_short(h, layers, norm_f, eps_f, d_inner, d_state, dt_rank, d_conv):
    """mtl_prefill_short: a short prompt's whole layer stack in one call.
    h [b, l, d_model] float32 holds the embedded tokens and is overwritten
    with the final residual stream; `layers` is a ctypes array of
    _lib.PrefillLayer (weights plus this call's cache pointers).  Returns
    norm_f(h) [b, l, d_model]."""
    _f32c(h, "h")
    _f32c(norm_f, "norm_f")
    b, l, M = h.shape
    rows, J = b * l, dt_rank + 2 * d_state
    if not prefill_short_ok(rows, M, d_inner, d_state, dt_rank, d_conv):
        raise ValueError("prefill_short: sizes outside mtl_prefill_short")
    if norm_f.numel() != M or norm_f.device != h.device:
        raise ValueError(f"prefill_short: norm_f must hold {M} floats on {h.device}")
    # one workspace, every buffer on a 256-byte boundary
    sizes = [rows * M, rows * d_inner, rows * d_inner, rows * d_inner, rows * d_inner, 16 * rows * J, rows * J,
             4 * rows * M]
    offs, n = [], 0
    for s in sizes:
        offs.append(n)
        n += -(-s // 64) * 64
    ws = torch.empty(n + rows * M, device=h.device, dtype=torch.float32)
    normed = ws[n:].view(b, l, M)
    base = ws.data_ptr()
    a = _lib.PrefillShortArgs()
    a.h = h.data_ptr()
    a.xn, a.u, a.z, a.dt, a.y, a.x_parts, a.x_dbl, a.y_parts = [base + 4 * o for o in offs]
    a.norm_f, a.normed_out, a.eps_f = norm_f.data_ptr(), normed.data_ptr(), float(eps_f)
    a.d_conv, a.n_layers = d_conv, len(layers)
    a.batch, a.seqlen, a.d_model, a.d_inner, a.d_state, a.dt_rank = b, l, M, d_inner, d_state, dt_rank
    with _dev_guard(h):
        _lib.check(_lib.load().mtl_prefill_short(ctypes.byref(a), layers, _stream(h)), "prefill_short")
    return normed


STEP_MAX_D_STATE = 16     # one state per lane of a 16-lane row in every step kernel
STEP_MAX_DT_RANK = 256    # dt_proj columns a step lane holds: 16 lanes x 16 registers


def check_step_shape(d_state, dt_rank) -> None:
    """ValueError for a model whose single-token step the step kernels do not
    take (more than STEP_MAX_D_STATE states or STEP_MAX_DT_RANK dt_proj
    columns), raised by the step entry points before anything is launched,
    so no cache is left half stepped."""
    if d_state > STEP_MAX_D_STATE or dt_rank > STEP_MAX_DT_RANK:
        raise ValueError(f"step: d_state {d_state}, dt_rank {dt_rank}; the step kernels take d_state <= "
                         f"{STEP_MAX_D_STATE} and dt_rank <= {STEP_MAX_DT_RANK}")


PREFILL_LONG_BLAS_WS = 32 << 20     # bytes of hipBLASLt workspace per mtl_prefill_long call


def prefill_long_ok(b, l, d_model, d_inner, d_state, dt_rank, d_conv) -> bool:
    """Whether mtl_prefill_long takes a prompt of b x l tokens of this layer
    shape (its size checks): b l <= 2^20, b <= 65535, l <= 1048560, d_model
    and d_inner in [1, 65536], d_state in [1, 32], dt_rank in [1, d_inner],
    d_conv in [1, 8]."""
    return (b >= 1 and l >= 1 and b * l <= 1 << 20 and b <= 65535 and l <= 65535 * 16
            and 1 <= d_model <= 1 << 16 and 1 <= d_inner <= 1 << 16 and 1 <= d_state <= 32
            and 1 <= dt_rank <= d_inner and 1 <= d_conv <= 8)


def prefill_long(h, layers, norm_f, eps_f, d_inner, d_state, dt_rank, d_conv, skinny_rows=0):
    """mtl_prefill_long: a prompt's whole layer stack in one call (any
    length, the projections on hipBLASLt; up to skinny_rows token rows on
    the library's skinny GEMM where the shapes fit it).  h [b, l, d_model]
    float32 holds the embedded tokens and is overwritten with the final
    residual stream; `layers` is a ctypes array of _lib.PrefillLayer
    (weights plus this call's cache pointers).  Returns norm_f(h)
    [b, l, d_model]."""
    _f32c(h, "h")
    _f32c(norm_f, "norm_f")
    b, l, M = h.shape
    rows, J = b * l, dt_rank + 2 * d_state
    if norm_f.numel() != M or norm_f.device != h.device:
        raise ValueError(f"prefill_long: norm_f must hold {M} floats on {h.device}")
    # one workspace, every buffer on a 256-byte boundary
    sizes = [rows * M, rows * 2 * d_inner, rows * d_inner, rows * J, rows * d_inner, rows * d_inner, rows * M,
             PREFILL_LONG_BLAS_WS // 4]
    offs, n = [], 0
    for sz in sizes:
        offs.append(n)
        n += -(-sz // 64) * 64
    ws = torch.empty(n + rows * M, device=h.device, dtype=torch.float32)
    normed = ws[n:].view(b, l, M)
    base = ws.data_ptr()
    a = _lib.PrefillLongArgs()
    a.h = h.data_ptr()
    a.xn, a.xz, a.u, a.x_dbl, a.dt, a.y, a.out, a.blas_ws = [base + 4 * o for o in offs]
    a.blas_ws_bytes = PREFILL_LONG_BLAS_WS
    a.norm_f, a.normed_out, a.eps_f = norm_f.data_ptr(), normed.data_ptr(), float(eps_f)
    a.d_conv, a.n_layers, a.skinny_rows = d_conv, len(layers), int(skinny_rows)
    a.batch, a.seqlen, a.d_model, a.d_inner, a.d_state, a.dt_rank = b, l, M, d_inner, d_state, dt_rank
    with _dev_guard(h):
        _lib.check(_lib.load().mtl_prefill_long(ctypes.byref(a), layers, _stream(h)), "prefill_long")
    return normed


def decode_step(layers, ids, emb, norm_f, eps_f, logits, xc, gz, y, xs, xpart, cfg, channels_per_block, split_k,
                xproj_parts):
    """mtl_decode_step: one fused decode step of every layer in one call.
    `layers` is a ctypes array of _lib.DecodeLayer (weights and this call's
    cache pointers); ids [b] int64; logits [b, vocab] receives norm_f + the
    tied lm_head; xc, gz, y [b, d_inner], xs three [b, d_model] and xpart
    [parts, b, J] are the workspace, all float32 contiguous on one device."""
    for t, name in ((emb, "emb"), (norm_f, "norm_f"), (logits, "logits"), (xc, "xc"), (gz, "gz"), (y, "y"),
                    (xpart, "xpart"), *((x, "xs") for x in xs)):
        _f32c(t, name)
    if ids.dtype != torch.int64 or not ids.is_contiguous():
        raise ValueError("decode_step: ids must be contiguous int64")
    b, D = xc.shape
    J = cfg.dt_rank + 2 * cfg.d_state
    if ids.numel() != b or tuple(logits.shape) != (b, emb.shape[0]) or xpart.shape[1:] != (b, J):
        raise ValueError("decode_step: ids [b], logits [b, vocab], xpart [parts, b, J] expected")
    a = _lib.DecodeStepArgs()
    a.ids, a.emb, a.norm_f, a.logits = ids.data_ptr(), emb.data_ptr(), norm_f.data_ptr(), logits.data_ptr()
    a.xc, a.gz, a.y, a.xpart = xc.data_ptr(), gz.data_ptr(), y.data_ptr(), xpart.data_ptr()
    a.x0, a.x1, a.resid = xs[0].data_ptr(), xs[1].data_ptr(), xs[2].data_ptr()
    a.eps_f, a.vocab, a.n_layers, a.batch = float(eps_f), emb.shape[0], len(layers), b
    a.d_model, a.d_inner, a.d_state, a.dt_rank, a.d_conv = emb.shape[1], D, cfg.d_state, cfg.dt_rank, cfg.d_conv
    a.channels_per_block, a.split_k, a.xproj_parts = channels_per_block, int(split_k), xproj_parts
    with _dev_guard(xc):
        _lib.check(_lib.load().mtl_decode_step(ctypes.byref(a), layers, _stream(xc)), "decode_step")
    return logits


def decode_step_batched(layers, h, norm_f, eps_f, cfg, fold):
    """mtl_decode_step_batched: a batched step of every layer in one call.
    `layers` is a ctypes array of _lib.DecodeLayer (weights with W_xT, and
    this call's cache pointers); h [b, d_model] float32 holds the step's
    embedding rows and is left holding the final residual stream.  Returns
    norm_f of it [b, d_model], the tied lm_head's input.  The workspace is
    allocated here (one float32 tensor, and with fold the zeroed counters)."""
    _f32c(h, "h")
    _f32c(norm_f, "norm_f")
    if h.dim() != 2 or h.data_ptr() % 16 or h.shape[1] != cfg.d_model:
        raise ValueError(f"decode_step_batched: h must be a 16-byte aligned [b, {cfg.d_model}] tensor")
    b, M = h.shape
    if norm_f.numel() != M or norm_f.device != h.device:
        raise ValueError(f"decode_step_batched: norm_f must hold {M} floats on {h.device}")
    D, J = cfg.d_inner, cfg.dt_rank + 2 * cfg.d_state
    nl = len(layers)
    pad = lambda n: -(-n // 64) * 64                      # 256-byte aligned slices
    sizes = {"normed_out": b * M, "inp": b * M, "xn": b * M, "xc": b * D, "z": b * D, "y": b * D,
             "xpart": (D // 16) * b * J, "x_dbl": b * J, "parts": 4 * b * M, "sq": (M // 16) * b}
    ws = torch.empty(sum(pad(n) for n in sizes.values()), device=h.device, dtype=torch.float32)
    a = _lib.DecodeStepBatchedArgs()
    off = 0
    for name, n in sizes.items():
        setattr(a, name, ws.data_ptr() + 4 * off)
        off += pad(n)
    counters = torch.zeros(max(nl - 1, 1), M // 16, device=h.device, dtype=torch.int32) if fold else None
    a.h, a.norm_f = h.data_ptr(), norm_f.data_ptr()
    a.counters = counters.data_ptr() if fold else None
    a.eps_f, a.n_layers, a.batch = float(eps_f), nl, b
    a.d_model, a.d_inner, a.d_state, a.dt_rank, a.d_conv = M, D, cfg.d_state, cfg.dt_rank, cfg.d_conv
    a.fold = int(bool(fold))
    with _dev_guard(h):
        _lib.check(_lib.load().mtl_decode_step_batched(ctypes.byref(a), layers, _stream(h)), "decode_step_batched")
    return ws[:b * M].view(b, M)


def decode_persist_workspace(cfg, device) -> torch.Tensor:
    """A zero-filled workspace for mtl_decode_step_persist (its exchange slots,
    epoch and error word), to be kept and reused by every call on `device`."""
    n = _lib.load().mtl_decode_persist_workspace_bytes(cfg.d_model, cfg.d_inner, cfg.d_state, cfg.dt_rank)
    return torch.zeros(n, dtype=torch.uint8, device=device)


def decode_persist_error(workspace) -> int:
    """The error word of a persistent-step workspace (synchronizes with the
    device): 0, or the code of a launch whose wait timed out.  After a
    nonzero word, reset_decode_persist_workspace() before the next call."""
    if workspace.dtype != torch.uint8 or workspace.numel() < 8:
        raise ValueError("decode_persist_error: not a persistent-step workspace")
    return int(workspace[4:8].view(torch.int32).item()) & 0xFFFFFFFF


def reset_decode_persist_workspace(workspace) -> None:
    """Zero-fill a persistent-step workspace (epoch, error word and slots), as
    after a call whose error word was nonzero.  Stream-ordered, no sync."""
    workspace.zero_()


def decode_step_persist(layers, layers_dev, ids, emb, norm_f, eps_f, logits, x0, workspace, cfg, blocking=0):
    """mtl_decode_step_persist: the batch-1 decode step of every layer as one
    persistent launch, then norm_f + the tied lm_head into logits [1, vocab].
    `layers` is the host ctypes array of _lib.DecodeLayer (weights with W_xT,
    and this call's cache pointers), `layers_dev` a uint8 device tensor
    holding a copy of its weight records; x0 [1, d_model] receives the final
    residual; workspace from decode_persist_workspace()."""
    for t, name in ((emb, "emb"), (norm_f, "norm_f"), (logits, "logits"), (x0, "x0")):
        _f32c(t, name)
    if ids.dtype != torch.int64 or not ids.is_contiguous() or ids.numel() != 1:
        raise ValueError("decode_step_persist: ids must be one contiguous int64 id")
    if tuple(logits.shape) != (1, emb.shape[0]) or tuple(x0.shape) != (1, emb.shape[1]):
        raise ValueError("decode_step_persist: logits [1, vocab] and x0 [1, d_model] expected")
    if layers_dev.dtype != torch.uint8 or layers_dev.numel() != ctypes.sizeof(layers) or not layers_dev.is_contiguous():
        raise ValueError("decode_step_persist: layers_dev must hold the layer records as contiguous uint8")
    if workspace.dtype != torch.uint8 or not workspace.is_contiguous():
        raise ValueError("decode_step_persist: workspace must be contiguous uint8")
    _same_device(x0, ids, emb, norm_f, logits, layers_dev, workspace)
    a = _lib.DecodeStepArgs()
    a.ids, a.emb, a.norm_f, a.logits, a.x0 = ids.data_ptr(), emb.data_ptr(), norm_f.data_ptr(), logits.data_ptr(), \
        x0.data_ptr()
    a.eps_f, a.vocab, a.n_layers, a.batch = float(eps_f), emb.shape[0], len(layers), 1
    a.d_model, a.d_inner, a.d_state, a.dt_rank, a.d_conv = emb.shape[1], cfg.d_inner, cfg.d_state, cfg.dt_rank, \
        cfg.d_conv
    with _dev_guard(x0):
        _lib.check(_lib.load().mtl_decode_step_persist(ctypes.byref(a), layers, layers_dev.data_ptr(),
                                                       workspace.data_ptr(), workspace.numel(), int(blocking),
                                                       _stream(x0)), "decode_step_persist")
    return logits


def _parts_array(parts):
    arr = (ctypes.c_void_p * len(parts))(*[p.data_ptr() for p in parts])
    return ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p)), arr


def quant_dequant_sum_int8_tok(parts, payloads=None, out=None, return_payloads=True):
    """Per-token int8 quantize -> dequantize-sum of `parts` (rank order),
    mtl_quant_dequant_sum_int8_tok.  parts: list of same-shape float32
    tensors (rows = leading dims, cols = last dim).  Returns (out, payloads)
    with payload r = [scales (4*rows bytes) || int8 codes] as uint8."""
    if not 1 <= len(parts) <= 8:
        raise ValueError("between 1 and 8 parts")
    p0 = parts[0]
    for p in parts:
        if p.shape != p0.shape or p.dtype != torch.float32 or not p.is_contiguous():
            raise ValueError("parts must be contiguous float32 tensors of one shape")
    cols = p0.shape[-1] if p0.dim() else 1
    rows = p0.numel() // cols if cols else 0
    if out is None:
        out = torch.empty_like(p0)
    elif out.shape != p0.shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be contiguous float32 like the parts")
    nbytes = rows * (cols + 4)
    if payloads is None and return_payloads:
        payloads = [torch.empty(nbytes, dtype=torch.uint8, device=p0.device) for _ in parts]
    if payloads is not None:
        if len(payloads) != len(parts) or any(q.dtype != torch.uint8 or q.numel() != nbytes or not q.is_contiguous()
                                              for q in payloads):
            raise ValueError(f"payloads must be {len(parts)} contiguous uint8 tensors of {nbytes} bytes")
    _same_device(p0, *parts, out, *(payloads or []))
    parr, keep1 = _parts_array(parts)
    qarr, keep2 = _parts_array(payloads) if payloads is not None else (None, None)
    with _dev_guard(p0):
        _lib.check(_lib.load().mtl_quant_dequant_sum_int8_tok(parr, len(parts), rows, cols, qarr, _ptr(out),
                                                              _stream(p0)), "quant_dequant_sum_int8_tok")
    return out, payloads


def quant_dequant_sum_fp16(parts, payloads=None, out=None, return_payloads=False):
    """fp16 cast -> sum (rank order) -> fp32 of `parts`
    (mtl_quant_dequant_sum_fp16).  Returns (out, payloads or None)."""
    if not 1 <= len(parts) <= 8:
        raise ValueError("between 1 and 8 parts")
    p0 = parts[0]
    for p in parts:
        if p.shape != p0.shape or p.dtype != torch.float32 or not p.is_contiguous():
            raise ValueError("parts must be contiguous float32 tensors of one shape")
    if out is None:
        out = torch.empty_like(p0)
    elif out.shape != p0.shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError("out must be contiguous float32 like the parts")
    if payloads is None and return_payloads:
        payloads = [torch.empty(p0.shape, dtype=torch.float16, device=p0.device) for _ in parts]
    if payloads is not None:
        if len(payloads) != len(parts) or any(q.dtype != torch.float16 or q.shape != p0.shape or not q.is_contiguous()
                                              for q in payloads):
            raise ValueError("payloads must be contiguous float16 tensors shaped like the parts")
    _same_device(p0, *parts, out, *(payloads or []))
    parr, keep1 = _parts_array(parts)
    qarr, keep2 = _parts_array(payloads) if payloads is not None else (None, None)
    with _dev_guard(p0):
        _lib.check(_lib.load().mtl_quant_dequant_sum_fp16(parr, len(parts), p0.numel(), qarr, _ptr(out),
                                                          _stream(p0)), "quant_dequant_sum_fp16")
    return out, payloads


# --------------------------------------------------------------------------- fused decode step
def _f32c(t, name):
    if t is None:
        return None
    if t.dtype != torch.float32 or not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous float32")
    return t


def decode_in(norm_w, eps, W_in, conv_state, conv_w, xc, gz, *, x=None, emb=None, ids=None, resid_out=None,
              b_in=None, conv_b=None, W_xT=None, xpart=None, channels_per_block=8):
    """mtl_decode_in: RMSNorm -> in_proj rows -> conv step (conv_state in
    place) -> xc = SiLU(conv), gz = SiLU(z), and optionally the x_proj split-K
    partials into xpart [nblk, b, J], nblk = ceil(D / channels_per_block)
    (8 or 4 channels per workgroup).  x [b, M] or (emb [V, M], ids [b])."""
    b, D = xc.shape
    M = norm_w.shape[0]
    K = conv_w.shape[1]
    for name, t in (("norm_w", norm_w), ("W_in", W_in), ("conv_state", conv_state), ("conv_w", conv_w),
                    ("xc", xc), ("gz", gz), ("x", x), ("emb", emb), ("resid_out", resid_out), ("b_in", b_in),
                    ("conv_b", conv_b), ("W_xT", W_xT), ("xpart", xpart)):
        _f32c(t, name)
    if tuple(W_in.shape) != (2 * D, M) or tuple(conv_state.shape) != (b, D, K - 1) or tuple(gz.shape) != (b, D):
        raise ValueError("decode_in: W_in [2D, M], conv_state [b, D, K-1], xc/gz [b, D] expected")
    if x is not None and tuple(x.shape) != (b, M):
        raise ValueError(f"x must be {(b, M)}")
    if ids is not None and (ids.dtype != torch.int64 or ids.numel() != b or not ids.is_contiguous()):
        raise ValueError("ids must be contiguous int64 with b entries")
    J = W_xT.shape[1] if W_xT is not None else 1
    if W_xT is not None:
        nblk = (D + channels_per_block - 1) // channels_per_block
        if tuple(W_xT.shape) != (D, J) or xpart is None or tuple(xpart.shape) != (nblk, b, J):
            raise ValueError("decode_in: W_xT [D, J] and xpart [nblk, b, J] expected")
    with _dev_guard(xc):
        _lib.check(_lib.load().mtl_decode_in(_ptr(x), _ptr(emb), _ptr(ids), emb.shape[0] if emb is not None else 0,
                                             _ptr(resid_out), _ptr(norm_w), float(eps),
                                             _ptr(W_in), _ptr(b_in), _ptr(conv_state), _ptr(conv_w), _ptr(conv_b),
                                             _ptr(W_xT), _ptr(xc), _ptr(gz), _ptr(xpart), b, M, D, K, J,
                                             channels_per_block, _stream(xc)), "decode_in")


def decode_gemv(v, W, out, bias=None, x_in=None):
    """mtl_decode_gemv: out [b, rows] = W [rows, cols] . v [b, cols] (+ bias)
    (+ x_in)."""
    for name, t in (("v", v), ("W", W), ("out", out), ("bias", bias), ("x_in", x_in)):
        _f32c(t, name)
    b, cols = v.shape
    rows = W.shape[0]
    if W.shape[1] != cols or tuple(out.shape) != (b, rows):
        raise ValueError("decode_gemv: W [rows, cols], v [b, cols], out [b, rows] expected")
    with _dev_guard(v):
        _lib.check(_lib.load().mtl_decode_gemv(_ptr(v), _ptr(W), _ptr(bias), _ptr(x_in), _ptr(out), b, rows, cols,
                                               _stream(v)), "decode_gemv")
    return out


SKINNY_MAX_ROWS = 64     # mtl_linear_skinny: rows of x per launch chunk
SKINNY_CHUNKED_MAX_ROWS = 64 * 65535   # rows of x over all chunks
IN_CONV_MAX_ROWS = 32    # mtl_in_proj_conv_xproj: batch rows


def linear_skinny_ok(x, W, max_rows=SKINNY_MAX_ROWS, bias=None) -> bool:
    """Whether mtl_linear_skinny takes y = x W^T (+ bias) for these operands
    in one chunk (or, with max_rows, in 64-row chunks): fp32 on the GPU,
    1..64 rows of x, K a multiple of 128, W rows a multiple of 4, 16-byte
    aligned rows and bias."""
    if x.dim() != 2 or W.dim() != 2 or x.dtype != torch.float32 or W.dtype != torch.float32:
        return False
    M, K = x.shape
    N = W.shape[0]
    return (x.is_cuda and W.is_cuda and 1 <= M <= max_rows and W.shape[1] == K and K % 128 == 0
            and N % 4 == 0 and x.stride(1) == 1 and x.stride(0) % 4 == 0 and W.is_contiguous()
            and x.data_ptr() % 16 == 0 and W.data_ptr() % 16 == 0 and aligned16(bias))


def linear_skinny(x, W, bias=None, out=None, ksplit=1, rows_per_block=None):
    """mtl_linear_skinny: out [M, N] = x [M, K] . W [N, K]^T (+ bias) on the
    matrix cores, for M <= 64 (the projections of a batched decode step,
    and of a prefill of at most 64 tokens), larger M in 64-row chunks.
    With ksplit > 1, out is [ksplit, M, N]: the partial products over K
    split into ksplit equal ranges (bias in part 0), to be added in order."""
    if not linear_skinny_ok(x, W, SKINNY_CHUNKED_MAX_ROWS, bias):
        raise ValueError("linear_skinny: fp32 x [M, K%128==0] (unit column stride, 16B rows), contiguous "
                         "W [N%4==0, K] and a 16-byte aligned bias expected")
    M, K = x.shape
    N = W.shape[0]
    if bias is not None:
        _f32_vec(bias, N, "bias")
    if K % (128 * ksplit):
        raise ValueError("linear_skinny: K must be a multiple of 128 * ksplit")
    shape = (M, N) if ksplit == 1 else (ksplit, M, N)
    if out is None:
        out = torch.empty(shape, device=x.device, dtype=torch.float32)
    elif tuple(out.shape) != shape or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"linear_skinny: out must be contiguous float32 {shape}")
    if rows_per_block is None:
        # 32-row tiles halve the re-reads of x where they still give every CU
        # a workgroup; at 16 rows or fewer of x the 16-row tiles stream faster
        # (past 32 rows of x, 32-row tiles need 96 KB of LDS: one workgroup per CU)
        rows_per_block = 32 if 16 < M <= 32 and (N + 31) // 32 * ksplit >= 256 else 16
    _same_device(x, W, bias, out)
    with _dev_guard(x):
        _lib.check(_lib.load().mtl_linear_skinny(_ptr(x), x.stride(0), _ptr(W), _ptr(bias), _ptr(out), N, M * N,
                                                 M, N, K, ksplit, rows_per_block, _stream(x)), "linear_skinny")
    return out


def residual_rows_per_block(M, N, ksplit) -> int:
    """linear_skinny's tile choice for out_proj with ksplit parts."""
    return 32 if 16 < M <= 32 and N % 32 == 0 and N // 32 * ksplit >= 256 else 16


def linear_skinny_residual(y, W, bias, h, w_next, x_next, sq, counters, ksplit, rows_per_block=None, parts=None):
    """mtl_linear_skinny_residual: out_proj of a batched step (y [M, K] .
    W [N, K]^T + bias, as ksplit partial products) with the residual add h
    += the parts in order (in place) and the next block's norm inputs:
    x_next = h * w_next, sq [N / rows_per_block, M] = per-tile sums of h^2.
    counters [N / rows_per_block] int32 must be zero (each call its own)."""
    if not linear_skinny_ok(y, W):
        raise ValueError("linear_skinny_residual: fp32 y [M<=32, K%128==0] and contiguous W [N, K] expected")
    M, K = y.shape
    N = W.shape[0]
    if M > 32:
        raise ValueError("linear_skinny_residual: at most 32 rows")
    if rows_per_block is None:
        rows_per_block = residual_rows_per_block(M, N, ksplit)
    tiles = N // rows_per_block
    for name, t, shape in (("h", h, (M, N)), ("x_next", x_next, (M, N)), ("sq", sq, (tiles, M))):
        _f32c(t, name)
        if tuple(t.shape) != shape:
            raise ValueError(f"linear_skinny_residual: {name} must be {shape}, got {tuple(t.shape)}")
    _f32_vec(w_next, N, "w_next")
    if bias is not None:
        _f32_vec(bias, N, "bias")
    if counters.dtype != torch.int32 or not counters.is_contiguous() or counters.numel() != tiles:
        raise ValueError(f"linear_skinny_residual: counters must be contiguous int32 [{tiles}]")
    if parts is None:
        parts = torch.empty(ksplit, M, N, device=y.device, dtype=torch.float32)
    elif tuple(parts.shape) != (ksplit, M, N) or parts.dtype != torch.float32 or not parts.is_contiguous():
        raise ValueError(f"linear_skinny_residual: parts must be contiguous float32 {(ksplit, M, N)}")
    _same_device(y, W, bias, h, w_next, x_next, sq, counters, parts)
    with _dev_guard(y):
        _lib.check(_lib.load().mtl_linear_skinny_residual(_ptr(y), y.stride(0), _ptr(W), _ptr(bias), _ptr(parts), M,
                                                          N, K, ksplit, rows_per_block, _ptr(h), _ptr(w_next),
                                                          _ptr(x_next), _ptr(sq), _ptr(counters), _stream(y)),
                   "linear_skinny_residual")
    return h, x_next, sq


def decode_gemv_parts(v, W, out_parts):
    """mtl_decode_gemv_parts: out_parts [P, b, rows], part p = W[:, p-th of P
    column ranges] . v[:, same range] (summed in order by decode_ssm)."""
    for name, t in (("v", v), ("W", W), ("out_parts", out_parts)):
        _f32c(t, name)
    b, cols = v.shape
    rows = W.shape[0]
    P = out_parts.shape[0]
    if W.shape[1] != cols or tuple(out_parts.shape) != (P, b, rows):
        raise ValueError("decode_gemv_parts: W [rows, cols], v [b, cols], out_parts [P, b, rows] expected")
    with _dev_guard(v):
        _lib.check(_lib.load().mtl_decode_gemv_parts(_ptr(v), _ptr(W), _ptr(out_parts), b, rows, cols, P, _stream(v)),
                   "decode_gemv_parts")
    return out_parts


def decode_norm_gemv(v, norm_w, eps, W, out, bias=None):
    """mtl_decode_norm_gemv: out [b, rows] = W [rows, cols] . RMSNorm(v) (+ bias),
    RMSNorm(v) = norm_w * v * rsqrt(mean(v^2) + eps) -- the final norm and
    lm_head of a decode step in one launch."""
    for name, t in (("v", v), ("norm_w", norm_w), ("W", W), ("out", out), ("bias", bias)):
        _f32c(t, name)
    b, cols = v.shape
    rows = W.shape[0]
    if W.shape[1] != cols or tuple(out.shape) != (b, rows) or tuple(norm_w.shape) != (cols,):
        raise ValueError("decode_norm_gemv: W [rows, cols], v [b, cols], norm_w [cols], out [b, rows] expected")
    with _dev_guard(v):
        _lib.check(_lib.load().mtl_decode_norm_gemv(_ptr(v), _ptr(norm_w), float(eps), _ptr(W), _ptr(bias), _ptr(out),
                                                    b, rows, cols, _stream(v)), "decode_norm_gemv")
    return out


def decode_ssm(xpart, xc, gz, W_dt, b_dt, A_log, Dv, ssm_state, y):
    """mtl_decode_ssm: reduce x_proj partials [nblk, b, J] -> dt_proj +
    softplus -> ssm_state update in place -> y = (C.h + D x) * gz."""
    for name, t in (("xpart", xpart), ("xc", xc), ("gz", gz), ("W_dt", W_dt), ("b_dt", b_dt), ("A_log", A_log),
                    ("Dv", Dv), ("ssm_state", ssm_state), ("y", y)):
        _f32c(t, name)
    b, D = xc.shape
    N = A_log.shape[1]
    R = W_dt.shape[1]
    if xpart.dim() != 3 or xpart.shape[1:] != (b, R + 2 * N) or tuple(ssm_state.shape) != (b, D, N):
        raise ValueError("decode_ssm: xpart [nblk, b, R+2N], ssm_state [b, D, N] expected")
    with _dev_guard(xc):
        _lib.check(_lib.load().mtl_decode_ssm(_ptr(xpart), xpart.shape[0], _ptr(xc), _ptr(gz), _ptr(W_dt),
                                              _ptr(b_dt), _ptr(A_log), _ptr(Dv), _ptr(ssm_state), _ptr(y), b, D, N,
                                              R, _stream(xc)), "decode_ssm")
    return y
