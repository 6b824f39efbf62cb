"""mtl_in_proj_conv_xproj (a batched step's in_proj, conv step and x_proj
partials in one launch, model.py:261-279) against a float64 reference of the
same three steps, tolerance 1e-5 relative: xc, z, the shifted conv history
and every channel block's x_proj partial; and against the two launches it
replaces (mtl_linear_skinny for in_proj, then mtl_conv_step_xproj): xc, z and
the history bit for bit (same summation orders), the partials to 1e-5 (they
are summed on the matrix cores here, channel by channel there).  Shapes: the mamba-1.4b
and 130m widths at 32 tokens, small and odd batch sizes, conv widths 2..4, J
up to 288, with and without the in_proj and conv biases."""
import pytest
import torch
import torch.nn.functional as F

from _util import assert_rel
from mamba_lite import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-5


def _operands(b, M, D, K, J, biases, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(b, M, device=DEV, generator=g)
    W_in = torch.randn(2 * D, M, device=DEV, generator=g) / M ** 0.5
    b_in = torch.randn(2 * D, device=DEV, generator=g) if biases else None
    state = torch.randn(b, D, K - 1, device=DEV, generator=g)
    conv_w = torch.randn(D, K, device=DEV, generator=g) / K ** 0.5
    conv_b = torch.randn(D, device=DEV, generator=g) if biases else None
    W_xT = torch.randn(D, J, device=DEV, generator=g) / D ** 0.5
    return x, W_in, b_in, state, conv_w, conv_b, W_xT


def _ref(x, W_in, b_in, state, conv_w, conv_b, W_xT, cpp):
    d = lambda t: None if t is None else t.double().cpu()
    x, W_in, b_in, state, conv_w, conv_b, W_xT = map(d, (x, W_in, b_in, state, conv_w, conv_b, W_xT))
    D = W_in.shape[0] // 2
    xz = x @ W_in.T + (b_in if b_in is not None else 0)
    window = torch.cat([state, xz[:, :D, None]], dim=2)                       # [b, D, K]
    pre = (window * conv_w[None]).sum(-1) + (conv_b if conv_b is not None else 0)
    xc = F.silu(pre)
    parts = torch.stack([xc[:, p * cpp:(p + 1) * cpp] @ W_xT[p * cpp:(p + 1) * cpp] for p in range(D // cpp)])
    return xc, xz[:, D:], window[:, :, 1:], parts


CASES = [  # b, d_model, d_inner, d_conv, J, channels_per_part, biases
    (32, 2048, 4096, 4, 160, 32, False),
    (32, 768, 1536, 4, 80, 16, False),
    (32, 768, 1536, 4, 80, 32, True),
    (5, 256, 64, 4, 40, 16, True),
    (17, 512, 96, 3, 288, 16, False),
    (17, 512, 96, 2, 288, 32, True),
    (1, 384, 32, 4, 18, 16, False),
    (16, 256, 128, 4, 97, 32, True),
]


@pytest.mark.parametrize("b,M,D,K,J,cpp,biases", CASES)
def test_in_proj_conv_xproj_vs_float64(b, M, D, K, J, cpp, biases):
    print(f"\n[in_proj_conv_xproj b={b} d_model={M} d_inner={D} d_conv={K} J={J} cpp={cpp} biases={biases}]",
          flush=True)
    x, W_in, b_in, state, conv_w, conv_b, W_xT = _operands(b, M, D, K, J, biases, b * 131 + M + D + K)
    r_xc, r_z, r_state, r_parts = _ref(x, W_in, b_in, state, conv_w, conv_b, W_xT, cpp)
    xc, z, xpart = ops.in_proj_conv_xproj(x, W_in, b_in, state, conv_w, conv_b, W_xT, channels_per_part=cpp)
    assert xpart.shape == (D // cpp, b, J)
    assert_rel(xc.cpu().numpy(), r_xc.numpy(), TOL, "xc")
    assert_rel(z.cpu().numpy(), r_z.numpy(), TOL, "z")
    assert_rel(state.cpu().numpy(), r_state.numpy(), TOL, "conv history")
    assert_rel(xpart.cpu().numpy(), r_parts.numpy(), TOL, "x_proj partials")
    assert_rel(ops.sum_parts(xpart).cpu().numpy(), r_parts.sum(0).numpy(), TOL, "x_dbl")


@pytest.mark.parametrize("b,M,D,K,J", [(32, 2048, 4096, 4, 160), (7, 768, 1536, 4, 80), (20, 256, 96, 3, 200)])
def test_in_proj_conv_xproj_equals_the_two_launches(b, M, D, K, J):
    """With 32-channel parts the in_proj tile product (the same as
    mtl_linear_skinny's) and the conv taps keep the unfused path's summation
    orders, so xc, z and the history match bit for bit; the x_proj partials
    of the same channel blocks agree to 1e-5."""
    print(f"\n[in_proj_conv_xproj == linear_skinny + conv_step_xproj b={b} d_model={M} d_inner={D}]", flush=True)
    x, W_in, b_in, state, conv_w, conv_b, W_xT = _operands(b, M, D, K, J, True, 7 * b + D)
    state2 = state.clone()
    xc, z, xpart = ops.in_proj_conv_xproj(x, W_in, b_in, state, conv_w, conv_b, W_xT, channels_per_part=32)
    xz = ops.linear_skinny(x, W_in, b_in)
    xc2, xpart2 = ops.conv_step_xproj(state2, xz[:, :D], conv_w, conv_b, W_xT)
    assert torch.equal(z, xz[:, D:])
    assert torch.equal(xc, xc2)
    assert torch.equal(state, state2)
    assert_rel(xpart.cpu().numpy(), xpart2.cpu().numpy(), TOL, "x_proj partials")


def test_in_proj_conv_xproj_rejects_what_it_does_not_cover():
    x, W_in, b_in, state, conv_w, conv_b, W_xT = _operands(4, 256, 64, 4, 40, False, 1)
    with pytest.raises(ValueError):
        ops.in_proj_conv_xproj(x[:, :128].contiguous(), W_in[:, :128].contiguous(), None, state, conv_w, None, W_xT)
    with pytest.raises(ValueError):   # conv history of the wrong width
        ops.in_proj_conv_xproj(x, W_in, None, state[:, :, :2].contiguous(), conv_w, None, W_xT)


PREFILL_CASES = [  # b, l, d_model, d_inner, d_conv, with history, biases
    (1, 64, 768, 1536, 4, False, False),
    (2, 20, 256, 512, 3, True, False),
    (4, 16, 128, 64, 2, True, True),
    (1, 1, 256, 32, 4, True, False),
    (3, 2, 128, 48, 4, True, True),
    (64, 1, 256, 96, 4, True, False),
    (2, 32, 2048, 4096, 4, True, False),
]


@pytest.mark.parametrize("b,l,M,D,K,hist,biases", PREFILL_CASES)
def test_in_proj_conv_prefill(b, l, M, D, K, hist, biases):
    """mtl_in_proj_conv_prefill (a short prefill's in_proj with the causal
    conv + SiLU and the final history as the epilogue, model.py:197-212):
    u, z and the final conv state bit for bit against mtl_linear_skinny +
    mtl_causal_conv1d_fwd, and against float64 at 1e-5; prompts shorter
    than the conv window (history and tokens mixed in the final state), one
    token per batch row, the 130m and 1.4b widths."""
    print(f"\n[in_proj_conv_prefill b={b} l={l} d_model={M} d_inner={D} d_conv={K} hist={hist} biases={biases}]",
          flush=True)
    g = torch.Generator(device=DEV).manual_seed(b * 97 + l + D + K)
    x = torch.randn(b * l, M, device=DEV, generator=g)
    W_in = torch.randn(2 * D, M, device=DEV, generator=g) / M ** 0.5
    b_in = torch.randn(2 * D, device=DEV, generator=g) if biases else None
    conv_w = torch.randn(D, K, device=DEV, generator=g) / K ** 0.5
    conv_b = torch.randn(D, device=DEV, generator=g) if biases else None
    h_in = torch.randn(b, D, K - 1, device=DEV, generator=g) if hist else None
    h_out = torch.empty(b, D, K - 1, device=DEV)
    u, z = ops.in_proj_conv_prefill(x, W_in, b_in, conv_w, conv_b, h_in, h_out, b, l)
    xz = ops.linear_skinny(x, W_in, b_in).view(b, l, 2 * D)
    u2, h2 = ops.causal_conv1d(xz[..., :D].transpose(1, 2), conv_w, conv_b, conv_state=h_in, silu=True)
    assert torch.equal(z.view(b, l, D), xz[..., D:])
    assert torch.equal(u.view(b, l, D), u2.transpose(1, 2))
    assert torch.equal(h_out, h2)
    xd = x.double().cpu().view(b, l, M)
    xzd = xd @ W_in.double().cpu().T + (b_in.double().cpu() if biases else 0)
    xsd = xzd[..., :D].transpose(1, 2)                                              # [b, D, l]
    pad = h_in.double().cpu() if hist else torch.zeros(b, D, K - 1, dtype=torch.float64)
    win = torch.cat([pad, xsd], dim=2)                                             # [b, D, K-1+l]
    pre = sum(win[..., k:k + l] * conv_w.double().cpu()[None, :, k, None] for k in range(K))
    pre = pre + (conv_b.double().cpu()[None, :, None] if biases else 0)
    assert_rel(u.view(b, l, D).cpu().numpy(), F.silu(pre).transpose(1, 2).numpy(), TOL, "u")
    assert_rel(h_out.cpu().numpy(), win[..., -(K - 1):].numpy(), TOL, "final history")


def test_in_proj_conv_prefill_strided_rows():
    """x as a row-strided view (row stride 2 d_model): the same u, z and
    history as from a contiguous copy, bit for bit."""
    print("\n[in_proj_conv_prefill strided x]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    b, l, M, D, K = 2, 24, 256, 128, 4
    wide = torch.randn(b * l, 2 * M, device=DEV, generator=g)
    x = wide[:, M:]
    W_in = torch.randn(2 * D, M, device=DEV, generator=g) / M ** 0.5
    conv_w = torch.randn(D, K, device=DEV, generator=g)
    h_in = torch.randn(b, D, K - 1, device=DEV, generator=g)
    h1, h2 = torch.empty(b, D, K - 1, device=DEV), torch.empty(b, D, K - 1, device=DEV)
    u1, z1 = ops.in_proj_conv_prefill(x, W_in, None, conv_w, None, h_in, h1, b, l)
    u2, z2 = ops.in_proj_conv_prefill(x.contiguous(), W_in, None, conv_w, None, h_in, h2, b, l)
    assert torch.equal(u1, u2) and torch.equal(z1, z2) and torch.equal(h1, h2)
