"""Conv (prefill + step), single-token SSM update and add+RMSNorm kernels vs
the oracle, on the GPU.  fp32 within 1e-4 relative; bf16 activations within
1e-2 of the oracle on bf16-rounded inputs."""
import numpy as np
import pytest
import torch

from _util import assert_rel, bf16_round
from mamba_lite import ops
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


@pytest.mark.parametrize("layout", ["cm", "tm"])
@pytest.mark.parametrize("L", [1, 2, 3, 4, 37, 100])
@pytest.mark.parametrize("with_state", [False, True])
def test_conv_fp32(layout, L, with_state):
    rng = np.random.default_rng(L * 10 + with_state)
    b, D, K = 2, 300, 4
    x = rng.standard_normal((b, D, L)).astype(np.float32)
    w = rng.standard_normal((D, K)).astype(np.float32)
    bias = rng.standard_normal(D).astype(np.float32)
    st = rng.standard_normal((b, D, K - 1)).astype(np.float32) if with_state else None
    X = _t(x) if layout == "cm" else _t(x.transpose(0, 2, 1)).transpose(1, 2)
    out, fs = ops.causal_conv1d(X, _t(w), _t(bias), conv_state=_t(st) if st is not None else None, silu=True)
    ref, ref_fs = om.causal_conv1d(x, w, bias, st, dtype=np.float64)
    assert_rel(out.cpu().numpy(), om.silu(ref), 1e-4, "conv out")
    assert np.array_equal(fs.cpu().numpy(), ref_fs.astype(np.float32)), "final conv state must be exact copies"


@pytest.mark.parametrize("D,offset", [(301, 0), (300, 1), (256, 0)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_state", [False, True])
def test_conv_token_major_views(D, offset, dtype, with_state):
    """Token-major views as the mixer passes them (the x half of in_proj's
    [b, l, 2D] output): vector path when channels are unit-stride and
    aligned, one channel per thread when D is odd or the view starts off a
    vector boundary; L = 70 spans five 16-step runs with a ragged last one."""
    rng = np.random.default_rng(D + offset + with_state)
    b, L, K = 3, 70, 4
    xz = rng.standard_normal((b, L, 2 * D + offset)).astype(np.float32)
    w = rng.standard_normal((D, K)).astype(np.float32)
    bias = rng.standard_normal(D).astype(np.float32)
    st = rng.standard_normal((b, D, K - 1)).astype(np.float32) if with_state else None
    XZ = _t(xz, dtype)
    X = XZ[..., offset:offset + D].transpose(1, 2)
    st_t = _t(st, dtype) if st is not None else None
    out, fs = ops.causal_conv1d(X, _t(w), _t(bias), conv_state=st_t, silu=True)
    xr = xz[..., offset:offset + D].transpose(0, 2, 1)
    if dtype == torch.bfloat16:
        xr = bf16_round(xr)
        st = bf16_round(st) if st is not None else None
    ref, ref_fs = om.causal_conv1d(np.ascontiguousarray(xr), w, bias, st, dtype=np.float64)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    assert_rel(out.float().cpu().numpy(), om.silu(ref), tol, "conv out")
    assert np.array_equal(fs.float().cpu().numpy(), ref_fs.astype(np.float32))


def test_conv_no_activation_and_widths():
    rng = np.random.default_rng(3)
    for K in (2, 3, 4, 5, 8):
        x = rng.standard_normal((1, 65, 19)).astype(np.float32)
        w = rng.standard_normal((65, K)).astype(np.float32)
        out, fs = ops.causal_conv1d(_t(x), _t(w), None, silu=False)
        ref, ref_fs = om.causal_conv1d(x, w, None, None, dtype=np.float64)
        assert_rel(out.cpu().numpy(), ref, 1e-4, f"K={K}")
        assert np.array_equal(fs.cpu().numpy(), ref_fs.astype(np.float32))


@pytest.mark.parametrize("K", [6, 8])
@pytest.mark.parametrize("L", [1, 5, 6, 9, 13])
def test_conv_short_runs_read_history_past_the_first_run(K, L):
    """Small grids use 4-step runs: with K - 1 > 4 the second run's window
    also starts inside the carried history, which must come from conv_state
    (not clamped inputs), in both layouts."""
    rng = np.random.default_rng(K * 100 + L)
    x = rng.standard_normal((2, 96, L)).astype(np.float32)
    w = rng.standard_normal((96, K)).astype(np.float32)
    bias = rng.standard_normal(96).astype(np.float32)
    st = rng.standard_normal((2, 96, K - 1)).astype(np.float32)
    ref, ref_fs = om.causal_conv1d(x, w, bias, st, dtype=np.float64)
    for X in (_t(x), _t(np.ascontiguousarray(x.transpose(0, 2, 1))).transpose(1, 2)):
        out, fs = ops.causal_conv1d(X, _t(w), _t(bias), conv_state=_t(st), silu=True)
        assert_rel(out.cpu().numpy(), om.silu(ref), 1e-4, f"K={K} L={L}")
        assert np.array_equal(fs.cpu().numpy(), ref_fs.astype(np.float32))


def test_conv_zero_length_passes_state_through():
    st = torch.randn(2, 64, 3, device=DEV)
    x = torch.empty(2, 64, 0, device=DEV)
    out, fs = ops.causal_conv1d(x, torch.randn(64, 4, device=DEV), conv_state=st)
    assert out.shape == (2, 64, 0) and torch.equal(fs, st)


def test_conv_bf16():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 256, 50)).astype(np.float32)
    w = rng.standard_normal((256, 4)).astype(np.float32)
    bias = rng.standard_normal(256).astype(np.float32)
    X = _t(x.transpose(0, 2, 1), torch.bfloat16).transpose(1, 2)
    out, fs = ops.causal_conv1d(X, _t(w), _t(bias))
    ref, ref_fs = om.causal_conv1d(bf16_round(x), w, bias, None, dtype=np.float64)
    assert out.dtype == torch.bfloat16
    assert_rel(out.float().cpu().numpy(), om.silu(ref), 1e-2, "conv bf16")
    assert np.array_equal(fs.float().cpu().numpy(), ref_fs.astype(np.float32))


def test_conv_step_in_place():
    rng = np.random.default_rng(5)
    b, D, K = 3, 200, 4
    st = rng.standard_normal((b, D, K - 1)).astype(np.float32)
    xz = rng.standard_normal((b, 2 * D)).astype(np.float32)
    w = rng.standard_normal((D, K)).astype(np.float32)
    bias = rng.standard_normal(D).astype(np.float32)
    S = _t(st)
    ptr = S.data_ptr()
    XZ = _t(xz)
    out = ops.conv_step(S, XZ[:, :D], _t(w), _t(bias))
    ref, ref_st = om.conv_step(st, xz[:, :D], w, bias, dtype=np.float64)
    assert S.data_ptr() == ptr
    assert_rel(out.cpu().numpy(), om.silu(ref), 1e-4, "conv step")
    assert np.array_equal(S.cpu().numpy(), ref_st.astype(np.float32))


@pytest.mark.parametrize("N,R", [(16, 48), (16, 128), (8, 2), (4, 5), (16, 256), (16, 32)])
@pytest.mark.parametrize("b", [1, 4, 11, 16, 17, 32, 40])
def test_selective_state_update(N, R, b):
    """b = 11 covers the 8-row batch blocks with a ragged last block; from 16
    rows (16 states, dt_rank a multiple of 16) the 32-row form with the dt
    dot on the matrix cores runs, b = 17 and 40 with a ragged last 32-row
    block, D = 200 with a ragged last 16-channel block."""
    print(f"state update N={N} R={R} b={b}", flush=True)
    rng = np.random.default_rng(N * 100 + R + b)
    D = 200
    h = rng.standard_normal((b, D, N)).astype(np.float32)
    x = rng.standard_normal((b, D)).astype(np.float32)
    z = rng.standard_normal((b, D)).astype(np.float32)
    xdbl = rng.standard_normal((b, R + 2 * N)).astype(np.float32)
    W = (rng.standard_normal((D, R)) / np.sqrt(R)).astype(np.float32)
    bdt = om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32)
    A_log = np.log(np.tile(np.arange(1, N + 1, dtype=np.float32), (D, 1)))
    Dv = rng.standard_normal(D).astype(np.float32)
    H = _t(h)
    y = ops.selective_state_update(H, _t(x), _t(z), _t(xdbl), _t(W), _t(bdt), _t(A_log), _t(Dv), a_is_log=True)
    y_ref, h_ref = om.selective_state_update(h, x, xdbl[:, :R], W, bdt, -np.exp(A_log.astype(np.float64)),
                                             xdbl[:, R:R + N], xdbl[:, R + N:], Dv, z, dtype=np.float64)
    assert_rel(y.cpu().numpy(), y_ref, 1e-4, "y")
    assert_rel(H.cpu().numpy(), h_ref, 1e-4, "state")


@pytest.mark.parametrize("b", [2, 16])
def test_selective_state_update_bf16(b):
    rng = np.random.default_rng(9 + b)
    D, N, R = 256, 16, 48
    h = rng.standard_normal((b, D, N)).astype(np.float32)
    x = rng.standard_normal((b, D)).astype(np.float32)
    z = rng.standard_normal((b, D)).astype(np.float32)
    xdbl = rng.standard_normal((b, R + 2 * N)).astype(np.float32)
    W = (rng.standard_normal((D, R)) / np.sqrt(R)).astype(np.float32)
    bdt = om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32)
    A = -np.tile(np.arange(1, N + 1, dtype=np.float32), (D, 1))
    Dv = np.ones(D, np.float32)
    H = _t(h)
    y = ops.selective_state_update(H, _t(x, torch.bfloat16), _t(z, torch.bfloat16), _t(xdbl, torch.bfloat16),
                                   _t(W), _t(bdt), _t(A), _t(Dv))
    xr, zr, dr = bf16_round(x), bf16_round(z), bf16_round(xdbl)
    y_ref, h_ref = om.selective_state_update(h, xr, dr[:, :R], W, bdt, A, dr[:, R:R + N], dr[:, R + N:], Dv, zr,
                                             dtype=np.float64)
    assert_rel(y.float().cpu().numpy(), y_ref, 1e-2, "y bf16")
    assert_rel(H.cpu().numpy(), h_ref, 1e-2, "state bf16")


def test_step_matches_one_token_prefill():
    """A single conv+SSM step from a given state equals a length-1 prefill
    through the conv and scan kernels from the same state."""
    rng = np.random.default_rng(10)
    b, D, N, R, K = 2, 192, 16, 12, 4
    cs = rng.standard_normal((b, D, K - 1)).astype(np.float32)
    hs = rng.standard_normal((b, D, N)).astype(np.float32)
    xz = rng.standard_normal((b, 2 * D)).astype(np.float32)
    w = rng.standard_normal((D, K)).astype(np.float32)
    cb = rng.standard_normal(D).astype(np.float32)
    xdbl = rng.standard_normal((b, R + 2 * N)).astype(np.float32)
    W = (rng.standard_normal((D, R)) / np.sqrt(R)).astype(np.float32)
    bdt = rng.standard_normal(D).astype(np.float32) - 3
    A = -np.tile(np.arange(1, N + 1, dtype=np.float32), (D, 1))
    Dv = rng.standard_normal(D).astype(np.float32)
    XZ = _t(xz)
    CS, HS = _t(cs), _t(hs)
    xc = ops.conv_step(CS, XZ[:, :D], _t(w), _t(cb))
    y = ops.selective_state_update(HS, xc, XZ[:, D:], _t(xdbl), _t(W), _t(bdt), _t(A), _t(Dv))
    u, fs = ops.causal_conv1d(_t(xz[:, :D, None]), _t(w), _t(cb), conv_state=_t(cs))
    dt = _t(xdbl[:, :R] @ W.T)[:, :, None]
    yp, hp = ops.selective_scan(u, dt, _t(A), _t(xdbl[:, R:R + N, None]), _t(xdbl[:, R + N:, None]), D=_t(Dv),
                                z=_t(xz[:, D:, None]), delta_bias=_t(bdt), h0=_t(hs))
    torch.cuda.synchronize()
    assert torch.equal(CS, fs)
    assert_rel(xc.cpu().numpy(), u[..., 0].cpu().numpy(), 1e-6, "conv")
    assert_rel(y.cpu().numpy(), yp[..., 0].cpu().numpy(), 1e-5, "y")
    assert_rel(HS.cpu().numpy(), hp.cpu().numpy(), 1e-5, "h")


@pytest.mark.parametrize("rows,cols", [(1, 768), (7, 2048), (64, 33), (3, 4096), (2, 5000)])
def test_add_rmsnorm(rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    y = rng.standard_normal((rows, cols)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    X = _t(x)
    out = ops.add_rmsnorm(X, _t(w), 1e-5, y=_t(y), x_out=X)
    assert_rel(X.cpu().numpy(), x.astype(np.float64) + y, 1e-6, "x_out")
    assert_rel(out.cpu().numpy(), om.rmsnorm(x.astype(np.float64) + y, w, 1e-5, np.float64), 1e-5, "normed")
    out2 = ops.add_rmsnorm(_t(x), _t(w), 1e-5)
    assert_rel(out2.cpu().numpy(), om.rmsnorm(x, w, 1e-5, np.float64), 1e-5, "norm only")


@pytest.mark.parametrize("rows,cols,nparts", [(32, 2048, 4), (32, 768, 4), (5, 768, 2), (3, 100, 1), (2, 4500, 3),
                                               (7, 300, 4)])
def test_add_rmsnorm_parts(rows, cols, nparts):
    """y given as split-K parts: x_out = x + ((p0 + p1) + ...), bit for bit
    what the parts summed in order and then mtl_add_rmsnorm give."""
    rng = np.random.default_rng(rows * 3 + cols + nparts)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    parts = rng.standard_normal((nparts, rows, cols)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    X = _t(x)
    out = ops.add_rmsnorm(X, _t(w), 1e-5, y_parts=_t(parts), x_out=X)
    ysum = parts[0].copy()
    for p in range(1, nparts):
        ysum = ysum + parts[p]                   # float32, part order
    X2 = _t(x)
    out2 = ops.add_rmsnorm(X2, _t(w), 1e-5, y=_t(ysum), x_out=X2)
    assert torch.equal(X, X2) and torch.equal(out, out2)
    assert_rel(out.cpu().numpy(), om.rmsnorm(x.astype(np.float64) + parts.astype(np.float64).sum(0), w, 1e-5,
                                             np.float64), 1e-5, "normed")


@pytest.mark.parametrize("nparts,n", [(1, 5), (3, 1000), (16, 5120), (32, 257), (33, 100), (64, 300), (97, 64),
                                      (128, 5120), (129, 70), (256, 1280), (320, 2560), (512, 64), (513, 100),
                                      (700, 33)])
def test_sum_parts_in_part_order(nparts, n):
    """mtl_sum_parts adds the parts in its documented fixed order (left to
    right up to 32 parts, four ordered quarters above), bit for bit."""
    rng = np.random.default_rng(nparts * 7 + n)
    scale = 10.0 ** rng.integers(-3, 4, (nparts, 1))
    parts = (rng.standard_normal((nparts, n)) * scale).astype(np.float32)
    assert parts.dtype == np.float32
    got = ops.sum_parts(_t(parts)).cpu().numpy()

    def ordered(ps):
        r = ps[0].copy()
        for p in ps[1:]:
            r = (r + p).astype(np.float32)
        return r
    if nparts <= 32:
        ref = ordered(parts)
    else:
        per = -(-nparts // 4)
        ref = ordered([ordered(parts[q * per:(q + 1) * per]) for q in range(4) if q * per < nparts])
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("b,D,J,K", [(1, 64, 36, 4), (5, 200, 80, 4), (8, 1536, 80, 4), (17, 333, 160, 3),
                                     (32, 4096, 160, 4), (32, 96, 288, 8)])
def test_conv_step_xproj_matches_conv_step_and_linear(b, D, J, K):
    """The fused batched conv step + x_proj partials: conv output and state
    equal mtl_conv_step's bit for bit; the block partials summed in order
    match x_proj of the conv output (1e-5)."""
    print(f"conv_step_xproj b={b} D={D} J={J} K={K}", flush=True)
    rng = np.random.default_rng(b * 1000 + D + J + K)
    st = rng.standard_normal((b, D, K - 1)).astype(np.float32)
    xz = rng.standard_normal((b, 2 * D)).astype(np.float32)
    w = rng.standard_normal((D, K)).astype(np.float32)
    bias = rng.standard_normal(D).astype(np.float32)
    Wx = (rng.standard_normal((J, D)) / np.sqrt(D)).astype(np.float32)
    S1, S2 = _t(st), _t(st)
    XZ = _t(xz)
    ref = ops.conv_step(S1, XZ[:, :D], _t(w), _t(bias))
    got, xpart = ops.conv_step_xproj(S2, XZ[:, :D], _t(w), _t(bias), _t(Wx.T))
    x_dbl = ops.sum_parts(xpart)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    assert torch.equal(S1, S2)
    xd_ref = ref.double().cpu().numpy() @ Wx.astype(np.float64).T
    assert_rel(x_dbl.cpu().numpy(), xd_ref, 1e-5, "x_dbl")


def _conv_sweep(n=20, seed=77):
    rng = np.random.default_rng(seed)
    return [(int(rng.integers(1, 4)), int(rng.choice([1, 3, 4, 63, 64, 130, 257])),
             int(rng.choice([1, 2, 15, 16, 17, 33, 80])), int(rng.integers(2, 9)), str(rng.choice(["cm", "tm"])),
             bool(rng.integers(0, 2)), 500 + i) for i in range(n)]


@pytest.mark.parametrize("b,D,L,K,layout,with_state,seed", _conv_sweep())
def test_conv_seeded_shape_sweep(b, D, L, K, layout, with_state, seed):
    """Seeded sweep over widths 2..8, channel counts with and without
    4-vector alignment, lengths around the 16-step run edge, both layouts:
    fp32 vs the float64 oracle, final state exact."""
    print(f"conv sweep b={b} D={D} L={L} K={K} {layout} state={with_state} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((b, D, L)).astype(np.float32)
    w = rng.standard_normal((D, K)).astype(np.float32)
    bias = rng.standard_normal(D).astype(np.float32)
    st = rng.standard_normal((b, D, K - 1)).astype(np.float32) if with_state else None
    X = _t(x) if layout == "cm" else _t(x.transpose(0, 2, 1)).transpose(1, 2)
    out, fs = ops.causal_conv1d(X, _t(w), _t(bias), conv_state=_t(st) if st is not None else None, silu=True)
    ref, ref_fs = om.causal_conv1d(x, w, bias, st, dtype=np.float64)
    assert_rel(out.cpu().numpy(), om.silu(ref), 1e-4, "conv out")
    assert np.array_equal(fs.cpu().numpy(), ref_fs.astype(np.float32))


def test_conv_shard_size_bf16_properties():
    """The conv at one TP rank's real shape: bf16 x [32, 2048, 2048] as the
    x half of a token-major [b, l, 2D] in_proj output.  (1) two halves with
    the carried history reproduce the one-pass output and final state bit for
    bit, (2) sampled channel blocks match the oracle (pre-activation conv,
    then SiLU) on the same bf16 values at 1e-2."""
    b, D, L, K = 32, 2048, 2048, 4
    print(f"conv shard size bf16 b={b} D={D} L={L}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(2)
    xz = torch.randn(b, L, 2 * D, device=DEV, generator=g).to(torch.bfloat16)
    x = xz[..., :D].transpose(1, 2)                     # [b, D, l] view, channel stride 1
    w = torch.randn(D, K, device=DEV, generator=g) * 0.5
    cb = torch.randn(D, device=DEV, generator=g) * 0.1
    out, fs = ops.causal_conv1d(x, w, cb)
    k = 1000
    o1, s1 = ops.causal_conv1d(x[..., :k], w, cb)
    o2, s2 = ops.causal_conv1d(x[..., k:], w, cb, conv_state=s1)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([o1, o2], -1), out) and torch.equal(s2, fs)
    for bi, c0 in ((0, 0), (19, 1024), (31, 1984)):
        sl = slice(c0, c0 + 64)
        xr = x[bi:bi + 1, sl].float().cpu().numpy()
        pre, st = om.causal_conv1d(xr, w[sl].cpu().numpy(), cb[sl].cpu().numpy(), None, dtype=np.float64)
        assert_rel(out[bi:bi + 1, sl].float().cpu().numpy(), om.silu(pre), 1e-2, f"out b={bi} c0={c0}")
        assert np.array_equal(fs[bi:bi + 1, sl].float().cpu().numpy(), st.astype(np.float32))
