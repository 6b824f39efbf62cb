"""Selective-scan kernel (mtl_selective_scan_fwd) vs the oracle, on the GPU.

Tolerances (stated per the parity bar): fp32 activations within 1e-4
relative of the float64 oracle; bf16 activations with fp32 state within
1e-2 relative of the oracle run on the same bf16-rounded inputs.
"""
import numpy as np
import pytest
import torch

from _util import assert_rel, bf16_round, scan_case
from mamba_lite import ops
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV, dtype)


def _run(c, layout="cm", h0=None, dtype=torch.float32, with_z=True, with_D=True, with_bias=True, a_is_log=False,
         algo="auto"):
    u, delta, z = c["u"], c["delta"], c["z"]
    if layout == "tm":   # token-major storage [b, l, D] viewed as [b, D, l]
        U = _t(u.transpose(0, 2, 1), dtype).transpose(1, 2)
        Dl = _t(delta.transpose(0, 2, 1), dtype).transpose(1, 2)
        Z = _t(z.transpose(0, 2, 1), dtype).transpose(1, 2)
        b, Dm, L = u.shape
        Y = torch.empty(b, L, Dm, device=DEV, dtype=dtype).transpose(1, 2)
        # B, C as column slices of an x_dbl-like [b, l, R + 2N] buffer
        N = c["B"].shape[1]
        xdbl = torch.zeros(b, L, 8 + 2 * N, device=DEV, dtype=dtype)
        xdbl[..., 8:8 + N] = _t(c["B"].transpose(0, 2, 1), dtype)
        xdbl[..., 8 + N:] = _t(c["C"].transpose(0, 2, 1), dtype)
        Bt, Ct = xdbl[..., 8:8 + N].transpose(1, 2), xdbl[..., 8 + N:].transpose(1, 2)
    else:
        U, Dl, Z = _t(u, dtype), _t(delta, dtype), _t(z, dtype)
        Bt, Ct = _t(c["B"], dtype), _t(c["C"], dtype)
        Y = None
    A = np.log(-c["A"]) if a_is_log else c["A"]
    y, h = ops.selective_scan(U, Dl, _t(A), Bt, Ct, D=_t(c["D"]) if with_D else None, z=Z if with_z else None,
                              delta_bias=_t(c["delta_bias"]) if with_bias else None,
                              h0=_t(h0) if h0 is not None else None, a_is_log=a_is_log, y=Y, algo=algo)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), h.cpu().numpy()


def _ref(c, h0=None, with_z=True, with_D=True, with_bias=True, round_bf16=False):
    g = (lambda a: bf16_round(a)) if round_bf16 else (lambda a: a)
    return om.selective_scan_bnl(g(c["u"]), g(c["delta"]), c["A"], g(c["B"]), g(c["C"]),
                                 c["D"] if with_D else None, g(c["z"]) if with_z else None,
                                 c["delta_bias"] if with_bias else None, h0, dtype=np.float64)


ALGOS = ["tiled", "chunked"]


@pytest.mark.parametrize("algo", ALGOS)
@pytest.mark.parametrize("layout", ["cm", "tm"])
@pytest.mark.parametrize("b,D,L,N", [(2, 64, 16, 16), (2, 200, 70, 16), (1, 96, 33, 8), (3, 70, 5, 4),
                                     (1, 64, 40, 32), (1, 130, 129, 1), (2, 32, 64, 16), (1, 48, 65, 16),
                                     (1, 20, 1000, 16), (2, 8, 191, 5), (1, 24, 300, 32), (1, 16, 260, 12)])
def test_scan_fp32_vs_oracle(algo, layout, b, D, L, N):
    """Chunk boundaries of the chunked kernel sit every 64 steps: lengths
    below, at and past one chunk, and many chunks (1000 steps).  Past 128
    steps on these small grids, 5 to 16 states take its long form (256-step
    chunks; 12 states: a partial group of four), 32 states the 64-step form."""
    print(f"scan fp32 {algo} {layout} b={b} D={D} L={L} N={N}", flush=True)
    c = scan_case(np.random.default_rng(b * 1000 + D + L + N), b, D, L, N)
    h0 = np.random.default_rng(7).standard_normal((b, D, N)).astype(np.float32)
    y, h = _run(c, layout, h0=h0, algo=algo)
    y_ref, h_ref = _ref(c, h0=h0)
    assert_rel(y, y_ref, 1e-4, "y")
    assert_rel(h, h_ref, 1e-4, "h")


@pytest.mark.parametrize("algo", ALGOS)
@pytest.mark.parametrize("opts", [dict(with_z=False), dict(with_D=False), dict(with_bias=False),
                                  dict(with_z=False, with_D=False, with_bias=False)])
def test_scan_optional_operands(opts, algo):
    c = scan_case(np.random.default_rng(11), 2, 96, 48, 16)
    y, h = _run(c, algo=algo, **opts)
    y_ref, h_ref = _ref(c, **opts)
    assert_rel(y, y_ref, 1e-4, f"y {opts}")
    assert_rel(h, h_ref, 1e-4, f"h {opts}")


@pytest.mark.parametrize("algo", ALGOS)
def test_scan_a_log_input(algo):
    c = scan_case(np.random.default_rng(12), 2, 64, 32, 16)
    y1, h1 = _run(c, a_is_log=True, algo=algo)
    y_ref, h_ref = _ref(c)
    assert_rel(y1, y_ref, 1e-4, "y")
    assert_rel(h1, h_ref, 1e-4, "h")


@pytest.mark.parametrize("algo", ALGOS)
def test_scan_zero_and_one_length(algo):
    c = scan_case(np.random.default_rng(13), 2, 64, 1, 16)
    h0 = np.random.default_rng(3).standard_normal((2, 64, 16)).astype(np.float32)
    y, h = _run(c, h0=h0, algo=algo)
    y_ref, h_ref = _ref(c, h0=h0)
    assert_rel(y, y_ref, 1e-4, "y L=1")
    assert_rel(h, h_ref, 1e-4, "h L=1")
    # L = 0: no output, state passes through unchanged
    u = torch.empty(2, 64, 0, device=DEV)
    B = torch.empty(2, 16, 0, device=DEV)
    y0, hz = ops.selective_scan(u, u, _t(c["A"]), B, B, h0=_t(h0), algo=algo)
    assert y0.shape == (2, 64, 0)
    assert torch.equal(hz.cpu(), torch.from_numpy(h0))


@pytest.mark.parametrize("algo", ALGOS)
@pytest.mark.parametrize("layout", ["cm", "tm"])
def test_scan_bf16_vs_oracle(layout, algo):
    c = scan_case(np.random.default_rng(21), 2, 128, 80, 16)
    y, h = _run(c, layout, dtype=torch.bfloat16, algo=algo)
    y_ref, h_ref = _ref(c, round_bf16=True)
    assert_rel(y, y_ref, 1e-2, "y bf16")
    assert_rel(h, h_ref, 1e-2, "h bf16")


@pytest.mark.parametrize("algo", ALGOS)
def test_scan_is_deterministic(algo):
    c = scan_case(np.random.default_rng(22), 2, 128, 100, 16)
    y1, h1 = _run(c, algo=algo)
    y2, h2 = _run(c, algo=algo)
    assert np.array_equal(y1, y2) and np.array_equal(h1, h2)


def test_scan_full_size_properties():
    """The isolated-op shape u,z [32,1536,1024]: (1) continuation from the
    carried state is bit-identical to the one-pass scan, (2) sampled channel
    blocks match the oracle, (3) every output is finite."""
    b, D, L, N = 32, 1536, 1024, 16
    print(f"scan full size b={b} D={D} L={L}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(0)
    u = torch.randn(b, D, L, device=DEV, generator=g)
    z = torch.randn(b, D, L, device=DEV, generator=g)
    delta = 0.5 * torch.randn(b, D, L, device=DEV, generator=g)
    Bm = torch.randn(b, N, L, device=DEV, generator=g)
    Cm = torch.randn(b, N, L, device=DEV, generator=g)
    rng = np.random.default_rng(5)
    bias = _t(om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32))
    A = -torch.arange(1, N + 1, device=DEV, dtype=torch.float32).repeat(D, 1).contiguous()
    Dv = torch.ones(D, device=DEV)
    y, h = ops.selective_scan(u, delta, A, Bm, Cm, D=Dv, z=z, delta_bias=bias)
    k = 512
    y1, h1 = ops.selective_scan(u[..., :k], delta[..., :k], A, Bm[..., :k], Cm[..., :k], D=Dv, z=z[..., :k],
                                delta_bias=bias)
    y2, h2 = ops.selective_scan(u[..., k:], delta[..., k:], A, Bm[..., k:], Cm[..., k:], D=Dv, z=z[..., k:],
                                delta_bias=bias, h0=h1)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all() and torch.isfinite(h).all()
    assert torch.equal(torch.cat([y1, y2], -1), y)
    assert torch.equal(h2, h)
    # oracle on sampled (batch, channel-block) pairs
    for bi, c0 in ((0, 0), (17, 704), (31, 1472)):
        sl = slice(c0, c0 + 64)
        yr, hr = om.selective_scan_bnl(u[bi:bi + 1, sl].cpu().numpy(), delta[bi:bi + 1, sl].cpu().numpy(),
                                       A[sl].cpu().numpy(), Bm[bi:bi + 1].cpu().numpy(), Cm[bi:bi + 1].cpu().numpy(),
                                       Dv[sl].cpu().numpy(), z[bi:bi + 1, sl].cpu().numpy(),
                                       bias[sl].cpu().numpy(), None, dtype=np.float64)
        assert_rel(y[bi:bi + 1, sl].cpu().numpy(), yr, 1e-4, f"y b={bi} c0={c0}")
        assert_rel(h[bi:bi + 1, sl].cpu().numpy(), hr, 1e-4, f"h b={bi} c0={c0}")


@pytest.mark.parametrize("algo", ALGOS)
def test_scan_channel_shard_equals_dense_slice(algo):
    """Per-channel independence the TP shard relies on (reference
    test_tp_correctness.py:76-79): scanning channels [1024, 2048) alone gives
    exactly the dense result's slice."""
    c = scan_case(np.random.default_rng(23), 2, 2048, 64, 16)
    y, h = _run(c, algo=algo)
    sub = {k: (v[:, 1024:] if k in ("u", "delta", "z") else v[1024:] if k in ("A", "D", "delta_bias") else v)
           for k, v in c.items()}
    ys, hs = _run(sub, algo=algo)
    assert np.array_equal(ys, y[:, 1024:]) and np.array_equal(hs, h[:, 1024:])


def test_zero_batch_and_zero_channels_are_no_ops():
    for b, D in ((0, 64), (2, 0)):
        u = torch.randn(b, D, 8, device=DEV)
        B = torch.randn(b, 16, 8, device=DEV)
        A = -torch.ones(D, 16, device=DEV)
        y, h = ops.selective_scan(u, u, A, B, B)
        assert y.shape == (b, D, 8) and h.shape == (b, D, 16)
        out, fs = ops.causal_conv1d(u, torch.randn(D, 4, device=DEV))
        assert out.shape == (b, D, 8) and fs.shape == (b, D, 3)
    torch.cuda.synchronize()


def _sweep_cases(n=24, seed=2024):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        cases.append((int(rng.integers(1, 4)), int(rng.choice([1, 7, 63, 64, 65, 128, 190, 257])),
                      int(rng.choice([1, 2, 15, 16, 17, 31, 32, 33, 64, 100])), int(rng.choice([1, 2, 4, 8, 12, 16, 32])),
                      str(rng.choice(["cm", "tm"])), bool(rng.integers(0, 2)), 1000 + i))
    return cases


@pytest.mark.parametrize("b,D,L,N,layout,with_h0,seed", _sweep_cases())
def test_scan_seeded_shape_sweep(b, D, L, N, layout, with_h0, seed):
    """Seeded sweep over ragged channel counts (tail channel blocks), lengths
    around the 16/32-step tile edges, state sizes 1..32, both layouts, with
    and without a carried state: fp32 vs the float64 oracle at 1e-4."""
    print(f"scan sweep b={b} D={D} L={L} N={N} {layout} h0={with_h0} seed={seed}", flush=True)
    c = scan_case(np.random.default_rng(seed), b, D, L, N)
    h0 = np.random.default_rng(seed + 1).standard_normal((b, D, N)).astype(np.float32) if with_h0 else None
    y, h = _run(c, layout, h0=h0)
    y_ref, h_ref = _ref(c, h0=h0)
    assert_rel(y, y_ref, 1e-4, "y")
    assert_rel(h, h_ref, 1e-4, "h")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scan_generic_bc_strides(dtype):
    """B and C with no unit stride at all (every other step of a wider
    buffer, state stride 3): the scan's generic B/C staging path, against the
    oracle on the same values."""
    b, D, L, N = 2, 96, 45, 16
    c = scan_case(np.random.default_rng(31), b, D, L, N)
    bigB = torch.zeros(b, 3 * N, 2 * L, device=DEV, dtype=dtype)
    bigC = torch.zeros(b, 3 * N, 2 * L, device=DEV, dtype=dtype)
    Bv, Cv = bigB[:, ::3, ::2], bigC[:, ::3, ::2]
    Bv.copy_(_t(c["B"], dtype)); Cv.copy_(_t(c["C"], dtype))
    assert Bv.stride(1) != 1 and Bv.stride(2) != 1
    y, h = ops.selective_scan(_t(c["u"], dtype), _t(c["delta"], dtype), _t(c["A"]), Bv, Cv, D=_t(c["D"]),
                              z=_t(c["z"], dtype), delta_bias=_t(c["delta_bias"]))
    torch.cuda.synchronize()
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    y_ref, h_ref = _ref(c, round_bf16=dtype == torch.bfloat16)
    assert_rel(y.float().cpu().numpy(), y_ref, tol, "y")
    assert_rel(h.cpu().numpy(), h_ref, tol, "h")


def test_scan_nan_delta_propagates_like_torch():
    """A NaN in delta + dt_bias makes dt NaN, as torch's softplus does in the
    reference (model.py:218): that channel's state and its outputs from that
    step on are NaN, the steps before it and every other channel are
    untouched (bit-identical to the clean run)."""
    b, D, L, N = 1, 64, 8, 16
    g = torch.Generator(device=DEV).manual_seed(0)
    u = torch.randn(b, D, L, device=DEV, generator=g)
    d = torch.randn(b, D, L, device=DEV, generator=g) * 0.5
    Bm = torch.randn(b, N, L, device=DEV, generator=g)
    Cm = torch.randn(b, N, L, device=DEV, generator=g)
    A = -torch.arange(1, N + 1, device=DEV, dtype=torch.float32).repeat(D, 1).contiguous()
    bias = torch.full((D,), -3.0, device=DEV)
    y0, h0 = ops.selective_scan(u, d, A, Bm, Cm, delta_bias=bias)
    dn = d.clone()
    dn[0, 5, 3] = float("nan")
    yn, hn = ops.selective_scan(u, dn, A, Bm, Cm, delta_bias=bias)
    torch.cuda.synchronize()
    assert torch.isnan(yn[0, 5, 3:]).all() and torch.isnan(hn[0, 5]).all()
    assert torch.equal(yn[0, 5, :3], y0[0, 5, :3])
    keep = [c for c in range(D) if c != 5]
    assert torch.equal(yn[0, keep], y0[0, keep]) and torch.equal(hn[0, keep], h0[0, keep])


def test_scan_shard_size_bf16_properties():
    """One TP rank's shard at its real shape: bf16 u, delta, z [32, 2048, 2048]
    token-major (as the mixer lays them out), B, C contiguous [32, 2048, 16],
    fp32 state.  (1) continuation from the carried state reproduces the
    one-pass scan bit for bit, (2) sampled channel blocks match the float64
    oracle on the same bf16 values at 1e-2, (3) every output is finite."""
    b, D, L, N = 32, 2048, 2048, 16
    print(f"scan shard size bf16 b={b} D={D} L={L}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(1)
    bf = torch.bfloat16
    mk = lambda *s: torch.randn(*s, device=DEV, generator=g).to(bf)
    u, z, Bin, Cin = mk(b, L, D), mk(b, L, D), mk(b, L, N), mk(b, L, N)
    delta = (0.5 * torch.randn(b, L, D, device=DEV, generator=g)).to(bf)
    rng = np.random.default_rng(6)
    bias = _t(om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32))
    A_log = torch.log(torch.arange(1, N + 1, device=DEV, dtype=torch.float32)).repeat(D, 1).contiguous()
    Dv = torch.ones(D, device=DEV)
    tv = lambda t: t.transpose(1, 2)
    y, h = ops.selective_scan(tv(u), tv(delta), A_log, tv(Bin), tv(Cin), D=Dv, z=tv(z), delta_bias=bias,
                              a_is_log=True)
    k = 1024
    y1, h1 = ops.selective_scan(tv(u[:, :k]), tv(delta[:, :k]), A_log, tv(Bin[:, :k]), tv(Cin[:, :k]), D=Dv,
                                z=tv(z[:, :k]), delta_bias=bias, a_is_log=True)
    y2, h2 = ops.selective_scan(tv(u[:, k:]), tv(delta[:, k:]), A_log, tv(Bin[:, k:]), tv(Cin[:, k:]), D=Dv,
                                z=tv(z[:, k:]), delta_bias=bias, h0=h1, a_is_log=True)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(h).all()
    assert torch.equal(torch.cat([y1, y2], -1), y) and torch.equal(h2, h)
    A = -np.exp(A_log.cpu().numpy())
    for bi, c0 in ((0, 0), (13, 1024), (31, 1984)):
        sl = slice(c0, c0 + 64)
        f = lambda t: t[bi:bi + 1].float().cpu().numpy()
        yr, hr = om.selective_scan_bnl(f(tv(u))[:, sl], f(tv(delta))[:, sl], A[sl], f(tv(Bin)), f(tv(Cin)),
                                       Dv[sl].cpu().numpy(), f(tv(z))[:, sl], bias[sl].cpu().numpy(), None,
                                       dtype=np.float64)
        assert_rel(y[bi:bi + 1, sl].float().cpu().numpy(), yr, 1e-2, f"y b={bi} c0={c0}")
        assert_rel(h[bi:bi + 1, sl].cpu().numpy(), hr, 1e-2, f"h b={bi} c0={c0}")


@pytest.mark.parametrize("dtype,L,Lp,N,full_ops", [(torch.float32, 1000, 1000, 16, True),
                                                   (torch.float32, 996, 1008, 13, False),
                                                   (torch.bfloat16, 1000, 1000, 16, True)])
def test_scan_large_ragged_grid(dtype, L, Lp, N, full_ops):
    """A 552-block channel-major grid, [24, 1472, L]: 23 channel blocks of
    64 per row (1472 = 23 * 64, so the grid is not a multiple of the CU
    count), L leaves a partial last 16-step sub-tile, and rows of Lp >= L
    steps make the inputs strided views.  Checked against (1) the float64
    oracle on sampled channel blocks, including the last one, (2) the same
    scan on a 3-block channel slice (a 72-block grid), bit for bit, and (3) bit-exact
    continuation split off the 16-step tile grid."""
    b, D = 24, 1472
    print(f"scan large ragged grid b={b} D={D} L={L} N={N} {dtype} full_ops={full_ops}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(7)
    mk = lambda *s, sc=1.0: (sc * torch.randn(*s[:-1], Lp, device=DEV, generator=g)).to(dtype)[..., :L]
    u, z, delta = mk(b, D, L), mk(b, D, L), mk(b, D, L, sc=0.5)
    Bm, Cm = mk(b, N, L), mk(b, N, L)
    if not full_ops:                    # delta is dt itself: keep it a small positive step
        delta.abs_().mul_(0.1)
    rng = np.random.default_rng(8)
    bias = _t(om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32))
    A = -torch.arange(1, N + 1, device=DEV, dtype=torch.float32).repeat(D, 1).contiguous()
    Dv = torch.linspace(0.5, 1.5, D, device=DEV)
    h0 = torch.randn(b, D, N, device=DEV, generator=g)
    kw = dict(D=Dv, z=z, delta_bias=bias, h0=h0) if full_ops else {}
    sp = full_ops                       # no bias / D / z / h0 and no softplus on the second case
    y, h = ops.selective_scan(u, delta, A, Bm, Cm, delta_softplus=sp, **kw)
    k = 504
    kw1 = dict(kw); kw2 = dict(kw)
    if full_ops:
        kw1["z"], kw2["z"] = z[..., :k], z[..., k:]
    y1, h1 = ops.selective_scan(u[..., :k], delta[..., :k], A, Bm[..., :k], Cm[..., :k], delta_softplus=sp, **kw1)
    kw2["h0"] = h1
    y2, h2 = ops.selective_scan(u[..., k:], delta[..., k:], A, Bm[..., k:], Cm[..., k:], delta_softplus=sp, **kw2)
    kws = {kk: (v[:192] if kk in ("D", "delta_bias") else v[:, :192]) for kk, v in kw.items()}
    if "h0" in kws:
        kws["h0"] = kws["h0"].contiguous()
    # a 72-block grid is one the automatic choice gives to the chunked kernel: force the tiled one,
    # whose results do not depend on the grid
    ys, hs = ops.selective_scan(u[:, :192], delta[:, :192], A[:192], Bm, Cm, delta_softplus=sp, algo="tiled",
                                **kws)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(h).all()
    assert torch.equal(torch.cat([y1, y2], -1), y) and torch.equal(h2, h)
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    assert torch.equal(y[:, :192], ys) and torch.equal(h[:, :192], hs)
    f = lambda t, bi: t[bi:bi + 1].float().cpu().numpy()
    for bi, c0 in ((0, 0), (11, 640), (23, 1408)):
        sl = slice(c0, c0 + 64)
        yr, hr = om.selective_scan_bnl(f(u, bi)[:, sl], f(delta, bi)[:, sl], A[sl].cpu().numpy(), f(Bm, bi),
                                       f(Cm, bi), Dv[sl].cpu().numpy() if full_ops else None,
                                       f(z, bi)[:, sl] if full_ops else None,
                                       bias[sl].cpu().numpy() if full_ops else None,
                                       f(h0, bi)[:, sl] if full_ops else None, delta_softplus=sp, dtype=np.float64)
        assert_rel(y[bi:bi + 1, sl].float().cpu().numpy(), yr, tol, f"y b={bi} c0={c0}")
        assert_rel(h[bi:bi + 1, sl].cpu().numpy(), hr, tol, f"h b={bi} c0={c0}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("b,L,k", [(2, 300, 77), (1, 300, 133), (1, 1000, 300)])
def test_chunked_matches_tiled_and_continues(dtype, b, L, k):
    """The two kernels on one mid-size mixer-layout input agree (fp32 1e-4,
    bf16 outputs within 1e-2), and the chunked kernel continued from its own
    state at a step that is not a chunk boundary reproduces its one-pass
    result.  At batch 1 (192 workgroups) sequences over 128 steps take the
    chunked kernel's long form (256-step chunks, 4 steps per lane), both
    parts of the 133 / 167 and 300 / 700 splits included; at batch 2 (384
    workgroups) the 64-step form."""
    D, N = 1536, 16
    print(f"scan chunked vs tiled {dtype} b={b} D={D} L={L} k={k}", flush=True)
    c = scan_case(np.random.default_rng(31), b, D, L, N)
    y1, h1 = _run(c, "tm", dtype=dtype, algo="tiled")
    y2, h2 = _run(c, "tm", dtype=dtype, algo="chunked")
    tol = 1e-4 if dtype == torch.float32 else 1e-2
    assert_rel(y2, y1, tol, "y chunked vs tiled")
    assert_rel(h2, h1, 1e-4, "h chunked vs tiled")
    cut = lambda a, sl: {**c, "u": a["u"][..., sl], "delta": a["delta"][..., sl], "z": a["z"][..., sl],
                         "B": a["B"][..., sl], "C": a["C"][..., sl]}
    ya, ha = _run(cut(c, slice(0, k)), "tm", dtype=dtype, algo="chunked")
    yb, hb = _run(cut(c, slice(k, L)), "tm", h0=ha, dtype=dtype, algo="chunked")
    assert_rel(np.concatenate([ya, yb], -1), y2, tol, "continued y")
    assert_rel(hb, h2, 1e-4, "continued h")
