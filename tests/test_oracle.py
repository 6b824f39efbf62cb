"""Pins the numpy oracle (CPU only, no GPU).

Each check computes the same quantity by an independent route (closed form,
np.convolve, float64 exact arithmetic, hand-computed rows, published byte
totals) so that a plausible slip in the oracle -- a dropped term, a wrong
sign, an off-by-one in time, a transposed operand -- fails here.
"""
import numpy as np
import pytest

from oracle import mixer as om
from oracle import pins
from oracle import quant as oq


def _rng(seed):
    return np.random.default_rng(seed)


def _scan_inputs(rng, b=2, D=5, l=12, N=16):
    u = rng.standard_normal((b, D, l))
    dt_bias = om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D)))
    delta = 0.5 * rng.standard_normal((b, D, l))
    A = -np.exp(rng.uniform(0, np.log(16), (D, N)))
    B = rng.standard_normal((b, l, N))
    C = rng.standard_normal((b, l, N))
    Dv = rng.standard_normal(D)
    z = rng.standard_normal((b, D, l))
    h0 = rng.standard_normal((b, D, N))
    return u, delta, A, B, C, Dv, z, dt_bias, h0


# --------------------------------------------------------------------------- scan
@pytest.mark.parametrize("N", [16, 8])
@pytest.mark.parametrize("with_h0", [False, True])
def test_scan_matches_closed_form(N, with_h0):
    u, delta, A, B, C, Dv, z, bias, h0 = _scan_inputs(_rng(1), N=N)
    h0 = h0[..., :N] if with_h0 else None
    y, h = om.selective_scan(u, delta, A, B, C, delta_bias=bias, h0=h0, dtype=np.float64)
    dt = om.softplus(delta + bias[None, :, None])
    y_cf, h_cf = pins.scan_closed_form(u, dt, A, B, C, h0)
    np.testing.assert_allclose(y, y_cf, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(h, h_cf, rtol=1e-10, atol=1e-12)


def test_scan_skip_and_gate_terms():
    u, delta, A, B, C, Dv, z, bias, h0 = _scan_inputs(_rng(2))
    y0, _ = om.selective_scan(u, delta, A, B, C, delta_bias=bias, dtype=np.float64)
    y1, _ = om.selective_scan(u, delta, A, B, C, D=Dv, z=z, delta_bias=bias, dtype=np.float64)
    sig = 1.0 / (1.0 + np.exp(-z))
    np.testing.assert_allclose(y1, (y0 + u * Dv[None, :, None]) * z * sig, rtol=1e-12, atol=1e-12)


def test_scan_zero_step_keeps_state():
    """delta -> -inf: softplus -> 0, dA = 1, dBx = 0 -> h stays h0 and
    y_t = <h0, C_t> + D u (before the gate)."""
    u, delta, A, B, C, Dv, z, bias, h0 = _scan_inputs(_rng(3))
    delta = np.full_like(delta, -1e4)
    y, h = om.selective_scan(u, delta, A, B, C, D=Dv, h0=h0, delta_bias=None, dtype=np.float64)
    np.testing.assert_array_equal(h, h0)
    expect = np.einsum("bdn,bln->bdl", h0, C) + u * Dv[None, :, None]
    np.testing.assert_allclose(y, expect, rtol=1e-12, atol=1e-12)


def test_scan_infinite_decay_is_memoryless():
    """A -> -inf: dA = 0, so h_t = dt_t B_t u_t and y_t = dt_t u_t <B_t, C_t>."""
    u, delta, A, B, C, Dv, z, bias, h0 = _scan_inputs(_rng(4))
    A = np.full_like(A, -1e300)
    y, h = om.selective_scan(u, delta, A, B, C, delta_bias=bias, h0=h0, dtype=np.float64)
    dt = om.softplus(delta + bias[None, :, None])
    expect = dt * u * np.einsum("bln,bln->bl", B, C)[:, None, :]
    np.testing.assert_allclose(y, expect, rtol=1e-12, atol=1e-12)


def test_scan_geometric_series():
    l = 40
    dtv, a, bx, c, h0 = 0.07, -2.5, 1.3, -0.8, 0.4
    u = np.full((1, 1, l), bx)
    delta = np.full((1, 1, l), dtv)
    A = np.array([[a]])
    B = np.ones((1, l, 1))
    C = np.full((1, l, 1), c)
    y, h = om.selective_scan(u, delta, A, B, C, h0=np.array([[[h0]]]), delta_softplus=False,
                             dtype=np.float64)
    np.testing.assert_allclose(y[0, 0], pins.scan_geometric(dtv, a, bx, c, l, h0), rtol=1e-12)


def test_scan_bnl_layout_is_a_transpose():
    u, delta, A, B, C, Dv, z, bias, h0 = _scan_inputs(_rng(5))
    y1, h1 = om.selective_scan(u, delta, A, B, C, Dv, z, bias, h0, dtype=np.float64)
    y2, h2 = om.selective_scan_bnl(u, delta, A, B.transpose(0, 2, 1), C.transpose(0, 2, 1), Dv, z,
                                   bias, h0, dtype=np.float64)
    np.testing.assert_array_equal(y1, y2)
    np.testing.assert_array_equal(h1, h2)


def test_scan_f32_tracks_f64():
    u, delta, A, B, C, Dv, z, bias, h0 = _scan_inputs(_rng(6), b=2, D=8, l=64)
    y32, h32 = om.selective_scan(u, delta, A, B, C, Dv, z, bias, h0, dtype=np.float32)
    y64, h64 = om.selective_scan(u, delta, A, B, C, Dv, z, bias, h0, dtype=np.float64)
    np.testing.assert_allclose(y32, y64, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(h32, h64, rtol=1e-4, atol=1e-5)


# --------------------------------------------------------------------------- softplus / silu / norm
def test_softplus_values():
    x = np.array([-30.0, -8.0, -1.0, 0.0, 1.0, 19.9, 20.0, 20.5, 50.0])
    # log(1 + e^x) through numpy's logaddexp; the threshold makes x > 20 exact identity
    expect = np.where(x > 20, x, np.logaddexp(0.0, x))
    np.testing.assert_allclose(om.softplus(x), expect, rtol=1e-14)
    assert om.softplus(np.array([20.5]))[0] == 20.5
    assert om.softplus(np.array([0.0]))[0] == np.log(2.0)
    # float32 result stays in float32 and matches log(2) to 1 ulp
    assert om.softplus(np.array([0.0], np.float32)).dtype == np.float32


def test_silu_values():
    x = np.array([-5.0, -1.0, 0.0, 2.0])
    np.testing.assert_allclose(om.silu(x), x / (1 + np.exp(-x)), rtol=1e-15)
    assert om.silu(np.array([0.0]))[0] == 0.0


def test_rmsnorm_constant_vector():
    c, M, eps = -3.0, 16, 1e-5
    w = np.linspace(0.5, 2.0, M)
    out = om.rmsnorm(np.full((2, M), c), w, eps, dtype=np.float64)
    np.testing.assert_allclose(out, np.broadcast_to(w * c / np.sqrt(c * c + eps), (2, M)), rtol=1e-14)


# --------------------------------------------------------------------------- conv
@pytest.mark.parametrize("l", [1, 2, 3, 9])
@pytest.mark.parametrize("with_state", [False, True])
def test_conv_matches_np_convolve(l, with_state):
    rng = _rng(10 + l)
    b, D, K = 2, 6, 4
    x = rng.standard_normal((b, D, l))
    w = rng.standard_normal((D, K))
    bias = rng.standard_normal(D)
    st = rng.standard_normal((b, D, K - 1)) if with_state else None
    out, fs = om.causal_conv1d(x, w, bias, st, dtype=np.float64)
    np.testing.assert_allclose(out, pins.conv_by_np_convolve(x, w, bias, st), rtol=1e-12, atol=1e-12)
    padded = np.concatenate([st if st is not None else np.zeros((b, D, K - 1)), x], axis=-1)
    np.testing.assert_array_equal(fs, padded[..., -(K - 1):])


def test_conv_step_equals_prefill_of_one():
    rng = _rng(20)
    b, D, K = 3, 7, 4
    st = rng.standard_normal((b, D, K - 1))
    x = rng.standard_normal((b, D))
    w = rng.standard_normal((D, K))
    bias = rng.standard_normal(D)
    o1, s1 = om.conv_step(st, x, w, bias, dtype=np.float64)
    o2, s2 = om.causal_conv1d(x[..., None], w, bias, st, dtype=np.float64)
    np.testing.assert_allclose(o1, o2[..., 0], rtol=1e-14)
    np.testing.assert_array_equal(s1, s2)


# --------------------------------------------------------------------------- mixer / LM
def make_mixer_weights(rng, M=32, D=64, N=8, R=None, K=4, bias=False):
    """Random mixer weights with the reference's SSM init (model.py:172-181)
    and the log-uniform dt_bias of HF Mamba (modeling_mamba.py:349-355)."""
    R = R or max(1, M // 16)
    s = lambda *shape: rng.standard_normal(shape) / np.sqrt(shape[-1])
    p = {
        "in_proj_w": s(2 * D, M), "conv_w": rng.standard_normal((D, K)) * 0.5,
        "conv_b": rng.standard_normal(D) * 0.1, "x_proj_w": s(R + 2 * N, D),
        "dt_proj_w": s(D, R), "dt_proj_b": om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))),
        "A_log": np.log(np.tile(np.arange(1, N + 1, dtype=np.float64), (D, 1))), "D": np.ones(D),
        "out_proj_w": s(M, D),
    }
    if bias:
        p["in_proj_b"] = rng.standard_normal(2 * D) * 0.1
        p["out_proj_b"] = rng.standard_normal(M) * 0.1
    return p


@pytest.mark.parametrize("bias", [False, True])
def test_mixer_l1_prefill_equals_step(bias):
    """prefill of one token from zero state == step from a zero cache
    (model.py:184-241 vs 249-294 are separate code paths)."""
    rng = _rng(30)
    p = make_mixer_weights(rng, bias=bias)
    x = rng.standard_normal((2, 1, 32))
    out_p, cs_p, h_p = om.mixer_prefill(p, x, dtype=np.float64)
    cs = np.zeros((2, 64, 3))
    hs = np.zeros((2, 64, 8))
    out_s = om.mixer_step(p, x[:, 0], cs, hs, dtype=np.float64)
    np.testing.assert_allclose(out_s, out_p[:, 0], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(cs, cs_p, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(hs, h_p, rtol=1e-12, atol=1e-14)


@pytest.mark.parametrize("k", [1, 2, 5])
def test_mixer_chunked_continuation(k):
    """prefill(x[:k]) then prefill(x[k:], cache) == prefill(x)
    (model.py:202-203, 226-230)."""
    rng = _rng(31)
    p = make_mixer_weights(rng)
    x = rng.standard_normal((2, 9, 32))
    out, cs, hs = om.mixer_prefill(p, x, dtype=np.float64)
    o1, c1, h1 = om.mixer_prefill(p, x[:, :k], dtype=np.float64)
    o2, c2, h2 = om.mixer_prefill(p, x[:, k:], c1, h1, dtype=np.float64)
    np.testing.assert_allclose(np.concatenate([o1, o2], axis=1), out, rtol=1e-11, atol=1e-12)
    np.testing.assert_allclose(c2, cs, rtol=1e-14)
    np.testing.assert_allclose(h2, hs, rtol=1e-11, atol=1e-13)


def make_lm_weights(rng, V=50, M=32, n_layer=2, **kw):
    return {
        "embedding": rng.standard_normal((V, M)),
        "norm_f": 1 + 0.1 * rng.standard_normal(M),
        "layers": [dict(make_mixer_weights(rng, M=M, **kw), norm=1 + 0.1 * rng.standard_normal(M))
                   for _ in range(n_layer)],
    }


def test_lm_teacher_forced_step_equals_prefill():
    """test_correctness.py:49-72 restated: prefill(ids[:, :1]) then step()
    with the actual next tokens reproduces full-prefill logits."""
    rng = _rng(32)
    W = make_lm_weights(rng)
    ids = rng.integers(0, 50, (2, 7))
    full, _ = om.lm_prefill(W, ids, dtype=np.float64)
    logits0, cache = om.lm_prefill(W, ids[:, :1], dtype=np.float64)
    got = [logits0]
    for t in range(1, 7):
        got.append(om.lm_step(W, ids[:, t:t + 1], cache, dtype=np.float64))
    np.testing.assert_allclose(np.concatenate(got, axis=1), full, rtol=1e-10, atol=1e-10)


def test_lm_f32_tracks_f64():
    rng = _rng(33)
    W = make_lm_weights(rng)
    ids = rng.integers(0, 50, (1, 12))
    l32, _ = om.lm_prefill(W, ids, dtype=np.float32)
    l64, _ = om.lm_prefill(W, ids, dtype=np.float64)
    np.testing.assert_allclose(l32, l64, rtol=1e-4, atol=1e-4)


# --------------------------------------------------------------------------- quant
def test_int8_hand_computed_row():
    # amax = 127 -> scale = 127/127 = 1.0 exactly, so codes = round-half-even(x)
    row = np.array([[2.5, 3.5, -2.5, -0.5, 0.5, 1.5, 127.0, -127.0, 126.5, -3.49]], np.float32)
    s, q = oq.quantize_int8_per_token(row)
    assert s.tolist() == [1.0]
    assert q.tolist() == [[2, 4, -2, 0, 0, 2, 127, -127, 126, -3]]


def test_int8_zero_and_tiny_rows():
    rows = np.zeros((2, 5), np.float32)
    rows[1, 3] = 1e-12
    s, q = oq.quantize_int8_per_token(rows)
    eps_scale = np.float32(np.float32(1e-8) / np.float32(127.0))
    assert s[0] == eps_scale and s[1] == eps_scale
    assert not q[0].any()
    assert q[1].tolist() == [0, 0, 0, 0, 0]   # 1e-12 / 7.9e-11 rounds to 0


def test_int8_amax_maps_to_127():
    rng = _rng(40)
    t = (rng.standard_t(3, (64, 768)) * 0.5).astype(np.float32)
    s, q = oq.quantize_int8_per_token(t)
    idx = np.abs(t).argmax(axis=1)
    assert np.array_equal(np.abs(q[np.arange(64), idx]), np.full(64, 127))
    assert np.array_equal(np.sign(q[np.arange(64), idx]), np.sign(t[np.arange(64), idx]).astype(np.int8))
    # quantization error bound |q s - t| <= s/2 (plus one rounding of the division)
    err = np.abs(q.astype(np.float64) * s[:, None] - t)
    assert (err <= s[:, None] * (0.5 + 1e-6)).all()


def test_int8_dequant_sum_exact_arithmetic():
    """out = fl32(fl32(q0 s0) + fl32(q1 s1)): recomputed in float64, where
    q*s is exact, then rounded explicitly."""
    rng = _rng(41)
    a = (rng.standard_t(3, (33, 80)) * 0.5).astype(np.float32)
    b = (rng.standard_t(3, (33, 80)) * 0.5).astype(np.float32)
    out, (p0, p1) = oq.quant_dequant_sum_int8_tok([a, b])
    s0, q0 = oq.unpack_payload(p0, 33, 80)
    s1, q1 = oq.unpack_payload(p1, 33, 80)
    t0 = (q0.astype(np.float64) * s0[:, None].astype(np.float64)).astype(np.float32)
    t1 = (q1.astype(np.float64) * s1[:, None].astype(np.float64)).astype(np.float32)
    expect = (t0.astype(np.float64) + t1.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(out, expect)
    # reference invariant (test_per_site_allreduce.py:108-112): error < 0.15 * max|dense|
    assert np.abs(out - (a + b)).max() < 0.15 * np.abs(a + b).max()


def test_payload_layout_and_published_bytes():
    t = np.arange(12, dtype=np.float32).reshape(3, 4) - 5
    s, q = oq.quantize_int8_per_token(t)
    p = oq.pack_payload(s, q)
    assert p.dtype == np.uint8 and p.size == oq.payload_nbytes(3, 4) == 3 * 4 + 4 * 3
    assert p[:12].tobytes() == s.astype("<f4").tobytes()
    assert p[12:].view(np.int8).tolist() == q.reshape(-1).tolist()
    # published wire bytes for one 130m prefill forward at b32 x 1024 on rank 0
    # (24 layers; sites x_proj: 48+2*16=80 cols, out_proj: 768 cols)
    rows, layers = 32 * 1024, 24
    assert layers * (oq.payload_nbytes(rows, 80) + oq.payload_nbytes(rows, 768)) == 673_185_792
    assert layers * rows * (80 + 768) * 2 == 1_333_788_672
    assert layers * rows * (80 + 768) * 4 == 2_667_577_344


def test_fp16_sum_is_single_rounding_of_exact_sum():
    rng = _rng(42)
    a = (rng.standard_t(3, 4096) * 0.5).astype(np.float32)
    b = (rng.standard_t(3, 4096) * 0.5).astype(np.float32)
    # include large/small magnitude pairs where the fp32 sum is inexact
    a[:4] = [32768.0, 1.0, -65504.0, 6e-8]
    b[:4] = [2.0 ** -24, 2.0 ** -24, 65504.0, 6e-8]
    out, lows = oq.fp16_sum([a, b])
    exact = lows[0].astype(np.float64) + lows[1].astype(np.float64)
    np.testing.assert_array_equal(out, exact.astype(np.float16).astype(np.float32))
    # test_quantized_allreduce.py:73-81: close at 1e-2, not exact at 1e-6
    assert np.allclose(out, a + b, atol=1e-2, rtol=1e-2)
    assert not np.allclose(out, a + b, atol=1e-6, rtol=0)


def test_mixer_prefill_activation_rounding_hook():
    """mixer_prefill(act=...): the identity hook reproduces the plain prefill
    bit for bit; a bf16 round leaves out (stored by out_proj) and the conv
    history (the stored in_proj output) exactly bf16-representable, keeps the
    float64 state off the bf16 grid, and moves the result by what bf16
    activations cost: here up to 1.2% of the output's rms, against 2^-9 per
    element for rounding the output alone -- so a bf16-activation path is
    compared with this model of it, not with the unrounded float64 result."""
    from _util import bf16_round
    import _golden as G
    p = G.oracle_mixer_dict(G.mixer_case_weights(7, 32, d_state=8))
    x = np.random.default_rng(8).standard_normal((1, 12, 32))
    o0, c0, h0 = om.mixer_prefill(p, x, dtype=np.float64)
    o1, c1, h1 = om.mixer_prefill(p, x, dtype=np.float64, act=lambda t: t)
    assert np.array_equal(o0, o1) and np.array_equal(c0, c1) and np.array_equal(h0, h1)
    ob, cb, hb = om.mixer_prefill(p, x, dtype=np.float64, act=bf16_round)
    assert np.array_equal(ob, bf16_round(ob)) and np.array_equal(cb, bf16_round(cb))
    assert not np.array_equal(hb, bf16_round(hb))
    rms = np.sqrt(np.mean(o0 ** 2))
    assert 2.0 ** -9 * rms < np.abs(ob - o0).max() < 3e-2 * rms


def _fl32(fr):
    """A Fraction rounded once to the nearest float32 (ties to even), from
    exact rational comparisons -- independent of numpy's float32 division."""
    from fractions import Fraction
    c = np.float32(float(fr))
    cands = [np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))]
    return min(cands, key=lambda v: (abs(Fraction(float(v)) - fr),
                                     int(np.frombuffer(np.float32(v).tobytes(), np.uint32)[0]) & 1))


def test_int8_row_with_a_scale_off_the_power_of_two_grid():
    """amax = 100: s = fl(100 / 127) = 0.7874016, not a power of two.  The
    codes are round-half-even of the correctly rounded fp32 quotient x / s
    (tp_utils.py:111-112), computed here by exact rational arithmetic; for
    these inputs the reciprocal form x * fl(1 / s) rounds to the code below,
    so an oracle slip to it fails."""
    from fractions import Fraction
    row = np.array([[100.0, 0.39370080828666687, 2.7559053897857666, 3.543307304382324, -4.3307085037231445,
                     -100.0]], np.float32)
    s, q = oq.quantize_int8_per_token(row)
    s_exact = _fl32(Fraction(100) / Fraction(127))
    assert s[0] == s_exact and s_exact not in (0.5, 1.0)
    want = [int(np.rint(_fl32(Fraction(float(x)) / Fraction(float(s_exact))))) for x in row[0]]
    assert q[0].tolist() == want == [127, 1, 4, 5, -6, -127]
    inv = np.float32(np.float32(1.0) / s_exact)
    recip = [int(np.rint(np.float32(x * inv))) for x in row[0]]
    assert recip[1:5] == [0, 3, 4, -5]


def test_inv_softplus_inverts_softplus():
    """inv_softplus builds every test's dt_bias: softplus(inv_softplus(y))
    returns y (float64, relative 1e-12) over the dt range [1e-3, 0.1] and
    beyond, and inv_softplus(log 2) = 0 (softplus(0) = log 2)."""
    y = np.exp(np.linspace(np.log(1e-6), np.log(30.0), 400))
    x = om.inv_softplus(y)
    back = np.log1p(np.exp(x))
    np.testing.assert_allclose(back, y, rtol=1e-12)
    lo = y <= 20
    np.testing.assert_allclose(om.softplus(x[lo]), y[lo], rtol=1e-12)
    # above 20 the oracle's softplus is the identity (torch's threshold), which
    # differs from log1p(exp(x)) by under e^-20 relative
    np.testing.assert_allclose(om.softplus(x[~lo]), y[~lo], rtol=np.exp(-20.0))
    assert abs(om.inv_softplus(np.log(2.0))) < 1e-15
    assert np.all(np.diff(x) > 0)                    # increasing, as softplus is
