"""Payload quantizer kernels vs the oracle, on the GPU: int8 codes, per-token
scales, payload bytes and the dequantize-sum output are BIT-EXACT; the fp16
cast-sum output is bit-exact too."""
import numpy as np
import pytest
import torch

from mamba_lite import ops, tp_utils
from oracle import quant as oq

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _student(rng, shape):
    return (rng.standard_t(3, shape) * 0.5).astype(np.float32)


@pytest.mark.parametrize("rows,cols", [(1024, 768), (1000, 80), (33, 160), (5, 2048), (3, 4097), (17, 1),
                                       (7, 1028), (9, 12), (4, 770)])
@pytest.mark.parametrize("nparts", [2, 1, 3])
def test_int8_tok_bit_exact(rows, cols, nparts):
    rng = np.random.default_rng(rows * 7 + cols + nparts)
    parts = [_student(rng, (rows, cols)) for _ in range(nparts)]
    out, pays = ops.quant_dequant_sum_int8_tok([torch.from_numpy(p).to(DEV) for p in parts])
    ref_out, ref_pays = oq.quant_dequant_sum_int8_tok(parts)
    for r in range(nparts):
        assert np.array_equal(pays[r].cpu().numpy(), ref_pays[r]), f"payload {r} differs"
    assert np.array_equal(out.cpu().numpy(), ref_out), "dequantized sum differs"


def test_int8_edge_rows():
    rows = np.zeros((6, 64), np.float32)
    rows[1, :9] = [2.5, 3.5, -2.5, -0.5, 0.5, 1.5, 127.0, -127.0, 126.5]   # scale exactly 1: ties to even
    rows[2, 5] = -3.0e-12                                                  # tiny: clamps to the 1e-8 floor
    rows[3] = np.linspace(-1e30, 1e30, 64, dtype=np.float32)              # huge magnitudes
    rows[4, ::2] = 7.0                                                     # exact +-amax -> +-127
    rows[4, 1::2] = -7.0
    rows[5] = np.float32(1e-38) * np.arange(64, dtype=np.float32)         # subnormal-range values
    b = np.flip(rows, 0).copy()
    out, pays = ops.quant_dequant_sum_int8_tok([torch.from_numpy(rows).to(DEV), torch.from_numpy(b).to(DEV)])
    ref_out, ref_pays = oq.quant_dequant_sum_int8_tok([rows, b])
    for r in range(2):
        assert np.array_equal(pays[r].cpu().numpy(), ref_pays[r])
    assert np.array_equal(out.cpu().numpy(), ref_out)
    s, q = oq.unpack_payload(pays[0].cpu().numpy(), 6, 64)
    assert q[1, :9].tolist() == [2, 4, -2, 0, 0, 2, 127, -127, 126]
    assert (np.abs(q[4]) == 127).all()


def _full_parts():
    """The payload workload: two [32*1024, 768] fp32 partials drawn
    Student-t(3) * 0.5 (heavy tails: the per-token scale varies widely)."""
    rng = np.random.default_rng(2024)
    return [_student(rng, (32 * 1024, 768)) for _ in range(2)]


def test_int8_full_payload_shape():
    """Every code, scale and output of the full workload, bit for bit."""
    print("\n[int8 payload 2 x [32768, 768] Student-t]", flush=True)
    parts = _full_parts()
    rows, cols = parts[0].shape
    out, pays = ops.quant_dequant_sum_int8_tok([torch.from_numpy(p).to(DEV) for p in parts])
    assert pays[0].numel() == tp_utils.int8_tok_payload_nbytes(rows, cols) == 25_296_896
    ref_out, ref_pays = oq.quant_dequant_sum_int8_tok(parts)
    for r in range(2):
        assert np.array_equal(pays[r].cpu().numpy(), ref_pays[r]), f"payload {r} differs"
    got = out.cpu().numpy()
    assert np.array_equal(got, ref_out), "dequantized sum differs"
    dense = parts[0] + parts[1]
    assert np.abs(got - dense).max() < 0.15 * np.abs(dense).max()


def test_fp16_full_payload_shape():
    print("\n[fp16 payload 2 x [32768, 768] Student-t]", flush=True)
    parts = _full_parts()
    out, pays = ops.quant_dequant_sum_fp16([torch.from_numpy(p.reshape(-1)).to(DEV) for p in parts],
                                           return_payloads=True)
    ref_out, ref_lows = oq.fp16_sum([p.reshape(-1) for p in parts])
    for r in range(2):
        assert np.array_equal(pays[r].cpu().numpy().view(np.uint16), ref_lows[r].view(np.uint16))
    assert np.array_equal(out.cpu().numpy(), ref_out)


@pytest.mark.parametrize("cols", [768, 770, 4097])
def test_int8_nan_row_propagates(cols):
    """A NaN in a row makes that row's scale NaN and its outputs NaN, as
    torch's amax and clamp do in the reference (tp_utils.py:111); its codes
    are 0, as numpy's and torch's CPU float -> int8 conversions turn NaN (the
    oracle's codes); the other rows stay bit-exact."""
    rng = np.random.default_rng(cols)
    parts = [_student(rng, (6, cols)) for _ in range(2)]
    parts[0][2, 5] = np.nan
    out, pays = ops.quant_dequant_sum_int8_tok([torch.from_numpy(p).to(DEV) for p in parts])
    got = out.cpu().numpy()
    s0, _ = oq.unpack_payload(pays[0].cpu().numpy(), 6, cols)
    s1, _ = oq.unpack_payload(pays[1].cpu().numpy(), 6, cols)
    assert np.isnan(s0[2]) and not np.isnan(s1[2])
    assert np.isnan(got[2]).all()
    keep = [0, 1, 3, 4, 5]
    with np.errstate(invalid="ignore"):
        ref_out, ref_pays = oq.quant_dequant_sum_int8_tok([p[keep] for p in parts])
    assert np.array_equal(got[keep], ref_out)
    rs, rq = oq.unpack_payload(ref_pays[0], 5, cols)
    g_s, g_q = oq.unpack_payload(pays[0].cpu().numpy(), 6, cols)
    assert np.array_equal(g_s[keep], rs) and np.array_equal(g_q[keep], rq)
    with np.errstate(invalid="ignore"):
        _, nan_codes = oq.quantize_int8_per_token(parts[0][2:3])
    assert (nan_codes == 0).all() and (g_q[2] == 0).all()


@pytest.mark.parametrize("cols", [768, 13])
def test_int8_inf_row_gives_an_infinite_scale_and_nan_outputs(cols):
    """An inf in a row: the reference's absmax is inf, so its scale is inf
    (tp_utils.py:111-112), every finite element quantizes to 0 and the inf
    element's quotient inf / inf is NaN, kept by torch.clamp and converted to
    int8 as 0; every output of the row is 0 * inf = NaN.  The same here:
    codes all 0, as the oracle's, scale inf, outputs NaN; the other rows stay
    bit-exact."""
    rng = np.random.default_rng(100 + cols)
    parts = [_student(rng, (6, cols)) for _ in range(2)]
    parts[1][4, 3] = -np.inf
    out, pays = ops.quant_dequant_sum_int8_tok([torch.from_numpy(p).to(DEV) for p in parts])
    got = out.cpu().numpy()
    s1, q1 = oq.unpack_payload(pays[1].cpu().numpy(), 6, cols)
    assert np.isposinf(s1[4])
    with np.errstate(invalid="ignore"):
        ref_s, ref_q = oq.quantize_int8_per_token(parts[1][4:5])
    assert np.isposinf(ref_s[0]) and (ref_q == 0).all() and (q1[4] == 0).all()
    assert np.isnan(got[4]).all()
    keep = [0, 1, 2, 3, 5]
    ref_out, ref_pays = oq.quant_dequant_sum_int8_tok([p[keep] for p in parts])
    assert np.array_equal(got[keep], ref_out)
    rs, rq = oq.unpack_payload(ref_pays[1], 5, cols)
    assert np.array_equal(s1[keep], rs) and np.array_equal(q1[keep], rq)


@pytest.mark.parametrize("n", [1, 1000, 65536 + 3, 4096])
@pytest.mark.parametrize("nparts", [1, 2, 3, 8])
def test_fp16_bit_exact(n, nparts):
    """n % 4 == 0 takes the 4-wide path, other n the scalar one."""
    rng = np.random.default_rng(n + nparts)
    parts = [_student(rng, (n,)) for _ in range(nparts)]
    if n >= 4 and nparts >= 2:
        parts[0][:4] = [32768.0, 1.0, -65504.0, 70000.0]
        parts[1][:4] = [2.0 ** -24, 2.0 ** -24, 65504.0, 1.0]
    out, pays = ops.quant_dequant_sum_fp16([torch.from_numpy(p).to(DEV) for p in parts], return_payloads=True)
    ref_out, ref_lows = oq.fp16_sum(parts)
    for r in range(nparts):
        assert np.array_equal(pays[r].cpu().numpy().view(np.uint16), ref_lows[r].view(np.uint16))
    assert np.array_equal(out.cpu().numpy(), ref_out)


def test_fp16_without_payloads_matches():
    rng = np.random.default_rng(77)
    parts = [_student(rng, (4096,)) for _ in range(2)]
    out, pays = ops.quant_dequant_sum_fp16([torch.from_numpy(p).to(DEV) for p in parts], return_payloads=False)
    assert pays is None
    ref_out, _ = oq.fp16_sum(parts)
    assert np.array_equal(out.cpu().numpy(), ref_out)


def test_tp_utils_wrappers_count_bytes():
    c = tp_utils.CommCounter()
    a = torch.randn(10, 80, device=DEV)
    b = torch.randn(10, 80, device=DEV)
    tp_utils.quant_dequant_sum_int8_tok([a, b], counter=c)
    tp_utils.quant_dequant_sum_fp16([a, b], counter=c)
    assert c.count == 2 and c.bytes == 10 * 84 + 10 * 80 * 2


def test_zero_rows_are_a_no_op():
    a = torch.empty(0, 768, device=DEV)
    out, pays = ops.quant_dequant_sum_int8_tok([a, a.clone()], return_payloads=True)
    assert out.shape == (0, 768)
    out16, _ = ops.quant_dequant_sum_fp16([a, a.clone()])
    assert out16.shape == (0, 768)
    torch.cuda.synchronize()
