"""mtl_linear_skinny (the matrix-core GEMM of the batched decode step's
projections, model.py:261, 293, 326) against a float64 reference of
y = x W^T + bias, tolerance 1e-5 relative (to each element plus the output's
rms): row counts 1..64 (one, two and four 16-row MFMA blocks), the mamba-130m and
1.4b projection shapes (and the 130m prefill's at 64 tokens), both workgroup tilings, K ranges of 1, 2, 3 and more
32-column stages per wavefront (every branch of the copy pipeline), weight
row counts that leave a tile partly filled, split K, strided x rows."""
import pytest
import torch

from _util import assert_rel
from mamba_lite import ops

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = 1e-5


def _ref(x, W, bias):
    y = x.double().cpu() @ W.double().cpu().T
    return (y + bias.double().cpu() if bias is not None else y).numpy()


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (5, 3072, 768), (16, 768, 1536), (17, 8192, 2048),
                                   (32, 2048, 4096), (32, 4, 128), (3, 50280, 256), (9, 1000, 384),
                                   (24, 200, 640), (33, 768, 1536), (48, 80, 1536), (64, 3072, 768),
                                   (64, 50280, 768), (64, 4, 128), (57, 1000, 384)])
@pytest.mark.parametrize("rows_per_block", [16, 32])
@pytest.mark.parametrize("with_bias", [False, True])
def test_linear_skinny_vs_float64(M, N, K, rows_per_block, with_bias):
    print(f"\n[linear_skinny M={M} N={N} K={K} rpb={rows_per_block} bias={with_bias}]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(M * 7 + N + K)
    x = torch.randn(M, K, device=DEV, generator=g)
    W = torch.randn(N, K, device=DEV, generator=g) / K ** 0.5
    bias = torch.randn(N, device=DEV, generator=g) if with_bias else None
    y = ops.linear_skinny(x, W, bias, rows_per_block=rows_per_block)
    assert_rel(y.cpu().numpy(), _ref(x, W, bias), TOL, "y")


@pytest.mark.parametrize("ksplit", [2, 4])
def test_linear_skinny_split_k_parts_add_up(ksplit):
    """Split-K parts: part s is the product over the s-th K range (bias in
    part 0), so their ordered sum is the full product."""
    print(f"\n[linear_skinny split K={ksplit}]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(ksplit)
    M, N, K = 32, 2048, 4096
    x = torch.randn(M, K, device=DEV, generator=g)
    W = torch.randn(N, K, device=DEV, generator=g) / K ** 0.5
    bias = torch.randn(N, device=DEV, generator=g)
    parts = ops.linear_skinny(x, W, bias, ksplit=ksplit)
    assert parts.shape == (ksplit, M, N)
    kc = K // ksplit
    for s in range(ksplit):
        ref = (x[:, s * kc:(s + 1) * kc].double().cpu() @ W[:, s * kc:(s + 1) * kc].double().cpu().T)
        if s == 0:
            ref = ref + bias.double().cpu()
        assert_rel(parts[s].cpu().numpy(), ref.numpy(), TOL, f"part {s}")
    assert_rel(ops.sum_parts(parts).cpu().numpy(), _ref(x, W, bias), TOL, "sum")


def test_linear_skinny_strided_rows_and_repeatability():
    """x as a row-strided view (the z half of an in_proj output, say) and two
    calls giving identical bits."""
    g = torch.Generator(device=DEV).manual_seed(3)
    base = torch.randn(20, 2 * 1536, device=DEV, generator=g)
    x = base[:, 1536:]
    W = torch.randn(768, 1536, device=DEV, generator=g)
    y1 = ops.linear_skinny(x, W)
    y2 = ops.linear_skinny(x, W)
    assert torch.equal(y1, y2)
    assert_rel(y1.cpu().numpy(), _ref(x, W, None), TOL, "y")
