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


@pytest.mark.parametrize("P,rows,J,R,D", [(12, 64, 80, 48, 1536), (4, 37, 160, 128, 4096), (1, 5, 36, 4, 128),
                                          (16, 64, 192, 160, 5120), (3, 17, 50, 7, 100)])
def test_xproj_sum_dt_vs_float64(P, rows, J, R, D):
    """mtl_xproj_sum_dt (x_proj's split-K parts summed, dt_proj on the sum,
    one launch): x_dbl bit for bit against mtl_sum_parts (same part order),
    dt against float64 at 1e-5; the mamba-130m, 1.4b and 2.8b widths, a
    single part, ragged row and channel counts."""
    print(f"\n[xproj_sum_dt P={P} rows={rows} J={J} R={R} D={D}]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(P * 31 + rows + D)
    parts = torch.randn(P, rows, J, device=DEV, generator=g)
    W_dt = torch.randn(D, R, device=DEV, generator=g) / R ** 0.5
    x_dbl, dt = ops.xproj_sum_dt(parts, W_dt)
    ref_x = ops.sum_parts(parts) if P > 1 else parts[0]
    assert torch.equal(x_dbl, ref_x)
    ref_dt = parts.double().sum(0)[:, :R].cpu() @ W_dt.double().cpu().T
    assert_rel(dt.cpu().numpy(), ref_dt.numpy(), TOL, "dt")
    if P == 1:
        x1, dt1 = ops.xproj_sum_dt(parts, W_dt, write_x_dbl=False)
        assert x1.data_ptr() == parts.data_ptr() and torch.equal(dt1, dt)


@pytest.mark.parametrize("M,N,K,ks", [(65, 3072, 768, 1), (128, 768, 1536, 4), (200, 80, 1536, 12),
                                      (256, 8192, 2048, 1), (129, 2048, 4096, 4), (300, 160, 4096, 16),
                                      (64 * 9 + 5, 1000, 384, 3)])
@pytest.mark.parametrize("rows_per_block", [16, 32])
def test_linear_skinny_row_chunks(M, N, K, ks, rows_per_block):
    """Past 64 rows of x the rows run as 64-row chunks of one launch: each
    chunk's outputs (every split-K part, bias in part 0) equal a launch over
    that chunk's rows alone bit for bit, and the whole is within 1e-5 of the
    float64 product.  x rows strided (a view of a wider tensor)."""
    print(f"\n[linear_skinny chunks M={M} N={N} K={K} ksplit={ks} rpb={rows_per_block}]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(M + N + K + ks)
    x = torch.randn(M, K + 64, device=DEV, generator=g)[:, 8:8 + K]
    W = torch.randn(N, K, device=DEV, generator=g) / K ** 0.5
    bias = torch.randn(N, device=DEV, generator=g)
    y = ops.linear_skinny(x, W, bias, ksplit=ks, rows_per_block=rows_per_block)
    parts = y.view(ks, M, N)
    for r0 in range(0, M, 64):
        xc = x[r0:r0 + 64]
        rpb = rows_per_block if xc.shape[0] > 32 else 16   # 32-row tiles at <= 32 rows pick other MFMA blocks
        alone = ops.linear_skinny(xc, W, bias, ksplit=ks, rows_per_block=rpb).view(ks, xc.shape[0], N)
        if xc.shape[0] > 32:
            assert torch.equal(parts[:, r0:r0 + 64], alone), f"chunk at row {r0}"
        else:
            assert_rel(parts[:, r0:r0 + 64].cpu().numpy(), alone.cpu().numpy(), TOL, f"chunk at row {r0}")
    full = ops.sum_parts(parts) if ks > 1 else y
    assert_rel(full.cpu().numpy(), _ref(x, W, bias), TOL, "y")
