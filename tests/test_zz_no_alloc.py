"""mtl_conv_step_xproj_noalloc (the allocation-free batched step) against
mtl_conv_step_xproj + mtl_sum_parts, through the C ABI: the conv output,
the shifted conv history and x_dbl bit for bit, on two calls in a row (the
second smaller, so it runs on what the first left in the library's scratch
array)."""
import ctypes

import numpy as np
import pytest
import torch

from mamba_lite import _lib, ops

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(rng, b, D, J, K):
    f = lambda *s: torch.from_numpy(rng.standard_normal(s).astype(np.float32)).to(DEV)
    return dict(state=f(b, D, K - 1), x=f(b, D), w=f(D, K) * 0.5, bias=f(D), WxT=f(D, J) * (D ** -0.5))


def _existing(c):
    state = c["state"].clone()
    xc, xpart = ops.conv_step_xproj(state, c["x"], c["w"], c["bias"], c["WxT"])
    return state, xc, ops.sum_parts(xpart)


def _noalloc(c):
    lib = _lib.load()
    b, D = c["x"].shape
    K, J = c["w"].shape[1], c["WxT"].shape[1]
    state = c["state"].clone()
    xc = torch.full((b, D), float("nan"), device=DEV)
    x_dbl = torch.full((b, J), float("nan"), device=DEV)
    rc = lib.mtl_conv_step_xproj_noalloc(state.data_ptr(), c["x"].data_ptr(), D, c["w"].data_ptr(),
                                         c["bias"].data_ptr(), xc.data_ptr(), D, c["WxT"].data_ptr(),
                                         x_dbl.data_ptr(), b, D, K, J, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "conv_step_xproj_noalloc")
    return state, xc, x_dbl


@pytest.mark.parametrize("shapes", [[(32, 4096, 160, 4), (4, 1536, 80, 4)],
                                    [(8, 5120, 192, 4), (1, 96, 36, 2)]])
def test_noalloc_matches_caller_buffer_entry_point(shapes):
    rng = np.random.default_rng(7)
    for b, D, J, K in shapes:
        print(f"\n[noalloc b={b} D={D} J={J} K={K}]", flush=True)
        c = _case(rng, b, D, J, K)
        s1, xc1, xd1 = _existing(c)
        s2, xc2, xd2 = _noalloc(c)
        torch.cuda.synchronize()
        assert torch.equal(xc1, xc2), "conv output"
        assert torch.equal(s1, s2), "conv history"
        assert torch.equal(xd1, xd2), "x_dbl"


def test_noalloc_on_a_side_stream_takes_that_streams_device():
    """A non-null stream: the scratch is looked up from the stream's device."""
    rng = np.random.default_rng(8)
    c = _case(rng, 4, 2048, 160, 4)
    s1, xc1, xd1 = _existing(c)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        print("\n[noalloc on a side stream b=4 D=2048 J=160]", flush=True)
        s2, xc2, xd2 = _noalloc(c)
    side.synchronize()
    assert torch.equal(xc1, xc2) and torch.equal(s1, s2) and torch.equal(xd1, xd2)


def test_noalloc_rejects_sizes_beyond_its_scratch():
    lib = _lib.load()
    P = ctypes.c_void_p(256)     # never dereferenced: the size check comes first
    rc = lib.mtl_conv_step_xproj_noalloc(P, P, 8192, P, None, P, 8192, P, P, 32, 8192, 4, 288, None)
    assert rc == 1 and b"scratch" in lib.mtl_last_error()
