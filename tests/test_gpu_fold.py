"""The batched step's residual add and RMSNorm folded into its projections
(mtl_linear_skinny_residual, mtl_in_proj_conv_xproj_normed), on the GPU:

  * the out_proj launch's parts are linear_skinny's bit for bit, its residual
    h equals mtl_add_rmsnorm_parts' x_out bit for bit, x_next = h * w equals
    torch's product bit for bit, and the per-tile sums of h^2 are within 1e-6
    of a float64 sum; each counter ends at the split count;
  * the normed in_proj (the norm applied to the dot products) is within 1e-5
    of the plain in_proj on mtl_add_rmsnorm's output (xc, z, the x_proj
    partials, the conv history);
  * MambaLM.step on the folded path against the float64 oracle (1e-4, the
    fp32 tolerance) and against the per-op step without the fold (1e-5), at
    b = 3, 8, 17 and 32, widths 256, 768 and 2048 (mamba-1.4b), with and
    without projection biases; graph replays equal eager bit for bit.
(model.py:130-135, 261-293, 303-311, 343-353)"""
import numpy as np
import pytest
import torch

import _golden as G
from _util import assert_rel
from mamba_lite import ops
from mamba_lite.cuda_graph import GraphedStepper
from mamba_lite.model import MambaConfig, MambaLM
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _n(t):
    return t.detach().double().cpu().numpy()


@pytest.mark.parametrize("M,N,K,ks", [(32, 2048, 4096, 4), (8, 768, 1536, 4), (17, 256, 512, 4), (3, 512, 1024, 2),
                                      (32, 256, 512, 1), (1, 128, 128, 1), (20, 1024, 2048, 4), (32, 768, 1536, 4)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_residual_out_proj_matches_parts_and_residual_add(M, N, K, ks, with_bias):
    print(f"\n[fold: out_proj residual M={M} N={N} K={K} ksplit={ks} bias={with_bias}]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(M * 131 + N + ks)
    y = torch.randn(M, K, device=DEV, generator=g)
    W = torch.randn(N, K, device=DEV, generator=g) / K ** 0.5
    bias = torch.randn(N, device=DEV, generator=g) if with_bias else None
    h = 2.0 * torch.randn(M, N, device=DEV, generator=g)
    w = 1.0 + 0.2 * torch.randn(N, device=DEV, generator=g)
    rpb = ops.residual_rows_per_block(M, N, ks)
    tiles = N // rpb
    parts_ref = ops.linear_skinny(y, W, bias, ksplit=ks, rows_per_block=rpb).view(ks, M, N)
    h_ref = h.clone()
    ops.add_rmsnorm(h_ref, w, 1e-5, y_parts=parts_ref, x_out=h_ref)

    hh, xn = h.clone(), torch.empty_like(h)
    sq = torch.empty(tiles, M, device=DEV)
    cnt = torch.zeros(tiles, device=DEV, dtype=torch.int32)
    parts = torch.empty(ks, M, N, device=DEV)
    ops.linear_skinny_residual(y, W, bias, hh, w, xn, sq, cnt, ks, rpb, parts)
    torch.cuda.synchronize()
    assert torch.equal(parts, parts_ref), "parts differ from linear_skinny's"
    assert torch.equal(hh, h_ref), "residual differs from add_rmsnorm_parts' x_out"
    assert torch.equal(xn, hh * w), "x_next differs from h * w"
    ref_sq = (_n(hh) ** 2).reshape(M, tiles, rpb).sum(-1).T
    assert_rel(_n(sq), ref_sq, 1e-6, "sq")
    assert (cnt == ks).all()


@pytest.mark.parametrize("b,d_model,d_inner,J", [(32, 2048, 4096, 160), (8, 768, 1536, 80), (17, 256, 512, 48),
                                                 (3, 256, 512, 40), (32, 768, 1536, 80)])
def test_normed_in_proj_matches_in_proj_of_the_norm(b, d_model, d_inner, J):
    print(f"\n[fold: normed in_proj b={b} d_model={d_model} d_inner={d_inner} J={J}]", flush=True)
    g = torch.Generator(device=DEV).manual_seed(b * 7 + d_model + J)
    eps = 1e-5
    h = 3.0 * torch.randn(b, d_model, device=DEV, generator=g)
    w = 1.0 + 0.2 * torch.randn(d_model, device=DEV, generator=g)
    normed = ops.add_rmsnorm(h.clone(), w, eps)
    rpb = ops.residual_rows_per_block(b, d_model, 4)
    tiles = d_model // rpb
    sq = (h.double() ** 2).view(b, tiles, rpb).sum(-1).t().float().contiguous()
    xn = h * w
    W_in = torch.randn(2 * d_inner, d_model, device=DEV, generator=g) / d_model ** 0.5
    b_in = 0.1 * torch.randn(2 * d_inner, device=DEV, generator=g)
    conv_w = 0.5 * torch.randn(d_inner, 4, device=DEV, generator=g)
    conv_b = 0.1 * torch.randn(d_inner, device=DEV, generator=g)
    W_xT = torch.randn(d_inner, J, device=DEV, generator=g) / d_inner ** 0.5
    cs0 = torch.randn(b, d_inner, 3, device=DEV, generator=g)
    cs_a, cs_b = cs0.clone(), cs0.clone()
    xc_a, z_a, xp_a = ops.in_proj_conv_xproj(normed, W_in, b_in, cs_a, conv_w, conv_b, W_xT)
    xc_b, z_b, xp_b = ops.in_proj_conv_xproj(xn, W_in, b_in, cs_b, conv_w, conv_b, W_xT, sq=sq, eps=eps)
    torch.cuda.synchronize()
    assert_rel(_n(xc_b), _n(xc_a), 1e-5, "xc")
    assert_rel(_n(z_b), _n(z_a), 1e-5, "z")
    assert_rel(_n(xp_b), _n(xp_a), 1e-5, "xpart")
    assert_rel(_n(cs_b), _n(cs_a), 1e-5, "conv_state")


def _lm(seed, d_model, n_layer, vocab, **kw):
    sd = G.lm_weights(seed, d_model, n_layer, vocab, **kw)
    lm = MambaLM(MambaConfig(d_model=d_model, n_layer=n_layer, vocab_size=vocab, **kw))
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    return lm.to(DEV).eval(), G.oracle_lm_dict(sd, n_layer)


@pytest.mark.parametrize("b,d_model,n_layer,kw", [
    (3, 256, 3, {}), (8, 256, 3, dict(bias=True)), (17, 256, 2, {}), (32, 256, 4, dict(bias=True)),
    (32, 768, 2, {}), (32, 2048, 2, dict(dt_rank=128)), (12, 2048, 2, dict(dt_rank=128))])
def test_folded_step_vs_oracle_and_unfolded(b, d_model, n_layer, kw, monkeypatch):
    """Past 16 rows the model keeps the add + norm launch (faster in graphs
    there); the limit is raised so the folded kernels are checked up to 32."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "STEP_NORM_FOLD_MAX_ROWS", 32)
    monkeypatch.setattr(mm, "BATCHED_STEP_NATIVE", False)     # the Python launches, counted below
    print(f"\n[fold: lm step b={b} d_model={d_model} layers={n_layer} {kw}]", flush=True)
    vocab = 512
    lm, W = _lm(60 + b + d_model, d_model, n_layer, vocab, **kw)
    calls = []
    real = ops.linear_skinny_residual
    monkeypatch.setattr(ops, "linear_skinny_residual", lambda *a, **k: calls.append(1) or real(*a, **k))
    rng = np.random.default_rng(b * 3 + d_model)
    plen, steps = 6, 3
    ids = rng.integers(0, vocab, (b, plen + steps), dtype=np.int64)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    with torch.no_grad():
        _, c_fold = lm.prefill(t(ids[:, :plen]))
        _, c_plain = lm.prefill(t(ids[:, :plen]))
        _, rcache = om.lm_prefill(W, ids[:, :plen], dtype=np.float64)
        for k in range(steps):
            s = ids[:, plen + k:plen + k + 1]
            got = lm.step(t(s), c_fold)
            monkeypatch.setattr(mm, "STEP_NORM_FOLD", False)
            plain = lm.step(t(s), c_plain)
            monkeypatch.setattr(mm, "STEP_NORM_FOLD", True)
            ref = om.lm_step(W, s, rcache, dtype=np.float64)
            assert_rel(_n(got), ref, 1e-4, f"step {k} logits vs oracle")
            assert_rel(_n(got), _n(plain), 1e-5, f"step {k} logits vs unfolded")
        for i, (lf, lp, (rc, rh)) in enumerate(zip(c_fold.layers, c_plain.layers, rcache)):
            assert_rel(_n(lf.conv_state), rc, 1e-4, f"layer {i} conv_state")
            assert_rel(_n(lf.ssm_state), rh, 1e-4, f"layer {i} ssm_state")
            assert_rel(_n(lf.ssm_state), _n(lp.ssm_state), 1e-5, f"layer {i} ssm_state vs unfolded")
    assert len(calls) == steps * (n_layer - 1), len(calls)


def test_fold_row_limit():
    """The default takes the fold up to 16 rows and the add + norm launch past
    them, eager and captured alike."""
    import mamba_lite.model as mm
    lm, _ = _lm(80, 256, 2, 512)
    for b, want in ((3, True), (16, True), (17, False), (32, False)):
        ids = torch.zeros(b, 4, dtype=torch.long, device=DEV)
        with torch.no_grad():
            _, cache = lm.prefill(ids)
            x = lm.embedding(ids[:, :1]).squeeze(1)
        assert lm._fold_ok(x, cache) == want, b
    assert mm.STEP_NORM_FOLD_MAX_ROWS == 16


@pytest.mark.parametrize("b", [8, 32])
def test_folded_step_graph_replays_equal_eager(b, monkeypatch):
    """Each replay zeroes its own counters (a fill kernel in the graph), so
    every replay, with eager work between them, equals the eager step."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "STEP_NORM_FOLD_MAX_ROWS", 32)
    print(f"\n[fold: graph replay b={b}]", flush=True)
    lm, _ = _lm(70 + b, 256, 3, 512, bias=True)
    rng = np.random.default_rng(b)
    ids = torch.from_numpy(rng.integers(0, 512, (b, 6), dtype=np.int64)).to(DEV)
    steps = [torch.from_numpy(rng.integers(0, 512, (b, 1), dtype=np.int64)).to(DEV) for _ in range(4)]
    with torch.no_grad():
        x = lm.embedding(steps[0]).squeeze(1)
        _, cache_e = lm.prefill(ids)
        assert lm._fold_ok(x, cache_e)
        eager = [lm.step(s, cache_e).clone() for s in steps]
        _, cache_g = lm.prefill(ids)
        st = GraphedStepper(lm, cache_g, b, "cuda")
        st.capture()
        for i, s in enumerate(steps):
            got = st.replay(s).clone()
            torch.cuda.synchronize()
            _ = lm.prefill(ids[:, :3])            # unrelated eager work between replays
            assert torch.equal(got, eager[i]), f"replay {i} differs"
    for le, lg in zip(cache_e.layers, cache_g.layers):
        assert torch.equal(le.ssm_state, lg.ssm_state) and torch.equal(le.conv_state, lg.conv_state)
