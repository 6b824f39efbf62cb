"""Fused decode step (mtl_decode_in / mtl_decode_gemv / mtl_decode_ssm) on
the GPU: against the per-op step path and the oracle, at the 130m width
(d_model 768: register-blocked rows, x_proj as split-K partials) and the
1.4b width (d_model 2048: x_proj as its own row GEMV), batch 1, 2 and 4.
fp32 within 1e-4 relative; the in-place cache and graph replay checks are
bit-exact."""
import numpy as np
import pytest
import torch

from _util import assert_rel
from mamba_lite import ops
from mamba_lite.cuda_graph import GraphedStepper
from mamba_lite.model import MambaConfig, MambaLM, MambaMixer
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _fused_up_to_batch_4(monkeypatch):
    """The fused kernels take 1, 2 or 4 rows; MambaLM.step sends batch 4 to
    the per-op path by default (faster there), so these tests raise the
    limit to keep the fused path covered at batch 4."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "FUSED_STEP_MAX_BATCH", 4)


def _np(t):
    return t.detach().float().cpu().numpy()


def _model(d_model, n_layer, vocab, seed):
    torch.manual_seed(seed)
    cfg = MambaConfig(d_model=d_model, n_layer=n_layer, vocab_size=vocab, d_state=16)
    with torch.device(DEV):
        m = MambaLM(cfg)
    rng = np.random.default_rng(seed)
    with torch.no_grad():
        for mx in m.modules():
            if isinstance(mx, MambaMixer):
                D = mx.dt_proj.bias.shape[0]
                mx.dt_proj.bias.copy_(torch.from_numpy(
                    om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32)))
    return m.eval()


def _per_op_step(model, ids, cache):
    """The unfused step: GEMMs + conv-step and SSM-update kernels."""
    x = model.embedding(ids).squeeze(1)
    xf = model._run(x, lambda i, xn: model.layers[i].mixer.step(xn, cache.layers[i]))
    return model.lm_head(xf).unsqueeze(1)


@pytest.mark.parametrize("d_model,split_max_b", [(768, 1), (2048, 0), (64, 4)])
@pytest.mark.parametrize("b", [1, 2, 4])
def test_fused_step_matches_per_op_step(d_model, split_max_b, b):
    """split_max_b: the largest batch whose x_proj runs as split-K partials
    (1 at the 130m width, never at the 1.4b width)."""
    print(f"fused decode d_model={d_model} b={b}", flush=True)
    model = _model(d_model, 2, 512, seed=d_model + b)
    assert model._decode_plan()["split_k_max_b"] == split_max_b
    ids = torch.randint(0, 512, (b, 6), device=DEV)
    with torch.no_grad():
        _, c1 = model.prefill(ids)
        _, c2 = model.prefill(ids)
        assert model._fused_step_ok(ids[:, :1], c1)
        ptrs = [(l.conv_state.data_ptr(), l.ssm_state.data_ptr()) for l in c1.layers]
        for t in range(3):
            nxt = torch.randint(0, 512, (b, 1), device=DEV)
            got = model.step(nxt, c1)
            ref = _per_op_step(model, nxt, c2)
            assert_rel(_np(got), _np(ref), 1e-4, f"logits step {t}")
        for l1, l2 in zip(c1.layers, c2.layers):
            assert_rel(_np(l1.ssm_state), _np(l2.ssm_state), 1e-4, "ssm_state")
            assert_rel(_np(l1.conv_state), _np(l2.conv_state), 1e-5, "conv_state")
        assert ptrs == [(l.conv_state.data_ptr(), l.ssm_state.data_ptr()) for l in c1.layers]


def test_fused_step_vs_oracle():
    model = _model(768, 2, 256, seed=11)
    W = {"embedding": _np(model.embedding.weight), "norm_f": _np(model.norm_f.weight), "layers": []}
    for blk in model.layers:
        m = blk.mixer
        W["layers"].append({"norm": _np(blk.norm.weight), "in_proj_w": _np(m.in_proj.weight),
                            "conv_w": _np(m.conv1d.weight)[:, 0, :], "conv_b": _np(m.conv1d.bias),
                            "x_proj_w": _np(m.x_proj.weight), "dt_proj_w": _np(m.dt_proj.weight),
                            "dt_proj_b": _np(m.dt_proj.bias), "A_log": _np(m.A_log), "D": _np(m.D),
                            "out_proj_w": _np(m.out_proj.weight)})
    ids = torch.randint(0, 256, (1, 5), device=DEV)
    with torch.no_grad():
        _, cache = model.prefill(ids[:, :4])
        got = model.step(ids[:, 4:5], cache)
    _, rc = om.lm_prefill(W, ids[:, :4].cpu().numpy(), dtype=np.float64)
    ref = om.lm_step(W, ids[:, 4:5].cpu().numpy(), rc, dtype=np.float64)
    assert_rel(_np(got), ref, 1e-4, "fused step vs oracle")


def test_fused_step_graph_replay_bit_identical():
    model = _model(768, 3, 1024, seed=5)
    ids = torch.randint(0, 1024, (1, 8), device=DEV)
    steps = [torch.randint(0, 1024, (1, 1), device=DEV) for _ in range(4)]
    with torch.no_grad():
        _, ce = model.prefill(ids)
        eager = [model.step(s, ce).clone() for s in steps]
        _, cg = model.prefill(ids)
        st = GraphedStepper(model, cg, 1, "cuda")
        st.capture()
        for i, s in enumerate(steps):
            g = st.replay(s).clone()
            torch.cuda.synchronize()
            assert torch.equal(g, eager[i]), f"replay {i}"
    for a, b in zip(ce.layers, cg.layers):
        assert torch.equal(a.ssm_state, b.ssm_state) and torch.equal(a.conv_state, b.conv_state)


def test_plan_refreshes_after_weight_change():
    model = _model(64, 1, 128, seed=3)
    ids = torch.randint(0, 128, (1, 3), device=DEV)
    with torch.no_grad():
        _, c1 = model.prefill(ids)
        model.step(ids[:, :1], c1)
        p1 = model._decode_plan()
        model.layers[0].mixer.x_proj.weight.mul_(0.5)
        p2 = model._decode_plan()
        assert p2 is not p1
        assert torch.equal(p2["layers"][0]["W_xT"], model.layers[0].mixer.x_proj.weight.t().contiguous())


def test_graph_replay_refuses_stale_weights():
    """The captured step reads copies derived from the weights (the fused
    plan); after an in-place weight update a replay raises instead of using
    them, and a new capture serves the updated weights."""
    model = _model(64, 1, 128, seed=4)
    ids = torch.randint(0, 128, (1, 4), device=DEV)
    tok = torch.randint(0, 128, (1, 1), device=DEV)
    with torch.no_grad():
        _, cg = model.prefill(ids)
        st = GraphedStepper(model, cg, 1, "cuda")
        st.capture()
        st.replay(tok)
        model.layers[0].mixer.x_proj.weight.mul_(0.5)
        with pytest.raises(RuntimeError, match="capture again"):
            st.replay(tok)
        _, ce = model.prefill(ids)
        _, cg = model.prefill(ids)
        st = GraphedStepper(model, cg, 1, "cuda")
        st.capture()
        g = st.replay(tok).clone()
        e = model.step(tok, ce)
        torch.cuda.synchronize()
        assert torch.equal(g, e)


@pytest.mark.parametrize("b", [1, 2, 4])
def test_fused_step_out_of_range_id_gives_nan_row(b):
    """An id outside [0, vocab) reads no memory outside the embedding: that
    batch row's logits are NaN, the other rows are unaffected."""
    model = _model(64, 2, 128, seed=6)
    ids = torch.randint(0, 128, (b, 4), device=DEV)
    tok = torch.randint(0, 128, (b, 1), device=DEV)
    bad = tok.clone()
    bad[b - 1, 0] = 128 if b != 2 else -1
    with torch.no_grad():
        _, c1 = model.prefill(ids)
        _, c2 = model.prefill(ids)
        assert model._fused_step_ok(tok, c1)
        good = model.step(tok, c1)
        got = model.step(bad, c2)
    assert torch.isnan(got[b - 1]).all()
    if b > 1:
        assert torch.equal(got[:b - 1], good[:b - 1])


@pytest.mark.parametrize("kw", [dict(d_state=8, d_conv=3, bias=True, conv_bias=False),
                                dict(d_state=4, d_conv=2, dt_rank=5),
                                dict(d_state=16, d_conv=8, bias=True),
                                dict(d_state=16, dt_rank=256)])
@pytest.mark.parametrize("b", [1, 4])
def test_fused_step_config_variants(kw, b):
    """Fused step with in/out_proj biases, no conv bias, N < 16, d_conv 2, 3
    and 8, a dt_rank that is not a multiple of 16, and dt_rank 256 (the
    largest the fused step takes: x_proj's 288 columns, more (column, row)
    pairs than a workgroup has threads): vs the per-op step."""
    print(f"fused decode variant {kw} b={b}", flush=True)
    torch.manual_seed(b)
    cfg = MambaConfig(d_model=96, n_layer=2, vocab_size=200, **kw)
    with torch.device(DEV):
        model = MambaLM(cfg)
    rng = np.random.default_rng(b)
    with torch.no_grad():
        for mx in model.modules():
            if isinstance(mx, MambaMixer):
                D = mx.dt_proj.bias.shape[0]
                mx.dt_proj.bias.copy_(torch.from_numpy(
                    om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32)))
                if mx.in_proj.bias is not None:
                    mx.in_proj.bias.normal_(0, 0.1)
                    mx.out_proj.bias.normal_(0, 0.1)
    model.eval()
    ids = torch.randint(0, 200, (b, 5), device=DEV)
    with torch.no_grad():
        _, c1 = model.prefill(ids)
        _, c2 = model.prefill(ids)
        assert model._fused_step_ok(ids[:, :1], c1)
        for t in range(3):
            nxt = torch.randint(0, 200, (b, 1), device=DEV)
            got = model.step(nxt, c1)
            ref = _per_op_step(model, nxt, c2)
            assert_rel(_np(got), _np(ref), 1e-4, f"logits step {t}")
        for l1, l2 in zip(c1.layers, c2.layers):
            assert_rel(_np(l1.ssm_state), _np(l2.ssm_state), 1e-4, "ssm_state")
            assert_rel(_np(l1.conv_state), _np(l2.conv_state), 1e-5, "conv_state")


@pytest.mark.parametrize("b,cols,rows,with_bias", [(1, 768, 50280, False), (2, 2048, 1001, True), (4, 64, 7, True),
                                                   (1, 4096, 300, False)])
def test_decode_norm_gemv_matches_rmsnorm_then_linear(b, cols, rows, with_bias):
    """mtl_decode_norm_gemv (the final norm_f and tied lm_head of a decode
    step in one launch) against torch fp32 RMSNorm followed by F.linear, at
    1e-4 relative: the lm_head shapes of the 130m and 1.4b widths, a ragged
    row count, the smallest width and the widest."""

    print(f"decode_norm_gemv b={b} cols={cols} rows={rows} bias={with_bias}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(cols + rows)
    v = 3.0 * torch.randn(b, cols, device=DEV, generator=g)
    w = 1.0 + 0.1 * torch.randn(cols, device=DEV, generator=g)
    W = torch.randn(rows, cols, device=DEV, generator=g) / cols ** 0.5
    bias = torch.randn(rows, device=DEV, generator=g) if with_bias else None
    out = torch.empty(b, rows, device=DEV)
    ops.decode_norm_gemv(v, w, 1e-5, W, out, bias=bias)
    vd, wd, Wd = v.double(), w.double(), W.double()
    ref = torch.nn.functional.linear(wd * vd * torch.rsqrt(vd.pow(2).mean(-1, keepdim=True) + 1e-5), Wd,
                                     bias.double() if with_bias else None)
    torch.cuda.synchronize()
    assert_rel(_np(out), ref.cpu().numpy(), 1e-4, "logits")


@pytest.mark.parametrize("b", [1, 2, 4])
@pytest.mark.parametrize("M,D", [(2048, 4096), (96, 192), (64, 100)])
def test_decode_in_channel_blocks_of_4_and_8(b, M, D):
    """mtl_decode_in with 4 and 8 channels per workgroup: every in_proj row is
    one wavefront's dot product in the same order either way, so xc, SiLU(z)
    and the shifted conv history match bit for bit; the x_proj partials of
    4- and 8-channel blocks add up to the same x_dbl within fp32 rounding."""
    print(f"decode_in blocks 4 vs 8: b={b} d_model={M} d_inner={D}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(b * 7 + M)
    K, J = 4, 40
    x = torch.randn(b, M, device=DEV, generator=g)
    norm_w = torch.rand(M, device=DEV, generator=g) + 0.5
    W_in = torch.randn(2 * D, M, device=DEV, generator=g) / M ** 0.5
    conv_w = torch.randn(D, K, device=DEV, generator=g) / 2
    conv_b = torch.randn(D, device=DEV, generator=g)
    state0 = torch.randn(b, D, K - 1, device=DEV, generator=g)
    W_xT = torch.randn(D, J, device=DEV, generator=g) / D ** 0.5
    outs = {}
    for cpb in (4, 8):
        for with_xp in (False, True):
            st = state0.clone()
            xc = torch.empty(b, D, device=DEV)
            gz = torch.empty(b, D, device=DEV)
            xpart = torch.empty(-(-D // cpb), b, J, device=DEV) if with_xp else None
            ops.decode_in(norm_w, 1e-5, W_in, st, conv_w, xc, gz, x=x, conv_b=conv_b,
                          W_xT=W_xT if with_xp else None, xpart=xpart, channels_per_block=cpb)
            outs[cpb, with_xp] = (xc, gz, st, None if xpart is None else xpart.sum(0))
    for with_xp in (False, True):
        for i in range(3):
            assert torch.equal(outs[4, with_xp][i], outs[8, with_xp][i]), (with_xp, i)
    assert_rel(_np(outs[4, True][3]), _np(outs[8, True][3]), 1e-5, "x_dbl")


@pytest.mark.parametrize("b,cols,rows,with_bias,with_x", [(1, 4096, 2048, False, True), (1, 1536, 768, True, True),
                                                          (2, 1536, 768, False, True), (4, 100, 9, True, False),
                                                          (1, 4, 3, True, False), (1, 4096, 160, False, False),
                                                          (4, 2048, 131, True, True)])
def test_decode_gemv_vs_float64(b, cols, rows, with_bias, with_x):
    """mtl_decode_gemv (the decode step's out_proj with the residual add, and
    x_proj at the 1.4b width) against float64 out = x_in + W v + bias, 1e-5
    relative: the out_proj shapes of the 1.4b and 130m widths at batch 1 and 2
    (one wavefront per row), batch 4 (four rows per workgroup), few long rows
    (a workgroup per row split four ways), ragged widths and row counts."""
    print(f"decode_gemv b={b} cols={cols} rows={rows} bias={with_bias} x_in={with_x}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(cols * 3 + rows + b)
    v = torch.randn(b, cols, device=DEV, generator=g)
    W = torch.randn(rows, cols, device=DEV, generator=g) / cols ** 0.5
    bias = torch.randn(rows, device=DEV, generator=g) if with_bias else None
    x_in = torch.randn(b, rows, device=DEV, generator=g) if with_x else None
    out = torch.empty(b, rows, device=DEV)
    ops.decode_gemv(v, W, out, bias=bias, x_in=x_in)
    ref = v.double().cpu() @ W.double().cpu().T
    if with_bias:
        ref = ref + bias.double().cpu()
    if with_x:
        ref = ref + x_in.double().cpu()
    assert_rel(_np(out), ref.numpy(), 1e-5, "out")


@pytest.mark.parametrize("cols,rows", [(4096, 2048), (1536, 768), (100, 9)])
def test_decode_gemv_row_kernel_equals_the_staged_kernel(cols, rows):
    """Batch 1 and 2 run one wavefront per row with v read from global
    memory, batch 4 four rows per workgroup with v staged in LDS; all take
    each lane's four-wide dot products in the same order and reduce over the
    wavefront the same way, so the rows of a batch-4 call equal batch-1 and
    batch-2 calls on the same v bit for bit."""
    print(f"decode_gemv b1, b2 == b4 rows cols={cols} rows={rows}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(cols + 5 * rows)
    v = torch.randn(4, cols, device=DEV, generator=g)
    W = torch.randn(rows, cols, device=DEV, generator=g) / cols ** 0.5
    bias = torch.randn(rows, device=DEV, generator=g)
    x_in = torch.randn(4, rows, device=DEV, generator=g)
    out4 = torch.empty(4, rows, device=DEV)
    ops.decode_gemv(v, W, out4, bias=bias, x_in=x_in)
    for i in range(4):
        out1 = torch.empty(1, rows, device=DEV)
        ops.decode_gemv(v[i:i + 1].clone(), W, out1, bias=bias, x_in=x_in[i:i + 1].clone())
        assert torch.equal(out1[0], out4[i]), i
    for i in (0, 2):
        out2 = torch.empty(2, rows, device=DEV)
        ops.decode_gemv(v[i:i + 2].clone(), W, out2, bias=bias, x_in=x_in[i:i + 2].clone())
        assert torch.equal(out2, out4[i:i + 2]), i


@pytest.mark.parametrize("d_model,b,fused_max", [(256, 1, 2), (256, 2, 2), (256, 4, 4), (2048, 1, 2), (2048, 2, 2)])
def test_native_decode_step_equals_the_per_layer_loop(d_model, b, fused_max, monkeypatch):
    """mtl_decode_step (every layer of a fused decode step in one C call)
    against the per-layer Python loop it replaces: logits and every layer's
    conv and SSM state bit for bit over three steps, at a width where
    decode_in forms the x_proj partials (d_model 256) and one where x_proj
    runs as its own column-part GEMV (d_model 2048)."""
    import mamba_lite.model as mm
    from mamba_lite import ops as mops
    from mamba_lite.model import MambaCache, MambaConfig, MambaLM
    monkeypatch.setattr(mm, "FUSED_STEP_MAX_BATCH", fused_max)
    print(f"native decode step d_model={d_model} b={b}", flush=True)
    torch.manual_seed(70 + b)
    cfg = MambaConfig(d_model=d_model, n_layer=2, vocab_size=320, d_state=16)
    with torch.device("cuda"):
        model = MambaLM(cfg).eval()
    calls = []
    real = mops.decode_step
    monkeypatch.setattr(mops, "decode_step", lambda *a, **k: calls.append(1) or real(*a, **k))
    ids = torch.randint(0, cfg.vocab_size, (b, 6), device="cuda")
    steps = [torch.randint(0, cfg.vocab_size, (b, 1), device="cuda") for _ in range(3)]

    def run():
        with torch.no_grad():
            _, cache = model.prefill(ids)
            out = [model.step(s, cache).clone() for s in steps]
        return out + [t for lc in cache.layers for t in (lc.conv_state, lc.ssm_state)]

    nat = run()
    assert len(calls) == 3
    monkeypatch.setattr(mm, "DECODE_STEP_NATIVE", False)
    per = run()
    assert len(calls) == 3
    for k, (x, y) in enumerate(zip(nat, per)):
        assert torch.equal(x, y), k


@pytest.mark.parametrize("bad", ["batch", "dtype", "strided", "layers"])
def test_fused_step_rejects_a_mismatched_cache_before_any_launch(bad):
    """A cache that does not match the step (a batch-1 cache stepped with
    batch-2 ids, a bfloat16 or strided state in a layer after the first, a
    cache with a layer missing) raises ValueError before any kernel runs: no
    layer's conv history or SSM state moves (the reference fails in
    torch.cat, model.py:264-266)."""
    print(f"fused step, mismatched cache: {bad}", flush=True)
    model = _model(768, 3, 512, seed=11)
    with torch.no_grad():
        _, cache = model.prefill(torch.randint(0, 512, (1, 6), device=DEV))
        ids = torch.randint(0, 512, (1, 1), device=DEV)
        if bad == "batch":
            ids = torch.randint(0, 512, (2, 1), device=DEV)
        elif bad == "dtype":
            cache.layers[1].ssm_state = cache.layers[1].ssm_state.bfloat16()
        elif bad == "strided":
            cs = cache.layers[2].conv_state
            cache.layers[2].conv_state = torch.zeros(cs.shape[0], cs.shape[2], cs.shape[1], device=DEV).transpose(1, 2)
        else:
            cache.layers.pop()
        before = [(l.conv_state.clone(), l.ssm_state.clone()) for l in cache.layers]
        assert model._fused_step_ok(ids, cache)
        with pytest.raises(ValueError, match="step:"):
            model.step(ids, cache)
        torch.cuda.synchronize()
        for (c0, h0), l in zip(before, cache.layers):
            assert torch.equal(c0, l.conv_state) and torch.equal(h0, l.ssm_state)


def _persist_err_word(model):
    from mamba_lite import ops
    ws = getattr(model, "_persist_ws", {})
    return [ops.decode_persist_error(t) for t in ws.values()]


@pytest.mark.parametrize("d_model,n_layer,blocking", [(64, 2, 0), (64, 2, 1), (64, 2, 2), (768, 3, 1), (768, 3, 2),
                                                      (512, 2, 0)])
def test_persistent_step_matches_the_three_kernel_step(d_model, n_layer, blocking, monkeypatch):
    """mtl_decode_step_persist (one launch for every layer) against the
    three-kernel fused step on the same weights: logits and both caches
    within 1e-4 over four steps (its x_proj partials are summed over
    different channel blocks), caches updated in place, no wait timed out."""
    import mamba_lite.model as mm
    print(f"persistent decode d_model={d_model} layers={n_layer} blocking={blocking}", flush=True)
    model = _model(d_model, n_layer, 512, seed=d_model + blocking)
    assert model._decode_plan()["persist"]
    ids = torch.randint(0, 512, (1, 6), device=DEV)
    toks = [torch.randint(0, 512, (1, 1), device=DEV) for _ in range(4)]
    with torch.no_grad():
        _, c_ref = model.prefill(ids)
        _, c = model.prefill(ids)
        monkeypatch.setattr(mm, "DECODE_PERSIST", False)
        refs = [model.step(t, c_ref).clone() for t in toks]
        monkeypatch.setattr(mm, "DECODE_PERSIST", True)
        monkeypatch.setattr(mm, "PERSIST_BLOCKING", blocking)
        ptrs = [(l.conv_state.data_ptr(), l.ssm_state.data_ptr()) for l in c.layers]
        for i, (t, r) in enumerate(zip(toks, refs)):
            assert_rel(_np(model.step(t, c)), _np(r), 1e-4, f"logits step {i}")
    for a, b in zip(c.layers, c_ref.layers):
        assert_rel(_np(a.ssm_state), _np(b.ssm_state), 1e-4, "ssm_state")
        assert_rel(_np(a.conv_state), _np(b.conv_state), 1e-5, "conv_state")
    assert ptrs == [(l.conv_state.data_ptr(), l.ssm_state.data_ptr()) for l in c.layers]
    assert _persist_err_word(model) == [0]


@pytest.mark.parametrize("kw", [dict(d_state=8, d_conv=3, bias=True, conv_bias=False),
                                dict(d_state=4, d_conv=2, dt_rank=5)])
def test_persistent_step_config_variants(kw, monkeypatch):
    """In/out_proj biases, no conv bias, N < 16, d_conv 2 and 3, a dt_rank
    that is not a multiple of 16: persistent step vs the three-kernel step."""
    import mamba_lite.model as mm
    print(f"persistent decode variant {kw}", flush=True)
    torch.manual_seed(3)
    cfg = MambaConfig(d_model=96, n_layer=2, vocab_size=200, **kw)
    with torch.device(DEV):
        model = MambaLM(cfg)
    with torch.no_grad():
        for mx in model.modules():
            if isinstance(mx, MambaMixer) and mx.in_proj.bias is not None:
                mx.in_proj.bias.normal_(0, 0.1)
                mx.out_proj.bias.normal_(0, 0.1)
    model.eval()
    ids = torch.randint(0, 200, (1, 5), device=DEV)
    with torch.no_grad():
        _, c_ref = model.prefill(ids)
        _, c = model.prefill(ids)
        for i in range(3):
            t = torch.randint(0, 200, (1, 1), device=DEV)
            monkeypatch.setattr(mm, "DECODE_PERSIST", False)
            ref = model.step(t, c_ref)
            monkeypatch.setattr(mm, "DECODE_PERSIST", True)
            assert_rel(_np(model.step(t, c)), _np(ref), 1e-4, f"step {i}")
    assert _persist_err_word(model) == [0]


def test_persistent_step_vs_oracle(monkeypatch):
    """The persistent step at the 130m width against the float64 oracle."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "DECODE_PERSIST", True)
    test_fused_step_vs_oracle()


def test_persistent_step_graph_replay_bit_identical(monkeypatch):
    """Captured as a HIP graph, the persistent launch (its epoch in the
    workspace advancing every replay) gives eager's bits, step after step,
    with eager steps between replays on the same workspace."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "DECODE_PERSIST", True)
    test_fused_step_graph_replay_bit_identical()


def test_persistent_step_out_of_range_id_gives_nan(monkeypatch):
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "DECODE_PERSIST", True)
    model = _model(64, 2, 128, seed=6)
    ids = torch.randint(0, 128, (1, 4), device=DEV)
    with torch.no_grad():
        _, c1 = model.prefill(ids)
        _, c2 = model.prefill(ids)
        got = model.step(torch.full((1, 1), 128, dtype=torch.long, device=DEV), c1)
        ok = model.step(torch.zeros((1, 1), dtype=torch.long, device=DEV), c2)
    # the NaN row also enters c1's states, as on every path; c2 is untouched
    assert torch.isnan(got).all() and torch.isfinite(ok).all()
    assert _persist_err_word(model) == [0]
