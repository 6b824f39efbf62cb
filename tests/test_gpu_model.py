"""Drop-in model API on the GPU: MambaMixer.prefill/step and MambaLM vs the
oracle, the reference's invariants (chunked continuation, teacher-forced
step == prefill, fresh prefill states vs in-place step), and hipGraph
replay == eager, bit for bit."""
import numpy as np
import pytest
import torch

from _util import assert_rel, bf16_round
from mamba_lite.cuda_graph import GraphedStepper
from mamba_lite.model import LayerCache, MambaCache, MambaConfig, MambaLM, MambaMixer
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _np(t):
    return t.detach().float().cpu().numpy()


def _mixer_weights(m):
    d = {"in_proj_w": _np(m.in_proj.weight), "conv_w": _np(m.conv1d.weight)[:, 0, :],
         "conv_b": _np(m.conv1d.bias) if m.conv1d.bias is not None else None, "x_proj_w": _np(m.x_proj.weight),
         "dt_proj_w": _np(m.dt_proj.weight), "dt_proj_b": _np(m.dt_proj.bias), "A_log": _np(m.A_log),
         "D": _np(m.D), "out_proj_w": _np(m.out_proj.weight)}
    if m.in_proj.bias is not None:
        d["in_proj_b"] = _np(m.in_proj.bias)
    if m.out_proj.bias is not None:
        d["out_proj_b"] = _np(m.out_proj.bias)
    return d


def _lm_weights(model):
    return {"embedding": _np(model.embedding.weight), "norm_f": _np(model.norm_f.weight),
            "layers": [dict(_mixer_weights(b.mixer), norm=_np(b.norm.weight)) for b in model.layers]}


def _init_dt_bias(module, seed):
    """dt_proj.bias = inv_softplus(log-uniform[1e-3, 0.1]) as HF Mamba inits it."""
    rng = np.random.default_rng(seed)
    with torch.no_grad():
        for m in module.modules():
            if isinstance(m, MambaMixer):
                D = m.dt_proj.bias.shape[0]
                m.dt_proj.bias.copy_(torch.from_numpy(
                    om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32)))


@pytest.fixture(scope="module")
def small_mixer():
    torch.manual_seed(0)
    cfg = MambaConfig(d_model=64, n_layer=1, vocab_size=100, d_state=16)
    m = MambaMixer(cfg, 0)
    _init_dt_bias(m, 0)
    return m.to(DEV).eval()


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("bias", [False, True])
def test_mixer_prefill_vs_oracle(bias, split, monkeypatch):
    """Both projection layouts: fused in_proj / x_proj with strided z, B, C
    views, and (forced here at a small size) the split GEMMs that give
    contiguous z, B, C."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "SPLIT_PROJ_MIN_TOKENS", 0 if split else 1 << 40)
    torch.manual_seed(1)
    cfg = MambaConfig(d_model=64, n_layer=1, vocab_size=100, d_state=16, bias=bias)
    m = MambaMixer(cfg, 0)
    _init_dt_bias(m, 1)
    m = m.to(DEV).eval()
    x = torch.randn(2, 37, 64, device=DEV)
    with torch.no_grad():
        out, cs, hs = m.prefill(x)
    ref, rcs, rhs = om.mixer_prefill(_mixer_weights(m), _np(x), dtype=np.float64)
    assert_rel(_np(out), ref, 1e-4, "out")
    assert np.array_equal(_np(cs), rcs.astype(np.float32)) or np.allclose(_np(cs), rcs, rtol=1e-6, atol=1e-6)
    assert_rel(_np(hs), rhs, 1e-4, "ssm_state")


def test_mixer_reference_test_config():
    """The reference TP tests' config: d_model 32, d_state 8, x [2,5,32]
    (test_tp_correctness.py:28-30, 47-48)."""
    torch.manual_seed(0)
    cfg = MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8, d_conv=4, expand=2)
    m = MambaMixer(cfg, 0).to(DEV).eval()
    torch.manual_seed(123)
    x = torch.randn(2, 5, 32).to(DEV)
    with torch.no_grad():
        out = m(x)
    ref, _, _ = om.mixer_prefill(_mixer_weights(m), _np(x), dtype=np.float64)
    assert_rel(_np(out), ref, 1e-4, "forward")


def test_mixer_chunked_continuation(small_mixer):
    m = small_mixer
    x = torch.randn(2, 50, 64, device=DEV)
    with torch.no_grad():
        out, cs, hs = m.prefill(x)
        o1, c1, h1 = m.prefill(x[:, :21])
        o2, c2, h2 = m.prefill(x[:, 21:], LayerCache(c1, h1))
    assert_rel(_np(torch.cat([o1, o2], 1)), _np(out), 1e-5, "out")
    # the carried conv history holds in_proj outputs; the GEMM library may pick
    # different kernels for different row counts, so equality holds to rounding
    assert_rel(_np(c2), _np(cs), 1e-5, "conv_state")
    assert_rel(_np(h2), _np(hs), 1e-5, "h")


def test_mixer_step_vs_oracle_and_in_place(small_mixer):
    m = small_mixer
    cfg = m.cfg
    cache = MambaCache.allocate(cfg, 3, DEV, torch.float32).layers[0]
    ptrs = (cache.conv_state.data_ptr(), cache.ssm_state.data_ptr())
    W = _mixer_weights(m)
    rcs = np.zeros((3, cfg.d_inner, 3))
    rhs = np.zeros((3, cfg.d_inner, cfg.d_state))
    for t in range(6):
        x = torch.randn(3, 64, device=DEV)
        with torch.no_grad():
            out = m.step(x, cache)
        ref = om.mixer_step(W, _np(x), rcs, rhs, dtype=np.float64)
        assert_rel(_np(out), ref, 1e-4, f"step {t}")
    assert (cache.conv_state.data_ptr(), cache.ssm_state.data_ptr()) == ptrs
    assert_rel(_np(cache.ssm_state), rhs, 1e-4, "ssm_state")
    assert_rel(_np(cache.conv_state), rcs, 1e-5, "conv_state")


def test_prefill_returns_fresh_state_and_leaves_cache(small_mixer):
    """model.py:334-341: prefill reads the cache but returns new tensors."""
    m = small_mixer
    cache = MambaCache.allocate(m.cfg, 1, DEV, torch.float32).layers[0]
    cache.ssm_state.normal_()
    before = cache.ssm_state.clone()
    with torch.no_grad():
        _, cs, hs = m.prefill(torch.randn(1, 9, 64, device=DEV), cache)
    assert torch.equal(cache.ssm_state, before)
    assert hs.data_ptr() != cache.ssm_state.data_ptr() and cs.data_ptr() != cache.conv_state.data_ptr()


@pytest.fixture(scope="module")
def small_lm():
    torch.manual_seed(2)
    cfg = MambaConfig(d_model=64, n_layer=3, vocab_size=203, d_state=16)
    model = MambaLM(cfg)
    _init_dt_bias(model, 2)
    return model.to(DEV).eval()


def test_lm_prefill_vs_oracle(small_lm):
    ids = torch.randint(0, small_lm.cfg.vocab_size, (2, 19), device=DEV)
    with torch.no_grad():
        logits, cache = small_lm.prefill(ids)
    ref, rcache = om.lm_prefill(_lm_weights(small_lm), ids.cpu().numpy(), dtype=np.float64)
    assert logits.shape == (2, 19, small_lm.cfg.vocab_size)
    assert_rel(_np(logits), ref, 1e-4, "logits")
    for lc, (rc, rh) in zip(cache.layers, rcache):
        assert_rel(_np(lc.ssm_state), rh, 1e-4, "ssm")


def test_lm_teacher_forced_step_matches_prefill(small_lm):
    """test_correctness.py:49-72 restated on random weights."""
    ids = torch.randint(0, small_lm.cfg.vocab_size, (1, 12), device=DEV)
    with torch.no_grad():
        full, _ = small_lm.prefill(ids)
        first, cache = small_lm.prefill(ids[:, :1])
        got = [first]
        for t in range(1, 12):
            got.append(small_lm.step(ids[:, t:t + 1], cache))
    assert_rel(_np(torch.cat(got, 1)), _np(full), 1e-4, "cached vs full")


def test_lm_generate_matches_eager_loop(small_lm):
    ids = torch.randint(0, small_lm.cfg.vocab_size, (2, 5), device=DEV)
    with torch.no_grad():
        toks = small_lm.generate(ids, max_new_tokens=6)
        logits, cache = small_lm.prefill(ids)
        nxt = logits[:, -1:].argmax(-1)
        seq = [ids, nxt]
        for _ in range(5):
            nxt = small_lm.step(nxt, cache)[:, -1, :].argmax(-1, keepdim=True)
            seq.append(nxt)
    assert torch.equal(toks, torch.cat(seq, 1))


@pytest.mark.parametrize("batch", [1, 4])
def test_graph_replay_bit_identical_to_eager(small_lm, batch):
    """run_tp.py:111-141 restated with a stricter bar: every replay's logits
    and the carried cache equal eager's bit for bit; eager work and syncs run
    between replays."""
    torch.manual_seed(3)
    ids = torch.randint(0, small_lm.cfg.vocab_size, (batch, 8), device=DEV)
    steps = [torch.randint(0, small_lm.cfg.vocab_size, (batch, 1), device=DEV) for _ in range(5)]
    with torch.no_grad():
        _, cache_e = small_lm.prefill(ids)
        eager = [small_lm.step(s, cache_e).clone() for s in steps]
        _, cache_g = small_lm.prefill(ids)
        st = GraphedStepper(small_lm, cache_g, batch, "cuda")
        st.capture()
        for i, s in enumerate(steps):
            g = st.replay(s).clone()
            torch.cuda.synchronize()
            _ = small_lm.prefill(ids[:, :3])   # unrelated eager work between replays
            assert torch.equal(g, eager[i]), f"replay {i} differs"
    for le, lg in zip(cache_e.layers, cache_g.layers):
        assert torch.equal(le.ssm_state, lg.ssm_state) and torch.equal(le.conv_state, lg.conv_state)


@pytest.mark.parametrize("batch", [8, 32])
def test_graph_replay_on_the_skinny_gemm_step(batch, monkeypatch):
    """The batched per-op step with in_proj fused with the conv step and the
    x_proj partials (mtl_in_proj_conv_xproj) and out_proj on mtl_linear_skinny
    (4 split-K parts summed by the residual add): graph replays equal eager
    bit for bit, with eager work between replays, and the eager step matches
    the float64 oracle."""
    import mamba_lite.model as mm
    from mamba_lite import ops as mops
    monkeypatch.setattr(mm, "BATCHED_STEP_NATIVE", False)     # the Python launches, counted below
    calls = []
    real = mops.linear_skinny
    monkeypatch.setattr(mops, "linear_skinny", lambda *a, **k: calls.append(k.get("ksplit", 1)) or real(*a, **k))
    real_ic = mops.in_proj_conv_xproj
    monkeypatch.setattr(mops, "in_proj_conv_xproj", lambda *a, **k: calls.append("fused") or real_ic(*a, **k))
    torch.manual_seed(6)
    cfg = MambaConfig(d_model=256, n_layer=2, vocab_size=512, d_state=16)
    model = MambaLM(cfg)
    _init_dt_bias(model, 6)
    model = model.to(DEV).eval()
    ids = torch.randint(0, 512, (batch, 6), device=DEV)
    steps = [torch.randint(0, 512, (batch, 1), device=DEV) for _ in range(4)]
    with torch.no_grad():
        _, cache_e = model.prefill(ids)
        calls.clear()                     # the prefill's own projections (<= 64 tokens) run there too
        eager = [model.step(s, cache_e).clone() for s in steps]
        assert "fused" in calls and 4 in calls and 1 not in calls, calls   # fused in_proj, out_proj in 4 parts
        ref_logits, rcache = om.lm_prefill(_lm_weights(model), ids.cpu().numpy(), dtype=np.float64)
        for k, s in enumerate(steps):
            ref = om.lm_step(_lm_weights(model), s.cpu().numpy(), rcache, dtype=np.float64)
            assert_rel(eager[k].cpu().numpy(), ref, 1e-4, f"step {k}")
        _, cache_g = model.prefill(ids)
        st = GraphedStepper(model, cache_g, batch, "cuda")
        st.capture()
        for i, s in enumerate(steps):
            g = st.replay(s).clone()
            torch.cuda.synchronize()
            _ = model.prefill(ids[:, :3])
            assert torch.equal(g, eager[i]), f"replay {i} differs"
    for le, lg in zip(cache_e.layers, cache_g.layers):
        assert torch.equal(le.ssm_state, lg.ssm_state) and torch.equal(le.conv_state, lg.conv_state)


@pytest.mark.parametrize("split", [False, True])
def test_bf16_mixer_shard_shape(split, monkeypatch):
    """bf16 activations, fp32 scan state, through conv + scan + gate at a
    reduced TP-rank shard shape, both projection layouts: vs the float64
    oracle on the same bf16-rounded weights and inputs, its activations
    rounded to bf16 where each op stores them, at 1e-2."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "SPLIT_PROJ_MIN_TOKENS", 0 if split else 1 << 40)
    torch.manual_seed(4)
    cfg = MambaConfig(d_model=128, n_layer=1, vocab_size=100, d_state=16)
    m = MambaMixer(cfg, 0)
    _init_dt_bias(m, 4)
    mb = m.to(DEV).to(torch.bfloat16)
    x = torch.randn(2, 40, 128, device=DEV).bfloat16()
    with torch.no_grad():
        outb, cb, hb = mb.prefill(x)
    assert outb.dtype == torch.bfloat16 and hb.dtype == torch.float32
    p = _mixer_weights(mb)
    ro, rc, rh = om.mixer_prefill(p, _np(x), dtype=np.float64, act=bf16_round)
    assert_rel(_np(outb), ro, 1e-2, "bf16 out vs oracle")
    assert_rel(_np(cb), rc, 1e-2, "bf16 conv_state vs oracle")
    assert_rel(_np(hb), rh, 1e-2, "fp32 state vs oracle")


@pytest.mark.parametrize("b", [8, 32, 40])
def test_mixer_step_batched_x_proj_chunks(b):
    """Batched per-op step: up to b = 32 the conv step and x_proj partials run
    in mtl_conv_step_xproj + mtl_sum_parts; above it (d_inner >= 1024) x_proj
    runs as chunked GEMMs + mtl_sum_parts.  Both match the oracle step."""
    print(f"batched mixer step b={b}", flush=True)
    torch.manual_seed(b)
    cfg = MambaConfig(d_model=512, n_layer=1, vocab_size=64, d_state=16)
    mx = MambaMixer(cfg, 0)
    _init_dt_bias(mx, b)
    mx = mx.to(DEV).eval()
    p = _mixer_weights(mx)
    rng = np.random.default_rng(b)
    D = cfg.d_inner
    cs = rng.standard_normal((b, D, cfg.d_conv - 1)).astype(np.float32)
    hs = (0.1 * rng.standard_normal((b, D, cfg.d_state))).astype(np.float32)
    x = rng.standard_normal((b, cfg.d_model)).astype(np.float32)
    lc = LayerCache(conv_state=torch.from_numpy(cs).to(DEV), ssm_state=torch.from_numpy(hs).to(DEV))
    with torch.no_grad():
        y = mx.step(torch.from_numpy(x).to(DEV), lc)
    cs_r, hs_r = cs.astype(np.float64), hs.astype(np.float64)
    y_ref = om.mixer_step(p, x.astype(np.float64), cs_r, hs_r, dtype=np.float64)
    assert mx._xproj_cache is not None
    assert_rel(y.cpu().numpy(), y_ref, 1e-4, "y")
    assert_rel(lc.ssm_state.cpu().numpy(), hs_r, 1e-4, "ssm_state")
    assert_rel(lc.conv_state.cpu().numpy(), cs_r, 1e-5, "conv_state")


def test_prefill_into_preallocated_cache():
    """prefill(..., out_cache=) writes the final states into the given
    tensors: bit-identical to a fresh prefill, addresses unchanged; and a
    chunked continuation can target its own input cache."""
    torch.manual_seed(21)
    cfg = MambaConfig(d_model=64, n_layer=2, vocab_size=128, d_state=16)
    with torch.device(DEV):
        model = MambaLM(cfg)
    _init_dt_bias(model, 21)
    model.eval()
    ids = torch.randint(0, 128, (2, 40), device=DEV)
    with torch.no_grad():
        ref_logits, ref_cache = model.prefill(ids)
        pre = MambaCache.allocate(cfg, 2, DEV, torch.float32)
        ptrs = [(l.conv_state.data_ptr(), l.ssm_state.data_ptr()) for l in pre.layers]
        logits, got = model.prefill(ids, out_cache=pre)
        assert got is pre
        assert ptrs == [(l.conv_state.data_ptr(), l.ssm_state.data_ptr()) for l in pre.layers]
        assert torch.equal(logits, ref_logits)
        for a, r in zip(pre.layers, ref_cache.layers):
            assert torch.equal(a.conv_state, r.conv_state) and torch.equal(a.ssm_state, r.ssm_state)
        # continuation written over its own input state
        _, c = model.prefill(ids[:, :25])
        _, c2 = model.prefill(ids[:, 25:], cache=c, out_cache=c)
        assert c2 is c
        for a, r in zip(c.layers, ref_cache.layers):
            assert_rel(_np(a.ssm_state), _np(r.ssm_state), 1e-5, "ssm_state")
            assert_rel(_np(a.conv_state), _np(r.conv_state), 1e-5, "conv_state")


@pytest.mark.parametrize("b", [1, 4])
def test_graph_serves_a_second_prompt_after_prefill_into_its_cache(b):
    """Capture once; prefill a new prompt into the captured cache; replays
    then equal eager steps from a fresh prefill of that prompt, bit for bit."""
    torch.manual_seed(22 + b)
    cfg = MambaConfig(d_model=64, n_layer=2, vocab_size=128, d_state=16)
    with torch.device(DEV):
        model = MambaLM(cfg)
    _init_dt_bias(model, 22)
    model.eval()
    p1 = torch.randint(0, 128, (b, 12), device=DEV)
    p2 = torch.randint(0, 128, (b, 9), device=DEV)
    steps = [torch.randint(0, 128, (b, 1), device=DEV) for _ in range(3)]
    with torch.no_grad():
        _, cache = model.prefill(p1)
        st = GraphedStepper(model, cache, b, "cuda")
        st.capture()
        st.replay(steps[0])
        model.prefill(p2, out_cache=cache)
        _, ce = model.prefill(p2)
        for s in steps:
            g = st.replay(s).clone()
            e = model.step(s, ce)
            torch.cuda.synchronize()
            assert torch.equal(g, e)


@pytest.mark.parametrize("d_model,b", [(768, 32), (2048, 1), (2048, 32)])
def test_tuned_gemm_table_loads_and_keeps_prefill_results(d_model, b):
    """mamba_lite.gemm_table: torch accepts the committed TunableOp table on
    this torch and ROCm, and a mixer prefill of b x 1024 tokens at the 130m and 1.4b
    widths (whose projection shapes are in the table: in_proj whole at 1 x
    1024, its halves at 32 x 1024, x_proj, dt_proj, out_proj) gives the same
    output and states within 1e-4 relative as the default GEMM paths."""
    import torch.cuda.tunable as tunable
    from mamba_lite import gemm_table
    print(f"\n[tuned table: mixer d_model={d_model} b={b} x 1024]", flush=True)
    torch.manual_seed(3)
    cfg = MambaConfig(d_model=d_model, n_layer=1, vocab_size=50280, d_state=16)
    with torch.device(DEV):
        mixer = MambaMixer(cfg, 0).eval()
    x = torch.randn(b, 1024, d_model, device=DEV)
    with torch.no_grad():
        ref, _, ref_h = mixer.prefill(x)
        try:
            assert gemm_table.enable()
            out, _, h = mixer.prefill(x)
            torch.cuda.synchronize()
        finally:
            tunable.enable(False)
    assert_rel(out[:4].cpu().numpy(), ref[:4].cpu().numpy(), 1e-4, "out")
    assert_rel(h.cpu().numpy(), ref_h.cpu().numpy(), 1e-4, "ssm_state")


def test_kernels_run_on_the_callers_current_stream():
    """The wrappers launch on torch's current stream of the operands' device
    (the raw-stream accessor): a prefill issued inside `torch.cuda.stream(s)`
    on a side stream, synchronized through that stream only, equals the same
    prefill on the default stream bit for bit."""
    torch.manual_seed(5)
    cfg = MambaConfig(d_model=64, n_layer=2, vocab_size=128, d_state=16)
    with torch.device(DEV):
        model = MambaLM(cfg).eval()
    ids = torch.randint(0, cfg.vocab_size, (2, 40), device=DEV)
    with torch.no_grad():
        ref, ref_cache = model.prefill(ids)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            from mamba_lite import ops
            assert ops._stream(ids) == side.cuda_stream
            out, cache = model.prefill(ids)
        side.synchronize()
    assert torch.equal(out, ref)
    for a, r in zip(cache.layers, ref_cache.layers):
        assert torch.equal(a.ssm_state, r.ssm_state) and torch.equal(a.conv_state, r.conv_state)


def test_prefill_leaves_the_blas_backend_alone():
    """No library call changes torch's process-wide BLAS backend choice (a
    GEMM another thread issues meanwhile keeps its backend and rounding)."""
    torch.manual_seed(6)
    cfg = MambaConfig(d_model=64, n_layer=1, vocab_size=128, d_state=16)
    with torch.device(DEV):
        model = MambaLM(cfg).eval()
    before = torch.backends.cuda.preferred_blas_library()
    with torch.no_grad():
        for l in (16, 100, 300):
            ids = torch.randint(0, cfg.vocab_size, (1, l), device=DEV)
            _, cache = model.prefill(ids)
            assert torch.backends.cuda.preferred_blas_library() == before
            model.step(ids[:, :1], cache)
            assert torch.backends.cuda.preferred_blas_library() == before


def test_graphed_prefill_replays_match_eager_and_feed_the_stepper():
    """GraphedPrefill: every replay equals an eager prefill on the graph's BLAS
    backend bit for bit (logits, and every layer's final states written into
    the shared cache); between replays the program runs its own eager work.  A GraphedStepper
    captured on the same cache then decodes from the graphed prompt exactly
    as eager steps decode from the eager prompt."""
    from mamba_lite import model as mm
    from mamba_lite.cuda_graph import GraphedPrefill
    torch.manual_seed(8)
    cfg = MambaConfig(d_model=128, n_layer=3, vocab_size=300, d_state=16)
    with torch.device(DEV):
        model = MambaLM(cfg).eval()
    b, l = 2, 24
    cache = MambaCache.allocate(cfg, b, DEV, torch.float32)
    gp = GraphedPrefill(model, cache, b, l, DEV)
    gp.capture()
    st = GraphedStepper(model, cache, b, DEV)
    st.capture()
    g = torch.Generator(device=DEV).manual_seed(3)
    with torch.no_grad():
        for k in range(3):
            print(f"graphed prefill replay {k}", flush=True)
            ids = torch.randint(0, cfg.vocab_size, (b, l), device=DEV, generator=g)
            logits = gp.replay(ids).clone()
            ref, rc = model.prefill(ids)
            assert torch.equal(logits, ref), k
            for a, r in zip(cache.layers, rc.layers):
                assert torch.equal(a.conv_state, r.conv_state) and torch.equal(a.ssm_state, r.ssm_state)
            nxt = ref[:, -1:].argmax(-1)
            for _ in range(4):
                got = st.replay(nxt).clone()
                exp = model.step(nxt, rc)
                assert torch.equal(got, exp)
                nxt = exp[:, -1].argmax(-1, keepdim=True)
    with pytest.raises(ValueError):
        gp.replay(torch.zeros(b, l + 1, dtype=torch.long, device=DEV))


@pytest.mark.parametrize("b,l", [(1, 64), (2, 20), (1, 17), (1, 1)])
def test_short_prefill_on_the_skinny_gemm_vs_oracle(b, l, monkeypatch):
    """A prefill of at most 64 tokens at a width whose projections all fit
    mtl_linear_skinny (K a multiple of 128): in_proj whole with the causal
    conv as its epilogue, x_proj split over K and summed, out_proj as 4 parts
    summed by the residual add.  Logits and
    final states against the float64 oracle at 1e-4, and against the same
    prefill on torch's GEMMs at 1e-5; the mixer's own prefill (out_proj as
    one tensor) against the oracle's mixer."""
    import mamba_lite.model as mm
    from mamba_lite import ops as mops
    monkeypatch.setattr(mm, "SHORT_PREFILL_NATIVE", False)    # the per-op launches themselves
    monkeypatch.setattr(mm, "LONG_PREFILL_NATIVE", False)
    torch.manual_seed(11)
    cfg = MambaConfig(d_model=256, n_layer=2, vocab_size=384, d_state=16)
    with torch.device(DEV):
        model = MambaLM(cfg).eval()
    ids = torch.randint(0, cfg.vocab_size, (b, l), device=DEV)
    calls = []
    real = mops.linear_skinny
    monkeypatch.setattr(mops, "linear_skinny", lambda *a, **k: calls.append(a[0].shape) or real(*a, **k))
    real_ipc = mops.in_proj_conv_prefill
    monkeypatch.setattr(mops, "in_proj_conv_prefill", lambda *a, **k: calls.append(a[0].shape) or real_ipc(*a, **k))
    with torch.no_grad():
        logits, cache = model.prefill(ids)
    # in_proj (with the conv), x_proj and out_proj of every layer
    assert all(s[0] == b * l for s in calls) and len(calls) == 3 * cfg.n_layer, calls
    ref, rcache = om.lm_prefill(_lm_weights(model), ids.cpu().numpy(), dtype=np.float64)
    assert_rel(logits.cpu().numpy(), ref, 1e-4, "logits")
    for lc, (rc, rh) in zip(cache.layers, rcache):
        assert_rel(lc.conv_state.cpu().numpy(), rc, 1e-4, "conv_state")
        assert_rel(lc.ssm_state.cpu().numpy(), rh, 1e-4, "ssm_state")
    monkeypatch.setattr(mm, "_SKINNY_PREFILL", False)
    with torch.no_grad():
        logits2, _ = model.prefill(ids)
    assert_rel(logits.cpu().numpy(), logits2.cpu().numpy(), 1e-5, "skinny vs torch GEMMs")
    monkeypatch.setattr(mm, "_SKINNY_PREFILL", True)
    mx = model.layers[0].mixer
    xin = torch.randn(b, l, cfg.d_model, device=DEV)
    with torch.no_grad():
        y, cs, hs = mx.prefill(xin)
    w = _lm_weights(model)["layers"][0]
    ry, rc, rh = om.mixer_prefill(w, xin.double().cpu().numpy(), None, None, np.float64)
    assert isinstance(y, torch.Tensor) and y.shape == (b, l, cfg.d_model)
    assert_rel(y.cpu().numpy(), ry, 1e-4, "mixer out")
    assert_rel(hs.cpu().numpy(), rh, 1e-4, "mixer ssm_state")


def test_short_prefill_continues_into_its_own_cache(monkeypatch):
    """A prompt of <= 64 tokens continued from a cache and written back into
    that same cache (out_cache=cache, as GraphedPrefill serves prompts) on
    the fused short-prefill kernels: the conv history read and the one
    written are the same tensor.  Logits and states against the float64
    oracle's continuation at 1e-4."""
    import mamba_lite.model as mm
    torch.manual_seed(21)
    cfg = MambaConfig(d_model=256, n_layer=2, vocab_size=384, d_state=16)
    with torch.device(DEV):
        model = MambaLM(cfg).eval()
    ids1 = torch.randint(0, cfg.vocab_size, (2, 13), device=DEV)
    ids2 = torch.randint(0, cfg.vocab_size, (2, 9), device=DEV)
    W = _lm_weights(model)
    with torch.no_grad():
        _, cache = model.prefill(ids1)
        logits, same = model.prefill(ids2, cache=cache, out_cache=cache)
    assert same is cache
    _, rc1 = om.lm_prefill(W, ids1.cpu().numpy(), dtype=np.float64)
    ref, rc2 = om.lm_prefill(W, ids2.cpu().numpy(), cache=rc1, dtype=np.float64)
    assert_rel(_np(logits), ref, 1e-4, "continued logits")
    for lc, (rcs, rhs) in zip(cache.layers, rc2):
        assert_rel(_np(lc.conv_state), rcs, 1e-4, "conv_state")
        assert_rel(_np(lc.ssm_state), rhs, 1e-4, "ssm_state")


@pytest.mark.parametrize("d_model", [64, 256])
def test_bf16_lm_prefill_step_generate(d_model):
    """MambaLM cast to bfloat16 (the reference's from_pretrained(dtype=...),
    model.py:368-372): prefill, teacher-forced steps and generate run on the
    per-op path with bf16 activations and caches, and match the float64
    oracle on the same (bf16-rounded) weights within 1e-2 on the logits."""
    torch.manual_seed(31 + d_model)
    cfg = MambaConfig(d_model=d_model, n_layer=2, vocab_size=300, d_state=16)
    with torch.device(DEV):
        m32 = MambaLM(cfg).eval()
    _init_dt_bias(m32, 31)
    with torch.device(DEV):
        m16 = MambaLM(cfg).eval()
    m16.load_state_dict(m32.state_dict())
    m16 = m16.to(torch.bfloat16)
    ids = torch.randint(0, cfg.vocab_size, (2, 11), device=DEV)
    with torch.no_grad():
        W = _lm_weights(m16)
        ref, rc = om.lm_prefill(W, ids[:, :8].cpu().numpy(), dtype=np.float64)
        l16, c16 = m16.prefill(ids[:, :8])
        assert l16.dtype == torch.bfloat16 and c16.layers[0].conv_state.dtype == torch.bfloat16
        assert_rel(_np(l16), ref, 1e-2, "bf16 prefill logits vs oracle")
        for t in range(8, 11):
            s16 = m16.step(ids[:, t:t + 1], c16)
            ref = om.lm_step(W, ids[:, t:t + 1].cpu().numpy(), rc, dtype=np.float64)
            assert s16.dtype == torch.bfloat16
            assert_rel(_np(s16), ref, 1e-2, f"bf16 step {t} vs oracle")
        toks = m16.generate(ids[:, :4], max_new_tokens=3)
    assert toks.shape == (2, 7) and torch.equal(toks[:, :4], ids[:, :4])


@pytest.mark.parametrize("d_conv,bias,b,l", [(2, False, 2, 32), (3, True, 4, 9), (4, True, 1, 64)])
def test_short_prefill_conv_widths_and_biases(d_conv, bias, b, l, monkeypatch):
    """The fused short-prefill path (in_proj with the conv epilogue, split
    x_proj with dt_proj, out_proj parts) at conv widths 2, 3, 4, with the
    in_proj / out_proj biases, against the float64 oracle at 1e-4.  At this
    width the one-call short prefill does not apply; the one-call long
    prefill, which would take the prompt, is switched off to reach the
    per-op launches."""
    import mamba_lite.model as mm
    from mamba_lite import ops as mops
    monkeypatch.setattr(mm, "LONG_PREFILL_NATIVE", False)
    torch.manual_seed(40 + d_conv)
    cfg = MambaConfig(d_model=128, n_layer=2, vocab_size=256, d_state=16, d_conv=d_conv, bias=bias)
    with torch.device(DEV):
        model = MambaLM(cfg).eval()
    _init_dt_bias(model, 40)
    calls = []
    real = mops.in_proj_conv_prefill
    monkeypatch.setattr(mops, "in_proj_conv_prefill", lambda *a, **k: calls.append(1) or real(*a, **k))
    ids = torch.randint(0, cfg.vocab_size, (b, l), device=DEV)
    with torch.no_grad():
        logits, cache = model.prefill(ids)
    assert len(calls) == cfg.n_layer
    ref, rcache = om.lm_prefill(_lm_weights(model), ids.cpu().numpy(), dtype=np.float64)
    assert_rel(_np(logits), ref, 1e-4, "logits")
    for lc, (rcs, rhs) in zip(cache.layers, rcache):
        assert_rel(_np(lc.conv_state), rcs, 1e-4, "conv_state")
        assert_rel(_np(lc.ssm_state), rhs, 1e-4, "ssm_state")


@pytest.mark.parametrize("d_conv,bias,b,l", [(4, False, 1, 64), (4, False, 2, 20), (3, True, 4, 9), (2, False, 1, 1),
                                             (4, True, 2, 32)])
def test_native_short_prefill_equals_the_per_op_path(d_conv, bias, b, l, monkeypatch):
    """mtl_prefill_short (a short prompt's layer stack as one C call) against
    the per-op path it replaces (the same kernels launched one by one from
    Python): logits and every final state bit for bit, for a fresh prompt
    and for one continued from a cache into that same cache; against the
    float64 oracle at 1e-4; and again after a weight is replaced by a tensor
    at another address (the call's pointer table is rebuilt)."""
    import mamba_lite.model as mm
    from mamba_lite import ops as mops
    print(f"native short prefill d_conv={d_conv} bias={bias} b={b} l={l}", flush=True)
    torch.manual_seed(50 + d_conv + l)
    cfg = MambaConfig(d_model=256, n_layer=3, vocab_size=320, d_state=16, d_conv=d_conv, bias=bias)
    with torch.device(DEV):
        model = MambaLM(cfg).eval()
    _init_dt_bias(model, 50)
    calls = []
    real = mops.prefill_short
    monkeypatch.setattr(mops, "prefill_short", lambda *a, **k: calls.append(1) or real(*a, **k))
    ids = torch.randint(0, cfg.vocab_size, (b, l), device=DEV)
    ids2 = torch.randint(0, cfg.vocab_size, (b, l), device=DEV)

    def run():
        with torch.no_grad():
            lg, c = model.prefill(ids)
            snap = [(x.conv_state.clone(), x.ssm_state.clone()) for x in c.layers]
            lg2, same = model.prefill(ids2, cache=c, out_cache=c)
        assert same is c
        return [lg, lg2] + [t for pair in snap for t in pair] + [t for x in c.layers for t in (x.conv_state,
                                                                                                x.ssm_state)]

    nat = run()
    assert len(calls) == 2
    monkeypatch.setattr(mm, "SHORT_PREFILL_NATIVE", False)
    monkeypatch.setattr(mm, "LONG_PREFILL_NATIVE", False)
    per = run()
    assert len(calls) == 2
    for k, (x, y) in enumerate(zip(nat, per)):
        assert torch.equal(x, y), k
    ref, rcache = om.lm_prefill(_lm_weights(model), ids.cpu().numpy(), dtype=np.float64)
    assert_rel(_np(nat[0]), ref, 1e-4, "logits")
    for i, (rcs, rhs) in enumerate(rcache):
        assert_rel(_np(nat[2 + 2 * i]), rcs, 1e-4, "conv_state")
        assert_rel(_np(nat[3 + 2 * i]), rhs, 1e-4, "ssm_state")
    w = model.layers[1].mixer.out_proj.weight
    w.data = (0.5 * w.data).clone()
    with torch.no_grad():
        lp, _ = model.prefill(ids)
        monkeypatch.setattr(mm, "SHORT_PREFILL_NATIVE", True)
        ln, _ = model.prefill(ids)
    assert len(calls) == 3 and torch.equal(ln, lp) and not torch.equal(ln, nat[0])


@pytest.mark.parametrize("b,kw,what", [(1, dict(d_state=32), "d_state 32"), (4, dict(d_state=32), "d_state 32"),
                                       (4, dict(dt_rank=300), "dt_rank 300")])
def test_a_step_past_the_step_kernels_limits_raises_before_touching_the_cache(b, kw, what):
    """The step kernels hold one state per lane of a 16-lane row and at most
    256 dt_proj columns; a model with 32 states or dt_rank 300 prefills (the
    scan takes up to 32 states, the per-op prefill any dt_rank) but its step
    raises ValueError before any launch, leaving every layer's conv history
    and SSM state as they were (the reference's torch step would run it)."""
    cfg = MambaConfig(d_model=256, n_layer=2, vocab_size=64, **kw)
    torch.manual_seed(b)
    with torch.device(DEV):
        lm = MambaLM(cfg).eval()
    ids = torch.randint(0, 64, (b, 9), device=DEV)
    with torch.no_grad():
        _, cache = lm.prefill(ids[:, :8])
        before = [(lc.conv_state.clone(), lc.ssm_state.clone()) for lc in cache.layers]
        with pytest.raises(ValueError, match=what):
            lm.step(ids[:, 8:], cache)
        torch.cuda.synchronize()
    for i, ((c, h), lc) in enumerate(zip(before, cache.layers)):
        assert torch.equal(c, lc.conv_state) and torch.equal(h, lc.ssm_state), f"layer {i} changed"
