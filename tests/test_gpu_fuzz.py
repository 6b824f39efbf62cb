"""Seeded random configurations of MambaLM against the float64 oracle.

Each case draws a model shape (d_model among sizes that do and do not take
the matrix-core paths, d_state 1-16, d_conv 1-4, expand 1-2, dt_rank, the
in/out and conv biases, 1-3 layers), a batch and two prompt lengths, then
checks at 1e-4 (relative to each element plus the tensor's rms):
  * the prefill logits and every layer's final conv and SSM states
    (reference model.py:328-341 over 184-241);
  * a continuation prefill from that cache (334-341 with a cache);
  * two teacher-forced steps from the continuation's cache, logits and the
    states after them (343-353 over 249-294).
The draws reach the matrix-core short-prompt projections (at most 64 token
rows, d_model a multiple of 128), the fused decode (batch 1 and 2) and the
per-op step (batch 3 and 5), the chunked and the tiled scan, and the
d_conv = 1 step that skips the conv; four fixed cases add the one-call short
prefill (d_inner a multiple of 512 as well).

A second sweep runs the mixer with bf16 activations and fp32 state (the
tensor-parallel shard's precision, tp_model.py:85-135) on random shapes,
both projection layouts, a prefill and a continuation from its cache,
against the oracle on the same bf16-rounded weights and inputs with its
activations rounded to bf16 where each op stores them, at 1e-2.

The first 24 random model shapes are also captured with GraphedStepper:
four replays equal four eager steps bit for bit, logits and caches
(reference cuda_graph.py:34-131); 12 more capture the prompt prefill
(GraphedPrefill): three replays of different prompts, eager work between
them, each equal to an eager prefill bit for bit.

A third sweep splits random mixers over 2 or 4 ranks on the one GPU
(tp_model.LocalTPMixer): the prefill output and each rank's states equal
the dense mixer's and its channel slices, and two steps the dense step, at
1e-4, with two all-reduces per call (tp_model.py:85-175, the reference's
tests/test_tp_correctness.py:76-80).
"""
import numpy as np
import pytest
import torch

import _golden as G
from _util import assert_rel, bf16_round
from mamba_lite.cuda_graph import GraphedPrefill, GraphedStepper
from mamba_lite.model import LayerCache, MambaCache, MambaConfig, MambaLM, MambaMixer
from mamba_lite.tp_model import LocalTPMixer
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"
N_CASES = 96


def _draw(seed):
    r = np.random.default_rng(1000 + seed)
    d_model = int(r.choice([32, 48, 64, 96, 128, 256, 384, 512]))
    cfg = dict(d_model=d_model, n_layer=int(r.integers(1, 4)), vocab_size=int(r.choice([64, 100])),
               d_state=int(r.choice([1, 4, 8, 13, 16])), d_conv=int(r.choice([1, 2, 3, 4])),
               expand=int(r.choice([1, 2])), bias=bool(r.integers(0, 2)), conv_bias=bool(r.integers(0, 2)))
    if r.integers(0, 2):
        cfg["dt_rank"] = int(r.integers(1, min(64, d_model) + 1))
    batch = int(r.choice([1, 2, 3, 5]))
    l0 = int(r.choice([1, 7, 33, 64, 65, 130]))
    if r.integers(0, 2):
        l0 = max(1, min(l0, 64 // batch))      # a short prompt: the one-call prefill where the shape allows
    l1 = int(r.choice([1, 5, 40]))
    return cfg, batch, l0, l1


# drawn so that the one-call short prefill takes them (fp32, at most 64 token
# rows, d_model a multiple of 128, d_inner a multiple of 512, J a multiple of 4)
SHORT_CASES = [
    (dict(d_model=512, n_layer=2, vocab_size=64, d_state=16, d_conv=4, expand=1, bias=True, conv_bias=False), 2, 17, 5),
    (dict(d_model=256, n_layer=1, vocab_size=100, d_state=8, d_conv=2, expand=2, dt_rank=16, bias=False,
          conv_bias=True), 1, 64, 1),
    (dict(d_model=512, n_layer=3, vocab_size=64, d_state=4, d_conv=3, expand=2, bias=False, conv_bias=True), 3, 21,
     40),
    (dict(d_model=384, n_layer=1, vocab_size=64, d_state=12, d_conv=4, expand=4, dt_rank=24, bias=True,
          conv_bias=True), 1, 1, 5),
]


def _case(i):
    return _draw(i) if i < N_CASES else SHORT_CASES[i - N_CASES]


def _cache_np(cache):
    return [(lc.conv_state.detach().float().cpu().numpy(), lc.ssm_state.detach().float().cpu().numpy())
            for lc in cache.layers]


def _check_cache(got, ref, what):
    for i, ((gc, gh), (rc, rh)) in enumerate(zip(got, ref)):
        assert_rel(gc, rc, 1e-4, f"{what} layer {i} conv_state")
        assert_rel(gh, rh, 1e-4, f"{what} layer {i} ssm_state")


@pytest.mark.parametrize("seed", range(N_CASES + len(SHORT_CASES)))
def test_random_config_prefill_continue_step_vs_oracle(seed):
    cfg_kw, batch, l0, l1 = _case(seed)
    print(f"\n[fuzz {seed}: {cfg_kw} batch={batch} prompt={l0} continuation={l1}]", flush=True)
    cfg = MambaConfig(**cfg_kw)
    extra = {k: cfg_kw[k] for k in ("d_state", "d_conv", "expand", "bias", "conv_bias", "dt_rank") if k in cfg_kw}
    sd = G.lm_weights(2000 + seed, cfg.d_model, cfg.n_layer, cfg.vocab_size, **extra)
    lm = MambaLM(cfg)
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    lm = lm.to(DEV).eval()
    W = G.oracle_lm_dict(sd, cfg.n_layer)
    ids = np.random.default_rng(3000 + seed).integers(0, cfg.vocab_size, (batch, l0 + l1 + 2), dtype=np.int64)
    tids = torch.from_numpy(ids).to(DEV)

    ref0, rc0 = om.lm_prefill(W, ids[:, :l0], dtype=np.float64)
    ref1, rc1 = om.lm_prefill(W, ids[:, l0:l0 + l1], cache=[(c.copy(), h.copy()) for c, h in rc0], dtype=np.float64)
    with torch.no_grad():
        if seed >= N_CASES:
            assert lm._native_prefill_kind(batch, l0) == "short", "the one-call short prefill"
        got0, c0 = lm.prefill(tids[:, :l0])
        assert_rel(got0.float().cpu().numpy(), ref0, 1e-4, "prefill logits")
        _check_cache(_cache_np(c0), rc0, "prefill")
        got1, c1 = lm.prefill(tids[:, l0:l0 + l1], c0)
        assert_rel(got1.float().cpu().numpy(), ref1, 1e-4, "continuation logits")
        _check_cache(_cache_np(c1), rc1, "continuation")
        ocache = [(c.copy(), h.copy()) for c, h in rc1]
        for k in range(2):
            t = l0 + l1 + k
            ref = om.lm_step(W, ids[:, t:t + 1], ocache, dtype=np.float64)
            got = lm.step(tids[:, t:t + 1], c1)
            assert_rel(got.float().cpu().numpy(), ref, 1e-4, f"step {k} logits")
    _check_cache(_cache_np(c1), ocache, "after the steps")


N_BF16 = 32


def _draw_bf16(seed):
    r = np.random.default_rng(5000 + seed)
    d_model = int(r.choice([64, 96, 128, 256, 512]))
    cfg = dict(d_model=d_model, n_layer=1, vocab_size=8, d_state=int(r.choice([4, 8, 16])),
               d_conv=int(r.choice([2, 3, 4])), expand=int(r.choice([1, 2])), bias=bool(r.integers(0, 2)),
               conv_bias=bool(r.integers(0, 2)))
    if r.integers(0, 2):
        cfg["dt_rank"] = int(r.integers(1, min(64, d_model) + 1))
    return cfg, int(r.choice([1, 2, 3, 4])), int(r.choice([1, 17, 64, 100, 300])), int(r.choice([1, 9, 40])), \
        bool(r.integers(0, 2))


@pytest.mark.parametrize("seed", range(N_BF16))
def test_random_bf16_mixer_prefill_and_continuation_vs_oracle(seed, monkeypatch):
    import mamba_lite.model as mm
    cfg_kw, batch, l0, l1, split = _draw_bf16(seed)
    print(f"\n[fuzz bf16 {seed}: {cfg_kw} batch={batch} prompt={l0} continuation={l1} split={split}]", flush=True)
    monkeypatch.setattr(mm, "SPLIT_PROJ_MIN_TOKENS", 0 if split else 1 << 40)
    cfg = MambaConfig(**cfg_kw)
    extra = {k: cfg_kw[k] for k in ("d_state", "d_conv", "expand", "bias", "conv_bias", "dt_rank") if k in cfg_kw}
    sd = {k: bf16_round(v) for k, v in G.mixer_case_weights(6000 + seed, cfg.d_model, **extra).items()}
    m = MambaMixer(cfg, 0)
    m.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    m = m.to(DEV).to(torch.bfloat16).eval()
    p = G.oracle_mixer_dict(sd)
    rng = np.random.default_rng(7000 + seed)
    x0 = bf16_round(rng.standard_normal((batch, l0, cfg.d_model)).astype(np.float32))
    x1 = bf16_round(rng.standard_normal((batch, l1, cfg.d_model)).astype(np.float32))
    ro, rc, rh = om.mixer_prefill(p, x0, dtype=np.float64, act=bf16_round)
    with torch.no_grad():
        out, cs, hs = m.prefill(torch.from_numpy(x0).to(DEV).bfloat16())
        assert out.dtype == torch.bfloat16 and hs.dtype == torch.float32
        _n = lambda t: t.detach().float().cpu().numpy()
        assert_rel(_n(out), ro, 1e-2, "prefill out")
        assert_rel(_n(cs), rc, 1e-2, "prefill conv_state")
        assert_rel(_n(hs), rh, 1e-2, "prefill ssm_state")
        # the continuation from the HIP path's own states (bf16 history, fp32 state)
        ro1, rc1, rh1 = om.mixer_prefill(p, x1, conv_state=_n(cs), ssm_state=_n(hs), dtype=np.float64, act=bf16_round)
        out1, cs1, hs1 = m.prefill(torch.from_numpy(x1).to(DEV).bfloat16(), LayerCache(cs, hs))
        assert_rel(_n(out1), ro1, 1e-2, "continuation out")
        assert_rel(_n(cs1), rc1, 1e-2, "continuation conv_state")
        assert_rel(_n(hs1), rh1, 1e-2, "continuation ssm_state")


N_TP = 16


def _draw_tp(seed):
    r = np.random.default_rng(8000 + seed)
    ws = int(r.choice([2, 4]))
    d_model = int(r.choice([32, 64, 96, 128, 256, 512]))
    cfg = dict(d_model=d_model, n_layer=1, vocab_size=8, d_state=int(r.choice([1, 4, 8, 16])),
               d_conv=int(r.choice([2, 3, 4])), expand=int(r.choice([1, 2])), bias=bool(r.integers(0, 2)),
               conv_bias=bool(r.integers(0, 2)))
    if r.integers(0, 2):
        cfg["dt_rank"] = int(r.integers(1, min(64, d_model) + 1))
    return cfg, ws, int(r.choice([1, 2, 3])), int(r.choice([1, 9, 40, 70]))


@pytest.mark.parametrize("seed", range(N_TP))
def test_random_tp_shards_match_the_dense_mixer(seed):
    cfg_kw, ws, batch, l = _draw_tp(seed)
    print(f"\n[fuzz tp {seed}: {cfg_kw} ws={ws} batch={batch} l={l}]", flush=True)
    cfg = MambaConfig(**cfg_kw)
    assert cfg.d_inner % ws == 0
    extra = {k: cfg_kw[k] for k in ("d_state", "d_conv", "expand", "bias", "conv_bias", "dt_rank") if k in cfg_kw}
    sd = G.mixer_case_weights(9000 + seed, cfg.d_model, **extra)
    dense = MambaMixer(cfg, 0)
    dense.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    dense = dense.to(DEV).eval()
    tp = LocalTPMixer.from_dense(dense, ws)
    g = torch.Generator(device=DEV).manual_seed(10000 + seed)
    x = torch.randn(batch, l + 2, cfg.d_model, device=DEV, generator=g)
    _n = lambda t: t.detach().float().cpu().numpy()
    S = cfg.d_inner // ws
    with torch.no_grad():
        ref, ref_conv, ref_ssm = dense.prefill(x[:, :l])
        out, conv, ssm = tp.prefill(x[:, :l])
        assert tp.comm.count == 2
        assert_rel(_n(out), _n(ref), 1e-4, "prefill out")
        for r in range(ws):
            sl = slice(r * S, (r + 1) * S)
            assert_rel(_n(conv[r]), _n(ref_conv[:, sl]), 1e-4, f"rank {r} conv_state")
            assert_rel(_n(ssm[r]), _n(ref_ssm[:, sl]), 1e-4, f"rank {r} ssm_state")
        caches = [LayerCache(c.clone(), h.clone()) for c, h in zip(conv, ssm)]
        dcache = LayerCache(ref_conv.clone(), ref_ssm.clone())
        for t in range(l, l + 2):
            o = tp.step(x[:, t], caches)
            od = dense.step(x[:, t], dcache)
            assert_rel(_n(o), _n(od), 1e-4, f"step {t - l}")
        assert tp.comm.count == 2 + 2 * 2
        assert_rel(_n(torch.cat([c.ssm_state for c in caches], 1)), _n(dcache.ssm_state), 1e-4, "states after steps")


@pytest.mark.parametrize("seed", range(24))
def test_random_config_graph_replay_equals_eager(seed):
    cfg_kw, batch, l0, _ = _draw(seed)
    print(f"\n[fuzz graph {seed}: {cfg_kw} batch={batch} prompt={l0}]", flush=True)
    cfg = MambaConfig(**cfg_kw)
    extra = {k: cfg_kw[k] for k in ("d_state", "d_conv", "expand", "bias", "conv_bias", "dt_rank") if k in cfg_kw}
    sd = G.lm_weights(2000 + seed, cfg.d_model, cfg.n_layer, cfg.vocab_size, **extra)
    lm = MambaLM(cfg)
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    lm = lm.to(DEV).eval()
    g = torch.Generator(device=DEV).manual_seed(11000 + seed)
    ids = torch.randint(0, cfg.vocab_size, (batch, l0), device=DEV, generator=g)
    toks = [torch.randint(0, cfg.vocab_size, (batch, 1), device=DEV, generator=g) for _ in range(4)]
    with torch.no_grad():
        _, ce = lm.prefill(ids)
        eager = [lm.step(t, ce).clone() for t in toks]
        _, cg = lm.prefill(ids)
        st = GraphedStepper(lm, cg, batch, "cuda")
        st.capture()
        for k, t in enumerate(toks):
            got = st.replay(t).clone()
            torch.cuda.synchronize()
            assert torch.equal(got, eager[k]), f"replay {k}"
    for i, (le, lg) in enumerate(zip(ce.layers, cg.layers)):
        assert torch.equal(le.conv_state, lg.conv_state) and torch.equal(le.ssm_state, lg.ssm_state), f"layer {i}"


@pytest.mark.parametrize("seed", range(24, 36))
def test_random_config_graphed_prefill_equals_eager(seed):
    cfg_kw, batch, l0, _ = _draw(seed)
    print(f"\n[fuzz graphed prefill {seed}: {cfg_kw} batch={batch} prompt={l0}]", flush=True)
    cfg = MambaConfig(**cfg_kw)
    extra = {k: cfg_kw[k] for k in ("d_state", "d_conv", "expand", "bias", "conv_bias", "dt_rank") if k in cfg_kw}
    sd = G.lm_weights(2000 + seed, cfg.d_model, cfg.n_layer, cfg.vocab_size, **extra)
    lm = MambaLM(cfg)
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    lm = lm.to(DEV).eval()
    cache = MambaCache.allocate(cfg, batch, DEV, torch.float32)
    gp = GraphedPrefill(lm, cache, batch, l0, DEV)
    gp.capture()
    g = torch.Generator(device=DEV).manual_seed(12000 + seed)
    with torch.no_grad():
        for k in range(3):
            ids = torch.randint(0, cfg.vocab_size, (batch, l0), device=DEV, generator=g)
            got = gp.replay(ids).clone()
            ref, rc = lm.prefill(ids)                       # eager work between the replays
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"replay {k} logits"
            for i, (a, r) in enumerate(zip(cache.layers, rc.layers)):
                assert torch.equal(a.conv_state, r.conv_state) and torch.equal(a.ssm_state, r.ssm_state), \
                    f"replay {k} layer {i}"
