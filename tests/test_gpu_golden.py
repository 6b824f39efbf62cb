"""The HIP path against the reference's own PyTorch outputs (the golden
vectors of tests/golden/, written by make_fixtures.py from mamba_lite/model.py
on the CPU): mixer prefill, continuation and in-place steps, the LM prefill
and teacher-forced steps on both decode paths and as a graph replay, and the
HF snapshot loader.  fp32 throughout, tolerance 1e-4 (relative to each
element plus the tensor's rms).
"""
import os

import numpy as np
import pytest
import torch

import _golden as G
from _util import assert_rel
from mamba_lite import model as mm
from mamba_lite.model import LayerCache, MambaCache, MambaConfig, MambaLM, MambaMixer

pytestmark = pytest.mark.gpu
TOL = 1e-4
DEV = "cuda"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _n(t):
    return t.detach().float().cpu().numpy()


def _mixer(seed, cfg):
    mc = MambaConfig(d_model=cfg["d_model"], n_layer=1, vocab_size=8, **G.lm_config_kw(cfg))
    m = MambaMixer(mc, 0)
    m.load_state_dict({k: torch.from_numpy(v) for k, v in G.mixer_case_weights(seed, **cfg).items()}, strict=True)
    return m.to(DEV).eval()


def _lm(seed, cfg):
    mc = MambaConfig(d_model=cfg["d_model"], n_layer=cfg["n_layer"], vocab_size=cfg["vocab_size"],
                     **G.lm_config_kw(cfg))
    lm = MambaLM(mc)
    sd = G.lm_weights(seed, cfg["d_model"], cfg["n_layer"], cfg["vocab_size"], **G.lm_config_kw(cfg))
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    return lm.to(DEV).eval()


@pytest.mark.parametrize("split", [False, True], ids=["fused_proj", "split_proj"])
@pytest.mark.parametrize("name,seed,cfg", G.MIXER_CASES, ids=[c[0] for c in G.MIXER_CASES])
def test_mixer_matches_reference_vectors(name, seed, cfg, split, monkeypatch):
    print(f"\n[golden mixer {name} split={split}]", flush=True)
    if split:   # both projection layouts of the prefill
        monkeypatch.setattr(mm, "SPLIT_PROJ_MIN_TOKENS", 1)
    f = G.load(name)
    m = _mixer(seed, cfg)
    with torch.no_grad():
        o0, c0, h0 = m.prefill(_t(f["x0"]))
        assert_rel(_n(o0), f["out0"], TOL, "prefill out")
        assert_rel(_n(c0), f["conv0"], TOL, "prefill conv_state")
        assert_rel(_n(h0), f["ssm0"], TOL, "prefill ssm_state")
        assert_rel(_n(m(_t(f["x0"]))), f["out0"], TOL, "forward")
        cache = LayerCache(conv_state=_t(f["conv0"]), ssm_state=_t(f["ssm0"]))
        o1, c1, h1 = m.prefill(_t(f["x1"]), cache)
        assert_rel(_n(o1), f["out1"], TOL, "continued prefill out")
        assert_rel(_n(c1), f["conv1"], TOL, "continued conv_state")
        assert_rel(_n(h1), f["ssm1"], TOL, "continued ssm_state")
        cache = LayerCache(conv_state=_t(f["conv1"]), ssm_state=_t(f["ssm1"]))
        ptrs = (cache.conv_state.data_ptr(), cache.ssm_state.data_ptr())
        for k in range(len(f["xs"])):
            out = m.step(_t(f["xs"][k]), cache)
            assert_rel(_n(out), f["step_out"][k], TOL, f"step {k} out")
            assert_rel(_n(cache.conv_state), f["step_conv"][k], TOL, f"step {k} conv_state")
            assert_rel(_n(cache.ssm_state), f["step_ssm"][k], TOL, f"step {k} ssm_state")
        assert (cache.conv_state.data_ptr(), cache.ssm_state.data_ptr()) == ptrs


def _check_lm(lm, f, plen, steps, what, stepper=None):
    ids = _t(f["ids"])
    with torch.no_grad():
        logits, cache = lm.prefill(ids[:, :plen])
        assert_rel(_n(logits), f["logits"], TOL, f"{what}: prefill logits")
        for i, lc in enumerate(cache.layers):
            assert_rel(_n(lc.conv_state), f[f"conv_{i}"], TOL, f"{what}: layer {i} conv_state")
            assert_rel(_n(lc.ssm_state), f[f"ssm_{i}"], TOL, f"{what}: layer {i} ssm_state")
        if stepper is not None:
            cache = stepper(cache)
        for k in range(steps):
            tok = ids[:, plen + k:plen + k + 1]
            lg = lm.step(tok, cache) if stepper is None else cache.replay(tok)
            assert_rel(_n(lg), f["step_logits"][k], TOL, f"{what}: step {k} logits")
        layers = cache.layers if stepper is None else cache.cache.layers
        for i, lc in enumerate(layers):
            assert_rel(_n(lc.conv_state), f[f"end_conv_{i}"], TOL, f"{what}: layer {i} conv_state after the steps")
            assert_rel(_n(lc.ssm_state), f[f"end_ssm_{i}"], TOL, f"{what}: layer {i} ssm_state after the steps")


@pytest.mark.parametrize("case", G.LM_CASES, ids=[c[0] for c in G.LM_CASES])
def test_lm_matches_reference_vectors(case, monkeypatch):
    """Prefill and teacher-forced steps on the fused decode path (batch 1, 2
    and 4), then again on the per-op path."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "FUSED_STEP_MAX_BATCH", 4)     # the fused kernels at every batch they take
    name, seed, cfg, batch, plen, steps = case
    print(f"\n[golden lm {name}]", flush=True)
    f = G.load(name)
    lm = _lm(seed, cfg)
    fused = lm._fused_step_ok(_t(f["ids"][:, :1]), MambaCache.allocate(lm.cfg, batch, DEV, torch.float32))
    assert fused == (batch in (1, 2, 4) and cfg.get("d_conv", 4) >= 2)
    _check_lm(lm, f, plen, steps, "fused step" if fused else "per-op step")
    monkeypatch.setattr(MambaLM, "_fused_step_ok", lambda self, ids, cache, **kw: False)
    _check_lm(lm, f, plen, steps, "per-op step")


@pytest.mark.parametrize("case", G.LM_CASES[:2], ids=[c[0] for c in G.LM_CASES[:2]])
def test_graph_replay_matches_reference_vectors(case):
    from mamba_lite.cuda_graph import GraphedStepper

    name, seed, cfg, batch, plen, steps = case
    print(f"\n[golden graph {name}]", flush=True)
    f = G.load(name)
    lm = _lm(seed, cfg)

    def stepper(cache):
        st = GraphedStepper(lm, cache, batch_size=batch, device=DEV)
        st.capture()
        return st
    _check_lm(lm, f, plen, steps, "graph replay", stepper=stepper)


@pytest.mark.parametrize("snapshot", ["hf_tiny", "hf_tiny_sharded"])
def test_from_pretrained_logits_match_reference(snapshot):
    print(f"\n[golden from_pretrained {snapshot}]", flush=True)
    f = G.load(G.HF_CASE[0])
    lm = MambaLM.from_pretrained(os.path.join(G.GOLDEN_DIR, snapshot)).to(DEV).eval()
    with torch.no_grad():
        logits, _ = lm.prefill(_t(f["ids"]))
    assert_rel(_n(logits), f["sharded_logits" if snapshot.endswith("sharded") else "logits"], TOL, "logits")
