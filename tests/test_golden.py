"""Pins the oracle's mixer and LM composition against vectors written by the
reference's own PyTorch model (tests/golden/make_fixtures.py), CPU only.

These cover what the closed forms of test_oracle.py cannot: which half of
in_proj is x and which is z (reference model.py:197-199), the [dt | B | C]
split order (215, 280), dt_proj on dt_low (216-218, 281), the residual
placement (303-311), norm_f and the tied lm_head (325-326, 339-340, 351-352),
the d_conv = 1 special case (210-212, 265-276) and the HF snapshot loader
(28-47, 367-397).  The reference ran in float32; the oracle runs in float64,
so the tolerance (1e-5, relative to each element plus the tensor's rms)
leaves room for the reference's roundings only.
"""
import numpy as np
import pytest
import torch

import _golden as G
from _util import assert_rel
from oracle import mixer as om

TOL = 1e-5


@pytest.mark.parametrize("name,seed,cfg", G.MIXER_CASES, ids=[c[0] for c in G.MIXER_CASES])
def test_oracle_mixer_matches_reference_vectors(name, seed, cfg):
    f = G.load(name)
    p = G.oracle_mixer_dict(G.mixer_case_weights(seed, **cfg))
    o0, c0, h0 = om.mixer_prefill(p, f["x0"], dtype=np.float64)
    assert_rel(o0, f["out0"], TOL, "prefill out")
    assert_rel(c0, f["conv0"], TOL, "prefill conv_state")
    assert_rel(h0, f["ssm0"], TOL, "prefill ssm_state")
    # continuation from the reference's own states, so each stage is pinned on its own
    o1, c1, h1 = om.mixer_prefill(p, f["x1"], f["conv0"].astype(np.float64), f["ssm0"].astype(np.float64),
                                  dtype=np.float64)
    assert_rel(o1, f["out1"], TOL, "continued prefill out")
    assert_rel(c1, f["conv1"], TOL, "continued conv_state")
    assert_rel(h1, f["ssm1"], TOL, "continued ssm_state")
    cs, hs = f["conv1"].astype(np.float64), f["ssm1"].astype(np.float64)
    for k in range(len(f["xs"])):
        out = om.mixer_step(p, f["xs"][k], cs, hs, dtype=np.float64)
        assert_rel(out, f["step_out"][k], TOL, f"step {k} out")
        assert_rel(cs, f["step_conv"][k], TOL, f"step {k} conv_state")
        assert_rel(hs, f["step_ssm"][k], TOL, f"step {k} ssm_state")


@pytest.mark.parametrize("case", G.LM_CASES, ids=[c[0] for c in G.LM_CASES])
def test_oracle_lm_matches_reference_vectors(case):
    name, seed, cfg, batch, plen, steps = case
    f = G.load(name)
    sd = G.lm_weights(seed, cfg["d_model"], cfg["n_layer"], cfg["vocab_size"], **G.lm_config_kw(cfg))
    W = G.oracle_lm_dict(sd, cfg["n_layer"])
    ids = f["ids"]
    logits, cache = om.lm_prefill(W, ids[:, :plen], dtype=np.float64)
    assert_rel(logits, f["logits"], TOL, "prefill logits")
    for i, (cs, hs) in enumerate(cache):
        assert_rel(cs, f[f"conv_{i}"], TOL, f"layer {i} conv_state")
        assert_rel(hs, f[f"ssm_{i}"], TOL, f"layer {i} ssm_state")
    for k in range(steps):
        lg = om.lm_step(W, ids[:, plen + k:plen + k + 1], cache, dtype=np.float64)
        assert_rel(lg, f["step_logits"][k], TOL, f"step {k} logits")
    for i, (cs, hs) in enumerate(cache):
        assert_rel(cs, f[f"end_conv_{i}"], TOL, f"layer {i} conv_state after the steps")
        assert_rel(hs, f[f"end_ssm_{i}"], TOL, f"layer {i} ssm_state after the steps")


def test_golden_weights_are_what_the_reference_loaded():
    """The seeded recipe rebuilds, bit for bit, the state dict that the
    reference's from_pretrained loaded from the committed snapshot."""
    name, seed, cfg = G.HF_CASE
    f = G.load(name)
    sd = G.lm_weights(seed, cfg["d_model"], cfg["n_layer"], cfg["vocab_size"], d_state=cfg["d_state"])
    ref_keys = sorted(k[3:] for k in f if k.startswith("sd."))
    assert ref_keys == sorted(sd)
    for k in ref_keys:
        np.testing.assert_array_equal(sd[k], f["sd." + k], err_msg=k)


@pytest.mark.parametrize("snapshot", ["hf_tiny", "hf_tiny_sharded"])
def test_from_pretrained_loads_the_reference_state_dict(snapshot):
    """Our from_pretrained on the synthetic snapshot (single file, and three
    shards with an index) gives the reference's config and exactly the state
    dict the reference's loader produced (model.py:367-397)."""
    import os
    from mamba_lite.model import MambaLM

    name, _, cfg = G.HF_CASE
    f = G.load(name)
    lm = MambaLM.from_pretrained(os.path.join(G.GOLDEN_DIR, snapshot))
    tag = "sharded_" if snapshot.endswith("sharded") else ""
    assert lm.cfg.vocab_size == int(f[tag + "vocab_size"]) and lm.cfg.dt_rank == int(f[tag + "dt_rank"])
    ours = lm.state_dict()
    ref_keys = sorted(k[3:] for k in f if k.startswith("sd."))
    assert sorted(ours) == ref_keys
    for k in ref_keys:
        got = ours[k]
        assert got.dtype == torch.float32, k
        np.testing.assert_array_equal(got.numpy(), f["sd." + k], err_msg=k)


def test_oracle_lm_on_the_loaded_snapshot():
    name, seed, cfg = G.HF_CASE
    f = G.load(name)
    sd = {k[3:]: f[k] for k in f if k.startswith("sd.")}
    W = G.oracle_lm_dict(sd, cfg["n_layer"])
    logits, _ = om.lm_prefill(W, f["ids"], dtype=np.float64)
    assert_rel(logits, f["logits"], TOL, "logits")
    assert_rel(logits, f["sharded_logits"], TOL, "logits (sharded snapshot)")
