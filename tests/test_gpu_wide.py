"""The mamba-1.4b width (d_model 2048, d_inner 4096, dt_rank 128) and wider
models against the float64 oracle, fp32, tolerance 1e-4 (relative to each
element plus the tensor's rms):

  * a 1024-token mixer prefill at batch 1 (model.py:184-241);
  * MambaMixer.step and MambaLM.step at batch 32 (the per-op step: in_proj
    fused with the conv step and the x_proj partials of each channel block,
    their ordered sum, the SSM update; model.py:249-294, 343-353);
  * MambaLM.step on the fused decode path at batch 1, 2 and 4;
  * d_model 2560 (d_inner 5120, past the fused decode path's 4096-channel
    limit: 320 x_proj partial blocks of 16 channels at batch 1 and 8, 160 of
    32 at batch 32);
  * the full-size mamba-130m model (24 layers, vocab 50280) on the fused
    decode path at batch 1.

Weights come from the seeded recipe of tests/_golden.py (A_log and D off
their constant init, so a channel-blind read shows)."""
import numpy as np
import pytest
import torch

import _golden as G
from _util import assert_rel
from mamba_lite.model import LayerCache, MambaConfig, MambaLM, MambaMixer
from oracle import mixer as om

pytestmark = pytest.mark.gpu
TOL = 1e-4
DEV = "cuda"
W14 = dict(d_model=2048, dt_rank=128)     # mamba-1.4b width: d_inner 4096, d_state 16, d_conv 4


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _n(t):
    return t.detach().float().cpu().numpy()


def _lm(seed, d_model, n_layer, vocab, **kw):
    sd = G.lm_weights(seed, d_model, n_layer, vocab, **kw)
    lm = MambaLM(MambaConfig(d_model=d_model, n_layer=n_layer, vocab_size=vocab, **kw))
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    return lm.to(DEV).eval(), G.oracle_lm_dict(sd, n_layer)


def test_mixer_prefill_1024_tokens_at_1p4b_width():
    print("\n[wide: mixer prefill b=1 l=1024 d_model=2048]", flush=True)
    sd = G.mixer_case_weights(41, **W14)
    m = MambaMixer(MambaConfig(d_model=2048, n_layer=1, vocab_size=8, dt_rank=128), 0)
    m.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    m = m.to(DEV).eval()
    x = np.random.default_rng(42).standard_normal((1, 1024, 2048)).astype(np.float32)
    with torch.no_grad():
        out, cs, hs = m.prefill(_t(x))
    ro, rc, rh = om.mixer_prefill(G.oracle_mixer_dict(sd), x, dtype=np.float64)
    assert_rel(_n(out), ro, TOL, "out")
    assert_rel(_n(cs), rc, TOL, "conv_state")
    assert_rel(_n(hs), rh, TOL, "ssm_state")


def test_mixer_step_batch32_at_1p4b_width():
    print("\n[wide: mixer step b=32 d_model=2048]", flush=True)
    sd = G.mixer_case_weights(43, **W14)
    m = MambaMixer(MambaConfig(d_model=2048, n_layer=1, vocab_size=8, dt_rank=128), 0)
    m.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    m = m.to(DEV).eval()
    p = G.oracle_mixer_dict(sd)
    rng = np.random.default_rng(44)
    x0 = rng.standard_normal((32, 6, 2048)).astype(np.float32)
    _, rc, rh = om.mixer_prefill(p, x0, dtype=np.float64)
    cache = LayerCache(conv_state=_t(rc.astype(np.float32)), ssm_state=_t(rh.astype(np.float32)))
    rc, rh = rc.astype(np.float32).astype(np.float64), rh.astype(np.float32).astype(np.float64)
    with torch.no_grad():
        for k in range(3):
            xt = rng.standard_normal((32, 2048)).astype(np.float32)
            got = m.step(_t(xt), cache)
            ref = om.mixer_step(p, xt, rc, rh, dtype=np.float64)
            assert_rel(_n(got), ref, TOL, f"step {k} out")
            assert_rel(_n(cache.conv_state), rc, TOL, f"step {k} conv_state")
            assert_rel(_n(cache.ssm_state), rh, TOL, f"step {k} ssm_state")


def _lm_steps_vs_oracle(lm, W, b, plen, steps, vocab, seed, expect_fused):
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, vocab, (b, plen + steps), dtype=np.int64)
    with torch.no_grad():
        logits, cache = lm.prefill(_t(ids[:, :plen]))
        assert lm._fused_step_ok(_t(ids[:, :1]), cache) == expect_fused
        ref_logits, ref_cache = om.lm_prefill(W, ids[:, :plen], dtype=np.float64)
        assert_rel(_n(logits), ref_logits, TOL, "prefill logits")
        for k in range(steps):
            got = lm.step(_t(ids[:, plen + k:plen + k + 1]), cache)
            ref = om.lm_step(W, ids[:, plen + k:plen + k + 1], ref_cache, dtype=np.float64)
            assert_rel(_n(got), ref, TOL, f"step {k} logits")
        for i, (lc, (rc, rh)) in enumerate(zip(cache.layers, ref_cache)):
            assert_rel(_n(lc.conv_state), rc, TOL, f"layer {i} conv_state")
            assert_rel(_n(lc.ssm_state), rh, TOL, f"layer {i} ssm_state")


@pytest.mark.parametrize("b,fused_max", [(1, 2), (2, 2), (4, 4), (4, 2), (32, 2)])
def test_lm_step_at_1p4b_width(b, fused_max, monkeypatch):
    """b = 1, 2 (and 4 with the fused limit raised): the fused decode path
    (x_proj as its own row GEMV at this width); b = 4 by default and 32:
    the per-op path."""
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "FUSED_STEP_MAX_BATCH", fused_max)
    print(f"\n[wide: lm step d_model=2048 b={b} fused up to {fused_max}]", flush=True)
    lm, W = _lm(45, 2048, 2, 2048, dt_rank=128)
    _lm_steps_vs_oracle(lm, W, b, 8, 3, 2048, 46 + b, expect_fused=b <= fused_max)


@pytest.mark.parametrize("b", [1, 8, 32])
def test_lm_step_d_inner_5120(b):
    """d_inner 5120: 320 x_proj partial blocks of 16 channels (batch 1, 8) or
    160 of 32 (batch 32), summed by the runtime-count form of mtl_sum_parts;
    the fused decode path stops at 4096."""
    print(f"\n[wide: lm step d_model=2560 b={b}]", flush=True)
    lm, W = _lm(47, 2560, 1, 512)
    _lm_steps_vs_oracle(lm, W, b, 5, 2, 512, 48 + b, expect_fused=False)


def test_lm_130m_full_depth_fused_step():
    """The mamba-130m model at full size (d_model 768, 24 layers, vocab
    50280, tied head) on the fused decode path at batch 1: prefill logits,
    three teacher-forced steps and every layer's states against the float64
    oracle (model.py:328-353)."""
    print("\n[wide: lm 130m 24 layers vocab 50280 b=1 fused]", flush=True)
    lm, W = _lm(49, 768, 24, 50280)
    _lm_steps_vs_oracle(lm, W, 1, 8, 3, 50280, 50, expect_fused=True)
