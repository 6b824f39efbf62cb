"""The benchmark workloads at their stated sizes, checked against the float64
oracle (fp32 at 1e-4, bf16 activations at 1e-2, relative to each element
plus the tensor's rms) or, where the oracle cannot run the whole case,
through a size-independent property:

  * mamba-130m, 24 layers, vocab 50280, batch 1: a 64-token prompt (the
    one-call short prefill with the chunked scan across lanes) and 32
    teacher-forced steps, prefill logits, every step's logits and every
    layer's final states (reference model.py:328-353); on the three-kernel
    fused step and on the persistent single-launch step;
  * the mamba-1.4b mixer (d_model 2048, d_inner 4096, dt_rank 128) prefilling
    32 x 1024 tokens -- the split-projection path of 16,384 tokens and more --
    with two batch rows recomputed by the oracle (model.py:184-241);
  * the 48-layer mamba-1.4b model (vocab 50280) after a 1024-token prefill at
    batch 1 and 32: 16 graph replays bit-identical to 16 eager steps, and
    the caches after them (reference run_tp.py:111-141, cuda_graph.py:34-131);
  * one tensor-parallel rank's shard of that mixer (d_inner 2048), bf16
    activations with fp32 state, prefilling 32 x 2048 tokens, two rows
    against the oracle on the same bf16-rounded weights and inputs, its
    activations rounded to bf16 where each op stores them (tp_model.py:85-135).
"""
import numpy as np
import pytest
import torch

import _golden as G
from _util import assert_rel, bf16_round
from mamba_lite.cuda_graph import GraphedStepper
from mamba_lite.model import MambaConfig, MambaLM, MambaMixer
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _n(t):
    return t.detach().float().cpu().numpy()


# ------------------------------------------------------------ mamba-130m, batch 1
_C1 = {}


def _c1_case():
    """Weights, ids and the oracle's prefill logits, 32 step logits and final
    states, computed once for both step paths."""
    if not _C1:
        sd = G.lm_weights(49, 768, 24, 50280)
        W = G.oracle_lm_dict(sd, 24)
        ids = np.random.default_rng(64).integers(0, 50280, (1, 64 + 32), dtype=np.int64)
        ref_prefill, cache = om.lm_prefill(W, ids[:, :64], dtype=np.float64)
        ref_steps = [om.lm_step(W, ids[:, 64 + k:65 + k], cache, dtype=np.float64) for k in range(32)]
        _C1.update(sd=sd, ids=ids, prefill=ref_prefill, steps=ref_steps, cache=cache)
    return _C1


@pytest.mark.parametrize("persist", [False, True])
def test_c1_130m_64_token_prompt_then_32_steps(persist, monkeypatch):
    import mamba_lite.model as mm
    monkeypatch.setattr(mm, "DECODE_PERSIST", persist)
    print(f"\n[C1: 130m, 24 layers, 64-token prompt + 32 steps, persistent={persist}]", flush=True)
    c = _c1_case()
    lm = MambaLM(MambaConfig(d_model=768, n_layer=24, vocab_size=50280))
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in c["sd"].items()}, strict=True)
    lm = lm.to(DEV).eval()
    ids = _t(c["ids"])
    with torch.no_grad():
        assert lm._native_prefill_kind(1, 64) == "short"                 # the one-call short prefill
        logits, cache = lm.prefill(ids[:, :64])
        assert_rel(_n(logits), c["prefill"], 1e-4, "prefill logits")
        assert lm._fused_step_ok(ids[:, :1], cache)
        for k in range(32):
            got = lm.step(ids[:, 64 + k:65 + k], cache)
            assert_rel(_n(got), c["steps"][k], 1e-4, f"step {k} logits")
    for i, (lc, (rc, rh)) in enumerate(zip(cache.layers, c["cache"])):
        assert_rel(_n(lc.conv_state), rc, 1e-4, f"layer {i} conv_state")
        assert_rel(_n(lc.ssm_state), rh, 1e-4, f"layer {i} ssm_state")


# ------------------------------------------------ mamba-1.4b mixer, 32 x 1024 tokens
def test_c4_1p4b_mixer_prefill_32x1024_split_projections():
    import mamba_lite.model as mm
    print("\n[C4: 1.4b mixer prefill b=32 l=1024, split projections]", flush=True)
    sd = G.mixer_case_weights(51, d_model=2048, dt_rank=128)
    m = MambaMixer(MambaConfig(d_model=2048, n_layer=1, vocab_size=8, dt_rank=128), 0)
    m.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    m = m.to(DEV).eval()
    b, l = 32, 1024
    assert b * l >= mm.SPLIT_PROJ_MIN_TOKENS
    x = torch.randn(b, l, 2048, device=DEV, generator=torch.Generator(device=DEV).manual_seed(52))
    with torch.no_grad():
        out, cs, hs = m.prefill(x)
    p = G.oracle_mixer_dict(sd)
    for row in (0, 29):
        ro, rc, rh = om.mixer_prefill(p, _n(x[row:row + 1]), dtype=np.float64)
        assert_rel(_n(out[row:row + 1]), ro, 1e-4, f"row {row} out")
        assert_rel(_n(cs[row:row + 1]), rc, 1e-4, f"row {row} conv_state")
        assert_rel(_n(hs[row:row + 1]), rh, 1e-4, f"row {row} ssm_state")


# ------------------------------------- 48-layer mamba-1.4b, graph replay == eager
_LM14 = {}


def _lm_1p4b():
    if not _LM14:
        torch.manual_seed(53)
        with torch.device(DEV):
            lm = MambaLM(MambaConfig(d_model=2048, n_layer=48, vocab_size=50280, dt_rank=128))
        rng = np.random.default_rng(54)
        with torch.no_grad():
            for mx in lm.modules():
                if isinstance(mx, MambaMixer):
                    D = mx.dt_proj.bias.shape[0]
                    mx.dt_proj.bias.copy_(torch.from_numpy(
                        om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32)))
        _LM14["lm"] = lm.eval()
    return _LM14["lm"]


@pytest.mark.parametrize("b", [1, 32])
def test_c4_1p4b_48_layers_graph_replay_equals_eager(b):
    print(f"\n[C4: 1.4b, 48 layers, 1024-token prefill, b={b}: 16 replays vs eager]", flush=True)
    lm = _lm_1p4b()
    g = torch.Generator(device=DEV).manual_seed(55 + b)
    ids = torch.randint(0, 50280, (b, 1024), device=DEV, generator=g)
    toks = [torch.randint(0, 50280, (b, 1), device=DEV, generator=g) for _ in range(16)]
    with torch.no_grad():
        _, ce = lm.prefill(ids)
        eager = [lm.step(t, ce).clone() for t in toks]
        _, cg = lm.prefill(ids)
        st = GraphedStepper(lm, cg, b, "cuda")
        st.capture()
        for k, t in enumerate(toks):
            got = st.replay(t).clone()
            torch.cuda.synchronize()
            assert torch.equal(got, eager[k]), f"replay {k}"
    assert all(torch.isfinite(e).all() for e in eager)
    for i, (le, lg) in enumerate(zip(ce.layers, cg.layers)):
        assert torch.equal(le.conv_state, lg.conv_state) and torch.equal(le.ssm_state, lg.ssm_state), f"layer {i}"


# --------------------------------------- one TP rank's shard, bf16, 32 x 2048 tokens
def test_c5_bf16_shard_mixer_32x2048_vs_oracle():
    """The rank's mixer: d_model 2048, its 2048 channels of d_inner (expand 1),
    dt_rank 128; bf16 weights and activations, fp32 SSM state."""
    print("\n[C5: bf16 shard mixer d_inner 2048, b=32 l=2048]", flush=True)
    sd = G.mixer_case_weights(57, d_model=2048, dt_rank=128, expand=1)
    sd_b = {k: bf16_round(v) for k, v in sd.items()}
    m = MambaMixer(MambaConfig(d_model=2048, n_layer=1, vocab_size=8, dt_rank=128, expand=1), 0)
    m.load_state_dict({k: torch.from_numpy(v) for k, v in sd_b.items()}, strict=True)
    m = m.to(DEV).to(torch.bfloat16).eval()
    x = torch.randn(32, 2048, 2048, device=DEV, generator=torch.Generator(device=DEV).manual_seed(58)).bfloat16()
    with torch.no_grad():
        out, cs, hs = m.prefill(x)
    assert out.dtype == torch.bfloat16 and hs.dtype == torch.float32
    p = G.oracle_mixer_dict(sd_b)
    for row in (0, 21):
        ro, rc, rh = om.mixer_prefill(p, _n(x[row:row + 1]), dtype=np.float64, act=bf16_round)
        assert_rel(_n(out[row:row + 1]), ro, 1e-2, f"row {row} out")
        assert_rel(_n(cs[row:row + 1]), rc, 1e-2, f"row {row} conv_state")
        assert_rel(_n(hs[row:row + 1]), rh, 1e-2, f"row {row} ssm_state")
