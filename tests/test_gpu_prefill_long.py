"""mtl_prefill_long: a prompt's whole layer stack in one C call past the
short-prompt limit, on the GPU (model.py:184-241, 303-306, 328-341):

  * logits and final states against the float64 oracle (1e-4, the fp32
    tolerance) and against the per-op Python path (1e-5: the GEMM picks
    differ, so the bits may), at the 130m and 1.4b widths and at small widths
    with biases, d_conv 1 and 3, 8 and 32 states;
  * continuation from a cache, written in place (h_out aliasing h0, the conv
    history read and written in different runs), and into a separate
    out_cache, with the projections on hipBLASLt and on the skinny GEMM;
  * a captured GraphedPrefill replays the eager bits, with eager work between
    replays;
  * which prompts take it (more than 64 tokens, or a shape the short path
    does not take, up to LONG_PREFILL_MAX_ELEMS token-channels);
  * two threads prefilling on their own streams at once get what each would
    alone, bit for bit;
  * up to LONG_PREFILL_SKINNY_ROWS rows, the projections on the skinny GEMM
    against the same call's hipBLASLt form and the oracle."""
import numpy as np
import pytest
import torch

import _golden as G
from _util import assert_rel
from mamba_lite import ops
from mamba_lite.cuda_graph import GraphedPrefill
from mamba_lite.model import MambaCache, MambaConfig, MambaLM
from oracle import mixer as om

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _n(t):
    return t.detach().double().cpu().numpy()


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _lm(seed, d_model, n_layer, vocab, **kw):
    sd = G.lm_weights(seed, d_model, n_layer, vocab, **kw)
    lm = MambaLM(MambaConfig(d_model=d_model, n_layer=n_layer, vocab_size=vocab, **kw))
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    return lm.to(DEV).eval(), G.oracle_lm_dict(sd, n_layer)


def _counting(monkeypatch):
    calls = []
    real = ops.prefill_long
    monkeypatch.setattr(ops, "prefill_long", lambda *a, **k: calls.append(1) or real(*a, **k))
    return calls


@pytest.mark.parametrize("b,l,d_model,n_layer,kw", [
    (1, 65, 768, 2, {}), (1, 300, 768, 2, {}), (2, 130, 256, 3, dict(bias=True)), (3, 40, 256, 2, {}),
    (1, 200, 2048, 1, dict(dt_rank=128)), (2, 70, 128, 2, dict(d_conv=1)), (1, 90, 256, 2, dict(d_conv=3, d_state=8)),
    (1, 100, 256, 2, dict(d_state=32)), (1, 9, 64, 2, {})])
def test_long_prefill_vs_oracle_and_per_op(b, l, d_model, n_layer, kw, monkeypatch):
    import mamba_lite.model as mm
    print(f"\n[prefill long b={b} l={l} d_model={d_model} layers={n_layer} {kw}]", flush=True)
    vocab = 512
    lm, W = _lm(90 + b + l + d_model, d_model, n_layer, vocab, **kw)
    calls = _counting(monkeypatch)
    ids = np.random.default_rng(b * 7 + l).integers(0, vocab, (b, l), dtype=np.int64)
    with torch.no_grad():
        logits, cache = lm.prefill(_t(ids))
        assert calls == [1], "the prompt did not take mtl_prefill_long"
        monkeypatch.setattr(mm, "LONG_PREFILL_NATIVE", False)
        ref_logits, ref_cache = lm.prefill(_t(ids))
        monkeypatch.setattr(mm, "LONG_PREFILL_NATIVE", True)
    o_logits, o_cache = om.lm_prefill(W, ids, dtype=np.float64)
    assert_rel(_n(logits), o_logits, 1e-4, "logits vs oracle")
    assert_rel(_n(logits), _n(ref_logits), 1e-5, "logits vs per-op path")
    for i, (lc, rc, (oc, oh)) in enumerate(zip(cache.layers, ref_cache.layers, o_cache)):
        assert_rel(_n(lc.ssm_state), oh, 1e-4, f"layer {i} ssm_state vs oracle")
        assert_rel(_n(lc.conv_state), oc, 1e-4, f"layer {i} conv_state vs oracle")
        assert_rel(_n(lc.ssm_state), _n(rc.ssm_state), 1e-5, f"layer {i} ssm_state vs per-op")


@pytest.mark.parametrize("b", [2, 1])
@pytest.mark.parametrize("in_place", [True, False])
def test_long_prefill_continues_a_cache(in_place, b, monkeypatch):
    """A 100-token prompt, then 150 more tokens from its cache: into the same
    cache (states rewritten in place) or into a separate out_cache; both
    against the oracle's continuation.  Two batch rows put both calls past
    the skinny-projection limit (200 and 300 token rows, hipBLASLt); one
    keeps both on the skinny GEMM (100 and 150 rows), whose second call reads
    the carried conv history and SSM state."""
    import mamba_lite.model as mm
    print(f"\n[prefill long continuation b={b} in_place={in_place}]", flush=True)
    assert (b * 150 <= mm.LONG_PREFILL_SKINNY_ROWS) == (b == 1) and 256 <= mm.LONG_PREFILL_SKINNY_MAX_D_MODEL
    lm, W = _lm(95, 256, 2, 512, bias=True)
    calls = _counting(monkeypatch)
    rng = np.random.default_rng(95)
    ids0, ids1 = rng.integers(0, 512, (b, 100)), rng.integers(0, 512, (b, 150))
    with torch.no_grad():
        _, cache = lm.prefill(_t(ids0))
        out = cache if in_place else MambaCache.allocate(lm.cfg, b, DEV, torch.float32)
        before = [lc.ssm_state.clone() for lc in cache.layers]
        logits, got = lm.prefill(_t(ids1), cache=cache, out_cache=out)
    assert got is out and len(calls) == 2
    if not in_place:
        assert all(torch.equal(a, lc.ssm_state) for a, lc in zip(before, cache.layers)), "input cache changed"
    _, oc = om.lm_prefill(W, ids0, dtype=np.float64)
    o_logits, oc2 = om.lm_prefill(W, ids1, cache=oc, dtype=np.float64)
    assert_rel(_n(logits), o_logits, 1e-4, "logits")
    for i, (lc, (c, h)) in enumerate(zip(got.layers, oc2)):
        assert_rel(_n(lc.ssm_state), h, 1e-4, f"layer {i} ssm_state")
        assert_rel(_n(lc.conv_state), c, 1e-4, f"layer {i} conv_state")


def test_graphed_long_prefill_replays_equal_eager(monkeypatch):
    print("\n[prefill long: graph replay]", flush=True)
    lm, _ = _lm(97, 768, 2, 512)
    calls = _counting(monkeypatch)
    rng = np.random.default_rng(97)
    prompts = [_t(rng.integers(0, 512, (1, 128))) for _ in range(3)]
    cache = MambaCache.allocate(lm.cfg, 1, DEV, torch.float32)
    gp = GraphedPrefill(lm, cache, 1, 128, "cuda")
    gp.capture()
    with torch.no_grad():
        for i, ids in enumerate(prompts):
            got = gp.replay(ids).clone()
            g_states = [lc.ssm_state.clone() for lc in cache.layers]
            torch.cuda.synchronize()
            ref, rcache = lm.prefill(ids)                       # eager work between replays
            assert torch.equal(got, ref), f"replay {i} differs from eager"
            assert all(torch.equal(a, lc.ssm_state) for a, lc in zip(g_states, rcache.layers))
    assert calls, "the captured prefill did not take mtl_prefill_long"


def test_native_prefill_kind():
    import mamba_lite.model as mm
    lm, _ = _lm(99, 768, 1, 512)
    assert lm._native_prefill_kind(1, 64) == "short"
    assert lm._native_prefill_kind(1, 65) == "long"
    assert lm._native_prefill_kind(4, 256) == "long"
    lim = mm.LONG_PREFILL_MAX_ELEMS // lm.cfg.d_inner
    assert lm._native_prefill_kind(1, lim) == "long"
    assert lm._native_prefill_kind(1, lim + 1) is None
    small, _ = _lm(99, 64, 1, 512)
    assert small._native_prefill_kind(1, 8) == "long"     # the short path takes d_model >= 256 only


def test_concurrent_long_prefills_on_two_streams():
    """Two threads prefill different prompts on their own streams at once
    (the library serializes the calls and shares its GEMM plans); each gets
    what a prefill on its own would give, bit for bit."""
    import threading
    print("\n[prefill long: two threads, two streams]", flush=True)
    lm, _ = _lm(101, 256, 2, 512)
    rng = np.random.default_rng(101)
    prompts = [_t(rng.integers(0, 512, (1, 200))), _t(rng.integers(0, 512, (2, 90)))]
    with torch.no_grad():
        alone = [lm.prefill(p)[0] for p in prompts]
    torch.cuda.synchronize()
    got = [None, None]

    def run(i):
        s = torch.cuda.Stream()
        with torch.no_grad(), torch.cuda.stream(s):
            for _ in range(5):
                got[i] = lm.prefill(prompts[i])[0]
        s.synchronize()

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(got[i], alone[i]), f"thread {i} differs"


@pytest.mark.parametrize("b,l,d_model,n_layer,kw", [
    (1, 65, 768, 2, {}), (1, 256, 768, 2, {}), (3, 50, 256, 3, dict(bias=True)), (1, 130, 2048, 1, dict(dt_rank=128)),
    (2, 100, 256, 2, dict(d_conv=3, d_state=8)), (1, 200, 512, 2, dict(d_state=32)),
    (2, 80, 512, 2, dict(d_conv=2, conv_bias=False))])
def test_long_prefill_skinny_projections(b, l, d_model, n_layer, kw, monkeypatch):
    """Up to LONG_PREFILL_SKINNY_ROWS token rows (raised here, and the width
    limit with it, to reach every case) the one call runs its projections on
    the skinny GEMM in 64-row chunks (x_proj as split-K parts
    summed with dt_proj applied, out_proj as parts summed by the residual
    norm): logits and states within 3e-5 of the same call's hipBLASLt form
    and within 1e-4 of the float64 oracle; the two forms round differently,
    so their logits differ in some bit (both forms ran)."""
    import mamba_lite.model as mm
    print(f"\n[prefill long skinny b={b} l={l} d_model={d_model} layers={n_layer} {kw}]", flush=True)
    vocab = 512
    lm, W = _lm(200 + b + l + d_model, d_model, n_layer, vocab, **kw)
    calls = _counting(monkeypatch)
    ids = np.random.default_rng(b * 11 + l).integers(0, vocab, (b, l), dtype=np.int64)
    with torch.no_grad():
        monkeypatch.setattr(mm, "LONG_PREFILL_SKINNY_ROWS", 4096)
        monkeypatch.setattr(mm, "LONG_PREFILL_SKINNY_MAX_D_MODEL", 4096)
        logits, cache = lm.prefill(_t(ids))
        monkeypatch.setattr(mm, "LONG_PREFILL_SKINNY_ROWS", 0)
        ref_logits, ref_cache = lm.prefill(_t(ids))
    assert calls == [1, 1], "the prompt did not take mtl_prefill_long"
    assert not torch.equal(logits, ref_logits), "the skinny form did not run"
    o_logits, o_cache = om.lm_prefill(W, ids, dtype=np.float64)
    assert_rel(_n(logits), o_logits, 1e-4, "logits vs oracle")
    # two fp32 forms of the same sums, rounded differently and carried through
    # the recurrence: 3e-5 between them, the oracle's 1e-4 for each
    assert_rel(_n(logits), _n(ref_logits), 3e-5, "logits vs the hipBLASLt form")
    for i, (lc, rc, (oc, oh)) in enumerate(zip(cache.layers, ref_cache.layers, o_cache)):
        assert_rel(_n(lc.ssm_state), oh, 1e-4, f"layer {i} ssm_state vs oracle")
        assert_rel(_n(lc.conv_state), oc, 1e-4, f"layer {i} conv_state vs oracle")
        assert_rel(_n(lc.ssm_state), _n(rc.ssm_state), 3e-5, f"layer {i} ssm_state vs the hipBLASLt form")


@pytest.mark.parametrize("l", [40, 100])
def test_a_changed_norm_eps_reaches_the_one_call_prefill(l, monkeypatch):
    """The one-call prefills (the short one at 40 tokens, the long one at
    100) keep their weight records between calls; a block norm's eps changed
    after a prompt is in the next one: it matches the per-op prefill with
    the new eps (1e-5) and differs from the prompt before the change."""
    import mamba_lite.model as mm
    print(f"\n[prefill: changed norm eps l={l}]", flush=True)
    lm, _ = _lm(170 + l, 256, 2, 512)
    calls = _counting(monkeypatch)
    ids = _t(np.random.default_rng(l).integers(0, 512, (1, l), dtype=np.int64))
    with torch.no_grad():
        before, _ = lm.prefill(ids)
        lm.layers[1].norm.eps = 3e-2
        logits, _ = lm.prefill(ids)
        monkeypatch.setattr(mm, "SHORT_PREFILL_NATIVE", False)
        monkeypatch.setattr(mm, "LONG_PREFILL_NATIVE", False)
        ref, _ = lm.prefill(ids)
    assert len(calls) == (2 if l > 64 else 0)
    assert not torch.equal(logits, before)
    assert_rel(_n(logits), _n(ref), 1e-5, "logits with the new eps vs per-op")
