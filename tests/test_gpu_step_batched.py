"""mtl_decode_step_batched: a batched step of the whole layer stack in one C
call, on the GPU (MambaLM.step, model.py:343-353 over MambaBlock.step 308-311
and MambaMixer.step 249-294):

  * logits and every layer's conv and SSM state equal the per-op Python
    step's bit for bit over three steps, with the residual add + norm folded
    (up to 16 rows) and not, at widths 256, 768 (mamba-130m) and 2048
    (mamba-1.4b), with and without projection and conv biases, d_conv 2 and
    3, 1 and 8 states, dt_rank 256 (x_proj's 288 columns, the most the call
    takes);
  * the same steps against the float64 oracle (1e-4, the fp32 tolerance);
  * a captured GraphedStepper replays the eager bits, with eager work
    between replays;
  * 24 seeded random shapes it takes (widths 256-1024, d_inner multiples of
    512, 1-16 states, d_conv 2-4, dt_rank, biases, 1-3 layers, 3-32 rows)
    against the per-op step bit for bit and the oracle at 1e-4;
  * a block norm's eps changed between steps reaches the next one;
  * biases, conv and norm weights that start off a 16-byte boundary send
    the step down paths that read them a float at a time (no entry point
    rejects them mid-step), matching the aligned model at 1e-4;
  * the model takes it only where every layer runs the per-op step's in_proj
    + conv + x_proj launch and split out_proj; elsewhere the per-op path runs,
    with its own checks (a cache of the wrong batch still raises
    ValueError)."""
import numpy as np
import pytest
import torch

import _golden as G
from _util import assert_rel
from mamba_lite import ops
from mamba_lite.cuda_graph import GraphedStepper
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
    real = ops.decode_step_batched
    monkeypatch.setattr(ops, "decode_step_batched", lambda *a, **k: calls.append(a[5]) or real(*a, **k))
    return calls


@pytest.mark.parametrize("b,d_model,n_layer,kw", [
    (3, 256, 3, {}), (4, 256, 2, dict(bias=True)), (8, 768, 2, {}), (8, 256, 2, dict(conv_bias=False)),
    (16, 256, 3, dict(bias=True)), (12, 256, 2, dict(d_state=8)), (17, 256, 2, {}), (24, 512, 2, dict(d_conv=3)),
    (32, 768, 2, {}), (32, 2048, 2, dict(dt_rank=128)), (8, 2048, 2, dict(dt_rank=128)),
    (5, 256, 1, {}), (20, 256, 2, dict(d_conv=2, bias=True)),
    # the largest x_proj width the call takes (dt_rank 256 + 2 x 16 states =
    # 288 columns), and one state
    (4, 256, 2, dict(dt_rank=256)), (6, 256, 2, dict(d_state=1))])
def test_batched_step_equals_per_op_and_oracle(b, d_model, n_layer, kw, monkeypatch):
    import mamba_lite.model as mm
    print(f"\n[batched step b={b} d_model={d_model} layers={n_layer} {kw}]", flush=True)
    vocab = 512
    lm, W = _lm(120 + b + d_model, d_model, n_layer, vocab, **kw)
    calls = _counting(monkeypatch)
    rng = np.random.default_rng(b * 5 + d_model)
    plen, steps = 6, 3
    ids = rng.integers(0, vocab, (b, plen + steps), dtype=np.int64)
    with torch.no_grad():
        _, c_nat = lm.prefill(_t(ids[:, :plen]))
        _, c_per = lm.prefill(_t(ids[:, :plen]))
        _, rcache = om.lm_prefill(W, ids[:, :plen], dtype=np.float64)
        fold = lm._fold_ok(lm.embedding(_t(ids[:, :1])).squeeze(1), c_nat)
        for k in range(steps):
            s = ids[:, plen + k:plen + k + 1]
            got = lm.step(_t(s), c_nat)
            monkeypatch.setattr(mm, "BATCHED_STEP_NATIVE", False)
            per = lm.step(_t(s), c_per)
            monkeypatch.setattr(mm, "BATCHED_STEP_NATIVE", True)
            ref = om.lm_step(W, s, rcache, dtype=np.float64)
            assert torch.equal(got, per), f"step {k}: logits differ from the per-op step"
            assert_rel(_n(got), ref, 1e-4, f"step {k} logits vs oracle")
    assert calls == [fold] * steps, (calls, fold)
    assert fold == (b <= mm.STEP_NORM_FOLD_MAX_ROWS and n_layer >= 2)
    for i, (ln, lp, (rc, rh)) in enumerate(zip(c_nat.layers, c_per.layers, rcache)):
        assert torch.equal(ln.conv_state, lp.conv_state), f"layer {i} conv_state"
        assert torch.equal(ln.ssm_state, lp.ssm_state), f"layer {i} ssm_state"
        assert_rel(_n(ln.ssm_state), rh, 1e-4, f"layer {i} ssm_state vs oracle")
        assert_rel(_n(ln.conv_state), rc, 1e-4, f"layer {i} conv_state vs oracle")


@pytest.mark.parametrize("b", [8, 32])
def test_batched_step_graph_replays_equal_eager(b, monkeypatch):
    """The captured step (the C call, the counters' fill kernel, the
    lm_head) replays the eager bits, with eager work between replays."""
    print(f"\n[batched step: graph replay b={b}]", flush=True)
    lm, _ = _lm(140 + b, 256, 3, 512, bias=True)
    calls = _counting(monkeypatch)
    rng = np.random.default_rng(b + 1)
    ids = _t(rng.integers(0, 512, (b, 6), dtype=np.int64))
    steps = [_t(rng.integers(0, 512, (b, 1), dtype=np.int64)) for _ in range(4)]
    with torch.no_grad():
        _, cache_e = lm.prefill(ids)
        eager = [lm.step(s, cache_e).clone() for s in steps]
        assert len(calls) == 4
        _, cache_g = lm.prefill(ids)
        st = GraphedStepper(lm, cache_g, b, "cuda")
        st.capture()
        for i, s in enumerate(steps):
            got = st.replay(s).clone()
            torch.cuda.synchronize()
            _ = lm.step(steps[0], MambaCache.allocate(lm.cfg, b, DEV, torch.float32))   # eager work between
            assert torch.equal(got, eager[i]), f"replay {i} differs"
    for le, lg in zip(cache_e.layers, cache_g.layers):
        assert torch.equal(le.ssm_state, lg.ssm_state) and torch.equal(le.conv_state, lg.conv_state)


def test_batched_step_is_taken_only_where_the_per_op_kernels_apply(monkeypatch):
    """d_conv 1 (no in_proj + conv launch) and a d_inner that is not a
    multiple of 512 (no 4-part out_proj) run op by op; so do a bfloat16 conv
    history and a cache of the wrong batch, which the per-op step rejects
    with ValueError."""
    calls = _counting(monkeypatch)
    rng = np.random.default_rng(3)
    for kw in (dict(d_conv=1), dict(expand=1)):
        d_model = 256 if "expand" not in kw else 384
        lm = MambaLM(MambaConfig(d_model=d_model, n_layer=2, vocab_size=512, **kw)).to(DEV).eval()
        ids = _t(rng.integers(0, 512, (4, 5), dtype=np.int64))
        with torch.no_grad():
            _, cache = lm.prefill(ids[:, :4])
            lm.step(ids[:, 4:], cache)
    assert calls == []
    lm, _ = _lm(150, 256, 2, 512)
    ids = _t(rng.integers(0, 512, (4, 1), dtype=np.int64))
    with torch.no_grad():
        x = lm.embedding(ids).squeeze(1)
        good = MambaCache.allocate(lm.cfg, 4, DEV, torch.float32)
        assert lm._batched_step_layers(x, good) is not None and lm._batched_step_layers(x, good)[1]
        half = MambaCache([type(lc)(lc.conv_state.bfloat16(), lc.ssm_state) for lc in good.layers])
        assert lm._batched_step_layers(x, half) is None
        wrong = MambaCache.allocate(lm.cfg, 8, DEV, torch.float32)
        assert lm._batched_step_layers(x, wrong) is None
        with pytest.raises(ValueError):
            lm.step(ids, wrong)
    assert calls == []


@pytest.mark.parametrize("b", [1, 8])
def test_a_changed_norm_eps_reaches_the_one_call_steps(b, monkeypatch):
    """The one-call steps keep their weight records between calls (the fused
    one at b = 1, the batched one at b = 8); a block norm's eps changed after
    a step is in the next one: it equals the per-op step bit for bit."""
    import mamba_lite.model as mm
    print(f"\n[one-call steps: changed norm eps b={b}]", flush=True)
    lm, _ = _lm(160 + b, 256, 2, 512)
    rng = np.random.default_rng(b + 9)
    ids = _t(rng.integers(0, 512, (b, 5), dtype=np.int64))
    steps = [_t(rng.integers(0, 512, (b, 1), dtype=np.int64)) for _ in range(2)]

    def per_op(s, cache):
        monkeypatch.setattr(mm, "BATCHED_STEP_NATIVE", False)
        monkeypatch.setattr(mm, "DECODE_STEP_NATIVE", False)
        out = lm.step(s, cache)
        monkeypatch.setattr(mm, "BATCHED_STEP_NATIVE", True)
        monkeypatch.setattr(mm, "DECODE_STEP_NATIVE", True)
        return out

    with torch.no_grad():
        _, c_nat = lm.prefill(ids)
        _, c_per = lm.prefill(ids)
        assert torch.equal(lm.step(steps[0], c_nat), per_op(steps[0], c_per))
        lm.layers[1].norm.eps = 3e-2
        got = lm.step(steps[1], c_nat)
        want = per_op(steps[1], c_per)
    assert torch.equal(got, want), "the changed eps did not reach the one-call step"


def _draw(seed):
    """A random model shape the one-call batched step takes: d_model a
    multiple of 128 from 256, d_inner a multiple of 512, d_state up to 16,
    d_conv 2..4, dt_rank with dt_rank + 2 d_state <= 288, biases on or off,
    1-3 layers, 3-32 rows."""
    r = np.random.default_rng(seed)
    d_model = int(r.choice([256, 384, 512, 768, 1024]))
    expand = int(r.choice([e for e in (1, 2, 3, 4) if (e * d_model) % 512 == 0]))
    d_state = int(r.choice([1, 4, 8, 12, 16]))
    cfg = dict(d_model=d_model, n_layer=int(r.integers(1, 4)), vocab_size=int(r.choice([64, 100])), d_state=d_state,
               d_conv=int(r.integers(2, 5)), expand=expand, bias=bool(r.integers(0, 2)),
               conv_bias=bool(r.integers(0, 2)))
    if r.integers(0, 2):
        cfg["dt_rank"] = int(r.integers(1, min(160, 288 - 2 * d_state) + 1))
    return cfg, int(r.integers(3, 33))


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_batched_step_equals_per_op(seed, monkeypatch):
    import mamba_lite.model as mm
    cfg_kw, b = _draw(seed)
    print(f"\n[batched step fuzz {seed}: {cfg_kw} batch={b}]", flush=True)
    cfg = MambaConfig(**cfg_kw)
    extra = {k: cfg_kw[k] for k in ("d_state", "d_conv", "expand", "dt_rank", "bias", "conv_bias") if k in cfg_kw}
    sd = G.lm_weights(4000 + seed, cfg.d_model, cfg.n_layer, cfg.vocab_size, **extra)
    lm = MambaLM(cfg)
    lm.load_state_dict({k: torch.from_numpy(v) for k, v in sd.items()}, strict=True)
    lm = lm.to(DEV).eval()
    W = G.oracle_lm_dict(sd, cfg.n_layer)
    calls = _counting(monkeypatch)
    ids = np.random.default_rng(5000 + seed).integers(0, cfg.vocab_size, (b, 7), dtype=np.int64)
    with torch.no_grad():
        _, c_nat = lm.prefill(_t(ids[:, :4]))
        _, c_per = lm.prefill(_t(ids[:, :4]))
        _, rcache = om.lm_prefill(W, ids[:, :4], dtype=np.float64)
        for k in range(3):
            s = ids[:, 4 + k:5 + k]
            got = lm.step(_t(s), c_nat)
            monkeypatch.setattr(mm, "BATCHED_STEP_NATIVE", False)
            per = lm.step(_t(s), c_per)
            monkeypatch.setattr(mm, "BATCHED_STEP_NATIVE", True)
            ref = om.lm_step(W, s, rcache, dtype=np.float64)
            assert torch.equal(got, per), f"step {k}: logits differ from the per-op step"
            assert_rel(_n(got), ref, 1e-4, f"step {k} logits vs oracle")
    assert len(calls) == 3
    for i, (ln, lp) in enumerate(zip(c_nat.layers, c_per.layers)):
        assert torch.equal(ln.conv_state, lp.conv_state) and torch.equal(ln.ssm_state, lp.ssm_state), f"layer {i}"


def _unaligned(p):
    """p's values in a parameter that starts 4 bytes past a 16-byte boundary
    (a view into a larger buffer)."""
    buf = torch.empty(p.numel() + 1, device=p.device, dtype=p.dtype)
    v = buf[1:].view_as(p)
    v.copy_(p.detach())
    return torch.nn.Parameter(v, requires_grad=False)


@pytest.mark.parametrize("b", [1, 4, 24])
def test_unaligned_vector_parameters_take_another_path_instead_of_raising(b, monkeypatch):
    """Biases, conv weights and norm weights that start off a 16-byte
    boundary cannot go to the entry points that load them in 16-byte runs
    (the one-call batched step, the folded step, the in_proj + conv + x_proj
    launch, the skinny GEMMs), which reject them: the step takes the paths
    that read them a float at a time (batch 1: the fused step, whose kernels
    do), and its logits and caches match the aligned model's at the fp32
    tolerance over three steps from a zero cache."""
    calls = _counting(monkeypatch)
    lm, _ = _lm(160, 256, 2, 512, bias=True)
    odd, _ = _lm(160, 256, 2, 512, bias=True)
    for blk in odd.layers:
        mx = blk.mixer
        mx.in_proj.bias = _unaligned(mx.in_proj.bias)
        mx.out_proj.bias = _unaligned(mx.out_proj.bias)
        mx.conv1d.weight = _unaligned(mx.conv1d.weight)
        mx.conv1d.bias = _unaligned(mx.conv1d.bias)
        blk.norm.weight = _unaligned(blk.norm.weight)
    assert all(blk.norm.weight.data_ptr() % 16 == 4 for blk in odd.layers)
    ids = _t(np.random.default_rng(160 + b).integers(0, 512, (b, 3), dtype=np.int64))
    ca = MambaCache.allocate(lm.cfg, b, DEV, torch.float32)
    co = MambaCache.allocate(odd.cfg, b, DEV, torch.float32)
    with torch.no_grad():
        for k in range(3):
            la = lm.step(ids[:, k:k + 1], ca)
            n = len(calls)
            lo = odd.step(ids[:, k:k + 1], co)
            assert len(calls) == n, "the unaligned model took the one-call batched step"
            assert_rel(_n(lo), _n(la), 1e-4, f"step {k} logits")
    assert len(calls) == (3 if b > 2 else 0)
    for i, (a_, o_) in enumerate(zip(ca.layers, co.layers)):
        assert_rel(_n(o_.conv_state), _n(a_.conv_state), 1e-4, f"layer {i} conv_state")
        assert_rel(_n(o_.ssm_state), _n(a_.ssm_state), 1e-4, f"layer {i} ssm_state")
