"""Tensor-parallel mixer and model with every rank on one GPU (mamba_lite.tp_model),
checked the way the reference checks its 2-process TPMambaMixer
(tests/test_tp_correctness.py:76-88, tests/test_quantized_allreduce.py:73-87,
tests/test_per_site_allreduce.py:77-112): the correct channel split equals the
dense mixer (1e-4) with exactly two all-reduces per call, the naive
packed-tensor split does not, an all-fp32 site map is bit-identical to the
global fp32 setting, an int8 site changes only its own site, fp16 is close but
not exact, and the per-token int8 all-reduce is close but lossy with under a
third of the fp32 wire bytes.  Beyond the reference's tests: prefill
continuation from per-rank caches, a teacher-forced step loop against the
dense step and the dense prefill, and the full TP model (LocalTPLM) against
the dense LM, loaded shard by shard from a local safetensors snapshot."""
import pytest
import torch

from _util import write_hf_snapshot
from mamba_lite.model import LayerCache, MambaConfig, MambaLM, MambaMixer
from mamba_lite.tp_model import LocalTPLM, LocalTPMixer

pytestmark = pytest.mark.gpu
DEV = "cuda"
LAYER = 3

CASES = [  # (d_model, d_state, batch, seqlen, world_size): the reference's small config, then the 130m width
    (32, 8, 2, 5, 2), (768, 16, 2, 33, 2), (768, 16, 1, 40, 4)]


def _dense(d_model, d_state, seed=0):
    torch.manual_seed(seed)
    cfg = MambaConfig(d_model=d_model, n_layer=1, vocab_size=100, d_state=d_state, d_conv=4, expand=2)
    with torch.device(DEV):
        return MambaMixer(cfg, layer_idx=0).eval()


def _x(b, l, d_model):
    torch.manual_seed(123)
    return torch.randn(b, l, d_model, device=DEV)


@pytest.mark.parametrize("d_model,d_state,b,l,ws", CASES)
def test_correct_split_matches_dense_with_two_allreduces(d_model, d_state, b, l, ws):
    print(f"tp local prefill d_model={d_model} b={b} l={l} ws={ws}", flush=True)
    dense = _dense(d_model, d_state)
    x = _x(b, l, d_model)
    tp = LocalTPMixer.from_dense(dense, ws)
    with torch.no_grad():
        ref, ref_conv, ref_ssm = dense.prefill(x)
        out, conv, ssm = tp.prefill(x)
    torch.testing.assert_close(out, ref, atol=1e-4, rtol=1e-4)
    assert tp.comm.count == 2
    S = dense.cfg.d_inner // ws
    for r in range(ws):
        sl = slice(r * S, (r + 1) * S)
        # the shard's in_proj is a GEMM of another shape: BLAS may sum in another order
        torch.testing.assert_close(conv[r], ref_conv[:, sl], atol=1e-4, rtol=1e-4)
        torch.testing.assert_close(ssm[r], ref_ssm[:, sl], atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("d_model,d_state,b,l,ws", CASES[1:])
def test_prefill_continues_from_rank_caches(d_model, d_state, b, l, ws):
    print(f"tp local continuation d_model={d_model} ws={ws}", flush=True)
    dense = _dense(d_model, d_state)
    x = _x(b, l, d_model)
    tp = LocalTPMixer.from_dense(dense, ws)
    k = l // 3
    with torch.no_grad():
        ref, _, ref_ssm = dense.prefill(x)
        _, conv, ssm = tp.prefill(x[:, :k])
        caches = [LayerCache(c, h) for c, h in zip(conv, ssm)]
        out, _, ssm2 = tp.prefill(x[:, k:], caches)
    torch.testing.assert_close(out, ref[:, k:], atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(torch.cat(ssm2, dim=1), ref_ssm, atol=1e-4, rtol=1e-4)
    assert tp.comm.count == 4


@pytest.mark.parametrize("d_model,d_state,b,l,ws", CASES)
def test_step_matches_dense_step_and_prefill(d_model, d_state, b, l, ws):
    print(f"tp local step d_model={d_model} b={b} ws={ws}", flush=True)
    dense = _dense(d_model, d_state)
    cfg = dense.cfg
    x = _x(b, l, d_model)
    tp = LocalTPMixer.from_dense(dense, ws)
    caches = tp.allocate_caches(b, device=DEV)
    dcache = LayerCache(torch.zeros(b, cfg.d_inner, cfg.d_conv - 1, device=DEV),
                        torch.zeros(b, cfg.d_inner, cfg.d_state, device=DEV))
    addrs = [(c.conv_state.data_ptr(), c.ssm_state.data_ptr()) for c in caches]
    with torch.no_grad():
        ref, ref_conv, ref_ssm = dense.prefill(x)
        for t in range(l):
            o = tp.step(x[:, t], caches)
            od = dense.step(x[:, t], dcache)
            torch.testing.assert_close(o, od, atol=1e-4, rtol=1e-4)
            torch.testing.assert_close(o, ref[:, t], atol=1e-4, rtol=1e-4)
    assert tp.comm.count == 2 * l
    assert [(c.conv_state.data_ptr(), c.ssm_state.data_ptr()) for c in caches] == addrs   # in place
    torch.testing.assert_close(torch.cat([c.conv_state for c in caches], 1), ref_conv, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(torch.cat([c.ssm_state for c in caches], 1), ref_ssm, atol=1e-4, rtol=1e-4)


def test_naive_split_gives_wrong_result():
    dense = _dense(32, 8)
    x = _x(2, 5, 32)
    with torch.no_grad():
        ref = dense(x)
        out = LocalTPMixer.from_dense(dense, 2, naive=True)(x)
    assert not torch.allclose(out, ref, atol=1e-2)


@pytest.mark.parametrize("d_model,d_state,b,l,ws", CASES[:2])
def test_fp16_allreduce_close_but_not_exact(d_model, d_state, b, l, ws):
    dense = _dense(d_model, d_state)
    x = _x(b, l, d_model)
    with torch.no_grad():
        ref = dense(x)
        out = LocalTPMixer.from_dense(dense, ws, allreduce_dtype="fp16")(x)
    torch.testing.assert_close(out, ref, atol=1e-2, rtol=1e-2)
    assert not torch.allclose(out, ref, atol=1e-6)


@pytest.mark.parametrize("d_model,d_state,b,l,ws", CASES[:2])
def test_int8_allreduce_close_but_lossy(d_model, d_state, b, l, ws):
    dense = _dense(d_model, d_state)
    x = _x(b, l, d_model)
    with torch.no_grad():
        ref = dense(x)
        tp8 = LocalTPMixer.from_dense(dense, ws, allreduce_dtype="int8_gather_tok")
        tp32 = LocalTPMixer.from_dense(dense, ws)
        out = tp8(x)
        tp32(x)
    torch.testing.assert_close(out, ref, atol=0.1, rtol=0.2)
    assert not torch.allclose(out, ref, atol=1e-6)
    assert (out - ref).abs().max().item() < 0.15 * ref.abs().max().item()
    assert tp8.comm.count == tp32.comm.count == 2 and tp8.comm.bytes < tp32.comm.bytes / 3


def test_per_site_dtype_map():
    """tests/test_per_site_allreduce.py:20-31, 77-112 on the sites built here."""
    specs = {
        "fp32_str": ("fp32", LAYER),
        "fp32_map": ({(LAYER, "x_proj"): "fp32", (LAYER, "out_proj"): "fp32"}, LAYER),
        "empty_map": ({}, LAYER),
        "int8_out_only_hit": ({(LAYER, "out_proj"): "int8_gather_tok"}, LAYER),
        "int8_out_only_miss": ({(LAYER, "out_proj"): "int8_gather_tok"}, LAYER + 1),
        "int8_x_only": ({(LAYER, "x_proj"): "int8_gather_tok"}, LAYER),
        "int8_gather_tok_all": ("int8_gather_tok", LAYER),
        "int8_all": ("int8", LAYER),
        "fp16_all": ("fp16", LAYER),
    }
    dense = _dense(32, 8)
    x = _x(2, 5, 32)
    res = {}
    with torch.no_grad():
        ref = dense(x)
        for name, (spec, layer) in specs.items():
            tp = LocalTPMixer.from_dense(dense, 2, allreduce_dtype=spec, layer_idx=layer)
            res[name] = (tp(x), tp.comm.count, tp.comm.bytes)
    base = res["fp32_str"][0]
    assert torch.equal(res["fp32_map"][0], base) and torch.equal(res["empty_map"][0], base)
    torch.testing.assert_close(base, ref, atol=1e-5, rtol=0)
    assert all(c == 2 for _, c, _ in res.values())
    assert not torch.equal(res["int8_out_only_hit"][0], base)
    assert torch.equal(res["int8_out_only_miss"][0], base)
    assert not torch.equal(res["int8_x_only"][0], base)
    assert torch.equal(res["int8_all"][0], res["int8_gather_tok_all"][0])
    assert res["int8_gather_tok_all"][2] < res["fp32_str"][2] / 3
    for name in ("int8_gather_tok_all", "fp16_all", "int8_x_only", "int8_out_only_hit"):
        assert (res[name][0] - ref).abs().max().item() < 0.15 * ref.abs().max().item(), name


def test_rank_caches_are_this_ranks_channels_only():
    dense = _dense(768, 16)
    tp = LocalTPMixer.from_dense(dense, 4)
    caches = tp.allocate_caches(3, device=DEV)
    assert len(caches) == 4
    for c in caches:
        assert tuple(c.conv_state.shape) == (3, 384, 3) and tuple(c.ssm_state.shape) == (3, 384, 16)
        assert c.ssm_state.dtype == torch.float32 and not c.conv_state.any() and not c.ssm_state.any()


@pytest.mark.parametrize("ws,shards", [(2, 1), (4, 3)])
def test_tp_lm_matches_dense_lm(tmp_path, ws, shards):
    """tests/test_tp_lm_correctness.py:43-81 on a synthetic local snapshot
    (no checkpoint is reachable offline): the TP LM loaded shard by shard
    from safetensors gives the dense LM's prefill logits and greedy tokens,
    with 2 AllReduces per prefill or step on layer 0 (prefill + generate of 8
    tokens = 2 * (1 + 1 + 7) = 18)."""
    print(f"tp local lm ws={ws} shards={shards}", flush=True)
    torch.manual_seed(0)
    cfg = MambaConfig(d_model=64, n_layer=3, vocab_size=256, d_state=16)
    src = MambaLM(cfg)
    write_hf_snapshot(tmp_path, cfg, {k: v.detach().clone() for k, v in src.state_dict().items()}, shards)
    dense = MambaLM.from_pretrained(str(tmp_path)).to(DEV).eval()
    tp = LocalTPLM.from_pretrained_shard(str(tmp_path), ws, device=DEV)
    torch.manual_seed(42)
    ids = torch.randint(0, cfg.vocab_size, (1, 12), device=DEV)
    with torch.no_grad():
        dense_logits, _ = dense.prefill(ids)
        dense_tokens = dense.generate(ids, max_new_tokens=8)
        tp_logits, _ = tp.prefill(ids)
        tp_tokens = tp.generate(ids, max_new_tokens=8)
    torch.testing.assert_close(tp_logits, dense_logits, atol=1e-4, rtol=1e-4)
    assert torch.equal(tp_tokens, dense_tokens), (tp_tokens.tolist(), dense_tokens.tolist())
    assert tp.layers[0].mixer.comm.count == 18


def test_tp_lm_teacher_forced_steps_match_prefill():
    """A prefill of the first token, then steps over the rest, reproduce the
    full prefill's logits (reference tests/test_correctness.py:49-72 on the
    TP model), from a dense LM sharded in memory at batch 2."""
    torch.manual_seed(1)
    cfg = MambaConfig(d_model=128, n_layer=2, vocab_size=300, d_state=16)
    with torch.device(DEV):
        dense = MambaLM(cfg).eval()
    tp = LocalTPLM.from_dense(dense, 2)
    ids = torch.randint(0, cfg.vocab_size, (2, 10), device=DEV)
    with torch.no_grad():
        full, _ = tp.prefill(ids)
        dense_full, _ = dense.prefill(ids)
        first, cache = tp.prefill(ids[:, :1])
        steps = [first] + [tp.step(ids[:, t:t + 1], cache) for t in range(1, ids.shape[1])]
    torch.testing.assert_close(full, dense_full, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(torch.cat(steps, 1), full, atol=1e-4, rtol=1e-4)
    assert len(cache.layers) == 2 and len(cache.layers[0]) == 2
    assert tuple(cache.layers[1][1].ssm_state.shape) == (2, cfg.d_inner // 2, 16)


def test_bf16_split_tracks_the_dense_bf16_mixer():
    """bf16 activations with fp32 SSM state, as the TP-rank shard workload
    runs: the split over 2 ranks tracks the dense bf16 mixer within the bf16
    tolerance (each rank's partial sums round to bf16 before the fp32
    all-reduce, the dense GEMM rounds once), and keeps fp32 rank states."""
    dense = _dense(256, 16).to(torch.bfloat16)
    x = _x(2, 37, 256).bfloat16()
    with torch.no_grad():
        ref, _, ref_h = dense.prefill(x)
        out, _, h = LocalTPMixer.from_dense(dense, 2).prefill(x)
    assert out.dtype == torch.bfloat16 and all(t.dtype == torch.float32 for t in h)
    torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(torch.cat(h, 1), ref_h, atol=2e-2, rtol=2e-2)
