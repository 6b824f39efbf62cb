"""Host-side logic of the drop-in API (CPU only)."""
import numpy as np
import pytest
import torch

from _util import write_hf_snapshot
from mamba_lite import ops, tp_utils
from mamba_lite.cuda_graph import CUDAGraphUnsupported, GraphedStepper
from mamba_lite.model import LayerCache, MambaCache, MambaConfig, MambaLM, MambaMixer


def test_config_defaults_and_padding():
    """reference model.py:64-76"""
    c = MambaConfig(d_model=768, n_layer=24, vocab_size=50277)
    assert c.d_inner == 1536 and c.dt_rank == 48 and c.vocab_size == 50280
    c2 = MambaConfig(d_model=2048, n_layer=48, vocab_size=50280)
    assert c2.d_inner == 4096 and c2.dt_rank == 128 and c2.vocab_size == 50280
    assert MambaConfig(d_model=8, n_layer=1, vocab_size=8).dt_rank == 1


def test_from_hf_config(tmp_path):
    import json
    p = tmp_path / "config.json"
    p.write_text(json.dumps({"hidden_size": 768, "num_hidden_layers": 24, "vocab_size": 50280, "state_size": 16,
                             "conv_kernel": 4, "expand": 2, "time_step_rank": 48, "use_conv_bias": True,
                             "use_bias": False}))
    c = MambaConfig.from_hf_config(str(p))
    assert (c.d_model, c.n_layer, c.d_inner, c.dt_rank, c.layer_norm_epsilon) == (768, 24, 1536, 48, 1e-5)


def test_cache_allocate_shapes_and_dtypes():
    cfg = MambaConfig(d_model=32, n_layer=3, vocab_size=100, d_state=8)
    cache = MambaCache.allocate(cfg, 2, "cpu", torch.float32)
    assert len(cache.layers) == 3
    assert cache.layers[0].conv_state.shape == (2, 64, 3) and cache.layers[0].ssm_state.shape == (2, 64, 8)
    assert all(float(l.ssm_state.abs().sum()) == 0 for l in cache.layers)
    c16 = MambaCache.allocate(cfg, 1, "cpu", torch.bfloat16)
    assert c16.layers[0].conv_state.dtype == torch.bfloat16
    assert c16.layers[0].ssm_state.dtype == torch.float32   # fp32 SSM state with bf16 activations


def test_parameter_names_match_reference_state_dict():
    """Same keys as reference MambaLM (model.py:148-170, 317-322) so its state
    dicts load strictly."""
    cfg = MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8)
    keys = set(MambaLM(cfg).state_dict())
    expect = {"embedding.weight", "norm_f.weight", "layers.0.norm.weight", "layers.0.mixer.in_proj.weight",
              "layers.0.mixer.conv1d.weight", "layers.0.mixer.conv1d.bias", "layers.0.mixer.x_proj.weight",
              "layers.0.mixer.dt_proj.weight", "layers.0.mixer.dt_proj.bias", "layers.0.mixer.A_log",
              "layers.0.mixer.D", "layers.0.mixer.out_proj.weight"}
    assert keys == expect


def test_ssm_param_init():
    """reference model.py:172-181: A_log = log(1..N) per channel, D = 1."""
    m = MambaMixer(MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8), 0)
    np.testing.assert_allclose(m.A_log.detach().numpy(), np.log(np.tile(np.arange(1, 9), (64, 1))), rtol=1e-7)
    assert torch.equal(m.D.detach(), torch.ones(64))


def test_cpu_tensors_raise_instead_of_falling_back():
    m = MambaMixer(MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8), 0)
    with pytest.raises(RuntimeError, match="GPU"):
        m.prefill(torch.randn(1, 3, 32))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.quant_dequant_sum_int8_tok([torch.randn(4, 8), torch.randn(4, 8)])


def test_shape_validation_before_launch():
    with pytest.raises(ValueError):
        ops.selective_scan(torch.randn(1, 8, 4), torch.randn(1, 8, 5), torch.randn(8, 4), torch.randn(1, 4, 4),
                           torch.randn(1, 4, 4))
    with pytest.raises(ValueError):
        ops.causal_conv1d(torch.randn(1, 8, 4), torch.randn(7, 4))
    # the one-call batched step takes d_model from h: a row of another width
    # or a norm_f of another length would stride the weights wrongly
    cfg = MambaConfig(d_model=256, n_layer=2, vocab_size=64)
    for h, nf in ((torch.zeros(4, 384), torch.ones(384)), (torch.zeros(4, 256), torch.ones(384))):
        with pytest.raises(ValueError):
            ops.decode_step_batched(None, h, nf, 1e-5, cfg, False)
    # the one-call prefills: a final norm of another width than h's rows
    for fn in (ops.prefill_short, ops.prefill_long):
        with pytest.raises(ValueError, match="norm_f"):
            fn(torch.zeros(1, 8, 256), None, torch.ones(384), 1e-5, 512, 16, 16, 4)


def test_graphed_stepper_rejects_cpu():
    """reference cuda_graph.py:62-65"""
    cfg = MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8)
    with pytest.raises(CUDAGraphUnsupported):
        GraphedStepper(MambaLM(cfg), MambaCache.allocate(cfg, 1, "cpu", torch.float32), 1, "cpu")


def test_graphed_prefill_rejects_cpu():
    from mamba_lite.cuda_graph import GraphedPrefill
    cfg = MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8)
    with pytest.raises(CUDAGraphUnsupported):
        GraphedPrefill(MambaLM(cfg), MambaCache.allocate(cfg, 1, "cpu", torch.float32), 1, 8, "cpu")


def test_graphed_stepper_rejects_int8_legacy():
    class M:
        allreduce_dtype = {(0, "x_proj"): "int8_legacy"}
    if not torch.cuda.is_available():
        pytest.skip("the device check fires first without a GPU")
    with pytest.raises(CUDAGraphUnsupported):
        GraphedStepper(M(), None, 1, "cuda")


def test_channel_slice_and_payload_bytes():
    assert tp_utils.channel_slice(1, 2, 4096) == slice(2048, 4096)
    with pytest.raises(AssertionError):
        tp_utils.channel_slice(0, 3, 4096)
    assert tp_utils.int8_tok_payload_nbytes(32768, 768) == 25_296_896


def test_shard_params_partition_the_dense_mixer():
    torch.manual_seed(0)
    cfg = MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8, bias=True)
    dense = MambaMixer(cfg, 0)
    s0 = tp_utils.shard_mixer_params(dense, 0, 2)
    s1 = tp_utils.shard_mixer_params(dense, 1, 2)
    Di = cfg.d_inner
    w = dense.in_proj.weight.detach()
    # x rows and z rows are split separately (reference tp_model.py:194-197)
    assert torch.equal(torch.cat([s0["in_proj.weight"][:Di // 2], s1["in_proj.weight"][:Di // 2]]), w[:Di])
    assert torch.equal(torch.cat([s0["in_proj.weight"][Di // 2:], s1["in_proj.weight"][Di // 2:]]), w[Di:])
    assert torch.equal(torch.cat([s0["x_proj.weight"], s1["x_proj.weight"]], 1), dense.x_proj.weight.detach())
    assert torch.equal(s1["out_proj.bias"], torch.zeros_like(dense.out_proj.bias))
    assert torch.equal(s0["out_proj.bias"], dense.out_proj.bias.detach())


def test_naive_shard_cuts_the_packed_in_proj():
    """Reference NaiveTPMambaMixer (tp_model.py:217-244): at world_size 2
    rank 0 gets only x rows and rank 1 only z rows."""
    torch.manual_seed(0)
    cfg = MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8)
    dense = MambaMixer(cfg, 0)
    Di = cfg.d_inner
    w = dense.in_proj.weight.detach()
    assert torch.equal(tp_utils.naive_shard_mixer_params(dense, 0, 2)["in_proj.weight"], w[:Di])
    n1 = tp_utils.naive_shard_mixer_params(dense, 1, 2)
    assert torch.equal(n1["in_proj.weight"], w[Di:])
    assert torch.equal(n1["x_proj.weight"], tp_utils.shard_mixer_params(dense, 1, 2)["x_proj.weight"])


def test_site_dtype_lookup():
    """Reference tests/test_per_site_allreduce.py:69-74, plus the variants not built here."""
    assert tp_utils.site_dtype("fp16", 5, "x_proj") == "fp16"
    m = {(2, "out_proj"): "int8_gather_tok"}
    assert tp_utils.site_dtype(m, 2, "out_proj") == "int8_gather_tok"
    assert tp_utils.site_dtype(m, 2, "x_proj") == "fp32"
    assert tp_utils.site_dtype(m, 3, "out_proj") == "fp32"
    assert tp_utils.site_dtype("int8", 0, "x_proj") == "int8"
    with pytest.raises(AssertionError):
        tp_utils.site_dtype("fp32", 0, "in_proj")
    with pytest.raises(AssertionError):
        tp_utils.site_dtype("bf8", 0, "x_proj")
    for unbuilt in ("int8_legacy", "int8_sum", "int8_gather"):
        with pytest.raises(NotImplementedError):
            tp_utils.site_dtype({(0, "x_proj"): unbuilt}, 0, "x_proj")


def test_layer_cache_is_a_dataclass_pair():
    lc = LayerCache(conv_state=torch.zeros(1, 2, 3), ssm_state=torch.zeros(1, 2, 4))
    assert lc.conv_state.shape == (1, 2, 3) and lc.ssm_state.shape == (1, 2, 4)


def test_product_package_never_imports_the_oracle():
    """The oracle is test infrastructure: nothing under the package may import
    or load it (no CPU fallback path)."""
    import os
    import re
    pkg = os.path.join(os.path.dirname(__file__), "..", "mamba-tp-lite_amd")
    pat = re.compile(r"^\s*(from\s+oracle\b|import\s+oracle\b)|['\"]oracle[/'\"]", re.M)
    hits = []
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".cpp", ".h")):
                path = os.path.join(dirpath, f)
                with open(path, encoding="utf-8") as fh:
                    if pat.search(fh.read()):
                        hits.append(path)
    assert hits == []


@pytest.mark.parametrize("shards", [1, 3])
def test_from_pretrained_local_snapshot(tmp_path, shards):
    """reference model.py:28-47 (single file or index-named shards) and
    367-397 (backbone. prefix, embeddings -> embedding, strict load)."""
    torch.manual_seed(0)
    cfg = MambaConfig(d_model=32, n_layer=2, vocab_size=64, d_state=8)
    src = MambaLM(cfg)
    with torch.no_grad():
        for p in src.parameters():
            p.normal_()
    sd = {k: v.detach().clone() for k, v in src.state_dict().items()}
    write_hf_snapshot(tmp_path, cfg, sd, shards)
    m = MambaLM.from_pretrained(str(tmp_path))
    got = m.state_dict()
    assert set(got) == set(sd)
    for k in sd:
        assert torch.equal(got[k], sd[k]), k
    assert m.cfg.d_inner == 64 and m.cfg.dt_rank == 2


def test_from_pretrained_missing_checkpoint(tmp_path):
    from mamba_lite.model import load_hf_state_dict
    with pytest.raises(FileNotFoundError):
        load_hf_state_dict(str(tmp_path))


def test_gemm_table_file_is_well_formed():
    """The committed TunableOp table: validator lines for torch, HIP,
    hipBLASLt, rocBLAS and gfx950, then one fp32 GEMM entry per tuned shape
    with a solution name and a time."""
    import csv
    from mamba_lite import gemm_table
    rows = list(csv.reader(open(gemm_table.TABLE)))
    validators = {r[1]: r[2] for r in rows if r[0] == "Validator"}
    assert {"PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION", "GCN_ARCH_NAME"} <= set(validators)
    assert validators["GCN_ARCH_NAME"].startswith("gfx950")
    gemms = [r for r in rows if r[0].startswith("GemmTunableOp_float")]
    assert len(gemms) >= 5 and all(len(r) == 4 and float(r[3]) > 0 for r in gemms)
    # a CPU-only process keeps the default GEMM paths
    if not __import__("torch").cuda.is_available():
        assert gemm_table.enable() is False


def test_local_tp_mixer_needs_a_divisible_world_size():
    """Reference tp_model.py:65 (d_inner % world_size == 0)."""
    from mamba_lite.tp_model import LocalTPMixer
    cfg = MambaConfig(d_model=32, n_layer=1, vocab_size=100, d_state=8)
    with pytest.raises(AssertionError):
        LocalTPMixer(cfg, world_size=3)
    with pytest.raises(RuntimeError, match="no shards"):
        LocalTPMixer(cfg, world_size=2).prefill(torch.randn(1, 2, 32))


def test_generate_has_no_sampling_path():
    """The reference's generate(greedy=False) leaves the first token None
    (model.py:359) and fails in its first step; here it is a clear error
    raised before any work (no GPU needed)."""
    cfg = MambaConfig(d_model=32, n_layer=1, vocab_size=64, d_state=8)
    model = MambaLM(cfg)
    with pytest.raises(NotImplementedError):
        model.generate(torch.zeros(1, 3, dtype=torch.long), 2, greedy=False)


@pytest.mark.parametrize("rows,M,D,N,R,K,ok", [
    (64, 768, 1536, 16, 48, 4, True),       # 130m shape, 64 tokens
    (1, 2048, 4096, 16, 128, 4, True),      # 1.4b shape, one token
    (65, 768, 1536, 16, 48, 4, False),      # more than 64 token rows
    (64, 128, 512, 16, 8, 4, False),        # d_model below 256
    (64, 320, 1024, 16, 20, 4, False),      # d_model not a multiple of 128
    (64, 384, 768, 16, 24, 4, False),       # d_inner not a multiple of 512
    (64, 768, 1536, 17, 48, 4, False),      # d_state above 16
    (64, 768, 1536, 15, 48, 4, False),      # dt_rank + 2 d_state not a multiple of 4
    (64, 768, 1536, 16, 161, 4, False),     # dt_rank above 160
    (64, 768, 1536, 16, 48, 5, False),      # conv width 5
    (64, 768, 1536, 16, 48, 1, False),      # conv width 1
])
def test_prefill_short_covers_the_sizes_its_kernels_take(rows, M, D, N, R, K, ok):
    """ops.prefill_short_ok admits exactly the sizes mtl_prefill_short
    checks on the host (the same bounds the C-ABI rejection tests hold)."""
    assert ops.prefill_short_ok(rows, M, D, N, R, K) is ok


@pytest.mark.parametrize("b,l,M,D,N,R,K,ok", [
    (1, 100, 256, 512, 16, 16, 4, True),
    (1, 100, 256, 512, 16, 16, 1, True),           # d_conv 1
    (1, 100, 96, 192, 16, 256, 4, False),          # dt_rank above d_inner
    (65536, 1, 256, 512, 16, 16, 4, False),        # batch rows
    (1, 1 << 20, 1, 1, 1, 1, 4, False),            # seqlen past the conv grid
    (1, 65535 * 16, 1, 1, 1, 1, 4, True),
    (4096, 257, 256, 512, 16, 16, 4, False),       # b l past 2^20
    (1, 100, 256, 512, 33, 16, 4, False),          # d_state
    (1, 100, 256, 512, 16, 16, 9, False),          # d_conv
    (1, 100, 1 << 17, 512, 16, 16, 4, False),      # d_model
])
def test_prefill_long_covers_the_sizes_its_checks_take(b, l, M, D, N, R, K, ok):
    """ops.prefill_long_ok admits exactly the sizes mtl_prefill_long checks
    before its first launch (the C-ABI rejection tests hold the same
    bounds), so MambaLM never hands it a prompt it rejects."""
    assert ops.prefill_long_ok(b, l, M, D, N, R, K) is ok


def test_a_dt_rank_above_d_inner_takes_the_per_op_prefill():
    """The reference allows dt_rank > d_inner (dt_proj is a Linear(dt_rank,
    d_inner)); neither one-call prefill takes it, so prefill() runs op by op
    for every prompt length."""
    model = MambaLM(MambaConfig(d_model=96, n_layer=1, vocab_size=64, dt_rank=256))
    assert model._native_prefill_kind(1, 5) is None and model._native_prefill_kind(2, 300) is None


def test_native_prefill_is_not_taken_off_the_gpu():
    """MambaLM._prefill_native declines CPU token ids (short and long
    prompts) before touching the library, so prefill() keeps its other paths
    there."""
    cfg = MambaConfig(d_model=256, n_layer=1, vocab_size=64, d_state=16)
    model = MambaLM(cfg)
    assert model._native_prefill_kind(1, 8) == "short" and model._native_prefill_kind(1, 300) == "long"
    for l in (8, 300):
        assert model._prefill_native(torch.zeros(1, l, dtype=torch.long), None, None) is None
    assert not hasattr(model, "_short_plan")


@pytest.mark.parametrize("bias,conv_bias", [(False, True), (True, False)])
def test_layer_tensors_are_the_step_parameters_in_order(bias, conv_bias):
    """MambaLM._layer_tensors() reads each layer's parameters through the
    modules' dicts: the very parameter objects attribute access gives, in the
    order of the _LT_* indices (the one-call steps build their weight
    records from it), with absent biases as None; a replaced weight is
    seen at once."""
    import mamba_lite.model as mm
    model = MambaLM(MambaConfig(d_model=64, n_layer=2, vocab_size=64, bias=bias, conv_bias=conv_bias))
    for blk, lt in zip(model.layers, model._layer_tensors()):
        mx = blk.mixer
        want = {mm._LT_NORM: blk.norm.weight, mm._LT_W_IN: mx.in_proj.weight, mm._LT_B_IN: mx.in_proj.bias,
                mm._LT_CONV_W: mx.conv1d.weight, mm._LT_CONV_B: mx.conv1d.bias, mm._LT_XPROJ: mx.x_proj.weight,
                mm._LT_W_DT: mx.dt_proj.weight, mm._LT_B_DT: mx.dt_proj.bias, mm._LT_A_LOG: mx.A_log,
                mm._LT_D: mx.D, mm._LT_W_OUT: mx.out_proj.weight, mm._LT_B_OUT: mx.out_proj.bias}
        assert len(lt) == len(want) == 12
        for k, t in want.items():
            assert lt[k] is t, k
        assert (lt[mm._LT_B_IN] is None) == (not bias) and (lt[mm._LT_CONV_B] is None) == (not conv_bias)
    model.layers[1].mixer.out_proj.weight = torch.nn.Parameter(torch.zeros(64, 128))
    assert model._layer_tensors()[1][mm._LT_W_OUT] is model.layers[1].mixer.out_proj.weight


def test_unaligned_parameters_keep_the_native_step_records_out():
    """The one-call steps' weight records (_batched_template,
    _decode_step_template) are built only from parameters the library can
    load in 16-byte runs; a parameter that starts 4 bytes off a 16-byte
    boundary (a view into a larger buffer) makes them None, so the step runs
    a path that takes it, instead of an entry point that rejects it."""
    model = MambaLM(MambaConfig(d_model=256, n_layer=2, vocab_size=64, bias=True)).eval()
    dev = torch.device("cpu")

    def unaligned(p):
        buf = torch.empty(p.numel() + 1, dtype=p.dtype)
        v = buf[1:].view_as(p)
        v.copy_(p.detach())
        return torch.nn.Parameter(v, requires_grad=False)

    assert model._batched_template(model._layer_tensors(), dev, 256) is not None
    for split_k in (True, False):
        assert model._decode_step_template(model._decode_plan(), split_k, dev) is not None
    mx = model.layers[1].mixer
    mx.out_proj.bias = unaligned(mx.out_proj.bias)
    assert model._batched_template(model._layer_tensors(), dev, 256) is None
    for split_k in (True, False):   # biases are read a float at a time there
        assert model._decode_step_template(model._decode_plan(), split_k, dev) is not None
    mx.in_proj.weight = unaligned(mx.in_proj.weight)
    for split_k in (True, False):
        assert model._decode_step_template(model._decode_plan(), split_k, dev) is None


def test_persistent_decode_grid_query():
    """mtl_decode_persist_grid: the 130m shape takes 64 workgroups with the
    first blocking and 128 with the second; shapes outside the kernel's
    register blocking return 0 (the step then runs kernel by kernel)."""
    from mamba_lite import _lib
    lib = _lib.load()
    assert lib.mtl_decode_persist_grid(768, 1536, 16, 48, 4, 24, 0) == 64
    assert lib.mtl_decode_persist_grid(768, 1536, 16, 48, 4, 24, 1) == 64
    assert lib.mtl_decode_persist_grid(768, 1536, 16, 48, 4, 24, 2) == 128
    assert lib.mtl_decode_persist_grid(2048, 4096, 16, 128, 4, 48, 0) == 0     # 1.4b: too wide
    assert lib.mtl_decode_persist_grid(1024, 2048, 16, 64, 4, 48, 0) == 0      # partials exceed the exchange lanes
    assert lib.mtl_decode_persist_grid(768, 1536, 16, 48, 4, 65, 0) == 0       # cache pointers: 64 layers at most
    assert lib.mtl_decode_persist_grid(768, 1536, 16, 48, 8, 24, 0) == 0       # d_conv 8


def test_persistent_workspace_error_word_and_reset():
    """The error word is bytes 4..8 of the workspace (an unsigned code, 0 when
    no wait timed out); the reset zero-fills epoch, error word and slots."""
    from mamba_lite import ops
    cfg = MambaConfig(d_model=768, n_layer=1, vocab_size=8)
    ws = ops.decode_persist_workspace(cfg, "cpu")
    assert ws.numel() == 256 + 8 * (288 * 80 + 2048 + 1024) and int(ws.sum()) == 0
    assert ops.decode_persist_error(ws) == 0
    ws[0:4].view(torch.int32)[0] = 7                       # an epoch
    ws[4:8].view(torch.int32)[0] = -3                      # code 0xFFFFFFFD
    ws[300] = 9                                           # a slot byte
    assert ops.decode_persist_error(ws) == 0xFFFFFFFD
    ops.reset_decode_persist_workspace(ws)
    assert int(ws.sum()) == 0 and ops.decode_persist_error(ws) == 0
    with pytest.raises(ValueError):
        ops.decode_persist_error(torch.zeros(4, dtype=torch.uint8))


def test_from_pretrained_loads_in_proj_bias_of_a_bias_snapshot(tmp_path):
    """A `use_bias: true` snapshot: the in_proj and out_proj biases are both
    loaded.  (The reference's loader remaps out_proj.bias only, so its strict
    load of such a snapshot stops on the missing in_proj.bias, model.py:
    392-396; loading it is this library's deliberate deviation.)"""
    import _golden as G
    import torch
    from _util import write_hf_snapshot
    from mamba_lite.model import MambaConfig, MambaLM
    cfg = MambaConfig(d_model=64, n_layer=2, vocab_size=128, bias=True)
    sd = G.lm_weights(12, 64, 2, 128, bias=True)
    write_hf_snapshot(tmp_path, cfg, {k: torch.from_numpy(v) for k, v in sd.items()})
    lm = MambaLM.from_pretrained(str(tmp_path))
    got = lm.state_dict()
    assert set(got) == set(sd)
    for k, v in sd.items():
        assert torch.equal(got[k], torch.from_numpy(v)), k
    assert lm.layers[1].mixer.in_proj.bias is not None and lm.layers[1].mixer.out_proj.bias is not None
