"""The C-ABI library loads and exports every symbol include/mtl.h declares
(CPU only: no kernel is launched)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mtl.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mtl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for n in ("mtl_selective_scan_fwd", "mtl_causal_conv1d_fwd", "mtl_conv_step", "mtl_selective_state_update",
              "mtl_add_rmsnorm", "mtl_quant_dequant_sum_int8_tok", "mtl_quant_dequant_sum_fp16",
              "mtl_last_error", "mtl_abi_version"):
        assert n in names


def test_library_loads_and_exports_every_declared_symbol():
    from mamba_lite import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: build with python mamba-tp-lite_amd/build.py")
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.mtl_abi_version() == _lib.ABI_VERSION
    assert lib.mtl_last_error() == b""


def test_struct_layouts_match_header():
    """ctypes mirrors follow the header field order: 8-byte fields, then four
    int32 flags."""
    from mamba_lite import _lib

    assert ctypes.sizeof(_lib.ScanParams) == 8 * (6 * 4 + 5 + 4) + 4 * 4
    assert ctypes.sizeof(_lib.ConvParams) == 8 * (2 * 4 + 4 + 3) + 4 * 4
    # mtl_prefill_layer: norm_w, eps + reserved, 15 pointers
    assert ctypes.sizeof(_lib.PrefillLayer) == 8 + 4 + 4 + 15 * 8
    assert _lib.PrefillLayer.W_in.offset == 16
    # mtl_prefill_short_args: 11 pointers, eps_f and three int32, six int64 sizes
    assert ctypes.sizeof(_lib.PrefillShortArgs) == 11 * 8 + 4 * 4 + 6 * 8
    assert _lib.PrefillShortArgs.batch.offset == 104
    # mtl_prefill_long_args: 9 pointers, blas_ws_bytes, 2 pointers, eps_f and three int32, six int64 sizes
    assert ctypes.sizeof(_lib.PrefillLongArgs) == 12 * 8 + 4 * 4 + 6 * 8
    assert _lib.PrefillLongArgs.batch.offset == 112
    # mtl_decode_layer: norm_w, eps + reserved, 14 pointers
    assert ctypes.sizeof(_lib.DecodeLayer) == 8 + 4 + 4 + 14 * 8
    # mtl_decode_step_args: 11 pointers, eps_f, then eleven int32
    assert ctypes.sizeof(_lib.DecodeStepArgs) == 11 * 8 + 4 + 11 * 4
    assert _lib.DecodeStepArgs.eps_f.offset == 88
    # mtl_decode_step_batched_args: 13 pointers, eps_f, then nine int32
    assert ctypes.sizeof(_lib.DecodeStepBatchedArgs) == 13 * 8 + 4 + 9 * 4
    assert _lib.DecodeStepBatchedArgs.eps_f.offset == 104
    assert _lib.DecodeStepBatchedArgs.fold.offset == 136


def test_invalid_arguments_are_rejected_without_a_gpu():
    """Host-side validation in the library returns an error code and a
    message before any launch."""
    from mamba_lite import _lib

    lib = _lib.load()
    p = _lib.ScanParams()
    p.batch, p.seqlen, p.dim, p.dstate = 1, 4, 8, 64   # dstate > 32
    rc = lib.mtl_selective_scan_fwd(ctypes.byref(p), None)
    assert rc == 1 and b"dstate" in lib.mtl_last_error()
    rc = lib.mtl_quant_dequant_sum_int8_tok(None, 2, 4, 4, None, None, None)
    assert rc == 1 and b"parts" in lib.mtl_last_error()
    c = _lib.ConvParams()
    c.batch, c.seqlen, c.dim, c.width = 1, 4, 8, 9     # width > 8
    assert lib.mtl_causal_conv1d_fwd(ctypes.byref(c), None) == 1
    assert b"width" in lib.mtl_last_error()


@pytest.mark.parametrize("case", [
    ("mtl_decode_in", dict(batch=3), b"batch must be 1, 2 or 4"),
    ("mtl_decode_in", dict(d_model=6), b"d_model"),
    ("mtl_decode_in", dict(channels_per_block=16), b"channels_per_block"),
    ("mtl_decode_in", dict(channels_per_block=2), b"channels_per_block must be 8 or 4"),
    ("mtl_decode_in", dict(d_conv=9), b"bad sizes"),
    ("mtl_decode_in", dict(d_conv=1), b"bad sizes"),
    ("mtl_decode_in", dict(first_layer=True, vocab=0), b"vocab"),
    ("mtl_decode_gemv", dict(batch=8), b"batch must be 1, 2 or 4"),
    ("mtl_decode_gemv", dict(cols=8192), b"cols"),
    ("mtl_decode_norm_gemv", dict(batch=3), b"batch must be 1, 2 or 4"),
    ("mtl_decode_norm_gemv", dict(cols=6), b"cols"),
    ("mtl_decode_ssm", dict(d_state=17), b"d_state"),
    ("mtl_decode_ssm", dict(dt_rank=300), b"dt_rank"),
    ("mtl_decode_ssm", dict(nblk=1000), b"partial blocks"),
    ("mtl_sum_parts", dict(nparts=0), b"nparts"),
    ("mtl_sum_parts", dict(nparts=-3), b"nparts"),
    ("mtl_conv_step_xproj", dict(batch=33), b"batch"),
    ("mtl_conv_step_xproj", dict(xdbl_cols=289), b"xdbl_cols"),
    ("mtl_conv_step_xproj", dict(width=9), b"width"),
    ("mtl_conv_step_xproj", dict(width=0), b"width"),
    ("mtl_selective_state_update", dict(dstate=17), b"dstate"),
    ("mtl_selective_state_update", dict(dt_rank=257), b"dt_rank"),
    ("mtl_conv_step", dict(width=9), b"width"),
    ("mtl_decode_gemv_parts", dict(nparts=0), b"nparts"),
    ("mtl_decode_gemv_parts", dict(cols=4100, nparts=4), b"multiple of 4 * nparts"),
    ("mtl_decode_gemv_parts", dict(cols=8192 * 4, nparts=4), b"at most 4096"),
    ("mtl_decode_gemv_parts", dict(batch=3), b"batch must be 1, 2 or 4"),
    ("mtl_linear_skinny", dict(M=64 * 65535 + 1), b"M (rows of x)"),
    ("mtl_in_proj_conv_prefill", dict(batch=5, seqlen=13), b"batch * seqlen"),
    ("mtl_in_proj_conv_prefill", dict(d_conv=5), b"d_conv"),
    ("mtl_in_proj_conv_prefill", dict(d_inner=40), b"multiple of 16"),
    ("mtl_in_proj_conv_prefill", dict(alias=True), b"alias"),
    ("mtl_xproj_sum_dt", dict(R=161), b"dt_rank"),
    ("mtl_xproj_sum_dt", dict(R=90, J=80), b"dt_rank"),
    ("mtl_xproj_sum_dt", dict(nparts=0), b"nparts"),
    ("mtl_linear_skinny", dict(M=0), b"M (rows of x)"),
    ("mtl_linear_skinny", dict(K=96), b"multiple of 128"),
    ("mtl_linear_skinny", dict(K=256, ksplit=4), b"multiple of 128 * ksplit"),
    ("mtl_linear_skinny", dict(N=6), b"multiple of 4"),
    ("mtl_linear_skinny", dict(rows_per_block=8), b"rows_per_block"),
    ("mtl_linear_skinny", dict(K=256, ksplit=2, y_ks=64), b"overlap"),
    ("mtl_prefill_short", dict(batch=5, seqlen=13), b"batch * seqlen"),
    ("mtl_prefill_short", dict(d_model=320), b"d_model"),
    ("mtl_prefill_short", dict(d_inner=768), b"d_inner"),
    ("mtl_prefill_short", dict(d_state=17), b"d_state"),
    ("mtl_prefill_short", dict(d_conv=5), b"d_conv"),
    ("mtl_prefill_short", dict(n_layers=0), b"n_layers"),
    ("mtl_prefill_short", dict(null_ws=True), b"null workspace"),
    ("mtl_prefill_short", dict(null_layer=True), b"layer 1: null required pointer"),
    ("mtl_prefill_short", dict(alias=True), b"layer 1: conv_state_out must not alias"),
    ("mtl_prefill_short", dict(d_state=15), b"multiple of 4"),
    ("mtl_decode_step", dict(batch=3), b"batch must be 1, 2 or 4"),
    ("mtl_decode_step", dict(cpb=16), b"channels_per_block"),
    ("mtl_decode_step", dict(d_state=17), b"d_state"),
    ("mtl_decode_step", dict(d_inner=8192), b"d_inner"),
    ("mtl_decode_step", dict(d_conv=9), b"d_conv"),
    ("mtl_decode_step", dict(n_layers=0), b"n_layers"),
    ("mtl_decode_step", dict(split_k=0, xproj_parts=0), b"xproj_parts"),
    ("mtl_decode_step", dict(null_ws=True), b"null workspace"),
    ("mtl_decode_step", dict(null_layer=True), b"layer 1: null required pointer"),
    ("mtl_decode_step", dict(split_k=0, xproj_parts=4, null_layer=False), b"layer 0: null required pointer"),
    # rejected before any launch: limits the per-layer calls would only meet
    # after layer 0's conv history had moved on
    ("mtl_decode_step", dict(batch=2, d_model=768, d_inner=1536, dt_rank=48), b"partial blocks"),
    ("mtl_decode_step", dict(split_k=0, xproj_parts=3), b"multiple of 4 * xproj_parts"),
    ("mtl_decode_step", dict(split_k=0, xproj_parts=65, d_inner=4096), b"xproj_parts must be in [1, 64]"),
    ("mtl_decode_step", dict(misaligned_layer=True), b"layer 1: W_in, W_out and W_x must be 16-byte aligned"),
    ("mtl_decode_step", dict(same_ws=True), b"x0, x1 and resid must be distinct"),
    ("mtl_decode_step", dict(batch=4, d_model=4096), b"batch * d_model too large"),
    ("mtl_decode_step_persist", dict(batch=2), b"batch must be 1"),
    ("mtl_decode_step_persist", dict(d_model=2048, d_inner=4096), b"d_model"),
    ("mtl_decode_step_persist", dict(n_layers=65), b"n_layers"),
    ("mtl_decode_step_persist", dict(dt_rank=80), b"dt_rank"),
    ("mtl_decode_step_persist", dict(d_conv=5), b"d_conv"),
    ("mtl_decode_step_persist", dict(ws_bytes=1024), b"workspace too small"),
    ("mtl_decode_step_persist", dict(blocking=3), b"blocking"),
    ("mtl_decode_step_persist", dict(null_xt=True), b"layer 1: null required pointer"),
    ("mtl_prefill_short", dict(misaligned_layer=True),
     b"layer 1: W_in, b_in, W_x, W_out and b_out must be 16-byte aligned"),
    ("mtl_decode_step_batched", dict(batch=33), b"batch must be in [1, 32]"),
    ("mtl_decode_step_batched", dict(n_layers=0), b"n_layers"),
    ("mtl_decode_step_batched", dict(d_model=320), b"d_model"),
    ("mtl_decode_step_batched", dict(d_inner=768), b"d_inner"),
    ("mtl_decode_step_batched", dict(d_state=17), b"d_state"),
    ("mtl_decode_step_batched", dict(dt_rank=260), b"dt_rank"),
    ("mtl_decode_step_batched", dict(d_conv=5), b"d_conv"),
    ("mtl_decode_step_batched", dict(null_ws=True), b"null workspace"),
    ("mtl_decode_step_batched", dict(fold=1, null_fold=True), b"fold needs xn, sq and counters"),
    ("mtl_decode_step_batched", dict(fold=1, xn_is_h=True), b"xn must not alias h or inp"),
    ("mtl_decode_step_batched", dict(null_layer=True), b"layer 1: null required pointer"),
    ("mtl_decode_step_batched", dict(misaligned_layer=True), b"layer 1: W_in, b_in, conv_state"),
    ("mtl_decode_step_batched", dict(fold=1, misaligned_norm=True), b"layer 1: W_in, b_in, conv_state"),
    ("mtl_decode_step_batched", dict(fold=1, d_model=2176), b"at most 128"),
    ("mtl_decode_step_batched", dict(inp_is_h=True), b"must not alias h"),
    ("mtl_decode_step_batched", dict(layer1_eps=-1.0), b"layer 1: eps must be >= 0"),
    # a NaN eps would pass a "not below zero" test and then fail in the folded
    # in_proj of layer 1, after layer 0 has stepped its caches
    ("mtl_decode_step_batched", dict(fold=1, layer1_eps=float("nan")), b"layer 1: eps must be >= 0"),
    ("mtl_in_proj_conv_xproj", dict(batch=33), b"batch must be in [1, 32]"),
    ("mtl_in_proj_conv_xproj", dict(d_model=128), b"at least 256"),
    ("mtl_in_proj_conv_xproj", dict(d_model=320), b"multiple of 128"),
    ("mtl_in_proj_conv_xproj", dict(cpp=8), b"channels_per_part"),
    ("mtl_in_proj_conv_xproj", dict(d_inner=48, cpp=32), b"multiple of channels_per_part"),
    ("mtl_in_proj_conv_xproj", dict(d_conv=5), b"d_conv"),
    ("mtl_in_proj_conv_xproj", dict(d_conv=1), b"d_conv"),
    ("mtl_in_proj_conv_xproj", dict(J=289), b"J (x_proj rows)"),
    ("mtl_prefill_long", dict(d_conv=9), b"d_conv"),
    ("mtl_prefill_long", dict(d_state=33), b"d_state"),
    ("mtl_prefill_long", dict(batch=1 << 12, seqlen=1 << 12), b"batch * seqlen"),
    ("mtl_prefill_long", dict(n_layers=0), b"n_layers"),
    ("mtl_prefill_long", dict(batch=65536, seqlen=1), b"batch must be <= 65535"),
    ("mtl_prefill_long", dict(batch=1, seqlen=1 << 20), b"seqlen must be <= 1048560"),
    ("mtl_prefill_long", dict(null_ws=True), b"null workspace"),
    ("mtl_prefill_long", dict(null_layer=True), b"layer 1: null required pointer"),
    ("mtl_prefill_long", dict(alias=True), b"layer 1: conv_state_out must not alias"),
    ("mtl_in_proj_conv_xproj_normed", dict(sq_tiles=129), b"sq_tiles must be in [1, 128]"),
    ("mtl_in_proj_conv_xproj_normed", dict(sq_tiles=0), b"sq_tiles must be in [1, 128]"),
    ("mtl_in_proj_conv_xproj_normed", dict(null_sq=True), b"null sq"),
    ("mtl_in_proj_conv_xproj_normed", dict(eps=-1.0), b"eps"),
    ("mtl_in_proj_conv_xproj_normed", dict(batch=33), b"batch must be in [1, 32]"),
    ("mtl_linear_skinny_residual", dict(M=33), b"M (rows of x) must be in [1, 32]"),
    ("mtl_linear_skinny_residual", dict(M=0), b"M (rows of x)"),
    ("mtl_linear_skinny_residual", dict(N=48, rpb=32), b"multiple of rows_per_block"),
    ("mtl_linear_skinny_residual", dict(rpb=8), b"rows_per_block must be 16 or 32"),
    ("mtl_linear_skinny_residual", dict(K=256, ksplit=4), b"multiple of 128 * ksplit"),
    ("mtl_linear_skinny_residual", dict(alias=True), b"x_next must not alias h"),
    ("mtl_linear_skinny_residual", dict(null_cnt=True), b"null required pointer"),
])
def test_entry_points_validate_sizes_on_the_host(case):
    """Each entry point rejects sizes its kernels do not cover, with a message,
    before any launch (the pointers below are never dereferenced)."""
    from mamba_lite import _lib

    lib = _lib.load()
    name, over, msg = case
    P = ctypes.c_void_p(16)     # a non-null, 16-byte aligned placeholder that is never used
    if name == "mtl_decode_in":
        a = dict(batch=1, d_model=64, d_inner=128, d_conv=4, xdbl_cols=36, channels_per_block=8, first_layer=False,
                 vocab=0)
        a.update(over)
        x, emb, ids = (None, P, P) if a["first_layer"] else (P, None, None)
        rc = lib.mtl_decode_in(x, emb, ids, a["vocab"], None, P, 1e-5, P, None, P, P, None, None, P, P, None,
                               a["batch"], a["d_model"], a["d_inner"], a["d_conv"], a["xdbl_cols"],
                               a["channels_per_block"], None)
    elif name == "mtl_decode_gemv":
        a = dict(batch=1, rows=8, cols=64)
        a.update(over)
        rc = lib.mtl_decode_gemv(P, P, None, None, P, a["batch"], a["rows"], a["cols"], None)
    elif name == "mtl_decode_norm_gemv":
        a = dict(batch=1, rows=8, cols=64)
        a.update(over)
        rc = lib.mtl_decode_norm_gemv(P, P, 1e-5, P, None, ctypes.c_void_p(32), a["batch"], a["rows"], a["cols"], None)
    elif name == "mtl_decode_ssm":
        a = dict(nblk=4, batch=1, d_inner=64, d_state=16, dt_rank=4)
        a.update(over)
        rc = lib.mtl_decode_ssm(P, a["nblk"], P, P, P, P, P, None, P, P, a["batch"], a["d_inner"], a["d_state"],
                                a["dt_rank"], None)
    elif name == "mtl_sum_parts":
        a = dict(nparts=2)
        a.update(over)
        rc = lib.mtl_sum_parts(P, a["nparts"], 16, P, None)
    elif name == "mtl_conv_step_xproj":
        a = dict(batch=8, width=4, xdbl_cols=160)
        a.update(over)
        rc = lib.mtl_conv_step_xproj(P, P, 64, P, None, P, 64, P, P, a["batch"], 64, a["width"], a["xdbl_cols"], None)
    elif name == "mtl_selective_state_update":
        a = dict(dstate=16, dt_rank=4)
        a.update(over)
        rc = lib.mtl_selective_state_update(P, P, 64, None, 0, P, 36, P, P, P, None, P, 64, 1, 64, a["dstate"],
                                            a["dt_rank"], 0, 0, None)
    elif name == "mtl_decode_gemv_parts":
        a = dict(batch=1, rows=8, cols=4096, nparts=4)
        a.update(over)
        rc = lib.mtl_decode_gemv_parts(P, P, P, a["batch"], a["rows"], a["cols"], a["nparts"], None)
    elif name == "mtl_in_proj_conv_prefill":
        a = dict(batch=1, seqlen=64, d_model=256, d_inner=512, d_conv=4, alias=False)
        a.update(over)
        Q = ctypes.c_void_p(32)
        rc = lib.mtl_in_proj_conv_prefill(P, a["d_model"], P, None, P, None, a["d_conv"], Q if a["alias"] else P, Q,
                                          P, P, a["batch"], a["seqlen"], a["d_model"], a["d_inner"], None)
    elif name == "mtl_xproj_sum_dt":
        a = dict(nparts=4, rows=64, J=80, R=48, D=1536)
        a.update(over)
        rc = lib.mtl_xproj_sum_dt(P, a["nparts"], a["rows"], a["J"], P, a["R"], a["D"], P, P, None)
    elif name == "mtl_linear_skinny":
        a = dict(M=8, N=64, K=128, ksplit=1, rows_per_block=16, y_ks=0)
        a.update(over)
        rc = lib.mtl_linear_skinny(P, a["K"], P, None, P, a["N"], a["y_ks"], a["M"], a["N"], a["K"], a["ksplit"],
                                   a["rows_per_block"], None)
    elif name == "mtl_prefill_short":
        a = dict(batch=1, seqlen=64, d_model=256, d_inner=512, d_state=16, d_conv=4, n_layers=2, null_ws=False,
                 null_layer=False, alias=False, misaligned_layer=False)
        a.update(over)
        args = _lib.PrefillShortArgs()
        for f, *_ in _lib.PrefillShortArgs._fields_[:11]:
            setattr(args, f, None if a["null_ws"] and f == "y" else 16)
        args.eps_f, args.d_conv, args.n_layers = 1e-5, a["d_conv"], a["n_layers"]
        args.batch, args.seqlen, args.d_model, args.d_inner = a["batch"], a["seqlen"], a["d_model"], a["d_inner"]
        args.d_state, args.dt_rank = a["d_state"], 16
        layers = (_lib.PrefillLayer * 2)()
        for i, L in enumerate(layers):
            for f, *_ in _lib.PrefillLayer._fields_:
                if f not in ("eps", "reserved"):
                    setattr(L, f, 16 * (len(f) + 1))
            L.conv_state_out = 32
            L.conv_state_in = 32 if a["alias"] and i == 1 else 48
            if a["null_layer"] and i == 1:
                L.W_dt = None
            if a["misaligned_layer"] and i == 1:
                L.W_out = 24
        rc = lib.mtl_prefill_short(ctypes.byref(args), layers, None)
    elif name == "mtl_prefill_long":
        a = dict(batch=1, seqlen=128, d_model=256, d_inner=512, d_state=16, d_conv=4, n_layers=2, null_ws=False,
                 null_layer=False, alias=False)
        a.update(over)
        args = _lib.PrefillLongArgs()
        for f in ("h", "xn", "xz", "u", "x_dbl", "dt", "y", "out", "blas_ws", "norm_f", "normed_out"):
            setattr(args, f, None if a["null_ws"] and f == "y" else 16)
        args.blas_ws_bytes = 1 << 20
        args.eps_f, args.d_conv, args.n_layers = 1e-5, a["d_conv"], a["n_layers"]
        args.batch, args.seqlen, args.d_model, args.d_inner = a["batch"], a["seqlen"], a["d_model"], a["d_inner"]
        args.d_state, args.dt_rank = a["d_state"], 16
        layers = (_lib.PrefillLayer * 2)()
        for i, L in enumerate(layers):
            for f, *_ in _lib.PrefillLayer._fields_:
                if f not in ("eps", "reserved"):
                    setattr(L, f, 16 * (len(f) + 1))
            L.conv_state_out = 32
            L.conv_state_in = 32 if a["alias"] and i == 1 else 48
            if a["null_layer"] and i == 1:
                L.W_dt = None
        rc = lib.mtl_prefill_long(ctypes.byref(args), layers, None)
    elif name == "mtl_decode_step":
        a = dict(batch=1, cpb=8, n_layers=2, split_k=1, xproj_parts=1, null_ws=False, null_layer=False, d_state=16,
                 d_inner=512, d_conv=4, d_model=256, dt_rank=16, misaligned_layer=False, same_ws=False)
        a.update(over)
        args = _lib.DecodeStepArgs()
        for k, (f, *_) in enumerate(_lib.DecodeStepArgs._fields_[:11]):
            # distinct 16-byte aligned placeholders, never dereferenced
            setattr(args, f, None if a["null_ws"] and f == "gz" else 16 if a["same_ws"] else 16 * (k + 1))
        args.eps_f, args.vocab, args.n_layers, args.batch = 1e-5, 64, a["n_layers"], a["batch"]
        args.d_model, args.d_inner, args.d_state, args.dt_rank, args.d_conv = a["d_model"], a["d_inner"], \
            a["d_state"], a["dt_rank"], a["d_conv"]
        args.channels_per_block, args.split_k, args.xproj_parts = a["cpb"], a["split_k"], a["xproj_parts"]
        layers = (_lib.DecodeLayer * 2)()
        for i, L in enumerate(layers):
            for f, *_ in _lib.DecodeLayer._fields_:
                if f not in ("eps", "reserved", "W_x"):       # W_x unset: only split_k layers are complete
                    setattr(L, f, 16)
            if a["null_layer"] and i == 1:
                L.A_log = None
            if a["misaligned_layer"] and i == 1:
                L.W_out = 24
        rc = lib.mtl_decode_step(ctypes.byref(args), layers, None)
    elif name == "mtl_decode_step_persist":
        a = dict(batch=1, n_layers=2, d_model=256, d_inner=512, d_state=16, dt_rank=16, d_conv=4, ws_bytes=1 << 20,
                 blocking=0, null_xt=False)
        a.update(over)
        args = _lib.DecodeStepArgs()
        for k, (f, *_) in enumerate(_lib.DecodeStepArgs._fields_[:11]):
            setattr(args, f, 16 * (k + 1))
        args.eps_f, args.vocab, args.n_layers, args.batch = 1e-5, 64, a["n_layers"], a["batch"]
        args.d_model, args.d_inner, args.d_state, args.dt_rank, args.d_conv = a["d_model"], a["d_inner"], \
            a["d_state"], a["dt_rank"], a["d_conv"]
        layers = (_lib.DecodeLayer * max(2, a["n_layers"]))()
        for i, L in enumerate(layers):
            for f, *_ in _lib.DecodeLayer._fields_:
                if f not in ("eps", "reserved", "W_x"):
                    setattr(L, f, 16)
            if a["null_xt"] and i == 1:
                L.W_xT = None
        rc = lib.mtl_decode_step_persist(ctypes.byref(args), layers, ctypes.c_void_p(256), ctypes.c_void_p(256),
                                         a["ws_bytes"], a["blocking"], None)
    elif name == "mtl_decode_step_batched":
        a = dict(batch=8, n_layers=2, d_model=256, d_inner=512, d_state=16, dt_rank=16, d_conv=4, fold=0,
                 null_ws=False, null_fold=False, xn_is_h=False, null_layer=False, misaligned_layer=False,
                 misaligned_norm=False, inp_is_h=False, layer1_eps=None)
        a.update(over)
        args = _lib.DecodeStepBatchedArgs()
        for k, (f, *_) in enumerate(_lib.DecodeStepBatchedArgs._fields_[:13]):
            # distinct 16-byte aligned placeholders, never dereferenced
            setattr(args, f, 16 * (k + 1))
        if a["null_ws"]:
            args.x_dbl = None
        if a["null_fold"]:
            args.sq = None
        if a["xn_is_h"]:
            args.xn = args.h
        if a["inp_is_h"]:
            args.inp = args.h
        args.eps_f, args.n_layers, args.batch, args.fold = 1e-5, a["n_layers"], a["batch"], a["fold"]
        args.d_model, args.d_inner, args.d_state, args.dt_rank, args.d_conv = a["d_model"], a["d_inner"], \
            a["d_state"], a["dt_rank"], a["d_conv"]
        layers = (_lib.DecodeLayer * 2)()
        for i, L in enumerate(layers):
            for f, *_ in _lib.DecodeLayer._fields_:
                if f not in ("eps", "reserved", "W_x"):
                    setattr(L, f, 16)
            if a["null_layer"] and i == 1:
                L.W_xT = None
            if a["misaligned_layer"] and i == 1:
                L.conv_state = 24
            if a["misaligned_norm"] and i == 1:
                L.norm_w = 20
            if a["layer1_eps"] is not None and i == 1:
                L.eps = a["layer1_eps"]
        rc = lib.mtl_decode_step_batched(ctypes.byref(args), layers, None)
    elif name == "mtl_in_proj_conv_xproj":
        a = dict(batch=8, d_model=256, d_inner=64, cpp=16, d_conv=4, J=40)
        a.update(over)
        rc = lib.mtl_in_proj_conv_xproj(P, a["d_model"], P, None, P, P, None, a["d_conv"], P, a["J"], P, P,
                                        a["d_inner"], P, a["batch"], a["d_model"], a["d_inner"], a["cpp"], None)
    elif name == "mtl_in_proj_conv_xproj_normed":
        a = dict(batch=8, d_model=256, d_inner=64, cpp=16, d_conv=4, J=40, sq_tiles=16, null_sq=False, eps=1e-5)
        a.update(over)
        rc = lib.mtl_in_proj_conv_xproj_normed(P, a["d_model"], P, None, P, P, None, a["d_conv"], P, a["J"], P, P,
                                               a["d_inner"], P, a["batch"], a["d_model"], a["d_inner"], a["cpp"],
                                               None if a["null_sq"] else P, a["sq_tiles"], a["eps"], None)
    elif name == "mtl_linear_skinny_residual":
        a = dict(M=8, N=256, K=512, ksplit=4, rpb=16, alias=False, null_cnt=False)
        a.update(over)
        xn = P if a["alias"] else ctypes.c_void_p(64)
        rc = lib.mtl_linear_skinny_residual(P, a["K"], P, None, P, a["M"], a["N"], a["K"], a["ksplit"], a["rpb"], P,
                                            P, xn, P, None if a["null_cnt"] else P, None)
    else:
        a = dict(width=4)
        a.update(over)
        rc = lib.mtl_conv_step(P, P, 64, P, None, P, 64, 1, 64, a["width"], 0, 1, None)
    assert rc == 1, (name, over)
    assert msg in lib.mtl_last_error(), lib.mtl_last_error()


@pytest.mark.parametrize("over,msg", [
    (dict(B_sn=-1), b"negative B/C stride"),
    (dict(C_sl=1 << 30), b"B/C strides too large"),
    (dict(u_sl=1 << 28, delta_sl=1 << 28, y_sl=1 << 28), b"token-major step stride too large"),
])
def test_scan_rejects_strides_outside_its_32_bit_offsets(over, msg):
    """The scan addresses B/C tiles and token-major rows with 32-bit byte
    offsets from a uniform base; strides that would overflow them, or point
    backwards, are refused on the host (pointers are placeholders)."""
    from mamba_lite import _lib

    lib = _lib.load()
    b, L, D, N = 2, 64, 64, 16
    p = _lib.ScanParams()
    P = 16
    p.u = p.delta = p.z = p.B = p.C = p.y = P
    p.A = P
    for t in ("u", "delta", "z", "y"):        # token-major [b, l, D]
        setattr(p, f"{t}_sb", L * D); setattr(p, f"{t}_sd", 1); setattr(p, f"{t}_sl", D)
    for t in ("B", "C"):                       # [b, l, N] viewed as [b, N, l]
        setattr(p, f"{t}_sb", L * N); setattr(p, f"{t}_sn", 1); setattr(p, f"{t}_sl", N)
    p.batch, p.seqlen, p.dim, p.dstate, p.dtype = b, L, D, N, 0
    for k, v in over.items():
        setattr(p, k, v)
    assert lib.mtl_selective_scan_fwd(ctypes.byref(p), None) == 1
    assert msg in lib.mtl_last_error(), lib.mtl_last_error()
