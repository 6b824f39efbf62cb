"""Benchmark of the Mamba mixer hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                   [--only scan|decode|quant|shard|prefill|prefill-short|prefill-long|copy|decode-counters|all]
                   [--decode-shapes 130m,1.4b] [--decode-batches B,...] [--decode-persist]
                   [--no-step-fold] [--no-cpu-baseline]

Headline (`value`): fused selective-scan prefill throughput, fp32, on the
isolated-op workload u, delta, z [32, 1536, 1024], B, C [32, 16, 1024],
A [1536, 16] = -(1..16), D = 1 (one step = one scan over the whole batch =
32,768 tokens), with `roofline` for the scan kernel (algorithmic bytes /
HIP-event kernel time vs 8 TB/s) and `cpu_baseline` (the numpy oracle's
materialize-then-loop scan on the host cores, same workload).

Reported beside it in the same JSON line, each with its own parity check:
  decode_us_per_token  hipGraph-replayed MambaLM.step, 130m shape b=1 and
                       1.4b shape b=1 / b=32 (random-init fp32 weights)
  prefill_tok_s        MambaLM.prefill, 130m shape (b=1 x 64, b=32 x 1024) and
                       1.4b shape (b=1 x 1024, b=32 x 1024)
  prefill_graph_tok_s  the b=1 x 64 prefill captured once (GraphedPrefill)
                       and replayed per prompt
  quant                per-token int8 and fp16 quantize->dequantize-sum of
                       two [32768, 768] fp32 partials (GB/s)
  shard_bf16           one TP rank's 1.4b channel shard (D=2048), bf16
                       activations, b=32 x 2048: conv and scan+gate kernels
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "mamba-tp-lite_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "prefill tok/s + scan HBM GB/s (% peak); decode µs/token, 130m & 1.4b shape"
HBM_PEAK_GBPS = 8000.0
# VALU roofline of the scans: a wave64 VALU instruction holds one of the 1024
# SIMDs for 4 cycles, a transcendental (half rate on gfx950) for 8; at the
# 2.4 GHz peak engine clock.  Instruction counts per launch from rocprofv3
# (SQ_INSTS_VALU, SQ_INSTS_VALU_TRANS_F32), recorded in profiles/.
SIMDS, CLOCK_HZ = 1024, 2.4e9
SCAN_VALU = {"fp32_b32_d1536_l1024": (80.2e6, 15.7e6), "bf16_b32_d2048_l2048": (223.5e6, 42.0e6)}


def valu_roofline(key, us):
    """VALU-bound time of a scan launch (every SIMD issuing every cycle) and
    the fraction of it the measured launch time reaches."""
    valu, trans = SCAN_VALU[key]
    floor_us = (valu + trans) * 4 / SIMDS / CLOCK_HZ * 1e6
    return {"bound": "valu", "floor_us": floor_us, "measured_us": us, "frac": floor_us / us,
            "sq_insts_valu": valu, "sq_insts_valu_trans_f32": trans,
            "how": "(SQ_INSTS_VALU + SQ_INSTS_VALU_TRANS_F32) x 4 cycles / 1024 SIMDs at 2.4 GHz"}

# isolated selective-scan workload
SCAN_B, SCAN_D, SCAN_L, SCAN_N = 32, 1536, 1024, 16
SCAN_BYTES = 4 * (4 * SCAN_B * SCAN_D * SCAN_L + 2 * SCAN_B * SCAN_N * SCAN_L + SCAN_D * SCAN_N + 2 * SCAN_D
                  + SCAN_B * SCAN_D * SCAN_N)  # u, delta, z, y + B, C + A + D, dt_bias + h_out = 812,756,992


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_info():
    """The host the cpu_baseline legs ran on: logical CPUs, torch's intra-op
    thread count and the CPU model string."""
    import torch
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_count": os.cpu_count(), "torch_num_threads": torch.get_num_threads(), "cpu_model": model}


def dt_bias_init(D, seed):
    """dt_proj.bias = inv_softplus(dt), dt log-uniform in [1e-3, 0.1] (the HF
    Mamba init): inv_softplus(y) = y + log(-expm1(-y))."""
    import numpy as np
    rng = np.random.default_rng(seed)
    dt = np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))
    return (dt + np.log(-np.expm1(-dt))).astype(np.float32)


def _timed(fn, iters, warmup, stream=None):
    """Mean ms per call of fn() over `iters` back-to-back calls, bracketed by
    HIP events on the stream the work is enqueued on."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    s.record(stream)
    for _ in range(iters):
        fn()
    e.record(stream)
    e.synchronize()
    return s.elapsed_time(e) / iters


def _median_trials(fn, iters, warmup, trials=5):
    import statistics
    vals = [_timed(fn, iters, warmup if i == 0 else 1) for i in range(trials)]
    return statistics.median(vals), vals


# --------------------------------------------------------------------------- scan (headline)
def make_scan_inputs(dev, seed=0):
    import torch
    g = torch.Generator(device=dev).manual_seed(seed)
    b, D, L, N = SCAN_B, SCAN_D, SCAN_L, SCAN_N
    bias = torch.from_numpy(dt_bias_init(D, seed))
    return dict(
        u=torch.randn(b, D, L, device=dev, generator=g),
        delta=0.5 * torch.randn(b, D, L, device=dev, generator=g),
        z=torch.randn(b, D, L, device=dev, generator=g),
        B=torch.randn(b, N, L, device=dev, generator=g),
        C=torch.randn(b, N, L, device=dev, generator=g),
        A=-torch.arange(1, N + 1, device=dev, dtype=torch.float32).repeat(D, 1).contiguous(),
        D=torch.ones(D, device=dev),
        delta_bias=bias.to(dev),
    )


# Wall time of scan launches run before the timed trials: the GPU's clocks
# and power state settle over the first second or two of sustained load (a
# short warmup left the first trials ~10% slow), so every run is timed in the
# same steady state.
SCAN_PREWARM_S = 2.0


def bench_scan(dev, steps, warmup):
    import torch
    from mamba_lite import ops
    x = make_scan_inputs(dev)
    y = torch.empty_like(x["u"])
    h = torch.empty(SCAN_B, SCAN_D, SCAN_N, device=dev)

    def step():
        ops.selective_scan(x["u"], x["delta"], x["A"], x["B"], x["C"], D=x["D"], z=x["z"],
                           delta_bias=x["delta_bias"], y=y, h_out=h)

    t0 = time.perf_counter()
    n_pre = 0
    while time.perf_counter() - t0 < SCAN_PREWARM_S:
        for _ in range(20):
            step()
        n_pre += 20
        torch.cuda.synchronize()
    prewarm_ms = (time.perf_counter() - t0) * 1e3
    ms, trials = _median_trials(step, steps, warmup)
    torch.cuda.synchronize()
    return ms, trials, (x, y, h), {"prewarm_ms": prewarm_ms, "prewarm_launches": n_pre}


def cpu_baseline_scan(workers, gpu_run):
    """cpu_baseline leg: the oracle's materialize-then-loop scan (numpy,
    float32) on the host cores over the whole isolated-op workload, one batch
    row per process; then the oracle (float64) on two sampled (row, 64-channel)
    blocks of the very inputs the GPU scanned, as the parity gate reported
    with the throughput."""
    import multiprocessing as mp
    import numpy as np
    from oracle import mixer as om
    t0 = time.perf_counter()
    with mp.get_context("spawn").Pool(workers) as pool:
        pool.map(_cpu_scan_row, range(SCAN_B))
    secs = time.perf_counter() - t0
    x, y, h = gpu_run
    err = 0.0
    for bi, c0 in ((0, 0), (29, 1408)):
        sl = slice(c0, c0 + 64)
        f = lambda t: t.cpu().numpy()
        yr, hr = om.selective_scan_bnl(f(x["u"][bi:bi + 1, sl]), f(x["delta"][bi:bi + 1, sl]), f(x["A"][sl]),
                                       f(x["B"][bi:bi + 1]), f(x["C"][bi:bi + 1]), f(x["D"][sl]),
                                       f(x["z"][bi:bi + 1, sl]), f(x["delta_bias"][sl]), None, dtype=np.float64)
        for got, ref in ((y[bi:bi + 1, sl], yr), (h[bi:bi + 1, sl], hr)):
            d = np.abs(f(got) - ref)
            err = max(err, float((d / (np.abs(ref) + np.sqrt(np.mean(ref ** 2)))).max()))
    return secs, err


def _cpu_scan_row(bi):
    import numpy as np
    from oracle import mixer as om
    rng = np.random.default_rng(1000 + bi)
    D, L, N = SCAN_D, SCAN_L, SCAN_N
    u = rng.standard_normal((1, D, L), dtype=np.float32)
    delta = (0.5 * rng.standard_normal((1, D, L), dtype=np.float32))
    z = rng.standard_normal((1, D, L), dtype=np.float32)
    B = rng.standard_normal((1, N, L), dtype=np.float32)
    C = rng.standard_normal((1, N, L), dtype=np.float32)
    A = -np.tile(np.arange(1, N + 1, dtype=np.float32), (D, 1))
    om.selective_scan_bnl(u, delta, A, B, C, np.ones(D, np.float32), z, dt_bias_init(D, bi), None,
                          dtype=np.float32)
    return bi


def traffic_from_profiles(key):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE + WRITE_SIZE
    (calibrated against a copy kernel) for `key`, if recorded."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get(key, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


# --------------------------------------------------------------------------- model decode / prefill
def build_lm(cfg, dev, seed=0):
    import torch
    from mamba_lite.model import MambaLM, MambaMixer
    torch.manual_seed(seed)
    with torch.device(dev):
        model = MambaLM(cfg)
    with torch.no_grad():
        for i, m in enumerate(x for x in model.modules() if isinstance(x, MambaMixer)):
            m.dt_proj.bias.copy_(torch.from_numpy(dt_bias_init(m.dt_proj.bias.shape[0], seed * 1000 + i)))
    return model.eval()


def bench_decode(model, batch, prompt, n_tokens, dev):
    import torch
    from mamba_lite.cuda_graph import GraphedStepper
    g = torch.Generator(device=dev).manual_seed(1234)
    ids = torch.randint(0, model.cfg.vocab_size, (batch, prompt), device=dev, generator=g)
    nxt = torch.zeros(batch, 1, dtype=torch.long, device=dev)
    with torch.no_grad():
        _, cache_e = model.prefill(ids)
        eager = [model.step(nxt, cache_e).clone() for _ in range(3)]
        _, cache = model.prefill(ids)
        st = GraphedStepper(model, cache, batch, "cuda")
        st.capture()
        ok = all(torch.equal(st.replay(nxt), e) for e in eager)   # graph == eager, bit for bit
        ms = _timed(lambda: st.replay(nxt), n_tokens, 3)
        # eager steps (what generate() runs), launched from the host one step at a time
        ms_eager = _timed(lambda: model.step(nxt, cache_e), 64, 3)
    return ms * 1000.0, ok, ms_eager * 1000.0


def _oracle_lm_weights(model):
    f = lambda p: p.detach().float().cpu().numpy()
    layers = []
    for blk in model.layers:
        m = blk.mixer
        d = {"norm": f(blk.norm.weight), "in_proj_w": f(m.in_proj.weight), "conv_w": f(m.conv1d.weight)[:, 0, :],
             "conv_b": f(m.conv1d.bias) if m.conv1d.bias is not None else None, "x_proj_w": f(m.x_proj.weight),
             "dt_proj_w": f(m.dt_proj.weight), "dt_proj_b": f(m.dt_proj.bias), "A_log": f(m.A_log), "D": f(m.D),
             "out_proj_w": f(m.out_proj.weight)}
        layers.append(d)
    return {"embedding": f(model.embedding.weight), "norm_f": f(model.norm_f.weight), "layers": layers}


def cpu_baseline_decode(model, dev, prompt=64, steps=32, name="130m", parity=True):
    """cpu_baseline leg of the decode metric, batch 1: the oracle's LM (numpy
    float32, the reference's materialize-then-loop prefill and its step) on
    the host, `prompt` ids then `steps` timed greedy steps (us/token); with
    `parity`, the GPU's fused step logits compared to the float64 oracle's on
    the same weights and tokens (three teacher-forced steps)."""
    import numpy as np
    import torch
    from oracle import mixer as om
    W = _oracle_lm_weights(model)
    g = torch.Generator(device=dev).manual_seed(99)
    ids = torch.randint(0, model.cfg.vocab_size, (1, prompt), device=dev, generator=g)
    _, cache = om.lm_prefill(W, ids.cpu().numpy(), dtype=np.float32)
    with torch.no_grad():
        logits, gcache = model.prefill(ids)
    nxt = ids[:, -1:].cpu().numpy()
    err = 0.0
    t0 = time.perf_counter()
    for _ in range(steps):
        ref = om.lm_step(W, nxt, cache, dtype=np.float32)
        nxt = ref[:, -1].argmax(-1)[:, None]
    secs = time.perf_counter() - t0
    out = {}
    if parity:
        # parity of the fused GPU step on the same tokens (teacher-forced)
        _, cache = om.lm_prefill(W, ids.cpu().numpy(), dtype=np.float64)
        tok = ids[:, -1:]
        with torch.no_grad():
            for _ in range(3):
                got = model.step(tok, gcache)
                ref = om.lm_step(W, tok.cpu().numpy(), cache, dtype=np.float64)
                err = max(err, float(np.abs(got.cpu().numpy() - ref).max() / np.abs(ref).max()))
                tok = got[:, -1].argmax(-1, keepdim=True)
        out["gpu_step_max_rel_err_vs_oracle_f64"] = err
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": secs / steps * 1e6, "unit": "us/token", "cores": cores, "kind": "port",
            "sample": f"{name} shape b=1: {prompt}-token prefill, then {steps} greedy steps timed (numpy float32 "
                      f"oracle; BLAS threads up to {cores})", **out, **host_info()}


def bench_prefill(model, batch, seqlen, dev, iters=None):
    import torch
    g = torch.Generator(device=dev).manual_seed(7)
    ids = torch.randint(0, model.cfg.vocab_size, (batch, seqlen), device=dev, generator=g)
    small = batch * seqlen <= 4096      # milliseconds per call: average more calls
    iters = iters or (20 if small else 3)
    with torch.no_grad():
        ms = _timed(lambda: model.prefill(ids), iters, 3 if small else 1)
    return batch * seqlen / (ms / 1000.0)


def bench_prefill_graph(model, batch, seqlen, dev, iters=20):
    """The same prefill captured once with cuda_graph.GraphedPrefill and
    replayed per prompt (final states into a preallocated cache).  Checks
    the replay against an eager prefill, bit for bit, before timing."""
    import torch
    from mamba_lite import model as mm
    from mamba_lite.cuda_graph import GraphedPrefill
    g = torch.Generator(device=dev).manual_seed(7)
    ids = torch.randint(0, model.cfg.vocab_size, (batch, seqlen), device=dev, generator=g)
    cache = mm.MambaCache.allocate(model.cfg, batch, dev, torch.float32)
    gp = GraphedPrefill(model, cache, batch, seqlen, "cuda")
    gp.capture()
    with torch.no_grad():
        got = gp.replay(ids).clone()
        ref, _ = model.prefill(ids)
    ms = _timed(lambda: gp.replay(ids), iters, 3)
    return {"tok_s": batch * seqlen / (ms / 1000.0), "ms_per_prompt": ms,
            "replay_equals_eager": bool(torch.equal(got, ref))}


# --------------------------------------------------------------------------- quant / shard
def _cpu_quant_chunk(args):
    """One process's share of the int8 CPU baseline: rows [r0, r1) of two
    Student-t(3) * 0.5 partials of 768 columns (seeded per chunk), quantized
    and dequant-summed by the oracle; returns the seconds it took."""
    import numpy as np
    from oracle import quant as oq
    r0, r1 = args
    rng = np.random.default_rng(1000 + r0)
    parts = [(rng.standard_t(3, (r1 - r0, 768)) * 0.5).astype(np.float32) for _ in range(2)]
    t0 = time.perf_counter()
    oq.quant_dequant_sum_int8_tok(parts)
    return time.perf_counter() - t0


def cpu_baseline_quant(parts, pays, out, rows=4096, workers=16):
    """cpu_baseline leg of the int8 payload op: the oracle's per-token int8
    quantize -> dequantize-sum (numpy, IEEE fp32 like the reference's torch
    CPU ops) over the full [32768, 768] workload split by rows over `workers`
    processes (each draws its rows of the same distribution), timed as wall
    clock; and, as its parity gate, the first `rows` rows of the very
    partials the GPU quantized compared byte for byte with the GPU payloads
    and output.  (torch's own GPU division on ROCm is not correctly rounded,
    so it cannot serve as the bit-exact reference.)"""
    import multiprocessing as mp
    import numpy as np
    from oracle import quant as oq
    cols = parts[0].shape[1]
    host = [p[:rows].cpu().numpy() for p in parts]
    t0 = time.perf_counter()
    ref_out, ref_pays = oq.quant_dequant_sum_int8_tok(host)
    secs = time.perf_counter() - t0
    R = parts[0].shape[0]
    exact = bool(np.array_equal(out[:rows].cpu().numpy(), ref_out))
    for p, rp in zip(pays, ref_pays):
        s, q = oq.unpack_payload(p.cpu().numpy(), R, cols)
        rs, rq = oq.unpack_payload(rp, rows, cols)
        exact = exact and bool(np.array_equal(s[:rows], rs) and np.array_equal(q[:rows], rq))
    step = (R + workers - 1) // workers
    chunks = [(r, min(R, r + step)) for r in range(0, R, step)]
    with mp.get_context("spawn").Pool(workers) as pool:
        per = pool.map(_cpu_quant_chunk, chunks)
    nbytes = 2 * R * cols * 4 + 2 * R * (cols + 4) + R * cols * 4
    one = 2 * rows * cols * 4 + 2 * rows * (cols + 4) + rows * cols * 4
    return {"value": nbytes / max(per) / 1e9, "unit": "GB/s", "cores": workers, "kind": "port",
            "sample": f"all {R} rows x {cols} columns split over {workers} processes running at once (numpy "
                      f"oracle; each draws its rows from the same distribution and times its own quantize + "
                      f"dequant-sum; value = all bytes / the slowest process, {max(per) * 1e3:.1f} ms); parity "
                      f"gate: the first {rows} rows of the GPU's own inputs, byte for byte",
            "single_core_gbps": one / secs / 1e9, "bit_exact_codes_scales_out": exact, **host_info()}


QUANT_PREWARM_S = 1.0


def bench_quant(dev, iters=20):
    import numpy as np
    import torch
    from mamba_lite import ops
    rows, cols = 32 * 1024, 768
    # Student-t(3) * 0.5 partials drawn on the host (seeded), then resident in HBM
    rng = np.random.default_rng(3)
    parts = [torch.from_numpy((rng.standard_t(3, (rows, cols)) * 0.5).astype(np.float32)).to(dev) for _ in range(2)]
    out = torch.empty_like(parts[0])
    pays = [torch.empty(rows * (cols + 4), dtype=torch.uint8, device=dev) for _ in range(2)]
    # back-to-back launches first, so the clocks have settled when timing
    # starts (run alone, the first timed calls otherwise read up to 2x slow)
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < QUANT_PREWARM_S:
        for _ in range(20):
            ops.quant_dequant_sum_int8_tok(parts, payloads=pays, out=out)
        torch.cuda.synchronize()
    ms8 = _timed(lambda: ops.quant_dequant_sum_int8_tok(parts, payloads=pays, out=out), iters, 3)
    torch.cuda.synchronize()
    cpu = cpu_baseline_quant(parts, pays, out)
    bytes8 = 2 * rows * cols * 4 + 2 * rows * (cols + 4) + rows * cols * 4
    p16 = [torch.empty(rows, cols, dtype=torch.float16, device=dev) for _ in range(2)]
    ms16 = _timed(lambda: ops.quant_dequant_sum_fp16(parts, payloads=p16, out=out), iters, 3)
    ref16 = (parts[0].half() + parts[1].half()).float()
    exact16 = bool(torch.equal(out, ref16))
    bytes16 = 2 * rows * cols * 4 + 2 * rows * cols * 2 + rows * cols * 4
    # cold-HBM rates: calls cycle over 4 distinct sets of partials (805 MB of
    # inputs against the 256 MB MALL), so each call reads its partials from
    # HBM; the back-to-back figures above re-read one 201 MB set, which the
    # MALL partly serves
    sets = [parts] + [[p.roll(k + 1, 0) for p in parts] for k in range(3)]
    ring = {"i": 0}

    def cold(fn):
        def call():
            ring["i"] = (ring["i"] + 1) % len(sets)
            fn(sets[ring["i"]])
        return call
    ms8c = _timed(cold(lambda ps: ops.quant_dequant_sum_int8_tok(ps, payloads=pays, out=out)), iters, 4)
    ms16c = _timed(cold(lambda ps: ops.quant_dequant_sum_fp16(ps, payloads=p16, out=out)), iters, 4)
    del sets
    # the headline rates are the cold-HBM ones: every call reads its inputs from HBM
    return {"int8_us": ms8c * 1e3, "int8_gbps": bytes8 / ms8c / 1e6,
            "int8_frac_hbm_peak": bytes8 / ms8c / 1e6 / HBM_PEAK_GBPS, "int8_cpu_baseline": cpu,
            "fp16_us": ms16c * 1e3, "fp16_gbps": bytes16 / ms16c / 1e6,
            "fp16_frac_hbm_peak": bytes16 / ms16c / 1e6 / HBM_PEAK_GBPS, "fp16_bit_exact_vs_torch": exact16,
            "how": "4 distinct partial sets (805 MB) cycled, so each call's inputs come from HBM, not the MALL",
            "mall_warm": {"int8_us": ms8 * 1e3, "int8_gbps": bytes8 / ms8 / 1e6,
                          "fp16_us": ms16 * 1e3, "fp16_gbps": bytes16 / ms16 / 1e6,
                          "how": "one 201 MB set re-read back to back, partly served by the 256 MB MALL"},
            "algorithmic_bytes": {"int8": bytes8, "fp16": bytes16}}


def _torch_scan_ref(u, delta, A, B, C, Dv, z, bias):
    """Sequential fp32 scan in torch on the GPU (reference model.py:216-238
    op order) for a small block: u, delta, z [D, L]; B, C [L, N]."""
    import torch
    import torch.nn.functional as F
    dt = F.softplus(delta + bias[:, None])
    h = torch.zeros(u.shape[0], A.shape[1], device=u.device)
    ys = []
    for t in range(u.shape[1]):
        h = torch.exp(dt[:, t, None] * A) * h + (dt[:, t, None] * B[t][None, :]) * u[:, t, None]
        ys.append(h @ C[t])
    y = torch.stack(ys, 1)
    return (y + u * Dv[:, None]) * F.silu(z)


def bench_shard(dev, iters=10):
    """One TP rank's channel shard of the 1.4b mixer (D = 2048 of 4096),
    bf16 activations with fp32 state, b=32 x l=2048, token-major layout as
    the mixer produces it."""
    import torch
    import torch.nn.functional as F
    from mamba_lite import ops
    b, L, D, N, R = 32, 2048, 2048, 16, 128
    g = torch.Generator(device=dev).manual_seed(5)
    bf = torch.bfloat16
    # the layouts MambaMixer.prefill produces: x and z as separate token-major
    # [b, l, D] in_proj outputs, B and C as separate [b, l, N] x_proj outputs
    xin = torch.randn(b, L, D, device=dev, generator=g).to(bf)
    zin = torch.randn(b, L, D, device=dev, generator=g).to(bf)
    Bin = torch.randn(b, L, N, device=dev, generator=g).to(bf)
    Cin = torch.randn(b, L, N, device=dev, generator=g).to(bf)
    delta = (0.5 * torch.randn(b, L, D, device=dev, generator=g)).to(bf)
    bias = torch.from_numpy(dt_bias_init(D, 5)).to(dev)
    w = torch.randn(D, 4, device=dev, generator=g) * 0.5
    cb = torch.randn(D, device=dev, generator=g) * 0.1
    A_log = torch.log(torch.arange(1, N + 1, device=dev, dtype=torch.float32)).repeat(D, 1).contiguous()
    Dv = torch.ones(D, device=dev)
    u = torch.empty(b, L, D, device=dev, dtype=bf)
    y = torch.empty(b, L, D, device=dev, dtype=bf)
    fs = torch.empty(b, D, 3, device=dev, dtype=bf)
    h = torch.empty(b, D, N, device=dev)
    xs, z = xin.transpose(1, 2), zin.transpose(1, 2)
    Bv, Cv = Bin.transpose(1, 2), Cin.transpose(1, 2)
    conv = lambda: ops.causal_conv1d(xs, w, cb, out=u.transpose(1, 2), final_state=fs)
    scan = lambda: ops.selective_scan(u.transpose(1, 2), delta.transpose(1, 2), A_log, Bv, Cv, D=Dv, z=z,
                                      delta_bias=bias, a_is_log=True, y=y.transpose(1, 2), h_out=h)
    t0 = time.perf_counter()      # settle clocks under sustained load first, as for the headline scan
    while time.perf_counter() - t0 < 1.5:
        scan()
        conv()
        torch.cuda.synchronize()
    ms_conv = _timed(conv, iters, 2)
    ms_scan = _timed(scan, iters, 2)
    torch.cuda.synchronize()
    # parity gate: batch row 0, channels 640..703, torch fp32 on the same bf16 inputs
    sl = slice(640, 704)
    with torch.no_grad():
        xr = F.pad(xs[0, sl].float(), (3, 0))
        cref = F.silu(F.conv1d(xr[None], w[sl][:, None, :], cb[sl], groups=64)[0])
        e_conv = float(((u[0, :, sl].float().T - cref).abs().max() / cref.abs().max()).item())
        yr = _torch_scan_ref(u[0, :, sl].float().T, delta[0, :, sl].float().T, -torch.exp(A_log[sl]),
                             Bv[0].float().T.contiguous(), Cv[0].float().T.contiguous(), Dv[sl], z[0, sl].float(),
                             bias[sl])
        e_scan = float(((y[0, :, sl].float().T - yr).abs().max() / yr.abs().max()).item())
    conv_bytes = 2 * b * L * D * 2 + b * D * 3 * 2 + D * 4 * 4 + D * 4   # x, u; final state out; w, bias
    scan_bytes = 4 * b * L * D * 2 + 2 * b * N * L * 2 + b * D * N * 4 + D * N * 4 + 2 * D * 4   # u,delta,z,y; B,C; h; A; D,bias
    return {"conv_us": ms_conv * 1e3, "conv_gbps": conv_bytes / ms_conv / 1e6,
            "scan_us": ms_scan * 1e3, "scan_gbps": scan_bytes / ms_scan / 1e6,
            "scan_frac_hbm_peak": scan_bytes / ms_scan / 1e6 / HBM_PEAK_GBPS,
            "scan_valu_roofline": valu_roofline("bf16_b32_d2048_l2048", ms_scan * 1e3),
            "tok_s": b * L / ((ms_conv + ms_scan) / 1000.0),
            "max_rel_err_vs_torch_fp32": {"conv": e_conv, "scan": e_scan},
            "algorithmic_bytes": {"conv": conv_bytes, "scan": scan_bytes}}


# --------------------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default="all",
                    choices=["all", "scan", "decode", "quant", "shard", "prefill", "prefill-short", "prefill-long",
                             "copy", "decode-counters"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode-shapes", default="130m,1.4b", help="comma list of 130m, 1.4b")
    ap.add_argument("--decode-batches", default="",
                    help="comma list of batch sizes for every decode shape (default: 1 at 130m, 1 and 32 at 1.4b)")
    ap.add_argument("--no-step-fold", action="store_true",
                    help="batched steps of 3-16 rows keep the add + norm launch between blocks (MambaLM folds it "
                         "into the projections by default)")
    ap.add_argument("--decode-persist", action="store_true",
                    help="decode batch 1 through the persistent single-launch step (off by default in MambaLM); "
                         "the shapes it does not take run their usual step")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU and has no multi-GPU mode (asked for --gpus {args.gpus}); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from mamba_lite import _lib
    from mamba_lite.model import MambaConfig
    _lib.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    result = {"metric": METRIC}
    extra = {}
    # the tuned projection GEMMs of the prefill shapes (mamba_lite/gemm_table.py)
    from mamba_lite import gemm_table
    gemm_ok = gemm_table.enable() if args.only != "copy" else False
    log(f"tuned GEMM table {'loaded' if gemm_ok else 'not used (default GEMM paths)'}")

    want = lambda s: args.only in ("all", s)
    if args.only == "copy":
        # calibration for rocprofv3 FETCH_SIZE / WRITE_SIZE: a plain device copy
        # of a known 1 GiB fp32 buffer, 5 times
        n = 1 << 28
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": n * 4, "launches": 5}), flush=True)
        return
    if args.only == "prefill-short":
        # the eager 64-token prompt alone (130m shape, b=1, fp32), for a
        # rocprofv3 trace of the one-call short prefill: 3 warmup prompts, then
        # the 20 timed ones of the prefill_tok_s entry
        model = build_lm(MambaConfig(d_model=768, n_layer=24, vocab_size=50280), dev)
        tok_s = bench_prefill(model, 1, 64, dev)
        log(f"prefill-short 130m b=1 x 64 eager: {tok_s:.0f} tok/s, {64 / tok_s * 1e6:.1f} us per prompt")
        print(json.dumps({"prefill_tok_s": {"130m_b1_l64": tok_s}}), flush=True)
        return
    if args.only == "prefill-long":
        # the 32 x 1024-token prefills alone (130m and 1.4b shapes, fp32), for
        # rocprofv3 traces of their GEMM / conv / scan split: 1 warmup + 3
        # timed prompts each
        for name, kw in (("130m", dict(d_model=768, n_layer=24, vocab_size=50280)),
                         ("1p4b", dict(d_model=2048, n_layer=48, vocab_size=50280))):
            model = build_lm(MambaConfig(**kw), dev)
            tok_s = bench_prefill(model, 32, 1024, dev, iters=3)
            log(f"prefill-long {name} b=32 x 1024: {tok_s:.0f} tok/s")
            print(json.dumps({"prefill_tok_s": {f"{name}_b32_l1024": tok_s}}), flush=True)
            del model
            torch.cuda.empty_cache()
        return
    if args.only == "decode-counters":
        # a short workload for rocprofv3 --pmc runs over the decode kernels
        # (counter collection serializes every dispatch, so the timed decode
        # bench's replays take minutes there): the 1.4b shape, a 16-token
        # prefill, then 4 eager steps at batch 1 (fused path) and batch 32
        # (per-op path), the same kernels on the same shapes as the graphs
        model = build_lm(MambaConfig(d_model=2048, n_layer=48, vocab_size=50280), dev)
        for b in (1, 32):
            g = torch.Generator(device=dev).manual_seed(1)
            ids = torch.randint(0, 50280, (b, 16), device=dev, generator=g)
            nxt = torch.zeros(b, 1, dtype=torch.long, device=dev)
            with torch.no_grad():
                _, cache = model.prefill(ids)
                for s in range(4):
                    model.step(nxt, cache)
                    torch.cuda.synchronize()
                    log(f"decode-counters 1.4b b={b}: step {s} done")
        return
    if want("scan"):
        log("scan: isolated selective scan fp32 [32,1536,1024]")
        t0 = time.perf_counter()
        ms, trials, gpu_run, prewarm = bench_scan(dev, args.steps, args.warmup)
        wall = time.perf_counter() - t0
        gbps = SCAN_BYTES / ms / 1e6
        result.update({
            "value": SCAN_B * SCAN_L / (ms / 1000.0), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded torch.Generator / numpy)",
            "config": {"workload": "isolated selective scan fp32: u, delta, z [32,1536,1024]; B, C [32,16,1024]; "
                                   "A [1536,16] = -(1..16); D = 1; y and final state h [32,1536,16]",
                       "batch": SCAN_B, "dim": SCAN_D, "seqlen": SCAN_L, "dstate": SCAN_N},
            "roofline": {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                         "frac": gbps / HBM_PEAK_GBPS,
                         "traffic": traffic_from_profiles("scan_fp32_b32_d1536_l1024"),
                         "kernel": "scan_fwd_kernel<float, NW=4, SPW=4, TT=16, channel-major>",
                         "algorithmic_bytes": SCAN_BYTES,
                         "limiter": "VALU issue and the access pattern together: 102 VALU instructions per 64 "
                                    "(channel, step) pairs, 80 of them the 16-state recurrence, 76% VALU busy "
                                    "(rocprofv3 counters; 156 us of VALU issue at 100% and the 2.4 GHz peak "
                                    "clock, scan_valu_roofline); the same channel-major "
                                    "u/delta/z/y stream with no arithmetic takes 173 us (4.65 TB/s)"},
        })
        extra["scan_valu_roofline"] = valu_roofline("fp32_b32_d1536_l1024", ms * 1e3)
        extra["scan_trials_ms"] = trials
        extra["scan_prewarm"] = prewarm
        log(f"scan: {ms*1000:.1f} us/call, {gbps:.0f} GB/s ({gbps/HBM_PEAK_GBPS:.1%} of peak), {wall:.1f}s")
        if not args.no_cpu_baseline:
            workers = max(1, min(16, os.cpu_count() or 1))
            log(f"cpu baseline: oracle scan, {workers} processes")
            secs, err = cpu_baseline_scan(workers, gpu_run)
            extra["scan_max_rel_err_vs_oracle"] = err
            result["cpu_baseline"] = {
                "value": SCAN_B * SCAN_L / secs, "unit": "tok/s", "cores": workers, "kind": "port",
                "sample": f"the full isolated-scan workload (32 rows x 1536 ch x 1024 steps x 16 states), numpy "
                          f"float32 materialize-then-loop, one batch row per process over {workers} processes; "
                          f"{secs:.1f} s wall",
                **host_info()}
            log(f"cpu baseline: {secs:.1f}s; GPU scan max rel err vs oracle {err:.2e}")

    if want("decode"):
        dec = {}
        if args.decode_persist:
            import mamba_lite.model as mm
            mm.DECODE_PERSIST = True
            extra["decode_persist"] = True
        if args.no_step_fold:
            import mamba_lite.model as mm
            mm.STEP_NORM_FOLD = False
            extra["step_fold"] = False
        only_b = tuple(int(v) for v in args.decode_batches.split(",") if v) if args.decode_batches else None
        for name, cfg_kw, batches, prompt, ntok in (
                ("130m", dict(d_model=768, n_layer=24, vocab_size=50280), (1,), 64, 256),
                ("1.4b", dict(d_model=2048, n_layer=48, vocab_size=50280), (1, 32), 1024, 256)):
            if name not in args.decode_shapes.split(","):
                continue
            try:
                log(f"decode {name}: building model")
                model = build_lm(MambaConfig(**cfg_kw), dev)
                for bsz in (only_b or batches):
                    us, ok, us_eager = bench_decode(model, bsz, prompt, ntok, dev)
                    dec[f"{name}_b{bsz}"] = {"us_per_step": us, "us_per_token": us / bsz, "graph_equals_eager": ok,
                                             "prompt": prompt, "tokens_timed": ntok, "eager_us_per_step": us_eager}
                    log(f"decode {name} b={bsz}: {us:.1f} us/step (graph==eager {ok}); eager {us_eager:.1f} us/step")
                if name == "130m" and not args.no_cpu_baseline:
                    cb = cpu_baseline_decode(model, dev)
                    dec.setdefault("130m_b1", {})["cpu_baseline"] = cb
                    log(f"decode cpu baseline: {cb['value']:.0f} us/token; GPU step rel err vs oracle "
                        f"{cb['gpu_step_max_rel_err_vs_oracle_f64']:.2e}")
                if name == "1.4b" and not args.no_cpu_baseline:
                    # reduced: a 16-token prompt (not 1024) and 8 timed steps at
                    # batch 1; the float64 parity of this shape is in the tests
                    cb = cpu_baseline_decode(model, dev, prompt=16, steps=8, name="1.4b", parity=False)
                    dec.setdefault("1.4b_b1", {})["cpu_baseline"] = cb
                    log(f"decode 1.4b cpu baseline: {cb['value']:.0f} us/token")
                del model
                torch.cuda.empty_cache()
            except Exception as e:  # report, keep the headline line
                dec[name] = {"error": repr(e)}
                log(f"decode {name} failed: {e!r}")
        extra["decode_us_per_token"] = dec

    if want("prefill"):
        try:
            model = build_lm(MambaConfig(d_model=768, n_layer=24, vocab_size=50280), dev)
            # 64 tokens: mtl_prefill_short; 256: mtl_prefill_long; 32 x 1024: the per-op path
            extra["prefill_tok_s"] = {"130m_b1_l64": bench_prefill(model, 1, 64, dev),
                                      "130m_b1_l256": bench_prefill(model, 1, 256, dev),
                                      "130m_b32_l1024": bench_prefill(model, 32, 1024, dev)}
            log(f"prefill: {extra['prefill_tok_s']}")
            extra["prefill_graph_tok_s"] = {"130m_b1_l64": bench_prefill_graph(model, 1, 64, dev)}
            log(f"prefill graph: {extra['prefill_graph_tok_s']}")
            del model
            torch.cuda.empty_cache()
            # the 1.4b shape's 1024-token prompts (48 layers, d_inner 4096)
            model = build_lm(MambaConfig(d_model=2048, n_layer=48, vocab_size=50280), dev)
            extra["prefill_tok_s"]["1p4b_b1_l128"] = bench_prefill(model, 1, 128, dev)
            extra["prefill_tok_s"]["1p4b_b1_l1024"] = bench_prefill(model, 1, 1024, dev, iters=5)
            extra["prefill_tok_s"]["1p4b_b32_l1024"] = bench_prefill(model, 32, 1024, dev, iters=2)
            log(f"prefill 1.4b: b=1 x 1024 {extra['prefill_tok_s']['1p4b_b1_l1024']:.0f} tok/s, "
                f"b=32 x 1024 {extra['prefill_tok_s']['1p4b_b32_l1024']:.0f} tok/s")
            del model
            torch.cuda.empty_cache()
        except Exception as e:
            extra.setdefault("prefill_tok_s", {})["error"] = repr(e)

    if want("quant"):
        try:
            extra["quant"] = bench_quant(dev)
            log(f"quant: {extra['quant']}")
        except Exception as e:
            extra["quant"] = {"error": repr(e)}

    if want("shard"):
        try:
            extra["shard_bf16"] = bench_shard(dev)
            log(f"shard: {extra['shard_bf16']}")
        except Exception as e:
            extra["shard_bf16"] = {"error": repr(e)}

    if "value" not in result:
        result.update({"value": None, "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                       "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                       "dtype": "f32", "data": "synthetic", "config": {"workload": f"partial run: {args.only}"}})
    result.update(extra)
    result["device"] = torch.cuda.get_device_name(dev)
    result["gemm_table"] = {"loaded": gemm_ok, "file": "mamba-tp-lite_amd/mamba_lite/gemm_table_gfx950.csv",
                            "covers": "prefill projection and lm_head shapes of the 130m model at 32 x 1024 tokens "
                                      "and the lm_head of its 64-token prompt; of the 1.4b model at 1 x 1024 and "
                                      "32 x 1024 tokens; the 1.4b batch-32 decode step's lm_head"}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
