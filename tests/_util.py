"""Shared test helpers (no test functions here)."""
from __future__ import annotations

import numpy as np

from oracle import mixer as om


def assert_rel(got, ref, tol, what=""):
    """Elementwise |got - ref| <= tol * |ref| + tol * rms(ref).

    The rms floor keeps entries that cancel to ~0 from demanding relative
    accuracy that no fp32 evaluation order has; everywhere else this is a
    plain relative tolerance of `tol`."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    if ref.size == 0:
        return
    floor = tol * np.sqrt(np.mean(ref * ref))
    err = np.abs(got - ref)
    bound = tol * np.abs(ref) + floor
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())}/{bad.size} elements off; worst at {i}: got {got[i]!r} "
                             f"ref {ref[i]!r} (|err| {err[i]:.3e} > {bound[i]:.3e}; tol {tol})")


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest even) and back to float32."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).bfloat16().float().numpy()


def scan_case(rng, b, D, L, N, dtype=np.float32):
    """Inputs distributed as the isolated selective-scan benchmark: u, z ~
    N(0,1); delta ~ N(0, 0.5^2) pre-bias with dt_bias = inv_softplus of a
    log-uniform [1e-3, 0.1] draw; B, C ~ N(0,1) as [b, N, L]; A = -(1..N);
    D = 1."""
    u = rng.standard_normal((b, D, L)).astype(dtype)
    delta = (0.5 * rng.standard_normal((b, D, L))).astype(dtype)
    bias = om.inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32)
    B = rng.standard_normal((b, N, L)).astype(dtype)
    C = rng.standard_normal((b, N, L)).astype(dtype)
    z = rng.standard_normal((b, D, L)).astype(dtype)
    A = -np.tile(np.arange(1, N + 1, dtype=np.float32), (D, 1))
    Dv = np.ones(D, np.float32)
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=Dv, z=z, delta_bias=bias)


def write_hf_snapshot(path, cfg, sd, shards=1):
    """A local `mamba-*-hf` style directory: config.json + safetensors with
    the `backbone.` names (embeddings, layers.{i}.mixer.*, norm_f)."""
    import json
    from safetensors.torch import save_file
    (path / "config.json").write_text(json.dumps({
        "hidden_size": cfg.d_model, "num_hidden_layers": cfg.n_layer, "vocab_size": cfg.vocab_size,
        "state_size": cfg.d_state, "conv_kernel": cfg.d_conv, "expand": cfg.expand, "time_step_rank": cfg.dt_rank,
        "use_conv_bias": cfg.conv_bias, "use_bias": cfg.bias}))
    hf = {}
    for k, v in sd.items():
        if k == "embedding.weight":
            hf["backbone.embeddings.weight"] = v
        elif k == "norm_f.weight":
            hf["backbone.norm_f.weight"] = v
        else:
            hf["backbone." + k] = v
    hf["lm_head.weight"] = sd["embedding.weight"].clone()   # tied; ignored by the loader
    keys = sorted(hf)
    if shards == 1:
        save_file({k: hf[k].contiguous() for k in keys}, str(path / "model.safetensors"))
        return
    weight_map = {}
    for s in range(shards):
        part = keys[s::shards]
        name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: hf[k].contiguous() for k in part}, str(path / name))
        weight_map.update({k: name for k in part})
    (path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
