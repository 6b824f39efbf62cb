"""Golden-vector recipes shared by tests/golden/make_fixtures.py (which runs
the reference's PyTorch model once, in the development container) and the
tests that read the vectors back.

Weights are not stored in the fixtures: each case names a seed, and
`mixer_weights` / `lm_weights` rebuild the same float32 arrays from it with
numpy's PCG64 generator, under the reference's parameter names
(mamba_lite/model.py:160-169, 300, 320-322).  A fixture file then holds the
inputs and the reference's outputs only.

The draws are chosen so that a wiring slip changes the result: A_log is
log(1..N) plus a per-(channel, state) offset and D, the norm weights and the
biases are not constants, so a transposed or channel-blind read of any of
them shows.
"""
from __future__ import annotations

import os

import numpy as np

GOLDEN_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _inv_softplus(y):
    y = np.asarray(y, np.float64)
    return y + np.log(-np.expm1(-y))


def _u(rng, shape, bound):
    return rng.uniform(-bound, bound, shape).astype(np.float32)


def mixer_weights(rng, d_model, d_state=16, d_conv=4, expand=2, dt_rank=None, bias=False, conv_bias=True,
                  prefix=""):
    """One MambaMixer's parameters (reference model.py:160-169) as float32
    numpy arrays keyed by their state-dict names (with `prefix`)."""
    D = expand * d_model
    R = dt_rank if dt_rank is not None else max(1, d_model // 16)
    N, K, M = d_state, d_conv, d_model
    w = {}
    w["in_proj.weight"] = _u(rng, (2 * D, M), M ** -0.5)
    if bias:
        w["in_proj.bias"] = _u(rng, (2 * D,), M ** -0.5)
    w["conv1d.weight"] = _u(rng, (D, 1, K), K ** -0.5)
    if conv_bias:
        w["conv1d.bias"] = _u(rng, (D,), K ** -0.5)
    w["x_proj.weight"] = _u(rng, (R + 2 * N, D), D ** -0.5)
    w["dt_proj.weight"] = _u(rng, (D, R), R ** -0.5)
    w["dt_proj.bias"] = _inv_softplus(np.exp(rng.uniform(np.log(1e-3), np.log(0.1), D))).astype(np.float32)
    w["A_log"] = (np.log(np.arange(1, N + 1, dtype=np.float64))[None, :]
                  + rng.uniform(-0.3, 0.3, (D, N))).astype(np.float32)
    w["D"] = rng.uniform(0.5, 1.5, D).astype(np.float32)
    w["out_proj.weight"] = _u(rng, (M, D), D ** -0.5)
    if bias:
        w["out_proj.bias"] = _u(rng, (M,), D ** -0.5)
    return {prefix + k: v for k, v in w.items()}


def lm_weights(seed, d_model, n_layer, vocab_size, **mixer_kw):
    """A MambaLM state dict (reference model.py:317-322): embedding ~ N(0, 1),
    per-layer norm weights U(0.8, 1.2), mixers as mixer_weights, norm_f
    U(0.8, 1.2).  vocab_size must already be padded (MambaConfig rounds it
    up to a multiple of 8)."""
    rng = np.random.default_rng(seed)
    sd = {"embedding.weight": rng.standard_normal((vocab_size, d_model)).astype(np.float32)}
    for i in range(n_layer):
        sd[f"layers.{i}.norm.weight"] = rng.uniform(0.8, 1.2, d_model).astype(np.float32)
        sd.update(mixer_weights(rng, d_model, prefix=f"layers.{i}.mixer.", **mixer_kw))
    sd["norm_f.weight"] = rng.uniform(0.8, 1.2, d_model).astype(np.float32)
    return sd


def mixer_case_weights(seed, d_model, **mixer_kw):
    return mixer_weights(np.random.default_rng(seed), d_model, **mixer_kw)


def oracle_mixer_dict(sd, prefix=""):
    """Reference state-dict names -> the oracle's mixer dict (oracle/mixer.py)."""
    g = lambda k: sd.get(prefix + k)
    d = {"in_proj_w": g("in_proj.weight"), "conv_w": g("conv1d.weight")[:, 0, :], "conv_b": g("conv1d.bias"),
         "x_proj_w": g("x_proj.weight"), "dt_proj_w": g("dt_proj.weight"), "dt_proj_b": g("dt_proj.bias"),
         "A_log": g("A_log"), "D": g("D"), "out_proj_w": g("out_proj.weight")}
    if g("in_proj.bias") is not None:
        d["in_proj_b"] = g("in_proj.bias")
    if g("out_proj.bias") is not None:
        d["out_proj_b"] = g("out_proj.bias")
    return d


def oracle_lm_dict(sd, n_layer):
    layers = []
    for i in range(n_layer):
        d = oracle_mixer_dict(sd, f"layers.{i}.mixer.")
        d["norm"] = sd[f"layers.{i}.norm.weight"]
        layers.append(d)
    return {"embedding": sd["embedding.weight"], "norm_f": sd["norm_f.weight"], "layers": layers}


# ---------------------------------------------------------------- the cases
# Mixer cases: (name, seed, config).  Each fixture holds, for a batch of 2:
# prefill of x0 without a cache, a continuation prefill of x1 from that
# cache, then three steps from the continuation's cache.
MIXER_CASES = [
    # the reference's own TP test configuration (tests/test_tp_correctness.py:28-30)
    ("mixer_d32_n8", 11, dict(d_model=32, d_state=8, d_conv=4, expand=2)),
    # in_proj / out_proj biases (MambaConfig.bias), 16 states
    ("mixer_d64_bias", 12, dict(d_model=64, d_state=16, d_conv=4, expand=2, bias=True)),
    # a 2-tap conv without bias, explicit dt_rank
    ("mixer_d48_k2", 13, dict(d_model=48, d_state=4, d_conv=2, expand=2, dt_rank=5, conv_bias=False)),
    # d_conv = 1: prefill applies the 1-tap conv and its bias, step skips it (model.py:206-212, 265-276)
    ("mixer_d32_k1", 14, dict(d_model=32, d_state=16, d_conv=1, expand=2)),
]
MIXER_LENGTHS = (7, 5)     # x0, x1 token counts
MIXER_STEPS = 3

# LM cases: (name, seed, config, batch, prompt length, teacher-forced steps)
LM_CASES = [
    ("lm_d64_l2", 21, dict(d_model=64, n_layer=2, vocab_size=104), 2, 9, 3),
    ("lm_d48_l3_k3", 22, dict(d_model=48, n_layer=3, vocab_size=64, d_state=8, d_conv=3), 1, 6, 3),
    # one layer at the mamba-1.4b width (d_model 2048, d_inner 4096, dt_rank 128)
    ("lm_1p4b_width_l1", 23, dict(d_model=2048, n_layer=1, vocab_size=256, dt_rank=128), 1, 12, 3),
]

# HF-snapshot loader case: config.json + safetensors written by the fixture
# script, and what the reference's from_pretrained (model.py:367-397) loads.
HF_CASE = ("hf_tiny", 31, dict(d_model=32, n_layer=2, vocab_size=64, d_state=8))


def lm_config_kw(cfg):
    return {k: v for k, v in cfg.items() if k not in ("d_model", "n_layer", "vocab_size")}


def load(name):
    path = os.path.join(GOLDEN_DIR, name + ".npz")
    with np.load(path, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}
