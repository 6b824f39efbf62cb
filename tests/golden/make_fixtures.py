"""Writes the golden vectors of tests/golden/ from the reference's own
PyTorch model (mamba-tp-lite, mamba_lite/model.py), run on the CPU in float32.

    python tests/golden/make_fixtures.py [--reference /root/reference]

Runs only where the reference checkout is present (the development
container); the tests read the .npz files it writes and never the reference.
Weights are rebuilt from seeds by tests/_golden.py, so the files hold inputs
and outputs only.  What each file holds:

  mixer_*.npz  MambaMixer (model.py:184-294), batch 2:
      x0 [2,l0,M]      -> out0, conv0, ssm0   prefill without a cache
      x1 [2,l1,M]      -> out1, conv1, ssm1   prefill continuing from (conv0, ssm0)
      xs [S,2,M]       -> step_out [S,2,M]    steps from (conv1, ssm1), state
                          after each step in step_conv [S,...], step_ssm [S,...]
  lm_*.npz     MambaLM (model.py:314-353):
      ids [b, l+S]     -> logits [b,l,V] and per-layer conv_i / ssm_i of the
                          prompt prefill of ids[:, :l]; step_logits [S,b,1,V]
                          of teacher-forced steps on ids[:, l:], and the
                          states after them (end_conv_i / end_ssm_i)
  hf_tiny/, hf_tiny_sharded/   a synthetic `mamba-*-hf` snapshot (config.json
      + safetensors, one file / three files with an index), and hf_tiny.npz:
      the state dict the reference's from_pretrained (model.py:367-397)
      loads from it (keys as `sd.<name>`) and its prefill logits on `ids`.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))   # tests/ for _golden
import _golden as G  # noqa: E402


def _load_reference(ref_root):
    path = os.path.join(ref_root, "mamba_lite", "model.py")
    spec = importlib.util.spec_from_file_location("reference_mamba_model", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod   # dataclasses resolve annotations through the module table
    spec.loader.exec_module(mod)
    return mod


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def _n(t):
    return t.detach().cpu().numpy().astype(np.float32, copy=True)


def _save(name, arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} B)")


def make_mixer(ref, name, seed, cfg):
    mc = ref.MambaConfig(d_model=cfg["d_model"], n_layer=1, vocab_size=8, **G.lm_config_kw(cfg))
    mixer = ref.MambaMixer(mc, layer_idx=0).eval()
    sd = G.mixer_case_weights(seed, **cfg)
    mixer.load_state_dict({k: _t(v) for k, v in sd.items()}, strict=True)
    rng = np.random.default_rng(seed + 1000)
    l0, l1 = G.MIXER_LENGTHS
    M = cfg["d_model"]
    x0 = rng.standard_normal((2, l0, M)).astype(np.float32)
    x1 = rng.standard_normal((2, l1, M)).astype(np.float32)
    xs = rng.standard_normal((G.MIXER_STEPS, 2, M)).astype(np.float32)
    out = {"x0": x0, "x1": x1, "xs": xs}
    with torch.no_grad():
        o0, c0, h0 = mixer.prefill(_t(x0), None)
        o1, c1, h1 = mixer.prefill(_t(x1), ref.LayerCache(conv_state=c0, ssm_state=h0))
        cache = ref.LayerCache(conv_state=c1.clone(), ssm_state=h1.clone())
        so, sc, sh = [], [], []
        for k in range(G.MIXER_STEPS):
            so.append(_n(mixer.step(_t(xs[k]), cache)))
            sc.append(_n(cache.conv_state))
            sh.append(_n(cache.ssm_state))
    out.update(out0=_n(o0), conv0=_n(c0), ssm0=_n(h0), out1=_n(o1), conv1=_n(c1), ssm1=_n(h1),
               step_out=np.stack(so), step_conv=np.stack(sc), step_ssm=np.stack(sh))
    _save(name, out)


def make_lm(ref, name, seed, cfg, batch, plen, steps):
    mc = ref.MambaConfig(d_model=cfg["d_model"], n_layer=cfg["n_layer"], vocab_size=cfg["vocab_size"],
                         **G.lm_config_kw(cfg))
    assert mc.vocab_size == cfg["vocab_size"], "fixture vocab sizes are multiples of 8"
    lm = ref.MambaLM(mc).eval()
    sd = G.lm_weights(seed, cfg["d_model"], cfg["n_layer"], cfg["vocab_size"], **G.lm_config_kw(cfg))
    lm.load_state_dict({k: _t(v) for k, v in sd.items()}, strict=True)
    rng = np.random.default_rng(seed + 1000)
    ids = rng.integers(0, cfg["vocab_size"], (batch, plen + steps), dtype=np.int64)
    out = {"ids": ids}
    with torch.no_grad():
        logits, cache = lm.prefill(_t(ids[:, :plen]))
        out["logits"] = _n(logits)
        for i, lc in enumerate(cache.layers):
            out[f"conv_{i}"] = _n(lc.conv_state)
            out[f"ssm_{i}"] = _n(lc.ssm_state)
        sl = [_n(lm.step(_t(ids[:, plen + k:plen + k + 1]), cache)) for k in range(steps)]
        out["step_logits"] = np.stack(sl)
        for i, lc in enumerate(cache.layers):
            out[f"end_conv_{i}"] = _n(lc.conv_state)
            out[f"end_ssm_{i}"] = _n(lc.ssm_state)
    _save(name, out)


def _write_snapshot(path, cfg, sd, shards):
    """config.json with the HF key names that MambaConfig.from_hf_config reads
    (model.py:79-93) and the weights under their `backbone.` names."""
    from safetensors.numpy import save_file

    os.makedirs(path, exist_ok=True)
    for f in os.listdir(path):
        os.remove(os.path.join(path, f))
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump({"hidden_size": cfg["d_model"], "num_hidden_layers": cfg["n_layer"],
                   "vocab_size": cfg["vocab_size"], "state_size": cfg.get("d_state", 16),
                   "conv_kernel": cfg.get("d_conv", 4), "expand": 2,
                   "time_step_rank": max(1, cfg["d_model"] // 16), "use_conv_bias": True, "use_bias": False,
                   "pad_vocab_size_multiple": 8, "layer_norm_epsilon": 1e-5}, f, indent=1, sort_keys=True)
    hf = {}
    for k, v in sd.items():
        if k == "embedding.weight":
            hf["backbone.embeddings.weight"] = v
        elif k == "norm_f.weight":
            hf["backbone.norm_f.weight"] = v
        else:
            hf["backbone." + k] = v
    hf["lm_head.weight"] = sd["embedding.weight"].copy()   # tied in the checkpoints; the loader skips it
    keys = sorted(hf)
    if shards == 1:
        save_file({k: hf[k] for k in keys}, os.path.join(path, "model.safetensors"))
        return
    weight_map = {}
    for s in range(shards):
        part = keys[s::shards]
        fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: hf[k] for k in part}, os.path.join(path, fname))
        weight_map.update({k: fname for k in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f, indent=1, sort_keys=True)


def make_hf(ref, name, seed, cfg):
    sd = G.lm_weights(seed, cfg["d_model"], cfg["n_layer"], cfg["vocab_size"], d_state=cfg["d_state"])
    single, sharded = os.path.join(HERE, name), os.path.join(HERE, name + "_sharded")
    _write_snapshot(single, cfg, sd, 1)
    _write_snapshot(sharded, cfg, sd, 3)
    rng = np.random.default_rng(seed + 1000)
    ids = rng.integers(0, cfg["vocab_size"], (2, 6), dtype=np.int64)
    out = {"ids": ids}
    for tag, path in (("", single), ("sharded_", sharded)):
        lm = ref.MambaLM.from_pretrained(path, dtype=torch.float32).eval()
        with torch.no_grad():
            logits, _ = lm.prefill(_t(ids))
        out[tag + "logits"] = _n(logits)
        if not tag:
            for k, v in lm.state_dict().items():
                out["sd." + k] = _n(v)
        out[tag + "vocab_size"] = np.int64(lm.cfg.vocab_size)
        out[tag + "dt_rank"] = np.int64(lm.cfg.dt_rank)
    _save(name, out)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args(argv)
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    ref = _load_reference(args.reference)
    for name, seed, cfg in G.MIXER_CASES:
        make_mixer(ref, name, seed, cfg)
    for name, seed, cfg, batch, plen, steps in G.LM_CASES:
        make_lm(ref, name, seed, cfg, batch, plen, steps)
    make_hf(ref, *G.HF_CASE)


if __name__ == "__main__":
    main()
