"""Drop-in Mamba (v1) model API backed by the MI355X kernels.

Same public surface as mamba-tp-lite's mamba_lite/model.py:
  MambaConfig, LayerCache, MambaCache.allocate, RMSNorm, MambaMixer
  (.prefill / .step / .forward), MambaBlock, MambaLM (.prefill / .step /
  .generate / .from_pretrained), load_hf_state_dict.
Parameter names and shapes match the reference, so its state dicts (and HF
`state-spaces/mamba-*-hf` checkpoints through from_pretrained) load as is.

What runs where: the prefill's in_proj / x_proj / dt_proj / out_proj and the
lm_head are torch GEMMs (hipBLASLt / rocBLAS).  The decode step's projections
run on libmtl kernels: GEMVs fused with the norm and the residual at batch
<= 4, matrix-core skinny GEMMs at <= 32 tokens (in_proj fused with the conv
step and x_proj).  The causal conv + SiLU, the selective scan (with dt bias,
softplus, D skip and SiLU gate fused), the single-token conv and SSM updates
and the residual + RMSNorm are libmtl HIP kernels as well.  The model runs on
the GPU only.

Deliberate deviation: with bfloat16 activations the SSM state stays float32
(the cache allocates it in float32 and prefill returns it in float32);
the reference casts it to the activation dtype (model.py:241).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib, ops


def load_hf_state_dict(hf_path: str) -> dict[str, torch.Tensor]:
    """Reads a HF checkpoint directory: model.safetensors, or the shards named
    by model.safetensors.index.json (reference model.py:28-47)."""
    from safetensors.torch import load_file

    single = os.path.join(hf_path, "model.safetensors")
    index = os.path.join(hf_path, "model.safetensors.index.json")
    if os.path.exists(single):
        return load_file(single)
    if os.path.exists(index):
        with open(index) as f:
            shards = sorted(set(json.load(f)["weight_map"].values()))
        merged: dict[str, torch.Tensor] = {}
        for name in shards:
            merged.update(load_file(os.path.join(hf_path, name)))
        return merged
    raise FileNotFoundError(f"no model.safetensors or model.safetensors.index.json under {hf_path}")


@dataclass
class MambaConfig:
    """Shape source of the model (reference model.py:50-93)."""

    d_model: int
    n_layer: int
    vocab_size: int
    d_state: int = 16
    d_conv: int = 4
    expand: int = 2
    dt_rank: int | None = None
    conv_bias: bool = True
    bias: bool = False
    pad_vocab_size_multiple: int = 8
    layer_norm_epsilon: float = 1e-5

    @property
    def d_inner(self) -> int:
        return self.expand * self.d_model

    def __post_init__(self):
        if self.dt_rank is None:
            self.dt_rank = max(1, self.d_model // 16)
        rem = self.vocab_size % self.pad_vocab_size_multiple
        if rem:
            self.vocab_size += self.pad_vocab_size_multiple - rem

    @classmethod
    def from_hf_config(cls, config_path: str) -> "MambaConfig":
        with open(config_path) as f:
            c = json.load(f)
        return cls(d_model=c["hidden_size"], n_layer=c["num_hidden_layers"], vocab_size=c["vocab_size"],
                   d_state=c["state_size"], d_conv=c["conv_kernel"], expand=c["expand"],
                   dt_rank=c["time_step_rank"], conv_bias=c["use_conv_bias"], bias=c["use_bias"],
                   pad_vocab_size_multiple=c.get("pad_vocab_size_multiple", 8),
                   layer_norm_epsilon=c.get("layer_norm_epsilon", 1e-5))


@dataclass
class LayerCache:
    """Per-layer recurrent state (reference model.py:96-101)."""

    conv_state: torch.Tensor  # [batch, d_inner, d_conv - 1]
    ssm_state: torch.Tensor   # [batch, d_inner, d_state], float32


def _state_dtype(dtype):
    return torch.float32 if dtype in (torch.bfloat16, torch.float16) else dtype


class MambaCache:
    """List of LayerCache (reference model.py:104-121).  step() mutates the
    tensors in place, so their addresses stay fixed for graph replay."""

    def __init__(self, layers: list[LayerCache]):
        self.layers = layers

    @staticmethod
    def allocate(config: MambaConfig, batch_size: int, device, dtype) -> "MambaCache":
        return MambaCache([
            LayerCache(
                conv_state=torch.zeros(batch_size, config.d_inner, config.d_conv - 1, device=device, dtype=dtype),
                ssm_state=torch.zeros(batch_size, config.d_inner, config.d_state, device=device,
                                      dtype=_state_dtype(dtype)),
            )
            for _ in range(config.n_layer)
        ])


# Prefill runs in_proj as two GEMMs (x / z halves) and copies B and C out of
# x_dbl once a call holds this many tokens: the scan then reads contiguous z
# rows and contiguous [b, l, N] B and C instead of strided slices.  Below it
# the extra launches cost more than the scan gains, so the fused projection
# is kept and the scan reads the slices through their strides.
SPLIT_PROJ_MIN_TOKENS = 16384


# Batched step projections run on mtl_linear_skinny (fp32, <= 32 tokens);
# out_proj as this many split-K parts.
SKINNY_OUT_SPLIT = 4

# A prefill of at most 64 tokens (b l rows of the projections, fp32) runs
# in_proj, x_proj and out_proj on mtl_linear_skinny as well: in_proj whole,
# x_proj (few weight rows) split over K into up to 16 parts that
# mtl_sum_parts adds, and, inside MambaLM.prefill, out_proj as
# SKINNY_OUT_SPLIT parts that the residual add sums.  The tied lm_head stays
# on the library GEMM (faster at 64 x 50280 x 768: 66 against 69 us).
# Prefills of more tokens keep torch's GEMMs on torch's own backend choice:
# the library never changes that process-wide setting.
_SKINNY_PREFILL = True

# A prompt of at most 64 tokens on an fp32 model runs its whole layer stack
# as one C call (mtl_prefill_short) launching the same kernels, in the same
# order, as the per-op path above: the bits are the same, and the ~100 us of
# Python per layer that bounds an eager short prefill goes away.
SHORT_PREFILL_NATIVE = True

# Longer prompts on an fp32 model run as one C call too (mtl_prefill_long),
# with the projections as hipBLASLt GEMMs launched from C++, up to
# LONG_PREFILL_MAX_ELEMS token-channels (b l d_inner): below it an eager
# per-op prefill is bound by its ~160 us of Python per layer.  Measured per
# prompt, one call against the per-op path: mamba-130m width 65 tokens 1.62
# against 3.94 ms, 256 tokens 1.70 against 3.91 ms, 1024 tokens 3.55 against
# 3.92 ms; mamba-1.4b width 128 tokens 4.82 against 8.10 ms, 512 tokens 12.87
# against 12.85 ms.  Past it the GPU time dominates and the per-op path keeps
# torch's GEMMs (and any tuned GEMM table: 1.4b 1024 tokens 23.4 against 23.9
# ms with it).  The C call's GEMM picks differ from torch's, so its logits
# differ from the per-op path's by float rounding.
LONG_PREFILL_NATIVE = True
LONG_PREFILL_MAX_ELEMS = 1 << 21
# Up to LONG_PREFILL_SKINNY_ROWS token rows, at widths up to
# LONG_PREFILL_SKINNY_MAX_D_MODEL, the one-call long prefill runs its
# projections on the library's skinny GEMM (64-row chunks) instead of
# hipBLASLt.  Eager prompts, skinny against hipBLASLt, one run: mamba-130m
# width 65 tokens 1199 against 1452 us, 128 tokens 1278 against 1498, 192
# tokens 1566 against 1727, 256 tokens 1700 against 1679, 512 tokens 2738
# against 2369; mamba-1.4b width 65 tokens 5978 against 4387 us, slower at
# every length (each further 64-row chunk streams the 67 MB in_proj weight
# again).
LONG_PREFILL_SKINNY_ROWS = 192
LONG_PREFILL_SKINNY_MAX_D_MODEL = 1024

# The fused decode step (fp32, batch 1 and 2) runs its whole layer stack as
# one C call (mtl_decode_step) launching the same kernels with the same
# arguments as the per-layer Python loop: the same bits, without the Python
# per launch that bounds an eager step.
DECODE_STEP_NATIVE = True

# The batched step (fp32, the rows the fused step does not take, up to 32)
# runs its layer stack as one C call too (mtl_decode_step_batched) when
# every layer takes the per-op path's in_proj + conv + x_proj launch and
# split out_proj: the same launches with the same tile choices, so the same
# bits, without the ~5 Python-launched ops per layer.
BATCHED_STEP_NATIVE = True

# With DECODE_PERSIST, the batch-1 fused decode of a model that fits its
# register blocking (d_model <= 1024, d_inner <= 2 d_model, dt_rank <= 64,
# d_conv <= 4, <= 64 layers) runs as one persistent launch,
# mtl_decode_step_persist, instead of three kernels per layer.  It is off:
# at the 130m shape, graph replays, it measured 449 us/token against 317-321
# us for the three-kernel layers (its three exchanges per layer cost 2-2.5
# us each on this part, and its 64 workgroups stream the weights at ~56 GB/s
# per CU).  PERSIST_BLOCKING 0 lets the library pick its grid.
DECODE_PERSIST = False
PERSIST_BLOCKING = 0


def _persist_grid(cfg: MambaConfig) -> int:
    """Workgroups mtl_decode_step_persist would launch for this shape, or 0
    when it does not take it (asked of the library: a register blocking must
    fit it)."""
    return int(_lib.load().mtl_decode_persist_grid(cfg.d_model, cfg.d_inner, cfg.d_state, cfg.dt_rank, cfg.d_conv,
                                                   cfg.n_layer, PERSIST_BLOCKING))


def _cu_count(device) -> int:
    return torch.cuda.get_device_properties(device).multi_processor_count


def _skinny_rows(x: torch.Tensor, w: torch.Tensor, enabled: bool = True, bias=None) -> torch.Tensor | None:
    """x [..., K] as the [rows, K] operand of mtl_linear_skinny (with this
    bias), or None where it does not apply."""
    if not (enabled and _SKINNY_PREFILL) or not x.is_contiguous():
        return None
    x2 = x.reshape(-1, x.shape[-1])
    return x2 if ops.linear_skinny_ok(x2, w, bias=bias) else None


def _skinny_split(K: int, most: int = 16) -> int:
    """The largest split of K into ranges of whole 128-column granules, at
    most `most` parts."""
    g = K // 128
    return max(p for p in range(1, min(g, most) + 1) if g % p == 0)

# column parts of the fused step's stand-alone x_proj GEMV
_XPROJ_PARTS = 4

# Largest batch that takes the fused decode step (its kernels take 1, 2 or
# 4 rows).  At 4 rows the per-op step on the matrix-core skinny GEMMs is as
# fast or faster (graph replays, A/B in one run: 130m 542 -> 501 us/step,
# 1.4b 2406 against 2414); at 2 rows the fused step is well ahead (130m 407
# against 475, 1.4b 1730 against 2343).
FUSED_STEP_MAX_BATCH = 2

# A batched fp32 step past FUSED_STEP_MAX_BATCH of at most
# STEP_NORM_FOLD_MAX_ROWS rows adds each block's residual in its out_proj
# launch, which also leaves the next block's norm inputs
# (mtl_linear_skinny_residual); the next in_proj applies that norm to its dot
# products (mtl_in_proj_conv_xproj_normed).  No add + norm launch runs
# between two blocks.  The last workgroup of each out_proj tile waits on
# three dependent memory round trips (its partial's stores, the count, the
# other partials' loads): with two or more workgroups per CU (up to 16 rows)
# other tiles' products hide them, at 32 rows (one per CU) they cost what the
# launch saves.  Graph replays, fold off -> on: mamba-1.4b width 8 rows 1945
# -> 1885 us, 16 rows 2027 -> 1995 us, 32 rows 2302-2307 -> 2312-2341 us;
# mamba-130m width 8 rows 550 -> 540 us, 32 rows 618 -> 621-629 us.  Eager steps gain 5-8%
# at every size (the add + norm launch's host time).  The same rule holds
# for eager and captured steps, so a graph replays the eager bits.
STEP_NORM_FOLD = True
STEP_NORM_FOLD_MAX_ROWS = 16


def _f32(t: torch.Tensor | None) -> torch.Tensor | None:
    if t is None:
        return None
    return t if t.dtype == torch.float32 and t.is_contiguous() else t.float().contiguous()


class RMSNorm(nn.Module):
    """w * x * rsqrt(mean(x^2) + eps) in float32 (reference model.py:124-135),
    one fused kernel per call."""

    def __init__(self, d_model: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d_model))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dtype = x.dtype
        out = ops.add_rmsnorm(x.float().contiguous(), _f32(self.weight), self.eps)
        return out.to(dtype)


class MambaMixer(nn.Module):
    """One Mamba mixer (reference model.py:138-294):
    in_proj -> causal conv1d + SiLU -> x_proj -> dt_proj -> selective scan
    (+ D skip, * SiLU(z)) -> out_proj."""

    def __init__(self, cfg: MambaConfig, layer_idx: int):
        super().__init__()
        self.cfg = cfg
        self.layer_idx = layer_idx
        d_inner, d_model, d_state, dt_rank, d_conv = cfg.d_inner, cfg.d_model, cfg.d_state, cfg.dt_rank, cfg.d_conv
        self.in_proj = nn.Linear(d_model, 2 * d_inner, bias=cfg.bias)
        self.conv1d = nn.Conv1d(d_inner, d_inner, kernel_size=d_conv, groups=d_inner, padding=d_conv - 1,
                                bias=cfg.conv_bias)
        self.x_proj = nn.Linear(d_inner, dt_rank + 2 * d_state, bias=False)
        self.dt_proj = nn.Linear(dt_rank, d_inner, bias=True)
        self.A_log = nn.Parameter(torch.empty(d_inner, d_state))
        self.D = nn.Parameter(torch.empty(d_inner))
        self.out_proj = nn.Linear(d_inner, d_model, bias=cfg.bias)
        self._reset_ssm_params()

    def _reset_ssm_params(self):
        """S4D-real init A_log = log(1..N) per channel, D = 1 (reference
        model.py:172-181)."""
        with torch.no_grad():
            n = self.A_log.shape[1]
            self.A_log.copy_(torch.log(torch.arange(1, n + 1, dtype=torch.float32)).expand_as(self.A_log))
            self.D.fill_(1.0)

    # small per-channel parameters are consumed in float32 by the kernels
    def _conv_w(self):
        w = self.conv1d.weight
        return _f32(w.reshape(w.shape[0], w.shape[-1]))

    def _step_conv(self):
        """(weight [D, K], bias) of the single-token conv.  With d_conv == 1 the
        reference's step uses x as is, with neither the 1-tap weight nor the
        conv bias (model.py:265-276), while its prefill applies both
        (206-208): the step then runs the kernel with a unit weight and no
        bias, which returns x exactly."""
        if self.cfg.d_conv > 1:
            return self._conv_w(), _f32(self.conv1d.bias)
        w = self.conv1d.weight
        ones = getattr(self, "_unit_conv_w", None)
        if ones is None or ones.device != w.device or ones.shape[0] != w.shape[0]:
            ones = torch.ones(w.shape[0], 1, device=w.device, dtype=torch.float32)
            self._unit_conv_w = ones
        return ones, None

    def prefill(self, x: torch.Tensor, cache: LayerCache | None = None, out: LayerCache | None = None):
        """x: [b, l, d_model] -> (out [b, l, d_model], conv_state [b, D, K-1],
        ssm_state [b, D, N]) -- reference model.py:184-241.  The cache is read
        as the initial state and never written; new state tensors are returned,
        or, with `out` (a preallocated LayerCache, which may be `cache` itself),
        the final states are written into out's tensors and those are returned."""
        return self._prefill(x, cache, out, parts_ok=False)

    def _prefill(self, x: torch.Tensor, cache: LayerCache | None, out: LayerCache | None, parts_ok: bool,
                 skinny: bool = True):
        """prefill(); with parts_ok, out_proj of a short prefill may come back
        as _Parts (split-K partial products for the residual add to sum);
        skinny=False keeps every projection on torch's GEMMs."""
        b, l, _ = x.shape
        Dm, N, R, K = self.cfg.d_inner, self.cfg.d_state, self.cfg.dt_rank, self.cfg.d_conv
        if out is not None:
            if tuple(out.conv_state.shape) != (b, Dm, K - 1) or out.conv_state.dtype != x.dtype or \
                    not out.conv_state.is_contiguous():
                raise ValueError(f"out.conv_state must be contiguous {(b, Dm, K - 1)} {x.dtype}")
            if tuple(out.ssm_state.shape) != (b, Dm, N) or out.ssm_state.dtype != torch.float32 or \
                    not out.ssm_state.is_contiguous():
                raise ValueError(f"out.ssm_state must be contiguous float32 {(b, Dm, N)}")
        split = b * l >= SPLIT_PROJ_MIN_TOKENS
        x2 = None if split else _skinny_rows(x, self.in_proj.weight, skinny, self.in_proj.bias)
        # in_proj with the causal conv as its epilogue (<= 64 tokens)
        fused_conv = x2 is not None and ops.in_proj_conv_prefill_ok(x2, self.in_proj.weight, K)
        if fused_conv:
            xs = z = None
        elif split:
            # in_proj as two GEMMs (x rows, z rows) so the conv and the scan read
            # whole contiguous [b, l, D] rows rather than halves of [b, l, 2D] rows
            w_in, b_in = self.in_proj.weight, self.in_proj.bias
            xs = F.linear(x, w_in[:Dm], b_in[:Dm] if b_in is not None else None).transpose(1, 2)   # [b, D, l]
            z = F.linear(x, w_in[Dm:], b_in[Dm:] if b_in is not None else None).transpose(1, 2)
        else:
            xz = (ops.linear_skinny(x2, self.in_proj.weight, self.in_proj.bias).view(b, l, 2 * Dm) if x2 is not None
                  else self.in_proj(x))                          # [b, l, 2D]
            xs = xz[..., :Dm].transpose(1, 2)                    # [b, D, l] view, D-stride 1
            z = xz[..., Dm:].transpose(1, 2)
        conv_in_state = cache.conv_state if cache is not None else None
        if conv_in_state is not None and conv_in_state.dtype != x.dtype:
            conv_in_state = conv_in_state.to(x.dtype)
        if conv_in_state is not None:
            conv_in_state = conv_in_state.contiguous()
            if out is not None and conv_in_state.data_ptr() == out.conv_state.data_ptr():
                conv_in_state = conv_in_state.clone()            # the conv reads and writes different runs
        if fused_conv:
            conv_state = (out.conv_state if out is not None
                          else torch.empty(b, Dm, K - 1, device=x.device, dtype=torch.float32))
            u_flat, z_flat = ops.in_proj_conv_prefill(x2, self.in_proj.weight, self.in_proj.bias, self._conv_w(),
                                                      _f32(self.conv1d.bias), conv_in_state, conv_state, b, l)
            u_store = u_flat.view(b, l, Dm)
            u = u_store.transpose(1, 2)                          # [b, D, l] views
            z = z_flat.view(b, l, Dm).transpose(1, 2)
        else:
            u_store = torch.empty(b, l, Dm, device=x.device, dtype=x.dtype)
            u, conv_state = ops.causal_conv1d(xs, self._conv_w(), _f32(self.conv1d.bias), conv_state=conv_in_state,
                                              silu=True, out=u_store.transpose(1, 2),
                                              final_state=out.conv_state if out is not None else None)
        w_x = self.x_proj.weight
        u2 = _skinny_rows(u_store, w_x, skinny)
        dt = None
        if u2 is not None:
            # x_proj split over K; its parts summed and dt_proj applied to the
            # sum in one launch (dt_proj's K = dt_rank is not the skinny GEMM's)
            ks = _skinny_split(Dm)
            parts = ops.linear_skinny(u2, w_x, ksplit=ks).view(ks, b * l, -1)
            if R <= ops.XPROJ_SUM_DT_MAX_R:
                x_dbl, dt = ops.xproj_sum_dt(parts, self.dt_proj.weight, write_x_dbl=ks > 1)
                dt = dt.view(b, l, Dm)
            else:
                x_dbl = ops.sum_parts(parts) if ks > 1 else parts[0]
            x_dbl = x_dbl.view(b, l, -1)
        else:
            x_dbl = F.linear(u_store, w_x)                        # [b, l, R+2N]
        dt_low = x_dbl[..., :R]
        if split:
            # B and C copied out of x_dbl into contiguous [b, l, N] (2 * b*l*N
            # elements, against re-reading u for two more GEMMs): a scan
            # tile's 16 steps of one of them are then one 16N-element run
            B = x_dbl[..., R:R + N].contiguous().transpose(1, 2)  # [b, N, l] view, N-stride 1
            C = x_dbl[..., R + N:].contiguous().transpose(1, 2)
        else:
            B = x_dbl[..., R:R + N].transpose(1, 2)               # [b, N, l] view, row stride R+2N
            C = x_dbl[..., R + N:].transpose(1, 2)
        if dt is None:
            dt = F.linear(dt_low, self.dt_proj.weight)            # [b, l, D]; bias fused in the scan
        h0 = None
        if cache is not None:
            h0 = cache.ssm_state.float().contiguous()
        y_store = torch.empty(b, l, Dm, device=x.device, dtype=x.dtype)
        # h_out may be h0: each state is read and written by the same thread
        _, h = ops.selective_scan(u, dt.transpose(1, 2), _f32(self.A_log), B, C, D=_f32(self.D), z=z,
                                  delta_bias=_f32(self.dt_proj.bias), h0=h0, delta_softplus=True, a_is_log=True,
                                  y=y_store.transpose(1, 2), h_out=out.ssm_state if out is not None else None)
        h = h if out is not None else h.to(_state_dtype(x.dtype))
        if parts_ok:
            w_out = self.out_proj.weight
            y2 = _skinny_rows(y_store, w_out, skinny, self.out_proj.bias)
            if y2 is not None and Dm % (128 * SKINNY_OUT_SPLIT) == 0:
                parts = ops.linear_skinny(y2, w_out, self.out_proj.bias, ksplit=SKINNY_OUT_SPLIT)
                return _Parts(parts.view(SKINNY_OUT_SPLIT, b, l, -1)), conv_state, h
        return self.out_proj(y_store), conv_state, h

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """No-cache forward (reference model.py:243-246)."""
        out, _, _ = self.prefill(x, cache=None)
        return out

    def step(self, x_t: torch.Tensor, cache: LayerCache):
        """x_t: [b, d_model] -> out [b, d_model]; updates cache.conv_state and
        cache.ssm_state in place (reference model.py:249-294).  No host sync,
        no allocation outside torch's caching allocator: graph-capturable."""
        return self.out_proj(self._step_y(x_t, cache))

    def _in_proj_step(self, x_t: torch.Tensor) -> torch.Tensor:
        """in_proj of a batched step: the matrix-core skinny GEMM where its
        operand rules hold, else nn.Linear.  Measured at 32 tokens with the
        weight cold in HBM, against the library's GEMM: the mamba-130m width
        9.8 -> 6.0 us, 1.4b 17.8-18.7 -> 15.6-15.8 us."""
        w = self.in_proj.weight
        if ops.linear_skinny_ok(x_t, w, bias=self.in_proj.bias):
            return ops.linear_skinny(x_t, w, self.in_proj.bias)
        return self.in_proj(x_t)

    def _out_proj_parts(self, y: torch.Tensor):
        """out_proj of a batched step as split-K partial products [P, b,
        d_model] (summed in order by the residual add that follows), or None
        where the skinny GEMM does not apply.  Measured at 32 tokens with the
        weight cold in HBM, against the library's GEMM: the mamba-1.4b
        out_proj 16.7 -> 10.0 us, 130m 7.9 -> 3.7 us."""
        w = self.out_proj.weight
        K = w.shape[1]
        if K % (128 * SKINNY_OUT_SPLIT) or not ops.linear_skinny_ok(y, w, bias=self.out_proj.bias):
            return None
        return ops.linear_skinny(y, w, self.out_proj.bias, ksplit=SKINNY_OUT_SPLIT)

    def _step_y(self, x_t: torch.Tensor, cache: LayerCache, sq: torch.Tensor | None = None,
                eps: float = 0.0) -> torch.Tensor:
        """The step up to the gated SSM output y [b, d_inner] (before out_proj).
        With sq, x_t is h * norm weight and sq the per-tile sums of h^2 that
        ops.linear_skinny_residual left: the in_proj input is RMSNorm(h)."""
        ops.check_step_shape(self.cfg.d_state, self.cfg.dt_rank)   # before the conv history moves
        Dm, R = self.cfg.d_inner, self.cfg.dt_rank
        b = x_t.shape[0]
        J = R + 2 * self.cfg.d_state
        conv_w, conv_b = self._step_conv()
        w_in = self.in_proj.weight
        if ops.in_proj_conv_xproj_ok(x_t, w_in, cache.conv_state, conv_w.shape[-1], J, self.in_proj.bias, conv_w,
                                     conv_b):
            # in_proj, the conv step and the x_proj partials of each channel
            # block in one launch (measured at the mamba-1.4b width, 32 tokens:
            # see in_proj_conv_xproj)
            xc, z, xpart = ops.in_proj_conv_xproj(x_t, w_in, self.in_proj.bias, cache.conv_state, conv_w, conv_b,
                                                  self._xproj_t(), sq=sq, eps=eps)
            return ops.selective_state_update(cache.ssm_state, xc, z, ops.sum_parts(xpart), _f32(self.dt_proj.weight),
                                              _f32(self.dt_proj.bias), _f32(self.A_log), _f32(self.D), a_is_log=True)
        if sq is not None:
            raise ValueError("step: a normed input needs the in_proj_conv_xproj path")
        xz = self._in_proj_step(x_t)                             # [b, 2D]
        if xz.dtype == torch.float32 and b <= 32 and J <= 288 and cache.conv_state.dtype == torch.float32:
            # conv step and the x_proj partials of 32-channel blocks in one kernel
            xc, xpart = ops.conv_step_xproj(cache.conv_state, xz[:, :Dm], conv_w, conv_b, self._xproj_t())
            x_dbl = ops.sum_parts(xpart)                         # [b, R+2N]
        else:
            xc = ops.conv_step(cache.conv_state, xz[:, :Dm], conv_w, conv_b, silu=True)
            x_dbl = self._x_proj_step(xc)                        # [b, R+2N]
        return ops.selective_state_update(cache.ssm_state, xc, xz[:, Dm:], x_dbl, _f32(self.dt_proj.weight),
                                          _f32(self.dt_proj.bias), _f32(self.A_log), _f32(self.D), a_is_log=True)


    # x_proj of a batched step: [b, D] x [D, R+2N] has too few output tiles
    # for one GEMM to fill the GPU, so it runs as D/128 GEMMs over channel
    # chunks (one batched call) whose outputs are added in chunk order
    _XPROJ_CHUNK = 128

    def _xproj_t(self) -> torch.Tensor:
        """x_proj weight transposed, contiguous [D, R+2N] (rebuilt when the
        weight changes: tracked by address and version)."""
        w = self.x_proj.weight
        key = (w.data_ptr(), w._version, w.dtype)
        cached = getattr(self, "_xproj_cache", None)
        if cached is None or cached[0] != key:
            with torch.no_grad():
                cached = (key, w.detach().t().contiguous())
            self._xproj_cache = cached
        return cached[1]

    def _xproj_chunks(self) -> torch.Tensor:
        wt = self._xproj_t()
        return wt.view(wt.shape[0] // self._XPROJ_CHUNK, self._XPROJ_CHUNK, wt.shape[1])

    def _x_proj_step(self, xc: torch.Tensor) -> torch.Tensor:
        b, D = xc.shape
        if b >= 8 and D >= 1024 and D % self._XPROJ_CHUNK == 0 and xc.dtype == torch.float32 and xc.is_cuda:
            wt = self._xproj_chunks()
            parts = torch.bmm(xc.view(b, wt.shape[0], self._XPROJ_CHUNK).transpose(0, 1), wt)   # [D/128, b, J]
            return ops.sum_parts(parts)
        return F.linear(xc, self.x_proj.weight)


# field order of MambaLM._layer_tensors()
(_LT_NORM, _LT_W_IN, _LT_B_IN, _LT_CONV_W, _LT_CONV_B, _LT_XPROJ, _LT_W_DT, _LT_B_DT, _LT_A_LOG, _LT_D, _LT_W_OUT,
 _LT_B_OUT) = range(12)


@dataclass
class _Parts:
    """A mixer output given as split-K partial products [P, b, d_model],
    added in order by the residual add that consumes it."""
    parts: torch.Tensor


class MambaBlock(nn.Module):
    """RMSNorm -> mixer -> residual (reference model.py:297-311)."""

    def __init__(self, cfg: MambaConfig, layer_idx: int):
        super().__init__()
        self.norm = RMSNorm(cfg.d_model, eps=cfg.layer_norm_epsilon)
        self.mixer = MambaMixer(cfg, layer_idx)

    def prefill(self, x, cache: LayerCache | None, out: LayerCache | None = None):
        y, conv_state, ssm_state = self.mixer.prefill(self.norm(x), cache, out)
        return x + y, conv_state, ssm_state

    def step(self, x_t, cache: LayerCache):
        return x_t + self.mixer.step(self.norm(x_t), cache)


class MambaLM(nn.Module):
    """Embedding -> n_layer MambaBlocks -> RMSNorm -> lm_head tied to the
    embedding (reference model.py:314-365).  Between blocks the residual add
    and the next block's RMSNorm run as one fused kernel."""

    def __init__(self, cfg: MambaConfig):
        super().__init__()
        self.cfg = cfg
        self.embedding = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.layers = nn.ModuleList([MambaBlock(cfg, i) for i in range(cfg.n_layer)])
        self.norm_f = RMSNorm(cfg.d_model, eps=cfg.layer_norm_epsilon)

    def lm_head(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(x, self.embedding.weight)

    def _norm_weight(self, i: int) -> torch.Tensor:
        mod = self.layers[i].norm if i < len(self.layers) else self.norm_f
        return _f32(mod.weight)

    def _eps(self, i: int) -> float:
        return (self.layers[i].norm if i < len(self.layers) else self.norm_f).eps

    def _run(self, x: torch.Tensor, per_layer):
        """Residual stream in float32: h_{i+1} = h_i + mixer_i(norm_i(h_i)),
        with each add fused into the following norm."""
        act = x.dtype
        h = x.float().contiguous()
        normed = ops.add_rmsnorm(h, self._norm_weight(0), self._eps(0))
        for i in range(len(self.layers)):
            y = per_layer(i, normed.to(act) if act != torch.float32 else normed)
            if isinstance(y, _Parts):
                normed = ops.add_rmsnorm(h, self._norm_weight(i + 1), self._eps(i + 1), y_parts=y.parts, x_out=h)
            else:
                normed = ops.add_rmsnorm(h, self._norm_weight(i + 1), self._eps(i + 1), y=y.float().contiguous(),
                                         x_out=h)
        return normed.to(act) if act != torch.float32 else normed

    def prefill(self, input_ids: torch.Tensor, cache: MambaCache | None = None,
                out_cache: MambaCache | None = None):
        """input_ids [b, l] -> (logits [b, l, vocab], new MambaCache)
        (reference model.py:328-341).  With `out_cache` (e.g. the cache a
        GraphedStepper captured, or `cache` itself) the final states are
        written into its tensors in place and out_cache is returned, so a
        captured decode graph can serve the next prompt without re-capture."""
        if out_cache is not None and len(out_cache.layers) != len(self.layers):
            raise ValueError("out_cache has the wrong number of layers")
        native = self._prefill_native(input_ids, cache, out_cache)
        if native is not None:
            return native
        x = self.embedding(input_ids)
        new_layers: list[LayerCache] = []

        def layer(i, xn):
            lc = cache.layers[i] if cache is not None else None
            oc = out_cache.layers[i] if out_cache is not None else None
            y, cs, hs = self.layers[i].mixer._prefill(xn, lc, oc, parts_ok=True)
            new_layers.append(LayerCache(conv_state=cs, ssm_state=hs))
            return y

        xf = self._run(x, layer)
        return self.lm_head(xf), (out_cache if out_cache is not None else MambaCache(new_layers))

    # ---- short prompt as one C call ----
    def _short_prefill_plan(self):
        """ctypes array of mtl_prefill_layer holding every layer's weight
        pointers, or None when a weight is not a contiguous float32 GPU
        tensor.  Rebuilt whenever any weight tensor's address or a block
        norm's eps changes."""
        ws = [t for lt in self._layer_tensors() for t in lt]     # 12 per layer, in mtl_prefill_layer's order
        ws.append(self.norm_f.weight)
        key = tuple(0 if t is None else t.data_ptr() for t in ws) + self._norm_eps()
        plan = getattr(self, "_short_plan", None)
        if plan is not None and plan[0] == key:
            return plan[1]
        arr = None
        if all(t is None or (t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()) for t in ws):
            arr = (_lib.PrefillLayer * len(self.layers))()
            for i, L in enumerate(arr):
                (L.norm_w, L.W_in, L.b_in, L.conv_w, L.conv_b, L.W_x, L.W_dt, L.dt_bias, L.A_log, L.Dv, L.W_out,
                 L.b_out) = key[12 * i:12 * i + 12]
                L.eps = self.layers[i].norm.eps
        self._short_plan = (key, arr)
        return arr

    def _native_prefill_kind(self, b, l):
        """'short' (mtl_prefill_short), 'long' (mtl_prefill_long) or None for
        a prompt of b x l tokens of this model's shape."""
        cfg = self.cfg
        D, N, K = cfg.d_inner, cfg.d_state, cfg.d_conv
        if SHORT_PREFILL_NATIVE and _SKINNY_PREFILL and ops.prefill_short_ok(b * l, cfg.d_model, D, N, cfg.dt_rank, K):
            return "short"
        if LONG_PREFILL_NATIVE and b * l * D <= LONG_PREFILL_MAX_ELEMS and \
                ops.prefill_long_ok(b, l, cfg.d_model, D, N, cfg.dt_rank, K):
            return "long"
        return None

    def _prefill_native(self, input_ids, cache, out_cache):
        """prefill() through mtl_prefill_short or mtl_prefill_long, or None
        where neither applies (a size or layer shape they do not take, a
        dtype other than float32, caches that are not contiguous float32)."""
        cfg = self.cfg
        if input_ids.dim() != 2 or not input_ids.is_cuda:
            return None
        b, l = input_ids.shape
        D, N, K = cfg.d_inner, cfg.d_state, cfg.d_conv
        kind = self._native_prefill_kind(b, l)
        if kind is None or self.embedding.weight.dtype != torch.float32:
            return None
        for c in (cache, out_cache):
            if c is not None and not all(
                    tuple(lc.conv_state.shape) == (b, D, K - 1) and lc.conv_state.dtype == torch.float32 and
                    lc.conv_state.is_contiguous() and tuple(lc.ssm_state.shape) == (b, D, N) and
                    lc.ssm_state.dtype == torch.float32 and lc.ssm_state.is_contiguous() for lc in c.layers):
                return None
        tmpl = self._short_prefill_plan()
        if tmpl is None:
            return None
        # a copy per call: the library reads it while ctypes has released the
        # GIL, so another thread's prefill must not rewrite its cache pointers
        arr = type(tmpl).from_buffer_copy(tmpl)
        new_layers, held = [], []
        for i, L in enumerate(arr):
            lc = cache.layers[i] if cache is not None else None
            if out_cache is not None:
                conv_out, h_out = out_cache.layers[i].conv_state, out_cache.layers[i].ssm_state
            else:
                conv_out = torch.empty(b, D, K - 1, device=input_ids.device, dtype=torch.float32)
                h_out = torch.empty(b, D, N, device=input_ids.device, dtype=torch.float32)
                new_layers.append(LayerCache(conv_state=conv_out, ssm_state=h_out))
            conv_in = lc.conv_state if lc is not None else None
            if conv_in is not None and conv_in.data_ptr() == conv_out.data_ptr():
                conv_in = conv_in.clone()        # the conv reads and writes different runs
                held.append(conv_in)
            L.conv_state_in = conv_in.data_ptr() if conv_in is not None else None
            L.conv_state_out = conv_out.data_ptr()
            L.h0 = lc.ssm_state.data_ptr() if lc is not None else None   # h_out may be h0
            L.h_out = h_out.data_ptr()
        h = self.embedding(input_ids).contiguous()
        if kind == "short":
            normed = ops.prefill_short(h, arr, self.norm_f.weight, self.norm_f.eps, D, N, cfg.dt_rank, K)
        else:
            skinny = LONG_PREFILL_SKINNY_ROWS if cfg.d_model <= LONG_PREFILL_SKINNY_MAX_D_MODEL else 0
            normed = ops.prefill_long(h, arr, self.norm_f.weight, self.norm_f.eps, D, N, cfg.dt_rank, K,
                                      skinny_rows=skinny)
        return self.lm_head(normed), (out_cache if out_cache is not None else MambaCache(new_layers))

    def step(self, input_ids: torch.Tensor, cache: MambaCache):
        """input_ids [b, 1] -> logits [b, 1, vocab]; cache updated in place
        (reference model.py:343-353).  fp32 models at batch 1 and 2
        (FUSED_STEP_MAX_BATCH) take the fused decode path (3-4 launches per
        layer); others run the per-op path (the matrix-core skinny GEMMs or
        the library's, the conv-step and SSM-update kernels)."""
        lt = self._layer_tensors()
        if self._fused_step_ok(input_ids, cache, lt=lt):
            return self._step_fused(input_ids, cache, lt=lt)
        x = self.embedding(input_ids).squeeze(1)
        if BATCHED_STEP_NATIVE:
            got = self._batched_step_layers(x, cache, lt)
            if got is not None:
                arr, fold = got
                normed = ops.decode_step_batched(arr, x, self.norm_f.weight, self.norm_f.eps, self.cfg, fold)
                return self.lm_head(normed).unsqueeze(1)
        if self._fold_ok(x, cache):
            return self._step_folded(x, cache)

        def layer(i, xn):
            mx = self.layers[i].mixer
            y = mx._step_y(xn, cache.layers[i])
            parts = mx._out_proj_parts(y)
            return mx.out_proj(y) if parts is None else _Parts(parts)

        xf = self._run(x, layer)
        return self.lm_head(xf).unsqueeze(1)

    # ---- batched step with the residual add and norm folded into the projections ----
    def _fold_ok(self, x, cache) -> bool:
        """Whether the batched step takes _step_folded: STEP_NORM_FOLD, fp32
        on the GPU, at most STEP_NORM_FOLD_MAX_ROWS (and 32) rows, two or more
        layers, and every layer on the in_proj + conv + x_proj launch and the
        split out_proj."""
        cfg = self.cfg
        if not STEP_NORM_FOLD or len(self.layers) < 2 or x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda:
            return False
        b, dm = x.shape
        J = cfg.dt_rank + 2 * cfg.d_state
        if b > min(32, STEP_NORM_FOLD_MAX_ROWS) or cfg.d_conv < 2 or cfg.d_inner % (128 * SKINNY_OUT_SPLIT) or \
                len(cache.layers) != len(self.layers):
            return False
        rpb = ops.residual_rows_per_block(b, dm, SKINNY_OUT_SPLIT)
        if dm % rpb or dm // rpb > 128:
            return False
        nl = len(self.layers)
        for i, (blk, lc) in enumerate(zip(self.layers, cache.layers)):
            mx = blk.mixer
            w = mx.out_proj.weight
            conv_w, conv_b = mx._step_conv()
            if not ops.in_proj_conv_xproj_ok(x, mx.in_proj.weight, lc.conv_state, cfg.d_conv, J, mx.in_proj.bias,
                                             conv_w, conv_b):
                return False
            if w.dtype != torch.float32 or not w.is_contiguous() or tuple(w.shape) != (dm, cfg.d_inner) or \
                    w.device != x.device or not ops.aligned16(w, mx.out_proj.bias):
                return False
            if i + 1 < nl and not ops.aligned16(self._norm_weight(i + 1)):   # the next norm, read by out_proj
                return False
        return True

    def _step_folded(self, x, cache):
        """MambaLM.step for b <= 32 fp32 rows with no add + norm launch between
        blocks: layer 0's norm runs as mtl_add_rmsnorm; each out_proj but the
        last adds the residual in place and leaves x_next = h * w_next and the
        per-tile sums of h^2 (ops.linear_skinny_residual), from which the next
        in_proj takes RMSNorm(h); the last out_proj's parts go to the final
        add + norm as before.  The residual stream equals the per-op path's bit
        for bit; each norm differs from it by float rounding (applied to the
        dot products)."""
        b, dm = x.shape
        nl = len(self.layers)
        rpb = ops.residual_rows_per_block(b, dm, SKINNY_OUT_SPLIT)
        tiles = dm // rpb
        h = x.float().contiguous()
        inp = ops.add_rmsnorm(h, self._norm_weight(0), self._eps(0))
        xn = torch.empty_like(h)
        sq = torch.empty(tiles, b, device=h.device, dtype=torch.float32)
        counters = torch.zeros(nl - 1, tiles, device=h.device, dtype=torch.int32)
        parts = torch.empty(SKINNY_OUT_SPLIT, b, dm, device=h.device, dtype=torch.float32)
        s = None
        for i, blk in enumerate(self.layers):
            mx = blk.mixer
            y = mx._step_y(inp, cache.layers[i], sq=s, eps=self._eps(i))
            if i + 1 < nl:
                ops.linear_skinny_residual(y, mx.out_proj.weight, mx.out_proj.bias, h, self._norm_weight(i + 1), xn,
                                           sq, counters[i], SKINNY_OUT_SPLIT, rpb, parts)
                inp, s = xn, sq
            else:
                p = ops.linear_skinny(y, mx.out_proj.weight, mx.out_proj.bias, ksplit=SKINNY_OUT_SPLIT)
                inp = ops.add_rmsnorm(h, self._norm_weight(nl), self._eps(nl), y_parts=p, x_out=h)
        return self.lm_head(inp).unsqueeze(1)

    def _batched_step_layers(self, x, cache, lt=None):
        """(ctypes array of mtl_decode_layer for mtl_decode_step_batched with
        this call's cache pointers, whether the residual add + norm fold),
        or None when some layer would not take the per-op path's in_proj +
        conv + x_proj launch and split out_proj, or a weight or cache tensor
        is not a contiguous float32 tensor of its shape on x's device (the
        step then runs op by op, with that path's checks and errors).  The
        weights are checked when their addresses (or x_proj's version, which
        its transposed copy follows) change; the cache tensors every call.
        The fold follows _fold_ok's rule, which on these layers reduces to
        the row count and the out_proj tile."""
        cfg = self.cfg
        nl = len(self.layers)
        if x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous() or \
                x.data_ptr() % 16 or len(cache.layers) != nl:
            return None
        b, dm = x.shape
        D, N, K, R = cfg.d_inner, cfg.d_state, cfg.d_conv, cfg.dt_rank
        if not (1 <= b <= ops.IN_CONV_MAX_ROWS and dm >= 256 and dm % 128 == 0 and D % (128 * SKINNY_OUT_SPLIT) == 0
                and N <= 16 and R <= 256 and 2 <= K <= 4 and R + 2 * N <= 288):
            return None
        dev = x.device
        lt = self._layer_tensors() if lt is None else lt
        sig = (dev, dm, tuple(0 if t is None else t.data_ptr() for ts in lt for t in ts),
               tuple(ts[_LT_XPROJ]._version for ts in lt), self._norm_eps())
        cached = getattr(self, "_batched_tmpl", None)
        if cached is None or cached[0] != sig:
            cached = (sig, self._batched_template(lt, dev, dm))
            self._batched_tmpl = cached
        tmpl = cached[1]
        if tmpl is None:
            return None
        cs_shape, hs_shape = (b, D, K - 1), (b, D, N)
        for lc in cache.layers:
            cs, hs = lc.conv_state, lc.ssm_state
            if cs.dtype != torch.float32 or hs.dtype != torch.float32 or cs.shape != cs_shape or \
                    hs.shape != hs_shape or not cs.is_contiguous() or not hs.is_contiguous() or cs.device != dev or \
                    hs.device != dev or cs.data_ptr() % 16:
                return None
        arr = type(tmpl).from_buffer_copy(tmpl)   # per call: read by the library without the GIL
        for L, lc in zip(arr, cache.layers):
            L.conv_state, L.ssm_state = lc.conv_state.data_ptr(), lc.ssm_state.data_ptr()
        rpb = ops.residual_rows_per_block(b, dm, SKINNY_OUT_SPLIT)
        fold = STEP_NORM_FOLD and nl >= 2 and b <= min(32, STEP_NORM_FOLD_MAX_ROWS) and dm % rpb == 0 and \
            dm // rpb <= 128
        return arr, fold

    def _batched_template(self, lt, dev, dm):
        """The weight half of _batched_step_layers: mtl_decode_layer records
        (W_xT = x_proj transposed, conv weights as [D, K] views), or None when
        a weight is not a contiguous float32 tensor of its shape on dev or one
        the library loads in 16-byte runs (norm, in_proj, conv, out_proj and
        their biases) is not 16-byte aligned."""
        cfg = self.cfg
        D, N, K, R = cfg.d_inner, cfg.d_state, cfg.d_conv, cfg.dt_rank
        ok = lambda t, shape: t.device == dev and t.dtype == torch.float32 and t.is_contiguous() and \
            tuple(t.shape) == shape
        opt = lambda t, shape: t is None or ok(t, shape)
        tmpl = (_lib.DecodeLayer * len(lt))()
        for i, (ts, L) in enumerate(zip(lt, tmpl)):
            if not (ok(ts[_LT_NORM], (dm,)) and ok(ts[_LT_W_IN], (2 * D, dm)) and opt(ts[_LT_B_IN], (2 * D,))
                    and ok(ts[_LT_CONV_W], (D, 1, K)) and opt(ts[_LT_CONV_B], (D,))
                    and ok(ts[_LT_XPROJ], (R + 2 * N, D)) and ok(ts[_LT_W_DT], (D, R)) and ok(ts[_LT_B_DT], (D,))
                    and ok(ts[_LT_A_LOG], (D, N)) and opt(ts[_LT_D], (D,)) and ok(ts[_LT_W_OUT], (dm, D))
                    and opt(ts[_LT_B_OUT], (dm,))):
                return None
            if not ops.aligned16(ts[_LT_NORM], ts[_LT_W_IN], ts[_LT_B_IN], ts[_LT_CONV_W], ts[_LT_CONV_B],
                                 ts[_LT_W_OUT], ts[_LT_B_OUT]):
                return None
            w_xt = self.layers[i].mixer._xproj_t()
            ptr = lambda t: 0 if t is None else t.data_ptr()
            (L.norm_w, L.W_in, L.b_in, L.conv_w, L.conv_b, L.W_xT, L.W_dt, L.dt_bias, L.A_log, L.Dv, L.W_out,
             L.b_out) = (ptr(ts[_LT_NORM]), ptr(ts[_LT_W_IN]), ptr(ts[_LT_B_IN]), ptr(ts[_LT_CONV_W]),
                         ptr(ts[_LT_CONV_B]), w_xt.data_ptr(), ptr(ts[_LT_W_DT]), ptr(ts[_LT_B_DT]),
                         ptr(ts[_LT_A_LOG]), ptr(ts[_LT_D]), ptr(ts[_LT_W_OUT]), ptr(ts[_LT_B_OUT]))
            L.eps = self.layers[i].norm.eps
        return tmpl

    # ---- fused decode step ----
    def _fused_step_ok(self, input_ids, cache, lt=None) -> bool:
        cfg = self.cfg
        b = input_ids.shape[0]
        if b not in (1, 2, 4) or b > FUSED_STEP_MAX_BATCH or cfg.d_state > 16 or cfg.d_model % 4 or \
                cfg.d_inner % 4 or b * cfg.d_model > 15 * 1024 or cfg.d_inner > 4096 or cfg.dt_rank > 256 or \
                not 2 <= cfg.d_conv <= 8:
            return False
        if self.embedding.weight.dtype != torch.float32 or not input_ids.is_cuda or \
                not ops.aligned16(self.embedding.weight):
            return False
        lc = cache.layers[0]
        if not (lc.conv_state.dtype == torch.float32 and lc.ssm_state.dtype == torch.float32 and
                lc.conv_state.is_contiguous() and lc.ssm_state.is_contiguous()):
            return False
        if DECODE_STEP_NATIVE:
            plan = self._decode_plan(lt)
            split_k = b <= plan["split_k_max_b"]
            tmpl = self._decode_step_template(plan, split_k, input_ids.device, lt)
            if tmpl is None:
                return False
            # the step that follows in the same call reuses them (keyed on this
            # call's parameter list, so no other call can pick them up)
            self._fused_memo = (lt, plan, tmpl) if lt is not None else None
        return True

    def _check_step_cache(self, cache, b: int, device):
        """Every layer's conv_state [b, D, K-1] and ssm_state [b, D, N] must be
        contiguous float32 on the ids' device before the one-call step hands
        their addresses to the kernels (the reference fails in torch.cat on a
        mismatched cache, model.py:264-266)."""
        cfg = self.cfg
        if len(cache.layers) != len(self.layers):
            raise ValueError(f"step: cache has {len(cache.layers)} layers, the model {len(self.layers)}")
        cs_shape = (b, cfg.d_inner, cfg.d_conv - 1)
        h_shape = (b, cfg.d_inner, cfg.d_state)
        for i, lc in enumerate(cache.layers):
            cs, hs = lc.conv_state, lc.ssm_state
            if cs.shape != cs_shape or cs.dtype != torch.float32 or not cs.is_contiguous() or cs.device != device:
                raise ValueError(f"step: layer {i} conv_state must be contiguous float32 {cs_shape} on {device}, "
                                 f"got {tuple(cs.shape)} {cs.dtype} on {cs.device}")
            if hs.shape != h_shape or hs.dtype != torch.float32 or not hs.is_contiguous() or hs.device != device:
                raise ValueError(f"step: layer {i} ssm_state must be contiguous float32 {h_shape} on {device}, "
                                 f"got {tuple(hs.shape)} {hs.dtype} on {hs.device}")

    def _layer_tensors(self):
        """Per layer, the parameters a one-call decode step reads, in the
        order _LT_* names: looked up through the modules' own dicts, not
        nn.Module attribute access (an eager step reads ~300 of them, and
        each attribute lookup through nn.Module costs ~0.2 us)."""
        out = []
        for blk in self.layers._modules.values():
            bm = blk._modules
            mx = bm["mixer"]
            sub, mp = mx._modules, mx._parameters
            ip, cv = sub["in_proj"]._parameters, sub["conv1d"]._parameters
            xp, dp, op = sub["x_proj"]._parameters, sub["dt_proj"]._parameters, sub["out_proj"]._parameters
            out.append((bm["norm"]._parameters["weight"], ip["weight"], ip.get("bias"), cv["weight"], cv.get("bias"),
                        xp["weight"], dp["weight"], dp.get("bias"), mp["A_log"], mp["D"], op["weight"],
                        op.get("bias")))
        return out

    def _norm_eps(self):
        """Every block norm's eps (the weight records carry them)."""
        return tuple(blk._modules["norm"].eps for blk in self.layers._modules.values())

    def _derived_key(self, lt=None):
        """(address, version) of the parameters that derived weight copies are
        built from: the fused decode plan and the per-op step's transposed
        x_proj.  A captured graph reads those copies, so it is stale once
        this key changes."""
        lt = self._layer_tensors() if lt is None else lt
        return tuple((t[_LT_XPROJ].data_ptr(), t[_LT_XPROJ]._version, t[_LT_CONV_W].data_ptr(),
                      t[_LT_CONV_W]._version) for t in lt)

    def _derived_tensors(self):
        """The derived copies a step reads now (held by a captured graph so a
        rebuild cannot free memory the graph still addresses)."""
        held = [getattr(self, "_plan", None), getattr(self, "_persist_tab", None),
                getattr(self, "_persist_ws", None)]
        for m in self.layers:
            held += [getattr(m.mixer, "_xproj_cache", None), getattr(m.mixer, "_unit_conv_w", None)]
        return held

    def _decode_plan(self, lt=None):
        """Per-layer tensors of the fused step: x_proj transposed [D, J] for the
        split-K partials, conv weights as [D, K].  Rebuilt whenever a source
        parameter changes (tracked by tensor version and address)."""
        key = self._derived_key(lt)
        plan = getattr(self, "_plan", None)
        if plan is not None and plan["key"] == key:
            return plan
        cfg = self.cfg
        J = cfg.dt_rank + 2 * cfg.d_state
        cpb = 8  # channels per decode_in workgroup when it also forms the x_proj partials
        nblk = (cfg.d_inner + cpb - 1) // cpb
        # every decode_ssm workgroup sums the x_proj partials with Q threads
        # per (j, batch) pair and one batch of <= 64 loads per thread; when
        # that does not cover nblk, x_proj runs as its own row GEMV instead
        def _fits(b):
            q = max(1, min(256 // (J * b), 8))
            return -(-nblk // q) <= 64
        split_k_max_b = max([b for b in (1, 2, 4) if _fits(b)], default=0)
        persist = _persist_grid(cfg)
        need_xt = split_k_max_b > 0 or persist > 0    # the persistent step reads x_proj transposed too
        layers = []
        with torch.no_grad():
            for m in self.layers:
                mx = m.mixer
                w = mx.conv1d.weight
                layers.append({
                    "W_xT": mx.x_proj.weight.detach().t().contiguous() if need_xt else None,
                    "conv_w": w.detach().reshape(w.shape[0], w.shape[-1]).contiguous(),
                })
        self._plan = {"key": key, "layers": layers, "cpb": cpb, "nblk": nblk, "J": J,
                      "split_k_max_b": split_k_max_b, "persist": persist}
        return self._plan

    def _persist_table(self, tmpl, device):
        """Device copy of the weight records in `tmpl` for the persistent step,
        rebuilt when the template changes; None when it would have to be
        uploaded inside a graph capture (that step then runs kernel by
        kernel)."""
        cached = getattr(self, "_persist_tab", None)
        if cached is not None and cached[0] is tmpl:
            return cached[1]
        if torch.cuda.is_current_stream_capturing():
            return None
        host = torch.frombuffer(bytearray(bytes(tmpl)), dtype=torch.uint8)
        dev_tab = host.to(device)
        self._persist_tab = (tmpl, dev_tab)
        return dev_tab

    def _persist_workspace(self, device):
        """The persistent step's workspace on `device` (exchange slots, epoch,
        error word), zero-filled once and kept."""
        ws = getattr(self, "_persist_ws", {})
        t = ws.get(device)
        if t is None:
            if torch.cuda.is_current_stream_capturing():
                return None
            t = ops.decode_persist_workspace(self.cfg, device)
            ws[device] = t
            self._persist_ws = ws
        return t

    def _decode_step_template(self, plan, split_k, device, lt=None):
        """ctypes array of mtl_decode_layer with every layer's weight pointers
        (x_proj transposed from the decode plan with split_k, as is without),
        or None when a weight is not a contiguous float32 tensor on `device`
        or in_proj, out_proj or (without split_k) x_proj is not 16-byte
        aligned (the step then runs op by op).  Rebuilt whenever any of those
        tensors' addresses change."""
        ws = []
        for t, lp in zip(self._layer_tensors() if lt is None else lt, plan["layers"]):
            ws += [t[_LT_NORM], t[_LT_W_IN], t[_LT_B_IN], lp["conv_w"], t[_LT_CONV_B],
                   lp["W_xT"] if split_k else None, None if split_k else t[_LT_XPROJ], t[_LT_W_DT], t[_LT_B_DT],
                   t[_LT_A_LOG], t[_LT_D], t[_LT_W_OUT], t[_LT_B_OUT]]
        key = tuple(0 if t is None else t.data_ptr() for t in ws) + self._norm_eps()
        cached = getattr(self, "_step_tmpl", {}).get(split_k)
        if cached is not None and cached[0] == key and cached[2] == device:
            return cached[1]
        arr = None
        if all(t is None or (t.device == device and t.dtype == torch.float32 and t.is_contiguous()) for t in ws) \
                and ops.aligned16(*ws[1::13], *ws[6::13], *ws[11::13]):   # W_in, W_x, W_out
            arr = (_lib.DecodeLayer * len(self.layers))()
            for i, L in enumerate(arr):
                (L.norm_w, L.W_in, L.b_in, L.conv_w, L.conv_b, L.W_xT, L.W_x, L.W_dt, L.dt_bias, L.A_log, L.Dv,
                 L.W_out, L.b_out) = key[13 * i:13 * i + 13]
                L.eps = self.layers[i].norm.eps
        if not hasattr(self, "_step_tmpl"):
            self._step_tmpl = {}
        self._step_tmpl[split_k] = (key, arr, device)
        return arr

    def _step_fused(self, input_ids, cache, lt=None):
        cfg = self.cfg
        memo = getattr(self, "_fused_memo", None)
        memo = memo if memo is not None and lt is not None and memo[0] is lt else None
        self._fused_memo = None
        plan = memo[1] if memo is not None else self._decode_plan(lt)
        b, M, D, J = input_ids.shape[0], cfg.d_model, cfg.d_inner, plan["J"]
        split_k = b <= plan["split_k_max_b"]
        dev = input_ids.device
        ids = input_ids.reshape(-1).contiguous()   # a column slice of a longer id tensor is strided
        f32 = dict(device=dev, dtype=torch.float32)
        xc = torch.empty(b, D, **f32)
        gz = torch.empty(b, D, **f32)
        y = torch.empty(b, D, **f32)
        xs = [torch.empty(b, M, **f32) for _ in range(3)]
        # without block partials, x_proj runs as its own row GEMV in column parts
        # (more workgroups on its 160 rows at the 1.4b width) that decode_ssm adds
        xp_parts = 1 if split_k else _XPROJ_PARTS if D % (4 * _XPROJ_PARTS) == 0 else 1
        xpart = torch.empty(plan["nblk"] if split_k else xp_parts, b, J, **f32)
        # decode_in at batch 1 without the partials: 4 channels per workgroup,
        # one in_proj row per wavefront, twice the workgroups on the weight
        # stream (measured at d_model 2048: 12.87 -> 12.63 us; at batch 2 and 4
        # the 8-channel blocks are faster)
        cpb = 4 if b == 1 and not split_k else plan["cpb"]
        # its workgroups must all be resident at once: a device with fewer CUs
        # than its grid (a partitioned GPU) runs the three-kernel step
        if DECODE_STEP_NATIVE and DECODE_PERSIST and b == 1 and 0 < plan["persist"] <= _cu_count(dev):
            self._check_step_cache(cache, b, dev)
            tmpl = self._decode_step_template(plan, True, dev, lt)
            tab = self._persist_table(tmpl, dev) if tmpl is not None else None
            wsp = self._persist_workspace(dev) if tab is not None else None
            if wsp is not None:
                arr = type(tmpl).from_buffer_copy(tmpl)
                for L, lc in zip(arr, cache.layers):
                    L.conv_state, L.ssm_state = lc.conv_state.data_ptr(), lc.ssm_state.data_ptr()
                logits = torch.empty(1, self.embedding.weight.shape[0], **f32)
                ops.decode_step_persist(arr, tab, ids, self.embedding.weight, _f32(self.norm_f.weight),
                                        self.norm_f.eps, logits, xs[0], wsp, cfg, PERSIST_BLOCKING)
                return logits.unsqueeze(1)
        if DECODE_STEP_NATIVE:
            self._check_step_cache(cache, b, dev)
            logits = torch.empty(b, self.embedding.weight.shape[0], **f32)
            tmpl = memo[2] if memo is not None else self._decode_step_template(plan, split_k, dev, lt)
            arr = type(tmpl).from_buffer_copy(tmpl)     # per call: read by the library without the GIL
            for L, lc in zip(arr, cache.layers):
                L.conv_state, L.ssm_state = lc.conv_state.data_ptr(), lc.ssm_state.data_ptr()
            ops.decode_step(arr, ids, self.embedding.weight, _f32(self.norm_f.weight), self.norm_f.eps, logits,
                            xc, gz, y, xs, xpart, cfg, cpb, split_k, xp_parts)
            return logits.unsqueeze(1)
        x_cur = None
        for i, blk in enumerate(self.layers):
            mx, lp, lc = blk.mixer, plan["layers"][i], cache.layers[i]
            resid = xs[2] if i == 0 else x_cur
            ops.decode_in(blk.norm.weight, blk.norm.eps, mx.in_proj.weight, lc.conv_state, lp["conv_w"], xc, gz,
                          x=x_cur, emb=self.embedding.weight if i == 0 else None, ids=ids if i == 0 else None,
                          resid_out=xs[2] if i == 0 else None, b_in=mx.in_proj.bias, conv_b=mx.conv1d.bias,
                          W_xT=lp["W_xT"] if split_k else None, xpart=xpart if split_k else None,
                          channels_per_block=cpb)
            if not split_k:
                ops.decode_gemv_parts(xc, mx.x_proj.weight, xpart)
            ops.decode_ssm(xpart, xc, gz, mx.dt_proj.weight, mx.dt_proj.bias, mx.A_log, mx.D, lc.ssm_state, y)
            x_next = xs[i % 2]
            ops.decode_gemv(y, mx.out_proj.weight, x_next, bias=mx.out_proj.bias, x_in=resid)
            x_cur = x_next
        # final norm_f + tied lm_head in one launch (reference model.py:351-352)
        logits = torch.empty(b, self.embedding.weight.shape[0], **f32)
        ops.decode_norm_gemv(x_cur, _f32(self.norm_f.weight), self.norm_f.eps, self.embedding.weight, logits)
        return logits.unsqueeze(1)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, greedy: bool = True):
        """Prefill once, then greedy decode through the cache (reference
        model.py:355-365).  Returns the full token sequence.  The reference
        has no sampling path: with greedy=False it sets the first token to
        None (model.py:359) and its first step fails; here that is a clear
        error before any work."""
        if not greedy:
            raise NotImplementedError("generate: only greedy decoding exists (the reference's greedy=False "
                                      "path has no sampler)")
        logits, cache = self.prefill(input_ids)
        next_id = logits[:, -1:].argmax(dim=-1)
        tokens = [input_ids, next_id]
        for _ in range(max_new_tokens - 1):
            logits = self.step(next_id, cache)
            next_id = logits[:, -1, :].argmax(dim=-1, keepdim=True)
            tokens.append(next_id)
        return torch.cat(tokens, dim=1)

    @classmethod
    def from_pretrained(cls, hf_path: str, dtype=torch.float32) -> "MambaLM":
        """Local HF `state-spaces/mamba-*-hf` snapshot -> MambaLM (reference
        model.py:367-397): `backbone.` prefix and `embeddings` renamed, strict
        load."""
        cfg = MambaConfig.from_hf_config(os.path.join(hf_path, "config.json"))
        model = cls(cfg).to(dtype)
        sd = load_hf_state_dict(hf_path)
        remapped = {"embedding.weight": sd["backbone.embeddings.weight"],
                    "norm_f.weight": sd["backbone.norm_f.weight"]}
        names = ["norm.weight", "mixer.in_proj.weight", "mixer.conv1d.weight", "mixer.x_proj.weight",
                 "mixer.dt_proj.weight", "mixer.dt_proj.bias", "mixer.A_log", "mixer.D", "mixer.out_proj.weight"]
        if cfg.conv_bias:
            names.append("mixer.conv1d.bias")
        if cfg.bias:
            names += ["mixer.in_proj.bias", "mixer.out_proj.bias"]
        for i in range(cfg.n_layer):
            for n in names:
                remapped[f"layers.{i}.{n}"] = sd[f"backbone.layers.{i}.{n}"]
        missing, unexpected = model.load_state_dict({k: v.to(dtype) for k, v in remapped.items()}, strict=True)
        assert not missing and not unexpected, (missing, unexpected)
        return model
