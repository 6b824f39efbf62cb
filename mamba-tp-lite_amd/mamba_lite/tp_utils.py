"""Payload quantizers of the tensor-parallel AllReduce, run as local ops, plus
the channel-shard helpers (mamba-tp-lite mamba_lite/tp_utils.py).

On one GPU there is no collective: the partial sums that ranks would
exchange are tensors in this GPU's memory, and the ops below do what the
reference does around its collective -- quantize each partial into its wire
payload, then dequantize and sum in rank order -- as one HIP kernel each.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops


class CommCounter:
    """Collective count and wire bytes (reference tp_utils.py:11-20)."""

    def __init__(self):
        self.count = 0
        self.bytes = 0

    def reset(self):
        self.count = 0
        self.bytes = 0


def int8_tok_payload_nbytes(rows: int, cols: int) -> int:
    """Wire bytes of one rank's per-token int8 payload: 4*rows scale bytes +
    rows*cols codes (reference tp_utils.py:113-117)."""
    return rows * (cols + 4)


def quant_dequant_sum_int8_tok(parts, counter: CommCounter | None = None, return_payloads: bool = False):
    """Local all_reduce_sum_int8_gather_tok (reference tp_utils.py:103-131,
    145-149) over `parts` (one fp32 tensor per rank, same shape).  Codes and
    per-token scales are bit-identical to the reference arithmetic."""
    out, payloads = ops.quant_dequant_sum_int8_tok([p.contiguous() for p in parts], return_payloads=True)
    if counter is not None:
        counter.count += 1
        counter.bytes += payloads[0].numel()
    return (out, payloads) if return_payloads else out


def quant_dequant_sum_fp16(parts, counter: CommCounter | None = None, return_payloads: bool = False):
    """Local all_reduce_sum_fp16 (reference tp_utils.py:31-42): fp16 cast,
    rank-ordered fp16 sum, back to fp32."""
    out, payloads = ops.quant_dequant_sum_fp16([p.contiguous() for p in parts], return_payloads=return_payloads)
    if counter is not None:
        counter.count += 1
        counter.bytes += parts[0].numel() * 2
    return (out, payloads) if return_payloads else out


def channel_slice(rank: int, world_size: int, total: int) -> slice:
    """Rank r's channel range of d_inner (reference tp_utils.py:163-166)."""
    assert total % world_size == 0, f"{total} not divisible by world_size={world_size}"
    shard = total // world_size
    return slice(rank * shard, (rank + 1) * shard)


def shard_mixer_params(dense, rank: int, world_size: int) -> dict[str, torch.Tensor]:
    """Rank r's parameter shard of a dense MambaMixer, sliced as the correct
    TP mixer slices it (reference tp_model.py:190-214): in_proj's x rows and
    z rows split separately, conv / dt_proj / A_log / D by channel, x_proj and
    out_proj by input column; the out_proj bias stays with rank 0."""
    cfg = dense.cfg
    sl = channel_slice(rank, world_size, cfg.d_inner)
    Di = cfg.d_inner
    w = dense.in_proj.weight
    p = {
        "in_proj.weight": torch.cat([w[:Di][sl], w[Di:][sl]], dim=0),
        "conv1d.weight": dense.conv1d.weight[sl],
        "x_proj.weight": dense.x_proj.weight[:, sl],
        "dt_proj.weight": dense.dt_proj.weight[sl],
        "dt_proj.bias": dense.dt_proj.bias[sl],
        "A_log": dense.A_log[sl],
        "D": dense.D[sl],
        "out_proj.weight": dense.out_proj.weight[:, sl],
    }
    if dense.in_proj.bias is not None:
        b = dense.in_proj.bias
        p["in_proj.bias"] = torch.cat([b[:Di][sl], b[Di:][sl]], dim=0)
    if dense.conv1d.bias is not None:
        p["conv1d.bias"] = dense.conv1d.bias[sl]
    if dense.out_proj.bias is not None:
        p["out_proj.bias"] = dense.out_proj.bias if rank == 0 else torch.zeros_like(dense.out_proj.bias)
    return {k: v.detach().contiguous() for k, v in p.items()}


def naive_shard_mixer_params(dense, rank: int, world_size: int) -> dict[str, torch.Tensor]:
    """The wrong split the reference keeps as a negative example
    (NaiveTPMambaMixer, tp_model.py:217-244): in_proj's packed [x | z] rows
    cut contiguously, so at world_size 2 rank 0 holds only x rows and rank 1
    only z rows; everything else as shard_mixer_params."""
    p = shard_mixer_params(dense, rank, world_size)
    full = channel_slice(rank, world_size, 2 * dense.cfg.d_inner)
    p["in_proj.weight"] = dense.in_proj.weight[full].detach().contiguous()
    if dense.in_proj.bias is not None:
        p["in_proj.bias"] = dense.in_proj.bias[full].detach().contiguous()
    return p


class ShardMixer:
    """One rank's channel shard of a MambaMixer (reference _TPMambaMixerBase,
    tp_model.py:44-179) on this GPU's kernels.

    The reference's two AllReduces split prefill and step into two stages
    each: stage 1 gives this rank's partial x_proj sums over its channels'
    share of the contraction, [.., R + 2N]; stage 2 takes the x_dbl summed
    over ranks and gives this rank's partial out_proj sums [.., d_model].
    The caller sums the partials of all ranks between the stages
    (LocalTPMixer does it in memory).  Caches hold this rank's channels only."""

    def __init__(self, dense, rank: int, world_size: int, naive: bool = False):
        cfg = dense.cfg
        self.cfg = cfg
        self.shard = cfg.d_inner // world_size
        self.p = (naive_shard_mixer_params if naive else shard_mixer_params)(dense, rank, world_size)
        w = self.p["conv1d.weight"]
        self.conv_w = w.reshape(w.shape[0], w.shape[-1]).float().contiguous()
        cb = self.p.get("conv1d.bias")
        self.conv_b = cb.float().contiguous() if cb is not None else None
        self.ssm = {k: self.p[k].float().contiguous() for k in ("dt_proj.weight", "dt_proj.bias", "A_log", "D")}

    def prefill_stage1(self, x: torch.Tensor, cache=None):
        """x [b, l, d_model] (replicated) -> (x_dbl partial [b, l, R+2N], saved).
        Conv history comes from cache.conv_state when a cache is given
        (tp_model.py:95-98)."""
        p, S = self.p, self.shard
        xz = F.linear(x, p["in_proj.weight"], p.get("in_proj.bias"))      # [b, l, 2S]: this rank's x | z
        xs, z = xz[..., :S].transpose(1, 2), xz[..., S:].transpose(1, 2)  # [b, S, l] views
        u_store = torch.empty(x.shape[0], x.shape[1], S, device=x.device, dtype=x.dtype)
        _, conv_state = ops.causal_conv1d(xs, self.conv_w, self.conv_b,
                                          conv_state=cache.conv_state if cache is not None else None,
                                          silu=True, out=u_store.transpose(1, 2))
        return F.linear(u_store, p["x_proj.weight"]), (u_store, z, conv_state)

    def prefill_stage2(self, x_dbl: torch.Tensor, saved, cache=None):
        """x_dbl [b, l, R+2N] (summed over ranks) -> (out_proj partial
        [b, l, d_model], conv_state [b, S, K-1], ssm_state [b, S, N]); the SSM
        starts from cache.ssm_state when a cache is given (tp_model.py:115-119)."""
        R, N = self.cfg.dt_rank, self.cfg.d_state
        u_store, z, conv_state = saved
        q = self.ssm
        dt = F.linear(x_dbl[..., :R], self.p["dt_proj.weight"])           # bias fused in the scan
        B, C = x_dbl[..., R:R + N].transpose(1, 2), x_dbl[..., R + N:].transpose(1, 2)
        y_store = torch.empty_like(u_store)
        _, h = ops.selective_scan(u_store.transpose(1, 2), dt.transpose(1, 2), q["A_log"], B, C, D=q["D"], z=z,
                                  delta_bias=q["dt_proj.bias"], a_is_log=True,
                                  h0=cache.ssm_state if cache is not None else None, y=y_store.transpose(1, 2))
        return F.linear(y_store, self.p["out_proj.weight"]), conv_state, h

    def step_stage1(self, x_t: torch.Tensor, cache):
        """x_t [b, d_model] -> (x_dbl partial [b, R+2N], saved); this rank's
        cache.conv_state advances in place (tp_model.py:142-158)."""
        S = self.shard
        xz = F.linear(x_t, self.p["in_proj.weight"], self.p.get("in_proj.bias"))  # [b, 2S]
        xc = ops.conv_step(cache.conv_state, xz[:, :S], self.conv_w, self.conv_b, silu=True)
        return F.linear(xc, self.p["x_proj.weight"]), (xc, xz[:, S:])

    def step_stage2(self, x_dbl: torch.Tensor, saved, cache):
        """x_dbl [b, R+2N] (summed over ranks) -> out_proj partial [b, d_model];
        cache.ssm_state advances in place (tp_model.py:160-174)."""
        xc, z = saved
        q = self.ssm
        y = ops.selective_state_update(cache.ssm_state, xc, z, x_dbl, q["dt_proj.weight"], q["dt_proj.bias"],
                                       q["A_log"], q["D"], a_is_log=True)
        return F.linear(y, self.p["out_proj.weight"])


def _sum_fp32(parts, counter: CommCounter | None = None):
    """Plain fp32 all-reduce, summed in rank order (the reference's fp32
    SUM of the same partials, tp_utils.py:23-28)."""
    out = parts[0].clone()
    for t in parts[1:]:
        out += t
    if counter is not None:
        counter.count += 1
        counter.bytes += parts[0].numel() * 4
    return out


# The all-reduce variants on this path, by the reference's dtype names
# (ALLREDUCE_FNS, tp_utils.py:150-158, where "int8" also names the per-token gather).
LOCAL_ALLREDUCE = {"fp32": _sum_fp32, "fp16": quant_dequant_sum_fp16, "int8": quant_dequant_sum_int8_tok,
                   "int8_gather_tok": quant_dequant_sum_int8_tok}
UNBUILT_ALLREDUCE = ("int8_legacy", "int8_sum", "int8_gather")  # per-tensor int8 variants of the reference
SITES = ("x_proj", "out_proj")


def site_dtype(spec, layer_idx: int, site: str) -> str:
    """The all-reduce dtype of one collective site (reference
    tp_utils.py:169-180): `spec` is one dtype name for every site or a
    {(layer_idx, site): dtype} map whose missing sites stay fp32.  `site` is
    "x_proj" (AllReduce #1) or "out_proj" (AllReduce #2)."""
    assert site in SITES, site
    dtype = spec if isinstance(spec, str) else spec.get((layer_idx, site), "fp32")
    if dtype in UNBUILT_ALLREDUCE:
        raise NotImplementedError(f"allreduce dtype {dtype!r} (per-tensor int8) is not built here; "
                                  f"built: {sorted(LOCAL_ALLREDUCE)}")
    assert dtype in LOCAL_ALLREDUCE, f"unknown allreduce dtype {dtype!r}"
    return dtype


class LocalTPMixer:
    """A tensor-parallel MambaMixer with all `world_size` ranks on this GPU:
    the reference's TPMambaMixer (tp_model.py:44-214, or NaiveTPMambaMixer,
    217-244, with naive=True) over channel shards of `dense`, with each of its
    two AllReduces per prefill or step done in memory, in rank order, by the
    LOCAL_ALLREDUCE op that `allreduce_dtype` names for that site (the
    payload quantizers of tp_utils.py:31-42 and 103-131 for fp16 and
    int8_gather_tok).  `comm` counts the collectives and one rank's wire
    bytes as the reference's CommCounter does.  Caches are one LayerCache
    per rank, holding that rank's channels."""

    def __init__(self, dense, world_size: int = 2, allreduce_dtype="fp32", layer_idx: int = 0, naive: bool = False):
        self.cfg = dense.cfg
        self.world_size = world_size
        self.layer_idx = layer_idx
        self.comm = CommCounter()
        self.shards = [ShardMixer(dense, r, world_size, naive=naive) for r in range(world_size)]
        self.out_bias = self.shards[0].p.get("out_proj.bias")
        self.set_allreduce_dtype(allreduce_dtype)

    def set_allreduce_dtype(self, allreduce_dtype) -> None:
        """Reference tp_model.py:76-79."""
        self.allreduce_dtype = allreduce_dtype
        self._ar_x = LOCAL_ALLREDUCE[site_dtype(allreduce_dtype, self.layer_idx, "x_proj")]
        self._ar_out = LOCAL_ALLREDUCE[site_dtype(allreduce_dtype, self.layer_idx, "out_proj")]

    def allocate_caches(self, batch: int, device=None, dtype=torch.float32):
        """One zeroed LayerCache per rank: conv_state [b, S, K-1] in `dtype`,
        ssm_state [b, S, N] fp32."""
        from .model import LayerCache
        cfg, S = self.cfg, self.shards[0].shard
        return [LayerCache(torch.zeros(batch, S, cfg.d_conv - 1, device=device, dtype=dtype),
                           torch.zeros(batch, S, cfg.d_state, device=device, dtype=torch.float32))
                for _ in range(self.world_size)]

    def _finish(self, parts, shape):
        out = self._ar_out(parts, counter=self.comm).reshape(shape)             # AllReduce #2
        return out + self.out_bias if self.out_bias is not None else out

    def prefill(self, x: torch.Tensor, caches=None):
        """x [b, l, d_model] -> (out [b, l, d_model], [conv_state per rank],
        [ssm_state per rank]) (tp_model.py:85-135).  With `caches`, each
        rank continues from its LayerCache, which is read, not written."""
        b, l, M = x.shape
        caches = caches if caches is not None else [None] * self.world_size
        s1 = [sh.prefill_stage1(x, c) for sh, c in zip(self.shards, caches)]
        J = s1[0][0].shape[-1]
        x_dbl = self._ar_x([part.reshape(b * l, J) for part, _ in s1], counter=self.comm).reshape(b, l, J)  # AR #1
        s2 = [sh.prefill_stage2(x_dbl, saved, c) for sh, (_, saved), c in zip(self.shards, s1, caches)]
        out = self._finish([part.reshape(b * l, M) for part, _, _ in s2], (b, l, M))
        return out, [cs for _, cs, _ in s2], [h for _, _, h in s2]

    def step(self, x_t: torch.Tensor, caches):
        """x_t [b, d_model] -> out [b, d_model]; every rank's LayerCache
        advances in place (tp_model.py:137-179)."""
        s1 = [sh.step_stage1(x_t, c) for sh, c in zip(self.shards, caches)]
        x_dbl = self._ar_x([part for part, _ in s1], counter=self.comm)                # AllReduce #1
        parts = [sh.step_stage2(x_dbl, saved, c) for sh, (_, saved), c in zip(self.shards, s1, caches)]
        return self._finish(parts, x_t.shape)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Full sequence, no cache (tp_model.py:81-83)."""
        return self.prefill(x)[0]

    __call__ = forward
