"""Payload quantizers of the tensor-parallel AllReduce, run as local ops, plus
the channel-shard helpers (mamba-tp-lite mamba_lite/tp_utils.py).

On one GPU there is no collective: the partial sums that ranks would
exchange are tensors in this GPU's memory, and the ops below do what the
reference does around its collective -- quantize each partial into its wire
payload, then dequantize and sum in rank order -- as one HIP kernel each.
"""
from __future__ import annotations

import torch

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


def shard_mixer_tensors(tensors, d_inner: int, rank: int, world_size: int,
                        naive: bool = False) -> dict[str, torch.Tensor]:
    """Rank r's shard of one dense mixer's tensors, given by their module
    names ("in_proj.weight", "A_log", ...; biases may be absent), sliced as
    the correct TP mixer slices them (reference tp_model.py:190-214): in_proj's
    x rows and z rows split separately, conv / dt_proj / A_log / D by channel,
    x_proj and out_proj by input column; the out_proj bias stays with rank 0.
    naive=True cuts in_proj's packed [x | z] rows contiguously instead, the
    wrong split of NaiveTPMambaMixer (tp_model.py:217-244): at world_size 2
    rank 0 then holds only x rows and rank 1 only z rows."""
    sl = channel_slice(rank, world_size, d_inner)
    t = tensors
    if naive:
        full = channel_slice(rank, world_size, 2 * d_inner)
        packed = lambda v: v[full]
    else:
        packed = lambda v: torch.cat([v[:d_inner][sl], v[d_inner:][sl]], dim=0)
    p = {
        "in_proj.weight": packed(t["in_proj.weight"]),
        "conv1d.weight": t["conv1d.weight"][sl],
        "x_proj.weight": t["x_proj.weight"][:, sl],
        "dt_proj.weight": t["dt_proj.weight"][sl],
        "dt_proj.bias": t["dt_proj.bias"][sl],
        "A_log": t["A_log"][sl],
        "D": t["D"][sl],
        "out_proj.weight": t["out_proj.weight"][:, sl],
    }
    if t.get("in_proj.bias") is not None:
        p["in_proj.bias"] = packed(t["in_proj.bias"])
    if t.get("conv1d.bias") is not None:
        p["conv1d.bias"] = t["conv1d.bias"][sl]
    if t.get("out_proj.bias") is not None:
        ob = t["out_proj.bias"]
        p["out_proj.bias"] = ob if rank == 0 else torch.zeros_like(ob)
    return {k: v.detach().contiguous() for k, v in p.items()}


def shard_mixer_params(dense, rank: int, world_size: int) -> dict[str, torch.Tensor]:
    """Rank r's parameter shard of a dense MambaMixer (shard_mixer_tensors)."""
    return shard_mixer_tensors(dict(dense.named_parameters()), dense.cfg.d_inner, rank, world_size)


def naive_shard_mixer_params(dense, rank: int, world_size: int) -> dict[str, torch.Tensor]:
    """The naive packed-tensor split of NaiveTPMambaMixer (tp_model.py:217-244)."""
    return shard_mixer_tensors(dict(dense.named_parameters()), dense.cfg.d_inner, rank, world_size, naive=True)


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
