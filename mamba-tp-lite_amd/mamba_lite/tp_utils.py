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
