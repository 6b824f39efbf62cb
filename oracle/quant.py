"""Bit-exact numpy restatement of the AllReduce payload quantizers
(test infrastructure).

Follows mamba-tp-lite `mamba_lite/tp_utils.py`:
  * per-token int8 gather, `_int8_gather(per_token=True)` (tp_utils.py:103-131,
    reached through `all_reduce_sum_int8_gather_tok`, 145-149);
  * fp16 cast -> sum -> cast back, `all_reduce_sum_fp16` (tp_utils.py:31-42).
The collective itself is replaced by the partial tensors held in memory: the
all-gather of payloads becomes "payload r is computed from partial r", and
the sum runs locally in rank order (tp_utils.py:127-130).

numpy float32 arithmetic is IEEE binary32 with one rounding per ufunc call
(no FMA contraction), np.rint is round-half-to-even like torch.round, and
float32 -> float16 casts round to nearest even -- the same roundings the
reference's torch CPU ops perform.

Parity: pinned in tests/test_oracle.py by hand-computed rows (exact scales,
ties-to-even, zero rows, +-amax -> +-127), the payload byte formula that
reproduces the published 673,185,792-byte prefill total, and the fp16 double
rounding identity (fp32 sum then fp16 == exact sum rounded once to fp16).
"""
from __future__ import annotations

import numpy as np

_EPS = np.float32(1e-8)     # clamp(min=1e-8) on a float32 tensor (tp_utils.py:111)
_QMAX = np.float32(127.0)   # "/ 127.0" (tp_utils.py:111)


def quantize_int8_per_token(t: np.ndarray):
    """tp_utils.py:106-112 with per_token=True: rows = all leading dims,
    scale_r = max(amax_r, 1e-8) / 127 (fp32), q = clamp(round(t / scale), +-127).
    Returns (scales float32 [rows], codes int8 [rows, cols])."""
    t = np.ascontiguousarray(t, dtype=np.float32)
    cols = t.shape[-1]
    t2 = t.reshape(-1, cols)
    amax = np.abs(t2).max(axis=1) if cols > 0 else np.zeros(t2.shape[0], np.float32)
    scale = (np.maximum(amax, _EPS) / _QMAX).astype(np.float32)
    q = np.clip(np.rint(t2 / scale[:, None]), -127, 127).astype(np.int8)
    return scale, q


def pack_payload(scale: np.ndarray, q: np.ndarray) -> np.ndarray:
    """tp_utils.py:113: [scales as little-endian fp32 bytes || int8 codes row-major]."""
    return np.concatenate([np.ascontiguousarray(scale, np.float32).view(np.uint8),
                           np.ascontiguousarray(q, np.int8).view(np.uint8).reshape(-1)])


def unpack_payload(payload: np.ndarray, rows: int, cols: int):
    """Inverse of pack_payload (tp_utils.py:129-130)."""
    s = np.ascontiguousarray(payload[:4 * rows]).view(np.float32)
    q = np.ascontiguousarray(payload[4 * rows:4 * rows + rows * cols]).view(np.int8).reshape(rows, cols)
    return s, q


def payload_nbytes(rows: int, cols: int) -> int:
    """Bytes on the wire per rank per call: 4*rows + rows*cols (tp_utils.py:113-117)."""
    return 4 * rows + rows * cols


def dequant_sum(payloads, rows: int, cols: int) -> np.ndarray:
    """tp_utils.py:127-130: out = 0; for r in rank order: out += q_r.float() * s_r."""
    out = np.zeros((rows, cols), np.float32)
    for p in payloads:
        s, q = unpack_payload(p, rows, cols)
        out = out + q.astype(np.float32) * s[:, None]
    return out


def quant_dequant_sum_int8_tok(parts):
    """Local restatement of all_reduce_sum_int8_gather_tok over the given
    partial tensors (one per rank).  Returns (out float32 of the parts' shape,
    list of payload byte arrays)."""
    parts = [np.ascontiguousarray(p, np.float32) for p in parts]
    shape = parts[0].shape
    cols = shape[-1]
    rows = int(np.prod(shape[:-1])) if len(shape) > 1 else 1
    payloads = [pack_payload(*quantize_int8_per_token(p)) for p in parts]
    return dequant_sum(payloads, rows, cols).reshape(shape), payloads


def fp16_sum(parts):
    """tp_utils.py:37-42 locally: low_r = fp16(part_r); SUM in fp16; back to
    fp32.  Returns (out float32, list of fp16 payloads)."""
    # values beyond the fp16 range become +-inf, as torch's .half() makes them
    with np.errstate(over="ignore"):
        lows = [np.ascontiguousarray(p, np.float32).astype(np.float16) for p in parts]
        acc = lows[0]
        for lo in lows[1:]:
            acc = (acc + lo).astype(np.float16)   # numpy half add: fp32 add rounded to fp16 (RNE)
    return acc.astype(np.float32), lows
