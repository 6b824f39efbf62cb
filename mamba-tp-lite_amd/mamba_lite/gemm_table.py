"""Tuned GEMM solutions for the projection shapes of the prefill workloads.

The projections (in_proj, x_proj, dt_proj, out_proj, the tied lm_head) are
torch fp32 GEMMs on hipBLASLt / rocBLAS.  `gemm_table_gfx950.csv` is a torch
TunableOp results table: for each prefill projection and lm_head shape of the
mamba-130m model at batch 32 x 1024 tokens (and the lm_head of its 64-token
prompt) and of the mamba-1.4b model at 1 x 1024 and 32 x 1024 tokens, it
names the hipBLASLt or rocBLAS solution that measured fastest on MI355X,
among all solutions both libraries offer.  It was recorded by running the
prefill benchmark with TunableOp tuning on (10 iterations or 10 ms per
candidate).  Against hipBLASLt's defaults, the 1.4b entries took the
1024-token prefill from 42.8 K to 43.4-43.5 K tok/s at batch 1 and from
50.4 K to 51.5-51.6 K tok/s at batch 32 (A/B in one run, twice).

`enable()` turns TunableOp on with tuning off and loads the table.  Shapes in
the table then run their tuned solution; every other GEMM keeps torch's
default path.  The table is tied to the builds it was measured with: torch
rejects it (and `enable` returns False) when torch, HIP, hipBLASLt or rocBLAS
versions or the GPU architecture differ, and every GEMM then keeps the
default path.  TunableOp is a process-wide torch setting, so this is opt-in.

Of the decode shapes only the 1.4b batch-32 step's tied lm_head (32 x 50280
x 2048, the one torch GEMM left in that step) is in the table: its pick took
the captured step from 2335-2336 to 2321 us.  The 32-row projections, when
they were torch GEMMs, ran slower inside the captured decode graph with the
tuner's picks than with hipBLASLt's default.  So
are the 64-token prompt's projections: the tuner's rocBLAS picks ran 1.528
ms per prompt inside a captured 130m prefill against 1.418 ms with
hipBLASLt's defaults (they now run on the library's own skinny GEMM).  The
64-token prompt's tied lm_head (64 x 50280 x 768) is in the table: its
rocBLAS pick takes the captured prompt from 876-878 to 863-866 us.
"""
from __future__ import annotations

import os

import torch

TABLE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gemm_table_gfx950.csv")


def enable(path: str = TABLE) -> bool:
    """Use the tuned GEMM table (TunableOp on, tuning off).  Returns True if
    torch accepted the table."""
    import torch.cuda.tunable as tunable

    if not torch.cuda.is_available() or not os.path.exists(path):
        return False
    tunable.enable(True)
    tunable.tuning_enable(False)
    return bool(tunable.read_file(path))
