"""CPU oracle for the Mamba mixer hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference
(`mamba_lite/model.py`, `mamba_lite/tp_utils.py` of mamba-tp-lite) so the HIP
kernels can be checked against it.  Only `tests/`, `__graft_entry__.smoke()`
and the `cpu_baseline` leg of `bench.py` may import it, and only to check
results against or to time as the CPU baseline.  The product package never
imports it and has no CPU fallback.

Modules
-------
mixer  -- causal conv1d, selective scan (materialize-then-loop form), mixer
          prefill/step, RMSNorm, LM prefill/step.  float32 follows the
          reference op order; float64 is the brute-force variant.
quant  -- per-token int8 quantize -> dequantize-sum and the fp16 cast-sum of
          the tensor-parallel AllReduce payload (bit-exact restatement).
pins   -- independent formulations used only to pin the restatement
          (closed-form scan, np.convolve conv, geometric series).

Parity status of each function is listed in the module docstrings; every
function here is pinned by a check in tests/test_oracle.py (none is
"parity unpinned").
"""
