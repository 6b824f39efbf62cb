"""hipGraph-captured decode step (same API as mamba-tp-lite's
mamba_lite/cuda_graph.py:29-131).

On ROCm, torch.cuda.graph / torch.cuda.CUDAGraph record a hipGraph.  The
whole MambaLM.step -- embedding, fused add+RMSNorm, the in_proj / x_proj /
out_proj / lm_head GEMMs and the libmtl conv-step and SSM-update kernels --
is captured once and replayed with one launch per token.  The step kernels
update the cache in place and never allocate, synchronize or touch host
memory, which is what makes the capture valid.
"""
from __future__ import annotations

import torch


class CUDAGraphUnsupported(RuntimeError):
    """Capture cannot proceed; the caller should fall back to eager decode
    (reference cuda_graph.py:29-30)."""


def _clone_cache(cache):
    """Disposable copy of a MambaCache for the warmup steps, so warmup does
    not advance the cache that gets captured (reference cuda_graph.py:34-48)."""
    from .model import LayerCache, MambaCache

    return MambaCache([LayerCache(conv_state=l.conv_state.clone(), ssm_state=l.ssm_state.clone())
                       for l in cache.layers])


class GraphedStepper:
    """Captures `model.step(static_ids, cache)` once, then replays it.

        stepper = GraphedStepper(model, cache, batch_size=1, device="cuda")
        stepper.capture()
        for _ in range(n_new_tokens):
            logits = stepper.replay(next_id)   # next_id: [batch, 1] int64
    """

    def __init__(self, model, cache, batch_size: int, device: str, n_warmup: int = 3):
        if device != "cuda" or not torch.cuda.is_available():
            raise CUDAGraphUnsupported("graph capture needs a GPU device ('cuda'); there is no CPU fallback.")
        allreduce_dtype = getattr(model, "allreduce_dtype", "fp32")
        names = {allreduce_dtype} if isinstance(allreduce_dtype, str) else set(allreduce_dtype.values())
        if "int8_legacy" in names:
            raise CUDAGraphUnsupported("int8_legacy synchronizes its scale through the host (.item()), "
                                       "which cannot be captured.")
        self.model = model
        self.cache = cache
        self.device = device
        self.static_ids = torch.zeros((batch_size, 1), dtype=torch.long, device=device)
        self.static_logits = None
        self.graph = None
        self.n_warmup = n_warmup

    def capture(self):
        # warmup on a side stream against a clone of the cache: settles the
        # caching allocator and the GEMM libraries' lazy initialization
        warm = _clone_cache(self.cache)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(self.n_warmup):
                self.model.step(self.static_ids, warm)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        del warm

        self.graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(self.graph), torch.no_grad():
                self.static_logits = self.model.step(self.static_ids, self.cache)
        except RuntimeError as e:
            self.graph = None
            raise CUDAGraphUnsupported(f"graph capture failed: {e}") from e
        # the step reads derived weight copies (transposed x_proj, the fused
        # decode plan) at addresses now baked into the graph: keep them alive,
        # and remember which parameter versions they were built from
        key_fn = getattr(self.model, "_derived_key", None)
        self._derived_key = key_fn() if key_fn is not None else None
        held_fn = getattr(self.model, "_derived_tensors", None)
        self._held = held_fn() if held_fn is not None else None

    def replay(self, next_id: torch.Tensor) -> torch.Tensor:
        if self.graph is None:
            raise RuntimeError("call capture() before replay()")
        if self._derived_key is not None and self.model._derived_key() != self._derived_key:
            # the reference's graph reads the parameters themselves; this one
            # reads copies made at capture, so a weight update needs a new capture
            raise RuntimeError("model weights changed after capture(); capture again before replaying")
        self.static_ids.copy_(next_id)
        self.graph.replay()
        return self.static_logits


class GraphedPrefill:
    """Captures `model.prefill(static_ids, out_cache=cache)` for one fixed
    [batch_size, seqlen] prompt shape, then replays it per prompt.

        prefill = GraphedPrefill(model, cache, batch_size=1, seqlen=64, device="cuda")
        prefill.capture()
        logits = prefill.replay(prompt_ids)    # [batch, seqlen] int64

    A replay writes the prompt's final conv and SSM states into `cache` in
    place and its logits into `static_logits`; the next replay overwrites
    both.  Passing the cache a GraphedStepper captured lets decoding continue
    from the prompt with no copy.  Every replay starts from zero state, as
    MambaLM.prefill without an incoming cache does.  A short prompt's eager
    prefill is bound by host time (about a hundred launches through torch and
    the kernel wrappers); a replay is one graph launch.  The reference graphs
    only the decode step; this is the same capture for the prompt."""

    def __init__(self, model, cache, batch_size: int, seqlen: int, device: str, n_warmup: int = 3):
        if device != "cuda" or not torch.cuda.is_available():
            raise CUDAGraphUnsupported("graph capture needs a GPU device ('cuda'); there is no CPU fallback.")
        if len(cache.layers) != len(model.layers):
            raise ValueError("cache has the wrong number of layers")
        self.model = model
        self.cache = cache
        self.static_ids = torch.zeros((batch_size, seqlen), dtype=torch.long, device=device)
        self.static_logits = None
        self.graph = None
        self.n_warmup = n_warmup

    def capture(self):
        warm = _clone_cache(self.cache)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(self.n_warmup):
                self.model.prefill(self.static_ids, out_cache=warm)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        del warm

        self.graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(self.graph), torch.no_grad():
                self.static_logits, _ = self.model.prefill(self.static_ids, out_cache=self.cache)
        except RuntimeError as e:
            self.graph = None
            raise CUDAGraphUnsupported(f"graph capture failed: {e}") from e

    def replay(self, ids: torch.Tensor) -> torch.Tensor:
        if tuple(ids.shape) != tuple(self.static_ids.shape):
            raise ValueError(f"ids must be {tuple(self.static_ids.shape)}, got {tuple(ids.shape)}")
        self.static_ids.copy_(ids)
        self.graph.replay()
        return self.static_logits
