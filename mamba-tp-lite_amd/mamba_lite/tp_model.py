"""Tensor-parallel Mamba with every rank's channel shard on one GPU
(mamba-tp-lite mamba_lite/tp_model.py).

The reference runs one process per rank and exchanges the two partial sums of
each mixer call over torch.distributed: the x_proj partials (AllReduce #1,
so every rank sees the same dt_low / B / C) and the out_proj partials
(AllReduce #2, bias added once).  Here all ranks' shards live on this GPU and
run the same kernels at the shard shape; each AllReduce is an in-memory sum
of the ranks' partials in rank order -- plain fp32, or the fp16 / per-token
int8 payload quantizers of tp_utils -- chosen per (layer, site) as the
reference's per-site dtype spec chooses it.  Every call keeps the
reference's two-stage split (ShardMixer stage 1 ends at the x_proj partial,
stage 2 at the out_proj partial), so a multi-GPU mixer is the same shard
code with the in-memory sum replaced by the collective.
"""
from __future__ import annotations

import os

import torch
import torch.nn.functional as F

from . import ops
from .model import LayerCache, MambaConfig, load_hf_state_dict
from .tp_utils import LOCAL_ALLREDUCE, CommCounter, shard_mixer_tensors, site_dtype


class ShardMixer:
    """One rank's channel shard of a MambaMixer (reference _TPMambaMixerBase,
    tp_model.py:44-179) on this GPU's kernels.  `params` is the rank's
    shard in shard_mixer_tensors' layout.

    prefill and step each run in two stages around the reference's two
    AllReduces: stage 1 gives this rank's partial x_proj sums over its
    channels' share of the contraction, [.., R + 2N]; stage 2 takes the x_dbl
    summed over ranks and gives this rank's partial out_proj sums
    [.., d_model].  Caches hold this rank's channels only."""

    def __init__(self, cfg: MambaConfig, params: dict[str, torch.Tensor]):
        self.cfg = cfg
        self.p = params
        self.shard = params["D"].shape[0]
        w = params["conv1d.weight"]
        self.conv_w = w.reshape(w.shape[0], w.shape[-1]).float().contiguous()
        cb = params.get("conv1d.bias")
        self.conv_b = cb.float().contiguous() if cb is not None else None
        self.ssm = {k: params[k].float().contiguous() for k in ("dt_proj.weight", "dt_proj.bias", "A_log", "D")}

    def prefill_stage1(self, x: torch.Tensor, cache: LayerCache | None = None):
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

    def prefill_stage2(self, x_dbl: torch.Tensor, saved, cache: LayerCache | None = None):
        """x_dbl [b, l, R+2N] (summed over ranks) -> (out_proj partial
        [b, l, d_model], conv_state [b, S, K-1], ssm_state [b, S, N] fp32);
        the SSM starts from cache.ssm_state when a cache is given
        (tp_model.py:115-119)."""
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

    def step_stage1(self, x_t: torch.Tensor, cache: LayerCache):
        """x_t [b, d_model] -> (x_dbl partial [b, R+2N], saved); this rank's
        cache.conv_state advances in place (tp_model.py:142-158)."""
        S = self.shard
        xz = F.linear(x_t, self.p["in_proj.weight"], self.p.get("in_proj.bias"))  # [b, 2S]
        xc = ops.conv_step(cache.conv_state, xz[:, :S], self.conv_w, self.conv_b, silu=True)
        return F.linear(xc, self.p["x_proj.weight"]), (xc, xz[:, S:])

    def step_stage2(self, x_dbl: torch.Tensor, saved, cache: LayerCache):
        """x_dbl [b, R+2N] (summed over ranks) -> out_proj partial [b, d_model];
        cache.ssm_state advances in place (tp_model.py:160-174)."""
        xc, z = saved
        q = self.ssm
        y = ops.selective_state_update(cache.ssm_state, xc, z, x_dbl, q["dt_proj.weight"], q["dt_proj.bias"],
                                       q["A_log"], q["D"], a_is_log=True)
        return F.linear(y, self.p["out_proj.weight"])


class LocalTPMixer:
    """A tensor-parallel MambaMixer with all `world_size` ranks on this GPU:
    the reference's TPMambaMixer (tp_model.py:44-214), or NaiveTPMambaMixer
    (217-244) when loaded with naive=True.  Each prefill or step does the two
    AllReduces in memory, in rank order, with the LOCAL_ALLREDUCE op that
    `allreduce_dtype` names for the site; partials are reduced in fp32 and
    cast back to the activation dtype.  `comm` counts collectives and one
    rank's wire bytes as the reference's CommCounter does.  Caches are one
    LayerCache per rank, holding that rank's channels."""

    def __init__(self, cfg: MambaConfig, world_size: int = 2, allreduce_dtype="fp32", layer_idx: int = 0):
        assert cfg.d_inner % world_size == 0
        self.cfg = cfg
        self.world_size = world_size
        self.layer_idx = layer_idx
        self.comm = CommCounter()
        self.shards: list[ShardMixer] = []
        self.out_bias = None
        self.set_allreduce_dtype(allreduce_dtype)

    @classmethod
    def from_dense(cls, dense, world_size: int = 2, allreduce_dtype="fp32", layer_idx: int = 0,
                   naive: bool = False) -> "LocalTPMixer":
        return cls(dense.cfg, world_size, allreduce_dtype, layer_idx).load_shard_from_dense(dense, naive)

    def load_shard_from_dense(self, dense, naive: bool = False) -> "LocalTPMixer":
        """Every rank's shard of `dense` (tp_model.py:190-214, or the naive
        split of 217-244)."""
        tensors = dict(dense.named_parameters())
        return self.load_shards([shard_mixer_tensors(tensors, self.cfg.d_inner, r, self.world_size, naive)
                                 for r in range(self.world_size)])

    def load_shards(self, params_per_rank) -> "LocalTPMixer":
        assert len(params_per_rank) == self.world_size
        self.shards = [ShardMixer(self.cfg, p) for p in params_per_rank]
        self.out_bias = params_per_rank[0].get("out_proj.bias")
        return self

    def set_allreduce_dtype(self, allreduce_dtype) -> None:
        """Reference tp_model.py:75-78."""
        self.allreduce_dtype = allreduce_dtype
        self._ar_x = LOCAL_ALLREDUCE[site_dtype(allreduce_dtype, self.layer_idx, "x_proj")]
        self._ar_out = LOCAL_ALLREDUCE[site_dtype(allreduce_dtype, self.layer_idx, "out_proj")]

    def allocate_caches(self, batch: int, device=None, dtype=torch.float32) -> list[LayerCache]:
        """One zeroed LayerCache per rank: conv_state [b, S, K-1] in `dtype`,
        ssm_state [b, S, N] fp32."""
        cfg, S = self.cfg, self.cfg.d_inner // self.world_size
        return [LayerCache(torch.zeros(batch, S, cfg.d_conv - 1, device=device, dtype=dtype),
                           torch.zeros(batch, S, cfg.d_state, device=device, dtype=torch.float32))
                for _ in range(self.world_size)]

    def _reduce(self, ar, parts, shape, dtype):
        rows = parts[0].numel() // shape[-1]
        out = ar([t.reshape(rows, shape[-1]).float() for t in parts], counter=self.comm)
        return out.reshape(shape).to(dtype)

    def prefill(self, x: torch.Tensor, caches: list[LayerCache] | None = None):
        """x [b, l, d_model] -> (out [b, l, d_model], [conv_state per rank],
        [ssm_state per rank]) (tp_model.py:85-135).  With `caches`, each rank
        continues from its LayerCache, which is read, not written."""
        if not self.shards:
            raise RuntimeError("no shards loaded: call load_shard_from_dense or load_shards first")
        b, l, M = x.shape
        caches = caches if caches is not None else [None] * self.world_size
        s1 = [sh.prefill_stage1(x, c) for sh, c in zip(self.shards, caches)]
        J = s1[0][0].shape[-1]
        x_dbl = self._reduce(self._ar_x, [part for part, _ in s1], (b, l, J), x.dtype)          # AllReduce #1
        s2 = [sh.prefill_stage2(x_dbl, saved, c) for sh, (_, saved), c in zip(self.shards, s1, caches)]
        out = self._reduce(self._ar_out, [part for part, _, _ in s2], (b, l, M), x.dtype)       # AllReduce #2
        if self.out_bias is not None:
            out = out + self.out_bias
        return out, [cs for _, cs, _ in s2], [h for _, _, h in s2]

    def step(self, x_t: torch.Tensor, caches: list[LayerCache]) -> torch.Tensor:
        """x_t [b, d_model] -> out [b, d_model]; every rank's LayerCache
        advances in place (tp_model.py:137-179)."""
        if not self.shards:
            raise RuntimeError("no shards loaded: call load_shard_from_dense or load_shards first")
        ops.check_step_shape(self.cfg.d_state, self.cfg.dt_rank)   # before any rank's conv history moves
        s1 = [sh.step_stage1(x_t, c) for sh, c in zip(self.shards, caches)]
        x_dbl = self._reduce(self._ar_x, [part for part, _ in s1], s1[0][0].shape, x_t.dtype)  # AllReduce #1
        parts = [sh.step_stage2(x_dbl, saved, c) for sh, (_, saved), c in zip(self.shards, s1, caches)]
        out = self._reduce(self._ar_out, parts, x_t.shape, x_t.dtype)                           # AllReduce #2
        return out + self.out_bias if self.out_bias is not None else out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Full sequence, no cache (tp_model.py:80-83)."""
        return self.prefill(x)[0]

    __call__ = forward


class LocalTPCache:
    """The caches of a LocalTPLM: layers[i][r] is layer i's LayerCache on
    rank r (the reference keeps one MambaCache per rank process, each holding
    that rank's channels)."""

    def __init__(self, layers: list[list[LayerCache]]):
        self.layers = layers

    @staticmethod
    def allocate(cfg: MambaConfig, world_size: int, batch_size: int, device, dtype=torch.float32) -> "LocalTPCache":
        mixer = LocalTPMixer(cfg, world_size)
        return LocalTPCache([mixer.allocate_caches(batch_size, device, dtype) for _ in range(cfg.n_layer)])


class LocalTPBlock:
    """RMSNorm weight + LocalTPMixer of one layer (reference TPMambaBlock,
    tp_model.py:247-262)."""

    def __init__(self, norm_weight: torch.Tensor, mixer: LocalTPMixer):
        self.norm_weight = norm_weight
        self.mixer = mixer


class LocalTPLM:
    """Tensor-parallel full model with every rank on this GPU (reference
    TPMambaLM, tp_model.py:271-384): embedding, norms and the tied lm_head
    replicated, each layer's mixer a LocalTPMixer.  The residual stream is
    float32 and each residual add runs fused with the next RMSNorm, as in
    MambaLM."""

    def __init__(self, cfg: MambaConfig, embedding: torch.Tensor, blocks: list[LocalTPBlock],
                 norm_f_weight: torch.Tensor):
        self.cfg = cfg
        self.embedding_weight = embedding
        self.layers = blocks
        self.norm_f_weight = norm_f_weight
        self._norm_w = [b.norm_weight.float().contiguous() for b in blocks] + [norm_f_weight.float().contiguous()]
        self.world_size = blocks[0].mixer.world_size if blocks else 1

    @classmethod
    def from_dense(cls, lm, world_size: int = 2, allreduce_dtype="fp32", naive: bool = False) -> "LocalTPLM":
        """Every rank's shard of a dense MambaLM."""
        blocks = [LocalTPBlock(blk.norm.weight.detach(),
                               LocalTPMixer.from_dense(blk.mixer, world_size, allreduce_dtype, i, naive))
                  for i, blk in enumerate(lm.layers)]
        return cls(lm.cfg, lm.embedding.weight.detach(), blocks, lm.norm_f.weight.detach())

    @classmethod
    def from_pretrained_shard(cls, hf_path: str, world_size: int = 2, allreduce_dtype="fp32",
                              dtype=torch.float32, device=None) -> "LocalTPLM":
        """A local HF `state-spaces/mamba-*-hf` snapshot (single or sharded
        safetensors), every mixer tensor sliced per rank straight from the
        checkpoint's state dict, with no dense model built (reference
        TPMambaLM.from_pretrained_shard, tp_model.py:335-384)."""
        cfg = MambaConfig.from_hf_config(os.path.join(hf_path, "config.json"))
        sd = load_hf_state_dict(hf_path)
        put = lambda t: t.to(device=device, dtype=dtype)
        names = ["in_proj.weight", "in_proj.bias", "conv1d.weight", "conv1d.bias", "x_proj.weight",
                 "dt_proj.weight", "dt_proj.bias", "A_log", "D", "out_proj.weight", "out_proj.bias"]
        blocks = []
        for i in range(cfg.n_layer):
            pre = f"backbone.layers.{i}."
            tensors = {n: put(sd[pre + "mixer." + n]) for n in names if pre + "mixer." + n in sd}
            mixer = LocalTPMixer(cfg, world_size, allreduce_dtype, i).load_shards(
                [shard_mixer_tensors(tensors, cfg.d_inner, r, world_size) for r in range(world_size)])
            blocks.append(LocalTPBlock(put(sd[pre + "norm.weight"]), mixer))
        return cls(cfg, put(sd["backbone.embeddings.weight"]), blocks, put(sd["backbone.norm_f.weight"]))

    def set_allreduce_dtype(self, allreduce_dtype) -> None:
        for blk in self.layers:
            blk.mixer.set_allreduce_dtype(allreduce_dtype)

    def lm_head(self, x: torch.Tensor) -> torch.Tensor:
        return F.linear(x, self.embedding_weight)

    def _run(self, x: torch.Tensor, per_layer) -> torch.Tensor:
        act = x.dtype
        eps = self.cfg.layer_norm_epsilon
        h = x.float().contiguous()
        normed = ops.add_rmsnorm(h, self._norm_w[0], eps)
        for i in range(len(self.layers)):
            y = per_layer(i, normed.to(act))
            normed = ops.add_rmsnorm(h, self._norm_w[i + 1], eps, y=y.float().contiguous(), x_out=h)
        return normed.to(act)

    def prefill(self, input_ids: torch.Tensor, cache: LocalTPCache | None = None):
        """input_ids [b, l] -> (logits [b, l, vocab], new LocalTPCache)
        (tp_model.py:305-315)."""
        x = F.embedding(input_ids, self.embedding_weight)
        new_layers: list[list[LayerCache]] = []

        def layer(i, xn):
            out, conv, ssm = self.layers[i].mixer.prefill(xn, cache.layers[i] if cache is not None else None)
            new_layers.append([LayerCache(c, h) for c, h in zip(conv, ssm)])
            return out

        xf = self._run(x, layer)
        return self.lm_head(xf), LocalTPCache(new_layers)

    def step(self, input_ids: torch.Tensor, cache: LocalTPCache) -> torch.Tensor:
        """input_ids [b, 1] -> logits [b, 1, vocab]; every rank's cache
        advances in place (tp_model.py:317-322)."""
        x = F.embedding(input_ids, self.embedding_weight).squeeze(1)
        xf = self._run(x, lambda i, xn: self.layers[i].mixer.step(xn, cache.layers[i]))
        return self.lm_head(xf).unsqueeze(1)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        """Greedy decode (tp_model.py:324-333): one prefill, then steps."""
        logits, cache = self.prefill(input_ids)
        next_id = logits[:, -1:].argmax(dim=-1)
        tokens = [input_ids, next_id]
        for _ in range(max_new_tokens - 1):
            logits = self.step(next_id, cache)
            next_id = logits[:, -1, :].argmax(dim=-1, keepdim=True)
            tokens.append(next_id)
        return torch.cat(tokens, dim=1)
