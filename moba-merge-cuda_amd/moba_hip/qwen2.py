"""Qwen2 as a consumer of the moba-hip API (no weights are downloaded; the
caller passes a transformers Qwen2 model).

* ``project_qkv`` / ``output_projection`` / ``decode_layer``: the projected,
  rotary-embedded Q/K/V adapter of examples/qwen2_attention.py:6-26, with the
  cache step served by :class:`~moba_hip.PagedKVCache` /
  :class:`~moba_hip.PreparedDecode`.
* :class:`Qwen2Session`: batch-1 full-model inference in the shape of
  examples/full_qwen2.py:19-215.  Prefill runs every layer's attention through
  the ``opt_hip`` MoBA prefill (topk 1 gives full causal attention) and fills
  one paged cache per layer; decode runs one prepared step per layer, either
  eagerly or as ONE hipGraph of the whole model step (``backend=
  "model_graph"``): the graph holds the projections, RoPE, every layer's
  fused decode launches, the MLPs and the LM head, and the host work of a
  step is the page planning of each layer (native code) plus one replay.
  The decode position comes from the device length of layer 0's cache, so
  replays need no new arguments.
"""
from __future__ import annotations

import torch

from .cache_layout import positive_int
from .grouped_attention import moba_hip_attention
from .kv_cache import PagedKVCache


def _rope():
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    return apply_rotary_pos_emb


def project_qkv(layer, hidden, cos, sin):
    """Q/K/V of ``hidden`` [b,t,hidden] through the layer's projections and
    rotary embedding, as [b*t, heads, head_dim] contiguous tensors."""
    b, t, _ = hidden.shape
    d = layer.head_dim
    q, k, v = (proj(hidden).view(b, t, -1, d).transpose(1, 2)
               for proj in (layer.q_proj, layer.k_proj, layer.v_proj))
    q, k = _rope()(q, k, cos, sin)
    return tuple(x.transpose(1, 2).reshape(b * t, -1, d).contiguous() for x in (q, k, v))


def output_projection(layer, attention_output):
    return layer.o_proj(attention_output.flatten(-2))


def decode_layer(layer, norm, hidden, cos, sin, cache_or_plan, *, graph=False, topk=4):
    """One decode token through one attention layer: project, then a prepared
    step (a PreparedDecode) or an append_and_attend (a cache); returns
    (o_proj output, DecodeResult, q, k, v)."""
    q, k, v = project_qkv(layer, norm(hidden), cos, sin)
    if hasattr(cache_or_plan, "step"):
        result = cache_or_plan.step(q, k, v, use_graph=graph)
    else:
        result = cache_or_plan.append_and_attend(q, k, v, sequence_ids=[0], topk=topk)
    return output_projection(layer, result.output), result, q, k, v


class Qwen2Session:
    def __init__(self, model, capacity, *, mode="moba", chunk=128, topk=4, page=16,
                 backend="eager"):
        if mode not in ("dense", "moba"):
            raise ValueError("mode")
        if backend not in ("eager", "model_graph"):
            raise ValueError("backend")
        cfg = model.config
        if cfg.model_type != "qwen2":
            raise ValueError("Qwen2 architecture required")
        if getattr(cfg, "use_sliding_window", False):
            raise ValueError("sliding window unsupported")
        if model.training or any(p.requires_grad for p in model.parameters()):
            raise ValueError("eval model with gradients disabled required")
        self.capacity = positive_int(capacity, "capacity")
        self.chunk, self.topk = positive_int(chunk, "chunk"), positive_int(topk, "topk")
        if self.topk > 9:
            raise ValueError("topk must be <=9")
        self.model, self.mode, self.backend = model, mode, backend
        self.device = next(model.parameters()).device
        if self.device.type != "cuda":
            raise ValueError("CUDA model required")
        self.dtype = next(model.parameters()).dtype
        self.hq, self.hk = cfg.num_attention_heads, cfg.num_key_value_heads
        self.dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // self.hq
        self.stream = torch.cuda.current_stream(self.device).cuda_stream
        self.caches = [PagedKVCache(1, self.capacity, self.hk, self.dim, page_size=page,
                                    chunk_size=self.chunk, dtype=self.dtype, device=self.device)
                       for _ in model.model.layers]
        self.plans, self.graph, self.closed, self.failed = [], None, False, False
        self.token = torch.zeros((1, 1), device=self.device, dtype=torch.long)
        self.logits = None

    def _check(self):
        if self.closed or self.failed:
            raise ValueError("closed/failed session")
        if torch.cuda.current_stream(self.device).cuda_stream != self.stream:
            raise ValueError("cross-stream session")

    def _prefill_config(self):
        # topk 1: the MoBA entry's full-causal fallback (one chunk per sequence)
        return {"chunk_size": self.chunk, "topk": self.topk if self.mode == "moba" else 1}

    @torch.no_grad()
    def prefill(self, ids):
        """Runs the prompt ``ids`` [1, t] (CUDA int64) through the model, filling
        every layer's cache; returns the logits of the last prompt token."""
        self._check()
        if self.plans or any(c.lengths[0] for c in self.caches):
            raise ValueError("fresh session required")
        if ids.dim() != 2 or ids.shape[0] != 1 or not 0 < ids.shape[1] < self.capacity:
            raise ValueError("batch=1, nonempty prefix below capacity required")
        if ids.device != self.device or ids.dtype != torch.long:
            raise ValueError("CUDA int64 token IDs required")
        m, t = self.model.model, ids.shape[1]
        h = m.embed_tokens(ids)
        cos, sin = m.rotary_emb(h, torch.arange(t, device=self.device)[None])
        cu = torch.tensor([0, t], device=self.device, dtype=torch.int32)
        for layer, cache in zip(m.layers, self.caches):
            q, k, v = project_qkv(layer.self_attn, layer.input_layernorm(h), cos, sin)
            cache.append(k, v, sequence_ids=[0], cu_seqlens=[0, t])
            out = moba_hip_attention(q, k, v, cu, t, self._prefill_config())
            h = h + output_projection(layer.self_attn, out[None])
            h = h + layer.mlp(layer.post_attention_layernorm(h))
        return self.model.lm_head(m.norm(h))[:, -1]

    @torch.no_grad()
    def prepare(self):
        """Leases every layer's cache for decode; with model_graph, captures
        one whole-model decode step."""
        self._check()
        if self.plans:
            raise ValueError("already prepared")
        if not self.caches[0].lengths[0]:
            raise ValueError("prefill first")
        self.plans = [c.prepare_decode([0], self.hq, mode=self.mode, topk=self.topk,
                                       check_finite=False) for c in self.caches]
        if self.backend == "model_graph":
            self._capture()

    def _compute_step(self):
        """Device work of one decode step on the current stream (capturable)."""
        m = self.model.model
        stream = torch.cuda.current_stream(self.device).cuda_stream
        h = m.embed_tokens(self.token)
        position = self.caches[0]._lengths[:1].to(torch.long).view(1, 1)
        cos, sin = m.rotary_emb(h, position)
        for layer, p in zip(m.layers, self.plans):
            q, k, v = project_qkv(layer.self_attn, layer.input_layernorm(h), cos, sin)
            p.q.copy_(q)
            p.k.copy_(k)
            p.v.copy_(v)
            p._launch_step(stream)
            h = h + output_projection(layer.self_attn, p.output.view(1, 1, self.hq, self.dim))
            h = h + layer.mlp(layer.post_attention_layernorm(h))
        self.logits = self.model.lm_head(m.norm(h))[:, -1]

    def _capture(self):
        # warm the torch ops (lazy kernels, allocator) on a side stream with
        # work that leaves every cache unchanged: a capture records, it does
        # not run, so the caches stay as they are
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            m = self.model.model
            h = m.embed_tokens(self.token)
            cos, sin = m.rotary_emb(h, torch.zeros((1, 1), device=self.device, dtype=torch.long))
            for layer in m.layers:
                project_qkv(layer.self_attn, layer.input_layernorm(h), cos, sin)
                layer.mlp(layer.post_attention_layernorm(h))
            self.model.lm_head(m.norm(h))
        torch.cuda.current_stream(self.device).wait_stream(side)
        with torch.cuda.graph(graph, stream=side):
            self._compute_step()
        self.graph = graph

    @torch.no_grad()
    def step(self, token):
        """Feeds one token; returns the logits [1, vocab] of the next one."""
        self._check()
        if isinstance(token, bool) or not isinstance(token, int) or \
                not 0 <= token < self.model.config.vocab_size:
            raise ValueError("one valid CPU token ID required")
        if not self.plans:
            raise ValueError("prepare first")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        for p in self.plans:  # host planning of every layer before any launch
            p._plan_step(stream)
        self.token.fill_(token)
        try:
            if self.graph is not None:
                self.graph.replay()
            else:
                self._compute_step()
            for p in self.plans:
                p._commit_step()
        except Exception:
            self.failed = True
            for p in self.plans:
                p.failed = True
            raise
        return self.logits

    def close(self):
        if self.closed:
            return
        for p in self.plans:
            p.close()
        self.graph, self.closed = None, True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
