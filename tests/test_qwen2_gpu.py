"""Qwen2 consumer of the API (examples/qwen2_attention.py:20-26,
examples/full_qwen2.py:96-187) on a small randomly initialised Qwen2 (no
weights are available offline):

* dense mode equals the transformers model's own forward (full causal
  attention) on the same token sequence, for the prefill logits and every
  decode step;
* MoBA mode: the whole-model hipGraph replays equal the eager steps bit for
  bit, and one layer's decode attention matches the FP64 oracle on the
  routes it took (decode_layer adapter).
"""
import pytest
import torch

from decode_check import check

pytestmark = pytest.mark.gpu


def _model(seed=0, layers=2):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    torch.manual_seed(seed)
    cfg = Qwen2Config(vocab_size=512, hidden_size=512, intermediate_size=1024,
                      num_hidden_layers=layers, num_attention_heads=8, num_key_value_heads=2,
                      max_position_embeddings=4096, attn_implementation="eager")
    m = Qwen2ForCausalLM(cfg).to("cuda", torch.bfloat16).eval()
    for p in m.parameters():
        p.requires_grad_(False)
    return m


def _tokens(n, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 512, (1, n), generator=g).to("cuda")


def test_dense_session_matches_transformers(cuda_device):
    from moba_hip.qwen2 import Qwen2Session
    model = _model()
    ids = _tokens(200, 1)
    extra = [int(x) for x in _tokens(5, 2)[0]]
    with Qwen2Session(model, 256, mode="dense", chunk=64, page=16) as s:
        got = [s.prefill(ids)]
        s.prepare()
        for t in extra:
            got.append(s.step(t).clone())
    full = torch.cat([ids, torch.tensor([extra], device="cuda")], 1)
    with torch.no_grad():
        ref = model(full).logits[0].float()
    want = [ref[199 + i] for i in range(len(got))]
    for i, (a, b) in enumerate(zip(got, want)):
        a = a.float().reshape(-1)
        cos = torch.nn.functional.cosine_similarity(a, b, dim=0).item()
        assert cos > 0.999, f"step {i}: cosine {cos}"
        assert (a - b).abs().max().item() < 0.05 * b.abs().max().item(), f"step {i}"


def test_moba_model_graph_equals_eager(cuda_device):
    from moba_hip.qwen2 import Qwen2Session
    model = _model(seed=3)
    ids = _tokens(300, 3)
    extra = [int(x) for x in _tokens(12, 4)[0]]
    logits = {}
    for backend in ("eager", "model_graph"):
        with Qwen2Session(model, 400, mode="moba", chunk=32, topk=3, page=16,
                          backend=backend) as s:
            out = [s.prefill(ids)]
            s.prepare()
            for t in extra:
                out.append(s.step(t).clone())
                torch.randn(100, device="cuda").sum().item()  # eager work between replays
            logits[backend] = out
    for a, b in zip(logits["eager"], logits["model_graph"]):
        assert torch.equal(a, b)


def test_decode_layer_adapter_matches_oracle(cuda_device):
    from moba_hip import PagedKVCache
    from moba_hip.qwen2 import decode_layer, project_qkv
    model = _model(seed=5, layers=1)
    m = model.model
    layer = m.layers[0]
    cache = PagedKVCache(1, 512, 2, 64, page_size=16, chunk_size=32, dtype=torch.bfloat16)
    with torch.no_grad():
        h = m.embed_tokens(_tokens(129, 6))
        cos, sin = m.rotary_emb(h, torch.arange(129, device="cuda")[None])
        _, k, v = project_qkv(layer.self_attn, layer.input_layernorm(h[:, :128]), cos[:, :128],
                              sin[:, :128])
        cache.append(k, v, sequence_ids=[0], cu_seqlens=[0, 128])
        with cache.prepare_decode([0], 8, topk=3) as plan:
            out, result, q, _, _ = decode_layer(layer.self_attn, layer.input_layernorm,
                                                h[:, 128:], cos[:, 128:], sin[:, 128:], plan)
            check(cache, result, q)
            assert out.shape == (1, 512)  # [b*t, hidden], as the reference adapter
