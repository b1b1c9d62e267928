"""The model oracle (oracle/model_ref.py) pinned on the CPU.

* against transformers' Qwen3ForCausalLM (the architecture the reference's
  target and draft share: serving/vendor/ssd/models/qwen3.py,
  models/d3d/modeling_d3d.py) with random weights copied in, under the
  target's causal mask, the draft's prefix-causal + bidirectional-block mask
  (serving/engine.py:41-42) and shifted positions;
* by closed forms: RMSNorm of a constant vector, RoPE's relative-position
  invariance and its norm preservation, GQA equal to explicitly repeated KV
  heads, and the mask helper's row counts.

Random (not unit) norm weights, distinct q/k/v/gate/up blocks and Hq != Hkv
make a swapped projection block, a wrong rotation half, a wrong GQA head map
or a dropped norm fail the comparison.
"""
from __future__ import annotations

import math

import pytest
import torch

from d3d_amd.model import ModelShape
from oracle import model_ref

transformers = pytest.importorskip("transformers")

SHAPE = ModelShape(layers=2, hidden=64, heads=4, kv_heads=2, head_dim=16, mlp=96, vocab=100)


def _hf_model(seed: int, shape: ModelShape = SHAPE):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    cfg = Qwen3Config(vocab_size=shape.vocab, hidden_size=shape.hidden, intermediate_size=shape.mlp,
                      num_hidden_layers=shape.layers, num_attention_heads=shape.heads,
                      num_key_value_heads=shape.kv_heads, head_dim=shape.head_dim, rope_theta=shape.rope_theta,
                      rms_norm_eps=shape.eps, tie_word_embeddings=False, attention_bias=False,
                      max_position_embeddings=1024)
    torch.manual_seed(seed)
    m = Qwen3ForCausalLM(cfg).eval()
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in m.named_parameters():
            if p.ndim == 1:  # norm weights: random around 1
                p.copy_(1.0 + 0.3 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.08 * torch.randn(p.shape, generator=g))
    return m


def _weights(m, shape: ModelShape = SHAPE):
    """The oracle's weight dict from the transformers module."""
    sd = {k: v.detach().float() for k, v in m.state_dict().items()}
    d = shape.head_dim
    half = d // 2
    layers = []
    for i in range(shape.layers):
        p = f"model.layers.{i}."
        layers.append(dict(
            qkv=torch.cat([sd[p + "self_attn.q_proj.weight"], sd[p + "self_attn.k_proj.weight"],
                           sd[p + "self_attn.v_proj.weight"]]),
            o=sd[p + "self_attn.o_proj.weight"],
            gate_up=torch.cat([sd[p + "mlp.gate_proj.weight"], sd[p + "mlp.up_proj.weight"]]),
            down=sd[p + "mlp.down_proj.weight"],
            ln1=sd[p + "input_layernorm.weight"], ln2=sd[p + "post_attention_layernorm.weight"],
            qn=sd[p + "self_attn.q_norm.weight"], kn=sd[p + "self_attn.k_norm.weight"]))
    inv_freq = 1.0 / (shape.rope_theta ** (torch.arange(0, half, dtype=torch.float32) * 2 / d))
    return dict(embed=sd["model.embed_tokens.weight"], norm=sd["model.norm.weight"], lm_head=sd["lm_head.weight"],
                inv_freq=inv_freq, layers=layers)


@pytest.mark.parametrize("prefix,block,bidirectional,shift", [(0, 12, False, 0), (9, 7, False, 5),
                                                              (10, 6, True, 0), (24, 16, True, 37)])
def test_model_ref_matches_transformers_qwen3(prefix, block, bidirectional, shift):
    m = _hf_model(prefix + block + shift)
    W = _weights(m)
    T = prefix + block
    ids = torch.randint(0, SHAPE.vocab, (T,), generator=torch.Generator().manual_seed(T))
    pos = torch.arange(T) + shift
    mask = model_ref.causal_then_block(prefix, block, bidirectional)
    with torch.no_grad():
        ref = m(ids[None], attention_mask=mask[None, None], position_ids=pos[None]).logits[0]
        got = model_ref.forward(W, SHAPE, ids, pos, mask)
    err = (got - ref).abs().max().item()
    assert err <= 2e-5 * max(ref.abs().max().item(), 1.0), err


def _layer_step_logits(W, shape, ids_new, pos_new, past, mask_new):
    """Chains model_ref.layer_step over every layer for the new rows, each
    layer attending to its cached prefix keys/values ``past[l]``, then the
    final norm and LM head."""
    x, residual = W["embed"][ids_new], None
    for L, (kp, vp) in zip(W["layers"], past):
        x, residual = model_ref.layer_step(L, shape, W["inv_freq"], x, residual, pos_new, kp, vp, mask_new)
    return model_ref._rms(residual + x, W["norm"], shape.eps) @ W["lm_head"].T


@pytest.mark.parametrize("layers,prefix,block,shift", [(1, 9, 7, 0), (2, 24, 16, 37), (2, 1, 5, 3)])
def test_layer_step_matches_transformers_with_cached_prefix(layers, prefix, block, shift):
    """layer_step (the CPU-baseline workload) against transformers' Qwen3:
    the prefix runs through transformers with its KV cache kept, the cache's
    per-layer keys (after k_norm and RoPE) and values feed layer_step for the
    new rows, and the chained result must equal transformers' logits of the
    whole sequence on those rows (causal), and model_ref.forward's under the
    prefix-causal + bidirectional-block mask."""
    shape = ModelShape(layers=layers, hidden=64, heads=4, kv_heads=2, head_dim=16, mlp=96, vocab=100)
    m = _hf_model(100 + prefix + block, shape)
    W = _weights(m, shape)
    T = prefix + block
    ids = torch.randint(0, shape.vocab, (T,), generator=torch.Generator().manual_seed(T + 1))
    pos = torch.arange(T) + shift
    with torch.no_grad():
        cache = m(ids[None, :prefix], position_ids=pos[None, :prefix], use_cache=True).past_key_values
        past = [(c.keys[0].transpose(0, 1).float(), c.values[0].transpose(0, 1).float()) for c in cache.layers]
        assert past[0][0].shape == (prefix, shape.kv_heads, shape.head_dim)
        for bidirectional in (False, True):
            mask = model_ref.causal_then_block(prefix, block, bidirectional)
            got = _layer_step_logits(W, shape, ids[prefix:], pos[prefix:], past, mask[prefix:])
            if bidirectional:
                ref = model_ref.forward(W, shape, ids, pos, mask)[prefix:]
            else:
                ref = m(ids[None], position_ids=pos[None]).logits[0, prefix:]
            err = (got - ref).abs().max().item()
            assert err <= 2e-5 * max(ref.abs().max().item(), 1.0), (bidirectional, err)


def test_layer_step_fails_with_a_shifted_cache():
    """Negative control: prefix keys cached one position off must break the match."""
    shape = ModelShape(layers=1, hidden=64, heads=4, kv_heads=2, head_dim=16, mlp=96, vocab=100)
    m = _hf_model(11, shape)
    W = _weights(m, shape)
    prefix, block = 8, 6
    ids = torch.arange(prefix + block) * 3 % shape.vocab
    pos = torch.arange(prefix + block)
    with torch.no_grad():
        c = m(ids[None, :prefix], position_ids=pos[None, :prefix] + 1, use_cache=True).past_key_values.layers[0]
        past = [(c.keys[0].transpose(0, 1).float(), c.values[0].transpose(0, 1).float())]
        mask = model_ref.causal_then_block(prefix, block, False)[prefix:]
        got = _layer_step_logits(W, shape, ids[prefix:], pos[prefix:], past, mask)
        ref = m(ids[None], position_ids=pos[None]).logits[0, prefix:]
    assert (got - ref).abs().max().item() > 1e-3


def test_model_ref_fails_with_a_swapped_projection():
    """Negative control: gate and up swapped in one layer must break the match."""
    m = _hf_model(3)
    W = _weights(m)
    L = W["layers"][1]
    gate, up = L["gate_up"].chunk(2)
    L["gate_up"] = torch.cat([up, gate])
    T = 10
    ids = torch.arange(T) * 7 % SHAPE.vocab
    mask = model_ref.causal_then_block(0, T, False)
    with torch.no_grad():
        ref = m(ids[None], attention_mask=mask[None, None]).logits[0]
        got = model_ref.forward(W, SHAPE, ids, torch.arange(T), mask)
    assert (got - ref).abs().max().item() > 1e-3


def test_rmsnorm_closed_form():
    x = torch.full((3, 8), 2.0)
    w = torch.arange(1.0, 9.0)
    eps = 1e-6
    want = 2.0 / math.sqrt(4.0 + eps) * w
    assert torch.allclose(model_ref._rms(x, w, eps), want.expand(3, 8), rtol=1e-6, atol=0)


def test_rope_relative_position_invariance_and_norm():
    g = torch.Generator().manual_seed(0)
    d = 16
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, d // 2, dtype=torch.float32) * 2 / d))
    q = torch.randn(5, 2, d, generator=g, dtype=torch.float64)
    k = torch.randn(5, 2, d, generator=g, dtype=torch.float64)
    p_q = torch.tensor([0, 3, 17, 100, 511])
    p_k = torch.tensor([0, 1, 9, 40, 500])

    def rope64(x, pos):
        freqs = pos.double()[:, None] * inv_freq.double()[None, :]
        cos, sin = freqs.cos()[:, None, :], freqs.sin()[:, None, :]
        x1, x2 = x.chunk(2, dim=-1)
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1)

    # The oracle's rotation (fp32) equals the float64 closed form ...
    assert torch.allclose(model_ref._rope(q.float(), p_q, inv_freq).double(), rope64(q, p_q), atol=2e-5)
    # ... which depends only on position differences and preserves norms.
    a = (rope64(q, p_q) * rope64(k, p_k)).sum(-1)
    b = (rope64(q, p_q + 1234) * rope64(k, p_k + 1234)).sum(-1)
    assert torch.allclose(a, b, atol=1e-9)
    assert torch.allclose(rope64(q, p_q).norm(dim=-1), q.norm(dim=-1), atol=1e-12)


def test_gqa_equals_repeated_kv_heads():
    """An Hkv=2 model equals the Hkv=4 model whose KV heads are the 2 heads
    repeated per query group (head h reads KV head h // (Hq / Hkv))."""
    m = _hf_model(5)
    W = _weights(m)
    d = SHAPE.head_dim
    full = ModelShape(layers=SHAPE.layers, hidden=SHAPE.hidden, heads=4, kv_heads=4, head_dim=d, mlp=SHAPE.mlp,
                      vocab=SHAPE.vocab)
    W2 = dict(W, layers=[])
    for L in W["layers"]:
        q, k, v = L["qkv"].split([4 * d, 2 * d, 2 * d])
        rep = lambda t: t.reshape(2, d, -1).repeat_interleave(2, 0).reshape(4 * d, -1)
        W2["layers"].append(dict(L, qkv=torch.cat([q, rep(k), rep(v)])))
    T = 14
    ids = torch.arange(T) * 5 % SHAPE.vocab
    mask = model_ref.causal_then_block(6, 8, True)
    a = model_ref.forward(W, SHAPE, ids, torch.arange(T), mask)
    b = model_ref.forward(W2, full, ids, torch.arange(T), mask)
    assert torch.allclose(a, b, atol=1e-5)


@pytest.mark.parametrize("prefix,block", [(0, 5), (7, 16)])
def test_causal_then_block_row_counts(prefix, block):
    for bidirectional in (False, True):
        m = model_ref.causal_then_block(prefix, block, bidirectional)
        counts = m.sum(1).tolist()
        T = prefix + block
        want = [i + 1 for i in range(prefix)] + [T if bidirectional else prefix + j + 1 for j in range(block)]
        assert counts == want
        # every row is a prefix of the columns (a single interval from 0)
        for r in range(T):
            assert m[r, :counts[r]].all() and not m[r, counts[r]:].any()
