"""ORACLE -- test infrastructure only.

fp32 torch-CPU restatement of the Qwen3-shaped target and D3D draft
forwards over a contiguous (unpaged) KV history with explicit attention
masks, used to check the paged model plumbing: slot mapping, page tables,
positions and the RoPE applied to cached keys.

Follows serving/vendor/ssd/models/qwen3.py:14-325 (target: RMSNorm in fp32,
rotary in fp32) and models/d3d/modeling_d3d.py:111-432 (draft: RoPE with
cos/sin in the activation dtype), computed here entirely in fp32.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope(x, pos, inv_freq):
    freqs = pos.float()[:, None] * inv_freq[None, :]
    cos, sin = freqs.cos()[:, None, :], freqs.sin()[:, None, :]
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1)


def weights_fp32(model):
    """Copy a Qwen3PagedModel's weights to fp32 CPU tensors."""
    cv = lambda t: t.detach().float().cpu()
    return dict(embed=cv(model.embed), norm=cv(model.norm), lm_head=cv(model.lm_head),
                inv_freq=cv(model.inv_freq), layers=[{k: cv(v) for k, v in L.items()} for L in model.layers])


def forward(W, shape, ids, positions, mask):
    """Logits [T, V] for tokens ids [T] at positions [T]; mask [T, T] bool (query, key)."""
    Hq, Hkv, d = shape.heads, shape.kv_heads, shape.head_dim
    x = W["embed"][ids]
    residual = None
    for L in W["layers"]:
        residual = x if residual is None else residual + x
        hs = _rms(residual, L["ln1"], shape.eps)
        q, k, v = (hs @ L["qkv"].T).split([Hq * d, Hkv * d, Hkv * d], -1)
        q = _rope(_rms(q.reshape(-1, Hq, d), L["qn"], shape.eps), positions, W["inv_freq"])
        k = _rope(_rms(k.reshape(-1, Hkv, d), L["kn"], shape.eps), positions, W["inv_freq"])
        v = v.reshape(-1, Hkv, d)
        G = Hq // Hkv
        kk = k.repeat_interleave(G, 1).transpose(0, 1)
        vv = v.repeat_interleave(G, 1).transpose(0, 1)
        o = F.scaled_dot_product_attention(q.transpose(0, 1), kk, vv, attn_mask=mask, scale=d ** -0.5)
        x = o.transpose(0, 1).reshape(-1, Hq * d) @ L["o"].T
        residual = residual + x
        hs = _rms(residual, L["ln2"], shape.eps)
        gate, up = (hs @ L["gate_up"].T).chunk(2, -1)
        x = (F.silu(gate) * up) @ L["down"].T
    return _rms(residual + x, W["norm"], shape.eps) @ W["lm_head"].T


def causal_then_block(prefix: int, block: int, bidirectional: bool):
    """Mask over prefix + block tokens: causal prefix, block causal or bidirectional."""
    T = prefix + block
    m = torch.ones(T, T).tril().bool()
    if bidirectional:
        m[prefix:, :] = True
    return m


def random_layer(shape, seed: int = 0):
    """fp32 weights of one decoder layer of ``shape`` (CPU), for timing."""
    g = torch.Generator().manual_seed(seed)
    h, d, Hq, Hkv = shape.hidden, shape.head_dim, shape.heads, shape.kv_heads
    w = lambda *dims: torch.randn(*dims, generator=g) * 0.02
    return dict(qkv=w((Hq + 2 * Hkv) * d, h), o=w(h, Hq * d), gate_up=w(2 * shape.mlp, h), down=w(h, shape.mlp),
                ln1=torch.ones(h), ln2=torch.ones(h), qn=torch.ones(d), kn=torch.ones(d))


def layer_step(L, shape, inv_freq, x, residual, pos, k_past, v_past, mask):
    """One decoder layer (the op sequence of ``forward``) over new rows x
    [T, h] attending to cached keys/values [P, Hkv, d] plus their own, under
    mask [T, P + T]; returns (x, residual) for the next layer."""
    Hq, Hkv, d = shape.heads, shape.kv_heads, shape.head_dim
    residual = x if residual is None else residual + x
    hs = _rms(residual, L["ln1"], shape.eps)
    q, k, v = (hs @ L["qkv"].T).split([Hq * d, Hkv * d, Hkv * d], -1)
    q = _rope(_rms(q.reshape(-1, Hq, d), L["qn"], shape.eps), pos, inv_freq)
    k = _rope(_rms(k.reshape(-1, Hkv, d), L["kn"], shape.eps), pos, inv_freq)
    v = v.reshape(-1, Hkv, d)
    k = torch.cat([k_past, k])
    v = torch.cat([v_past, v])
    G = Hq // Hkv
    kk = k.repeat_interleave(G, 1).transpose(0, 1)
    vv = v.repeat_interleave(G, 1).transpose(0, 1)
    o = F.scaled_dot_product_attention(q.transpose(0, 1), kk, vv, attn_mask=mask, scale=d ** -0.5)
    x = o.transpose(0, 1).reshape(-1, Hq * d) @ L["o"].T
    residual = residual + x
    hs = _rms(residual, L["ln2"], shape.eps)
    gate, up = (hs @ L["gate_up"].T).chunk(2, -1)
    return (F.silu(gate) * up) @ L["down"].T, residual
