"""Fused per-layer glue of the paged Qwen3 target and D3D draft forwards.

* ``add_rmsnorm``     -- RMSDNorm.add_norm_forward / norm_forward
                         (serving/vendor/ssd/layers/layernorm.py:53-98)
* ``qk_rope_append``  -- q/k RMSHeadNorm (layernorm.py:1-52), rotary
                         embedding (serving/vendor/ssd/layers/rotary_embedding.py:6-16
                         for the target, models/d3d/modeling_d3d.py:164-187 for
                         the draft) and the KV-cache store of
                         serving/vendor/ssd/layers/attention.py:21-22, one launch
* ``silu_mul``        -- SiluAndMul (serving/vendor/ssd/layers/activation.py:6-14)

Each is one gfx950 kernel; there is no CPU path.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import _lib


def _bf16_rows(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous bf16 tensor")


def add_rmsnorm(x: Optional[torch.Tensor], residual: torch.Tensor, weight: torch.Tensor, eps: float,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = RMSNorm(x + residual) * weight; residual <- bf16(x + residual) in place.

    With ``x`` None the residual is normalised as it is and not written.
    Rows are the last dimension of ``residual`` (H <= 8192, H % 8 == 0).
    """
    dev = _lib.require_device(x, residual, weight, out)
    _bf16_rows(residual, "residual")
    _bf16_rows(weight, "weight")
    H = residual.shape[-1]
    if weight.numel() != H:
        raise ValueError("weight must have one entry per hidden unit")
    if x is not None:
        _bf16_rows(x, "x")
        if x.shape != residual.shape:
            raise ValueError("x and residual shapes differ")
    if out is None:
        out = torch.empty_like(residual)
    else:
        _bf16_rows(out, "out")
        if out.shape != residual.shape:
            raise ValueError("out and residual shapes differ")
    T = residual.numel() // H
    st = _lib.load().d3d_add_rmsnorm(_lib.ptr(x), residual.data_ptr(), weight.data_ptr(), out.data_ptr(), T, H,
                                     float(eps), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_add_rmsnorm")
    return out


def qk_rope_append(qkv: torch.Tensor, positions: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor,
                   inv_freq: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   slot_mapping: torch.Tensor, heads: int, kv_heads: int, eps: float, *, draft_rope: bool,
                   q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Normalise and rotate q and k, store k and v in the paged cache; returns q [T, Hq, D].

    ``qkv`` [T, (Hq + 2 Hkv) * D] bf16, ``positions`` and ``slot_mapping``
    [T] int64, caches [num_pages, page_size, Hkv, D] bf16.  Slots outside
    the cache are skipped.
    """
    dev = _lib.require_device(qkv, positions, q_norm, k_norm, inv_freq, k_cache, v_cache, slot_mapping)
    _bf16_rows(qkv, "qkv")
    P, ps, Hkv, D = k_cache.shape
    if v_cache.shape != k_cache.shape or Hkv != kv_heads:
        raise ValueError("cache shapes do not match the model's kv heads")
    _bf16_rows(k_cache, "k_cache")
    _bf16_rows(v_cache, "v_cache")
    T = qkv.numel() // ((heads + 2 * kv_heads) * D)
    if qkv.numel() != T * (heads + 2 * kv_heads) * D:
        raise ValueError("qkv row width must be (heads + 2 kv_heads) * head_dim")
    if positions.dtype != torch.int64 or slot_mapping.dtype != torch.int64:
        raise ValueError("positions and slot_mapping must be int64")
    if positions.numel() != T or slot_mapping.numel() != T:
        raise ValueError("positions and slot_mapping need one entry per token")
    if inv_freq.dtype != torch.float32 or inv_freq.numel() != D // 2:
        raise ValueError("inv_freq must be fp32 [head_dim / 2]")
    if q_out is None:
        q_out = torch.empty(T, heads, D, dtype=torch.bfloat16, device=dev)
    st = _lib.load().d3d_qk_rope_append(
        qkv.data_ptr(), positions.data_ptr(), q_norm.data_ptr(), k_norm.data_ptr(), inv_freq.data_ptr(),
        q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(), T, heads, kv_heads, D,
        float(eps), int(bool(draft_rope)), P * ps, _lib.stream_ptr(dev))
    _lib.check(st, "d3d_qk_rope_append")
    return q_out


def silu_mul(gate_up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(gate) * up for gate_up [..., 2M] = [gate | up]; returns [..., M] bf16."""
    dev = _lib.require_device(gate_up, out)
    _bf16_rows(gate_up, "gate_up")
    M = gate_up.shape[-1] // 2
    if out is None:
        out = torch.empty(*gate_up.shape[:-1], M, dtype=torch.bfloat16, device=dev)
    T = gate_up.numel() // (2 * M)
    st = _lib.load().d3d_silu_mul(gate_up.data_ptr(), out.data_ptr(), T, M, _lib.stream_ptr(dev))
    _lib.check(st, "d3d_silu_mul")
    return out
