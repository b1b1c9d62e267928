"""Fused per-layer glue of the paged Qwen3 target and D3D draft forwards.

* ``add_rmsnorm``     -- RMSDNorm.add_norm_forward / norm_forward
                         (serving/vendor/ssd/layers/layernorm.py:53-98)
* ``qk_rope_append``  -- q/k RMSHeadNorm (layernorm.py:1-52), rotary
                         embedding (serving/vendor/ssd/layers/rotary_embedding.py:6-16
                         for the target, models/d3d/modeling_d3d.py:164-187 for
                         the draft) and the KV-cache store of
                         serving/vendor/ssd/layers/attention.py:21-22, one launch
* ``silu_mul``        -- SiluAndMul (serving/vendor/ssd/layers/activation.py:6-14)
* ``project``         -- the decoder layer's F.linear for blocks of at most
                         64 rows (the qkv, o and down projections of a verify
                         or draft block), by a weight-streaming HIP GEMM whose
                         K-split partials ``add_rmsnorm`` and
                         ``qk_rope_append`` sum on the way in

Each is one gfx950 kernel; there is no CPU path.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Union

import torch
import torch.nn.functional as F

from . import _lib

ROWS64 = 64  # largest block project() runs on the HIP GEMM


@dataclass(frozen=True)
class SplitProduct:
    """x @ w.T as ``splits`` fp32 partial products over K ranges,
    ``parts`` [splits, M, N]; its value is bf16(sum of the splits in order)."""
    parts: torch.Tensor
    splits: int

    def __post_init__(self):
        # The consumers read splits x M x N floats from parts: a leading
        # dimension other than splits would send them past the allocation.
        if self.parts.ndim != 3 or self.splits < 1 or self.parts.shape[0] != self.splits:
            raise ValueError(f"split partials must be [splits={self.splits}, M, N], got {tuple(self.parts.shape)}")

    @property
    def shape(self):
        return self.parts.shape[1:]

    def value(self) -> torch.Tensor:
        """The bf16 product (the splits summed in order, then rounded)."""
        acc = self.parts[0].clone()
        for s in range(1, self.splits):
            acc += self.parts[s]
        return acc.to(torch.bfloat16)


Product = Union[torch.Tensor, SplitProduct]


def rows64_splits(N: int, K: int) -> int:
    """The split count project() runs d3d_gemm_rows64 with for a 64-row
    block times weight [N, K], or 0 where it uses hipBLASLt instead.

    The kernel holds two workgroups per CU (256 CUs); its grid is N / 64
    column tiles times the splits.  Grids of 128 to 256 workgroups and of
    exactly 512 are at least even with hipBLASLt on every 64-row projection
    of both models (graph-replayed, HBM-resident weights): the 6144 x 4096
    target qkv at 192 workgroups 16.6 against 17.5-18.3 us, the 12288 x 2048
    draft gate-up at 192 14.8-16.2 against 15.7 us on its tuned library
    solution and 17.2-18.2 on the default one.  A round and a half (the
    24576 x 4096 target gate-up at 384: 48.0 against 46.9 us) and smaller
    grids stay with hipBLASLt.
    """
    if N % 64 or K % 128:
        return 0
    splits = _lib.load().d3d_gemm_rows64_splits(N, K)
    grid = (N // 64) * splits
    return splits if 128 <= grid <= 256 or grid == 512 else 0


def project(x: torch.Tensor, weight: torch.Tensor) -> Product:
    """F.linear(x, weight) for bf16 x [M, K] and weight [N, K].

    Contiguous, 16-byte aligned blocks of at most 64 rows with N % 64 == 0
    and K % 128 == 0 run d3d_gemm_rows64 where rows64_splits says so; when
    it splits K the result is a SplitProduct for add_rmsnorm or
    qk_rope_append to consume.  Other shapes use F.linear (hipBLASLt).
    """
    M, K = x.shape
    N = weight.shape[0]
    if (M > ROWS64 or N % 64 or K % 128 or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16
            or not x.is_contiguous() or not weight.is_contiguous()
            or x.data_ptr() % 16 or weight.data_ptr() % 16):  # the kernel's 16-byte row loads
        return F.linear(x, weight)
    dev = _lib.require_device(x, weight)
    lib = _lib.load()
    splits = rows64_splits(N, K)
    if not splits:
        return F.linear(x, weight)
    if splits == 1:
        y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        st = lib.d3d_gemm_rows64(x.data_ptr(), weight.data_ptr(), y.data_ptr(), None, M, N, K, 1, _lib.stream_ptr(dev))
        _lib.check(st, "d3d_gemm_rows64")
        return y
    parts = torch.empty(splits, M, N, dtype=torch.float32, device=dev)
    st = lib.d3d_gemm_rows64(x.data_ptr(), weight.data_ptr(), None, parts.data_ptr(), M, N, K, splits,
                             _lib.stream_ptr(dev))
    _lib.check(st, "d3d_gemm_rows64")
    return SplitProduct(parts, splits)


def rows64_silu_ok(H: int, K: int) -> bool:
    """Whether gate_up_silu runs the fused d3d_gemm_rows64_silu_mul for a
    gate-up weight [2H, K] (its grid is 2H / 64 workgroups; the same grids
    as rows64_splits, and the step counts the kernel is built for)."""
    grid = 2 * H // 64
    return H % 32 == 0 and K % 128 == 0 and K // 128 in (8, 16, 24, 32, 48, 64) and (128 <= grid <= 256 or grid == 512)


def gate_up_silu(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """silu_mul(F.linear(x, weight)) for bf16 x [M, K] and a gate-up weight
    [2H, K] (gate rows, then up rows), the MLP's gate_up_proj + SiluAndMul.

    Blocks of at most 64 rows whose shape rows64_silu_ok accepts run one
    fused launch (d3d_gemm_rows64_silu_mul), equal bit for bit to
    d3d_gemm_rows64 followed by silu_mul; others run F.linear (hipBLASLt)
    and silu_mul."""
    M, K = x.shape
    H = weight.shape[0] // 2
    if (M > ROWS64 or weight.shape[0] % 2 or not rows64_silu_ok(H, K) or x.dtype != torch.bfloat16
            or weight.dtype != torch.bfloat16 or not x.is_contiguous() or not weight.is_contiguous()
            or x.data_ptr() % 16 or weight.data_ptr() % 16 or weight.shape[1] != K):
        return silu_mul(F.linear(x, weight))
    dev = _lib.require_device(x, weight)
    y = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    st = _lib.load().d3d_gemm_rows64_silu_mul(x.data_ptr(), weight.data_ptr(), y.data_ptr(), M, H, K,
                                              _lib.stream_ptr(dev))
    _lib.check(st, "d3d_gemm_rows64_silu_mul")
    return y


def _bf16_rows(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous bf16 tensor")


def add_rmsnorm(x: Optional[Product], residual: torch.Tensor, weight: torch.Tensor, eps: float,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out = RMSNorm(x + residual) * weight; residual <- bf16(x + residual) in place.

    With ``x`` None the residual is normalised as it is and not written.
    ``x`` may be a SplitProduct of ``project``.  Rows are the last dimension
    of ``residual`` (H <= 8192, H % 8 == 0).
    """
    if isinstance(x, SplitProduct):
        return _add_rmsnorm_parts(x, residual, weight, eps, out)
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


def qk_rope_append(qkv: Product, positions: torch.Tensor, q_norm: torch.Tensor, k_norm: torch.Tensor,
                   inv_freq: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   slot_mapping: torch.Tensor, heads: int, kv_heads: int, eps: float, *, draft_rope: bool,
                   q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Normalise and rotate q and k, store k and v in the paged cache; returns q [T, Hq, D].

    ``qkv`` [T, (Hq + 2 Hkv) * D] bf16, or a SplitProduct of ``project``;
    ``positions`` and ``slot_mapping`` [T] int64, caches
    [num_pages, page_size, Hkv, D] bf16.  Slots outside the cache are
    skipped.
    """
    split = qkv if isinstance(qkv, SplitProduct) else None
    src = split.parts if split is not None else qkv
    dev = _lib.require_device(src, positions, q_norm, k_norm, inv_freq, k_cache, v_cache, slot_mapping)
    if split is not None:
        if split.parts.dtype != torch.float32 or not split.parts.is_contiguous():
            raise ValueError("split partials must be contiguous fp32")
        if split.parts.shape[2] != (heads + 2 * kv_heads) * k_cache.shape[3]:
            raise ValueError("qkv row width must be (heads + 2 kv_heads) * head_dim")
        qkv = split.parts[0]
    else:
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
    lib = _lib.load()
    tail = (positions.data_ptr(), q_norm.data_ptr(), k_norm.data_ptr(), inv_freq.data_ptr(), q_out.data_ptr(),
            k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(), T, heads, kv_heads, D, float(eps),
            int(bool(draft_rope)), P * ps, _lib.stream_ptr(dev))
    if split is not None:
        st = lib.d3d_qk_rope_append_parts(split.parts.data_ptr(), split.splits, *tail)
        _lib.check(st, "d3d_qk_rope_append_parts")
    else:
        st = lib.d3d_qk_rope_append(qkv.data_ptr(), *tail)
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


def _add_rmsnorm_parts(x: SplitProduct, residual: torch.Tensor, weight: torch.Tensor, eps: float,
                       out: Optional[torch.Tensor]) -> torch.Tensor:
    dev = _lib.require_device(x.parts, residual, weight, out)
    _bf16_rows(residual, "residual")
    _bf16_rows(weight, "weight")
    H = residual.shape[-1]
    T = residual.numel() // H
    if weight.numel() != H:
        raise ValueError("weight must have one entry per hidden unit")
    if x.parts.dtype != torch.float32 or not x.parts.is_contiguous() or tuple(x.parts.shape) != (x.splits, T, H):
        raise ValueError("split partials must be contiguous fp32 [splits, T, H] matching the residual")
    if out is None:
        out = torch.empty_like(residual)
    else:
        _bf16_rows(out, "out")
        if out.shape != residual.shape:
            raise ValueError("out and residual shapes differ")
    st = _lib.load().d3d_add_rmsnorm_parts(x.parts.data_ptr(), x.splits, residual.data_ptr(), weight.data_ptr(),
                                           out.data_ptr(), T, H, float(eps), _lib.stream_ptr(dev))
    _lib.check(st, "d3d_add_rmsnorm_parts")
    return out
