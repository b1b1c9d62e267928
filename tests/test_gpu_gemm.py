"""The 64-row weight-streaming GEMM and the kernels that sum its K splits (GPU).

* d3d_gemm_rows64 (through layers.project) against the fp64 product of the
  same bf16 operands, at the qkv / o / gate-up / down shapes of the Qwen3-8B
  target and the Qwen3-1.7B draft and at 1, 5, 37 and 64 rows.  Bound per
  entry: one bf16 step of the exact value (the final rounding) plus
  2 K 2^-24 sum_k |x_k w_k|, twice the classical error bound of an fp32 sum
  of K products in any order -- so a misplaced tile or a stale stage fails,
  while the kernel's own summation order passes.
* Every split count gives the same product to fp32 rounding, and the splits
  of a given count always sum to the same bits; k-step counts outside the
  register-staged kernel's unrolled set (the direct-to-LDS kernel) meet the
  same bound.
* d3d_gemm_rows64_silu_mul equals d3d_gemm_rows64 followed by silu_mul bit
  for bit.
* d3d_add_rmsnorm_parts and d3d_qk_rope_append_parts equal the bf16 kernels
  fed bf16(sum of the splits in order) -- the SplitProduct's value -- bit for
  bit, residual and cache included.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from d3d_amd import _lib
from d3d_amd import layers as ly

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
BF = torch.bfloat16

SHAPES = {  # name: (N, K)
    "target_qkv": (6144, 4096), "target_o": (4096, 4096), "target_gate_up": (24576, 4096),
    "target_down": (4096, 12288), "draft_qkv": (4096, 2048), "draft_o": (2048, 2048),
    "draft_gate_up": (12288, 2048), "draft_down": (2048, 6144),
}


def _operands(M, N, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=DEV).to(BF)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(BF)
    return x, w


def _reference(x: torch.Tensor, w: torch.Tensor):
    """fp64 product and the per-entry bound of the module docstring."""
    K = x.shape[1]
    ref = x.double() @ w.double().T
    slack = (x.double().abs() @ w.double().abs().T) * (2.0 * K * 2.0 ** -24)
    ulp = torch.clamp(ref.abs(), min=2.0 ** -100).log2().floor().exp2() * 2.0 ** -7
    return ref, ulp + slack


def _within(y: torch.Tensor, ref_bound):
    ref, bound = ref_bound
    err = (y.double() - ref).abs()
    assert bool((err <= bound).all()), float((err / bound).max())


@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("M", [1, 5, 37, 64])
def test_rows64_matches_exact_product(name, M):
    N, K = SHAPES[name]
    x, w = _operands(M, N, K, seed=M * 31 + N + K)
    got = ly.project(x, w)
    y = got.value() if isinstance(got, ly.SplitProduct) else got
    assert y.shape == (M, N) and y.dtype == BF
    _within(y, _reference(x, w))


@pytest.mark.parametrize("N,K", [(4096, 12288), (2048, 2048)])
def test_every_split_count_agrees(N, K):
    lib = _lib.load()
    M = 64
    x, w = _operands(M, N, K, seed=7)
    st = torch.cuda.current_stream(DEV).cuda_stream
    y1 = torch.empty(M, N, dtype=BF, device=DEV)
    assert lib.d3d_gemm_rows64(x.data_ptr(), w.data_ptr(), y1.data_ptr(), None, M, N, K, 1, st) == 0
    rb = _reference(x, w)
    _within(y1, rb)
    for s in (2, 4, 8, 16):
        if K % (128 * s):
            continue
        parts = torch.empty(s, M, N, dtype=torch.float32, device=DEV)
        for rep in range(2):
            assert lib.d3d_gemm_rows64(x.data_ptr(), w.data_ptr(), None, parts.data_ptr(), M, N, K, s, st) == 0
            total = ly.SplitProduct(parts, s).value()
            if rep == 0:
                first = total.clone()
            else:
                assert torch.equal(total, first), s
        _within(total, rb)


@pytest.mark.parametrize("K,splits", [(640, 1), (1280, 1), (1280, 2), (128 * 7 * 4, 4), (128 * 48, 1)])
@pytest.mark.parametrize("M", [1, 37, 64])
def test_step_counts_outside_the_unrolled_set(K, splits, M):
    """k-step counts per split (5, 10, 7, 48) that the register-staged kernel
    is not unrolled for run on the direct-to-LDS kernel: same bound."""
    lib = _lib.load()
    N = 256
    x, w = _operands(M, N, K, seed=K + splits + M)
    st = torch.cuda.current_stream(DEV).cuda_stream
    if splits == 1:
        y = torch.empty(M, N, dtype=BF, device=DEV)
        assert lib.d3d_gemm_rows64(x.data_ptr(), w.data_ptr(), y.data_ptr(), None, M, N, K, 1, st) == 0
    else:
        parts = torch.empty(splits, M, N, dtype=torch.float32, device=DEV)
        assert lib.d3d_gemm_rows64(x.data_ptr(), w.data_ptr(), None, parts.data_ptr(), M, N, K, splits, st) == 0
        y = ly.SplitProduct(parts, splits).value()
    _within(y, _reference(x, w))


@pytest.mark.parametrize("H,K", [(6144, 2048), (12288, 4096), (256, 1024)])
@pytest.mark.parametrize("M", [1, 5, 37, 64])
def test_fused_gate_up_silu_equals_the_two_kernels(H, K, M):
    """d3d_gemm_rows64_silu_mul equals d3d_gemm_rows64 (one split) on the
    gate-up weight followed by silu_mul, bit for bit, and the product stays
    within the exact-product bound."""
    lib = _lib.load()
    x, w = _operands(M, 2 * H, K, seed=H + K + M)
    st = torch.cuda.current_stream(DEV).cuda_stream
    gu = torch.empty(M, 2 * H, dtype=BF, device=DEV)
    assert lib.d3d_gemm_rows64(x.data_ptr(), w.data_ptr(), gu.data_ptr(), None, M, 2 * H, K, 1, st) == 0
    want = ly.silu_mul(gu)
    got = torch.empty(M, H, dtype=BF, device=DEV)
    assert lib.d3d_gemm_rows64_silu_mul(x.data_ptr(), w.data_ptr(), got.data_ptr(), M, H, K, st) == 0
    assert torch.equal(got, want)
    _within(gu, _reference(x, w))
    if ly.rows64_silu_ok(H, K):
        assert torch.equal(ly.gate_up_silu(x, w), want)
    else:
        assert torch.equal(ly.gate_up_silu(x, w), ly.silu_mul(F.linear(x, w)))


def test_split_sum_kernels_equal_bf16_path():
    T, H = 64, 4096
    g = torch.Generator(device=DEV).manual_seed(3)
    x, w = _operands(T, H, 4096, seed=11)
    prod = ly.project(x, w)
    assert isinstance(prod, ly.SplitProduct) and prod.splits > 1
    r0 = (torch.randn(T, H, generator=g, device=DEV) * 2).to(BF)
    nw = (1 + 0.1 * torch.randn(H, generator=g, device=DEV)).to(BF)
    ra, rb = r0.clone(), r0.clone()
    out_a = ly.add_rmsnorm(prod, ra, nw, 1e-6)
    out_b = ly.add_rmsnorm(prod.value(), rb, nw, 1e-6)
    assert torch.equal(ra, rb) and torch.equal(out_a, out_b)

    Hq, Hkv, D = 16, 8, 128  # the draft's qkv: 4096 x 2048, split 4 ways
    K = 2048
    xq, wq = _operands(T, (Hq + 2 * Hkv) * D, K, seed=13)
    qkv = ly.project(xq, wq)
    assert isinstance(qkv, ly.SplitProduct)
    pages, ps = 8, 16
    pos = torch.arange(100, 100 + T, device=DEV)
    slots = torch.randperm(pages * ps, device=DEV)[:T]
    qn = (1 + 0.1 * torch.randn(D, generator=g, device=DEV)).to(BF)
    kn = (1 + 0.1 * torch.randn(D, generator=g, device=DEV)).to(BF)
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, D // 2, device=DEV, dtype=torch.float32) * 2 / D))
    for draft_rope in (False, True):
        caches = []
        qs = []
        for src in (qkv, qkv.value()):
            kc = torch.zeros(pages, ps, Hkv, D, dtype=BF, device=DEV)
            vc = torch.zeros_like(kc)
            qs.append(ly.qk_rope_append(src, pos, qn, kn, inv_freq, kc, vc, slots, Hq, Hkv, 1e-6,
                                        draft_rope=draft_rope))
            caches.append((kc, vc))
        assert torch.equal(qs[0], qs[1])
        assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])


def test_project_falls_back_beyond_64_rows_and_odd_shapes():
    x, w = _operands(65, 2048, 2048, seed=5)
    y = ly.project(x, w)
    assert isinstance(y, torch.Tensor) and torch.equal(y, F.linear(x, w))
    x2, w2 = _operands(16, 2000, 2048, seed=6)  # N not a multiple of 64
    assert torch.equal(ly.project(x2, w2), F.linear(x2, w2))
    # a round and a half of workgroups goes to hipBLASLt
    x3, w3 = _operands(64, 24576, 4096, seed=7)  # 384 tiles x 1 split
    assert torch.equal(ly.project(x3, w3), F.linear(x3, w3))
    x6, w6 = _operands(64, 6144, 4096, seed=9)  # 96 tiles x 2 splits: the HIP GEMM
    assert isinstance(ly.project(x6, w6), ly.SplitProduct)
    x4, w4 = _operands(64, 2048, 6144, seed=8)  # 32 tiles x 8 splits
    assert isinstance(ly.project(x4, w4), ly.SplitProduct)
    # a contiguous view 2 bytes off 16-byte alignment
    buf = torch.empty(64 * 6144 + 1, dtype=BF, device=DEV)
    x5 = buf[1:].view(64, 6144)
    x5.copy_(x4)
    y5 = ly.project(x5, w4)
    assert isinstance(y5, torch.Tensor) and torch.equal(y5, F.linear(x5, w4))
