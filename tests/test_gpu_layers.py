"""Fused layer kernels against fp32 torch restatements of the reference's ops (GPU).

The restatements follow the reference's operation order and casts:
RMSDNorm.add_norm_forward (serving/vendor/ssd/layers/layernorm.py:76-87),
RMSHeadNorm + apply_rotary_emb (layernorm.py:17-26,
serving/vendor/ssd/layers/rotary_embedding.py:6-16), the draft's HF RoPE with
bf16 cos/sin (models/d3d/modeling_d3d.py:164-187) and SiluAndMul.  The
residual and the cache copies are bit-exact; normalised and rotated values
may differ by one bf16 rounding step (fp32 sums in another order, rsqrt
and exp on the device): at most 2 ulp anywhere and 1 ulp on >= 99 % of
entries.  Where a rotation cancels, one such step in a rotated input (or,
for the draft's RoPE, in a bf16-rounded cos / sin) moves a tiny result by
many of its own ulps; the rotation tests add that propagated step, entry by
entry, as slack.
"""
from __future__ import annotations

import pytest
import torch

from d3d_amd import layers as ly

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
BF = torch.bfloat16


def _ulp_close(got: torch.Tensor, ref32: torch.Tensor, max_ulp: int = 2, frac_one: float = 0.99,
               atol=0.0):
    """got (bf16) within max_ulp bf16 steps (+ atol, a number or a per-entry
    tensor) of ref32 rounded to bf16, and within one step on at least
    frac_one of the entries."""
    ref = ref32.to(BF).float()
    got = got.float().cpu()
    ulp = torch.clamp(ref.abs(), min=2.0 ** -126).log2().floor().exp2() * 2.0 ** -7
    err = (got - ref).abs()
    assert bool((err <= max_ulp * ulp + atol).all()), float(((err - atol) / ulp).max())
    assert (err <= ulp + atol).float().mean() >= frac_one


def _rms_ref(s32, w, eps):
    # x.float() ... x.to(bf16).mul_(weight): bf16 normalised value times the weight, rounded
    n = (s32 * torch.rsqrt(s32.pow(2).mean(-1, keepdim=True) + eps)).to(BF).float()
    return n * w.float()


@pytest.mark.parametrize("T,H", [(1, 2048), (37, 4096), (128, 2048), (1088, 2048), (5, 8192), (3, 264)])
@pytest.mark.parametrize("with_x", [False, True])
def test_add_rmsnorm(T, H, with_x):
    g = torch.Generator().manual_seed(T * 7 + H)
    r = (torch.randn(T, H, generator=g) * 3).to(BF)
    x = (torch.randn(T, H, generator=g)).to(BF) if with_x else None
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(BF)
    rd = r.to(DEV)
    out = ly.add_rmsnorm(x.to(DEV) if with_x else None, rd, w.to(DEV), 1e-6)
    s32 = r.float() + (x.float() if with_x else 0.0)
    assert torch.equal(rd.cpu(), s32.to(BF)), "residual must be bf16(x + residual) bit for bit"
    _ulp_close(out, _rms_ref(s32, w, 1e-6))


def test_add_rmsnorm_zero_rows_and_bad_shapes():
    r = torch.zeros(0, 256, dtype=BF, device=DEV)
    w = torch.ones(256, dtype=BF, device=DEV)
    assert ly.add_rmsnorm(None, r, w, 1e-6).shape == (0, 256)
    with pytest.raises(ValueError):
        ly.add_rmsnorm(None, torch.zeros(2, 12, dtype=BF, device=DEV), torch.ones(12, dtype=BF, device=DEV), 1e-6)
    with pytest.raises(ValueError):
        ly.add_rmsnorm(None, torch.zeros(2, 16384, dtype=BF, device=DEV),
                       torch.ones(16384, dtype=BF, device=DEV), 1e-6)
    # an all-zero row normalises to zero (rsqrt(eps) * 0)
    z = torch.zeros(1, 512, dtype=BF, device=DEV)
    assert torch.count_nonzero(ly.add_rmsnorm(None, z, torch.ones(512, dtype=BF, device=DEV), 1e-6)) == 0


def test_unaligned_rows_are_rejected():
    """add_rmsnorm and silu_mul move 16-byte vectors: a row pointer off a
    16-byte boundary is refused with an argument error instead of being read."""
    buf = torch.zeros(2 * 512 + 8, dtype=BF, device=DEV)
    r = buf[1:1 + 2 * 512].view(2, 512)  # 2-byte offset, still contiguous
    with pytest.raises(ValueError):
        ly.add_rmsnorm(None, r, torch.ones(512, dtype=BF, device=DEV), 1e-6)
    with pytest.raises(ValueError):
        ly.silu_mul(buf[1:1 + 2 * 16].view(2, 16))


def _cos_sin(pos, inv_freq):
    """cos/sin of positions * inv_freq computed on the device in fp32, as the
    reference builds its rotary cache (rotary_embedding.py:19-60)."""
    f = pos.to(DEV).float()[:, None] * inv_freq.to(DEV)[None, :]
    return f.cos().cpu()[:, None, :], f.sin().cpu()[:, None, :]


def _rope_ref(y, pos, inv_freq, draft):
    """y [T, H, D] fp32 holding bf16 values -> rotated, fp32 holding bf16 values."""
    cos, sin = _cos_sin(pos, inv_freq)
    y1, y2 = y.chunk(2, -1)
    if draft:
        c, s_ = cos.to(BF).float(), sin.to(BF).float()
        r = lambda t: t.to(BF).float()
        return torch.cat([r(r(y1 * c) + r(-y2 * s_)), r(r(y2 * c) + r(y1 * s_))], -1)
    return torch.cat([y1 * cos - y2 * sin, y2 * cos + y1 * sin], -1)


def _bf_ulp(v):
    return torch.clamp(v.abs(), min=2.0 ** -126).log2().floor().exp2() * 2.0 ** -7


def _rope_slack(y, pos, inv_freq, draft):
    """Per-entry change of the rotated value when one rotated input moves by
    one bf16 step (and, with draft RoPE, when cos or sin rounds to the other
    neighbouring bf16 value), to first order.  y is [T, H, D] as in _rope_ref."""
    cos, sin = _cos_sin(pos, inv_freq)
    y1, y2 = y.chunk(2, -1)
    c, s_ = cos.abs(), sin.abs()
    s1 = _bf_ulp(y1) * c + _bf_ulp(y2) * s_
    s2 = _bf_ulp(y2) * c + _bf_ulp(y1) * s_
    if draft:
        uc, us = _bf_ulp(cos), _bf_ulp(sin)
        s1 = s1 + uc * y1.abs() + us * y2.abs()
        s2 = s2 + uc * y2.abs() + us * y1.abs()
    return torch.cat([s1, s2], -1)


@pytest.mark.parametrize("draft", [False, True])
# 8 + 2 x 2 heads leave a partly empty workgroup; 1088 is the packed draft
# block of four requests.
@pytest.mark.parametrize("Hq,Hkv,T", [(32, 8, 128), (16, 8, 16), (8, 2, 3), (32, 8, 300), (8, 2, 257),
                                      (16, 8, 1088)])
def test_qk_rope_append(draft, Hq, Hkv, T):
    D, ps = 128, 16
    P = max(32, -(-T // ps) + 4)
    g = torch.Generator().manual_seed(Hq * 131 + T + draft)
    qkv = (torch.randn(T, (Hq + 2 * Hkv) * D, generator=g) * 2).to(BF)
    pos = torch.randint(0, 40000, (T,), generator=g)
    slots = torch.randperm(P * ps, generator=g)[:T]
    if T > 2:
        slots[1] = -1  # skipped
    qn = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
    kn = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
    inv_freq = 1.0 / (1_000_000.0 ** (torch.arange(0, D // 2, dtype=torch.float32) * 2 / D))
    kc = torch.zeros(P, ps, Hkv, D, dtype=BF, device=DEV)
    vc = torch.zeros_like(kc)
    q = ly.qk_rope_append(qkv.to(DEV), pos.to(DEV), qn.to(DEV), kn.to(DEV), inv_freq.to(DEV), kc, vc,
                          slots.to(DEV), Hq, Hkv, 1e-6, draft_rope=draft)
    q_in, k_in, v_in = qkv.float().split([Hq * D, Hkv * D, Hkv * D], -1)
    qh = _rms_ref(q_in.reshape(T, Hq, D), qn, 1e-6).to(BF).float()
    kh = _rms_ref(k_in.reshape(T, Hkv, D), kn, 1e-6).to(BF).float()
    # Slack: one bf16 step of a rotated input (or of the draft's bf16 cos /
    # sin) carried through the rotation, plus 2^-20 of the largest entry for
    # fp32 contraction where a result cancels to nearly zero.
    floor = 2.0 ** -20 * float(qkv.float().abs().max())
    _ulp_close(q.reshape(T, Hq, D), _rope_ref(qh, pos, inv_freq, draft),
               atol=_rope_slack(qh, pos, inv_freq, draft) + floor)
    kflat, vflat = kc.reshape(-1, Hkv, D).cpu(), vc.reshape(-1, Hkv, D).cpu()
    ok = slots >= 0
    _ulp_close(kflat[slots[ok]], _rope_ref(kh, pos, inv_freq, draft)[ok],
               atol=(_rope_slack(kh, pos, inv_freq, draft) + floor)[ok])
    assert torch.equal(vflat[slots[ok]], v_in.reshape(T, Hkv, D).to(BF)[ok])
    untouched = torch.ones(P * ps, dtype=torch.bool)
    untouched[slots[ok]] = False
    assert torch.count_nonzero(kflat[untouched]) == 0 and torch.count_nonzero(vflat[untouched]) == 0


def test_qk_rope_position_zero_is_norm_only():
    """At position 0 the rotation is the identity: q is exactly the head norm."""
    D, Hq, Hkv, T = 128, 4, 2, 5
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, generator=g).to(BF)
    kc = torch.zeros(4, 16, Hkv, D, dtype=BF, device=DEV)
    inv = torch.rand(D // 2, generator=g).to(DEV)
    ones = torch.ones(D, dtype=BF, device=DEV)
    for draft in (False, True):
        q = ly.qk_rope_append(qkv.to(DEV), torch.zeros(T, dtype=torch.int64, device=DEV), ones, ones, inv, kc,
                              torch.zeros_like(kc), torch.arange(T, device=DEV), Hq, Hkv, 1e-6, draft_rope=draft)
        ref = _rms_ref(qkv.float()[:, :Hq * D].reshape(T, Hq, D), ones.cpu(), 1e-6)
        _ulp_close(q, ref, max_ulp=1)


@pytest.mark.parametrize("T,M", [(1, 6144), (128, 12288), (7, 8), (1088, 6144), (70000, 8), (3, 2056)])
def test_silu_mul(T, M):
    """Rows past the launch's 65,535 grid rows (T = 70000) are taken by the
    grid-stride loop; M = 2056 leaves a partial workgroup of vectors."""
    g = torch.Generator().manual_seed(T + M)
    gu = (torch.randn(T, 2 * M, generator=g) * 4).to(BF)
    out = ly.silu_mul(gu.to(DEV))
    gate, up = gu.float().chunk(2, -1)
    _ulp_close(out, torch.nn.functional.silu(gate.double()).float() * up)
