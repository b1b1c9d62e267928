"""Speculative acceptance on the gfx950 fused-acceptance kernel.

Drop-in for the reference module ``single/speculative_sampling.py``: same
names, signatures, result type and ``ValueError`` messages.  Two differences
are additions, not changes:

* the uniforms are accepted explicitly, as keyword-only ``uniforms`` ([B, K]
  fp32) and ``resample_uniform`` ([B] fp32).  When omitted they are drawn
  with ``torch.rand`` on the inputs' device (optionally from ``generator``),
  so reference-style calls keep working;
* ``torch.multinomial`` is replaced by an inverse CDF driven by
  ``resample_uniform``: token = first t with C_t > u * W over the (residual
  or bonus) weights, else the last t with positive weight.

Batched entry points (``accept_fused``, ``accept_fused_sparse``,
``greedy_accept``) take B requests in one launch; the reference functions
keep the reference's B == 1 rule.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple, Optional

import torch

from . import _lib


@dataclass(frozen=True)
class SpeculativeSampleResult:
    """single/speculative_sampling.py:8-12."""

    accepted_draft_tokens: int
    correction_token: torch.Tensor
    all_accepted: bool


# Messages for the out_token sentinels, as the reference's checks word them:
# an out-of-range draft token fails the gather of single/speculative_sampling.py
# :50-54, and torch.multinomial (:71) rejects a distribution without mass.
_SENTINEL_ERRORS = {
    _lib.D3D_TOKEN_BAD_DRAFT: (ValueError, "draft token id outside the vocabulary"),
    _lib.D3D_TOKEN_EMPTY_DISTRIBUTION: (RuntimeError, "invalid multinomial distribution (sum of probabilities <= 0)"),
    _lib.D3D_TOKEN_TIMEOUT: (RuntimeError, "acceptance residual hand-off timed out"),
}


def _raise_for_token(token: int, request: Optional[int] = None) -> None:
    err = _SENTINEL_ERRORS.get(int(token))
    if err is None:
        if token < 0:
            raise RuntimeError(f"acceptance returned an unknown status {token}")
        return
    cls, msg = err
    raise cls(msg if request is None else f"request {request}: {msg}")


class AcceptOutput(NamedTuple):
    """Device tensors written by one fused-acceptance launch.

    ``out_token`` holds a token id (>= 0) or, for a request whose draw could
    not be made, a negative status: ``D3D_TOKEN_BAD_DRAFT`` (a draft token
    outside [0, V)), ``D3D_TOKEN_EMPTY_DISTRIBUTION`` (no probability mass to
    draw from) or ``D3D_TOKEN_TIMEOUT``.  ``valid`` is the per-request mask of
    real tokens, computed on the device; :meth:`check` reads the tokens once
    and raises the reference's error for the first bad request.
    """

    accepted: torch.Tensor  # [B] int32, accepted draft tokens (0..K)
    accept_mask: torch.Tensor  # [B, K] bool, per-position decision
    out_token: torch.Tensor  # [B] int64, correction or bonus token, or a status < 0
    all_accepted: torch.Tensor  # [B] bool
    posterior: Optional[torch.Tensor]  # [B, K+1] int64, argmax of every target row; None if not asked for

    @property
    def valid(self) -> torch.Tensor:
        """[B] bool on the device: the request's out_token is a token id."""
        return self.out_token >= 0

    def check(self) -> "AcceptOutput":
        """Raise ValueError / RuntimeError if any request carries a status
        instead of a token (one host synchronisation); returns self."""
        for b, token in enumerate(self.out_token.tolist()):
            if token < 0:
                _raise_for_token(token, b if self.out_token.numel() > 1 else None)
        return self


def _prep(t: torch.Tensor) -> torch.Tensor:
    if t.dtype not in (torch.float32, torch.bfloat16):
        t = t.float()
    return t.contiguous()


def _outputs(B: int, K: int, dev: torch.device, posterior: bool = True):
    return (torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, K, dtype=torch.uint8, device=dev),
            torch.empty(B, dtype=torch.int64, device=dev), torch.empty(B, dtype=torch.uint8, device=dev),
            torch.empty(B, K + 1, dtype=torch.int64, device=dev) if posterior else None)


def accept_fused(
    target: torch.Tensor,
    draft: Optional[torch.Tensor],
    draft_tokens: torch.Tensor,
    *,
    temperature: float = 1.0,
    uniforms: Optional[torch.Tensor] = None,
    resample_uniform: Optional[torch.Tensor] = None,
    input_kind: str = "logits",
    generator: Optional[torch.Generator] = None,
    posterior: bool = True,
) -> AcceptOutput:
    """Batched fused acceptance: B requests of K draft tokens, one launch.

    ``target`` [B, K+1, V] and ``draft`` [B, K, V] are logits
    (``input_kind="logits"``: softmax at ``temperature``, the reference's
    ``_sampling_probs`` at single/eval_sync.py:287-305; ``temperature <= 1e-5``
    is greedy acceptance, single/eval_sync.py:1223-1234, and ignores draft and
    uniforms) or probabilities (``input_kind="probs"``, normalised by their sum
    as at single/speculative_sampling.py:37-40).  No host synchronisation.
    ``posterior=False`` leaves out the argmax of the target rows
    (``AcceptOutput.posterior`` is None) for a caller that does not use it;
    greedy acceptance computes it regardless, since its decision is made of it.
    """
    if target.ndim != 3 or draft_tokens.ndim != 2:
        raise ValueError("expected draft_tokens [B,K] and target [B,K+1,V]")
    B, K = draft_tokens.shape
    if target.shape[0] != B or target.shape[1] != K + 1:
        raise ValueError("target must contain K draft rows plus one bonus row")
    V = target.shape[2]
    kind = {"logits": _lib.D3D_INPUT_LOGITS, "probs": _lib.D3D_INPUT_PROBS}.get(input_kind)
    if kind is None:
        raise ValueError(f"input_kind must be 'logits' or 'probs', got {input_kind!r}")
    greedy = kind == _lib.D3D_INPUT_LOGITS and not (temperature > 1e-5)
    dev = _lib.require_device(target, draft_tokens, None if greedy else draft)
    target = _prep(target)
    if not greedy:
        if draft is None or draft.ndim != 3 or draft.shape[:2] != (B, K) or draft.shape[2] != V:
            raise ValueError("draft must be [B,K,V] with the target's vocabulary")
        draft = _prep(draft)
        if draft.dtype != target.dtype:
            draft = draft.to(target.dtype)
        if uniforms is None:
            uniforms = torch.rand(B, K, device=dev, generator=generator)
        if resample_uniform is None:
            resample_uniform = torch.rand(B, device=dev, generator=generator)
        uniforms = uniforms.to(device=dev, dtype=torch.float32).reshape(B, K).contiguous()
        resample_uniform = resample_uniform.to(device=dev, dtype=torch.float32).reshape(B).contiguous()
    else:
        draft = uniforms = resample_uniform = None
    tokens = draft_tokens.to(device=dev, dtype=torch.int64).contiguous()

    accepted, mask, out_token, all_acc, post = _outputs(B, K, dev, posterior or greedy)
    lib = _lib.load()
    nbytes = lib.d3d_accept_workspace_bytes(B, K, V)
    ws = _lib.workspace(dev, "accept", nbytes)
    status = lib.d3d_accept_fused(
        _lib.ptr(target), _lib.ptr(draft), _lib.dtype_code(target), kind,
        _lib.ptr(tokens), _lib.ptr(uniforms), _lib.ptr(resample_uniform),
        float(temperature), B, K, V,
        _lib.ptr(accepted), _lib.ptr(mask), _lib.ptr(out_token), _lib.ptr(all_acc),
        _lib.ptr(post), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev),
    )
    _lib.check(status, "d3d_accept_fused")
    return AcceptOutput(accepted, mask.bool(), out_token, all_acc.bool(), post)


def accept_fused_sparse(
    target: torch.Tensor,
    draft_tokens: torch.Tensor,
    draft_token_ids: torch.Tensor,
    draft_token_probs: torch.Tensor,
    *,
    temperature: float = 1.0,
    uniforms: Optional[torch.Tensor] = None,
    resample_uniform: Optional[torch.Tensor] = None,
    input_kind: str = "probs",
    generator: Optional[torch.Generator] = None,
    posterior: bool = True,
) -> AcceptOutput:
    """Batched fused acceptance against sparse proposals, one launch.

    ``target`` [B, K+1, V] as in :func:`accept_fused`; the draft side is
    ``draft_token_ids`` / ``draft_token_probs`` [B, K, S] (S <= 1024), the
    proposal support of single/speculative_sampling.py:79-143.  Support ids
    outside [0, V) carry no mass.  No host synchronisation; statuses in
    ``out_token`` and ``posterior`` as for :func:`accept_fused`.
    """
    if target.ndim != 3 or draft_tokens.ndim != 2:
        raise ValueError("expected draft_tokens [B,K] and target [B,K+1,V]")
    if draft_token_ids.ndim != 3 or draft_token_probs.ndim != 3:
        raise ValueError("expected sparse draft ids/probs [B,K,S]")
    B, K = draft_tokens.shape
    if target.shape[0] != B or target.shape[1] != K + 1:
        raise ValueError("target must contain K draft rows plus one bonus row")
    if draft_token_ids.shape[:2] != (B, K):
        raise ValueError("sparse draft support must contain one row per draft token")
    if draft_token_probs.shape != draft_token_ids.shape:
        raise ValueError("sparse draft ids and probs must have identical shapes")
    V, S = target.shape[2], draft_token_ids.shape[2]
    kind = {"logits": _lib.D3D_INPUT_LOGITS, "probs": _lib.D3D_INPUT_PROBS}.get(input_kind)
    if kind is None:
        raise ValueError(f"input_kind must be 'logits' or 'probs', got {input_kind!r}")
    dev = _lib.require_device(target, draft_tokens, draft_token_ids, draft_token_probs)
    target = _prep(target)
    if uniforms is None:
        uniforms = torch.rand(B, K, device=dev, generator=generator)
    if resample_uniform is None:
        resample_uniform = torch.rand(B, device=dev, generator=generator)
    uniforms = uniforms.to(device=dev, dtype=torch.float32).reshape(B, K).contiguous()
    resample_uniform = resample_uniform.to(device=dev, dtype=torch.float32).reshape(B).contiguous()
    tokens = draft_tokens.to(device=dev, dtype=torch.int64).contiguous()
    q_ids = draft_token_ids.to(dtype=torch.int64).contiguous()
    q_probs = draft_token_probs.to(dtype=torch.float32).contiguous()

    accepted, mask, out_token, all_acc, post = _outputs(B, K, dev, posterior)
    lib = _lib.load()
    ws = _lib.workspace(dev, "accept", lib.d3d_accept_workspace_bytes(B, K, V))
    status = lib.d3d_accept_fused_sparse(
        _lib.ptr(target), _lib.dtype_code(target), kind, _lib.ptr(tokens), _lib.ptr(q_ids), _lib.ptr(q_probs),
        S, _lib.ptr(uniforms), _lib.ptr(resample_uniform), float(temperature), B, K, V,
        _lib.ptr(accepted), _lib.ptr(mask), _lib.ptr(out_token), _lib.ptr(all_acc),
        _lib.ptr(post), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev),
    )
    _lib.check(status, "d3d_accept_fused_sparse")
    return AcceptOutput(accepted, mask.bool(), out_token, all_acc.bool(), post)


def _to_result(out: AcceptOutput) -> SpeculativeSampleResult:
    packed = torch.stack(
        [out.accepted[0].long(), out.out_token[0], out.all_accepted[0].long()]
    ).cpu().tolist()
    n, token, all_acc = packed
    _raise_for_token(token)
    return SpeculativeSampleResult(
        accepted_draft_tokens=int(n),
        correction_token=out.out_token[:1].clone(),
        all_accepted=bool(all_acc),
    )


def verify_speculative_block(
    draft_tokens: torch.Tensor,
    target_probs: torch.Tensor,
    draft_probs: torch.Tensor,
    *,
    uniforms: Optional[torch.Tensor] = None,
    resample_uniform: Optional[torch.Tensor] = None,
    generator: Optional[torch.Generator] = None,
) -> SpeculativeSampleResult:
    """Verify a sampled draft block with standard p/q rejection sampling.

    single/speculative_sampling.py:15-76: ``draft_tokens`` [B, K],
    ``target_probs`` [B, K+1, V] (last row is the bonus distribution),
    ``draft_probs`` [B, K, V]; B must be 1, as in the reference.
    """
    if draft_tokens.ndim != 2 or target_probs.ndim != 3 or draft_probs.ndim != 3:
        raise ValueError("expected draft_tokens [B,K], target_probs/draft_probs [B,K,V]")
    batch, draft_len = draft_tokens.shape
    if target_probs.shape[0] != batch or target_probs.shape[1] != draft_len + 1:
        raise ValueError("target_probs must contain K draft rows plus one bonus row")
    if draft_probs.shape[0] != batch or draft_probs.shape[1] != draft_len:
        raise ValueError("draft_probs must contain one row per draft token")
    if target_probs.shape[-1] != draft_probs.shape[-1]:
        raise ValueError("target and draft vocabularies must match")
    if batch != 1:
        raise ValueError("standard verification currently supports batch size 1")
    out = accept_fused(
        target_probs, draft_probs, draft_tokens,
        uniforms=uniforms, resample_uniform=resample_uniform,
        input_kind="probs", generator=generator, posterior=False,
    )
    return _to_result(out)


def verify_speculative_block_sparse(
    draft_tokens: torch.Tensor,
    target_probs: torch.Tensor,
    draft_token_ids: torch.Tensor,
    draft_token_probs: torch.Tensor,
    *,
    uniforms: Optional[torch.Tensor] = None,
    resample_uniform: Optional[torch.Tensor] = None,
    generator: Optional[torch.Generator] = None,
) -> SpeculativeSampleResult:
    """Verify against an exact sparse proposal distribution.

    single/speculative_sampling.py:79-143: ``draft_tokens`` [B, K],
    ``target_probs`` [B, K+1, V], ``draft_token_ids`` / ``draft_token_probs``
    [B, K, S]; B must be 1, as in the reference.
    """
    if draft_tokens.ndim != 2 or target_probs.ndim != 3:
        raise ValueError("expected draft_tokens [B,K] and target_probs [B,K+1,V]")
    if draft_token_ids.ndim != 3 or draft_token_probs.ndim != 3:
        raise ValueError("expected sparse draft ids/probs [B,K,S]")
    batch, draft_len = draft_tokens.shape
    if batch != 1:
        raise ValueError("standard verification currently supports batch size 1")
    if target_probs.shape[:2] != (batch, draft_len + 1):
        raise ValueError("target_probs must contain K draft rows plus one bonus row")
    if draft_token_ids.shape[:2] != (batch, draft_len):
        raise ValueError("sparse draft support must contain one row per draft token")
    if draft_token_probs.shape != draft_token_ids.shape:
        raise ValueError("sparse draft ids and probs must have identical shapes")
    out = accept_fused_sparse(
        target_probs, draft_tokens, draft_token_ids, draft_token_probs,
        uniforms=uniforms, resample_uniform=resample_uniform, input_kind="probs", generator=generator,
        posterior=False,
    )
    return _to_result(out)


def greedy_accept(target_logits: torch.Tensor, block: torch.Tensor) -> AcceptOutput:
    """Greedy acceptance of B blocks (anchor + K draft tokens) in one launch.

    single/eval_sync.py:1223-1234 and serving/engine.py:138-145: posterior =
    argmax of each target row; accepted = leading draft tokens equal to the
    posterior of the row before them; out_token = posterior[accepted].  The
    engine's commit length is ``accepted + 1``.
    """
    if block.ndim != 2 or target_logits.ndim != 3 or target_logits.shape[:2] != block.shape:
        raise ValueError("expected block [B,K+1] and target_logits [B,K+1,V]")
    return accept_fused(target_logits, None, block[:, 1:], temperature=0.0)
