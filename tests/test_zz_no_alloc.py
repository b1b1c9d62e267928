"""d3d_accept_fused_noalloc against d3d_accept_fused, through the C ABI (GPU).

The allocation-free entry point runs the same kernels with the row
statistics in a static device array instead of a caller workspace.  Two
calls in a row -- the second with a smaller batch, so stale scratch from
the first is present -- must reproduce the workspace entry point's outputs
bit for bit (accept mask, accepted count, output token, all-accepted flag,
posterior), at T = 1 over logits, over probabilities, and greedy.  A size
whose workspace exceeds the scratch is refused before any launch.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from d3d_amd import _lib
from d3d_amd import workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _outputs(B, K):
    return dict(acc=torch.full((B,), -7, dtype=torch.int32, device=DEV),
                mask=torch.full((B, K), 9, dtype=torch.uint8, device=DEV),
                tok=torch.full((B,), -7, dtype=torch.int64, device=DEV),
                alla=torch.full((B,), 9, dtype=torch.uint8, device=DEV),
                post=torch.full((B, K + 1), -7, dtype=torch.int64, device=DEV))


def _call(noalloc, t, d, kind, tok, u, ru, T):
    lib = _lib.load()
    B, K1, V = t.shape
    K = K1 - 1
    o = _outputs(B, K)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    common = (t.data_ptr(), d.data_ptr(), _lib.D3D_DTYPE_F32, kind, tok.data_ptr(), u.data_ptr(), ru.data_ptr(),
              float(T), B, K, V, o["acc"].data_ptr(), o["mask"].data_ptr(), o["tok"].data_ptr(),
              o["alla"].data_ptr(), o["post"].data_ptr())
    if noalloc:
        st = lib.d3d_accept_fused_noalloc(*common, stream)
    else:
        n = lib.d3d_accept_workspace_bytes(B, K, V)
        ws = torch.empty(n, dtype=torch.uint8, device=DEV)
        st = lib.d3d_accept_fused(*common, ws.data_ptr(), n, stream)
    assert st == 0, lib.d3d_status_string(st)
    torch.cuda.synchronize()
    return {k: v.cpu() for k, v in o.items()}


@pytest.mark.parametrize("mode", ["logits", "probs", "greedy"])
def test_noalloc_matches_workspace_entry_point_twice(mode):
    kind = _lib.D3D_INPUT_PROBS if mode == "probs" else _lib.D3D_INPUT_LOGITS
    T = 0.0 if mode == "greedy" else 1.0
    for seed, B in ((11, 8), (12, 3)):  # the second call is smaller
        inp = workloads.accept_inputs(seed, B=B, K=15, temperature=T, device="cuda")
        t, d = inp.target, inp.draft
        if mode == "probs":
            t, d = torch.softmax(t, -1).contiguous(), torch.softmax(d, -1).contiguous()
        args = (t, d, kind, inp.tokens, inp.uniforms, inp.resample_u, T)
        want = _call(False, *args)
        got = _call(True, *args)
        for k in want:
            assert torch.equal(got[k], want[k]), (mode, B, k)
        assert (got["acc"] >= 0).all() and (got["tok"] >= 0).all()


def test_noalloc_refuses_sizes_beyond_the_scratch():
    lib = _lib.load()
    K, V = 15, 151936
    B = 214
    assert lib.d3d_accept_workspace_bytes(B, K, V) > _lib.D3D_ACCEPT_NOALLOC_SCRATCH_BYTES
    assert lib.d3d_accept_workspace_bytes(213, K, V) <= _lib.D3D_ACCEPT_NOALLOC_SCRATCH_BYTES
    # Refused on the host before any pointer is touched or kernel launched.
    null = ctypes.c_void_p(0)
    st = lib.d3d_accept_fused_noalloc(null, null, _lib.D3D_DTYPE_F32, _lib.D3D_INPUT_LOGITS, null, null, null,
                                      1.0, B, K, V, null, null, null, null, null, null)
    assert st == -3  # D3D_E_WORKSPACE
