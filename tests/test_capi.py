"""The C ABI library loads and exports every entry point include/d3d_hip.h declares.

CPU only: no kernel is launched here.  Argument validation happens on the
host before any HIP call, so invalid calls are exercised with null pointers.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from d3d_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "d3d_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(d3d_\w+)\s*\(", text)))


def test_header_declares_functions():
    names = declared_functions()
    assert "d3d_accept_fused" in names and len(names) >= 4


def test_every_declared_function_is_exported_and_bound(d3d_lib):
    for name in declared_functions():
        assert hasattr(d3d_lib, name), f"{name} not exported by {_lib.LIB_PATH.name}"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(declared_functions())


def test_status_strings_and_version(d3d_lib):
    assert d3d_lib.d3d_status_string(0) == b"ok"
    assert b"shape" in d3d_lib.d3d_status_string(-1)
    assert d3d_lib.d3d_version() >= 100


def test_accept_workspace_bytes(d3d_lib):
    small = d3d_lib.d3d_accept_workspace_bytes(1, 15, 151936)
    big = d3d_lib.d3d_accept_workspace_bytes(8, 15, 151936)
    assert 0 < small < big
    assert d3d_lib.d3d_accept_workspace_bytes(0, 15, 100) == 0


@pytest.mark.parametrize(
    "B,K,V,dtype,kind,expect",
    [
        (0, 15, 100, 0, 0, -1),      # no requests
        (1, 0, 100, 0, 0, -1),       # no draft tokens
        (1, 128, 100, 0, 0, -1),     # K above the supported 127
        (1, 15, 0, 0, 0, -1),        # empty vocabulary
        (1, 15, 100, 7, 0, -2),      # unknown dtype
        (1, 15, 100, 0, 9, -5),      # unknown input kind
        (1, 15, 100, 0, 0, -4),      # null pointers
    ],
)
def test_accept_rejects_invalid_arguments_without_launching(d3d_lib, B, K, V, dtype, kind, expect):
    st = d3d_lib.d3d_accept_fused(None, None, dtype, kind, None, None, None, 1.0, B, K, V,
                                  None, None, None, None, None, None, 0, None)
    assert st == expect
    with pytest.raises(ValueError):
        _lib.check(st, "d3d_accept_fused")


def test_accept_rejects_small_workspace(d3d_lib):
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    st = d3d_lib.d3d_accept_fused(p, p, 0, 0, p, p, p, 1.0, 1, 15, 151936,
                                  p, p, p, p, None, p, 64, None)
    assert st == -3


def test_gemm_rows64_splits_and_argument_checks(d3d_lib):
    lib = d3d_lib
    # one round of 512 resident workgroups, at least two 128-wide k steps per
    # split, at most 16,384 partial floats per row below K = 8192
    assert lib.d3d_gemm_rows64_splits(4096, 12288) == 4
    assert lib.d3d_gemm_rows64_splits(2048, 2048) == 8
    assert lib.d3d_gemm_rows64_splits(2048, 6144) == 8
    assert lib.d3d_gemm_rows64_splits(4096, 2048) == 4
    assert lib.d3d_gemm_rows64_splits(4096, 4096) == 4
    assert lib.d3d_gemm_rows64_splits(24576, 4096) == 1
    assert lib.d3d_gemm_rows64_splits(12288, 2048) == 1
    assert lib.d3d_gemm_rows64_splits(6144, 4096) == 2
    assert lib.d3d_gemm_rows64_splits(2000, 2048) == 1 and lib.d3d_gemm_rows64_splits(2048, 100) == 1
    # layers.project takes the kernel on grids of 128 to 256 workgroups and of 512
    from d3d_amd import layers as ly
    routed = {(N, K): ly.rows64_splits(N, K) for N, K in ((6144, 4096), (4096, 4096), (24576, 4096),
                                                          (4096, 12288), (4096, 2048), (2048, 2048),
                                                          (12288, 2048), (2048, 6144), (2000, 2048))}
    assert routed == {(6144, 4096): 2, (4096, 4096): 4, (24576, 4096): 0, (4096, 12288): 4, (4096, 2048): 4,
                      (2048, 2048): 8, (12288, 2048): 1, (2048, 6144): 8, (2000, 2048): 0}
    null = ctypes.c_void_p(0)
    dummy = ctypes.c_void_p(256)
    # the fused gate-up + SiLU-mul: shape, step-count and pointer checks before any launch
    for M, H, K in ((0, 64, 1024), (65, 64, 1024), (8, 48, 1024), (8, 64, 1000), (8, 64, 1152)):
        assert lib.d3d_gemm_rows64_silu_mul(dummy, dummy, dummy, M, H, K, null) in (-1, -5), (M, H, K)
    assert lib.d3d_gemm_rows64_silu_mul(dummy, dummy, dummy, 8, 64, 1152, null) == -5  # 9 steps: D3D_E_UNSUPPORTED
    assert lib.d3d_gemm_rows64_silu_mul(null, dummy, dummy, 8, 64, 1024, null) == -4
    for M, N, K, s in ((0, 64, 128, 1), (65, 64, 128, 1), (8, 100, 128, 1), (8, 64, 100, 1), (8, 64, 128, 2),
                       (8, 64, 4096, 3), (8, 64, 4096, 32)):
        assert lib.d3d_gemm_rows64(dummy, dummy, dummy, dummy, M, N, K, s, null) == -1, (M, N, K, s)
    assert lib.d3d_gemm_rows64(null, dummy, dummy, dummy, 8, 64, 128, 1, null) == -4  # D3D_E_NULL
    assert lib.d3d_gemm_rows64(dummy, dummy, null, dummy, 8, 64, 128, 1, null) == -4
    assert lib.d3d_gemm_rows64(dummy, dummy, dummy, null, 8, 64, 256, 2, null) == -4
    assert lib.d3d_add_rmsnorm_parts(dummy, 0, dummy, dummy, dummy, 4, 64, 1e-6, null) == -1
    assert lib.d3d_add_rmsnorm_parts(null, 2, dummy, dummy, dummy, 4, 64, 1e-6, null) == -4
