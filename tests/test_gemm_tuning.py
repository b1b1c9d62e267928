"""The shipped library-GEMM solution file and the step shapes it covers.

CPU only: the file's format (TunableOp's CSV: validator lines, then one
``op,params,solution,ms`` line per shape) and its coverage of the engine
step's library GEMMs; whether torch loads it is a GPU test."""
import re

import pytest

from d3d_amd import gemm_tuning, layers as ly
from d3d_amd.model import D3D_1P7B, QWEN3_8B


def _rows():
    lines = gemm_tuning.RESULTS.read_text().splitlines()
    val = [l.split(",") for l in lines if l.startswith("Validator,")]
    res = [l.split(",") for l in lines if not l.startswith("Validator,")]
    return val, res


def test_results_file_has_validators_and_one_entry_per_step_shape():
    val, res = _rows()
    assert {v[1] for v in val} >= {"PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "GCN_ARCH_NAME",
                                   "ROCBLAS_VERSION"}
    arch = dict((v[1], v[2]) for v in val)["GCN_ARCH_NAME"]
    assert arch.startswith("gfx950")
    shapes = []
    for op, params, solution, ms in res:
        assert op == "GemmTunableOp_BFloat16_TN"
        # F.linear(x [M, K], w [N, K]) is the column-major TN GEMM N x M x K
        m = re.fullmatch(r"tn_(\d+)_(\d+)_(\d+)_ld_(\d+)_(\d+)_(\d+)", params)
        assert m, params
        N, M, K, lda, ldb, ldc = map(int, m.groups())
        assert (lda, ldb, ldc) == (K, K, N)
        assert solution == "Default" or re.fullmatch(r"Gemm_(Hipblaslt|Rocblas)_-?\d+", solution), solution
        assert float(ms) > 0
        shapes.append((M, N, K))
    assert len(shapes) == len(set(shapes))
    assert sorted(shapes) == gemm_tuning.step_gemm_shapes(QWEN3_8B, D3D_1P7B)


def test_step_shapes_leave_out_what_runs_on_the_hip_gemm():
    """At 64 rows and fewer the projections layers.project runs on
    d3d_gemm_rows64 are not library GEMMs; the LM heads always are, and the
    packed predict (more than 64 rows) runs every projection on the library."""
    got = gemm_tuning.step_gemm_shapes(QWEN3_8B, D3D_1P7B, batches=(4,), anchors=(1,))
    V = QWEN3_8B.vocab
    assert got == sorted([
        (64, 24576, 4096), (64, V, 4096),                              # target gate-up, LM head
        (64, V, 2048),                                                 # draft recovery LM head
        (1088, 4096, 2048), (1088, 2048, 2048), (1088, 12288, 2048),   # packed predict: 4 x 272 rows
        (1088, 2048, 6144), (1088, V, 2048),
    ])
    for M, N, K in got:
        if M <= ly.ROWS64 and N != V:
            assert ly.rows64_splits(N, K) == 0


def test_enable_without_a_gpu_leaves_torch_defaults(tmp_path):
    if gemm_tuning.torch.cuda.is_available():
        pytest.skip("CPU-only check")
    assert gemm_tuning.enable() is False
    assert gemm_tuning.enable(tmp_path / "missing.csv") is False


def test_corun_shapes_stay_on_the_library_default():
    """The packed predict's qkv and down projections and the verify's
    gate-up run beside the other forward; the file keeps them on the default
    solution, every other shape on a timed choice (which may also be the
    default)."""
    _, res = _rows()
    sol = {}
    for _, params, solution, _ in res:
        N, M, K = map(int, params.split("_")[1:4])
        sol[(M, N, K)] = solution
    keep = gemm_tuning.corun_default_shapes(QWEN3_8B, D3D_1P7B)
    assert len(keep) == 20 and set(keep) <= set(sol)
    assert all(sol[s] == "Default" for s in keep)
    assert (1088, 4096, 2048) in keep and (1088, 2048, 6144) in keep and (64, 24576, 4096) in keep
    assert (1088, 12288, 2048) not in keep and (1088, 2048, 2048) not in keep
    assert (64, QWEN3_8B.vocab, 4096) not in keep
