"""Library GEMMs on the shipped TunableOp solution choices: the file loads on
this GPU, tuned products stay within bf16 GEMM rounding of an fp32 product,
and HIP-graph replays of them equal their eager calls (replayed several
times, with eager work and synchronisations between the replays)."""
import pytest
import torch
import torch.nn.functional as F

from d3d_amd import gemm_tuning

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
BF = torch.bfloat16
V = 151936
# The batch-4, one-anchor engine step's library GEMMs (M, N, K).
SHAPES = [(64, 6144, 4096), (64, 24576, 4096), (64, V, 4096), (64, 12288, 2048), (64, V, 2048),
          (1088, 4096, 2048), (1088, 2048, 2048), (1088, 12288, 2048), (1088, 2048, 6144), (1088, V, 2048)]


@pytest.fixture(scope="module", autouse=True)
def tuned():
    was = torch.cuda.tunable.is_enabled()
    assert gemm_tuning.enable(), "the shipped results file did not load on this GPU"
    yield
    if not was:
        gemm_tuning.disable()


def _operands(M, N, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=DEV).to(BF)
    w = (torch.randn(N, K, generator=g, device=DEV) * 0.02).to(BF)
    return x, w


@pytest.mark.parametrize("M,N,K", SHAPES)
def test_tuned_product_within_bf16_rounding(M, N, K):
    x, w = _operands(M, N, K, seed=M + N + K)
    y = F.linear(x, w).float()
    ref = x.float() @ w.float().t()
    # fp32 accumulation, one bf16 rounding of the output: |err| <= 2^-8 |y|
    # plus accumulation-order noise of K products of magnitude ~0.02 * 1.
    bound = ref.abs() * 2.0 ** -8 + 1e-3 * (K / 4096) ** 0.5
    assert bool(((y - ref).abs() <= bound).all()), float((y - ref).abs().max())


@torch.inference_mode()  # as the engine captures its step graphs
def test_graph_replays_of_tuned_gemms_equal_eager():
    ops = [_operands(M, N, K, seed=7 * M + N) for M, N, K in SHAPES]
    eager = [F.linear(x, w) for x, w in ops]
    s = torch.cuda.Stream(DEV)
    outs = [torch.empty_like(e) for e in eager]
    with torch.cuda.stream(s):
        for (x, w), o in zip(ops, outs):
            torch.mm(x, w.t(), out=o)
        torch.cuda.synchronize(DEV)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for (x, w), o in zip(ops, outs):
                torch.mm(x, w.t(), out=o)
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize(DEV)
        g.replay()
        torch.cuda.synchronize(DEV)
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o, e), (rep, SHAPES[i])
        # eager work between replays
        F.linear(*ops[rep % len(ops)])
        torch.cuda.synchronize(DEV)
