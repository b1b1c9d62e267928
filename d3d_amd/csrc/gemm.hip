// Weight-streaming GEMM for blocks of at most 64 rows:  Y[M, N] = X[M, K] W[N, K]^T
// (bf16 in, fp32 accumulation), the projections of a 64-token verify or draft
// block (serving/vendor/ssd/layers/linear.py: F.linear on bf16 weights).
//
// At M <= 64 the weights dominate the traffic (a 64-row block reads each
// weight once and each activation once per 64 output columns), so the
// kernel is built to stream W:
//
// * Workgroup (column tile of 64, K split s): four waves; each k step moves
//   a 64 x 128 tile of W and the 64 x 128 tile of X straight from global
//   memory into LDS (global_load_lds, 16 bytes per lane: every wave
//   instruction reads four full 256-byte row segments), two stages deep, so
//   the loads in flight cost no registers.  Within a row the 16-byte chunk
//   q is stored at slot q ^ (row & 7): the MFMA operand reads of 16
//   consecutive rows then spread over the LDS banks.
// * Wave w multiplies the 64 rows of X by columns 16w .. 16w + 15 of the
//   tile with v_mfma_f32_16x16x32_bf16, both operands read from LDS.
// * Small N leaves too few column tiles to fill 256 CUs, so K is split over
//   `splits` workgroups per tile (d3d_gemm_rows64_splits picks the count).
//   With one split the result is rounded to bf16 into Y; with several,
//   each split writes its fp32 partial [splits][M][N] and the consumer of
//   the product sums the splits in order (d3d_add_rmsnorm_parts,
//   d3d_qk_rope_append_parts) -- no extra launch, no atomics, and the sum
//   has the same bits on every call.
#include "d3d_common.hpp"
#include "../../include/d3d_hip.h"

namespace d3d {
namespace gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int NT = 256;                  // four waves
constexpr int TN = 64;                   // output columns per workgroup
constexpr int TK = 128;                  // k per stage
constexpr int ST = 2;                    // stages
constexpr int ROWB = TK * 2;             // bytes of one tile row
constexpr int CPR = ROWB / 16;           // 16-byte chunks per tile row
constexpr int TILEB = 64 * ROWB;         // one 64-row tile (W or X), 16 KB
constexpr int STAGEB = 2 * TILEB;        // W tile, then X tile
constexpr int RPI = kWave / CPR;         // tile rows per wave instruction
constexpr int LPW = TILEB / 1024 / 4;    // load instructions per wave per tile
constexpr int kMaxSplits = 16;
static_assert(ST * STAGEB <= 64 * 1024, "LDS per workgroup");

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__global__ __launch_bounds__(NT) void gemm_rows64_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w,
                                                         uint16_t* __restrict__ y, float* __restrict__ parts,
                                                         int M, int N, int K, int KR) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    const int c16 = lane & 15, g4 = lane >> 4;
    const int n0 = blockIdx.x * TN;
    const int kb = blockIdx.y * KR;
    const int steps = KR / TK;
    // This lane's source rows and LDS rows: wave wv fills rows
    // (wv * LPW + j) * RPI + lane / CPR of both tiles, chunk lane % CPR
    // read from global chunk (lane % CPR) ^ (row & 7).
    const int lr = lane / CPR, lc = lane % CPR;
    const uint16_t* wsrc[LPW];
    const uint16_t* xsrc[LPW];
    int lofs[LPW];
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
        const int rb = (wv * LPW + j) * RPI, r = rb + lr;
        const int q = lc ^ (r & 7);
        wsrc[j] = w + (size_t)(n0 + r) * K + kb + 8 * q;
        xsrc[j] = x + (size_t)min(r, M - 1) * K + kb + 8 * q;
        lofs[j] = rb * ROWB;
    }
    f32x4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = {0.f, 0.f, 0.f, 0.f};
    // Stage 0 in flight before the loop; each iteration issues the next
    // stage, waits for the current one (its own loads, then the barrier for
    // everyone's), multiplies it, and frees it with a second barrier.
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
        __builtin_amdgcn_global_load_lds(wsrc[j], smem + lofs[j], 16, 0, 0);
        __builtin_amdgcn_global_load_lds(xsrc[j], smem + TILEB + lofs[j], 16, 0, 0);
    }
    const int rB = 16 * wv + c16;
    for (int step = 0; step < steps; ++step) {
        if (step + 1 < steps) {
            char* nxt = smem + ((step + 1) % ST) * STAGEB;
            const int ko = (step + 1) * TK;
#pragma unroll
            for (int j = 0; j < LPW; ++j) {
                __builtin_amdgcn_global_load_lds(wsrc[j] + ko, nxt + lofs[j], 16, 0, 0);
                __builtin_amdgcn_global_load_lds(xsrc[j] + ko, nxt + TILEB + lofs[j], 16, 0, 0);
            }
            wait_vmcnt<2 * LPW>();
        } else {
            wait_vmcnt<0>();
        }
        __syncthreads();
        const char* cur = smem + (step % ST) * STAGEB;
#pragma unroll
        for (int ks = 0; ks < TK / 32; ++ks) {
            const int q = 4 * ks + g4;
            const u32x4 bw = *reinterpret_cast<const u32x4*>(cur + rB * ROWB + 16 * (q ^ (rB & 7)));
            u32x4 ax[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int m = 16 * t + c16;
                ax[t] = *reinterpret_cast<const u32x4*>(cur + TILEB + m * ROWB + 16 * (q ^ (m & 7)));
            }
#pragma unroll
            for (int t = 0; t < 4; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ax[t]),
                                                                 __builtin_bit_cast(bf16x8, bw), acc[t], 0, 0, 0);
        }
        __syncthreads();
    }
    // Lane (c16, g4) holds rows 16t + 4 g4 + r of column 16 wv + c16.
    const int n = n0 + 16 * wv + c16;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 16 * t + 4 * g4 + r;
            if (m < M) {
                if (gridDim.y == 1)
                    y[(size_t)m * N + n] = f32_to_bf16_bits(acc[t][r]);
                else
                    parts[((size_t)blockIdx.y * M + m) * N + n] = acc[t][r];
            }
        }
}

}  // namespace gemm
}  // namespace d3d

using namespace d3d;

extern "C" int d3d_gemm_rows64_splits(int N, int K) {
    if (N < gemm::TN || N % gemm::TN || K < gemm::TK || K % gemm::TK) return 1;
    // The most splits whose grid is one round of resident workgroups (two
    // per CU with 64 KB of LDS each: 512), leaving every split at least two
    // k steps, and -- below K = 8192, where more splits buy less -- at most
    // 16,384 partial floats per output row: the consumer of the product
    // reads every partial back, about 1 us per 4 MB at 64 rows.  Measured
    // on the 64-row projections of both models with 1-16 splits, counting
    // that read, this is within 0.3 us of the fastest count on each.
    const int tiles = N / gemm::TN;
    int s = 1;
    while (s < gemm::kMaxSplits && tiles * 2 * s <= 512 && K % (gemm::TK * 2 * s) == 0 &&
           K / (2 * s) >= 2 * gemm::TK && (K >= 8192 || (int64_t)2 * s * N <= 16384))
        s *= 2;
    return s;
}

extern "C" int d3d_gemm_rows64(const void* x, const void* w, void* y, float* parts, int M, int N, int K,
                               int splits, void* stream) {
    if (M < 1 || M > 64 || N < gemm::TN || N % gemm::TN || K < gemm::TK) return D3D_E_SHAPE;
    if (splits < 1 || splits > gemm::kMaxSplits || K % (gemm::TK * splits)) return D3D_E_SHAPE;
    if (!x || !w || (splits == 1 ? !y : !parts)) return D3D_E_NULL;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16) return D3D_E_UNSUPPORTED;
    hipLaunchKernelGGL(gemm::gemm_rows64_kernel, dim3(N / gemm::TN, splits), dim3(gemm::NT), gemm::ST * gemm::STAGEB,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x),
                       static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y), parts, M, N, K, K / splits);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
