// Weight-streaming GEMM for blocks of at most 64 rows:  Y[M, N] = X[M, K] W[N, K]^T
// (bf16 in, fp32 accumulation), the projections of a 64-token verify or draft
// block (serving/vendor/ssd/layers/linear.py: F.linear on bf16 weights).
//
// At M <= 64 the weights dominate the traffic (a 64-row block reads each
// weight once and each activation once per 64 output columns), so the
// kernel is built to stream W:
//
// * Workgroup (column tile of 64, K split s), four waves; each k step moves
//   a 64 x 128 tile of W and the 64 x 128 tile of X.  Every wave
//   instruction reads four full 256-byte row segments (16 bytes per lane),
//   the order that streams the weights fastest of those measured.  Within
//   a row the 16-byte chunk q is stored at slot q ^ (row & 7) of LDS, so
//   the MFMA operand reads of 16 consecutive rows spread over the banks.
// * Register-staged pipeline (gemm_rows64_kernel): the loads of the next
//   two k steps are in flight in registers while a step is stored to one of
//   two LDS buffers and multiplied from it, one barrier per step.  The k
//   loop is unrolled for the step counts the models use (STEPS), so the
//   compiler's wait before each store counts exactly the loads issued after
//   it.  Measured against the earlier form (direct global -> LDS loads, two
//   stages, two barriers per step; kept as gemm_rows64_dma_kernel for other
//   step counts), graph-replayed on HBM-resident weights: target o 14.7 ->
//   9.9 us, target down 29.8 -> 23.5, draft qkv 9.2 -> 7.1, draft o 6.7 ->
//   6.0, draft down 12.4 -> 8.9; the same kernel without loads of X or
//   without the MFMAs was only 10-15 % faster, so the direct-to-LDS loads
//   with one stage ahead were the bound.
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

// One k step from an LDS stage (W tile, then X tile): wave wv multiplies the
// 64 rows of X by columns 16 wv .. 16 wv + 15 of the tile.
__device__ __forceinline__ void mma_step(const char* cur, f32x4 (&acc)[4], int wv, int c16, int g4) {
    const int rB = 16 * wv + c16;
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
}

// Lane (c16, g4) holds rows 16t + 4 g4 + r of column n: bf16 into Y (one
// split) or the fp32 partial of split blockIdx.y.
__device__ __forceinline__ void store_tile(const f32x4 (&acc)[4], uint16_t* y, float* parts, int M, int N, int n,
                                           int g4) {
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

// Direct global -> LDS form (global_load_lds, two stages): the kernel for
// step counts gemm_rows64_kernel is not unrolled for.
__global__ __launch_bounds__(NT) void gemm_rows64_dma_kernel(const uint16_t* __restrict__ x,
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
        mma_step(smem + (step % ST) * STAGEB, acc, wv, c16, g4);
        __syncthreads();
    }
    store_tile(acc, y, parts, M, N, n0 + 16 * wv + c16, g4);
}

// Register-staged form of the kernel above (same tiles, LDS layout and
// results): stage st of a lane is rw / rx[st % 2] until it is stored to
// LDS buffer st % 2; the loads of stage st + 2 then reuse those registers.
//
// SILU: W is a gate-up weight [2 H, K] (gate rows, then up rows) and Y
// [M, H] = silu(bf16(X Wg^T)) * bf16(X Wu^T), each product rounded as the
// bf16 GEMM output would be, then evaluated as d3d_silu_mul does.  Tile t
// stands for output columns 32 t .. 32 t + 31: tile row 16 w + c is gate
// row 32 t + 8 w + c (c < 8) or the up row of column 32 t + 8 w + c - 8, so
// a lane's gate and up products of one column sit in lanes c and c + 8 of
// its 16-lane row.
template <int STEPS, bool SILU = false>
__global__ __launch_bounds__(NT, 2) void gemm_rows64_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w,
                                                            uint16_t* __restrict__ y, float* __restrict__ parts,
                                                            int M, int N, int K, int KR) {
    constexpr int P = 2;  // k steps in flight in registers
    extern __shared__ __attribute__((aligned(16))) char smem[];
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    const int c16 = lane & 15, g4 = lane >> 4;
    const int n0 = blockIdx.x * TN;
    const int kb = blockIdx.y * KR;
    // This lane's source rows and LDS slots: wave wv loads rows
    // (wv * LPW + j) * RPI + lane / CPR of both tiles, global chunk
    // (lane % CPR) ^ (row & 7) into LDS chunk lane % CPR.
    const int lr = lane / CPR, lc = lane % CPR;
    const uint16_t* wsrc[LPW];
    const uint16_t* xsrc[LPW];
    int lofs[LPW];
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
        const int r = (wv * LPW + j) * RPI + lr;
        const int q = lc ^ (r & 7);
        int wrow = n0 + r;
        if constexpr (SILU) {
            const int col = 32 * blockIdx.x + 8 * (r >> 4) + (r & 7);
            wrow = (r & 8) ? N / 2 + col : col;
        }
        wsrc[j] = w + (size_t)wrow * K + kb + 8 * q;
        xsrc[j] = x + (size_t)min(r, M - 1) * K + kb + 8 * q;
        lofs[j] = r * ROWB + lc * 16;
    }
    u32x4 rw[P][LPW], rx[P][LPW];
    auto load = [&](int st, int sl) {
#pragma unroll
        for (int j = 0; j < LPW; ++j) {
            rw[sl][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wsrc[j] + st * TK));
            rx[sl][j] = *reinterpret_cast<const u32x4*>(xsrc[j] + st * TK);
        }
    };
    f32x4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < P; ++p)
        if (p < STEPS) load(p, p);
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
        // Buffer st % 2 was last read in step st - 2, which every wave
        // finished before the barrier of step st - 1.
        char* buf = smem + (st & 1) * STAGEB;
#pragma unroll
        for (int j = 0; j < LPW; ++j) {
            *reinterpret_cast<u32x4*>(buf + lofs[j]) = rw[st % P][j];
            *reinterpret_cast<u32x4*>(buf + TILEB + lofs[j]) = rx[st % P][j];
        }
        if (st + P < STEPS) load(st + P, st % P);
        __syncthreads();
        mma_step(buf, acc, wv, c16, g4);
    }
    if constexpr (SILU) {
        const int H = N / 2, col = 32 * blockIdx.x + 8 * wv + (c16 & 7);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float mine = acc[t][r], other = __shfl_xor(mine, 8, kWave);
                const int m = 16 * t + 4 * g4 + r;
                if (c16 < 8 && m < M) {
                    const float gv = bf16_bits_to_f32(f32_to_bf16_bits(mine));
                    const float uv = bf16_bits_to_f32(f32_to_bf16_bits(other));
                    y[(size_t)m * H + col] = __builtin_bit_cast(uint16_t, (__bf16)(gv / (1.0f + expf(-gv)) * uv));
                }
            }
    } else {
        store_tile(acc, y, parts, M, N, n0 + 16 * wv + c16, g4);
    }
}

}  // namespace gemm
}  // namespace d3d

using namespace d3d;

extern "C" int d3d_gemm_rows64_splits(int N, int K) {
    if (N < gemm::TN || N % gemm::TN || K < gemm::TK || K % gemm::TK) return 1;
    // The most splits whose grid is at most one workgroup per CU (256),
    // leaving every split at least two k steps, and -- below K = 8192, where
    // more splits buy less -- at most 16,384 partial floats per output row:
    // the consumer of the product reads every partial back, about 1 us per
    // 4 MB at 64 rows.  Measured with that consumer (d3d_add_rmsnorm_parts)
    // on rotating HBM-resident weights: 4096 x 12288 at 4 splits 27.6 us
    // against 31.2 at 8 (a full round of two per CU), 4096 x 4096 at 4
    // splits 14.9 against 17.9 at 8, 2048 x 6144 at 8 splits 13.8 against
    // 15.4 at 4 and 16.6 at 16.
    const int tiles = N / gemm::TN;
    int s = 1;
    while (s < gemm::kMaxSplits && tiles * 2 * s <= 256 && K % (gemm::TK * 2 * s) == 0 &&
           K / (2 * s) >= 2 * gemm::TK && (K >= 8192 || (int64_t)2 * s * N <= 16384))
        s *= 2;
    return s;
}

extern "C" int d3d_gemm_rows64_silu_mul(const void* x, const void* w_gate_up, void* y, int M, int H, int K,
                                        void* stream) {
    if (M < 1 || M > 64 || H < 32 || H % 32 || K < gemm::TK || K % gemm::TK) return D3D_E_SHAPE;
    if (!x || !w_gate_up || !y) return D3D_E_NULL;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w_gate_up) % 16) return D3D_E_UNSUPPORTED;
    const dim3 grid(H / 32), block(gemm::NT);
    const size_t lds = gemm::ST * gemm::STAGEB;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    const uint16_t* wp = static_cast<const uint16_t*>(w_gate_up);
    uint16_t* yp = static_cast<uint16_t*>(y);
    switch (K / gemm::TK) {
#define D3D_ROWS64_SILU(n)                                                                                      \
    case n:                                                                                                    \
        hipLaunchKernelGGL((gemm::gemm_rows64_kernel<n, true>), grid, block, lds, s, xp, wp, yp, nullptr, M, 2 * H, K, \
                           K);                                                                                 \
        break;
        D3D_ROWS64_SILU(8) D3D_ROWS64_SILU(16) D3D_ROWS64_SILU(24) D3D_ROWS64_SILU(32) D3D_ROWS64_SILU(48)
        D3D_ROWS64_SILU(64)
#undef D3D_ROWS64_SILU
        default:
            return D3D_E_UNSUPPORTED;
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

extern "C" int d3d_gemm_rows64(const void* x, const void* w, void* y, float* parts, int M, int N, int K,
                               int splits, void* stream) {
    if (M < 1 || M > 64 || N < gemm::TN || N % gemm::TN || K < gemm::TK) return D3D_E_SHAPE;
    if (splits < 1 || splits > gemm::kMaxSplits || K % (gemm::TK * splits)) return D3D_E_SHAPE;
    if (!x || !w || (splits == 1 ? !y : !parts)) return D3D_E_NULL;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16) return D3D_E_UNSUPPORTED;
    const dim3 grid(N / gemm::TN, splits), block(gemm::NT);
    const size_t lds = gemm::ST * gemm::STAGEB;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t* xp = static_cast<const uint16_t*>(x);
    const uint16_t* wp = static_cast<const uint16_t*>(w);
    uint16_t* yp = static_cast<uint16_t*>(y);
    const int KR = K / splits;
    switch (KR / gemm::TK) {
#define D3D_ROWS64_STEPS(n) \
    case n: hipLaunchKernelGGL(gemm::gemm_rows64_kernel<n>, grid, block, lds, s, xp, wp, yp, parts, M, N, K, KR); break;
        D3D_ROWS64_STEPS(1) D3D_ROWS64_STEPS(2) D3D_ROWS64_STEPS(3) D3D_ROWS64_STEPS(4) D3D_ROWS64_STEPS(6)
        D3D_ROWS64_STEPS(8) D3D_ROWS64_STEPS(12) D3D_ROWS64_STEPS(16) D3D_ROWS64_STEPS(24) D3D_ROWS64_STEPS(32)
#undef D3D_ROWS64_STEPS
        default:
            hipLaunchKernelGGL(gemm::gemm_rows64_dma_kernel, grid, block, lds, s, xp, wp, yp, parts, M, N, K, KR);
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
