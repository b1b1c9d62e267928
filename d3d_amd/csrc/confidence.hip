// Confidence and top-k unmask for one diffusion-draft denoise iteration.
//
// Reference behaviour (D3D repository):
//   single/eval_sync.py:447-465  _select_transfer: scores = confidence where
//       the block holds MASK_ID (else -1), top-k, block[idx] = x0[idx]
//   single/eval_sync.py:713-717  greedy confidence: x0 = argmax(logits),
//       x0_p = max softmax(logits) probability
//   third_party/sglang/python/sglang/srt/dllm/algorithm/low_confidence.py:32-35
//       the same confidence for SGLang's LowConfidence
//   single/eval_sync.py:287-291, :323-338  greedy _sample_with_prob: the
//       one-hot distribution, so every position's confidence is 1.0 and
//       top-k among masked positions reduces to the tie order
//   single/eval_sync.py:453-462  "dynamic" remasking: the masked positions
//       with confidence >= threshold, at most k of them (the k most
//       confident), or the plain top-k when none reaches the threshold
// Confidence modes: D3D_CONF_MAX_SOFTMAX (the :713-717 metrics confidence,
// SGLang's LowConfidence) or D3D_CONF_ONE_HOT (the reference's greedy
// low_confidence steps: 1.0 everywhere, so the lowest masked positions are
// taken first, the index order in which torch's CUDA top-k gathers tied
// values).  Differences, on purpose: selection is per request (the
// reference applies row 0's indices to every row, eval_sync.py:461-464), and
// ties in confidence go to the lowest position.  With temperature T > 1e-5
// (max-softmax mode only) the confidence is the argmax token's probability
// under softmax(logits / T); x0 stays the argmax.
//
// Two kernels: row statistics of every (request, position) row, streamed once
// in 4096-entry chunks (HBM-bound), then one workgroup per request merges the
// chunk records, computes conf = 1 / sum exp(z - max z) and x0, ranks the
// masked positions and writes the unmasked tokens into the block in place.
#include "d3d_common.hpp"
#include "rowstats.hpp"
#include "../../include/d3d_hip.h"

#include <limits.h>

namespace d3d {
namespace conf {

using namespace rows;

constexpr int kMaxQ = 1024;  // positions per request

struct Params {
    const void* logits;  // [B, Q, V]
    int64_t* block;      // [B, Q]
    int64_t mask_id;
    int k;
    float T;
    int one_hot;      // confidence 1.0 for every position
    int dynamic;      // threshold remasking
    float threshold;
    int Q, V, C;
    RowStat* stats;  // [B][Q][C]
    int64_t* x0;     // [B, Q] (may be null)
    float* conf;     // [B, Q] (may be null)
};

template <int DT, bool VEC>
__global__ __launch_bounds__(NT) void conf_stats_kernel(Params P) {
    constexpr int E = Vec<DT>::E;
    const int c = blockIdx.x, i = blockIdx.y, b = blockIdx.z;
    __shared__ float rf[NT / kWave];
    __shared__ int ri[NT / kWave];
    const void* row = row_ptr<DT>(P.logits, (size_t)b * P.Q + i, P.V);
    const int first = c * kChunk + threadIdx.x * E;
    float x[L];
    load_tile<DT, VEC, true, L>(row, P.V, first, NT * E, fill_value<kLogits>(), x);
    const RowStat st = P.T == 1.0f ? chunk_stats<DT, kLogits, true>(x, first, P.T, true, rf, ri)
                                   : chunk_stats<DT, kLogits, false>(x, first, P.T, true, rf, ri);
    if (threadIdx.x == 0) P.stats[((size_t)b * P.Q + i) * P.C + c] = st;
}

// Number of positions to unmask: k, or with dynamic remasking the count of
// masked positions whose confidence reaches the threshold when that count is
// positive and below k (eval_sync.py:453-462).
__device__ __forceinline__ int transfer_count(int k, int dynamic, int n_confident) {
    return (dynamic && n_confident > 0) ? min(k, n_confident) : k;
}

// Among positions with mask[i], the kk highest confidences (ties: lower
// position; all of them when kk >= their count) take x0 in block; selected
// (may be null) records which positions were unmasked.  Rank of position i:
// the number of masked positions with higher confidence, or equal
// confidence and a lower index.
//
// Wave-parallel: each wave takes 64 candidate positions at a time, one per
// lane, and walks the positions 64 at a time too: its lanes load 64 of them
// (one each) and every candidate counts the ones ranked above it by reading
// those 64 confidences and masks across lanes.  Q <= 64, the draft block's
// size, is one step of each loop and one wave.
__device__ __forceinline__ void rank_and_unmask(int64_t* block, int Q, int k, int n_masked, const uint8_t* mask,
                                                const float* conf, const int* x0, uint8_t* selected) {
    const int kk = min(k, n_masked);
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    for (int i0 = wv * kWave; i0 < Q; i0 += NT) {
        const int i = i0 + lane;
        const bool mi = i < Q && mask[i];
        const float ci = i < Q ? conf[i] : 0.f;
        int rank = 0;
        for (int j0 = 0; j0 < Q; j0 += kWave) {
            const int j = j0 + lane;
            const bool mj = j < Q && mask[j];
            const float cj = j < Q ? conf[j] : 0.f;
            const int tn = min(kWave, Q - j0);  // the same for every lane
#pragma unroll 16
            for (int t = 0; t < tn; ++t) {
                const float c = __shfl(cj, t, kWave);
                const int m = __shfl((int)mj, t, kWave);
                rank += m && (c > ci || (c == ci && j0 + t < i));
            }
        }
        const bool pick = mi && rank < kk;
        if (pick) block[i] = x0[i];
        if (selected && i < Q) selected[i] = pick;
    }
}

// Masked positions and, of those, the ones whose confidence reaches the
// threshold (for "dynamic" remasking), over the workgroup: one ballot per
// wave and a fixed-order sum of the wave counts.
__device__ __forceinline__ int2 count_masked(const uint8_t* mask, const float* conf, int Q, float threshold,
                                             int2* s_w) {
    int n = 0, nc = 0;
    for (int i0 = 0; i0 < Q; i0 += NT) {
        const int i = i0 + (int)threadIdx.x;
        const bool m = i < Q && mask[i];
        const bool c = m && conf[i] >= threshold;
        n += __popcll(__ballot(m));
        nc += __popcll(__ballot(c));
    }
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) s_w[threadIdx.x / kWave] = make_int2(n, nc);
    __syncthreads();
    int2 t = make_int2(0, 0);
#pragma unroll
    for (int w = 0; w < NT / kWave; ++w) {
        t.x += s_w[w].x;
        t.y += s_w[w].y;
    }
    return t;
}

// Top-k unmask with caller-given tokens and confidences (the sampled draft
// path): one workgroup per request.
__global__ __launch_bounds__(NT) void select_transfer_kernel(int64_t* block, int64_t mask_id, int k, int dynamic,
                                                             float threshold, const int64_t* x0, const float* conf,
                                                             uint8_t* selected, int Q) {
    const int b = blockIdx.x;
    __shared__ float sC[kMaxQ];
    __shared__ int sX[kMaxQ];
    __shared__ uint8_t sMask[kMaxQ];
    __shared__ int2 s_w[NT / kWave];
    for (int i = threadIdx.x; i < Q; i += NT) {
        const size_t e = (size_t)b * Q + i;
        sMask[i] = block[e] == mask_id;
        sC[i] = conf[e];
        sX[i] = (int)x0[e];
    }
    __syncthreads();
    const int2 cnt = count_masked(sMask, sC, Q, threshold, s_w);
    rank_and_unmask(block + (size_t)b * Q, Q, transfer_count(k, dynamic, cnt.y), cnt.x, sMask, sC, sX,
                    selected ? selected + (size_t)b * Q : nullptr);
}

__global__ __launch_bounds__(NT) void conf_select_kernel(Params P) {
    const int b = blockIdx.x;
    const int Q = P.Q;
    __shared__ RowStat lds[kMaxStatLds];
    __shared__ float sM[kMaxQ], sS[kMaxQ];
    __shared__ int sArg[kMaxQ];
    __shared__ uint8_t sMask[kMaxQ];
    __shared__ int2 s_w[NT / kWave];

    // Block ids are loaded before the merge so the load overlaps it.
    for (int i = threadIdx.x; i < Q; i += NT) sMask[i] = P.block[(size_t)b * Q + i] == P.mask_id;
    merge_row_stats<kLogits>(P.stats + (size_t)b * Q * P.C, Q, P.C, Q, sM, sS, sArg, lds);
    // The argmax entry's probability is exp(z_max - M) / S = 1 / S (1.0 in
    // one-hot mode).
    for (int i = threadIdx.x; i < Q; i += NT) {
        const float cf = P.one_hot ? 1.0f : 1.0f / sS[i];
        sS[i] = cf;
        if (P.conf) P.conf[(size_t)b * Q + i] = cf;
        if (P.x0) P.x0[(size_t)b * Q + i] = sArg[i];
    }
    __syncthreads();
    const int2 cnt = count_masked(sMask, sS, Q, P.threshold, s_w);
    rank_and_unmask(P.block + (size_t)b * Q, Q, transfer_count(P.k, P.dynamic, cnt.y), cnt.x, sMask, sS, sArg,
                    nullptr);
}

template <int DT, bool VEC>
static hipError_t launch(const Params& P, int B, hipStream_t s) {
    hipLaunchKernelGGL((conf_stats_kernel<DT, VEC>), dim3(P.C, P.Q, B), dim3(NT), 0, s, P);
    hipLaunchKernelGGL(conf_select_kernel, dim3(B), dim3(NT), 0, s, P);
    return hipGetLastError();
}

static int num_chunks(int64_t V) { return (int)((V + kChunk - 1) / kChunk); }

}  // namespace conf
}  // namespace d3d

using namespace d3d;

extern "C" size_t d3d_confidence_workspace_bytes(int B, int Q, int64_t V) {
    if (B < 1 || Q < 1 || V < 1) return 0;
    return ((size_t)B * Q * conf::num_chunks(V) * sizeof(rows::RowStat) + 255) & ~(size_t)255;
}

extern "C" int d3d_select_transfer(int64_t* block_ids, int64_t mask_id, int k, int dynamic, float threshold,
                                   const int64_t* x0, const float* conf, uint8_t* selected_out, int B, int Q,
                                   void* stream) {
    using namespace conf;
    if (B < 1 || B > 65535 || Q < 1 || Q > kMaxQ || k < 0) return D3D_E_SHAPE;
    if (dynamic && !(threshold == threshold)) return D3D_E_VALUE;
    if (!block_ids || !x0 || !conf) return D3D_E_NULL;
    hipLaunchKernelGGL(select_transfer_kernel, dim3(B), dim3(rows::NT), 0, static_cast<hipStream_t>(stream),
                       block_ids, mask_id, k, dynamic ? 1 : 0, threshold, x0, conf, selected_out, Q);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

extern "C" int d3d_confidence_topk_unmask(const void* logits, int dtype, int64_t* block_ids, int64_t mask_id,
                                          int k, float temperature, int conf_mode, int dynamic, float threshold,
                                          int B, int Q, int64_t V, int64_t* x0_out, float* conf_out,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    using namespace conf;
    if (B < 1 || B > 65535 || Q < 1 || Q > kMaxQ || V < 1 || V > (int64_t)kMaxStatLds * kChunk || k < 0)
        return D3D_E_SHAPE;
    if (dtype != D3D_DTYPE_F32 && dtype != D3D_DTYPE_BF16) return D3D_E_DTYPE;
    if (conf_mode != D3D_CONF_MAX_SOFTMAX && conf_mode != D3D_CONF_ONE_HOT) return D3D_E_VALUE;
    // One-hot confidences are the greedy draw's; a sampled draw has its own.
    if (conf_mode == D3D_CONF_ONE_HOT && temperature > 1e-5f) return D3D_E_UNSUPPORTED;
    if (dynamic && !(threshold == threshold)) return D3D_E_VALUE;
    if (!logits || !block_ids || !workspace) return D3D_E_NULL;
    if (workspace_bytes < d3d_confidence_workspace_bytes(B, Q, V)) return D3D_E_WORKSPACE;
    Params P;
    P.logits = logits;
    P.block = block_ids;
    P.mask_id = mask_id;
    P.k = k;
    P.T = temperature > 1e-5f ? temperature : 1.0f;
    P.one_hot = conf_mode == D3D_CONF_ONE_HOT;
    P.dynamic = dynamic ? 1 : 0;
    P.threshold = threshold;
    P.Q = Q;
    P.V = (int)V;
    P.C = num_chunks(V);
    P.stats = static_cast<rows::RowStat*>(workspace);
    P.x0 = x0_out;
    P.conf = conf_out;
    const size_t esize = dtype == D3D_DTYPE_F32 ? 4 : 2;
    const bool vec = ((uintptr_t)logits % 16 == 0) && ((size_t)V * esize) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t err;
    if (dtype == D3D_DTYPE_F32)
        err = vec ? launch<kF32, true>(P, B, s) : launch<kF32, false>(P, B, s);
    else
        err = vec ? launch<kBF16, true>(P, B, s) : launch<kBF16, false>(P, B, s);
    return err == hipSuccess ? D3D_OK : (int)err;
}
