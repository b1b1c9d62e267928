// Top-k token ids of logits rows for the draft's anchor proposals.
//
// Reference behaviour (D3D repository):
//   serving/backend.py:84-93  Runner._run: per 256-row chunk of hidden
//       states, logits = lm_head(h); greedy = logits.argmax(-1);
//       top = logits.topk(k).indices (k = anchor_num + 1), used by
//       Engine._recover / Engine._predict (serving/engine.py:54-131) to pick
//       the anchor tokens of the packed branches
//
// Order: descending value, equal values by ascending index, so top[0] is
// torch.argmax's first maximum.  NaN entries are never selected.  With
// log_softmax the values are returned as log-probabilities x - logsumexp(x)
// (single/eval_sync.py:763-768, torch.topk of log_softmax: the same ids).
//
// Two kernels: (1) grid (chunks, rows): each workgroup takes k rounds of a
// workgroup argmax over its 4096-entry chunk (each thread holds 16 entries
// in registers and excludes the ones already taken) and writes k (value,
// index) candidates; (2) one workgroup per row merges the chunk candidates
// the same way.  Streaming the logits once is the HBM-bound part.
#include "d3d_common.hpp"
#include "rowstats.hpp"
#include "../../include/d3d_hip.h"

#include <limits.h>

namespace d3d {
namespace topk {

using namespace rows;

constexpr int kMaxK = 64;
constexpr int kMaxCand = 8192;  // chunk candidates per row merged in LDS

struct Cand {
    float v;
    int i;
};

struct Params {
    const void* logits;  // [N, V]
    int N, V, C, k;
    Cand* cand;       // [N][C][k]
    float2* lse;      // [N][C] chunk (max, sum exp(x - max)) when log-probabilities are asked for
    int64_t* ids;     // [N, k]
    float* vals;      // [N, k] (may be null)
};

template <int DT, bool VEC>
__global__ __launch_bounds__(NT) void topk_chunk_kernel(Params P) {
    constexpr int E = Vec<DT>::E;
    const int c = blockIdx.x, n = blockIdx.y;
    __shared__ float sv[NT / kWave];
    __shared__ int si[NT / kWave];
    const void* row = row_ptr<DT>(P.logits, n, P.V);
    const int first = c * kChunk + threadIdx.x * E;
    float x[L];
    load_tile<DT, VEC, true, L>(row, P.V, first, NT * E, -INFINITY, x);
    uint32_t taken = 0;  // bit l: entry l already selected
    for (int r = 0; r < P.k; ++r) {
        float bv = -INFINITY;
        int bi = INT_MAX;
#pragma unroll
        for (int l = 0; l < L; ++l) {
            const int e = tile_index<DT>(first, NT * E, l);
            if (!((taken >> l) & 1u) && e < P.V) argmax_merge(bv, bi, x[l], e);
        }
        float wv = bv;
        int wi = bi;
        block_argmax<NT>(wv, wi, sv, si);
        // The owner of the winning entry excludes it from later rounds.
#pragma unroll
        for (int l = 0; l < L; ++l)
            if (tile_index<DT>(first, NT * E, l) == wi) taken |= 1u << l;
        if (threadIdx.x == 0) P.cand[((size_t)n * P.C + c) * P.k + r] = Cand{wv, wi};
        if (r == 0 && P.lse) {
            // Round 0's winner is the chunk max: the chunk's share of logsumexp.
            float se = 0.f;
            if (wv != -INFINITY) {
#pragma unroll
                for (int l = 0; l < L; ++l)
                    if (tile_index<DT>(first, NT * E, l) < P.V) se += expf(x[l] - wv);
            }
            se = block_sum<NT>(se, sv);
            if (threadIdx.x == 0) P.lse[(size_t)n * P.C + c] = make_float2(wv, se);
        }
    }
}

__global__ __launch_bounds__(NT) void topk_merge_kernel(Params P) {
    const int n = blockIdx.x;
    __shared__ Cand lds[kMaxCand];
    __shared__ float sv[NT / kWave];
    __shared__ int si[NT / kWave];
    const int total = P.C * P.k;
    for (int e = threadIdx.x; e < total; e += NT) lds[e] = P.cand[(size_t)n * total + e];
    float logz = 0.f;
    if (P.lse) {
        // logsumexp over the chunk records, in a fixed order.
        float mx = -INFINITY;
        for (int c = threadIdx.x; c < P.C; c += NT) mx = fmaxf(mx, P.lse[(size_t)n * P.C + c].x);
        mx = block_max<NT>(mx, sv);
        float se = 0.f;
        for (int c = threadIdx.x; c < P.C; c += NT) {
            const float2 t = P.lse[(size_t)n * P.C + c];
            if (t.x != -INFINITY) se += t.y * expf(t.x - mx);
        }
        se = block_sum<NT>(se, sv);
        logz = mx + logf(se);
    }
    __syncthreads();
    for (int r = 0; r < P.k; ++r) {
        float bv = -INFINITY;
        int bi = INT_MAX, bp = -1;
        for (int e = threadIdx.x; e < total; e += NT) {
            const Cand cd = lds[e];
            if (cd.i == INT_MAX) continue;  // taken, or a chunk with fewer than k entries
            const float v0 = bv;
            const int i0 = bi;
            argmax_merge(bv, bi, cd.v, cd.i);
            if (bv != v0 || bi != i0) bp = e;
        }
        float wv = bv;
        int wi = bi;
        block_argmax<NT>(wv, wi, sv, si);
        if (threadIdx.x == 0) {
            P.ids[(size_t)n * P.k + r] = wi == INT_MAX ? -1 : wi;
            if (P.vals) P.vals[(size_t)n * P.k + r] = P.lse ? wv - logz : wv;
        }
        // Token ids are unique among candidates: the holder marks its entry.
        if (bp >= 0 && bi == wi && wi != INT_MAX) lds[bp].i = INT_MAX;
        __syncthreads();
    }
}

}  // namespace topk
}  // namespace d3d

using namespace d3d;

static size_t cand_bytes(int N, int64_t V, int k) {
    const size_t C = (size_t)((V + rows::kChunk - 1) / rows::kChunk);
    return ((size_t)N * C * k * sizeof(topk::Cand) + 255) & ~(size_t)255;
}

extern "C" size_t d3d_topk_workspace_bytes(int N, int64_t V, int k) {
    if (N < 1 || V < 1 || k < 1) return 0;
    const size_t C = (size_t)((V + rows::kChunk - 1) / rows::kChunk);
    return cand_bytes(N, V, k) + (((size_t)N * C * sizeof(float2) + 255) & ~(size_t)255);
}

extern "C" int d3d_topk_rows(const void* logits, int dtype, int N, int64_t V, int k, int log_softmax,
                             int64_t* ids_out, float* vals_out, void* workspace, size_t workspace_bytes,
                             void* stream) {
    using namespace topk;
    if (N < 0 || V < 1 || V > INT_MAX / 2 || k < 1 || k > kMaxK || k > V) return D3D_E_SHAPE;
    if (dtype != D3D_DTYPE_F32 && dtype != D3D_DTYPE_BF16) return D3D_E_DTYPE;
    if (N == 0) return D3D_OK;
    if (N > 65535) return D3D_E_SHAPE;
    if (!logits || !ids_out || !workspace) return D3D_E_NULL;
    Params P;
    P.logits = logits;
    P.N = N;
    P.V = (int)V;
    P.C = (int)((V + rows::kChunk - 1) / rows::kChunk);
    P.k = k;
    if ((int64_t)P.C * k > kMaxCand) return D3D_E_SHAPE;
    if (workspace_bytes < d3d_topk_workspace_bytes(N, V, k)) return D3D_E_WORKSPACE;
    P.cand = static_cast<Cand*>(workspace);
    P.lse = (log_softmax && vals_out)
                ? reinterpret_cast<float2*>(static_cast<char*>(workspace) + cand_bytes(N, V, k))
                : nullptr;
    P.ids = ids_out;
    P.vals = vals_out;
    const size_t esize = dtype == D3D_DTYPE_F32 ? 4 : 2;
    const bool vec = ((uintptr_t)logits % 16 == 0) && ((size_t)V * esize) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 g1(P.C, N);
    if (dtype == D3D_DTYPE_F32) {
        if (vec)
            hipLaunchKernelGGL((topk_chunk_kernel<kF32, true>), g1, dim3(rows::NT), 0, s, P);
        else
            hipLaunchKernelGGL((topk_chunk_kernel<kF32, false>), g1, dim3(rows::NT), 0, s, P);
    } else {
        if (vec)
            hipLaunchKernelGGL((topk_chunk_kernel<kBF16, true>), g1, dim3(rows::NT), 0, s, P);
        else
            hipLaunchKernelGGL((topk_chunk_kernel<kBF16, false>), g1, dim3(rows::NT), 0, s, P);
    }
    hipLaunchKernelGGL(topk_merge_kernel, dim3(N), dim3(rows::NT), 0, s, P);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
