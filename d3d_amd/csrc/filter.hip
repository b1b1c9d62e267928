// Row filters of the draft's proposal distributions, and wide sparse
// supports, over rows of V logits.
//
// Reference behaviour (D3D repository):
//   single/eval_sync.py:292-295  top-k: z = logits.float() / T, entries with
//       z below the k-th largest z are masked out (ties with it are kept)
//   single/eval_sync.py:296-303  top-p: sort z descending, softmax, cumsum;
//       entry j > 0 of the sorted order goes when the cumulative probability
//       of entries 0..j-1 exceeds top_p (the crossing entry is kept)
//   single/eval_sync.py:341-367  _sample_with_sparse_probs: the support is
//       torch.topk(z, S) in descending order (S = V when top_k = 0), the
//       nucleus filter over that order, softmax, a draw from the support
//
// A filter is one record per row, (zf, lim): entry e with scaled logit z is
// kept iff z > zf, or z == zf and e <= lim.  Sorted orders break ties by the
// lower id (the order of a stable descending sort), so a cut through a run
// of equal values keeps its lowest ids.
//
// d3d_row_filter runs one workgroup per row and makes several passes over
// the row (it stays in L2 after the first): the row maximum, an exact radix
// select of the k-th largest value (four 8-bit digit passes of counts over
// order-preserving 32-bit keys), and for top-p a radix descent over the same
// digits with mass histograms: each entry adds w = exp(z - max) as a 64-bit
// fixed-point integer (2^-40 units), so the sums are exact integers and the
// cut does not depend on the order of the atomic adds.  The entry where the
// cumulative mass first exceeds top_p * sum(w) fixes (zf, lim); one more
// pass in id order finds the tie limit when the cut falls inside a run of
// equal values.
//
// Wide supports (S > 64): d3d_support_gather writes each kept entry of the
// exact top-S filter as one 50-bit key ((~key(z)) << 18 | id: ascending
// keys are descending values, ties by ascending id, every key distinct),
// rocPRIM's segmented radix sort orders them, and one workgroup per row
// forms softmax over the support, the nucleus filter in support order and
// the inverse-CDF draw (first s with C_s > u * W, else the last s with
// positive weight).
#include "d3d_common.hpp"
#include "rowstats.hpp"
#include "../../include/d3d_hip.h"

#include <limits.h>

#include <algorithm>
#include <rocprim/device/device_segmented_radix_sort.hpp>

namespace d3d {
namespace filt {

constexpr int NTF = 1024;              // threads per row workgroup
constexpr int kWaves = NTF / kWave;    // 16
constexpr int kIdBits = 18;            // ids < 2^18 in a support key
constexpr int64_t kMaxV = 1 << kIdBits;
constexpr double kFix = 1099511627776.0;  // 2^40: fixed-point unit of the masses

// Order-preserving key of a float: a < b (as floats) iff key(a) < key(b);
// -0 is read as +0 and NaN as the lowest key.
__device__ __forceinline__ uint32_t key_of(float z) {
    if (z != z) return 0u;
    if (z == 0.f) z = 0.f;
    const uint32_t u = __float_as_uint(z);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float float_of(uint32_t k) {
    const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

template <int DT>
__device__ __forceinline__ float scaled(const void* row, int e, float T, bool unit) {
    const float x = rows::load_one<DT>(row, e);
    return unit ? x : x / T;
}

// Calls f(e, z) for every entry of the row; thread t visits e = t, t + NTF, ...
template <int DT, typename F>
__device__ __forceinline__ void for_row(const void* row, int V, float T, bool unit, F&& f) {
    for (int e = threadIdx.x; e < V; e += NTF) f(e, scaled<DT>(row, e, T, unit));
}

__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) s[threadIdx.x / kWave] = v;
    __syncthreads();
    uint32_t t = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += s[w];
    return t;
}

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) s[threadIdx.x / kWave] = v;
    __syncthreads();
    uint64_t t = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) t += s[w];
    return t;
}

__device__ __forceinline__ float block_max_f(float v, float* s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) s[threadIdx.x / kWave] = v;
    __syncthreads();
    float t = s[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) t = fmaxf(t, s[w]);
    return t;
}

__device__ __forceinline__ uint64_t weight_fx(float z, float M) {
    if (!(z > -INFINITY)) return 0;  // -inf and NaN carry no mass
    return (uint64_t)((double)expf(z - M) * kFix);
}

// Id of the q-th entry (1-based, ascending id) with key == v, by a pass in
// id order (rounds of NTF consecutive entries, block-wide exclusive scans of
// the per-round counts).
template <int DT>
__device__ int nth_tie(const void* row, int V, float T, bool unit, uint32_t v, uint32_t q, uint32_t* s_u, int* s_i) {
    uint32_t before = 0;
    for (int base = 0; base < V; base += NTF) {
        const int e = base + threadIdx.x;
        const bool hit = e < V && key_of(scaled<DT>(row, e, T, unit)) == v;
        const uint64_t bal = __ballot(hit);
        const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
        __syncthreads();
        if (lane == 0) s_u[w] = (uint32_t)__popcll(bal);
        __syncthreads();
        uint32_t off = before;
        for (int k = 0; k < w; ++k) off += s_u[k];
        uint32_t total = before;
        for (int k = 0; k < kWaves; ++k) total += s_u[k];
        const uint32_t rank = off + (uint32_t)__popcll(bal & ((1ull << lane) - 1)) + 1;
        if (threadIdx.x == 0) *s_i = -1;
        __syncthreads();
        if (hit && rank == q) *s_i = e;
        __syncthreads();
        if (*s_i >= 0) return *s_i;
        before = total;
    }
    return V - 1;
}

struct FilterParams {
    const void* logits;  // [N, V]
    int V;
    float T;
    int top_k;    // 0: off
    float top_p;  // >= 1: off
    int exact;    // the top-k filter keeps exactly top_k entries (ties by id)
    float* zf;    // [N]
    int32_t* lim; // [N]
};

template <int DT>
__global__ __launch_bounds__(NTF) void row_filter_kernel(FilterParams P) {
    __shared__ uint32_t s_cnt[256];
    __shared__ unsigned long long s_mass[256];
    __shared__ uint32_t s_u[kWaves];
    __shared__ uint64_t s_u64[kWaves];
    __shared__ float s_f[kWaves];
    __shared__ int s_i;
    __shared__ uint32_t s_pick[2];
    const int n = blockIdx.x, V = P.V;
    const void* row = rows::row_ptr<DT>(P.logits, n, V);
    const bool unit = P.T == 1.0f;
    const float T = P.T;

    // Top-k: the key K of the k-th largest entry, by digit-wise descent on
    // counts of the entries that share the digits chosen so far.
    uint32_t K = 0;      // keep key >= K (all ties) unless exact
    int lim_k = INT_MAX;
    const bool use_k = P.top_k > 0 && P.top_k < V;
    if (use_k) {
        uint32_t prefix = 0, mask = 0, need = (uint32_t)P.top_k;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int b = threadIdx.x; b < 256; b += NTF) s_cnt[b] = 0;
            __syncthreads();
            for_row<DT>(row, V, T, unit, [&](int, float z) {
                const uint32_t k = key_of(z);
                if ((k & mask) == prefix) atomicAdd(&s_cnt[(k >> shift) & 255u], 1u);
            });
            __syncthreads();
            if (threadIdx.x == 0) {
                uint32_t acc = 0;
                int b = 255;
                for (; b > 0; --b) {
                    if (acc + s_cnt[b] >= need) break;
                    acc += s_cnt[b];
                }
                s_pick[0] = (uint32_t)b;
                s_pick[1] = need - acc;  // rank of the k-th entry within bin b
            }
            __syncthreads();
            prefix |= s_pick[0] << shift;
            mask |= 255u << shift;
            need = s_pick[1];
            __syncthreads();
        }
        K = prefix;
        // Exactly top_k entries: the `need` lowest ids among the ties at K.
        if (P.exact) lim_k = nth_tie<DT>(row, V, T, unit, K, need, s_u, &s_i);
    }
    float zf = use_k ? float_of(K) : -INFINITY;
    int lim = use_k ? lim_k : INT_MAX;

    if (P.top_p < 1.0f) {
        auto kept = [&](int e, float z) {
            const uint32_t k = key_of(z);
            return !use_k || k > K || (k == K && e <= lim_k);
        };
        // Row maximum and total mass over the entries the top-k filter keeps.
        float mx = -INFINITY;
        for_row<DT>(row, V, T, unit, [&](int e, float z) {
            if (kept(e, z) && z > mx) mx = z;
        });
        const float M = block_max_f(mx, s_f);
        uint64_t tot = 0;
        for_row<DT>(row, V, T, unit, [&](int e, float z) {
            if (kept(e, z)) tot += weight_fx(z, M);
        });
        const uint64_t S = block_sum_u64(tot, s_u64);
        const uint64_t target = (uint64_t)((double)P.top_p * (double)S);
        // The largest key v with mass(key >= v) > target: digit descent on
        // the mass of the entries that share the digits chosen so far; A is
        // the mass strictly above the current range.
        uint32_t prefix = 0, mask = 0;
        uint64_t A = 0;
        bool cut = true;
        for (int shift = 24; shift >= 0 && cut; shift -= 8) {
            for (int b = threadIdx.x; b < 256; b += NTF) s_mass[b] = 0;
            __syncthreads();
            for_row<DT>(row, V, T, unit, [&](int e, float z) {
                const uint32_t k = key_of(z);
                if ((k & mask) == prefix && kept(e, z)) {
                    const uint64_t w = weight_fx(z, M);
                    if (w) atomicAdd(&s_mass[(k >> shift) & 255u], (unsigned long long)w);
                }
            });
            __syncthreads();
            if (threadIdx.x == 0) {
                uint64_t acc = 0;
                int b = 255;
                for (; b >= 0; --b) {
                    if (A + acc + s_mass[b] > target) break;
                    acc += s_mass[b];
                }
                s_pick[0] = b < 0 ? 0xffffffffu : (uint32_t)b;
                s_u64[0] = A + acc;
            }
            __syncthreads();
            if (s_pick[0] == 0xffffffffu) {
                cut = false;  // rounding left the whole mass at or below target
            } else {
                prefix |= s_pick[0] << shift;
                mask |= 255u << shift;
                A = s_u64[0];
            }
            __syncthreads();
        }
        if (cut) {
            // Entries with key == prefix all weigh w; the cut keeps the first
            // q of them (ascending id): A + q w > target >= A + (q - 1) w.
            const float zc = float_of(prefix);
            const uint64_t w = weight_fx(zc, M);
            const uint64_t q = w ? (target - A) / w + 1 : 1;
            zf = zc;
            // Every entry with key == prefix >= K passes the top-k filter
            // (ties with the k-th value are kept), so the count runs over all.
            lim = nth_tie<DT>(row, V, T, unit, prefix, (uint32_t)q, s_u, &s_i);
        }
    }
    if (threadIdx.x == 0) {
        P.zf[n] = zf;
        P.lim[n] = lim;
    }
}

// Wide supports ---------------------------------------------------------------

// Workgroup (chunk, row): the kept entries of its 4096-entry chunk, as
// support keys, at consecutive slots reserved with one atomic per chunk.
template <int DT>
__global__ __launch_bounds__(rows::NT) void support_gather_kernel(const void* logits, int V, float T,
                                                                  const float* zf, const int32_t* lim, int S,
                                                                  uint64_t* keys, uint32_t* counters) {
    constexpr int NT = rows::NT;
    const int c = blockIdx.x, n = blockIdx.y;
    const void* row = rows::row_ptr<DT>(logits, n, V);
    const bool unit = T == 1.0f;
    const float f = zf[n];
    const int l = lim[n];
    const uint32_t kf = key_of(f);
    __shared__ uint32_t s_w[NT / kWave];
    __shared__ uint32_t s_base;
    constexpr int PER = rows::kChunk / NT;  // 16 entries per thread
    uint64_t mine[PER];
    uint32_t cnt = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = c * rows::kChunk + j * NT + threadIdx.x;
        mine[j] = ~0ull;
        if (e < V) {
            const uint32_t k = key_of(scaled<DT>(row, e, T, unit));
            if (k > kf || (k == kf && e <= l)) {
                mine[j] = ((uint64_t)(~k) << kIdBits) | (uint64_t)e;
                ++cnt;
            }
        }
    }
    // Exclusive offset of this thread among the chunk's kept entries.
    uint32_t incl = cnt;
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += t;
    }
    if (lane == kWave - 1) s_w[w] = incl;
    __syncthreads();
    uint32_t off = incl - cnt, total = 0;
#pragma unroll
    for (int k = 0; k < NT / kWave; ++k) {
        if (k < w) off += s_w[k];
        total += s_w[k];
    }
    if (threadIdx.x == 0) s_base = total ? atomicAdd(&counters[n], total) : 0u;
    __syncthreads();
    uint64_t* out = keys + (size_t)n * S;
    uint32_t slot = s_base + off;
#pragma unroll
    for (int j = 0; j < PER; ++j)
        if (mine[j] != ~0ull) {
            if (slot < (uint32_t)S) out[slot] = mine[j];  // the filter keeps exactly S
            ++slot;
        }
}

__device__ __forceinline__ float key_value(uint64_t k) {
    return float_of(~(uint32_t)(k >> kIdBits));
}

// Inclusive scan over the workgroup in thread order.
__device__ __forceinline__ float block_incl(float v, float* s, float* tot) {
    const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const float t = __shfl_up(v, o, kWave);
        if (lane >= o) v += t;
    }
    __syncthreads();
    if (lane == kWave - 1) s[w] = v;
    __syncthreads();
    float off = 0.f, t = 0.f;
#pragma unroll
    for (int k = 0; k < kWaves; ++k) {
        if (k < w) off += s[k];
        t += s[k];
    }
    *tot = t;
    return v + off;
}

// One workgroup per row over its sorted support keys [S]: ids, softmax over
// the support (max = the first value), the nucleus filter in support order,
// the draw.  A slot the gather left unwritten (only a NaN logit can leave
// the filter short of S entries) holds ~0: weight 0, id -1.
__global__ __launch_bounds__(NTF) void support_draw_kernel(const uint64_t* keys, int S, float top_p,
                                                           const float* u, int64_t* tok, int64_t* ids_out,
                                                           float* probs_out, float* tok_prob) {
    __shared__ float s_w[kWaves];
    __shared__ int s_i[2];
    const int n = blockIdx.x;
    const uint64_t* k = keys + (size_t)n * S;
    int64_t* ids = ids_out + (size_t)n * S;
    float* probs = probs_out + (size_t)n * S;
    const float M = key_value(k[0]);
    auto weight = [&](int s) {
        const uint64_t kk = k[s];
        const float z = key_value(kk);
        return (kk != ~0ull && z > -INFINITY) ? expf(z - M) : 0.f;
    };
    // Z = sum of the weights, in a fixed order.
    float part = 0.f;
    for (int s = threadIdx.x; s < S; s += NTF) part += weight(s);
    float Z;
    block_incl(part, s_w, &Z);
    // Nucleus filter: entry s > 0 goes when the inclusive probability of
    // entries 0..s-1 exceeds top_p; `keep` is the kept prefix length.
    int keep = S;
    if (top_p < 1.0f && Z > 0.f) {
        float carry = 0.f;
        if (threadIdx.x == 0) s_i[0] = S;
        __syncthreads();
        for (int base = 0; base < S; base += NTF) {
            const int s = base + threadIdx.x;
            const float p = s < S ? weight(s) / Z : 0.f;
            float t;
            const float incl = carry + block_incl(p, s_w, &t);
            if (s < S && s > 0 && incl - p > top_p) atomicMin(&s_i[0], s);
            __syncthreads();
            carry += t;
            if (s_i[0] < S) break;
        }
        keep = s_i[0];
        __syncthreads();
    }
    float Zk = Z;
    if (keep < S) {
        part = 0.f;
        for (int s = threadIdx.x; s < keep; s += NTF) part += weight(s);
        block_incl(part, s_w, &Zk);
    }
    auto prob = [&](int s) { return (s < keep && Zk > 0.f) ? weight(s) / Zk : 0.f; };
    float tot_p = 0.f;
    part = 0.f;
    for (int s = threadIdx.x; s < S; s += NTF) {
        const float p = prob(s);
        ids[s] = k[s] == ~0ull ? -1 : (int64_t)(k[s] & ((1ull << kIdBits) - 1));
        probs[s] = p;
        part += p;
    }
    block_incl(part, s_w, &tot_p);
    // Draw in support order over the same probabilities.
    const float target = u[n] * tot_p;
    float carry = 0.f;
    if (threadIdx.x == 0) {
        s_i[0] = INT_MAX;
        s_i[1] = -1;
    }
    __syncthreads();
    for (int base = 0; base < S; base += NTF) {
        const int s = base + threadIdx.x;
        const float p = s < S ? prob(s) : 0.f;
        float t;
        const float incl = carry + block_incl(p, s_w, &t);
        if (s < S && p > 0.f) {
            atomicMax(&s_i[1], s);
            if (incl > target) atomicMin(&s_i[0], s);
        }
        __syncthreads();
        carry += t;
        if (s_i[0] != INT_MAX) break;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const int pick = s_i[0] != INT_MAX ? s_i[0] : s_i[1];
        tok[n] = pick >= 0 ? (int64_t)(k[pick] & ((1ull << kIdBits) - 1)) : (int64_t)D3D_TOKEN_EMPTY_DISTRIBUTION;
        if (tok_prob) tok_prob[n] = pick >= 0 ? prob(pick) : 0.f;
    }
}

struct SupportLayout {
    size_t keys_in, keys_out, counters, offsets, temp, temp_bytes, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static hipError_t sort_temp_bytes(int N, int S, size_t* bytes) {
    *bytes = 0;
    return rocprim::segmented_radix_sort_keys(nullptr, *bytes, (const uint64_t*)nullptr, (uint64_t*)nullptr,
                                              (unsigned int)((size_t)N * S), (unsigned int)N, (const int*)nullptr,
                                              (const int*)nullptr, 0, 32 + kIdBits, (hipStream_t)0, false);
}

static SupportLayout support_layout(int N, int S, size_t temp) {
    SupportLayout l;
    const size_t keys = align256((size_t)N * S * sizeof(uint64_t));
    l.keys_in = 0;
    l.keys_out = keys;
    l.counters = 2 * keys;
    l.offsets = l.counters + align256((size_t)N * sizeof(uint32_t));
    l.temp = l.offsets + align256((size_t)(N + 1) * sizeof(int));
    l.temp_bytes = temp;
    l.total = l.temp + align256(temp);
    return l;
}

// Per-row slot counters at 0, segment offsets n * S, every key slot ~0.
__global__ void support_setup_kernel(uint32_t* counters, int* offsets, uint64_t* keys, int N, int S) {
    const size_t total = (size_t)N * S;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x)
        keys[i] = ~0ull;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < N) counters[i] = 0;
    if (i <= N) offsets[i] = i * S;
}

}  // namespace filt
}  // namespace d3d

using namespace d3d;

extern "C" int d3d_row_filter(const void* logits, int dtype, int N, int64_t V, float temperature, int top_k,
                              float top_p, float* zfloor_out, int32_t* zlimit_out, void* stream) {
    using namespace filt;
    if (N < 0 || N > 65535 || V < 1 || V > (int64_t)INT_MAX / 2 || top_k < 0) return D3D_E_SHAPE;
    if (dtype != D3D_DTYPE_F32 && dtype != D3D_DTYPE_BF16) return D3D_E_DTYPE;
    if (!(temperature > 1e-5f)) return D3D_E_UNSUPPORTED;
    if (!(top_p > 0.f && top_p <= 1.f)) return D3D_E_VALUE;
    if (N == 0) return D3D_OK;
    if (!logits || !zfloor_out || !zlimit_out) return D3D_E_NULL;
    FilterParams P{logits, (int)V, temperature, top_k, top_p, 0, zfloor_out, zlimit_out};
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == D3D_DTYPE_F32)
        hipLaunchKernelGGL(row_filter_kernel<kF32>, dim3(N), dim3(NTF), 0, s, P);
    else
        hipLaunchKernelGGL(row_filter_kernel<kBF16>, dim3(N), dim3(NTF), 0, s, P);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

extern "C" size_t d3d_support_workspace_bytes(int N, int S) {
    using namespace filt;
    if (N < 1 || S < 1) return 0;
    size_t temp = 0;
    if (sort_temp_bytes(N, S, &temp) != hipSuccess) return 0;
    return support_layout(N, S, temp).total;
}

extern "C" int d3d_sample_support_wide(const void* logits, int dtype, int N, int64_t V, float temperature, int S,
                                       float top_p, const float* uniforms, int64_t* tokens_out,
                                       int64_t* support_ids_out, float* support_probs_out, float* token_probs_out,
                                       void* workspace, size_t workspace_bytes, void* stream) {
    using namespace filt;
    if (N < 0 || N > 65535 || V < 1 || V > kMaxV || S < 1 || S > V) return D3D_E_SHAPE;
    if ((size_t)N * S > (size_t)UINT_MAX) return D3D_E_SHAPE;
    if (dtype != D3D_DTYPE_F32 && dtype != D3D_DTYPE_BF16) return D3D_E_DTYPE;
    if (!(temperature > 1e-5f)) return D3D_E_UNSUPPORTED;
    if (!(top_p > 0.f && top_p <= 1.f)) return D3D_E_VALUE;
    if (N == 0) return D3D_OK;
    if (!logits || !uniforms || !tokens_out || !support_ids_out || !support_probs_out || !workspace)
        return D3D_E_NULL;
    size_t temp = 0;
    hipError_t err = sort_temp_bytes(N, S, &temp);
    if (err != hipSuccess) return (int)err;
    const SupportLayout lay = support_layout(N, S, temp);
    if (workspace_bytes < lay.total) return D3D_E_WORKSPACE;
    char* ws = static_cast<char*>(workspace);
    uint64_t* kin = reinterpret_cast<uint64_t*>(ws + lay.keys_in);
    uint64_t* kout = reinterpret_cast<uint64_t*>(ws + lay.keys_out);
    uint32_t* counters = reinterpret_cast<uint32_t*>(ws + lay.counters);
    int* offsets = reinterpret_cast<int*>(ws + lay.offsets);
    // The exact top-S filter's (zf, lim) live in the keys_out region until
    // the gather has read them (the sort writes keys_out afterwards).
    float* zf = reinterpret_cast<float*>(kout);
    int32_t* lim = reinterpret_cast<int32_t*>(kout) + N;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const size_t slots = (size_t)N * S;
    const int setup_blocks = (int)std::min<size_t>(1024, std::max<size_t>((N + 1 + 255) / 256, (slots + 255) / 256));
    hipLaunchKernelGGL(support_setup_kernel, dim3(setup_blocks), dim3(256), 0, s, counters, offsets, kin, N, S);
    FilterParams P{logits, (int)V, temperature, S < V ? S : 0, 1.0f, 1, zf, lim};
    const int C = (int)((V + rows::kChunk - 1) / rows::kChunk);
    if (S == V) {
        // The whole vocabulary: every entry is kept (zf = -inf keeps all but
        // NaN, which the key maps below -inf; those are dropped).
        FilterParams Q = P;
        Q.top_k = 0;
        if (dtype == D3D_DTYPE_F32)
            hipLaunchKernelGGL(row_filter_kernel<kF32>, dim3(N), dim3(NTF), 0, s, Q);
        else
            hipLaunchKernelGGL(row_filter_kernel<kBF16>, dim3(N), dim3(NTF), 0, s, Q);
    } else if (dtype == D3D_DTYPE_F32) {
        hipLaunchKernelGGL(row_filter_kernel<kF32>, dim3(N), dim3(NTF), 0, s, P);
    } else {
        hipLaunchKernelGGL(row_filter_kernel<kBF16>, dim3(N), dim3(NTF), 0, s, P);
    }
    if (dtype == D3D_DTYPE_F32)
        hipLaunchKernelGGL(support_gather_kernel<kF32>, dim3(C, N), dim3(rows::NT), 0, s, logits, (int)V,
                           temperature, zf, lim, S, kin, counters);
    else
        hipLaunchKernelGGL(support_gather_kernel<kBF16>, dim3(C, N), dim3(rows::NT), 0, s, logits, (int)V,
                           temperature, zf, lim, S, kin, counters);
    err = hipGetLastError();
    if (err != hipSuccess) return (int)err;
    size_t tb = lay.temp_bytes;
    err = rocprim::segmented_radix_sort_keys(ws + lay.temp, tb, kin, kout, (unsigned int)((size_t)N * S),
                                             (unsigned int)N, offsets, offsets + 1, 0, 32 + kIdBits, s, false);
    if (err != hipSuccess) return (int)err;
    hipLaunchKernelGGL(support_draw_kernel, dim3(N), dim3(NTF), 0, s, kout, S, top_p, uniforms, tokens_out,
                       support_ids_out, support_probs_out, token_probs_out);
    err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
