// Fused per-layer glue of the Qwen3-shaped target and draft forwards.
//
// Each kernel replaces a chain of small tensor operations with one pass:
//
//   add_rmsnorm      residual += x (rounded to bf16), out = RMSNorm(sum) * w
//                    serving/vendor/ssd/layers/layernorm.py:53-98 (RMSDNorm:
//                    fp32 sum and statistics, bf16 normalised value times a
//                    bf16 weight)
//   qk_rope_append   per token: q/k head RMSNorm (RMSHeadNorm,
//                    layernorm.py:1-52), rotary embedding, q written out, k and
//                    v appended to the paged cache at the token's slot
//                    (serving/vendor/ssd/layers/attention.py:21-22).  Target
//                    RoPE rotates in fp32 (rotary_embedding.py:6-16); draft
//                    RoPE follows models/d3d/modeling_d3d.py:164-187 with cos
//                    and sin rounded to bf16 and each product rounded to bf16.
//   silu_mul         out = silu(gate) * up computed in fp32 and rounded once
//                    to bf16, as the compiled SiluAndMul of
//                    serving/vendor/ssd/layers/activation.py:6-14 evaluates it
//
// Rows are bf16; the head dim is 128, split between lane l (entry l) and
// lane l + 64 of a wave (entry l + 64), which are exactly the pairs the
// rotate-half RoPE mixes.
//
// The *_parts forms take their GEMM input as the fp32 partials of a K-split
// GEMM (d3d_gemm_rows64, [splits][T][width]): each entry is the partials
// summed in split order and rounded to bf16, the value a bf16 GEMM output
// holds, and then everything proceeds as in the bf16 form.
#include "d3d_common.hpp"
#include "../../include/d3d_hip.h"

namespace d3d {
namespace layers {

constexpr int NT = 256;
constexpr int HD = 128;  // head dim

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even, on the convert unit (v_cvt_pk_bf16_f32,
// two values per instruction): the bits f32_to_bf16_bits gives for every
// input but NaN, which stays a NaN.  The kernels here are bound by their
// VALU work, of which the rounding was the largest part.
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ uint16_t bits1(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float bf(uint16_t b) { return bf16_bits_to_f32(b); }
__device__ __forceinline__ float rbf(float f) { return bf16_bits_to_f32(bits1(f)); }
// Both values of a pair rounded to bf16 with one conversion.
__device__ __forceinline__ void rbf2(float& a, float& b) {
    const uint32_t p = pack2(a, b);
    a = __uint_as_float(p << 16);
    b = __uint_as_float(p & 0xffff0000u);
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Entries e .. e + 7 of a K-split product: the fp32 partials summed in
// split order, rounded to bf16 and packed in pairs like a bf16 row.
__device__ __forceinline__ u32x4 sum_parts8(const float* parts, int splits, size_t stride, size_t e) {
    float a[8];
    {
        const f32x4 p0 = *reinterpret_cast<const f32x4*>(parts + e);
        const f32x4 p1 = *reinterpret_cast<const f32x4*>(parts + e + 4);
        a[0] = p0.x; a[1] = p0.y; a[2] = p0.z; a[3] = p0.w;
        a[4] = p1.x; a[5] = p1.y; a[6] = p1.z; a[7] = p1.w;
    }
    for (int sp = 1; sp < splits; ++sp) {
        const float* q = parts + (size_t)sp * stride + e;
        const f32x4 p0 = *reinterpret_cast<const f32x4*>(q);
        const f32x4 p1 = *reinterpret_cast<const f32x4*>(q + 4);
        a[0] += p0.x; a[1] += p0.y; a[2] += p0.z; a[3] += p0.w;
        a[4] += p1.x; a[5] += p1.y; a[6] += p1.z; a[7] += p1.w;
    }
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h)
        o[h] = pack2(a[2 * h], a[2 * h + 1]);
    return o;
}

// One entry of a K-split product, as bf16 bits.
__device__ __forceinline__ uint16_t sum_parts1(const float* parts, int splits, size_t stride, size_t e) {
    float a = parts[e];
    for (int sp = 1; sp < splits; ++sp) a += parts[(size_t)sp * stride + e];
    return bits1(a);
}

// One workgroup per row of H entries (H a multiple of 8).  One wave per row
// (no block reduction) measured slower -- 5.1 -> 7.2 us at 1088 x 2048 and
// 3.8 -> 8.8 us at 64 x 4096 -- because it leaves a quarter of the waves to
// hide the load latency.
template <bool PARTS>
__global__ __launch_bounds__(NT) void add_rmsnorm_kernel(const uint16_t* __restrict__ x, const float* __restrict__ parts,
                                                         int splits, size_t stride, uint16_t* residual,
                                                         const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                         int H, float eps) {
    const size_t row = blockIdx.x;
    __shared__ float red[NT / kWave];
    constexpr int kMaxVec = 4;  // up to 4 vectors of 8 per thread: H <= 8192
    float v[kMaxVec][8];
    u32x4 wreg[kMaxVec];  // the weights load with the row, not after the reduction
    const int nvec = H / 8;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxVec; ++j) {
        const int vi = threadIdx.x + j * NT;
        if (vi >= nvec) break;
        const size_t off = row * H + vi * 8;
        wreg[j] = *reinterpret_cast<const u32x4*>(w + vi * 8);
        const u32x4 r = *reinterpret_cast<const u32x4*>(residual + off);
        u32x4 a = {0u, 0u, 0u, 0u};
        if constexpr (PARTS) a = sum_parts8(parts, splits, stride, off);
        else if (x) a = *reinterpret_cast<const u32x4*>(x + off);
        u32x4 rs;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            float lo = bf16_bits_to_f32(r[h] & 0xffffu), hi = bf16_bits_to_f32(r[h] >> 16);
            if (PARTS || x) {
                lo += bf16_bits_to_f32(a[h] & 0xffffu);
                hi += bf16_bits_to_f32(a[h] >> 16);
            }
            v[j][2 * h] = lo;
            v[j][2 * h + 1] = hi;
            ss += lo * lo + hi * hi;
            rs[h] = pack2(lo, hi);
        }
        if (PARTS || x) *reinterpret_cast<u32x4*>(residual + off) = rs;
    }
    const float tot = block_sum<NT>(ss, red);
    const float rstd = rsqrtf(tot / (float)H + eps);
#pragma unroll
    for (int j = 0; j < kMaxVec; ++j) {
        const int vi = threadIdx.x + j * NT;
        if (vi >= nvec) break;
        const size_t off = row * H + vi * 8;
        const u32x4 wv = wreg[j];
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            float lo = v[j][2 * h] * rstd, hi = v[j][2 * h + 1] * rstd;
            rbf2(lo, hi);
            o[h] = pack2(lo * bf16_bits_to_f32(wv[h] & 0xffffu), hi * bf16_bits_to_f32(wv[h] >> 16));
        }
        *reinterpret_cast<u32x4*>(out + off) = o;
    }
}

// One wave per (token, head): grid (tokens, ceil(heads / 4)).  A workgroup
// per token with 16-byte vectors (eight lanes per head, cos / sin once per
// token in LDS) measured 10.9 -> 9.5 us at 1088 draft rows but 2.8 -> 3.7 us
// at 64 target rows, where more waves hide the latency.  Query heads
// (norm + rope -> q_out), key heads (norm + rope -> k_cache) and value heads
// (copy -> v_cache).  Lane l holds entries l and l + 64 of a head, the pair
// the rotate-half RoPE mixes, and computes that pair's cos / sin itself.
template <bool DRAFT_ROPE, bool PARTS>
__global__ __launch_bounds__(NT) void qk_rope_append_kernel(
    const uint16_t* __restrict__ qkv, const float* __restrict__ parts, int splits, size_t stride,
    const int64_t* __restrict__ positions, const uint16_t* __restrict__ qn,
    const uint16_t* __restrict__ kn, const float* __restrict__ inv_freq, uint16_t* __restrict__ q_out,
    uint16_t* k_cache, uint16_t* v_cache, const int64_t* __restrict__ slots, int Hq, int Hkv, float eps,
    int64_t num_slots) {
    const size_t t = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int h = blockIdx.y * (NT / kWave) + (threadIdx.x >> 6);
    const int heads = Hq + 2 * Hkv;
    if (h >= heads) return;  // whole wave; no barrier in this kernel
    // Every load of this wave at once.
    const size_t e = (t * (size_t)heads + h) * HD;
    uint16_t a, b;
    if constexpr (PARTS) {
        a = sum_parts1(parts, splits, stride, e + lane);
        b = sum_parts1(parts, splits, stride, e + lane + 64);
    } else {
        a = qkv[e + lane];
        b = qkv[e + lane + 64];
    }
    const int64_t slot = slots[t];
    const bool store = slot >= 0 && slot < num_slots;
    if (h >= Hq + Hkv) {  // value head: copy into the cache
        if (store) {
            uint16_t* dst = v_cache + ((size_t)slot * Hkv + (h - Hq - Hkv)) * HD;
            dst[lane] = a;
            dst[lane + 64] = b;
        }
        return;
    }
    const bool is_q = h < Hq;
    const uint16_t* nw = is_q ? qn : kn;
    const float w0 = bf(nw[lane]), w1 = bf(nw[lane + 64]);
    const int64_t pos = positions[t];
    const float f = (float)pos * inv_freq[lane];
    const float x0 = bf(a), x1 = bf(b);
    const float rstd = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / (float)HD + eps);
    float y0 = x0 * rstd, y1 = x1 * rstd;
    rbf2(y0, y1);
    y0 *= w0;
    y1 *= w1;
    rbf2(y0, y1);
    // cos / sin of this lane's frequency (entries lane and lane + 64).
    const float cs = cosf(f), sn = sinf(f);
    float o0, o1;
    if constexpr (DRAFT_ROPE) {
        float c = cs, s = sn;
        rbf2(c, s);
        float p0 = y0 * c, p1 = -y1 * s, p2 = y1 * c, p3 = y0 * s;
        rbf2(p0, p1);
        rbf2(p2, p3);
        o0 = p0 + p1;
        o1 = p2 + p3;
    } else {
        o0 = y0 * cs - y1 * sn;
        o1 = y1 * cs + y0 * sn;
    }
    uint16_t* dst;
    if (is_q) {
        dst = q_out + (t * Hq + h) * HD;
    } else {
        if (!store) return;
        dst = k_cache + ((size_t)slot * Hkv + (h - Hq)) * HD;
    }
    const uint32_t ob = pack2(o0, o1);
    dst[lane] = (uint16_t)(ob & 0xffffu);
    dst[lane + 64] = (uint16_t)(ob >> 16);
}

// silu(g) * u of 8 bf16 columns (16-byte vectors).
__device__ __forceinline__ void silu_mul_vec(const uint16_t* gp, const uint16_t* up, uint16_t* op) {
    const u32x4 g = *reinterpret_cast<const u32x4*>(gp);
    const u32x4 u = *reinterpret_cast<const u32x4*>(up);
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        float r[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float gv = bf16_bits_to_f32(k ? (g[h] >> 16) : (g[h] & 0xffffu));
            const float uv = bf16_bits_to_f32(k ? (u[h] >> 16) : (u[h] & 0xffffu));
            r[k] = gv / (1.0f + expf(-gv)) * uv;
        }
        o[h] = pack2(r[0], r[1]);
    }
    *reinterpret_cast<u32x4*>(op) = o;
}

// out[t, i] = silu(gate[t, i]) * up[t, i] with gate_up = [gate | up] per row.
// Thread (x, y) takes 8-column vector x of rows y, y + gridDim.y, ... (no
// per-thread division).
__global__ __launch_bounds__(NT) void silu_mul_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                      int M, int T) {
    const int c = blockIdx.x * NT + threadIdx.x;
    if (c >= M / 8) return;
    for (int t = blockIdx.y; t < T; t += gridDim.y) {
        silu_mul_vec(gu + (size_t)t * 2 * M + (size_t)c * 8, gu + (size_t)t * 2 * M + M + (size_t)c * 8,
                     out + (size_t)t * M + (size_t)c * 8);
    }
}

}  // namespace layers
}  // namespace d3d

using namespace d3d;

// add_rmsnorm and silu_mul move rows as 16-byte vectors.
static bool unaligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 != 0; }

static int add_rmsnorm(const void* x, const float* parts, int splits, void* residual, const void* weight, void* out,
                       int T, int H, float eps, void* stream) {
    if (T < 0 || H < 8 || H % 8 || H > 8 * 4 * layers::NT) return D3D_E_SHAPE;
    if (T == 0) return D3D_OK;
    if (!residual || !weight || !out) return D3D_E_NULL;
    if (unaligned16(x) || unaligned16(parts) || unaligned16(residual) || unaligned16(weight) || unaligned16(out))
        return D3D_E_UNSUPPORTED;
    const size_t stride = (size_t)T * H;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (parts)
        hipLaunchKernelGGL(layers::add_rmsnorm_kernel<true>, dim3(T), dim3(layers::NT), 0, s, nullptr, parts, splits,
                           stride, static_cast<uint16_t*>(residual), static_cast<const uint16_t*>(weight),
                           static_cast<uint16_t*>(out), H, eps);
    else
        hipLaunchKernelGGL(layers::add_rmsnorm_kernel<false>, dim3(T), dim3(layers::NT), 0, s,
                           static_cast<const uint16_t*>(x), nullptr, 0, stride, static_cast<uint16_t*>(residual),
                           static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(out), H, eps);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

extern "C" int d3d_add_rmsnorm(const void* x, void* residual, const void* weight, void* out, int T, int H,
                               float eps, void* stream) {
    return add_rmsnorm(x, nullptr, 0, residual, weight, out, T, H, eps, stream);
}

extern "C" int d3d_add_rmsnorm_parts(const float* parts, int splits, void* residual, const void* weight, void* out,
                                     int T, int H, float eps, void* stream) {
    if (splits < 1) return D3D_E_SHAPE;
    if (!parts) return D3D_E_NULL;
    return add_rmsnorm(nullptr, parts, splits, residual, weight, out, T, H, eps, stream);
}

static int qk_rope_append(const void* qkv, const float* parts, int splits, const int64_t* positions,
                          const void* q_norm_w, const void* k_norm_w, const float* inv_freq, void* q_out,
                          void* k_cache, void* v_cache, const int64_t* slot_mapping, int T, int Hq, int Hkv, int D,
                          float eps, int draft_rope, int64_t num_slots, void* stream) {
    if (T < 0 || Hq < 1 || Hkv < 1 || num_slots < 1) return D3D_E_SHAPE;
    if (D != layers::HD) return D3D_E_UNSUPPORTED;
    if (T == 0) return D3D_OK;
    if ((!qkv && !parts) || !positions || !q_norm_w || !k_norm_w || !inv_freq || !q_out || !k_cache || !v_cache ||
        !slot_mapping)
        return D3D_E_NULL;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto* a = static_cast<const uint16_t*>(qkv);
    const size_t stride = (size_t)T * (Hq + 2 * Hkv) * layers::HD;
    const dim3 grid(T, (Hq + 2 * Hkv + layers::NT / kWave - 1) / (layers::NT / kWave));
    const auto* qn = static_cast<const uint16_t*>(q_norm_w);
    const auto* kn = static_cast<const uint16_t*>(k_norm_w);
    auto* qo = static_cast<uint16_t*>(q_out);
    auto* kc = static_cast<uint16_t*>(k_cache);
    auto* vc = static_cast<uint16_t*>(v_cache);
    if (parts) {
        if (draft_rope)
            hipLaunchKernelGGL((layers::qk_rope_append_kernel<true, true>), grid, dim3(layers::NT), 0, s, nullptr,
                               parts, splits, stride, positions, qn, kn, inv_freq, qo, kc, vc, slot_mapping, Hq, Hkv,
                               eps, num_slots);
        else
            hipLaunchKernelGGL((layers::qk_rope_append_kernel<false, true>), grid, dim3(layers::NT), 0, s, nullptr,
                               parts, splits, stride, positions, qn, kn, inv_freq, qo, kc, vc, slot_mapping, Hq, Hkv,
                               eps, num_slots);
    } else {
        if (draft_rope)
            hipLaunchKernelGGL((layers::qk_rope_append_kernel<true, false>), grid, dim3(layers::NT), 0, s, a,
                               nullptr, 0, stride, positions, qn, kn, inv_freq, qo, kc, vc, slot_mapping, Hq, Hkv,
                               eps, num_slots);
        else
            hipLaunchKernelGGL((layers::qk_rope_append_kernel<false, false>), grid, dim3(layers::NT), 0, s, a,
                               nullptr, 0, stride, positions, qn, kn, inv_freq, qo, kc, vc, slot_mapping, Hq, Hkv,
                               eps, num_slots);
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

extern "C" int d3d_qk_rope_append(const void* qkv, const int64_t* positions, const void* q_norm_w,
                                  const void* k_norm_w, const float* inv_freq, void* q_out, void* k_cache,
                                  void* v_cache, const int64_t* slot_mapping, int T, int Hq, int Hkv, int D,
                                  float eps, int draft_rope, int64_t num_slots, void* stream) {
    if (!qkv) return D3D_E_NULL;
    return qk_rope_append(qkv, nullptr, 0, positions, q_norm_w, k_norm_w, inv_freq, q_out, k_cache, v_cache,
                          slot_mapping, T, Hq, Hkv, D, eps, draft_rope, num_slots, stream);
}

extern "C" int d3d_qk_rope_append_parts(const float* parts, int splits, const int64_t* positions,
                                        const void* q_norm_w, const void* k_norm_w, const float* inv_freq,
                                        void* q_out, void* k_cache, void* v_cache, const int64_t* slot_mapping,
                                        int T, int Hq, int Hkv, int D, float eps, int draft_rope,
                                        int64_t num_slots, void* stream) {
    if (splits < 1) return D3D_E_SHAPE;
    if (!parts) return D3D_E_NULL;
    return qk_rope_append(nullptr, parts, splits, positions, q_norm_w, k_norm_w, inv_freq, q_out, k_cache, v_cache,
                          slot_mapping, T, Hq, Hkv, D, eps, draft_rope, num_slots, stream);
}

extern "C" int d3d_silu_mul(const void* gate_up, void* out, int T, int M, void* stream) {
    if (T < 0 || M < 8 || M % 8) return D3D_E_SHAPE;
    if (T == 0) return D3D_OK;
    if (!gate_up || !out) return D3D_E_NULL;
    if (unaligned16(gate_up) || unaligned16(out)) return D3D_E_UNSUPPORTED;
    const dim3 grid((unsigned)((M / 8 + layers::NT - 1) / layers::NT), (unsigned)(T < 65535 ? T : 65535));
    hipLaunchKernelGGL(layers::silu_mul_kernel, grid, dim3(layers::NT), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), M, T);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
