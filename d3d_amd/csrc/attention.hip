// Paged block attention for gfx950: block-verify (causal within the block)
// and diffusion-draft block (bidirectional within the block) over a paged
// KV cache, plus the KV append that precedes them.
//
// Reference behaviour (D3D repository):
//   serving/vendor/ssd/layers/attention.py:21-22   KV append by slot mapping
//   serving/vendor/ssd/layers/attention.py:38-41   flash_attn_with_kvcache(
//       q, k_cache, v_cache, cache_seqlens, block_table, causal=True): query i
//       of a block of Q sees keys j <= ctx - Q + i (bottom-right causal)
//   serving/vendor/ssd/layers/attention.py:42-52 with serving/engine.py:41-42
//       draft recovery: every block query sees keys j < ctx (prefix + block)
//   models/d3d/modeling_d3d.py:190-200             GQA: head h reads KV head
//       h / (Hq / Hkv)
//   serving/engine.py:35-52 with :73-131           packed multi-branch draft:
//       the pending block (causal over prefix + block) followed by branch
//       blocks that see the prefix, the first n pending tokens and their
//       own block (bidirectional); here a per-query descriptor replaces the
//       materialised [B, 1, Q, S] bool mask
//
// Layouts (bf16): q and out [B, Q, Hq, D]; caches [num_pages, page, Hkv, D]
// (the reference's layout, serving/backend.py:46-48); block_table
// [B, max_pages] int32; context_lens [B] int32 = prefix + Q (the block's own
// keys are already appended).
//
// Work decomposition: workgroup (work item * Hkv + kv_head, query tile).
// Request b's context is cut into S_b = ceil(ctx_b / split_tokens) splits
// of whole 64-token tiles; for up to kMaxPackedB requests the work items
// (b, split) are numbered consecutively over the requests' actual split
// counts, so the grid's tail holds only empty items and short requests leave
// no idle workgroups in the middle of the launch.
// The G = Hq/Hkv query heads of the group times QT queries of the block
// form the MFMA rows (row r = g*QT + qi, 16 rows per wave, at most 16 x kMaxWaves).
// Key t is visible to a row iff t < A or S_lo <= t < S_hi (two ranges):
// causal A = ctx - Q + qi + 1; bidirectional A = ctx; packed A = prefix +
// vis[qi][0], [S_lo, S_hi) = prefix + [vis[qi][1], vis[qi][2]).  Each workgroup walks its split of the
// context in 64-token tiles staged in LDS; all waves share a tile.  Scores
// are computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32_bf16: the
// result layout (lane l holds tokens 4*(l/16)+r of row l%16) is, two 16-token
// sub-tiles at a time, the operand layout of P^T in O^T = V^T P^T, so
// probabilities never leave registers, and the O^T accumulators keep each
// lane on the query row whose softmax statistics it holds (rescaling and
// normalising need no cross-lane moves).  V is read 4 columns at a time (one
// 8-byte LDS read serves four 16-dim output tiles): tile (h, q) holds dim
// 64h + 4j + q in accumulator row j.  Online softmax runs in the log2
// domain.  With more than one split, (m, l, O) partials go to the workspace
// and a combine kernel merges them.
#include "d3d_common.hpp"
#include "../../include/d3d_hip.h"

#include <limits.h>

namespace d3d {
namespace attn {

constexpr int D = 128;         // head dimension
constexpr int TILE = 64;       // tokens per KV tile
// LDS bytes per token row.  K rows are read 16 B per lane, 16 rows per
// instruction: a 272-byte stride (68 banks) puts the 16 rows on 16 disjoint
// 4-bank groups.  V rows are read 8 B per lane with 4 token rows (4 apart)
// per wave: a 288-byte stride puts rows 4 apart 32 banks apart.
constexpr int ROWB = D * 2 + 16;     // K
constexpr int ROWB_V = D * 2 + 32;   // V
constexpr int LDS_V = TILE * ROWB;   // V region offset
// Up to 16 * kMaxWaves MFMA rows per workgroup (32 rows per wave with two
// row tiles).  Four waves (64 rows) run three workgroups per CU; eight-wave
// workgroups (128 rows) fit only one per CU at this register count and
// measured slower on the packed draft block (end-to-end 66.5 -> 68.9 steps/s
// with four).
constexpr int kMaxWaves = 4;
constexpr int kMaxSplitPages = 1024;  // page ids staged per split

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));

struct Params {
    const uint16_t* q;
    const uint16_t* k_cache;
    const uint16_t* v_cache;
    const int32_t* block_table;
    const int32_t* context_lens;
    uint16_t* out;
    _Float16* part_o;  // [B][nqt][Hkv][splits][M][D], O / l per split
    float* part_ml;    // [B][nqt][Hkv][splits][M][4], (m, l, 2^e, 0) per split
    int B, Q, Hq, Hkv, G, M;
    int page_size, max_pages, num_pages;
    int page_shift;  // log2(page_size) for powers of two, else -1
    int split_tokens, num_splits;  // tokens per split, splits per request at most
    int QT, nqt;        // queries per workgroup, query tiles per request
    const int32_t* vis; // packed mode: [Q][3] visibility descriptor
    float scale_log2;   // softmax scale * log2(e)
};

enum : int { kCausal = 0, kFull = 1, kPacked = 2 };

constexpr int kMaxPackedB = 64;  // requests whose work items are numbered consecutively

// Splits of request b: at least 1, at most num_splits (keys past
// num_splits * split_tokens, beyond the max_context bound, are not read).
__device__ __forceinline__ int splits_of(const Params& P, int b) {
    const int ctx = min(P.context_lens[b], P.max_pages * P.page_size);
    const int n = ctx > 0 ? (ctx + P.split_tokens - 1) / P.split_tokens : 1;
    return min(n, P.num_splits);
}

// Work item -> (request, split); b = -1 past the last item.
__device__ __forceinline__ void item_of(const Params& P, int item, int& b, int& s, int& nsplit) {
    b = -1;
    s = 0;
    nsplit = 1;
    if (P.B <= kMaxPackedB) {
        int acc = 0;
        for (int i = 0; i < P.B; ++i) {
            const int si = splits_of(P, i);
            if (item < acc + si) {
                b = i;
                s = item - acc;
                nsplit = si;
                return;
            }
            acc += si;
        }
    } else {
        const int bi = item / P.num_splits, si = item - bi * P.num_splits;
        const int n = splits_of(P, bi);
        if (si < n) {
            b = bi;
            s = si;
            nsplit = n;
        }
    }
}

// Butterfly steps across lane groups with gfx950's permlane swaps (VALU,
// no LDS round trip).  permlane16_swap(v, v) returns rows {0,0,2,2} and
// {1,1,3,3} of v, permlane32_swap(v, v) halves {lo,lo} and {hi,hi}: the max
// (or sum) of the pair is the xor-16 (xor-32) reduction step, and each lane
// adds its own value and its partner's, which commute exactly.
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Bits 0 .. n - 1 set: none for n <= 0, all 64 for n >= 64.
__device__ __forceinline__ uint64_t bits_below(int n) {
    return n <= 0 ? 0ull : n >= 64 ? ~0ull : (1ull << n) - 1ull;
}

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 pair -> packed bf16 (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Exponent e of the fp16 partial-output scale for a row whose largest
// magnitude is amax: amax * 2^-e lies in [2^14, 2^15) for normal amax; e is
// clamped to [-110, 110] so that 2^e and 2^-e are normal floats (zero,
// subnormal, Inf and NaN rows stay finite-scaled; Inf / NaN propagate).
__device__ __forceinline__ int row_scale_exp(float amax) {
    const int ex = (int)((__float_as_uint(amax) >> 23) & 0xffu) - 127;
    return min(max(ex - 14, -110), 110);
}

// Stages tokens [t0, t0 + TILE) of one KV head into registers.  Sixteen
// threads cover one 256-byte token row (16-byte segment tid % 16); pass p of
// NPASS handles token tid / 16 + p * (NT / 16), and each pass loads the
// token's K and V segments (reg[p] and reg[NPASS + p]).  Tokens at or past
// t_end, or on a page id outside the pool, load the split's first row (a
// valid address) and are then zeroed, so masked probabilities (exactly 0)
// never meet NaN or Inf garbage and no load is divergent.
template <int NT>
__device__ __forceinline__ void fetch_tile(const Params& P, int kvh, int t0, int t_begin, int t_end,
                                           const int* pages, size_t safe_row, u32x4 (&reg)[2 * TILE * 16 / NT],
                                           int& okmask) {
    constexpr int NPASS = TILE * 16 / NT;
    const int seg = threadIdx.x & 15;
    const size_t row_elems = (size_t)P.Hkv * D;
#pragma unroll
    for (int pss = 0; pss < NPASS; ++pss) {
        const int t = t0 + (int)(threadIdx.x >> 4) + pss * (NT / 16);
        const int rel = t - t_begin;
        const int pidx = P.page_shift >= 0 ? rel >> P.page_shift : rel / P.page_size;
        const int slot = P.page_shift >= 0 ? t & (P.page_size - 1) : t % P.page_size;
        const bool live = t < t_end;
        const int page = live ? pages[live ? pidx : 0] : -1;  // index stays inside the split
        const bool ok = page >= 0 && page < P.num_pages;
        const size_t row = ok ? (size_t)(page * P.page_size + slot) : safe_row;
        const size_t off = row * row_elems + (size_t)kvh * D + seg * 8;
        reg[pss] = *reinterpret_cast<const u32x4*>(P.k_cache + off);
        reg[NPASS + pss] = *reinterpret_cast<const u32x4*>(P.v_cache + off);
        // Zeroing happens at store time so that this load is not waited on here.
        okmask = pss == 0 ? (int)ok : (okmask | ((int)ok << pss));
    }
}

// Wave-uniform variant for power-of-two pages of at least 4 tokens.  A
// wave's 64 lanes cover 4 consecutive token rows starting at a multiple of 4
// (tiles start at page- and 64-aligned split offsets), so the 4 rows share
// one page: the page id and the rows' base address are scalar, and each lane
// adds a fixed 32-bit offset (row in the group, KV head, 16-byte segment).
template <int NT>
__device__ __forceinline__ void fetch_tile_u(const Params& P, int t0, int t_begin, int t_end, const int* pages,
                                             int safe_row, uint32_t lane_off, u32x4 (&reg)[2 * TILE * 16 / NT],
                                             int& okmask) {
    constexpr int NPASS = TILE * 16 / NT;
    const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int rl = (int)(threadIdx.x >> 4) & 3;
    const size_t row_bytes = (size_t)P.Hkv * D * 2;
    int pg[NPASS];
#pragma unroll
    for (int pss = 0; pss < NPASS; ++pss) {
        const int tw = t0 + 4 * w + pss * (NT / 16);
        pg[pss] = tw < t_end ? pages[(tw - t_begin) >> P.page_shift] : -1;  // index inside the split
    }
    okmask = 0;
#pragma unroll
    for (int pss = 0; pss < NPASS; ++pss) {
        const int tw = t0 + 4 * w + pss * (NT / 16);
        const int page = __builtin_amdgcn_readfirstlane(pg[pss]);
        const bool pok = page >= 0 && page < P.num_pages;
        const int base = pok ? page * P.page_size + (tw & (P.page_size - 1)) : safe_row;
        const char* kb = reinterpret_cast<const char*>(P.k_cache) + (size_t)base * row_bytes;
        const char* vb = reinterpret_cast<const char*>(P.v_cache) + (size_t)base * row_bytes;
        reg[pss] = *reinterpret_cast<const u32x4*>(kb + lane_off);
        reg[NPASS + pss] = *reinterpret_cast<const u32x4*>(vb + lane_off);
        okmask |= (int)(pok && tw + rl < t_end) << pss;
    }
}

// clean: every row of the tile is live and on an in-pool page (uniform), so
// no row needs zeroing.
template <int NT>
__device__ __forceinline__ void store_tile(char* lds, const u32x4 (&reg)[2 * TILE * 16 / NT], int okmask,
                                           bool clean) {
    constexpr int NPASS = TILE * 16 / NT;
    const int seg = threadIdx.x & 15;
    const u32x4 z = {0u, 0u, 0u, 0u};
    if (clean) {
#pragma unroll
        for (int pss = 0; pss < NPASS; ++pss) {
            const int tl = (int)(threadIdx.x >> 4) + pss * (NT / 16);
            *reinterpret_cast<u32x4*>(lds + tl * ROWB + seg * 16) = reg[pss];
            *reinterpret_cast<u32x4*>(lds + LDS_V + tl * ROWB_V + seg * 16) = reg[NPASS + pss];
        }
        return;
    }
#pragma unroll
    for (int pss = 0; pss < NPASS; ++pss) {
        const int tl = (int)(threadIdx.x >> 4) + pss * (NT / 16);
        const bool ok = (okmask >> pss) & 1;
        *reinterpret_cast<u32x4*>(lds + tl * ROWB + seg * 16) = ok ? reg[pss] : z;
        *reinterpret_cast<u32x4*>(lds + LDS_V + tl * ROWB_V + seg * 16) = ok ? reg[NPASS + pss] : z;
    }
}

// Launch bounds ask for at least two workgroups per CU; at the register
// counts the compiler reaches, four-wave workgroups run three per CU.
// UPG: pages are a power of two of at least 4 tokens (wave-uniform page ids).
// RT: row tiles of 16 per wave.  With RT = 2 each K fragment and each
// permuted V operand read from LDS feeds two MFMAs (blocks of more than 64
// rows per KV head: the packed draft block).
template <int NW, int MODE, bool UPG, int RT>
__global__ __launch_bounds__(NW * 64, 2) void attn_split_kernel(Params P) {
    constexpr int NT = NW * 64;
    const int kvh = blockIdx.x % P.Hkv, qt = blockIdx.y;
    int b, s, nsplit, ctx;
    // One request whose split spans at most NT pages: the item is the split,
    // and its page ids (one per thread) load together with the context
    // length instead of after it.
    const bool spec = P.B == 1 && (P.split_tokens + P.page_size - 1) / P.page_size <= NT;
    int pg_spec = 0;
    if (spec) {
        b = 0;
        s = blockIdx.x / P.Hkv;  // < num_splits, so the split starts inside the table
        const int raw = P.context_lens[0];
        const int p0 = s * P.split_tokens / P.page_size;
        const int span = min((P.split_tokens + P.page_size - 1) / P.page_size, P.max_pages - p0);
        if ((int)threadIdx.x < span) pg_spec = P.block_table[p0 + threadIdx.x];
        ctx = min(raw, P.max_pages * P.page_size);
        nsplit = min(ctx > 0 ? (ctx + P.split_tokens - 1) / P.split_tokens : 1, P.num_splits);
        if (s >= nsplit) return;  // past the last split (uniform, before any barrier)
    } else {
        item_of(P, blockIdx.x / P.Hkv, b, s, nsplit);
        if (b < 0) return;  // past the last work item (uniform, before any barrier)
        ctx = min(P.context_lens[b], P.max_pages * P.page_size);
    }
    const int q0 = qt * P.QT;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g4 = lane >> 4, c16 = lane & 15;

    __shared__ __attribute__((aligned(16))) char lds[TILE * (ROWB + ROWB_V)];
    __shared__ int pages[kMaxSplitPages];
    __shared__ int s_lim[2][NW];
    __shared__ uint32_t s_tiles[2][NW];

    // This lane's query row in row tile rt (wave w holds rows w*16*RT ..
    // w*16*RT + 16*RT - 1) for the Q^T operand and the softmax statistics.
    int row[RT], qi[RT], head[RT], va[RT], vlo[RT], vhi[RT];
    bool row_ok[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        row[rt] = (w * RT + rt) * 16 + c16;
        const int gh = row[rt] / P.QT;
        qi[rt] = q0 + (row[rt] - gh * P.QT);
        row_ok[rt] = row[rt] < P.M && qi[rt] < P.Q;
        head[rt] = kvh * P.G + (row_ok[rt] ? gh : 0);
        // Visible keys: t < va, or vlo <= t < vhi.
        va[rt] = vlo[rt] = vhi[rt] = 0;
        if (row_ok[rt]) {
            if constexpr (MODE == kCausal) {
                va[rt] = ctx - P.Q + qi[rt] + 1;
            } else if constexpr (MODE == kFull) {
                va[rt] = ctx;
            } else {
                const int pre = ctx - P.Q;
                va[rt] = pre + P.vis[qi[rt] * 3 + 0];
                vlo[rt] = pre + P.vis[qi[rt] * 3 + 1];
                vhi[rt] = pre + P.vis[qi[rt] * 3 + 2];
            }
            va[rt] = min(va[rt], ctx);
            vhi[rt] = min(vhi[rt], ctx);
        }
    }
    // Workgroup bounds: keys below a_min are visible to every row; none at
    // or past w_end is visible to any (w_end >= 0).  Causal and bidirectional
    // blocks have them in closed form: every query q0 .. min(q0 + QT, Q) - 1
    // of the tile has rows, and a row's frontier grows with its query.
    // Packed blocks reduce their descriptors over the workgroup.
    // Packed blocks also mark which of the split's first 64 tiles hold a
    // key that some row sees (bit i: tokens t_begin + TILE i ..): each
    // query tile sees the prefix, the pending block and its own branches,
    // not the other branches' keys, so most tiles past the prefix are
    // skipped.  A skipped tile would add exactly nothing to any row's
    // (m, l, O).
    int a_min = INT_MAX, w_end = 0;
    uint64_t tile_vis = ~0ull;
    if constexpr (MODE == kPacked) {
        int amin = INT_MAX, wend = 0;
        uint64_t tv = 0;
        const int tb = s * P.split_tokens;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
            if (row_ok[rt]) {
                amin = min(amin, va[rt]);
                wend = max(wend, max(va[rt], vhi[rt]));
                // keys below va: tiles [0, ceil((va - tb) / TILE));
                // keys [vlo, vhi): tiles floor((vlo - tb) / TILE) .. ceil((vhi - tb) / TILE) - 1
                tv |= bits_below(va[rt] > tb ? (va[rt] - tb + TILE - 1) / TILE : 0);
                if (vlo[rt] < vhi[rt] && vhi[rt] > tb)
                    tv |= bits_below((vhi[rt] - tb + TILE - 1) / TILE) &
                          ~bits_below(vlo[rt] > tb ? (vlo[rt] - tb) / TILE : 0);
            }
        uint32_t tv_lo = (uint32_t)tv, tv_hi = (uint32_t)(tv >> 32);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            amin = min(amin, __shfl_xor(amin, o, 64));
            wend = max(wend, __shfl_xor(wend, o, 64));
            tv_lo |= (uint32_t)__shfl_xor((int)tv_lo, o, 64);
            tv_hi |= (uint32_t)__shfl_xor((int)tv_hi, o, 64);
        }
        if (lane == 0) {
            s_lim[0][w] = amin;
            s_lim[1][w] = wend;
            s_tiles[0][w] = tv_lo;
            s_tiles[1][w] = tv_hi;
        }
        __syncthreads();
        tv_lo = tv_hi = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            a_min = min(a_min, s_lim[0][i]);
            w_end = max(w_end, s_lim[1][i]);
            tv_lo |= s_tiles[0][i];
            tv_hi |= s_tiles[1][i];
        }
        tile_vis = ((uint64_t)tv_hi << 32) | tv_lo;
    } else if constexpr (MODE == kCausal) {
        a_min = min(ctx - P.Q + q0 + 1, ctx);
        w_end = max(0, min(ctx - P.Q + min(q0 + P.QT, P.Q), ctx));
    } else {
        a_min = ctx;
        w_end = max(0, ctx);
    }
    const int t_begin = s * P.split_tokens;
    const int t_end = min(min(t_begin + P.split_tokens, ctx), w_end);
    // Page ids of the whole split in one round trip (split starts are page aligned).
    const int p0 = t_begin / P.page_size;
    const int np = t_end > t_begin ? (t_end - 1) / P.page_size - p0 + 1 : 0;
    int bad_page = 0;
    if (spec) {
        if ((int)threadIdx.x < np) {  // np <= span: the split's pages are a prefix of the span
            pages[threadIdx.x] = pg_spec;
            bad_page = pg_spec < 0 || pg_spec >= P.num_pages;
        }
    } else {
        for (int i = threadIdx.x; i < np; i += NT) {
            const int pg = P.block_table[(size_t)b * P.max_pages + p0 + i];
            pages[i] = pg;
            bad_page |= pg < 0 || pg >= P.num_pages;
        }
    }
    const bool pages_ok = !__syncthreads_or(bad_page);
    // A row every masked lane may read: the first in-pool page of the split
    // (or cache row 0).
    int safe_row = 0;
    for (int i = 0; i < np; ++i)
        if (pages[i] >= 0 && pages[i] < P.num_pages) {
            safe_row = pages[i] * P.page_size;
            break;
        }
    const uint32_t lane_off = (uint32_t)(((threadIdx.x >> 4) & 3) * P.Hkv * D * 2 + kvh * D * 2 + (threadIdx.x & 15) * 16);
    // Stage tokens [t0, t0 + TILE) into registers / store them to LDS.
    auto fetch = [&](int t0, u32x4 (&reg)[2 * TILE * 16 / NT], int& ok) {
        if constexpr (UPG)
            fetch_tile_u<NT>(P, t0, t_begin, t_end, pages, safe_row, lane_off, reg, ok);
        else
            fetch_tile<NT>(P, kvh, t0, t_begin, t_end, pages, (size_t)safe_row, reg, ok);
    };


    // Q^T operand of v_mfma_f32_16x16x32_bf16: lane l holds row l%16, head
    // dims 32*ks + 8*(l/16) + 0..7.  K is read with the same dim assignment,
    // so the product sums over every dim whatever order the hardware uses.
    bf16x8 qop[RT][D / 32];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (row_ok[rt])
                v = *reinterpret_cast<const u32x4*>(P.q + (((size_t)b * P.Q + qi[rt]) * P.Hq + head[rt]) * D +
                                                    ks * 32 + g4 * 8);
            qop[rt][ks] = __builtin_bit_cast(bf16x8, v);
        }

    f32x4 o[RT][D / 16];
    float m_run[RT], l_run[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
#pragma unroll
        for (int n = 0; n < D / 16; ++n) o[rt][n] = {0.f, 0.f, 0.f, 0.f};
        m_run[rt] = -INFINITY;
        l_run[rt] = 0.f;
    }

    // One 64-token tile from LDS into the running (m, l, O) of each row.
    auto compute = [&](int t0) {
        const char* kl = lds;
        const char* vl = lds + LDS_V;
        // S^T sub-tiles: sc[rt][m][r] = score of token t0 + 16m + 4*g4 + r for
        // row c16 of row tile rt.
        float sc[RT][TILE / 16][4];
        {
            // Four independent accumulation chains per row tile, interleaved;
            // each K fragment serves every row tile.
            f32x4 acc[RT][TILE / 16];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int m = 0; m < TILE / 16; ++m) acc[rt][m] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
                u32x4 kf[TILE / 16];
#pragma unroll
                for (int m = 0; m < TILE / 16; ++m)
                    kf[m] = *reinterpret_cast<const u32x4*>(kl + (16 * m + c16) * ROWB + (ks * 32 + g4 * 8) * 2);
#pragma unroll
                for (int m = 0; m < TILE / 16; ++m)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        acc[rt][m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[m]),
                                                                           qop[rt][ks], acc[rt][m], 0, 0, 0);
            }
            // Raw scores; the softmax scale is applied inside the exponent.
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int m = 0; m < TILE / 16; ++m)
#pragma unroll
                    for (int r = 0; r < 4; ++r) sc[rt][m][r] = acc[rt][m][r];
        }
        // Masking only where the tile crosses the split end or the
        // visibility frontier of some row (a uniform test).
        if (t0 + TILE > min(t_end, a_min)) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int m = 0; m < TILE / 16; ++m)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int t = t0 + 16 * m + 4 * g4 + r;
                        const bool vis = t < va[rt] || (MODE == kPacked && t >= vlo[rt] && t < vhi[rt]);
                        if (!(vis && t < t_end)) sc[rt][m][r] = -INFINITY;
                    }
        }
        // P as the P^T operand of 16x16x32: sub-tiles 2mp and 2mp+1 give the
        // 8 token slots (4*g4 + r, then 16 + 4*g4 + r) of row c16.
        // A row with no visible key so far has m_run = -inf and only -inf
        // scores: exp2(-inf) = 0 with the offset taken as 0.
        uint32_t pw[RT][TILE / 16][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            float tmax = -INFINITY;
#pragma unroll
            for (int m = 0; m < TILE / 16; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sc[rt][m][r]);
            tmax = xor32_max(xor16_max(tmax));
            // Rescale only when the running max of some row grows (log2 domain:
            // scale * max raw score; the scale is positive, so the max commutes).
            const float m_new = fmaxf(m_run[rt], tmax * P.scale_log2);
            const bool grow = m_new > m_run[rt];
            if (__any(grow)) {
                const float alpha =
                    grow ? (m_run[rt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[rt] - m_new)) : 1.f;
                l_run[rt] *= alpha;
                // O^T accumulators: every entry of this lane belongs to row c16.
#pragma unroll
                for (int n = 0; n < D / 16; ++n) o[rt][n] *= alpha;
                m_run[rt] = m_new;
            }
            float psum = 0.f;
            const float m_off = m_run[rt] == -INFINITY ? 0.f : m_run[rt];
#pragma unroll
            for (int m = 0; m < TILE / 16; ++m) {
                float pr[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pr[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[rt][m][r], P.scale_log2, -m_off));
                    psum += pr[r];
                }
                pw[rt][m][0] = pack_bf16x2(pr[0], pr[1]);
                pw[rt][m][1] = pack_bf16x2(pr[2], pr[3]);
            }
            l_run[rt] += psum;
        }
#pragma unroll
        for (int mp = 0; mp < TILE / 32; ++mp) {
            bf16x8 pop[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const u32x4 pv = {pw[rt][2 * mp][0], pw[rt][2 * mp][1], pw[rt][2 * mp + 1][0], pw[rt][2 * mp + 1][1]};
                pop[rt] = __builtin_bit_cast(bf16x8, pv);
            }
#pragma unroll
            for (int h = 0; h < D / 64; ++h) {
                // V rows of the 8 token slots, 4 columns 64h + 4*c16 .. +3 each.
                u32x2 vr[8];
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const int t = 32 * mp + 16 * (kk >> 2) + 4 * g4 + (kk & 3);
                    vr[kk] = *reinterpret_cast<const u32x2*>(vl + t * ROWB_V + (64 * h + 4 * c16) * 2);
                }
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    // Column qq of each row: low or high half of word qq/2.
                    const uint32_t sel = (qq & 1) ? 0x07060302u : 0x05040100u;
                    const int word = qq >> 1;
                    const u32x4 vw = {__builtin_amdgcn_perm(vr[1][word], vr[0][word], sel),
                                      __builtin_amdgcn_perm(vr[3][word], vr[2][word], sel),
                                      __builtin_amdgcn_perm(vr[5][word], vr[4][word], sel),
                                      __builtin_amdgcn_perm(vr[7][word], vr[6][word], sel)};
                    // O^T = V^T P^T: the same registers with the operands
                    // swapped (A = V^T, lane l row dim 64h + 4(l%16) + qq;
                    // B = P^T, lane l column = query row l%16), so the
                    // accumulator rows are dims and its columns query rows.
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        o[rt][4 * h + qq] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, vw), pop[rt], o[rt][4 * h + qq], 0, 0, 0);
                }
            }
        }
    };

    // Tiles are staged global -> registers -> LDS with one register set in
    // flight while the current tile is computed.  A second set (218 VGPRs,
    // two waves per SIMD, loads checked in the assembly to stay outstanding
    // across the compute) measured batch-8 verify 35.4 -> 35.0 us and nothing
    // at batch 1 or end to end: the tile loop is bound by its dependency
    // chain, not by load latency.
    // The first tile at or after t (a tile start) that some row sees;
    // every tile for causal and bidirectional blocks, and past the 64
    // tiles the packed mask covers.
    auto next_tile = [&](int t) -> int {
        if constexpr (MODE == kPacked) {
            const int i = (t - t_begin) / TILE;
            if (i < 64) {
                const uint64_t m = tile_vis >> i;
                return m ? t + TILE * (int)__builtin_ctzll(m) : t_begin + 64 * TILE;
            }
        }
        return t;
    };
    u32x4 regA[2 * TILE * 16 / NT];
    int okA = 0;
    int t0 = next_tile(t_begin);
    if (t0 < t_end) fetch(t0, regA, okA);
    // Whole tiles on in-pool pages store without zeroing; the split's
    // partial last tile (and every tile of a split that names an
    // out-of-pool page) zeroes its dead rows.  Two loops rather than a
    // per-tile branch: with the branch inside one loop the compiler
    // waits for the next tile's loads before the first MFMA.
    if (pages_ok) {
        while (t0 + TILE <= t_end) {
            __syncthreads();
            store_tile<NT>(lds, regA, okA, true);
            __syncthreads();
            const int tn = next_tile(t0 + TILE);
            if (tn < t_end) fetch(tn, regA, okA);
            compute(t0);
            t0 = tn;
        }
    }
    while (t0 < t_end) {
        __syncthreads();
        store_tile<NT>(lds, regA, okA, false);
        __syncthreads();
        const int tn = next_tile(t0 + TILE);
        if (tn < t_end) fetch(tn, regA, okA);
        compute(t0);
        t0 = tn;
    }

    // Row sums: reduce the per-lane partials over the 4 lanes of a row.
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) l_run[rt] = xor32_sum(xor16_sum(l_run[rt]));

    // Lane (g4, c16) holds row c16 of row tile rt at dims 64h + 16 g4 + 4r +
    // qq in o[rt][4h + qq][r]: four consecutive dims per (h, r).
    if (nsplit == 1) {
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float inv = l_run[rt] > 0.f ? 1.f / l_run[rt] : 0.f;
            if (row_ok[rt]) {
                uint16_t* dst = P.out + (((size_t)b * P.Q + qi[rt]) * P.Hq + head[rt]) * D + 16 * g4;
#pragma unroll
                for (int h = 0; h < D / 64; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const u32x2 v = {pack_bf16x2(o[rt][4 * h + 0][r] * inv, o[rt][4 * h + 1][r] * inv),
                                         pack_bf16x2(o[rt][4 * h + 2][r] * inv, o[rt][4 * h + 3][r] * inv)};
                        *reinterpret_cast<u32x2*>(dst + 64 * h + 4 * r) = v;
                    }
            }
        }
    } else {
        // Normalised partial O / l in fp16 with a power-of-two row scale
        // 2^e chosen so that the row's largest |O / l| lands in [2^14, 2^15):
        // no overflow for bf16 values past fp16's 65504 and no subnormal loss
        // for tiny ones.  (m, l, 2^e) in fp32.
        const size_t unit = (((size_t)b * P.nqt + qt) * P.Hkv + kvh) * P.num_splits + s;
        _Float16* po = P.part_o + unit * P.M * D;
        float4* pml = reinterpret_cast<float4*>(P.part_ml) + unit * P.M;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
            const float inv = l_run[rt] > 0.f ? 1.f / l_run[rt] : 0.f;
            float amax = 0.f;
#pragma unroll
            for (int n = 0; n < D / 16; ++n)
#pragma unroll
                for (int r = 0; r < 4; ++r) amax = fmaxf(amax, fabsf(o[rt][n][r] * inv));
            amax = xor32_max(xor16_max(amax));  // the 4 lanes of row c16
            const int e = row_scale_exp(amax);
            const float down = __uint_as_float((uint32_t)(127 - e) << 23) * inv;  // 2^-e / l
            if (row[rt] < P.M) {
#pragma unroll
                for (int h = 0; h < D / 64; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const h16x4 v = {(_Float16)(o[rt][4 * h + 0][r] * down), (_Float16)(o[rt][4 * h + 1][r] * down),
                                         (_Float16)(o[rt][4 * h + 2][r] * down), (_Float16)(o[rt][4 * h + 3][r] * down)};
                        *reinterpret_cast<h16x4*>(po + (size_t)row[rt] * D + 64 * h + 16 * g4 + 4 * r) = v;
                    }
            }
            if (g4 == 0 && row_ok[rt])
                pml[row[rt]] = make_float4(m_run[rt], l_run[rt], __uint_as_float((uint32_t)(127 + e) << 23), 0.f);
        }
    }
}

// Merges the split partials: workgroup (row block, kv_head, b) handles
// kRowsPerCombine rows; 32 threads per row, 4 columns each.  All split
// statistics are loaded at once, then the weighted partial outputs.
constexpr int kRowsPerCombine = 8;
constexpr int kMaxSplits = 256;

// Up to kSpecSplits splits per request (8 rows x 32 splits = one thread per
// statistic) and at most kSpecBatch requests, every load of the combine --
// split statistics, partial outputs and the request's context length -- is
// issued at once, from clamped slots inside the workspace; slots at or past
// the request's split count are then excluded by selects (their bits may be
// stale), never by a multiply.  One round trip instead of three: batch-1
// verify 12.55 -> 12.43 us, batch-4 draft block 13.86 -> 13.53 us.  NSPEC
// (4, 8, 16, 20, 24 or 32, the smallest at least num_splits) bounds the
// partial outputs each thread loads.  The 17 splits of a 2064-key context
// took 32 slots (118 VGPRs, each thread's loads and conversions issued in
// one long chain) before the 20- and 24-slot forms: batch-1 verify 13.49 ->
// 11.96 us, batch-4 draft block 13.32 -> 11.86 us.  Larger batches of mixed lengths would read
// many stale slots (about 4 MB at the batch-8 draw), so they keep the exact
// loop (NSPEC = 0), or with CTX_FIRST read the request's context length
// first and clamp every slot to its own split count: two round trips and no
// stale slots (batch-8 draw 34.3 -> 32.8 us for the whole call, against the
// exact loop's three round trips).
constexpr int kSpecSplits = 32;
constexpr int kSpecBatch = 4;

template <int NSPEC, bool CTX_FIRST = false>
__global__ __launch_bounds__(256) void attn_combine_kernel(Params P) {
    const int r0 = blockIdx.x * kRowsPerCombine, kvh = blockIdx.y;
    const int b = blockIdx.z / P.nqt, q0 = (blockIdx.z - b * P.nqt) * P.QT;
    const size_t unit0 = ((size_t)blockIdx.z * P.Hkv + kvh) * P.num_splits;
    constexpr bool SPEC = NSPEC > 0;
    __shared__ float wts[kRowsPerCombine][SPEC ? kSpecSplits : kMaxSplits];
    __shared__ float lsum[kRowsPerCombine][SPEC ? kSpecSplits : kMaxSplits];
    __shared__ float pscale[kRowsPerCombine][SPEC ? kSpecSplits : kMaxSplits];
    __shared__ float inv_den[kRowsPerCombine];
    // Output mapping: 32 threads per row, 4 columns each.
    const int rr = threadIdx.x / 32, c4 = (threadIdx.x % 32) * 4, row = r0 + rr;
    const int row_c = row < P.M ? row : P.M - 1;
    int S;
    if constexpr (SPEC) {
        static_assert(kRowsPerCombine * kSpecSplits == 256, "one statistic per thread");
        int slots = P.num_splits;  // slots loaded are clamped below this
        if constexpr (CTX_FIRST) {
            S = splits_of(P, b);
            if (S == 1) return;  // the split kernel wrote this request's output
            slots = S;
        }
        const int er = threadIdx.x / kSpecSplits, esp = threadIdx.x % kSpecSplits;
        const int erow = min(r0 + er, P.M - 1);
        const int esp_c = min(esp, slots - 1);
        const float4 ml = reinterpret_cast<const float4*>(P.part_ml)[(unit0 + esp_c) * P.M + erow];
        h16x4 hv[NSPEC > 0 ? NSPEC : 1];
#pragma unroll
        for (int sp = 0; sp < NSPEC; ++sp) {
            const int spc = min(sp, slots - 1);
            hv[sp] = *reinterpret_cast<const h16x4*>(P.part_o + ((unit0 + spc) * P.M + row_c) * D + c4);
        }
        if constexpr (!CTX_FIRST) {
            S = splits_of(P, b);
            if (S == 1) return;  // the split kernel wrote this request's output
        }
        const bool live = esp < S && r0 + er < P.M;
        wts[er][esp] = live ? ml.x : -INFINITY;
        lsum[er][esp] = live ? ml.y : 0.f;
        pscale[er][esp] = ml.z;
        __syncthreads();
        // One wave per two rows: lanes 0..31 and 32..63 fold one row each.
        {
            const int wv = threadIdx.x / 64, lane = threadIdx.x % 64;
            const int r2 = 2 * wv + lane / 32, l32 = lane % 32;
            float mx = wts[r2][l32];
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            const float m = wts[r2][l32];
            const float wgt = (m == -INFINITY) ? 0.f : exp2f(m - mx) * lsum[r2][l32];
            float den = wgt;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
            wts[r2][l32] = wgt * pscale[r2][l32];  // each lane rewrites only the entry it read
            if (l32 == 0) inv_den[r2] = den > 0.f ? 1.f / den : 0.f;
        }
        __syncthreads();
        const int oh = kvh * P.G + row / P.QT, oq = q0 + row % P.QT;
        if (row >= P.M || oq >= P.Q) return;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sp = 0; sp < NSPEC; ++sp) {
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            const f32x4 o = {(float)hv[sp][0], (float)hv[sp][1], (float)hv[sp][2], (float)hv[sp][3]};
            acc += wts[rr][sp] * (sp < S ? o : z);
        }
        const float sc = inv_den[rr];
        const u32x2 v = {pack_bf16x2(acc[0] * sc, acc[1] * sc), pack_bf16x2(acc[2] * sc, acc[3] * sc)};
        *reinterpret_cast<u32x2*>(P.out + (((size_t)b * P.Q + oq) * P.Hq + oh) * D + c4) = v;
        return;
    }
    S = splits_of(P, b);
    if (S == 1) return;  // the split kernel wrote this request's output
    // Statistics of every (row, split) in one round trip.
    for (int e = threadIdx.x; e < kRowsPerCombine * S; e += 256) {
        const int er = e / S, sp = e % S, erow = r0 + er;
        float m = -INFINITY, l = 0.f, sc = 1.f;
        if (erow < P.M) {
            const float4 ml = reinterpret_cast<const float4*>(P.part_ml)[(unit0 + sp) * P.M + erow];
            m = ml.x;
            l = ml.y;
            sc = ml.z;
        }
        wts[er][sp] = m;
        lsum[er][sp] = l;
        pscale[er][sp] = sc;
    }
    __syncthreads();
    // One wave per row: lanes fold splits, then a butterfly (fixed order).
    {
        const int wv = threadIdx.x / 64, lane = threadIdx.x % 64;
        for (int r2 = wv; r2 < kRowsPerCombine; r2 += 4) {
            float mx = -INFINITY;
            for (int sp = lane; sp < S; sp += 64) mx = fmaxf(mx, wts[r2][sp]);
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            float den = 0.f;
            for (int sp = lane; sp < S; sp += 64) {
                const float m = wts[r2][sp];
                const float w = (m == -INFINITY) ? 0.f : exp2f(m - mx);
                // Weight of the stored partial (O / l) * 2^-e; the denominator
                // takes the unscaled weight.
                wts[r2][sp] = w * lsum[r2][sp] * pscale[r2][sp];
                den += w * lsum[r2][sp];
            }
            for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
            if (lane == 0) inv_den[r2] = den > 0.f ? 1.f / den : 0.f;
        }
    }
    __syncthreads();
    const int oh = kvh * P.G + row / P.QT, oq = q0 + row % P.QT;
    if (row >= P.M || oq >= P.Q) return;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int sp = 0; sp < S; ++sp) {
        const float w = wts[rr][sp];
        const h16x4 h = *reinterpret_cast<const h16x4*>(P.part_o + ((unit0 + sp) * P.M + row) * D + c4);
        const f32x4 o = {(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
        acc += w * o;
    }
    const float sc = inv_den[rr];
    const u32x2 v = {pack_bf16x2(acc[0] * sc, acc[1] * sc), pack_bf16x2(acc[2] * sc, acc[3] * sc)};
    *reinterpret_cast<u32x2*>(P.out + (((size_t)b * P.Q + oq) * P.Hq + oh) * D + c4) = v;
}

// Combine with every load issued at once, NSPEC the smallest of 4, 8, 16,
// 20, 24, 32 covering ns splits.
template <bool CTX_FIRST>
static void launch_slot_combine(int ns, dim3 grid, hipStream_t s, const Params& P) {
    if (ns <= 4)
        hipLaunchKernelGGL((attn_combine_kernel<4, CTX_FIRST>), grid, dim3(256), 0, s, P);
    else if (ns <= 8)
        hipLaunchKernelGGL((attn_combine_kernel<8, CTX_FIRST>), grid, dim3(256), 0, s, P);
    else if (ns <= 16)
        hipLaunchKernelGGL((attn_combine_kernel<16, CTX_FIRST>), grid, dim3(256), 0, s, P);
    else if (ns <= 20)
        hipLaunchKernelGGL((attn_combine_kernel<20, CTX_FIRST>), grid, dim3(256), 0, s, P);
    else if (ns <= 24)
        hipLaunchKernelGGL((attn_combine_kernel<24, CTX_FIRST>), grid, dim3(256), 0, s, P);
    else
        hipLaunchKernelGGL((attn_combine_kernel<32, CTX_FIRST>), grid, dim3(256), 0, s, P);
}

// KV append: one workgroup per token, 16 bytes per thread (K then V).
__global__ __launch_bounds__(256) void kv_append_kernel(const uint16_t* k, const uint16_t* v, uint16_t* k_cache,
                                                        uint16_t* v_cache, const int64_t* slots, int row_elems,
                                                        int64_t num_slots) {
    const int n = blockIdx.x;
    const int64_t slot = slots[n];
    if (slot < 0 || slot >= num_slots) return;
    const int vecs = row_elems / 8;
    for (int u = threadIdx.x; u < 2 * vecs; u += blockDim.x) {
        const int kv = u / vecs, seg = u % vecs;
        const uint16_t* src = (kv == 0 ? k : v) + (size_t)n * row_elems + seg * 8;
        uint16_t* dst = (kv == 0 ? k_cache : v_cache) + (size_t)slot * row_elems + seg * 8;
        *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
    }
}

struct Plan {
    int waves, rt, split_tokens, num_splits, QT, nqt;
    bool valid;
    size_t part_o_bytes, part_ml_bytes, total;
};

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Work items if every request were max_context long: about one round of the
// 768 resident four-wave workgroups (three per CU).  Mixed lengths fill less:
// at batch 8 (contexts 873..6219) 768 gives 448 items of 9 tiles and measured
// 37.8 -> 35.2 us against 2048 (992 items of 4 tiles; half the fp16 partials
// and none of the second round's idle slots); batch 1 and the draft block
// keep their plans (the two-tile minimum and one-tile splits bind).  With
// the context-first combine the batch-8 optimum stays at 768: 512 / 640 /
// 768 / 1024 / 1280 / 1536 measured 39.5 / 34.6 / 33.0 / 34.5 / 38.6 /
// 38.7 us.
constexpr int kTargetItems = 768;

static Plan plan(int B, int Q, int Hq, int Hkv, int max_context, int page_size) {
    Plan p;
    const int G = Hq / Hkv;
    // Blocks of more than 64 rows per KV head (G x Q) take two row tiles per
    // wave in four-wave workgroups: 128 rows, each LDS fragment used twice.
    p.rt = G * Q > 64 ? 2 : 1;
    const int rows = kMaxWaves * 16 * p.rt;
    p.QT = Q < rows / G ? Q : rows / G;
    p.nqt = (Q + p.QT - 1) / p.QT;
    const int M = G * p.QT;
    // One row tile per wave: M <= 64 rows (G <= 64 is validated), so two or
    // four waves.
    p.waves = p.rt == 2 ? 4 : (M <= 32 ? 2 : 4);
    const int tiles = (max_context + TILE - 1) / TILE;
    // Tiles per split: about kTargetItems (request, split, kv head, query
    // tile) items if every request were max_context long.
    const int64_t units = (int64_t)B * p.nqt * Hkv;
    // Two-row-tile workgroups (238 VGPRs) run two per CU, not three: about
    // one round of them is 512 items.
    const int64_t target = p.rt == 2 ? 512 : kTargetItems;
    int64_t tps = (units * tiles + target - 1) / target;
    // Four-wave workgroups take at least two tiles per split: at batch 1
    // (2064 keys) that halves the fp16 partials and measured 14.9 -> 14.0 us;
    // two-wave workgroups (the 32-row draft block) keep one-tile splits,
    // which measured faster there.
    const int min_tps = p.waves >= 4 ? 2 : 1;
    tps = tps < min_tps ? min_tps : tps;
    tps = tps > tiles ? tiles : tps;
    int tiles_per_split = (int)tps;
    if ((tiles + tiles_per_split - 1) / tiles_per_split > kMaxSplits) tiles_per_split = (tiles + kMaxSplits - 1) / kMaxSplits;
    // Split starts must be page aligned and a split's pages must fit in LDS.
    const int unit_tokens = page_size % TILE == 0 ? page_size : (TILE % page_size == 0 ? TILE : TILE * page_size);
    int split_tokens = tiles_per_split * TILE;
    split_tokens = (split_tokens + unit_tokens - 1) / unit_tokens * unit_tokens;
    while (split_tokens / page_size + 1 > kMaxSplitPages && split_tokens > unit_tokens) split_tokens -= unit_tokens;
    p.split_tokens = split_tokens;
    p.num_splits = (max_context + p.split_tokens - 1) / p.split_tokens;
    if (p.num_splits < 1) p.num_splits = 1;
    p.valid = p.num_splits <= kMaxSplits && p.split_tokens / page_size + 1 <= kMaxSplitPages;
    if (p.num_splits == 1) {
        p.part_o_bytes = p.part_ml_bytes = 0;
    } else {
        p.part_o_bytes = align256((size_t)B * p.nqt * Hkv * p.num_splits * M * D * sizeof(_Float16));
        p.part_ml_bytes = align256((size_t)B * p.nqt * Hkv * p.num_splits * M * 4 * sizeof(float));
    }
    p.total = p.part_o_bytes + p.part_ml_bytes;
    if (p.total == 0) p.total = 256;
    return p;
}

static int validate(int B, int Q, int Hq, int Hkv, int D_, int page_size, int max_pages, int num_pages,
                    int max_context) {
    if (B < 1 || B > 65535 || Q < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv) return D3D_E_SHAPE;
    if (D_ != D) return D3D_E_UNSUPPORTED;
    if (Hq / Hkv > kMaxWaves * 16) return D3D_E_UNSUPPORTED;
    if ((int64_t)B * ((Q + 127) / 128) * (Hq / Hkv) > 65535 * 128) return D3D_E_SHAPE;
    if (page_size < 1 || max_pages < 1 || num_pages < 1 || max_context < 1) return D3D_E_SHAPE;
    if ((int64_t)max_pages * page_size < max_context) return D3D_E_SHAPE;
    return D3D_OK;
}

template <int MODE>
static int run(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
               const int32_t* context_lens, const int32_t* vis, void* out, int B, int Q, int Hq, int Hkv, int D_,
               int page_size, int max_pages, int num_pages, float scale, int max_context, void* workspace,
               size_t ws_bytes, void* stream) {
    const int st = validate(B, Q, Hq, Hkv, D_, page_size, max_pages, num_pages, max_context);
    if (st != D3D_OK) return st;
    if (!q || !k_cache || !v_cache || !block_table || !context_lens || !out) return D3D_E_NULL;
    if (MODE == kPacked && !vis) return D3D_E_NULL;
    const Plan pl = plan(B, Q, Hq, Hkv, max_context, page_size);
    if (!pl.valid) return D3D_E_UNSUPPORTED;
    if ((int64_t)B * pl.nqt > 65535 || (int64_t)B * pl.num_splits * Hkv > INT_MAX / 2) return D3D_E_SHAPE;
    if (pl.num_splits > 1 && (!workspace || ws_bytes < pl.total)) return D3D_E_WORKSPACE;
    Params P;
    P.q = static_cast<const uint16_t*>(q);
    P.k_cache = static_cast<const uint16_t*>(k_cache);
    P.v_cache = static_cast<const uint16_t*>(v_cache);
    P.block_table = block_table;
    P.context_lens = context_lens;
    P.out = static_cast<uint16_t*>(out);
    P.part_o = pl.num_splits > 1 ? reinterpret_cast<_Float16*>(workspace) : nullptr;
    P.part_ml = pl.num_splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + pl.part_o_bytes)
                                  : nullptr;
    P.B = B;
    P.Q = Q;
    P.Hq = Hq;
    P.Hkv = Hkv;
    P.G = Hq / Hkv;
    P.QT = pl.QT;
    P.nqt = pl.nqt;
    P.M = P.G * pl.QT;
    P.vis = vis;
    P.page_size = page_size;
    P.page_shift = -1;
    if ((page_size & (page_size - 1)) == 0) {
        int sh = 0;
        while ((1 << sh) < page_size) ++sh;
        P.page_shift = sh;
    }
    P.max_pages = max_pages;
    P.num_pages = num_pages;
    P.split_tokens = pl.split_tokens;
    P.num_splits = pl.num_splits;
    P.scale_log2 = scale * 1.4426950408889634f;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // x = work item * Hkv + kv head; items past the requests' splits exit.
    const dim3 grid(B * pl.num_splits * Hkv, pl.nqt);
    // Power-of-two pages of at least 4 tokens take the wave-uniform fetch.
    const bool upg = P.page_shift >= 2;
    switch (pl.waves) {
        case 2:
            if (upg)
                hipLaunchKernelGGL((attn_split_kernel<2, MODE, true, 1>), grid, dim3(128), 0, s, P);
            else
                hipLaunchKernelGGL((attn_split_kernel<2, MODE, false, 1>), grid, dim3(128), 0, s, P);
            break;
        case 4:
            if (pl.rt == 2) {
                if (upg)
                    hipLaunchKernelGGL((attn_split_kernel<4, MODE, true, 2>), grid, dim3(256), 0, s, P);
                else
                    hipLaunchKernelGGL((attn_split_kernel<4, MODE, false, 2>), grid, dim3(256), 0, s, P);
            } else {
                if (upg)
                    hipLaunchKernelGGL((attn_split_kernel<4, MODE, true, 1>), grid, dim3(256), 0, s, P);
                else
                    hipLaunchKernelGGL((attn_split_kernel<4, MODE, false, 1>), grid, dim3(256), 0, s, P);
            }
            break;
        default:
            return D3D_E_UNSUPPORTED;
    }
    if (pl.num_splits > 1)
    {
        const dim3 cgrid((P.M + kRowsPerCombine - 1) / kRowsPerCombine, Hkv, B * pl.nqt);
        const int ns = pl.num_splits;
        if (ns > kSpecSplits)
            hipLaunchKernelGGL(attn_combine_kernel<0>, cgrid, dim3(256), 0, s, P);
        else if (B > kSpecBatch)
            launch_slot_combine<true>(ns, cgrid, s, P);
        else
            launch_slot_combine<false>(ns, cgrid, s, P);
    }
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}

}  // namespace attn
}  // namespace d3d

using namespace d3d;

extern "C" size_t d3d_attn_workspace_bytes(int B, int Q, int Hq, int Hkv, int D, int page_size,
                                           int max_context) {
    if (B < 1 || Q < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv || D != attn::D || max_context < 1 || page_size < 1)
        return 0;
    return attn::plan(B, Q, Hq, Hkv, max_context, page_size).total;
}

extern "C" int d3d_verify_attn_paged(const void* q, const void* k_cache, const void* v_cache,
                                     const int32_t* block_table, const int32_t* context_lens, void* out, int B,
                                     int Q, int Hq, int Hkv, int D, int page_size, int max_pages, int num_pages,
                                     float scale, int max_context, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    return attn::run<attn::kCausal>(q, k_cache, v_cache, block_table, context_lens, nullptr, out, B, Q, Hq, Hkv, D,
                                    page_size, max_pages, num_pages, scale, max_context, workspace,
                                    workspace_bytes, stream);
}

extern "C" int d3d_draft_block_attn(const void* q, const void* k_cache, const void* v_cache,
                                    const int32_t* block_table, const int32_t* context_lens, void* out, int B,
                                    int Q, int Hq, int Hkv, int D, int page_size, int max_pages, int num_pages,
                                    float scale, int max_context, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    return attn::run<attn::kFull>(q, k_cache, v_cache, block_table, context_lens, nullptr, out, B, Q, Hq, Hkv, D,
                                  page_size, max_pages, num_pages, scale, max_context, workspace, workspace_bytes,
                                  stream);
}

extern "C" int d3d_packed_block_attn(const void* q, const void* k_cache, const void* v_cache,
                                     const int32_t* block_table, const int32_t* context_lens,
                                     const int32_t* q_visibility, void* out, int B, int Q, int Hq, int Hkv, int D,
                                     int page_size, int max_pages, int num_pages, float scale, int max_context,
                                     void* workspace, size_t workspace_bytes, void* stream) {
    return attn::run<attn::kPacked>(q, k_cache, v_cache, block_table, context_lens, q_visibility, out, B, Q, Hq,
                                    Hkv, D, page_size, max_pages, num_pages, scale, max_context, workspace,
                                    workspace_bytes, stream);
}

extern "C" int d3d_kv_append(const void* k, const void* v, void* k_cache, void* v_cache,
                             const int64_t* slot_mapping, int n_tokens, int Hkv, int D, int64_t num_slots,
                             void* stream) {
    if (n_tokens < 0 || Hkv < 1 || D < 8 || D % 8 || num_slots < 1) return D3D_E_SHAPE;
    if (n_tokens == 0) return D3D_OK;
    if (!k || !v || !k_cache || !v_cache || !slot_mapping) return D3D_E_NULL;
    hipLaunchKernelGGL(attn::kv_append_kernel, dim3(n_tokens), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                       static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), slot_mapping, Hkv * D,
                       num_slots);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? D3D_OK : (int)err;
}
