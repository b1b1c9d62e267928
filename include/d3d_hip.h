/*
 * libd3d_hip -- C ABI of the MI355X (gfx950) kernels for D3D's per-step
 * speculative hot path: fused acceptance, paged block-verify attention,
 * KV append, diffusion-draft block attention (recovery and packed
 * multi-branch), confidence/top-k unmask and the fused per-layer glue of the
 * target and draft forwards.
 *
 * Conventions shared by every entry point:
 *  - All tensor arguments are device pointers to contiguous row-major data
 *    owned by the caller.  The library allocates nothing.
 *  - `stream` is a hipStream_t passed as void* (0 = the null stream).  Work is
 *    enqueued on it; no entry point synchronises the host.
 *  - Return value: 0 on success, a negative D3D_E_* code for an argument that
 *    fails validation (nothing is launched), or a positive hipError_t when a
 *    launch fails.
 *  - Workspaces: size them with the matching *_workspace_bytes() call.  No
 *    initialisation is needed; a workspace can be reused by later calls on
 *    the same stream, but calls that share one workspace must not overlap
 *    in time (use one workspace per stream).
 */
#ifndef D3D_HIP_H
#define D3D_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of logits / probabilities. */
#define D3D_DTYPE_F32 0
#define D3D_DTYPE_BF16 1

/* What the acceptance inputs hold. */
#define D3D_INPUT_LOGITS 0 /* softmax(x / temperature); temperature <= 1e-5 selects greedy */
#define D3D_INPUT_PROBS 1  /* (unnormalised) probabilities, divided by max(sum, 1e-12) */

/* Status codes. */
#define D3D_OK 0
#define D3D_E_SHAPE (-1)
#define D3D_E_DTYPE (-2)
#define D3D_E_WORKSPACE (-3)
#define D3D_E_NULL (-4)
#define D3D_E_UNSUPPORTED (-5)
#define D3D_E_VALUE (-6) /* a scalar argument outside its domain (mode, threshold, top_p) */

/* Confidence of a greedy draft token (d3d_confidence_topk_unmask). */
#define D3D_CONF_MAX_SOFTMAX 0 /* softmax(logits / T')[argmax]: the metrics confidence */
#define D3D_CONF_ONE_HOT 1     /* 1.0: the reference's greedy low_confidence steps */

/* Sentinels written to out_token[b] by the acceptance kernels. */
#define D3D_TOKEN_EMPTY_DISTRIBUTION (-1) /* the resampling weights sum to zero */
/* A draft token id lies outside [0, V) (stochastic modes: the token indexes p
 * and q; accepted = 0, all_accepted = 0 and the mask is 0 at bad positions).
 * Greedy acceptance only compares tokens with the argmax, so there such a
 * token is a mismatch and the request is decided as usual. */
#define D3D_TOKEN_BAD_DRAFT (-2)
/* The residual reduction's cross-workgroup wait (for the other parts of the
 * same request) did not end within its bound of over 100 ms.  Not expected:
 * workgroups are dispatched in order.  Every output but out_token is valid. */
#define D3D_TOKEN_TIMEOUT (-3)

/* Short description of a status code (static storage). */
const char* d3d_status_string(int status);

/* Library version, major * 10000 + minor * 100 + patch. */
int d3d_version(void);

/*
 * Bytes of workspace d3d_accept_fused needs for B requests of K draft tokens
 * over a vocabulary of V entries (same for every dtype, input kind and mode).
 */
size_t d3d_accept_workspace_bytes(int B, int K, int64_t V);

/*
 * Fused acceptance for B independent requests in one HBM-streaming pass.
 *
 * Replaces, per request:
 *   single/eval_sync.py:287-305        _sampling_probs (temperature softmax)
 *   single/speculative_sampling.py:15-76 verify_speculative_block
 *   single/eval_sync.py:1223-1234      greedy acceptance (cumprod of matches)
 *   serving/engine.py:138-145          Engine._accepted
 *
 * target   [B, K+1, V]  rows 0..K-1 score draft token i, row K is the bonus row
 * draft    [B, K, V]    proposal rows (unused in greedy mode; may be NULL)
 * dtype    D3D_DTYPE_F32 or D3D_DTYPE_BF16 (both tensors)
 * input_kind  D3D_INPUT_LOGITS or D3D_INPUT_PROBS
 * draft_tokens [B, K] int64
 * uniforms     [B, K] fp32 in [0, 1): position i accepted iff u_i <= a_i,
 *              a_i = min(1, p_i(x_i) / max(q_i(x_i), 1e-12))
 * resample_u   [B] fp32 in [0, 1): drives the inverse-CDF draw of the
 *              correction (or bonus) token
 * temperature  logits mode only; <= 1e-5 selects greedy acceptance
 *              (uniforms, resample_u and draft unused, may be NULL)
 *
 * Outputs (device):
 *   accepted     [B] int32  accepted draft tokens, 0..K
 *   accept_mask  [B, K] uint8  the per-position decision at every position
 *   out_token    [B] int64  correction token (or bonus token when all K are
 *                accepted); D3D_TOKEN_* sentinels on invalid input
 *   all_accepted [B] uint8
 *   posterior    [B, K+1] int64  argmax of every target row (may be NULL;
 *                the stochastic modes then skip the argmax reduction)
 */
int d3d_accept_fused(const void* target, const void* draft, int dtype, int input_kind,
                     const int64_t* draft_tokens, const float* uniforms,
                     const float* resample_u, float temperature, int B, int K, int64_t V,
                     int32_t* accepted, uint8_t* accept_mask, int64_t* out_token,
                     uint8_t* all_accepted, int64_t* posterior, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * Fused acceptance against sparse proposals: as d3d_accept_fused, with the
 * draft side given as S (id, probability) pairs per position.
 *
 * Replaces single/speculative_sampling.py:79-143
 * (verify_speculative_block_sparse), batched over B requests:
 *   q_i(x)  = sum over s with q_ids[b,i,s] == x of q_probs[b,i,s] / Z_i,
 *             Z_i = max(sum_s q_probs[b,i,s], 1e-12)
 *   residual at the first reject j: p_j minus every q_probs[b,j,s] / Z_j at
 *   q_ids[b,j,s] (subtracted in support order, duplicates accumulate), then
 *   clamped at zero; p_j itself when that mass is <= 1e-12.
 *
 * q_ids [B, K, S] int64 (ids outside [0, V) carry no mass), q_probs
 * [B, K, S] fp32, 1 <= S <= 1024.  Uses d3d_accept_workspace_bytes.  In
 * greedy mode (logits, temperature <= 1e-5) the proposals are unused and
 * the result is d3d_accept_fused's greedy acceptance.
 */
int d3d_accept_fused_sparse(const void* target, int dtype, int input_kind,
                            const int64_t* draft_tokens, const int64_t* q_ids, const float* q_probs,
                            int S, const float* uniforms, const float* resample_u, float temperature,
                            int B, int K, int64_t V, int32_t* accepted, uint8_t* accept_mask,
                            int64_t* out_token, uint8_t* all_accepted, int64_t* posterior,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Size of the static scratch d3d_accept_fused_noalloc uses on each GPU. */
#define D3D_ACCEPT_NOALLOC_SCRATCH_BYTES (4u << 20)

/*
 * d3d_accept_fused without a caller workspace and without any allocation:
 * the same kernels, arguments and outputs, with the row statistics kept in
 * a file-scope device array of D3D_ACCEPT_NOALLOC_SCRATCH_BYTES (4 MiB) that
 * each GPU the library runs on holds until the process ends.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).
 *
 * Sizes whose workspace (d3d_accept_workspace_bytes(B, K, V)) exceeds the
 * scratch return D3D_E_WORKSPACE before anything is launched: at K = 15 and
 * V = 151,936 that is B > 213.  The scratch needs no clearing between calls.
 * The first call on a device looks the array's address up (once per
 * device, with that device current); make it before any graph capture.
 * Every call on one GPU shares that GPU's array: calls that overlap in time
 * on one GPU (different streams, or different threads) race.
 */
int d3d_accept_fused_noalloc(const void* target, const void* draft, int dtype, int input_kind,
                             const int64_t* draft_tokens, const float* uniforms,
                             const float* resample_u, float temperature, int B, int K, int64_t V,
                             int32_t* accepted, uint8_t* accept_mask, int64_t* out_token,
                             uint8_t* all_accepted, int64_t* posterior, void* stream);

/*
 * Bytes of workspace the paged attention entry points need (split-context
 * partials).  max_context bounds every context_lens[b]; the same value must
 * be passed to the attention call.
 */
size_t d3d_attn_workspace_bytes(int B, int Q, int Hq, int Hkv, int D, int page_size,
                                int max_context);

/*
 * Block-verify attention over a paged KV cache, causal within the block.
 *
 * Replaces flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens,
 * block_table, causal=True, softmax_scale) at
 * serving/vendor/ssd/layers/attention.py:38-41.
 *
 * q, out       [B, Q, Hq, D] bf16
 * k_cache, v_cache [num_pages, page_size, Hkv, D] bf16 (layout of
 *              serving/backend.py:46-48)
 * block_table  [B, max_pages] int32 page ids
 * context_lens [B] int32, keys per request including the block's own Q
 *              keys (already appended); query i sees keys
 *              j <= context_lens[b] - Q + i
 * D must be 128; Hq / Hkv <= 128 (blocks of more than 128 / (Hq / Hkv)
 * queries are tiled over workgroups).  Page ids outside [0, num_pages)
 * read as zero keys/values instead of faulting.
 */
int d3d_verify_attn_paged(const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_table, const int32_t* context_lens, void* out,
                          int B, int Q, int Hq, int Hkv, int D, int page_size, int max_pages,
                          int num_pages, float scale, int max_context, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * Diffusion-draft block attention: as d3d_verify_attn_paged, but every
 * query of the block sees every key j < context_lens[b] (prefix plus the
 * bidirectional block).
 *
 * Replaces the draft branch of serving/vendor/ssd/layers/attention.py:42-52
 * under the recovery mask of serving/engine.py:41-42 (cols < prefix + Q), and
 * the all-true block mask of the single-request draft step
 * (single/eval_sync.py:531-540 with models/d3d/modeling_d3d.py:345-364).
 */
int d3d_draft_block_attn(const void* q, const void* k_cache, const void* v_cache,
                         const int32_t* block_table, const int32_t* context_lens, void* out,
                         int B, int Q, int Hq, int Hkv, int D, int page_size, int max_pages,
                         int num_pages, float scale, int max_context, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * Packed multi-branch draft attention: as d3d_draft_block_attn, with the
 * visible keys of each query given by a descriptor instead of a mask.
 * With prefix = context_lens[b] - Q (the block's Q keys are appended after
 * the prefix), query i sees key t iff
 *     t < prefix + q_visibility[i][0]
 *  or prefix + q_visibility[i][1] <= t < prefix + q_visibility[i][2].
 * q_visibility [Q][3] int32 is shared by the B requests.  Q is unbounded
 * (queries are tiled over workgroups).
 *
 * Replaces the draft branch of serving/vendor/ssd/layers/attention.py:42-52
 * under the packed mask of serving/engine.py:43-50 (Engine._mask with
 * branch specs): the pending block's rows i see (prefix + i + 1) keys,
 * i.e. {i + 1, 0, 0}; rows of the branch at offset off with n accepted
 * pending tokens see {n, off, off + K}.  Uses d3d_attn_workspace_bytes.
 */
int d3d_packed_block_attn(const void* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_table, const int32_t* context_lens,
                          const int32_t* q_visibility, void* out, int B, int Q, int Hq, int Hkv,
                          int D, int page_size, int max_pages, int num_pages, float scale,
                          int max_context, void* workspace, size_t workspace_bytes, void* stream);

/*
 * KV append: k_cache.view(-1, Hkv, D)[slot_mapping] = k (and v), as at
 * serving/vendor/ssd/layers/attention.py:21-22.  k, v [n_tokens, Hkv, D]
 * bf16; slot_mapping [n_tokens] int64; num_slots = num_pages * page_size.
 * Slots outside [0, num_slots) are skipped.
 */
int d3d_kv_append(const void* k, const void* v, void* k_cache, void* v_cache,
                  const int64_t* slot_mapping, int n_tokens, int Hkv, int D, int64_t num_slots,
                  void* stream);

/* Bytes of workspace d3d_confidence_topk_unmask needs. */
size_t d3d_confidence_workspace_bytes(int B, int Q, int64_t V);

/*
 * One denoise iteration of the diffusion draft: greedy token and confidence
 * for every position, then top-k unmask of the masked positions, in place.
 *
 * Replaces single/eval_sync.py:447-465 (_select_transfer) with x0 =
 * argmax(logits) and, by conf_mode, either the metrics confidence of
 * single/eval_sync.py:713-717 (D3D_CONF_MAX_SOFTMAX: conf =
 * softmax(logits / T')[x0], T' = T when T > 1e-5, else 1) or the one-hot
 * confidence of the greedy _sample_with_prob, single/eval_sync.py:287-291
 * and :323-338 (D3D_CONF_ONE_HOT: conf = 1.0, greedy only, else
 * D3D_E_UNSUPPORTED).  Among positions with block_ids == mask_id the kk
 * highest confidences (ties: lowest position; all of them when kk >= their
 * count) take x0, where kk = k, or with dynamic != 0 ("dynamic" remasking,
 * single/eval_sync.py:453-462) kk = min(k, n) when n > 0 masked positions
 * have conf >= threshold.  Selection is per request.
 *
 * logits [B, Q, V] fp32 or bf16; block_ids [B, Q] int64 (in/out);
 * x0_out [B, Q] int64 and conf_out [B, Q] fp32 may be NULL.  Q <= 1024.
 */
int d3d_confidence_topk_unmask(const void* logits, int dtype, int64_t* block_ids, int64_t mask_id,
                               int k, float temperature, int conf_mode, int dynamic, float threshold,
                               int B, int Q, int64_t V, int64_t* x0_out, float* conf_out,
                               void* workspace, size_t workspace_bytes, void* stream);

/*
 * Top-k unmask with caller-given tokens and confidences: among positions
 * with block_ids == mask_id, the kk highest conf (ties: lowest position; all
 * of them when kk >= their count) take x0, in place, with kk as in
 * d3d_confidence_topk_unmask (dynamic threshold remasking when dynamic !=
 * 0); selected_out [B, Q] uint8 (may be NULL) marks the positions unmasked.
 * x0 [B, Q] int64, conf [B, Q] fp32, Q <= 1024.
 *
 * Replaces _select_transfer, single/eval_sync.py:447-465, when x0 and its
 * confidence come from the sampled proposal (_sample_with_prob or the
 * sparse support, single/eval_sync.py:560-576); selection is per request.
 */
int d3d_select_transfer(int64_t* block_ids, int64_t mask_id, int k, int dynamic, float threshold,
                        const int64_t* x0, const float* conf, uint8_t* selected_out, int B, int Q,
                        void* stream);

/* Bytes of workspace d3d_topk_rows needs. */
size_t d3d_topk_workspace_bytes(int N, int64_t V, int k);

/*
 * Top-k token ids of N logits rows [N, V] (fp32 or bf16): ids_out [N, k]
 * int64 in descending order of value, equal values by ascending id (so
 * ids_out[n][0] is the argmax with torch's first-maximum rule); NaN entries
 * are never selected.  vals_out [N, k] fp32 may be NULL; with log_softmax
 * != 0 it holds log_softmax(x) of the selected entries (x - logsumexp(x)),
 * else the raw values.  1 <= k <= 64, N <= 65535, ceil(V / 4096) * k <= 8192.
 *
 * Replaces logits.argmax(-1) and logits.topk(k).indices in Runner._run,
 * serving/backend.py:84-93, which feed the anchor choice of
 * Engine._recover / Engine._predict (serving/engine.py:54-131), and
 * torch.topk(log_softmax(logits), k) of the anchor draft,
 * single/eval_sync.py:763-768.
 */
int d3d_topk_rows(const void* logits, int dtype, int N, int64_t V, int k, int log_softmax,
                  int64_t* ids_out, float* vals_out, void* workspace, size_t workspace_bytes,
                  void* stream);

/*
 * Block inputs of B requests from a device-resident page-table pool
 * page_pool [pool_rows, pool_width] int32 (one row of page ids per sequence,
 * -1 past its page list; rows[b] the row of request b): tables_out [B, width]
 * int32 (the row's first width entries with -1 shown as 0, 0 past the pool
 * width or for a row outside the pool), slots_out [B, Q] int64 = page *
 * page_size + pos % page_size with page = row[pos / page_size] for pos =
 * starts[b] + i (-1 when that page index is past width or the entry is -1:
 * d3d_kv_append skips the token),
 * positions_out [B, Q] int64 = pos and context_lens_out [B] int32 =
 * starts[b] + Q (either may be NULL).  All pointers are device memory.
 *
 * Replaces the per-step host list work of Runner._tables and the slot
 * mapping of Runner.forward, serving/backend.py:73-76 and :123-124.
 */
int d3d_block_inputs(const int32_t* page_pool, int pool_rows, int pool_width, const int32_t* rows,
                     const int32_t* starts, int B, int Q, int width, int page_size, int32_t* tables_out,
                     int64_t* slots_out, int64_t* positions_out, int32_t* context_lens_out, void* stream);

/* Bytes of workspace d3d_lmhead_topk needs. */
size_t d3d_lmhead_workspace_bytes(int T, int64_t V, int k);

/*
 * Fused LM head + top-k: the logits hidden [T, H] x weight[V, H]^T (bf16,
 * row-major, 16-byte aligned, H a multiple of 32) rounded to bf16 and
 * reduced without being written: ids_out [T, k] int64 in descending order of
 * value, equal values by ascending id (ids_out[t][0] is the argmax with
 * torch's first-maximum rule); vals_out [T, k] fp32 (may be NULL) holds the
 * bf16 logits, or with log_softmax != 0 their log-softmax x - logsumexp(x)
 * over the whole row.  1 <= k <= 8, T <= 65535.  Hidden rows are taken 64
 * at a time and the weight is streamed once per 64 rows: meant for up to 64
 * rows (one pass over the weight), correct for any T.
 *
 * Replaces lm_head(h) followed by logits.argmax(-1) / logits.topk(k) in
 * Runner._run, serving/backend.py:84-93, and the draft's argmax and
 * torch.topk(log_softmax(logits), k), single/eval_sync.py:713-717 and
 * :763-768; the [T, V] logits are never materialised.
 */
int d3d_lmhead_topk(const void* hidden, const void* weight, int T, int H, int64_t V, int k,
                    int log_softmax, int64_t* ids_out, float* vals_out, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Bytes of workspace d3d_sample_rows needs. */
size_t d3d_sample_workspace_bytes(int N, int64_t V);

/*
 * One proposal token per logits row [N, V] (fp32 or bf16) and its
 * probability.  temperature <= 1e-5: the argmax (first maximum) with
 * probability 1 (uniforms and kth unused, may be NULL).  Otherwise p =
 * softmax(z) over z = logits / T, restricted, when kth (may be NULL) is
 * given, to the entries with z >= kth[n] / T (top-k filtering: kth[n] is the
 * row's k-th largest logit, so ties with it are kept), and token = the first
 * t with C_t > u[n] * W over the softmax weights, else the last t with
 * positive weight (inverse CDF in place of torch.multinomial); probs_out[n]
 * = p[token] (may be NULL).  zfloor / zlimit [N] (both NULL, or both given:
 * the row filter of d3d_row_filter) further restrict the entries to z >
 * zfloor[n], or z == zfloor[n] at ids <= zlimit[n].  N <= 65535.
 * D3D_TOKEN_EMPTY_DISTRIBUTION if a row has no finite entry.
 *
 * Replaces _sample_tokens / _sample_with_prob over _sampling_probs,
 * single/eval_sync.py:287-338 (top-k filtering :293-295; top-p is served by
 * d3d_sample_support).
 */
int d3d_sample_rows(const void* logits, int dtype, int N, int64_t V, float temperature,
                    const float* kth, const float* zfloor, const int32_t* zlimit, const float* uniforms,
                    int64_t* tokens_out, float* probs_out, void* workspace, size_t workspace_bytes,
                    void* stream);

/*
 * The dense proposal distribution of N logits rows [N, V]: probs_out [N, V]
 * fp32 = softmax(logits / T) over the entries kept by the top-k floor kth
 * (as in d3d_sample_rows; may be NULL), 0 elsewhere; temperature <= 1e-5
 * gives the one-hot row at the argmax (first maximum).  Workspace as
 * d3d_sample_workspace_bytes(N, V).
 *
 * Replaces _sampling_probs, single/eval_sync.py:287-305, where the draft
 * keeps proposal_probs (:566-570, :577-584) for verify_speculative_block.
 */
int d3d_softmax_rows(const void* logits, int dtype, int N, int64_t V, float temperature, const float* kth,
                     const float* zfloor, const int32_t* zlimit, float* probs_out, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * The per-row filter of _sampling_probs' top-k and top-p options
 * (single/eval_sync.py:292-303) over N logits rows [N, V] at temperature T >
 * 1e-5, for d3d_sample_rows / d3d_softmax_rows: with z = logits / T (fp32),
 * top_k in 1..V-1 keeps the entries at or above the k-th largest z (ties
 * kept; 0 or >= V: off); top_p < 1 then sorts the kept entries by z
 * descending (ties by ascending id), and keeps the shortest prefix whose
 * softmax mass exceeds top_p (the entry that crosses it included).  The
 * result is zfloor_out / zlimit_out [N]: entry e is kept iff z > zfloor, or
 * z == zfloor and e <= zlimit.  NaN entries are never kept.  0 < top_p <= 1.
 */
int d3d_row_filter(const void* logits, int dtype, int N, int64_t V, float temperature, int top_k, float top_p,
                   float* zfloor_out, int32_t* zlimit_out, void* stream);

/* Bytes of workspace d3d_sample_support_wide needs. */
size_t d3d_support_workspace_bytes(int N, int S);

/*
 * _sample_with_sparse_probs (single/eval_sync.py:341-367) for supports of
 * any size 1 <= S <= V (V <= 2^18; S = V is top_k = 0, the whole vocabulary):
 * support_ids_out [N, S] int64 = the S largest z = logits / T in descending
 * order (ties by ascending id), support_probs_out [N, S] = softmax over the
 * support after the nucleus filter (top_p < 1: entry s > 0 is dropped when
 * the inclusive probability of entries 0..s-1 exceeds top_p, the rest
 * renormalised), tokens_out [N] = the inverse-CDF draw over the support in
 * support order at uniforms[n], token_probs_out [N] (may be NULL) its
 * probability.  T > 1e-5, 0 < top_p <= 1.  Workspace:
 * d3d_support_workspace_bytes(N, S).  d3d_topk_rows + d3d_sample_support
 * cover S <= 64 in one launch pair.
 */
int d3d_sample_support_wide(const void* logits, int dtype, int N, int64_t V, float temperature, int S,
                            float top_p, const float* uniforms, int64_t* tokens_out, int64_t* support_ids_out,
                            float* support_probs_out, float* token_probs_out, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Sparse proposal over a top-S support: support_vals / support_ids [N, S]
 * are the S largest logits of each row in descending order with their ids
 * (d3d_topk_rows).  support_probs_out [N, S] = softmax(support_vals / T),
 * and with top_p < 1 the nucleus filter: entry s > 0 is dropped (probability
 * 0, the rest renormalised) when the inclusive sum of the first s
 * probabilities exceeds top_p; tokens_out[n] = support_ids[n, s] for the
 * first s whose inclusive sum exceeds u[n] * W (else the last positive
 * entry); token_probs_out (may be NULL) the drawn entry's probability.
 * 1 <= S <= 64, temperature > 1e-5, 0 < top_p <= 1.
 *
 * Replaces _sample_with_sparse_probs, single/eval_sync.py:341-367.
 */
int d3d_sample_support(const float* support_vals, const int64_t* support_ids, int N, int S,
                       float temperature, float top_p, const float* uniforms, int64_t* tokens_out,
                       float* support_probs_out, float* token_probs_out, void* stream);

/*
 * Residual add + RMSNorm over rows of H bf16 entries (H a multiple of 8,
 * H <= 8192): s = x + residual in fp32, residual = bf16(s) (in place),
 * out = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * weight).  With x == NULL the
 * residual is only normalised (the first layer's input norm) and left as is.
 * Every pointer must be 16-byte aligned (D3D_E_UNSUPPORTED otherwise).
 *
 * Replaces RMSDNorm.add_norm_forward / norm_forward,
 * serving/vendor/ssd/layers/layernorm.py:53-98, as called by the decoder
 * layers of serving/vendor/ssd/models/qwen3.py and the draft's
 * models/d3d/modeling_d3d.py.
 */
int d3d_add_rmsnorm(const void* x, void* residual, const void* weight, void* out, int T, int H,
                    float eps, void* stream);

/*
 * Per-token attention input: for each of T tokens, qkv [T, (Hq + 2 Hkv) * D]
 * bf16 holds q, k and v heads.  q and k heads get RMSNorm over D with
 * q_norm_w / k_norm_w (RMSHeadNorm, serving/vendor/ssd/layers/layernorm.py:1-52)
 * and rotate-half RoPE at positions[t] with angle positions[t] * inv_freq[i]
 * (inv_freq [D/2] fp32).  draft_rope == 0 rotates in fp32 and rounds once
 * (serving/vendor/ssd/layers/rotary_embedding.py:6-16); draft_rope != 0
 * rounds cos, sin and every product and sum to bf16
 * (models/d3d/modeling_d3d.py:164-187).  q goes to q_out [T, Hq, D]; k and
 * v go to the paged caches at slot_mapping[t] as d3d_kv_append stores them
 * (serving/vendor/ssd/layers/attention.py:21-22).  D must be 128.
 */
int d3d_qk_rope_append(const void* qkv, const int64_t* positions, const void* q_norm_w,
                       const void* k_norm_w, const float* inv_freq, void* q_out, void* k_cache,
                       void* v_cache, const int64_t* slot_mapping, int T, int Hq, int Hkv, int D,
                       float eps, int draft_rope, int64_t num_slots, void* stream);

/*
 * out [T, M] = silu(gate) * up for gate_up [T, 2M] = [gate | up] bf16,
 * evaluated in fp32 and rounded once (SiluAndMul,
 * serving/vendor/ssd/layers/activation.py:6-14).  M a multiple of 8;
 * gate_up and out 16-byte aligned (D3D_E_UNSUPPORTED otherwise).
 */
int d3d_silu_mul(const void* gate_up, void* out, int T, int M, void* stream);

/*
 * Projection of a block of at most 64 rows: Y[M, N] = X[M, K] W[N, K]^T with
 * bf16 X (row-major, row stride K) and W (the [out, in] weight), fp32
 * accumulation.  Replaces the F.linear of the decoder layer's qkv, o and
 * down projections (serving/vendor/ssd/models/qwen3.py, as linear.py runs
 * them) for verify and draft blocks.  1 <= M <= 64, N a multiple of 64, K a
 * multiple of 128 * splits, X and W 16-byte aligned.  splits == 1 writes Y
 * as bf16 [M, N]; splits > 1 (at most 16) writes the fp32 partial products
 * of the splits' K ranges to parts [splits, M, N] instead, for
 * d3d_add_rmsnorm_parts or d3d_qk_rope_append_parts to sum.  Y (or parts)
 * must not overlap X or W.
 */
int d3d_gemm_rows64(const void* x, const void* w, void* y, float* parts, int M, int N, int K, int splits,
                    void* stream);

/*
 * The decoder layer's gate-up projection and SiluAndMul in one launch for a
 * block of at most 64 rows (Qwen3MLP.forward, serving/vendor/ssd/models/
 * qwen3.py:139-142: gate_up_proj, then act_fn = SiluAndMul,
 * serving/vendor/ssd/layers/activation.py:6-14): y [M, H] bf16 =
 * silu(g) * u, where g and u are the bf16-rounded products X Wg^T and
 * X Wu^T of w_gate_up [2H, K] = [gate rows | up rows] -- the values
 * d3d_gemm_rows64 (one split) followed by d3d_silu_mul give, bit for bit.
 * 1 <= M <= 64, H a multiple of 32, K / 128 in {8, 16, 24, 32, 48, 64}
 * (D3D_E_UNSUPPORTED otherwise), X and W 16-byte aligned.
 */
int d3d_gemm_rows64_silu_mul(const void* x, const void* w_gate_up, void* y, int M, int H, int K, void* stream);

/* The split count d3d_gemm_rows64 is fastest with for an [N, K] weight (1 when N or K
 * is not a multiple of 64 or 128). */
int d3d_gemm_rows64_splits(int N, int K);

/*
 * d3d_add_rmsnorm with x given as the partials of d3d_gemm_rows64:
 * x[t, i] = bf16(sum over s in order of parts[s, t, i]), parts
 * [splits, T, H] fp32, 16-byte aligned.
 */
int d3d_add_rmsnorm_parts(const float* parts, int splits, void* residual, const void* weight, void* out, int T,
                          int H, float eps, void* stream);

/*
 * d3d_qk_rope_append with qkv given as the partials of d3d_gemm_rows64:
 * qkv[t, i] = bf16(sum over s in order of parts[s, t, i]), parts
 * [splits, T, (Hq + 2 Hkv) * D] fp32.
 */
int d3d_qk_rope_append_parts(const float* parts, int splits, const int64_t* positions, const void* q_norm_w,
                             const void* k_norm_w, const float* inv_freq, void* q_out, void* k_cache,
                             void* v_cache, const int64_t* slot_mapping, int T, int Hq, int Hkv, int D,
                             float eps, int draft_rope, int64_t num_slots, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* D3D_HIP_H */
