/*
 * ORACLE -- test infrastructure only.
 *
 * A CPU restatement, in double precision, of D3D's per-step acceptance
 * arithmetic.  The tests compare the HIP kernels in d3d_amd/csrc against it;
 * it is never linked into, called by, or shipped with the product path: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
 *
 * Reference behaviour restated here (paths relative to the D3D repository):
 *   single/eval_sync.py:287-305          _sampling_probs (temperature softmax,
 *                                        one-hot argmax at T <= 1e-5)
 *   single/speculative_sampling.py:37-40 p / p.sum().clamp_min(1e-12)
 *   single/speculative_sampling.py:46-56 a_i = min(1, p_tok / max(q_tok, 1e-12)),
 *                                        accept iff u_i <= a_i
 *   single/speculative_sampling.py:57-69 first reject, bonus row when none,
 *                                        residual max(p - q, 0) with the
 *                                        mass <= 1e-12 fallback to p
 *   single/speculative_sampling.py:99-135 sparse proposal: q_tok by support
 *                                        match, residual by scatter-add of -q
 *   single/eval_sync.py:1223-1234        greedy: leading matches of the draft
 *                                        against argmax, correction = argmax[n]
 *
 * torch.multinomial (single/speculative_sampling.py:71, :138) is replaced by
 * a defined inverse CDF driven by a caller-supplied uniform v in [0, 1):
 *   token = min{ t : C_t > v * W },  C_t = sum_{s <= t} w_s,  W = C_{V-1}
 * over the unnormalised weights w (residual, or p).  When rounding leaves no
 * such t, the last t with w_t > 0 is taken.  W <= 0 yields -1 (the reference
 * raises from torch.multinomial there).
 *
 * A draft token outside [0, V) makes the reference's gather p[.., token_ids]
 * (speculative_sampling.py:50-54, :108-110) raise: such a request reports
 * out_token = -2 with accepted = 0 and all_accepted = 0; its mask holds the
 * decision of every in-range position and 0 at the bad ones, and both
 * margins are +inf (no rounding can change that outcome).  Greedy acceptance
 * only compares tokens with the argmax (eval_sync.py:1223-1234), so there an
 * out-of-range token is a mismatch like any other.
 *
 * Each routine also reports its decision margins, which the fixture writer
 * uses to keep only inputs whose result does not depend on fp32 rounding:
 *   u_margin   = min_i |u_i - a_i| over every draft position
 *   cdf_margin = min(v*W - C_{t-1}, C_t - v*W) / W at the chosen token
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_KIND_LOGITS 0
#define ORACLE_KIND_PROBS 1

/* torch.argmax tie rule: the first index holding the maximum. */
long oracle_argmax_f32(const float* x, long V) {
    long best = 0;
    for (long t = 1; t < V; ++t)
        if (x[t] > x[best]) best = t;
    return best;
}

/* One probability row.  kind LOGITS: softmax(x / T) (eval_sync.py:292-305),
 * one-hot argmax when T <= 1e-5 (:288-291).  kind PROBS: x as given.  Both
 * are then divided by max(sum, 1e-12) (speculative_sampling.py:37-40). */
void oracle_row_probs(const float* x, long V, int kind, double T, double* p) {
    if (kind == ORACLE_KIND_LOGITS && T <= 1e-5) {
        memset(p, 0, sizeof(double) * (size_t)V);
        p[oracle_argmax_f32(x, V)] = 1.0;
    } else if (kind == ORACLE_KIND_LOGITS) {
        double m = -INFINITY;
        for (long t = 0; t < V; ++t) {
            double z = (double)x[t] / T;
            if (z > m) m = z;
        }
        double s = 0.0;
        for (long t = 0; t < V; ++t) {
            p[t] = exp((double)x[t] / T - m);
            s += p[t];
        }
        for (long t = 0; t < V; ++t) p[t] /= s;
    } else {
        for (long t = 0; t < V; ++t) p[t] = (double)x[t];
    }
    double s = 0.0;
    for (long t = 0; t < V; ++t) s += p[t];
    if (s < 1e-12) s = 1e-12;
    for (long t = 0; t < V; ++t) p[t] /= s;
}

/* Inverse CDF over unnormalised weights; see the header comment. */
long oracle_inverse_cdf(const double* w, long V, double v, double* margin) {
    double W = 0.0;
    for (long t = 0; t < V; ++t) W += w[t];
    if (!(W > 0.0)) {
        if (margin) *margin = 0.0;
        return -1;
    }
    double target = v * W, c = 0.0;
    for (long t = 0; t < V; ++t) {
        double prev = c;
        c += w[t];
        if (c > target) {
            if (margin) {
                double lo = target - prev, hi = c - target;
                *margin = (lo < hi ? lo : hi) / W;
            }
            return t;
        }
    }
    if (margin) *margin = 0.0;
    for (long t = V - 1; t >= 0; --t)
        if (w[t] > 0.0) return t;
    return -1;
}

static double accept_prob(double p_tok, double q_tok) {
    double r = p_tok / (q_tok > 1e-12 ? q_tok : 1e-12);
    return r < 1.0 ? r : 1.0;
}

/*
 * Dense acceptance for B independent requests (the reference handles B = 1,
 * speculative_sampling.py:44-45; each request here follows that rule).
 *   target [B, K+1, V], draft [B, K, V] fp32, tokens [B, K], u [B, K], ru [B]
 * Outputs: mask [B, K] (u_i <= a_i at every position), accepted [B],
 * out_token [B], all_accepted [B], u_margin [B], cdf_margin [B].
 */
void oracle_accept_dense(const float* target, const float* draft, int kind, double T,
                         const int64_t* tokens, const float* u, const float* ru,
                         int B, int K, long V, uint8_t* mask, int32_t* accepted,
                         int64_t* out_token, uint8_t* all_accepted, double* u_margin,
                         double* cdf_margin) {
    double* p = (double*)malloc(sizeof(double) * (size_t)V);
    double* q = (double*)malloc(sizeof(double) * (size_t)V);
    for (int b = 0; b < B; ++b) {
        const float* tb = target + (size_t)b * (K + 1) * V;
        const float* db = draft + (size_t)b * K * V;
        int n = K, bad = 0;
        double um = INFINITY;
        for (int i = 0; i < K; ++i) {
            long tok = (long)tokens[(size_t)b * K + i];
            if (tok < 0 || tok >= V) {
                mask[(size_t)b * K + i] = 0;
                bad = 1;
                continue;
            }
            oracle_row_probs(tb + (size_t)i * V, V, kind, T, p);
            oracle_row_probs(db + (size_t)i * V, V, kind, T, q);
            double a = accept_prob(p[tok], q[tok]);
            double ui = (double)u[(size_t)b * K + i];
            int acc = ui <= a;
            mask[(size_t)b * K + i] = (uint8_t)acc;
            double d = fabs(ui - a);
            if (d < um) um = d;
            if (!acc && n == K) n = i;
        }
        if (bad) {
            accepted[b] = 0;
            all_accepted[b] = 0;
            out_token[b] = -2;
            u_margin[b] = INFINITY;
            cdf_margin[b] = INFINITY;
            continue;
        }
        u_margin[b] = um;
        accepted[b] = n;
        all_accepted[b] = (uint8_t)(n == K);
        oracle_row_probs(tb + (size_t)n * V, V, kind, T, p);
        if (n < K) {
            oracle_row_probs(db + (size_t)n * V, V, kind, T, q);
            double mass = 0.0;
            for (long t = 0; t < V; ++t) {
                q[t] = p[t] - q[t] > 0.0 ? p[t] - q[t] : 0.0;
                mass += q[t];
            }
            if (mass > 1e-12) memcpy(p, q, sizeof(double) * (size_t)V);
        }
        out_token[b] = oracle_inverse_cdf(p, V, (double)ru[b], &cdf_margin[b]);
    }
    free(p);
    free(q);
}

/*
 * Sparse-proposal acceptance (speculative_sampling.py:79-143), batched the
 * same way.  q_ids / q_probs [B, K, S]; q_probs rows are normalised over S.
 * Support ids outside [0, V) are ignored.
 */
void oracle_accept_sparse(const float* target, int kind, double T, const int64_t* tokens,
                          const int64_t* q_ids, const float* q_probs, int S, const float* u,
                          const float* ru, int B, int K, long V, uint8_t* mask,
                          int32_t* accepted, int64_t* out_token, uint8_t* all_accepted,
                          double* u_margin, double* cdf_margin) {
    double* p = (double*)malloc(sizeof(double) * (size_t)V);
    for (int b = 0; b < B; ++b) {
        const float* tb = target + (size_t)b * (K + 1) * V;
        int n = K, bad = 0;
        double um = INFINITY;
        for (int i = 0; i < K; ++i) {
            size_t row = ((size_t)b * K + i) * S;
            long tok = (long)tokens[(size_t)b * K + i];
            if (tok < 0 || tok >= V) {
                mask[(size_t)b * K + i] = 0;
                bad = 1;
                continue;
            }
            oracle_row_probs(tb + (size_t)i * V, V, kind, T, p);
            double qs = 0.0, qt = 0.0;
            for (int s = 0; s < S; ++s) qs += (double)q_probs[row + s];
            if (qs < 1e-12) qs = 1e-12;
            for (int s = 0; s < S; ++s)
                if ((long)q_ids[row + s] == tok) qt += (double)q_probs[row + s] / qs;
            double a = accept_prob(p[tok], qt);
            double ui = (double)u[(size_t)b * K + i];
            int acc = ui <= a;
            mask[(size_t)b * K + i] = (uint8_t)acc;
            double d = fabs(ui - a);
            if (d < um) um = d;
            if (!acc && n == K) n = i;
        }
        if (bad) {
            accepted[b] = 0;
            all_accepted[b] = 0;
            out_token[b] = -2;
            u_margin[b] = INFINITY;
            cdf_margin[b] = INFINITY;
            continue;
        }
        u_margin[b] = um;
        accepted[b] = n;
        all_accepted[b] = (uint8_t)(n == K);
        oracle_row_probs(tb + (size_t)n * V, V, kind, T, p);
        if (n < K) {
            size_t row = ((size_t)b * K + n) * S;
            double qs = 0.0;
            for (int s = 0; s < S; ++s) qs += (double)q_probs[row + s];
            if (qs < 1e-12) qs = 1e-12;
            double* r = (double*)malloc(sizeof(double) * (size_t)V);
            memcpy(r, p, sizeof(double) * (size_t)V);
            for (int s = 0; s < S; ++s) {
                long id = (long)q_ids[row + s];
                if (id >= 0 && id < V) r[id] -= (double)q_probs[row + s] / qs;
            }
            double mass = 0.0;
            for (long t = 0; t < V; ++t) {
                if (r[t] < 0.0) r[t] = 0.0;
                mass += r[t];
            }
            if (mass > 1e-12) memcpy(p, r, sizeof(double) * (size_t)V);
            free(r);
        }
        out_token[b] = oracle_inverse_cdf(p, V, (double)ru[b], &cdf_margin[b]);
    }
    free(p);
}

/*
 * Greedy acceptance (eval_sync.py:1223-1234; engine.py:138-145): posterior =
 * argmax of every target row, accepted = number of leading draft tokens equal
 * to the posterior of the row before them, correction = posterior[accepted].
 * mask[i] = (tokens[i] == posterior[i]) at every position.
 */
void oracle_accept_greedy(const float* target, const int64_t* tokens, int B, int K, long V,
                          int64_t* posterior, uint8_t* mask, int32_t* accepted,
                          int64_t* out_token, uint8_t* all_accepted) {
    for (int b = 0; b < B; ++b) {
        const float* tb = target + (size_t)b * (K + 1) * V;
        for (int i = 0; i <= K; ++i)
            posterior[(size_t)b * (K + 1) + i] = oracle_argmax_f32(tb + (size_t)i * V, V);
        int n = K;
        for (int i = 0; i < K; ++i) {
            int m = tokens[(size_t)b * K + i] == posterior[(size_t)b * (K + 1) + i];
            mask[(size_t)b * K + i] = (uint8_t)m;
            if (!m && n == K) n = i;
        }
        accepted[b] = n;
        all_accepted[b] = (uint8_t)(n == K);
        out_token[b] = posterior[(size_t)b * (K + 1) + n];
    }
}

/*
 * _select_transfer (eval_sync.py:447-465) for one request with given x0 and
 * conf [Q]: among positions holding mask_id, the kk highest confidences
 * (ties: lowest index) take their x0 (selection by repeated maximum); kk as
 * in oracle_confidence_topk.  selected [Q] (may be NULL) marks them.
 */
void oracle_select_transfer(int64_t* blk, int64_t mask_id, int k, int dynamic, double threshold,
                            const int64_t* x0, const float* conf, uint8_t* selected, int Q) {
    int masked = 0, confident = 0;
    for (int i = 0; i < Q; ++i) {
        masked += blk[i] == mask_id;
        confident += blk[i] == mask_id && conf[i] >= (float)threshold;
    }
    int kk = (dynamic && confident > 0) ? (k < confident ? k : confident) : k;
    if (kk > masked) kk = masked;
    if (Q <= 0) return;
    uint8_t* taken = (uint8_t*)calloc((size_t)(unsigned)Q, 1);
    for (int r = 0; r < kk; ++r) {
        int best = -1;
        for (int i = 0; i < Q; ++i) {
            if (blk[i] != mask_id || taken[i]) continue;
            if (best < 0 || conf[i] > conf[best]) best = i;
        }
        taken[best] = 1;
    }
    for (int i = 0; i < Q; ++i) {
        if (taken[i]) blk[i] = x0[i];
        if (selected) selected[i] = taken[i];
    }
    free(taken);
}

/*
 * Confidence and top-k unmask for one denoise iteration
 * (eval_sync.py:447-465 _select_transfer), per request rather than with row
 * 0's indices applied to every row (:461-464).
 *   logits [B, Q, V] fp32, block [B, Q] in/out.  x0 = argmax of each row and
 *   conf = its softmax(logits / T) probability, with T taken as 1 when
 *   T <= 1e-5 (the greedy confidence of eval_sync.py:713-717 and of SGLang's
 *   low_confidence.py:32-35), or 1.0 with one_hot (the greedy
 *   _sample_with_prob of eval_sync.py:287-291, :323-338).  Among positions
 *   holding mask_id, the kk highest confidences (ties: lowest index) take
 *   their x0; kk = k, except with dynamic remasking (eval_sync.py:453-462):
 *   when n > 0 masked positions have conf >= threshold (compared in fp32, as
 *   torch compares a float32 tensor with a Python float), kk = min(k, n).
 *   x0 [B, Q] and conf [B, Q] are written for every row.
 */
void oracle_confidence_topk(const float* logits, int64_t* block, int64_t mask_id, int k,
                            double T, int one_hot, int dynamic, double threshold, int B, int Q, long V,
                            int64_t* x0, float* conf) {
    for (int b = 0; b < B; ++b) {
        for (int i = 0; i < Q; ++i) {
            const float* x = logits + ((size_t)b * Q + i) * V;
            long a = oracle_argmax_f32(x, V);
            x0[(size_t)b * Q + i] = a;
            double Te = T <= 1e-5 ? 1.0 : T;
            double m = (double)x[a] / Te, s = 0.0;
            for (long t = 0; t < V; ++t) s += exp((double)x[t] / Te - m);
            conf[(size_t)b * Q + i] = one_hot ? 1.0f : (float)(1.0 / s);
        }
        oracle_select_transfer(block + (size_t)b * Q, mask_id, k, dynamic, threshold, x0 + (size_t)b * Q,
                               conf + (size_t)b * Q, NULL, Q);
    }
}
