/*
 * TEST INFRASTRUCTURE -- the CPU float64 oracle of the Block AttnRes operator.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline). No
 * product path calls it.
 *
 * It restates, in plain C double precision, the algorithm of the reference:
 *   forward   src/switchyard/reference.py:98-104 (rms_norm) and :130-133
 *             (k = rms_norm(v); logits = <w, k>; alpha = softmax over n;
 *             out = sum_n alpha_n v_n), the float64 oracle of :136-146.
 *   backward  the closed form documented at src/switchyard/triton_op.py:205-214
 *             (the reference computes it in _bwd_resident, :234-264).
 *   stats     attn_with_stats, src/switchyard/reference.py:195-216.
 *   merge     merge_online_softmax, src/switchyard/reference.py:219-233.
 *   batched   block_attn_res_batched's contract, triton_op.py:438-462:
 *             entry s equals the single-query forward with queries[s].
 *
 * Layout: v [N][T][D] (T = B*T tokens), out/g [T][D], w [D], all contiguous.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Per-token softmax weights over the N sources (reference.py:130-132).
 * The key is materialised element by element, k = v * rsqrt(mean(v^2)+eps),
 * before the dot with w, as the reference's einsum over rms_norm(v) does. */
static void token_alpha(const double* v, const double* w, int64_t n, int64_t t, int64_t tok,
                        int64_t d, double eps, double* logit, double* alpha, double* rinv) {
  double m = -INFINITY;
  for (int64_t i = 0; i < n; ++i) {
    const double* x = v + (i * t + tok) * d;
    double ss = 0.0;
    for (int64_t k = 0; k < d; ++k) ss += x[k] * x[k];
    const double r = 1.0 / sqrt(ss / (double)d + eps);
    double lg = 0.0;
    for (int64_t k = 0; k < d; ++k) lg += w[k] * (x[k] * r);
    logit[i] = lg;
    if (rinv) rinv[i] = r;
    if (lg > m) m = lg;
  }
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    alpha[i] = exp(logit[i] - m);
    s += alpha[i];
  }
  for (int64_t i = 0; i < n; ++i) alpha[i] /= s;
}

/* out[t][d] = sum_n alpha_n v_n[t][d]. alpha_out [N][T] may be NULL. */
int oracle_forward(const double* v, const double* w, double* out, double* alpha_out, int64_t n,
                   int64_t t, int64_t d, double eps) {
  if (n < 1 || t < 0 || d < 1) return -1;
  double* buf = (double*)malloc(sizeof(double) * 2 * (size_t)n);
  if (!buf) return -2;
  double *logit = buf, *alpha = buf + n;
  for (int64_t tok = 0; tok < t; ++tok) {
    token_alpha(v, w, n, t, tok, d, eps, logit, alpha, NULL);
    double* o = out + tok * d;
    for (int64_t k = 0; k < d; ++k) o[k] = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      const double* x = v + (i * t + tok) * d;
      for (int64_t k = 0; k < d; ++k) o[k] += alpha[i] * x[k];
      if (alpha_out) alpha_out[i * t + tok] = alpha[i];
    }
  }
  free(buf);
  return 0;
}

/* Gradients of out with respect to v and w for upstream gradient g, by the
 * closed form (triton_op.py:205-214): with r_n = rsqrt(ssq_n/D + eps),
 * a_n = <w, v_n>, G_n = <g, v_n>, S = sum_n alpha_n G_n,
 *   dlogit_n = alpha_n (G_n - S), da_n = dlogit_n r_n,
 *   dssq_n = -dlogit_n a_n r_n^3 / (2D),
 *   dv_n = alpha_n g + da_n w + 2 dssq_n v_n,  dw = sum_tokens sum_n da_n v_n.
 * G_n - S is evaluated as (G_n - G_m) - sum_k alpha_k (G_k - G_m), m the
 * row with the largest logit: the same number (alpha sums to one), but with
 * no cancellation when the softmax saturates (alpha_m -> 1, G_m - S -> 0).
 * dv [N][T][D], dw [D] (overwritten). */
int oracle_backward(const double* v, const double* w, const double* g, double* dv, double* dw,
                    int64_t n, int64_t t, int64_t d, double eps) {
  if (n < 1 || t < 0 || d < 1) return -1;
  double* buf = (double*)malloc(sizeof(double) * 4 * (size_t)n);
  if (!buf) return -2;
  double *logit = buf, *alpha = buf + n, *rinv = buf + 2 * n, *gdot = buf + 3 * n;
  for (int64_t k = 0; k < d; ++k) dw[k] = 0.0;
  for (int64_t tok = 0; tok < t; ++tok) {
    token_alpha(v, w, n, t, tok, d, eps, logit, alpha, rinv);
    const double* gt = g + tok * d;
    int64_t top = 0;
    for (int64_t i = 0; i < n; ++i) {
      const double* x = v + (i * t + tok) * d;
      double gg = 0.0;
      for (int64_t k = 0; k < d; ++k) gg += gt[k] * x[k];
      gdot[i] = gg;
      if (logit[i] > logit[top]) top = i;
    }
    const double gref = gdot[top];
    double s = 0.0; /* S - G_top */
    for (int64_t i = 0; i < n; ++i) s += alpha[i] * (gdot[i] - gref);
    for (int64_t i = 0; i < n; ++i) {
      const double* x = v + (i * t + tok) * d;
      double* dx = dv + (i * t + tok) * d;
      const double r = rinv[i];
      const double a = logit[i] / r; /* <w, v_i> */
      const double dlogit = alpha[i] * ((gdot[i] - gref) - s);
      const double da = dlogit * r;
      const double dssq = -dlogit * a * r * r * r / (2.0 * (double)d);
      for (int64_t k = 0; k < d; ++k) {
        dx[k] = alpha[i] * gt[k] + da * w[k] + 2.0 * dssq * x[k];
        dw[k] += da * x[k];
      }
    }
  }
  free(buf);
  return 0;
}

/* attn_with_stats (reference.py:195-216): o = sum_n exp(logit_n - m) v_n,
 * m = max logit, ell = sum_n exp(logit_n - m). o [T][D], m/ell [T]. */
int oracle_attn_with_stats(const double* v, const double* w, double* o, double* m, double* ell,
                           int64_t n, int64_t t, int64_t d, double eps) {
  if (n < 1 || t < 0 || d < 1) return -1;
  double* logit = (double*)malloc(sizeof(double) * (size_t)n);
  if (!logit) return -2;
  for (int64_t tok = 0; tok < t; ++tok) {
    double mx = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
      const double* x = v + (i * t + tok) * d;
      double ss = 0.0;
      for (int64_t k = 0; k < d; ++k) ss += x[k] * x[k];
      const double r = 1.0 / sqrt(ss / (double)d + eps);
      double lg = 0.0;
      for (int64_t k = 0; k < d; ++k) lg += w[k] * (x[k] * r);
      logit[i] = lg;
      if (lg > mx) mx = lg;
    }
    double* ot = o + tok * d;
    for (int64_t k = 0; k < d; ++k) ot[k] = 0.0;
    double l = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      const double p = exp(logit[i] - mx);
      const double* x = v + (i * t + tok) * d;
      for (int64_t k = 0; k < d; ++k) ot[k] += p * x[k];
      l += p;
    }
    m[tok] = mx;
    ell[tok] = l;
  }
  free(logit);
  return 0;
}

/* merge_online_softmax (reference.py:219-233): the (o, m, ell) of the union of
 * two disjoint source groups. Outputs may alias neither input. */
void oracle_merge(const double* o1, const double* m1, const double* l1, const double* o2,
                  const double* m2, const double* l2, double* o, double* m, double* l, int64_t t,
                  int64_t d) {
  for (int64_t tok = 0; tok < t; ++tok) {
    const double mm = m1[tok] > m2[tok] ? m1[tok] : m2[tok];
    const double s1 = exp(m1[tok] - mm), s2 = exp(m2[tok] - mm);
    for (int64_t k = 0; k < d; ++k) o[tok * d + k] = o1[tok * d + k] * s1 + o2[tok * d + k] * s2;
    m[tok] = mm;
    l[tok] = l1[tok] * s1 + l2[tok] * s2;
  }
}

/* out[s] = forward(v, q[s]) for s < S (triton_op.py:438-462). out [S][T][D]. */
int oracle_batched(const double* v, const double* q, double* out, int64_t n, int64_t s, int64_t t,
                   int64_t d, double eps) {
  for (int64_t i = 0; i < s; ++i) {
    const int rc = oracle_forward(v, q + i * d, out + i * t * d, NULL, n, t, d, eps);
    if (rc) return rc;
  }
  return 0;
}

/* Gradient of attn_with_stats for upstream (go [T][D], gm [T], gl [T]).
 * Derivation (no reference counterpart; written from reference.py:195-216):
 * with k the first row holding the max logit m, p_i = exp(logit_i - m) and
 * G_i = <go, v_i>, the loss depends on logit_i through p_i (o and ell) and,
 * for i = k, through m itself:
 *   dlogit_i = p_i (G_i + gl)                           i != k
 *   dlogit_k = gm - sum_{i != k} p_i (G_i + gl)         (p_k = 1)
 * and the chain through logit_i = r_i <w, v_i> is the one of oracle_backward,
 * with p_i in place of alpha_i in the direct term p_i * go. */
int oracle_attn_with_stats_backward(const double* v, const double* w, const double* go,
                                    const double* gm, const double* gl, double* dv, double* dw,
                                    int64_t n, int64_t t, int64_t d, double eps) {
  if (n < 1 || t < 0 || d < 1) return -1;
  double* buf = (double*)malloc(sizeof(double) * 4 * (size_t)n);
  if (!buf) return -2;
  double *logit = buf, *p = buf + n, *rinv = buf + 2 * n, *dlg = buf + 3 * n;
  for (int64_t k = 0; k < d; ++k) dw[k] = 0.0;
  for (int64_t tok = 0; tok < t; ++tok) {
    token_alpha(v, w, n, t, tok, d, eps, logit, p, rinv);
    int64_t top = 0;
    for (int64_t i = 1; i < n; ++i)
      if (logit[i] > logit[top]) top = i;
    const double* gt = go + tok * d;
    double other = 0.0;
    for (int64_t i = 0; i < n; ++i) {
      const double* x = v + (i * t + tok) * d;
      double gg = 0.0;
      for (int64_t k = 0; k < d; ++k) gg += gt[k] * x[k];
      p[i] = exp(logit[i] - logit[top]);
      dlg[i] = p[i] * (gg + gl[tok]);
      if (i != top) other += dlg[i];
    }
    dlg[top] = gm[tok] - other;
    for (int64_t i = 0; i < n; ++i) {
      const double* x = v + (i * t + tok) * d;
      double* dx = dv + (i * t + tok) * d;
      const double r = rinv[i];
      const double a = logit[i] / r;
      const double da = dlg[i] * r;
      const double dssq = -dlg[i] * a * r * r * r / (2.0 * (double)d);
      for (int64_t k = 0; k < d; ++k) {
        dx[k] = p[i] * gt[k] + da * w[k] + 2.0 * dssq * x[k];
        dw[k] += da * x[k];
      }
    }
  }
  free(buf);
  return 0;
}

/* Gradient of oracle_merge for upstream (go [T][D], gm [T], gl [T]). With
 * s_i = exp(m_i - m) and k the group holding the max (group 1 on a tie):
 *   do_i = s_i go, dl_i = s_i gl, ds_i = <go, o_i> + gl l_i,
 *   dm_j = s_j ds_j for the other group j, dm_k = gm - s_j ds_j. */
void oracle_merge_backward(const double* o1, const double* m1, const double* l1, const double* o2,
                           const double* m2, const double* l2, const double* go, const double* gm,
                           const double* gl, double* do1, double* dm1, double* dl1, double* do2,
                           double* dm2, double* dl2, int64_t t, int64_t d) {
  for (int64_t tok = 0; tok < t; ++tok) {
    const int first = m1[tok] >= m2[tok];
    const double mm = first ? m1[tok] : m2[tok];
    const double s1 = exp(m1[tok] - mm), s2 = exp(m2[tok] - mm);
    double d1 = 0.0, d2 = 0.0;
    for (int64_t k = 0; k < d; ++k) {
      const double g = go[tok * d + k];
      d1 += g * o1[tok * d + k];
      d2 += g * o2[tok * d + k];
      do1[tok * d + k] = s1 * g;
      do2[tok * d + k] = s2 * g;
    }
    const double ds1 = d1 + gl[tok] * l1[tok], ds2 = d2 + gl[tok] * l2[tok];
    dl1[tok] = s1 * gl[tok];
    dl2[tok] = s2 * gl[tok];
    if (first) {
      dm2[tok] = s2 * ds2;
      dm1[tok] = gm[tok] - s2 * ds2;
    } else {
      dm1[tok] = s1 * ds1;
      dm2[tok] = gm[tok] - s1 * ds1;
    }
  }
}

/* Gradient of oracle_batched for upstream g [S][T][D]: the S queries are S
 * independent operators sharing v, so dv = sum_s dv_s and dq[s] = dw_s of
 * oracle_backward(v, q[s], g[s]). dv [N][T][D], dq [S][D]. */
int oracle_batched_backward(const double* v, const double* q, const double* g, double* dv,
                            double* dq, int64_t n, int64_t s, int64_t t, int64_t d, double eps) {
  if (n < 1 || s < 1 || t < 0 || d < 1) return -1;
  const size_t vol = (size_t)n * (size_t)t * (size_t)d;
  double* tmp = (double*)malloc(sizeof(double) * (vol > 0 ? vol : 1));
  if (!tmp) return -2;
  for (size_t k = 0; k < vol; ++k) dv[k] = 0.0;
  for (int64_t i = 0; i < s; ++i) {
    const int rc = oracle_backward(v, q + i * d, g + i * t * d, tmp, dq + i * d, n, t, d, eps);
    if (rc) {
      free(tmp);
      return rc;
    }
    for (size_t k = 0; k < vol; ++k) dv[k] += tmp[k];
  }
  free(tmp);
  return 0;
}
