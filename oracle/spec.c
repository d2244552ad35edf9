/*
 * ORACLE ONLY (test infrastructure): CPU restatement of speculative acceptance
 * sampling, emulating the fp32 reduction order of the GPU kernel exactly, so
 * accept counts and tokens can be compared bit for bit given identical logits
 * and uniforms. Must be built with -ffp-contract=off.
 *
 * Rule (Leviathan et al. 2023; Chen et al. 2023), generalising the reference's
 * greedy-draft case (engine/speculative.py:74-81, where q is one-hot):
 *   z = logits * inv_temp, p = softmax(z_target), q = softmax(z_draft)
 *   for i < k: accept draft d_i iff u_i * q_i(d_i) < p_i(d_i)
 *   first rejection at n: token ~ max(0, p_n - q_n); all accepted: token ~ p_k.
 * Written without division: with e = exp(z - max), S = sum e,
 *   accept iff u * e_q(d) * S_p < e_p(d) * S_q,
 *   residual weight w_j = max(0, e_p(j) * S_q - e_q(j) * S_p),
 *   bonus weight w_j = e_p(j).
 * One-hot q (no draft logits): e_q = [j == d], S_q = 1. A draft id outside
 * [0, V) is rejected. NaN logits are not supported.
 * Greedy (reference sampler.greedy, engine/speculative.py:75-77): accept iff
 * argmax(target_i) == d_i (first maximal index), token = argmax of row n.
 *
 * Filtering of the target rows (Sampler.scores, engine/sampler.py:30-52):
 *   presence penalty: x' = x - penalty * s(j), s(j) = 1 for the tokens of
 *     `seen` and, in verify row i, for the drafts d_0..d_{i-1} that precede it
 *     (the reference's extra_seen=draft for its bonus row), else seen[j];
 *   greedy scores are x' (argmax as above); otherwise z = x' * inv_temp;
 *   top-k (1 <= top_k <= 64): c_0 >= ... >= c_{K-1}, the K largest z (with
 *     multiplicity); cutoff = c_{K-1};
 *   top-p (0 < top_p < 1, needs top_k): e_i = exp(c_i - c_0), S = sum e_i in
 *     order, p_i = e_i / S, running inclusive sums r_i, keep i iff
 *     (r_i - p_i) < top_p (mx.cumsum(probs) - probs < top_p); cutoff = min kept c_i;
 *   kept set: z >= cutoff; p(j) = exp(z_j - c_0) / S_p on the kept set with
 *     S_p = sum_{i: c_i > cutoff} exp(c_i - c_0) + n_eq * exp(cutoff - c_0),
 *     n_eq = number of tokens of the row with z == cutoff.
 * Wide form (64 < top_k < V, or top-p with no top-k; top_k >= V means no
 * top-k, engine/sampler.py:44-47): masses m(z) = trunc(exp(z - c_0) * 2^32)
 * as uint64 (exact, order-free sums); v_k = the top_k-th largest z (with
 * multiplicity); S_cand = sum of m over the top_k candidates (z > v_k, plus
 * top_k - #(z > v_k) copies of m(v_k)), or over the whole row; cutoff = the
 * smallest row value v >= v_k with M(> v) < top_p * S_cand in double, where
 * M(> v) = sum of m over z > v (engine/sampler.py:47-50 with exact sums; v_k
 * itself without top-p); S_p = sum of exp(z - c_0) over z >= cutoff in fp32,
 * logical thread t of 1024 owning elements 4 (t + 1024 i) + e in (i, e) order,
 * xor butterflies per 64-thread wave, then the 16 wave sums in order. The
 * integer parts are computed here by sorting, not by the kernel's radix descent.
 * Draft rows (draft logits) are never filtered.
 *
 * Reduction order (shared with the kernel): a row is cut into parts of 8192;
 * in a part, logical thread t (0..255) owns elements
 *   base + 4*(t + 256*i) + e,  i = 0..7, e = 0..3  (in that order),
 * summed sequentially; thread sums combine with an xor butterfly over each
 * 64-lane wave (32,16,8,4,2,1) and then ((w0 + w1) + w2) + w3.
 * Parts combine as m = max m_p, S = sum_p S_p * exp(m_p - m) left to right.
 * Inverse-CDF sampling walks the same order: parts, then threads, then elements,
 * with running fp32 prefix sums; when rounding leaves the walk without a hit, the
 * last positive weight of the scope is taken.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define PART 8192
#define NT 256
#define NI 8

/* exp(x): Cody-Waite reduction x = n*ln2 + r (ln2 split hi/lo), Taylor series of
 * degree 7 for e^r in Horner form with fmaf, scaled by 2^n; 0 below -69 (keeps
 * every product formed with it in the normal range). */
float orc_expf(float x) {
  if (!(x >= -69.0f)) return 0.0f;
  if (x > 88.0f) return INFINITY;
  const float n = rintf(x * 1.44269504f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.428606765330187e-06f, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int e = (int)n;
  uint32_t bits = (uint32_t)(e + 127) << 23;
  float scale;
  memcpy(&scale, &bits, 4);
  return p * scale;
}

static int nparts(int V) { return (V + PART - 1) / PART; }

/* element j of logical thread t, slot s = 4*i + e, in part p; -1 if past V */
static inline int elem(int V, int p, int t, int s) {
  const int i = s >> 2, e = s & 3;
  const int j = p * PART + 4 * (t + NT * i) + e;
  const int end = (p + 1) * PART < V ? (p + 1) * PART : V;
  return j < end ? j : -1;
}

/* first element of logical thread t in part p is past the end: the thread owns nothing */
static inline int thread_empty(int V, int p, int t) { return elem(V, p, t, 0) < 0; }

static float block_sum(const float* tsum) {
  float w[4];
  for (int wv = 0; wv < 4; ++wv) {
    float v[64], nv[64];
    for (int l = 0; l < 64; ++l) v[l] = tsum[wv * 64 + l];
    for (int o = 32; o >= 1; o >>= 1) {
      for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ o];
      memcpy(v, nv, sizeof(v));
    }
    w[wv] = v[0];
  }
  return ((w[0] + w[1]) + w[2]) + w[3];
}

typedef struct { float m, s, cutoff; } rowstat;

/* sampling-side filter of a target row: penalty inputs and the tokens that
 * count as seen in this row in addition to `seen` */
typedef struct {
  const float* seen; /* [V] or NULL */
  float pen;
  const int32_t* extra; /* drafts d_0 .. d_{n_extra-1} */
  int n_extra;
} pfilt;

/* penalised logit x - pen * s(j) (no subtraction at all without a penalty) */
static inline float pen_logit(const float* row, int j, const pfilt* f) {
  const float x = row[j];
  if (!f || (!f->seen && f->n_extra == 0) || f->pen == 0.0f) return x;
  float sj = f->seen ? f->seen[j] : 0.0f;
  for (int q = 0; q < f->n_extra; ++q)
    if (f->extra[q] == j) sj = 1.0f;
  return x - f->pen * sj;
}

static int cmp_desc(const void* a, const void* b) {
  const float x = *(const float*)a, y = *(const float*)b;
  return (x < y) - (x > y);
}

/* filtered statistics of a target row (top_k >= 1): m = c_0, s = S_p, cutoff */
static rowstat filtered_stats(const float* row, int V, float inv_temp, const pfilt* f, int top_k, float top_p) {
  float* z = (float*)malloc(sizeof(float) * (size_t)V);
  for (int j = 0; j < V; ++j) z[j] = pen_logit(row, j, f) * inv_temp;
  float* srt = (float*)malloc(sizeof(float) * (size_t)V);
  memcpy(srt, z, sizeof(float) * (size_t)V);
  qsort(srt, (size_t)V, sizeof(float), cmp_desc);
  const int K = top_k;
  const float c0 = srt[0];
  float cutoff = srt[K - 1];
  if (top_p > 0.0f && top_p < 1.0f) {
    float e[64], S = 0.0f;
    for (int i = 0; i < K; ++i) {
      e[i] = orc_expf(srt[i] - c0);
      S = S + e[i];
    }
    float run = 0.0f, mn = INFINITY;
    for (int i = 0; i < K; ++i) {
      const float pi = e[i] / S;
      const float incl = run + pi;
      if ((incl - pi) < top_p && srt[i] < mn) mn = srt[i];
      run = incl;
    }
    cutoff = mn;
  }
  int n_gt = 0;
  while (n_gt < K && srt[n_gt] > cutoff) ++n_gt;
  int n_eq = 0;
  for (int j = 0; j < V; ++j) n_eq += (z[j] == cutoff);
  float S = 0.0f;
  for (int i = 0; i < n_gt; ++i) S = S + orc_expf(srt[i] - c0);
  S = S + (float)n_eq * orc_expf(cutoff - c0);
  free(z);
  free(srt);
  rowstat r;
  r.m = c0;
  r.s = S;
  r.cutoff = cutoff;
  return r;
}

static inline uint64_t fx_mass(float z, float c0) { return (uint64_t)(orc_expf(z - c0) * 4294967296.0f); }

#define WT 1024

/* wide-form statistics of a target row (see the header): m = c_0, s = S_p, cutoff */
static rowstat wide_stats(const float* row, int V, float inv_temp, const pfilt* f, int K, float top_p) {
  float* z = (float*)malloc(sizeof(float) * (size_t)V);
  for (int j = 0; j < V; ++j) z[j] = pen_logit(row, j, f) * inv_temp;
  float* srt = (float*)malloc(sizeof(float) * (size_t)V);
  memcpy(srt, z, sizeof(float) * (size_t)V);
  qsort(srt, (size_t)V, sizeof(float), cmp_desc);
  const float c0 = srt[0];
  const float vk = K > 0 ? srt[K - 1] : -INFINITY;
  float cutoff = vk;
  if (top_p > 0.0f && top_p < 1.0f) {
    uint64_t S = 0;
    if (K > 0) {
      int n_gt = 0;
      while (srt[n_gt] > vk) S += fx_mass(srt[n_gt++], c0);
      S += (uint64_t)(K - n_gt) * fx_mass(vk, c0);
    } else {
      for (int j = 0; j < V; ++j) S += fx_mass(srt[j], c0);
    }
    const double T = (double)top_p * (double)S;
    /* walk the distinct values downwards; M = mass of the values above */
    uint64_t M = 0;
    int i = 0;
    cutoff = srt[0];
    while (i < V && srt[i] >= vk) {
      const float v = srt[i];
      if (!((double)M < T)) break;
      cutoff = v;
      while (i < V && srt[i] == v) M += fx_mass(srt[i++], c0);
    }
  }
  /* S_p in the kernel's order */
  float tsum[WT];
  for (int t = 0; t < WT; ++t) {
    float acc = 0.0f;
    for (int j = 4 * t; j < V; j += 4 * WT)
      for (int e = 0; e < 4; ++e) acc = acc + (z[j + e] >= cutoff ? orc_expf(z[j + e] - c0) : 0.0f);
    tsum[t] = acc;
  }
  float S = 0.0f;
  for (int w = 0; w < WT / 64; ++w) {
    float v[64], nv[64];
    for (int l = 0; l < 64; ++l) v[l] = tsum[w * 64 + l];
    for (int o = 32; o >= 1; o >>= 1) {
      for (int l = 0; l < 64; ++l) nv[l] = v[l] + v[l ^ o];
      memcpy(v, nv, sizeof(v));
    }
    S = w == 0 ? v[0] : S + v[0];
  }
  free(z);
  free(srt);
  rowstat r;
  r.m = c0;
  r.s = S;
  r.cutoff = cutoff;
  return r;
}

static rowstat row_stats(const float* row, int V, float inv_temp, const pfilt* f) {
  const int P = nparts(V);
  float mp[4096], sp[4096];
  for (int p = 0; p < P; ++p) {
    float m = -INFINITY;
    const int b0 = p * PART, e0 = (p + 1) * PART < V ? (p + 1) * PART : V;
    for (int j = b0; j < e0; ++j) {
      const float z = pen_logit(row, j, f) * inv_temp;
      if (z > m) m = z;
    }
    float ts[NT];
    for (int t = 0; t < NT; ++t) {
      float acc = 0.0f;
      if (!thread_empty(V, p, t))
        for (int s = 0; s < 4 * NI; ++s) {
          const int j = elem(V, p, t, s);
          if (j < 0) break;
          acc = acc + orc_expf(pen_logit(row, j, f) * inv_temp - m);
        }
      ts[t] = acc;
    }
    mp[p] = m;
    sp[p] = block_sum(ts);
  }
  rowstat r;
  float m = -INFINITY;
  for (int p = 0; p < P; ++p)
    if (mp[p] > m) m = mp[p];
  float s = 0.0f;
  for (int p = 0; p < P; ++p) s = s + sp[p] * orc_expf(mp[p] - m);
  r.m = m;
  r.s = s;
  r.cutoff = -INFINITY;
  return r;
}

/* first index of the maximum of the (penalised) row (greedy) */
static int row_argmax(const float* row, int V, const pfilt* f) {
  int bj = 0;
  float bv = pen_logit(row, 0, f);
  for (int j = 1; j < V; ++j) {
    const float v = pen_logit(row, j, f);
    if (v > bv) {
      bv = v;
      bj = j;
    }
  }
  return bj;
}

/* sampling weight of element j */
typedef struct {
  const float* tp; /* target row */
  const float* tq; /* draft row or NULL */
  int d;           /* draft id (one-hot q when tq == NULL) */
  int mode;        /* 0 = residual, 1 = plain p */
  float inv_temp;
  rowstat sp, sq;
  const pfilt* f;  /* penalty of the target row */
} wctx;

static inline float weight(const wctx* c, int j) {
  const float z = pen_logit(c->tp, j, c->f) * c->inv_temp;
  const float ep = z >= c->sp.cutoff ? orc_expf(z - c->sp.m) : 0.0f;
  if (c->mode == 1) return ep;
  float eq, Sq;
  if (c->tq) {
    eq = orc_expf(c->tq[j] * c->inv_temp - c->sq.m);
    Sq = c->sq.s;
  } else {
    eq = (j == c->d) ? 1.0f : 0.0f;
    Sq = 1.0f;
  }
  const float r = ep * Sq - eq * c->sp.s;
  return r > 0.0f ? r : 0.0f;
}

static int sample(const wctx* c, int V, float u) {
  const int P = nparts(V);
  float* T = (float*)malloc(sizeof(float) * (size_t)P * NT);
  float* Wp = (float*)malloc(sizeof(float) * (size_t)P);
  for (int p = 0; p < P; ++p) {
    for (int t = 0; t < NT; ++t) {
      float acc = 0.0f;
      if (!thread_empty(V, p, t))
        for (int s = 0; s < 4 * NI; ++s) {
          const int j = elem(V, p, t, s);
          if (j < 0) break;
          acc = acc + weight(c, j);
        }
      T[(size_t)p * NT + t] = acc;
    }
    Wp[p] = block_sum(T + (size_t)p * NT);
  }
  float W = 0.0f;
  for (int p = 0; p < P; ++p) W = W + Wp[p];
  int result = -1;
  if (W > 0.0f) {
    const float th = u * W;
    float cacc = 0.0f;
    int ps = -1;
    for (int p = 0; p < P; ++p) {
      const float nx = cacc + Wp[p];
      if (nx > th) { ps = p; break; }
      cacc = nx;
    }
    int fallback = 0;
    if (ps < 0) {
      for (int p = P - 1; p >= 0; --p)
        if (Wp[p] > 0.0f) { ps = p; break; }
      fallback = 1;
    }
    int ts = -1;
    if (!fallback) {
      for (int t = 0; t < NT; ++t) {
        const float nx = cacc + T[(size_t)ps * NT + t];
        if (nx > th) { ts = t; break; }
        cacc = nx;
      }
    }
    if (ts < 0) {
      for (int t = NT - 1; t >= 0; --t)
        if (T[(size_t)ps * NT + t] > 0.0f) { ts = t; break; }
      fallback = 1;
    }
    if (!fallback) {
      for (int s = 0; s < 4 * NI; ++s) {
        const int j = elem(V, ps, ts, s);
        if (j < 0) break;
        cacc = cacc + weight(c, j);
        if (cacc > th) { result = j; break; }
      }
    }
    if (result < 0) {
      for (int s = 4 * NI - 1; s >= 0; --s) {
        const int j = elem(V, ps, ts, s);
        if (j >= 0 && weight(c, j) > 0.0f) { result = j; break; }
      }
    }
  }
  free(T);
  free(Wp);
  return result;
}

void orc_spec_accept_filtered(const float* target, const float* draft, const int32_t* draft_ids,
                              const float* u_accept, const float* u_sample, float inv_temp, const float* seen,
                              float presence_penalty, int top_k, float top_p, int32_t* n_accept,
                              int32_t* out_token, int S, int k, int V, int threads) {
  const int greedy = !(inv_temp > 0.0f);
#pragma omp parallel for schedule(dynamic) num_threads(threads > 0 ? threads : 1)
  for (int st = 0; st < S; ++st) {
    const float* tgt = target + (size_t)st * (k + 1) * V;
    const float* drf = draft ? draft + (size_t)st * k * V : NULL;
    const int32_t* d = draft_ids + (size_t)st * k;
    pfilt pf[65];
    for (int i = 0; i <= k; ++i) {
      pf[i].seen = seen;
      pf[i].pen = presence_penalty;
      pf[i].extra = d;
      pf[i].n_extra = i;
    }
    int n = k, tok = -1;
    if (greedy) {
      for (int i = 0; i < k; ++i) {
        const int am = row_argmax(tgt + (size_t)i * V, V, &pf[i]);
        if (am != d[i]) { n = i; tok = am; break; }
      }
      if (n == k) tok = row_argmax(tgt + (size_t)k * V, V, &pf[k]);
    } else {
      rowstat rp[65], rq[64];
      const int tk = (top_k > 0 && top_k < V) ? top_k : 0;
      const int use_p = top_p > 0.0f && top_p < 1.0f;
      for (int i = 0; i <= k; ++i) {
        const float* ri = tgt + (size_t)i * V;
        if (tk >= 1 && tk <= 64) rp[i] = filtered_stats(ri, V, inv_temp, &pf[i], tk, top_p);
        else if (tk > 64 || use_p) rp[i] = wide_stats(ri, V, inv_temp, &pf[i], tk, top_p);
        else rp[i] = row_stats(ri, V, inv_temp, &pf[i]);
      }
      if (drf)
        for (int i = 0; i < k; ++i) rq[i] = row_stats(drf + (size_t)i * V, V, inv_temp, NULL);
      for (int i = 0; i < k; ++i) {
        const int di = d[i];
        if (di < 0 || di >= V) { n = i; break; } /* an out-of-range draft is rejected */
        const float zd = pen_logit(tgt + (size_t)i * V, di, &pf[i]) * inv_temp;
        const float ep = zd >= rp[i].cutoff ? orc_expf(zd - rp[i].m) : 0.0f;
        float eq = 1.0f, Sq = 1.0f;
        if (drf) {
          eq = orc_expf(drf[(size_t)i * V + di] * inv_temp - rq[i].m);
          Sq = rq[i].s;
        }
        const float lhs = u_accept[(size_t)st * k + i] * eq * rp[i].s;
        const float rhs = ep * Sq;
        if (!(lhs < rhs)) { n = i; break; }
      }
      wctx c;
      c.inv_temp = inv_temp;
      c.sp = rp[n];
      c.f = &pf[n];
      if (n < k) {
        c.tp = tgt + (size_t)n * V;
        c.tq = drf ? drf + (size_t)n * V : NULL;
        c.d = d[n];
        c.mode = 0;
        if (drf) c.sq = rq[n];
        tok = sample(&c, V, u_sample[st]);
        if (tok < 0) { /* residual vanished in fp32: fall back to p_n */
          c.mode = 1;
          tok = sample(&c, V, u_sample[st]);
        }
      } else {
        c.tp = tgt + (size_t)k * V;
        c.tq = NULL;
        c.d = -1;
        c.mode = 1;
        tok = sample(&c, V, u_sample[st]);
      }
    }
    n_accept[st] = n;
    out_token[st] = tok;
  }
}

/* the filter record (c_0, S_p, cutoff) of one target row, as the accept and
 * scores kernels use it (row_stats for an unfiltered sampling row) */
void orc_row_filter(const float* row, int V, float inv_temp, const float* seen, float presence_penalty, int top_k,
                    float top_p, float out[3]) {
  pfilt pf = {seen, presence_penalty, NULL, 0};
  const int tk = (top_k > 0 && top_k < V) ? top_k : 0;
  const int use_p = top_p > 0.0f && top_p < 1.0f;
  rowstat r;
  if (tk >= 1 && tk <= 64) r = filtered_stats(row, V, inv_temp, &pf, tk, top_p);
  else if (tk > 64 || use_p) r = wide_stats(row, V, inv_temp, &pf, tk, top_p);
  else r = row_stats(row, V, inv_temp, &pf);
  out[0] = r.m;
  out[1] = r.s;
  out[2] = r.cutoff;
}

void orc_spec_accept(const float* target, const float* draft, const int32_t* draft_ids,
                     const float* u_accept, const float* u_sample, float inv_temp,
                     int32_t* n_accept, int32_t* out_token, int S, int k, int V, int threads) {
  orc_spec_accept_filtered(target, draft, draft_ids, u_accept, u_sample, inv_temp, NULL, 0.0f, 0, 1.0f, n_accept,
                           out_token, S, k, V, threads);
}
