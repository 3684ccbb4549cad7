/*
 * ORACLE — TEST INFRASTRUCTURE ONLY.  Never linked into or called by the product
 * (batchspec_amd); only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
 * leg load it, as the checker.
 *
 * Plain-C restatement of the top-k / top-p renormalisation of
 * batchspec/backends/utils/sampling.py:18-58 (get_sampling_probs: softmax(logits/T),
 * then top-p renorm if top_p > 0 (:51-52), then top-k renorm if top_k > 0 (:55-56)),
 * of the non-greedy sample() of :61-115 with explicit uniforms, and of the sampling
 * branch of MTPEngine.evaluate_posterior (batchspec/backends/mtp_engine.py:561-575)
 * fed those filtered distributions.  Compiled into liboracle.so with accept.c,
 * whose canonical row statistics and exp2 it uses.
 *
 * Definition of the filtered distribution of a row x[0..V) at temperature T
 * (deterministic, as documented by the GPU kernels):
 *   (M, Z)  canonical row statistics (accept.c), C = log2(e) * (1/T);
 *   w(x)    = exp2(fma(x, C, -(M*C)));  m(x) = trunc(w(x) * 2^40)  (64-bit integer);
 *   key(x)  = order-preserving 32-bit image of x (-0 counts as +0);
 *   top-k is on iff 0 < top_k < V;  top-p is on iff 0 < top_p < 1;
 *   target  = ceil(fl(top_p * Z) * 2^40);
 *   walking the distinct keys from the largest down, with cnt / mass = number /
 *   sum of m of the elements whose key is >= the current one, the threshold t* is
 *   the first key where (top-k on and cnt >= top_k) or (top-p on and mass >= target);
 *   if there is none, t* is the smallest key (everything kept).
 *   Z_K = float(mass at t*, rounded to nearest even) * 2^-40;
 *   p'(x) = key(x) >= t* ? w(x) * (1/Z_K) : 0.
 * This is the reference's order: the nucleus is taken on the full distribution and
 * top-k on the renormalised one; both keep an upper set of values, so the result
 * keeps the smaller of the two sets.  Ties at the threshold are all kept.
 *
 * Draw from non-negative weights r (floats): r_fx(v) = trunc(r(v) * 2^40),
 * total = sum r_fx; t = floor(u * total) in binary64 (t = 0 for u <= 0 or NaN);
 * the result is the first index v (ascending) whose running sum exceeds t, or the
 * last index with r_fx > 0 if none does; -1 when total == 0.
 *
 * Chain: accept x_i iff u_i * q'_i(x_i) < p'_i(x_i) (q' one-hot, or the draft
 * logits filtered the same way); at the first rejection j draw from
 * max(0, p'_j - q'_j) (or from p'_j if that has no mass); if all k pass draw the
 * bonus from p'_k; the draws use u_k.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

void oc_row_stats(const float* x, int64_t V, float c, float* M, float* Z);
float oc_exp2(float y);
void oc_softmax(const float* logits, int64_t rows, int64_t V, float T, float* probs);
void oc_chain_logits(const float* draft_logits, const int64_t* draft_ids,
                     const float* target_logits, float T, const float* uniforms, int B, int k,
                     int64_t V, int32_t* out_ids, int32_t* accepted, int32_t* emitted);

static const float LOG2E_F = 0x1.715476p+0f;

uint32_t oc_okey(float x) {
  uint32_t b;
  memcpy(&b, &x, 4);
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static float key_value(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  float x;
  memcpy(&x, &b, 4);
  return x;
}

static uint64_t fx40(float w) { return w > 0.0f ? (uint64_t)(w * 0x1p40f) : 0u; }

/* Round-to-nearest-even conversion of a 64-bit integer to binary32. */
float oc_u64_to_f32(uint64_t v) {
  if (v < (1ull << 24)) return (float)(uint32_t)v;
  int n = 64 - __builtin_clzll(v); /* bit length, > 24 */
  int sh = n - 24;
  uint64_t mant = v >> sh;
  uint64_t rem = v & ((1ull << sh) - 1);
  uint64_t half = 1ull << (sh - 1);
  if (rem > half || (rem == half && (mant & 1))) ++mant;
  return ldexpf((float)mant, sh); /* mant <= 2^24: exact */
}

static float weight(float x, float c, float neg_mc) { return oc_exp2(fmaf(x, c, neg_mc)); }

typedef struct {
  float m;      /* row max M */
  float inv_k;  /* 1 / Z_K */
  uint32_t t;   /* threshold key t* */
  int filtered; /* 0: no filter on (p' = w / Z) */
} row_filter;

static int cmp_key_desc(const void* a, const void* b) {
  uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

static row_filter filter_row(const float* x, int64_t V, float c, int top_k, float top_p,
                             uint64_t* zk_out) {
  row_filter f;
  float M, Z;
  oc_row_stats(x, V, c, &M, &Z);
  f.m = M;
  const int use_k = top_k > 0 && (int64_t)top_k < V;
  const int use_p = top_p > 0.0f && top_p < 1.0f;
  f.filtered = use_k || use_p;
  if (!f.filtered) {
    f.inv_k = 1.0f / Z;
    f.t = 0u;
    if (zk_out) *zk_out = 0;
    return f;
  }
  const float neg = -(M * c);
  const uint64_t target = use_p ? (uint64_t)ceilf((top_p * Z) * 0x1p40f) : 0u;
  uint32_t* keys = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)V);
  for (int64_t v = 0; v < V; ++v) keys[v] = oc_okey(x[v]);
  qsort(keys, (size_t)V, sizeof(uint32_t), cmp_key_desc);
  uint64_t cnt = 0, mass = 0;
  uint32_t t = keys[V - 1];
  uint64_t zk = 0;
  int found = 0;
  for (int64_t i = 0; i < V;) {
    int64_t j = i;
    while (j < V && keys[j] == keys[i]) ++j;
    const uint64_t n = (uint64_t)(j - i);
    cnt += n;
    mass += fx40(weight(key_value(keys[i]), c, neg)) * n;
    if ((use_k && cnt >= (uint64_t)top_k) || (use_p && mass >= target)) {
      t = keys[i];
      zk = mass;
      found = 1;
      break;
    }
    i = j;
  }
  if (!found) zk = mass;
  free(keys);
  f.t = t;
  f.inv_k = 1.0f / (oc_u64_to_f32(zk) * 0x1p-40f);
  if (zk_out) *zk_out = zk;
  return f;
}

static float filtered_p(const row_filter* f, float x, float c) {
  if (oc_okey(x) < f->t) return 0.0f;
  return weight(x, c, -(f->m * c)) * f->inv_k;
}

/* Exported for tests: threshold key, Z_K numerator and row max of one row. */
void oc_filter_row(const float* x, int64_t V, float T, int top_k, float top_p, float* M,
                   float* inv_k, uint32_t* t_key, uint64_t* zk_fx) {
  const float c = LOG2E_F * (1.0f / T);
  row_filter f = filter_row(x, V, c, top_k, top_p, zk_fx);
  *M = f.m;
  *inv_k = f.inv_k;
  *t_key = f.t;
}

static uint64_t draw_point(float u, uint64_t total) {
  if (!(u > 0.0f)) return 0u;
  return (uint64_t)floor((double)u * (double)total);
}

int64_t oc_fx_draw(const float* r, int64_t V, float u) {
  uint64_t total = 0;
  for (int64_t v = 0; v < V; ++v) total += fx40(r[v]);
  if (total == 0) return -1;
  const uint64_t t = draw_point(u, total);
  uint64_t cum = 0;
  int64_t last = -1;
  for (int64_t v = 0; v < V; ++v) {
    const uint64_t w = fx40(r[v]);
    if (w == 0) continue;
    cum += w;
    last = v;
    if (cum > t) return v;
  }
  return last;
}

/* Filtered probabilities of rows [rows, V] (get_sampling_probs). */
void oc_filtered_probs(const float* logits, int64_t rows, int64_t V, float T, int top_k,
                       float top_p, float* probs) {
  const float c = LOG2E_F * (1.0f / T);
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = logits + r * V;
    row_filter f = filter_row(x, V, c, top_k, top_p, NULL);
    if (!f.filtered) {
      oc_softmax(x, 1, V, T, probs + r * V);
      continue;
    }
    for (int64_t v = 0; v < V; ++v) probs[r * V + v] = filtered_p(&f, x[v], c);
  }
}

void oc_chain_filtered(const float* draft_logits, const int64_t* draft_ids,
                       const float* target_logits, float T, int top_k, float top_p,
                       const float* uniforms, int B, int k, int64_t V, int32_t* out_ids,
                       int32_t* accepted, int32_t* emitted) {
  const int use_k = top_k > 0 && (int64_t)top_k < V;
  const int use_p = top_p > 0.0f && top_p < 1.0f;
  if (!use_k && !use_p) {
    oc_chain_logits(draft_logits, draft_ids, target_logits, T, uniforms, B, k, V, out_ids,
                    accepted, emitted);
    return;
  }
  const float c = LOG2E_F * (1.0f / T);
  row_filter* ft = (row_filter*)malloc(sizeof(row_filter) * (size_t)(k + 1));
  row_filter* fd = (row_filter*)malloc(sizeof(row_filter) * (size_t)(k > 0 ? k : 1));
  float* r = (float*)malloc(sizeof(float) * (size_t)V);
  for (int b = 0; b < B; ++b) {
    const float* tl = target_logits + (int64_t)b * (k + 1) * V;
    const float* dl = draft_logits ? draft_logits + (int64_t)b * k * V : NULL;
    const int64_t* ids = k > 0 ? draft_ids + (int64_t)b * k : NULL;
    const float* u = uniforms + (int64_t)b * (k + 1);
    for (int i = 0; i <= k; ++i) ft[i] = filter_row(tl + (int64_t)i * V, V, c, top_k, top_p, NULL);
    if (dl)
      for (int i = 0; i < k; ++i) fd[i] = filter_row(dl + (int64_t)i * V, V, c, top_k, top_p, NULL);
    int j = k, cnt = 0;
    for (int i = 0; i < k; ++i) {
      const int64_t x = ids[i];
      int acc = 0;
      if (x >= 0 && x < V) {
        const float p = filtered_p(&ft[i], tl[(int64_t)i * V + x], c);
        const float q = dl ? filtered_p(&fd[i], dl[(int64_t)i * V + x], c) : 1.0f;
        acc = u[i] * q < p;
      }
      cnt += acc;
      if (!acc && j == k) j = i;
    }
    const float* prow = tl + (int64_t)j * V;
    int64_t tok = -1;
    if (j < k) {
      for (int64_t v = 0; v < V; ++v) {
        const float p = filtered_p(&ft[j], prow[v], c);
        const float q = dl ? filtered_p(&fd[j], dl[(int64_t)j * V + v], c) : (v == ids[j] ? 1.0f : 0.0f);
        const float d = p - q;
        r[v] = d > 0.0f ? d : 0.0f;
      }
      tok = oc_fx_draw(r, V, u[k]);
    }
    if (tok < 0) {
      for (int64_t v = 0; v < V; ++v) r[v] = filtered_p(&ft[j], prow[v], c);
      tok = oc_fx_draw(r, V, u[k]);
    }
    int32_t* out = out_ids + (int64_t)b * (k + 1);
    for (int i = 0; i <= k; ++i) out[i] = i < j ? (int32_t)ids[i] : (i == j ? (int32_t)tok : -1);
    accepted[b] = cnt;
    emitted[b] = j;
  }
  free(r);
  free(fd);
  free(ft);
}

/* sample() of sampling.py:61-115 for temperature > 0: one draw per row with
 * uniforms[row] (the chain with no draft tokens). */
void oc_sample(const float* logits, int64_t rows, int64_t V, float T, int top_k, float top_p,
               const float* uniforms, int64_t* out) {
  int32_t id, acc, emi;
  for (int64_t r = 0; r < rows; ++r) {
    oc_chain_filtered(NULL, NULL, logits + r * V, T, top_k, top_p, uniforms + r, 1, 0, V, &id,
                      &acc, &emi);
    out[r] = id;
  }
}
