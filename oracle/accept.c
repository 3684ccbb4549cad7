/*
 * ORACLE — TEST INFRASTRUCTURE ONLY.  Never linked into or called by the product
 * (batchspec_amd); only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
 * leg load it, as the checker.
 *
 * Plain-C restatement of speculative acceptance with explicit uniforms, following
 *   - batchspec/backends/mtp_engine.py:561-575  (evaluate_posterior, sampling branch:
 *     softmax probabilities, one-hot draft probabilities, chain speculative sampling)
 *   - batchspec/backends/utils/sampling.py:18-58 (get_sampling_probs: softmax(logits/T),
 *     top-p/top-k off)
 *   - the chain rule of FlashInfer chain_speculative_sampling (called at
 *     mtp_engine.py:569): accept x_i iff u_i*q_i(x_i) < p_i(x_i); on the first rejection
 *     j draw from norm(max(0, p_j - q_j)); if all accepted draw the bonus from p_k.
 *
 * Floating-point values follow the deterministic ("canonical") order the GPU kernels
 * document, restated here from that specification:
 *   exp2(y): n = floor(y) saturated to int32 (NaN: INT32_MAX); f = min(fl(y - n),
 *            largest float < 1), 0 for an infinite or NaN y; P(f) = Horner-fma of
 *            the degree-4 polynomial with P(0) = 1 fitted to 2^f on [0, 1) for
 *            relative error (binary32 coefficients below); ldexp(P, n).
 *   weights: w(x) = exp2(fma(x, C, -(M*C))), C = log2(e) * (1/T).
 *   groups of 8 consecutive elements; lane (8t+i) owns groups t + 256*i + 2048*j.
 *   row stats: per lane, running max m and an integer-valued reference r (start
 *   -2^127; per group r' = max(r, ceil(fl(gm*C))), the lane sum rescaled by
 *   ldexp(s, sat_int32(r - r'))), weights 2^fma(x, C, -r); then every lane rescaled
 *   once to the row max, s * exp2(r - fl(M*C)), and summed by the tree over lanes.
 *   sums: group sums left to right, lane sums over groups in j order, balanced tree
 *   over lanes; draws walk down that tree.
 * Build: cc -O2 -ffp-contract=off -fPIC -shared (see oracle/build.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define NGROUP 8
#define NT 256
#define NL 2048

static const float LOG2E = 0x1.715476p+0f;
static const float POLY[5] = {0x1.0p+0f, 0x1.62d6c2p-1f, 0x1.ee24b2p-3f, 0x1.abf636p-5f,
                              0x1.b7fb26p-7f};

float oc_exp2(float y) {
  float f;
  int n;
  if (y != y) { /* the GPU's clamped fract gives 0, its floor conversion INT32_MAX */
    f = 0.0f;
    n = INT32_MAX;
  } else {
    const float fl = floorf(y);
    f = fl == y ? 0.0f : y - fl; /* 0 for an integer or infinite y */
    if (f > 0x1.fffffep-1f) f = 0x1.fffffep-1f; /* fract is below 1 */
    n = fl >= 0x1p31f ? INT32_MAX : (fl < -0x1p31f ? INT32_MIN : (int)fl);
  }
  float p = POLY[4];
  for (int i = 3; i >= 0; --i) p = fmaf(p, f, POLY[i]);
  return ldexpf(p, n);
}

static float weight(float x, float c, float neg_mc) { return oc_exp2(fmaf(x, c, neg_mc)); }

static int64_t ngroups(int64_t V) { return (V + NGROUP - 1) / NGROUP; }

/* lane index -> first group and stride */
static int64_t lane_first_group(int lam) { return (int64_t)(lam >> 3) + 256 * (lam & 7); }

/* Balanced binary tree sum of NL values (destroys the array). */
static float tree_sum(float* v) {
  for (int width = NL; width > 1; width >>= 1)
    for (int i = 0; i < width / 2; ++i) v[i] = v[2 * i] + v[2 * i + 1];
  return v[0];
}

/* Conversion toward zero, saturated at the int32 range (-inf: INT32_MIN). */
static int sat_i32(float v) {
  if (v != v) return 0;
  return v <= -0x1p31f ? INT32_MIN : (v >= 0x1p31f ? INT32_MAX : (int)v);
}

/* (M, Z) of one row of V values: per lane a running max m, a sum s and an
 * integer-valued reference r (start -2^127, below fl(x*C) of every admissible x);
 * per group r' = max(r, ceil(fl(gm*C))), s = ldexp(s, sat(r - r')), r = r', then the
 * weights 2^fma(x, C, -r) summed in.  M = max over lanes, Z = tree over lanes of
 * s * 2^(r - fl(M*C)). */
void oc_row_stats(const float* x, int64_t V, float c, float* M, float* Z) {
  const int64_t G = ngroups(V);
  float* lr = (float*)malloc(sizeof(float) * NL);
  float* ls = (float*)malloc(sizeof(float) * NL);
  float mx = -INFINITY;
  for (int lam = 0; lam < NL; ++lam) {
    float m = -INFINITY, s = 0.0f, r = -0x1p127f;
    for (int64_t g = lane_first_group(lam); g < G; g += NL) {
      int64_t v0 = g * NGROUP;
      int n = (int)((V - v0) < NGROUP ? (V - v0) : NGROUP);
      float gm = x[v0];
      for (int e = 1; e < n; ++e)
        if (x[v0 + e] > gm) gm = x[v0 + e];
      const float rn = fmaxf(r, ceilf(gm * c));
      s = ldexpf(s, sat_i32(r - rn));
      r = rn;
      if (gm > m) m = gm;
      float gs = 0.0f;
      for (int e = 0; e < n; ++e) gs = gs + weight(x[v0 + e], c, -r);
      s = s + gs;
    }
    lr[lam] = r;
    ls[lam] = s;
    if (m > mx) mx = m;
  }
  const float rho = mx * c;
  for (int lam = 0; lam < NL; ++lam) ls[lam] = ls[lam] * oc_exp2(lr[lam] - rho);
  *M = mx;
  *Z = tree_sum(ls);
  free(ls);
  free(lr);
}

void oc_softmax(const float* logits, int64_t rows, int64_t V, float T, float* probs) {
  const float c = LOG2E * (1.0f / T);
  for (int64_t r = 0; r < rows; ++r) {
    float M, Z;
    oc_row_stats(logits + r * V, V, c, &M, &Z);
    float neg = -(M * c), inv = 1.0f / Z;
    for (int64_t v = 0; v < V; ++v) probs[r * V + v] = weight(logits[r * V + v], c, neg) * inv;
  }
}

/* Draw from weights r[0..V) (all >= 0) with uniform u by the canonical tree walk.
 * Returns -1 if every weight is zero. */
int64_t oc_tree_draw(const float* r, int64_t V, float u) {
  const int64_t G = ngroups(V);
  float* gsum = (float*)malloc(sizeof(float) * (size_t)(G > 0 ? G : 1));
  float* tree = (float*)malloc(sizeof(float) * 2 * NL);
  for (int64_t g = 0; g < G; ++g) {
    int64_t v0 = g * NGROUP;
    int n = (int)((V - v0) < NGROUP ? (V - v0) : NGROUP);
    float s = 0.0f;
    for (int e = 0; e < n; ++e) s = s + r[v0 + e];
    gsum[g] = s;
  }
  for (int lam = 0; lam < NL; ++lam) {
    float s = 0.0f;
    for (int64_t g = lane_first_group(lam); g < G; g += NL) s = s + gsum[g];
    tree[lam] = s;
  }
  /* levels stored consecutively: level l starts at off[l] */
  int off[12];
  off[0] = 0;
  int n = NL;
  for (int l = 1; l < 12; ++l) {
    off[l] = off[l - 1] + n;
    for (int i = 0; i < n / 2; ++i) tree[off[l] + i] = tree[off[l - 1] + 2 * i] + tree[off[l - 1] + 2 * i + 1];
    n >>= 1;
  }
  int64_t result = -1;
  float total = tree[off[11]];
  if (total > 0.0f) {
    float t = u * total;
    int idx = 0;
    for (int l = 11; l >= 1; --l) {
      float left = tree[off[l - 1] + 2 * idx];
      float right = tree[off[l - 1] + 2 * idx + 1];
      if (t < left || !(right > 0.0f)) {
        idx = 2 * idx;
      } else {
        t = t - left;
        idx = 2 * idx + 1;
      }
    }
    float c = 0.0f, c_at = 0.0f, c_last = 0.0f;
    int64_t chosen = -1, last_pos = -1;
    for (int64_t g = lane_first_group(idx); g < G; g += NL) {
      float cn = c + gsum[g];
      if (gsum[g] > 0.0f) {
        last_pos = g;
        c_last = c;
      }
      if (t < cn) {
        chosen = g;
        c_at = c;
        break;
      }
      c = cn;
    }
    if (chosen < 0) {
      chosen = last_pos;
      c_at = c_last;
    }
    if (chosen >= 0) {
      float tl = t - c_at, s = 0.0f;
      int64_t v0 = chosen * NGROUP, last_e = -1;
      int ne = (int)((V - v0) < NGROUP ? (V - v0) : NGROUP);
      for (int e = 0; e < ne; ++e) {
        s = s + r[v0 + e];
        if (r[v0 + e] > 0.0f) last_e = e;
        if (tl < s) {
          result = v0 + e;
          break;
        }
      }
      if (result < 0 && last_e >= 0) result = v0 + last_e;
    }
  }
  free(tree);
  free(gsum);
  return result;
}

/* Shared chain logic once p/q rows are materialised as weights.
 * p_rows: k+1 rows of target probabilities; q_rows: k rows or NULL (one-hot). */
static void chain_one(const float* p_rows, const float* q_rows, const int64_t* draft, const float* u,
                      int k, int64_t V, float* scratch, int32_t* out, int32_t* accepted,
                      int32_t* emitted) {
  int j = k, cnt = 0;
  for (int i = 0; i < k; ++i) {
    int64_t x = draft[i];
    int acc = 0;
    if (x >= 0 && x < V) {
      float p = p_rows[(int64_t)i * V + x];
      float q = q_rows ? q_rows[(int64_t)i * V + x] : 1.0f;
      acc = u[i] * q < p;
    }
    cnt += acc;
    if (!acc && j == k) j = i;
  }
  const float* prow = p_rows + (int64_t)j * V;
  if (j < k) {
    for (int64_t v = 0; v < V; ++v) {
      float q = q_rows ? q_rows[(int64_t)j * V + v] : (v == draft[j] ? 1.0f : 0.0f);
      float d = prow[v] - q;
      scratch[v] = d > 0.0f ? d : 0.0f;
    }
  } else {
    memcpy(scratch, prow, sizeof(float) * (size_t)V);
  }
  int64_t tok = oc_tree_draw(scratch, V, u[k]);
  if (tok < 0 && j < k) tok = oc_tree_draw(prow, V, u[k]); /* no residual mass: draw p_j */
  for (int i = 0; i <= k; ++i) out[i] = i < j ? (int32_t)draft[i] : (i == j ? (int32_t)tok : -1);
  *accepted = cnt;
  *emitted = j;
}

/* Probability inputs: target_probs [B,k+1,V], draft_probs [B,k,V] or NULL. */
void oc_chain_probs(const float* draft_probs, const int64_t* draft_ids, const float* target_probs,
                    const float* uniforms, int B, int k, int64_t V, int32_t* out_ids,
                    int32_t* accepted, int32_t* emitted) {
  float* scratch = (float*)malloc(sizeof(float) * (size_t)V);
  for (int b = 0; b < B; ++b)
    chain_one(target_probs + (int64_t)b * (k + 1) * V,
              draft_probs ? draft_probs + (int64_t)b * k * V : NULL, draft_ids + (int64_t)b * k,
              uniforms + (int64_t)b * (k + 1), k, V, scratch, out_ids + (int64_t)b * (k + 1),
              accepted + b, emitted + b);
  free(scratch);
}

/* Logit inputs (already widened to fp32): softmax at temperature T, then the chain. */
void oc_chain_logits(const float* draft_logits, const int64_t* draft_ids, const float* target_logits,
                     float T, const float* uniforms, int B, int k, int64_t V, int32_t* out_ids,
                     int32_t* accepted, int32_t* emitted) {
  float* p = (float*)malloc(sizeof(float) * (size_t)(k + 1) * (size_t)V);
  float* q = draft_logits ? (float*)malloc(sizeof(float) * (size_t)(k > 0 ? k : 1) * (size_t)V) : NULL;
  float* scratch = (float*)malloc(sizeof(float) * (size_t)V);
  for (int b = 0; b < B; ++b) {
    oc_softmax(target_logits + (int64_t)b * (k + 1) * V, k + 1, V, T, p);
    if (q) oc_softmax(draft_logits + (int64_t)b * k * V, k, V, T, q);
    chain_one(p, q, draft_ids + (int64_t)b * k, uniforms + (int64_t)b * (k + 1), k, V, scratch,
              out_ids + (int64_t)b * (k + 1), accepted + b, emitted + b);
  }
  free(scratch);
  free(q);
  free(p);
}
