// Speculative acceptance (piece 3 of the verification path) and softmax.
//
// Greedy: MTPEngine.evaluate_posterior greedy branch
// (batchspec/backends/mtp_engine.py:553-560) with the argmax of
// mtp_engine.py:747 fused in:
//   flags_i = preds_i == draft_i;  accept = sum(flags)+1 (reference rule) or the
//   longest matching prefix + 1;  bonus = preds[accept-1];
//   eos_accepted = any(draft_i == eos and flags_i).
// Argmax follows torch.argmax: the first maximum wins and NaN counts as maximum.
//
// Stochastic: chain speculative sampling (the FlashInfer call at
// mtp_engine.py:569) with caller-supplied uniforms u[B, k+1]:
//   accept draft token x_i  iff  u_i * q_i(x_i) < p_i(x_i),  i = 0..k-1 in order;
//   at the first rejection j, emit a draw from max(0, p_j - q_j) (normalised) using
//   u_k; if all k are accepted, emit a draw from p_k using u_k.
// All floating-point values the decisions depend on follow the canonical order of
// canon.h, so the token ids match a CPU restatement bit for bit.  The draw is an
// inverse-CDF walk down the 2048-lane reduction tree: at each node go left iff
// t < sum(left) (or the right subtree is empty), else t -= sum(left); inside the
// chosen lane the groups, then the elements, are scanned left to right.
//
// This translation unit is compiled with -ffp-contract=off: every multiply-add
// that the canonical order fuses is an explicit fmaf.
#include <algorithm>
#include <mutex>

#include "common.h"
#include "canon.h"
#include "page_update.h"
#include "rows.h"

namespace bsx {
namespace acc {

// rows [0, n_a) come from tensor a, rows [n_a, n_a + n_b) from tensor b.
template <int DT>
__global__ void __launch_bounds__(256) stats_kernel(const void* a, int64_t n_a, const void* b,
                                                    int64_t V, float c, float2* stats) {
  const int64_t r = blockIdx.x;
  const size_t esz = DT == BSX_DTYPE_FP32 ? 4 : 2;
  const char* base = r < n_a ? static_cast<const char*>(a) + r * V * esz
                             : static_cast<const char*>(b) + (r - n_a) * V * esz;
  const bool vec = ((V * esz) % 16 == 0) && (((uintptr_t)base) % 16 == 0);
  float m, z;
  row_stats<DT>(base, V, vec, c, &m, &z);
  if (threadIdx.x == 0) stats[r] = make_float2(m, z);
}

// ----------------------------------------------------------------------------
// Chain decision (identical in every kernel that needs it).
// ----------------------------------------------------------------------------
struct ChainArgs {
  // logits path
  const void* t_logits;  // [B, k+1, V]
  const void* d_logits;  // [B, k, V] or null (one-hot draft)
  const float2* stats;   // [B*(k+1)] target rows, then [B*k] draft rows
  float c;
  // probs path
  const float* t_probs;  // [B, k+1, V]
  const float* d_probs;  // [B, k, V] or null
  // common
  const int64_t* draft_ids;  // [B, k]
  const float* uniforms;     // [B, k+1]
  int B, k;
  int64_t V;
  float* lanes;  // [B, 2048]
  int32_t* dec;  // [B, 2]: the residual kernel's decision (j, independent accepts)
  int32_t* out_ids;
  int32_t* accepted;
  int32_t* emitted;
};

template <int DT, bool LOGITS>
struct Chain {
  const ChainArgs& a;
  __device__ Chain(const ChainArgs& args) : a(args) {}

  __device__ __forceinline__ float2 tstat(int b, int i) const { return a.stats[(int64_t)b * (a.k + 1) + i]; }
  __device__ __forceinline__ float2 dstat(int b, int i) const {
    return a.stats[(int64_t)a.B * (a.k + 1) + (int64_t)b * a.k + i];
  }
  __device__ __forceinline__ const void* trow(int b, int i) const {
    const size_t esz = LOGITS ? (DT == BSX_DTYPE_FP32 ? 4 : 2) : 4;
    const char* base = LOGITS ? static_cast<const char*>(a.t_logits)
                              : reinterpret_cast<const char*>(a.t_probs);
    return base + (((int64_t)b * (a.k + 1) + i) * a.V) * esz;
  }
  __device__ __forceinline__ const void* drow(int b, int i) const {
    const size_t esz = LOGITS ? (DT == BSX_DTYPE_FP32 ? 4 : 2) : 4;
    const char* base = LOGITS ? static_cast<const char*>(a.d_logits)
                              : reinterpret_cast<const char*>(a.d_probs);
    return base + (((int64_t)b * a.k + i) * a.V) * esz;
  }
  __device__ __forceinline__ bool has_draft_dist() const {
    return LOGITS ? a.d_logits != nullptr : a.d_probs != nullptr;
  }

  // p_i(v), q_i(v) as defined by the canonical order.
  __device__ __forceinline__ float p_at(int b, int i, int64_t v) const {
    if constexpr (LOGITS) {
      const float2 s = tstat(b, i);
      const float x = load_one<DT>(trow(b, i), v);
      return canon::weight(x, a.c, -(s.x * a.c)) * (1.0f / s.y);
    } else {
      return static_cast<const float*>(trow(b, i))[v];
    }
  }
  __device__ __forceinline__ float q_at(int b, int i, int64_t v, int64_t draft_tok) const {
    if (!has_draft_dist()) return v == draft_tok ? 1.0f : 0.0f;
    if constexpr (LOGITS) {
      const float2 s = dstat(b, i);
      const float x = load_one<DT>(drow(b, i), v);
      return canon::weight(x, a.c, -(s.x * a.c)) * (1.0f / s.y);
    } else {
      return static_cast<const float*>(drow(b, i))[v];
    }
  }

  // Ratio test of draft position i: accept iff u_i * q_i(x_i) < p_i(x_i).
  __device__ __forceinline__ bool accepts(int b, int i) const {
    const int64_t x = a.draft_ids[(int64_t)b * a.k + i];
    if (x < 0 || x >= a.V) return false;
    const float p = p_at(b, i, x);
    const float q = q_at(b, i, x, x);
    const float u = a.uniforms[(int64_t)b * (a.k + 1) + i];
    return u * q < p;
  }

  // j (first rejected position, k if none) and the independent accept count, for the
  // whole workgroup: the first wave runs the k ratio tests in parallel (lane i, test i).
  // With k < 64 (LOGITS), lane i also reads the statistics of target row i and draft
  // row i up front, and the lane of row j hands them to the workgroup (pre_*), so the
  // residual's first loads do not wait for another round trip.
  bool pre = false;
  float2 pre_ts, pre_ds;

  __device__ __forceinline__ int decide(int b, int* n_accept) {
    __shared__ int s_j, s_n;
    __shared__ float2 s_ts, s_ds;
    const bool stage = LOGITS && a.k < 64;
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      float2 ts = {0.f, 0.f}, ds = {0.f, 0.f};
      if (stage && lane <= a.k) {
        ts = tstat(b, lane);
        if (lane < a.k && has_draft_dist()) ds = dstat(b, lane);
      }
      int j = a.k, cnt = 0;
      for (int i0 = 0; i0 < a.k; i0 += 64) {
        const int i = i0 + lane;
        const bool acc = i < a.k && accepts(b, i);
        const uint64_t acc_bits = __builtin_amdgcn_ballot_w64(acc);
        const uint64_t rej_bits = __builtin_amdgcn_ballot_w64(i < a.k && !acc);
        cnt += __builtin_popcountll(acc_bits);
        if (j == a.k && rej_bits != 0) j = i0 + __builtin_ctzll(rej_bits);
      }
      if (lane == 0) {
        s_j = j;
        s_n = cnt;
      }
      if (stage && lane == j) {
        s_ts = ts;
        s_ds = ds;
      }
    }
    __syncthreads();
    *n_accept = s_n;
    if (stage) {
      pre = true;
      pre_ts = s_ts;
      pre_ds = s_ds;
    }
    return s_j;
  }

  // What the residual of row j needs, computed once: row pointers, whether they can be
  // read in 16-byte vectors, and the normalisers of p_j and q_j.
  // (j == k: target row k alone; fallback: p_j alone, used when the residual has no
  // mass.)
  struct ResidualRow {
    const void* tr;
    const void* dr;
    bool tvec, dvec, with_q, dist;
    float tnmc, tinv, dnmc, dinv;
    int64_t x;  // the draft token of row j (one-hot drafts)
  };
  __device__ __forceinline__ ResidualRow residual_row(int b, int j, bool fallback) const {
    ResidualRow rr;
    const int64_t V = a.V;
    const int esz = LOGITS && DT != BSX_DTYPE_FP32 ? 2 : 4;
    rr.x = j < a.k ? a.draft_ids[(int64_t)b * a.k + j] : -1;
    rr.tr = trow(b, j);
    rr.tvec = (((uintptr_t)rr.tr) % 16 == 0) && ((V * esz) % 16 == 0);
    rr.with_q = j < a.k && !fallback;
    rr.dist = has_draft_dist();
    rr.dr = rr.with_q && rr.dist ? drow(b, j) : rr.tr;
    rr.dvec = (((uintptr_t)rr.dr) % 16 == 0) && ((V * esz) % 16 == 0);
    rr.tnmc = rr.tinv = rr.dnmc = rr.dinv = 0.f;
    if constexpr (LOGITS) {
      const float2 ts = pre ? pre_ts : tstat(b, j);
      rr.tnmc = -(ts.x * a.c);
      rr.tinv = 1.0f / ts.y;
      if (rr.with_q && rr.dist) {
        const float2 ds = pre ? pre_ds : dstat(b, j);
        rr.dnmc = -(ds.x * a.c);
        rr.dinv = 1.0f / ds.y;
      }
    }
    return rr;
  }

  // Residual weights of group g of the row prepared in rr.
  __device__ __forceinline__ int residual_group(const ResidualRow& rr, int64_t g, float r[8]) const {
    const int64_t V = a.V;
    float xt[8], xd[8];
    const int n = LOGITS ? load_group<DT>(rr.tr, g, V, rr.tvec, xt)
                         : load_group<BSX_DTYPE_FP32>(rr.tr, g, V, rr.tvec, xt);
    if (rr.with_q && rr.dist) {
      if constexpr (LOGITS) load_group<DT>(rr.dr, g, V, rr.dvec, xd);
      else load_group<BSX_DTYPE_FP32>(rr.dr, g, V, rr.dvec, xd);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float p = 0.f, q = 0.f;
      if (e < n) {
        if constexpr (LOGITS) p = canon::weight(xt[e], a.c, rr.tnmc) * rr.tinv;
        else p = xt[e];
        if (rr.with_q) {
          if (rr.dist) {
            if constexpr (LOGITS) q = canon::weight(xd[e], a.c, rr.dnmc) * rr.dinv;
            else q = xd[e];
          } else {
            q = (g * kGroup + e == rr.x) ? 1.0f : 0.0f;
          }
        }
      }
      r[e] = rr.with_q ? fmaxf(p - q, 0.0f) : p;
    }
    return n;
  }

  // Sum of a group's residual values, left to right from 0 (canonical).
  __device__ __forceinline__ static float group_sum(const float (&r)[8], int n) {
    float gs = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < n) gs = gs + r[e];
    return gs;
  }

  // Lane lam = 8*tt + ii of row j: its group sums and the lane sum.  Groups are computed
  // NB at a time (their loads issued together), summed in canonical order.
  __device__ __forceinline__ float lane_sum(int b, int j, int lam, bool fallback) const {
    constexpr int NB = 4;
    const int64_t G = ceil_div(a.V, kGroup);
    const int tt = lam >> 3, ii = lam & 7;
    const ResidualRow rr = residual_row(b, j, fallback);
    float s = 0.f;
    for (int64_t g0 = (int64_t)tt + 256 * ii; g0 < G; g0 += (int64_t)NB * kLanes) {
      float r[NB][8];
      int n[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int64_t g = g0 + (int64_t)u * kLanes;
        n[u] = residual_group(rr, g < G ? g : g0, r[u]);
      }
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int64_t g = g0 + (int64_t)u * kLanes;
        if (g < G) {
          s = s + group_sum(r[u], n[u]);
        }
      }
    }
    return s;
  }
};

// grid (B, 8): part w computes the lanes 8*tau + w, tau = threadIdx.x.
template <int DT, bool LOGITS>
__global__ void __launch_bounds__(256) residual_kernel(ChainArgs a) {
  Chain<DT, LOGITS> ch(a);
  const int b = blockIdx.x;
  const int w = blockIdx.y;
  int nacc;
  const int j = ch.decide(b, &nacc);
  if (w == 0 && threadIdx.x == 0) {  // for the pick kernel
    a.dec[2 * b] = j;
    a.dec[2 * b + 1] = nacc;
  }
  const int lam = 8 * threadIdx.x + w;
  a.lanes[(int64_t)b * kLanes + lam] = ch.lane_sum(b, j, lam, false);
}

// Levels 1..11 of the canonical tree over the 2048 lane sums (v: lanes 8t .. 8t+7 of
// thread t), each node the sum of its two children, stored at tree[4096 - (4096 >> l) + i]
// for node i of level l (level 0 included): levels 1-3 from registers, 4-9 across the
// wave by shuffles, 10-11 from the four wave nodes.  Every thread calls it; it ends with
// a barrier.
__device__ __forceinline__ void build_lane_tree(float* tree, const float (&v)[8]) {
  const int t = threadIdx.x, lane = t & 63;
  float a1[4], a2[2];
#pragma unroll
  for (int i = 0; i < 8; ++i) tree[8 * t + i] = v[i];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a1[i] = v[2 * i] + v[2 * i + 1];
    tree[2048 + 4 * t + i] = a1[i];
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    a2[i] = a1[2 * i] + a1[2 * i + 1];
    tree[3072 + 2 * t + i] = a2[i];
  }
  float s = a2[0] + a2[1];
  tree[3584 + t] = s;
#pragma unroll
  for (int d = 1, l = 4; d < 64; d <<= 1, ++l) {
    const float o = __shfl_xor(s, d);
    s = (lane & d) ? o + s : s + o;  // left child + right child
    if ((lane & (2 * d - 1)) == 0) tree[4096 - (4096 >> l) + (t >> (l - 3))] = s;
  }
  __syncthreads();
  if (t == 0) {
    const float x0 = tree[4088] + tree[4089], x1 = tree[4090] + tree[4091];
    tree[4092] = x0;
    tree[4093] = x1;
    tree[4094] = x0 + x1;
  }
  __syncthreads();
}

// grid B: tree over the 2048 lane sums, inverse-CDF walk, outputs.
template <int DT, bool LOGITS>
__global__ void __launch_bounds__(256) pick_kernel(ChainArgs a) {
  __shared__ float tree[2 * kLanes];  // level l at [4096 - (4096 >> l), ...)
  __shared__ float gs_lane[256];
  __shared__ float gv[256][8];  // the residual values of those groups
  __shared__ int s_lane;
  __shared__ float s_tg;
  Chain<DT, LOGITS> ch(a);
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int j = a.dec[2 * b];  // the residual kernel's decision
  const int nacc = a.dec[2 * b + 1];
  const int64_t G = ceil_div(a.V, kGroup);

  // The row statistics of row j are read now, before the tree is built (the walk's
  // group sums need them).
  auto rr = ch.residual_row(b, j, false);
  {
    float v[8];
    const float* ls = a.lanes + (int64_t)b * kLanes + 8 * t;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = ls[i];
    build_lane_tree(tree, v);
  }
  bool fallback = false;
  if (!(tree[2 * kLanes - 2] > 0.f)) {
    // No residual mass (p_j <= q_j everywhere in fp32): draw from p_j instead.
    fallback = true;
    rr.with_q = false;
    rr.dr = rr.tr;
    rr.dvec = rr.tvec;
    float v[8];
    for (int w = 0; w < 8; ++w) v[w] = ch.lane_sum(b, j, 8 * t + w, true);
    __syncthreads();
    build_lane_tree(tree, v);
  }
  if (t == 0) {
    const float u = a.uniforms[(int64_t)b * (a.k + 1) + a.k];
    float tg = u * tree[2 * kLanes - 2];
    int idx = 0;
    for (int l = 11; l >= 1; --l) {
      const int off = 4096 - (4096 >> (l - 1));  // level l - 1
      const float left = tree[off + 2 * idx];
      const float right = tree[off + 2 * idx + 1];
      if (tg < left || !(right > 0.f)) {
        idx = 2 * idx;
      } else {
        tg = tg - left;
        idx = 2 * idx + 1;
      }
    }
    s_lane = idx;
    s_tg = tg;
  }
  __syncthreads();
  // The lane's groups g = tt + 256 ii + 2048 m in order: their sums computed again, one
  // group per thread (the residual kernel keeps none), then scanned by thread 0; the
  // values of a chunk's groups stay in LDS for the element scan.
  const int lane = s_lane;
  const float tg = s_tg;
  const int64_t g_first = (int64_t)(lane >> 3) + 256 * (lane & 7);
  const int64_t n_groups = g_first < G ? ceil_div(G - g_first, (int64_t)kLanes) : 0;
  float cacc = 0.f, c_at = 0.f, c_last = 0.f;
  int64_t chosen = -1, last_pos = -1;
  float rc[8];
  int nc = 0;
  for (int64_t m0 = 0; m0 < n_groups; m0 += 256) {
    if (m0 + t < n_groups) {
      float r[8];
      const int n = ch.residual_group(rr, g_first + (m0 + t) * kLanes, r);
      gs_lane[t] = Chain<DT, LOGITS>::group_sum(r, n);
#pragma unroll
      for (int e = 0; e < 8; ++e) gv[t][e] = e < n ? r[e] : 0.f;
    }
    __syncthreads();
    if (t == 0 && chosen < 0) {
      const int cnt = (int)min<int64_t>(256, n_groups - m0);
      for (int q = 0; q < cnt; ++q) {
        const int64_t g = g_first + (m0 + q) * kLanes;
        const float gsv = gs_lane[q];
        const float cn = cacc + gsv;
        if (gsv > 0.f) {
          last_pos = g;
          c_last = cacc;
        }
        if (tg < cn) {
          chosen = g;
          c_at = cacc;
          nc = (int)min<int64_t>(kGroup, a.V - g * kGroup);
#pragma unroll
          for (int e = 0; e < 8; ++e) rc[e] = gv[q][e];
          break;
        }
        cacc = cn;
      }
    }
    __syncthreads();
  }
  if (t == 0) {
    if (chosen < 0 && last_pos >= 0) {
      // the last group with mass (its values may have left LDS with a later chunk)
      chosen = last_pos;
      c_at = c_last;
      nc = ch.residual_group(rr, chosen, rc);
    }
    int64_t tok = -1;
    if (chosen >= 0) {
      const float tl = tg - c_at;
      float s = 0.f;
      int64_t last_e = -1;
      for (int e = 0; e < nc; ++e) {
        s = s + rc[e];
        if (rc[e] > 0.f) last_e = e;
        if (tl < s) {
          tok = chosen * kGroup + e;
          break;
        }
      }
      if (tok < 0 && last_e >= 0) tok = chosen * kGroup + last_e;
    }
    int32_t* out = a.out_ids + (int64_t)b * (a.k + 1);
    for (int i = 0; i <= a.k; ++i) {
      int32_t v = -1;
      if (i < j) v = (int32_t)a.draft_ids[(int64_t)b * a.k + i];
      else if (i == j) v = (int32_t)tok;
      out[i] = v;
    }
    a.accepted[b] = nacc;
    a.emitted[b] = j;
  }
}

// ----------------------------------------------------------------------------
// Softmax: probs = weight(x) / Z with the canonical (M, Z).
// ----------------------------------------------------------------------------
template <int DT>
__global__ void __launch_bounds__(256) softmax_norm_kernel(const void* logits, int64_t V, float c,
                                                           const float2* stats, float* probs) {
  const int64_t r = blockIdx.x;
  const float2 s = stats[r];
  const float nmc = -(s.x * c);
  const float inv = 1.0f / s.y;
  const size_t esz = DT == BSX_DTYPE_FP32 ? 4 : 2;
  const char* row = static_cast<const char*>(logits) + r * V * esz;
  float* out = probs + r * V;
  for (int64_t v = (int64_t)blockIdx.y * 256 + threadIdx.x; v < V; v += (int64_t)gridDim.y * 256)
    out[v] = canon::weight(load_one<DT>(row, v), c, nmc) * inv;
}

// ----------------------------------------------------------------------------
// Argmax (torch semantics: the first maximum wins, NaN counts as the maximum).
//
// Every row is cut into `parts` equal column ranges, one workgroup each, sized so that
// a thread issues all of its loads of the range at once (one memory round trip per
// workgroup, and every workgroup of a [320, 128256] call resident at the same time),
// then a small combine over the parts of a row in column order.  A thread visits its
// columns in increasing order, so ties keep the earlier column with a strict
// comparison; each 8-element vector costs a NaN-propagating maximum reduction and a
// branch-free update of (running maximum, vector holding it), and the column inside
// the winning vector is located once, from registers.
// ----------------------------------------------------------------------------
constexpr int kArgmaxThreads = 256;
// Bytes a thread loads per batch: 8 16-byte loads in flight.  Measured at [64, 5, 128256]
// bf16 (kernel trace, rotating buffers): 16 loads per thread (1280 workgroups, all
// resident, every workgroup computing only after its loads) 18.1 us; 8 (2560 workgroups,
// about 1.7 per slot, so the maxima of early workgroups overlap the loads of later ones)
// 15.9 us; 4 16.3 us.
constexpr int kArgmaxBytesPerThread = 128;

struct ArgmaxSplit {
  int64_t parts;  // workgroups per row
  int64_t chunk;  // columns per workgroup (multiple of 8)
};

static ArgmaxSplit argmax_split(int64_t rows, int64_t V, int elem_bytes) {
  const int64_t cols_per_wg = (int64_t)kArgmaxThreads * kArgmaxBytesPerThread / elem_bytes;
  int64_t parts = ceil_div(V, cols_per_wg);
  // few rows: more, smaller parts (at least ~512 workgroups, parts of >= 4096 columns)
  parts = std::max(parts, std::min(ceil_div(V, 4096), ceil_div(512, std::max<int64_t>(rows, 1))));
  ArgmaxSplit a;
  a.chunk = ceil_div(ceil_div(V, parts), 8) * 8;
  a.parts = ceil_div(V, a.chunk);
  return a;
}

// (av, ac) ranks before (bv, bc): NaN first (lowest column among NaNs), then the
// larger value, then the lower column.
__device__ __forceinline__ bool better(float av, int ac, float bv, int bc) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ac < bc);
  return av > bv || (av == bv && ac < bc);
}

__device__ __forceinline__ void take(float x, int col, float& bv, int& bc) {
  // columns arrive in increasing order: strict rule, NaN sticks once seen
  const bool upd = (bc == INT_MAX) || (x > bv) || ((x != x) && (bv == bv));
  if (upd) {
    bv = x;
    bc = col;
  }
}

// The 8 values of a vector as fp32.
template <int DT>
__device__ __forceinline__ void vec8(const u32x4* p, float (&x)[8]) {
  if constexpr (DT == BSX_DTYPE_FP32) {
    const f32x4 a = __builtin_bit_cast(f32x4, p[0]);
    const f32x4 b = __builtin_bit_cast(f32x4, p[1]);
    x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
    x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
  } else {
    const u32x4 w = p[0];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x[2 * q] = lo_f32<DT>(w[q]);
      x[2 * q + 1] = hi_f32<DT>(w[q]);
    }
  }
}

__device__ __forceinline__ float max8(const float (&x)[8]) {
  return __builtin_elementwise_maximum(
      __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[0], x[1]),
                                    __builtin_elementwise_maximum(x[2], x[3])),
      __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[4], x[5]),
                                    __builtin_elementwise_maximum(x[6], x[7])));
}

// First position in x of the value m (NaN matches NaN).
__device__ __forceinline__ int first_of(const float (&x)[8], float m) {
  int e = 7;
#pragma unroll
  for (int q = 6; q >= 0; --q)
    if (x[q] == m || (m != m && x[q] != x[q])) e = q;
  return e;
}

// Reduce (bv, bc) over the workgroup; every thread gets the result.
__device__ __forceinline__ void block_best(float& bv, int& bc) {
  constexpr int NW = kArgmaxThreads / 64;
  __shared__ float s_v[NW];
  __shared__ int s_c[NW];
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float ov = __shfl_xor(bv, m);
    const int oc = __shfl_xor(bc, m);
    if (better(ov, oc, bv, bc)) {
      bv = ov;
      bc = oc;
    }
  }
  __syncthreads();  // previous readers of s_v / s_c are done
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = bv;
    s_c[threadIdx.x >> 6] = bc;
  }
  __syncthreads();
  bv = s_v[0];
  bc = s_c[0];
#pragma unroll
  for (int q = 1; q < NW; ++q)
    if (better(s_v[q], s_c[q], bv, bc)) {
      bv = s_v[q];
      bc = s_c[q];
    }
}

// grid rows * parts: workgroup (r, p) takes columns [p*chunk, min(V, (p+1)*chunk)) of row r.
// (Evaluating the greedy acceptance inside this launch, by the workgroup that finishes
// last, was measured slower on MI355X than the separate small kernel: the partials must
// cross the XCDs' separate L2 caches, by a release fence per workgroup (an L2 write-back
// each) or by written-through stores and uncached reads.)
template <int DT>
__global__ void __launch_bounds__(kArgmaxThreads) argmax_part_kernel(const void* logits, int64_t V,
                                                           int64_t row_stride, int64_t parts,
                                                           int64_t chunk, float* pval,
                                                           int32_t* pcol) {
  constexpr int ES = DT == BSX_DTYPE_FP32 ? 4 : 2;
  constexpr int VW = ES / 2;  // 16-byte loads per 8-element vector
  constexpr int NT = kArgmaxThreads;
  constexpr int U = kArgmaxBytesPerThread / (16 * VW);  // vectors per thread per batch
  const int64_t wg = blockIdx.x;
  const int64_t r = wg / parts;
  const int64_t part = wg - r * parts;
  const int64_t c0 = part * chunk;
  const int64_t c1 = min(V, c0 + chunk);
  const int t = threadIdx.x;
  const char* row = static_cast<const char*>(logits) + r * row_stride * ES;
  float bv = -INFINITY;
  int bc = INT_MAX;
  // head (unaligned), body (8-element vectors), tail: each thread's columns ascend
  int64_t a0 = c0, a1 = c0;
  if ((((uintptr_t)row) % 16) == 0) {
    a0 = min(c1, (c0 + 7) / 8 * 8);
    a1 = max(a0, c1 / 8 * 8);
  }
  if (c0 + t < a0) take(load_one<DT>(row, c0 + t), (int)(c0 + t), bv, bc);
  const int64_t nv = (a1 - a0) / 8;
  const u32x4* vbase = reinterpret_cast<const u32x4*>(row + a0 * ES);
  // The logits are read once: non-temporal loads, all U vectors of a batch issued
  // together (indices past the range are clamped to its last vector and not used).
  for (int64_t v0 = 0; v0 < nv; v0 += (int64_t)U * NT) {
    u32x4 buf[U][VW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t v = min(v0 + t + (int64_t)u * NT, nv - 1);
#pragma unroll
      for (int h = 0; h < VW; ++h) buf[u][h] = __builtin_nontemporal_load(vbase + v * VW + h);
    }
    // running maximum of the batch and the first vector holding it (vectors arrive in
    // increasing column order: strict rule, NaN sticks once seen); no branches
    float m = bv;
    int bu = -1;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float x[8];
      vec8<DT>(buf[u], x);
      const float m8 = max8(x);
      const bool ok = v0 + t + (int64_t)u * NT < nv;
      const bool upd = ok && ((bc == INT_MAX && bu < 0) || (m8 > m) || ((m8 != m8) && (m == m)));
      m = upd ? m8 : m;
      bu = upd ? u : bu;
    }
    if (bu >= 0) {  // locate the column inside the winning vector (registers only)
      float x[8];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (u == bu) vec8<DT>(buf[u], x);
      bv = m;
      bc = (int)(a0 + 8 * (v0 + t + (int64_t)bu * NT)) + first_of(x, m);
    }
  }
  for (int64_t c = a1 + t; c < c1; c += NT) take(load_one<DT>(row, c), (int)c, bv, bc);
  block_best(bv, bc);
  if (t == 0) {
    pval[wg] = bv;
    pcol[wg] = bc;
  }
}

// argmax of row r from the partials of its parts, combined in column order.
__device__ __forceinline__ int64_t row_argmax(const float* pval, const int32_t* pcol, int64_t r,
                                              int64_t parts) {
  // the first 8 parts in one round of loads, any further ones after
  constexpr int P = 8;
  float v[P];
  int c[P];
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const int64_t i = r * parts + min((int64_t)q, parts - 1);
    v[q] = pval[i];
    c[q] = pcol[i];
  }
  float bv = v[0];
  int bc = c[0];
#pragma unroll
  for (int q = 1; q < P; ++q)
    if (q < parts && better(v[q], c[q], bv, bc)) {
      bv = v[q];
      bc = c[q];
    }
  for (int64_t q = P; q < parts; ++q) {
    const float x = pval[r * parts + q];
    const int cx = pcol[r * parts + q];
    if (better(x, cx, bv, bc)) {
      bv = x;
      bc = cx;
    }
  }
  return bc;
}

__global__ void argmax_final_kernel(const float* pval, const int32_t* pcol, int64_t rows,
                                    int64_t parts, int64_t* out) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r < rows) out[r] = row_argmax(pval, pcol, r, parts);
}

// One wave per request: lane i < k+1 owns row (b, i); the evaluation of
// mtp_engine.py:553-560 runs on ballots and shuffles.
__global__ void __launch_bounds__(256) greedy_eval_kernel(
    const int64_t* draft, const int64_t* target_ids, const float* pval, const int32_t* pcol,
    int64_t parts, int B, int k, int64_t eos, int mode, int64_t* bonus, int64_t* accept,
    uint8_t* eos_acc) {
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (b >= B) return;
  const int i = threadIdx.x & 63;
  int64_t pred = -1;
  if (i <= k) {
    const int64_t r = (int64_t)b * (k + 1) + i;
    pred = target_ids ? target_ids[r] : row_argmax(pval, pcol, r, parts);
  }
  const int64_t d = i < k ? draft[(int64_t)b * k + i] : -2;
  const bool flag = i < k && pred == d;
  const uint64_t fl = __builtin_amdgcn_ballot_w64(flag);
  uint64_t counted;
  if (mode == 0) {
    counted = fl;
  } else {
    // longest matching prefix: the run of ones from bit 0
    const uint64_t miss = ~fl;
    const int first_miss = miss ? __builtin_ctzll(miss) : 64;
    counted = first_miss >= 64 ? fl : (fl & ((1ull << first_miss) - 1));
  }
  const int n = __builtin_popcountll(counted);
  const bool my_counted = (counted >> i) & 1ull;
  const uint64_t eh = __builtin_amdgcn_ballot_w64(my_counted && d == eos);
  const int64_t bonus_v = __shfl(pred, n);
  if (i == 0) {
    accept[b] = n + 1;
    bonus[b] = bonus_v;
    eos_acc[b] = eh ? 1 : 0;
  }
}

// Greedy acceptance evaluated inside the page-table delete that consumes its accept
// counts (the verify step's next operation: delete_kv(n_inserted - accept_nums)), one
// workgroup of pt::kThreads threads.  The waves evaluate the requests, packed: lane l of
// a wave holds request slot l / (k+1) and row l % (k+1), so a wave covers 64 / (k+1)
// requests per round (12 at k = 4) and every request of the step is evaluated in one
// round of partial loads; the accept counts stay in LDS for the delete, which is
// page_table_kernel's update (page_update.h) with d_r = n_inserted - accept_r.
constexpr int kFusedMaxBatch = 8192;

__global__ void __launch_bounds__(pt::kThreads) greedy_eval_delete_kernel(
    const int64_t* draft, const int64_t* target_ids, const float* pval, const int32_t* pcol,
    int64_t parts, int B, int k, int64_t eos, int mode, int64_t* bonus, int64_t* accept,
    uint8_t* eos_acc, int32_t n_inserted, pt::Args pa) {
  __shared__ int32_t s_acc[kFusedMaxBatch];
  constexpr int NW = pt::kThreads / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int R = k + 1;
  const int per_wave = 64 / R;
  const int slot = lane / R;
  const int i = lane - slot * R;
  const int sbit = slot * R;  // <= 63
  const uint64_t seg_mask = R >= 64 ? ~0ull : ((1ull << R) - 1);
  for (int b0 = wave * per_wave; b0 < B; b0 += NW * per_wave) {
    const int b = b0 + slot;
    const bool active = slot < per_wave && b < B;
    int64_t pred = -1;
    if (active) {
      const int64_t r = (int64_t)b * R + i;
      pred = target_ids ? target_ids[r] : row_argmax(pval, pcol, r, parts);
    }
    const int64_t d = active && i < k ? draft[(int64_t)b * k + i] : -2;
    const bool flag = active && i < k && pred == d;
    const uint64_t seg = (__builtin_amdgcn_ballot_w64(flag) >> sbit) & seg_mask;
    int n;
    uint64_t counted;
    if (mode == 0) {
      counted = seg;
      n = __builtin_popcountll(seg);
    } else {
      // longest matching prefix: the run of ones from the request's row 0
      const uint64_t miss = ~seg;
      n = miss ? __builtin_ctzll(miss) : 64;
      counted = n >= 64 ? ~0ull : ((1ull << n) - 1);
    }
    const bool my_counted = i < 64 && ((counted >> i) & 1ull);
    const uint64_t eh =
        (__builtin_amdgcn_ballot_w64(active && my_counted && d == eos) >> sbit) & seg_mask;
    const int64_t bonus_v = __shfl(pred, min(sbit + n, 63));
    if (active && i == 0) {
      accept[b] = n + 1;
      bonus[b] = bonus_v;
      eos_acc[b] = eh ? 1 : 0;
      s_acc[b] = n + 1;
    }
  }
  lds_barrier();  // (s_acc; the output stores need not land first)
  pt::update_pages(pa, [&](int r) -> int32_t { return n_inserted - s_acc[r]; });
}

static int elem_bytes_of(int dtype) { return dtype == BSX_DTYPE_FP32 ? 4 : 2; }

static int dispatch_argmax_parts(const void* logits, int dtype, int64_t rows, int64_t V,
                                 int64_t stride, const ArgmaxSplit& sp, float* pv, int32_t* pc,
                                 hipStream_t st) {
  const dim3 grid((unsigned)(rows * sp.parts));
  switch (dtype) {
    case BSX_DTYPE_BF16:
      hipLaunchKernelGGL((argmax_part_kernel<BSX_DTYPE_BF16>), grid, dim3(kArgmaxThreads), 0, st,
                         logits, V, stride, sp.parts, sp.chunk, pv, pc);
      break;
    case BSX_DTYPE_FP16:
      hipLaunchKernelGGL((argmax_part_kernel<BSX_DTYPE_FP16>), grid, dim3(kArgmaxThreads), 0, st,
                         logits, V, stride, sp.parts, sp.chunk, pv, pc);
      break;
    case BSX_DTYPE_FP32:
      hipLaunchKernelGGL((argmax_part_kernel<BSX_DTYPE_FP32>), grid, dim3(kArgmaxThreads), 0, st,
                         logits, V, stride, sp.parts, sp.chunk, pv, pc);
      break;
    default:
      set_error("unknown dtype %d", dtype);
      return BSX_ERR_INVALID;
  }
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace acc
}  // namespace bsx

using namespace bsx;

// Partials of one (row, part) pair each; sized for fp32 logits, whose split has the
// most parts, so one workspace serves every dtype.
static int64_t argmax_partials(int64_t rows, int64_t vocab) {
  return rows * acc::argmax_split(rows, vocab, 4).parts;
}

// Workspace: [partial values][partial columns].
static int64_t argmax_values_offset() { return 0; }
static int64_t argmax_columns_offset(int64_t rows, int64_t vocab) {
  return acc::align256(argmax_partials(rows, vocab) * 4);
}

extern "C" int64_t bsx_argmax_ws_bytes(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 256;
  return argmax_columns_offset(rows, vocab) + argmax_partials(rows, vocab) * 4;
}

extern "C" int bsx_argmax(const void* logits_d, int dtype, int64_t rows, int64_t vocab,
                          int64_t row_stride, int64_t* out_d, void* ws_d, int64_t ws_bytes,
                          void* stream) {
  BSX_REQUIRE(rows >= 0 && vocab > 0 && vocab < (1LL << 31), BSX_ERR_INVALID,
              "bad shape rows=%lld vocab=%lld", (long long)rows, (long long)vocab);
  if (rows == 0) return BSX_OK;
  BSX_REQUIRE(logits_d && out_d && ws_d, BSX_ERR_INVALID, "null pointer");
  BSX_REQUIRE(row_stride >= vocab, BSX_ERR_INVALID, "row_stride smaller than vocab");
  BSX_REQUIRE(ws_bytes >= bsx_argmax_ws_bytes(rows, vocab), BSX_ERR_CAPACITY,
              "argmax workspace too small");
  BSX_REQUIRE(dtype == BSX_DTYPE_BF16 || dtype == BSX_DTYPE_FP16 || dtype == BSX_DTYPE_FP32,
              BSX_ERR_INVALID, "unknown dtype %d", dtype);
  const acc::ArgmaxSplit sp = acc::argmax_split(rows, vocab, acc::elem_bytes_of(dtype));
  BSX_REQUIRE(rows * sp.parts < (1LL << 31), BSX_ERR_UNSUPPORTED, "too many rows for one launch");
  float* pv = reinterpret_cast<float*>(static_cast<char*>(ws_d) + argmax_values_offset());
  int32_t* pc = reinterpret_cast<int32_t*>(static_cast<char*>(ws_d) +
                                           argmax_columns_offset(rows, vocab));
  hipStream_t st = as_stream(stream);
  int rc = acc::dispatch_argmax_parts(logits_d, dtype, rows, vocab, row_stride, sp, pv, pc, st);
  if (rc != BSX_OK) return rc;
  hipLaunchKernelGGL(acc::argmax_final_kernel, dim3((unsigned)ceil_div(rows, 256)), dim3(256), 0,
                     st, pv, pc, rows, sp.parts, out_d);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

extern "C" int64_t bsx_accept_greedy_ws_bytes(int B, int k, int64_t vocab) {
  return bsx_argmax_ws_bytes((int64_t)B * (k + 1), vocab);
}

extern "C" int bsx_accept_greedy(const int64_t* draft_d, const int64_t* target_ids_d,
                                 const void* target_logits_d, int dtype, int B, int k,
                                 int64_t vocab, int64_t eos_id, int mode, int64_t* bonus_d,
                                 int64_t* accept_d, uint8_t* eos_acc_d, void* ws_d,
                                 int64_t ws_bytes, void* stream) {
  BSX_REQUIRE(B >= 0 && k >= 0 && k <= 63, BSX_ERR_INVALID, "bad B=%d / k=%d (k <= 63)", B, k);
  BSX_REQUIRE(mode == 0 || mode == 1, BSX_ERR_INVALID, "mode must be 0 or 1");
  if (B == 0) return BSX_OK;
  BSX_REQUIRE(bonus_d && accept_d && eos_acc_d && (k == 0 || draft_d), BSX_ERR_INVALID,
              "null pointer");
  BSX_REQUIRE(target_ids_d || target_logits_d, BSX_ERR_INVALID, "need target ids or logits");
  hipStream_t st = as_stream(stream);
  const int64_t rows = (int64_t)B * (k + 1);
  float* pv = nullptr;
  int32_t* pc = nullptr;
  acc::ArgmaxSplit sp = {1, 8};
  if (!target_ids_d) {
    BSX_REQUIRE(vocab > 0 && vocab < (1LL << 31), BSX_ERR_INVALID, "vocab must be in (0, 2^31)");
    BSX_REQUIRE(ws_d && ws_bytes >= bsx_accept_greedy_ws_bytes(B, k, vocab), BSX_ERR_CAPACITY,
                "greedy workspace too small");
    BSX_REQUIRE(dtype == BSX_DTYPE_BF16 || dtype == BSX_DTYPE_FP16 || dtype == BSX_DTYPE_FP32,
                BSX_ERR_INVALID, "unknown dtype %d", dtype);
    sp = acc::argmax_split(rows, vocab, acc::elem_bytes_of(dtype));
    BSX_REQUIRE(rows * sp.parts < (1LL << 31), BSX_ERR_UNSUPPORTED, "too many rows for one launch");
    pv = reinterpret_cast<float*>(static_cast<char*>(ws_d) + argmax_values_offset());
    pc = reinterpret_cast<int32_t*>(static_cast<char*>(ws_d) + argmax_columns_offset(rows, vocab));
    int rc = acc::dispatch_argmax_parts(target_logits_d, dtype, rows, vocab, vocab, sp, pv, pc, st);
    if (rc != BSX_OK) return rc;
  }
  hipLaunchKernelGGL(acc::greedy_eval_kernel, dim3((unsigned)ceil_div(B, 4)), dim3(256), 0, st,
                     draft_d, target_ids_d, pv, pc, sp.parts, B, k, eos_id, mode, bonus_d,
                     accept_d, eos_acc_d);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

extern "C" int bsx_accept_greedy_delete(
    const int64_t* draft_d, const int64_t* target_ids_d, const void* target_logits_d, int dtype,
    int B, int k, int64_t vocab, int64_t eos_id, int mode, int64_t* bonus_d, int64_t* accept_d,
    uint8_t* eos_acc_d, void* ws_d, int64_t ws_bytes, int32_t n_inserted, int32_t* num_pages_d,
    int32_t* last_len_d, int32_t* cachelens_d, int page_size, int max_pages, int32_t* indptr_d,
    int32_t* indices_d, void* stream) {
  BSX_REQUIRE(B >= 0 && k >= 0 && k <= 63, BSX_ERR_INVALID, "bad B=%d / k=%d (k <= 63)", B, k);
  BSX_REQUIRE(mode == 0 || mode == 1, BSX_ERR_INVALID, "mode must be 0 or 1");
  if (B == 0) return BSX_OK;
  BSX_REQUIRE(B <= acc::kFusedMaxBatch, BSX_ERR_UNSUPPORTED,
              "the fused acceptance + delete takes at most %d requests (got %d)",
              acc::kFusedMaxBatch, B);
  BSX_REQUIRE(n_inserted >= k + 1, BSX_ERR_INVALID,
              "n_inserted (%d) must cover the k + 1 = %d verified tokens", n_inserted, k + 1);
  BSX_REQUIRE(bonus_d && accept_d && eos_acc_d && (k == 0 || draft_d), BSX_ERR_INVALID,
              "null pointer");
  BSX_REQUIRE(target_ids_d || target_logits_d, BSX_ERR_INVALID, "need target ids or logits");
  BSX_REQUIRE(page_size > 0 && max_pages > 0, BSX_ERR_INVALID, "bad page_size or max_pages");
  BSX_REQUIRE((int64_t)B * max_pages < (1LL << 31), BSX_ERR_UNSUPPORTED, "page table too large");
  BSX_REQUIRE(num_pages_d && last_len_d && indptr_d && indices_d, BSX_ERR_INVALID,
              "null page-table pointer");
  hipStream_t st = as_stream(stream);
  const int64_t rows = (int64_t)B * (k + 1);
  float* pv = nullptr;
  int32_t* pc = nullptr;
  acc::ArgmaxSplit sp = {1, 8};
  if (!target_ids_d) {
    BSX_REQUIRE(vocab > 0 && vocab < (1LL << 31), BSX_ERR_INVALID, "vocab must be in (0, 2^31)");
    BSX_REQUIRE(ws_d && ws_bytes >= bsx_accept_greedy_ws_bytes(B, k, vocab), BSX_ERR_CAPACITY,
                "greedy workspace too small");
    BSX_REQUIRE(dtype == BSX_DTYPE_BF16 || dtype == BSX_DTYPE_FP16 || dtype == BSX_DTYPE_FP32,
                BSX_ERR_INVALID, "unknown dtype %d", dtype);
    sp = acc::argmax_split(rows, vocab, acc::elem_bytes_of(dtype));
    BSX_REQUIRE(rows * sp.parts < (1LL << 31), BSX_ERR_UNSUPPORTED, "too many rows for one launch");
    pv = reinterpret_cast<float*>(static_cast<char*>(ws_d) + argmax_values_offset());
    pc = reinterpret_cast<int32_t*>(static_cast<char*>(ws_d) + argmax_columns_offset(rows, vocab));
    int rc = acc::dispatch_argmax_parts(target_logits_d, dtype, rows, vocab, vocab, sp, pv, pc, st);
    if (rc != BSX_OK) return rc;
  }
  pt::Args pa;
  pa.num_pages = num_pages_d;
  pa.last_len = last_len_d;
  pa.cachelens = cachelens_d;
  pa.d = nullptr;
  pa.d_scalar = 0;
  pa.sign = -1;
  pa.B = B;
  pa.page_size = page_size;
  pa.max_pages = max_pages;
  pa.indptr = indptr_d;
  pa.indices = indices_d;
  pa.errors = nullptr;  // a delete never exceeds the page budget
  hipLaunchKernelGGL(acc::greedy_eval_delete_kernel, dim3(1), dim3(pt::kThreads), 0, st, draft_d,
                     target_ids_d, pv, pc, sp.parts, B, k, eos_id, mode, bonus_d, accept_d,
                     eos_acc_d, n_inserted, pa);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

// ---- greedy acceptance without a caller workspace ----------------------------------
// The argmax partials live in a file-scope device array (one copy per GPU, held until
// the process ends).  Host code never passes the array's name to a kernel: its device
// address is looked up once per device with hipGetSymbolAddress, with that device
// current, and kept in g_scratch_addr.  Calls on one GPU share the array, so calls
// that overlap in time on one GPU (different streams without ordering) race; the
// partials are fully written before they are read, so nothing in it must start at zero.
namespace {
constexpr int kMaxScratchDevices = 64;
__device__ __align__(256) unsigned char scratch[BSX_NOALLOC_SCRATCH_BYTES];
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxScratchDevices];
}  // namespace

static int scratch_address(void** out) {
  int dev = -1;
  BSX_HIP_CHECK(hipGetDevice(&dev));
  BSX_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, BSX_ERR_UNSUPPORTED,
              "device %d beyond the %d devices the allocation-free scratch supports", dev,
              kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    BSX_REQUIRE(e == hipSuccess && p != nullptr, BSX_ERR_HIP,
                "hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return BSX_OK;
}

extern "C" int bsx_accept_greedy_noalloc(const int64_t* draft_d, const int64_t* target_ids_d,
                                         const void* target_logits_d, int dtype, int B, int k,
                                         int64_t vocab, int64_t eos_id, int mode,
                                         int64_t* bonus_d, int64_t* accept_d,
                                         uint8_t* eos_acc_d, void* stream) {
  if (target_ids_d == nullptr && B > 0 && k >= 0 && vocab > 0) {
    const int64_t need = bsx_accept_greedy_ws_bytes(B, k, vocab);
    BSX_REQUIRE(need <= (int64_t)BSX_NOALLOC_SCRATCH_BYTES, BSX_ERR_CAPACITY,
                "B=%d k=%d vocab=%lld needs %lld bytes of argmax partials; the "
                "allocation-free scratch holds %lld (use bsx_accept_greedy with a workspace)",
                B, k, (long long)vocab, (long long)need, (long long)BSX_NOALLOC_SCRATCH_BYTES);
  }
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != BSX_OK) return rc;
  return bsx_accept_greedy(draft_d, target_ids_d, target_logits_d, dtype, B, k, vocab, eos_id,
                           mode, bonus_d, accept_d, eos_acc_d, ws,
                           (int64_t)BSX_NOALLOC_SCRATCH_BYTES, stream);
}

static int64_t chain_ws_layout(int B, int k, int64_t V, bool logits, int64_t* off_lanes,
                               int64_t* off_dec) {
  (void)V;
  const int64_t rows = (int64_t)B * (2 * k + 1);
  const int64_t stats = logits ? acc::align256(rows * 8) : 0;
  *off_lanes = stats;
  *off_dec = stats + acc::align256((int64_t)B * canon::kLanes * 4);
  return *off_dec + acc::align256((int64_t)B * 8);
}

extern "C" int64_t bsx_chain_ws_bytes(int B, int k, int64_t vocab) {
  int64_t a, b;
  return chain_ws_layout(B, k, vocab, true, &a, &b);
}

template <int DT, bool LOGITS>
static int launch_chain(acc::ChainArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((acc::residual_kernel<DT, LOGITS>), dim3(a.B, 8), dim3(256), 0, st, a);
  BSX_LAUNCH_CHECK();
  hipLaunchKernelGGL((acc::pick_kernel<DT, LOGITS>), dim3(a.B), dim3(256), 0, st, a);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

static int check_chain_common(const int64_t* draft_ids_d, const float* uniforms_d, int B, int k,
                              int64_t vocab, int32_t* out_ids_d, int32_t* accepted_d,
                              int32_t* emitted_d) {
  BSX_REQUIRE(B >= 0 && k >= 0 && vocab > 0, BSX_ERR_INVALID, "bad B=%d k=%d vocab=%lld", B, k,
              (long long)vocab);
  BSX_REQUIRE(vocab < (1LL << 31), BSX_ERR_UNSUPPORTED, "vocab too large");
  if (B == 0) return BSX_OK;
  BSX_REQUIRE(uniforms_d && out_ids_d && accepted_d && emitted_d && (k == 0 || draft_ids_d),
              BSX_ERR_INVALID, "null pointer");
  return BSX_OK;
}

extern "C" int bsx_chain_speculative_sampling(const float* draft_probs_d,
                                              const int64_t* draft_ids_d,
                                              const float* target_probs_d,
                                              const float* uniforms_d, int B, int k,
                                              int64_t vocab, int32_t* out_ids_d,
                                              int32_t* accepted_d, int32_t* emitted_d, void* ws_d,
                                              int64_t ws_bytes, void* stream) {
  int rc = check_chain_common(draft_ids_d, uniforms_d, B, k, vocab, out_ids_d, accepted_d, emitted_d);
  if (rc != BSX_OK || B == 0) return rc;
  BSX_REQUIRE(target_probs_d, BSX_ERR_INVALID, "null target_probs");
  int64_t off_lanes, off_dec;
  const int64_t need = chain_ws_layout(B, k, vocab, false, &off_lanes, &off_dec);
  BSX_REQUIRE(ws_d && ws_bytes >= need, BSX_ERR_CAPACITY, "chain workspace too small (%lld < %lld)",
              (long long)ws_bytes, (long long)need);
  acc::ChainArgs a{};
  a.t_probs = target_probs_d;
  a.d_probs = draft_probs_d;
  a.draft_ids = draft_ids_d;
  a.uniforms = uniforms_d;
  a.B = B;
  a.k = k;
  a.V = vocab;
  a.lanes = reinterpret_cast<float*>(static_cast<char*>(ws_d) + off_lanes);
  a.dec = reinterpret_cast<int32_t*>(static_cast<char*>(ws_d) + off_dec);
  a.out_ids = out_ids_d;
  a.accepted = accepted_d;
  a.emitted = emitted_d;
  return launch_chain<BSX_DTYPE_FP32, false>(a, as_stream(stream));
}

template <int DT>
static int chain_logits_impl(acc::ChainArgs& a, hipStream_t st) {
  const int64_t n_t = (int64_t)a.B * (a.k + 1);
  const int64_t n_d = a.d_logits ? (int64_t)a.B * a.k : 0;
  float2* stats = const_cast<float2*>(a.stats);
  hipLaunchKernelGGL((acc::stats_kernel<DT>), dim3((unsigned)(n_t + n_d)), dim3(256), 0, st,
                     a.t_logits, n_t, a.d_logits, a.V, a.c, stats);
  BSX_LAUNCH_CHECK();
  return launch_chain<DT, true>(a, st);
}

extern "C" int bsx_chain_speculative_sampling_logits(const void* draft_logits_d,
                                                     const int64_t* draft_ids_d,
                                                     const void* target_logits_d, int dtype,
                                                     float temperature, const float* uniforms_d,
                                                     int B, int k, int64_t vocab,
                                                     int32_t* out_ids_d, int32_t* accepted_d,
                                                     int32_t* emitted_d, void* ws_d,
                                                     int64_t ws_bytes, void* stream) {
  BSX_REQUIRE(row_bytes_ok(vocab, dtype), BSX_ERR_UNSUPPORTED,
              "a row of %lld logits is 2^31 bytes or more", (long long)vocab);
  int rc = check_chain_common(draft_ids_d, uniforms_d, B, k, vocab, out_ids_d, accepted_d, emitted_d);
  if (rc != BSX_OK || B == 0) return rc;
  BSX_REQUIRE(target_logits_d, BSX_ERR_INVALID, "null target_logits");
  BSX_REQUIRE(temperature > 0.f && temperature == temperature, BSX_ERR_INVALID,
              "temperature must be > 0 (greedy acceptance has its own entry point)");
  int64_t off_lanes, off_dec;
  const int64_t need = chain_ws_layout(B, k, vocab, true, &off_lanes, &off_dec);
  BSX_REQUIRE(ws_d && ws_bytes >= need, BSX_ERR_CAPACITY, "chain workspace too small (%lld < %lld)",
              (long long)ws_bytes, (long long)need);
  acc::ChainArgs a{};
  a.t_logits = target_logits_d;
  a.d_logits = draft_logits_d;
  a.stats = static_cast<const float2*>(ws_d);
  a.c = canon::scale_for_temperature(temperature);
  a.draft_ids = draft_ids_d;
  a.uniforms = uniforms_d;
  a.B = B;
  a.k = k;
  a.V = vocab;
  a.lanes = reinterpret_cast<float*>(static_cast<char*>(ws_d) + off_lanes);
  a.dec = reinterpret_cast<int32_t*>(static_cast<char*>(ws_d) + off_dec);
  a.out_ids = out_ids_d;
  a.accepted = accepted_d;
  a.emitted = emitted_d;
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case BSX_DTYPE_BF16: return chain_logits_impl<BSX_DTYPE_BF16>(a, st);
    case BSX_DTYPE_FP16: return chain_logits_impl<BSX_DTYPE_FP16>(a, st);
    case BSX_DTYPE_FP32: return chain_logits_impl<BSX_DTYPE_FP32>(a, st);
  }
  set_error("unknown dtype %d", dtype);
  return BSX_ERR_INVALID;
}

extern "C" int64_t bsx_softmax_ws_bytes(int64_t rows) { return acc::align256(rows * 8); }

template <int DT>
static int softmax_impl(const void* logits, int64_t rows, int64_t V, float c, float* probs,
                        float2* stats, hipStream_t st) {
  hipLaunchKernelGGL((acc::stats_kernel<DT>), dim3((unsigned)rows), dim3(256), 0, st, logits,
                     rows, nullptr, V, c, stats);
  BSX_LAUNCH_CHECK();
  const int parts = (int)std::min<int64_t>(64, std::max<int64_t>(1, ceil_div(V, 4096)));
  hipLaunchKernelGGL((acc::softmax_norm_kernel<DT>), dim3((unsigned)rows, parts), dim3(256), 0, st,
                     logits, V, c, stats, probs);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

extern "C" int bsx_softmax(const void* logits_d, int dtype, float temperature, int64_t rows,
                           int64_t vocab, float* probs_d, void* ws_d, int64_t ws_bytes,
                           void* stream) {
  BSX_REQUIRE(rows >= 0 && vocab > 0, BSX_ERR_INVALID, "bad shape");
  BSX_REQUIRE(row_bytes_ok(vocab, dtype), BSX_ERR_UNSUPPORTED,
              "a row of %lld logits is 2^31 bytes or more", (long long)vocab);
  if (rows == 0) return BSX_OK;
  BSX_REQUIRE(logits_d && probs_d && ws_d, BSX_ERR_INVALID, "null pointer");
  BSX_REQUIRE(temperature > 0.f, BSX_ERR_INVALID, "temperature must be > 0");
  BSX_REQUIRE(ws_bytes >= bsx_softmax_ws_bytes(rows), BSX_ERR_CAPACITY, "softmax workspace too small");
  const float c = canon::scale_for_temperature(temperature);
  float2* stats = static_cast<float2*>(ws_d);
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case BSX_DTYPE_BF16: return softmax_impl<BSX_DTYPE_BF16>(logits_d, rows, vocab, c, probs_d, stats, st);
    case BSX_DTYPE_FP16: return softmax_impl<BSX_DTYPE_FP16>(logits_d, rows, vocab, c, probs_d, stats, st);
    case BSX_DTYPE_FP32: return softmax_impl<BSX_DTYPE_FP32>(logits_d, rows, vocab, c, probs_d, stats, st);
  }
  set_error("unknown dtype %d", dtype);
  return BSX_ERR_INVALID;
}
