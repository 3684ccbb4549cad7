// Top-k / top-p renormalisation fused into acceptance and sampling.
//
// Replaces, for top-p and/or top-k on:
//   * get_sampling_probs (batchspec/backends/utils/sampling.py:18-58): softmax(x/T),
//     then top-p renorm if top_p > 0 (:51-52), then top-k renorm if top_k > 0 (:55-56);
//   * the non-greedy sample() (:61-115), with an explicit uniform per row;
//   * the sampling branch of MTPEngine.evaluate_posterior
//     (batchspec/backends/mtp_engine.py:561-575) fed those filtered distributions.
//
// The filtered distribution of a row is defined exactly (the CPU restatement computes
// the same bits):
//   (M, Z)  canonical row statistics (canon.h), C = log2(e)/T;
//   w(x) = exp2(fma(x, C, -(M*C))),  m(x) = trunc(w(x) * 2^40) as a 64-bit integer;
//   key(x)  order-preserving 32-bit image of x;
//   top-k is on iff 0 < top_k < V, top-p iff 0 < top_p < 1;
//   target = ceil(fl(top_p * Z) * 2^40);
//   walking the distinct keys downwards with cnt / mass = number / sum of m of the
//   elements at or above the key, t* is the first key where (top-k on and
//   cnt >= top_k) or (top-p on and mass >= target); the smallest key if none is;
//   Z_K = float(mass at t*) * 2^-40 (round to nearest even);
//   p'(x) = key(x) >= t* ? w(x) / Z_K : 0   (computed as w(x) * (1/Z_K)).
// That is the reference's order: the nucleus is cut on the full distribution, top-k
// on the renormalised one, and the result keeps the smaller of the two upper sets;
// ties at the threshold are kept.  Integer counts and masses make the threshold
// independent of the reduction order, so no canonical tree is needed here.
//
// Draws are an inverse CDF over fixed-point weights r_fx = trunc(r * 2^40) in
// ascending vocabulary order: t = floor(u * total) (binary64), the first index whose
// running sum exceeds t (the last non-zero index if none does).
//
// Kernels:
//   filter_rows_kernel: one 256-thread workgroup per row.
//     1. canonical (M, Z), keeping the 2048 lane maxima;
//     2. a lower bound L of t*: the k-th largest lane maximum is at most the k-th
//        largest element, so the lower edge of its 12-bit key bin bounds t* from
//        below (for top-p alone the bound of rank 64 is used and checked afterwards);
//     3. the row is read again (the first pass left it in the memory-side cache) and
//        the elements >= L are listed in LDS;
//     4. with at most kCap of them, every listed element gets its count and mass of
//        listed elements at or above it (all of the row's elements there are listed),
//        which gives t* and Z_K exactly; the kept elements are written out;
//     5. otherwise (ties, a large k, a wide nucleus), an exact radix select over the
//        key bits, 8 per pass, with counts and fixed-point masses per digit in LDS,
//        and the row gets no list.
//   filter_chain_kernel: one workgroup per request: the ratio tests, then the draw
//     from the row the chain stops at, over its kept list, or over the whole row in
//     contiguous chunks when it has none.
//   filtered_probs_kernel: p'(x) for every element (get_sampling_probs).
#include <limits.h>

#include <algorithm>

#include "bsx.h"
#include "common.h"
#include "canon.h"
#include "rows.h"

namespace bsx {
namespace filt {

using acc::load_one;
using canon::fx40;
using canon::key_value;
using canon::okey;

constexpr int kThreads = 256;
constexpr int kCap = 256;         // listed candidates per row (fast path)
constexpr int kTopPProbe = 64;    // rank of the lane-maximum bound for top-p alone
constexpr int kBinShift = 20;     // 12-bit key bins for the bound
constexpr int kBins = 1 << (32 - kBinShift);
constexpr int kFirstFiniteBin = 8;  // bins below hold -inf and NaN images only
static_assert(kCap <= kThreads, "one listed candidate per thread");

struct RowInfo {
  float m;        // row max M
  float inv_k;    // 1 / Z_K
  uint32_t t_key; // threshold key t*
  int32_t n_list; // kept elements listed, or -1 (no list)
};

struct RowsArgs {
  const void* a;  // rows [0, n_a)
  int64_t n_a;
  const void* b;  // rows [n_a, ...)
  int64_t V;
  float c;
  int top_k;      // <= 0 or >= V: off
  float top_p;    // <= 0 or >= 1: off
  RowInfo* info;
  int32_t* lists; // [rows][kCap]
};

__device__ __forceinline__ bool reached(bool use_k, bool use_p, uint32_t cnt, uint64_t mass,
                                        int top_k, uint64_t target) {
  return (use_k && cnt >= (uint32_t)top_k) || (use_p && mass >= target);
}

// Bits of the key that vary for each logit type (the rest are constant for a sign):
// bf16 16, fp16 19 (24 after rounding up to whole passes), fp32 32.
template <int DT>
constexpr int radix_passes() {
  return DT == BSX_DTYPE_BF16 ? 2 : (DT == BSX_DTYPE_FP16 ? 3 : 4);
}

// Calls f(x, v) for every element of the row (16-byte loads when vec).
template <int DT, typename F>
__device__ __forceinline__ void for_each_element(const void* row, int64_t V, bool vec, F&& f) {
  constexpr int EPV = DT == BSX_DTYPE_FP32 ? 4 : 8;
  const int t = threadIdx.x;
  int64_t done = 0;
  if (vec) {
    const int64_t nv = V / EPV;
    const u32x4* p = static_cast<const u32x4*>(row);
    constexpr int U = 4;
    for (int64_t v0 = t; v0 < nv; v0 += (int64_t)kThreads * U) {
      u32x4 w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = v0 + (int64_t)kThreads * u;
        w[u] = p[i < nv ? i : v0];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t i = v0 + (int64_t)kThreads * u;
        if (i < nv) {
#pragma unroll
          for (int e = 0; e < EPV; ++e) {
            float x;
            if constexpr (DT == BSX_DTYPE_FP32) x = __uint_as_float(w[u][e]);
            else x = (e & 1) ? hi_f32<DT>(w[u][e >> 1]) : lo_f32<DT>(w[u][e >> 1]);
            f(x, i * EPV + e);
          }
        }
      }
    }
    done = nv * EPV;
  }
  for (int64_t v = done + t; v < V; v += kThreads) f(load_one<DT>(row, v), v);
}

template <int DT>
__global__ void __launch_bounds__(kThreads) filter_rows_kernel(RowsArgs a) {
  __shared__ __align__(16) uint32_t hist[kBins];  // bound histogram; reused by the radix select
  __shared__ uint32_t part[kThreads];
  __shared__ uint32_t ckey[kCap];
  __shared__ int32_t cidx[kCap];
  __shared__ uint64_t cmass[kCap];
  __shared__ float s_m, s_z;
  __shared__ int s_bin, s_count, s_nk;
  __shared__ uint32_t s_t;
  __shared__ uint64_t s_zk;

  const int t = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int64_t V = a.V;
  const size_t esz = DT == BSX_DTYPE_FP32 ? 4 : 2;
  const char* row = r < a.n_a ? static_cast<const char*>(a.a) + r * V * esz
                              : static_cast<const char*>(a.b) + (r - a.n_a) * V * esz;
  const bool vec = ((V * esz) % 16 == 0) && (((uintptr_t)row) % 16 == 0);
  const float c = a.c;
  const bool use_k = a.top_k > 0 && (int64_t)a.top_k < V;
  const bool use_p = a.top_p > 0.f && a.top_p < 1.f;

  // 1. canonical statistics and lane maxima
  float lm[8];
  acc::row_stats<DT, true>(row, V, vec, c, &s_m, &s_z, lm);
  const float M = s_m, Z = s_z;
  const float neg = -(M * c);
  const uint64_t target = use_p ? (uint64_t)ceilf((a.top_p * Z) * 0x1p40f) : 0ull;

  // 2. bound: the lower edge of the bin of the k_eff-th largest lane maximum
  const int k_eff = use_k ? a.top_k : kTopPProbe;
  for (int i = t; i < kBins; i += kThreads) hist[i] = 0u;
  if (t == 0) {
    s_count = 0;
    s_nk = 0;
    s_t = 0u;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) atomicAdd(&hist[okey(lm[i]) >> kBinShift], 1u);
  __syncthreads();
  {
    uint32_t ps = 0;
    for (int i = 0; i < kBins / kThreads; ++i) ps += hist[t * (kBins / kThreads) + i];
    part[t] = ps;
  }
  __syncthreads();
  if (t < 64) {
    // lane l: bins [64 l, 64 l + 64); inclusive suffix sums over lanes
    const uint32_t q = part[4 * t] + part[4 * t + 1] + part[4 * t + 2] + part[4 * t + 3];
    uint32_t s = q;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = __shfl_down(s, d);
      if (t + d < 64) s += o;
    }
    const uint64_t mask = __builtin_amdgcn_ballot_w64(k_eff <= 2048 && s >= (uint32_t)k_eff);
    const int ls = mask ? 63 - __builtin_clzll(mask) : -1;
    if (ls < 0) {
      if (t == 0) s_bin = -1;
    } else if (t == ls) {
      uint32_t cum = s - q;
      int bin = 64 * t;
      for (int i = 64 * t + 63; i >= 64 * t; --i) {
        cum += hist[i];
        if (cum >= (uint32_t)k_eff) {
          bin = i;
          break;
        }
      }
      s_bin = bin;
    }
  }
  __syncthreads();
  const bool all = s_bin < kFirstFiniteBin;
  const float lf = all ? -INFINITY : key_value((uint32_t)s_bin << kBinShift);

  // 3./4. list the elements >= L and walk them
  bool listed = false;
  if (!all || V <= kCap) {
    for_each_element<DT>(row, V, vec, [&](float x, int64_t v) {
      if (x >= lf) {
        const int slot = atomicAdd(&s_count, 1);
        if (slot < kCap) {
          ckey[slot] = okey(x);
          cidx[slot] = (int32_t)v;
        }
      }
    });
    __syncthreads();
    const int n = s_count;
    if (n <= kCap) {
      uint32_t key = 0u;
      uint64_t mass = 0ull;
      if (t < n) {
        key = ckey[t];
        cmass[t] = fx40(canon::weight(key_value(key), c, neg));
      }
      __syncthreads();
      if (t < n) {
        uint32_t cnt = 0u;
        for (int q = 0; q < n; ++q) {
          if (ckey[q] >= key) {
            ++cnt;
            mass += cmass[q];
          }
        }
        if (reached(use_k, use_p, cnt, mass, a.top_k, target)) atomicMax(&s_t, key);
      }
      __syncthreads();
      const uint32_t tk = s_t;
      // a finite element's key is never 0: 0 means no listed key reached the target
      // (top-p alone with the nucleus below the bound)
      if (tk != 0u) {
        if (t < n && key == tk) s_zk = mass;  // equal keys hold equal masses
        if (t < n && key >= tk) {
          const int slot = atomicAdd(&s_nk, 1);
          a.lists[r * kCap + slot] = cidx[t];
        }
        __syncthreads();
        listed = true;
      }
    }
  }

  // 5. exact radix select
  if (!listed) {
    uint32_t* hc = hist;                                  // [256]
    uint64_t* hm = reinterpret_cast<uint64_t*>(hist + 256);  // [256]
    __shared__ uint32_t s_prefix, s_above_c;
    __shared__ uint64_t s_above_m;
    constexpr int NP = radix_passes<DT>();
    if (t == 0) {
      s_prefix = 0u;
      s_above_c = 0u;
      s_above_m = 0ull;
    }
    for (int pass = 0; pass < NP; ++pass) {
      const int shift = 24 - 8 * pass;
      hc[t] = 0u;
      hm[t] = 0ull;
      __syncthreads();
      const uint32_t prefix = s_prefix;
      for_each_element<DT>(row, V, vec, [&](float x, int64_t) {
        const uint32_t key = okey(x);
        if (pass == 0 || (key >> (shift + 8)) == prefix) {
          const uint32_t d = (key >> shift) & 255u;
          atomicAdd(&hc[d], 1u);
          const uint64_t m = fx40(canon::weight(x, c, neg));
          if (m != 0ull) atomicAdd(reinterpret_cast<unsigned long long*>(&hm[d]),
                                   (unsigned long long)m);
        }
      });
      __syncthreads();
      if (t == 0) {
        uint32_t cum_c = s_above_c;
        uint64_t cum_m = s_above_m;
        int chosen = -1;
        uint32_t ch_prev_c = 0u, ch_c = 0u;
        uint64_t ch_prev_m = 0ull, ch_m = 0ull;
        for (int d = 255; d >= 0; --d) {
          if (hc[d] == 0u) continue;
          const uint32_t pc = cum_c;
          const uint64_t pm = cum_m;
          cum_c += hc[d];
          cum_m += hm[d];
          chosen = d;  // the lowest non-empty digit so far
          ch_prev_c = pc;
          ch_prev_m = pm;
          ch_c = cum_c;
          ch_m = cum_m;
          if (reached(use_k, use_p, cum_c, cum_m, a.top_k, target)) break;
        }
        s_prefix = (pass == 0 ? 0u : (prefix << 8)) | (uint32_t)chosen;
        s_above_c = ch_prev_c;
        s_above_m = ch_prev_m;
        s_zk = ch_m;
        (void)ch_c;
      }
      __syncthreads();
    }
    if (t == 0) {
      constexpr int low_bits = 32 - 8 * NP;
      uint32_t tk = low_bits == 0 ? s_prefix : (s_prefix << low_bits);
      // the bits below the varying ones are 0 for positive values, 1 for negative
      if (low_bits > 0 && !(tk & 0x80000000u)) tk |= (1u << low_bits) - 1u;
      s_t = tk;
      s_nk = -1;
    }
    __syncthreads();
  }

  if (t == 0) {
    RowInfo ri;
    ri.m = M;
    ri.inv_k = 1.0f / (canon::u64_to_f32(s_zk) * 0x1p-40f);
    ri.t_key = s_t;
    ri.n_list = s_nk;
    a.info[r] = ri;
  }
}

// ----------------------------------------------------------------------------
// Acceptance and draws over filtered rows.
// ----------------------------------------------------------------------------
struct ChainArgs {
  const void* t_logits;  // [B, k+1, V]
  const void* d_logits;  // [B, k, V] or null (one-hot draft)
  const RowInfo* info;   // [B*(k+1)] target rows, then [B*k] draft rows
  const int32_t* lists;
  const int64_t* draft_ids;  // [B, k]
  const float* uniforms;     // [B, k+1]
  int B, k;
  int64_t V;
  float c;
  int32_t* out_ids;  // [B, k+1]
  int32_t* accepted;
  int32_t* emitted;
};

template <int DT>
struct Filtered {
  const void* row;
  float c, nmc, inv;
  uint32_t tk;
  __device__ __forceinline__ float p(int64_t v) const {
    const float x = load_one<DT>(row, v);
    return okey(x) >= tk ? canon::weight(x, c, nmc) * inv : 0.0f;
  }
};

template <int DT>
__device__ __forceinline__ Filtered<DT> filtered_row(const void* base, int64_t row, int64_t V,
                                                     const RowInfo& ri, float c) {
  Filtered<DT> f;
  f.row = static_cast<const char*>(base) + row * V * (DT == BSX_DTYPE_FP32 ? 4 : 2);
  f.c = c;
  f.nmc = -(ri.m * c);
  f.inv = ri.inv_k;
  f.tk = ri.t_key;
  return f;
}

__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, uint64_t* s_acc) {
  if (threadIdx.x == 0) *s_acc = 0ull;
  __syncthreads();
  if (v != 0ull) atomicAdd(reinterpret_cast<unsigned long long*>(s_acc), (unsigned long long)v);
  __syncthreads();
  const uint64_t total = *s_acc;
  __syncthreads();
  return total;
}

template <int DT>
__global__ void __launch_bounds__(kThreads) filter_chain_kernel(ChainArgs a) {
  __shared__ int s_j, s_n, s_tok, s_last;
  __shared__ int32_t lv[kCap];
  __shared__ uint64_t lr[kCap];
  __shared__ uint64_t s_acc;
  __shared__ uint64_t excl[kThreads];
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int k = a.k;
  const int64_t V = a.V;
  const int64_t trow0 = (int64_t)b * (k + 1);
  const int64_t drow0 = (int64_t)a.B * (k + 1) + (int64_t)b * k;

  // ratio tests: lane i of the first wave tests draft position i
  if (t < 64) {
    int j = k, cnt = 0;
    for (int i0 = 0; i0 < k; i0 += 64) {
      const int i = i0 + t;
      bool acc = false;
      if (i < k) {
        const int64_t x = a.draft_ids[(int64_t)b * k + i];
        if (x >= 0 && x < V) {
          const float p = filtered_row<DT>(a.t_logits, trow0 + i, V, a.info[trow0 + i], a.c).p(x);
          const float q = a.d_logits
                              ? filtered_row<DT>(a.d_logits, (int64_t)b * k + i, V,
                                                 a.info[drow0 + i], a.c).p(x)
                              : 1.0f;
          acc = a.uniforms[trow0 + i] * q < p;
        }
      }
      const uint64_t acc_bits = __builtin_amdgcn_ballot_w64(acc);
      const uint64_t rej_bits = __builtin_amdgcn_ballot_w64(i < k && !acc);
      cnt += __builtin_popcountll(acc_bits);
      if (j == k && rej_bits != 0) j = i0 + __builtin_ctzll(rej_bits);
    }
    if (t == 0) {
      s_j = j;
      s_n = cnt;
      s_tok = INT_MAX;
      s_last = -1;
    }
  }
  __syncthreads();
  const int j = s_j;
  const RowInfo ti = a.info[trow0 + j];
  const Filtered<DT> P = filtered_row<DT>(a.t_logits, trow0 + j, V, ti, a.c);
  const bool has_q = j < k;
  const int64_t xj = has_q ? a.draft_ids[(int64_t)b * k + j] : -1;
  Filtered<DT> Q{};
  if (has_q && a.d_logits) Q = filtered_row<DT>(a.d_logits, (int64_t)b * k + j, V, a.info[drow0 + j], a.c);
  auto r_at = [&](int64_t v, bool with_q) -> uint64_t {
    const float p = P.p(v);
    if (!with_q) return fx40(p);
    const float q = a.d_logits ? Q.p(v) : (v == xj ? 1.0f : 0.0f);
    return fx40(fmaxf(p - q, 0.0f));
  };
  const float u = a.uniforms[trow0 + k];
  int tok = -1;
  if (ti.n_list >= 0) {
    const int n = ti.n_list;
    const int32_t v = t < n ? a.lists[(trow0 + j) * kCap + t] : 0;
    uint64_t total = 0ull;
    for (int pass = 0; pass < 2; ++pass) {
      const bool with_q = has_q && pass == 0;
      if (pass == 1 && !has_q) break;
      const uint64_t w = t < n ? r_at(v, with_q) : 0ull;
      if (t < n) {
        lv[t] = v;
        lr[t] = w;
      }
      total = block_sum_u64(w, &s_acc);
      if (total != 0ull) break;
    }
    if (total != 0ull) {
      const uint64_t tp = canon::draw_point(u, total);
      if (t < n && lr[t] != 0ull) {
        uint64_t prefix = 0ull;
        for (int q = 0; q < n; ++q)
          if (lv[q] <= v) prefix += lr[q];
        if (prefix > tp) atomicMin(&s_tok, (int)v);
        atomicMax(&s_last, (int)v);
      }
      __syncthreads();
      tok = s_tok != INT_MAX ? s_tok : s_last;
    }
  } else {
    // no list: the whole row, thread t owning the contiguous chunk [lo, hi)
    const int64_t chunk = ceil_div(V, (int64_t)kThreads);
    const int64_t lo = min((int64_t)t * chunk, V);
    const int64_t hi = min(lo + chunk, V);
    uint64_t total = 0ull;
    bool with_q = has_q;
    uint64_t sum = 0ull;
    for (int pass = 0; pass < 2; ++pass) {
      with_q = has_q && pass == 0;
      if (pass == 1 && !has_q) break;
      sum = 0ull;
      for (int64_t v = lo; v < hi; ++v) sum += r_at(v, with_q);
      excl[t] = sum;
      __syncthreads();
      if (t == 0) {
        uint64_t run = 0ull;
        for (int i = 0; i < kThreads; ++i) {
          const uint64_t s = excl[i];
          excl[i] = run;
          run += s;
        }
        s_acc = run;
      }
      __syncthreads();
      total = s_acc;
      __syncthreads();
      if (total != 0ull) break;
    }
    if (total != 0ull) {
      const uint64_t tp = canon::draw_point(u, total);
      const uint64_t e0 = excl[t];
      if (sum != 0ull) {
        if (tp >= e0 && tp < e0 + sum) {
          uint64_t cum = e0;
          for (int64_t v = lo; v < hi; ++v) {
            cum += r_at(v, with_q);
            if (cum > tp) {
              s_tok = (int)v;
              break;
            }
          }
        }
        int64_t last = -1;
        for (int64_t v = hi - 1; v >= lo; --v)
          if (r_at(v, with_q) != 0ull) {
            last = v;
            break;
          }
        atomicMax(&s_last, (int)last);
      }
      __syncthreads();
      tok = s_tok != INT_MAX ? s_tok : s_last;
    }
  }
  if (t == 0) {
    int32_t* out = a.out_ids + (int64_t)b * (k + 1);
    for (int i = 0; i <= k; ++i) {
      int32_t o = -1;
      if (i < j) o = (int32_t)a.draft_ids[(int64_t)b * k + i];
      else if (i == j) o = tok;
      out[i] = o;
    }
    a.accepted[b] = s_n;
    a.emitted[b] = j;
  }
}

// p'(x) for every element of every row (grid: rows x parts).
template <int DT>
__global__ void __launch_bounds__(kThreads) filtered_probs_kernel(const void* logits, int64_t V,
                                                                  float c, const RowInfo* info,
                                                                  float* probs) {
  const int64_t r = blockIdx.x;
  const Filtered<DT> f = filtered_row<DT>(logits, r, V, info[r], c);
  float* out = probs + r * V;
  for (int64_t v = (int64_t)blockIdx.y * kThreads + threadIdx.x; v < V;
       v += (int64_t)gridDim.y * kThreads)
    out[v] = f.p(v);
}

static int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

}  // namespace filt
}  // namespace bsx

using namespace bsx;

extern "C" int64_t bsx_filter_ws_bytes(int64_t rows) {
  return filt::align256(rows * (int64_t)sizeof(filt::RowInfo)) +
         filt::align256(rows * filt::kCap * 4);
}

static bool filters_on(int top_k, float top_p, int64_t vocab) {
  return (top_k > 0 && (int64_t)top_k < vocab) || (top_p > 0.f && top_p < 1.f);
}

template <int DT>
static int launch_filter_rows(const void* a, int64_t n_a, const void* b, int64_t n_b, int64_t V,
                              float c, int top_k, float top_p, void* ws, hipStream_t st) {
  filt::RowsArgs ra;
  ra.a = a;
  ra.n_a = n_a;
  ra.b = b;
  ra.V = V;
  ra.c = c;
  ra.top_k = top_k;
  ra.top_p = top_p;
  ra.info = static_cast<filt::RowInfo*>(ws);
  ra.lists = reinterpret_cast<int32_t*>(static_cast<char*>(ws) +
                                        filt::align256((n_a + n_b) * (int64_t)sizeof(filt::RowInfo)));
  hipLaunchKernelGGL((filt::filter_rows_kernel<DT>), dim3((unsigned)(n_a + n_b)),
                     dim3(filt::kThreads), 0, st, ra);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

template <int DT>
static int filtered_chain_impl(filt::ChainArgs& ca, void* ws, hipStream_t st, int top_k,
                               float top_p) {
  const int64_t n_t = (int64_t)ca.B * (ca.k + 1);
  const int64_t n_d = ca.d_logits ? (int64_t)ca.B * ca.k : 0;
  int rc = launch_filter_rows<DT>(ca.t_logits, n_t, ca.d_logits, n_d, ca.V, ca.c, top_k, top_p,
                                  ws, st);
  if (rc != BSX_OK) return rc;
  hipLaunchKernelGGL((filt::filter_chain_kernel<DT>), dim3((unsigned)ca.B), dim3(filt::kThreads),
                     0, st, ca);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

extern "C" int64_t bsx_chain_filtered_ws_bytes(int B, int k, int64_t vocab) {
  const int64_t f = bsx_filter_ws_bytes((int64_t)B * (2 * k + 1));
  const int64_t u = bsx_chain_ws_bytes(B, k, vocab);
  return f > u ? f : u;
}

extern "C" int bsx_chain_speculative_sampling_filtered(
    const void* draft_logits_d, const int64_t* draft_ids_d, const void* target_logits_d,
    int dtype, float temperature, int top_k, float top_p, const float* uniforms_d, int B, int k,
    int64_t vocab, int32_t* out_ids_d, int32_t* accepted_d, int32_t* emitted_d, void* ws_d,
    int64_t ws_bytes, void* stream) {
  if (!filters_on(top_k, top_p, vocab))
    return bsx_chain_speculative_sampling_logits(draft_logits_d, draft_ids_d, target_logits_d,
                                                 dtype, temperature, uniforms_d, B, k, vocab,
                                                 out_ids_d, accepted_d, emitted_d, ws_d,
                                                 ws_bytes, stream);
  BSX_REQUIRE(B >= 0 && k >= 0 && vocab > 0, BSX_ERR_INVALID, "bad B=%d k=%d vocab=%lld", B, k,
              (long long)vocab);
  BSX_REQUIRE(vocab < (1LL << 31), BSX_ERR_UNSUPPORTED, "vocab too large");
  if (B == 0) return BSX_OK;
  BSX_REQUIRE(target_logits_d && uniforms_d && out_ids_d && accepted_d && emitted_d &&
                  (k == 0 || draft_ids_d),
              BSX_ERR_INVALID, "null pointer");
  BSX_REQUIRE(temperature > 0.f && temperature == temperature, BSX_ERR_INVALID,
              "temperature must be > 0 (greedy acceptance has its own entry point)");
  const int64_t need = bsx_filter_ws_bytes((int64_t)B * (2 * k + 1));
  BSX_REQUIRE(ws_d && ws_bytes >= need, BSX_ERR_CAPACITY, "filter workspace too small (%lld < %lld)",
              (long long)ws_bytes, (long long)need);
  filt::ChainArgs ca{};
  ca.t_logits = target_logits_d;
  ca.d_logits = draft_logits_d;
  ca.info = static_cast<const filt::RowInfo*>(ws_d);
  const int64_t rows = (int64_t)B * (k + 1) + (draft_logits_d ? (int64_t)B * k : 0);
  ca.lists = reinterpret_cast<const int32_t*>(static_cast<char*>(ws_d) +
                                              filt::align256(rows * (int64_t)sizeof(filt::RowInfo)));
  ca.draft_ids = draft_ids_d;
  ca.uniforms = uniforms_d;
  ca.B = B;
  ca.k = k;
  ca.V = vocab;
  ca.c = canon::scale_for_temperature(temperature);
  ca.out_ids = out_ids_d;
  ca.accepted = accepted_d;
  ca.emitted = emitted_d;
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case BSX_DTYPE_BF16: return filtered_chain_impl<BSX_DTYPE_BF16>(ca, ws_d, st, top_k, top_p);
    case BSX_DTYPE_FP16: return filtered_chain_impl<BSX_DTYPE_FP16>(ca, ws_d, st, top_k, top_p);
    case BSX_DTYPE_FP32: return filtered_chain_impl<BSX_DTYPE_FP32>(ca, ws_d, st, top_k, top_p);
  }
  set_error("unknown dtype %d", dtype);
  return BSX_ERR_INVALID;
}

extern "C" int64_t bsx_sample_ws_bytes(int64_t rows, int64_t vocab) {
  const int64_t f = bsx_chain_filtered_ws_bytes((int)rows, 0, vocab);
  return f + filt::align256(rows * 8);
}

extern "C" int bsx_sample(const void* logits_d, int dtype, float temperature, int top_k,
                          float top_p, const float* uniforms_d, int64_t rows, int64_t vocab,
                          int32_t* out_d, void* ws_d, int64_t ws_bytes, void* stream) {
  BSX_REQUIRE(rows >= 0 && rows < (1LL << 31) && vocab > 0, BSX_ERR_INVALID, "bad shape");
  if (rows == 0) return BSX_OK;
  BSX_REQUIRE(logits_d && uniforms_d && out_d && ws_d, BSX_ERR_INVALID, "null pointer");
  const int64_t need = bsx_sample_ws_bytes(rows, vocab);
  BSX_REQUIRE(ws_bytes >= need, BSX_ERR_CAPACITY, "sample workspace too small (%lld < %lld)",
              (long long)ws_bytes, (long long)need);
  const int64_t main = bsx_chain_filtered_ws_bytes((int)rows, 0, vocab);
  int32_t* scratch = reinterpret_cast<int32_t*>(static_cast<char*>(ws_d) + main);
  return bsx_chain_speculative_sampling_filtered(nullptr, nullptr, logits_d, dtype, temperature,
                                                 top_k, top_p, uniforms_d, (int)rows, 0, vocab,
                                                 out_d, scratch, scratch + rows, ws_d, main,
                                                 stream);
}

extern "C" int64_t bsx_sampling_probs_ws_bytes(int64_t rows) {
  const int64_t f = bsx_filter_ws_bytes(rows);
  const int64_t s = bsx_softmax_ws_bytes(rows);
  return f > s ? f : s;
}

template <int DT>
static int sampling_probs_impl(const void* logits, int64_t rows, int64_t V, float c, int top_k,
                               float top_p, float* probs, void* ws, hipStream_t st) {
  int rc = launch_filter_rows<DT>(logits, rows, nullptr, 0, V, c, top_k, top_p, ws, st);
  if (rc != BSX_OK) return rc;
  const int parts = (int)std::min<int64_t>(64, std::max<int64_t>(1, ceil_div(V, 4096)));
  hipLaunchKernelGGL((filt::filtered_probs_kernel<DT>), dim3((unsigned)rows, parts),
                     dim3(filt::kThreads), 0, st, logits, V, c,
                     static_cast<const filt::RowInfo*>(ws), probs);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

extern "C" int bsx_sampling_probs(const void* logits_d, int dtype, float temperature, int top_k,
                                  float top_p, int64_t rows, int64_t vocab, float* probs_d,
                                  void* ws_d, int64_t ws_bytes, void* stream) {
  if (!filters_on(top_k, top_p, vocab))
    return bsx_softmax(logits_d, dtype, temperature, rows, vocab, probs_d, ws_d, ws_bytes, stream);
  BSX_REQUIRE(rows >= 0 && rows < (1LL << 31) && vocab > 0 && vocab < (1LL << 31),
              BSX_ERR_INVALID, "bad shape");
  if (rows == 0) return BSX_OK;
  BSX_REQUIRE(logits_d && probs_d && ws_d, BSX_ERR_INVALID, "null pointer");
  BSX_REQUIRE(temperature > 0.f, BSX_ERR_INVALID, "temperature must be > 0");
  BSX_REQUIRE(ws_bytes >= bsx_filter_ws_bytes(rows), BSX_ERR_CAPACITY,
              "sampling-probs workspace too small");
  const float c = canon::scale_for_temperature(temperature);
  hipStream_t st = as_stream(stream);
  switch (dtype) {
    case BSX_DTYPE_BF16:
      return sampling_probs_impl<BSX_DTYPE_BF16>(logits_d, rows, vocab, c, top_k, top_p, probs_d, ws_d, st);
    case BSX_DTYPE_FP16:
      return sampling_probs_impl<BSX_DTYPE_FP16>(logits_d, rows, vocab, c, top_k, top_p, probs_d, ws_d, st);
    case BSX_DTYPE_FP32:
      return sampling_probs_impl<BSX_DTYPE_FP32>(logits_d, rows, vocab, c, top_k, top_p, probs_d, ws_d, st);
  }
  set_error("unknown dtype %d", dtype);
  return BSX_ERR_INVALID;
}
