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
//     1. the canonical (M, Z) pass lists candidates on the way: the k-th largest of
//        the maxima of 2048 disjoint groups (read first) bounds t* from below; groups
//        are listed only when their maximum reaches it (for top-p alone the bound of
//        rank 64 is used); with at most kCands candidates, each gets the count and
//        mass of the listed keys at or above its own (every element of the row there
//        is listed), which gives t* and Z_K exactly, and the kept indices are written
//        out;
//     2. if the list overflowed (or the row is too short for step 1), the bound of all
//        2048 lane maxima and a second read of the row list the candidates again;
//     a row that neither lists (a top_k above kCands, a nucleus below the bound) is
//     left, for top-p alone or a top_k above kDeferTopK, to
//   filter_deferred_kernel: one workgroup per row, the others leave at once;
//     otherwise (rare: ties) it takes step 4 in place.
//     3. a histogram of counts and masses over 1024 bins of the weight's exponent
//        picks the bin that holds t*; its elements (or, for a bin of more than kCands,
//        those of one of its 1024 sub-bins, after a histogram of them) are listed and
//        walked with the count and mass above them as the base; the row gets no list;
//     4. if a sub-bin is still too dense (ties), an exact radix select over the key
//        bits, 8 per pass, with counts and fixed-point masses per digit in LDS.
//   filter_tiles_kernel: (request, part) workgroups: the ratio tests, then, when the
//     row the chain stops at has no kept list, the fixed-point sums of its draw weights
//     over wave-sized tiles of the row, 8 tiles per workgroup;
//   filter_chain_kernel: one workgroup per request: the ratio tests, then the draw
//     from the row the chain stops at, over its kept list, or from the tile sums (their
//     prefix, the tile, the lane, the element) without one.
//   filtered_probs_kernel: p'(x) for every element (get_sampling_probs).
#include <limits.h>

#include <algorithm>

#include "bsx.h"
#include "common.h"
#include "canon.h"
#include "rows.h"

namespace bsx {
namespace filt {

using acc::load_group;
using acc::load_one;
using canon::kLanes;
using canon::LaneState;
using canon::fx40;
using canon::kGroup;
using canon::key_value;
using canon::okey;

constexpr int kThreads = 256;
constexpr int kCands = 1024;      // candidates listed in LDS per row
constexpr int kCap = 256;         // kept elements listed per row for the draw
constexpr int kTopPProbe = 64;    // rank of the lane-maximum bound for top-p alone
constexpr int kDeferTopK = 64;    // top_k above which unlisted rows go to the second kernel
constexpr int kMaxTiles = 2048;   // tiles of a whole-row draw
constexpr int kBinShift = 21;     // 11-bit key bins for the bound
constexpr int kBins = 1 << (32 - kBinShift);
constexpr int kFirstFiniteBin = 4;  // bins below hold -inf and NaN images only
static_assert(kCap <= kThreads, "one kept element per thread in the draw");
static_assert(kMaxTiles % kThreads == 0, "tiles split evenly over threads");
static_assert(kCands % kThreads == 0 && kCands * 8 <= kBins * 4, "candidate masses fit hist");
static_assert(kBins % (4 * kThreads) == 0 && 4 * (kBins / kThreads) <= 64, "bound scan layout");
// Log2-weight bins of the large-threshold select: kYScale bins per unit of the weight's
// exponent y, the last bin from y <= -(kYBins - 1) / kYScale < -40.9 on, where every
// fixed-point mass is 0.
constexpr int kYBins = 1024;
constexpr float kYScale = 25.0f;
static_assert(kYBins * 8 <= kBins * 4 && kYBins <= kCands && kYBins % kThreads == 0,
              "bin masses fit hist, bin counts fit ckey / cidx");
static_assert((kYBins - 1) / kYScale > 40.5f, "the last bin holds mass 0 only");

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
  int defer;      // rows that list neither go to filter_deferred_kernel (else step 4 here)
};

constexpr int32_t kDeferred = -2;  // n_list of a row whose threshold is not found yet

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

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m);
  const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += shfl_xor_u64(v, m);
  return v;
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ uint64_t wave_prefix_u64(uint64_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t lo = __shfl_up((uint32_t)v, d);
    const uint32_t hi = __shfl_up((uint32_t)(v >> 32), d);
    if (lane >= d) v += ((uint64_t)hi << 32) | lo;
  }
  return v;
}

// LDS of filter_rows_kernel.  hist is the bound histogram, then (as uint64) the
// candidate masses of a walk, or the digit counts and masses of the radix select.
struct RowsLds {
  uint32_t hist[kBins];
  uint32_t part[kThreads];
  uint32_t ckey[kCands];
  int32_t cidx[kCands];
  float m, z;
  int bin, count, rcount, ng, nk;
  uint32_t above, rkey, tk, prefix, above_c;
  uint64_t zk, above_m;
};

// Inclusive suffix sum over the 64 lanes of a wave (lane l: sum of lanes l..63).
__device__ __forceinline__ uint32_t wave_suffix_u32(uint32_t v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_down(v, d);
    if (lane + d < 64) v += o;
  }
  return v;
}

// Bin (11-bit key prefix) holding the k-th largest of the 2048 values lm (8 per
// thread); -1 if k > 2048 or if that value is -inf or NaN (those are not counted: a
// list of candidates padded with -inf would otherwise pile its atomics onto one bin).
// L.above receives the number of values in higher bins.  Every thread of the workgroup
// calls it.
__device__ __forceinline__ int kth_bin(RowsLds& L, const float (&lm)[8], int k) {
  constexpr int PER = kBins / kThreads;  // bins summed per thread
  const int t = threadIdx.x;
  u32x4* h4 = reinterpret_cast<u32x4*>(L.hist);
#pragma unroll
  for (int i = 0; i < PER / 4; ++i) h4[t * (PER / 4) + i] = u32x4{0u, 0u, 0u, 0u};
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t bin = okey(lm[i]) >> kBinShift;
    if (bin >= (uint32_t)kFirstFiniteBin) atomicAdd(&L.hist[bin], 1u);
  }
  __syncthreads();
  {
    uint32_t ps = 0;
#pragma unroll
    for (int i = 0; i < PER / 4; ++i) {
      const u32x4 v = h4[t * (PER / 4) + i];
      ps += (v[0] + v[1]) + (v[2] + v[3]);
    }
    L.part[t] = ps;
  }
  __syncthreads();
  if (t < 64) {
    // lane l: the bins of threads 4l .. 4l+3, i.e. [4 PER l, 4 PER (l+1))
    const uint32_t q = L.part[4 * t] + L.part[4 * t + 1] + L.part[4 * t + 2] + L.part[4 * t + 3];
    const uint32_t s = wave_suffix_u32(q);
    const uint64_t mask = __builtin_amdgcn_ballot_w64(k <= 2048 && s >= (uint32_t)k);
    const int ls = mask ? 63 - __builtin_clzll(mask) : -1;  // uniform
    if (ls < 0) {
      if (t == 0) L.bin = -1;
    } else {
      // the chunk of lane ls (4 PER <= 64 bins), one bin per lane, suffix sums again
      constexpr int CH = 4 * PER;
      const uint32_t above_chunk = __shfl(s - q, ls);
      const uint32_t hv = t < CH ? L.hist[CH * ls + t] : 0u;
      const uint32_t sb = wave_suffix_u32(hv) + above_chunk;
      const uint64_t m2 = __builtin_amdgcn_ballot_w64(t < CH && sb >= (uint32_t)k);
      const int lb = 63 - __builtin_clzll(m2);  // non-empty: the chunk holds the k-th
      if (t == lb) {
        L.bin = CH * ls + lb;
        L.above = sb - hv;
      }
    }
  }
  __syncthreads();
  return L.bin;
}

// Key of the k-th largest of the 2048 values lm (k <= 2048), exact when at most
// kThreads of them share its 12-bit bin (else the bin's lower edge, a smaller bound);
// 0 when that value is -inf or k > 2048.  Uses hist and part.  Every thread calls it.
__device__ __forceinline__ uint32_t kth_key(RowsLds& L, const float (&lm)[8], int k) {
  const int t = threadIdx.x;
  const int bin = kth_bin(L, lm, k);
  if (bin < kFirstFiniteBin) return 0u;
  if (t == 0) {
    L.rcount = 0;
    L.rkey = 0u;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t key = okey(lm[i]);
    if ((int)(key >> kBinShift) == bin) {
      const int slot = atomicAdd(&L.rcount, 1);
      if (slot < kThreads) L.part[slot] = key;
    }
  }
  __syncthreads();
  const int n = L.rcount;
  uint32_t result = (uint32_t)bin << kBinShift;
  if (n <= kThreads) {
    // the largest key of the bin with at least k values at or above it
    if (t < n) {
      const uint32_t key = L.part[t];
      uint32_t cnt = L.above;
      for (int q = 0; q < n; ++q) cnt += L.part[q] >= key ? 1u : 0u;
      if (cnt >= (uint32_t)k) atomicMax(&L.rkey, key);
    }
    __syncthreads();
    result = L.rkey;
  }
  __syncthreads();
  return result;
}

// kth_key as a call: for the statistics pass's first round and the list tightening, where
// inlining it would raise
// the pass's registers (and with them the rows a compute unit holds).  The values go by
// value, in registers (an array by reference would go through scratch memory).
__device__ __noinline__ uint32_t kth_key_call(RowsLds& L, float v0, float v1, float v2, float v3,
                                              float v4, float v5, float v6, float v7, int k) {
  const float lm[8] = {v0, v1, v2, v3, v4, v5, v6, v7};
  return kth_key(L, lm, k);
}

// The 8 elements of a complete group of a row with 16-byte aligned groups.
template <int DT>
__device__ __forceinline__ void load8(const void* row, int64_t g, float (&x)[8]) {
  if constexpr (DT == BSX_DTYPE_FP32) {
    const f32x4 a = static_cast<const f32x4*>(row)[2 * g];
    const f32x4 b = static_cast<const f32x4*>(row)[2 * g + 1];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x[q] = a[q];
      x[4 + q] = b[q];
    }
  } else {
    const u32x4 w = static_cast<const u32x4*>(row)[g];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      x[2 * q] = lo_f32<DT>(w[q]);
      x[2 * q + 1] = hi_f32<DT>(w[q]);
    }
  }
}

__device__ __forceinline__ void push_candidate(RowsLds& L, float x, int64_t v) {
  const int slot = atomicAdd(&L.count, 1);
  if (slot < kCands) {
    L.ckey[slot] = okey(x);
    L.cidx[slot] = (int32_t)v;
  }
}

// Lists the row's elements >= a bound lf during the statistics pass.  In whole round
// r = c0/8 each thread only sets bits 8r + i of a 128-bit register mask for its groups
// t + 256*(c0 + i) whose maximum reaches the bound (at most 16 whole rounds); such
// groups are rare, and their elements are read again after the pass (anything heavier
// inside the pass's loop costs the loop occupancy).  Groups of the partial rounds list
// their elements directly.
constexpr int kMaxHitRounds = 16;

template <int DT>
struct Collector {
  RowsLds* L;
  float lf;
  bool on;  // same value in every thread
  int k;
  uint64_t hits[2];
  __device__ bool wants_first() const { return on; }
  // The bound from the maxima of the first round's groups t + 256 i, i < 8: they are
  // disjoint, so the k-th largest of the 2048 has at least k elements of the row at or
  // above it, and so has t*.
  __device__ void first(const float (&gm)[8]) {
    const uint32_t kb =
        kth_key_call(*L, gm[0], gm[1], gm[2], gm[3], gm[4], gm[5], gm[6], gm[7], k);
    if (kb == 0u) on = false;
    else lf = key_value(kb);
  }
  __device__ void round(int64_t c0, const float (&gm)[8]) {
    if (!on) return;
    uint64_t h = 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) h |= (gm[i] >= lf ? 1ull : 0ull) << i;
    const int r = (int)(c0 / 8);
    if (r < 8) hits[0] |= h << (8 * r);
    else hits[1] |= h << (8 * (r - 8));
  }
  __device__ void group(int64_t g, const float* x, int n, float gm) {
    if (!on || !(gm >= lf)) return;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < n && x[e] >= lf) push_candidate(*L, x[e], g * kGroup + e);
  }
};

// Threshold from a complete list of the candidates [0, n) (every element of the row
// at or above the smallest listed key and below the keys counted in base_c / base_m
// is listed): each candidate gets base_c / base_m plus the count and mass of the listed
// keys at or above its own; t* is the largest key that reaches the target.  Writes the
// kept indices (at most kCap, else the row gets no list; no list either when list_out
// is null).  Returns false (in every thread) when no listed key reaches the target.
__device__ __forceinline__ bool walk(RowsLds& L, int n, float c, float neg, bool use_k,
                                     bool use_p, int top_k, uint64_t target, int32_t* list_out,
                                     uint32_t base_c = 0u, uint64_t base_m = 0ull) {
  typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
  const int t = threadIdx.x;
  uint64_t* cm = reinterpret_cast<uint64_t*>(L.hist);
  constexpr int PER = kCands / kThreads;
  const int n8 = (n + 7) & ~7;  // padded with key 0 (below every element's key), mass 0
  if (t == 0) {
    L.tk = 0u;
    L.nk = 0;
  }
  for (int s = t; s < n8; s += kThreads) {
    if (s < n) {
      cm[s] = fx40(canon::weight(key_value(L.ckey[s]), c, neg));
    } else {
      cm[s] = 0ull;
      L.ckey[s] = 0u;
    }
  }
  __syncthreads();
  if (!use_k) {
    // top-p alone: t* is listed only if the listed mass reaches the target
    uint64_t mine = 0ull;
    for (int s = t; s < n; s += kThreads) mine += cm[s];
    if (t == 0) L.zk = 0ull;
    __syncthreads();
    if (mine != 0ull) atomicAdd(reinterpret_cast<unsigned long long*>(&L.zk), (unsigned long long)mine);
    __syncthreads();
    const bool enough = base_m + L.zk >= target;
    __syncthreads();
    if (!enough) return false;
  }
  uint32_t key[PER];
  uint32_t cnt[PER];
  uint64_t mass[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int s = t + kThreads * j;
    key[j] = s < n ? L.ckey[s] : 0xffffffffu;
    cnt[j] = base_c;
    mass[j] = base_m;
  }
  if (n <= kThreads) {
    // one candidate per thread; every listed key against it, 8 at a time from 16-byte
    // reads; threads (and waves) without a candidate skip the loop
    if (t < n) {
      const u32x4* k4 = reinterpret_cast<const u32x4*>(L.ckey);
      const u64x2* m2 = reinterpret_cast<const u64x2*>(cm);
      for (int q = 0; q < n8; q += 8) {
        const u32x4 ka = k4[q / 4], kb = k4[q / 4 + 1];
        const u64x2 m01 = m2[q / 2], m23 = m2[q / 2 + 1], m45 = m2[q / 2 + 2], m67 = m2[q / 2 + 3];
        const uint32_t kk[8] = {ka[0], ka[1], ka[2], ka[3], kb[0], kb[1], kb[2], kb[3]};
        const uint64_t mm[8] = {m01[0], m01[1], m23[0], m23[1], m45[0], m45[1], m67[0], m67[1]};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const bool ge = kk[e] >= key[0];
          cnt[0] += ge ? 1u : 0u;
          mass[0] += ge ? mm[e] : 0ull;
        }
      }
    }
  } else {
    for (int q = 0; q < n; ++q) {
      const uint32_t kq = L.ckey[q];
      const uint64_t mq = cm[q];
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (kq >= key[j]) {
          ++cnt[j];
          mass[j] += mq;
        }
    }
  }
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (t + kThreads * j < n && reached(use_k, use_p, cnt[j], mass[j], top_k, target))
      atomicMax(&L.tk, key[j]);
  __syncthreads();
  const uint32_t tk = L.tk;
  // a finite element's key is never 0
  if (tk == 0u) return false;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int s = t + kThreads * j;
    if (s < n) {
      if (key[j] == tk) L.zk = mass[j];  // equal keys hold equal masses
      if (list_out != nullptr && key[j] >= tk) {
        const int slot = atomicAdd(&L.nk, 1);
        if (slot < kCap) list_out[slot] = L.cidx[s];
      }
    }
  }
  lds_barrier();  // (the list stores need not land first)
  if (t == 0 && (list_out == nullptr || L.nk > kCap)) L.nk = -1;
  lds_barrier();
  return true;
}

// Position of an element on the log2-weight axis: q = -y * kYScale with
// y = fma(x, C, -(M C)), the exponent of its weight.  Its bin is floor(q) below
// kYBins - 1 and the last bin otherwise (NaN included); the sub-bins of bin b split
// [b, b + 1) into kYBins.  A larger key never gets a larger q, bin or sub-bin, so every
// bin (sub-bin) holds a contiguous range of keys.
__device__ __forceinline__ float ypos(float x, float c, float neg) {
  return -fmaf(x, c, neg) * kYScale;
}
__device__ __forceinline__ int ybin(float q) {
  return q < (float)(kYBins - 1) ? (int)fmaxf(q, 0.0f) : kYBins - 1;
}
// q - b is exact for q in [b, b + 1) (b >= 1), and q itself for b = 0.
__device__ __forceinline__ int ysub(float q, int b) {
  return min((int)fmaxf((q - (float)b) * (float)kYBins, 0.0f), kYBins - 1);
}

// The first of the bins [0, nb) (in decreasing key order) at which base + the running
// count / mass of cnt / mass reaches the threshold.  Returns it (-1 if none does) and
// leaves what lies above it in L.above_c / L.above_m and its own count in L.rcount.
// Uses part.  Every thread calls it.
__device__ __forceinline__ int ybin_first(RowsLds& L, const uint32_t* cnt, const uint64_t* mass,
                                          int nb, uint32_t base_c, uint64_t base_m, bool use_k,
                                          bool use_p, int top_k, uint64_t target) {
  constexpr int PER = kYBins / kThreads;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  uint32_t cc[PER];
  uint64_t mm[PER];
  uint64_t sc = 0ull, sm = 0ull;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    cc[i] = cnt[PER * t + i];
    mm[i] = mass[PER * t + i];
    sc += cc[i];
    sm += mm[i];
  }
  const uint64_t ic = wave_prefix_u64(sc), im = wave_prefix_u64(sm);
  uint64_t* wt = reinterpret_cast<uint64_t*>(L.part);  // wave totals: counts, then masses
  if (lane == 63) {
    wt[wave] = ic;
    wt[kThreads / 64 + wave] = im;
  }
  if (t == 0) L.bin = INT_MAX;
  __syncthreads();
  uint64_t ac = base_c + (ic - sc), am = base_m + (im - sm);
  for (int w = 0; w < wave; ++w) {
    ac += wt[w];
    am += wt[kThreads / 64 + w];
  }
  int mine = -1;
  uint32_t my_c = 0u, my_n = 0u;
  uint64_t my_m = 0ull;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int b = PER * t + i;
    if (mine < 0 && b < nb &&
        reached(use_k, use_p, (uint32_t)(ac + cc[i]), am + mm[i], top_k, target)) {
      mine = b;
      my_c = (uint32_t)ac;
      my_m = am;
      my_n = cc[i];
    }
    ac += cc[i];
    am += mm[i];
  }
  if (mine >= 0) atomicMin(&L.bin, mine);
  __syncthreads();
  const int first = L.bin;
  if (mine >= 0 && mine == first) {
    L.above_c = my_c;
    L.above_m = my_m;
    L.rcount = (int)my_n;
  }
  __syncthreads();
  return first == INT_MAX ? -1 : first;
}

// fx40(2^y) for y in (-41, 1): the 2^8 scale of fx40 folded into the exponent,
// ldexp(P(f), n + 8) = ldexp(P(f), n) * 2^8 exactly (both normal), then its two
// conversions.
__device__ __forceinline__ uint64_t mass_of_exponent(float y) {
  int n;
  const float p = canon::exp2_parts(y, &n);
  const float a = ldexpf(p, n + 8);
  const uint32_t hi = (uint32_t)a;
  const uint32_t lo = (uint32_t)((a - (float)hi) * 0x1p32f);
  return ((uint64_t)hi << 32) | lo;
}

// What an exponent-bin histogram holds: counts (top-k on), fixed-point masses (top-p on).
constexpr int kHistCount = 1, kHistMass = 2;

// Counts (in ckey) and masses (in hist) of the elements per bin (SUB false; the last bin
// left out) or per sub-bin of bin b0, whose elements are those in [xlo, xhi] (SUB true);
// what MODE leaves out stays 0.
template <int DT, int MODE, bool SUB>
__device__ void ybin_hist(RowsLds& L, const void* row, int64_t V, bool vec, float c, float neg,
                          int b0, float xlo, float xhi) {
  uint32_t* cnt = L.ckey;
  uint64_t* mass = reinterpret_cast<uint64_t*>(L.hist);
  for (int i = threadIdx.x; i < kYBins; i += kThreads) {
    cnt[i] = 0u;
    mass[i] = 0ull;
  }
  __syncthreads();
  for_each_element<DT>(row, V, vec, [&](float x, int64_t) {
    const float y = fmaf(x, c, neg);
    const float q = -y * kYScale;  // ypos(x, c, neg)
    int b;
    if constexpr (SUB) {
      if (!(x >= xlo && x <= xhi)) return;
      b = ysub(q, b0);
    } else {
      if (!(q < (float)(kYBins - 1))) return;
      b = (int)fmaxf(q, 0.0f);
    }
    if constexpr ((MODE & kHistCount) != 0) atomicAdd(&cnt[b], 1u);
    if constexpr ((MODE & kHistMass) != 0)
      atomicAdd(reinterpret_cast<unsigned long long*>(&mass[b]),
                (unsigned long long)mass_of_exponent(y));
  });
  __syncthreads();
}

template <int DT, bool SUB>
__device__ void ybin_hist_for(int mode, RowsLds& L, const void* row, int64_t V, bool vec, float c,
                              float neg, int b0, float xlo, float xhi) {
  if (mode == kHistCount) ybin_hist<DT, kHistCount, SUB>(L, row, V, vec, c, neg, b0, xlo, xhi);
  else if (mode == kHistMass) ybin_hist<DT, kHistMass, SUB>(L, row, V, vec, c, neg, b0, xlo, xhi);
  else ybin_hist<DT, kHistCount | kHistMass, SUB>(L, row, V, vec, c, neg, b0, xlo, xhi);
}

// The first key k in [lo, hi) with pred(k), pred non-decreasing in k and taken as true
// at hi; hi if none.  The range is split 64 ways per step (one candidate per lane of
// the calling wave), so a 32-bit range takes about 6 steps.  Wave-uniform.
template <typename P>
__device__ uint64_t wave_first_key(uint64_t lo, uint64_t hi, P&& pred) {
  const uint64_t lane = threadIdx.x & 63;
  while (lo < hi) {
    const uint64_t step = (hi - lo + 63) / 64;
    const uint64_t k = lo + lane * step;
    const uint64_t m = __builtin_amdgcn_ballot_w64(k >= hi || pred((uint32_t)k));
    if (m == 0ull) {
      lo += 63 * step + 1;  // false up to the last lane's key
    } else {
      const uint64_t f = (uint64_t)__builtin_ctzll(m);
      if (f == 0) return lo;
      const uint64_t nhi = lo + f * step < hi ? lo + f * step : hi;
      lo += (f - 1) * step + 1;
      hi = nhi;
    }
  }
  return lo;
}

// Float range [xlo, xhi] of the keys of bin b0 (b1 < 0) or of its sub-bin b1: bins and
// sub-bins are contiguous key ranges, found by two searches over the finite and
// infinite keys.  Every thread calls it; the set must hold at least one key.
__device__ void ybin_range(RowsLds& L, int b0, int b1, float c, float neg, float* xlo,
                           float* xhi) {
  float* xr = reinterpret_cast<float*>(L.part);
  if (threadIdx.x < 64) {
    const int target = b0 * kYBins + (b1 >= 0 ? b1 : 0);
    auto pos = [&](uint32_t k) {
      const float q = ypos(key_value(k), c, neg);
      const int b = ybin(q);
      return b * kYBins + (b1 >= 0 && b == b0 ? ysub(q, b0) : 0);
    };
    const uint64_t k_lo = okey(-INFINITY), k_end = (uint64_t)okey(INFINITY) + 1;
    const uint64_t first = wave_first_key(k_lo, k_end, [&](uint32_t k) { return pos(k) <= target; });
    const uint64_t past = wave_first_key(first, k_end, [&](uint32_t k) { return pos(k) < target; });
    if (threadIdx.x == 0) {
      xr[0] = key_value((uint32_t)first);
      xr[1] = key_value((uint32_t)(past - 1));
    }
  }
  __syncthreads();
  *xlo = xr[0];
  *xhi = xr[1];
  __syncthreads();
}

// Threshold of a row whose upper set is too large to list: the first log2-weight bin
// (one histogram pass) at which the running count / mass reaches the target, then the
// elements of that bin listed and walked with what lies above as the base.  A bin of
// more than kCands elements is narrowed to one of its 1024 sub-bins by a histogram of
// them (a second pass) before it is listed; a listed bin of more than kThreads elements
// is narrowed to one of its sub-bins in LDS.  The histograms hold counts for top-k
// (for top-k alone the listing pass then sums the masses above) and masses for top-p
// (for top-p alone a bin is known to be too large only once listed).  The row gets no
// list.  Returns false (in every thread) when the threshold is not found this way (a
// sub-bin too dense, or a target beyond the mass of the bins).  Needs a finite row max.
template <int DT>
__device__ __forceinline__ bool ybin_threshold(
    RowsLds& L, const void* row, int64_t V, bool vec, float c, float neg, bool use_k,
    bool use_p, int top_k, uint64_t target) {
  const int t = threadIdx.x;
  const int mode = (use_k ? kHistCount : 0) | (use_p ? kHistMass : 0);
  ybin_hist_for<DT, false>(mode, L, row, V, vec, c, neg, -1, 0.f, 0.f);
  const int b0 = ybin_first(L, L.ckey, reinterpret_cast<const uint64_t*>(L.hist), kYBins - 1,
                            0u, 0ull, use_k, use_p, top_k, target);
  if (b0 < 0) return false;
  uint32_t base_c = L.above_c;
  uint64_t base_m = L.above_m;
  int b1 = -1;
  float xlo, xhi;
  // narrows bin b0 to the sub-bin b1 that holds the threshold
  auto narrow = [&]() -> bool {
    ybin_range(L, b0, -1, c, neg, &xlo, &xhi);
    ybin_hist_for<DT, true>(mode, L, row, V, vec, c, neg, b0, xlo, xhi);
    b1 = ybin_first(L, L.ckey, reinterpret_cast<const uint64_t*>(L.hist), kYBins, base_c,
                    base_m, use_k, use_p, top_k, target);
    if (b1 < 0 || (use_k && L.rcount > kCands)) return false;
    base_c = L.above_c;
    base_m = L.above_m;
    return true;
  };
  // lists the elements of bin b0 (sub-bin b1)
  auto list = [&]() {
    ybin_range(L, b0, b1, c, neg, &xlo, &xhi);
    if (t == 0) {
      L.count = 0;
      L.zk = 0ull;
    }
    __syncthreads();
    uint64_t above = 0ull;  // top-k alone: the mass of the elements above the listed ones
    for_each_element<DT>(row, V, vec, [&](float x, int64_t) {
      if (x >= xlo && x <= xhi) {
        const int slot = atomicAdd(&L.count, 1);
        if (slot < kCands) L.ckey[slot] = okey(x);
      } else if (!use_p && x > xhi) {
        above += mass_of_exponent(fmaf(x, c, neg));
      }
    });
    if (!use_p) {
      above = wave_sum_u64(above);
      if ((t & 63) == 0 && above != 0ull)
        atomicAdd(reinterpret_cast<unsigned long long*>(&L.zk), (unsigned long long)above);
    }
    __syncthreads();
    if (!use_p) base_m = L.zk;
  };
  if (use_k && L.rcount > kCands && !narrow()) return false;
  list();
  if (!use_k && L.count > kCands) {
    // a bin of uncounted elements (top-p alone) too large to list
    __syncthreads();
    if (!narrow()) return false;
    list();
  }
  int n = L.count;
  if (n > kCands) return false;
  if (n > kThreads && b1 < 0) {
    // sub-bins of the listed elements: counts in cidx, masses in hist
    uint32_t* cnt = reinterpret_cast<uint32_t*>(L.cidx);
    uint64_t* mass = reinterpret_cast<uint64_t*>(L.hist);
    for (int i = t; i < kYBins; i += kThreads) {
      cnt[i] = 0u;
      mass[i] = 0ull;
    }
    __syncthreads();
    for (int s = t; s < n; s += kThreads) {
      const float x = key_value(L.ckey[s]);
      const int sb = ysub(ypos(x, c, neg), b0);
      atomicAdd(&cnt[sb], 1u);
      const uint64_t m = fx40(canon::weight(x, c, neg));
      if (m != 0ull) atomicAdd(reinterpret_cast<unsigned long long*>(&mass[sb]), (unsigned long long)m);
    }
    __syncthreads();
    const int s1 = ybin_first(L, cnt, mass, kYBins, base_c, base_m, use_k, use_p, top_k, target);
    if (s1 < 0) return false;
    base_c = L.above_c;
    base_m = L.above_m;
    // keep the elements of sub-bin s1, in place
    constexpr int PER = kCands / kThreads;
    uint32_t kk[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int s = t + kThreads * j;
      kk[j] = s < n ? L.ckey[s] : 0u;
    }
    if (t == 0) L.count = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (t + kThreads * j < n && ysub(ypos(key_value(kk[j]), c, neg), b0) == s1)
        L.ckey[atomicAdd(&L.count, 1)] = kk[j];
    __syncthreads();
    n = L.count;
  }
  return walk(L, n, c, neg, use_k, use_p, top_k, target, nullptr, base_c, base_m);
}

// Step 4: exact radix select over the key bits, 8 per pass, counts and fixed-point
// masses per digit in LDS.  Leaves t* in L.tk, Z_K in L.zk, no list.
template <int DT>
__device__ __forceinline__ void radix_threshold(
    RowsLds& L, const void* row, int64_t V, bool vec, float c, float neg, bool use_k,
    bool use_p, int top_k, uint64_t target) {
  const int t = threadIdx.x;
  uint32_t* hc = L.hist;                                     // [256]
  uint64_t* hm = reinterpret_cast<uint64_t*>(L.hist + 256);  // [256]
  constexpr int NP = radix_passes<DT>();
  if (t == 0) {
    L.prefix = 0u;
    L.above_c = 0u;
    L.above_m = 0ull;
  }
  for (int pass = 0; pass < NP; ++pass) {
    const int shift = 24 - 8 * pass;
    hc[t] = 0u;
    hm[t] = 0ull;
    __syncthreads();
    const uint32_t prefix = L.prefix;
    for_each_element<DT>(row, V, vec, [&](float x, int64_t) {
      const uint32_t key = okey(x);
      if (pass == 0 || (key >> (shift + 8)) == prefix) {
        const uint32_t d = (key >> shift) & 255u;
        atomicAdd(&hc[d], 1u);
        const uint64_t m = fx40(canon::weight(x, c, neg));
        if (m != 0ull)
          atomicAdd(reinterpret_cast<unsigned long long*>(&hm[d]), (unsigned long long)m);
      }
    });
    __syncthreads();
    if (t == 0) {
      uint32_t cum_c = L.above_c;
      uint64_t cum_m = L.above_m;
      int chosen = -1;
      uint32_t ch_prev_c = 0u;
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
        ch_m = cum_m;
        if (reached(use_k, use_p, cum_c, cum_m, top_k, target)) break;
      }
      L.prefix = (pass == 0 ? 0u : (prefix << 8)) | (uint32_t)chosen;
      L.above_c = ch_prev_c;
      L.above_m = ch_prev_m;
      L.zk = ch_m;
    }
    __syncthreads();
  }
  if (t == 0) {
    constexpr int low_bits = 32 - 8 * NP;
    uint32_t tk = low_bits == 0 ? L.prefix : (L.prefix << low_bits);
    // the bits below the varying ones are 0 for positive values, 1 for negative
    if (low_bits > 0 && !(tk & 0x80000000u)) tk |= (1u << low_bits) - 1u;
    L.tk = tk;
    L.nk = -1;
  }
  __syncthreads();
}

// Steps 3 and 4 for a row whose upper set could not be listed.
template <int DT>
__device__ __forceinline__ void large_threshold(
    RowsLds& L, const void* row, int64_t V, bool vec, float c, float neg, bool use_k,
    bool use_p, int top_k, uint64_t target) {
  bool found = false;
  if (neg > -INFINITY && neg < INFINITY)
    found = ybin_threshold<DT>(L, row, V, vec, c, neg, use_k, use_p, top_k, target);
  if (!found) radix_threshold<DT>(L, row, V, vec, c, neg, use_k, use_p, top_k, target);
}

__device__ __forceinline__ void write_info(RowsLds& L, RowInfo* info, float M) {
  if (threadIdx.x == 0) {
    RowInfo ri;
    ri.m = M;
    ri.inv_k = 1.0f / (canon::u64_to_f32(L.zk) * 0x1p-40f);
    ri.t_key = L.tk;
    ri.n_list = L.nk;
    *info = ri;
  }
}

template <int DT>
__global__ void __launch_bounds__(kThreads) filter_rows_kernel(RowsArgs a) {
  __shared__ __align__(16) RowsLds L;
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
  const int k_eff = use_k ? a.top_k : kTopPProbe;
  int32_t* list_out = a.lists + r * kCap;

  // 1. canonical statistics, listing candidates on the way when every thread has a
  //    whole first round
  if (t == 0) L.count = 0;
  // Candidates are listed during the pass when every thread has a whole first round
  // (the bound comes from it) and the hit masks cover the whole rounds.
  const int64_t G_whole = V / kGroup;
  Collector<DT> col{&L, INFINITY,
                    vec && k_eff <= kCands && ceil_div(G_whole, (int64_t)kThreads * 8) <= kMaxHitRounds,
                    k_eff, {0ull, 0ull}};
  float lm[8];
  acc::row_stats<DT, true, Collector<DT>>(row, V, vec, c, &L.m, &L.z, lm, &col);
  const float M = L.m, Z = L.z;
  const float neg = -(M * c);
  const uint64_t target = use_p ? (uint64_t)ceilf((a.top_p * Z) * 0x1p40f) : 0ull;
  if (col.on) {
    // the noted groups of the whole rounds: their indices listed in LDS, then one
    // group per thread read again (a single round trip for the usual few hundred)
    if (t == 0) L.ng = 0;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      uint64_t h = col.hits[w];
#pragma unroll 1
      while (h != 0ull) {
        const int bit = __builtin_ctzll(h);
        h &= h - 1ull;
        const int slot = atomicAdd(&L.ng, 1);
        // bit 8r + i: group t + 256(8r + i)
        if (slot < kBins) L.hist[slot] = (uint32_t)(t + 256 * (64 * w + bit));
      }
    }
    __syncthreads();
    const int ng = min(L.ng, kBins);
    for (int q = t; q < ng; q += kThreads) {
      const int64_t g = L.hist[q];
      float x[8];
      load8<DT>(row, g, x);
      uint32_t hb = 0u;
#pragma unroll
      for (int e = 0; e < 8; ++e) hb |= (x[e] >= col.lf ? 1u : 0u) << e;
#pragma unroll 1
      while (hb != 0u) {
        const int e = __builtin_ctz(hb);
        hb &= hb - 1u;
        // the element again from cache: indexing x by a run-time e would put x in
        // scratch memory
        push_candidate(L, load_one<DT>(row, g * kGroup + e), g * kGroup + e);
      }
    }
    __syncthreads();
    if (L.ng > kBins && t == 0) L.count = kCands + 1;  // could not list them all
    __syncthreads();
  }

  if (col.on && use_k && L.count > 2 * k_eff && L.count <= kCands) {
    // With top-k on, t* is at or above the k-th largest listed key: every element of the
    // row at or above the bound is listed, so that is the row's k-th largest.  Keeping only
    // the keys at or above it leaves the walk about top_k of them.
    constexpr int PER = kCands / kThreads;
    static_assert(PER <= 8, "the k-th selection takes 8 values per thread");
    const int n = L.count;
    uint32_t ck[PER];
    int32_t ci[PER];
    float cv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cv[j] = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int s = t + kThreads * j;
      ck[j] = s < n ? L.ckey[s] : 0u;
      ci[j] = s < n ? L.cidx[s] : 0;
      if (s < n) cv[j] = key_value(ck[j]);
    }
    const uint32_t kb = kth_key_call(L, cv[0], cv[1], cv[2], cv[3], cv[4], cv[5], cv[6], cv[7],
                                     k_eff);  // 0 (keep all) with fewer than k finite
    if (t == 0) L.count = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (t + kThreads * j < n && ck[j] >= kb) {
        const int slot = atomicAdd(&L.count, 1);
        L.ckey[slot] = ck[j];
        L.cidx[slot] = ci[j];
      }
    __syncthreads();
  }

  bool listed = false;
  const bool early = col.on && L.count <= kCands;
  if (early) {
    listed = walk(L, L.count, c, neg, use_k, use_p, a.top_k, target, list_out);
  } else if (k_eff <= kCands) {
    // 2. otherwise the bound of all lane maxima, and a second read of the row (a list
    //    cannot hold more than kCands of the top-k).  On this branch only, so that the
    //    lane maxima need not stay live across the walk above.
    const uint32_t kb = kth_key(L, lm, k_eff);
    const bool all = kb == 0u;
    if (!all || V <= kCands) {
      const float lf = all ? -INFINITY : key_value(kb);
      for_each_element<DT>(row, V, vec, [&](float x, int64_t v) {
        if (x >= lf) push_candidate(L, x, v);
      });
      __syncthreads();
      const int n = L.count;
      if (n <= kCands) listed = walk(L, n, c, neg, use_k, use_p, a.top_k, target, list_out);
    }
  }

  if (!listed && a.defer) {
    // steps 3 and 4 in filter_deferred_kernel (kept out of this kernel, whose registers
    // bound how many rows it holds at once)
    if (t == 0) a.info[r] = RowInfo{M, Z, 0u, kDeferred};
    return;
  }
  if (!listed) radix_threshold<DT>(L, row, V, vec, c, neg, use_k, use_p, a.top_k, target);
  write_info(L, a.info + r, M);
}

// Steps 3 and 4 of the rows filter_rows_kernel could not list (their statistics in the
// row info: M, and Z in place of 1 / Z_K); the other rows are left as they are.  Its
// registers let the device hold every row at once.
template <int DT>
__global__ void __launch_bounds__(kThreads) filter_deferred_kernel(RowsArgs a) {
  __shared__ __align__(16) RowsLds L;
  const int64_t r = blockIdx.x;
  const RowInfo ri = a.info[r];
  if (ri.n_list != kDeferred) return;
  const int64_t V = a.V;
  const size_t esz = DT == BSX_DTYPE_FP32 ? 4 : 2;
  const char* row = r < a.n_a ? static_cast<const char*>(a.a) + r * V * esz
                              : static_cast<const char*>(a.b) + (r - a.n_a) * V * esz;
  const bool vec = ((V * esz) % 16 == 0) && (((uintptr_t)row) % 16 == 0);
  const float c = a.c;
  const bool use_k = a.top_k > 0 && (int64_t)a.top_k < V;
  const bool use_p = a.top_p > 0.f && a.top_p < 1.f;
  const float M = ri.m, Z = ri.inv_k;
  const float neg = -(M * c);
  const uint64_t target = use_p ? (uint64_t)ceilf((a.top_p * Z) * 0x1p40f) : 0ull;
  large_threshold<DT>(L, row, V, vec, c, neg, use_k, use_p, a.top_k, target);
  write_info(L, a.info + r, M);
}

// ----------------------------------------------------------------------------
// Few rows: each row split over kParts workgroups (top-k on, top_k <= kDeferTopK).
// ----------------------------------------------------------------------------
// With one workgroup per row, a few hundred rows (the reference's default sampling at
// the MTP verify shape: 320 rows of 128256) leave most compute units without work and
// every row's pass latency-bound.  filter_parts_kernel gives each row kParts workgroups:
// part p takes the canonical threads [64 p, 64 p + 64) (lanes [512 p, 512 p + 512), the
// lanes 8t + i of canon.h), wave h of the part the lanes i = 2h, 2h + 1 of its 64
// threads.  Every lane runs the canonical update of canon.h over its groups in order,
// so the lane states are exactly those of the one-workgroup pass; they go to the
// workspace, and filter_combine_kernel rescales them to the row max and sums them over
// the same tree (row_stats' epilogue), giving the same (M, Z) bit for bit.
// Candidates: part p's bound is the k-th largest of the maxima of its 512 first-round
// groups (disjoint, so at least k of the part's elements reach it, and t* is at or above
// the row's k-th largest element, which is at or above it); the part lists its elements
// at or above the bound, keeps those at or above its own k-th largest listed key kb_p
// (the part's k-th largest element) and writes them.  Every element of the row at or
// above B = max_p kb_p is then written by its part, and t* >= the row's k-th largest
// >= B, so the walk over the written keys at or above B finds t* and Z_K exactly.  A
// part that cannot list (too many elements at its bound, a first round without k finite
// maxima) sends the row to the exact threshold search of steps 3 and 4 in the combine
// kernel.
constexpr int kParts = 4;
constexpr int kPartThreads = kThreads / kParts;  // canonical threads per part
constexpr int kSplitMaxRows = 512;
constexpr int64_t kSplitMinVocab = 8 * kLanes;  // every part has whole first-round groups
constexpr int64_t kSplitMaxVocab = 16 * 8 * kLanes;  // at most 16 rounds: 32 hit bits
constexpr int kSplitRounds = 2;                 // rounds per batch of loads (4, two batches in flight)
constexpr int kPartList = kCap;                 // keys a part writes (about top_k + ties)
static_assert(kThreads / 64 * 2 == 8, "a wave of a part holds two lanes of each thread");

struct PartOut {
  float m;        // maximum over the part's lanes (fmaxf-reduced)
  uint32_t kb;    // the part's k-th largest listed key
  int32_t count;  // keys written (>= kb), or -1: the part could not list
  int32_t pad;
};

struct SplitArgs {
  const void* a;  // rows [0, n_a)
  int64_t n_a;
  const void* b;  // rows [n_a, ...)
  int64_t V;
  float c;
  int top_k;
  float top_p;
  RowInfo* info;
  int32_t* lists;    // [rows][kCap]
  float* lane_s;     // [rows][8][kThreads]: lane 8 t + i at [i][t]
  float* lane_r;     // [rows][8][kThreads]
  PartOut* parts;    // [rows][kParts]
  uint32_t* ckeys;   // [rows][kParts][kPartList]
  int32_t* cidx;     // [rows][kParts][kPartList]
};

// A lower bound of the k-th largest of the keys (N per thread, 0 = no value), from a
// 256-bin histogram of their distance to the largest key at bf16 resolution (key >> 16):
// the lower edge of the first bin, from the top, at which k keys are reached.  At least
// k of the keys are at or above it, and it is within one bf16 step of the k-th largest.
// Returns 0 when the k largest do not fit the 256 bins (or there are fewer than k).
// Every thread calls it; uses hist, part and bin of L.  Its barriers order only LDS
// (lds_barrier): global loads the caller has in flight stay in flight across it when it
// is inlined (fine_bound_inline).

template <int N>
__device__ __forceinline__ uint32_t fine_bound_inline(RowsLds& L, const uint32_t (&key)[N],
                                                      int k) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  uint32_t kmax = 0u;
#pragma unroll
  for (int i = 0; i < N; ++i) kmax = max(kmax, key[i]);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, m));
  if (lane == 0) L.part[wave] = kmax;
  L.hist[t] = 0u;
  lds_barrier();
  kmax = max(max(L.part[0], L.part[1]), max(L.part[2], L.part[3]));
  const uint32_t top = kmax >> 16;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t d = top - (key[i] >> 16);
    if (key[i] != 0u && d < 256u) atomicAdd(&L.hist[d], 1u);
  }
  lds_barrier();
  if (t < 64) {
    const u32x4 c = reinterpret_cast<const u32x4*>(L.hist)[t];
    const uint32_t s = (c[0] + c[1]) + (c[2] + c[3]);
    uint32_t incl = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t o = (uint32_t)__shfl_up((int)incl, d);
      if (lane >= d) incl += o;
    }
    const uint64_t reach = __builtin_amdgcn_ballot_w64(k <= 1024 && incl >= (uint32_t)k);
    int bin = -1;
    if (reach != 0ull) {
      const int ls = __builtin_ctzll(reach);  // first lane (from the top) reaching k
      uint32_t cum = (uint32_t)__shfl((int)(incl - s), ls);
      const u32x4 cl = reinterpret_cast<const u32x4*>(L.hist)[ls];
      bool found = false;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        cum += cl[q];
        if (!found && cum >= (uint32_t)k) {
          bin = 4 * ls + q;
          found = true;
        }
      }
    }
    if (t == 0) L.bin = kmax == 0u ? -1 : bin;
  }
  lds_barrier();
  const int bin = L.bin;
  lds_barrier();
  return bin < 0 ? 0u : (top - (uint32_t)bin) << 16;
}

// Out-of-line form of four keys per thread.  The keys travel by value, in registers: an
// array passed by reference to a call would be stored to scratch memory and read back.
__device__ __noinline__ uint32_t fine_bound4(RowsLds& L, u32x4 key4, int k) {
  const uint32_t key[4] = {key4[0], key4[1], key4[2], key4[3]};
  return fine_bound_inline<4>(L, key, k);
}

template <int DT>
__device__ __forceinline__ const char* split_row(const SplitArgs& a, int64_t r) {
  const size_t esz = DT == BSX_DTYPE_FP32 ? 4 : 2;
  return r < a.n_a ? static_cast<const char*>(a.a) + r * a.V * esz
                   : static_cast<const char*>(a.b) + (r - a.n_a) * a.V * esz;
}

template <int DT>
__global__ void __launch_bounds__(kThreads) filter_parts_kernel(SplitArgs a) {
  __shared__ __align__(16) RowsLds L;
  __shared__ float s_max[kThreads / 64];
  constexpr int VW = DT == BSX_DTYPE_FP32 ? 2 : 1;
  const int t = threadIdx.x;
  // wave-uniform (scalar) so the lanes' group offsets below are scalar operands
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t r = blockIdx.x / kParts;
  const int p = (int)(blockIdx.x % kParts);
  const int64_t V = a.V;
  const char* row = split_row<DT>(a, r);
  const float c = a.c;
  const int k = a.top_k;
  const int ct = p * kPartThreads + (t & 63);  // canonical thread
  const int i0 = 2 * wave;                     // its lanes i0, i0 + 1
  const int64_t G = ceil_div(V, (int64_t)kGroup);
  const int64_t G_whole = V / kGroup;
  const __amdgpu_buffer_rsrc_t rsrc = row_rsrc(row, V * (int64_t)(VW == 2 ? 4 : 2));
  LaneState st[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    st[e].m = -INFINITY;
    st[e].s = 0.f;
    st[e].r = canon::kRefStart;
  }
  if (t == 0) L.count = 0;
  float lf = INFINITY;
  uint32_t hits = 0u;  // bit 2 j + e: group ct + 256 (8 j + i0 + e) reached the bound

  // Loads of the groups of rounds [cq, cq + 8 NR) of this thread's two lanes; a load past
  // the row returns 0 (buffer range), and groups past G_whole are not used from it.
  auto load_rounds = [&](int64_t cq, auto& w, auto nr_tag) {
    constexpr int NR = decltype(nr_tag)::value;
#pragma unroll
    for (int q = 0; q < NR; ++q)
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int h = 0; h < VW; ++h)
          w[q][e][h] = load_nt_b128(rsrc, (ct * VW + h) * 16,
                                    (int)(cq + 8 * q + i0 + e) * 4096 * VW);
  };
  auto unpack = [&](const u32x4 (&wv)[VW], float (&x)[8]) {
    if constexpr (DT == BSX_DTYPE_FP32) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x[u] = __uint_as_float(wv[0][u]);
        x[4 + u] = __uint_as_float(wv[1][u]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        x[2 * u] = lo_f32<DT>(wv[0][u]);
        x[2 * u + 1] = hi_f32<DT>(wv[0][u]);
      }
    }
  };
  auto max8f = [](const float (&x)[8]) {
    return __builtin_elementwise_maximum(
        __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[0], x[1]),
                                      __builtin_elementwise_maximum(x[2], x[3])),
        __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[4], x[5]),
                                      __builtin_elementwise_maximum(x[6], x[7])));
  };
  // One round cq of the two lanes, with the arithmetic of row_stats: a round whole for
  // the canonical thread (all 8 of its groups complete) by the whole-round path, the
  // other rounds group by group.
  auto do_round = [&](int64_t cq, const u32x4 (&wr)[2][VW], const float (&gm)[2],
                      const float (&x)[2][8]) {
    const bool whole_round = (int64_t)ct + 256 * (cq + 7) < G_whole;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int64_t g = (int64_t)ct + 256 * (cq + i0 + e);
      if (g < G_whole && !whole_round) {
        float gmf = x[e][0];
#pragma unroll
        for (int u = 1; u < 8; ++u) gmf = fmaxf(gmf, x[e][u]);
        canon::lane_update(st[e], x[e], 8, gmf, c);
        if (gmf >= lf) {
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (x[e][u] >= lf) push_candidate(L, x[e][u], g * kGroup + u);
        }
      } else if (g < G_whole) {
        const float rr = canon::lane_reference(st[e], gm[e], c);
        // = 0 + w0 + ... exactly: weights are >= +0
        float gs = canon::weight(x[e][0], c, -rr);
#pragma unroll
        for (int u = 1; u < 8; ++u) gs = gs + canon::weight(x[e][u], c, -rr);
        st[e].s = st[e].s + gs;
        hits |= (gm[e] >= lf ? 1u : 0u) << (2 * (int)(cq >> 3) + e);
      } else if (g < G) {
        float xp[8];
        const int n = load_group<DT>(row, g, V, true, xp);
        float gmp = xp[0];
#pragma unroll
        for (int u = 1; u < 8; ++u)
          if (u < n) gmp = fmaxf(gmp, xp[u]);
        canon::lane_update(st[e], xp, n, gmp, c);
        if (gmp >= lf) {
#pragma unroll
          for (int u = 0; u < 8; ++u)
            if (u < n && xp[u] >= lf) push_candidate(L, xp[u], g * kGroup + u);
        }
      }
    }
  };

  // The rounds after round 0 that are whole for every thread of the part run in batches
  // of kSplitRounds, software-pipelined over two register sets: each batch's loads go
  // out before the previous batch is computed, so a wave's arithmetic overlaps its own
  // loads (the workgroups of all rows start together and would otherwise alternate
  // between loading and computing in step).  Rounds [8, c_whole) are whole for every
  // thread of the part (its largest canonical thread is the binding one), in whole
  // batches; the rounds after them (at most a few) take do_round's per-group rules.
  constexpr int NR = kSplitRounds;
  const std::integral_constant<int, NR> nr;
  const int64_t ct_max = (int64_t)p * kPartThreads + kPartThreads - 1;
  const int64_t n_whole = G_whole > ct_max + 256 * 7 ? (G_whole - 1 - ct_max - 256 * 7) / 2048 + 1 : 0;
  const int64_t c_whole = 8 + ((n_whole - 1) / NR) * NR * 8;  // end of the batched rounds
  u32x4 wa[NR][2][VW], wb[NR][2][VW];

  // Round 0 on its own (the vocabulary is at least kSplitMinVocab, so all its groups are
  // whole): the part's bound is the k-th largest of its 512 first-round group maxima
  // (every thread calls the selection; -inf values are not counted).  The first batch's
  // loads go out before the selection, whose barriers order only LDS.
  {
    u32x4 w[1][2][VW];
    load_rounds(0, w, std::integral_constant<int, 1>());
    // (unconditional, so the load counts agree on every path; a load past the row
    // returns 0 and is not used when there is no batch)
    load_rounds(8, wa, nr);
    float x[2][8], gm[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      unpack(w[0][e], x[e]);
      gm[e] = max8f(x[e]);
    }
    // (-inf and negative NaN images are left out, as kth_key does)
    uint32_t gk[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      gk[e] = okey(gm[e]);
      if ((gk[e] >> kBinShift) < (uint32_t)kFirstFiniteBin) gk[e] = 0u;
    }
    uint32_t kb = fine_bound_inline<2>(L, gk, k);
    if (kb == 0u)  // the k largest spread over more than 256 bf16 steps
      kb = kth_key_call(L, gm[0], gm[1], -INFINITY, -INFINITY, -INFINITY, -INFINITY, -INFINITY,
                        -INFINITY, k);
    lf = kb == 0u ? INFINITY : key_value(kb);
    if (t == 0 && kb == 0u) L.count = kCands + 1;  // cannot list: the combine searches
    do_round(0, w[0], gm, x);
  }
  // Whole-round arithmetic only (a branch in this loop, even a rare one, costs it about
  // 40 registers): the groups whose maximum reaches the bound are noted as bits of hits.
  auto compute_whole = [&](int64_t cq0, const u32x4 (&w)[NR][2][VW]) {
#pragma unroll
    for (int q = 0; q < NR; ++q) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        float x[8];
        unpack(w[q][e], x);
        const float gm = max8f(x);
        const float rr = canon::lane_reference(st[e], gm, c);
        float gs = canon::weight(x[0], c, -rr);
#pragma unroll
        for (int u = 1; u < 8; ++u) gs = gs + canon::weight(x[u], c, -rr);
        st[e].s = st[e].s + gs;
        hits |= (gm >= lf ? 1u : 0u) << (2 * (int)((cq0 + 8 * q) >> 3) + e);
      }
    }
  };
  // wa holds rounds [8, 8 + 8 NR).  Every batch's loads are issued unconditionally (the
  // batch after the last one holds the first rounds after the loop), so the load counts
  // agree on every path and the wait before a batch's arithmetic leaves the next
  // batch's loads in flight.
  int64_t c0 = 8;
  if (c_whole > 8) {
    for (;;) {
      load_rounds(c0 + 8 * NR, wb, nr);
      compute_whole(c0, wa);
      c0 += 8 * NR;
      if (c0 >= c_whole) {
#pragma unroll
        for (int q = 0; q < NR; ++q)
#pragma unroll
          for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int h = 0; h < VW; ++h) wa[q][e][h] = wb[q][e][h];
        break;
      }
      load_rounds(c0 + 8 * NR, wa, nr);
      compute_whole(c0, wb);
      c0 += 8 * NR;
      if (c0 >= c_whole) break;
    }
  }
  // the rounds after the batches: the first NR from wa (loaded), the rest (if any) here
#pragma unroll
  for (int q = 0; q < NR; ++q) {
    const int64_t cq = c0 + 8 * q;
    if ((int64_t)ct + 256 * cq < G) {
      float x[2][8], gm[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        unpack(wa[q][e], x[e]);
        gm[e] = max8f(x[e]);
      }
      do_round(cq, wa[q], gm, x);
    }
  }
  for (int64_t cq = c0 + 8 * NR; (int64_t)ct + 256 * cq < G; cq += 8) {
    u32x4 w[1][2][VW];
    load_rounds(cq, w, std::integral_constant<int, 1>());
    float x[2][8], gm[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      unpack(w[0][e], x[e]);
      gm[e] = max8f(x[e]);
    }
    do_round(cq, w[0], gm, x);
  }
  // lane states and the part's maximum
  // lane 8 ct + i at [i][ct]: a wave's stores of one i cover 64 consecutive floats
  float* ls = a.lane_s + r * kLanes;
  float* lr = a.lane_r + r * kLanes;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    ls[(i0 + e) * kThreads + ct] = st[e].s;
    lr[(i0 + e) * kThreads + ct] = st[e].r;
  }
  float mx = fmaxf(st[0].m, st[1].m);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  if ((t & 63) == 0) s_max[wave] = mx;
  // The groups that reached the bound (a few hundred per part) are listed in LDS and
  // read again one per thread: a single round trip, where a thread reading its own noted
  // groups in turn would put several dependent ones on the workgroup's tail.
  if (t == 0) L.ng = 0;
  lds_barrier();  // (the lane-state stores need not land first)
  uint32_t hb = hits;
#pragma unroll 1
  while (hb != 0u) {
    const int bit = __builtin_ctz(hb);
    hb &= hb - 1u;
    const int slot = atomicAdd(&L.ng, 1);
    if (slot < kBins) L.hist[slot] = (uint32_t)(ct + 256 * (8 * (bit >> 1) + i0 + (bit & 1)));
  }
  __syncthreads();
  const int ng = min(L.ng, kBins);
  for (int q = t; q < ng; q += kThreads) {
    const int64_t g = L.hist[q];
    float xg[8];
    load8<DT>(row, g, xg);
    uint32_t hm = 0u;
#pragma unroll
    for (int u = 0; u < 8; ++u) hm |= (xg[u] >= lf ? 1u : 0u) << u;
#pragma unroll 1
    while (hm != 0u) {
      const int u = __builtin_ctz(hm);
      hm &= hm - 1u;
      // the element again from cache: indexing xg by a run-time u would put it in
      // scratch memory
      push_candidate(L, load_one<DT>(row, g * kGroup + u), g * kGroup + u);
    }
  }
  __syncthreads();
  if (L.ng > kBins && t == 0) L.count = kCands + 1;  // could not note them all
  __syncthreads();
  const int n = L.count;
  PartOut po;
  po.m = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  po.kb = 0u;
  po.count = -1;
  po.pad = 0;
  if (n <= kCands) {
    // keep the keys at or above the part's k-th largest listed key (its k-th largest
    // element: every element at or above the bound is listed)
    constexpr int PER = kCands / kThreads;
    uint32_t ck[PER];
    int32_t ci[PER];
    float cv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cv[j] = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int s = t + kThreads * j;
      ck[j] = s < n ? L.ckey[s] : 0u;
      ci[j] = s < n ? L.cidx[s] : 0;
      if (s < n) cv[j] = key_value(ck[j]);
    }
    static_assert(PER == 4, "fine_bound4 takes four keys per thread");
    uint32_t lk[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) lk[j] = t + kThreads * j < n ? ck[j] : 0u;
    uint32_t kb = fine_bound4(L, u32x4{lk[0], lk[1], lk[2], lk[3]}, k);
    if (kb == 0u)
      kb = kth_key_call(L, cv[0], cv[1], cv[2], cv[3], cv[4], cv[5], cv[6], cv[7], k);
    if (t == 0) L.nk = 0;
    __syncthreads();
    uint32_t* okeys = a.ckeys + (r * kParts + p) * kPartList;
    int32_t* oidx = a.cidx + (r * kParts + p) * kPartList;
    if (kb != 0u) {
#pragma unroll
      for (int j = 0; j < PER; ++j)
        if (t + kThreads * j < n && ck[j] >= kb) {
          const int slot = atomicAdd(&L.nk, 1);
          if (slot < kPartList) {
            okeys[slot] = ck[j];
            oidx[slot] = ci[j];
          }
        }
    }
    lds_barrier();  // (the key stores need not land first)
    if (kb != 0u && L.nk <= kPartList) {
      po.kb = kb;
      po.count = L.nk;
    }
  }
  if (t == 0) a.parts[r * kParts + p] = po;
}

// The combine of row r by the whole workgroup (filter_combine_kernel, and the fallback of
// filter_request_kernel).
template <int DT>
__device__ __forceinline__ void combine_row(const SplitArgs& a, int64_t r, RowsLds& L,
                                            float (&wave_val)[kThreads / 64]) {
  const int t = threadIdx.x;
  const int64_t V = a.V;
  const char* row = split_row<DT>(a, r);
  const float c = a.c;
  const bool use_k = a.top_k > 0 && (int64_t)a.top_k < V;
  const bool use_p = a.top_p > 0.f && a.top_p < 1.f;
  // Every load of the row's records goes out at once: the part records, the lane states
  // and all kParts * kPartList key slots of the parts (masked by their counts below).
  PartOut po[kParts];
#pragma unroll
  for (int q = 0; q < kParts; ++q) po[q] = a.parts[r * kParts + q];
  constexpr int SL = kParts * kPartList / kThreads;
  static_assert(kParts * kPartList % kThreads == 0, "key slots split evenly over threads");
  uint32_t sk[SL];
  int32_t si[SL];
#pragma unroll
  for (int j = 0; j < SL; ++j) {
    const int64_t slot = r * kParts * kPartList + t + kThreads * j;
    sk[j] = a.ckeys[slot];
    si[j] = a.cidx[slot];
  }
  // (M, Z): row_stats' epilogue on the lane states of the parts
  float mx = po[0].m;
#pragma unroll
  for (int q = 1; q < kParts; ++q) mx = fmaxf(mx, po[q].m);
  const float rho_m = mx * c;
  // lane 8 t + i of the row at [i][t] (the parts' layout)
  const float* lsr = a.lane_s + r * kLanes + t;
  const float* lrr = a.lane_r + r * kLanes + t;
  float sv[8], rv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    sv[i] = lsr[i * kThreads];
    rv[i] = lrr[i * kThreads];
  }
  float rs[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) rs[i] = canon::lane_rescaled(LaneState{-INFINITY, sv[i], rv[i]}, rho_m);
  float sum = ((rs[0] + rs[1]) + (rs[2] + rs[3])) + ((rs[4] + rs[5]) + (rs[6] + rs[7]));
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) sum = sum + __shfl_xor(sum, m);
  if ((t & 63) == 0) wave_val[t >> 6] = sum;
  if (t == 0) L.count = 0;
  __syncthreads();
  const float M = mx;
  const float Z = (wave_val[0] + wave_val[1]) + (wave_val[2] + wave_val[3]);
  const float neg = -(M * c);
  const uint64_t target = use_p ? (uint64_t)ceilf((a.top_p * Z) * 0x1p40f) : 0ull;

  bool listed = false;
  bool can = true;
  uint32_t bkey = 0u;
#pragma unroll
  for (int q = 0; q < kParts; ++q) {
    can = can && po[q].count >= 0;
    bkey = max(bkey, po[q].kb);
  }
  if (can) {
    // the written keys at or above B = max kb_p: every element of the row there
#pragma unroll
    for (int j = 0; j < SL; ++j) {
      const int slot = t + kThreads * j;
      const int q = slot / kPartList;
      int cnt = po[0].count;
#pragma unroll
      for (int qq = 1; qq < kParts; ++qq) cnt = q == qq ? po[qq].count : cnt;
      if (slot - q * kPartList < cnt && sk[j] >= bkey) {
        const int at = atomicAdd(&L.count, 1);
        if (at < kCands) {
          L.ckey[at] = sk[j];
          L.cidx[at] = si[j];
        }
      }
    }
    __syncthreads();
    const int n = L.count;
    if (n <= kCands) listed = walk(L, n, c, neg, use_k, use_p, a.top_k, target, a.lists + r * kCap);
  }
  if (!listed) {
    const size_t esz = DT == BSX_DTYPE_FP32 ? 4 : 2;
    const bool vec = ((V * esz) % 16 == 0) && (((uintptr_t)row) % 16 == 0);
    large_threshold<DT>(L, row, V, vec, c, neg, use_k, use_p, a.top_k, target);
  }
  write_info(L, a.info + r, M);
}

template <int DT>
__global__ void __launch_bounds__(kThreads) filter_combine_kernel(SplitArgs a) {
  __shared__ __align__(16) RowsLds L;
  __shared__ float wave_val[kThreads / 64];
  combine_row<DT>(a, blockIdx.x, L, wave_val);
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
  uint64_t* tiles;   // [B][2][draw_tiles(V)] tile sums of the whole-row draws
  int tiles_ready;   // filter_tiles_kernel ran (else a row without a list sums its tiles
                     // in filter_chain_kernel)
  int32_t* out_ids;  // [B, k+1]
  int32_t* accepted;
  int32_t* emitted;
};

// Tiles of a whole-row draw: 64 lanes x E consecutive elements (E a multiple of 8), at
// most kMaxTiles of them; filter_tiles_kernel sums kTilesPerPart per workgroup.
constexpr int kTilesPerPart = 8;
static_assert(kTilesPerPart % (kThreads / 64) == 0, "whole tiles per wave");
__host__ __device__ inline int draw_tile_elems(int64_t V) {
  return kGroup * (int)ceil_div(V, (int64_t)kMaxTiles * 64 * kGroup);
}
__host__ __device__ inline int draw_tiles(int64_t V) {
  return (int)ceil_div(V, 64LL * draw_tile_elems(V));
}

template <int DT>
struct Filtered {
  const void* row;
  float c, nmc, inv;
  uint32_t tk;
  __device__ __forceinline__ float p(int64_t v) const {
    const float x = load_one<DT>(row, v);
    return okey(x) >= tk ? canon::weight(x, c, nmc) * inv : 0.0f;
  }
  // p of the 8 elements [v0, v0 + 8) of a 16-byte aligned row (v0 a multiple of 8)
  __device__ __forceinline__ void p8(int64_t v0, float (&out)[8]) const {
    float x[8];
    load8<DT>(row, v0 / kGroup, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = okey(x[e]) >= tk ? canon::weight(x[e], c, nmc) * inv : 0.0f;
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

// Ratio tests of request b, by the first wave (lane i tests draft position i): the
// first rejected position (k if none) in *s_j, the number accepted in *s_n.
template <int DT>
__device__ void ratio_tests(const ChainArgs& a, int b, int* s_j, int* s_n) {
  const int t = threadIdx.x;
  if (t >= 64) return;
  const int k = a.k;
  const int64_t V = a.V;
  const int64_t trow0 = (int64_t)b * (k + 1);
  const int64_t drow0 = (int64_t)a.B * (k + 1) + (int64_t)b * k;
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
    *s_j = j;
    *s_n = cnt;
  }
}

// Fixed-point weights of the draw of a request whose chain stops at position j:
// r(v) = fx40(max(p'(v) - q'(v), 0)) against the draft (its filtered probability, or one
// at the draft token for a one-hot draft) when j < k, and fx40(p'(v)) without it (all
// accepted, or a residual that sums to 0).
template <int DT>
struct DrawRow {
  Filtered<DT> P, Q;
  bool has_q, qlog, vec8;
  int64_t xj, V;

  __device__ uint64_t at(int64_t v, bool with_q) const {
    const float p = P.p(v);
    if (!with_q) return fx40(p);
    const float q = qlog ? Q.p(v) : (v == xj ? 1.0f : 0.0f);
    return fx40(fmaxf(p - q, 0.0f));
  }
  // both weights of the 8 elements [v0, v0 + 8) (v0 a multiple of 8): rq against the
  // draft (when has_q), rp without; one 16-byte load per row when the rows allow it
  __device__ void at8(int64_t v0, uint64_t (&rq)[8], uint64_t (&rp)[8]) const {
    if (vec8 && v0 + 8 <= V) {
      float p[8], q[8];
      P.p8(v0, p);
      if (has_q && qlog) Q.p8(v0, q);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        rp[e] = fx40(p[e]);
        if (has_q) {
          const float qe = qlog ? q[e] : (v0 + e == xj ? 1.0f : 0.0f);
          rq[e] = fx40(fmaxf(p[e] - qe, 0.0f));
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        rp[e] = v0 + e < V ? at(v0 + e, false) : 0ull;
        if (has_q) rq[e] = v0 + e < V ? at(v0 + e, true) : 0ull;
      }
    }
  }
  // sums of rq and rp over the E elements [v0, v0 + E) (E a multiple of 8)
  __device__ void sums(int64_t v0, int E, uint64_t& sq, uint64_t& sp) const {
    sq = 0ull;
    sp = 0ull;
    for (int e0 = 0; e0 < E && v0 + e0 < V; e0 += 8) {
      uint64_t rq[8], rp[8];
      at8(v0 + e0, rq, rp);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sp += rp[e];
        if (has_q) sq += rq[e];
      }
    }
  }
};

template <int DT>
__device__ DrawRow<DT> draw_row(const ChainArgs& a, int b, int j) {
  const int k = a.k;
  const int64_t V = a.V;
  const int64_t trow = (int64_t)b * (k + 1) + j;
  DrawRow<DT> d;
  d.V = V;
  d.P = filtered_row<DT>(a.t_logits, trow, V, a.info[trow], a.c);
  d.has_q = j < k;
  d.qlog = d.has_q && a.d_logits != nullptr;
  d.xj = d.has_q ? a.draft_ids[(int64_t)b * k + j] : -1;
  d.Q = Filtered<DT>{};
  if (d.qlog)
    d.Q = filtered_row<DT>(a.d_logits, (int64_t)b * k + j, V,
                           a.info[(int64_t)a.B * (k + 1) + (int64_t)b * k + j], a.c);
  const size_t esz = DT == BSX_DTYPE_FP32 ? 4 : 2;
  d.vec8 = (V * (int64_t)esz) % 16 == 0 && ((uintptr_t)d.P.row) % 16 == 0 &&
           (!d.qlog || ((uintptr_t)d.Q.row) % 16 == 0);
  return d;
}

// Tile sums of a whole-row draw: grid (B, parts); part p sums the tiles
// [kTilesPerPart p, kTilesPerPart (p + 1)) of the row request b's chain stops at, one
// wave per tile, into tiles[b][0][T] (against the draft) and tiles[b][1][T] (without),
// unless that row has a kept list.
template <int DT>
__global__ void __launch_bounds__(kThreads) filter_tiles_kernel(ChainArgs a) {
  __shared__ int s_j, s_n;
  const int b = blockIdx.x;
  // nothing to sum when every target row of the request has a kept list (the usual case
  // with a small top_k): one read of the row infos instead of the ratio tests
  {
    const int tw = threadIdx.x & 63;
    bool listed = true;
    for (int i = tw; i <= a.k; i += 64) listed &= a.info[(int64_t)b * (a.k + 1) + i].n_list >= 0;
    if (__builtin_amdgcn_ballot_w64(!listed) == 0ull) return;  // the same in every wave
  }
  ratio_tests<DT>(a, b, &s_j, &s_n);
  __syncthreads();
  const int j = s_j;
  if (a.info[(int64_t)b * (a.k + 1) + j].n_list >= 0) return;
  const DrawRow<DT> R = draw_row<DT>(a, b, j);
  const int E = draw_tile_elems(a.V);
  const int ntiles = draw_tiles(a.V);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint64_t* ts = a.tiles + (int64_t)b * 2 * ntiles;
  constexpr int U = kTilesPerPart / (kThreads / 64);
  uint64_t sq[U], sp[U];
  // the tiles of a wave summed together: their loads go out together
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int T = blockIdx.y * kTilesPerPart + (kThreads / 64) * u + wave;
    R.sums((int64_t)(T < ntiles ? T : 0) * 64 * E + (int64_t)lane * E, E, sq[u], sp[u]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int T = blockIdx.y * kTilesPerPart + (kThreads / 64) * u + wave;
    const uint64_t q = R.has_q ? wave_sum_u64(sq[u]) : 0ull;
    const uint64_t p = wave_sum_u64(sp[u]);
    if (lane == 0 && T < ntiles) {
      ts[T] = q;
      ts[ntiles + T] = p;
    }
  }
}

// LDS of the chain of one request.
struct ChainLds {
  int s_j, s_n, s_tok, s_last, s_tile, s_last_tile;
  int32_t lv[kCap];
  uint64_t lr[kCap];
  uint64_t s_acc, s_tbase;
  uint64_t excl[kThreads];
  uint64_t s_wave[kThreads / 64];
  uint64_t tsum[kMaxTiles];
  uint64_t tloc[2][kMaxTiles];  // tile sums made here (tiles_ready == 0)
};

// The chain of request b by the whole workgroup, from the row infos and lists in the
// workspace (filter_chain_kernel, and the fallback of filter_request_kernel).
template <int DT>
__device__ __forceinline__ void chain_request(const ChainArgs& a, int b, ChainLds& S) {
  int &s_j = S.s_j, &s_n = S.s_n, &s_tok = S.s_tok, &s_last = S.s_last, &s_tile = S.s_tile,
      &s_last_tile = S.s_last_tile;
  int32_t(&lv)[kCap] = S.lv;
  uint64_t(&lr)[kCap] = S.lr;
  uint64_t &s_acc = S.s_acc, &s_tbase = S.s_tbase;
  uint64_t(&excl)[kThreads] = S.excl;
  uint64_t(&s_wave)[kThreads / 64] = S.s_wave;
  uint64_t(&tsum)[kMaxTiles] = S.tsum;
  uint64_t(&tloc)[2][kMaxTiles] = S.tloc;
  const int t = threadIdx.x;
  const int k = a.k;
  const int64_t V = a.V;
  const int64_t trow0 = (int64_t)b * (k + 1);

  ratio_tests<DT>(a, b, &s_j, &s_n);
  if (t == 0) {
    s_tok = INT_MAX;
    s_last = -1;
    s_last_tile = 0;
  }
  __syncthreads();
  const int j = s_j;
  const RowInfo ti = a.info[trow0 + j];
  const DrawRow<DT> R = draw_row<DT>(a, b, j);
  const bool has_q = R.has_q;
  const float u = a.uniforms[trow0 + k];
  int tok = -1;
  if (ti.n_list >= 0) {
    const int n = ti.n_list;
    const int32_t v = t < n ? a.lists[(trow0 + j) * kCap + t] : 0;
    uint64_t total = 0ull;
    for (int pass = 0; pass < 2; ++pass) {
      const bool with_q = has_q && pass == 0;
      if (pass == 1 && !has_q) break;
      const uint64_t w = t < n ? R.at(v, with_q) : 0ull;
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
    // No list: the tile sums of filter_tiles_kernel (tiles of 64 lanes x E consecutive
    // elements), their prefix, then the lane and the element inside the tile that holds
    // the draw point.
    const int E = draw_tile_elems(V);
    const int64_t tile = 64LL * E;
    const int ntiles = draw_tiles(V);
    const uint64_t* ts = a.tiles + (int64_t)b * 2 * ntiles;
    const int wave = t >> 6, lane = t & 63;
    if (!a.tiles_ready) {
      // the tile sums of filter_tiles_kernel, here (it was not launched: with a small
      // top_k every row is expected to list, and a row that does not is rare); each wave
      // sums 8 of its tiles per round, their loads together
      constexpr int U = 8;
      for (int T0 = wave; T0 < ntiles; T0 += (kThreads / 64) * U) {
        uint64_t sq[U], sp[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int T = T0 + (kThreads / 64) * u;
          R.sums((int64_t)(T < ntiles ? T : 0) * tile + (int64_t)lane * E, E, sq[u], sp[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int T = T0 + (kThreads / 64) * u;
          const uint64_t q = has_q ? wave_sum_u64(sq[u]) : 0ull;
          const uint64_t pp = wave_sum_u64(sp[u]);
          if (lane == 0 && T < ntiles) {
            tloc[0][T] = q;
            tloc[1][T] = pp;
          }
        }
      }
      __syncthreads();
    }
    uint64_t total = 0ull;
    bool with_q = has_q;
    for (int pass = 0; pass < 2; ++pass) {
      with_q = has_q && pass == 0;
      if (pass == 1 && !has_q) break;
      for (int T = t; T < ntiles; T += kThreads)
        tsum[T] = a.tiles_ready ? ts[(with_q ? 0 : ntiles) + T] : tloc[with_q ? 0 : 1][T];
      __syncthreads();
      // thread t: tiles [8t, 8t + 8); exclusive prefix of those groups
      uint64_t mine = 0ull;
      for (int i = 0; i < kMaxTiles / kThreads; ++i) {
        const int T = t * (kMaxTiles / kThreads) + i;
        if (T < ntiles) mine += tsum[T];
      }
      const uint64_t incl = wave_prefix_u64(mine);
      if (lane == 63) s_wave[wave] = incl;
      __syncthreads();
      uint64_t off = 0ull;
      total = 0ull;
      for (int w = 0; w < kThreads / 64; ++w) {
        if (w < wave) off += s_wave[w];
        total += s_wave[w];
      }
      excl[t] = off + (incl - mine);
      __syncthreads();
      if (total != 0ull) break;
    }
    if (total != 0ull) {
      const uint64_t tp = canon::draw_point(u, total);
      if (t == 0) s_tile = -1;
      __syncthreads();
      // the tile whose running sum first exceeds tp (else the last non-empty tile)
      uint64_t base = excl[t];
      for (int i = 0; i < kMaxTiles / kThreads; ++i) {
        const int T = t * (kMaxTiles / kThreads) + i;
        if (T >= ntiles) break;
        const uint64_t x = tsum[T];
        if (x != 0ull) {
          if (tp >= base && tp < base + x) {
            s_tile = T;
            s_tbase = base;
          }
          atomicMax(&s_last_tile, T);
        }
        base += x;
      }
      __syncthreads();
      const bool found = s_tile >= 0;
      const int T = found ? s_tile : s_last_tile;
      if (wave == 0) {
        const int64_t v0 = T * tile + (int64_t)lane * E;
        uint64_t sq, sp;
        R.sums(v0, E, sq, sp);
        const uint64_t ls = with_q ? sq : sp;
        const uint64_t incl = wave_prefix_u64(ls);
        const uint64_t lexcl = incl - ls;
        if (found) {
          const uint64_t tt = tp - s_tbase;
          if (ls != 0ull && tt >= lexcl && tt < incl) {
            uint64_t cum = lexcl;
            bool done = false;
            for (int e0 = 0; e0 < E && v0 + e0 < V && !done; e0 += 8) {
              uint64_t rq[8], rp[8];
              R.at8(v0 + e0, rq, rp);
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                cum += with_q ? rq[e] : rp[e];
                if (!done && cum > tt) {
                  s_tok = (int)(v0 + e0 + e);
                  done = true;
                }
              }
            }
          }
        } else {
          const uint64_t nz = __builtin_amdgcn_ballot_w64(ls != 0ull);
          if (nz != 0ull && lane == 63 - __builtin_clzll(nz)) {
            for (int e = E - 1; e >= 0; --e)
              if (v0 + e < V && R.at(v0 + e, with_q) != 0ull) {
                s_tok = (int)(v0 + e);
                break;
              }
          }
        }
      }
      __syncthreads();
      tok = s_tok != INT_MAX ? s_tok : -1;
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

template <int DT>
__global__ void __launch_bounds__(kThreads) filter_chain_kernel(ChainArgs a) {
  __shared__ ChainLds S;
  chain_request<DT>(a, blockIdx.x, S);
}

// ---- The split path's tail in one launch per request --------------------------------
//
// filter_request_kernel (grid B, four waves) replaces filter_combine_kernel +
// filter_chain_kernel for requests of at most kFastRows rows with one-hot drafts.  It
// keeps filter_combine_kernel's arithmetic and order:
//   - (M, Z): wave w evaluates slice w of every row's canonical tree (canonical threads
//     64 w .. 64 w + 63: the same eight-term sums and the same butterfly within the
//     slice), and Z is the same sum of the four slice sums;
//   - the walk of row i (wave i mod 4) over the parts' keys at or above the largest part
//     bound: t* is the largest key whose count (keys at or above it) reaches top_k or
//     whose mass reaches the target.  Counts and masses are integers, so any evaluation
//     order gives the same t* and Z_K.  Here the top_k-th largest key T is selected first
//     (a bitwise search over ballots), and only the keys at or above T get their count
//     and mass: T itself reaches by count, so t* >= T.  With fewer than top_k keys, T is
//     0 and every key is examined, as in the workgroup walk.
// It covers the rows whose parts each listed at most kFastPart keys and whose walk finds
// t* among them.  A request with any other row runs combine_row on those rows and
// chain_request (the whole workgroup, through the workspace), which give the same bits.
// The chain then runs on the first wave from the rows' infos and kept keys in LDS; an
// element's weight is a function of its key (key_value(okey(x)) is x, or +0 for -0,
// whose weight is the same).
constexpr int kFastRows = 8;                    // rows of a request (k + 1)
constexpr int kFastPart = 32;                   // keys of a part read by the walk
constexpr int kFastCands = kParts * kFastPart;  // candidate slots of a row: two per lane
constexpr int kFastTopK = kFastPart - 8;        // largest top_k sent to filter_request_kernel
static_assert(kFastCands == 128 && kFastPart <= kPartList, "two candidate slots per lane");

struct FastLds {
  uint32_t key[kFastRows][kFastCands];  // the kept keys of the row (keys >= t*)
  int32_t idx[kFastRows][kFastCands];   // and their indices
  uint32_t tkey[kFastRows][kFastCands]; // the walk's keys >= T, pads of key 0 to x4
  uint64_t tm[kFastRows][kFastCands];   // their masses (the chain's row: draw weights)
  RowInfo info[kFastRows];
  int ok[kFastRows];                    // the wave walk finished the row
  float zs[kFastRows][kThreads / 64];   // slice sums of the canonical trees
  int64_t xid[kFastRows];               // draft token of position i
  float xval[kFastRows];                // the target logit of row i at it (when in range)
};

// Set bits of m in the lanes below this one.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Wave reductions on the DPP network (no LDS round trips): quad permutations [1,0,3,2]
// and [2,3,0,1] (partners l ^ 1, l ^ 2), then the mirrors within 8 and 16 lanes, which
// reach the other half of the 8 / 16 lanes once each half holds one value, then the four
// rows of 16 read as scalars.  For the float sum this is the butterfly
// s = s + shfl_xor(s, m), m = 1 .. 32, bit for bit: each step adds the same two values
// as the butterfly (in either order, which addition does not see), and the last two
// steps are (R0 + R1) + (R2 + R3) over the row sums.  Every lane must be active.
constexpr int kDppXor1 = 0xb1, kDppXor2 = 0x4e, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  return ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)v);
}

__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}

__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int l) {
  return ((uint64_t)lane_u32((uint32_t)(v >> 32), l) << 32) | lane_u32((uint32_t)v, l);
}

__device__ __forceinline__ float wave_tree_sum(float s) {
  s = s + __uint_as_float(dpp_u32<kDppXor1>(__float_as_uint(s)));
  s = s + __uint_as_float(dpp_u32<kDppXor2>(__float_as_uint(s)));
  s = s + __uint_as_float(dpp_u32<kDppHalfMirror>(__float_as_uint(s)));
  s = s + __uint_as_float(dpp_u32<kDppMirror>(__float_as_uint(s)));
  const float r0 = __uint_as_float(lane_u32(__float_as_uint(s), 0));
  const float r1 = __uint_as_float(lane_u32(__float_as_uint(s), 16));
  const float r2 = __uint_as_float(lane_u32(__float_as_uint(s), 32));
  const float r3 = __uint_as_float(lane_u32(__float_as_uint(s), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<kDppXor1>(v));
  v = max(v, dpp_u32<kDppXor2>(v));
  v = max(v, dpp_u32<kDppHalfMirror>(v));
  v = max(v, dpp_u32<kDppMirror>(v));
  return max(max(lane_u32(v, 0), lane_u32(v, 16)), max(lane_u32(v, 32), lane_u32(v, 48)));
}

__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
  v |= dpp_u32<kDppXor1>(v);
  v |= dpp_u32<kDppXor2>(v);
  v |= dpp_u32<kDppHalfMirror>(v);
  v |= dpp_u32<kDppMirror>(v);
  return (lane_u32(v, 0) | lane_u32(v, 16)) | (lane_u32(v, 32) | lane_u32(v, 48));
}

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  v = min(v, dpp_u64<kDppXor1>(v));
  v = min(v, dpp_u64<kDppXor2>(v));
  v = min(v, dpp_u64<kDppHalfMirror>(v));
  v = min(v, dpp_u64<kDppMirror>(v));
  return min(min(lane_u64(v, 0), lane_u64(v, 16)), min(lane_u64(v, 32), lane_u64(v, 48)));
}

__device__ __forceinline__ uint64_t wave_add_u64(uint64_t v) {
  v += dpp_u64<kDppXor1>(v);
  v += dpp_u64<kDppXor2>(v);
  v += dpp_u64<kDppHalfMirror>(v);
  v += dpp_u64<kDppMirror>(v);
  return (lane_u64(v, 0) + lane_u64(v, 16)) + (lane_u64(v, 32) + lane_u64(v, 48));
}

__device__ __forceinline__ int wave_min_i32(int v) {
  v = min(v, (int)dpp_u32<kDppXor1>((uint32_t)v));
  v = min(v, (int)dpp_u32<kDppXor2>((uint32_t)v));
  v = min(v, (int)dpp_u32<kDppHalfMirror>((uint32_t)v));
  v = min(v, (int)dpp_u32<kDppMirror>((uint32_t)v));
  return min(min((int)lane_u32(v, 0), (int)lane_u32(v, 16)),
             min((int)lane_u32(v, 32), (int)lane_u32(v, 48)));
}

__device__ __forceinline__ int wave_max_i32(int v) {
  v = max(v, (int)dpp_u32<kDppXor1>((uint32_t)v));
  v = max(v, (int)dpp_u32<kDppXor2>((uint32_t)v));
  v = max(v, (int)dpp_u32<kDppHalfMirror>((uint32_t)v));
  v = max(v, (int)dpp_u32<kDppMirror>((uint32_t)v));
  return max(max((int)lane_u32(v, 0), (int)lane_u32(v, 16)),
             max((int)lane_u32(v, 32), (int)lane_u32(v, 48)));
}

// What the walk of a row reads: the part records and the first kFastPart key slots of
// each part (slot s = lane + 64 h of the lane: part s / kFastPart).
struct WalkIn {
  PartOut po[kParts];
  uint32_t sk[2];
  int32_t si[2];
};

__device__ __forceinline__ void walk_load(const SplitArgs& a, int64_t r, WalkIn& in) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int q = 0; q < kParts; ++q) in.po[q] = a.parts[r * kParts + q];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int s = lane + 64 * h;
    const int64_t at = (r * kParts + s / kFastPart) * kPartList + s % kFastPart;
    in.sk[h] = a.ckeys[at];
    in.si[h] = a.cidx[at];
  }
}

// Loaded values in registers here: a wave's loads are in flight together before the
// first wait (the compiler would otherwise move loads into the branches that use them).
__device__ __forceinline__ void walk_pin(const WalkIn& in) {
#pragma unroll
  for (int q = 0; q < kParts; ++q)
    asm volatile("" ::"v"(in.po[q].m), "v"(in.po[q].kb), "v"(in.po[q].count));
  asm volatile("" ::"v"(in.sk[0]), "v"(in.sk[1]), "v"(in.si[0]), "v"(in.si[1]));
}

// The top_k-th largest of the keys held (kj[h] where val[h]), or 0 when fewer than top_k
// are held: the largest T with at least top_k keys >= T, built bit by bit from the top.
// Every held key has the largest key's bits outside `diff` (the bits where some key
// differs from it), so T starts from those and only the bits of diff are decided.
__device__ __forceinline__ uint32_t kth_largest_held(const uint32_t (&kj)[2], const bool (&val)[2],
                                                     int top_k) {
  const int held = __builtin_popcountll(__builtin_amdgcn_ballot_w64(val[0])) +
                   __builtin_popcountll(__builtin_amdgcn_ballot_w64(val[1]));
  if (held < top_k) return 0u;
  const uint32_t hi = wave_max_u32(max(val[0] ? kj[0] : 0u, val[1] ? kj[1] : 0u));
  uint32_t diff = wave_or_u32((val[0] ? kj[0] ^ hi : 0u) | (val[1] ? kj[1] ^ hi : 0u));
  uint32_t T = hi & ~diff;
  while (diff != 0u) {
    const uint32_t bit = 1u << (31 - __builtin_clz(diff));
    diff &= ~bit;
    const uint32_t cand = T | bit;
    const int c = __builtin_popcountll(__builtin_amdgcn_ballot_w64(val[0] && kj[0] >= cand)) +
                  __builtin_popcountll(__builtin_amdgcn_ballot_w64(val[1] && kj[1] >= cand));
    if (c >= top_k) T = cand;
  }
  return T;
}

// The walk of row r by one wave, with its statistics (M, Z): its info and kept list into
// the workspace and F (slot `slot`).  Returns false (in every lane, writing no info)
// when the row needs the workgroup's combine.
__device__ __forceinline__ bool fast_walk(const SplitArgs& a, int64_t r, int slot,
                                          const WalkIn& in, float M, float Z, FastLds& F) {
  const int lane = threadIdx.x & 63;
  const float c = a.c;
  const bool use_k = a.top_k > 0 && (int64_t)a.top_k < a.V;
  const bool use_p = a.top_p > 0.f && a.top_p < 1.f;
  if (!use_k) return false;
  bool can = true;
  uint32_t bkey = 0u;
#pragma unroll
  for (int q = 0; q < kParts; ++q) {
    can = can && in.po[q].count >= 0 && in.po[q].count <= kFastPart;
    bkey = max(bkey, in.po[q].kb);
  }
  if (!can) return false;
  const float neg = -(M * c);
  const uint64_t target = use_p ? (uint64_t)ceilf((a.top_p * Z) * 0x1p40f) : 0ull;
  // the written keys at or above B = max kb_p: every element of the row there
  bool val[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int s = lane + 64 * h;
    const int q = s / kFastPart;
    int cnt = in.po[0].count;
#pragma unroll
    for (int qq = 1; qq < kParts; ++qq) cnt = q == qq ? in.po[qq].count : cnt;
    val[h] = s % kFastPart < cnt && in.sk[h] >= bkey;
  }
  const uint32_t T = kth_largest_held(in.sk, val, a.top_k);
  // count and mass of each key >= T over the keys >= T (every key at or above one of
  // them is one of them); the keys in turn, from the ballot of each slot
  bool top[2];
  uint64_t cm[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    top[h] = val[h] && in.sk[h] >= T;
    cm[h] = top[h] ? fx40(canon::weight(key_value(in.sk[h]), c, neg)) : 0ull;
  }
  // the keys >= T and their masses into LDS (slot order, pads of key 0 and mass 0 to a
  // multiple of 4), then each key's count and mass over them, four per read
  typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
  const uint64_t t0 = __builtin_amdgcn_ballot_w64(top[0]);
  const uint64_t t1 = __builtin_amdgcn_ballot_w64(top[1]);
  const int m0 = __builtin_popcountll(t0);
  const int m = m0 + __builtin_popcountll(t1);
  const int m4 = (m + 3) & ~3;
  uint32_t* tkey = F.tkey[slot];
  uint64_t* tm = F.tm[slot];
  if (top[0]) {
    tkey[lanes_below(t0)] = in.sk[0];
    tm[lanes_below(t0)] = cm[0];
  }
  if (top[1]) {
    tkey[m0 + lanes_below(t1)] = in.sk[1];
    tm[m0 + lanes_below(t1)] = cm[1];
  }
  if (lane < m4 - m) {
    tkey[m + lane] = 0u;
    tm[m + lane] = 0ull;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  uint32_t cnt[2] = {0u, 0u};
  uint64_t ms[2] = {0ull, 0ull};
  for (int q = 0; q < m4; q += 4) {
    const u32x4 kk = *reinterpret_cast<const u32x4*>(tkey + q);
    const u64x2 ma = *reinterpret_cast<const u64x2*>(tm + q);
    const u64x2 mb = *reinterpret_cast<const u64x2*>(tm + q + 2);
    const uint64_t mm[4] = {ma[0], ma[1], mb[0], mb[1]};
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bool ge = kk[e] >= in.sk[h];
        cnt[h] += ge ? 1u : 0u;
        ms[h] += ge ? mm[e] : 0ull;
      }
  }
  // t* = the largest key that reaches; Z_K = its mass, which is the smallest mass of the
  // keys that reach (mass does not increase with the key; equal keys hold equal masses)
  uint32_t best = 0u;
  uint64_t least = ~0ull;
#pragma unroll
  for (int h = 0; h < 2; ++h)
    if (top[h] && reached(use_k, use_p, cnt[h], ms[h], a.top_k, target)) {
      best = max(best, in.sk[h]);
      least = min(least, ms[h]);
    }
  const uint32_t tk = wave_max_u32(best);
  const uint64_t zk = wave_min_u64(least);
  if (tk == 0u) return false;
  // the kept keys (>= t*) with their indices, in slot order
  const bool k0 = val[0] && in.sk[0] >= tk;
  const bool k1 = val[1] && in.sk[1] >= tk;
  const uint64_t l0 = __builtin_amdgcn_ballot_w64(k0);
  const uint64_t l1 = __builtin_amdgcn_ballot_w64(k1);
  const int nl0 = __builtin_popcountll(l0);
  int32_t* lo = a.lists + r * kCap;
  if (k0) {
    const int p = lanes_below(l0);
    lo[p] = in.si[0];
    F.key[slot][p] = in.sk[0];
    F.idx[slot][p] = in.si[0];
  }
  if (k1) {
    const int p = nl0 + lanes_below(l1);
    lo[p] = in.si[1];
    F.key[slot][p] = in.sk[1];
    F.idx[slot][p] = in.si[1];
  }
  RowInfo ri;
  ri.m = M;
  ri.inv_k = 1.0f / (canon::u64_to_f32(zk) * 0x1p-40f);
  ri.t_key = tk;
  ri.n_list = nl0 + __builtin_popcountll(l1);
  if (lane == 0) {
    a.info[r] = ri;
    F.info[slot] = ri;
  }
  return true;
}

template <int DT>
__global__ void __launch_bounds__(kThreads) filter_request_kernel(SplitArgs sa, ChainArgs ca) {
  __shared__ __align__(16) FastLds F;
  __shared__ __align__(16) RowsLds L;
  __shared__ float wave_val[kThreads / 64];
  __shared__ ChainLds S;
  const int b = blockIdx.x;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int k = ca.k;
  const int nrows = k + 1;
  const int64_t V = ca.V;
  const int64_t trow0 = (int64_t)b * nrows;
  const float c = ca.c;
  static_assert(kFastRows == 2 * (kThreads / 64), "two walk rows per wave at most");
  const int i0 = wave, i1 = wave + kThreads / 64;  // the wave's walk rows

  // Every load first: the draft tokens (the last wave), the lane states of slice `wave`
  // and the part maxima of every row, and the walk rows' records and key slots (of the
  // last row for a wave without a row: loaded, unused).
  const bool x_lane = wave == kThreads / 64 - 1 && lane < k;
  const int64_t xid = x_lane ? ca.draft_ids[(int64_t)b * k + lane] : -1;
  float sv[kFastRows][8], rv[kFastRows][8], pm[kFastRows][kParts];
  const float* pmf = reinterpret_cast<const float*>(sa.parts);
  constexpr int kPartFloats = sizeof(PartOut) / 4;
#pragma unroll
  for (int i = 0; i < kFastRows; ++i)
    if (i < nrows) {
      const int64_t r = trow0 + i;
      const float* lsr = sa.lane_s + r * kLanes + 64 * wave + lane;
      const float* lrr = sa.lane_r + r * kLanes + 64 * wave + lane;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sv[i][e] = lsr[e * kThreads];
        rv[i][e] = lrr[e * kThreads];
      }
#pragma unroll
      for (int q = 0; q < kParts; ++q) pm[i][q] = pmf[(r * kParts + q) * kPartFloats];
    }
  WalkIn w0, w1;
  walk_load(sa, trow0 + min(i0, nrows - 1), w0);
  walk_load(sa, trow0 + min(i1, nrows - 1), w1);
#pragma unroll
  for (int i = 0; i < kFastRows; ++i)
    if (i < nrows) {
#pragma unroll
      for (int e = 0; e < 8; ++e) asm volatile("" ::"v"(sv[i][e]), "v"(rv[i][e]));
#pragma unroll
      for (int q = 0; q < kParts; ++q) asm volatile("" ::"v"(pm[i][q]));
    }
  walk_pin(w0);
  walk_pin(w1);
  // the target logit at the draft token (every lane: no branch to wait in; its round
  // trip overlaps the trees and the walks)
  const char* xrow = static_cast<const char*>(ca.t_logits) +
                     (trow0 + (x_lane ? lane : 0)) * V * (DT == BSX_DTYPE_FP32 ? 4 : 2);
  const bool x_in = xid >= 0 && xid < V;
  const float xval = load_one<DT>(xrow, x_in ? xid : 0);

  // slice `wave` of every row's canonical tree
#pragma unroll
  for (int i = 0; i < kFastRows; ++i)
    if (i < nrows) {
      float mx = pm[i][0];
#pragma unroll
      for (int q = 1; q < kParts; ++q) mx = fmaxf(mx, pm[i][q]);
      const float rho_m = mx * c;
      float rs[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        rs[e] = canon::lane_rescaled(LaneState{-INFINITY, sv[i][e], rv[i][e]}, rho_m);
      const float zs =
          wave_tree_sum(((rs[0] + rs[1]) + (rs[2] + rs[3])) + ((rs[4] + rs[5]) + (rs[6] + rs[7])));
      if (lane == 0) F.zs[i][wave] = zs;
    }
  __syncthreads();
  // the walks
  auto walk_row = [&](int i, const WalkIn& in) {
    const float Z = (F.zs[i][0] + F.zs[i][1]) + (F.zs[i][2] + F.zs[i][3]);
    float M = in.po[0].m;
#pragma unroll
    for (int q = 1; q < kParts; ++q) M = fmaxf(M, in.po[q].m);
    const bool ok = fast_walk(sa, trow0 + i, i, in, M, Z, F);
    if (lane == 0) F.ok[i] = ok ? 1 : 0;
  };
  if (i0 < nrows) walk_row(i0, w0);
  if (i1 < nrows) walk_row(i1, w1);
  if (x_lane) {
    F.xid[lane] = xid;
    F.xval[lane] = x_in ? xval : 0.0f;
  }
  __syncthreads();
  bool all_ok = true;
  for (int i = 0; i < nrows; ++i) all_ok = all_ok && F.ok[i] != 0;
  if (!all_ok) {
    for (int i = 0; i < nrows; ++i)
      if (F.ok[i] == 0) {
        combine_row<DT>(sa, trow0 + i, L, wave_val);
        __syncthreads();
      }
    chain_request<DT>(ca, b, S);
    return;
  }
  if (wave != 0) return;

  // ratio tests (lane i: draft position i), with the one-hot draft q = 1
  const float* uni = ca.uniforms + trow0;
  bool acc = false;
  if (lane < k) {
    const int64_t x = F.xid[lane];
    if (x >= 0 && x < V) {
      const RowInfo ri = F.info[lane];
      const float xv = F.xval[lane];
      const float p = okey(xv) >= ri.t_key ? canon::weight(xv, c, -(ri.m * c)) * ri.inv_k : 0.0f;
      acc = uni[lane] * 1.0f < p;
    }
  }
  const uint64_t acc_bits = __builtin_amdgcn_ballot_w64(acc);
  const uint64_t rej_bits = __builtin_amdgcn_ballot_w64(lane < k && !acc);
  const int j = rej_bits != 0ull ? __builtin_ctzll(rej_bits) : k;

  // the draw from row j over its kept keys (entry s in lane s mod 64): r = fx40(max(p' -
  // q', 0)) against the draft (one at its token) when j < k, else (or when that has no
  // mass) fx40(p')
  const RowInfo ri = F.info[j];
  const int n = ri.n_list;
  const bool has_q = j < k;
  const int64_t xj = has_q ? F.xid[j] : -1;
  const float nmc = -(ri.m * c);
  bool kept[2];
  int32_t vid[2];
  float p[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int s = lane + 64 * h;
    kept[h] = s < n;
    vid[h] = kept[h] ? F.idx[j][s] : 0;
    p[h] = kept[h] ? canon::weight(key_value(F.key[j][s]), c, nmc) * ri.inv_k : 0.0f;
  }
  uint64_t w[2] = {0ull, 0ull};
  uint64_t total = 0ull;
  for (int pass = 0; pass < 2; ++pass) {
    const bool with_q = has_q && pass == 0;
    if (pass == 1 && !has_q) break;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float q = with_q && (int64_t)vid[h] == xj ? 1.0f : 0.0f;
      w[h] = !kept[h] ? 0ull : (with_q ? fx40(fmaxf(p[h] - q, 0.0f)) : fx40(p[h]));
    }
    total = wave_add_u64(w[0] + w[1]);
    if (total != 0ull) break;
  }
  int tok = -1;
  if (total != 0ull) {
    const uint64_t tp = canon::draw_point(uni[k], total);
    // the first index (ascending) whose running sum exceeds tp, else the last index with
    // weight: each weighted entry sums the weights at or below its index, the weighted
    // entries in turn
    typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
    typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
    uint64_t* fw = F.tm[j];  // (the walk's masses are not needed any more)
    int32_t* fi = F.idx[j];
    const int n4 = (n + 3) & ~3;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (lane + 64 * h < n4) fw[lane + 64 * h] = w[h];  // (pads: weight 0)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    uint64_t prefix[2] = {0ull, 0ull};
    for (int q = 0; q < n4; q += 4) {
      const i32x4 ii = *reinterpret_cast<const i32x4*>(fi + q);
      const u64x2 wa = *reinterpret_cast<const u64x2*>(fw + q);
      const u64x2 wb = *reinterpret_cast<const u64x2*>(fw + q + 2);
      const uint64_t ww[4] = {wa[0], wa[1], wb[0], wb[1]};
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int h = 0; h < 2; ++h) prefix[h] += ii[e] <= vid[h] ? ww[e] : 0ull;
    }
    int first = INT_MAX, last = -1;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (w[h] != 0ull) {
        if (prefix[h] > tp) first = min(first, (int)vid[h]);
        last = max(last, (int)vid[h]);
      }
    first = wave_min_i32(first);
    last = wave_max_i32(last);
    tok = first != INT_MAX ? first : last;
  }
  if (lane <= k) {
    int32_t o = -1;
    if (lane < j) o = (int32_t)F.xid[lane];
    else if (lane == j) o = tok;
    ca.out_ids[trow0 + lane] = o;
  }
  if (lane == 0) {
    ca.accepted[b] = __builtin_popcountll(acc_bits);
    ca.emitted[b] = j;
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

// Workspace of the split rows (few rows): lane states, part records, part lists.
// Non-decreasing in rows (a caller sizing for more rows always has room for the split
// region of fewer), so sized for kSplitMaxRows above it.
static int64_t split_ws_bytes(int64_t rows) {
  rows = std::min<int64_t>(rows, filt::kSplitMaxRows);
  return 2 * filt::align256(rows * canon::kLanes * 4) +
         filt::align256(rows * filt::kParts * (int64_t)sizeof(filt::PartOut)) +
         2 * filt::align256(rows * filt::kParts * filt::kPartList * 4);
}

static int64_t rows_ws_bytes(int64_t rows) {
  return filt::align256(rows * (int64_t)sizeof(filt::RowInfo)) +
         filt::align256(rows * filt::kCap * 4);
}

extern "C" int64_t bsx_filter_ws_bytes(int64_t rows) {
  return rows_ws_bytes(rows) + split_ws_bytes(rows);
}

static bool filters_on(int top_k, float top_p, int64_t vocab) {
  return (top_k > 0 && (int64_t)top_k < vocab) || (top_p > 0.f && top_p < 1.f);
}

// The split path (each row over kParts workgroups, then one combine per row) takes few
// rows of a vocabulary in its range, with a small top_k and 16-byte aligned rows.
template <int DT>
static bool split_applies(const void* a, const void* b, int64_t rows, int64_t V, int top_k) {
  const int64_t esz = DT == BSX_DTYPE_FP32 ? 4 : 2;
  const bool aligned = (V * esz) % 16 == 0 && (uintptr_t)a % 16 == 0 &&
                       (b == nullptr || (uintptr_t)b % 16 == 0);
  const bool use_k = top_k > 0 && (int64_t)top_k < V;
  return use_k && top_k <= filt::kDeferTopK && rows <= filt::kSplitMaxRows &&
         V >= filt::kSplitMinVocab && V <= filt::kSplitMaxVocab && aligned;
}

// The split path's arguments: row infos and lists at the start of ws (as for
// filter_rows_kernel), then lane states, part records and part lists.
static filt::SplitArgs split_args(const void* a, int64_t n_a, const void* b, int64_t rows,
                                  int64_t V, float c, int top_k, float top_p, void* ws) {
  filt::SplitArgs sa;
  sa.a = a;
  sa.n_a = n_a;
  sa.b = b;
  sa.V = V;
  sa.c = c;
  sa.top_k = top_k;
  sa.top_p = top_p;
  sa.info = static_cast<filt::RowInfo*>(ws);
  sa.lists = reinterpret_cast<int32_t*>(static_cast<char*>(ws) +
                                        filt::align256(rows * (int64_t)sizeof(filt::RowInfo)));
  char* base = static_cast<char*>(ws) + rows_ws_bytes(rows);
  sa.lane_s = reinterpret_cast<float*>(base);
  base += filt::align256(rows * canon::kLanes * 4);
  sa.lane_r = reinterpret_cast<float*>(base);
  base += filt::align256(rows * canon::kLanes * 4);
  sa.parts = reinterpret_cast<filt::PartOut*>(base);
  base += filt::align256(rows * filt::kParts * (int64_t)sizeof(filt::PartOut));
  sa.ckeys = reinterpret_cast<uint32_t*>(base);
  base += filt::align256(rows * filt::kParts * filt::kPartList * 4);
  sa.cidx = reinterpret_cast<int32_t*>(base);
  return sa;
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
  // Top-p alone and a top_k above kDeferTopK expect rows whose upper set cannot be
  // listed: those finish in filter_deferred_kernel.  Below it such rows (ties) are rare
  // and take the radix select in place, without a second launch.
  const bool use_k = top_k > 0 && (int64_t)top_k < V;
  const bool use_p = top_p > 0.f && top_p < 1.f;
  ra.defer = (use_p && !use_k) || (use_k && top_k > filt::kDeferTopK);
  const int64_t rows = n_a + n_b;
  if (split_applies<DT>(a, b, rows, V, top_k)) {
    // few rows: each row over kParts workgroups, then one combine per row
    const filt::SplitArgs sa = split_args(a, n_a, b, rows, V, c, top_k, top_p, ws);
    hipLaunchKernelGGL((filt::filter_parts_kernel<DT>), dim3((unsigned)(rows * filt::kParts)),
                       dim3(filt::kThreads), 0, st, sa);
    BSX_LAUNCH_CHECK();
    hipLaunchKernelGGL((filt::filter_combine_kernel<DT>), dim3((unsigned)rows),
                       dim3(filt::kThreads), 0, st, sa);
    BSX_LAUNCH_CHECK();
    return BSX_OK;
  }
  hipLaunchKernelGGL((filt::filter_rows_kernel<DT>), dim3((unsigned)(n_a + n_b)),
                     dim3(filt::kThreads), 0, st, ra);
  BSX_LAUNCH_CHECK();
  if (ra.defer) {
    hipLaunchKernelGGL((filt::filter_deferred_kernel<DT>), dim3((unsigned)(n_a + n_b)),
                       dim3(filt::kThreads), 0, st, ra);
    BSX_LAUNCH_CHECK();
  }
  return BSX_OK;
}

template <int DT>
static int filtered_chain_impl(filt::ChainArgs& ca, void* ws, hipStream_t st, int top_k,
                               float top_p) {
  const int64_t n_t = (int64_t)ca.B * (ca.k + 1);
  const int64_t n_d = ca.d_logits ? (int64_t)ca.B * ca.k : 0;
  if (ca.d_logits == nullptr && ca.k + 1 <= filt::kFastRows && top_k <= filt::kFastTopK &&
      split_applies<DT>(ca.t_logits, nullptr, n_t, ca.V, top_k)) {
    // few rows with one-hot drafts (the MTP engine's sampling verification): the parts,
    // then the combine and the chain of each request in one workgroup
    const filt::SplitArgs sa = split_args(ca.t_logits, n_t, nullptr, n_t, ca.V, ca.c, top_k,
                                          top_p, ws);
    ca.tiles_ready = 0;
    hipLaunchKernelGGL((filt::filter_parts_kernel<DT>), dim3((unsigned)(n_t * filt::kParts)),
                       dim3(filt::kThreads), 0, st, sa);
    BSX_LAUNCH_CHECK();
    hipLaunchKernelGGL((filt::filter_request_kernel<DT>), dim3((unsigned)ca.B),
                       dim3(filt::kThreads), 0, st, sa, ca);
    BSX_LAUNCH_CHECK();
    return BSX_OK;
  }
  int rc = launch_filter_rows<DT>(ca.t_logits, n_t, ca.d_logits, n_d, ca.V, ca.c, top_k, top_p,
                                  ws, st);
  if (rc != BSX_OK) return rc;
  // With a small top_k every row is expected to list its kept set: the chain kernel sums
  // the tiles itself for the rare row that does not (ties), and the tile-sum launch is
  // left out.  Otherwise (top-p alone, a large top_k) the tile sums come first.
  const bool use_k = top_k > 0 && (int64_t)top_k < ca.V;
  ca.tiles_ready = !(use_k && top_k <= filt::kDeferTopK);
  if (ca.tiles_ready) {
    const int parts = (int)ceil_div(filt::draw_tiles(ca.V), filt::kTilesPerPart);
    hipLaunchKernelGGL((filt::filter_tiles_kernel<DT>), dim3((unsigned)ca.B, (unsigned)parts),
                       dim3(filt::kThreads), 0, st, ca);
    BSX_LAUNCH_CHECK();
  }
  hipLaunchKernelGGL((filt::filter_chain_kernel<DT>), dim3((unsigned)ca.B), dim3(filt::kThreads),
                     0, st, ca);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

// Row infos and lists of the filtered rows, then the tile sums of the whole-row draws.
static int64_t filtered_chain_tiles_bytes(int B, int64_t vocab) {
  return filt::align256((int64_t)B * 2 * filt::draw_tiles(vocab) * 8);
}

extern "C" int64_t bsx_chain_filtered_ws_bytes(int B, int k, int64_t vocab) {
  const int64_t f = bsx_filter_ws_bytes((int64_t)B * (2 * k + 1)) +
                    filtered_chain_tiles_bytes(B, vocab);
  const int64_t u = bsx_chain_ws_bytes(B, k, vocab);
  return f > u ? f : u;
}

extern "C" int bsx_chain_speculative_sampling_filtered(
    const void* draft_logits_d, const int64_t* draft_ids_d, const void* target_logits_d,
    int dtype, float temperature, int top_k, float top_p, const float* uniforms_d, int B, int k,
    int64_t vocab, int32_t* out_ids_d, int32_t* accepted_d, int32_t* emitted_d, void* ws_d,
    int64_t ws_bytes, void* stream) {
  BSX_REQUIRE(row_bytes_ok(vocab, dtype), BSX_ERR_UNSUPPORTED,
              "a row of %lld logits is 2^31 bytes or more", (long long)vocab);
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
  const int64_t need = bsx_filter_ws_bytes((int64_t)B * (2 * k + 1)) +
                       filtered_chain_tiles_bytes(B, vocab);
  BSX_REQUIRE(ws_d && ws_bytes >= need, BSX_ERR_CAPACITY, "filter workspace too small (%lld < %lld)",
              (long long)ws_bytes, (long long)need);
  filt::ChainArgs ca{};
  ca.t_logits = target_logits_d;
  ca.d_logits = draft_logits_d;
  ca.info = static_cast<const filt::RowInfo*>(ws_d);
  const int64_t rows = (int64_t)B * (k + 1) + (draft_logits_d ? (int64_t)B * k : 0);
  ca.lists = reinterpret_cast<const int32_t*>(static_cast<char*>(ws_d) +
                                              filt::align256(rows * (int64_t)sizeof(filt::RowInfo)));
  ca.tiles = reinterpret_cast<uint64_t*>(static_cast<char*>(ws_d) + bsx_filter_ws_bytes(rows));
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
  BSX_REQUIRE(row_bytes_ok(vocab, dtype), BSX_ERR_UNSUPPORTED,
              "a row of %lld logits is 2^31 bytes or more", (long long)vocab);
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
  BSX_REQUIRE(row_bytes_ok(vocab, dtype), BSX_ERR_UNSUPPORTED,
              "a row of %lld logits is 2^31 bytes or more", (long long)vocab);
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
