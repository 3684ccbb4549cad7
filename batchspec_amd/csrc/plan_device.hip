// Device-side schedule of the verify-attention kernels (no counterpart in the
// reference: its plan() always schedules on the host, from host copies of the page
// table, batchspec/backends/base/attn_wrapper.py:33-72).
//
// One 1024-thread workgroup reads the device page table (qo_indptr, kv_indptr,
// kv_last_page_len) and writes the blob layout of bsx_attn_plan_device_shape:
//   seq[b]          = {qo_start, qo_len, kv_len, page_start}, kv_len by the
//                     get_seq_lens formula (batchspec/models/modules/kv_cache.py:66-70);
//   work units      = a request's kv tiles [0, ceil(kv_len / 32)), or for the
//                     sink+window view the sink tiles and the window tiles (as
//                     bsx_attn_plan); requests without query tokens have none;
//   costs           = max(1, tiles) + kSegmentCost per unit; their prefix over the
//                     batch lays the units on a line of total cost T;
//   shares          = workgroup w of W' = min(W, T) takes the positions
//                     [floor(w T / W'), floor((w+1) T / W')): tile i of a unit starting
//                     at s sits at s + kSegmentCost + i, an empty unit's output at
//                     s + kSegmentCost;
//   segments        = each unit's tiles cut at the share boundaries, in position order
//                     (which is workgroup order), with partial slots for requests cut
//                     into several segments and one merge record per such request;
//   dyn             = {split requests, error code, segments, 0}.
// A malformed table (including one whose kv_indptr[B] exceeds the entries of
// kv_indices) leaves an empty schedule and the most negative error code of its
// violations (no output is written); the launch itself never fails on data.
#include "common.h"
#include "attn_shape.h"

namespace bsx {
namespace pland {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
using attn_shape::kMaxDevicePlanBatch;
using attn_shape::kMaxDevicePlanCtas;
constexpr int kMaxSegs = kMaxDevicePlanCtas + 2 * kMaxDevicePlanBatch;
using attn_shape::kSegmentCost;
using attn_shape::kTileTokens;

struct Args {
  const int32_t* qo_indptr;
  const int32_t* kv_indptr;
  const int32_t* last_len;
  int32_t* blob;
  int64_t kv_indices_len;  // entries of kv_indices (< 0: not checked)
  int B, W, page_size, mask_mode, sink, window, max_qo;
  int off_seg_indptr, off_segments, off_merge, off_part, off_dyn;
};

struct Units {
  int n;       // 0, 1 or 2
  int b0, e0;  // tile ranges
  int b1, e1;
};

__device__ __forceinline__ Units units_of(const Args& a, int qlen, int kl) {
  Units u{0, 0, 0, 0, 0};
  if (qlen == 0) return u;
  const int nt = (kl + kTileTokens - 1) / kTileTokens;
  if (a.mask_mode == BSX_MASK_STREAMING && kl > a.sink + a.window) {
    const int a_end = (a.sink + kTileTokens - 1) / kTileTokens;
    const int w_beg = max(0, kl - a.window) / kTileTokens;
    if (w_beg <= a_end) {
      u.n = 1, u.b0 = 0, u.e0 = nt;
    } else if (a_end > 0) {
      u.n = 2, u.b0 = 0, u.e0 = a_end, u.b1 = w_beg, u.e1 = nt;
    } else {
      u.n = 1, u.b0 = w_beg, u.e0 = nt;
    }
  } else {
    u.n = 1, u.b0 = 0, u.e0 = nt;
  }
  return u;
}

__device__ __forceinline__ int64_t unit_cost(int tb, int te) {
  return (int64_t)max(1, te - tb) + kSegmentCost;
}

// Exclusive scan over the workgroup; every thread gets its prefix and the total.
template <typename T>
__device__ __forceinline__ T block_exclusive(T v, T* s_wave, T* total) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  T x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const T o = __shfl_up(x, d);
    if (lane >= d) x += o;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  T base = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const T sw = s_wave[w];
    if (w < wave) base += sw;
    tot += sw;
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

__global__ void __launch_bounds__(kThreads) plan_kernel(Args a) {
  __shared__ int32_t s_qlen[kMaxDevicePlanBatch];
  __shared__ int32_t s_kl[kMaxDevicePlanBatch];
  __shared__ int64_t s_cpre[kMaxDevicePlanBatch];  // cost position of the request's units
  __shared__ int16_t s_segwg[kMaxSegs];             // share of each segment (ascending)
  __shared__ int64_t s_w64[kWaves];
  __shared__ int32_t s_w32[kWaves];
  __shared__ int s_err;
  const int t = threadIdx.x;
  const int B = a.B;
  int32_t* blob = a.blob;
  if (t == 0) s_err = 0;
  __syncthreads();

  // 1. lengths, checks, unit costs and their prefix over the batch
  int64_t carry = 0;
  for (int c0 = 0; c0 < B; c0 += kThreads) {
    const int b = c0 + t;
    int64_t cost = 0;
    if (b < B) {
      const int q0 = a.qo_indptr[b], q1 = a.qo_indptr[b + 1];
      const int p0 = a.kv_indptr[b], p1 = a.kv_indptr[b + 1];
      const int last = a.last_len[b];
      const int np = p1 - p0, qlen = q1 - q0;
      int err = 0;
      if ((b == 0 && (q0 != 0 || p0 != 0)) || qlen < 0 || np < 0) err = BSX_ERR_INVALID;
      if (last < 0 || last > a.page_size) err = BSX_ERR_INVALID;
      if (qlen > a.max_qo) err = BSX_ERR_UNSUPPORTED;
      const int64_t kl = np > 0 ? (int64_t)(np - 1) * a.page_size + last : 0;
      if (kl >= (1LL << 30)) err = BSX_ERR_UNSUPPORTED;
      if (err) atomicMin(&s_err, err);
      const int qv = err ? 0 : qlen;
      const int kv = err ? 0 : (int)kl;
      s_qlen[b] = qv;
      s_kl[b] = kv;
      blob[4 * b + 0] = q0;
      blob[4 * b + 1] = qv;
      blob[4 * b + 2] = kv;
      blob[4 * b + 3] = p0;
      const Units u = units_of(a, qv, kv);
      if (u.n > 0) cost += unit_cost(u.b0, u.e0);
      if (u.n > 1) cost += unit_cost(u.b1, u.e1);
    }
    int64_t tot;
    const int64_t pre = block_exclusive<int64_t>(cost, s_w64, &tot);
    if (b < B) s_cpre[b] = carry + pre;
    carry += tot;
  }
  if (t == 0 && (a.kv_indptr[B] < 1 ||
                 (a.kv_indices_len >= 0 && a.kv_indptr[B] > a.kv_indices_len)))
    atomicMin(&s_err, (int)BSX_ERR_INVALID);
  __syncthreads();
  const int err = s_err;
  const int64_t T = err ? 0 : carry;
  const int64_t Wn = min((int64_t)a.W, T);  // workgroups with a non-empty share
  // share of position pos, and the first position of share w
  auto wg_of = [&](int64_t pos) -> int64_t { return ((pos + 1) * Wn - 1) / T; };
  auto share_begin = [&](int64_t w) -> int64_t { return w * T / Wn; };

  // 2. per request: segments (cuts of its units at share boundaries), partial slots,
  // merge records; then the segments themselves
  int seg_carry = 0, part_carry = 0, merge_carry = 0;
  for (int c0 = 0; c0 < B; c0 += kThreads) {
    const int b = c0 + t;
    int nseg = 0;
    Units u{0, 0, 0, 0, 0};
    int64_t s0 = 0, s1 = 0;
    if (b < B && T > 0) {
      u = units_of(a, s_qlen[b], s_kl[b]);
      s0 = s_cpre[b];
      s1 = s0 + (u.n > 0 ? unit_cost(u.b0, u.e0) : 0);
      for (int k = 0; k < u.n; ++k) {
        const int64_t s = k ? s1 : s0;
        const int n = k ? u.e1 - u.b1 : u.e0 - u.b0;
        const int64_t wf = wg_of(s + kSegmentCost);
        const int64_t wl = n > 0 ? wg_of(s + kSegmentCost + n - 1) : wf;
        nseg += (int)(wl - wf + 1);
      }
    }
    const bool split = nseg > 1;
    int tot_seg, tot_part, tot_merge;
    const int seg_pre = seg_carry + block_exclusive<int32_t>(nseg, s_w32, &tot_seg);
    const int part_pre = part_carry + block_exclusive<int32_t>(split ? nseg : 0, s_w32, &tot_part);
    const int merge_pre = merge_carry + block_exclusive<int32_t>(split ? 1 : 0, s_w32, &tot_merge);
    if (b < B) {
      blob[a.off_part + b] = part_pre;
      if (split) {
        int32_t* m = blob + a.off_merge + 4 * merge_pre;
        m[0] = part_pre;
        m[1] = part_pre + nseg;
        m[2] = a.qo_indptr[b];
        m[3] = s_qlen[b];
      }
      int si = seg_pre, piece = 0;
      for (int k = 0; k < u.n; ++k) {
        const int64_t s = (k ? s1 : s0) + kSegmentCost;  // position of the first tile
        const int tb = k ? u.b1 : u.b0;
        const int n = k ? u.e1 - u.b1 : u.e0 - u.b0;
        const int64_t wf = wg_of(s);
        const int64_t wl = n > 0 ? wg_of(s + n - 1) : wf;
        for (int64_t w = wf; w <= wl; ++w) {
          const int64_t lo = max(share_begin(w), s), hi = min(share_begin(w + 1), s + n);
          int32_t* sg = blob + a.off_segments + 4 * si;
          sg[0] = b;
          sg[1] = n > 0 ? tb + (int)(lo - s) : tb;
          sg[2] = n > 0 ? tb + (int)(hi - s) : tb;
          sg[3] = split ? part_pre + piece : -1;
          s_segwg[si] = (int16_t)w;
          ++si;
          ++piece;
        }
      }
    }
    seg_carry += tot_seg;
    part_carry += tot_part;
    merge_carry += tot_merge;
  }
  // 3. seg_indptr[w] = segments in shares before w (the segments' shares ascend:
  // binary search)
  __syncthreads();
  for (int w = t; w <= a.W; w += kThreads) {
    int lo = 0, hi = seg_carry;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_segwg[mid] < w) lo = mid + 1;
      else hi = mid;
    }
    blob[a.off_seg_indptr + w] = lo;
  }
  if (t == 0) {
    blob[a.off_part + B] = part_carry;
    blob[a.off_dyn + 0] = merge_carry;
    blob[a.off_dyn + 1] = err;
    blob[a.off_dyn + 2] = seg_carry;
    blob[a.off_dyn + 3] = 0;
  }
}

}  // namespace pland
}  // namespace bsx

using namespace bsx;

extern "C" int bsx_attn_plan_device(const bsx_attn_plan_t* plan, const int32_t* qo_indptr_d,
                                    const int32_t* kv_indptr_d, const int32_t* kv_last_page_len_d,
                                    int64_t kv_indices_len, int32_t* plan_blob_d, void* stream) {
  BSX_REQUIRE(plan != nullptr && plan->device_plan == 1, BSX_ERR_INVALID,
              "plan was not made by bsx_attn_plan_device_shape");
  BSX_REQUIRE(plan->batch >= 1 && plan->batch <= attn_shape::kMaxDevicePlanBatch,
              BSX_ERR_INVALID, "bad batch %d", plan->batch);
  BSX_REQUIRE(qo_indptr_d && kv_indptr_d && kv_last_page_len_d && plan_blob_d, BSX_ERR_INVALID,
              "null pointer");
  pland::Args a;
  a.qo_indptr = qo_indptr_d;
  a.kv_indptr = kv_indptr_d;
  a.last_len = kv_last_page_len_d;
  a.blob = plan_blob_d;
  a.kv_indices_len = kv_indices_len;
  a.B = plan->batch;
  a.W = plan->num_ctas;
  a.page_size = plan->page_size;
  a.mask_mode = plan->mask_mode;
  a.sink = plan->sink_tokens;
  a.window = plan->window_tokens;
  a.max_qo = plan->max_qo_len;
  a.off_seg_indptr = plan->off_seg_indptr;
  a.off_segments = plan->off_segments;
  a.off_merge = plan->off_merge_seqs;
  a.off_part = plan->off_part_indptr;
  a.off_dyn = plan->off_dyn;
  hipLaunchKernelGGL(pland::plan_kernel, dim3(1), dim3(pland::kThreads), 0, as_stream(stream), a);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}
