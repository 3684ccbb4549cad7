// Device-side body of the sync-free page-table update, shared by page_table_kernel
// (page_table.hip) and the fused greedy acceptance + delete (accept.hip).
//
// Replaces PageTable.insert_kv / delete_kv (batchspec/backends/base/page_table.py:55-137)
// with PageManager.allocate / free (batchspec/backends/utils/paging.py:155-277):
//   per request r: total = (pages_r - 1) * page_size + last_r (+ dec or - del);
//   insert: pages only grow (the tail pages of the new total are appended);
//   delete: total clamped at 0, tail pages dropped;  pages >= 1 always;
//   last_r = (total - 1) % page_size + 1 (0 for an empty request);
//   cachelens_r = max(cachelens_r +/- d_r, 0);
//   when no d_r > 0, nothing changes (the reference returns early);
//   an insert that would give some request more than max_pages pages changes nothing
//   and increments *errors (the reference raises before touching its state).
// Page k of request r has id r * max_pages + k (the reference allocator's ids), so the
// packed CSR (indptr = exclusive scan of page counts, indices) is rebuilt from the counts.
#pragma once

#include "common.h"

namespace bsx {
namespace pt {

constexpr int kThreads = 1024;

struct Args {
  int32_t* num_pages;
  int32_t* last_len;
  int32_t* cachelens;  // may be null
  const int32_t* d;    // [B] or null (then d_scalar)
  int32_t d_scalar;
  int sign;            // +1 insert, -1 delete
  int B, page_size, max_pages;
  int32_t* indptr;     // [B + 1]
  int32_t* indices;    // [B * max_pages]
  int32_t* errors;     // may be null
};

// The whole update by one workgroup of kThreads threads; delta(r) gives d_r.
template <class Delta>
__device__ __forceinline__ void update_pages(const Args& a, Delta delta) {
  __shared__ int32_t s_scan[kThreads];
  __shared__ int32_t s_pages[kThreads];
  __shared__ int32_t s_wave[kThreads / 64];
  __shared__ int32_t s_flag[2][kThreads / 64];
  __shared__ int32_t s_base;
  const int t = threadIdx.x;
  const int ps = a.page_size;
  // anything to do? and would any request overflow?
  int any_pos = 0, over = 0;
  for (int r = t; r < a.B; r += kThreads) {
    const int32_t d = delta(r);
    any_pos |= d > 0;
    if (a.sign > 0) {
      const int64_t total = (int64_t)(a.num_pages[r] - 1) * ps + a.last_len[r] + d;
      const int64_t full = total > 0 ? (total - 1) / ps : 0;
      const int64_t pages = max((int64_t)a.num_pages[r], full + 1);
      over |= pages > a.max_pages;
    }
  }
  // (per-wave flags through LDS: no wait for global stores the caller has in flight)
  const bool wpos = __builtin_amdgcn_ballot_w64(any_pos != 0) != 0ull;
  const bool wover = __builtin_amdgcn_ballot_w64(over != 0) != 0ull;
  if ((t & 63) == 0) {
    s_flag[0][t >> 6] = wpos ? 1 : 0;
    s_flag[1][t >> 6] = wover ? 1 : 0;
  }
  lds_barrier();
  any_pos = 0;
  over = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) {
    any_pos |= s_flag[0][w];
    over |= s_flag[1][w];
  }
  if (!any_pos) return;
  if (over) {
    if (t == 0 && a.errors) a.errors[0] += 1;
    return;
  }

  // new counts and tails (each thread owns its requests)
  for (int r = t; r < a.B; r += kThreads) {
    const int32_t d = delta(r);
    const int32_t old_pages = a.num_pages[r];
    int64_t total = (int64_t)(old_pages - 1) * ps + a.last_len[r] + (int64_t)a.sign * d;
    if (total < 0) total = 0;
    const int64_t full = total > 0 ? (total - 1) / ps : 0;
    const int32_t tail = total > 0 ? (int32_t)((total - 1) % ps + 1) : 0;
    const int32_t pages = a.sign > 0 ? max(old_pages, (int32_t)(full + 1))
                                     : min(old_pages, (int32_t)(full + 1));
    a.num_pages[r] = pages;
    a.last_len[r] = tail;
    if (a.cachelens) {
      const int64_t cl = (int64_t)a.cachelens[r] + (int64_t)a.sign * d;
      a.cachelens[r] = cl > 0 ? (int32_t)cl : 0;
    }
  }

  // indptr (exclusive scan of the page counts) and indices, kThreads requests at a
  // time; each chunk's counts and starts stay in LDS for the index writes.  A thread
  // reads back only the counts it wrote itself (request r0 + t), so the barriers here
  // order LDS only and never wait for the global stores in flight.
  if (t == 0) s_base = 0;
  lds_barrier();
  for (int r0 = 0; r0 < a.B; r0 += kThreads) {
    const int r = r0 + t;
    const int32_t v = r < a.B ? a.num_pages[r] : 0;
    s_pages[t] = v;
    // inclusive scan: within each wave by shuffles, then over the wave totals
    const int lane = t & 63, wave = t >> 6;
    int32_t x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int32_t o = __shfl_up(x, d);
      if (lane >= d) x += o;
    }
    if (lane == 63) s_wave[wave] = x;
    lds_barrier();
    if (t < 64) {
      int32_t w = t < kThreads / 64 ? s_wave[t] : 0;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int32_t o = __shfl_up(w, d);
        if (t >= d) w += o;
      }
      if (t < kThreads / 64) s_wave[t] = w;  // inclusive over waves
    }
    lds_barrier();
    s_scan[t] = x + (wave > 0 ? s_wave[wave - 1] : 0);
    lds_barrier();
    const int32_t base = s_base;
    if (r < a.B) a.indptr[r] = base + s_scan[t] - v;
    const int nr = min(kThreads, a.B - r0);
    // the chunk's requests one after another, each request's pages over the workgroup
    for (int q = 0; q < nr; ++q) {
      const int32_t n = s_pages[q];
      const int32_t beg = base + s_scan[q] - n;
      for (int k = t; k < n; k += kThreads) a.indices[beg + k] = (r0 + q) * a.max_pages + k;
    }
    lds_barrier();
    if (t == kThreads - 1) s_base = base + s_scan[t];
    lds_barrier();
  }
  if (t == 0) a.indptr[a.B] = s_base;
}

}  // namespace pt
}  // namespace bsx
