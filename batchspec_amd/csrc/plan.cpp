// Host-side planner of the verify-attention kernel (pure C++, no GPU needed).
//
// Plays the role of BatchPrefillWithPagedKVCacheWrapper.plan() as called at
// batchspec/backends/standard_engine.py:132-143 and
// batchspec/backends/mtp_engine.py:420-432: it reads the host copies of the CSR
// page table, validates them, derives every request's kv length with the
// get_seq_lens formula (batchspec/models/modules/kv_cache.py:66-70), and cuts the
// whole kv work into equal shares for a persistent grid.
//
// Device blob layout (int32):
//   seq[batch][4]      qo_start, qo_len, kv_len, page_start
//   seg_indptr[ctas+1] segments of workgroup w are [seg_indptr[w], seg_indptr[w+1])
//   segments[S][4]     request, first tile, end tile, partial slot (-1 = final)
//   merge[M][4]        per request whose kv range spans several segments (16-byte
//                      aligned): first partial slot, end slot, qo_start, qo_len
//   part_indptr[b+1]   partial slots of request b are [part_indptr[b], part_indptr[b+1])
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <vector>

#include "../../include/bsx.h"
#include "attn_shape.h"

namespace bsx {
void set_error(const char* fmt, ...);
}

#define PLAN_REQUIRE(cond, code, ...)  \
  do {                                 \
    if (!(cond)) {                     \
      ::bsx::set_error(__VA_ARGS__);   \
      return (code);                   \
    }                                  \
  } while (0)

namespace {

using bsx::attn_shape::kMaxWavesPerCta;
using bsx::attn_shape::kTileTokens;
constexpr int64_t kSegmentCost = bsx::attn_shape::kSegmentCost;

struct Unit {
  int b;
  int tb;
  int te;
};

struct Seg {
  int b, tb, te;
};

// Greedy packing of the units, in order, into workgroups of capacity `cap` (cost
// units: one per tile plus kSegmentCost per segment).  Returns the number of
// workgroups used, or -1 when more than `max_ctas` would be needed.
int64_t pack_units(const std::vector<Unit>& units, int64_t cap, int64_t max_ctas,
                   std::vector<std::vector<Seg>>* out) {
  if (out) out->assign(1, {});
  int64_t used = 1, rem = cap;
  for (const Unit& u : units) {
    int left = u.te - u.tb;
    int pos = u.tb;
    bool placed_empty = false;
    while (left > 0 || (u.te == u.tb && !placed_empty)) {
      if (rem < kSegmentCost + 1) {
        if (++used > max_ctas) return -1;
        rem = cap;
        if (out) out->emplace_back();
      }
      const int take = (int)std::min<int64_t>(left, rem - kSegmentCost);
      if (out) out->back().push_back({u.b, pos, pos + take});
      rem -= take + kSegmentCost;
      if (u.te == u.tb) {
        rem -= 1;  // an empty request still writes its (zero) output
        placed_empty = true;
      }
      left -= take;
      pos += take;
    }
  }
  return used;
}

}  // namespace

// Resident waves per SIMD of each kernel variant (from the compiler's register
// report; 512 VGPRs per SIMD lane are shared by the resident waves).
static int waves_per_simd(int head_dim, int qrow_tile) {
  if (head_dim == 128) return 2;
  return qrow_tile == 16 ? 4 : 3;
}

// Workgroup shape and persistent grid of the attention kernels for query rows per kv
// head of up to max_qo * group (shared by the host and the device planner).
struct GridShape {
  int qrow_tile, qrow_blocks, hpc, qbpc, n_qgroups, num_ctas;
  bool shared;
};

static GridShape grid_shape(int max_qo, int group, int num_kv_heads, int head_dim, int page_size,
                     int num_cus, int mask_mode) {
  GridShape g;
  // Query rows per kv head = qo_len * group.  A wave covers 16 or 32 of them.
  const int64_t max_rows = (int64_t)max_qo * group;
  g.qrow_tile = max_rows <= 16 ? 16 : 32;
  g.qrow_blocks = (int)std::max<int64_t>(1, (max_rows + g.qrow_tile - 1) / g.qrow_tile);
  // Several waves per kv head: they share each K/V tile through LDS when a 16-token
  // subtile always lies inside one page (the shared kernel's loads assume it).
  // (a general custom mask runs on the per-wave kernel, which reads the mask bits)
  g.shared = g.qrow_blocks > 1 && page_size >= 16 && mask_mode != BSX_MASK_CUSTOM;
  g.hpc = 1;  // kv heads per workgroup: largest divisor of num_kv_heads that fits
  if (g.shared) {
    g.qbpc = g.qrow_blocks <= 2 ? 2 : g.qrow_blocks <= 4 ? 4 : 8;
    for (int c = 1; c <= num_kv_heads; ++c)
      if (num_kv_heads % c == 0 && c <= bsx::attn_shape::shared_max_heads(head_dim, g.qbpc))
        g.hpc = c;
  } else {
    for (int c = 1; c <= num_kv_heads; ++c)
      if (num_kv_heads % c == 0 &&
          c * std::min(g.qrow_blocks, kMaxWavesPerCta) <= kMaxWavesPerCta)
        g.hpc = c;
    g.qbpc = g.qrow_blocks;
    while (g.qbpc * g.hpc > kMaxWavesPerCta) g.qbpc = (g.qbpc + 1) / 2;
  }
  g.n_qgroups = (g.qrow_blocks + g.qbpc - 1) / g.qbpc;
  const int cta_waves = g.hpc * g.qbpc;
  // One grid row (blockIdx.y) per (kv-head group, query group); size grid.x so that
  // all workgroups are resident at once on num_cus compute units (4 SIMDs each; the
  // shared kernel's LDS ring also bounds its workgroups per compute unit).
  const int grid_y = (num_kv_heads / g.hpc) * g.n_qgroups;
  int resident_per_cu = std::max(1, 4 * waves_per_simd(head_dim, g.qrow_tile) / cta_waves);
  if (g.shared)
    resident_per_cu = std::max(
        1, std::min(resident_per_cu, bsx::attn_shape::kLdsPerCu /
                                         bsx::attn_shape::shared_lds_bytes(head_dim, g.qbpc)));
  g.num_ctas = std::max(1, (num_cus * resident_per_cu) / grid_y);
  return g;
}

extern "C" int64_t bsx_attn_plan_ints_bound(int batch, int num_cus) {
  if (batch < 0 || num_cus < 1) return -1;
  const int64_t num_ctas = (int64_t)num_cus * 16;
  // seq 4B + seg_indptr (W+1) + segments 4*(2W + 2B) + merge records 4B (+3 to align)
  // + part_indptr (B+1)
  return 4LL * batch + (num_ctas + 1) + 4LL * (2 * num_ctas + 2LL * batch) + 4LL * batch + 3 +
         (batch + 1) + 16;
}

// Validated page table and its greedy schedule over a persistent grid of at most
// `max_ctas` workgroups (shared by the compact and the fixed-layout host plans).
struct HostSchedule {
  std::vector<int32_t> qo_len, kv_len;
  int max_qo = 0;
  int safe_pos = -1;  // first position of kv_indices that belongs to a request
  int64_t total_tiles = 0;
  std::vector<std::vector<Seg>> per_cta;  // segments of each used workgroup
  std::vector<int> units_of;              // segments per request
  std::vector<int32_t> part_indptr;       // partial slots per request
  std::vector<int32_t> merge_seqs;        // requests cut into several segments
  int nseg = 0;
};

static int validate_table(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                          const int32_t* kv_last_page_len_h, int batch, int page_size,
                          int mask_mode, int64_t kv_indices_len, HostSchedule* hs) {
  PLAN_REQUIRE(qo_indptr_h[0] == 0 && kv_indptr_h[0] == 0, BSX_ERR_INVALID,
               "qo_indptr[0] and paged_kv_indptr[0] must be 0");
  hs->qo_len.assign(batch, 0);
  hs->kv_len.assign(batch, 0);
  for (int b = 0; b < batch; ++b) {
    const int q = qo_indptr_h[b + 1] - qo_indptr_h[b];
    const int np = kv_indptr_h[b + 1] - kv_indptr_h[b];
    const int last = kv_last_page_len_h[b];
    PLAN_REQUIRE(q >= 0, BSX_ERR_INVALID, "qo_indptr not non-decreasing at request %d", b);
    PLAN_REQUIRE(np >= 0, BSX_ERR_INVALID, "paged_kv_indptr not non-decreasing at request %d", b);
    PLAN_REQUIRE(last >= 0 && last <= page_size, BSX_ERR_INVALID,
                 "paged_kv_last_page_len[%d] = %d outside [0, page_size=%d]", b, last, page_size);
    const int64_t kl = np > 0 ? (int64_t)(np - 1) * page_size + last : 0;
    PLAN_REQUIRE(kl < (1LL << 30), BSX_ERR_UNSUPPORTED, "kv length too large at request %d", b);
    hs->qo_len[b] = q;
    hs->kv_len[b] = (int32_t)kl;
    if (np > 0 && hs->safe_pos < 0) hs->safe_pos = kv_indptr_h[b];
    if (mask_mode == BSX_MASK_TREE)
      PLAN_REQUIRE(q <= 32, BSX_ERR_UNSUPPORTED,
                   "tree mask supports at most 32 query tokens per request (request %d has %d)", b,
                   q);
    hs->max_qo = std::max(hs->max_qo, q);
  }
  PLAN_REQUIRE(kv_indices_len < 0 || kv_indptr_h[batch] <= kv_indices_len, BSX_ERR_INVALID,
               "paged_kv_indptr[-1] = %d exceeds the %lld entries of paged_kv_indices",
               kv_indptr_h[batch], (long long)kv_indices_len);
  return BSX_OK;
}

static void schedule(int batch, int mask_mode, int sink_tokens, int window_tokens, int max_ctas,
                     HostSchedule* hs) {
  // Work units: contiguous tile ranges per request (two for the sink+window view).
  std::vector<Unit> units;
  units.reserve(2 * (size_t)batch);
  hs->total_tiles = 0;
  for (int b = 0; b < batch; ++b) {
    if (hs->qo_len[b] == 0) continue;
    const int kl = hs->kv_len[b];
    const int ntiles = (kl + kTileTokens - 1) / kTileTokens;
    if (mask_mode == BSX_MASK_STREAMING && kl > sink_tokens + window_tokens) {
      const int a_end = (sink_tokens + kTileTokens - 1) / kTileTokens;
      const int w_beg = std::max(0, (kl - window_tokens)) / kTileTokens;
      if (w_beg <= a_end) {
        units.push_back({b, 0, ntiles});
      } else {
        if (a_end > 0) units.push_back({b, 0, a_end});
        units.push_back({b, w_beg, ntiles});
      }
    } else {
      units.push_back({b, 0, ntiles});
    }
  }
  int64_t total_cost = 0;
  for (const Unit& u : units) {
    hs->total_tiles += u.te - u.tb;
    total_cost += std::max(1, u.te - u.tb) + kSegmentCost;
  }

  // Smallest per-workgroup capacity whose greedy packing fits the grid.
  hs->per_cta.clear();
  if (!units.empty()) {
    const int64_t W = max_ctas;
    int64_t lo = std::max<int64_t>(kSegmentCost + 1, (total_cost + W - 1) / W);
    int64_t hi = total_cost + kSegmentCost + 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi) / 2;
      if (pack_units(units, mid, W, nullptr) >= 0)
        hi = mid;
      else
        lo = mid + 1;
    }
    pack_units(units, lo, W, &hs->per_cta);
  }
  if (hs->per_cta.empty()) hs->per_cta.resize(1);

  hs->units_of.assign(batch, 0);
  hs->nseg = 0;
  for (const auto& v : hs->per_cta) {
    hs->nseg += (int)v.size();
    for (const Seg& sg : v) hs->units_of[sg.b]++;
  }
  // Partial slots for requests that ended up in more than one segment.
  hs->part_indptr.assign(batch + 1, 0);
  hs->merge_seqs.clear();
  for (int b = 0; b < batch; ++b) {
    const int n = hs->units_of[b];
    hs->part_indptr[b + 1] = hs->part_indptr[b] + (n > 1 ? n : 0);
    if (n > 1) hs->merge_seqs.push_back(b);
  }
}

// Writes seq records, seg_indptr (workgroups past the used ones get empty ranges),
// segments, merge records and part_indptr at the given offsets.
static void write_blob(const HostSchedule& hs, const int32_t* qo_indptr_h,
                       const int32_t* kv_indptr_h, int batch, int blob_batch, int W,
                       int off_seq, int off_seg_indptr, int off_segments, int off_merge,
                       int off_part, int32_t* blob) {
  for (int b = 0; b < blob_batch; ++b) {
    const bool live = b < batch;
    blob[off_seq + 4 * b + 0] = live ? qo_indptr_h[b] : qo_indptr_h[batch];
    blob[off_seq + 4 * b + 1] = live ? hs.qo_len[b] : 0;
    blob[off_seq + 4 * b + 2] = live ? hs.kv_len[b] : 0;
    blob[off_seq + 4 * b + 3] = live ? kv_indptr_h[b] : kv_indptr_h[batch];
  }
  std::vector<int32_t> next_slot(hs.part_indptr.begin(), hs.part_indptr.end() - 1);
  int si = 0;
  for (int w = 0; w < W; ++w) {
    blob[off_seg_indptr + w] = si;
    if (w >= (int)hs.per_cta.size()) continue;
    for (const Seg& sg : hs.per_cta[w]) {
      blob[off_segments + 4 * si + 0] = sg.b;
      blob[off_segments + 4 * si + 1] = sg.tb;
      blob[off_segments + 4 * si + 2] = sg.te;
      blob[off_segments + 4 * si + 3] = hs.units_of[sg.b] > 1 ? next_slot[sg.b]++ : -1;
      ++si;
    }
  }
  blob[off_seg_indptr + W] = si;
  for (int i = off_segments + 4 * si; i < off_merge; ++i) blob[i] = 0;
  for (size_t i = 0; i < hs.merge_seqs.size(); ++i) {
    const int b = hs.merge_seqs[i];
    blob[off_merge + 4 * (int)i + 0] = hs.part_indptr[b];
    blob[off_merge + 4 * (int)i + 1] = hs.part_indptr[b + 1];
    blob[off_merge + 4 * (int)i + 2] = qo_indptr_h[b];
    blob[off_merge + 4 * (int)i + 3] = hs.qo_len[b];
  }
  for (int b = 0; b <= blob_batch; ++b)
    blob[off_part + b] = hs.part_indptr[std::min(b, batch)];
}

#define PLAN_COMMON_CHECKS()                                                                    \
  PLAN_REQUIRE(num_kv_heads > 0 && num_qo_heads > 0 && num_qo_heads % num_kv_heads == 0,        \
               BSX_ERR_INVALID,                                                                 \
               "num_qo_heads (%d) must be a positive multiple of num_kv_heads (%d)",            \
               num_qo_heads, num_kv_heads);                                                     \
  PLAN_REQUIRE(head_dim == 64 || head_dim == 128, BSX_ERR_UNSUPPORTED,                          \
               "head_dim %d not supported (64 or 128)", head_dim);                              \
  PLAN_REQUIRE(page_size >= 1 && page_size <= 1024 && (page_size & (page_size - 1)) == 0,       \
               BSX_ERR_UNSUPPORTED, "page_size %d must be a power of two <= 1024", page_size);  \
  PLAN_REQUIRE(mask_mode >= BSX_MASK_NONE && mask_mode <= BSX_MASK_CUSTOM, BSX_ERR_INVALID,     \
               "unknown mask mode %d", mask_mode);                                              \
  PLAN_REQUIRE(num_cus >= 1, BSX_ERR_INVALID, "num_cus must be >= 1");                          \
  PLAN_REQUIRE(mask_mode != BSX_MASK_STREAMING || (sink_tokens >= 0 && window_tokens >= 0),     \
               BSX_ERR_INVALID, "streaming view needs sink >= 0 and window >= 0")

// The wave-split kernel fits: at most 16 query rows per kv head (one 16-row tile), pages
// of 16 or more tokens, a causal / no / sink + window mask, (request, kv head) pairs that
// fill the compute units, and no request with more than kSplitMaxTiles visible tiles.
static bool wave_split_fits(const HostSchedule& hs, const GridShape& gs, int batch,
                            int num_kv_heads, int group, int head_dim, int page_size,
                            int mask_mode, int sink_tokens, int window_tokens, int num_cus) {
  namespace as = bsx::attn_shape;
  if (gs.shared || gs.qrow_tile != 16 || gs.qrow_blocks != 1 || page_size < 16) return false;
  if (mask_mode != BSX_MASK_NONE && mask_mode != BSX_MASK_CAUSAL &&
      mask_mode != BSX_MASK_STREAMING)
    return false;
  const int64_t pairs = (int64_t)batch * num_kv_heads;
  if (2 * pairs < num_cus || pairs > num_cus) return false;
  int longest = 0;
  int64_t tiles = 0;
  for (int b = 0; b < batch; ++b) {
    const int kl = hs.kv_len[b];
    const int ntiles = (kl + kTileTokens - 1) / kTileTokens;
    int visible = ntiles;
    if (mask_mode == BSX_MASK_STREAMING && kl > sink_tokens + window_tokens) {
      const int a_end = (sink_tokens + kTileTokens - 1) / kTileTokens;
      const int w_beg = std::max(0, kl - window_tokens) / kTileTokens;
      if (w_beg > a_end) visible = a_end + (ntiles - w_beg);
    }
    if (visible > as::kSplitMaxTiles) return false;
    if (hs.qo_len[b] > 0) {
      longest = std::max(longest, visible);
      tiles += visible;
    }
  }
  const double mb = (double)tiles * num_kv_heads * as::head_tile_bytes(head_dim) * 1e-6;
  // a wave's tile time scales with the head dim (its bytes and its matrix products)
  const double wave_tile_us = as::kWsWaveTileUs * head_dim / 128.0;
  const double ws_us = std::max(as::kWsLatencyUs + wave_tile_us * longest / as::kSplitWaves,
                                as::kWsFixedUs + as::kWsUsPerMB * mb);
  const double sk_us = as::kSkFixedUs + as::kSkUsPerMB * mb +
                       as::kSkRowUs * std::max(0, hs.max_qo * group - 4);
  return ws_us < sk_us;
}

extern "C" int bsx_attn_plan(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                             const int32_t* kv_last_page_len_h, int batch, int num_qo_heads,
                             int num_kv_heads, int head_dim, int page_size, int mask_mode,
                             int sink_tokens, int window_tokens, float sm_scale, int num_cus,
                             int64_t kv_indices_len, int32_t* plan_blob_h,
                             int64_t blob_capacity_ints, bsx_attn_plan_t* out) {
  PLAN_REQUIRE(qo_indptr_h && kv_indptr_h && kv_last_page_len_h && plan_blob_h && out,
               BSX_ERR_INVALID, "null argument to bsx_attn_plan");
  PLAN_REQUIRE(batch >= 0, BSX_ERR_INVALID, "batch must be >= 0 (got %d)", batch);
  PLAN_COMMON_CHECKS();

  HostSchedule hs;
  int rc = validate_table(qo_indptr_h, kv_indptr_h, kv_last_page_len_h, batch, page_size,
                          mask_mode, kv_indices_len, &hs);
  if (rc != BSX_OK) return rc;
  const int group = num_qo_heads / num_kv_heads;
  const GridShape gs =
      grid_shape(hs.max_qo, group, num_kv_heads, head_dim, page_size, num_cus, mask_mode);
  schedule(batch, mask_mode, sink_tokens, window_tokens, gs.num_ctas, &hs);
  const int W = (int)hs.per_cta.size();
  const int nseg = hs.nseg;
  const int nmerge = (int)hs.merge_seqs.size();
  const int64_t need = 4LL * batch + (W + 1) + 4LL * nseg + 3 + 4LL * nmerge + (batch + 1);
  PLAN_REQUIRE(need <= blob_capacity_ints, BSX_ERR_CAPACITY,
               "plan blob needs %lld int32 entries, capacity %lld", (long long)need,
               (long long)blob_capacity_ints);
  const int off_seq = 0;
  const int off_seg_indptr = off_seq + 4 * batch;
  const int off_segments = off_seg_indptr + W + 1;
  const int off_merge = (off_segments + 4 * nseg + 3) & ~3;  // 16-byte records
  const int off_part = off_merge + 4 * nmerge;
  write_blob(hs, qo_indptr_h, kv_indptr_h, batch, batch, W, off_seq, off_seg_indptr,
             off_segments, off_merge, off_part, plan_blob_h);

  memset(out, 0, sizeof(*out));
  out->batch = batch;
  out->num_qo_heads = num_qo_heads;
  out->num_kv_heads = num_kv_heads;
  out->head_dim = head_dim;
  out->page_size = page_size;
  out->mask_mode = mask_mode;
  out->group_size = group;
  out->qrow_tile = gs.qrow_tile;
  out->qrow_blocks = gs.qrow_blocks;
  out->heads_per_cta = gs.hpc;
  out->qblocks_per_cta = gs.qbpc;
  out->num_qgroups = gs.n_qgroups;
  out->num_ctas = W;
  out->num_segments = nseg;
  out->num_partials = hs.part_indptr[batch];
  out->num_split_requests = nmerge;
  out->max_qo_len = hs.max_qo;
  out->tile_tokens = kTileTokens;
  out->sink_tokens = sink_tokens;
  out->window_tokens = window_tokens;
  out->off_seq = off_seq;
  out->off_seg_indptr = off_seg_indptr;
  out->off_segments = off_segments;
  out->off_merge_seqs = off_merge;
  out->off_part_indptr = off_part;
  out->plan_ints = (int32_t)need;
  const int64_t rows_total = (int64_t)gs.qrow_tile * gs.qrow_blocks;
  // partial outputs in the input dtype plus their fp32 log-sum-exp
  out->float_ws_bytes =
      (int64_t)out->num_partials * num_kv_heads * rows_total * (head_dim * 2 + 4);
  out->sm_scale = sm_scale > 0.f ? sm_scale : 1.0f / std::sqrt((float)head_dim);
  out->total_qo = batch > 0 ? qo_indptr_h[batch] : 0;
  out->safe_page_pos = hs.safe_pos;
  out->total_tiles = hs.total_tiles;
  out->shared_kv_tiles = gs.shared ? 1 : 0;
  out->off_dyn = -1;
  if (wave_split_fits(hs, gs, batch, num_kv_heads, group, head_dim, page_size, mask_mode,
                      sink_tokens, window_tokens, num_cus)) {
    // one workgroup per (request, kv head), its waves merging in LDS: no partials, no
    // merge launch (the blob keeps its request records; the segments go unused)
    out->shared_kv_tiles = bsx::attn_shape::kPlanWaveSplit;
    out->heads_per_cta = 1;
    out->qblocks_per_cta = 1;
    out->num_qgroups = 1;
    out->num_ctas = batch;
    out->num_partials = 0;
    out->num_split_requests = 0;
    out->float_ws_bytes = 0;
  }
  return BSX_OK;
}

extern "C" int bsx_attn_plan_fixed(const bsx_attn_plan_t* shape, const int32_t* qo_indptr_h,
                                   const int32_t* kv_indptr_h,
                                   const int32_t* kv_last_page_len_h, int batch,
                                   int64_t kv_indices_len, int32_t* plan_blob_h,
                                   int64_t blob_capacity_ints, bsx_attn_plan_t* out) {
  PLAN_REQUIRE(shape && qo_indptr_h && kv_indptr_h && kv_last_page_len_h && plan_blob_h && out,
               BSX_ERR_INVALID, "null argument to bsx_attn_plan_fixed");
  PLAN_REQUIRE(shape->device_plan == 1, BSX_ERR_INVALID,
               "shape was not made by bsx_attn_plan_device_shape");
  PLAN_REQUIRE(batch >= 1 && batch <= shape->batch, BSX_ERR_INVALID,
               "batch %d outside the fixed shape's 1..%d requests", batch, shape->batch);
  PLAN_REQUIRE(blob_capacity_ints >= shape->plan_ints, BSX_ERR_CAPACITY,
               "plan blob needs %d int32 entries, capacity %lld", shape->plan_ints,
               (long long)blob_capacity_ints);
  HostSchedule hs;
  int rc = validate_table(qo_indptr_h, kv_indptr_h, kv_last_page_len_h, batch,
                          shape->page_size, shape->mask_mode, kv_indices_len, &hs);
  if (rc != BSX_OK) return rc;
  PLAN_REQUIRE(hs.max_qo <= shape->max_qo_len, BSX_ERR_CAPACITY,
               "a request has %d query tokens, the fixed shape allows %d", hs.max_qo,
               shape->max_qo_len);
  PLAN_REQUIRE(hs.safe_pos >= 0, BSX_ERR_INVALID, "the page table holds no page");
  schedule(batch, shape->mask_mode, shape->sink_tokens, shape->window_tokens, shape->num_ctas,
           &hs);
  const int W = shape->num_ctas;
  PLAN_REQUIRE(hs.nseg <= shape->num_segments, BSX_ERR_CAPACITY,
               "schedule of %d segments exceeds the fixed bound %d", hs.nseg,
               shape->num_segments);
  // the merge-record region between off_merge_seqs and off_part_indptr holds one record
  // per request of the shape; the partial slots are bounded by the segments above
  PLAN_REQUIRE((int64_t)hs.merge_seqs.size() <= shape->batch &&
                   (int64_t)hs.part_indptr[batch] <= shape->num_partials,
               BSX_ERR_CAPACITY, "schedule of %d merge records / %d partial slots exceeds the "
               "fixed bounds %d / %d", (int)hs.merge_seqs.size(), (int)hs.part_indptr[batch],
               shape->batch, shape->num_partials);
  write_blob(hs, qo_indptr_h, kv_indptr_h, batch, shape->batch, W, shape->off_seq,
             shape->off_seg_indptr, shape->off_segments, shape->off_merge_seqs,
             shape->off_part_indptr, plan_blob_h);
  int32_t* dyn = plan_blob_h + shape->off_dyn;
  dyn[0] = (int32_t)hs.merge_seqs.size();
  dyn[1] = 0;
  dyn[2] = hs.nseg;
  dyn[3] = 0;
  *out = *shape;
  out->total_qo = qo_indptr_h[batch];
  out->total_tiles = hs.total_tiles;
  return BSX_OK;
}

// Device-planned attention: shape, grid and a blob layout sized by bounds (the
// device planner, plan_device.hip, fills the blob from the device page table).
extern "C" int bsx_attn_plan_device_shape(int batch, int num_qo_heads, int num_kv_heads,
                                          int head_dim, int page_size, int mask_mode,
                                          int sink_tokens, int window_tokens, float sm_scale,
                                          int num_cus, int max_qo_len, bsx_attn_plan_t* out) {
  PLAN_REQUIRE(out, BSX_ERR_INVALID, "null plan");
  PLAN_REQUIRE(batch >= 1 && batch <= bsx::attn_shape::kMaxDevicePlanBatch, BSX_ERR_UNSUPPORTED,
               "device plans take 1..%d requests (got %d)", bsx::attn_shape::kMaxDevicePlanBatch,
               batch);
  PLAN_REQUIRE(num_kv_heads > 0 && num_qo_heads > 0 && num_qo_heads % num_kv_heads == 0,
               BSX_ERR_INVALID, "num_qo_heads (%d) must be a positive multiple of num_kv_heads (%d)",
               num_qo_heads, num_kv_heads);
  PLAN_REQUIRE(head_dim == 64 || head_dim == 128, BSX_ERR_UNSUPPORTED,
               "head_dim %d not supported (64 or 128)", head_dim);
  PLAN_REQUIRE(page_size >= 1 && page_size <= 1024 && (page_size & (page_size - 1)) == 0,
               BSX_ERR_UNSUPPORTED, "page_size %d must be a power of two <= 1024", page_size);
  PLAN_REQUIRE(mask_mode >= BSX_MASK_NONE && mask_mode <= BSX_MASK_STREAMING, BSX_ERR_INVALID,
               "unknown mask mode %d", mask_mode);
  PLAN_REQUIRE(num_cus >= 1, BSX_ERR_INVALID, "num_cus must be >= 1");
  PLAN_REQUIRE(mask_mode != BSX_MASK_STREAMING || (sink_tokens >= 0 && window_tokens >= 0),
               BSX_ERR_INVALID, "streaming view needs sink >= 0 and window >= 0");
  PLAN_REQUIRE(max_qo_len >= 1, BSX_ERR_INVALID, "max_qo_len must be >= 1");
  PLAN_REQUIRE(mask_mode != BSX_MASK_TREE || max_qo_len <= 32, BSX_ERR_UNSUPPORTED,
               "tree mask supports at most 32 query tokens per request");
  const int group = num_qo_heads / num_kv_heads;
  const GridShape gs =
      grid_shape(max_qo_len, group, num_kv_heads, head_dim, page_size, num_cus, mask_mode);
  const int W = gs.num_ctas;
  PLAN_REQUIRE(W <= bsx::attn_shape::kMaxDevicePlanCtas, BSX_ERR_UNSUPPORTED,
               "grid of %d workgroups too large for a device plan", W);
  const int64_t max_segs = (int64_t)W + 2LL * batch;
  const int64_t off_seg_indptr = 4LL * batch;
  const int64_t off_segments = off_seg_indptr + W + 1;
  const int64_t off_merge = (off_segments + 4 * max_segs + 3) & ~3LL;
  const int64_t off_part = off_merge + 4LL * batch;
  const int64_t off_dyn = off_part + batch + 1;
  const int64_t ints = off_dyn + 4;
  PLAN_REQUIRE(ints < (1LL << 31), BSX_ERR_UNSUPPORTED, "batch too large for a device plan");

  memset(out, 0, sizeof(*out));
  out->batch = batch;
  out->num_qo_heads = num_qo_heads;
  out->num_kv_heads = num_kv_heads;
  out->head_dim = head_dim;
  out->page_size = page_size;
  out->mask_mode = mask_mode;
  out->group_size = group;
  out->qrow_tile = gs.qrow_tile;
  out->qrow_blocks = gs.qrow_blocks;
  out->heads_per_cta = gs.hpc;
  out->qblocks_per_cta = gs.qbpc;
  out->num_qgroups = gs.n_qgroups;
  out->num_ctas = W;
  out->num_segments = (int32_t)max_segs;
  out->num_partials = (int32_t)max_segs;
  out->num_split_requests = batch;  // bound: the merge grid covers every request
  out->max_qo_len = max_qo_len;
  out->tile_tokens = kTileTokens;
  out->sink_tokens = sink_tokens;
  out->window_tokens = window_tokens;
  out->off_seq = 0;
  out->off_seg_indptr = (int32_t)off_seg_indptr;
  out->off_segments = (int32_t)off_segments;
  out->off_merge_seqs = (int32_t)off_merge;
  out->off_part_indptr = (int32_t)off_part;
  out->plan_ints = (int32_t)ints;
  const int64_t rows_total = (int64_t)gs.qrow_tile * gs.qrow_blocks;
  out->float_ws_bytes = max_segs * num_kv_heads * rows_total * (head_dim * 2 + 4);
  out->sm_scale = sm_scale > 0.f ? sm_scale : 1.0f / std::sqrt((float)head_dim);
  out->total_qo = batch * max_qo_len;  // bound: q / out need this many token rows
  out->safe_page_pos = 0;  // the table holds a page (checked by the planner)
  out->shared_kv_tiles = gs.shared ? 1 : 0;
  out->total_tiles = -1;
  out->device_plan = 1;
  out->off_dyn = (int32_t)off_dyn;
  return BSX_OK;
}
