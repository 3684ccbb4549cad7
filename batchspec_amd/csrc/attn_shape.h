// Workgroup-shape rules of the verify-attention kernels, shared by the host planner
// (plan.cpp) and the kernels (attn.hip).
#pragma once

namespace bsx {
namespace attn_shape {

constexpr int kTileTokens = 32;     // kv tokens per inner-loop tile
// Planner cost of starting a segment, in kv tiles: the Q load of the new request (one
// memory latency) and the write of its (partial) result, measured on MI355X at about
// two tile times together.
constexpr int kSegmentCost = 2;
// Largest batch and grid a device-side plan handles (its per-request and
// per-segment state lives in LDS).
constexpr int kMaxDevicePlanBatch = 2048;
constexpr int kMaxDevicePlanCtas = 4096;
constexpr int kMaxWavesPerCta = 8;
constexpr int kLdsPerCu = 160 * 1024;

// Bytes of one kv head's K and V tile.
constexpr int head_tile_bytes(int head_dim) { return 2 * kTileTokens * head_dim * 2; }

// Shared-tile kernel with qb waves per kv head: at most shared_max_heads kv heads per
// workgroup, a ring of shared_stages tile stages.  Adjacent kv heads share a
// workgroup: the DRAM channels of a head's 256-byte slices of the token rows depend on
// the head (measured on MI355X: one fixed head per workgroup streams at 6.4 TB/s,
// two adjacent heads at 6.7 TB/s), and a workgroup's pace follows its slices.
constexpr int shared_max_heads(int head_dim, int qb) { return 8 / qb; }
constexpr int shared_stages(int head_dim, int qb) { return (head_dim == 128 && qb == 2) ? 2 : 4; }
constexpr int shared_lds_bytes(int head_dim, int qb) {
  return shared_stages(head_dim, qb) * shared_max_heads(head_dim, qb) * head_tile_bytes(head_dim);
}

// Wave-split kernel (bsx_attn_plan_t.shared_kv_tiles == kPlanWaveSplit): one workgroup
// of kSplitWaves waves per (request, kv head), the waves splitting the request's visible
// tiles and merging in LDS.  Planned for at most 16 query rows per kv head, pages of 16+
// tokens, causal / no / sink + window masks, no request with more than kSplitMaxTiles
// visible tiles, and between half the compute units and all of them in (request, kv
// head) pairs, when the time model below puts it ahead of the split-KV schedule.
constexpr int kPlanWaveSplit = 2;
constexpr int kSplitWaves = 8;
constexpr int kSplitMaxTiles = 4 * kSplitWaves;

// Time model of the two schedules in microseconds, fitted on MI355X to the measured
// kernel times (head dim 128, bf16) of decode and 4-token draft batches with 128..512
// (request, kv head) pairs and views of 10..32 tiles; MB = visible K/V bytes / 1e6.
// Checked at head dim 64 and at 8 query heads per kv head (128..256 pairs).
//   wave-split: max(kWsLatencyUs + kWsWaveTileUs * (D / 128) * (longest view's tiles)
//                   / kSplitWaves, kWsFixedUs + kWsUsPerMB * MB)
//     the longest view's run per wave, or the workgroups' streaming (5.5 TB/s)
//   split-KV:   kSkFixedUs + kSkUsPerMB * MB + kSkRowUs * (query rows per kv head - 4)
//     the merge launch and partials, the balanced stream (7.0 TB/s), the partial rows
// Above one workgroup per compute unit the wave-split kernel's two co-resident
// workgroups per unit fall behind the balanced split (measured 4-36% slower at 288-2048
// pairs, except sink + window views within 5%), so it is not planned there.
constexpr double kWsLatencyUs = 7.55;
constexpr double kWsWaveTileUs = 3.47;
constexpr double kWsFixedUs = 6.25;
constexpr double kWsUsPerMB = 0.182;
constexpr double kSkFixedUs = 11.81;
constexpr double kSkUsPerMB = 0.143;
constexpr double kSkRowUs = 0.294;

}  // namespace attn_shape
}  // namespace bsx
