// Workgroup-shape rules of the verify-attention kernels, shared by the host planner
// (plan.cpp) and the kernels (attn.hip).
#pragma once

namespace bsx {
namespace attn_shape {

constexpr int kTileTokens = 32;     // kv tokens per inner-loop tile
constexpr int kMaxWavesPerCta = 8;
constexpr int kSharedLdsBytes = 128 * 1024;  // LDS of the shared-tile kernel

// Bytes of one kv head's K and V tile.
constexpr int head_tile_bytes(int head_dim) { return 2 * kTileTokens * head_dim * 2; }

// Ring depth of the shared-tile kernel with qb waves per kv head: the deepest ring
// that holds 8 / qb heads in kSharedLdsBytes.
constexpr int shared_stages(int head_dim, int qb) { return (head_dim == 128 && qb == 2) ? 2 : 4; }

// Whether a workgroup of `heads` kv heads fits the shared-tile kernel's LDS.
constexpr bool shared_fits(int head_dim, int qb, int heads) {
  return shared_stages(head_dim, qb) * heads * head_tile_bytes(head_dim) <= kSharedLdsBytes;
}

}  // namespace attn_shape
}  // namespace bsx
