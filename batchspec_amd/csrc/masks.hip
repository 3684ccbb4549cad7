// Draft-tree masks and positions on the device (a "next" row of the path).
//
// Replaces the host-side mask producers of the verify step:
//   * MTPEngine._setup_common_attn_mask_and_position_ids
//     (batchspec/backends/mtp_engine.py:172-208): the (k+1)^2 MTP layout, whose mask is
//     the ancestor relation of a tree (parent(x_g) = x_{g-1}, parent(m_1@g) = x_g,
//     parent(m_r@g) = m_{r-1}@g) and whose position ids g + r are the node depths;
//   * the per-request Python loop that concatenates ones(S, cachelen_b) with that mask
//     before plan() (mtp_engine.py:410-417), and the position ids
//     cachelens[:, None] + common_position_ids (mtp_engine.py:381);
//   * EAGLE-style token trees given by a parent array.
// Output: per token one uint32 word, bit j set iff draft token j is the token itself or
// one of its ancestors (the attention's tree-mask format: every cached column is
// visible), and position = cachelen_b + depth.
//
// One thread per (request, token) walks up its parent chain (at most n <= 32 steps).
// A parent that does not precede its token (parent >= i, or < -1) ends the chain there,
// so any input terminates and addresses only its own request's row.
#include "common.h"

namespace bsx {
namespace masks {

__global__ void __launch_bounds__(256) tree_mask_kernel(const int32_t* parents,
                                                        int64_t parents_stride, int n,
                                                        const int32_t* cachelens, int B,
                                                        uint32_t* words, int64_t* positions) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)B * n) return;
  const int b = (int)(gid / n);
  const int i = (int)(gid - (int64_t)b * n);
  const int32_t* par = parents + (int64_t)b * parents_stride;
  uint32_t w = 1u << i;
  int depth = 0;
  int j = i;
  for (int step = 0; step < n; ++step) {
    const int p = par[j];
    if (p < 0 || p >= j) break;
    w |= 1u << p;
    ++depth;
    j = p;
  }
  words[gid] = w;
  if (positions != nullptr) positions[gid] = (cachelens ? (int64_t)cachelens[b] : 0) + depth;
}

}  // namespace masks
}  // namespace bsx

using namespace bsx;

extern "C" int bsx_tree_masks(const int32_t* parents_d, int64_t parents_stride, int n,
                              const int32_t* cachelens_d, int B, uint32_t* words_d,
                              int64_t* positions_d, void* stream) {
  BSX_REQUIRE(B >= 0 && n >= 0, BSX_ERR_INVALID, "bad B=%d n=%d", B, n);
  BSX_REQUIRE(n <= 32, BSX_ERR_UNSUPPORTED, "at most 32 draft tokens per request (n=%d)", n);
  if (B == 0 || n == 0) return BSX_OK;
  BSX_REQUIRE(parents_d && words_d, BSX_ERR_INVALID, "null pointer");
  BSX_REQUIRE(parents_stride == 0 || parents_stride >= n, BSX_ERR_INVALID,
              "parents_stride must be 0 (shared) or >= n");
  const int64_t total = (int64_t)B * n;
  BSX_REQUIRE(total < (1LL << 31), BSX_ERR_UNSUPPORTED, "too many tokens");
  hipLaunchKernelGGL(masks::tree_mask_kernel, dim3((unsigned)ceil_div(total, (int64_t)256)),
                     dim3(256), 0, as_stream(stream), parents_d, parents_stride, n, cachelens_d,
                     B, words_d, positions_d);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}
