// Accepted-KV compaction after a verify step (the first "next" row of the path).
//
// Replaces MTPEngine.collate_accepted_kv_cache (batchspec/backends/mtp_engine.py:577-631).
// The verify step inserted (k+1)^2 KV rows per request starting at prev_cachelens[b]:
// regular token i sits at position prev + i*(k+1), followed by its k mask tokens.  The
// first accept_nums[b] regular tokens are kept, moved to positions prev + i.  The
// reference does this with a permute/reshape that copies every layer's whole cache
// each step and assumes each request's pages are contiguous (page id r*max_pages+k);
// here only the accepted rows move, in place, addressed through the page table.
//
// Race freedom: for 1 <= i < accept <= k+1 the destinations prev+1 .. prev+k lie below
// every source prev + j*(k+1), j >= 1, so no move reads a row another move writes
// (i = 0 is the identity and is skipped).  Requests own disjoint pages.
//
// One workgroup per (request, layer); each thread copies 16-byte vectors of the K and
// V rows.  Accept counts are clamped to [0, k+1] and positions beyond the request's
// pages are skipped, so no input can address outside the request's pages.
#include "common.h"

namespace bsx {
namespace collate {

struct Args {
  const int64_t* accept_nums;
  const int32_t* prev_cachelens;
  const int32_t* kv_indptr;
  const int32_t* kv_indices;
  const int64_t* k_bases;  // per-layer base addresses
  const int64_t* v_bases;
  int64_t page_stride_bytes;
  int stride;  // draft_length + 1
  int num_kv_heads, row_bytes, page_size, vecs_per_token;
};

__global__ void __launch_bounds__(256) collate_kernel(Args a) {
  const int b = blockIdx.x;
  const int layer = blockIdx.y;
  const int64_t acc = a.accept_nums[b];
  const int accept = (int)(acc < 0 ? 0 : (acc > a.stride ? a.stride : acc));
  if (accept <= 1) return;
  const int prev = a.prev_cachelens[b];
  const int p0 = a.kv_indptr[b];
  const int npos = (a.kv_indptr[b + 1] - p0) * a.page_size;
  char* kc = reinterpret_cast<char*>(a.k_bases[layer]);
  char* vc = reinterpret_cast<char*>(a.v_bases[layer]);
  const int per_move = a.vecs_per_token;  // vectors of one K (or V) token row
  const int total = (accept - 1) * per_move;
  for (int t = threadIdx.x; t < total; t += blockDim.x) {
    const int i = 1 + t / per_move;
    const int c = t - (i - 1) * per_move;
    const int src = prev + i * a.stride;
    const int dst = prev + i;
    if (prev < 0 || src >= npos) continue;
    const int sp = a.kv_indices[p0 + src / a.page_size];
    const int dp = a.kv_indices[p0 + dst / a.page_size];
    const int64_t so = (int64_t)sp * a.page_stride_bytes +
                       (int64_t)(src % a.page_size) * a.vecs_per_token * 16 + 16 * (int64_t)c;
    const int64_t dof = (int64_t)dp * a.page_stride_bytes +
                        (int64_t)(dst % a.page_size) * a.vecs_per_token * 16 + 16 * (int64_t)c;
    const u32x4 kv = *reinterpret_cast<const u32x4*>(kc + so);
    const u32x4 vv = *reinterpret_cast<const u32x4*>(vc + so);
    *reinterpret_cast<u32x4*>(kc + dof) = kv;
    *reinterpret_cast<u32x4*>(vc + dof) = vv;
  }
}

}  // namespace collate
}  // namespace bsx

using namespace bsx;

extern "C" int bsx_collate_accepted_kv(const int64_t* accept_nums_d,
                                       const int32_t* prev_cachelens_d, int batch,
                                       int draft_length, const int32_t* kv_indptr_d,
                                       const int32_t* kv_indices_d, const int64_t* k_bases_d,
                                       const int64_t* v_bases_d, int num_layers,
                                       int64_t page_stride, int num_kv_heads, int head_dim,
                                       int page_size, int elem_bytes, void* stream) {
  BSX_REQUIRE(batch >= 0 && num_layers >= 0, BSX_ERR_INVALID, "batch and num_layers must be >= 0");
  if (batch == 0 || num_layers == 0) return BSX_OK;
  BSX_REQUIRE(accept_nums_d && prev_cachelens_d && kv_indptr_d && kv_indices_d && k_bases_d &&
                  v_bases_d,
              BSX_ERR_INVALID, "null pointer to collate");
  BSX_REQUIRE(draft_length >= 0, BSX_ERR_INVALID, "draft_length must be >= 0");
  BSX_REQUIRE(elem_bytes == 2 || elem_bytes == 4, BSX_ERR_INVALID, "elem_bytes must be 2 or 4");
  BSX_REQUIRE(num_kv_heads > 0 && head_dim > 0 && page_size > 0, BSX_ERR_INVALID,
              "bad kv shape");
  const int64_t row_bytes = (int64_t)head_dim * elem_bytes;
  BSX_REQUIRE(row_bytes % 16 == 0 && (page_stride * elem_bytes) % 16 == 0, BSX_ERR_UNSUPPORTED,
              "head_dim*elem_bytes and the page stride must be multiples of 16 bytes");
  BSX_REQUIRE(batch <= 65535 * 1024 && num_layers <= 65535, BSX_ERR_UNSUPPORTED,
              "too many requests or layers for one launch");
  collate::Args a;
  a.accept_nums = accept_nums_d;
  a.prev_cachelens = prev_cachelens_d;
  a.kv_indptr = kv_indptr_d;
  a.kv_indices = kv_indices_d;
  a.k_bases = k_bases_d;
  a.v_bases = v_bases_d;
  a.page_stride_bytes = page_stride * elem_bytes;
  a.stride = draft_length + 1;
  a.num_kv_heads = num_kv_heads;
  a.row_bytes = (int)row_bytes;
  a.page_size = page_size;
  a.vecs_per_token = (int)(num_kv_heads * row_bytes / 16);
  hipLaunchKernelGGL(collate::collate_kernel, dim3(batch, num_layers), dim3(256), 0,
                     as_stream(stream), a);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}
