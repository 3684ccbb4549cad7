// Paged KV append (piece 2 of the verification path).
//
// Replaces the FlashInfer triple used by StandardKVCache.update
// (batchspec/models/modules/kv_cache.py:64-83):
//   seq_len[b]  = (kv_indptr[b+1] - kv_indptr[b] - 1) * page_size + last_page_len[b]
//   token i of request b (append_indptr[b] <= i < append_indptr[b+1]) lands at
//   pos = seq_len[b] - (append_indptr[b+1] - append_indptr[b]) + (i - append_indptr[b])
//   cache[kv_indices[kv_indptr[b] + pos / page_size], k|v, pos % page_size, h, :] = k|v[i, h, :]
// The page table already counts the new tokens (insert_kv runs before the layer
// loop, batchspec/backends/continuous/batch_builder.py:75).
//
// The copy is one 16-byte vector per thread; a thread finds its request by binary
// search over append_indptr, so no host read of append_indptr[-1] is needed.
#include "common.h"

namespace bsx {
namespace append {

__device__ __forceinline__ int seq_len_of(const int32_t* kv_indptr, const int32_t* last, int b,
                                          int page_size) {
  const int np = kv_indptr[b + 1] - kv_indptr[b];
  return np > 0 ? (np - 1) * page_size + last[b] : 0;
}

// Largest b with indptr[b] <= i (indptr non-decreasing, indptr[0] = 0 <= i < indptr[batch]).
__device__ __forceinline__ int find_request(const int32_t* indptr, int batch, int i) {
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (indptr[mid] <= i)
      lo = mid;
    else
      hi = mid - 1;
  }
  return lo;
}

__global__ void seq_lens_kernel(const int32_t* kv_indptr, const int32_t* last, int batch,
                                int page_size, int32_t* out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < batch) out[b] = seq_len_of(kv_indptr, last, b, page_size);
}

__global__ void batch_pos_kernel(const int32_t* append_indptr, const int32_t* seq_lens, int batch,
                                 int nnz, int32_t* bidx, int32_t* pos) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nnz) return;
  const int b = find_request(append_indptr, batch, i);
  const int n = append_indptr[b + 1] - append_indptr[b];
  bidx[i] = b;
  pos[i] = seq_lens[b] - n + (i - append_indptr[b]);
}

// Element bytes are 2 (bf16/fp16) or 4 (fp32): VPR 16-byte vectors per (token, head) row.
struct CopyArgs {
  const char* k;
  const char* v;
  int64_t k_stride_bytes, v_stride_bytes;  // between tokens
  char* k_cache;
  char* v_cache;
  int64_t page_stride_bytes;
  const int32_t* kv_indices;
  const int32_t* kv_indptr;
  int num_kv_heads, row_bytes, page_size;
  int vecs_per_row;
};

__device__ __forceinline__ void copy_one(const CopyArgs& a, int i, int b, int pos, int rem) {
  // rem = vector index inside the token: head h = rem / vecs_per_row, vector c.
  // A position outside the request's pages has no slot: nothing is written (the
  // reference would index a neighbouring request's page; we refuse to).
  if (b < 0 || pos < 0) return;
  if (pos >= (a.kv_indptr[b + 1] - a.kv_indptr[b]) * a.page_size) return;
  const int h = rem / a.vecs_per_row;
  const int c = rem - h * a.vecs_per_row;
  const int page = a.kv_indices[a.kv_indptr[b] + pos / a.page_size];
  const int slot = pos % a.page_size;
  const int64_t dst = (int64_t)page * a.page_stride_bytes +
                      ((int64_t)slot * a.num_kv_heads + h) * a.row_bytes + 16 * c;
  const int64_t srck = (int64_t)i * a.k_stride_bytes + (int64_t)h * a.row_bytes + 16 * c;
  const int64_t srcv = (int64_t)i * a.v_stride_bytes + (int64_t)h * a.row_bytes + 16 * c;
  *reinterpret_cast<u32x4*>(a.k_cache + dst) = *reinterpret_cast<const u32x4*>(a.k + srck);
  *reinterpret_cast<u32x4*>(a.v_cache + dst) = *reinterpret_cast<const u32x4*>(a.v + srcv);
}

__global__ void append_kernel(CopyArgs a, const int32_t* bidx, const int32_t* pos, int nnz) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_tok = a.num_kv_heads * a.vecs_per_row;
  const int64_t i = t / per_tok;
  if (i >= nnz) return;
  copy_one(a, (int)i, bidx[i], pos[i], (int)(t - i * per_tok));
}

__global__ void fused_append_kernel(CopyArgs a, const int32_t* append_indptr,
                                    const int32_t* kv_last_page_len, int batch, int nnz) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_tok = a.num_kv_heads * a.vecs_per_row;
  const int64_t i = t / per_tok;
  if (i >= nnz) return;
  const int ii = (int)i;
  if (ii >= append_indptr[batch]) return;  // k has more rows than the indptr covers
  const int b = find_request(append_indptr, batch, ii);
  const int n = append_indptr[b + 1] - append_indptr[b];
  const int sl = seq_len_of(a.kv_indptr, kv_last_page_len, b, a.page_size);
  copy_one(a, ii, b, sl - n + (ii - append_indptr[b]), (int)(t - i * per_tok));
}

static int make_args(CopyArgs& a, const void* k, const void* v, int64_t ks, int64_t vs, void* kc,
                     void* vc, int64_t page_stride, const int32_t* kv_indices,
                     const int32_t* kv_indptr, int num_kv_heads, int head_dim, int page_size,
                     int elem_bytes) {
  BSX_REQUIRE(k && v && kc && vc && kv_indices && kv_indptr, BSX_ERR_INVALID,
              "null pointer to kv append");
  BSX_REQUIRE(elem_bytes == 2 || elem_bytes == 4, BSX_ERR_INVALID, "elem_bytes must be 2 or 4");
  BSX_REQUIRE(num_kv_heads > 0 && head_dim > 0 && page_size > 0, BSX_ERR_INVALID,
              "bad kv shape");
  const int row_bytes = head_dim * elem_bytes;
  BSX_REQUIRE(row_bytes % 16 == 0, BSX_ERR_UNSUPPORTED,
              "head_dim*elem_bytes must be a multiple of 16 (got %d)", row_bytes);
  BSX_REQUIRE(((uintptr_t)k | (uintptr_t)v | (uintptr_t)kc | (uintptr_t)vc) % 16 == 0 &&
                  (ks * elem_bytes) % 16 == 0 && (vs * elem_bytes) % 16 == 0 &&
                  (page_stride * elem_bytes) % 16 == 0,
              BSX_ERR_INVALID, "kv append needs 16-byte aligned pointers and strides");
  a.k = static_cast<const char*>(k);
  a.v = static_cast<const char*>(v);
  a.k_stride_bytes = ks * elem_bytes;
  a.v_stride_bytes = vs * elem_bytes;
  a.k_cache = static_cast<char*>(kc);
  a.v_cache = static_cast<char*>(vc);
  a.page_stride_bytes = page_stride * elem_bytes;
  a.kv_indices = kv_indices;
  a.kv_indptr = kv_indptr;
  a.num_kv_heads = num_kv_heads;
  a.row_bytes = row_bytes;
  a.page_size = page_size;
  a.vecs_per_row = row_bytes / 16;
  return BSX_OK;
}

}  // namespace append
}  // namespace bsx

using namespace bsx;

extern "C" int bsx_get_seq_lens(const int32_t* kv_indptr_d, const int32_t* kv_last_page_len_d,
                                int batch, int page_size, int32_t* seq_lens_d, void* stream) {
  BSX_REQUIRE(batch >= 0 && page_size > 0, BSX_ERR_INVALID, "bad batch/page_size");
  if (batch == 0) return BSX_OK;
  BSX_REQUIRE(kv_indptr_d && kv_last_page_len_d && seq_lens_d, BSX_ERR_INVALID, "null pointer");
  hipLaunchKernelGGL(append::seq_lens_kernel, dim3((batch + 255) / 256), dim3(256), 0,
                     as_stream(stream), kv_indptr_d, kv_last_page_len_d, batch, page_size,
                     seq_lens_d);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

extern "C" int bsx_get_batch_indices_positions(const int32_t* append_indptr_d,
                                               const int32_t* seq_lens_d, int batch, int nnz,
                                               int32_t* batch_indices_d, int32_t* positions_d,
                                               void* stream) {
  BSX_REQUIRE(batch >= 0 && nnz >= 0, BSX_ERR_INVALID, "bad batch/nnz");
  if (nnz == 0) return BSX_OK;
  BSX_REQUIRE(batch > 0, BSX_ERR_INVALID, "nnz > 0 with an empty batch");
  BSX_REQUIRE(append_indptr_d && seq_lens_d && batch_indices_d && positions_d, BSX_ERR_INVALID,
              "null pointer");
  hipLaunchKernelGGL(append::batch_pos_kernel, dim3((nnz + 255) / 256), dim3(256), 0,
                     as_stream(stream), append_indptr_d, seq_lens_d, batch, nnz, batch_indices_d,
                     positions_d);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

extern "C" int bsx_append_paged_kv_cache(const void* append_key_d, const void* append_value_d,
                                         int64_t key_stride_tok, int64_t value_stride_tok,
                                         const int32_t* batch_indices_d,
                                         const int32_t* positions_d, int nnz, void* k_cache_d,
                                         void* v_cache_d, int64_t page_stride,
                                         const int32_t* kv_indices_d, const int32_t* kv_indptr_d,
                                         int num_kv_heads, int head_dim, int page_size,
                                         int elem_bytes, void* stream) {
  BSX_REQUIRE(nnz >= 0, BSX_ERR_INVALID, "nnz must be >= 0");
  if (nnz == 0) return BSX_OK;
  BSX_REQUIRE(batch_indices_d && positions_d, BSX_ERR_INVALID, "null batch_indices/positions");
  append::CopyArgs a;
  int rc = append::make_args(a, append_key_d, append_value_d, key_stride_tok, value_stride_tok,
                             k_cache_d, v_cache_d, page_stride, kv_indices_d, kv_indptr_d,
                             num_kv_heads, head_dim, page_size, elem_bytes);
  if (rc != BSX_OK) return rc;
  const int64_t threads = (int64_t)nnz * num_kv_heads * a.vecs_per_row;
  hipLaunchKernelGGL(append::append_kernel, dim3((unsigned)ceil_div(threads, 256)), dim3(256), 0,
                     as_stream(stream), a, batch_indices_d, positions_d, nnz);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

extern "C" int bsx_kv_append(const void* k_d, const void* v_d, int64_t k_stride_tok,
                             int64_t v_stride_tok, const int32_t* append_indptr_d,
                             const int32_t* kv_indptr_d, const int32_t* kv_indices_d,
                             const int32_t* kv_last_page_len_d, int batch, int nnz,
                             void* k_cache_d, void* v_cache_d, int64_t page_stride,
                             int num_kv_heads, int head_dim, int page_size, int elem_bytes,
                             void* stream) {
  BSX_REQUIRE(batch >= 0 && nnz >= 0, BSX_ERR_INVALID, "bad batch/nnz");
  if (nnz == 0 || batch == 0) return BSX_OK;
  BSX_REQUIRE(append_indptr_d && kv_last_page_len_d, BSX_ERR_INVALID, "null pointer");
  append::CopyArgs a;
  int rc = append::make_args(a, k_d, v_d, k_stride_tok, v_stride_tok, k_cache_d, v_cache_d,
                             page_stride, kv_indices_d, kv_indptr_d, num_kv_heads, head_dim,
                             page_size, elem_bytes);
  if (rc != BSX_OK) return rc;
  const int64_t threads = (int64_t)nnz * num_kv_heads * a.vecs_per_row;
  hipLaunchKernelGGL(append::fused_append_kernel, dim3((unsigned)ceil_div(threads, 256)),
                     dim3(256), 0, as_stream(stream), a, append_indptr_d, kv_last_page_len_d,
                     batch, nnz);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}
