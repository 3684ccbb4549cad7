// Boolean custom attention masks packed on the device.
//
// The MTP engine passes plan() a flattened boolean mask, per request
// cat(ones(qo_len, cachelen), common_attn_mask) of qo_len x kv_len entries
// (batchspec/backends/mtp_engine.py:399-432), and FlashInfer's plan() packs it into bits
// on the device (custom_mask: "the flattened boolean mask, sum(qo_len[i] * kv_len[i])
// entries").  Here:
//   1. packbits_kernel: bit u of word w = entry 32 w + u of the flattened mask (little
//      bit order, the flat order of the reference's mask); one padding word follows.
//   2. mask_rows_kernel, one workgroup per request: whether the request's mask has the
//      tree form (every row sees its first kv_len - qo_len tokens, qo_len <= 32), and
//      then each query token's tree word (bit c = entry (i, kv_len - qo_len + c)), the
//      attention's fast mask; otherwise the request needs the general mask (per-tile
//      bit words read from the packed bits by the attention kernel).
// Descriptor layout (uint32): [batch] bit offsets of the requests' masks, then the
// packed bits (their word 0 at index batch).
#include "common.h"

namespace bsx {
namespace cmask {

__device__ __forceinline__ uint32_t nz_bits4(uint32_t v) {
  return ((v & 0xffu) != 0u ? 1u : 0u) | ((v & 0xff00u) != 0u ? 2u : 0u) |
         ((v & 0xff0000u) != 0u ? 4u : 0u) | ((v & 0xff000000u) != 0u ? 8u : 0u);
}

__global__ void __launch_bounds__(256) packbits_kernel(const uint8_t* m, int64_t n, bool vec,
                                                       uint32_t* bits, int64_t nwords) {
  const int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (w > nwords) return;  // word nwords is the padding word
  const int64_t b0 = 32 * w;
  uint32_t word = 0u;
  if (vec && b0 + 32 <= n) {
    const uint4 a = reinterpret_cast<const uint4*>(m + b0)[0];
    const uint4 c = reinterpret_cast<const uint4*>(m + b0)[1];
    word = nz_bits4(a.x) | nz_bits4(a.y) << 4 | nz_bits4(a.z) << 8 | nz_bits4(a.w) << 12 |
           nz_bits4(c.x) << 16 | nz_bits4(c.y) << 20 | nz_bits4(c.z) << 24 | nz_bits4(c.w) << 28;
  } else {
    for (int u = 0; u < 32; ++u)
      if (b0 + u < n && m[b0 + u] != 0) word |= 1u << u;
  }
  bits[w] = word;
}

// 32 mask bits starting at bit f (f + 32 may run into the padding word).
__device__ __forceinline__ uint32_t bits_at(const uint32_t* bits, int64_t f) {
  const int64_t w = f >> 5;
  const uint64_t pair = ((uint64_t)bits[w + 1] << 32) | bits[w];
  return (uint32_t)(pair >> (f & 31));
}

// req: [batch][4] = (qo_start, qo_len, kv_len, bit offset).  general[b]: 0 tree form,
// 1 general mask, 2 malformed (the request's bits do not lie inside the mask).
__global__ void __launch_bounds__(256) mask_rows_kernel(const int32_t* req, int64_t n,
                                                        uint32_t* desc, int batch,
                                                        uint32_t* tree_words, int32_t* general) {
  __shared__ int s_bad;
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int qo_start = req[4 * b], q = req[4 * b + 1], k = req[4 * b + 2];
  const int64_t off = req[4 * b + 3];
  const uint32_t* bits = desc + batch;
  if (t == 0) {
    desc[b] = (uint32_t)off;
    s_bad = 0;
  }
  __syncthreads();
  int g;
  if (q < 0 || k < 0 || off < 0 || off + (int64_t)q * k > n) {
    g = 2;
  } else if (q == 0) {
    g = 0;
  } else if (q > 32 || k < q) {
    g = 1;
  } else {
    // every row's first k - q entries set
    const int pre = k - q;
    const int nchunk = (pre + 31) / 32;
    bool bad = false;
    for (int64_t idx = t; idx < (int64_t)q * nchunk; idx += blockDim.x) {
      const int i = (int)(idx / nchunk);
      const int c = (int)(idx - (int64_t)i * nchunk);
      const int len = min(32, pre - 32 * c);
      const uint32_t need = len == 32 ? ~0u : (1u << len) - 1u;
      if ((bits_at(bits, off + (int64_t)i * k + 32 * c) & need) != need) bad = true;
    }
    if (bad) s_bad = 1;  // (any writer sets the same value)
    __syncthreads();
    g = s_bad ? 1 : 0;
    if (g == 0) {
      const uint32_t keep = q == 32 ? ~0u : (1u << q) - 1u;
      for (int i = t; i < q; i += blockDim.x)
        tree_words[qo_start + i] = bits_at(bits, off + (int64_t)i * k + pre) & keep;
    }
  }
  if (t == 0) general[b] = g;
}

}  // namespace cmask
}  // namespace bsx

using namespace bsx;

extern "C" int bsx_custom_mask_prepare(const void* mask_d, int64_t n_bools, const int32_t* req_d,
                                       int batch, uint32_t* desc_d, uint32_t* tree_words_d,
                                       int32_t* general_d, void* stream) {
  BSX_REQUIRE(batch >= 0 && n_bools >= 0, BSX_ERR_INVALID, "batch and n_bools must be >= 0");
  BSX_REQUIRE(n_bools < (1LL << 31), BSX_ERR_UNSUPPORTED,
              "custom masks hold fewer than 2^31 entries (got %lld)", (long long)n_bools);
  if (batch == 0) return BSX_OK;
  BSX_REQUIRE(req_d && desc_d && tree_words_d && general_d && (mask_d || n_bools == 0),
              BSX_ERR_INVALID, "null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t nwords = (n_bools + 31) / 32;
  const bool vec = (reinterpret_cast<uintptr_t>(mask_d) % 16) == 0;
  hipLaunchKernelGGL(cmask::packbits_kernel, dim3((unsigned)ceil_div(nwords + 1, 256)), dim3(256),
                     0, st, static_cast<const uint8_t*>(mask_d), n_bools, vec, desc_d + batch,
                     nwords);
  BSX_LAUNCH_CHECK();
  hipLaunchKernelGGL(cmask::mask_rows_kernel, dim3((unsigned)batch), dim3(256), 0, st, req_d,
                     n_bools, desc_d, batch, tree_words_d, general_d);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}
