// Sync-free page-table update (a "next" row of the path): one workgroup per call, the
// update rule in page_update.h.
#include "page_update.h"

namespace bsx {
namespace pt {

__global__ void __launch_bounds__(kThreads) page_table_kernel(Args a) {
  update_pages(a, [&](int r) -> int32_t { return a.d ? a.d[r] : a.d_scalar; });
}

}  // namespace pt
}  // namespace bsx

using namespace bsx;

extern "C" int bsx_page_table_update(int32_t* num_pages_d, int32_t* last_len_d,
                                     int32_t* cachelens_d, const int32_t* d_d,
                                     int32_t d_scalar, int sign, int B, int page_size,
                                     int max_pages, int32_t* indptr_d, int32_t* indices_d,
                                     int32_t* errors_d, void* stream) {
  BSX_REQUIRE(B >= 0, BSX_ERR_INVALID, "bad batch %d", B);
  if (B == 0) return BSX_OK;
  BSX_REQUIRE(sign == 1 || sign == -1, BSX_ERR_INVALID, "sign must be +1 (insert) or -1 (delete)");
  BSX_REQUIRE(page_size > 0 && max_pages > 0, BSX_ERR_INVALID, "bad page_size or max_pages");
  BSX_REQUIRE((int64_t)B * max_pages < (1LL << 31), BSX_ERR_UNSUPPORTED, "page table too large");
  BSX_REQUIRE(num_pages_d && last_len_d && indptr_d && indices_d, BSX_ERR_INVALID,
              "null pointer");
  pt::Args a;
  a.num_pages = num_pages_d;
  a.last_len = last_len_d;
  a.cachelens = cachelens_d;
  a.d = d_d;
  a.d_scalar = d_scalar;
  a.sign = sign;
  a.B = B;
  a.page_size = page_size;
  a.max_pages = max_pages;
  a.indptr = indptr_d;
  a.indices = indices_d;
  a.errors = errors_d;
  hipLaunchKernelGGL(pt::page_table_kernel, dim3(1), dim3(pt::kThreads), 0, as_stream(stream), a);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}
