// Streaming-read probe: a kernel that only reads its input once, with the load pattern
// of the acceptance kernels (non-temporal 16-byte loads, every load of a thread issued
// before any is used), in a configurable launch shape.  Its time for a buffer of the
// size a one-pass kernel reads is the floor that kernel is measured against (the greedy
// argmax reads the [B, k+1, V] logits once).  No counterpart in the reference.
#include "common.h"

namespace bsx {
namespace probe {

template <int U>
__global__ void read_probe_kernel(const u32x4* src, int64_t n16, uint32_t* sink) {
  const int64_t base = (int64_t)blockIdx.x * blockDim.x * U + threadIdx.x;
  u32x4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = min(base + (int64_t)u * blockDim.x, n16 - 1);
    v[u] = __builtin_nontemporal_load(src + i);
  }
  uint32_t x = 0;
#pragma unroll
  for (int u = 0; u < U; ++u) x ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  if (x == 0x9e3779b9u) sink[0] = x;  // keeps the loads live; the value is irrelevant
}

template <int U>
static void launch(const void* src, int64_t n16, int threads, uint32_t* sink, hipStream_t st) {
  const int64_t per_wg = (int64_t)threads * U;
  const dim3 grid((unsigned)((n16 + per_wg - 1) / per_wg));
  hipLaunchKernelGGL((read_probe_kernel<U>), grid, dim3(threads), 0, st,
                     static_cast<const u32x4*>(src), n16, sink);
}

}  // namespace probe
}  // namespace bsx

using namespace bsx;

extern "C" int bsx_read_probe(const void* src_d, int64_t bytes, int threads,
                              int loads_per_thread, uint32_t* sink_d, void* stream) {
  BSX_REQUIRE(src_d && sink_d, BSX_ERR_INVALID, "null pointer");
  BSX_REQUIRE(bytes > 0 && bytes % 16 == 0, BSX_ERR_INVALID,
              "bytes must be a positive multiple of 16 (got %lld)", (long long)bytes);
  BSX_REQUIRE(threads == 64 || threads == 128 || threads == 256 || threads == 512 ||
                  threads == 1024,
              BSX_ERR_INVALID, "threads must be 64, 128, 256, 512 or 1024");
  const int64_t n16 = bytes / 16;
  const int64_t wgs = (n16 + (int64_t)threads * loads_per_thread - 1) /
                      ((int64_t)threads * loads_per_thread);
  BSX_REQUIRE(wgs < (1LL << 31), BSX_ERR_UNSUPPORTED, "buffer too large for one launch");
  hipStream_t st = as_stream(stream);
  switch (loads_per_thread) {
    case 1: probe::launch<1>(src_d, n16, threads, sink_d, st); break;
    case 2: probe::launch<2>(src_d, n16, threads, sink_d, st); break;
    case 4: probe::launch<4>(src_d, n16, threads, sink_d, st); break;
    case 8: probe::launch<8>(src_d, n16, threads, sink_d, st); break;
    case 16: probe::launch<16>(src_d, n16, threads, sink_d, st); break;
    case 32: probe::launch<32>(src_d, n16, threads, sink_d, st); break;
    default:
      set_error("loads_per_thread must be 1, 2, 4, 8, 16 or 32 (got %d)", loads_per_thread);
      return BSX_ERR_INVALID;
  }
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}
