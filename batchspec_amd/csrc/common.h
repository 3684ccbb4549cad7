// Shared host/device helpers for the bsx C ABI: error reporting, argument checks,
// vector types and dtype conversion.  gfx950 (CDNA4) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/bsx.h"

namespace bsx {

// Thread-local last error, returned by bsx_last_error().
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

}  // namespace bsx

#define BSX_REQUIRE(cond, code, ...)   \
  do {                                 \
    if (!(cond)) {                     \
      ::bsx::set_error(__VA_ARGS__);   \
      return (code);                   \
    }                                  \
  } while (0)

#define BSX_HIP_CHECK(expr)                                                       \
  do {                                                                            \
    hipError_t _e = (expr);                                                       \
    if (_e != hipSuccess) {                                                       \
      ::bsx::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(_e),     \
                       __FILE__, __LINE__);                                       \
      return BSX_ERR_HIP;                                                         \
    }                                                                             \
  } while (0)

#define BSX_LAUNCH_CHECK()                                                         \
  do {                                                                            \
    hipError_t _e = hipGetLastError();                                            \
    if (_e != hipSuccess) {                                                       \
      ::bsx::set_error("kernel launch failed: %s (%s:%d)", hipGetErrorString(_e), \
                       __FILE__, __LINE__);                                       \
      return BSX_ERR_HIP;                                                         \
    }                                                                             \
  } while (0)

namespace bsx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Rows read through buffer descriptors are addressed with 32-bit byte offsets: a row of
// logits must stay below 2^31 bytes (entry points reject larger ones).
inline bool row_bytes_ok(int64_t vocab, int dtype) {
  return vocab > 0 && vocab * (dtype == BSX_DTYPE_FP32 ? 4 : 2) < (1LL << 31);
}

// Buffer descriptor of `bytes` bytes from `base` (below 2^31): raw 32-bit data, no
// stride; a load at or past `bytes` returns 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000 /* data format: 32 bits */);
}
// Non-temporal 16-byte load at voffset (per thread) + soffset (wave-uniform) bytes.
__device__ __forceinline__ u32x4 load_nt_b128(__amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset,
                                                                         2 /* nt */));
}

// 16-bit float element -> fp32 (exact) for the two storage dtypes.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
  return (float)h;
}

template <int DT>
__device__ __forceinline__ float half_bits_to_f32(uint32_t bits16) {
  if constexpr (DT == BSX_DTYPE_BF16) {
    return bf16_bits_to_f32(bits16);
  } else {
    return f16_bits_to_f32(bits16);
  }
}

// Low / high 16-bit element of a packed dword -> fp32.
template <int DT>
__device__ __forceinline__ float lo_f32(uint32_t w) {
  if constexpr (DT == BSX_DTYPE_BF16) return __uint_as_float(w << 16);
  else return f16_bits_to_f32(w & 0xFFFFu);
}
template <int DT>
__device__ __forceinline__ float hi_f32(uint32_t w) {
  if constexpr (DT == BSX_DTYPE_BF16) return __uint_as_float(w & 0xFFFF0000u);
  else return f16_bits_to_f32(w >> 16);
}

// fp32 -> 16-bit storage (round to nearest even).
template <int DT>
__device__ __forceinline__ uint16_t f32_to_half_bits(float f) {
  if constexpr (DT == BSX_DTYPE_BF16) {
    __bf16 h = (__bf16)f;
    return __builtin_bit_cast(uint16_t, h);
  } else {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
  }
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Workgroup barrier that orders LDS only (s_waitcnt lgkmcnt(0); s_barrier): unlike
// __syncthreads it does not wait for the global loads and stores in flight, so a barrier
// that follows global stores read only by later kernels (lists, lane states, records,
// page-table arrays) does not pay their round trip.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace bsx
