// Row access and canonical row statistics shared by the acceptance, softmax and
// sampling-filter kernels (the arithmetic is specified in canon.h).
#pragma once

#include <type_traits>

#include "common.h"
#include "canon.h"

namespace bsx {
namespace acc {

using canon::kGroup;
using canon::kLanes;
using canon::LaneState;

// ----------------------------------------------------------------------------
// Row access: group g of a row of V elements, as fp32 (exact conversion).
// ----------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ int load_group(const void* row, int64_t g, int64_t V, bool vec,
                                          float x[8]) {
  const int64_t v0 = g * kGroup;
  const int n = (int)min((int64_t)kGroup, V - v0);
  if constexpr (DT == BSX_DTYPE_FP32) {
    const float* r = static_cast<const float*>(row) + v0;
    if (vec && n == 8) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(r);
      const f32x4 b = *reinterpret_cast<const f32x4*>(r + 4);
      x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
      x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = e < n ? r[e] : 0.f;
    }
  } else {
    const uint16_t* r = static_cast<const uint16_t*>(row) + v0;
    if (vec && n == 8) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(r);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        x[2 * q] = lo_f32<DT>(w[q]);
        x[2 * q + 1] = hi_f32<DT>(w[q]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = e < n ? half_bits_to_f32<DT>(r[e]) : 0.f;
    }
  }
  return n;
}

template <int DT>
__device__ __forceinline__ float load_one(const void* row, int64_t v) {
  if constexpr (DT == BSX_DTYPE_FP32) return static_cast<const float*>(row)[v];
  else return half_bits_to_f32<DT>(static_cast<const uint16_t*>(row)[v]);
}

// ----------------------------------------------------------------------------
// Row statistics (M, Z): online lane states, one rescale per lane to the row max,
// then the canonical binary tree over lanes.  One 256-thread workgroup per row;
// thread t owns lanes 8t+i (its groups t + 256*c, lane i = c mod 8).
// ----------------------------------------------------------------------------
// With LANES, lane_max[i] receives the maximum of lane 8t+i (-inf for a lane without
// groups).  A Hook observes the pass without changing the statistics:
// hook->round(c0, gm) in each whole round (groups t + 256*(c0 + i), i < 8, gm[i]
// their maxima), hook->group(g, x, n, gm) for each group of the remaining partial
// rounds (x its n elements), and, when hook->wants_first() (same value in every
// thread) and every thread has a whole first round, hook->first(gm) before that
// round's hook->round (called by every thread; the first round runs outside the loop).
struct NoRowHook {};

template <int DT, bool LANES = false, typename Hook = NoRowHook>
__device__ void row_stats(const void* row, int64_t V, bool vec, float c, float* out_m,
                          float* out_z, float* lane_max = nullptr, Hook* hook = nullptr) {
  constexpr bool HOOKED = !std::is_same<Hook, NoRowHook>::value;
  __shared__ float wave_val[4];
  const int t = threadIdx.x;
  const int64_t G = ceil_div(V, kGroup);
  LaneState st[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    st[i].m = -INFINITY;
    st[i].s = 0.f;
    st[i].r = canon::kRefStart;
  }
  int64_t c0 = 0;
  if (vec) {
    // Whole rounds: the 8 groups t + 256*(c0 + i), i < 8, all exist and are complete.
    // Their loads go out together; then each lane's reference update (branch-free: an
    // exact power-of-two rescale) and its weights, in the canonical order.
    const int64_t G_whole = V / kGroup;
    constexpr int VW = DT == BSX_DTYPE_FP32 ? 2 : 1;
    // Buffer loads: the row's base in a descriptor, the thread's offset in a register and
    // the group's offset in a scalar register, so no vector instruction computes an
    // address (and a load past the row's bytes returns 0).
    const __amdgpu_buffer_rsrc_t rsrc = row_rsrc(row, V * (int64_t)(VW == 2 ? 4 : 2));
    auto whole_round = [&](int64_t c0, auto first_tag) {
      constexpr bool FIRST = decltype(first_tag)::value;
      u32x4 w[8][VW];
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int h = 0; h < VW; ++h)
          w[i][h] = load_nt_b128(rsrc, (t * VW + h) * 16, (int)(c0 + i) * 4096 * VW);
      float x[8][8], gm[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (DT == BSX_DTYPE_FP32) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            x[i][q] = __uint_as_float(w[i][0][q]);
            x[i][4 + q] = __uint_as_float(w[i][1][q]);
          }
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            x[i][2 * q] = lo_f32<DT>(w[i][0][q]);
            x[i][2 * q + 1] = hi_f32<DT>(w[i][0][q]);
          }
        }
        gm[i] = __builtin_elementwise_maximum(
            __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[i][0], x[i][1]),
                                          __builtin_elementwise_maximum(x[i][2], x[i][3])),
            __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[i][4], x[i][5]),
                                          __builtin_elementwise_maximum(x[i][6], x[i][7])));
      }
      if constexpr (HOOKED) {
        if constexpr (FIRST) hook->first(gm);
        hook->round(c0, gm);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float r = canon::lane_reference(st[i], gm[i], c);
        // = 0 + w0 + ... exactly: weights are >= +0
        float gs = canon::weight(x[i][0], c, -r);
#pragma unroll
        for (int e = 1; e < 8; ++e) gs = gs + canon::weight(x[i][e], c, -r);
        st[i].s = st[i].s + gs;
      }
    };
    if constexpr (HOOKED) {
      // The first round on its own when every thread has one and the hook wants it
      // (hook->first(gm) is called by every thread, outside the loop).
      if (255 + 256 * 7 < G_whole && hook->wants_first()) {
        whole_round(0, std::true_type());
        c0 = 8;
      }
    }
    for (; (int64_t)t + 256 * (c0 + 7) < G_whole; c0 += 8) whole_round(c0, std::false_type());
  }
  for (; (int64_t)t + 256 * c0 < G; c0 += 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t g = (int64_t)t + 256 * (c0 + i);
      if (g < G) {
        float x[8];
        const int n = load_group<DT>(row, g, V, vec, x);
        float gm = x[0];
#pragma unroll
        for (int e = 1; e < 8; ++e)
          if (e < n) gm = fmaxf(gm, x[e]);
        if (n == 8) {
          canon::lane_update(st[i], x, 8, gm, c);
        } else {
          canon::lane_update(st[i], x, n, gm, c);
        }
        if constexpr (HOOKED) hook->group(g, x, n, gm);
      }
    }
  }
  if constexpr (LANES) {
#pragma unroll
    for (int i = 0; i < 8; ++i) lane_max[i] = st[i].m;
  }
  // row max (order-free)
  float mx = st[0].m;
#pragma unroll
  for (int i = 1; i < 8; ++i) mx = fmaxf(mx, st[i].m);
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) mx = fmaxf(mx, __shfl_xor(mx, m));
  if ((t & 63) == 0) wave_val[t >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wave_val[0], wave_val[1]), fmaxf(wave_val[2], wave_val[3]));
  __syncthreads();
  const float rho_m = mx * c;
  // lanes 8t+i rescaled once, then the tree over i, over t in the wave, over waves
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = canon::lane_rescaled(st[i], rho_m);
  float s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) s = s + __shfl_xor(s, m);
  if ((t & 63) == 0) wave_val[t >> 6] = s;
  __syncthreads();
  if (t == 0) {
    *out_m = mx;
    *out_z = (wave_val[0] + wave_val[1]) + (wave_val[2] + wave_val[3]);
  }
  __syncthreads();
}

}  // namespace acc
}  // namespace bsx
