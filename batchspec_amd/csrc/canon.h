// Deterministic ("canonical") arithmetic of the acceptance and softmax kernels.
//
// Acceptance must give bit-identical token ids on the GPU and on a CPU restatement
// fed the same uniforms.  That requires every floating-point value the decisions
// depend on to be produced by the same sequence of IEEE-754 binary32 operations:
//   * exp is our own: 2^y = ldexp(P(f), n), n = floor(y) saturated to the int32 range,
//     f = fl(y - n) capped at the largest float below 1 (the GPU's v_cvt_flr_i32_f32
//     and v_fract_f32, the latter with its clamp modifier, so that f = 0 for an
//     infinite y), P a degree-4 polynomial with P(0) = 1 fitted to 2^f on [0, 1) for
//     relative error (minimax by linear programming over 20000 points of [0, 1),
//     coefficients rounded to binary32; no last-bit change of them does better),
//     evaluated by Horner with fused multiply-add; relative error at most 3.0e-6 from
//     2^y (P(f) < 2 at the largest f, and P rises with f).  exp2(-inf) = 0 (n = INT_MIN); arguments far below -150 underflow to 0 in
//     ldexp without a clamp.
//   * every sum runs over a fixed tree, independent of the launch configuration:
//       - a row of V values is cut into groups of 8 consecutive elements
//         (group g = elements [8g, 8g+8) ∩ [0, V));
//       - the groups are dealt to NL = 2048 lanes: lane λ = 8t + i owns groups
//         g = t + 256*i + 2048*j for j = 0, 1, ... (t < 256, i < 8);
//       - a group sum adds its elements left to right starting from 0;
//       - a lane sum adds its group sums in increasing j starting from 0;
//       - the row sum is the balanced binary tree over the 2048 lane sums
//         (node = left child + right child).
//   * softmax statistics use the same lanes.  C = log2(e) * (1/T).  A lane keeps its
//     running max m, its sum s and an integer-valued reference r, which starts at
//     R0 = -2^127 (below fl(x·C) of every admissible x).  For each group, with group
//     max gm: r' = max(r, ceil(fl(gm·C))); s = ldexp(s, sat(r - r')) (sat: conversion
//     to int32, saturated; an exact power-of-two rescale, 0 for a lane that has only
//     seen -inf); r = r'; m = max(m, gm); then s += the group sum of the weights
//     2^fma(x, C, -r).
//     The row max M is the max over lanes; the row sum Z is the binary tree over
//     lanes of s_lane·2^(r_lane - rho(M)), rho(M) = fl(M·C) (each lane rescaled
//     exactly once).  Later weights are 2^fma(x, C, -rho(M)).
// Inputs are finite or -inf (a row needs at least one finite logit), with |x * C| below
// 2^31 for finite x: a weight's exponent is at most the rounding error of fl(x * C), so
// below 2^31 every weight stays under 2^64.  Beyond it weights can overflow and a row's
// Z become inf or NaN, the same on the CPU and the GPU.
#pragma once

#include <math.h>
#include <stdint.h>

#ifndef __HIP__
#define BSX_HD inline
#else
#define BSX_HD __host__ __device__ inline __attribute__((always_inline))
#endif

namespace bsx {
namespace canon {

constexpr int kGroup = 8;         // elements per group
constexpr int kThreads = 256;     // t range
constexpr int kLanesPerThread = 8;  // i range
constexpr int kLanes = kThreads * kLanesPerThread;  // 2048
constexpr int kLaneStride = kLanes;                  // groups between consecutive j

constexpr float kLog2e = 0x1.715476p+0f;
constexpr float kC0 = 0x1.0p+0f;
constexpr float kC1 = 0x1.62d6c2p-1f;
constexpr float kC2 = 0x1.ee24b2p-3f;
constexpr float kC3 = 0x1.abf636p-5f;
constexpr float kC4 = 0x1.b7fb26p-7f;

// 2^y = ldexp(P(f), n): returns P(f) and sets n.
BSX_HD float exp2_parts(float y, int* n_out) {
#ifdef __HIP_DEVICE_COMPILE__
  float f;
  asm("v_fract_f32_e64 %0, %1 clamp" : "=v"(f) : "v"(y));
  int n;
  asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(n) : "v"(y));
#else
  float f;
  int n;
  if (y != y) {
    f = 0.0f;
    n = INT32_MAX;
  } else {
    const float fl = floorf(y);
    f = fl == y ? 0.0f : fminf(y - fl, 0x1.fffffep-1f);
    n = fl >= 0x1p31f ? INT32_MAX : (fl < -0x1p31f ? INT32_MIN : (int)fl);
  }
#endif
  float p = kC4;
  p = fmaf(p, f, kC3);
  p = fmaf(p, f, kC2);
  p = fmaf(p, f, kC1);
  p = fmaf(p, f, kC0);
  *n_out = n;
  return p;
}

BSX_HD float exp2(float y) {
  int n;
  const float p = exp2_parts(y, &n);
  return ldexpf(p, n);
}

// Scale C = log2(e) / T.
BSX_HD float scale_for_temperature(float temperature) {
  float inv_t = 1.0f / temperature;
  return kLog2e * inv_t;
}

// Weight of a logit relative to the row max: 2^(fma(x, C, -(M*C))).
BSX_HD float weight(float x, float c, float neg_mc) { return exp2(fmaf(x, c, neg_mc)); }

// Maximum of two non-NaN floats (on the device without the NaN-quieting of fmaxf).
BSX_HD float max_nn(float a, float b) {
#ifdef __HIP_DEVICE_COMPILE__
  return __builtin_elementwise_maximum(a, b);
#else
  return fmaxf(a, b);
#endif
}

// Conversion to int32 toward zero, saturated at the int32 range (-inf: INT32_MIN).
BSX_HD int sat_i32(float v) {
#ifdef __HIP_DEVICE_COMPILE__
  int n;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(n) : "v"(v));
  return n;
#else
  if (v != v) return 0;
  return v <= -0x1p31f ? INT32_MIN : (v >= 0x1p31f ? INT32_MAX : (int)v);
#endif
}

// Start value of a lane's reference: below fl(x*C) of every admissible finite x.
constexpr float kRefStart = -0x1p127f;

// Online lane state: running max m, weight sum s, integer-valued reference r.
struct LaneState {
  float m;
  float s;
  float r;
};

// Reference update for a group with maximum gm: returns the new reference and rescales
// the lane sum by the exact power of two between the two references.
BSX_HD float lane_reference(LaneState& st, float gm, float c) {
  const float r = max_nn(st.r, ceilf(gm * c));
  st.s = ldexpf(st.s, sat_i32(st.r - r));
  st.r = r;
  st.m = max_nn(st.m, gm);
  return r;
}

// Fold one group (n elements, group max gm) into a lane.
BSX_HD void lane_update(LaneState& st, const float* x, int n, float gm, float c) {
  const float r = lane_reference(st, gm, c);
  float gs = 0.f;
  for (int e = 0; e < n; ++e) gs = gs + weight(x[e], c, -r);
  st.s = st.s + gs;
}

// A lane's sum expressed relative to the row max M (rho_m = M*C).
BSX_HD float lane_rescaled(LaneState st, float rho_m) { return st.s * exp2(st.r - rho_m); }

// ---- top-k / top-p filtering and fixed-point draws ----------------------------
// Order-preserving 32-bit image of a finite float (-0 maps like +0).
BSX_HD uint32_t okey(float x) {
  uint32_t b = __builtin_bit_cast(uint32_t, x);
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
BSX_HD float key_value(uint32_t k) {
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// Fixed-point mass of a weight: trunc(w * 2^40) (w * 2^40 is exact), 0 unless w > 0
// (finite w below 2^23).  On the device from a = w * 2^8 with two conversions: the
// integer part floor(a) * 2^32 + trunc(fract(a) * 2^32), both parts exact; on the host
// read off the bits.
BSX_HD uint64_t fx40(float w) {
#ifdef __HIP_DEVICE_COMPILE__
  const float a = fmaxf(w, 0.0f) * 0x1p8f;  // NaN and w <= 0 give 0
  const uint32_t hi = (uint32_t)a;
  const uint32_t lo = (uint32_t)((a - (float)hi) * 0x1p32f);
  return ((uint64_t)hi << 32) | lo;
#else
  if (!(w > 0.0f)) return 0ull;
  const uint32_t b = __builtin_bit_cast(uint32_t, w * 0x1p40f);
  const int e = (int)(b >> 23) - 150;  // value = mant * 2^e
  const uint64_t mant = (uint64_t)((b & 0x7fffffu) | 0x800000u);
  if ((b >> 23) == 0u) return 0ull;    // below 1
  return e >= 0 ? mant << e : (e > -24 ? mant >> -e : 0ull);
#endif
}
// Round-to-nearest-even conversion of a 64-bit integer to binary32.
BSX_HD float u64_to_f32(uint64_t v) {
  if (v < (1ull << 24)) return (float)(uint32_t)v;
  const int n = 64 - __builtin_clzll(v);
  const int sh = n - 24;
  uint64_t mant = v >> sh;
  const uint64_t rem = v & ((1ull << sh) - 1);
  const uint64_t half = 1ull << (sh - 1);
  if (rem > half || (rem == half && (mant & 1))) ++mant;
  return ldexpf((float)(uint32_t)mant, sh);
}
// Draw point of a uniform over a fixed-point total: floor(u * total) in binary64
// (0 for u <= 0 or NaN).
BSX_HD uint64_t draw_point(float u, uint64_t total) {
  if (!(u > 0.0f)) return 0ull;
  return (uint64_t)floor((double)u * (double)total);
}

}  // namespace canon
}  // namespace bsx
