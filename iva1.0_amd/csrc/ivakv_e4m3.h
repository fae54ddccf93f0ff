// OCP e4m3fn codes for FP8 KV pages: conversion in integer arithmetic (round to
// nearest even, saturating at +-448, so the codes do not depend on a hardware rounding
// mode) and the per-row scaling factor, shared by the FP8 append / gather kernels and
// the fused FP8 decode merge.
#pragma once
#include "ivakv_internal.h"

namespace ivakv {

constexpr float kFp8Max = 448.f;

// float -> e4m3fn code, round to nearest even, saturating at +-448 (NaN -> 0x7F).
// Both ranges are computed and one is selected (no branch: a divergent branch per code
// costs more than the arithmetic of the path not taken).
__device__ inline uint32_t e4m3_encode(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t au = u & 0x7fffffffu;
  const float a = __uint_as_float(au);
  // below 2^-6: subnormal grid step 2^-9, codes 0..8 (8 = smallest normal)
  const uint32_t sub = (uint32_t)__builtin_rintf(fminf(a, 0.015625f) * 512.f);
  // from 2^-6 on: keep 3 mantissa bits with round-to-nearest-even on the float's own
  // bits, then rebias the exponent from 127 to 7 (saturating at 0x7E = 448)
  const uint32_t r = (au + 0x7FFFFu + ((au >> 20) & 1u)) >> 20;
  const uint32_t nrm = r >= (127u - 7u) * 8u + 0x7Fu ? 0x7Eu : r - (127u - 7u) * 8u;
  uint32_t code = a < 0.015625f ? sub : nrm;
  code = code > 0x7Eu ? 0x7Eu : code;
  code = au > 0x7f800000u ? 0x7Fu : code;  // NaN
  return sign | code;
}

// e4m3fn code -> float, exactly.
__device__ inline float e4m3_decode(uint32_t b) {
  const uint32_t e = (b >> 3) & 0xFu, m = b & 7u;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;                       // m * 2^-9
  else if (e == 15 && m == 7) v = __uint_as_float(0x7fc00000u);  // NaN
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -v : v;
}

// max(a, b) that keeps a NaN (fmaxf drops it): a row holding a NaN has a NaN max |x|.
__device__ inline float nan_max(float a, float b) { return (a > b || a != a) ? a : b; }

// Scaling factor of a row with max |x| = amax, the reference's rule
// (src/quant/fp8_runtime.py:67-76): 1 for amax == 0, else 448 / amax clamped to
// [1e-8, 1e8] as max(1e-8, min(sf, 1e8)) evaluates in Python, so a NaN amax gives 1e-8
// (and an infinite one 448 / inf = 0, also 1e-8).
__device__ inline float row_sf(float amax) {
  if (amax == 0.f) return 1.f;
  const float sf = kFp8Max / amax;
  return sf != sf ? 1e-8f : fminf(fmaxf(sf, 1e-8f), 1e8f);
}

}  // namespace ivakv
