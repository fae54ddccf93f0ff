// RoPE arithmetic shared by the rotation kernels (ivakv_rope.hip) and the FP8 append
// (ivakv_fp8.hip), so every path rotates a pair with the same float operations.
//
// RoPE as the reference's RoPE module defines it (src/core/rope_kv.py:22-50): dims
// (2i, 2i+1) of a head form a pair rotated by angle a = p * f_i at absolute position
// p, with f_i = 1 / theta^(2i / D) (computed in double, stored as float, as the
// reference's float32 buffer holds it) and a = float(p) * f_i in float:
//   y[2i]   = x[2i] cos a - x[2i+1] sin a
//   y[2i+1] = x[2i] sin a + x[2i+1] cos a
// evaluated in fp32 (each as one product rounded, then a fused multiply-add) and rounded
// once to the element type.
#pragma once
#include "ivakv_internal.h"

namespace ivakv {

template <typename E>
__device__ inline float rope_ld(E x) { return (float)x; }

// The products and sums are spelled as explicit fused multiply-adds, so every kernel
// that inlines this rotates a pair to the same float, whatever contraction the compiler
// would otherwise choose in its context.
template <typename E>
__device__ inline void rotate_pair(E& x0, E& x1, float c, float s) {
  const float a = rope_ld(x0), b = rope_ld(x1);
  x0 = (E)__builtin_fmaf(a, c, -(b * s));
  x1 = (E)__builtin_fmaf(a, s, b * c);
}

// f_i = 1 / theta^(2i / D), in double, stored as float.
__device__ inline float inv_freq(int i, int D, float theta) {
  return (float)(1.0 / pow((double)theta, (double)(2 * i) / (double)D));
}

// Each workgroup computes f_i once into LDS (head_dim up to 2 * kFreqTable) instead of
// once per (token, head, pair): the double pow costs more than the row's memory traffic.
// Pairs past the table compute f_i directly, to the same float.
constexpr int kFreqTable = 1024;

// Fills f[0, min(half, kFreqTable)); every thread of the workgroup must call it.
__device__ inline void fill_freqs(float* f, int half, int D, float theta) {
  for (int i = threadIdx.x; i < half && i < kFreqTable; i += blockDim.x) f[i] = inv_freq(i, D, theta);
  __syncthreads();
}

// cos / sin of pair i at position p (accurate library sin / cos of the float angle).
__device__ inline void pair_angle(const float* f, int p, int i, int D, float theta, float& c,
                                  float& s) {
  const float fi = i < kFreqTable ? f[i] : inv_freq(i, D, theta);
  const float ang = (float)p * fi;
  sincosf(ang, &s, &c);
}

}  // namespace ivakv
