// Ceiling kernels for bench.py --workload ceiling (measurement only: not
// part of libivakv's C ABI).  The two read kernels read HBM and write one 16-byte word
// per wave, so the traffic is the bytes read; the MFMA kernel reads nothing.
//
//   ceiling_stream_read: the buffer read front to back, 16 bytes per lane per load, a
//     grid-stride loop with four loads in flight per lane.
//   ceiling_tile_read: the access pattern of the decode walk without its arithmetic:
//     n_tiles tiles of tile_bytes (4096 = one 16-row K or V page of one kv head at
//     head_dim 128, fp16) at the offsets idx[i] * tile_bytes, dealt in equal contiguous
//     shares to a grid of 4-wave workgroups, one tile in flight per wave (the bytes in
//     flight per CU are set by the workgroups per CU).
//   ceiling_mfma_f16: dense fp16 16x16x32 MFMA throughput (the prefill's instruction)
//     on random operands, with no memory traffic in the loop.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void ceiling_stream_read(const u32x4* __restrict__ src,
                                                           int64_t n_vec, u32x4* sink) {
  u32x4 acc = {0, 0, 0, 0};
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n_vec; i += 4 * stride) {
    const u32x4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n_vec; i += stride) acc ^= src[i];
  // one word per wave keeps the loads live
  for (int off = 32; off > 0; off >>= 1) {
    acc.x ^= __shfl_xor(acc.x, off);
    acc.y ^= __shfl_xor(acc.y, off);
    acc.z ^= __shfl_xor(acc.z, off);
    acc.w ^= __shfl_xor(acc.w, off);
  }
  if ((threadIdx.x & 63) == 0) sink[(blockIdx.x * blockDim.x + threadIdx.x) >> 6] = acc;
}

template <int PER_LANE>
__global__ __launch_bounds__(256) void ceiling_tile_read(const u32x4* __restrict__ src,
                                                         const int32_t* __restrict__ idx,
                                                         int64_t n_tiles, u32x4* sink) {
  constexpr int tile_vec = 64 * PER_LANE;  // 16-byte words per tile
  const int lane = threadIdx.x & 63;
  // wave-uniform index (readfirstlane), so the tile ids are read through the scalar cache
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) +
                       __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
  const int64_t t0 = wave * n_tiles / waves, t1 = (wave + 1) * n_tiles / waves;
  u32x4 acc = {0, 0, 0, 0};
  // One tile in flight per wave: the bytes in flight come from the waves per CU.
  for (int64_t t = t0; t < t1; ++t) {
    const u32x4* p = src + (int64_t)idx[t] * tile_vec + lane;
    u32x4 v[PER_LANE];
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) v[j] = p[64 * j];
#pragma unroll
    for (int j = 0; j < PER_LANE; ++j) acc ^= v[j];
  }
  for (int off = 32; off > 0; off >>= 1) {
    acc.x ^= __shfl_xor(acc.x, off);
    acc.y ^= __shfl_xor(acc.y, off);
    acc.z ^= __shfl_xor(acc.z, off);
    acc.w ^= __shfl_xor(acc.w, off);
  }
  if (lane == 0) sink[wave] = acc;
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Dense fp16 MFMA throughput: every wave runs `iters` rounds of kChains independent
// 16x16x32 accumulations (no loads in the loop), so nothing but the matrix cores and
// the clock bounds it.  The four operand vectors of each wave are read once from
// `ops` (random fp16 values, 1024 waves' worth): operands that toggle as many bits as
// real data draw the power, and so set the clock, that real data does.
constexpr int kChains = 8;
__global__ __launch_bounds__(256, 2) void ceiling_mfma_f16(int iters, const f16x8* __restrict__ ops,
                                                           f32x4* sink) {
  const int lane = threadIdx.x & 63;
  const int w = (blockIdx.x * 4 + (threadIdx.x >> 6)) & 1023;
  const f16x8 a0 = ops[(w * 4 + 0) * 64 + lane], b0 = ops[(w * 4 + 1) * 64 + lane];
  const f16x8 a1 = ops[(w * 4 + 2) * 64 + lane], b1 = ops[(w * 4 + 3) * 64 + lane];
  f32x4 acc[kChains];
#pragma unroll
  for (int k = 0; k < kChains; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < kChains; ++k)
      acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16((k & 1) ? a1 : a0, (k & 2) ? b1 : b0, acc[k], 0, 0, 0);
  }
  f32x4 s = acc[0];
#pragma unroll
  for (int k = 1; k < kChains; ++k) s += acc[k];
  if (lane == 0) sink[(blockIdx.x * blockDim.x + threadIdx.x) >> 6] = s;
}

}  // namespace

// Runs grid workgroups of 4 waves, each wave iters x 8 MFMAs of 16x16x32 (16,384 FLOP
// each) on operands read from ops (1024 * 4 * 64 vectors of 8 fp16, 4 MiB); sink holds
// one 16-byte word per wave (grid * 4 words).  Returns the HIP error code of the launch.
extern "C" int ceiling_mfma(int iters, const void* ops, void* sink, int grid, hipStream_t stream) {
  ceiling_mfma_f16<<<grid, 256, 0, stream>>>(iters, static_cast<const f16x8*>(ops),
                                             static_cast<f32x4*>(sink));
  return (int)hipGetLastError();
}

// Reads n_bytes (a multiple of 16) of src; sink holds one 16-byte word per wave of the
// grid (grid * 4 words).  Returns the HIP error code of the launch.
extern "C" int ceiling_stream(const void* src, int64_t n_bytes, void* sink, int grid,
                              hipStream_t stream) {
  ceiling_stream_read<<<grid, 256, 0, stream>>>(static_cast<const u32x4*>(src), n_bytes / 16,
                                                static_cast<u32x4*>(sink));
  return (int)hipGetLastError();
}

// Reads tiles idx[0..n_tiles) of tile_bytes (4096, or 8192 = a K + V pair's bytes) each
// from src, one tile in flight per wave of a grid of `grid` 4-wave workgroups; sink holds
// one 16-byte word per wave (grid * 4 words).  Returns -1 for another tile size, else
// the HIP error code of the launch.
extern "C" int ceiling_tiles(const void* src, const int32_t* idx, int64_t n_tiles,
                             int tile_bytes, void* sink, int grid, hipStream_t stream) {
  const u32x4* s = static_cast<const u32x4*>(src);
  u32x4* k = static_cast<u32x4*>(sink);
  if (tile_bytes == 4096) ceiling_tile_read<4><<<grid, 256, 0, stream>>>(s, idx, n_tiles, k);
  else if (tile_bytes == 8192) ceiling_tile_read<8><<<grid, 256, 0, stream>>>(s, idx, n_tiles, k);
  else return -1;
  return (int)hipGetLastError();
}
