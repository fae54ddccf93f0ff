// Ceiling kernels for bench.py --workload ceiling (measurement only: not
// part of libivakv's C ABI).  The two read kernels read HBM and write one 16-byte word
// per wave, so the traffic is the bytes read; the MFMA kernel reads nothing.
//
//   ceiling_stream_read<U, NT>: each wave streams its own contiguous share of the
//     buffer front to back, U 16-byte loads per lane per slot (U KiB per wave), two
//     slots in flight (the next slot's loads are issued before the current one is
//     consumed), so 2U KiB stay in flight per wave without a bubble.  NT: the loads
//     carry the non-temporal hint (read-once data).
//   ceiling_tile_read<PER_LANE, RING, NT>: the access pattern of the decode walk without
//     its arithmetic: n_tiles tiles of 1024 * PER_LANE bytes (4096 = one 16-row K or V
//     page of one kv head at head_dim 128, fp16) at the offsets idx[i] * tile_bytes,
//     dealt in equal contiguous shares to the waves, RING tiles in flight per wave
//     (RING 4 of 4 KiB = the walk's two ring slots of K + V, 16 KiB).
//   ceiling_mfma_f16: dense fp16 16x16x32 MFMA throughput (the prefill's instruction)
//     on random operands, with no memory traffic in the loop.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ inline u32x4 load16(const u32x4* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}

// XOR-folds acc over the wave and stores one word (keeps every load live).
__device__ inline void sink_wave(u32x4 acc, u32x4* sink, int64_t wave) {
  for (int off = 32; off > 0; off >>= 1) {
    acc.x ^= __shfl_xor(acc.x, off);
    acc.y ^= __shfl_xor(acc.y, off);
    acc.z ^= __shfl_xor(acc.z, off);
    acc.w ^= __shfl_xor(acc.w, off);
  }
  if ((threadIdx.x & 63) == 0) sink[wave] = acc;
}

__device__ inline int64_t wave_id() {
  return (int64_t)blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

template <int U, bool NT>
__global__ __launch_bounds__(256) void ceiling_stream_read(const u32x4* __restrict__ src,
                                                           int64_t n_vec, u32x4* sink) {
  constexpr int64_t kSlot = 64 * U;  // 16-byte words of one slot
  const int lane = threadIdx.x & 63;
  const int64_t wave = wave_id();
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
  const int64_t slots = n_vec / kSlot;
  const int64_t s0 = wave * slots / waves, s1 = (wave + 1) * slots / waves;
  u32x4 acc = {0, 0, 0, 0};
  if (s0 < s1) {
    u32x4 a[U], b[U];
    const u32x4* base = src + lane;
#pragma unroll
    for (int j = 0; j < U; ++j) a[j] = load16<NT>(base + s0 * kSlot + 64 * j);
    // Slot s is in a, s + 1 in b; past the share the last slot is re-read (an L2
    // hit), so the loop has no branch that would drain the loads in flight.
    for (int64_t s = s0; s < s1; s += 2) {
      const int64_t sb = s + 1 < s1 ? s + 1 : s1 - 1;
#pragma unroll
      for (int j = 0; j < U; ++j) b[j] = load16<NT>(base + sb * kSlot + 64 * j);
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < U; ++j) acc ^= a[j];
      const int64_t sa = s + 2 < s1 ? s + 2 : s1 - 1;
#pragma unroll
      for (int j = 0; j < U; ++j) a[j] = load16<NT>(base + sa * kSlot + 64 * j);
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < U; ++j) acc ^= b[j];
    }
  }
  sink_wave(acc, sink, wave);
}

template <int PER_LANE, int RING, bool NT>
__global__ __launch_bounds__(256) void ceiling_tile_read(const u32x4* __restrict__ src,
                                                         const int32_t* __restrict__ idx,
                                                         int64_t n_tiles, u32x4* sink) {
  constexpr int64_t kTileVec = 64 * PER_LANE;  // 16-byte words per tile
  const int lane = threadIdx.x & 63;
  const int64_t wave = wave_id();
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x >> 6);
  const int64_t t0 = wave * n_tiles / waves, t1 = (wave + 1) * n_tiles / waves;
  u32x4 acc = {0, 0, 0, 0};
  if (t0 < t1) {
    u32x4 v[RING][PER_LANE];
    auto load = [&](int r, int64_t t) __attribute__((always_inline)) {
      const u32x4* p = src + (int64_t)idx[t < t1 ? t : t1 - 1] * kTileVec + lane;
#pragma unroll
      for (int j = 0; j < PER_LANE; ++j) v[r][j] = load16<NT>(p + 64 * j);
      __asm__ volatile("" ::: "memory");
    };
#pragma unroll
    for (int r = 0; r < RING; ++r) load(r, t0 + r);
    // Tile t sits in slot (t - t0) % RING; consuming it frees the slot for tile t + RING.
    for (int64_t t = t0; t < t1; t += RING) {
#pragma unroll
      for (int r = 0; r < RING; ++r) {
#pragma unroll
        for (int j = 0; j < PER_LANE; ++j) acc ^= v[r][j];
        load(r, t + RING + r);
      }
    }
  }
  sink_wave(acc, sink, wave);
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

template <int U, bool NT>
void launch_stream(const void* src, int64_t n_bytes, void* sink, int grid, hipStream_t stream) {
  ceiling_stream_read<U, NT><<<grid, 256, 0, stream>>>(static_cast<const u32x4*>(src), n_bytes / 16,
                                                       static_cast<u32x4*>(sink));
}

template <int RING, bool NT>
void launch_tiles(const void* src, const int32_t* idx, int64_t n_tiles, int tile_bytes, void* sink,
                  int grid, hipStream_t stream) {
  const u32x4* s = static_cast<const u32x4*>(src);
  u32x4* k = static_cast<u32x4*>(sink);
  if (tile_bytes == 4096) ceiling_tile_read<4, RING, NT><<<grid, 256, 0, stream>>>(s, idx, n_tiles, k);
  else ceiling_tile_read<8, RING, NT><<<grid, 256, 0, stream>>>(s, idx, n_tiles, k);
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

// Reads n_bytes (a multiple of 16 * 64 * per_lane) of src, each wave a contiguous share,
// per_lane (4 or 8) 16-byte loads per lane per slot, two slots in flight, with the
// non-temporal hint when nt != 0; sink holds one 16-byte word per wave of the grid
// (grid * 4 words).  Returns -1 for another per_lane, else the HIP error code.
extern "C" int ceiling_stream(const void* src, int64_t n_bytes, void* sink, int grid, int per_lane,
                              int nt, hipStream_t stream) {
  if (per_lane == 4) {
    if (nt) launch_stream<4, true>(src, n_bytes, sink, grid, stream);
    else launch_stream<4, false>(src, n_bytes, sink, grid, stream);
  } else if (per_lane == 8) {
    if (nt) launch_stream<8, true>(src, n_bytes, sink, grid, stream);
    else launch_stream<8, false>(src, n_bytes, sink, grid, stream);
  } else {
    return -1;
  }
  return (int)hipGetLastError();
}

// Reads tiles idx[0..n_tiles) of tile_bytes (4096, or 8192 = a K + V pair's bytes) each
// from src, ring (1, 2 or 4) tiles in flight per wave of a grid of `grid` 4-wave
// workgroups, with the non-temporal hint when nt != 0; sink holds one 16-byte word per
// wave (grid * 4 words).  Returns -1 for another tile size or ring, else the HIP error
// code of the launch.
extern "C" int ceiling_tiles(const void* src, const int32_t* idx, int64_t n_tiles, int tile_bytes,
                             int ring, int nt, void* sink, int grid, hipStream_t stream) {
  if (tile_bytes != 4096 && tile_bytes != 8192) return -1;
  switch (ring * 2 + (nt ? 1 : 0)) {
    case 2: launch_tiles<1, false>(src, idx, n_tiles, tile_bytes, sink, grid, stream); break;
    case 3: launch_tiles<1, true>(src, idx, n_tiles, tile_bytes, sink, grid, stream); break;
    case 4: launch_tiles<2, false>(src, idx, n_tiles, tile_bytes, sink, grid, stream); break;
    case 5: launch_tiles<2, true>(src, idx, n_tiles, tile_bytes, sink, grid, stream); break;
    case 8: launch_tiles<4, false>(src, idx, n_tiles, tile_bytes, sink, grid, stream); break;
    case 9: launch_tiles<4, true>(src, idx, n_tiles, tile_bytes, sink, grid, stream); break;
    default: return -1;
  }
  return (int)hipGetLastError();
}
