// Rotary position embedding fused into the paged append, rotation of query rows in
// place, and page moves for pool compaction, on gfx950.  The rotation itself (RoPE of
// src/core/rope_kv.py:22-50) is in ivakv_rope.h; the FP8 pools' fused append is in
// ivakv_fp8.hip.
#include "ivakv_rope.h"

namespace ivakv {
namespace {

constexpr int64_t kMaxGridR = 0x7fffffff;

struct alignas(16) Chunk16 {
  uint32_t w[4];
};

// x [n_tok][H][D] with element strides (token, head), rotated in place at positions[t].
// One thread per (token, head, pair).
template <typename E>
__global__ __launch_bounds__(256) void rope_kernel(E* x, int64_t ts, int64_t hs,
                                                   const int32_t* pos, int n_tok, int H, int D,
                                                   float theta) {
  __shared__ float s_freq[kFreqTable];
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int half = D / 2;
  fill_freqs(s_freq, half, D, theta);
  if (gid >= (int64_t)n_tok * H * half) return;
  const int i = (int)(gid % half);
  const int64_t th = gid / half;
  const int h = (int)(th % H);
  const int64_t t = th / H;
  float c, s;
  pair_angle(s_freq, pos[t], i, D, theta, c, s);
  E* row = x + t * ts + h * hs;
  rotate_pair(row[2 * i], row[2 * i + 1], c, s);
}

// Paged append with K rotated: one thread per (token, group of up to eight kv heads,
// 16-byte chunk), the chunk's pairs rotated before the store.  Sources and pools that
// allow it (16-byte aligned rows) move whole 16-byte chunks (VEC), whose loads and K
// stores carry the non-temporal hint (8192 rows: 15.6 µs against 19.2 µs without).
struct AppendRopeArgs {
  const void* k_new;
  const void* v_new;
  int64_t kts, khs, vts, vhs;
  void* k_pool;
  void* v_pool;
  const int32_t* slots;
  const int32_t* pos;
  int n_tok, Hkv, D, bs;
  int64_t n_slots;
  float theta;
};

// Lanes rotate up to kRopeHeads kv heads of one (token, chunk): cos / sin depend on the
// position and the pair only, so they are computed once per lane, not once per head.
// Few rows (decode steps, short chunks) take one head per lane in 64-thread
// workgroups (HEADS = 1), spreading the stores over many CUs, as ivakv_append does.
constexpr int kRopeHeads = 8;
constexpr int64_t kFewRopeThreads = 1024 * 64;  // below 1024 waves: one head per lane

template <typename E, bool VEC, int HEADS>
__global__ __launch_bounds__(256) void append_rope_kernel(AppendRopeArgs a) {
  constexpr int X = 16 / sizeof(E);
  const int nch = a.D / X;
  const int ngrp = cdiv(a.Hkv, HEADS);
  // Thread order (token % 16, chunk, head group, token / 16), as in append_kernel: 16
  // consecutive tokens (consecutive slots of a page in a chunk append) per lane group,
  // so K and V stores coalesce; workgroups in XCD-contiguous order, as append_vec_kernel.
  __shared__ float s_freq[kFreqTable];
  fill_freqs(s_freq, a.D / 2, a.D, a.theta);
  const int64_t gid = xcd_contiguous_block(blockIdx.x, gridDim.x) * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)cdiv(a.n_tok, 16) * 16 * ngrp * nch) return;
  const int t_lo = (int)(gid & 15);
  const int64_t g1 = gid >> 4;
  const int c = (int)(g1 % nch);
  const int64_t g2 = g1 / nch;
  const int h0 = (int)(g2 % ngrp) * HEADS;
  const int64_t t = (g2 / ngrp) * 16 + t_lo;
  if (t >= a.n_tok) return;
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.n_slots) return;
  const int64_t page = slot / a.bs;
  const int off = (int)(slot - page * a.bs);
  const int nh = min(HEADS, a.Hkv - h0);
  const E* __restrict__ kb = static_cast<const E*>(a.k_new) + t * a.kts + (int64_t)c * X;
  const E* __restrict__ vb = static_cast<const E*>(a.v_new) + t * a.vts + (int64_t)c * X;
  E* __restrict__ kp = static_cast<E*>(a.k_pool);
  E* __restrict__ vp = static_cast<E*>(a.v_pool);
  union Row {
    Chunk16 c;
    E e[X];
  };
  E k[HEADS][X], v[HEADS][X];
#pragma unroll
  for (int u = 0; u < HEADS; ++u) {
    if (u < nh) {
      if constexpr (VEC) {  // 16-byte source chunks
        Row rk, rv;
        rk.c = ld<true, Chunk16>(kb + (h0 + u) * a.khs);
        rv.c = ld<true, Chunk16>(vb + (h0 + u) * a.vhs);
#pragma unroll
        for (int j = 0; j < X; ++j) {
          k[u][j] = rk.e[j];
          v[u][j] = rv.e[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < X; ++j) {
          k[u][j] = kb[(h0 + u) * a.khs + j];
          v[u][j] = vb[(h0 + u) * a.vhs + j];
        }
      }
    }
  }
  const int p = a.pos[t];
  float cs[X / 2], sn[X / 2];
#pragma unroll
  for (int j = 0; j < X / 2; ++j) pair_angle(s_freq, p, c * (X / 2) + j, a.D, a.theta, cs[j], sn[j]);
#pragma unroll
  for (int u = 0; u < HEADS; ++u) {
    if (u < nh) {
#pragma unroll
      for (int j = 0; j < X / 2; ++j) rotate_pair(k[u][2 * j], k[u][2 * j + 1], cs[j], sn[j]);
      const int64_t head_base = page * a.Hkv + h0 + u;
      E* kd = kp + ((head_base * nch + c) * a.bs + off) * X;
      E* vd = vp + head_base * a.D * a.bs + (int64_t)c * X * a.bs + off;
      if constexpr (VEC) {
        Row rk;
#pragma unroll
        for (int j = 0; j < X; ++j) rk.e[j] = k[u][j];
        st<true, Chunk16>(kd, rk.c);
      } else {
#pragma unroll
        for (int j = 0; j < X; ++j) kd[j] = k[u][j];
      }
#pragma unroll
      for (int j = 0; j < X; ++j) vd[(int64_t)j * a.bs] = v[u][j];
    }
  }
}

// Page moves: page src[i] -> dst[i] of every pool tensor (K and V tiles of all kv
// heads, and the FP8 scaling factors when given).  Grid (chunk block, move), 16
// bytes per thread.  A move whose source or destination id lies outside
// [0, num_pages) is skipped.  Reads and writes carry the non-temporal hint (4096 moves:
// 82 µs against 89 µs without).
__global__ __launch_bounds__(256) void copy_pages_kernel(Chunk16* k, Chunk16* v, Chunk16* ks,
                                                         Chunk16* vs, const int32_t* src,
                                                         const int32_t* dst, int num_pages,
                                                         int64_t page_chunks,
                                                         int64_t scale_chunks) {
  const int64_t s = src[blockIdx.y], d = dst[blockIdx.y];
  if (s < 0 || s >= num_pages || d < 0 || d >= num_pages) return;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < page_chunks;
       i += (int64_t)gridDim.x * blockDim.x) {
    st<true, Chunk16>(k + d * page_chunks + i, ld<true, Chunk16>(k + s * page_chunks + i));
    st<true, Chunk16>(v + d * page_chunks + i, ld<true, Chunk16>(v + s * page_chunks + i));
    if (ks && i < scale_chunks) {
      st<true, Chunk16>(ks + d * scale_chunks + i, ld<true, Chunk16>(ks + s * scale_chunks + i));
      st<true, Chunk16>(vs + d * scale_chunks + i, ld<true, Chunk16>(vs + s * scale_chunks + i));
    }
  }
}

}  // namespace
}  // namespace ivakv

using namespace ivakv;

extern "C" int ivakv_rope(void* x, int64_t tok_stride, int64_t head_stride,
                          const int32_t* positions, int n_tok, int num_heads, int head_dim,
                          float theta, int dtype, hipStream_t stream) {
  static const char* name = "ivakv_rope";
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (n_tok < 0 || num_heads <= 0 || head_dim <= 0 || head_dim % 2)
    return fail(IVAKV_E_ARG, "%s: bad sizes n_tok=%d H=%d D=%d (D must be even)", name, n_tok,
                num_heads, head_dim);
  if (!(theta > 0.f)) return fail(IVAKV_E_ARG, "%s: theta must be positive", name);
  if (n_tok == 0) return IVAKV_OK;
  if (!x || !positions) return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (tok_stride < 0 || head_stride < 0) return fail(IVAKV_E_ARG, "%s: negative stride", name);
  const int64_t total = (int64_t)n_tok * num_heads * (head_dim / 2);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > kMaxGridR) return fail(IVAKV_E_SHAPE, "%s: too many rows", name);
  switch (dtype) {
    case IVAKV_F16:
      rope_kernel<_Float16><<<(unsigned)blocks, 256, 0, stream>>>(
          static_cast<_Float16*>(x), tok_stride, head_stride, positions, n_tok, num_heads, head_dim, theta);
      break;
    case IVAKV_BF16:
      rope_kernel<__bf16><<<(unsigned)blocks, 256, 0, stream>>>(
          static_cast<__bf16*>(x), tok_stride, head_stride, positions, n_tok, num_heads, head_dim, theta);
      break;
    default:
      rope_kernel<float><<<(unsigned)blocks, 256, 0, stream>>>(
          static_cast<float*>(x), tok_stride, head_stride, positions, n_tok, num_heads, head_dim, theta);
      break;
  }
  return launch_status(name);
}

extern "C" int ivakv_append_rope(const void* k_new, const void* v_new, int64_t k_tok_stride,
                                 int64_t k_head_stride, int64_t v_tok_stride,
                                 int64_t v_head_stride, void* k_pool, void* v_pool,
                                 const int32_t* slot_mapping, const int32_t* positions, int n_tok,
                                 int num_kv_heads, int head_dim, int block_size, int num_pages,
                                 float theta, int dtype, hipStream_t stream) {
  static const char* name = "ivakv_append_rope";
  const int es = dtype_size(dtype);
  if (es == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (n_tok < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_pages < 0)
    return fail(IVAKV_E_ARG, "%s: bad sizes n_tok=%d Hkv=%d D=%d block_size=%d num_pages=%d",
                name, n_tok, num_kv_heads, head_dim, block_size, num_pages);
  const int X = 16 / es;
  if (head_dim % X != 0)
    return fail(IVAKV_E_SHAPE, "%s: head_dim %d must be a multiple of %d", name, head_dim, X);
  if (!(theta > 0.f)) return fail(IVAKV_E_ARG, "%s: theta must be positive", name);
  if (n_tok == 0) return IVAKV_OK;
  if (!k_new || !v_new || !k_pool || !v_pool || !slot_mapping || !positions)
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (k_tok_stride < 0 || k_head_stride < 0 || v_tok_stride < 0 || v_head_stride < 0)
    return fail(IVAKV_E_ARG, "%s: negative stride", name);
  AppendRopeArgs a{k_new, v_new, k_tok_stride, k_head_stride, v_tok_stride, v_head_stride,
                   k_pool, v_pool, slot_mapping, positions, n_tok, num_kv_heads, head_dim,
                   block_size, (int64_t)num_pages * block_size, theta};
  const int64_t lanes = (int64_t)cdiv(n_tok, 16) * 16 * (head_dim / X);  // per head group
  const bool few = lanes * cdiv(num_kv_heads, kRopeHeads) < kFewRopeThreads;
  const int64_t total = lanes * (few ? num_kv_heads : cdiv(num_kv_heads, kRopeHeads));
  const int threads = few ? 64 : 256;
  const int64_t blocks = (total + threads - 1) / threads;
  if (blocks > kMaxGridR) return fail(IVAKV_E_SHAPE, "%s: too many rows", name);
  // 16-byte K / V chunk accesses when every source row and the pools allow them
  const bool vec = aligned16(k_new) && aligned16(v_new) && aligned16(k_pool) && aligned16(v_pool) &&
                   (k_tok_stride % X == 0) && (k_head_stride % X == 0) &&
                   (v_tok_stride % X == 0) && (v_head_stride % X == 0);
  const unsigned g = (unsigned)blocks;
#define IVAKV_APPEND_ROPE(E)                                                                     \
  if (few) {                                                                                     \
    if (vec) append_rope_kernel<E, true, 1><<<g, threads, 0, stream>>>(a);                       \
    else append_rope_kernel<E, false, 1><<<g, threads, 0, stream>>>(a);                          \
  } else {                                                                                       \
    if (vec) append_rope_kernel<E, true, kRopeHeads><<<g, threads, 0, stream>>>(a);              \
    else append_rope_kernel<E, false, kRopeHeads><<<g, threads, 0, stream>>>(a);                 \
  }
  switch (dtype) {
    case IVAKV_F16: IVAKV_APPEND_ROPE(_Float16); break;
    case IVAKV_BF16: IVAKV_APPEND_ROPE(__bf16); break;
    default: IVAKV_APPEND_ROPE(float); break;
  }
#undef IVAKV_APPEND_ROPE
  return launch_status(name);
}

extern "C" int ivakv_copy_pages(void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                                const int32_t* src_pages, const int32_t* dst_pages, int n_moves,
                                int num_pages, int num_kv_heads, int head_dim, int block_size,
                                int elem_bytes, hipStream_t stream) {
  static const char* name = "ivakv_copy_pages";
  if (n_moves < 0 || num_pages < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4))
    return fail(IVAKV_E_ARG,
                "%s: bad sizes moves=%d pages=%d Hkv=%d D=%d block_size=%d elem_bytes=%d", name,
                n_moves, num_pages, num_kv_heads, head_dim, block_size, elem_bytes);
  const int64_t page_bytes = (int64_t)num_kv_heads * head_dim * block_size * elem_bytes;
  const int64_t scale_bytes = (int64_t)num_kv_heads * block_size * 4;
  if (page_bytes % 16 || (k_scale && scale_bytes % 16))
    return fail(IVAKV_E_SHAPE, "%s: page of %lld bytes is not a multiple of 16", name,
                (long long)page_bytes);
  if (n_moves == 0) return IVAKV_OK;
  if (!k_pool || !v_pool || !src_pages || !dst_pages || (!k_scale != !v_scale))
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (!aligned16(k_pool) || !aligned16(v_pool) || (k_scale && (!aligned16(k_scale) || !aligned16(v_scale))))
    return fail(IVAKV_E_ARG, "%s: pools must be 16-byte aligned", name);
  if (n_moves > 65535) return fail(IVAKV_E_SHAPE, "%s: at most 65535 moves per call", name);
  const int64_t chunks = page_bytes / 16;
  const unsigned bx = (unsigned)((chunks + 255) / 256 < 64 ? (chunks + 255) / 256 : 64);
  copy_pages_kernel<<<dim3(bx, (unsigned)n_moves), 256, 0, stream>>>(
      static_cast<Chunk16*>(k_pool), static_cast<Chunk16*>(v_pool),
      reinterpret_cast<Chunk16*>(k_scale), reinterpret_cast<Chunk16*>(v_scale), src_pages,
      dst_pages, num_pages, chunks, k_scale ? scale_bytes / 16 : 0);
  return launch_status(name);
}
