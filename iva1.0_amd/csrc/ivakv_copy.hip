// Bit-exact KV data movement on gfx950: paged append (scatter into slots), paged
// gather (pages -> contiguous rows) and the index gather/scatter of a contiguous
// [B, H, S, D] cache.  Elements are moved as raw 16/32-bit words, so every
// kernel here is exact for any dtype of that size.
//
// All kernels are HBM-bound copies: each thread moves one 16-byte chunk
// (8 half / 4 float elements) per row, so a wavefront reads or writes 1 KiB
// per instruction in the layout-favoured direction.
#include "ivakv_internal.h"

namespace ivakv {
namespace {

struct alignas(16) Chunk16 {
  uint32_t w[4];
};

// ---------------------------------------------------------------------------
// append: new rows [n_tok][Hkv][D] (strided) -> k_pool / v_pool slots
// ---------------------------------------------------------------------------
struct AppendArgs {
  const void* k_new;
  const void* v_new;
  int64_t kts, khs, vts, vhs;  // element strides (token, head)
  void* k_pool;
  void* v_pool;
  const int32_t* slots;
  int n_tok, Hkv, D, bs;
  int64_t n_slots;  // num_pages * bs
};

// Element path (sources or pools not 16-byte aligned): one thread per (token, head,
// chunk of X elements).  Thread order (token % 16, chunk, head, token / 16): the 16
// lanes of a token group cover 16 consecutive tokens, which a chunk append puts in
// consecutive slots of one page, so their K elements are 256 contiguous bytes per
// chunk and each V dim's elements one 32-byte row.
template <typename E>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
  constexpr int X = 16 / sizeof(E);
  const int nch = a.D / X;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)cdiv(a.n_tok, 16) * 16 * a.Hkv * nch;
  if (gid >= total) return;
  const int t_lo = (int)(gid & 15);
  const int64_t g1 = gid >> 4;
  const int c = (int)(g1 % nch);
  const int64_t g2 = g1 / nch;
  const int h = (int)(g2 % a.Hkv);
  const int64_t t = (g2 / a.Hkv) * 16 + t_lo;
  if (t >= a.n_tok) return;
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.n_slots) return;
  const int64_t page = slot / a.bs;
  const int off = (int)(slot - page * a.bs);
  const int64_t head_base = page * a.Hkv + h;
  const E* ks = static_cast<const E*>(a.k_new) + t * a.kts + h * a.khs + (int64_t)c * X;
  const E* vs = static_cast<const E*>(a.v_new) + t * a.vts + h * a.vhs + (int64_t)c * X;
  E* kd = static_cast<E*>(a.k_pool) + ((head_base * nch + c) * a.bs + off) * X;
  E* vd = static_cast<E*>(a.v_pool) + head_base * a.D * a.bs + (int64_t)c * X * a.bs + off;
#pragma unroll
  for (int i = 0; i < X; ++i) kd[i] = ks[i];
#pragma unroll
  for (int i = 0; i < X; ++i) vd[(int64_t)i * a.bs] = vs[i];
}

// 16-byte path: one thread per (token, group of up to kAppendHeads kv heads, 16-byte
// chunk), thread order (token % 16, chunk, head group, token / 16).  A lane issues the
// K and V loads of all its heads before the first store, so a wave keeps 16 KiB of
// source rows in flight and a chunk append runs in about one round of resident waves
// (one head per lane: eight rounds of single round trips).  K chunks are stored whole
// (256 contiguous bytes per 16 consecutive slots); each V chunk is spread over X rows
// of the page's [D][bs] tile.  Row loads and K stores carry the non-temporal hint
// (8192 rows from HBM: 14.9 µs against 17.7 µs with neither).  Blocks run in
// XCD-contiguous order (xcd_contiguous_block).  Groups of 32 or 64 consecutive tokens
// per lane group (fewer split pages, 16 / 32 bytes per token per load) measured
// 21 / 33 µs against 14.8 µs on 8192 aligned rows.
// Few rows (a decode step's one token per sequence, each to its own page; short
// chunks): one head per lane in 64-thread workgroups (HEADS = 1), so the stores spread
// over many CUs instead of the few workgroups eight heads per lane would give.  Rows of
// 8 kv heads x 128 dims from HBM: a 32-sequence decode step 14.0 -> 2.9 us, 256
// sequences 16.4 -> 5.7 us, one 512-row chunk 6.1 -> 3.2 us, 2048 rows 7.6 -> 7.1 us;
// at 8192 rows eight heads per lane stay ahead (15.6 against 18.5 us).
constexpr int kAppendHeads = 8;
constexpr int64_t kFewAppendThreads = 1024 * 64;  // below 1024 waves: one head per lane

template <typename E, int HEADS>
__global__ __launch_bounds__(256) void append_vec_kernel(AppendArgs a) {
  constexpr int X = 16 / sizeof(E);
  const int nch = a.D / X;
  const int ngrp = cdiv(a.Hkv, HEADS);
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
  const E* ks = static_cast<const E*>(a.k_new) + t * a.kts + (int64_t)c * X;
  const E* vs = static_cast<const E*>(a.v_new) + t * a.vts + (int64_t)c * X;
  union Row {
    Chunk16 c16;
    E e[X];
  };
  Row k[HEADS], v[HEADS];
#pragma unroll
  for (int u = 0; u < HEADS; ++u) {
    if (u < nh) {
      k[u].c16 = ld<true, Chunk16>(ks + (h0 + u) * a.khs);
      v[u].c16 = ld<true, Chunk16>(vs + (h0 + u) * a.vhs);
    }
  }
#pragma unroll
  for (int u = 0; u < HEADS; ++u) {
    if (u < nh) {
      const int64_t head_base = page * a.Hkv + h0 + u;
      E* kd = static_cast<E*>(a.k_pool) + ((head_base * nch + c) * a.bs + off) * X;
      E* vd = static_cast<E*>(a.v_pool) + head_base * a.D * a.bs + (int64_t)c * X * a.bs + off;
      st<true, Chunk16>(kd, k[u].c16);
#pragma unroll
      for (int i = 0; i < X; ++i) vd[(int64_t)i * a.bs] = v[u].e[i];
    }
  }
}

// ---------------------------------------------------------------------------
// gather: pages -> k_out / v_out = [B][Hkv][out_len][D]
// ---------------------------------------------------------------------------
struct GatherArgs {
  const void* k_pool;
  const void* v_pool;
  const int32_t* bt;
  const int32_t* ctx;
  int max_blocks, Hkv, D, bs, num_pages, out_len;
  void* k_out;
  void* v_out;
};

// Any element size, page size and head_dim (gather16_kernel takes 2-byte elements on
// 16-row pages at head_dim 64 / 128 / 256).  Grid (logical page, group of H kv heads,
// sequence), 256 threads per kv head.  Thread index (within a head) = chunk * bs + row, so
// the K page (stored [D/X][bs][X]) is read as one contiguous run and each
// 16-byte V chunk is assembled from X row-adjacent elements of the [D][bs]
// page (consecutive lanes read consecutive rows).  K reads carry the non-temporal hint
// (each page is read once); the output stores do not (C2 batch at one kv head per
// workgroup: 161 µs, against 178 µs with the hint on the stores too).
template <typename E, int H>
__global__ __launch_bounds__(256 * H) void gather_kernel(GatherArgs a) {
  constexpr int X = 16 / sizeof(E);
  const int hl = threadIdx.x >> 8, tl = threadIdx.x & 255;
  const int j = blockIdx.x, h = blockIdx.y * H + hl, b = blockIdx.z;
  if (h >= a.Hkv) return;
  const int nch = a.D / X;
  int L = a.ctx[b];
  L = L < 0 ? 0 : L;
  const int lim = L < a.out_len ? L : a.out_len;
  int64_t phys = -1;
  if (j < a.max_blocks && (int64_t)j * a.bs < lim) {
    const int64_t p = a.bt[(int64_t)b * a.max_blocks + j];
    if (p >= 0 && p < a.num_pages) phys = p;
  }
  const int rows = nch * a.bs;
  for (int idx = tl; idx < rows; idx += 256) {
    const int t = idx % a.bs;
    const int c = idx / a.bs;
    const int64_t pos = (int64_t)j * a.bs + t;
    if (pos >= a.out_len) continue;
    const int64_t orow = (((int64_t)b * a.Hkv + h) * a.out_len + pos) * a.D + (int64_t)c * X;
    union {
      Chunk16 c16;
      E e[X];
    } kv, vv;
    kv.c16 = Chunk16{{0u, 0u, 0u, 0u}};
    vv.c16 = Chunk16{{0u, 0u, 0u, 0u}};
    if (phys >= 0 && pos < lim) {
      const int64_t head_base = phys * a.Hkv + h;
      kv.c16 = ld<true, Chunk16>(static_cast<const E*>(a.k_pool) + ((head_base * nch + c) * a.bs + t) * X);
      const E* vb = static_cast<const E*>(a.v_pool) + head_base * a.D * a.bs + (int64_t)c * X * a.bs + t;
#pragma unroll
      for (int i = 0; i < X; ++i) vv.e[i] = vb[(int64_t)i * a.bs];
    }
    st<false, Chunk16>(static_cast<E*>(a.k_out) + orow, kv.c16);
    st<false, Chunk16>(static_cast<E*>(a.v_out) + orow, vv.c16);
  }
}

// The same gather for 2-byte elements on 16-row pages: grid (logical page, group of H kv
// heads, sequence), 2 D threads per kv head.  Thread t of a head takes row t / (D/8) and
// 8-element chunk t % (D/8): its K chunk is one 16-byte load (the K page keeps a row's
// chunk contiguous); the V page ([D][16]) is staged in LDS with one 16-byte load per
// thread and read back as the row's 8 elements of the chunk.  Consecutive threads store
// consecutive chunks of a row, so a wave stores whole output rows.  All loads of a thread
// are issued before the barrier; rows past the context or on an invalid page are stored
// as zeros without loads.  C2's batch: 147 us against 152.5 us for gather_kernel at four
// kv heads per workgroup (lanes along the rows, each V chunk from 8 two-byte loads).
template <int D, int H>
__global__ __launch_bounds__(1024) void gather16_kernel(GatherArgs a) {
  constexpr int NC = D / 8;  // 16-byte chunks per row
  __shared__ Chunk16 s_v[H][2 * D];
  const int hl = threadIdx.x / (2 * D), t = threadIdx.x - hl * (2 * D);
  const int j = blockIdx.x, h = blockIdx.y * H + hl, b = blockIdx.z;
  int L = a.ctx[b];
  L = L < 0 ? 0 : L;
  const int lim = L < a.out_len ? L : a.out_len;
  int64_t phys = -1;
  if (h < a.Hkv && j < a.max_blocks && (int64_t)j * 16 < lim) {
    const int64_t p = a.bt[(int64_t)b * a.max_blocks + j];
    if (p >= 0 && p < a.num_pages) phys = p;
  }
  const int r = t / NC, c = t - r * NC;
  const int64_t pos = (int64_t)j * 16 + r;
  const bool has = phys >= 0 && pos < lim;
  Chunk16 kv = Chunk16{{0u, 0u, 0u, 0u}};
  if (phys >= 0) {  // uniform per kv head
    const int64_t tile = (phys * a.Hkv + h) * (int64_t)(16 * D);  // elements
    s_v[hl][t] = ld<true, Chunk16>(static_cast<const uint16_t*>(a.v_pool) + tile + 8 * t);
    if (has) kv = ld<true, Chunk16>(static_cast<const uint16_t*>(a.k_pool) + tile + (c * 16 + r) * 8);
  }
  __syncthreads();
  if (h >= a.Hkv || pos >= a.out_len) return;
  Chunk16 vv = Chunk16{{0u, 0u, 0u, 0u}};
  if (has) {
    const uint16_t* sv = reinterpret_cast<const uint16_t*>(s_v[hl]);
    uint16_t e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = sv[(8 * c + i) * 16 + r];
    vv = __builtin_bit_cast(Chunk16, e);
  }
  const int64_t orow = (((int64_t)b * a.Hkv + h) * a.out_len + pos) * D + 8 * c;
  st<false, Chunk16>(static_cast<uint16_t*>(a.k_out) + orow, kv);
  st<false, Chunk16>(static_cast<uint16_t*>(a.v_out) + orow, vv);
}

// ---------------------------------------------------------------------------
// index gather / scatter on a contiguous-layout [B][H][S][D] cache
// ---------------------------------------------------------------------------
struct IndexArgs {
  const void* src;
  void* dst;
  int64_t s_b, s_h, s_s, s_d;  // strides of the indexed cache
  int64_t o_b, o_h, o_s, o_d;  // strides of the dense side (gather out / scatter values)
  const int64_t* idx;
  int n_idx, H, S, D;
  int64_t total;
};

// Elements per thread (grid-stride).  On the ops bench's 1024 of 4096 positions (fp16,
// 8 heads, D 128): gather / scatter 25.0 / 25.0 us at 1, 24.6-24.8 / 23.6 us at 2, 26.4 /
// 25.1 us at 4, 28.3 / 26.7 us at 8.
constexpr int kIdxU = 2;

// kIdxU elements per thread, gid + u * (grid threads), in three phases so every load of
// the thread is in flight together: the elements' indices, then their source rows, then
// the stores.  GATHER: out[b,h,j] = kv[b,h,idx[j]] (zero row for an out-of-range index).
// SCATTER: kv[b,h,idx[j]] = values[b,h,j] (out-of-range index skipped).  16-byte stores
// carry the non-temporal hint, and so do the gather's cache reads (the scatter's dense
// reads measured faster without).
template <typename E, bool VEC, bool GATHER>
__global__ __launch_bounds__(256) void index_copy_kernel(IndexArgs a) {
  constexpr int X = VEC ? 16 / (int)sizeof(E) : 1;
  using V = typename std::conditional<VEC, Chunk16, E>::type;
  const int per_row = a.D / X;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int e[kIdxU], jj[kIdxU];
  int64_t bh[kIdxU], ix[kIdxU];
#pragma unroll
  for (int u = 0; u < kIdxU; ++u) {
    const int64_t g = gid + u * stride < a.total ? gid + u * stride : 0;
    e[u] = (int)(g % per_row);
    const int64_t r = g / per_row;
    jj[u] = (int)(r % a.n_idx);
    bh[u] = r / a.n_idx;  // b * H + h
    ix[u] = a.idx[jj[u]];
  }
  int64_t cache_row[kIdxU], dense_row[kIdxU];
  bool ok[kIdxU];
  V val[kIdxU];
#pragma unroll
  for (int u = 0; u < kIdxU; ++u) {
    const int h = (int)(bh[u] % a.H);
    const int64_t b = bh[u] / a.H;
    ok[u] = gid + u * stride < a.total && ix[u] >= 0 && ix[u] < a.S;
    cache_row[u] = b * a.s_b + h * a.s_h + (ok[u] ? ix[u] : 0) * a.s_s + (int64_t)e[u] * X * a.s_d;
    dense_row[u] = b * a.o_b + h * a.o_h + (int64_t)jj[u] * a.o_s + (int64_t)e[u] * X * a.o_d;
    const E* src = static_cast<const E*>(a.src) + (GATHER ? cache_row[u] : dense_row[u]);
    if constexpr (VEC) {
      val[u] = Chunk16{{0u, 0u, 0u, 0u}};
      if (ok[u]) val[u] = GATHER ? ld<true, Chunk16>(src) : ld<false, Chunk16>(src);
    } else {
      val[u] = ok[u] ? *src : E(0);
    }
  }
#pragma unroll
  for (int u = 0; u < kIdxU; ++u) {
    if (gid + u * stride >= a.total) continue;
    if constexpr (GATHER) {
      E* o = static_cast<E*>(a.dst) + dense_row[u];
      if constexpr (VEC) st<true, Chunk16>(o, val[u]);
      else *o = val[u];
    } else {
      if (!ok[u]) continue;
      E* o = static_cast<E*>(a.dst) + cache_row[u];
      if constexpr (VEC) st<true, Chunk16>(o, val[u]);
      else *o = val[u];
    }
  }
}

inline unsigned blocks_for(int64_t total, int per_block) {
  return (unsigned)((total + per_block - 1) / per_block);
}

constexpr int64_t kMaxGrid = 2147483647LL;

}  // namespace
}  // namespace ivakv

using namespace ivakv;

extern "C" int ivakv_append(const void* k_new, const void* v_new, int64_t k_tok_stride,
                            int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
                            void* k_pool, void* v_pool, const int32_t* slot_mapping, int n_tok,
                            int num_kv_heads, int head_dim, int block_size, int num_pages,
                            int dtype, hipStream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0) return fail(IVAKV_E_DTYPE, "ivakv_append: unknown dtype code %d", dtype);
  if (n_tok < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 || num_pages < 0)
    return fail(IVAKV_E_ARG,
                "ivakv_append: bad sizes n_tok=%d Hkv=%d D=%d block_size=%d num_pages=%d", n_tok,
                num_kv_heads, head_dim, block_size, num_pages);
  const int X = 16 / es;
  if (head_dim % X != 0)
    return fail(IVAKV_E_SHAPE, "ivakv_append: head_dim %d must be a multiple of %d", head_dim, X);
  if (n_tok == 0) return IVAKV_OK;
  if (!k_new || !v_new || !k_pool || !v_pool || !slot_mapping)
    return fail(IVAKV_E_ARG, "ivakv_append: null pointer argument");
  if (k_tok_stride < 0 || k_head_stride < 0 || v_tok_stride < 0 || v_head_stride < 0)
    return fail(IVAKV_E_ARG, "ivakv_append: negative stride");
  AppendArgs a{k_new, v_new, k_tok_stride, k_head_stride, v_tok_stride, v_head_stride,
               k_pool, v_pool, slot_mapping, n_tok, num_kv_heads, head_dim, block_size,
               (int64_t)num_pages * block_size};
  const bool vec = aligned16(k_new) && aligned16(v_new) && aligned16(k_pool) && aligned16(v_pool) &&
                   (k_tok_stride % X == 0) && (k_head_stride % X == 0) &&
                   (v_tok_stride % X == 0) && (v_head_stride % X == 0);
  const int64_t lanes_per_head_group = (int64_t)cdiv(n_tok, 16) * 16 * (head_dim / X);
  const bool few = vec && lanes_per_head_group * cdiv(num_kv_heads, kAppendHeads) < kFewAppendThreads;
  const int64_t per_tok = vec && !few ? (int64_t)cdiv(num_kv_heads, kAppendHeads) : num_kv_heads;
  const int64_t total = lanes_per_head_group * per_tok;
  const int threads = few ? 64 : 256;
  const unsigned grid = blocks_for(total, threads);
  if ((int64_t)grid > kMaxGrid) return fail(IVAKV_E_SHAPE, "ivakv_append: too many rows");
  if (es == 4) {
    if (few) append_vec_kernel<uint32_t, 1><<<grid, threads, 0, stream>>>(a);
    else if (vec) append_vec_kernel<uint32_t, kAppendHeads><<<grid, threads, 0, stream>>>(a);
    else append_kernel<uint32_t><<<grid, threads, 0, stream>>>(a);
  } else {
    if (few) append_vec_kernel<uint16_t, 1><<<grid, threads, 0, stream>>>(a);
    else if (vec) append_vec_kernel<uint16_t, kAppendHeads><<<grid, threads, 0, stream>>>(a);
    else append_kernel<uint16_t><<<grid, threads, 0, stream>>>(a);
  }
  return launch_status("ivakv_append");
}

// kv heads per workgroup of the gather (C2 batch: 1 / 2 / 4 heads 161 / 156.5 / 152.5 us)
constexpr int kGatherHeads = 4;

extern "C" int ivakv_gather(const void* k_pool, const void* v_pool, const int32_t* block_tables,
                            const int32_t* context_lens, int batch, int max_blocks,
                            int num_kv_heads, int head_dim, int block_size, int num_pages,
                            int out_len, void* k_out, void* v_out, int dtype,
                            hipStream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0) return fail(IVAKV_E_DTYPE, "ivakv_gather: unknown dtype code %d", dtype);
  if (batch < 0 || max_blocks < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_pages < 0 || out_len < 0)
    return fail(IVAKV_E_ARG,
                "ivakv_gather: bad sizes B=%d max_blocks=%d Hkv=%d D=%d block_size=%d "
                "num_pages=%d out_len=%d",
                batch, max_blocks, num_kv_heads, head_dim, block_size, num_pages, out_len);
  const int X = 16 / es;
  if (head_dim % X != 0)
    return fail(IVAKV_E_SHAPE, "ivakv_gather: head_dim %d must be a multiple of %d", head_dim, X);
  if (batch == 0 || out_len == 0) return IVAKV_OK;
  if (!k_pool || !v_pool || !context_lens || !k_out || !v_out || (max_blocks > 0 && !block_tables))
    return fail(IVAKV_E_ARG, "ivakv_gather: null pointer argument");
  if (!aligned16(k_pool) || !aligned16(v_pool) || !aligned16(k_out) || !aligned16(v_out))
    return fail(IVAKV_E_ARG, "ivakv_gather: pools and outputs must be 16-byte aligned");
  if (batch > 65535 || num_kv_heads > 65535)
    return fail(IVAKV_E_SHAPE, "ivakv_gather: batch and num_kv_heads must be <= 65535");
  GatherArgs a{k_pool, v_pool, block_tables, context_lens, max_blocks, num_kv_heads, head_dim,
               block_size, num_pages, out_len, k_out, v_out};
  if (es == 2 && block_size == 16 && (head_dim == 64 || head_dim == 128 || head_dim == 256)) {
    // 1024 threads: 2 D per kv head
    const int hpw = 512 / head_dim;
    const dim3 g16((unsigned)cdiv(out_len, 16), (unsigned)cdiv(num_kv_heads, hpw), (unsigned)batch);
    switch (head_dim) {
      case 64: gather16_kernel<64, 8><<<g16, 1024, 0, stream>>>(a); break;
      case 128: gather16_kernel<128, 4><<<g16, 1024, 0, stream>>>(a); break;
      default: gather16_kernel<256, 2><<<g16, 1024, 0, stream>>>(a); break;
    }
    return launch_status("ivakv_gather");
  }
  constexpr int kH = kGatherHeads;
  dim3 grid((unsigned)cdiv(out_len, block_size), (unsigned)cdiv(num_kv_heads, kH), (unsigned)batch);
  if (es == 4) gather_kernel<uint32_t, kH><<<grid, 256 * kH, 0, stream>>>(a);
  else gather_kernel<uint16_t, kH><<<grid, 256 * kH, 0, stream>>>(a);
  return launch_status("ivakv_gather");
}

namespace {

int index_copy(bool gather, const char* name, const void* src, void* dst, int64_t s_b, int64_t s_h,
               int64_t s_s, int64_t s_d, int64_t o_b, int64_t o_h, int64_t o_s, int64_t o_d,
               const int64_t* indices, int n_idx, int batch, int n_heads, int seq_len,
               int head_dim, int dtype, hipStream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (n_idx < 0 || batch < 0 || n_heads < 0 || seq_len < 0 || head_dim < 0)
    return fail(IVAKV_E_ARG, "%s: negative size", name);
  const int64_t rows = (int64_t)batch * n_heads * n_idx;
  if (rows == 0 || head_dim == 0) return IVAKV_OK;
  if (!src || !dst || !indices) return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  const int X = 16 / es;
  const bool vec = s_d == 1 && o_d == 1 && head_dim % X == 0 && aligned16(src) && aligned16(dst) &&
                   s_b % X == 0 && s_h % X == 0 && s_s % X == 0 && o_b % X == 0 &&
                   o_h % X == 0 && o_s % X == 0;
  IndexArgs a{src, dst, s_b, s_h, s_s, s_d, o_b, o_h, o_s, o_d, indices, n_idx, n_heads, seq_len,
              head_dim, rows * (vec ? head_dim / X : head_dim)};
  const unsigned grid = blocks_for((a.total + kIdxU - 1) / kIdxU, 256);
  if ((int64_t)grid > kMaxGrid) return fail(IVAKV_E_SHAPE, "%s: too many rows", name);
#define IVAKV_IDX_LAUNCH(E)                                                              \
  do {                                                                                   \
    if (gather) {                                                                        \
      if (vec) index_copy_kernel<E, true, true><<<grid, 256, 0, stream>>>(a);            \
      else index_copy_kernel<E, false, true><<<grid, 256, 0, stream>>>(a);               \
    } else {                                                                             \
      if (vec) index_copy_kernel<E, true, false><<<grid, 256, 0, stream>>>(a);           \
      else index_copy_kernel<E, false, false><<<grid, 256, 0, stream>>>(a);              \
    }                                                                                    \
  } while (0)
  if (es == 4) IVAKV_IDX_LAUNCH(uint32_t);
  else IVAKV_IDX_LAUNCH(uint16_t);
#undef IVAKV_IDX_LAUNCH
  return launch_status(name);
}

}  // namespace

extern "C" int ivakv_index_gather(const void* kv, int64_t s_b, int64_t s_h, int64_t s_s,
                                  int64_t s_d, const int64_t* indices, int n_idx, int batch,
                                  int n_heads, int seq_len, int head_dim, void* out, int dtype,
                                  hipStream_t stream) {
  const int64_t o_s = head_dim, o_h = (int64_t)n_idx * head_dim, o_b = (int64_t)n_heads * o_h;
  return index_copy(true, "ivakv_index_gather", kv, out, s_b, s_h, s_s, s_d, o_b, o_h, o_s, 1,
                    indices, n_idx, batch, n_heads, seq_len, head_dim, dtype, stream);
}

extern "C" int ivakv_index_scatter(void* kv, int64_t s_b, int64_t s_h, int64_t s_s, int64_t s_d,
                                   const int64_t* indices, int n_idx, const void* values,
                                   int64_t v_b, int64_t v_h, int64_t v_s, int64_t v_d, int batch,
                                   int n_heads, int seq_len, int head_dim, int dtype,
                                   hipStream_t stream) {
  return index_copy(false, "ivakv_index_scatter", values, kv, s_b, s_h, s_s, s_d, v_b, v_h, v_s,
                    v_d, indices, n_idx, batch, n_heads, seq_len, head_dim, dtype, stream);
}
