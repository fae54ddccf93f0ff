// FP8 (OCP e4m3fn) KV pages on gfx950: append with per-(slot, kv head) scaling and
// dequantizing gather.  Decode attention over these pages is ivakv_decode_attn_fp8
// (ivakv_decode.hip).
//
// Pool layout (bytes): k_pool [page][Hkv][D/16][16][16] (16-byte chunks of 16 dims,
// rows of a chunk column contiguous), v_pool [page][Hkv][16 * D] with the byte of
// (dim d, key r) at fp8_v_offset(d, r, D) = order [d%16][r/4][d/16][r%4] (each lane of
// the decode walk reads its V bytes as whole 16-byte loads), k_scale / v_scale
// [page][Hkv][16] fp32.  A row x of one (token, kv head) is
// stored as codes e4m3(x * sf) with sf = 448 / max|x| (1 for an all-zero row),
// clamped to [1e-8, 1e8] -- the reference's scaling rule
// (src/quant/fp8_runtime.py:66-76) applied per row -- and read back as code / sf.
//
// Conversions are written out in integer arithmetic (round to nearest even,
// saturating at +-448), so the codes do not depend on a hardware rounding mode.
#include "ivakv_e4m3.h"

namespace ivakv {
namespace {

constexpr int64_t kMaxGrid8 = 0x7fffffff;

template <typename E>
__device__ inline float to_f(E x) { return (float)x; }
template <>
__device__ inline float to_f<float>(float x) { return x; }

struct Append8Args {
  const void* k_new;
  const void* v_new;
  int64_t kts, khs, vts, vhs;  // element strides (token, head)
  uint8_t* k_pool;
  uint8_t* v_pool;
  float* k_scale;
  float* v_scale;
  const int32_t* slots;
  int n_tok, Hkv, D;
  int64_t n_slots;
};

// One wave per (token, kv head) row: lane l holds dims l*PER .. l*PER+PER-1 of K
// and V, the wave reduces max|x|, and every lane stores its codes.
template <typename E, int PER>
__global__ __launch_bounds__(256) void append8_kernel(Append8Args a) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= (int64_t)a.n_tok * a.Hkv) return;  // whole wave
  const int h = (int)(row % a.Hkv);
  const int64_t t = row / a.Hkv;
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.n_slots) return;
  const int64_t page = slot / 16;
  const int off = (int)(slot - page * 16);
  const int64_t tile = page * a.Hkv + h;
  const E* ks = static_cast<const E*>(a.k_new) + t * a.kts + h * a.khs;
  const E* vs = static_cast<const E*>(a.v_new) + t * a.vts + h * a.vhs;
  float kx[PER], vx[PER];
  float kmax = 0.f, vmax = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    kx[i] = to_f(ks[lane * PER + i]);
    vx[i] = to_f(vs[lane * PER + i]);
    kmax = fmaxf(kmax, fabsf(kx[i]));
    vmax = fmaxf(vmax, fabsf(vx[i]));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    kmax = fmaxf(kmax, __shfl_xor(kmax, o));
    vmax = fmaxf(vmax, __shfl_xor(vmax, o));
  }
  const float ksf = row_sf(kmax), vsf = row_sf(vmax);
  uint8_t* kp = a.k_pool + tile * (int64_t)a.D * 16;
  uint8_t* vp = a.v_pool + tile * (int64_t)a.D * 16;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int d = lane * PER + i;
    kp[((d >> 4) * 16 + off) * 16 + (d & 15)] = (uint8_t)e4m3_encode(kx[i] * ksf);
    vp[fp8_v_offset(d, off, a.D)] = (uint8_t)e4m3_encode(vx[i] * vsf);
  }
  if (lane == 0) {
    a.k_scale[tile * 16 + off] = ksf;
    a.v_scale[tile * 16 + off] = vsf;
  }
}

struct Gather8Args {
  const uint8_t* k_pool;
  const uint8_t* v_pool;
  const float* k_scale;
  const float* v_scale;
  const int32_t* bt;
  const int32_t* ctx;
  int max_blocks, Hkv, D, num_pages, out_len;
  void* k_out;
  void* v_out;
};

// Grid (position block of 16, kv head, sequence), 256 threads: thread i handles
// dims i, i+256, ... of the block's 16 x D elements.  Out of the context or on
// an invalid page the rows are zero.
template <typename E>
__global__ __launch_bounds__(256) void gather8_kernel(Gather8Args a) {
  const int blk = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int L = a.ctx[b];
  const int64_t page = blk < a.max_blocks ? (int64_t)a.bt[(int64_t)b * a.max_blocks + blk] : -1;
  const bool page_ok = page >= 0 && page < a.num_pages;
  const int64_t tile = (page_ok ? page : 0) * a.Hkv + h;
  E* ko = static_cast<E*>(a.k_out) + (((int64_t)b * a.Hkv + h) * a.out_len) * a.D;
  E* vo = static_cast<E*>(a.v_out) + (((int64_t)b * a.Hkv + h) * a.out_len) * a.D;
  for (int i = threadIdx.x; i < 16 * a.D; i += blockDim.x) {
    const int r = i / a.D, d = i - r * a.D;
    const int pos = blk * 16 + r;
    if (pos >= a.out_len) continue;
    float kv = 0.f, vv = 0.f;
    if (page_ok && pos < L) {
      const uint32_t kc = a.k_pool[tile * (int64_t)a.D * 16 + ((d >> 4) * 16 + r) * 16 + (d & 15)];
      const uint32_t vc = a.v_pool[tile * (int64_t)a.D * 16 + fp8_v_offset(d, r, a.D)];
      kv = e4m3_decode(kc) / a.k_scale[tile * 16 + r];
      vv = e4m3_decode(vc) / a.v_scale[tile * 16 + r];
    }
    ko[(int64_t)pos * a.D + d] = (E)kv;
    vo[(int64_t)pos * a.D + d] = (E)vv;
  }
}

}  // namespace
}  // namespace ivakv

using namespace ivakv;

extern "C" int ivakv_append_fp8(const void* k_new, const void* v_new, int64_t k_tok_stride,
                                int64_t k_head_stride, int64_t v_tok_stride,
                                int64_t v_head_stride, void* k_pool, void* v_pool, float* k_scale,
                                float* v_scale, const int32_t* slot_mapping, int n_tok,
                                int num_kv_heads, int head_dim, int block_size, int num_pages,
                                int dtype, hipStream_t stream) {
  static const char* name = "ivakv_append_fp8";
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (n_tok < 0 || num_kv_heads <= 0 || num_pages < 0)
    return fail(IVAKV_E_ARG, "%s: bad sizes n_tok=%d Hkv=%d num_pages=%d", name, n_tok,
                num_kv_heads, num_pages);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IVAKV_E_SHAPE, "%s: head_dim %d not in {64,128,256}", name, head_dim);
  if (block_size != 16) return fail(IVAKV_E_SHAPE, "%s: block_size %d != 16", name, block_size);
  if (n_tok == 0) return IVAKV_OK;
  if (!k_new || !v_new || !k_pool || !v_pool || !k_scale || !v_scale || !slot_mapping)
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (k_tok_stride < 0 || k_head_stride < 0 || v_tok_stride < 0 || v_head_stride < 0)
    return fail(IVAKV_E_ARG, "%s: negative stride", name);
  Append8Args a{k_new, v_new, k_tok_stride, k_head_stride, v_tok_stride, v_head_stride,
                static_cast<uint8_t*>(k_pool), static_cast<uint8_t*>(v_pool), k_scale, v_scale,
                slot_mapping, n_tok, num_kv_heads, head_dim, (int64_t)num_pages * 16};
  const int64_t blocks = ((int64_t)n_tok * num_kv_heads + 3) / 4;
  if (blocks > kMaxGrid8) return fail(IVAKV_E_SHAPE, "%s: too many rows", name);
  const dim3 grid((unsigned)blocks);
#define IVAKV_APPEND8(E)                                                            \
  switch (head_dim) {                                                               \
    case 64: append8_kernel<E, 1><<<grid, 256, 0, stream>>>(a); break;              \
    case 128: append8_kernel<E, 2><<<grid, 256, 0, stream>>>(a); break;             \
    default: append8_kernel<E, 4><<<grid, 256, 0, stream>>>(a); break;              \
  }
  switch (dtype) {
    case IVAKV_F16: IVAKV_APPEND8(_Float16); break;
    case IVAKV_BF16: IVAKV_APPEND8(__bf16); break;
    default: IVAKV_APPEND8(float); break;
  }
#undef IVAKV_APPEND8
  return launch_status(name);
}

extern "C" int ivakv_gather_fp8(const void* k_pool, const void* v_pool, const float* k_scale,
                                const float* v_scale, const int32_t* block_tables,
                                const int32_t* context_lens, int batch, int max_blocks,
                                int num_kv_heads, int head_dim, int block_size, int num_pages,
                                int out_len, void* k_out, void* v_out, int dtype,
                                hipStream_t stream) {
  static const char* name = "ivakv_gather_fp8";
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (batch < 0 || max_blocks < 0 || num_kv_heads <= 0 || num_pages < 0 || out_len < 0)
    return fail(IVAKV_E_ARG, "%s: bad sizes B=%d max_blocks=%d Hkv=%d num_pages=%d out_len=%d",
                name, batch, max_blocks, num_kv_heads, num_pages, out_len);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IVAKV_E_SHAPE, "%s: head_dim %d not in {64,128,256}", name, head_dim);
  if (block_size != 16) return fail(IVAKV_E_SHAPE, "%s: block_size %d != 16", name, block_size);
  if (batch == 0 || out_len == 0) return IVAKV_OK;
  if (!k_pool || !v_pool || !k_scale || !v_scale || !context_lens || !k_out || !v_out ||
      (max_blocks > 0 && !block_tables))
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (batch > 65535 || num_kv_heads > 65535)
    return fail(IVAKV_E_SHAPE, "%s: batch and num_kv_heads must be <= 65535", name);
  Gather8Args a{static_cast<const uint8_t*>(k_pool), static_cast<const uint8_t*>(v_pool),
                k_scale, v_scale, block_tables, context_lens, max_blocks, num_kv_heads, head_dim,
                num_pages, out_len, k_out, v_out};
  const dim3 grid((unsigned)cdiv(out_len, 16), (unsigned)num_kv_heads, (unsigned)batch);
  switch (dtype) {
    case IVAKV_F16: gather8_kernel<_Float16><<<grid, 256, 0, stream>>>(a); break;
    case IVAKV_BF16: gather8_kernel<__bf16><<<grid, 256, 0, stream>>>(a); break;
    default: gather8_kernel<float><<<grid, 256, 0, stream>>>(a); break;
  }
  return launch_status(name);
}
