// FP8 (OCP e4m3fn) KV pages on gfx950: append with per-(slot, kv head) scaling (plain,
// or with K rotated by RoPE on the way in) and dequantizing gather.  Decode attention over these pages is ivakv_decode_attn_fp8
// (ivakv_decode.hip).
//
// Pool layout (bytes): k_pool [page][Hkv][D/16][16][16] (16-byte chunks of 16 dims,
// rows of a chunk column contiguous), v_pool [page][Hkv][16 * D] with the byte of
// (dim d, key r) at fp8_v_offset(d, r, D) = order [d%16][r/4][d/16][r%4] (each lane of
// the decode walk reads its V bytes as whole 16-byte loads), k_scale / v_scale
// [page][Hkv][16] fp32.  A row x of one (token, kv head) is
// stored as codes e4m3(x * sf) with sf = 448 / max|x| (1 for an all-zero row),
// clamped to [1e-8, 1e8] (1e-8 for a row holding a NaN or an infinity) -- the
// reference's scaling rule
// (src/quant/fp8_runtime.py:66-76) applied per row -- and read back as code / sf.
//
// Conversions are written out in integer arithmetic (round to nearest even,
// saturating at +-448), so the codes do not depend on a hardware rounding mode.
#include "ivakv_e4m3.h"
#include "ivakv_rope.h"

namespace ivakv {
namespace {

struct Append8Args {
  const void* k_new;
  const void* v_new;
  int64_t kts, khs, vts, vhs;  // element strides (token, head)
  uint8_t* k_pool;
  uint8_t* v_pool;
  float* k_scale;
  float* v_scale;
  const int32_t* slots;
  const int32_t* pos;  // RoPE positions (the RoPE variant only)
  int n_tok, Hkv;
  int64_t n_slots;
  float theta;
};

// Codes of a, b, c, d packed into a word (byte i: the i-th value).  hw: the hardware
// conversion (round to nearest even), for rows whose scaled values all lie below 464,
// where it agrees with e4m3_encode (a GPU test checks every code, tie and neighbouring
// float; values in (448, 464) round to 448 either way); rows beyond (an inf or NaN
// element, or a max |x| so large that the clamped factor leaves it above 448) keep
// e4m3_encode's saturation and NaN code.
__device__ inline uint32_t encode4(float a, float b, float c, float d, bool hw) {
  if (hw) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
  }
  return e4m3_encode(a) | (e4m3_encode(b) << 8) | (e4m3_encode(c) << 16) | (e4m3_encode(d) << 24);
}

// Value of lane l ^ 1 (ctrl 0xB1) or l ^ 2 (0x4E) inside each group of four lanes (DPP
// quad permutation; every lane of the wave active).
template <int kCtrl>
__device__ inline float quad_swap(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),
                                                               kCtrl, 0xF, 0xF, false));
}

// One lane's share of a token's K or V row: chunks g, g + 4, .. of 16 elements, each
// loaded as whole 16-byte words.
template <typename E, int D>
struct RowShare {
  static constexpr int kWords = sizeof(E);  // 16-byte words per 16-element chunk
  uint4 w[D / 64][kWords];
};
template <typename E>
struct Chunk16 {
  E e[16];
};

template <typename E, int D>
__device__ inline void load_share(const E* row, int g, RowShare<E, D>& s) {
#pragma unroll
  for (int j = 0; j < D / 64; ++j)
#pragma unroll
    for (int w = 0; w < RowShare<E, D>::kWords; ++w)
      s.w[j][w] = *reinterpret_cast<const uint4*>(row + 16 * (g + 4 * j) + w * (16 / (int)sizeof(E)));
}

// One workgroup per 16 consecutive tokens (token groups in XCD-contiguous order,
// xcd_contiguous_block) and group of kv heads (grid y): wave w of
// workgroup (x, y) takes kv heads 4y + w, 4y + w + 4 gridDim.y, ... (a few tokens: one
// head per wave, so the rows' round trips overlap; many: every head in one workgroup).
// Each lane holds one token r and chunk group g: the 16-dim chunks g, g + 4, .. of
// that token's K and V rows (D / 64 chunks).  A group whose 16 tokens fill one page in
// order (a page-aligned chunk append) puts the tokens across lanes (r = l % 16,
// g = l / 16: each K store instruction writes 16 consecutive rows of a chunk, 256
// contiguous bytes); any other group puts a token's four lanes side by side (r = l / 4,
// g = l % 4), so the V byte stores of a group split over two pages touch fewer lines
// (8192 rows as 16 chunks starting mid-page 15.4 -> 14.5 us, and 13.4 -> 12.8 us aligned
// with the uniform branch below).  A row's max |x| is reduced over the four lanes of its
// token (shuffles, or DPP quad permutations); each lane then stores its K chunks as
// whole 16-byte code chunks and its V codes byte by byte (assembling 4-byte words
// across lanes measured slower).  The codes come from the hardware conversion
// (encode4) in one branch-free block when every row of the wave allows it.
// ROPE: K is rotated first (rotate_pair, rounded once to the source dtype, as
// ivakv_rope rounds it), with cos / sin of the workgroup's 16 tokens x D/2 pairs
// computed once into LDS and shared by every kv head.
template <typename E, int D, bool ROPE, int WPB>
__global__ __launch_bounds__(256) void append8_kernel(Append8Args a) {
  constexpr int NC = D / 64;  // chunks per lane
  constexpr int HALF = D / 2;
  __shared__ float s_cs[ROPE ? 16 * HALF : 1], s_sn[ROPE ? 16 * HALF : 1];
  __shared__ float s_freq[ROPE ? kFreqTable : 1];
  const int64_t t0 = xcd_contiguous_block(blockIdx.x, gridDim.x) * 16;
  if constexpr (ROPE) {
    fill_freqs(s_freq, HALF, D, a.theta);
    for (int e = threadIdx.x; e < 16 * HALF; e += blockDim.x) {
      const int64_t tt = t0 + e / HALF;
      const int p = tt < a.n_tok ? a.pos[tt] : 0;
      pair_angle(s_freq, p, e % HALF, D, a.theta, s_cs[e], s_sn[e]);
    }
    __syncthreads();
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Lane layout only (any slots are handled either way): the group's first and last
  // tokens at the first and last row of one page.
  const int32_t s_first = a.slots[t0];
  const int32_t s_last = t0 + 15 < a.n_tok ? a.slots[t0 + 15] : -1;
  const bool whole = s_first >= 0 && (s_first & 15) == 0 && s_last == s_first + 15;
  const int r = whole ? (lane & 15) : (lane >> 2), g = whole ? (lane >> 4) : (lane & 3);
  const int64_t t = t0 + r;
  const bool tok = t < a.n_tok;
  const int64_t slot = tok ? a.slots[t] : -1;
  const bool ok = slot >= 0 && slot < a.n_slots;  // the same for the four lanes of a token
  const int64_t page = ok ? slot / 16 : 0;
  const int off = ok ? (int)(slot - page * 16) : 0;
  const int64_t tc = tok ? t : t0;  // rows past the batch read the group's first row
  for (int h = WPB * (int)blockIdx.y + wave; h < a.Hkv; h += WPB * (int)gridDim.y) {
    RowShare<E, D> kr, vr;
    load_share<E, D>(static_cast<const E*>(a.k_new) + tc * a.kts + h * a.khs, g, kr);
    load_share<E, D>(static_cast<const E*>(a.v_new) + tc * a.vts + h * a.vhs, g, vr);
    E ke[NC][16];
    float kx[NC][16], vx[NC][16];
    // max |x| drops NaN (fmaxf); the sum of |x| is non-finite exactly when the row holds
    // an infinity or a NaN, or is so large that its factor clamps to 1e-8 anyway, so
    // a non-finite sum stands for the reference rule's 1e-8 (row_sf of a NaN max)
    float kmax = 0.f, vmax = 0.f, ksum = 0.f, vsum = 0.f;
#pragma unroll
    for (int j = 0; j < NC; ++j) {
      const int c = g + 4 * j;
      const Chunk16<E> kc = __builtin_bit_cast(Chunk16<E>, kr.w[j]);
      const Chunk16<E> vc = __builtin_bit_cast(Chunk16<E>, vr.w[j]);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        ke[j][i] = kc.e[i];
        vx[j][i] = rope_ld(vc.e[i]);
      }
      if constexpr (ROPE) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int e = r * HALF + 8 * c + q;
          rotate_pair(ke[j][2 * q], ke[j][2 * q + 1], s_cs[e], s_sn[e]);
        }
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        kx[j][i] = rope_ld(ke[j][i]);
        kmax = fmaxf(kmax, fabsf(kx[j][i]));
        vmax = fmaxf(vmax, fabsf(vx[j][i]));
        ksum += fabsf(kx[j][i]);
        vsum += fabsf(vx[j][i]);
      }
    }
    if (whole) {
      kmax = fmaxf(kmax, __shfl_xor(kmax, 16));
      kmax = fmaxf(kmax, __shfl_xor(kmax, 32));
      vmax = fmaxf(vmax, __shfl_xor(vmax, 16));
      vmax = fmaxf(vmax, __shfl_xor(vmax, 32));
      ksum += __shfl_xor(ksum, 16);
      ksum += __shfl_xor(ksum, 32);
      vsum += __shfl_xor(vsum, 16);
      vsum += __shfl_xor(vsum, 32);
    } else {
      kmax = fmaxf(kmax, quad_swap<0xB1>(kmax));
      vmax = fmaxf(vmax, quad_swap<0xB1>(vmax));
      ksum += quad_swap<0xB1>(ksum);
      vsum += quad_swap<0xB1>(vsum);
      kmax = fmaxf(kmax, quad_swap<0x4E>(kmax));
      vmax = fmaxf(vmax, quad_swap<0x4E>(vmax));
      ksum += quad_swap<0x4E>(ksum);
      vsum += quad_swap<0x4E>(vsum);
    }
    const bool kfin = __builtin_isfinite(ksum), vfin = __builtin_isfinite(vsum);
    const float ksf = kfin ? row_sf(kmax) : 1e-8f, vsf = vfin ? row_sf(vmax) : 1e-8f;
    const bool khw = kfin && kmax * ksf < 464.f, vhw = vfin && vmax * vsf < 464.f;
    // wave-uniform: every row of the wave takes the hardware conversion
    const bool all_hw = __builtin_amdgcn_ballot_w64(ok && !(khw && vhw)) == 0;
    if (!ok) continue;  // a token's four lanes share ok: reductions read active lanes only
    const int64_t tile = page * a.Hkv + h;
    // The lane's K chunk g and V byte of (dim 16 g, row off); every other store of the
    // head is at a compile-time distance from these (fp8_v_offset(16 c + dl, off, D) =
    // dl * D + (off / 4) * (D / 4) + 4 c + off % 4), so one address serves them all.
    uint8_t* kp = a.k_pool + tile * (int64_t)D * 16 + (g * 16 + off) * 16;
    uint8_t* vp = a.v_pool + tile * (int64_t)D * 16 + fp8_v_offset(16 * g, off, D);
    auto put = [&](bool kh, bool vh) {
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        uint32_t w[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          w[u] = encode4(kx[j][4 * u] * ksf, kx[j][4 * u + 1] * ksf, kx[j][4 * u + 2] * ksf,
                         kx[j][4 * u + 3] * ksf, kh);
        *reinterpret_cast<uint4*>(kp + j * 4 * 16 * 16) = make_uint4(w[0], w[1], w[2], w[3]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t v4 = encode4(vx[j][4 * u] * vsf, vx[j][4 * u + 1] * vsf,
                                      vx[j][4 * u + 2] * vsf, vx[j][4 * u + 3] * vsf, vh);
#pragma unroll
          for (int e = 0; e < 4; ++e) vp[(4 * u + e) * D + 16 * j] = (uint8_t)(v4 >> (8 * e));
        }
      }
    };
    if (all_hw)
      put(true, true);
    else
      put(khw, vhw);
    if (g == 0) {
      a.k_scale[tile * 16 + off] = ksf;
      a.v_scale[tile * 16 + off] = vsf;
    }
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

template <typename E>
struct alignas(16) Out16 {
  E e[16];
};

// The same gather on 16-byte aligned pools and outputs: grid (position block of 16, group
// of H kv heads, sequence), H x D threads, D per kv head.  Thread t of a head takes row
// t / (D/16) and 16-dim chunk t % (D/16) of the block's K and of its V: the K chunk is one 16-byte load (the K tile order keeps
// a row's chunk contiguous); the V tile (16 x D codes in the FP8 V order) is staged in
// LDS with one 16-byte load per thread and read back in row order.  All loads of a thread
// are issued before the barrier.  Codes are decoded and divided by the row's factor in
// float32, as gather8_kernel does, and each chunk is stored as 16 contiguous outputs
// (consecutive threads: consecutive chunks of a row, so a wave stores whole rows).
// Rows past the context or on an invalid page are stored as zeros without loads.
// (C2's batch into fp16: 279 -> 154 us.  The gather is bound by its zero-padded output:
// one reciprocal per row with an FMA correction per element instead of the division
// measured 159 us, a bare multiply 158 us.)
template <typename E, int D, int H>
__global__ __launch_bounds__(1024) void gather8_vec_kernel(Gather8Args a) {
  constexpr int NC = D / 16;
  constexpr int64_t kTile = 16 * D;
  __shared__ uint4 s_v[H][D];  // the V tiles: D 16-byte chunks per kv head
  const int blk = blockIdx.x, b = blockIdx.z;
  const int hl = threadIdx.x / D, t = threadIdx.x - hl * D;
  const int h = blockIdx.y * H + hl;
  const int L = a.ctx[b];
  const int64_t page = blk < a.max_blocks ? (int64_t)a.bt[(int64_t)b * a.max_blocks + blk] : -1;
  const bool page_ok = page >= 0 && page < a.num_pages && h < a.Hkv;
  const int64_t tile = (page_ok ? page * a.Hkv + h : 0);
  const int rows = h < a.Hkv ? min(16, a.out_len - blk * 16) : 0;
  const int live = page_ok ? max(0, min(rows, L - blk * 16)) : 0;  // uniform per kv head
  const int r = t / NC, c = t - r * NC;
  const bool has = r < live;
  uint4 kw = make_uint4(0, 0, 0, 0);
  float ksf = 1.f, vsf = 1.f;
  if (live > 0) {
    s_v[hl][t] = reinterpret_cast<const uint4*>(a.v_pool + tile * kTile)[t];
    if (has) {
      kw = *reinterpret_cast<const uint4*>(a.k_pool + tile * kTile + (c * 16 + r) * 16);
      ksf = a.k_scale[tile * 16 + r];
      vsf = a.v_scale[tile * 16 + r];
    }
  }
  __syncthreads();
  if (r >= rows) return;
  const uint8_t* sv = reinterpret_cast<const uint8_t*>(s_v[hl]);
  const uint8_t* kb = reinterpret_cast<const uint8_t*>(&kw);
  Out16<E> ko, vo;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    ko.e[i] = (E)(has ? e4m3_decode(kb[i]) / ksf : 0.f);
    vo.e[i] = (E)(has ? e4m3_decode(sv[fp8_v_offset(16 * c + i, r, D)]) / vsf : 0.f);
  }
  const int64_t o = (((int64_t)b * a.Hkv + h) * a.out_len + blk * 16 + r) * D + 16 * c;
  *reinterpret_cast<Out16<E>*>(static_cast<E*>(a.k_out) + o) = ko;
  *reinterpret_cast<Out16<E>*>(static_cast<E*>(a.v_out) + o) = vo;
}

}  // namespace
}  // namespace ivakv

using namespace ivakv;

namespace {

// kv heads per workgroup of the FP8 gather (C2's batch: 1 / 2 / 4 / 8 heads 165 / 157 /
// 154 / 166 us)
constexpr int kGather8Heads = 4;

// Shared checks and launch of the two FP8 appends (positions == nullptr: no RoPE).
constexpr int kFewAppend8Tokens = 512;
int append8_entry(const char* name, const void* k_new, const void* v_new, int64_t k_tok_stride,
                  int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
                  void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                  const int32_t* slot_mapping, const int32_t* positions, bool rope, int n_tok,
                  int num_kv_heads, int head_dim, int block_size, int num_pages, float theta,
                  int dtype, hipStream_t stream) {
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (n_tok < 0 || num_kv_heads <= 0 || num_pages < 0)
    return fail(IVAKV_E_ARG, "%s: bad sizes n_tok=%d Hkv=%d num_pages=%d", name, n_tok,
                num_kv_heads, num_pages);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IVAKV_E_SHAPE, "%s: head_dim %d not in {64,128,256}", name, head_dim);
  if (block_size != 16) return fail(IVAKV_E_SHAPE, "%s: block_size %d != 16", name, block_size);
  if (rope && !(theta > 0.f)) return fail(IVAKV_E_ARG, "%s: theta must be positive", name);
  if (n_tok == 0) return IVAKV_OK;
  if (!k_new || !v_new || !k_pool || !v_pool || !k_scale || !v_scale || !slot_mapping ||
      (rope && !positions))
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (k_tok_stride < 0 || k_head_stride < 0 || v_tok_stride < 0 || v_head_stride < 0)
    return fail(IVAKV_E_ARG, "%s: negative stride", name);
  Append8Args a{k_new, v_new, k_tok_stride, k_head_stride, v_tok_stride, v_head_stride,
                static_cast<uint8_t*>(k_pool), static_cast<uint8_t*>(v_pool), k_scale, v_scale,
                slot_mapping, positions, n_tok, num_kv_heads, (int64_t)num_pages * 16, theta};
  // Every kv head in one workgroup when the tokens alone fill the device (the RoPE
  // angles are then computed once per token); else one kv head per wave, and for a
  // few rows without RoPE (decode steps) one wave per workgroup, so the stores spread
  // over more CUs (32 rows of 8 heads: 6.2 -> 3.8 us, 256 rows 7.2 -> 4.6 us; with
  // RoPE the angle table each workgroup computes costs what that gains).
  const bool one_wave = !rope && n_tok < kFewAppend8Tokens;
  const dim3 grid((unsigned)cdiv(n_tok, 16),
                  n_tok >= 2048 ? 1u : (unsigned)cdiv(num_kv_heads, one_wave ? 1 : 4));
#define IVAKV_APPEND8(E, R)                                                                      \
  switch (head_dim) {                                                                            \
    case 64:                                                                                     \
      if (one_wave) append8_kernel<E, 64, R, 1><<<grid, 64, 0, stream>>>(a);                     \
      else append8_kernel<E, 64, R, 4><<<grid, 256, 0, stream>>>(a);                             \
      break;                                                                                     \
    case 128:                                                                                    \
      if (one_wave) append8_kernel<E, 128, R, 1><<<grid, 64, 0, stream>>>(a);                    \
      else append8_kernel<E, 128, R, 4><<<grid, 256, 0, stream>>>(a);                            \
      break;                                                                                     \
    default:                                                                                     \
      if (one_wave) append8_kernel<E, 256, R, 1><<<grid, 64, 0, stream>>>(a);                    \
      else append8_kernel<E, 256, R, 4><<<grid, 256, 0, stream>>>(a);                            \
      break;                                                                                     \
  }
#define IVAKV_APPEND8_DT(R)                                                         \
  switch (dtype) {                                                                  \
    case IVAKV_F16: IVAKV_APPEND8(_Float16, R); break;                              \
    case IVAKV_BF16: IVAKV_APPEND8(__bf16, R); break;                               \
    default: IVAKV_APPEND8(float, R); break;                                        \
  }
  if (rope) {
    IVAKV_APPEND8_DT(true);
  } else {
    IVAKV_APPEND8_DT(false);
  }
#undef IVAKV_APPEND8_DT
#undef IVAKV_APPEND8
  return launch_status(name);
}

}  // namespace

extern "C" int ivakv_append_fp8(const void* k_new, const void* v_new, int64_t k_tok_stride,
                                int64_t k_head_stride, int64_t v_tok_stride,
                                int64_t v_head_stride, void* k_pool, void* v_pool, float* k_scale,
                                float* v_scale, const int32_t* slot_mapping, int n_tok,
                                int num_kv_heads, int head_dim, int block_size, int num_pages,
                                int dtype, hipStream_t stream) {
  return append8_entry("ivakv_append_fp8", k_new, v_new, k_tok_stride, k_head_stride,
                       v_tok_stride, v_head_stride, k_pool, v_pool, k_scale, v_scale,
                       slot_mapping, nullptr, false, n_tok, num_kv_heads, head_dim, block_size,
                       num_pages, 1.f, dtype, stream);
}

extern "C" int ivakv_append_rope_fp8(const void* k_new, const void* v_new, int64_t k_tok_stride,
                                     int64_t k_head_stride, int64_t v_tok_stride,
                                     int64_t v_head_stride, void* k_pool, void* v_pool,
                                     float* k_scale, float* v_scale, const int32_t* slot_mapping,
                                     const int32_t* positions, int n_tok, int num_kv_heads,
                                     int head_dim, int block_size, int num_pages, float theta,
                                     int dtype, hipStream_t stream) {
  return append8_entry("ivakv_append_rope_fp8", k_new, v_new, k_tok_stride, k_head_stride,
                       v_tok_stride, v_head_stride, k_pool, v_pool, k_scale, v_scale,
                       slot_mapping, positions, true, n_tok, num_kv_heads, head_dim, block_size,
                       num_pages, theta, dtype, stream);
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
  if (aligned16(k_pool) && aligned16(v_pool) && aligned16(k_out) && aligned16(v_out)) {
    constexpr int kH = kGather8Heads;
    const dim3 vgrid((unsigned)cdiv(out_len, 16), (unsigned)cdiv(num_kv_heads, kH), (unsigned)batch);
#define IVAKV_GATHER8_VEC(E)                                                                \
  switch (head_dim) {                                                                       \
    case 64: gather8_vec_kernel<E, 64, kH><<<vgrid, 64 * kH, 0, stream>>>(a); break;        \
    case 128: gather8_vec_kernel<E, 128, kH><<<vgrid, 128 * kH, 0, stream>>>(a); break;     \
    default: gather8_vec_kernel<E, 256, kH><<<vgrid, 256 * kH, 0, stream>>>(a); break;      \
  }
    switch (dtype) {
      case IVAKV_F16: IVAKV_GATHER8_VEC(_Float16); break;
      case IVAKV_BF16: IVAKV_GATHER8_VEC(__bf16); break;
      default: IVAKV_GATHER8_VEC(float); break;
    }
#undef IVAKV_GATHER8_VEC
    return launch_status(name);
  }
  switch (dtype) {
    case IVAKV_F16: gather8_kernel<_Float16><<<grid, 256, 0, stream>>>(a); break;
    case IVAKV_BF16: gather8_kernel<__bf16><<<grid, 256, 0, stream>>>(a); break;
    default: gather8_kernel<float><<<grid, 256, 0, stream>>>(a); break;
  }
  return launch_status(name);
}
