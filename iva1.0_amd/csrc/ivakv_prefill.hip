// Paged multi-query causal attention (prefill and chunked prefill) for gfx950.
//
// Sequence b contributes n_b query rows (a chunk of new tokens whose K/V are
// already in the pages) at absolute positions L_b - n_b .. L_b - 1, L_b =
// context_lens[b].  Query row i at position p attends to the keys j <= p that
// lie in the sliding window (j > p - window) or among the first n_sink
// positions, over the sequence's paged K/V; query head h*G + g reads kv head h.
//
// Work split: the query rows of one (sequence, kv head) are flattened
// position-major over the G heads of the group, r = i*G + g, so a block of 16
// rows spans as few positions as possible (tight causal ranges).  A workgroup
// of 4 waves takes 4*16*NR consecutive rows; each wave walks the pages its own
// rows can see, two pages (32 keys) at a time, through a 2-deep ring of
// register buffers:
//   S^T[key][row]  = K_page(16 x D) . Q^T(D x 16)        v_mfma 16x16x32, per page
//   O^T[dim][row] += V^T_pair(D x 32) . P^T(32 x 16)     v_mfma 16x16x32, per pair
// The QK accumulator of lane l holds keys 4*(l/16)+r of row l%16 for each page
// of the pair; those 8 values are exactly the k-slots of the PV MFMA's B
// operand (slot 8*(l/16)+r = page A key 4*(l/16)+r, slot +4 = page B key), and
// the V chunks of the two pages are paired the same way, so P never leaves
// registers.  Online softmax in fp32, log2 domain, as in the decode kernel.
#include "ivakv_tile.h"

namespace ivakv {
namespace {

constexpr int kPfWaves = 4;
constexpr int kPfThreads = 64 * kPfWaves;

struct PrefillArgs {
  const void* q;  // [n_tok, Hq, D], rows of sequence b at query_start[b] ..
  const void* k_pool;
  const void* v_pool;
  void* out;      // like q
  int batch, Hkv, G, max_blocks, num_pages;
  float scale_log2;
  int window, n_sink;
};

// Rows per workgroup of the kernel instance for head_dim D.
template <int D>
struct PrefillShape {
  static constexpr int NR = D <= 128 ? 2 : 1;  // 16-row blocks per wave
  static constexpr int kRowsWave = 16 * NR;
  static constexpr int kRowsWG = kRowsWave * kPfWaves;
};

template <int DT, int D>
__global__ __launch_bounds__(kPfThreads) void prefill_kernel(PrefillArgs a,
                                                             const int32_t* __restrict__ bt,
                                                             const int32_t* __restrict__ ctx,
                                                             const int32_t* __restrict__ qstart) {
  using Tr = Traits<DT>;
  using E = typename Tr::E;
  using VChunk = typename Tr::VChunk;
  constexpr int X = 16 / (int)sizeof(E);
  constexpr int KLD = D / X / 4;  // 16-byte K loads per lane per page
  constexpr int NB = D / 16;      // 16-dim blocks
  constexpr int NR = PrefillShape<D>::NR;
  constexpr int64_t kTile = (int64_t)D * kBS;

  const int h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63, ln = lane & 15, lq = lane >> 4;
  const int wave = uni(threadIdx.x >> 6);
  const int G = a.G, Hkv = a.Hkv, Hq = Hkv * G;
  const int q0 = qstart[b];
  const int n = qstart[b + 1] - q0;
  const int L = ctx[b];
  const int rows = n * G;
  const int r_w = blockIdx.x * PrefillShape<D>::kRowsWG + wave * PrefillShape<D>::kRowsWave;
  if (n <= 0 || r_w >= rows) return;
  const int first_pos = L - n;  // position of query row 0 of the chunk
  const int r_last = min(r_w + PrefillShape<D>::kRowsWave, rows) - 1;
  const int p_lo = max(first_pos + r_w / G, 0);
  const int p_hi = first_pos + r_last / G;

  // Keys any row of the wave can see: positions <= p_hi, from p_lo - window + 1
  // on, plus the sinks.  (All rows before position 0: nothing to walk.)
  const PageWalk w = make_walk(p_hi >= 0 ? p_hi + 1 : 0, a.window > 0 ? a.window + (p_hi - p_lo) : 0,
                               a.n_sink, kBS);
  const int n_eff = table_pages(w, a.max_blocks, kBS);

  // Query rows of the lane (column ln of each row block).  Rows past the chunk
  // or before position 0 see no key; their loads are clamped to row 0.
  int qpos[NR];
  Chunk16 qr[NR][KLD];
#pragma unroll
  for (int rb = 0; rb < NR; ++rb) {
    const int r = r_w + 16 * rb + ln;
    const int pos = first_pos + r / G;
    qpos[rb] = (r < rows && pos >= 0) ? pos : -1;
    const int rc = r < rows ? r : 0;
    const E* qb = static_cast<const E*>(a.q) + ((int64_t)(q0 + rc / G) * Hq + h * G + rc % G) * D;
#pragma unroll
    for (int j = 0; j < KLD; ++j) qr[rb][j] = *reinterpret_cast<const Chunk16*>(qb + (4 * j + lq) * X);
  }

  f32x4 acc[NR][NB];
  float m_run[NR], l_run[NR];
#pragma unroll
  for (int rb = 0; rb < NR; ++rb) {
#pragma unroll
    for (int m = 0; m < NB; ++m) acc[rb][m] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run[rb] = kNegInf;
    l_run[rb] = 0.f;
  }

  // Ring of two page pairs.  Effective pages past n_eff are clamped to the last
  // one (an L2 hit) and fully masked, so the loop body carries no branch around
  // the loads.
  Chunk16 kb[2][2][KLD];
  VChunk vb[2][2][NB];
  int lp_buf[2][2];
  bool ok_buf[2][2];
  auto issue = [&](int s, int pair) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int v = 2 * pair + half;
      const int vc = v < n_eff ? v : n_eff - 1;
      const int lp = logical_page(w, vc);
      const int64_t pp = bt[(int64_t)b * a.max_blocks + lp];
      const bool ok = v < n_eff && pp >= 0 && pp < a.num_pages;
      lp_buf[s][half] = lp;
      ok_buf[s][half] = ok;
      const int64_t tile = (((pp >= 0 && pp < a.num_pages) ? pp : 0) * Hkv + h) * kTile;
      const E* kp = static_cast<const E*>(a.k_pool) + tile;
      const E* vp = static_cast<const E*>(a.v_pool) + tile;
#pragma unroll
      for (int j = 0; j < KLD; ++j)
        kb[s][half][j] = *reinterpret_cast<const Chunk16*>(kp + ((4 * j + lq) * kBS + ln) * X);
#pragma unroll
      for (int m = 0; m < NB; ++m)
        vb[s][half][m] = *reinterpret_cast<const VChunk*>(vp + (16 * m + ln) * kBS + 4 * lq);
    }
    __asm__ volatile("" ::: "memory");
  };

  auto compute = [&](int s) {
    // V rows outside the context (tail of the last page, invalid pages) may hold
    // any bits; zero them (0 * NaN would poison the accumulator).
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      bool vrow[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) vrow[r] = ok_buf[s][half] && lp_buf[s][half] * kBS + 4 * lq + r < L;
#pragma unroll
      for (int m = 0; m < NB; ++m) Tr::mask_rows(vb[s][half][m], vrow);
    }
#pragma unroll
    for (int rb = 0; rb < NR; ++rb) {
      f32x4 sa = f32x4{0.f, 0.f, 0.f, 0.f}, sb = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KLD; ++j) {
        sa = Tr::qk(kb[s][0][j], qr[rb][j], sa);
        sb = Tr::qk(kb[s][1][j], qr[rb][j], sb);
      }
      const int qp = qpos[rb];
      float pa[4], pb[4], sl[8];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ka = lp_buf[s][0] * kBS + 4 * lq + r;
        const int kb_ = lp_buf[s][1] * kBS + 4 * lq + r;
        const bool va = ok_buf[s][0] && ka <= qp && (a.window <= 0 || ka > qp - a.window || ka < a.n_sink);
        const bool vb_ = ok_buf[s][1] && kb_ <= qp && (a.window <= 0 || kb_ > qp - a.window || kb_ < a.n_sink);
        sl[r] = va ? sa[r] * a.scale_log2 : kNegInf;
        sl[4 + r] = vb_ ? sb[r] * a.scale_log2 : kNegInf;
      }
      float mx = sl[0];
#pragma unroll
      for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sl[i]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run[rb], mx);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      const float alpha = exp2_fast(m_run[rb] - m_use);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = exp2_fast(sl[r] - m_use);
        pb[r] = exp2_fast(sl[4 + r] - m_use);
      }
      l_run[rb] = l_run[rb] * alpha + (((pa[0] + pa[1]) + (pa[2] + pa[3])) +
                                       ((pb[0] + pb[1]) + (pb[2] + pb[3])));
      m_run[rb] = m_new;
      const typename Tr::P8 p8 = Tr::pack_p8(pa, pb);
#pragma unroll
      for (int m = 0; m < NB; ++m) acc[rb][m] = Tr::pv32(vb[s][0][m], vb[s][1][m], p8, acc[rb][m] * alpha);
    }
  };

  if (n_eff > 0) {
    const int n_pairs = (n_eff + 1) / 2;
    issue(0, 0);
    issue(1, 1);
    for (int pi = 0; pi < n_pairs; pi += 2) {
      compute(0);
      issue(0, pi + 2);
      compute(1);
      issue(1, pi + 3);
    }
  }

  // O = acc / l, rows of this lane's column; the row sum is split over the 4 k-groups.
#pragma unroll
  for (int rb = 0; rb < NR; ++rb) {
    float l = l_run[rb] + __shfl_xor(l_run[rb], 16);
    l = l + __shfl_xor(l, 32);
    const int r = r_w + 16 * rb + ln;
    if (r < rows) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      E* o = static_cast<E*>(a.out) + ((int64_t)(q0 + r / G) * Hq + h * G + r % G) * D + 4 * lq;
#pragma unroll
      for (int m = 0; m < NB; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[16 * m + i] = Tr::from_float(acc[rb][m][i] * inv);
    }
  }
}

template <int DT>
void launch_prefill(int head_dim, dim3 grid, hipStream_t stream, const PrefillArgs& a,
                    const int32_t* bt, const int32_t* ctx, const int32_t* qs) {
  switch (head_dim) {
    case 64: prefill_kernel<DT, 64><<<grid, kPfThreads, 0, stream>>>(a, bt, ctx, qs); break;
    case 128: prefill_kernel<DT, 128><<<grid, kPfThreads, 0, stream>>>(a, bt, ctx, qs); break;
    default: prefill_kernel<DT, 256><<<grid, kPfThreads, 0, stream>>>(a, bt, ctx, qs); break;
  }
}

int rows_per_workgroup(int head_dim) {
  switch (head_dim) {
    case 64: return PrefillShape<64>::kRowsWG;
    case 128: return PrefillShape<128>::kRowsWG;
    default: return PrefillShape<256>::kRowsWG;
  }
}

}  // namespace
}  // namespace ivakv

using namespace ivakv;

extern "C" int ivakv_prefill_attn(const void* q, const void* k_pool, const void* v_pool,
                                  const int32_t* block_tables, const int32_t* context_lens,
                                  const int32_t* query_start, void* out, int batch,
                                  int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                  int max_blocks, int num_pages, int max_query_len, float scale,
                                  int window, int n_sink, int dtype, hipStream_t stream) {
  static const char* name = "ivakv_prefill_attn";
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_blocks < 0 || max_query_len < 0)
    return fail(IVAKV_E_ARG, "%s: bad sizes B=%d Hq=%d Hkv=%d max_blocks=%d max_query_len=%d",
                name, batch, num_q_heads, num_kv_heads, max_blocks, max_query_len);
  if (num_q_heads % num_kv_heads != 0)
    return fail(IVAKV_E_SHAPE, "%s: num_q_heads %d not a multiple of num_kv_heads %d", name,
                num_q_heads, num_kv_heads);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IVAKV_E_SHAPE, "%s: head_dim %d not in {64,128,256}", name, head_dim);
  if (block_size != kBS)
    return fail(IVAKV_E_SHAPE, "%s: block_size %d != %d", name, block_size, kBS);
  if (n_sink < 0) return fail(IVAKV_E_ARG, "%s: negative n_sink", name);
  if (batch == 0 || max_query_len == 0) return IVAKV_OK;
  if (num_pages < 1) return fail(IVAKV_E_ARG, "%s: num_pages must be >= 1", name);
  if (!q || !k_pool || !v_pool || !context_lens || !query_start || !out ||
      (max_blocks > 0 && !block_tables))
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (!aligned16(q) || !aligned16(k_pool) || !aligned16(v_pool) || !aligned16(out))
    return fail(IVAKV_E_ARG, "%s: q, pools and out must be 16-byte aligned", name);
  if (batch > 65535 || num_kv_heads > 65535)
    return fail(IVAKV_E_SHAPE, "%s: batch and num_kv_heads must be <= 65535", name);
  if (!(scale == scale)) return fail(IVAKV_E_ARG, "%s: scale is NaN", name);
  const int G = num_q_heads / num_kv_heads;
  const int64_t rows = (int64_t)max_query_len * G;
  const int64_t blocks_x = (rows + rows_per_workgroup(head_dim) - 1) / rows_per_workgroup(head_dim);
  if (blocks_x > 0x7fffffff) return fail(IVAKV_E_SHAPE, "%s: max_query_len too large", name);

  PrefillArgs a;
  a.q = q;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.out = out;
  a.batch = batch;
  a.Hkv = num_kv_heads;
  a.G = G;
  a.max_blocks = max_blocks;
  a.num_pages = num_pages;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  a.window = window > 0 ? window : 0;
  a.n_sink = n_sink;
  const dim3 grid((unsigned)blocks_x, (unsigned)num_kv_heads, (unsigned)batch);
  switch (dtype) {
    case IVAKV_F16: launch_prefill<IVAKV_F16>(head_dim, grid, stream, a, block_tables, context_lens, query_start); break;
    case IVAKV_BF16: launch_prefill<IVAKV_BF16>(head_dim, grid, stream, a, block_tables, context_lens, query_start); break;
    default: launch_prefill<IVAKV_F32>(head_dim, grid, stream, a, block_tables, context_lens, query_start); break;
  }
  return launch_status(name);
}
