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
// of W waves takes 32*W consecutive rows (two 16-row blocks per wave) and walks
// the pages its rows can see two at a time (32 keys):
// the pair's K and V tiles move HBM -> registers -> an LDS ring (eight buffers
// for the pipelined loop, two otherwise) once per workgroup, and every wave
// reads them from LDS in MFMA operand order (the pools' tile layout is kept in
// LDS):
//   S^T[key][row]  = K_page(16 x D) . Q^T(D x 16)        v_mfma 16x16x32, per page
//   O^T[dim][row] += V^T_pair(D x 32) . P^T(32 x 16)     v_mfma 16x16x32, per pair
// The QK accumulator of lane l holds keys 4*(l/16)+r of row l%16 for each page
// of the pair; those 8 values are exactly the k-slots of the PV MFMA's B
// operand (slot 8*(l/16)+r = page A key 4*(l/16)+r, slot +4 = page B key), and
// the V chunks of the two pages are paired the same way, so P never leaves
// registers.  Online softmax in fp32, log2 domain, as in the decode kernel.
// A wave skips pairs that lie entirely after its last row; only the pairs on
// its causal diagonal (or window edge, or the context's end) need masks.
//
// FP8 pages (kFp8): the staging loads e4m3fn codes (half the bytes) and their
// per-key scaling factors, and the LDS store converts them, code * (1 / sf) in
// fp32 rounded once to the query dtype, into the same LDS layout; the loop over
// pairs is the 16-bit one.  8-byte units (8 dims of one key of K, or 4 keys of
// two dims of V) spread the conversion over all threads.
#include "ivakv_tile.h"

namespace ivakv {
namespace {

// Log2-domain headroom of the lazy row max: p = exp2(s - m) stays <= 2^8, well
// inside fp16 / bf16 range.
constexpr float kLazyMax = 8.f;

struct PrefillArgs {
  const void* q;  // [n_tok, Hq, D], rows of sequence b at query_start[b] ..
  const void* k_pool;
  const void* v_pool;
  void* out;      // like q
  int n_tok;      // rows of q and out
  int batch, Hkv, G, max_blocks, num_pages;
  float scale_log2;
  int window, n_sink;
  int blocks_x;  // row-block workgroups per (sequence, kv head)
  const float* k_scale;  // FP8 pools: [num_pages][Hkv][16] fp32 scaling factors
  const float* v_scale;
  // Split walks: partial slots [slot][rows_wg][D] (acc) and [slot][rows_wg][2]
  // (running max, row sum) of the split workspace.
  float* part_acc;
  float* part_ml;
};

// Shape of the kernel instance.  fp16 / bf16 up to head_dim 128: 8 waves of
// two 16-row blocks (two waves per SIMD, under 256 registers each, so one
// wave's softmax overlaps the other's MFMAs) and two pairs in flight in
// registers; fp32 and head_dim 256: 4 waves (one per SIMD, the accumulator in
// AGPRs) and one pair in flight.
template <int DT, int D>
struct PrefillShape {
  static constexpr int kESize = DT == IVAKV_F32 ? 4 : 2;
  static constexpr int kWaves = (DT == IVAKV_F32 || D == 256) ? 4 : 8;
  static constexpr int kThreads = 64 * kWaves;
  // Row blocks per wave; one for fp32 at head_dim 256, whose q rows and accumulators
  // for two blocks would not fit 512 registers.
  static constexpr int NR = (DT == IVAKV_F32 && D == 256) ? 1 : 2;
  static constexpr int kStages = kWaves == 8 ? 2 : 1;  // pairs in flight in registers
  static constexpr int kRowsWave = 16 * NR;
  static constexpr int kRowsWG = kRowsWave * kWaves;
  static constexpr int kPageElems = kBS * D;          // one K or V page tile
  static constexpr int kPairElems = 4 * kPageElems;   // K_A, K_B, V_A, V_B
  // LDS pair buffers: eight for the pipelined loop (two stage sets; it needs five,
  // and a power of two makes the ring index a mask), else two.
  static constexpr int kBufs = kStages == 2 ? 8 : 2;
  static constexpr size_t kLdsBytes = kBufs * (size_t)kPairElems * kESize;
};

// Geometry of row block xb (rows xb * rows_wg ..) of sequence b: its rows, positions
// and the page walk that covers every key any of its rows can see.  ok is false
// when the block has no row to compute (a sequence whose rows do not lie inside q,
// an empty chunk, a block past the chunk's rows).
struct RowBlock {
  bool ok;
  int q0, rows, L, first_pos, r_wg;
  PageWalk w;
  int n_eff, n_pairs;  // effective pages of the walk, and pairs of them (32 keys)
};

__device__ inline RowBlock row_block(const PrefillArgs& a, const int32_t* ctx, const int32_t* qstart,
                                     int b, int xb, int rows_wg) {
  RowBlock rb;
  rb.ok = false;
  // The sequence's rows [q0, q1) must lie inside q / out; a range that does not is
  // skipped (its rows are not written).
  const int64_t q0l = qstart[b], q1l = qstart[b + 1];
  if (q0l < 0 || q1l <= q0l || q1l > a.n_tok) return rb;
  const int n = (int)(q1l - q0l);
  rb.q0 = (int)q0l;
  rb.L = ctx[b];
  rb.rows = n * a.G;
  rb.r_wg = xb * rows_wg;
  if (rb.r_wg >= rb.rows) return rb;
  rb.first_pos = rb.L - n;  // position of query row 0 of the chunk
  // Keys any row of the block can see: positions <= p_hi, from p_lo - window + 1 on,
  // plus the sinks.  (All rows before position 0: nothing to walk.)
  const int p_lo = max(rb.first_pos + rb.r_wg / a.G, 0);
  const int p_hi = rb.first_pos + (min(rb.r_wg + rows_wg, rb.rows) - 1) / a.G;
  rb.w = make_walk(p_hi >= 0 ? p_hi + 1 : 0, a.window > 0 ? a.window + (p_hi - p_lo) : 0,
                   a.n_sink, kBS);
  rb.n_eff = table_pages(rb.w, a.max_blocks, kBS);
  rb.n_pairs = (rb.n_eff + 1) / 2;
  rb.ok = true;
  return rb;
}

// Row block xb of (sequence b, kv head h) over pairs [pair_lo, pair_hi) of its walk
// (pair_lo even).  slot < 0: the block's whole walk, normalized rows into out; slot
// >= 0: one segment of a split walk, its unnormalized rows (acc, running max, row sum)
// into partial slot `slot` of the split workspace, for merge_rows.  Every
// thread of the workgroup calls it with the same arguments (the returns and barriers
// inside are uniform).
template <int DT, int D, bool kFp8>
__device__ __attribute__((always_inline)) inline void prefill_rows(
    const PrefillArgs& a, const int32_t* __restrict__ bt, const int32_t* __restrict__ ctx,
    const int32_t* __restrict__ qstart, int b, int h, int xb, int pair_lo, int pair_hi, int slot) {
  using Tr = Traits<DT>;
  using E = typename Tr::E;
  using S = PrefillShape<DT, D>;
  constexpr int X = 16 / (int)sizeof(E);
  constexpr int KLD = D / X / 4;  // 16-byte K reads per lane per page
  constexpr int NB = D / 16;      // 16-dim blocks
  constexpr int NR = S::NR;
  constexpr int64_t kTile = (int64_t)D * kBS;
  extern __shared__ Chunk16 lds[];  // 2 x [K_A | K_B | V_A | V_B], global tile layout

  const int tid = threadIdx.x;
  const int lane = tid & 63, ln = lane & 15, lq = lane >> 4;
  const int wave = uni(tid >> 6);
  const int G = a.G, Hkv = a.Hkv, Hq = Hkv * G;
  const RowBlock blk = row_block(a, ctx, qstart, b, xb, S::kRowsWG);
  if (!blk.ok) return;  // uniform over the workgroup
  const int q0 = blk.q0, L = blk.L, rows = blk.rows, r_wg = blk.r_wg, first_pos = blk.first_pos;
  const PageWalk w = blk.w;
  const int n_eff = blk.n_eff;
  // This call's pairs: [p0, n_pairs) with n_pairs the segment's end.
  const int n_pairs = min(blk.n_pairs, pair_hi);
  const int p0 = pair_lo;
  // Pages loads may touch: the segment's (loads past its last pair repeat its last
  // page, an L2 hit).
  const int v_end = min(n_eff, 2 * n_pairs);

  // This wave's rows: the last position any of them has (pairs entirely past it
  // are skipped) and, per lane, the position of row ln of each block.
  const int r_w = r_wg + wave * S::kRowsWave;
  const int wave_p_hi = r_w < rows ? first_pos + (min(r_w + S::kRowsWave, rows) - 1) / G : -1;
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
  // Scores are kept raw (q.k) and scaled inside the exponent, exp2(s*c - m), with
  // c = |scale * log2(e)| > 0; a negative scale negates q instead (exact), so
  // max(s*c) = c*max(s) always holds.  (A zero scale uses the smallest normal c.)
  const float c_log2 = fmaxf(fabsf(a.scale_log2), 1.17549435e-38f);
  if (a.scale_log2 < 0.f) {
    const uint32_t sign = sizeof(E) == 2 ? 0x80008000u : 0x80000000u;
#pragma unroll
    for (int rb = 0; rb < NR; ++rb)
#pragma unroll
      for (int j = 0; j < KLD; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) qr[rb][j].w[i] ^= sign;
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

  // Pair staging, HBM -> registers -> LDS.  An LDS buffer holds
  //   [K_A | K_B]  the two K tiles in the pools' layout (16-byte chunks), and
  //   V pair       row d (32 keys) = granules A0 B0 A1 B1 A2 B2 A3 B3, granule
  //                Pg = keys 4g..4g+3 of page P (4 elements),
  // so a lane's PV operand (granule lq of page A and of page B for dim d) is one
  // contiguous 2-granule read and a wave's V reads are conflict-free.  Thread
  // tid moves 16-byte LDS chunks tid + T*c of each part.  Pages past n_eff are
  // clamped to the last one (masked later); invalid ids read page 0.
  constexpr int kPageChunks = S::kPageElems * (int)sizeof(E) / 16;
  constexpr int kGran = 4 * (int)sizeof(E);  // bytes of one V granule
  constexpr int kKPer = (2 * kPageChunks + S::kThreads - 1) / S::kThreads;
  constexpr int kVPer = kKPer;               // the V pair has as many 16-byte chunks
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 stK[S::kStages][kKPer], stV[S::kStages][kVPer];  // vector types: kept in registers
  // Page ids.  Lanes fetch the block-table entries of a pair two loads ahead
  // with vector loads (no scalar-memory wait inside a step: the scalar and LDS
  // counters are shared), into the slot of the pair's parity; load() moves them
  // to scalar registers and records each page's validity (id in range, page
  // inside the walk) in okmask, bits 2 (pair % 16) and + 1, which the pair's
  // step reads.  Pages past n_eff are the last one (masked later); invalid ids
  // read page 0.
  auto lpage = [&](int v) IVAKV_INLINE -> int { return logical_page(w, v < v_end ? v : v_end - 1); };
  const int32_t* bt_row = bt + (int64_t)b * a.max_blocks;
  int ids_a[2], ids_b[2];
  uint32_t okmask = 0;
  auto fetch_ids = [&](int pair, int par) IVAKV_INLINE {
    int z = 0;
    asm volatile("" : "+v"(z));  // a vector-register offset: a vector load
    ids_a[par] = bt_row[lpage(2 * pair) + z];
    ids_b[par] = bt_row[lpage(2 * pair + 1) + z];
  };
  auto take_ids = [&](int pair, int par, int64_t& pa, int64_t& pb) IVAKV_INLINE {
    const int ia = __builtin_amdgcn_readfirstlane(ids_a[par]);
    const int ib = __builtin_amdgcn_readfirstlane(ids_b[par]);
    const bool va = ia >= 0 && ia < a.num_pages, vb = ib >= 0 && ib < a.num_pages;
    const int sh = 2 * (pair & 15);
    okmask = (okmask & ~(3u << sh)) | ((uint32_t)(va && 2 * pair < n_eff) << sh) |
             ((uint32_t)(vb && 2 * pair + 1 < n_eff) << (sh + 1));
    pa = va ? ia : 0;
    pb = vb ? ib : 0;
  };
  auto pair_ok = [&](int pair) IVAKV_INLINE -> uint32_t { return (okmask >> (2 * (pair & 15))) & 3u; };
  auto load_pair = [&](int pair, int set, int par) IVAKV_INLINE {
    int64_t pa, pb;
    take_ids(pair, par, pa, pb);
    const E* kpa = static_cast<const E*>(a.k_pool) + (pa * Hkv + h) * kTile;
    const E* kpb = static_cast<const E*>(a.k_pool) + (pb * Hkv + h) * kTile;
    const E* vpa = static_cast<const E*>(a.v_pool) + (pa * Hkv + h) * kTile;
    const E* vpb = static_cast<const E*>(a.v_pool) + (pb * Hkv + h) * kTile;
#pragma unroll
    for (int c = 0; c < kKPer; ++c) {
      const int idx = min(tid + S::kThreads * c, 2 * kPageChunks - 1);
      const E* src = idx < kPageChunks ? kpa : kpb;
      stK[set][c] = *reinterpret_cast<const u32x4*>(src + (idx % kPageChunks) * (16 / (int)sizeof(E)));
    }
#pragma unroll
    for (int c = 0; c < kVPer; ++c) {
      const int v = min(tid + S::kThreads * c, 2 * kPageChunks - 1);
      if constexpr (kGran == 8) {  // 16-bit: chunk v = row v/4, granule v%4 of A and B
        const int off = (v >> 2) * kBS + 4 * (v & 3);
        const u32x2 ga = *reinterpret_cast<const u32x2*>(vpa + off);
        const u32x2 gb = *reinterpret_cast<const u32x2*>(vpb + off);
        stV[set][c] = u32x4{ga[0], ga[1], gb[0], gb[1]};
      } else {  // fp32: chunk v = row v/8, granule (v%8)/2 of page v%2
        const int off = (v >> 3) * kBS + 4 * ((v & 7) >> 1);
        stV[set][c] = *reinterpret_cast<const u32x4*>(((v & 1) ? vpb : vpa) + off);
      }
    }
    fetch_ids(pair + 2, par);
  };
  // V values of keys no row may see (past the context, on an invalid page) are
  // zeroed as the pair enters LDS, once for the whole workgroup: 0 * NaN would
  // poison the PV accumulator.  Only a pair that reaches past the context or
  // holds an invalid page takes this branch.
  auto pair_needs_vmask = [&](int pair) IVAKV_INLINE -> bool {
    return pair_ok(pair) != 3u || lpage(2 * pair + 1) * kBS + kBS > L;
  };
  auto v_keys_ok = [&](int pair, int pg, int g, bool (&vis)[4]) IVAKV_INLINE {
    const bool page_ok = ((pair_ok(pair) >> pg) & 1u) != 0;
    const int k0 = lpage(2 * pair + pg) * kBS + 4 * g;
#pragma unroll
    for (int r = 0; r < 4; ++r) vis[r] = page_ok && k0 + r < L;
  };
  auto store_pair = [&](int buf, int set, int pair) IVAKV_INLINE {
    u32x4* dk = reinterpret_cast<u32x4*>(lds + buf * (4 * kPageChunks));
    u32x4* dv = dk + 2 * kPageChunks;
    if (pair_needs_vmask(pair)) {
#pragma unroll
      for (int c = 0; c < kVPer; ++c) {
        const int v = min(tid + S::kThreads * c, 2 * kPageChunks - 1);
        if constexpr (kGran == 8) {  // granule v%4 of pages A and B
          bool va[4], vb[4];
          v_keys_ok(pair, 0, v & 3, va);
          v_keys_ok(pair, 1, v & 3, vb);
          Chunk16 ch = __builtin_bit_cast(Chunk16, stV[set][c]);
          mask_pair16(ch, va, vb);
          stV[set][c] = __builtin_bit_cast(u32x4, ch);
        } else {  // granule (v%8)/2 of page v%2
          bool vis[4];
          v_keys_ok(pair, v & 1, (v & 7) >> 1, vis);
#pragma unroll
          for (int r = 0; r < 4; ++r) stV[set][c][r] = vis[r] ? stV[set][c][r] : 0u;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < kKPer; ++c)
      if ((2 * kPageChunks) % S::kThreads == 0 || tid + S::kThreads * c < 2 * kPageChunks)
        dk[tid + S::kThreads * c] = stK[set][c];
#pragma unroll
    for (int c = 0; c < kVPer; ++c)
      if ((2 * kPageChunks) % S::kThreads == 0 || tid + S::kThreads * c < 2 * kPageChunks)
        dv[tid + S::kThreads * c] = stV[set][c];
  };

  // FP8 staging.  A pair holds 4D 8-byte units of K codes and as many of V codes
  // (units [0, 2D) page A, [2D, 4D) page B).  K unit j of a page: codes of dims
  // 16(j/32) + 8(j%2) .. +8 of key (j/2)%16, which become the 16-bit pool layout's
  // chunk (2(j/32) + j%2)*16 + key.  V unit j: words 2j, 2j+1 of the tile's FP8
  // order [d%16][key/4][d/16][key%4] (ivakv_internal.h fp8_v_offset), i.e. keys
  // 4g..4g+3 of dims dl + 16m and dl + 16(m+1), which become granule (g, page) of
  // those two LDS V rows.
  constexpr int kUnits = 4 * D;                                  // per pair, K or V
  constexpr int kU8 = kFp8 ? (kUnits + S::kThreads - 1) / S::kThreads : 1;
  constexpr int kNB8 = D / 16;
  u32x2 st8K[S::kStages][kU8], st8V[S::kStages][kU8];
  float sc8K[S::kStages][kU8];
  f32x4 sc8V[S::kStages][kU8];
  auto load_pair8 = [&](int pair, int set, int par) IVAKV_INLINE {
    if constexpr (kFp8) {
    int64_t pa, pb;
    take_ids(pair, par, pa, pb);
    const int64_t tA = pa * Hkv + h, tB = pb * Hkv + h;
    const uint8_t* k8 = static_cast<const uint8_t*>(a.k_pool);
    const uint8_t* v8 = static_cast<const uint8_t*>(a.v_pool);
#pragma unroll
    for (int c = 0; c < kU8; ++c) {
      const int u = min(tid + S::kThreads * c, kUnits - 1);
      const int64_t t = u < 2 * D ? tA : tB;
      const int j = u % (2 * D);
      st8K[set][c] = *reinterpret_cast<const u32x2*>(k8 + t * kTile + 8 * j);
      sc8K[set][c] = a.k_scale[t * kBS + ((j >> 1) & 15)];
      st8V[set][c] = *reinterpret_cast<const u32x2*>(v8 + t * kTile + 8 * j);
      sc8V[set][c] = *reinterpret_cast<const f32x4*>(a.v_scale + t * kBS + 4 * (((2 * j) / kNB8) & 3));
    }
    fetch_ids(pair + 2, par);
    }
  };
  // Four codes (one 32-bit word) times four factors, as four values of E.
  auto dequant4 = [&](uint32_t w, float s0, float s1, float s2, float s3) IVAKV_INLINE -> u32x2 {
    if constexpr (kFp8) {
      const f32x2 lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false);
      const f32x2 hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, true);
      return u32x2{Tr::pack2(lo[0] * s0, lo[1] * s1), Tr::pack2(hi[0] * s2, hi[1] * s3)};
    } else {
      return u32x2{0u, 0u};
    }
  };
  auto store_pair8 = [&](int buf, int set, int pair) IVAKV_INLINE {
    if constexpr (kFp8) {
    u32x4* dk = reinterpret_cast<u32x4*>(lds + buf * (4 * kPageChunks));
    u32x2* dv = reinterpret_cast<u32x2*>(dk + 2 * kPageChunks);  // V rows of 8 granules
#pragma unroll
    for (int c = 0; c < kU8; ++c) {
      if (kUnits % S::kThreads != 0 && tid + S::kThreads * c >= kUnits) continue;
      const int u = tid + S::kThreads * c;
      const int pg = u < 2 * D ? 0 : 1, j = u % (2 * D);
      // K: one key's 8 dims, one 16-byte LDS chunk
      const float ik = __builtin_amdgcn_rcpf(sc8K[set][c]);
      const u32x2 k0 = dequant4(st8K[set][c][0], ik, ik, ik, ik);
      const u32x2 k1 = dequant4(st8K[set][c][1], ik, ik, ik, ik);
      const int key = (j >> 1) & 15, ch = (2 * (j >> 5) + (j & 1)) * 16 + key;
      dk[pg * kPageChunks + ch] = u32x4{k0[0], k0[1], k1[0], k1[1]};
      // V: keys 4g..4g+3 of two dims, one 8-byte granule in each of two rows
      const f32x4 sv = sc8V[set][c];
      const float i0 = __builtin_amdgcn_rcpf(sv[0]), i1 = __builtin_amdgcn_rcpf(sv[1]);
      const float i2 = __builtin_amdgcn_rcpf(sv[2]), i3 = __builtin_amdgcn_rcpf(sv[3]);
      const int w0 = 2 * j, m = w0 % kNB8, g = (w0 / kNB8) & 3, dl = w0 / (4 * kNB8);
      u32x2 vv[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) vv[e] = dequant4(st8V[set][c][e], i0, i1, i2, i3);
      if (pair_needs_vmask(pair)) {
        bool vis[4];
        v_keys_ok(pair, pg, g, vis);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          Chunk8 h = __builtin_bit_cast(Chunk8, vv[e]);
          mask_rows16(h, vis);
          vv[e] = __builtin_bit_cast(u32x2, h);
        }
      }
#pragma unroll
      for (int e = 0; e < 2; ++e) dv[(dl + 16 * (m + e)) * 8 + 2 * g + pg] = vv[e];
    }
    }
  };
  auto load = [&](int pair, int set, int par) IVAKV_INLINE {
    if constexpr (kFp8) load_pair8(pair, set, par);
    else load_pair(pair, set, par);
  };
  auto store = [&](int buf, int set, int pair) IVAKV_INLINE {
    if constexpr (kFp8) store_pair8(buf, set, pair);
    else store_pair(buf, set, pair);
  };

  // Scores of one pair (pages A, B) for every row block of the wave.
  struct PairS {
    f32x4 sa[NR], sb[NR];
  };
  // A pair past the walk or entirely after every row of the wave is skipped.
  auto pair_live = [&](int pair) IVAKV_INLINE -> bool {
    return pair < n_pairs && lpage(2 * pair) * kBS <= wave_p_hi;
  };
  auto read_k = [&](int buf, Chunk16 (&ka)[KLD], Chunk16 (&kb)[KLD]) IVAKV_INLINE {
    const E* kA = reinterpret_cast<const E*>(lds + buf * (4 * kPageChunks));
    const E* kB = kA + S::kPageElems;
#pragma unroll
    for (int j = 0; j < KLD; ++j) {
      ka[j] = *reinterpret_cast<const Chunk16*>(kA + ((4 * j + lq) * kBS + ln) * X);
      kb[j] = *reinterpret_cast<const Chunk16*>(kB + ((4 * j + lq) * kBS + ln) * X);
    }
  };
  using VPair = typename Tr::VPair;
  auto read_v = [&](int buf, VPair (&vp)[NB]) IVAKV_INLINE {
    const char* vP = reinterpret_cast<const char*>(lds + buf * (4 * kPageChunks) + 2 * kPageChunks);
#pragma unroll
    for (int m = 0; m < NB; ++m) vp[m] = Tr::read_vpair(vP + (16 * m + ln) * (8 * kGran) + lq * (2 * kGran));
  };
  auto qk_mfma = [&](const Chunk16 (&ka)[KLD], const Chunk16 (&kb)[KLD], PairS& sc) IVAKV_INLINE {
#pragma unroll
    for (int rb = 0; rb < NR; ++rb) {
      sc.sa[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
      sc.sb[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KLD; ++j) {
        sc.sa[rb] = Tr::qk(ka[j], qr[rb][j], sc.sa[rb]);
        sc.sb[rb] = Tr::qk(kb[j], qr[rb][j], sc.sb[rb]);
      }
    }
  };
  auto qk_pair = [&](int buf, PairS& sc) IVAKV_INLINE {
    Chunk16 ka[KLD], kb[KLD];
    read_k(buf, ka, kb);
    qk_mfma(ka, kb, sc);
  };
  // This lane's 8 scores of row block rb (keys 4lq.. of page A, then of page B).
  auto lane_scores = [&](const PairS& sc, int rb, float (&sl)[8]) IVAKV_INLINE {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sl[r] = sc.sa[rb][r];
      sl[4 + r] = sc.sb[rb][r];
    }
  };
  auto scaled_max = [&](const float (&sl)[8]) IVAKV_INLINE -> float {
    float lmx = sl[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) lmx = fmaxf(lmx, sl[i]);
    return lmx * c_log2;
  };
  // Lazy rescaling: the reference max m_run of a row (log2 units) only moves
  // (with a cross-lane max and a rescale of acc and l) when a scaled score exceeds
  // it by more than kLazyMax; otherwise p = exp2(s*c - m_run) <= 2^kLazyMax and
  // the final O = acc / l is unchanged.
  auto grows = [&](int rb, float lmx) IVAKV_INLINE -> bool { return lmx > m_run[rb] + kLazyMax; };
  auto rescale = [&](int rb, float lmx) IVAKV_INLINE {
    if (__builtin_amdgcn_ballot_w64(grows(rb, lmx)) != 0) {
      float mx = fmaxf(lmx, __shfl_xor(lmx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run[rb], mx);
      const float alpha = m_new == kNegInf ? 1.f : exp2_fast(m_run[rb] - m_new);
      l_run[rb] *= alpha;
#pragma unroll
      for (int m = 0; m < NB; ++m) acc[rb][m] *= alpha;
      m_run[rb] = m_new;
    }
  };
  // p = exp2(s*c - m_run) of the lane's 8 scores, their sum into l, PV.
  auto exp_pv = [&](int rb, const float (&sl)[8], const VPair (&vp)[NB]) IVAKV_INLINE {
    const float m_use = m_run[rb] == kNegInf ? 0.f : m_run[rb];
    float pa[4], pb[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pa[r] = exp2_fast(__builtin_fmaf(sl[r], c_log2, -m_use));
      pb[r] = exp2_fast(__builtin_fmaf(sl[4 + r], c_log2, -m_use));
    }
    l_run[rb] += ((pa[0] + pa[1]) + (pa[2] + pa[3])) + ((pb[0] + pb[1]) + (pb[2] + pb[3]));
    const typename Tr::PP8 p8 = Tr::pack_pp8(pa, pb);
#pragma unroll
    for (int m = 0; m < NB; ++m) acc[rb][m] = Tr::pv_pair(vp[m], p8, acc[rb][m]);
  };
  // Masks of a pair that is not interior for this wave, applied to its scores in
  // place: keys a row must not see (after its position, outside its window and
  // not a sink, past the context, on an invalid page) get score -inf.
  auto mask_scores = [&](int pair, PairS& sc) IVAKV_INLINE {
    const uint32_t ok = pair_ok(pair);
    const bool oka = (ok & 1u) != 0, okb = (ok & 2u) != 0;
    const int ka0 = lpage(2 * pair) * kBS + 4 * lq, kb0 = lpage(2 * pair + 1) * kBS + 4 * lq;
#pragma unroll
    for (int rb = 0; rb < NR; ++rb) {
      const int qp = qpos[rb];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ka_ = ka0 + r, kb_ = kb0 + r;
        const bool visa = oka && ka_ <= qp && (a.window <= 0 || ka_ > qp - a.window || ka_ < a.n_sink);
        const bool visb = okb && kb_ <= qp && (a.window <= 0 || kb_ > qp - a.window || kb_ < a.n_sink);
        sc.sa[rb][r] = visa ? sc.sa[rb][r] : kNegInf;
        sc.sb[rb][r] = visb ? sc.sb[rb][r] : kNegInf;
      }
    }
  };
  // A pair is interior for this wave when every key is visible to every row of
  // the wave: both pages valid and inside the walk, every key at or before the
  // wave's first row position and inside the window of its last row.  (Rows past
  // the chunk's end read row 0's query, so their scores stay finite; they are
  // never stored.)
  const int wave_pos_lo = first_pos + r_w / G;  // may be negative: then no pair is
  auto interior = [&](int pair) IVAKV_INLINE -> bool {
    return wave_pos_lo >= 0 && pair_ok(pair) == 3u &&
           lpage(2 * pair + 1) * kBS + kBS - 1 <= wave_pos_lo &&
           (a.window <= 0 || lpage(2 * pair) * kBS > wave_p_hi - a.window);
  };
  // Softmax and PV of a pair, with the next pair's QK (with_next): one test for
  // any row max growing (rare), then one block with no branch: the next pair's K
  // reads and QK MFMAs, this pair's V reads, exponentials and PV MFMAs.
  auto softmax_pv = [&](auto with_next, int bn, PairS& sn, int bc, const PairS& sc) IVAKV_INLINE {
    constexpr bool kNext = decltype(with_next)::value;
    float sl[NR][8], lmx[NR];
    bool any = false;
#pragma unroll
    for (int rb = 0; rb < NR; ++rb) {
      lane_scores(sc, rb, sl[rb]);
      lmx[rb] = scaled_max(sl[rb]);
      any = any || grows(rb, lmx[rb]);
    }
    if (__builtin_amdgcn_ballot_w64(any) != 0) {
#pragma unroll
      for (int rb = 0; rb < NR; ++rb) rescale(rb, lmx[rb]);
    }
    if constexpr (kNext) qk_pair(bn, sn);
    VPair vp[NB];
    read_v(bc, vp);
#pragma unroll
    for (int rb = 0; rb < NR; ++rb) exp_pv(rb, sl[rb], vp);
  };
  // One step of the pipelined loop: this pair's softmax + PV and the next pair's
  // QK (a pair past this wave's rows is skipped, and so is every later one; the
  // next pair's QK is harmless when it is not live).
  auto step = [&](int bn, PairS& sn, int bc, int pc, PairS& sc) IVAKV_INLINE {
    if (!pair_live(pc)) return;
    if (!interior(pc)) mask_scores(pc, sc);
    softmax_pv(std::true_type{}, bn, sn, bc, sc);
  };
  // One pair, QK then softmax + PV (the unpipelined loop).
  auto compute = [&](int buf, int pair) IVAKV_INLINE {
    if (!pair_live(pair)) return;
    PairS sc;
    qk_pair(buf, sc);
    if (!interior(pair)) mask_scores(pair, sc);
    softmax_pv(std::false_type{}, buf, sc, buf, sc);
  };

  // Ring: pair i is in LDS buffer i % 2 while pair i + 1 travels from HBM / L2
  // into the staging registers; one barrier per pair.  Page ids are fetched two
  // loads ahead, in the slot of the pair's parity.
  if (n_pairs > p0) {
    fetch_ids(p0, 0);
    fetch_ids(p0 + 1, 1);
    if constexpr (S::kStages == 2) {
      // Software pipeline over eight LDS buffers (pair p in buffer p & 7) and two
      // stage sets (pair p in set p % 2), two steps and one barrier per
      // iteration.  Step i issues the QK MFMAs of pair i + 1, then runs pair i's
      // softmax (on the VALU while those MFMAs execute) and PV.  An iteration
      // (steps i, i + 1) reads pairs i .. i + 2, published by the barrier before
      // it, and stores pairs i + 3 and i + 4 into the buffers of pairs i - 5 and
      // i - 4, which earlier barriers retired; its own barrier publishes them.  Loads
      // (pairs i + 5, i + 6) refill the stage sets just stored.  Loads past the
      // last pair repeat the last page (an L2 hit) into buffers nobody reads;
      // being unconditional keeps the stage in registers.
      PairS s0, s1;
      load(p0, 0, 0);
      load(p0 + 1, 1, 1);
      store(p0 & 7, 0, p0);
      load(p0 + 2, 0, 0);
      store((p0 + 1) & 7, 1, p0 + 1);
      load(p0 + 3, 1, 1);
      store((p0 + 2) & 7, 0, p0 + 2);
      load(p0 + 4, 0, 0);
      __syncthreads();
      if (pair_live(p0)) qk_pair(p0 & 7, s0);
      for (int i = p0; i < n_pairs; i += 2) {
        store((i + 3) & 7, 1, i + 3);
        load(i + 5, 1, 1);
        step((i + 1) & 7, s1, i & 7, i, s0);
        store((i + 4) & 7, 0, i + 4);
        load(i + 6, 0, 0);
        step((i + 2) & 7, s0, (i + 1) & 7, i + 1, s1);
        __syncthreads();
      }
    } else {
      // Two pairs per iteration so that the page-id slot (the pair's parity) is
      // known at compile time; a pair past the walk is skipped.
      load(p0, 0, 0);
      store(0, 0, p0);
      __syncthreads();
      for (int i = p0; i < n_pairs; i += 2) {
        load(i + 1, 0, 1);
        compute(0, i);
        store(1, 0, i + 1);
        __syncthreads();
        load(i + 2, 0, 0);
        compute(1, i + 1);
        store(0, 0, i + 2);
        __syncthreads();
      }
    }
  }

  // O = acc / l, rows of this lane's column; the row sum is split over the 4 k-groups.
  // A segment of a split walk stores acc, the running max and the row sum instead
  // (row r_w + 16 rb + ln - r_wg of the slot).
#pragma unroll
  for (int rb = 0; rb < NR; ++rb) {
    float l = l_run[rb] + __shfl_xor(l_run[rb], 16);
    l = l + __shfl_xor(l, 32);
    const int r = r_w + 16 * rb + ln;
    if (r < rows) {
      if (slot >= 0) {
        const int64_t pr = (int64_t)slot * S::kRowsWG + (r - r_wg);
        float* po = a.part_acc + pr * D + 4 * lq;
#pragma unroll
        for (int m = 0; m < NB; ++m) *reinterpret_cast<f32x4*>(po + 16 * m) = acc[rb][m];
        if (lq == 0) *reinterpret_cast<f32x2*>(a.part_ml + 2 * pr) = f32x2{m_run[rb], l};
      } else {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        E* o = static_cast<E*>(a.out) + ((int64_t)(q0 + r / G) * Hq + h * G + r % G) * D + 4 * lq;
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[16 * m + i] = Tr::from_float(acc[rb][m][i] * inv);
      }
    }
  }
}

// One workgroup per row block, in XCD-aware order: the dispatcher deals workgroup
// ids round-robin to the 8 XCDs, so unit u = (sequence, kv head) gets ids == u % 8
// (mod 8) and all its row blocks run on one XCD, close in time: its pages come from
// HBM once per XCD and are L2 hits for the other row blocks.  A unit's row blocks go
// last first: later rows see more keys, so the longest blocks are dispatched first
// and the shortest fill the tail.
template <int DT, int D, bool kFp8>
__global__ __launch_bounds__((PrefillShape<DT, D>::kThreads)) void prefill_kernel(PrefillArgs a,
                                                             const int32_t* __restrict__ bt,
                                                             const int32_t* __restrict__ ctx,
                                                             const int32_t* __restrict__ qstart) {
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int unit = (slot / a.blocks_x) * 8 + xcd;
  if (unit >= a.batch * a.Hkv) return;
  const int b = unit / a.Hkv, h = unit % a.Hkv;
  const int xb = a.blocks_x - 1 - slot % a.blocks_x;
  prefill_rows<DT, D, kFp8>(a, bt, ctx, qstart, b, h, xb, 0, 0x7fffffff, -1);
}

// ---------------------------------------------------------------------------
// Split walks (ivakv_prefill_attn_split).  A row block walks every pair its rows can
// see, so a chunk late in a long context is one workgroup's serial walk: a single
// 512-token chunk at 16k keys fills 64 of 256 CUs.  The split path cuts each row
// block's walk into segments of seg_pairs pairs, sized so that the batch's work
// spreads over every CU (seg_pairs ~ total pairs / CUs), runs (row block, segment)
// items on a persistent grid that takes them from per-XCD queues, and merges the
// segments of each split row block by log-sum-exp.  Two launches:
//   prefill_plan_kernel   one workgroup: segment size, the item queues (longest
//                         sequences first), partial slots, and the queues' and the
//                         split blocks' counters reset to zero (so the workspace needs
//                         no initialisation);
//   prefill_split_kernel  one workgroup per CU, items until its XCD's queue is empty;
//                         the workgroup that completes a split block's last segment
//                         merges the block's partials into out.
// ---------------------------------------------------------------------------

// Partial slots (row-block segments) the split workspace holds; the plan doubles the
// segment length until the split row blocks fit.
constexpr int kSplitSlots = 512;
// Shortest segment, in pairs of pages (32 keys each); even, as the pair loop needs.
constexpr int kSplitMinPairs = 16;
// The plan ranks the sequences by their longest row block in LDS, up to this batch
// (the split path's largest batch), and keeps the row blocks' pair counts in LDS up to
// kPlanCache row blocks (more: in the workspace).
constexpr int kPlanMaxBatch = 2048;
constexpr int kPlanSortBatch = 256;
constexpr int kPlanCache = 8192;
constexpr int kPlanThreads = 256;

// Split workspace.  ctl: [0] virtual units V, [1] split row blocks, [2] segment
// length in pairs, [3] partial slots used, [32 + 4x] the queue counter of XCD x.  A virtual unit (sequence b,
// kv head h, segment s) is packed (b | h << 16, s); the queue of XCD x holds virtual
// units x, x + 8, ... and a ticket j of it is row block blocks_x - 1 - j % blocks_x of
// unit x + 8 (j / blocks_x).  rb[b * blocks_x + xb] = (first slot, segments) of a
// split row block ((-1, 1) unsplit, (-1, 0) no rows); the slot of segment s of kv
// head h is first + h * segments + s; arrive[first] counts that block's finished
// segments.
struct SplitWs {
  int32_t* ctl;
  int2* vus;       // [batch * Hkv + kSplitSlots]
  int2* rb;        // [batch * blocks_x]
  int32_t* arrive; // [kSplitSlots]
  float* acc;      // [kSplitSlots][rows_wg][D]
  float* ml;       // [kSplitSlots][rows_wg][2]
};

// Byte layout of the split workspace (each part 256-byte aligned).
struct SplitLayout {
  size_t ctl, vus, rb, arrive, acc, ml, total;
};
inline SplitLayout split_layout(int batch, int num_kv_heads, int blocks_x, int rows_wg, int head_dim) {
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  SplitLayout l;
  l.ctl = 0;
  l.vus = up(l.ctl + 64 * sizeof(int32_t));
  l.rb = up(l.vus + ((size_t)batch * num_kv_heads + kSplitSlots) * sizeof(int2));
  l.arrive = up(l.rb + (size_t)batch * blocks_x * sizeof(int2));
  l.acc = up(l.arrive + (size_t)kSplitSlots * sizeof(int32_t));
  l.ml = up(l.acc + (size_t)kSplitSlots * rows_wg * head_dim * sizeof(float));
  l.total = up(l.ml + (size_t)kSplitSlots * rows_wg * 2 * sizeof(float));
  return l;
}

// Sum of v over the workgroup (kPlanThreads threads), returned to every thread.
__device__ inline int64_t plan_sum(int64_t v, int64_t* s_red64) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int lo = __shfl_xor((int)(uint32_t)v, off), hi = __shfl_xor((int)(v >> 32), off);
    v += (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
  }
  const int wv = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) s_red64[wv] = v;
  __syncthreads();
  int64_t t = 0;
  for (int i = 0; i < kPlanThreads / 64; ++i) t += s_red64[i];
  return t;
}

// Exclusive prefix of v over the workgroup in thread order; *total gets the sum.
__device__ inline int plan_scan(int v, int* s_red, int* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(incl, off);
    if (lane >= off) incl += u;
  }
  __syncthreads();
  if (lane == 63) s_red[wv] = incl;
  __syncthreads();
  int before = 0, t = 0;
  for (int i = 0; i < kPlanThreads / 64; ++i) {
    before += i < wv ? s_red[i] : 0;
    t += s_red[i];
  }
  *total = t;
  return before + incl - v;
}

// Segments of a row block of n pairs (one when it is not split).
__device__ inline int n_segments(int n_pairs, int seg) { return n_pairs > seg ? (n_pairs + seg - 1) / seg : 1; }

__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(PrefillArgs a,
                                                                    const int32_t* __restrict__ ctx,
                                                                    const int32_t* __restrict__ qstart,
                                                                    SplitWs ws, int rows_wg, int n_cu) {
  __shared__ int s_red[kPlanThreads / 64];
  __shared__ int64_t s_red64[kPlanThreads / 64];
  __shared__ int s_key[kPlanMaxBatch];   // longest row block (pairs) per sequence, -1: none
  __shared__ int s_order[kPlanMaxBatch];  // sequences by rank
  __shared__ int s_pref[kPlanMaxBatch + 1];
  __shared__ int s_np[kPlanCache];        // pairs of row block e (-1: no rows)
  const int tid = threadIdx.x;
  const int B = a.batch, Hkv = a.Hkv, BX = a.blocks_x;
  const int E = B * BX;
  const bool cached = E <= kPlanCache;
  // Row block e's pair count, written and read by the thread of e in every pass.
  auto np_of = [&](int e) -> int { return cached ? s_np[e] : ws.rb[e].x; };
  for (int b = tid; b < B; b += kPlanThreads) s_key[b] = -1;
  __syncthreads();
  // 1. Pairs of every row block, the batch's total and each sequence's longest block.
  int64_t part = 0;
  for (int e = tid; e < E; e += kPlanThreads) {
    const RowBlock blk = row_block(a, ctx, qstart, e / BX, e % BX, rows_wg);
    const int np = blk.ok ? blk.n_pairs : -1;
    if (cached) s_np[e] = np;
    else ws.rb[e].x = np;
    if (blk.ok) {
      part += np;
      atomicMax(&s_key[e / BX], np);
    }
  }
  const int64_t total = plan_sum(part, s_red64) * Hkv;
  // 2. Segment length: the work of one CU, at least kSplitMinPairs, even; doubled
  //    until the split row blocks' segments fit the slots.
  int seg = (int)min<int64_t>((total + n_cu - 1) / n_cu, 1 << 28);
  seg = max(kSplitMinPairs, (seg + 1) & ~1);
  for (;;) {
    int64_t need = 0;
    for (int e = tid; e < E; e += kPlanThreads) {
      const int np = np_of(e);
      if (np > seg) need += n_segments(np, seg);
    }
    if (plan_sum(need, s_red64) * Hkv <= kSplitSlots) break;
    seg *= 2;
  }
  // 3. Sequences by their longest row block, longest first (ties by index): the
  //    queues then hold the longest items first.  (A larger batch keeps its order:
  //    the ranking is quadratic.)
  for (int b = tid; b < B; b += kPlanThreads) {
    int r = b;
    if (B <= kPlanSortBatch) {
      const int kb = s_key[b];
      r = 0;
      for (int o = 0; o < B; ++o) {
        const int ko = s_key[o];
        r += (ko > kb || (ko == kb && o < b)) ? 1 : 0;
      }
    }
    s_order[r] = b;
  }
  __syncthreads();
  // 4. Virtual units in rank order: every kv head of every segment of the sequence
  //    (none for a sequence without rows).  Unit g goes to the queue of XCD g % 8.
  int V = 0;
  for (int r0 = 0; r0 < B; r0 += kPlanThreads) {
    const int r = r0 + tid;
    int cnt = 0;
    if (r < B) {
      const int kb = s_key[s_order[r]];
      cnt = kb < 0 ? 0 : Hkv * (kb > seg ? (kb + seg - 1) / seg : 1);
    }
    int chunk;
    const int ex = plan_scan(cnt, s_red, &chunk);
    if (r < B) s_pref[r] = V + ex;
    V += chunk;
  }
  if (tid == 0) s_pref[B] = V;
  __syncthreads();
  for (int g = tid; g < V; g += kPlanThreads) {
    int lo = 0, hi = B;  // last r with s_pref[r] <= g
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_pref[mid] <= g) lo = mid;
      else hi = mid;
    }
    const int b = s_order[lo], local = g - s_pref[lo];
    ws.vus[g] = int2{b | ((local % Hkv) << 16), local / Hkv};
  }
  // 5. Slots of the split row blocks, in (sequence, row block) order.
  int slot0 = 0, n_split = 0;
  for (int e0 = 0; e0 < E; e0 += kPlanThreads) {
    const int e = e0 + tid;
    const int np = e < E ? np_of(e) : -1;
    const int ns = np > seg ? n_segments(np, seg) : 0;
    int t_slots;
    const int ex_slots = plan_scan(Hkv * ns, s_red, &t_slots);
    if (e < E) ws.rb[e] = ns > 0 ? int2{slot0 + ex_slots, ns} : int2{-1, np < 0 ? 0 : 1};
    n_split += ns > 0 ? 1 : 0;
    slot0 += t_slots;
  }
  n_split = (int)plan_sum(n_split, s_red64);
  if (tid == 0) {
    ws.ctl[0] = V;
    ws.ctl[1] = n_split;
    ws.ctl[2] = seg;
    ws.ctl[3] = slot0;
  }
  if (tid < 8) ws.ctl[32 + 4 * tid] = 0;
  for (int i = tid; i < kSplitSlots; i += kPlanThreads) ws.arrive[i] = 0;
}

// Log-sum-exp merge of the n_seg segments (partial slots first ..) of row block blk of
// kv head h into out, by the whole workgroup.  A thread takes EG f32x4 elements (rows
// x 4 dims) at once and folds their segments U at a time, so EG * U partial loads are
// in flight per step rather than one element's.
template <int DT, int D>
__device__ inline void merge_rows(const PrefillArgs& a, const SplitWs& ws, const RowBlock& blk,
                                  int h, int first, int n_seg, int rows_wg) {
  using Tr = Traits<DT>;
  using E = typename Tr::E;
  constexpr int DV = D / 4;
  constexpr int EG = D == 256 ? 2 : 4;
  constexpr int U = 4;
  const int G = a.G, Hq = a.Hkv * G;
  const int n_el = rows_wg * DV, nt = blockDim.x;
  for (int t0 = threadIdx.x; t0 < n_el; t0 += EG * nt) {
    float M[EG], L[EG];
    f32x4 O[EG];
#pragma unroll
    for (int k = 0; k < EG; ++k) {
      M[k] = kNegInf;
      L[k] = 0.f;
      O[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int s0 = 0; s0 < n_seg; s0 += U) {
      float mv[EG][U], lv[EG][U];
      f32x4 ov[EG][U];
#pragma unroll
      for (int k = 0; k < EG; ++k) {
        const int t = min(t0 + k * nt, n_el - 1);
        const int rl = t / DV, d4 = 4 * (t % DV);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t pr = (int64_t)(first + min(s0 + u, n_seg - 1)) * rows_wg + rl;
          mv[k][u] = ws.ml[pr * 2];
          lv[k][u] = ws.ml[pr * 2 + 1];
          ov[k][u] = *reinterpret_cast<const f32x4*>(ws.acc + pr * D + d4);
        }
      }
#pragma unroll
      for (int k = 0; k < EG; ++k) {
        float mc = M[k];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          mv[k][u] = s0 + u < n_seg ? mv[k][u] : kNegInf;
          mc = fmaxf(mc, mv[k][u]);
        }
        const float m_use = mc == kNegInf ? 0.f : mc;
        const float f = exp2_fast(M[k] - m_use);
        L[k] *= f;
        O[k] *= f;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float w = exp2_fast(mv[k][u] - m_use);
          L[k] += lv[k][u] * w;
          O[k] += ov[k][u] * w;
        }
        M[k] = mc;
      }
    }
#pragma unroll
    for (int k = 0; k < EG; ++k) {
      const int t = t0 + k * nt;
      const int rl = t / DV, d4 = 4 * (t % DV);
      const int r = blk.r_wg + rl;
      if (t >= n_el || r >= blk.rows) continue;
      const float inv = L[k] > 0.f ? 1.f / L[k] : 0.f;
      E* o = static_cast<E*>(a.out) + ((int64_t)(blk.q0 + r / G) * Hq + h * G + r % G) * D + d4;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = Tr::from_float(O[k][i] * inv);
    }
  }
}

// Persistent grid of the split path: workgroup w serves the queue of XCD w % 8 (the
// dispatcher deals workgroup ids round-robin to the XCDs, so a unit's row blocks and
// segments share one L2), taking tickets from the queue's counter until it is empty.
template <int DT, int D, bool kFp8>
__global__ __launch_bounds__((PrefillShape<DT, D>::kThreads)) void prefill_split_kernel(
    PrefillArgs a, const int32_t* __restrict__ bt, const int32_t* __restrict__ ctx,
    const int32_t* __restrict__ qstart, SplitWs ws) {
  using S = PrefillShape<DT, D>;
  __shared__ int s_ticket[2];
  __shared__ int s_last;
  const int x = blockIdx.x & 7;
  // (V is at most the unit list's capacity; the clamp keeps every list read inside it.)
  const int V = min(ws.ctl[0], a.batch * a.Hkv + kSplitSlots), seg = max(ws.ctl[2], 2);
  const int tickets = (V > x ? (V - x + 7) / 8 : 0) * a.blocks_x;
  int* counter = ws.ctl + 32 + 4 * x;
  for (int it = 0;; ++it) {
    // Two ticket cells used in turn: a thread may still read the last ticket while
    // thread 0 writes the next one.
    if (threadIdx.x == 0)
      s_ticket[it & 1] = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    const int j = s_ticket[it & 1];
    if (j >= tickets) break;  // uniform
    const int2 vu = ws.vus[x + 8 * (j / a.blocks_x)];
    const int xb = a.blocks_x - 1 - j % a.blocks_x;
    const int b = vu.x & 0xffff, h = vu.x >> 16, s = vu.y;
    const int2 rb = ws.rb[b * a.blocks_x + xb];
    if (s >= rb.y) continue;  // the block has no rows, or fewer segments
    if (rb.y == 1) {
      prefill_rows<DT, D, kFp8>(a, bt, ctx, qstart, b, h, xb, 0, 0x7fffffff, -1);
      continue;
    }
    prefill_rows<DT, D, kFp8>(a, bt, ctx, qstart, b, h, xb, s * seg, (s + 1) * seg,
                              rb.x + h * rb.y + s);
    // Count the segment in: every wave waits until its partial stores have reached this
    // XCD's L2 (the barrier alone waits only for LDS traffic), then thread 0's
    // agent-scope release writes them back where the other XCDs read, and the arrival
    // is counted.  The workgroup that counts the last segment acquires (drops its
    // L2's stale lines) and merges the block.  (The item is read again from its
    // ticket, which stays in LDS until the next one: nothing of it stays live across
    // the walk.)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int2 vu2 = ws.vus[x + 8 * (s_ticket[it & 1] / a.blocks_x)];
    const int xb2 = a.blocks_x - 1 - s_ticket[it & 1] % a.blocks_x;
    const int b2 = vu2.x & 0xffff, h2 = vu2.x >> 16;
    const int2 rb2 = ws.rb[b2 * a.blocks_x + xb2];
    const int first = rb2.x + h2 * rb2.y;
    if (threadIdx.x == 0) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      s_last = __hip_atomic_fetch_add(ws.arrive + first, 1, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == rb2.y - 1;
    }
    __syncthreads();
    if (s_last) {  // uniform
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      const RowBlock blk = row_block(a, ctx, qstart, b2, xb2, S::kRowsWG);
      merge_rows<DT, D>(a, ws, blk, h2, first, rb2.y, S::kRowsWG);
    }
  }
}

template <int DT, int D, bool kFp8>
void launch_prefill_d(dim3 grid, hipStream_t stream, const PrefillArgs& a, const int32_t* bt,
                      const int32_t* ctx, const int32_t* qs) {
  // LDS beyond 64 KiB (fp32 with head_dim 256) must be allowed per kernel once.
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&prefill_kernel<DT, D, kFp8>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)PrefillShape<DT, D>::kLdsBytes);
  (void)attr;
  prefill_kernel<DT, D, kFp8><<<grid, PrefillShape<DT, D>::kThreads, PrefillShape<DT, D>::kLdsBytes, stream>>>(a, bt, ctx, qs);
}

template <int DT, bool kFp8 = false>
void launch_prefill(int head_dim, dim3 grid, hipStream_t stream, const PrefillArgs& a,
                    const int32_t* bt, const int32_t* ctx, const int32_t* qs) {
  switch (head_dim) {
    case 64: launch_prefill_d<DT, 64, kFp8>(grid, stream, a, bt, ctx, qs); break;
    case 128: launch_prefill_d<DT, 128, kFp8>(grid, stream, a, bt, ctx, qs); break;
    default: launch_prefill_d<DT, 256, kFp8>(grid, stream, a, bt, ctx, qs); break;
  }
}

// The split path's two launches (see prefill_plan_kernel); n_wg workgroups, a
// multiple of 8, for the persistent kernel.
template <int DT, int D, bool kFp8>
void launch_split_d(int n_wg, hipStream_t stream, const PrefillArgs& a, const int32_t* bt,
                    const int32_t* ctx, const int32_t* qs, const SplitWs& ws) {
  using S = PrefillShape<DT, D>;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&prefill_split_kernel<DT, D, kFp8>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kLdsBytes);
  (void)attr;
  prefill_plan_kernel<<<1, kPlanThreads, 0, stream>>>(a, ctx, qs, ws, S::kRowsWG, n_wg);
  prefill_split_kernel<DT, D, kFp8><<<n_wg, S::kThreads, S::kLdsBytes, stream>>>(a, bt, ctx, qs, ws);
}

template <int DT, bool kFp8 = false>
void launch_split(int head_dim, int n_wg, hipStream_t stream, const PrefillArgs& a,
                  const int32_t* bt, const int32_t* ctx, const int32_t* qs, const SplitWs& ws) {
  switch (head_dim) {
    case 64: launch_split_d<DT, 64, kFp8>(n_wg, stream, a, bt, ctx, qs, ws); break;
    case 128: launch_split_d<DT, 128, kFp8>(n_wg, stream, a, bt, ctx, qs, ws); break;
    default: launch_split_d<DT, 256, kFp8>(n_wg, stream, a, bt, ctx, qs, ws); break;
  }
}

// Workgroups of the split path's persistent grid: one per CU of the current device,
// rounded down to a multiple of the 8 XCD queues.
int split_workgroups() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus = 256;
  return cus >= 16 ? cus & ~7 : 8;
}

template <int DT>
int rows_per_workgroup_t(int head_dim) {
  switch (head_dim) {
    case 64: return PrefillShape<DT, 64>::kRowsWG;
    case 128: return PrefillShape<DT, 128>::kRowsWG;
    default: return PrefillShape<DT, 256>::kRowsWG;
  }
}

int rows_per_workgroup(int dtype, int head_dim) {
  switch (dtype) {
    case IVAKV_F16: return rows_per_workgroup_t<IVAKV_F16>(head_dim);
    case IVAKV_BF16: return rows_per_workgroup_t<IVAKV_BF16>(head_dim);
    default: return rows_per_workgroup_t<IVAKV_F32>(head_dim);
  }
}

int prefill_entry(const char* name, const void* q, const void* k_pool, const void* v_pool,
                  const float* k_scale, const float* v_scale, const int32_t* block_tables,
                  const int32_t* context_lens, const int32_t* query_start, int n_tok, void* out,
                  int batch, int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                  int max_blocks, int num_pages, int max_query_len, float scale, int window,
                  int n_sink, int dtype, hipStream_t stream, bool fp8, bool split = false,
                  void* workspace = nullptr, size_t workspace_bytes = 0) {
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (fp8 && dtype != IVAKV_F16 && dtype != IVAKV_BF16)
    return fail(IVAKV_E_DTYPE, "%s: FP8 pools take fp16 or bf16 queries (dtype %d)", name, dtype);
  if (batch < 0 || n_tok < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_blocks < 0 ||
      max_query_len < 0)
    return fail(IVAKV_E_ARG,
                "%s: bad sizes B=%d n_tok=%d Hq=%d Hkv=%d max_blocks=%d max_query_len=%d", name,
                batch, n_tok, num_q_heads, num_kv_heads, max_blocks, max_query_len);
  if (num_q_heads % num_kv_heads != 0)
    return fail(IVAKV_E_SHAPE, "%s: num_q_heads %d not a multiple of num_kv_heads %d", name,
                num_q_heads, num_kv_heads);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IVAKV_E_SHAPE, "%s: head_dim %d not in {64,128,256}", name, head_dim);
  if (block_size != kBS)
    return fail(IVAKV_E_SHAPE, "%s: block_size %d != %d", name, block_size, kBS);
  if (n_sink < 0) return fail(IVAKV_E_ARG, "%s: negative n_sink", name);
  if (batch == 0 || max_query_len == 0 || n_tok == 0) return IVAKV_OK;
  if (num_pages < 1) return fail(IVAKV_E_ARG, "%s: num_pages must be >= 1", name);
  if (!q || !k_pool || !v_pool || !context_lens || !query_start || !out ||
      (max_blocks > 0 && !block_tables))
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (!aligned16(q) || !aligned16(k_pool) || !aligned16(v_pool) || !aligned16(out))
    return fail(IVAKV_E_ARG, "%s: q, pools and out must be 16-byte aligned", name);
  if (fp8 && (!k_scale || !v_scale || !aligned16(k_scale) || !aligned16(v_scale)))
    return fail(IVAKV_E_ARG, "%s: k_scale / v_scale must be 16-byte aligned device pointers", name);
  if (!(scale == scale)) return fail(IVAKV_E_ARG, "%s: scale is NaN", name);
  const int G = num_q_heads / num_kv_heads;
  const int64_t rows = (int64_t)max_query_len * G;
  const int rows_wg = rows_per_workgroup(dtype, head_dim);
  const int64_t blocks_x = (rows + rows_wg - 1) / rows_wg;
  if (blocks_x > 0x7fffffff) return fail(IVAKV_E_SHAPE, "%s: max_query_len too large", name);

  PrefillArgs a;
  a.q = q;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.out = out;
  a.n_tok = n_tok;
  a.batch = batch;
  a.Hkv = num_kv_heads;
  a.G = G;
  a.max_blocks = max_blocks;
  a.num_pages = num_pages;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  a.window = window > 0 ? window : 0;
  a.n_sink = n_sink;
  a.blocks_x = (int)blocks_x;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.part_acc = nullptr;
  a.part_ml = nullptr;
  if (split) {
    if (batch > kPlanMaxBatch || num_kv_heads > 32767)
      return fail(IVAKV_E_SHAPE, "%s: the split path takes batch <= %d and num_kv_heads <= 32767 "
                  "(got %d, %d); use ivakv_prefill_attn", name, kPlanMaxBatch, batch, num_kv_heads);
    if (((int64_t)batch * num_kv_heads + kSplitSlots) * blocks_x > 0x7fffffff)
      return fail(IVAKV_E_SHAPE, "%s: launch too large", name);
    const SplitLayout lay = split_layout(batch, num_kv_heads, (int)blocks_x, rows_wg, head_dim);
    if (!workspace || workspace_bytes < lay.total || !aligned16(workspace))
      return fail(IVAKV_E_WORKSPACE, "%s: workspace of %zu bytes (16-byte aligned) required, got %zu",
                  name, lay.total, workspace ? workspace_bytes : (size_t)0);
    char* w = static_cast<char*>(workspace);
    SplitWs ws;
    ws.ctl = reinterpret_cast<int32_t*>(w + lay.ctl);
    ws.vus = reinterpret_cast<int2*>(w + lay.vus);
    ws.rb = reinterpret_cast<int2*>(w + lay.rb);
    ws.arrive = reinterpret_cast<int32_t*>(w + lay.arrive);
    ws.acc = reinterpret_cast<float*>(w + lay.acc);
    ws.ml = reinterpret_cast<float*>(w + lay.ml);
    a.part_acc = ws.acc;
    a.part_ml = ws.ml;
    const int n_wg = split_workgroups();
    if (fp8) {
      if (dtype == IVAKV_F16) launch_split<IVAKV_F16, true>(head_dim, n_wg, stream, a, block_tables, context_lens, query_start, ws);
      else launch_split<IVAKV_BF16, true>(head_dim, n_wg, stream, a, block_tables, context_lens, query_start, ws);
      return launch_status(name);
    }
    switch (dtype) {
      case IVAKV_F16: launch_split<IVAKV_F16>(head_dim, n_wg, stream, a, block_tables, context_lens, query_start, ws); break;
      case IVAKV_BF16: launch_split<IVAKV_BF16>(head_dim, n_wg, stream, a, block_tables, context_lens, query_start, ws); break;
      default: launch_split<IVAKV_F32>(head_dim, n_wg, stream, a, block_tables, context_lens, query_start, ws); break;
    }
    return launch_status(name);
  }
  // 1-D grid in XCD-aware order (see prefill_kernel): 8 interleaved unit streams.
  const int64_t units_per_xcd = ((int64_t)batch * num_kv_heads + 7) / 8;
  const int64_t n_wg = units_per_xcd * blocks_x * 8;
  if (n_wg > 0x7fffffff) return fail(IVAKV_E_SHAPE, "%s: launch too large", name);
  const dim3 grid((unsigned)n_wg);
  if (fp8) {
    if (dtype == IVAKV_F16) launch_prefill<IVAKV_F16, true>(head_dim, grid, stream, a, block_tables, context_lens, query_start);
    else launch_prefill<IVAKV_BF16, true>(head_dim, grid, stream, a, block_tables, context_lens, query_start);
    return launch_status(name);
  }
  switch (dtype) {
    case IVAKV_F16: launch_prefill<IVAKV_F16>(head_dim, grid, stream, a, block_tables, context_lens, query_start); break;
    case IVAKV_BF16: launch_prefill<IVAKV_BF16>(head_dim, grid, stream, a, block_tables, context_lens, query_start); break;
    default: launch_prefill<IVAKV_F32>(head_dim, grid, stream, a, block_tables, context_lens, query_start); break;
  }
  return launch_status(name);
}

}  // namespace
}  // namespace ivakv

using namespace ivakv;

extern "C" int ivakv_prefill_attn(const void* q, const void* k_pool, const void* v_pool,
                                  const int32_t* block_tables, const int32_t* context_lens,
                                  const int32_t* query_start, int n_tok, void* out, int batch,
                                  int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                                  int max_blocks, int num_pages, int max_query_len, float scale,
                                  int window, int n_sink, int dtype, hipStream_t stream) {
  return prefill_entry("ivakv_prefill_attn", q, k_pool, v_pool, nullptr, nullptr, block_tables,
                       context_lens, query_start, n_tok, out, batch, num_q_heads, num_kv_heads,
                       head_dim, block_size, max_blocks, num_pages, max_query_len, scale, window,
                       n_sink, dtype, stream, false);
}

extern "C" int ivakv_prefill_attn_fp8(const void* q, const void* k_pool, const void* v_pool,
                                      const float* k_scale, const float* v_scale,
                                      const int32_t* block_tables, const int32_t* context_lens,
                                      const int32_t* query_start, int n_tok, void* out,
                                      int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                      int block_size, int max_blocks, int num_pages,
                                      int max_query_len, float scale, int window, int n_sink,
                                      int dtype, hipStream_t stream) {
  return prefill_entry("ivakv_prefill_attn_fp8", q, k_pool, v_pool, k_scale, v_scale,
                       block_tables, context_lens, query_start, n_tok, out, batch, num_q_heads,
                       num_kv_heads, head_dim, block_size, max_blocks, num_pages, max_query_len,
                       scale, window, n_sink, dtype, stream, true);
}

extern "C" int ivakv_prefill_split_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                                  int head_dim, int max_query_len, int dtype,
                                                  size_t* bytes) {
  if (!bytes) return fail(IVAKV_E_ARG, "ivakv_prefill_split_workspace_size: null bytes");
  *bytes = 0;
  if (dtype_size(dtype) == 0)
    return fail(IVAKV_E_DTYPE, "ivakv_prefill_split_workspace_size: unknown dtype code %d", dtype);
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_query_len < 0 ||
      num_q_heads % num_kv_heads != 0 || (head_dim != 64 && head_dim != 128 && head_dim != 256))
    return fail(IVAKV_E_ARG, "ivakv_prefill_split_workspace_size: bad geometry B=%d Hq=%d Hkv=%d "
                "D=%d max_query_len=%d", batch, num_q_heads, num_kv_heads, head_dim, max_query_len);
  const int rows_wg = rows_per_workgroup(dtype, head_dim);
  const int64_t blocks_x = ((int64_t)max_query_len * (num_q_heads / num_kv_heads) + rows_wg - 1) / rows_wg;
  if (blocks_x > 0x7fffffff)
    return fail(IVAKV_E_SHAPE, "ivakv_prefill_split_workspace_size: max_query_len too large");
  *bytes = split_layout(batch, num_kv_heads, (int)blocks_x, rows_wg, head_dim).total;
  return IVAKV_OK;
}

extern "C" int ivakv_prefill_attn_split(const void* q, const void* k_pool, const void* v_pool,
                                        const int32_t* block_tables, const int32_t* context_lens,
                                        const int32_t* query_start, int n_tok, void* out,
                                        void* workspace, size_t workspace_bytes, int batch,
                                        int num_q_heads, int num_kv_heads, int head_dim,
                                        int block_size, int max_blocks, int num_pages,
                                        int max_query_len, float scale, int window, int n_sink,
                                        int dtype, hipStream_t stream) {
  return prefill_entry("ivakv_prefill_attn_split", q, k_pool, v_pool, nullptr, nullptr,
                       block_tables, context_lens, query_start, n_tok, out, batch, num_q_heads,
                       num_kv_heads, head_dim, block_size, max_blocks, num_pages, max_query_len,
                       scale, window, n_sink, dtype, stream, false, true, workspace,
                       workspace_bytes);
}

extern "C" int ivakv_prefill_attn_split_fp8(const void* q, const void* k_pool, const void* v_pool,
                                            const float* k_scale, const float* v_scale,
                                            const int32_t* block_tables,
                                            const int32_t* context_lens,
                                            const int32_t* query_start, int n_tok, void* out,
                                            void* workspace, size_t workspace_bytes, int batch,
                                            int num_q_heads, int num_kv_heads, int head_dim,
                                            int block_size, int max_blocks, int num_pages,
                                            int max_query_len, float scale, int window,
                                            int n_sink, int dtype, hipStream_t stream) {
  return prefill_entry("ivakv_prefill_attn_split_fp8", q, k_pool, v_pool, k_scale, v_scale,
                       block_tables, context_lens, query_start, n_tok, out, batch, num_q_heads,
                       num_kv_heads, head_dim, block_size, max_blocks, num_pages, max_query_len,
                       scale, window, n_sink, dtype, stream, true, true, workspace,
                       workspace_bytes);
}
