// Paged single-query (decode) attention for gfx950.
//
// One tile = one (page, kv head): 16 rows of K and of V, 2 * 16 * D * esize
// contiguous bytes in the pools.  A wavefront scores a tile for all Hq/Hkv
// query heads of its kv head at once (GQA reuse of every byte loaded).
//
// Per tile a wave issues D/X/4 16-byte K loads and D/16 V loads per lane.  The
// pool layout puts these loads directly in MFMA operand order:
//   S^T[row][head]  = K_page(16 x D) . Q^T(D x 16)      v_mfma 16x16x32 (f16/bf16)
//   O^T[dim][head] += V^T_page(D x 16) . P^T(16 x 16)   v_mfma 16x16x16 (f16/bf16)
// (16x16x4 f32 MFMAs for fp32).  The QK accumulator of lane l holds rows
// 4*(l/16)+r of head l%16, which is exactly the B operand layout the PV MFMA
// wants, so P never leaves registers.  Only heads l%16 < Hq/Hkv carry data.
// Softmax runs online in fp32 in the log2 domain (scale*log2(e) folded into the
// scores, v_exp_f32).
//
// Two walks share that tile code:
//   stream walk (default): a fixed set of waves, sized to
//     what the CUs hold at once, each takes an equal contiguous share of the
//     flattened (sequence, kv head, page) tile list and streams it through a
//     ring of register page buffers, crossing (sequence, kv head) boundaries
//     without draining.  Exact load balance in bytes whatever the context
//     lengths; a unit split between waves leaves one partial per wave that
//     decode_stream_merge_kernel folds together (log-sum-exp).
//   partitioned walk (partition_pages > 0, or a batch too large for the
//     stream walk's page prefix in LDS): grid (kv head, sequence, partition) of 4-wave
//     workgroups; a partition of part_pages pages is split over the 4 waves
//     and merged through LDS, then across partitions by decode_merge_kernel.
#include <type_traits>

#include "ivakv_e4m3.h"
#include "ivakv_tile.h"

namespace ivakv {
namespace {

constexpr int kWaves = 4;     // wavefronts per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kDefaultPartitionPages = 32;
constexpr int kPageBufs = 2;  // register page buffers per wave (ring)
// Workgroups per CU the partitioned walk is built for: two 4-wave groups (2 waves
// per SIMD, up to 256 registers each), or one at head_dim 256, whose two-tile ring
// alone takes 128 (16-bit) or 256 (fp32) registers per lane: one wave per SIMD gets
// 512, so nothing spills to scratch.
constexpr int partial_wgs_per_cu(int D) { return D == 256 ? 1 : 2; }
// Stream walk workgroup: kStreamWaves independent waves, one per SIMD; how many
// workgroups share a CU is a property of the tile operations (Ops::kWGsPerCU).
// Then the wave budget the workspace is sized for, the fewest tiles worth giving
// a wave, and the largest batch whose page prefix fits the workgroup's LDS.
constexpr int kStreamWaves = 4;
constexpr int kStreamThreads = 64 * kStreamWaves;
constexpr int kMaxStreamWaves = 4096;
constexpr int kMinTilesPerWave = 4;
constexpr int kMaxStreamBatch = 8192;
// Stream walk workgroups per CU from the bytes one ring slot holds (K + V of one
// tile).  One 4-wave workgroup per CU keeps 2 x 8 KiB slots per wave in flight at
// D 128 on 16-bit pages, enough to hold HBM busy; 4 KiB slots (D 64 at 16 bits,
// D 128 on FP8 pages) need two workgroups per CU for as many bytes in flight.
// (Deeper rings at one workgroup per CU, 3 or 4 slots of 4 KiB, measured no faster
// on the C2 FP8 walk: 42.0-43.2 against 41.8-42.0 µs per attention.)
constexpr int64_t kWG2SlotBytes = 4096;
constexpr int walk_wgs_per_cu(int64_t slot_bytes) { return slot_bytes <= kWG2SlotBytes ? 2 : 1; }

struct DecodeArgs {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const int32_t* bt;
  const int32_t* ctx;
  void* out;
  float* ws_acc;       // partitioned: [B][Hkv][n_parts_max][G][D]; stream: [slot][G][D]
  float* ws_ml;        // same slots x [G][2]  (max, sum)
  int32_t* ws_pref;    // stream: [B + 1] page prefix of the batch (written by workgroup 0)
  int batch, Hkv, G, max_blocks, num_pages;
  float scale_log2;
  int window, n_sink, part_pages, n_parts_max;
  int n_waves;         // stream: waves launched
  // Fused append (ivakv_decode_append_attn): position L-1 of every sequence is the new
  // token, whose rows come from k_new / v_new ([B][Hkv][D] dense) instead of the pool.
  const void* k_new;
  const void* v_new;
  int fused;
  // FP8 pools: per-(slot, kv head) scaling factors, [num_pages][Hkv][16] fp32.
  const float* k_scale;
  const float* v_scale;
};



// Page walk of a sequence of context length L as the stream walk reads it: with the
// fused append the pool covers positions < L - 1 only (the window and sinks are
// still those of length L); the new token at L - 1 is folded in by the merge.
__device__ inline PageWalk seq_walk(const DecodeArgs& a, int L) {
  PageWalk w = make_walk(L, a.window, a.n_sink, kBS);
  if (a.fused && w.L > 0) {
    w.L -= 1;
    const int n_log = cdiv(w.L, kBS);
    w.n_eff = w.sink_pages + (n_log > w.win_first ? n_log - w.win_first : 0);
  }
  return w;
}

// Partitions of one sequence, capped at the grid's partition count.  The cap only
// bites when context_lens[b] exceeds what the block table can address; every
// effective page it drops lies past max_blocks and would be masked anyway.
__device__ inline int num_partitions(const PageWalk& w, const DecodeArgs& a) {
  const int n = w.n_eff > 0 ? cdiv(w.n_eff, a.part_pages) : 1;
  return n < a.n_parts_max ? n : a.n_parts_max;
}

// Lazy rescaling: the reference max m_run of a head moves only when a tile's max
// exceeds it by more than kLazyLog2 (log2 units), so the weights p = 2^(s - m_run)
// stay <= 2^kLazyLog2 (exact in the 16-bit P operands) and the O and l rescale,
// NB * 4 multiplies per tile, runs only on those rare tiles (a wave-uniform branch).
// (O, l) relative to any m_run is a valid log-sum-exp state, so the merges are
// unchanged.
constexpr float kLazyLog2 = 8.f;

// Online-softmax state of one wave: lane holds head ln's reference max (the same
// in every k-group), its k-group's share of the running sum, and
// O^T[16m + 4lq + r][ln] in acc[m][r].
template <int NB, bool LAZY = true>
struct SoftmaxState {
  f32x4 acc[NB];
  float m_run, l_run;
  __device__ inline void reset() {
#pragma unroll
    for (int m = 0; m < NB; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_run = kNegInf;
    l_run = 0.f;
  }
  // Sum of head ln over the four k-groups.
  __device__ inline float total() const {
    float l = l_run + __shfl_xor(l_run, 16);
    return l + __shfl_xor(l, 32);
  }
  // Folds scaled scores sl (masked rows at -inf) and returns the weights p;
  // the caller then accumulates P . V.
  __device__ inline void fold(const float sl[4], float p[4]) {
    float mx = fmaxf(fmaxf(sl[0], sl[1]), fmaxf(sl[2], sl[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // -inf + kLazyLog2 is -inf: the first finite tile max always moves it.  Without
    // LAZY (fp32 at head_dim 256, where the branch costs registers the ring needs) the
    // reference max follows every increase and the rescale runs every tile.
    const bool grow = LAZY ? mx > m_run + kLazyLog2 : mx > m_run;
    if (!LAZY || __builtin_amdgcn_ballot_w64(grow) != 0) {
      const float m_new = grow ? mx : m_run;
      const float alpha = grow ? exp2_fast(m_run - m_new) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int m = 0; m < NB; ++m) acc[m] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == kNegInf ? 0.f : m_run;
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = exp2_fast(sl[r] - m_use);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);
  }
};

// Physical page of logical page lp of sequence b, or -1 when the table entry
// is outside the pool.  The tile of an invalid page is read from page 0 and
// fully masked.
__device__ inline int64_t phys_page(const DecodeArgs& a, const int32_t* bt, int b, int lp) {
  const int64_t p = bt[(int64_t)b * a.max_blocks + lp];
  return (p < 0 || p >= a.num_pages) ? -1 : p;
}

// Visibility of rows 4*lq + r of logical page lp for the walk w.
__device__ inline void rows_visible(const PageWalk& w, int lp, bool live, const DecodeArgs& a,
                                    int lq, bool vis[4]) {
  const int pos0 = lp * kBS + 4 * lq;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int pos = pos0 + r;
    vis[r] = live && pos < w.L && (pos >= w.win_start || pos < a.n_sink);
  }
}

// Whether every row of logical page lp is visible (wave-uniform: lp, live and the
// walk are): then no V row needs masking.
__device__ inline bool page_visible(const PageWalk& w, int lp, bool live, const DecodeArgs& a) {
  const int pos0 = lp * kBS;
  return live && pos0 + kBS <= w.L && (pos0 >= w.win_start || pos0 + kBS <= a.n_sink);
}

// Register-level tile machinery of one wave (lane = 16 * lq + ln) for pools of
// the query dtype DT.  Interface shared with TileOps8: QReg / TileReg register
// sets, load_q, load_tile, score.
template <int DT, int D>
struct TileOps {
  using Tr = Traits<DT>;
  using E = typename Tr::E;
  using VChunk = typename Tr::VChunk;
  static constexpr int kD = D;
  // Stream walk occupancy.  At D 128 (8 KiB slots) one workgroup per CU: 1024 waves
  // keep HBM as busy as 2048 (C2: 54.9 against 55.7 µs) with fewer partials; deeper
  // rings measured slower.
  static constexpr int kWGsPerCU = walk_wgs_per_cu(2 * (int64_t)D * kBS * sizeof(E));
  static constexpr int X = 16 / (int)sizeof(E);  // elements per 16-byte K chunk
  static constexpr int KLD = D / X / 4;          // K loads per lane per tile
  static constexpr int NB = D / 16;              // 16-dim blocks (PV MFMAs per tile)
  static constexpr int64_t kTile = (int64_t)D * kBS;  // elements of one tile
  static constexpr int kRing = kPageBufs;             // stream walk: tiles in flight
  // Query rows reloaded into every ring slot (false) or only when a slot's unit
  // changes: the reload is hidden behind 8 KiB tiles (C2 walk 47.5 µs against 48.2
  // with the per-unit form).
  static constexpr bool kQPerUnit = false;
  // fp32 at head_dim 256: a two-tile ring takes 256 of the 512 registers, and the
  // branches below would spill; its masking and rescaling stay branch-free.
  static constexpr bool kMaskBranch = !(DT == IVAKV_F32 && D == 256);
  using State = SoftmaxState<NB, kMaskBranch>;
  struct QReg {
    Chunk16 c[KLD];
  };
  struct TileReg {
    Chunk16 k[KLD];
    VChunk v[NB];
  };

  // Query rows of kv head h's group for sequence b, in K-chunk order (chunk
  // 4*j + lq).  MFMA columns ln >= G repeat head G-1: their scores are never
  // written out, and the loads stay unconditional (no exec-masked branch,
  // whose join would make the compiler wait for every outstanding load).
  static __device__ inline void load_q(const DecodeArgs& a, int b, int h, int ln, int lq, QReg& qr) {
    const int g = ln < a.G ? ln : a.G - 1;
    const E* qb = static_cast<const E*>(a.q) + ((int64_t)b * a.Hkv * a.G + h * a.G + g) * D;
#pragma unroll
    for (int j = 0; j < KLD; ++j) qr.c[j] = *reinterpret_cast<const Chunk16*>(qb + (4 * j + lq) * X);
  }

  // Issues the loads of one tile.  The empty asm with a memory clobber pins
  // them here: loads of read-only memory may otherwise be sunk down to their
  // first use in the next ring step, which serialises load and compute.
  static __device__ inline void load_tile(const DecodeArgs& a, int64_t phys, int h, int ln, int lq,
                                          TileReg& t) {
    const int64_t tile = ((phys < 0 ? 0 : phys) * a.Hkv + h) * kTile;
    const E* kp = static_cast<const E*>(a.k_pool) + tile;
    const E* vp = static_cast<const E*>(a.v_pool) + tile;
#pragma unroll
    for (int j = 0; j < KLD; ++j) t.k[j] = load_once<Chunk16>(kp + ((4 * j + lq) * kBS + ln) * X);
#pragma unroll
    for (int m = 0; m < NB; ++m) t.v[m] = load_once<VChunk>(vp + (16 * m + ln) * kBS + 4 * lq);
    __asm__ volatile("" ::: "memory");
  }

  // Scores one loaded tile of logical page lp and folds it into st.  With
  // live == false (a padding slot of the ring) every row is masked.
  static __device__ inline void score(State& st, TileReg& t, const QReg& qr, const PageWalk& w,
                                      int lp, bool live, const DecodeArgs& a, int lq) {
    // S^T = K . Q^T : lane holds rows 4*lq + r of head ln.
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KLD; ++j) s = Tr::qk(t.k[j], qr.c[j], s);
    bool vis[4];
    rows_visible(w, lp, live, a, lq, vis);
    float sl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) sl[r] = vis[r] ? s[r] * a.scale_log2 : kNegInf;
    // Rows that are not attended may hold any bits (0 * NaN would poison acc): a
    // page with such rows (a sequence's last, a window's first, padding or an invalid
    // id) zeroes them, behind a wave-uniform branch that full pages skip (except for
    // fp32 at head_dim 256, whose two-tile ring leaves no registers for it).  The
    // scores above are selects, so no block boundary separates the MFMAs from their
    // first use.
    if (!kMaskBranch || !page_visible(w, lp, live, a)) {
#pragma unroll
      for (int m = 0; m < NB; ++m) Tr::mask_rows(t.v[m], vis);
    }
    float p[4];
    st.fold(sl, p);
    // O^T += V^T . P^T
    const typename Tr::PVec pv = Tr::pack_p(p);
#pragma unroll
    for (int m = 0; m < NB; ++m) st.acc[m] = Tr::pv(t.v[m], pv, st.acc[m]);
  }
};

// The same for FP8 (OCP e4m3fn) pools with per-(slot, kv head) scaling factors
// (quantized = x * sf, sf = 448 / amax of the row; k_scale / v_scale [page][Hkv][16]
// fp32), queries and output of dtype DT (fp16 or bf16).  Layout: k_pool
// [page][Hkv][D/16][16][16] bytes, v_pool [page][Hkv][16 * D] bytes in the order of
// fp8_v_offset ([d%16][r/4][d/16][r%4]: a lane's V words are consecutive).  A lane's 16-byte K
// chunk holds dims 16c .. 16c+15 (c = 4i + lq) of row ln; it is converted to two
// 8-element operands (v_cvt_scalef32_pk_*_fp8, exact) for two 16x16x32 MFMAs, whose
// query chunks are loaded in the same dim order.  Per key, 1/sf_k joins the score
// scale and 1/sf_v multiplies p before the PV product.
template <int DT, int D>
struct TileOps8 {
  using Tr = Traits<DT>;
  using E = typename Tr::E;
  using VChunk = typename Tr::VChunk;
  static constexpr int kD = D;
  // At D 128 (4 KiB slots) two workgroups per CU: 41.6 µs on C2 against 44.6 µs at one.
  static constexpr int kWGsPerCU = walk_wgs_per_cu(2 * (int64_t)D * kBS);
  static constexpr int KL = D / 64;   // 16-byte K loads (16 dims) per lane per tile
  static constexpr int NB = D / 16;
  static constexpr int64_t kTileBytes = (int64_t)D * kBS;
  // The plain ring: a deeper one (as many bytes in flight as for 16-bit pages)
  // measured slower.
  static constexpr int kRing = kPageBufs;
  // Query rows loaded into a ring slot only when the slot's unit changes: with 4 KiB
  // tiles the per-slot reload costs (C2 FP8 attention 41.2-41.5 µs against
  // 38.7-38.8 µs loading per unit).
  static constexpr bool kQPerUnit = true;
  using State = SoftmaxState<NB>;
  struct QReg {
    Chunk16 c[2 * KL];  // c[2i + half]: dims 16 * (4i + lq) + 8 * half .. + 8
  };
  struct TileReg {
    Chunk16 k[KL];
    uint32_t v[NB];  // keys 4lq .. 4lq+3 of dim 16m + ln, one byte each
    f32x4 ks, vs;    // scaling factors of keys 4lq .. 4lq+3
  };

  static __device__ inline void load_q(const DecodeArgs& a, int b, int h, int ln, int lq, QReg& qr) {
    const int g = ln < a.G ? ln : a.G - 1;
    const E* qb = static_cast<const E*>(a.q) + ((int64_t)b * a.Hkv * a.G + h * a.G + g) * D;
#pragma unroll
    for (int i = 0; i < KL; ++i)
#pragma unroll
      for (int half = 0; half < 2; ++half)
        qr.c[2 * i + half] = *reinterpret_cast<const Chunk16*>(qb + 16 * (4 * i + lq) + 8 * half);
  }

  static __device__ inline void load_tile(const DecodeArgs& a, int64_t phys, int h, int ln, int lq,
                                          TileReg& t) {
    const int64_t tile = (phys < 0 ? 0 : phys) * a.Hkv + h;
    const uint8_t* kp = static_cast<const uint8_t*>(a.k_pool) + tile * kTileBytes;
    const uint8_t* vp = static_cast<const uint8_t*>(a.v_pool) + tile * kTileBytes;
#pragma unroll
    for (int i = 0; i < KL; ++i) t.k[i] = load_once<Chunk16>(kp + ((4 * i + lq) * kBS + ln) * 16);
    // Words m = 0 .. NB-1 (dims 16m + ln, keys 4lq .. 4lq+3) are consecutive in the
    // FP8 V tile order (fp8_v_offset): NB / 4 16-byte loads.
    const uint8_t* vl = vp + fp8_v_offset(ln, 4 * lq, D);
#pragma unroll
    for (int m = 0; m < NB; m += 4) {
      const Chunk16 c = load_once<Chunk16>(vl + 4 * m);
#pragma unroll
      for (int j = 0; j < 4; ++j) t.v[m + j] = c.w[j];
    }
    t.ks = load_once<f32x4>(a.k_scale + tile * kBS + 4 * lq);
    t.vs = load_once<f32x4>(a.v_scale + tile * kBS + 4 * lq);
    __asm__ volatile("" ::: "memory");
  }

  // Two fp8 values (bytes 2*HI, 2*HI+1 of w) as two DT values, exactly.
  template <bool HI>
  static __device__ inline uint32_t cvt2(uint32_t w) {
    if constexpr (DT == IVAKV_F16)
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
    else
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
  }

  static __device__ inline void score(State& st, TileReg& t, const QReg& qr, const PageWalk& w,
                                      int lp, bool live, const DecodeArgs& a, int lq) {
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const Chunk16 lo{{cvt2<false>(t.k[i].w[0]), cvt2<true>(t.k[i].w[0]),
                        cvt2<false>(t.k[i].w[1]), cvt2<true>(t.k[i].w[1])}};
      const Chunk16 hi{{cvt2<false>(t.k[i].w[2]), cvt2<true>(t.k[i].w[2]),
                        cvt2<false>(t.k[i].w[3]), cvt2<true>(t.k[i].w[3])}};
      s = Tr::qk(lo, qr.c[2 * i], s);
      s = Tr::qk(hi, qr.c[2 * i + 1], s);
    }
    bool vis[4];
    rows_visible(w, lp, live, a, lq, vis);
    float sl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sl[r] = vis[r] ? s[r] * (a.scale_log2 * __builtin_amdgcn_rcpf(t.ks[r])) : kNegInf;
    // Zero the bytes of rows that are not attended (any bits, NaN codes included),
    // on pages that have such rows (a wave-uniform branch full pages skip).
    if (!page_visible(w, lp, live, a)) {
      const uint32_t keep = (vis[0] ? 0xFFu : 0u) | (vis[1] ? 0xFF00u : 0u) |
                            (vis[2] ? 0xFF0000u : 0u) | (vis[3] ? 0xFF000000u : 0u);
#pragma unroll
      for (int m = 0; m < NB; ++m) t.v[m] &= keep;
    }
    float p[4];
    st.fold(sl, p);
    float pv_in[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pv_in[r] = p[r] * __builtin_amdgcn_rcpf(t.vs[r]);
    const typename Tr::PVec pv = Tr::pack_p(pv_in);
#pragma unroll
    for (int m = 0; m < NB; ++m) {
      const Chunk8 vh{{cvt2<false>(t.v[m]), cvt2<true>(t.v[m])}};
      st.acc[m] = Tr::pv(vh, pv, st.acc[m]);
    }
  }
};

// ---------------------------------------------------------------------------
// partitioned walk
// ---------------------------------------------------------------------------

// Wave w of partition `part` owns effective pages part*part_pages + w + 4*i,
// i = 0 .. n_mine-1, and streams them through a ring of kPageBufs register
// page buffers.  Loads are never skipped: past the wave's last page the index
// is clamped to that page (an L2 hit) and the duplicate is fully masked, so the
// loop body has no branches and the compiler's vmcnt waits only cover the
// buffer about to be consumed.
//
// Built for two workgroups per CU (one at head_dim 256): with a higher
// occupancy target the scheduler sinks each load next to its use and the ring
// stops overlapping loads with compute.
// Block table and context lengths come in as __restrict__ parameters, which
// keeps their reads on the scalar cache (see decode_stream_kernel).
//
// kFp8: FP8 pools (the fused step's single launch only): tiles through TileOps8, and the
// new rows quantized as ivakv_append_fp8 does (per-row factor from a wave reduction of
// max |x|, codes e4m3(x * sf)), attended as their dequantized values and stored as codes
// and factors, as decode_fused_merge_kernel does on the stream walk.
template <int DT, int D, bool kFp8 = false>
__global__ __launch_bounds__(kThreads, partial_wgs_per_cu(D)) void decode_partial_kernel(
    DecodeArgs a, const int32_t* __restrict__ bt, const int32_t* __restrict__ ctx) {
  using Ops = typename std::conditional<kFp8, TileOps8<DT, D>, TileOps<DT, D>>::type;
  using E = typename Ops::E;
  constexpr int NB = Ops::NB;

  const int h = blockIdx.x, b = blockIdx.y, part = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15;
  const int lq = lane >> 4;
  const PageWalk w = seq_walk(a, ctx[b]);  // fused: the positions before the new token
  const int n_parts = num_partitions(w, a);
  if (part >= n_parts) return;

  const int G = a.G;
  const int Hq = a.Hkv * G;
  const bool g_ok = ln < G;

  typename Ops::QReg qr;
  Ops::load_q(a, b, h, ln, lq, qr);
  typename Ops::State st;
  st.reset();

  // Fused (one partition per sequence): the new token's operands are loaded before
  // the walk, so they arrive with its first tiles: the slot's page id, for the
  // dot products q_g . k_new the lane-strided dims of k_new and of the wave's
  // heads g = wave + 4t (G <= 16), and this thread's element of v_new (the output
  // loop's dim is threadIdx.x % D in every round).  Every load is unconditional
  // (valid addresses when not fused, values then unused): a conditional load
  // would be waited for at the branch's join.
  constexpr int DJ = D / 64;
  const int L_ctx = ctx[b];
  const bool slot_in_table = a.fused && L_ctx > 0 && (L_ctx - 1) / kBS < a.max_blocks;
  const int32_t slot_entry = slot_in_table ? bt[(int64_t)b * a.max_blocks + (L_ctx - 1) / kBS]
                                           : ctx[b];
  const int64_t row_nh = ((int64_t)b * a.Hkv + h) * D;
  const E* qb = static_cast<const E*>(a.q) + ((int64_t)b * Hq + h * G) * D;
  const E* kn = a.fused ? static_cast<const E*>(a.k_new) + row_nh : qb;
  const E* vn = a.fused ? static_cast<const E*>(a.v_new) + row_nh : qb;
  float kd[DJ], qd[4][DJ], vd[kFp8 ? DJ : 1];
#pragma unroll
  for (int j = 0; j < DJ; ++j) kd[j] = (float)kn[lane + 64 * j];
  if constexpr (kFp8) {  // the V row's lane-strided dims, for its factor
#pragma unroll
    for (int j = 0; j < DJ; ++j) vd[j] = (float)vn[lane + 64 * j];
  }
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int j = 0; j < DJ; ++j) qd[t][j] = (float)qb[min(wave + 4 * t, G - 1) * D + lane + 64 * j];
  float v_own = (float)vn[threadIdx.x % D];

  const int v_begin = part * a.part_pages + wave;
  const int v_end = min(min((part + 1) * a.part_pages, w.n_eff), table_pages(w, a.max_blocks));
  const int n_mine = v_begin < v_end ? cdiv(v_end - v_begin, kWaves) : 0;
  // Effective page of the wave's i-th slot, clamped to its last page.
  auto eff_page = [&](int i) { return v_begin + kWaves * min(i, n_mine - 1); };

  if (n_mine > 0) {
    typename Ops::TileReg tb[kPageBufs];
    int64_t pb[kPageBufs];
#pragma unroll
    for (int s = 0; s < kPageBufs; ++s) {
      pb[s] = phys_page(a, bt, b, logical_page(w, eff_page(s)));
      Ops::load_tile(a, pb[s], h, ln, lq, tb[s]);
    }
    for (int i = 0; i < n_mine; i += kPageBufs) {
#pragma unroll
      for (int s = 0; s < kPageBufs; ++s) {
        Ops::score(st, tb[s], qr, w, logical_page(w, eff_page(i + s)),
                   i + s < n_mine && pb[s] >= 0, a, lq);
        pb[s] = phys_page(a, bt, b, logical_page(w, eff_page(i + s + kPageBufs)));
        Ops::load_tile(a, pb[s], h, ln, lq, tb[s]);
      }
    }
  }

  const float l_tot = st.total();

  // Merge the four waves through LDS.
  extern __shared__ float smem[];
  float* s_m = smem;                       // [kWaves][16]
  float* s_l = s_m + kWaves * 16;          // [kWaves][16]
  float* s_fin = s_l + kWaves * 16;        // [16][2] merged (max, sum)
  float* s_acc = s_fin + 32;               // [kWaves][G][D + 4]
  constexpr int kRow = D + 4;
  float* s_dot = s_acc + kWaves * G * kRow;  // [G] fused: q_g . k_new
  if (lq == 0) {
    s_m[wave * 16 + ln] = st.m_run;
    s_l[wave * 16 + ln] = l_tot;
  }
  __syncthreads();
  float M = kNegInf;
#pragma unroll
  for (int u = 0; u < kWaves; ++u) M = fmaxf(M, s_m[u * 16 + ln]);
  const float M_use = M == kNegInf ? 0.f : M;
  if (g_ok) {
    const float f = exp2_fast(st.m_run - M_use);
    float* dst = s_acc + (wave * G + ln) * kRow + 4 * lq;
#pragma unroll
    for (int m = 0; m < NB; ++m) *reinterpret_cast<f32x4*>(dst + 16 * m) = st.acc[m] * f;
    if (wave == 0 && lq == 0) {
      float L = 0.f;
#pragma unroll
      for (int u = 0; u < kWaves; ++u) L += s_l[u * 16 + ln] * exp2_fast(s_m[u * 16 + ln] - M_use);
      s_fin[2 * ln] = M;
      s_fin[2 * ln + 1] = L;
    }
  }
  // Fused: the new token's scores q_g . k_new from the prefetched operands, one
  // head per wave in turn, a wave reduction each.  FP8: every wave first reduces the
  // new rows' max |x| (NaN kept) to the factors and rounds its operands to the values
  // the codes decode to.
  float sfk = 1.f, sfv = 1.f;
  if (a.fused) {
    if constexpr (kFp8) {
      float ka = 0.f, va = 0.f;
#pragma unroll
      for (int j = 0; j < DJ; ++j) {
        ka = nan_max(ka, fabsf(kd[j]));
        va = nan_max(va, fabsf(vd[j]));
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        ka = nan_max(ka, __shfl_xor(ka, o));
        va = nan_max(va, __shfl_xor(va, o));
      }
      sfk = row_sf(ka);
      sfv = row_sf(va);
#pragma unroll
      for (int j = 0; j < DJ; ++j) kd[j] = e4m3_decode(e4m3_encode(kd[j] * sfk)) / sfk;
      v_own = e4m3_decode(e4m3_encode(v_own * sfv)) / sfv;
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (wave + 4 * t >= G) break;
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < DJ; ++j) dot += qd[t][j] * kd[j];
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) dot += __shfl_xor(dot, o);
      if (lane == 0) s_dot[wave + 4 * t] = dot;
    }
  }
  __syncthreads();

  const bool direct = n_parts == 1;
  // The new token's slot (position L-1); an invalid page id there means it is
  // neither stored nor attended, as in the stream walk's fused merge.
  const int64_t new_page = slot_in_table ? (int64_t)slot_entry : -1;
  const bool new_ok = new_page >= 0 && new_page < a.num_pages;
  const int64_t part_base = (((int64_t)b * a.Hkv + h) * a.n_parts_max + part) * G;
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int gg = idx / D, d = idx - (idx / D) * D;
    float o = 0.f;
#pragma unroll
    for (int u = 0; u < kWaves; ++u) o += s_acc[(u * G + gg) * kRow + d];
    if (direct) {
      float L = s_fin[2 * gg + 1];
      if (a.fused) {  // fold the new token (o and L are relative to max(M, 0 if none))
        const float M = s_fin[2 * gg];
        const float sc = s_dot[gg] * a.scale_log2;
        const float mn = fmaxf(M, sc);
        const float f = !new_ok ? 1.f : (M == kNegInf ? 0.f : exp2_fast(M - mn));
        const float wn = new_ok ? exp2_fast(sc - mn) : 0.f;
        L = L * f + wn;
        o = o * f + v_own * wn;
      }
      const float r = L > 0.f ? o / L : 0.f;
      static_cast<E*>(a.out)[((int64_t)b * Hq + h * G + gg) * D + d] = Ops::Tr::from_float(r);
    } else {
      a.ws_acc[part_base * D + idx] = o;
      if (d == 0) {
        a.ws_ml[(part_base + gg) * 2] = s_fin[2 * gg];
        a.ws_ml[(part_base + gg) * 2 + 1] = s_fin[2 * gg + 1];
      }
    }
  }
  // Fused: the new rows go to the slot of position L-1 (after every wave's reads
  // of that page, which the barriers above order).
  if (new_ok) {
    const int row = (L_ctx - 1) % kBS;
    if constexpr (kFp8) {
      const int64_t tile = new_page * a.Hkv + h;
      uint8_t* kp = static_cast<uint8_t*>(const_cast<void*>(a.k_pool)) + tile * D * kBS;
      uint8_t* vp = static_cast<uint8_t*>(const_cast<void*>(a.v_pool)) + tile * D * kBS;
      for (int d = threadIdx.x; d < D; d += kThreads) {
        kp[((d >> 4) * kBS + row) * 16 + (d & 15)] = (uint8_t)e4m3_encode((float)kn[d] * sfk);
        vp[fp8_v_offset(d, row, D)] = (uint8_t)e4m3_encode((float)vn[d] * sfv);
      }
      if (threadIdx.x == 0) {
        const_cast<float*>(a.k_scale)[tile * kBS + row] = sfk;
        const_cast<float*>(a.v_scale)[tile * kBS + row] = sfv;
      }
    } else {
      constexpr int X = 16 / (int)sizeof(E);
      const int64_t tile = (new_page * a.Hkv + h) * (int64_t)D * kBS;
      E* kp = static_cast<E*>(const_cast<void*>(a.k_pool)) + tile;
      E* vp = static_cast<E*>(const_cast<void*>(a.v_pool)) + tile;
      for (int d = threadIdx.x; d < D; d += kThreads) {
        kp[((d / X) * kBS + row) * X + d % X] = kn[d];
        vp[d * kBS + row] = vn[d];
      }
    }
  }
}

// Log-sum-exp fold of n partial (max, sum, acc) slots into one running state
// (M, L, O) of VEC consecutive output elements idx .. idx+VEC-1 (query head g; idx
// a multiple of VEC, so they share the head); slot(i) gives the workspace slot of
// the i-th partial.  One online pass loads U partials' (max, sum, acc) together, so
// the merge costs one memory round trip per U partials instead of separate max / sum
// / accumulate passes; U is sized to the partials a unit usually has (loads past n
// repeat the last slot, so a larger U only adds load instructions).
template <int VEC, int U, typename SlotFn>
__device__ inline void fold_slots(const DecodeArgs& a, int g, int idx, int D, int n, SlotFn slot,
                                  float& M, float& L,
                                  typename std::conditional<VEC == 4, f32x4, float>::type& O) {
  using OV = typename std::conditional<VEC == 4, f32x4, float>::type;
  const int G = a.G;
  for (int i0 = 0; i0 < n; i0 += U) {
    float mv[U], lv[U];
    OV av[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t sl = slot(min(i0 + u, n - 1));
      mv[u] = a.ws_ml[(sl * G + g) * 2];
      lv[u] = a.ws_ml[(sl * G + g) * 2 + 1];
      av[u] = *reinterpret_cast<const OV*>(a.ws_acc + sl * G * D + idx);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) mv[u] = i0 + u < n ? mv[u] : kNegInf;
    float mc = M;
#pragma unroll
    for (int u = 0; u < U; ++u) mc = fmaxf(mc, mv[u]);
    const float m_use = mc == kNegInf ? 0.f : mc;
    const float f = exp2_fast(M - m_use);
    L *= f;
    O *= f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float w = exp2_fast(mv[u] - m_use);
      L += lv[u] * w;
      O += av[u] * w;
    }
    M = mc;
  }
}

// Merges with VEC = 4 output elements per thread (16-byte partial loads, a quarter
// of the threads) pay when units are many; with few, long units the merge needs
// the parallelism of one element per thread, and below kMergeSplitUnits units
// (many partials per unit) four lanes share each element: lane l of a wave takes
// element l % 16 of the wave's 16-element block and the quarter l / 16 of the
// unit's partials, so each lane folds its quarter in one round trip of loads and
// the four states are combined across lanes.
constexpr int kMergeVec4Units = 1024;
constexpr int kMergeSplitUnits = 256;
constexpr int kSplitters = 4;
// Partials the stream walk's merges fold per round trip, by merge shape: a unit has
// about waves / units + 1 fragments, so at most 2 when units are many enough for
// four-element lanes (>= kMergeVec4Units), about 5 for one element per thread, and up
// to hundreds (a quarter per splitter lane) below kMergeSplitUnits.
constexpr int stream_fold_width(int vec, int splitters) {
  return vec == 4 ? 4 : splitters > 1 ? 16 : 8;
}

// Log-sum-exp combine of the (M, L, O) states of lanes l, l ^ 16, l ^ 32, l ^ 48.
__device__ inline void combine_splitters(float& M, float& L, float& O) {
#pragma unroll
  for (int off = 16; off <= 32; off <<= 1) {
    const float Mo = __shfl_xor(M, off), Lo = __shfl_xor(L, off), Oo = __shfl_xor(O, off);
    const float mc = fmaxf(M, Mo);
    const float m_use = mc == kNegInf ? 0.f : mc;
    const float fa = exp2_fast(M - m_use), fb = exp2_fast(Mo - m_use);
    L = L * fa + Lo * fb;
    O = O * fa + Oo * fb;
    M = mc;
  }
}

// Output elements of a merge thread: VEC consecutive ones per thread over the
// workgroup and grid z (S == 1), or one per lane with S lanes per element (S == 4,
// see kMergeSplitUnits); `split` is the lane's quarter of the partials.  first
// and step are uniform over a wave up to the lane's element offset, and G * D is a
// multiple of 64, so every lane of a wave runs the same number of iterations.
template <int VEC, int S>
struct MergeLanes {
  int first, step, split;
  __device__ MergeLanes() {
    if constexpr (S == 1) {
      first = VEC * (threadIdx.x + blockIdx.z * blockDim.x);
      step = VEC * blockDim.x * gridDim.z;
      split = 0;
    } else {
      const int lane = threadIdx.x & 63;
      const int waves = blockDim.x >> 6;
      first = 16 * ((threadIdx.x >> 6) + waves * blockIdx.z) + (lane & 15);
      step = 16 * waves * gridDim.z;
      split = lane >> 4;
    }
  }
  // Partials [begin, begin + count) of n this lane folds.
  __device__ void range(int n, int& begin, int& count) const {
    const int chunk = S == 1 ? n : (n + S - 1) / S;
    begin = split * chunk;
    count = max(0, min(chunk, n - begin));
  }
};

// Merge of n partial slots into the out rows of unit (b, h), over the elements of
// MergeLanes<VEC, S> (spread over the workgroup and grid z: a unit is split across
// workgroups when units are fewer than CUs).
template <int DT, int VEC, int S, int U, typename SlotFn>
__device__ inline void merge_slots(const DecodeArgs& a, int b, int h, int n, int D, SlotFn slot) {
  using E = typename Traits<DT>::E;
  const int G = a.G;
  const int Hq = a.Hkv * G;
  E* out = static_cast<E*>(a.out) + ((int64_t)b * Hq + h * G) * D;
  const MergeLanes<VEC, S> ml;
  int i0, cnt;
  ml.range(n, i0, cnt);
  for (int idx = ml.first; idx < G * D; idx += ml.step) {
    float M = kNegInf, L = 0.f;
    typename std::conditional<VEC == 4, f32x4, float>::type O = {};
    fold_slots<VEC, U>(a, idx / D, idx, D, cnt, [&](int i) { return slot(i0 + i); }, M, L, O);
    if constexpr (VEC == 4) {
#pragma unroll
      for (int r = 0; r < 4; ++r) out[idx + r] = Traits<DT>::from_float(L > 0.f ? O[r] / L : 0.f);
    } else {
      if constexpr (S > 1) combine_splitters(M, L, O);
      if (ml.split == 0) out[idx] = Traits<DT>::from_float(L > 0.f ? O / L : 0.f);
    }
  }
}

// Partitioned walk's merge: grid (kv head, sequence), 256 threads.
template <int DT>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a, int D) {
  const int h = blockIdx.x, b = blockIdx.y;
  const PageWalk w = make_walk(a.ctx[b], a.window, a.n_sink, kBS);
  const int n_parts = num_partitions(w, a);
  if (n_parts <= 1) return;
  const int64_t base = ((int64_t)b * a.Hkv + h) * a.n_parts_max;
  merge_slots<DT, 1, 1, 16>(a, b, h, n_parts, D, [&](int i) { return base + i; });
}

// ---------------------------------------------------------------------------
// stream walk
// ---------------------------------------------------------------------------

// n / d for n >= 0, d > 0: one 32-bit division when both fit in 32 bits (the
// usual case; a uniform branch), else the 64-bit routine, a loop of ~100
// instructions per bit pair that sits on the walk's and the merges' start-up path.
__device__ inline int64_t div_nn(int64_t n, int64_t d) {
  if (((uint64_t)n | (uint64_t)d) >> 32 == 0) return (int64_t)((uint32_t)n / (uint32_t)d);
  return n / d;
}

// Waves that share T tiles: every wave gets at least kMinTilesPerWave.
__device__ inline int64_t stream_waves(int64_t T, int n_waves) {
  const int64_t want = (T + kMinTilesPerWave - 1) / kMinTilesPerWave;
  return want < n_waves ? (want > 0 ? want : 1) : n_waves;
}

// Split of T flat tiles over W waves: wave k owns tiles [start(k), start(k + 1))
// with start(k) = k * T / W; owner(t) inverts it (the k with start(k) <= t <
// start(k + 1)).
struct WaveSplit {
  int64_t T, W;
  __device__ WaveSplit(int64_t T_, const DecodeArgs& a) : T(T_), W(stream_waves(T_, a.n_waves)) {}
  __device__ int64_t start(int64_t k) const { return div_nn(k * T, W); }
  __device__ int64_t owner(int64_t t) const { return div_nn((t + 1) * W - 1, T); }
};

// Flat tile order: sequence-major, then kv head, then effective page.  Unit
// (b, h) = tiles [Hkv*pref[b] + h*n_b, ... + n_b) with n_b = pref[b+1] - pref[b].
// A fragment (the part of a unit inside one wave's range) is identified by
// (wave k, unit u = b*Hkv + h); k + u increases strictly along the flat order,
// so it is the fragment's workspace slot (< kMaxStreamWaves + B*Hkv).
//
// The block table and context lengths also come in as __restrict__ parameters:
// with the workspace and output stores in the loop, that is what lets the
// compiler read them through the scalar cache (s_load, lgkmcnt) instead of
// vector loads whose vmcnt wait would drain the page ring.
template <class Ops>
__global__ __launch_bounds__(kStreamThreads, Ops::kWGsPerCU) void decode_stream_kernel(
    DecodeArgs a, const int32_t* __restrict__ bt, const int32_t* __restrict__ ctx) {
  using E = typename Ops::E;
  constexpr int D = Ops::kD, NB = Ops::NB;
  constexpr int kRing = Ops::kRing;  // tiles in flight per wave
  extern __shared__ int32_t s_pref[];  // [B + 1] page prefix, then per-wave scan totals
  int32_t* s_scan = s_pref + a.batch + 1;

  const int B = a.batch, Hkv = a.Hkv, G = a.G;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int ln = lane & 15;
  const int lq = lane >> 4;

  // 1. Page prefix of the batch: thread t sums a contiguous chunk of sequences;
  //    an inclusive scan of the chunk sums within each wave (lane shuffles) plus
  //    the totals of the waves before it (two barriers in all), then the chunk
  //    prefixes.
  const int chunk = cdiv(B, kStreamThreads);
  const int c0 = min(tid * chunk, B), c1 = min(c0 + chunk, B);
  int local = 0;
  for (int bb = c0; bb < c1; ++bb) {
    const int n = table_pages(seq_walk(a, ctx[bb]), a.max_blocks);
    s_pref[bb + 1] = n;
    local += n;
  }
  int incl = local;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off);
    if (lane >= off) incl += v;
  }
  if (lane == 63) s_scan[tid >> 6] = incl;
  __syncthreads();
  {
    int run = incl - local;  // exclusive prefix of this chunk
    for (int w = 0; w < (tid >> 6); ++w) run += s_scan[w];
    if (tid == 0) s_pref[0] = 0;
    for (int bb = c0; bb < c1; ++bb) {
      run += s_pref[bb + 1];
      s_pref[bb + 1] = run;
    }
  }
  __syncthreads();
  if (blockIdx.x == 0)
    for (int bb = tid; bb <= B; bb += kStreamThreads) a.ws_pref[bb] = s_pref[bb];

  const int64_t T = (int64_t)Hkv * uni(s_pref[B]);
  if (T == 0) return;
  const WaveSplit split(T, a);
  const int64_t k = (int64_t)blockIdx.x * kStreamWaves + __builtin_amdgcn_readfirstlane(tid >> 6);
  if (k >= split.W) return;
  const int64_t t_begin = split.start(k), t_end = split.start(k + 1);
  if (t_begin >= t_end) return;
  const int count = (int)(t_end - t_begin);

  // 2. Unit and page of the first tile: the last sequence b with
  //    pref[b] <= t_begin / Hkv (it is non-empty), then kv head and page.
  //    pref is non-decreasing, so b is the count of entries <= key, less one:
  //    one ballot when the batch fits a wave, else a binary search.
  int lo = 0, hi = B;
  {
    const int key = (int)div_nn(t_begin, Hkv);
    if (B <= 64) {
      const bool le = lane < B && s_pref[lane < B ? lane : 0] <= key;
      lo = __popcll(__ballot(le)) - 1;
    } else {
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (uni(s_pref[mid]) <= key) lo = mid;
        else hi = mid;
      }
    }
  }
  // A cursor walks (sequence, kv head, effective page) in flat order.
  struct Cursor {
    int b, h, v, n;
    PageWalk w;
  };
  Cursor c0r;
  c0r.b = lo;
  c0r.n = uni(s_pref[lo + 1]) - uni(s_pref[lo]);
  {
    const int64_t r = t_begin - (int64_t)Hkv * uni(s_pref[lo]);
    c0r.h = (int)div_nn(r, c0r.n);
    c0r.v = (int)(r - (int64_t)c0r.h * c0r.n);
  }
  c0r.w = seq_walk(a, ctx[c0r.b]);
  auto advance = [&](Cursor& c) {
    if (++c.v < c.n) return;
    c.v = 0;
    if (++c.h < Hkv) return;
    c.h = 0;
    do {
      ++c.b;
    } while (c.b < B && uni(s_pref[c.b + 1]) == uni(s_pref[c.b]));
    if (c.b < B) {
      c.n = uni(s_pref[c.b + 1]) - uni(s_pref[c.b]);
      c.w = seq_walk(a, ctx[c.b]);
    }
  };

  // 3. The ring: the load cursor runs kRing tiles ahead of the compute
  //    cursor.  Past the wave's last tile it stays there and loads padding slots
  //    that score() masks, from page 0 (as for an invalid page id): every wave
  //    reads that same tile, an L2 hit, where re-reading the wave's own last tile
  //    would miss (the streaming hint lets its lines go early).  Each slot holds
  //    the query rows of its tile's unit: loaded with every tile (an L2 hit after
  //    the first), or with kQPerUnit only when the slot's unit changes (a
  //    wave-uniform branch; the waits on the ring's tiles stay as they are).
  Cursor lc = c0r, cc = c0r;
  int issued = 0;
  typename Ops::QReg qb[kRing];
  typename Ops::TileReg tb[kRing];
  int64_t pb[kRing];
  int qunit[kRing];  // unit (b * Hkv + h) whose query rows qb[s] holds (kQPerUnit)
#pragma unroll
  for (int s = 0; s < kRing; ++s) qunit[s] = -1;
  auto issue = [&](int s) {
    if constexpr (Ops::kQPerUnit) {
      const int unit = lc.b * Hkv + lc.h;  // wave-uniform
      if (unit != qunit[s]) {
        Ops::load_q(a, lc.b, lc.h, ln, lq, qb[s]);
        qunit[s] = unit;
      }
    } else {
      Ops::load_q(a, lc.b, lc.h, ln, lq, qb[s]);
    }
    const int64_t p = phys_page(a, bt, lc.b, logical_page(lc.w, lc.v));
    pb[s] = issued < count ? p : -1;
    Ops::load_tile(a, pb[s], lc.h, ln, lq, tb[s]);
    if (++issued < count) advance(lc);
  };
#pragma unroll
  for (int s = 0; s < kRing; ++s) issue(s);

  typename Ops::State st;
  st.reset();
  bool fresh = true;   // next live tile starts a fragment
  int frag_first = 0;  // first page of the current fragment
  const int Hq = Hkv * G;
  for (int i = 0; i < count; i += kRing) {
#pragma unroll
    for (int s = 0; s < kRing; ++s) {
      const bool live = i + s < count;
      if (live && fresh) {
        st.reset();
        frag_first = cc.v;
        fresh = false;
      }
      Ops::score(st, tb[s], qb[s], cc.w, logical_page(cc.w, cc.v), live && pb[s] >= 0, a, lq);
      if (live) {
        const bool unit_end = cc.v == cc.n - 1;
        if (unit_end || i + s == count - 1) {
          // Flush the fragment: the whole unit goes straight to `out`,
          // a piece of it to workspace slot k + u.
          const float l_tot = st.total();
          if (ln < G) {
            if (frag_first == 0 && unit_end && !a.fused) {
              const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
              E* o = static_cast<E*>(a.out) + ((int64_t)cc.b * Hq + cc.h * G + ln) * D + 4 * lq;
#pragma unroll
              for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[16 * m + r] = Ops::Tr::from_float(st.acc[m][r] * inv);
            } else {
              const int64_t slot = k + (int64_t)cc.b * Hkv + cc.h;
              float* o = a.ws_acc + (slot * G + ln) * D + 4 * lq;
#pragma unroll
              for (int m = 0; m < NB; ++m) *reinterpret_cast<f32x4*>(o + 16 * m) = st.acc[m];
              if (lq == 0) {
                a.ws_ml[(slot * G + ln) * 2] = st.m_run;
                a.ws_ml[(slot * G + ln) * 2 + 1] = l_tot;
              }
            }
          }
          fresh = true;
        }
        advance(cc);
      }
      issue(s);
    }
  }
}

// Stream walk's merge: grid (kv head, sequence, column split), 256 or 64 threads.  Writes zeros for
// an empty unit, skips a unit one wave finished (written directly), and folds
// the fragments of a split unit (slots k + u, k = first..last wave).
template <int DT, int VEC, int S>
__global__ __launch_bounds__(256) void decode_stream_merge_kernel(DecodeArgs a, int D) {
  using E = typename Traits<DT>::E;
  const int h = blockIdx.x, b = blockIdx.y;
  const int Hkv = a.Hkv, G = a.G;
  const int p0 = a.ws_pref[b], p1 = a.ws_pref[b + 1], ptot = a.ws_pref[a.batch];
  asm volatile("" ::"s"(p0), "s"(p1), "s"(ptot));  // all three loads before the branch
  const int64_t pb = p0;
  const int n = p1 - p0;
  const int64_t T = (int64_t)Hkv * ptot;
  if (n == 0) {
    E* o = static_cast<E*>(a.out) + ((int64_t)b * Hkv * G + h * G) * D;
    for (int idx = threadIdx.x + blockIdx.z * blockDim.x; idx < G * D; idx += blockDim.x * gridDim.z)
      o[idx] = Traits<DT>::from_float(0.f);
    return;
  }
  const WaveSplit split(T, a);
  const int64_t first_tile = (int64_t)Hkv * pb + (int64_t)h * n;
  const int64_t k0 = split.owner(first_tile), k1 = split.owner(first_tile + n - 1);
  if (k0 == k1) return;
  const int64_t base = k0 + (int64_t)b * Hkv + h;
  merge_slots<DT, VEC, S, stream_fold_width(VEC, S)>(a, b, h, (int)(k1 - k0 + 1), D,
                                                    [&](int i) { return base + i; });
}

// Fused append's merge: grid (kv head, sequence, column split), 256 or 64 threads.  Scores the new
// token (position L-1) of every query head of the unit from k_new, folds it as one
// more log-sum-exp term (weight exp2(s - M), value row v_new) with the pool walk's
// partials of positions < L-1, writes `out`, and stores the new K/V rows into the
// token's slot for later steps.  Every unit is merged here (the fused walk never
// writes `out` directly).
//
// FP8 pools (kFp8): the new rows are quantized as ivakv_append_fp8 does (per-row
// factor sf = row_sf(max |x|) from a wave reduction over the row, codes e4m3(x * sf)),
// attended as their dequantized values code / sf -- what an append followed by the
// walk would read -- and their codes and factors are stored into the slot.
template <int DT, int D, bool kFp8, int VEC, int S>
__global__ __launch_bounds__(256) void decode_fused_merge_kernel(DecodeArgs a) {
  using Tr = Traits<DT>;
  using E = typename Tr::E;
  constexpr int DL = D / 64;  // dims of the new token's dot product per lane
  const int h = blockIdx.x, b = blockIdx.y;
  const int Hkv = a.Hkv, G = a.G, Hq = Hkv * G;
  const int lane = threadIdx.x & 63;
  // Every index the merge needs is loaded up front, in one round trip (the
  // empty asm keeps the compiler from sinking the prefix loads below the first
  // branch).
  const int L = a.ctx[b];
  const int p0 = a.ws_pref[b], p1 = a.ws_pref[b + 1], ptot = a.ws_pref[a.batch];
  asm volatile("" ::"s"(L), "s"(p0), "s"(p1), "s"(ptot));
  const int64_t pb = p0;
  const int n = p1 - p0;
  const int64_t T = (int64_t)Hkv * ptot;
  E* out = static_cast<E*>(a.out) + ((int64_t)b * Hq + h * G) * D;
  if (L <= 0) {
    for (int idx = threadIdx.x + blockIdx.z * blockDim.x; idx < G * D; idx += blockDim.x * gridDim.z)
      out[idx] = Tr::from_float(0.f);
    return;
  }
  // The new token's slot; an invalid page id there means it is neither stored nor
  // attended (as ivakv_append skips the slot and the walk masks the row).
  // The entry is loaded unconditionally (from context_lens when it lies outside
  // the table), through an offset that an empty asm turns into a vector
  // register: a conditional load, or one whose value is moved to a scalar
  // register, would be waited for at once instead of alongside the partials.
  const int pos = L - 1, row = pos % kBS, lp = pos / kBS;
  const bool in_table = lp < a.max_blocks;
  int64_t off = in_table ? (int64_t)b * a.max_blocks + lp : b;
  asm volatile("" : "+v"(off));
  const int32_t entry = (in_table ? a.bt : a.ctx)[off];
  const int64_t page = in_table ? (int64_t)entry : -1;
  const bool new_ok = page >= 0 && page < a.num_pages;
  const E* kn = static_cast<const E*>(a.k_new) + ((int64_t)b * Hkv + h) * D;
  const E* vn = static_cast<const E*>(a.v_new) + ((int64_t)b * Hkv + h) * D;
  const E* qb = static_cast<const E*>(a.q) + ((int64_t)b * Hq + h * G) * D;

  // Partials of the pool walk (positions < L-1): fragments k0..k1 of the unit.
  int64_t k0 = 0, nf = 0;
  if (n > 0) {
    const WaveSplit split(T, a);
    const int64_t first_tile = (int64_t)Hkv * pb + (int64_t)h * n;
    k0 = split.owner(first_tile);
    nf = split.owner(first_tile + n - 1) - k0 + 1;
  }
  const int64_t base = k0 + (int64_t)b * Hkv + h;
  // FP8: the new rows' factors, as ivakv_append_fp8 computes them (max |x| over the
  // row; every wave reduces the whole row, lanes strided over the dims), so every
  // thread holds them for the element loop and the append.
  float sfk = 1.f, sfv = 1.f;
  if constexpr (kFp8) {
    float ka = 0.f, va = 0.f;
#pragma unroll
    for (int j = 0; j < DL; ++j) {
      ka = nan_max(ka, fabsf((float)kn[lane + 64 * j]));
      va = nan_max(va, fabsf((float)vn[lane + 64 * j]));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      ka = nan_max(ka, __shfl_xor(ka, o));
      va = nan_max(va, __shfl_xor(va, o));
    }
    sfk = row_sf(ka);
    sfv = row_sf(va);
  }
  // Each thread owns VEC consecutive outputs idx .. of one query head g (D is a
  // multiple of 64), or with S == 4 a quarter of one output's partials
  // (MergeLanes).  The new token's dot product q_g . k_new: with VEC == 1 the
  // outputs of a wave share g and the wave sums lane-strided products (dims lane +
  // 64j); with VEC == 4 each lane sums its own four dims and the D/4 lanes of the
  // head reduce.  The operands (and the value elements) are loaded before the
  // partials, so every load of the thread is in flight at once; then the partials
  // are folded (and the splitters' states combined), then the new token.
  constexpr int NQ = VEC == 4 ? 4 : D / 64;  // dot-product terms per lane
  constexpr int kDotLanes = VEC == 4 ? D / 4 : 64;
  const MergeLanes<VEC, S> ml;
  int f0, fcnt;
  ml.range((int)nf, f0, fcnt);
  for (int idx = ml.first; idx < G * D; idx += ml.step) {
    const int g = idx / D, col = idx - g * D;
    float qv[NQ], kv[NQ], vv[VEC];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int d = VEC == 4 ? col + j : lane + 64 * j;
      qv[j] = (float)qb[g * D + d];
      kv[j] = (float)kn[d];
    }
#pragma unroll
    for (int r = 0; r < VEC; ++r) vv[r] = (float)vn[col + r];
    if constexpr (kFp8) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) kv[j] = e4m3_decode(e4m3_encode(kv[j] * sfk)) / sfk;
#pragma unroll
      for (int r = 0; r < VEC; ++r) vv[r] = e4m3_decode(e4m3_encode(vv[r] * sfv)) / sfv;
    }
    float M = kNegInf, L_sum = 0.f;
    typename std::conditional<VEC == 4, f32x4, float>::type O = {};
    fold_slots<VEC, stream_fold_width(VEC, S)>(a, g, idx, D, fcnt,
                                               [&](int i) { return base + f0 + i; }, M, L_sum, O);
    if constexpr (S > 1) combine_splitters(M, L_sum, O);
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < NQ; ++j) dot += qv[j] * kv[j];
#pragma unroll
    for (int o = 1; o < kDotLanes; o <<= 1) dot += __shfl_xor(dot, o);
    // Selects, not a branch: the page id's load is then waited for only here,
    // after the partials' loads were issued.
    const float sc = dot * a.scale_log2;
    const float mn = fmaxf(M, sc);
    const float f = new_ok ? exp2_fast(M - mn) : 1.f, w = new_ok ? exp2_fast(sc - mn) : 0.f;
    L_sum = L_sum * f + w;
    if (ml.split == 0) {
#pragma unroll
      for (int r = 0; r < VEC; ++r) {
        float o;
        if constexpr (VEC == 4) o = O[r];
        else o = O;
        out[idx + r] = Tr::from_float(L_sum > 0.f ? (o * f + vv[r] * w) / L_sum : 0.f);
      }
    }
  }

  // Append: the new rows go to the slot of position L-1.
  if (new_ok && blockIdx.z == 0) {
    if constexpr (kFp8) {
      const int64_t tile = page * Hkv + h;
      uint8_t* kp = static_cast<uint8_t*>(const_cast<void*>(a.k_pool)) + tile * D * kBS;
      uint8_t* vp = static_cast<uint8_t*>(const_cast<void*>(a.v_pool)) + tile * D * kBS;
      for (int d = threadIdx.x; d < D; d += blockDim.x) {
        kp[((d >> 4) * kBS + row) * 16 + (d & 15)] = (uint8_t)e4m3_encode((float)kn[d] * sfk);
        vp[fp8_v_offset(d, row, D)] = (uint8_t)e4m3_encode((float)vn[d] * sfv);
      }
      if (threadIdx.x == 0) {
        const_cast<float*>(a.k_scale)[tile * kBS + row] = sfk;
        const_cast<float*>(a.v_scale)[tile * kBS + row] = sfv;
      }
    } else {
      constexpr int X = 16 / (int)sizeof(E);
      const int64_t tile = (page * Hkv + h) * (int64_t)D * kBS;
      E* kp = static_cast<E*>(const_cast<void*>(a.k_pool)) + tile;
      E* vp = static_cast<E*>(const_cast<void*>(a.v_pool)) + tile;
      for (int d = threadIdx.x; d < D; d += blockDim.x) {
        kp[((d / X) * kBS + row) * X + d % X] = kn[d];
        vp[d * kBS + row] = vn[d];
      }
    }
  }
}

enum Stage { kFull = 0, kPartial = 1, kMerge = 2, kFused = 3 };

struct Plan {
  bool stream;
  int G, n_parts_max, part_pages;
  size_t acc_elems, ml_elems, pref_elems;
  size_t ws_bytes;
};

int make_plan(const char* name, Stage stage, int batch, int num_q_heads, int num_kv_heads,
              int head_dim, int block_size, int max_blocks, int window, int n_sink,
              int partition_pages, Plan* plan) {
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || max_blocks < 0)
    return fail(IVAKV_E_ARG, "%s: bad sizes B=%d Hq=%d Hkv=%d max_blocks=%d", name, batch,
                num_q_heads, num_kv_heads, max_blocks);
  if (num_q_heads % num_kv_heads != 0)
    return fail(IVAKV_E_SHAPE, "%s: num_q_heads %d not a multiple of num_kv_heads %d", name,
                num_q_heads, num_kv_heads);
  const int G = num_q_heads / num_kv_heads;
  if (G > 16) return fail(IVAKV_E_SHAPE, "%s: GQA group %d > 16 is not supported", name, G);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(IVAKV_E_SHAPE, "%s: head_dim %d not in {64,128,256}", name, head_dim);
  if (block_size != kBS)
    return fail(IVAKV_E_SHAPE, "%s: block_size %d != %d", name, block_size, kBS);
  if (n_sink < 0) return fail(IVAKV_E_ARG, "%s: negative n_sink", name);
  plan->G = G;
  plan->stream = partition_pages <= 0 && batch <= kMaxStreamBatch;
  const size_t units = (size_t)batch * num_kv_heads;
  if (plan->stream) {
    plan->part_pages = 0;
    plan->n_parts_max = 0;
    const size_t slots = (size_t)kMaxStreamWaves + units;
    plan->acc_elems = slots * G * (size_t)head_dim;
    plan->ml_elems = slots * G * 2;
    plan->pref_elems = (((size_t)batch + 1) + 3) & ~(size_t)3;
    plan->ws_bytes = (plan->acc_elems + plan->ml_elems + plan->pref_elems) * 4;
    return IVAKV_OK;
  }
  const int pp = partition_pages > 0 ? partition_pages : kDefaultPartitionPages;
  const int max_eff = max_effective_pages(max_blocks, window, n_sink, kBS);
  const int n_parts_max = max_eff > 0 ? cdiv(max_eff, pp) : 1;
  if (n_parts_max > 65535)
    return fail(IVAKV_E_SHAPE, "%s: %d partitions per sequence exceed 65535; raise partition_pages",
                name, n_parts_max);
  if (stage == kFused && n_parts_max > 1)
    return fail(IVAKV_E_SHAPE, "%s: the fused append runs on the stream walk (batch <= %d) or "
                "on one partition per sequence", name, kMaxStreamBatch);
  plan->part_pages = pp;
  plan->n_parts_max = n_parts_max;
  plan->pref_elems = 0;
  if (n_parts_max > 1) {
    plan->acc_elems = units * n_parts_max * G * (size_t)head_dim;
    plan->ml_elems = units * n_parts_max * G * 2;
    plan->ws_bytes = (plan->acc_elems + plan->ml_elems) * 4;
  } else {
    plan->acc_elems = plan->ml_elems = 0;
    plan->ws_bytes = 0;
  }
  return IVAKV_OK;
}

template <int DT, bool kFp8 = false>
void launch_partial(int D, dim3 grid, size_t smem, hipStream_t stream, const DecodeArgs& a) {
  switch (D) {
    case 64: decode_partial_kernel<DT, 64, kFp8><<<grid, kThreads, smem, stream>>>(a, a.bt, a.ctx); break;
    case 128: decode_partial_kernel<DT, 128, kFp8><<<grid, kThreads, smem, stream>>>(a, a.bt, a.ctx); break;
    default: decode_partial_kernel<DT, 256, kFp8><<<grid, kThreads, smem, stream>>>(a, a.bt, a.ctx); break;
  }
}

// The walk for pools of the query dtype, or of FP8 with per-slot scales.
template <int DT, bool kFp8, int D>
using WalkOps = typename std::conditional<kFp8, TileOps8<DT, D>, TileOps<DT, D>>::type;

template <int DT, bool kFp8 = false>
void launch_stream(Stage stage, int D, dim3 grid, size_t smem, hipStream_t stream,
                   const DecodeArgs& a) {
  if (stage != kMerge) {
    switch (D) {
      case 64: decode_stream_kernel<WalkOps<DT, kFp8, 64>><<<grid, kStreamThreads, smem, stream>>>(a, a.bt, a.ctx); break;
      case 128: decode_stream_kernel<WalkOps<DT, kFp8, 128>><<<grid, kStreamThreads, smem, stream>>>(a, a.bt, a.ctx); break;
      default: decode_stream_kernel<WalkOps<DT, kFp8, 256>><<<grid, kStreamThreads, smem, stream>>>(a, a.bt, a.ctx); break;
    }
  }
  // Merge grid: (kv head, sequence, column split) with one or four output elements
  // per thread, so every partial load of a unit is in flight at once; 64-thread
  // workgroups with four lanes per element when units are fewer than CUs, so few,
  // long sequences (many partials each) still merge on many CUs in one round trip.
  const int units = a.Hkv * a.batch;
  const bool vec4 = units >= kMergeVec4Units;
  const bool split = units < kMergeSplitUnits;
  // (four-element lanes: 128 threads hold a GQA-4, head_dim-128 unit's 512 outputs, so
  // no wave idles; C5's decode step 286.9 -> 285.8 us against 256-thread workgroups)
  const int threads = split ? 64 : vec4 ? 128 : 256;
  const int elems_per_wg = vec4 ? 4 * threads : split ? 16 * (threads / 64) : threads;
  const int zsplit = cdiv(a.G * D, elems_per_wg);
  const dim3 mgrid((unsigned)a.Hkv, (unsigned)a.batch, (unsigned)zsplit);
  if (stage == kFused) {
    if (vec4) {
      switch (D) {
        case 64: decode_fused_merge_kernel<DT, 64, kFp8, 4, 1><<<mgrid, threads, 0, stream>>>(a); break;
        case 128: decode_fused_merge_kernel<DT, 128, kFp8, 4, 1><<<mgrid, threads, 0, stream>>>(a); break;
        default: decode_fused_merge_kernel<DT, 256, kFp8, 4, 1><<<mgrid, threads, 0, stream>>>(a); break;
      }
    } else if (split) {
      switch (D) {
        case 64: decode_fused_merge_kernel<DT, 64, kFp8, 1, kSplitters><<<mgrid, threads, 0, stream>>>(a); break;
        case 128: decode_fused_merge_kernel<DT, 128, kFp8, 1, kSplitters><<<mgrid, threads, 0, stream>>>(a); break;
        default: decode_fused_merge_kernel<DT, 256, kFp8, 1, kSplitters><<<mgrid, threads, 0, stream>>>(a); break;
      }
    } else {
      switch (D) {
        case 64: decode_fused_merge_kernel<DT, 64, kFp8, 1, 1><<<mgrid, threads, 0, stream>>>(a); break;
        case 128: decode_fused_merge_kernel<DT, 128, kFp8, 1, 1><<<mgrid, threads, 0, stream>>>(a); break;
        default: decode_fused_merge_kernel<DT, 256, kFp8, 1, 1><<<mgrid, threads, 0, stream>>>(a); break;
      }
    }
  } else if (stage != kPartial) {
    if (vec4) decode_stream_merge_kernel<DT, 4, 1><<<mgrid, threads, 0, stream>>>(a, D);
    else if (split) decode_stream_merge_kernel<DT, 1, kSplitters><<<mgrid, threads, 0, stream>>>(a, D);
    else decode_stream_merge_kernel<DT, 1, 1><<<mgrid, threads, 0, stream>>>(a, D);
  }
}

// Workgroups of the stream walk on the current device: what its CUs hold at
// once, within the workspace's wave budget.
int stream_workgroups(int per_cu) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = kMaxStreamWaves / (kStreamWaves * per_cu);
  const int wgs = cus * per_cu;
  return wgs < kMaxStreamWaves / kStreamWaves ? wgs : kMaxStreamWaves / kStreamWaves;
}

// Fused calls on short tables whose batch has one to four (sequence, kv head) units
// per CU take one partition per sequence: a workgroup per unit walks it, merges its
// waves in LDS, folds the new token and writes out, with no merge kernel (C3's
// decode shape: 9.9 against 14.9 us for walk + merge; 512 units of 32 / 63 pages
// 28.4 / 49.1 against 32.4 / 52.9 us).  From four units per CU the stream walk's even
// shares win (1024 units: 54.6 / 94.9 against 57.2 / 98.7 us; 2048: 102.7 / 182.8
// against 115.8 / 204.0 us).  Returns the partition size for that, or 0 for the
// stream walk.
constexpr int kSinglePartitionMaxPages = 64;
int single_partition_pages(int batch, int num_kv_heads, int max_blocks, int window, int n_sink) {
  const int max_eff = max_effective_pages(max_blocks, window, n_sink, kBS);
  if (max_eff <= 0 || max_eff > kSinglePartitionMaxPages || batch > 65535) return 0;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  const int64_t units = (int64_t)batch * num_kv_heads;
  return units >= cus && units < 4 * (int64_t)cus ? max_eff : 0;
}

int decode_entry(Stage stage, const char* name, const void* q, const void* k_pool,
                 const void* v_pool, const int32_t* block_tables, const int32_t* context_lens,
                 void* out, void* workspace, size_t workspace_bytes, int batch, int num_q_heads,
                 int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_pages,
                 float scale, int window, int n_sink, int partition_pages, int dtype,
                 hipStream_t stream, const void* k_new = nullptr, const void* v_new = nullptr,
                 const float* k_scale = nullptr, const float* v_scale = nullptr, bool fp8 = false) {
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  if (fp8) {
    if (dtype != IVAKV_F16 && dtype != IVAKV_BF16)
      return fail(IVAKV_E_DTYPE, "%s: FP8 pools take fp16 or bf16 queries (dtype %d)", name, dtype);
    if (partition_pages > 0 || batch > kMaxStreamBatch)
      return fail(IVAKV_E_ARG, "%s: FP8 pools use the stream walk (partition_pages <= 0, "
                  "batch <= %d)", name, kMaxStreamBatch);
    if (batch > 0 && (!k_scale || !v_scale || !aligned16(k_scale) || !aligned16(v_scale)))
      return fail(IVAKV_E_ARG, "%s: k_scale / v_scale must be 16-byte aligned device pointers", name);
  }
  // The single launch for a full decode too (attention alone, the same kernel with no new
  // token): 256 units of 32 pages 18.3 -> 14.4 us, C3's layer shape 14.1 -> 9.8 us.
  if ((stage == kFused || stage == kFull) && partition_pages <= 0 && block_size == kBS &&
      n_sink >= 0)
    partition_pages = single_partition_pages(batch, num_kv_heads, max_blocks, window, n_sink);
  Plan plan;
  int st = make_plan(name, stage, batch, num_q_heads, num_kv_heads, head_dim, block_size,
                     max_blocks, window, n_sink, partition_pages, &plan);
  if (st != IVAKV_OK) return st;
  if (batch == 0) return IVAKV_OK;
  // An invalid page id is read as page 0 (then masked), so the pool needs a page.
  if (num_pages < 1) return fail(IVAKV_E_ARG, "%s: num_pages must be >= 1", name);
  if (!q || !k_pool || !v_pool || !context_lens || !out || (max_blocks > 0 && !block_tables))
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
  if (stage == kFused && (!k_new || !v_new))
    return fail(IVAKV_E_ARG, "%s: null k_new / v_new", name);
  if (!aligned16(q) || !aligned16(k_pool) || !aligned16(v_pool) || !aligned16(out))
    return fail(IVAKV_E_ARG, "%s: q, pools and out must be 16-byte aligned", name);
  if (plan.ws_bytes > 0 && (!workspace || workspace_bytes < plan.ws_bytes || !aligned16(workspace)))
    return fail(IVAKV_E_WORKSPACE, "%s: workspace of %zu bytes (16-byte aligned) required, got %zu",
                name, plan.ws_bytes, workspace ? workspace_bytes : (size_t)0);
  if (batch > 65535 || num_kv_heads > 65535)
    return fail(IVAKV_E_SHAPE, "%s: batch and num_kv_heads must be <= 65535", name);
  if (!(scale == scale)) return fail(IVAKV_E_ARG, "%s: scale is NaN", name);

  DecodeArgs a;
  a.q = q;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.bt = block_tables;
  a.ctx = context_lens;
  a.out = out;
  float* ws = static_cast<float*>(workspace);
  a.ws_acc = plan.ws_bytes ? ws : nullptr;
  a.ws_ml = plan.ws_bytes ? ws + plan.acc_elems : nullptr;
  a.ws_pref = plan.pref_elems ? reinterpret_cast<int32_t*>(ws + plan.acc_elems + plan.ml_elems)
                              : nullptr;
  a.batch = batch;
  a.Hkv = num_kv_heads;
  a.G = plan.G;
  a.max_blocks = max_blocks;
  a.num_pages = num_pages;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  a.window = window > 0 ? window : 0;
  a.n_sink = n_sink;
  a.part_pages = plan.part_pages;
  a.n_parts_max = plan.n_parts_max;
  a.n_waves = 0;
  a.k_new = k_new;
  a.v_new = v_new;
  a.fused = stage == kFused;
  a.k_scale = k_scale;
  a.v_scale = v_scale;

  if (plan.stream) {
    const int esize = fp8 ? 1 : dtype_size(dtype);
    const int wgs = stream_workgroups(walk_wgs_per_cu(2 * (int64_t)head_dim * kBS * esize));
    a.n_waves = wgs * kStreamWaves;
    const size_t smem = sizeof(int32_t) * ((size_t)batch + 1 + kStreamThreads);
    const dim3 grid((unsigned)wgs);
    if (fp8) {
      if (dtype == IVAKV_F16) launch_stream<IVAKV_F16, true>(stage, head_dim, grid, smem, stream, a);
      else launch_stream<IVAKV_BF16, true>(stage, head_dim, grid, smem, stream, a);
      return launch_status(name);
    }
    switch (dtype) {
      case IVAKV_F16: launch_stream<IVAKV_F16>(stage, head_dim, grid, smem, stream, a); break;
      case IVAKV_BF16: launch_stream<IVAKV_BF16>(stage, head_dim, grid, smem, stream, a); break;
      default: launch_stream<IVAKV_F32>(stage, head_dim, grid, smem, stream, a); break;
    }
    return launch_status(name);
  }
  if (stage == kFull || stage == kPartial || stage == kFused) {
    // Partition slowest: consecutive workgroups (which the dispatcher deals
    // round-robin to the 8 XCDs) are different kv heads / sequences of equal
    // partition index, so every XCD gets an even share of the pages.
    dim3 grid((unsigned)num_kv_heads, (unsigned)batch, (unsigned)plan.n_parts_max);
    const size_t smem =
        sizeof(float) * (2 * kWaves * 16 + 32 + (size_t)kWaves * plan.G * (head_dim + 4) + 16);
    if (fp8) {  // the fused step's single launch (FP8 pools take no partitions otherwise)
      if (dtype == IVAKV_F16) launch_partial<IVAKV_F16, true>(head_dim, grid, smem, stream, a);
      else launch_partial<IVAKV_BF16, true>(head_dim, grid, smem, stream, a);
      return launch_status(name);
    }
    switch (dtype) {
      case IVAKV_F16: launch_partial<IVAKV_F16>(head_dim, grid, smem, stream, a); break;
      case IVAKV_BF16: launch_partial<IVAKV_BF16>(head_dim, grid, smem, stream, a); break;
      default: launch_partial<IVAKV_F32>(head_dim, grid, smem, stream, a); break;
    }
    st = launch_status(name);
    if (st != IVAKV_OK) return st;
  }
  if ((stage == kFull || stage == kMerge) && plan.n_parts_max > 1) {
    dim3 grid((unsigned)num_kv_heads, (unsigned)batch);
    switch (dtype) {
      case IVAKV_F16: decode_merge_kernel<IVAKV_F16><<<grid, 256, 0, stream>>>(a, head_dim); break;
      case IVAKV_BF16: decode_merge_kernel<IVAKV_BF16><<<grid, 256, 0, stream>>>(a, head_dim); break;
      default: decode_merge_kernel<IVAKV_F32><<<grid, 256, 0, stream>>>(a, head_dim); break;
    }
    st = launch_status(name);
  }
  return st;
}

}  // namespace
}  // namespace ivakv

using namespace ivakv;

extern "C" int ivakv_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                           int head_dim, int block_size, int max_blocks,
                                           int window, int n_sink, int partition_pages,
                                           size_t* bytes) {
  if (!bytes) return fail(IVAKV_E_ARG, "ivakv_decode_workspace_size: null output pointer");
  Plan plan;
  const int st = make_plan("ivakv_decode_workspace_size", kFull, batch, num_q_heads, num_kv_heads,
                           head_dim, block_size, max_blocks, window, n_sink, partition_pages,
                           &plan);
  if (st != IVAKV_OK) return st;
  *bytes = plan.ws_bytes;
  return IVAKV_OK;
}

#define IVAKV_DECODE_ENTRY(fn, stage)                                                           \
  extern "C" int fn(const void* q, const void* k_pool, const void* v_pool,                      \
                    const int32_t* block_tables, const int32_t* context_lens, void* out,        \
                    void* workspace, size_t workspace_bytes, int batch, int num_q_heads,        \
                    int num_kv_heads, int head_dim, int block_size, int max_blocks,             \
                    int num_pages, float scale, int window, int n_sink, int partition_pages,    \
                    int dtype, hipStream_t stream) {                                            \
    return decode_entry(stage, #fn, q, k_pool, v_pool, block_tables, context_lens, out,         \
                        workspace, workspace_bytes, batch, num_q_heads, num_kv_heads, head_dim, \
                        block_size, max_blocks, num_pages, scale, window, n_sink,               \
                        partition_pages, dtype, stream);                                        \
  }

IVAKV_DECODE_ENTRY(ivakv_decode_attn, kFull)
IVAKV_DECODE_ENTRY(ivakv_decode_attn_partial, kPartial)
IVAKV_DECODE_ENTRY(ivakv_decode_attn_merge, kMerge)

extern "C" int ivakv_decode_append_attn(const void* q, const void* k_new, const void* v_new,
                                        void* k_pool, void* v_pool, const int32_t* block_tables,
                                        const int32_t* context_lens, void* out, void* workspace,
                                        size_t workspace_bytes, int batch, int num_q_heads,
                                        int num_kv_heads, int head_dim, int block_size,
                                        int max_blocks, int num_pages, float scale, int window,
                                        int n_sink, int dtype, hipStream_t stream) {
  return decode_entry(kFused, "ivakv_decode_append_attn", q, k_pool, v_pool, block_tables,
                      context_lens, out, workspace, workspace_bytes, batch, num_q_heads,
                      num_kv_heads, head_dim, block_size, max_blocks, num_pages, scale, window,
                      n_sink, 0, dtype, stream, k_new, v_new);
}

extern "C" int ivakv_decode_append_attn_fp8(const void* q, const void* k_new, const void* v_new,
                                            void* k_pool, void* v_pool, float* k_scale,
                                            float* v_scale, const int32_t* block_tables,
                                            const int32_t* context_lens, void* out,
                                            void* workspace, size_t workspace_bytes, int batch,
                                            int num_q_heads, int num_kv_heads, int head_dim,
                                            int block_size, int max_blocks, int num_pages,
                                            float scale, int window, int n_sink, int dtype,
                                            hipStream_t stream) {
  return decode_entry(kFused, "ivakv_decode_append_attn_fp8", q, k_pool, v_pool, block_tables,
                      context_lens, out, workspace, workspace_bytes, batch, num_q_heads,
                      num_kv_heads, head_dim, block_size, max_blocks, num_pages, scale, window,
                      n_sink, 0, dtype, stream, k_new, v_new, k_scale, v_scale, true);
}

extern "C" int ivakv_decode_attn_fp8(const void* q, const void* k_pool, const void* v_pool,
                                     const float* k_scale, const float* v_scale,
                                     const int32_t* block_tables, const int32_t* context_lens,
                                     void* out, void* workspace, size_t workspace_bytes,
                                     int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                     int block_size, int max_blocks, int num_pages, float scale,
                                     int window, int n_sink, int dtype, hipStream_t stream) {
  return decode_entry(kFull, "ivakv_decode_attn_fp8", q, k_pool, v_pool, block_tables,
                      context_lens, out, workspace, workspace_bytes, batch, num_q_heads,
                      num_kv_heads, head_dim, block_size, max_blocks, num_pages, scale, window,
                      n_sink, 0, dtype, stream, nullptr, nullptr, k_scale, v_scale, true);
}

// The fused decode step with a workspace of at most `capacity` bytes that get_ws
// supplies (called once, after the plan, when the plan needs one and a launch follows):
// ivakv_decode_append_attn_noalloc (ivakv_noalloc.hip) passes its static scratch.
// Same plan, kernels and results as ivakv_decode_append_attn.
int ivakv::decode_append_attn_capped(const char* name, const void* q, const void* k_new,
                                     const void* v_new, void* k_pool, void* v_pool,
                                     const int32_t* block_tables, const int32_t* context_lens,
                                     void* out, int batch, int num_q_heads, int num_kv_heads,
                                     int head_dim, int block_size, int max_blocks, int num_pages,
                                     float scale, int window, int n_sink, int dtype,
                                     hipStream_t stream, size_t capacity, WorkspaceSource get_ws) {
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  const int pp = block_size == kBS && n_sink >= 0
                     ? single_partition_pages(batch, num_kv_heads, max_blocks, window, n_sink)
                     : 0;
  Plan plan;
  const int st = make_plan(name, kFused, batch, num_q_heads, num_kv_heads, head_dim, block_size,
                           max_blocks, window, n_sink, pp, &plan);
  if (st != IVAKV_OK) return st;
  if (plan.ws_bytes > capacity)
    return fail(IVAKV_E_WORKSPACE,
                "%s: this geometry needs %zu bytes of workspace, more than the %zu bytes of "
                "the library's static scratch; call ivakv_decode_append_attn with a workspace",
                name, plan.ws_bytes, capacity);
  if (batch == 0) return IVAKV_OK;
  void* ws = nullptr;
  const int sst = get_ws(name, &ws);
  if (sst != IVAKV_OK) return sst;
  return decode_entry(kFused, name, q, k_pool, v_pool, block_tables, context_lens, out, ws,
                      capacity, batch, num_q_heads, num_kv_heads, head_dim, block_size,
                      max_blocks, num_pages, scale, window, n_sink, pp, dtype, stream, k_new,
                      v_new);
}
