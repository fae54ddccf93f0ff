// Paged single-query (decode) attention for gfx950.
//
// Work split: grid (partition, kv head, sequence), 4 wavefronts per workgroup.
// A partition is `part_pages` consecutive effective pages of one (sequence,
// kv head); wave w of the workgroup walks pages w, w+4, w+8, ... of it.  All
// Hq/Hkv query heads of the kv head share every page the wave loads (GQA reuse).
//
// Per page (16 rows) a wave issues D/X/4 16-byte K loads and D/16 V loads per
// lane.  The pool layout puts these loads directly in MFMA operand order:
//   S^T[row][head]  = K_page(16 x D) . Q^T(D x 16)      v_mfma 16x16x32 (f16/bf16)
//   O^T[dim][head] += V^T_page(D x 16) . P^T(16 x 16)   v_mfma 16x16x16 (f16/bf16)
// (16x16x4 f32 MFMAs for fp32).  The QK accumulator of lane l holds rows
// 4*(l/16)+r of head l%16, which is exactly the B operand layout the PV MFMA
// wants, so P never leaves registers.  Only heads l%16 < Hq/Hkv carry data.
//
// Softmax runs online in fp32 in the log2 domain (scale*log2(e) folded into the
// scores, v_exp_f32).  The four waves merge through LDS; a sequence that fits in
// one partition writes `out` directly, otherwise each partition writes an
// unnormalised (max, sum, acc) triple that decode_merge_kernel folds together.
#include "ivakv_internal.h"

namespace ivakv {
namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct alignas(16) Chunk16 {
  uint32_t w[4];
};
struct alignas(8) Chunk8 {
  uint32_t w[2];
};

constexpr int kBS = 16;       // rows per page == MFMA tile edge
constexpr int kWaves = 4;     // wavefronts per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kDefaultPartitionPages = 16;
constexpr float kNegInf = -__builtin_huge_valf();

struct DecodeArgs {
  const void* q;
  const void* k_pool;
  const void* v_pool;
  const int32_t* bt;
  const int32_t* ctx;
  void* out;
  float* ws_acc;  // [B][Hkv][n_parts_max][G][D]
  float* ws_ml;   // [B][Hkv][n_parts_max][G][2]  (max, sum)
  int Hkv, G, max_blocks, num_pages;
  float scale_log2;
  int window, n_sink, part_pages, n_parts_max;
};

// Zeroes the 16-bit V elements of rows that are not attended.  A row outside
// the context (tail of the last page, an invalid page) may hold any bits, and
// 0 * NaN would poison the PV accumulator even though its weight is zero.
__device__ inline void mask_rows16(Chunk8& v, const bool vis[4]) {
  v.w[0] &= (vis[0] ? 0x0000FFFFu : 0u) | (vis[1] ? 0xFFFF0000u : 0u);
  v.w[1] &= (vis[2] ? 0x0000FFFFu : 0u) | (vis[3] ? 0xFFFF0000u : 0u);
}

template <int DT>
struct Traits;

template <>
struct Traits<IVAKV_F16> {
  using E = _Float16;
  using VChunk = Chunk8;  // 4 consecutive rows of one dim
  using PVec = f16x4;
  static __device__ inline f32x4 qk(const Chunk16& k, const Chunk16& q, f32x4 s) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, k),
                                                  __builtin_bit_cast(f16x8, q), s, 0, 0, 0);
  }
  static __device__ inline PVec pack_p(const float p[4]) {
    return PVec{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
  }
  static __device__ inline f32x4 pv(const VChunk& v, const PVec& p, f32x4 acc) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, v), p, acc, 0, 0, 0);
  }
  static __device__ inline E from_float(float x) { return (E)x; }
  static __device__ inline void mask_rows(VChunk& v, const bool vis[4]) { mask_rows16(v, vis); }
};

// bf16 keeps only 8 significant bits, so P is carried as a hi + lo pair of bf16
// values (p = hi + lo to ~16 bits) and the PV product takes two MFMAs.
struct BF16Pair {
  i16x4 hi, lo;
};

template <>
struct Traits<IVAKV_BF16> {
  using E = __bf16;
  using VChunk = Chunk8;
  using PVec = BF16Pair;
  static __device__ inline f32x4 qk(const Chunk16& k, const Chunk16& q, f32x4 s) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, k),
                                                   __builtin_bit_cast(bf16x8, q), s, 0, 0, 0);
  }
  static __device__ inline PVec pack_p(const float p[4]) {
    bf16x4 hi{(__bf16)p[0], (__bf16)p[1], (__bf16)p[2], (__bf16)p[3]};
    bf16x4 lo{(__bf16)(p[0] - (float)hi[0]), (__bf16)(p[1] - (float)hi[1]),
              (__bf16)(p[2] - (float)hi[2]), (__bf16)(p[3] - (float)hi[3])};
    return PVec{__builtin_bit_cast(i16x4, hi), __builtin_bit_cast(i16x4, lo)};
  }
  static __device__ inline f32x4 pv(const VChunk& v, const PVec& p, f32x4 acc) {
    const i16x4 va = __builtin_bit_cast(i16x4, v);
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, p.hi, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, p.lo, acc, 0, 0, 0);
  }
  static __device__ inline E from_float(float x) { return (E)x; }
  static __device__ inline void mask_rows(VChunk& v, const bool vis[4]) { mask_rows16(v, vis); }
};

template <>
struct Traits<IVAKV_F32> {
  using E = float;
  using VChunk = Chunk16;
  using PVec = f32x4;
  static __device__ inline f32x4 qk(const Chunk16& k, const Chunk16& q, f32x4 s) {
    const f32x4 kf = __builtin_bit_cast(f32x4, k);
    const f32x4 qf = __builtin_bit_cast(f32x4, q);
#pragma unroll
    for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[i], qf[i], s, 0, 0, 0);
    return s;
  }
  static __device__ inline PVec pack_p(const float p[4]) { return PVec{p[0], p[1], p[2], p[3]}; }
  static __device__ inline f32x4 pv(const VChunk& v, const PVec& p, f32x4 acc) {
    const f32x4 vf = __builtin_bit_cast(f32x4, v);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[r], p[r], acc, 0, 0, 0);
    return acc;
  }
  static __device__ inline E from_float(float x) { return x; }
  static __device__ inline void mask_rows(VChunk& v, const bool vis[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) v.w[r] = vis[r] ? v.w[r] : 0u;
  }
};

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Partitions of one sequence, capped at the grid's partition count.  The cap only
// bites when context_lens[b] exceeds what the block table can address; every
// effective page it drops lies past max_blocks and would be masked anyway.
__device__ inline int num_partitions(const PageWalk& w, const DecodeArgs& a) {
  const int n = w.n_eff > 0 ? cdiv(w.n_eff, a.part_pages) : 1;
  return n < a.n_parts_max ? n : a.n_parts_max;
}

__device__ inline int logical_page(const PageWalk& w, int v) {
  return v < w.sink_pages ? v : w.win_first + (v - w.sink_pages);
}

template <int DT, int D>
__global__ __launch_bounds__(kThreads) void decode_partial_kernel(DecodeArgs a) {
  using Tr = Traits<DT>;
  using E = typename Tr::E;
  using VChunk = typename Tr::VChunk;
  constexpr int X = 16 / (int)sizeof(E);  // elements per 16-byte K chunk
  constexpr int KLD = D / X / 4;          // K loads per lane per page
  constexpr int NB = D / 16;              // 16-dim blocks (PV MFMAs per page)
  constexpr int64_t kTile = (int64_t)D * kBS;  // elements of one (page, head) tile

  const int part = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ln = lane & 15;  // MFMA column (query head) / row (K row, V dim)
  const int lq = lane >> 4;  // MFMA k-group
  const PageWalk w = make_walk(a.ctx[b], a.window, a.n_sink, kBS);
  const int n_parts = num_partitions(w, a);
  if (part >= n_parts) return;

  const int G = a.G;
  const int Hq = a.Hkv * G;
  const bool g_ok = ln < G;

  // Query rows of this kv head's group, in K-chunk order: chunk 4*j + lq.
  Chunk16 qr[KLD];
  {
    const E* qb = static_cast<const E*>(a.q) + ((int64_t)b * Hq + h * G + (g_ok ? ln : 0)) * D;
#pragma unroll
    for (int j = 0; j < KLD; ++j) {
      qr[j] = g_ok ? *reinterpret_cast<const Chunk16*>(qb + (4 * j + lq) * X) : Chunk16{{0u, 0u, 0u, 0u}};
    }
  }

  f32x4 acc[NB];
#pragma unroll
  for (int m = 0; m < NB; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;  // running max (log2 domain) of head ln
  float l_run = 0.f;      // this lane's share of the running sum

  const int v_first = part * a.part_pages + wave;
  const int v_stop = min((part + 1) * a.part_pages, w.n_eff);
  const E* kpool = static_cast<const E*>(a.k_pool);
  const E* vpool = static_cast<const E*>(a.v_pool);
  const int32_t* bt_row = a.bt + (int64_t)b * a.max_blocks;

  Chunk16 kc[KLD];
  VChunk vc[NB];
  int64_t cur_phys = -1;

  auto load_page = [&](int v, Chunk16* kd, VChunk* vd) -> int64_t {
    const int lp = logical_page(w, v);
    int64_t phys = lp < a.max_blocks ? (int64_t)bt_row[lp] : -1;
    if (phys < 0 || phys >= a.num_pages) phys = -1;
    const int64_t tile = ((phys < 0 ? 0 : phys) * a.Hkv + h) * kTile;
    const E* kp = kpool + tile;
    const E* vp = vpool + tile;
#pragma unroll
    for (int j = 0; j < KLD; ++j) kd[j] = *reinterpret_cast<const Chunk16*>(kp + ((4 * j + lq) * kBS + ln) * X);
#pragma unroll
    for (int m = 0; m < NB; ++m) vd[m] = *reinterpret_cast<const VChunk*>(vp + (16 * m + ln) * kBS + 4 * lq);
    return phys;
  };

  if (v_first < v_stop) cur_phys = load_page(v_first, kc, vc);
  for (int v = v_first; v < v_stop; v += kWaves) {
    Chunk16 kn[KLD];
    VChunk vn[NB];
    int64_t next_phys = -1;
    const bool more = v + kWaves < v_stop;
    if (more) next_phys = load_page(v + kWaves, kn, vn);

    // S^T = K . Q^T : lane holds rows 4*lq + r of head ln.
    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KLD; ++j) s = Tr::qk(kc[j], qr[j], s);

    const int pos0 = logical_page(w, v) * kBS + 4 * lq;
    float sl[4];
    bool vis[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int pos = pos0 + r;
      vis[r] = cur_phys >= 0 && pos < w.L && (pos >= w.win_start || pos < a.n_sink);
      sl[r] = vis[r] ? s[r] * a.scale_log2 : kNegInf;
    }
    // Unconditional (branch-free): a branch here would separate the QK MFMAs
    // from the first read of their accumulator by a basic-block boundary.
#pragma unroll
    for (int m = 0; m < NB; ++m) Tr::mask_rows(vc[m], vis);
    float mx = fmaxf(fmaxf(sl[0], sl[1]), fmaxf(sl[2], sl[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == kNegInf ? 0.f : m_new;
    const float alpha = exp2_fast(m_run - m_use);
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = exp2_fast(sl[r] - m_use);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    m_run = m_new;
#pragma unroll
    for (int m = 0; m < NB; ++m) acc[m] *= alpha;

    // O^T += V^T . P^T
    const typename Tr::PVec pv = Tr::pack_p(p);
#pragma unroll
    for (int m = 0; m < NB; ++m) acc[m] = Tr::pv(vc[m], pv, acc[m]);

    if (more) {
#pragma unroll
      for (int j = 0; j < KLD; ++j) kc[j] = kn[j];
#pragma unroll
      for (int m = 0; m < NB; ++m) vc[m] = vn[m];
      cur_phys = next_phys;
    }
  }

  // Row sum of head ln over the four k-groups.
  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot += __shfl_xor(l_tot, 32);

  // Merge the four waves through LDS.
  extern __shared__ float smem[];
  float* s_m = smem;                       // [kWaves][16]
  float* s_l = s_m + kWaves * 16;          // [kWaves][16]
  float* s_fin = s_l + kWaves * 16;        // [16][2] merged (max, sum)
  float* s_acc = s_fin + 32;               // [kWaves][G][D + 4]
  constexpr int kRow = D + 4;
  if (lq == 0) {
    s_m[wave * 16 + ln] = m_run;
    s_l[wave * 16 + ln] = l_tot;
  }
  __syncthreads();
  float M = kNegInf;
#pragma unroll
  for (int u = 0; u < kWaves; ++u) M = fmaxf(M, s_m[u * 16 + ln]);
  const float M_use = M == kNegInf ? 0.f : M;
  if (g_ok) {
    const float f = exp2_fast(m_run - M_use);
    float* dst = s_acc + (wave * G + ln) * kRow + 4 * lq;
#pragma unroll
    for (int m = 0; m < NB; ++m) *reinterpret_cast<f32x4*>(dst + 16 * m) = acc[m] * f;
    if (wave == 0 && lq == 0) {
      float L = 0.f;
#pragma unroll
      for (int u = 0; u < kWaves; ++u) L += s_l[u * 16 + ln] * exp2_fast(s_m[u * 16 + ln] - M_use);
      s_fin[2 * ln] = M;
      s_fin[2 * ln + 1] = L;
    }
  }
  __syncthreads();

  const bool direct = n_parts == 1;
  const int64_t part_base = (((int64_t)b * a.Hkv + h) * a.n_parts_max + part) * G;
  for (int idx = threadIdx.x; idx < G * D; idx += kThreads) {
    const int gg = idx / D, d = idx - (idx / D) * D;
    float o = 0.f;
#pragma unroll
    for (int u = 0; u < kWaves; ++u) o += s_acc[(u * G + gg) * kRow + d];
    if (direct) {
      const float L = s_fin[2 * gg + 1];
      const float r = L > 0.f ? o / L : 0.f;
      static_cast<E*>(a.out)[((int64_t)b * Hq + h * G + gg) * D + d] = Tr::from_float(r);
    } else {
      a.ws_acc[part_base * D + idx] = o;
      if (d == 0) {
        a.ws_ml[(part_base + gg) * 2] = s_fin[2 * gg];
        a.ws_ml[(part_base + gg) * 2 + 1] = s_fin[2 * gg + 1];
      }
    }
  }
}

// Log-sum-exp merge of the partitions of one (sequence, kv head).
template <int DT>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a, int D) {
  using Tr = Traits<DT>;
  using E = typename Tr::E;
  const int b = blockIdx.y, h = blockIdx.x;
  const PageWalk w = make_walk(a.ctx[b], a.window, a.n_sink, kBS);
  const int n_parts = num_partitions(w, a);
  if (n_parts <= 1) return;
  const int G = a.G;
  const int Hq = a.Hkv * G;
  const int64_t base = ((int64_t)b * a.Hkv + h) * a.n_parts_max;
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int gg = idx / D;
    float M = kNegInf;
    for (int p = 0; p < n_parts; ++p) M = fmaxf(M, a.ws_ml[((base + p) * G + gg) * 2]);
    const float M_use = M == kNegInf ? 0.f : M;
    float L = 0.f, o = 0.f;
    for (int p = 0; p < n_parts; ++p) {
      const float f = exp2_fast(a.ws_ml[((base + p) * G + gg) * 2] - M_use);
      L += a.ws_ml[((base + p) * G + gg) * 2 + 1] * f;
      o += a.ws_acc[(base + p) * G * D + idx] * f;
    }
    const float r = L > 0.f ? o / L : 0.f;
    static_cast<E*>(a.out)[((int64_t)b * Hq + h * G) * D + idx] = Tr::from_float(r);
  }
}

enum Stage { kFull = 0, kPartial = 1, kMerge = 2 };

struct Plan {
  int G, n_parts_max, part_pages;
  size_t ws_bytes;
};

int make_plan(const char* name, int batch, int num_q_heads, int num_kv_heads, int head_dim,
              int block_size, int max_blocks, int window, int n_sink, int partition_pages,
              Plan* plan) {
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
  const int pp = partition_pages > 0 ? partition_pages : kDefaultPartitionPages;
  const int max_eff = max_effective_pages(max_blocks, window, n_sink, kBS);
  const int n_parts_max = max_eff > 0 ? cdiv(max_eff, pp) : 1;
  plan->G = G;
  plan->part_pages = pp;
  plan->n_parts_max = n_parts_max;
  plan->ws_bytes = n_parts_max > 1 ? (size_t)batch * num_kv_heads * n_parts_max * G *
                                         ((size_t)head_dim + 2) * sizeof(float)
                                   : 0;
  return IVAKV_OK;
}

template <int DT>
void launch_partial(int D, dim3 grid, size_t smem, hipStream_t stream, const DecodeArgs& a) {
  switch (D) {
    case 64: decode_partial_kernel<DT, 64><<<grid, kThreads, smem, stream>>>(a); break;
    case 128: decode_partial_kernel<DT, 128><<<grid, kThreads, smem, stream>>>(a); break;
    default: decode_partial_kernel<DT, 256><<<grid, kThreads, smem, stream>>>(a); break;
  }
}

int decode_entry(Stage stage, const char* name, const void* q, const void* k_pool,
                 const void* v_pool, const int32_t* block_tables, const int32_t* context_lens,
                 void* out, void* workspace, size_t workspace_bytes, int batch, int num_q_heads,
                 int num_kv_heads, int head_dim, int block_size, int max_blocks, int num_pages,
                 float scale, int window, int n_sink, int partition_pages, int dtype,
                 hipStream_t stream) {
  if (dtype_size(dtype) == 0) return fail(IVAKV_E_DTYPE, "%s: unknown dtype code %d", name, dtype);
  Plan plan;
  int st = make_plan(name, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks,
                     window, n_sink, partition_pages, &plan);
  if (st != IVAKV_OK) return st;
  if (batch == 0) return IVAKV_OK;
  // An invalid page id is read as page 0 (then masked), so the pool needs a page.
  if (num_pages < 1) return fail(IVAKV_E_ARG, "%s: num_pages must be >= 1", name);
  if (!q || !k_pool || !v_pool || !context_lens || !out || (max_blocks > 0 && !block_tables))
    return fail(IVAKV_E_ARG, "%s: null pointer argument", name);
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
  const size_t acc_elems = (size_t)batch * num_kv_heads * plan.n_parts_max * plan.G * head_dim;
  a.ws_acc = plan.ws_bytes ? ws : nullptr;
  a.ws_ml = plan.ws_bytes ? ws + acc_elems : nullptr;
  a.Hkv = num_kv_heads;
  a.G = plan.G;
  a.max_blocks = max_blocks;
  a.num_pages = num_pages;
  a.scale_log2 = (float)((double)scale * 1.4426950408889634);
  a.window = window > 0 ? window : 0;
  a.n_sink = n_sink;
  a.part_pages = plan.part_pages;
  a.n_parts_max = plan.n_parts_max;

  if (stage == kFull || stage == kPartial) {
    dim3 grid((unsigned)plan.n_parts_max, (unsigned)num_kv_heads, (unsigned)batch);
    const size_t smem = sizeof(float) * (2 * kWaves * 16 + 32 + (size_t)kWaves * plan.G * (head_dim + 4));
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
  const int st = make_plan("ivakv_decode_workspace_size", batch, num_q_heads, num_kv_heads,
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
