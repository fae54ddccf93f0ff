/*
 * ivakv.h -- C ABI of libivakv.so, the MI355X (gfx950) paged KV-cache library.
 *
 * Scope: the paged KV-cache hot path of IVA1.0 -- appending new K/V rows into
 * block-table pages, gathering pages back to contiguous K/V, and paged
 * single-query (decode) attention with grouped-query heads, sliding window and
 * attention sinks -- plus the reference's index gather/scatter op.
 *
 * Conventions
 *   - Every entry point returns IVAKV_OK (0) or a negative IVAKV_E_* code and
 *     never throws across the ABI.  On error, ivakv_last_error() returns a
 *     thread-local message describing it.
 *   - All pointers except `stream` and host scalars are DEVICE pointers owned by
 *     the caller (the library never allocates or frees device memory).
 *   - Work is enqueued asynchronously on `stream` (NULL = the default stream).
 *     Argument checks run on the host before any launch.
 *   - Integer indices read from device memory (slot ids, page ids, context
 *     lengths, positions) are bounds-checked inside the kernels: an out-of-range
 *     slot is skipped by append/scatter, an out-of-range page reads as empty.
 *
 * Paged pool layout (esize = bytes per element, X = 16 / esize, BS = block_size):
 *   k_pool = [num_pages][Hkv][D / X][BS][X]   K(page,h,t,d) at ((d/X)*BS + t)*X + d%X
 *   v_pool = [num_pages][Hkv][D][BS]          V(page,h,t,d) at d*BS + t
 * Both pools are dense.  A slot s names page s / BS, in-page row s % BS.
 * A 16-row page of one KV head is 16*D*esize contiguous bytes for K and for V
 * (4 KiB each at D=128 fp16): one page is a handful of fully-coalesced 1 KiB
 * wavefront loads, already in the operand order of the 16x16 MFMA tiles.
 *
 * Reference interfaces replaced (paths relative to the IVA1.0 source tree):
 *   src/core/rope_kv.py:71-137        KVCache (contiguous [B,H,S,D] cache)
 *   src/core/attention.py:61-102      AttentionTorch.forward cache append + math
 *   src/kernels_t/kv_ops_triton.py:18-156  kv_gather/kv_scatter kernels, kv_ops_triton
 */
#ifndef IVAKV_H
#define IVAKV_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IVAKV_ABI_VERSION 2

/* status codes */
#define IVAKV_OK            0
#define IVAKV_E_ARG        -1  /* null pointer, negative size, bad stride */
#define IVAKV_E_DTYPE      -2  /* unknown dtype code */
#define IVAKV_E_SHAPE      -3  /* geometry the kernels do not support */
#define IVAKV_E_LAUNCH     -4  /* HIP reported an error at launch */
#define IVAKV_E_WORKSPACE  -5  /* workspace missing or too small */

/* dtype codes (element type of K, V, Q and outputs) */
#define IVAKV_F32   0
#define IVAKV_F16   1
#define IVAKV_BF16  2

/* ABI version compiled into the library (== IVAKV_ABI_VERSION). */
int ivakv_abi_version(void);

/* Thread-local description of the last error returned on this thread. */
const char* ivakv_last_error(void);

/*
 * Append: scatter n_tok new K/V rows into their slots.
 *   k_new(t, h, d) = k_new[t*k_tok_stride + h*k_head_stride + d]   (elements)
 *   slot_mapping[t] = slot of token t; -1 (or any id outside
 *   [0, num_pages*block_size)) leaves the pools untouched for that token.
 * Bit-exact data movement.  Duplicate slots in one call: one of the writers
 * wins (unspecified which), as for the reference scatter.
 * Replaces: KVCache.update slice-assign (src/core/rope_kv.py:98-110), the
 * torch.cat append (src/core/attention.py:61-63) and the scatter branch of
 * KVOpsTriton (src/kernels_t/kv_ops_triton.py:43-65,125-140).
 */
int ivakv_append(const void* k_new, const void* v_new,
                 int64_t k_tok_stride, int64_t k_head_stride,
                 int64_t v_tok_stride, int64_t v_head_stride,
                 void* k_pool, void* v_pool, const int32_t* slot_mapping,
                 int n_tok, int num_kv_heads, int head_dim, int block_size,
                 int num_pages, int dtype, hipStream_t stream);

/*
 * Gather: pages -> contiguous k_out/v_out = [batch][Hkv][out_len][D] (dense).
 * Row p < min(context_lens[b], out_len) of sequence b comes from slot
 * block_tables[b*max_blocks + p/BS]*BS + p%BS; all other rows are zero.
 * Output keeps the pool dtype.  Bit-exact data movement.
 * Replaces: KVCache.get_slice / .k / .v (src/core/rope_kv.py:136-137) and the
 * gather branch of KVOpsTriton (src/kernels_t/kv_ops_triton.py:18-40,111-123).
 */
int ivakv_gather(const void* k_pool, const void* v_pool,
                 const int32_t* block_tables, const int32_t* context_lens,
                 int batch, int max_blocks, int num_kv_heads, int head_dim,
                 int block_size, int num_pages, int out_len,
                 void* k_out, void* v_out, int dtype, hipStream_t stream);

/*
 * Bytes of device workspace ivakv_decode_attn (and its _partial/_merge halves)
 * needs for this geometry.  The default walk (partition_pages <= 0, batch <=
 * 8192) keeps one fp32 partial (max, sum, acc[G][D]) per wave of its wave
 * budget (4096) plus one per (sequence, kv head), and the batch's page prefix.
 * partition_pages > 0 selects the partitioned walk, whose workspace holds one
 * partial per (sequence, kv head, partition) and is 0 when no sequence spans
 * more than one partition.  The contents need no initialisation; calls that
 * share a workspace must not run concurrently.
 */
int ivakv_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                int head_dim, int block_size, int max_blocks,
                                int window, int n_sink, int partition_pages,
                                size_t* bytes);

/*
 * Paged decode attention (one query row per sequence):
 *   out[b, hq, :] = softmax_j(scale * q[b,hq,:] . K_b[j,:]) V_b[j,:]
 * over the visible positions j of sequence b, with L = context_lens[b]:
 *   j < L  and  (window <= 0  or  j >= L - window  or  j < n_sink).
 * KV head of query head hq is hq / (num_q_heads / num_kv_heads).
 * q, out = [batch][num_q_heads][D] dense.  L == 0 gives a zero row.
 * fp32 accumulation.  Default walk: the (sequence, kv head, page) tiles of the
 * whole batch are dealt out in equal contiguous shares to a fixed set of
 * wavefronts sized to the device; a (sequence, kv head) split between
 * wavefronts is merged with a log-sum-exp reduction.  partition_pages > 0
 * instead splits each sequence into partitions of that many pages (one
 * workgroup each) merged the same way.  With partition_pages <= 0, a batch of one
 * to four (sequence, kv head) units per CU on tables of at most 64 effective pages
 * takes one partition per sequence in a single launch (no merge: the call then
 * accepts a null workspace; ivakv_decode_workspace_size still reports the stream
 * walk's need, which covers it).
 * Supported: block_size 16, head_dim 64/128/256, num_q_heads/num_kv_heads
 * (the GQA group) any integer from 1 to 16.
 * Replaces: the cache branch of AttentionTorch.forward -- scores, causal /
 * sliding-window / sink masks, softmax, PV (src/core/attention.py:77-102,
 * 115-148) -- on the paged cache.
 */
int ivakv_decode_attn(const void* q, const void* k_pool, const void* v_pool,
                      const int32_t* block_tables, const int32_t* context_lens,
                      void* out, void* workspace, size_t workspace_bytes,
                      int batch, int num_q_heads, int num_kv_heads, int head_dim,
                      int block_size, int max_blocks, int num_pages, float scale,
                      int window, int n_sink, int partition_pages, int dtype,
                      hipStream_t stream);

/*
 * The two launches of ivakv_decode_attn, same arguments and same walk.
 * _partial runs the paged walk (writing `out` directly for every (sequence, kv
 * head) a single wavefront or partition covers); _merge folds the partials of
 * the others into `out` (and zero-fills empty sequences).  Exposed so a caller
 * can time the walk alone or merge partials that come from several devices
 * (context-parallel sharding of one sequence).
 * Replaces: same reference code as ivakv_decode_attn.
 */
int ivakv_decode_attn_partial(const void* q, const void* k_pool, const void* v_pool,
                              const int32_t* block_tables, const int32_t* context_lens,
                              void* out, void* workspace, size_t workspace_bytes,
                              int batch, int num_q_heads, int num_kv_heads, int head_dim,
                              int block_size, int max_blocks, int num_pages, float scale,
                              int window, int n_sink, int partition_pages, int dtype,
                              hipStream_t stream);
int ivakv_decode_attn_merge(const void* q, const void* k_pool, const void* v_pool,
                            const int32_t* block_tables, const int32_t* context_lens,
                            void* out, void* workspace, size_t workspace_bytes,
                            int batch, int num_q_heads, int num_kv_heads, int head_dim,
                            int block_size, int max_blocks, int num_pages, float scale,
                            int window, int n_sink, int partition_pages, int dtype,
                            hipStream_t stream);

/*
 * Fused decode step: append, then attend.  Position L-1 = context_lens[b]-1 of every
 * sequence is the new token; its rows k_new / v_new ([batch][Hkv][D] dense, pool
 * dtype) are written to that position's slot (block_tables[b][(L-1)/BS]*BS +
 * (L-1)%BS; skipped when that page id is outside the table or the pool) and
 * attended together with positions < L-1 read from the pools.  Same result as
 * ivakv_append of those rows followed by ivakv_decode_attn, in two launches
 * instead of three: the pool walk skips position L-1 and the merge scores the new
 * token straight from k_new.  When the batch has one to four (sequence, kv head)
 * units per CU of the device and the table holds at most 64 effective pages per
 * sequence (max_blocks, or the window and sinks), one launch: a workgroup per unit
 * walks it, merges its waves in LDS, folds in the new token and stores its rows.
 * Workspace: ivakv_decode_workspace_size with partition_pages <= 0 (enough for
 * either).  Supported geometry as ivakv_decode_attn, batch <= 8192.
 * Replaces: the append + score sequence of AttentionTorch.forward with a cache
 * (src/core/attention.py:61-102): torch.cat of the new K/V, then the attention
 * math over the extended cache.
 */
int ivakv_decode_append_attn(const void* q, const void* k_new, const void* v_new,
                             void* k_pool, void* v_pool, const int32_t* block_tables,
                             const int32_t* context_lens, void* out, void* workspace,
                             size_t workspace_bytes, int batch, int num_q_heads,
                             int num_kv_heads, int head_dim, int block_size, int max_blocks,
                             int num_pages, float scale, int window, int n_sink, int dtype,
                             hipStream_t stream);

/*
 * ivakv_decode_append_attn without a workspace argument: the same plan, kernels and
 * results as ivakv_decode_append_attn, with the decode workspace taken from a
 * file-scope device array of the library (64 MiB per device).  The array sits in a code
 * object of its own (ivakv_noalloc.hip), which a device maps on the first call of this
 * entry point there and holds until the process ends; the library's other entry points
 * leave it unmapped.  It allocates nothing: no hipMalloc, hipFree or allocating library
 * call.  A geometry whose workspace exceeds 64 MiB (see ivakv_decode_workspace_size: at
 * GQA 4, D 128 a slot takes 2080 B and 4096 slots are the wave budget, so more than
 * ~28k (sequence, kv head) units, ~3.5k sequences at 8 kv heads) returns
 * IVAKV_E_WORKSPACE before any launch.  Every call on one device shares
 * that device's array: calls that overlap on one device (different streams, or
 * threads) race and must be serialised by the caller.  Nothing in the array needs to
 * start at zero.
 * No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 */
int ivakv_decode_append_attn_noalloc(const void* q, const void* k_new, const void* v_new,
                                     void* k_pool, void* v_pool, const int32_t* block_tables,
                                     const int32_t* context_lens, void* out, int batch,
                                     int num_q_heads, int num_kv_heads, int head_dim,
                                     int block_size, int max_blocks, int num_pages, float scale,
                                     int window, int n_sink, int dtype, hipStream_t stream);

/*
 * FP8 KV pages (OCP e4m3fn codes, one byte per element) with one fp32 scaling factor
 * per (slot, kv head):
 *   k_pool  [num_pages][Hkv][D/16][BS][16] bytes (16-byte chunks of 16 dims)
 *   v_pool  [num_pages][Hkv][D * BS] bytes; within a tile the code of (dim d,
 *           key t) is at ((d%16 * 4 + t/4) * D/16 + d/16) * 4 + t%4, so each lane of
 *           the decode walk reads its V bytes as whole 16-byte loads
 *   k_scale, v_scale [num_pages][Hkv][BS] fp32
 * A row x of one (token, kv head) is stored as e4m3(x * sf), sf = 448 / max|x|
 * (1 for an all-zero row), clamped to [1e-8, 1e8] (a row holding a NaN or an infinity
 * gets 1e-8, as the reference's rule evaluates), rounded to nearest even and saturated
 * at +-448 (NaN code 0x7F); it reads back as code / sf.  BS = 16, head_dim in {64,128,256}.
 * Replaces: the reference's kv_cache_dtype "fp8" (configs/quant_infer.yaml:22,52),
 * with its scaling rule (src/quant/fp8_runtime.py:66-76) applied per row.
 *
 * ivakv_append_fp8: ivakv_append for FP8 pools; k_new / v_new rows of dtype f32 / f16 /
 * bf16 with element strides as in ivakv_append.  Skips slots outside the pool.
 */
int ivakv_append_fp8(const void* k_new, const void* v_new, int64_t k_tok_stride,
                     int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
                     void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                     const int32_t* slot_mapping, int n_tok, int num_kv_heads, int head_dim,
                     int block_size, int num_pages, int dtype, hipStream_t stream);
/*
 * ivakv_gather_fp8: ivakv_gather for FP8 pools, dequantized (code / sf) into outputs of
 * dtype `dtype` (f32 / f16 / bf16, [batch][Hkv][out_len][D] dense); zero past the
 * context or on an invalid page id.  16-byte aligned pools and outputs take a kernel
 * that moves 16-element chunks; any other alignment an element-wise one (same values).
 */
int ivakv_gather_fp8(const void* k_pool, const void* v_pool, const float* k_scale,
                     const float* v_scale, const int32_t* block_tables,
                     const int32_t* context_lens, int batch, int max_blocks, int num_kv_heads,
                     int head_dim, int block_size, int num_pages, int out_len, void* k_out,
                     void* v_out, int dtype, hipStream_t stream);
/*
 * ivakv_decode_attn_fp8: ivakv_decode_attn over FP8 pools (stream walk); q and out of
 * dtype f16 or bf16 (`dtype`), scores and softmax in fp32 on the dequantized keys and
 * values.  Workspace: ivakv_decode_workspace_size with partition_pages <= 0;
 * batch <= 8192.  k_scale / v_scale 16-byte aligned.
 */
int ivakv_decode_attn_fp8(const void* q, const void* k_pool, const void* v_pool,
                          const float* k_scale, const float* v_scale,
                          const int32_t* block_tables, const int32_t* context_lens, void* out,
                          void* workspace, size_t workspace_bytes, int batch, int num_q_heads,
                          int num_kv_heads, int head_dim, int block_size, int max_blocks,
                          int num_pages, float scale, int window, int n_sink, int dtype,
                          hipStream_t stream);

/*
 * ivakv_decode_append_attn_fp8: ivakv_decode_append_attn over FP8 pools.  The new rows
 * k_new / v_new ([batch][Hkv][D], dtype `dtype` like q) are quantized exactly as
 * ivakv_append_fp8 quantizes them (the pools and factors afterwards are byte-identical
 * to that append's), attended as their dequantized values, and stored into the slot of
 * position L-1; positions < L-1 come from the pools as in ivakv_decode_attn_fp8.  Same
 * result as ivakv_append_fp8 followed by ivakv_decode_attn_fp8, in two launches
 * instead of three (one on the batches where ivakv_decode_append_attn takes one).
 * Workspace, geometry and alignment as ivakv_decode_attn_fp8.
 * Replaces: the append + score sequence of AttentionTorch.forward with a cache
 * (src/core/attention.py:61-102) on a kv_cache_dtype "fp8" cache
 * (configs/quant_infer.yaml:22,52; scaling rule src/quant/fp8_runtime.py:66-76).
 */
int ivakv_decode_append_attn_fp8(const void* q, const void* k_new, const void* v_new,
                                 void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                                 const int32_t* block_tables, const int32_t* context_lens,
                                 void* out, void* workspace, size_t workspace_bytes, int batch,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 int block_size, int max_blocks, int num_pages, float scale,
                                 int window, int n_sink, int dtype, hipStream_t stream);

/*
 * Rotary position embedding as the reference's RoPE module defines it
 * (src/core/rope_kv.py:22-50): dims (2i, 2i+1) of a head rotate by a = p * f_i at absolute
 * position p, f_i = 1 / theta^(2i/D) (double, stored as float), a = float(p) * f_i:
 *   y[2i] = x[2i] cos a - x[2i+1] sin a,  y[2i+1] = x[2i] sin a + x[2i+1] cos a
 * in fp32, rounded once to the element type.  The reference computes this state but its
 * attention leaves q and k unrotated (attention.py:57-59,112-113); these entry points are
 * the rotation it describes.
 *
 * ivakv_rope: x [n_tok][num_heads][D] (element strides per token and head), rotated in
 * place at positions[t] (int32).  D even.
 */
int ivakv_rope(void* x, int64_t tok_stride, int64_t head_stride, const int32_t* positions,
               int n_tok, int num_heads, int head_dim, float theta, int dtype,
               hipStream_t stream);
/*
 * ivakv_append_rope: ivakv_append with every K row rotated at positions[t] on its way into
 * the page (V rows unchanged).  Replaces: the k rotation of AttentionTorch.forward
 * (attention.py:57-59) followed by the cache append (attention.py:61-63).
 */
int ivakv_append_rope(const void* k_new, const void* v_new, int64_t k_tok_stride,
                      int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
                      void* k_pool, void* v_pool, const int32_t* slot_mapping,
                      const int32_t* positions, int n_tok, int num_kv_heads, int head_dim,
                      int block_size, int num_pages, float theta, int dtype, hipStream_t stream);
/*
 * ivakv_append_rope_fp8: ivakv_append_fp8 with every K row rotated at positions[t] first
 * (the rotation of ivakv_append_rope, rounded once to the source dtype; V rows
 * unchanged): codes and factors equal those of ivakv_rope on the K rows followed by
 * ivakv_append_fp8, in one launch.  Source dtype f32 / f16 / bf16, head_dim in
 * {64, 128, 256}, block_size 16; slots outside the pool are skipped.  Replaces: the k
 * rotation of AttentionTorch.forward (attention.py:57-59) followed by the cache append
 * (attention.py:61-63) on a kv_cache_dtype "fp8" cache (configs/quant_infer.yaml:22,52).
 */
int ivakv_append_rope_fp8(const void* k_new, const void* v_new, int64_t k_tok_stride,
                          int64_t k_head_stride, int64_t v_tok_stride, int64_t v_head_stride,
                          void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                          const int32_t* slot_mapping, const int32_t* positions, int n_tok,
                          int num_kv_heads, int head_dim, int block_size, int num_pages,
                          float theta, int dtype, hipStream_t stream);
/*
 * ivakv_copy_pages: page moves src_pages[i] -> dst_pages[i] (int32, n_moves <= 65535) of a
 * pool pair of num_pages pages, K and V tiles of every kv head (elem_bytes 1, 2 or 4), plus
 * the FP8 scaling factors when k_scale / v_scale are given (both or neither).  The source
 * and destination sets must be disjoint.  A move whose source or destination id lies
 * outside [0, num_pages) is skipped.  Used by pool compaction (PagedKVPool.compact), the
 * paged counterpart of kv_compact_triton (src/kernels_t/kv_ops_triton.py:68-92,159-181).
 */
int ivakv_copy_pages(void* k_pool, void* v_pool, float* k_scale, float* v_scale,
                     const int32_t* src_pages, const int32_t* dst_pages, int n_moves,
                     int num_pages, int num_kv_heads, int head_dim, int block_size,
                     int elem_bytes, hipStream_t stream);

/*
 * Paged multi-query causal attention (prefill / chunked prefill).  Sequence b owns
 * query rows query_start[b] .. query_start[b+1]-1 of q ([n_tok][Hq][D] dense, pool
 * dtype); with n_b rows and context length L = context_lens[b], row i sits at
 * absolute position p = L - n_b + i and its K/V must already be in the pages
 * (ivakv_append first).  Row i of query head h attends to the keys j <= p of
 * kv head h / (Hq/Hkv) with j > p - window (all when window <= 0) or j < n_sink,
 * over valid page ids; out has q's shape.  A row at a negative position (n_b > L)
 * and a row that sees no key are written as zeros.  max_query_len must be >= every
 * n_b (rows past it are not computed).  query_start is int32 [batch+1], non-
 * decreasing, query_start[0] = 0 and query_start[batch] <= n_tok (the rows of q and
 * out).  The kernel reads it from device memory and skips (writes nothing for) a
 * sequence whose rows [query_start[b], query_start[b+1]) do not lie in [0, n_tok).
 * Geometry: head_dim in {64, 128, 256}, block_size 16, any GQA group.
 * Replaces: AttentionTorch.forward with a cache and seq_len > 1
 * (src/core/attention.py:61-102): torch.cat of the chunk's K/V, scores, causal /
 * window / sink masks (attention.py:79-93,115-148) at absolute positions, softmax, PV.
 */
int ivakv_prefill_attn(const void* q, const void* k_pool, const void* v_pool,
                       const int32_t* block_tables, const int32_t* context_lens,
                       const int32_t* query_start, int n_tok, void* out, int batch,
                       int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                       int max_blocks, int num_pages, int max_query_len, float scale,
                       int window, int n_sink, int dtype, hipStream_t stream);

/*
 * ivakv_prefill_attn_fp8: ivakv_prefill_attn over FP8 pools (layout and factors as
 * ivakv_append_fp8 writes them); q and out of dtype f16 or bf16 (`dtype`).  Keys and
 * values are dequantized, code / sf rounded once to `dtype`, as they are staged into
 * LDS; the attention is then the 16-bit kernel's.  k_scale / v_scale 16-byte aligned.
 * Replaces: the same reference code as ivakv_prefill_attn on a kv_cache_dtype "fp8"
 * cache (configs/quant_infer.yaml:22,52; scaling rule src/quant/fp8_runtime.py:66-76).
 */
int ivakv_prefill_attn_fp8(const void* q, const void* k_pool, const void* v_pool,
                           const float* k_scale, const float* v_scale,
                           const int32_t* block_tables, const int32_t* context_lens,
                           const int32_t* query_start, int n_tok, void* out, int batch,
                           int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                           int max_blocks, int num_pages, int max_query_len, float scale,
                           int window, int n_sink, int dtype, hipStream_t stream);

/*
 * Bytes of device workspace ivakv_prefill_attn_split(_fp8) needs for this geometry:
 * the plan (item queues, per-row-block segments), and 512 fp32 partial slots of one
 * row block each (the rows of one workgroup: 256 at head_dim <= 128 in fp16 / bf16)
 * with a running max and row sum per row: about 65 MiB at head_dim 128.
 */
int ivakv_prefill_split_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                       int head_dim, int max_query_len, int dtype,
                                       size_t* bytes);

/*
 * ivakv_prefill_attn with each row block's walk split along the keys: the same
 * arguments and results (within the attention tolerance: segments round P to the
 * query dtype against their own running maxima), for batches whose longest chunks
 * sit on long contexts.  ivakv_prefill_attn gives a row block one workgroup, so a
 * 512-token chunk at 16k keys occupies 64 workgroups for the whole launch; here a plan
 * kernel cuts every row block's walk into segments of about (total work / CUs), and a
 * persistent grid (one workgroup per CU) runs the (row block, segment) items, longest
 * sequences first, from per-XCD queues; the workgroup that finishes a split block's
 * last segment folds its segments by log-sum-exp.  Two launches, no host
 * synchronisation (graph capture safe).  batch <= 2048, num_kv_heads <= 32767.  The
 * workspace (ivakv_prefill_split_workspace_size) needs no initialisation; calls that
 * share a workspace must not run concurrently.
 * Replaces: the same reference code as ivakv_prefill_attn.
 */
int ivakv_prefill_attn_split(const void* q, const void* k_pool, const void* v_pool,
                             const int32_t* block_tables, const int32_t* context_lens,
                             const int32_t* query_start, int n_tok, void* out,
                             void* workspace, size_t workspace_bytes, int batch,
                             int num_q_heads, int num_kv_heads, int head_dim, int block_size,
                             int max_blocks, int num_pages, int max_query_len, float scale,
                             int window, int n_sink, int dtype, hipStream_t stream);

/* ivakv_prefill_attn_split over FP8 pools, as ivakv_prefill_attn_fp8. */
int ivakv_prefill_attn_split_fp8(const void* q, const void* k_pool, const void* v_pool,
                                 const float* k_scale, const float* v_scale,
                                 const int32_t* block_tables, const int32_t* context_lens,
                                 const int32_t* query_start, int n_tok, void* out,
                                 void* workspace, size_t workspace_bytes, int batch,
                                 int num_q_heads, int num_kv_heads, int head_dim,
                                 int block_size, int max_blocks, int num_pages,
                                 int max_query_len, float scale, int window, int n_sink,
                                 int dtype, hipStream_t stream);

/*
 * Index gather on a contiguous-layout cache kv = [batch][n_heads][seq_len][D]
 * with element strides (s_b, s_h, s_s, s_d):
 *   out[b, h, j, :] = kv[b, h, indices[j], :]      out = [B][H][n_idx][D] dense
 * indices are int64 on the device, shared by every (b, h).  An index outside
 * [0, seq_len) yields a zero row.
 * Replaces: kv_gather_kernel + the gather branch of KVOpsTriton
 * (src/kernels_t/kv_ops_triton.py:18-40,111-123).
 */
int ivakv_index_gather(const void* kv, int64_t s_b, int64_t s_h, int64_t s_s, int64_t s_d,
                       const int64_t* indices, int n_idx,
                       int batch, int n_heads, int seq_len, int head_dim,
                       void* out, int dtype, hipStream_t stream);

/*
 * Index scatter, in place: kv[b, h, indices[j], :] = values[b, h, j, :] with
 * values strides (v_b, v_h, v_s, v_d).  Indices outside [0, seq_len) are
 * skipped.  With duplicate indices each 16-byte chunk of such a row comes from one of
 * the duplicates (unspecified which, and not necessarily the same for every chunk), as
 * torch's index_put leaves duplicates unspecified.
 * Replaces: kv_scatter_kernel + the scatter branch of KVOpsTriton
 * (src/kernels_t/kv_ops_triton.py:43-65,125-140); the functional (clone, then
 * scatter) form is kept by the Python op.
 */
int ivakv_index_scatter(void* kv, int64_t s_b, int64_t s_h, int64_t s_s, int64_t s_d,
                        const int64_t* indices, int n_idx,
                        const void* values, int64_t v_b, int64_t v_h, int64_t v_s, int64_t v_d,
                        int batch, int n_heads, int seq_len, int head_dim,
                        int dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* IVAKV_H */
