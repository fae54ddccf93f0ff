// Internal helpers shared by the libivakv translation units (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "ivakv.h"

namespace ivakv {

// Records a printf-style message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps the state after a launch to a status: IVAKV_E_LAUNCH with HIP's message
// when the launch failed, IVAKV_OK otherwise.
int launch_status(const char* what);

// Supplies a workspace's device address for the entry point `name`, or an error status.
typedef int (*WorkspaceSource)(const char* name, void** ptr);

// ivakv_decode_append_attn with its workspace from get_ws instead of an argument, for a
// plan of at most `capacity` bytes (IVAKV_E_WORKSPACE beyond, before any launch).
// Defined in ivakv_decode.hip.
int decode_append_attn_capped(const char* name, const void* q, const void* k_new,
                              const void* v_new, void* k_pool, void* v_pool,
                              const int32_t* block_tables, const int32_t* context_lens, void* out,
                              int batch, int num_q_heads, int num_kv_heads, int head_dim,
                              int block_size, int max_blocks, int num_pages, float scale,
                              int window, int n_sink, int dtype, hipStream_t stream,
                              size_t capacity, WorkspaceSource get_ws);

inline int dtype_size(int dtype) {
  switch (dtype) {
    case IVAKV_F32: return 4;
    case IVAKV_F16: return 2;
    case IVAKV_BF16: return 2;
    default: return 0;
  }
}

// Non-temporal (streaming) load / store of a 4-, 8- or 16-byte value: the hint for
// data a kernel touches once, which HBM-bound kernels here read and write faster with
// it (measured per kernel; plain where a kernel's measurements favoured plain).
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t nt_u32x2 __attribute__((ext_vector_type(2)));
template <class T>
__device__ inline T load_nt(const void* p) {
  static_assert(sizeof(T) == 16 || sizeof(T) == 8 || sizeof(T) == 4, "4, 8 or 16 bytes");
  if constexpr (sizeof(T) == 16)
    return __builtin_bit_cast(T, __builtin_nontemporal_load(static_cast<const nt_u32x4*>(p)));
  else if constexpr (sizeof(T) == 8)
    return __builtin_bit_cast(T, __builtin_nontemporal_load(static_cast<const nt_u32x2*>(p)));
  else
    return __builtin_bit_cast(T, __builtin_nontemporal_load(static_cast<const uint32_t*>(p)));
}
template <class T>
__device__ inline void store_nt(void* p, const T& v) {
  static_assert(sizeof(T) == 16 || sizeof(T) == 8 || sizeof(T) == 4, "4, 8 or 16 bytes");
  if constexpr (sizeof(T) == 16)
    __builtin_nontemporal_store(__builtin_bit_cast(nt_u32x4, v), static_cast<nt_u32x4*>(p));
  else if constexpr (sizeof(T) == 8)
    __builtin_nontemporal_store(__builtin_bit_cast(nt_u32x2, v), static_cast<nt_u32x2*>(p));
  else
    __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, v), static_cast<uint32_t*>(p));
}
// Load / store with the hint when NT.
template <bool NT, class T>
__device__ inline T ld(const void* p) {
  if constexpr (NT) return load_nt<T>(p);
  else return *static_cast<const T*>(p);
}
template <bool NT, class T>
__device__ inline void st(void* p, const T& v) {
  if constexpr (NT) store_nt<T>(p, v);
  else *static_cast<T*>(p) = v;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Logical index of workgroup b of n (a 1-D grid dimension) such that each XCD runs a
// contiguous range of them: workgroups are dispatched to the 8 XCDs round-robin (b on
// XCD b % 8), and XCD x takes logical blocks x * q + min(x, r) .. (q = n / 8, r = n % 8).
// A bijection on [0, n) whatever the dispatch does; with round-robin dispatch,
// neighbouring logical blocks share an L2.  The appends use it so the partial 32-byte
// sectors where a chunk's pages straddle two token groups merge in one L2 before they
// are written back (a page-unaligned 8192-row chunk append: 20.4 -> 17.4 us).
__device__ inline int64_t xcd_contiguous_block(int64_t b, int64_t n) {
  const int64_t q = n >> 3, r = n & 7, x = b & 7;
  return x * q + (x < r ? x : r) + (b >> 3);
}

// Ceil division for non-negative ints.
__host__ __device__ inline int cdiv(int a, int b) { return (a + b - 1) / b; }

// Visible-page walk of one sequence for decode attention.  The visible key
// positions of a sequence of length L are
//   { j < L : window <= 0 or j >= L - window or j < n_sink }
// i.e. the attention-sink prefix [0, n_sink) united with the window [L-window, L).
// They are covered by "effective" pages 0..n_eff-1: effective page v < sink_pages
// is logical page v, and v >= sink_pages is logical page win_first + v - sink_pages.
struct PageWalk {
  int L;           // context length
  int win_start;   // first window position (0 when there is no window)
  int sink_pages;  // pages holding sink positions that lie before the window
  int win_first;   // first logical page of the window range
  int n_eff;       // number of effective pages
};

__host__ __device__ inline PageWalk make_walk(int L, int window, int n_sink, int bs) {
  PageWalk w;
  w.L = L < 0 ? 0 : L;
  w.win_start = (window > 0 && w.L > window) ? w.L - window : 0;
  int sink_len = (n_sink > 0) ? (n_sink < w.win_start ? n_sink : w.win_start) : 0;
  w.sink_pages = cdiv(sink_len, bs);
  int wf = w.win_start / bs;
  w.win_first = wf > w.sink_pages ? wf : w.sink_pages;
  int n_log = cdiv(w.L, bs);
  w.n_eff = w.sink_pages + (n_log > w.win_first ? n_log - w.win_first : 0);
  return w;
}

// Logical page of effective page v.
__host__ __device__ inline int logical_page(const PageWalk& w, int v) {
  return v < w.sink_pages ? v : w.win_first + (v - w.sink_pages);
}

// Byte of (dim d, key r) in an FP8 V tile (head_dim D, 16 keys): order
// [d % 16][r / 4][d / 16][r % 4].  Lane (ln, lq) of the decode walk needs keys
// 4lq .. 4lq+3 of dims ln, 16 + ln, ..., one 4-byte word per 16 dims: in this
// order its D/16 words are consecutive, D/64 16-byte loads.
__host__ __device__ inline int fp8_v_offset(int d, int r, int D) {
  return (((d & 15) * 4 + (r >> 2)) * (D >> 4) + (d >> 4)) * 4 + (r & 3);
}

// Effective pages of a walk whose logical page lies inside the block table
// (logical_page is increasing, so these are the first ones).  Positions on the
// pages past the table are never attended, so the walks stop there.
__host__ __device__ inline int table_pages(const PageWalk& w, int max_blocks, int bs = 16) {
  const int sink = w.sink_pages < max_blocks ? w.sink_pages : max_blocks;
  const int n_log = cdiv(w.L, bs);
  const int win = (n_log < max_blocks ? n_log : max_blocks) - w.win_first;
  return sink + (win > 0 ? win : 0);
}

// Largest n_eff any sequence can have for a block table of max_blocks columns.
inline int max_effective_pages(int max_blocks, int window, int n_sink, int bs) {
  if (window <= 0) return max_blocks;
  int bound = cdiv(n_sink > 0 ? n_sink : 0, bs) + cdiv(window, bs) + 1;
  return bound < max_blocks ? bound : max_blocks;
}

}  // namespace ivakv
