// ivakv_decode_append_attn_noalloc: the fused decode step with its workspace in a
// file-scope device array, so the entry point allocates nothing.  The array lives in
// this translation unit's own code object, which holds no kernel: a device maps it
// (64 MiB) when this entry point first looks up its address there, not when the
// library's other kernels load.
#include <mutex>

#include "ivakv_internal.h"

namespace ivakv {
namespace {

// The decode workspace (one fp32 partial per wave budget slot and per (sequence, kv
// head), then the batch's page prefix).  Every device the entry point runs on holds its
// own copy until the process ends.  In host code the name `scratch` is a host-side
// stand-in, not a device address: the address comes from hipGetSymbolAddress, looked up
// once per device (with that device current) and kept.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of the current device's scratch array (looked up on the first call per
// device).
int scratch_address(const char* name, void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(IVAKV_E_LAUNCH, "%s: hipGetDevice: %s", name, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(IVAKV_E_ARG, "%s: device %d outside the %d devices the scratch table holds", name,
                dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(IVAKV_E_LAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", name, dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return IVAKV_OK;
}

}  // namespace
}  // namespace ivakv

// The fused decode step with its workspace in the static scratch (no allocation
// anywhere).  Same plan, kernels and results as ivakv_decode_append_attn.
extern "C" int ivakv_decode_append_attn_noalloc(const void* q, const void* k_new,
                                                const void* v_new, void* k_pool, void* v_pool,
                                                const int32_t* block_tables,
                                                const int32_t* context_lens, void* out,
                                                int batch, int num_q_heads, int num_kv_heads,
                                                int head_dim, int block_size, int max_blocks,
                                                int num_pages, float scale, int window,
                                                int n_sink, int dtype, hipStream_t stream) {
  return ivakv::decode_append_attn_capped(
      "ivakv_decode_append_attn_noalloc", q, k_new, v_new, k_pool, v_pool, block_tables,
      context_lens, out, batch, num_q_heads, num_kv_heads, head_dim, block_size, max_blocks,
      num_pages, scale, window, n_sink, dtype, stream, ivakv::kScratchBytes,
      ivakv::scratch_address);
}
