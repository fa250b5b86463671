// ir_paged_decode_noalloc: ir_paged_decode for callers that cannot allocate
// device memory (code under hipGraph capture, tight serving loops, harnesses
// that forbid it). The split-KV arrival counters and fp32 partial rows that
// ir_paged_decode takes from the caller live here in one file-scope device
// array instead, which every GPU the library runs on holds until the process
// ends.
//
// In host code `scratch` names a host-side stand-in, not a device address:
// the address of each device's copy comes from hipGetSymbolAddress, taken
// once per device (with that device current) on the entry point's first call
// there, and only that address is passed to kernels.
//
// Every call on one GPU shares that GPU's array: calls that overlap on one GPU
// (different streams, or graphs replayed concurrently) race on it. Calls in
// one stream's order are safe: each leaves the counters it used at zero, and
// the partial rows are scratch rewritten before they are read.
#include <mutex>

#include "status.hpp"

namespace ir {
namespace {

constexpr int64_t kNoAllocCounterBytes = 64 << 10;  // 16,384 arrival counters
constexpr int64_t kNoAllocScratchBytes = 16 << 20;  // counters + partial rows
constexpr int64_t kNoAllocPartialBytes = kNoAllocScratchBytes - kNoAllocCounterBytes;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

__global__ __launch_bounds__(256) void zero_words_kernel(int32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0;
}

std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array. The first call on a
// device looks it up and clears the counter region on `s` (a fill kernel, so
// the clear is also safe inside a captured graph); the counters stay zero at
// rest from then on.
int scratch_of_current_device(hipStream_t s, uint8_t** out) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess) return fail(IR_ELAUNCH, "ir_paged_decode_noalloc: hipGetDevice: %s", hipGetErrorString(ge));
  if (dev < 0 || dev >= kMaxDevices) return fail(IR_EUNSUPPORTED, "ir_paged_decode_noalloc: device %d", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(IR_ELAUNCH, "ir_paged_decode_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
    hipLaunchKernelGGL(zero_words_kernel, dim3(16), dim3(256), 0, s, (int32_t*)p, kNoAllocCounterBytes / 4);
    const int rc = check_launch("ir_paged_decode_noalloc (scratch clear)");
    if (rc != IR_OK) return rc;
    g_scratch_ptr[dev] = (uint8_t*)p;
  }
  *out = g_scratch_ptr[dev];
  return IR_OK;
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_paged_decode_noalloc(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                                       const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                                       int64_t cache_head_stride, int64_t num_blocks, int block_size,
                                       const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                                       const int32_t* context_lens, void* out, int64_t out_seq_stride,
                                       int64_t out_head_stride, int num_seqs, int num_q_heads, int num_kv_heads,
                                       int head_dim, float scale, int dtype, int partition_tokens,
                                       int32_t* err_flags, ir_stream_t stream) {
  // sizes first: a request beyond the array is refused before any device call
  const int64_t ws = ir_paged_decode_workspace_size(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                                    max_blocks_per_seq, block_size, partition_tokens);
  const int64_t ctr = ir_paged_decode_num_counters(num_seqs, num_q_heads, num_kv_heads);
  if (ws > kNoAllocPartialBytes || ctr * 4 > kNoAllocCounterBytes)
    return fail(IR_EWORKSPACE,
                "ir_paged_decode_noalloc: this call needs %lld bytes of partial rows and %lld arrival counters; "
                "the no-alloc scratch holds %lld bytes and %lld counters (use ir_paged_decode with a workspace)",
                (long long)ws, (long long)ctr, (long long)kNoAllocPartialBytes, (long long)(kNoAllocCounterBytes / 4));
  uint8_t* base = nullptr;
  if (ws > 0) {
    const int rc = scratch_of_current_device((hipStream_t)stream, &base);
    if (rc != IR_OK) return rc;
  }
  return ir_paged_decode(q, q_seq_stride, q_head_stride, k_cache, v_cache, cache_slot_stride, cache_head_stride,
                         num_blocks, block_size, block_tables, bt_stride, max_blocks_per_seq, context_lens, out,
                         out_seq_stride, out_head_stride, num_seqs, num_q_heads, num_kv_heads, head_dim, scale, dtype,
                         partition_tokens, base ? (int32_t*)base : nullptr, base ? kNoAllocCounterBytes / 4 : 0,
                         base ? base + kNoAllocCounterBytes : nullptr, base ? kNoAllocPartialBytes : 0, err_flags,
                         stream);
}
