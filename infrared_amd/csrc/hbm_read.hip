// Read-only HBM streaming roof: the rate at which this device reads a large
// contiguous buffer with the decode kernels' load form (non-temporal 16-byte
// loads, every lane's loads of a round in flight together). A measurement
// utility beside the kernels, so the decode's achieved bandwidth can be held
// against a read-only roof measured on the same device, not only against a
// copy (which reads and writes) or the published peak.
#include "common.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kReadThreads = 256;
constexpr int kReadUnroll = 8;  // 16-byte loads in flight per lane
constexpr int64_t kReadChunk = (int64_t)kReadThreads * kReadUnroll;  // 16-byte pieces per round

// Workgroup i reads rounds i, i + grid, ... of kReadChunk pieces; the pieces a
// lane loads in one round are kReadThreads apart, so each load instruction of
// a wavefront covers 1 KiB contiguous. The XOR of everything read is stored
// only if it equals a value no caller expects, which keeps the loads live
// without writing per workgroup.
__global__ __launch_bounds__(kReadThreads) void hbm_read_kernel(const u32x4* src, int64_t rounds, uint32_t* sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t r = blockIdx.x; r < rounds; r += gridDim.x) {
    const u32x4* p = src + r * kReadChunk + threadIdx.x;
    u32x4 v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) v[u] = load_nt(p + u * kReadThreads);
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u];
  }
  const uint32_t x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x9e3779b9u) sink[0] = x;
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int64_t ir_hbm_read_granule(void) { return kReadChunk * 16; }

extern "C" int ir_hbm_read(const void* src, int64_t bytes, uint32_t* sink, int workgroups, ir_stream_t stream) {
  IR_REQUIRE(src && sink, "ir_hbm_read: null pointer");
  IR_REQUIRE(aligned16(src), "ir_hbm_read: src must be 16-byte aligned");
  IR_REQUIRE(bytes > 0 && bytes % (kReadChunk * 16) == 0, "ir_hbm_read: bytes must be a positive multiple of %lld",
             (long long)(kReadChunk * 16));
  IR_REQUIRE(workgroups >= 0, "ir_hbm_read: bad workgroup count");
  const int64_t rounds = bytes / (kReadChunk * 16);
  int64_t grid = workgroups > 0 ? workgroups : (int64_t)device_cus() * 8;
  if (grid > rounds) grid = rounds;
  hipLaunchKernelGGL(hbm_read_kernel, dim3((unsigned)grid), dim3(kReadThreads), 0, (hipStream_t)stream,
                     (const u32x4*)src, rounds, sink);
  return check_launch("ir_hbm_read");
}
