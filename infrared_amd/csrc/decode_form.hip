// Block tables from the reference engine's decode metadata.
//
// The reference's eager decode hands the attention seam per-key slots and an
// additive mask (infrared/engine/paged_engine.py:306-314, :630-638):
//   gather_slots[i, p] = bt_i[p / bs] * bs + p % bs   for p < ctx_i (0 after),
//   mask[i, 0, 0, p]   = 0 for p < ctx_i, finfo(dtype).min after.
// One workgroup per sequence recovers ctx_i (the mask's zeros) and bt_i[j] =
// gather_slots[i, j * bs] / bs, and verifies the form exactly: the zeros are a
// prefix, every later mask value is at most -6e4 (masked in any dtype, fp16's
// finfo.min included), every slot below ctx_i follows the closed form and
// every block id lies in the pool, and at least one key is visible (a row
// masked entirely is the mask kernel's uniform average over its keys, not an
// empty context). Each workgroup leaves its sequence's flag in bad[1 + i]; a
// one-workgroup launch after it ORs them into bad[0] (so nothing needs clearing
// before the call). A violation sets bad[0]; the caller then runs the mask
// kernel, which reads the metadata as given.
//
// Where the host does not wait for the verdict -- under hipGraph capture, or
// an eager caller that launches before the verdict is known -- both kernels
// run and the verdict gates them on the device: with IR_FORM_CLEAR_ON_FAIL the
// second launch also sets every context length to 0 when bad[0] is set (the
// block-table decode then reads nothing and writes zero rows), and the mask
// kernel, given bad[0] as its run_if gate, runs after it only in that case.
// The second launch can also publish the verdict, tagged, into pinned host
// memory, where the host reads it when it arrives without synchronising.
#include "common.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kFormThreads = 256;
constexpr int kFormBatch = 16;  // loads a lane has in flight per pass

template <int DT>
__device__ __forceinline__ float mask_at(const void* m, int64_t off) {
  if constexpr (DT == IR_DTYPE_F32) return ((const float*)m)[off];
  const uint32_t h = ((const uint16_t*)m)[off];
  return DT == IR_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

// Each phase issues a lane's kFormBatch loads before it inspects any of them,
// so a sequence of T keys costs about T / (kFormThreads * kFormBatch) round
// trips per phase. Slots are divided in 32 bits when every slot of the pool
// fits (the uniform `narrow`).
template <int DT>
__global__ __launch_bounds__(kFormThreads) void decode_form_kernel(const int64_t* gs, int64_t gs_b, int64_t gs_t,
                                                                   const void* mask, int64_t m_b, int64_t m_t, int T,
                                                                   int bs, int64_t num_blocks, int32_t* bt,
                                                                   int64_t bt_stride, int width, int32_t* ctx_out,
                                                                   int32_t* seq_bad) {
  __shared__ int s_zeros, s_first, s_bad;
  const int b = blockIdx.x, tid = threadIdx.x;
  if (tid == 0) {
    s_zeros = 0;
    s_first = T;
    s_bad = 0;
  }
  __syncthreads();
  const int64_t* g = gs + (int64_t)b * gs_b;
  const int64_t mrow = (int64_t)b * m_b;
  const int64_t n_slots = num_blocks * bs;
  const bool narrow = n_slots <= 0x7fffffff;
  int zeros = 0, first = T, wrong = 0;
  for (int base = 0; base < T; base += kFormThreads * kFormBatch) {
    float x[kFormBatch];
#pragma unroll
    for (int i = 0; i < kFormBatch; ++i) {  // past T: key T - 1 again, not inspected
      const int t = min(base + i * kFormThreads + tid, T - 1);
      x[i] = mask_at<DT>(mask, mrow + (int64_t)t * m_t);
    }
#pragma unroll
    for (int i = 0; i < kFormBatch; ++i) {
      const int t = base + i * kFormThreads + tid;
      if (t < T && x[i] == 0.f) ++zeros;
      if (t < T && x[i] != 0.f) {
        first = min(first, t);
        wrong |= !(x[i] <= -6e4f);
      }
    }
  }
  atomicAdd(&s_zeros, zeros);
  atomicMin(&s_first, first);
  if (wrong) s_bad = 1;
  __syncthreads();
  const int ctx = s_zeros;
  if (s_first < ctx) s_bad = 1;  // a masked key before the last visible one
  if (ctx == 0 && T > 0) s_bad = 1;  // no visible key: the mask kernel's uniform average
  // block id of a block's first slot, or -1 unless it is a block start in the pool
  auto block_of = [&](int64_t head) -> int64_t {
    if (head < 0 || head >= n_slots) return -1;
    if (narrow) {
      const int h = (int)head;
      return h % bs == 0 ? h / bs : -1;
    }
    return head % bs == 0 ? head / bs : -1;
  };
  for (int base = 0; base < ctx; base += kFormThreads * kFormBatch) {
    int64_t slot[kFormBatch], head[kFormBatch];
#pragma unroll
    for (int i = 0; i < kFormBatch; ++i) {
      const int t = base + i * kFormThreads + tid;
      const bool in = t < ctx;
      slot[i] = in ? g[(int64_t)t * gs_t] : 0;
      head[i] = in ? g[(int64_t)(t / bs) * bs * gs_t] : 0;
    }
#pragma unroll
    for (int i = 0; i < kFormBatch; ++i) {
      const int t = base + i * kFormThreads + tid;
      if (t >= ctx) break;
      const int64_t id = block_of(head[i]);
      if (id < 0 || slot[i] != id * bs + t % bs) s_bad = 1;
    }
  }
  for (int j = tid; j < width; j += kFormThreads) {
    const int p = j * bs;
    const int64_t id = p < ctx ? block_of(g[(int64_t)p * gs_t]) : 0;
    bt[(int64_t)b * bt_stride + j] = (int32_t)max(id, (int64_t)0);
  }
  __syncthreads();
  if (tid == 0) {
    ctx_out[b] = ctx;
    seq_bad[b] = s_bad;
  }
}

// After the check, one workgroup: bad[0] = any sequence's flag; when asked,
// every context length becomes 0 if the check failed; and, when given, the
// host record receives tag << 32 | verdict in one 8-byte store, then a
// system-scope fence.
constexpr int kFinishThreads = 1024;
__global__ __launch_bounds__(kFinishThreads) void decode_form_finish_kernel(int32_t* bad, int batch, int32_t* ctx_out,
                                                                           int clear, uint64_t* host, uint32_t tag) {
  __shared__ int s_bad;
  if (threadIdx.x == 0) s_bad = 0;
  __syncthreads();
  int v = 0;
  for (int b = threadIdx.x; b < batch; b += kFinishThreads) v |= bad[1 + b];
  if (v) s_bad = 1;
  __syncthreads();
  const int verdict = s_bad;
  if (threadIdx.x == 0) {
    bad[0] = verdict;
    if (host != nullptr) {
      host[0] = (uint64_t)tag << 32 | (uint32_t)verdict;
      __threadfence_system();
    }
  }
  if (clear && verdict)
    for (int b = threadIdx.x; b < batch; b += kFinishThreads) ctx_out[b] = 0;
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_decode_form(const int64_t* gather_slots, int64_t gs_b_stride, int64_t gs_t_stride,
                              const void* mask, int64_t mask_b_stride, int64_t mask_t_stride, int mask_dtype,
                              int batch, int seq_k, int block_size, int64_t num_blocks, int32_t* block_tables,
                              int64_t bt_stride, int max_blocks_per_seq, int32_t* context_lens, int32_t* bad,
                              int flags, uint64_t* host_verdict, uint32_t tag, ir_stream_t stream) {
  IR_REQUIRE(dtype_bytes(mask_dtype) > 0, "ir_decode_form: unknown mask dtype %d", mask_dtype);
  IR_REQUIRE((flags & ~IR_FORM_CLEAR_ON_FAIL) == 0, "ir_decode_form: unknown flags %#x", flags);
  IR_REQUIRE(batch >= 0 && seq_k >= 0 && block_size > 0 && num_blocks >= 0, "ir_decode_form: bad sizes");
  IR_REQUIRE(max_blocks_per_seq >= (seq_k + block_size - 1) / block_size && bt_stride >= max_blocks_per_seq,
             "ir_decode_form: block tables of %d ids cannot hold %d keys", max_blocks_per_seq, seq_k);
  if (batch == 0) return ok();
  IR_REQUIRE(gather_slots && mask && block_tables && context_lens && bad, "ir_decode_form: null pointer");
  uint64_t* host_dev = nullptr;
  if (host_verdict != nullptr) {
    const hipError_t e = hipHostGetDevicePointer((void**)&host_dev, host_verdict, 0);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // not left for the next launch check to report
      return fail(IR_EINVAL, "ir_decode_form: host_verdict is not pinned host memory: %s", hipGetErrorString(e));
    }
  }
  hipStream_t s = (hipStream_t)stream;
  int32_t* seq_bad = bad + 1;
  if (mask_dtype == IR_DTYPE_F32)
    hipLaunchKernelGGL(decode_form_kernel<IR_DTYPE_F32>, dim3(batch), dim3(kFormThreads), 0, s, gather_slots,
                       gs_b_stride, gs_t_stride, mask, mask_b_stride, mask_t_stride, seq_k, block_size, num_blocks,
                       block_tables, bt_stride, max_blocks_per_seq, context_lens, seq_bad);
  else if (mask_dtype == IR_DTYPE_BF16)
    hipLaunchKernelGGL(decode_form_kernel<IR_DTYPE_BF16>, dim3(batch), dim3(kFormThreads), 0, s, gather_slots,
                       gs_b_stride, gs_t_stride, mask, mask_b_stride, mask_t_stride, seq_k, block_size, num_blocks,
                       block_tables, bt_stride, max_blocks_per_seq, context_lens, seq_bad);
  else
    hipLaunchKernelGGL(decode_form_kernel<IR_DTYPE_F16>, dim3(batch), dim3(kFormThreads), 0, s, gather_slots,
                       gs_b_stride, gs_t_stride, mask, mask_b_stride, mask_t_stride, seq_k, block_size, num_blocks,
                       block_tables, bt_stride, max_blocks_per_seq, context_lens, seq_bad);
  hipLaunchKernelGGL(decode_form_finish_kernel, dim3(1), dim3(kFinishThreads), 0, s, bad, batch, context_lens,
                     (flags & IR_FORM_CLEAR_ON_FAIL) ? 1 : 0, host_dev, tag);
  return check_launch("ir_decode_form");
}
