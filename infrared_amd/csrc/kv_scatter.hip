// KV-slot scatter (PagedKVPool.write) and block-table gather (PagedKVPool.gather
// through the closed-form slot map) for gfx950.
//
// The scatter is a pure copy: each new token's [num_kv_heads, head_dim] row is
// written to row slot_mapping[i] of the layer's pool. Rows are moved in 16-byte
// pieces, one piece per lane, so one wavefront moves 1 KiB of contiguous row
// data per instruction; misaligned layouts take an element-wise kernel.
#include "common.hpp"
#include "status.hpp"

namespace ir {
namespace {

struct ScatterArgs {
  const uint8_t* k;
  const uint8_t* v;
  int64_t k_tok, k_head, v_tok, v_head;  // bytes
  uint8_t* kc;
  uint8_t* vc;
  int64_t c_slot, c_head;  // bytes
  int64_t num_slots;
  const int64_t* slots;
  int64_t n_tokens;
  int num_kv_heads;
  int row_bytes;  // head_dim * element bytes
  int32_t* err;
};

// One lane per 16-byte piece of a (token, head) row. The slot and both source
// pieces are loaded before the slot is inspected (the sources are in bounds
// for every lane of the grid), so a lane waits for one round trip, not two.
// NARROW: the grid's piece count fits 31 bits, so the index math is 32-bit.
template <bool NARROW>
__global__ __launch_bounds__(256) void kv_scatter_vec16(ScatterArgs a) {
  const int pieces = a.row_bytes >> 4;
  int64_t tok;
  int head, piece;
  if constexpr (NARROW) {
    const int per_tok = pieces * a.num_kv_heads;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int)a.n_tokens * per_tok) return;
    const int t = idx / per_tok;
    const int rem = idx - t * per_tok;
    tok = t;
    head = rem / pieces;
    piece = rem - head * pieces;
  } else {
    const int64_t per_tok = (int64_t)pieces * a.num_kv_heads;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.n_tokens * per_tok) return;
    tok = idx / per_tok;
    const int rem = (int)(idx - tok * per_tok);
    head = rem / pieces;
    piece = rem - head * pieces;
  }
  const int64_t off = (int64_t)piece * 16;
  const int64_t slot = a.slots[tok];
  const u32x4 kx = *(const u32x4*)(a.k + tok * a.k_tok + head * a.k_head + off);
  const u32x4 vx = *(const u32x4*)(a.v + tok * a.v_tok + head * a.v_head + off);
  if (slot < 0) return;  // padding sentinel
  if (slot >= a.num_slots) {
    flag_error(a.err, IR_ERR_SLOT_RANGE);
    return;
  }
  *(u32x4*)(a.kc + slot * a.c_slot + head * a.c_head + off) = kx;
  *(u32x4*)(a.vc + slot * a.c_slot + head * a.c_head + off) = vx;
}

// Element-wise fallback for layouts that are not 16-byte aligned.
template <typename S>
__global__ __launch_bounds__(256) void kv_scatter_elem(ScatterArgs a) {
  const int ebytes = (int)sizeof(S);
  const int head_dim = a.row_bytes / ebytes;
  const int64_t per_tok = (int64_t)head_dim * a.num_kv_heads;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.n_tokens * per_tok) return;
  const int64_t tok = idx / per_tok;
  const int rem = (int)(idx - tok * per_tok);
  const int head = rem / head_dim;
  const int d = rem - head * head_dim;
  const int64_t slot = a.slots[tok];
  if (slot < 0) return;
  if (slot >= a.num_slots) {
    flag_error(a.err, IR_ERR_SLOT_RANGE);
    return;
  }
  const int64_t off = (int64_t)d * ebytes;
  *(S*)(a.kc + slot * a.c_slot + head * a.c_head + off) =
      *(const S*)(a.k + tok * a.k_tok + head * a.k_head + off);
  *(S*)(a.vc + slot * a.c_slot + head * a.c_head + off) =
      *(const S*)(a.v + tok * a.v_tok + head * a.v_head + off);
}

// out[i] = cache[slots[i]] (the reference's `self.k[layer_idx, flat]`): one
// lane per 16-byte piece of a (row, head); slots outside the pool read as zero
// and are flagged.
__global__ __launch_bounds__(256) void kv_gather_slots_vec16(ScatterArgs a) {
  const int pieces = a.row_bytes >> 4;
  const int64_t per_tok = (int64_t)pieces * a.num_kv_heads;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.n_tokens * per_tok) return;
  const int64_t tok = idx / per_tok;
  const int rem = (int)(idx - tok * per_tok);
  const int head = rem / pieces;
  const int piece = rem - head * pieces;
  const int64_t slot = a.slots[tok];
  const int64_t off = (int64_t)piece * 16;
  u32x4 kx = {0u, 0u, 0u, 0u}, vx = {0u, 0u, 0u, 0u};
  if (slot >= 0 && slot < a.num_slots) {
    kx = *(const u32x4*)(a.kc + slot * a.c_slot + head * a.c_head + off);
    vx = *(const u32x4*)(a.vc + slot * a.c_slot + head * a.c_head + off);
  } else if (piece == 0 && head == 0) {
    flag_error(a.err, IR_ERR_GATHER_RANGE);
  }
  // k/v here are the (contiguous) outputs
  *(u32x4*)((uint8_t*)a.k + tok * a.k_tok + head * a.k_head + off) = kx;
  *(u32x4*)((uint8_t*)a.v + tok * a.v_tok + head * a.v_head + off) = vx;
}

template <typename S>
__global__ __launch_bounds__(256) void kv_gather_slots_elem(ScatterArgs a) {
  const int ebytes = (int)sizeof(S);
  const int head_dim = a.row_bytes / ebytes;
  const int64_t per_tok = (int64_t)head_dim * a.num_kv_heads;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.n_tokens * per_tok) return;
  const int64_t tok = idx / per_tok;
  const int rem = (int)(idx - tok * per_tok);
  const int head = rem / head_dim;
  const int d = rem - head * head_dim;
  const int64_t slot = a.slots[tok];
  const int64_t off = (int64_t)d * ebytes;
  S kx = 0, vx = 0;
  if (slot >= 0 && slot < a.num_slots) {
    kx = *(const S*)(a.kc + slot * a.c_slot + head * a.c_head + off);
    vx = *(const S*)(a.vc + slot * a.c_slot + head * a.c_head + off);
  } else if (d == 0 && head == 0) {
    flag_error(a.err, IR_ERR_GATHER_RANGE);
  }
  *(S*)((uint8_t*)a.k + tok * a.k_tok + head * a.k_head + off) = kx;
  *(S*)((uint8_t*)a.v + tok * a.v_tok + head * a.v_head + off) = vx;
}

struct GatherArgs {
  const uint8_t* kc;
  const uint8_t* vc;
  int64_t c_slot, c_head;  // bytes
  int64_t num_blocks;
  int bs;
  const int32_t* bt;
  int64_t bt_stride;
  int max_blocks;
  const int32_t* ctx;
  int num_seqs, max_ctx, num_kv_heads;
  int row_bytes;
  uint8_t* ok;
  uint8_t* ov;
  int32_t* err;
};

// One lane per element-sized piece (bytes `P`) of out[b, t, h, :].
template <typename P>
__global__ __launch_bounds__(256) void paged_gather_kernel(GatherArgs a) {
  const int pieces = a.row_bytes / (int)sizeof(P);
  const int64_t per_tok = (int64_t)pieces * a.num_kv_heads;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.num_seqs * a.max_ctx * per_tok;
  if (idx >= total) return;
  const int64_t bt_idx = idx / per_tok;  // b * max_ctx + t
  const int rem = (int)(idx - bt_idx * per_tok);
  const int head = rem / pieces;
  const int piece = rem - head * pieces;
  const int b = (int)(bt_idx / a.max_ctx);
  const int t = (int)(bt_idx - (int64_t)b * a.max_ctx);
  int ctx = a.ctx[b];
  const int cap = a.max_blocks * a.bs;
  if (ctx > cap || ctx < 0) {
    flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    ctx = ctx < 0 ? 0 : cap;
  }
  const int64_t out_off = (bt_idx * a.num_kv_heads + head) * a.row_bytes + (int64_t)piece * sizeof(P);
  P kx = P(), vx = P();
  if (t < ctx) {
    const int64_t slot = token_slot(a.bt + (int64_t)b * a.bt_stride, t, a.bs, a.num_blocks, a.err);
    if (slot >= 0) {
      const int64_t in_off = slot * a.c_slot + head * a.c_head + (int64_t)piece * sizeof(P);
      kx = *(const P*)(a.kc + in_off);
      vx = *(const P*)(a.vc + in_off);
    }
  }
  *(P*)(a.ok + out_off) = kx;
  *(P*)(a.ov + out_off) = vx;
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_kv_scatter(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                             const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                             void* k_cache, void* v_cache, int64_t cache_slot_stride,
                             int64_t cache_head_stride, int64_t num_slots,
                             const int64_t* slot_mapping, int64_t n_tokens, int num_kv_heads,
                             int head_dim, int dtype, int32_t* err_flags, ir_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  IR_REQUIRE(eb > 0, "ir_kv_scatter: unknown dtype %d", dtype);
  IR_REQUIRE(n_tokens >= 0 && num_kv_heads > 0 && head_dim > 0 && num_slots >= 0,
             "ir_kv_scatter: bad sizes n_tokens=%lld heads=%d head_dim=%d num_slots=%lld",
             (long long)n_tokens, num_kv_heads, head_dim, (long long)num_slots);
  if (n_tokens == 0) return ok();
  IR_REQUIRE(k && v && k_cache && v_cache && slot_mapping, "ir_kv_scatter: null pointer");
  ScatterArgs a;
  a.k = (const uint8_t*)k;
  a.v = (const uint8_t*)v;
  a.k_tok = k_tok_stride * eb;
  a.k_head = k_head_stride * eb;
  a.v_tok = v_tok_stride * eb;
  a.v_head = v_head_stride * eb;
  a.kc = (uint8_t*)k_cache;
  a.vc = (uint8_t*)v_cache;
  a.c_slot = cache_slot_stride * eb;
  a.c_head = cache_head_stride * eb;
  a.num_slots = num_slots;
  a.slots = slot_mapping;
  a.n_tokens = n_tokens;
  a.num_kv_heads = num_kv_heads;
  a.row_bytes = head_dim * eb;
  a.err = err_flags;
  const bool vec = (a.row_bytes % 16 == 0) && aligned16(k) && aligned16(v) && aligned16(k_cache) &&
                   aligned16(v_cache) && a.k_tok % 16 == 0 && a.k_head % 16 == 0 &&
                   a.v_tok % 16 == 0 && a.v_head % 16 == 0 && a.c_slot % 16 == 0 &&
                   a.c_head % 16 == 0;
  hipStream_t s = (hipStream_t)stream;
  if (vec) {
    const int64_t total = n_tokens * num_kv_heads * (a.row_bytes / 16);
    const dim3 grid((unsigned)((total + 255) / 256));
    if (total + 255 < ((int64_t)1 << 31))
      hipLaunchKernelGGL(kv_scatter_vec16<true>, grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(kv_scatter_vec16<false>, grid, dim3(256), 0, s, a);
  } else {
    const int64_t total = n_tokens * num_kv_heads * (int64_t)head_dim;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (eb == 4)
      hipLaunchKernelGGL(kv_scatter_elem<uint32_t>, grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(kv_scatter_elem<uint16_t>, grid, dim3(256), 0, s, a);
  }
  return check_launch("ir_kv_scatter");
}

extern "C" int ir_gather_slots(const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                               int64_t cache_head_stride, int64_t num_slots, const int64_t* slots,
                               int64_t n, int num_kv_heads, int head_dim, int dtype, void* out_k,
                               void* out_v, int32_t* err_flags, ir_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  IR_REQUIRE(eb > 0, "ir_gather_slots: unknown dtype %d", dtype);
  IR_REQUIRE(n >= 0 && num_kv_heads > 0 && head_dim > 0 && num_slots >= 0, "ir_gather_slots: bad sizes");
  if (n == 0) return ok();
  IR_REQUIRE(k_cache && v_cache && slots && out_k && out_v, "ir_gather_slots: null pointer");
  ScatterArgs a;
  a.row_bytes = head_dim * eb;
  a.k = (const uint8_t*)out_k;
  a.v = (const uint8_t*)out_v;
  a.k_tok = a.v_tok = (int64_t)num_kv_heads * a.row_bytes;
  a.k_head = a.v_head = a.row_bytes;
  a.kc = (uint8_t*)k_cache;
  a.vc = (uint8_t*)v_cache;
  a.c_slot = cache_slot_stride * eb;
  a.c_head = cache_head_stride * eb;
  a.num_slots = num_slots;
  a.slots = slots;
  a.n_tokens = n;
  a.num_kv_heads = num_kv_heads;
  a.err = err_flags;
  const bool vec = (a.row_bytes % 16 == 0) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out_k) &&
                   aligned16(out_v) && a.c_slot % 16 == 0 && a.c_head % 16 == 0;
  hipStream_t s = (hipStream_t)stream;
  if (vec) {
    const int64_t total = n * num_kv_heads * (a.row_bytes / 16);
    hipLaunchKernelGGL(kv_gather_slots_vec16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, a);
  } else {
    const int64_t total = n * num_kv_heads * (int64_t)head_dim;
    const dim3 grid((unsigned)((total + 255) / 256));
    if (eb == 4)
      hipLaunchKernelGGL(kv_gather_slots_elem<uint32_t>, grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(kv_gather_slots_elem<uint16_t>, grid, dim3(256), 0, s, a);
  }
  return check_launch("ir_gather_slots");
}

extern "C" int ir_paged_gather(const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                               int64_t cache_head_stride, int64_t num_blocks, int block_size,
                               const int32_t* block_tables, int64_t bt_stride,
                               int max_blocks_per_seq, const int32_t* context_lens, int num_seqs,
                               int max_ctx, int num_kv_heads, int head_dim, int dtype,
                               void* out_k, void* out_v, int32_t* err_flags, ir_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  IR_REQUIRE(eb > 0, "ir_paged_gather: unknown dtype %d", dtype);
  IR_REQUIRE(num_seqs >= 0 && max_ctx >= 0 && num_kv_heads > 0 && head_dim > 0 &&
                 block_size > 0 && max_blocks_per_seq >= 0 && num_blocks >= 0,
             "ir_paged_gather: bad sizes");
  if ((int64_t)num_seqs * max_ctx == 0) return ok();
  IR_REQUIRE(k_cache && v_cache && block_tables && context_lens && out_k && out_v,
             "ir_paged_gather: null pointer");
  GatherArgs a;
  a.kc = (const uint8_t*)k_cache;
  a.vc = (const uint8_t*)v_cache;
  a.c_slot = cache_slot_stride * eb;
  a.c_head = cache_head_stride * eb;
  a.num_blocks = num_blocks;
  a.bs = block_size;
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks_per_seq;
  a.ctx = context_lens;
  a.num_seqs = num_seqs;
  a.max_ctx = max_ctx;
  a.num_kv_heads = num_kv_heads;
  a.row_bytes = head_dim * eb;
  a.ok = (uint8_t*)out_k;
  a.ov = (uint8_t*)out_v;
  a.err = err_flags;
  const bool vec = (a.row_bytes % 16 == 0) && aligned16(k_cache) && aligned16(v_cache) &&
                   aligned16(out_k) && aligned16(out_v) && a.c_slot % 16 == 0 && a.c_head % 16 == 0;
  hipStream_t s = (hipStream_t)stream;
  const int piece = vec ? 16 : eb;
  const int64_t total = (int64_t)num_seqs * max_ctx * num_kv_heads * (a.row_bytes / piece);
  const dim3 grid((unsigned)((total + 255) / 256));
  if (vec)
    hipLaunchKernelGGL(paged_gather_kernel<u32x4>, grid, dim3(256), 0, s, a);
  else if (eb == 4)
    hipLaunchKernelGGL(paged_gather_kernel<uint32_t>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(paged_gather_kernel<uint16_t>, grid, dim3(256), 0, s, a);
  return check_launch("ir_paged_gather");
}
