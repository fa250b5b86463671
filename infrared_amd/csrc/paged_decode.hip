// GQA paged decode attention for gfx950 (split-KV partitions) and the C ABI
// of the decode entry points.
//
// One workgroup per (unit, partition of `part_tokens` keys); the tile math is
// in paged_decode.hpp. The wavefronts' (max, sum, acc) states merge through
// LDS. A sequence that fits one partition writes its output directly. Longer
// ones write fp32 partials (device-scope stores) that the last workgroup of
// the unit to finish -- found with an arrival counter -- merges with
// log-sum-exp weights before it resets the counter (or, with
// IR_DECODE_MERGE=kernel, a second launch merges them).
#include <stdlib.h>
#include <string.h>

#include "paged_decode.hpp"
#include "status.hpp"

namespace ir {
namespace {

// Log-sum-exp merge of the partitions of (seq, heads head0..head0+nh) into out;
// DEV: the partials were written by other workgroups of this launch and are
// read at device scope (byte offsets below 2 GiB, checked by the host).
template <int DT, int D, bool DEV>
__device__ __forceinline__ void merge_partials(const DecodeArgs& a, int seq, int head0, int nh, int nparts,
                                               int tid, int nthreads) {
  constexpr int EB = TileShape<DT, D>::EB;
  for (int it = tid; it < nh * (D / 4); it += nthreads) {
    const int hc = it / (D / 4);
    const int d0 = (it - hc * (D / 4)) * 4;
    const int64_t row0 = ((int64_t)seq * a.num_q_heads + head0 + hc) * a.max_parts;
    float o[4], L;
    if constexpr (DEV)
      lse_merge_dev<D>(dev_rsrc(a.ws_o), dev_rsrc(a.ws_ml), (int)row0, 1, nparts, d0, o, L);
    else
      lse_merge(a.ws_o + row0 * D + d0, D, a.ws_ml + row0 * 2, 2, nparts, [](const float* p) { return *p; }, o,
                L);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    store4<DT>((uint8_t*)a.out + ((int64_t)seq * a.o_seq + (int64_t)(head0 + hc) * a.o_head + d0) * EB, o, inv);
  }
}

// FUSED: partials are merged by the last workgroup to arrive (device-scope
// counter); otherwise paged_decode_reduce merges them in a second launch.
// 16-bit dtypes: two wavefronts per SIMD (<= 256 registers each) keep two
// resident workgroups' worth of loads in flight per CU. fp32 tiles are twice
// the registers and run one per SIMD.
template <int DT, int D, bool BS16, int NW, bool FUSED, int DEPTH>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(DT == IR_DTYPE_F32 ? 1 : 2)))
void paged_decode_kernel(DecodeArgs a) {
  typedef TileShape<DT, D> Sh;
  constexpr int EB = Sh::EB;
  __shared__ MergeSmem<NW, D> sm;
  __shared__ __attribute__((aligned(16))) uint8_t kstage[NW][KStage<DT, D>::BYTES];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;

  const int unit = blockIdx.x;  // (seq, kv head, head group)
  int idx = unit;
  const int hg = idx % a.n_hg;
  idx /= a.n_hg;
  const int kvh = idx % a.num_kv_heads;
  const int seq = idx / a.num_kv_heads;
  const int part = blockIdx.y;

  const int ctx = clamp_ctx(a, seq, part == 0 && threadIdx.x == 0 && hg == 0 && kvh == 0);
  const int nparts = ctx > 0 ? (ctx + a.part_tokens - 1) / a.part_tokens : 1;
  if (part >= nparts) return;
  const int t_begin = part * a.part_tokens;
  const int t_end = min(ctx, t_begin + a.part_tokens);
  const int tile_lo = t_begin >> 4;
  // (an empty pool has nothing to read: every key is unusable)
  const int tile_hi = (t_end > t_begin && a.num_blocks > 0) ? (t_end + 15) >> 4 : tile_lo;

  const int h_local = hg * 16 + c;
  const int32_t* bt_row = a.bt + (int64_t)seq * a.bt_stride;
  const uint8_t* kc = (const uint8_t*)a.kc + (int64_t)kvh * a.c_head * EB;
  const uint8_t* vc = (const uint8_t*)a.vc + (int64_t)kvh * a.c_head * EB;
  const LaneOffsets<DT, D> lo = lane_offsets<DT, D>(lane, a.c_slot * EB);
  uint32_t qr[Sh::KDW];
  load_query<DT, D>(a, seq, kvh * a.n_rep + h_local, h_local < a.n_rep, g, qr);

  State<D> st;
  state_init(st);
  bool bad = false;
  attend_tiles<DT, D, BS16, NW, DEPTH>(a, bt_row, kc, vc, lo, qr, tile_lo, tile_hi, t_end, kstage[w], lane, w, st,
                                       bad);
  if (bad) flag_error(a.err, IR_ERR_BLOCK_RANGE);
  st.l = wave_sum_groups(st.l);

  // ---- merge the wavefronts of this workgroup through LDS
  merge_publish<NW, D>(sm, st, w, g, c);
  __syncthreads();

  const int nh = min(16, a.n_rep - hg * 16);
  const int head0 = kvh * a.n_rep + hg * 16;
  if (nparts == 1) {
    store_merged<DT, D, NW>(a, sm, seq, head0, nh);
    return;
  }

  // ---- split-KV: publish this partition's partial
  for (int it = threadIdx.x; it < nh * (D / 4); it += NW * 64) {
    const int hc = it / (D / 4);
    const int d0 = (it - hc * (D / 4)) * 4;
    float M, L, o[4];
    merge_column<NW, D>(sm, hc, d0, M, L, o);
    const int64_t row = ((int64_t)seq * a.num_q_heads + head0 + hc) * a.max_parts + part;
    float* wo = a.ws_o + row * D + d0;
    if constexpr (FUSED) {
      store_dev4(dev_rsrc(a.ws_o), (int)(row * D + d0) * 4, f32x4{o[0], o[1], o[2], o[3]});
      if (d0 == 0) store_dev2(dev_rsrc(a.ws_ml), (int)row * 8, f32x2{M, L});
    } else {
      *(f32x4*)wo = f32x4{o[0], o[1], o[2], o[3]};
      if (d0 == 0) {
        a.ws_ml[row * 2 + 0] = M;
        a.ws_ml[row * 2 + 1] = L;
      }
    }
  }
  if constexpr (FUSED) {
    // Every thread's partial stores have completed at device scope before the
    // arrival is counted; the last arrival reads them back at device scope.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
      const int prev = __hip_atomic_fetch_add(a.counters + unit, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = prev == nparts - 1;
    }
    __syncthreads();
    if (!s_last) return;
    merge_partials<DT, D, true>(a, seq, head0, nh, nparts, threadIdx.x, NW * 64);
    if (threadIdx.x == 0)
      __hip_atomic_store(a.counters + unit, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Second-launch merge: one workgroup per (seq, kv head, head group).
template <int DT, int D>
__global__ __launch_bounds__(256) void paged_decode_reduce(DecodeArgs a) {
  const int unit = blockIdx.x;
  int idx = unit;
  const int hg = idx % a.n_hg;
  idx /= a.n_hg;
  const int kvh = idx % a.num_kv_heads;
  const int seq = idx / a.num_kv_heads;
  const int ctx = clamp_ctx(a, seq, false);
  const int nparts = ctx > 0 ? (ctx + a.part_tokens - 1) / a.part_tokens : 1;
  if (nparts <= 1) return;
  const int nh = min(16, a.n_rep - hg * 16);
  merge_partials<DT, D, false>(a, seq, kvh * a.n_rep + hg * 16, nh, nparts, threadIdx.x, 256);
}

// (sequence, KV head) units that alone cover the 256 CUs: the default takes one
// partition per unit from here on.
constexpr int64_t kUnitsForCUs = 256;

int max_parts_for(int max_blocks, int bs, int part_tokens) {
  const int64_t cap = (int64_t)max_blocks * bs;
  const int64_t p = (cap + part_tokens - 1) / part_tokens;
  return p < 1 ? 1 : (int)p;
}

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

// Workspace layout: [partial acc: rows x D fp32][max,sum: rows x 2 fp32], each
// region 256-byte aligned. The arrival counters live in their own buffer:
// every call leaves them at zero, so one counters buffer may serve calls of
// any shape, while partial rows are scratch that differs from call to call.
struct WsLayout {
  int64_t acc_bytes, ml_bytes;
  int64_t total() const { return acc_bytes + ml_bytes; }
};

WsLayout ws_layout(int num_seqs, int num_q_heads, int head_dim, int max_parts) {
  const int64_t rows = (int64_t)num_seqs * num_q_heads * max_parts;
  return WsLayout{align256(rows * head_dim * 4), align256(rows * 2 * 4)};
}

// Launch shape knobs, read once from the environment for tuning runs:
// IR_DECODE_WAVES (4 or 8 wavefronts per workgroup, default 4),
// IR_DECODE_MERGE ("fused" (default): the last-arriving workgroup merges
// split-KV partials, when the partial rows sit below 2 GiB; "kernel": a second
// launch merges them) and IR_DECODE_DEPTH (tile loads a wavefront keeps in its
// register ring: 1, 2 or 3; by default 2 when the units alone cover the CUs,
// else 1). With one workgroup per unit, contexts of unequal length leave the
// call's tail to a few CUs, each of which then needs two tiles in flight per
// wavefront (64 sequences of 512..4096 keys: 59 us at 2, 79 us at 1); split
// small batches run faster with one, the shorter memory queues speeding up
// their merges (8 fp32 sequences of <= 512 keys: 8.2 us with a second merge
// launch and 2 -> 7.06 us fused with 1; 16 long-context bf16 sequences 35.9 ->
// 33.6 us).
struct LaunchKnobs {
  int waves = 4;
  bool fused = true;
  int depth = 0;  // 0: by batch, as above
  LaunchKnobs() {
    if (const char* e = getenv("IR_DECODE_WAVES")) waves = atoi(e) == 8 ? 8 : 4;
    if (const char* e = getenv("IR_DECODE_MERGE")) fused = strcmp(e, "kernel") != 0;
    if (const char* e = getenv("IR_DECODE_DEPTH")) depth = atoi(e) == 3 ? 3 : atoi(e) == 2 ? 2 : atoi(e) == 1 ? 1 : 0;
  }
};

const LaunchKnobs& knobs() {
  static const LaunchKnobs k;
  return k;
}

template <int DT, int D, bool BS16, int NW, int DEPTH>
void launch_main(const DecodeArgs& a, bool fused, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)a.num_seqs * a.num_kv_heads * a.n_hg), (unsigned)a.max_parts);
  if (fused)
    hipLaunchKernelGGL((paged_decode_kernel<DT, D, BS16, NW, true, DEPTH>), grid, dim3(NW * 64), 0, s, a);
  else
    hipLaunchKernelGGL((paged_decode_kernel<DT, D, BS16, NW, false, DEPTH>), grid, dim3(NW * 64), 0, s, a);
}

template <int DT, int D, bool BS16, int NW>
void launch_depth(const DecodeArgs& a, int depth, bool fused, hipStream_t s) {
  if (depth == 3) launch_main<DT, D, BS16, NW, 3>(a, fused, s);
  else if (depth == 1) launch_main<DT, D, BS16, NW, 1>(a, fused, s);
  else launch_main<DT, D, BS16, NW, 2>(a, fused, s);
}

template <int DT, int D>
int launch_decode(const DecodeArgs& a, bool bs16, bool fused, hipStream_t s) {
  const LaunchKnobs& k = knobs();
  const int depth = k.depth ? k.depth : ((int64_t)a.num_seqs * a.num_kv_heads >= kUnitsForCUs ? 2 : 1);
  if (bs16) {
    if (k.waves == 8) launch_depth<DT, D, true, 8>(a, depth, fused, s);
    else launch_depth<DT, D, true, 4>(a, depth, fused, s);
  } else {
    if (k.waves == 8) launch_depth<DT, D, false, 8>(a, depth, fused, s);
    else launch_depth<DT, D, false, 4>(a, depth, fused, s);
  }
  if (!fused && a.max_parts > 1)
    hipLaunchKernelGGL((paged_decode_reduce<DT, D>), dim3((unsigned)((int64_t)a.num_seqs * a.num_kv_heads * a.n_hg)),
                       dim3(256), 0, s, a);
  return check_launch("ir_paged_decode");
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_paged_decode_default_partition(int num_seqs, int num_kv_heads, int max_blocks_per_seq,
                                                 int block_size) {
  // One partition per (sequence, KV head) when those units alone cover the
  // 256 CUs: no split-KV merge, fewest per-workgroup prologues. Smaller
  // batches split their keys so the table capacity spreads over about 128
  // workgroups or more, in partitions of 64 (one tile per wavefront) to 1024
  // tokens (measured: 8 fp32 sequences of <= 512 keys 6.85 us at 64, 7.25 us
  // at 128, 10.4 us at 512; 16 long-context sequences are fastest at 1024).
  const int64_t units = (int64_t)num_seqs * num_kv_heads;
  if (units >= kUnitsForCUs) return kMaxPartition;
  const int64_t cap = (int64_t)max_blocks_per_seq * block_size;
  int64_t p = (units * cap / 128 + 15) / 16 * 16;
  if (p < 64) p = 64;
  if (p > 1024) p = 1024;
  return (int)p;
}

extern "C" int64_t ir_paged_decode_workspace_size(int num_seqs, int num_q_heads, int num_kv_heads,
                                                  int head_dim, int max_blocks_per_seq, int block_size,
                                                  int partition_tokens) {
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      max_blocks_per_seq < 0)
    return 0;
  if (partition_tokens <= 0)
    partition_tokens = ir_paged_decode_default_partition(num_seqs, num_kv_heads, max_blocks_per_seq, block_size);
  if (num_q_heads % num_kv_heads) return 0;
  const int mp = max_parts_for(max_blocks_per_seq, block_size, partition_tokens);
  if (mp <= 1) return 0;
  return ws_layout(num_seqs, num_q_heads, head_dim, mp).total();
}

extern "C" int64_t ir_paged_decode_num_counters(int num_seqs, int num_q_heads, int num_kv_heads) {
  if (num_seqs <= 0 || num_q_heads <= 0 || num_kv_heads <= 0 || num_q_heads % num_kv_heads) return 0;
  return (int64_t)num_seqs * num_kv_heads * ((num_q_heads / num_kv_heads + 15) / 16);
}

extern "C" int ir_paged_decode(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                               const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                               int64_t cache_head_stride, int64_t num_blocks, int block_size,
                               const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                               const int32_t* context_lens, void* out, int64_t out_seq_stride,
                               int64_t out_head_stride, int num_seqs, int num_q_heads, int num_kv_heads,
                               int head_dim, float scale, int dtype, int partition_tokens,
                               int32_t* counters, int64_t num_counters, void* workspace,
                               int64_t workspace_bytes, int32_t* err_flags, ir_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  IR_REQUIRE(eb > 0, "ir_paged_decode: unknown dtype %d", dtype);
  IR_REQUIRE(num_seqs >= 0 && num_q_heads > 0 && num_kv_heads > 0 && block_size > 0 &&
                 max_blocks_per_seq >= 0 && num_blocks >= 0,
             "ir_paged_decode: bad sizes");
  IR_REQUIRE(num_q_heads % num_kv_heads == 0, "ir_paged_decode: num_q_heads %d not a multiple of num_kv_heads %d",
             num_q_heads, num_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return fail(IR_EUNSUPPORTED, "ir_paged_decode: head_dim %d not supported (64, 128)", head_dim);
  if (num_seqs == 0) return ok();
  IR_REQUIRE(q && k_cache && v_cache && block_tables && context_lens && out, "ir_paged_decode: null pointer");
  IR_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
             "ir_paged_decode: q, caches and out must be 16-byte aligned");
  IR_REQUIRE((q_seq_stride * eb) % 16 == 0 && (q_head_stride * eb) % 16 == 0 &&
                 (cache_slot_stride * eb) % 16 == 0 && (cache_head_stride * eb) % 16 == 0 &&
                 (out_seq_stride * eb) % 16 == 0 && (out_head_stride * eb) % 16 == 0,
             "ir_paged_decode: strides must be multiples of 16 bytes");
  if (partition_tokens <= 0)
    partition_tokens = ir_paged_decode_default_partition(num_seqs, num_kv_heads, max_blocks_per_seq, block_size);
  IR_REQUIRE(partition_tokens % 16 == 0 && partition_tokens <= kMaxPartition,
             "ir_paged_decode: partition_tokens %d must be a multiple of 16 and at most %d", partition_tokens,
             kMaxPartition);
  IR_REQUIRE((int64_t)max_blocks_per_seq * block_size <= (int64_t)1 << 30,
             "ir_paged_decode: block tables of %d x %d tokens exceed 2^30 keys", max_blocks_per_seq, block_size);
  // A 16-token tile starting at a multiple of 16 stays inside one block when the
  // block size is a multiple of 16: then the block id is wave-uniform.
  const bool bs16 = block_size % 16 == 0;

  DecodeArgs a;
  a.q = q;
  a.q_seq = q_seq_stride;
  a.q_head = q_head_stride;
  a.kc = k_cache;
  a.vc = v_cache;
  a.c_slot = cache_slot_stride;
  a.c_head = cache_head_stride;
  a.num_blocks = num_blocks;
  a.bs = block_size;
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks_per_seq;
  a.ctx = context_lens;
  a.out = out;
  a.o_seq = out_seq_stride;
  a.o_head = out_head_stride;
  a.num_seqs = num_seqs;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.n_rep = num_q_heads / num_kv_heads;
  a.n_hg = (a.n_rep + 15) / 16;
  a.scale_log2 = scale * kLog2e;
  a.part_tokens = partition_tokens;
  a.n_ups = num_kv_heads * a.n_hg;
  a.counters = nullptr;
  a.ws_o = nullptr;
  a.ws_ml = nullptr;
  a.err = err_flags;
  a.max_parts = max_parts_for(max_blocks_per_seq, block_size, partition_tokens);
  bool fused = false;
  IR_REQUIRE(a.max_parts <= 65535, "ir_paged_decode: %d partitions exceed the grid limit", a.max_parts);
  if (a.max_parts > 1) {
    const int64_t need = ir_paged_decode_workspace_size(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                                        max_blocks_per_seq, block_size, partition_tokens);
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u))
      return fail(IR_EWORKSPACE, "ir_paged_decode: workspace of %lld bytes (256-byte aligned) required, got %lld",
                  (long long)need, (long long)workspace_bytes);
    const int64_t units = ir_paged_decode_num_counters(num_seqs, num_q_heads, num_kv_heads);
    if (!counters || num_counters < units)
      return fail(IR_EWORKSPACE, "ir_paged_decode: %lld arrival counters required, got %lld", (long long)units,
                  (long long)num_counters);
    const WsLayout ly = ws_layout(num_seqs, num_q_heads, head_dim, a.max_parts);
    a.counters = counters;
    a.ws_o = (float*)workspace;
    a.ws_ml = (float*)((uint8_t*)workspace + ly.acc_bytes);
    fused = knobs().fused && ly.acc_bytes < ((int64_t)1 << 31);
  }
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case IR_DTYPE_BF16:
      return head_dim == 128 ? launch_decode<IR_DTYPE_BF16, 128>(a, bs16, fused, s)
                             : launch_decode<IR_DTYPE_BF16, 64>(a, bs16, fused, s);
    case IR_DTYPE_F16:
      return head_dim == 128 ? launch_decode<IR_DTYPE_F16, 128>(a, bs16, fused, s)
                             : launch_decode<IR_DTYPE_F16, 64>(a, bs16, fused, s);
    default:
      return head_dim == 128 ? launch_decode<IR_DTYPE_F32, 128>(a, bs16, fused, s)
                             : launch_decode<IR_DTYPE_F32, 64>(a, bs16, fused, s);
  }
}
