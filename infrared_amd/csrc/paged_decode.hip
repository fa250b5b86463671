// GQA paged decode attention for gfx950 (one query token per sequence).
//
// Work decomposition: one workgroup per (sequence, KV head, head group of <=16
// query heads, partition of `part_tokens` keys). Its kWaves wavefronts take
// the partition's 16-token tiles round-robin. Per tile a wavefront
//   1. loads the 16 K rows and 16 V rows of its KV head straight from the pool
//      with 16-byte loads (each row of one head is head_dim contiguous
//      elements; the K/V tile is fetched once and serves every query head of
//      the GQA group),
//   2. scores S^T[token][head] = K . Q^T with MFMA (rows = 16 tokens, columns =
//      the group's query heads, padded to 16),
//   3. runs the online softmax in base 2 on the MFMA accumulator: per head the
//      16 scores sit in 4 registers of 4 lane groups, so the tile max needs two
//      cross-group shuffles,
//   4. accumulates O^T[d][head] += V^T . P^T with MFMA, where the P^T operand is
//      exactly the lane's own four probabilities and the V^T operand is a
//      register-level 4x(head_dim/16) transpose of the loaded V rows.
// Loads run one tile ahead of the math (a register ring), and the block ids
// of a wavefront's tiles are fetched up front, one per lane, so no load waits
// on a block-table read.
//
// The wavefronts' (max, sum, acc) states merge through LDS. A sequence that
// fits one partition writes its output directly. Longer ones write fp32
// partials; the last workgroup of a (sequence, KV head, head group) to finish
// -- found with an arrival counter in the workspace -- merges them with
// log-sum-exp weights and resets the counter to zero, so one launch does the
// whole call and the workspace is clean for the next one.
//
// Algorithm parity: the one-shot softmax of infrared/model/layers.py:102-118
// over the gathered history (infrared/model/triton_attention.py:110-129), with
// the streaming max/sum update of infrared/model/triton_attention.py:135-177 and
// the exp2 fold of infrared/model/triton_attention.py:249. For 16-bit dtypes
// the probabilities are rounded to the input dtype before the PV product, as
// `softmax(scores.float()).to(q.dtype)` does in the reference.
#include <stdlib.h>
#include <string.h>

#include "attn_tile.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kMaxWaveTiles = 64;  // tiles per wavefront (one block id per lane)
constexpr int kMaxPartition = 16 * kMaxWaveTiles * 4;  // tokens (4 wavefronts)

struct DecodeArgs {
  const void* q;
  int64_t q_seq, q_head;  // elements
  const void* kc;
  const void* vc;
  int64_t c_slot, c_head;  // elements
  int64_t num_blocks;
  int bs;
  const int32_t* bt;
  int64_t bt_stride;
  int max_blocks;
  const int32_t* ctx;
  void* out;
  int64_t o_seq, o_head;  // elements
  int num_seqs, num_q_heads, num_kv_heads, n_rep, n_hg;
  float scale_log2;
  int part_tokens, max_parts;
  int32_t* counters;  // [seq][kv_head][head group], zero at rest
  float* ws_o;        // [seq][q_head][part][D]
  float* ws_ml;       // [seq][q_head][part][2]
  int32_t* err;
};

// Issues the loads of the tile starting at key t0 and returns a 4-bit mask of
// which of this lane's keys 4r+g (r = 0..3) may be used (the keys whose scores
// and V rows this lane holds, see staged_token). Every load is issued unconditionally and nothing else
// touches memory here: an unusable key (bad block id, past the context) reads
// row 0 of the pool instead and is masked in the math, and a bad block id only
// sets `bad` (reported once after the loop). That keeps the hardware wait
// counts exact, with no load-free or extra-memory-op path.
// BS16: `bid` is the tile's wave-uniform block id; otherwise every lane
// resolves its own keys through the block table.
// Per-lane byte offsets of this lane's K pieces and V rows inside a 16-token
// tile, relative to the tile's first row; constant across tiles when the tile
// is one block's contiguous rows, so a tile load is uniform base + offset.
template <int DT, int D>
struct LaneOffsets {
  uint32_t k[KStage<DT, D>::NI];
  uint32_t v[4];
};

template <int DT, int D>
__device__ __forceinline__ LaneOffsets<DT, D> lane_offsets(int lane, int64_t slot_bytes) {
  typedef TileShape<DT, D> Sh;
  LaneOffsets<DT, D> o;
  const int g = lane >> 4, c = lane & 15;
#pragma unroll
  for (int i = 0; i < KStage<DT, D>::NI; ++i)
    o.k[i] = (uint32_t)(kstage_row<DT, D>(i, lane) * slot_bytes + 16 * kstage_chunk<DT, D>(lane));
#pragma unroll
  for (int r = 0; r < 4; ++r) o.v[r] = (uint32_t)((4 * r + g) * slot_bytes + Sh::TILES * c * Sh::EB);
  return o;
}

template <int DT, int D, bool BS16>
__device__ __forceinline__ uint32_t load_tile(const DecodeArgs& a, const int32_t* bt_row, int32_t bid,
                                              const uint8_t* kc, const uint8_t* vc, const LaneOffsets<DT, D>& lo,
                                              int t0, int t_end, int lane, Tile<DT, D>& tl, bool& bad) {
  typedef TileShape<DT, D> Sh;
  const int g = lane >> 4, c = lane & 15;
  const int64_t slot_bytes = a.c_slot * Sh::EB;
  if constexpr (BS16) {
    // The whole tile lies in one block, and every row of a block is inside the
    // pool even past the context end. The tile base is wave-uniform.
    const int blk = t0 / a.bs;
    const bool ok = bid >= 0 && (int64_t)bid < a.num_blocks;
    bad |= !ok;
    const int64_t base = ok ? (int64_t)bid * a.bs + (t0 - blk * a.bs) : 0;
    const uint8_t* tk = kc + base * slot_bytes;
    const uint8_t* tv = vc + base * slot_bytes;
#pragma unroll
    for (int i = 0; i < KStage<DT, D>::NI; ++i) {
      const u32x4 x = __builtin_nontemporal_load((const u32x4*)(tk + lo.k[i]));
      tl.k[4 * i + 0] = x[0];
      tl.k[4 * i + 1] = x[1];
      tl.k[4 * i + 2] = x[2];
      tl.k[4 * i + 3] = x[3];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) load_dwords_nt<Sh::VDW, true>(tv + lo.v[r], tl.v[r]);
    uint32_t m = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) m |= (ok && t0 + 4 * r + g < t_end) ? (1u << r) : 0u;
    return m;
  } else {
    kstage_load<DT, D, true>(
        [&](int t) {
          const int tk = t0 + t;
          const int64_t ks = tk < t_end ? token_slot_or_neg(bt_row, tk, a.bs, a.num_blocks) : 0;
          bad |= ks < 0;
          return kc + (ks >= 0 ? ks : 0) * slot_bytes;
        },
        lane, tl.k);
    uint32_t m = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tv = t0 + 4 * r + g;
      const int64_t vs = tv < t_end ? token_slot_or_neg(bt_row, tv, a.bs, a.num_blocks) : -1;
      load_v_nt<DT, D, true>(vc + (vs >= 0 ? vs : 0) * slot_bytes, c, tl.v[r]);
      m |= vs >= 0 ? (1u << r) : 0u;
    }
    return m;
  }
}

// kmask: which of this lane's keys 4r+g are usable; a tile whose keys are
// all usable in every lane takes the unmasked path.
template <int DT, int D>
__device__ __forceinline__ void compute_tile(const Tile<DT, D>& tl, const uint32_t (&qr)[TileShape<DT, D>::KDW],
                                             uint32_t kmask, float scale_log2, uint8_t* kst, int lane, State<D>& st) {
  uint32_t kop[TileShape<DT, D>::KDW];
  kstage_transpose<DT, D>(kst, lane, tl.k, kop);
  const f32x4 s = qk_tile<DT, D>(kop, qr);
  float sv[4];
  bool vok[4];
  if (__all(kmask == 0xfu)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      vok[r] = true;
      sv[r] = s[r] * scale_log2;
    }
    softmax_pv<DT, D, true>(sv, tl.v, vok, st);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      vok[r] = (kmask >> r) & 1u;
      sv[r] = vok[r] ? s[r] * scale_log2 : kNegInf;
    }
    softmax_pv<DT, D, false>(sv, tl.v, vok, st);
  }
}

// Context length of `seq`, clamped to what its block table can hold (flagged).
__device__ __forceinline__ int clamp_ctx(const DecodeArgs& a, int seq, bool report) {
  int ctx = a.ctx[seq];
  const int cap = a.max_blocks * a.bs;
  if (ctx < 0 || ctx > cap) {
    if (report) flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    ctx = ctx < 0 ? 0 : cap;
  }
  return ctx;
}

// Device-scope (sc1) accesses for the split-KV partials: written through to
// the device coherence point and read back from it, so one workgroup can merge
// what workgroups on other XCDs wrote without a cache-wide fence.
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Log-sum-exp merge of the partitions of (seq, heads head0..head0+nh) into out.
template <int DT, int D, bool DEV>
__device__ __forceinline__ void merge_partials(const DecodeArgs& a, int seq, int head0, int nh, int nparts,
                                               int tid, int nthreads) {
  constexpr int EB = TileShape<DT, D>::EB;
  for (int it = tid; it < nh * (D / 4); it += nthreads) {
    const int hc = it / (D / 4);
    const int d0 = (it - hc * (D / 4)) * 4;
    const int64_t row0 = ((int64_t)seq * a.num_q_heads + head0 + hc) * a.max_parts;
    const float* ml = a.ws_ml + row0 * 2;
    float M = kNegInf;
    for (int p = 0; p < nparts; ++p) M = fmaxf(M, DEV ? load_dev(ml + 2 * p) : ml[2 * p]);
    float L = 0.f;
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < nparts; ++p) {
      const float mp = DEV ? load_dev(ml + 2 * p) : ml[2 * p];
      const float lp = DEV ? load_dev(ml + 2 * p + 1) : ml[2 * p + 1];
      const float wt = mp == kNegInf ? 0.f : fast_exp2(mp - M);
      L += wt * lp;
      const float* src = a.ws_o + (row0 + p) * D + d0;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] += wt * (DEV ? load_dev(src + k) : src[k]);
    }
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
  // (an empty pool has nothing to read: every key is unusable)
  const int ntiles = (t_end > t_begin && a.num_blocks > 0) ? (t_end - t_begin + 15) >> 4 : 0;
  // this wavefront's tiles: partition tiles w, w + NW, ...
  const int my_tiles = ntiles > w ? (ntiles - w + NW - 1) / NW : 0;

  const int h_local = hg * 16 + c;
  const bool head_ok = h_local < a.n_rep;
  const int qh = kvh * a.n_rep + h_local;

  const int32_t* bt_row = a.bt + (int64_t)seq * a.bt_stride;
  // Block ids of this wavefront's tiles, lane j holding tile j (a wavefront
  // has at most kMaxWaveTiles tiles), fetched once so no tile load waits on a
  // block-table read.
  int32_t bid_lane = 0;
  if constexpr (BS16) {
    if (lane < my_tiles) bid_lane = bt_row[(t_begin + 16 * (w + NW * lane)) / a.bs];
  }
  const uint8_t* kc = (const uint8_t*)a.kc + (int64_t)kvh * a.c_head * EB;
  const uint8_t* vc = (const uint8_t*)a.vc + (int64_t)kvh * a.c_head * EB;
  const LaneOffsets<DT, D> lo = lane_offsets<DT, D>(lane, a.c_slot * EB);

  // Q^T operand, same k-slot assignment as the K loads; padded heads are zero.
  uint32_t qr[Sh::KDW];
  if (head_ok)
    load_k<DT, D>((const uint8_t*)a.q + ((int64_t)seq * a.q_seq + (int64_t)qh * a.q_head) * EB, g, qr);
  else
    zero_dwords(qr);

  State<D> st;
  state_init(st);

  auto tile_t0 = [&](int i) { return t_begin + 16 * (w + NW * i); };
  bool bad = false;
  auto issue = [&](int i, Tile<DT, D>& tl) -> uint32_t {
    const int32_t bid = BS16 ? __builtin_amdgcn_readlane(bid_lane, i) : 0;
    return load_tile<DT, D, BS16>(a, bt_row, bid, kc, vc, lo, tile_t0(i), t_end, lane, tl, bad);
  };

  // Register ring of DEPTH tiles: while one tile is in the math, the next
  // DEPTH-1 tiles' loads are in flight. The loop body is straight-line so the
  // loads' wait counts stay exact: issues past the end re-read the last tile
  // (still in L2) and a slot past the end is computed with an empty key mask,
  // which changes nothing.
  if (my_tiles > 0) {
    const int last = my_tiles - 1;
    Tile<DT, D> ring[DEPTH];
    uint32_t mk[DEPTH];
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) mk[r] = issue(min(r, last), ring[r]);
    for (int i = 0; i < my_tiles; i += DEPTH) {
#pragma unroll
      for (int r = 0; r < DEPTH; ++r) {
        compute_tile<DT, D>(ring[r], qr, i + r < my_tiles ? mk[r] : 0u, a.scale_log2, kstage[w], lane, st);
        mk[r] = issue(min(i + r + DEPTH, last), ring[r]);
      }
    }
  }
  if (bad) flag_error(a.err, IR_ERR_BLOCK_RANGE);
  st.l = wave_sum_groups(st.l);

  // ---- merge the wavefronts of this workgroup through LDS
  merge_publish<NW, D>(sm, st, w, g, c);
  __syncthreads();

  const int nh = min(16, a.n_rep - hg * 16);
  const int head0 = kvh * a.n_rep + hg * 16;
  if (nparts == 1) {
    for (int it = threadIdx.x; it < nh * (D / 4); it += NW * 64) {
      const int hc = it / (D / 4);
      const int d0 = (it - hc * (D / 4)) * 4;
      float M, L, o[4];
      merge_column<NW, D>(sm, hc, d0, M, L, o);
      const float inv = L > 0.f ? 1.f / L : 0.f;
      store4<DT>((uint8_t*)a.out + ((int64_t)seq * a.o_seq + (int64_t)(head0 + hc) * a.o_head + d0) * EB, o, inv);
    }
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
#pragma unroll
      for (int k = 0; k < 4; ++k) store_dev(wo + k, o[k]);
      if (d0 == 0) {
        store_dev(a.ws_ml + row * 2 + 0, M);
        store_dev(a.ws_ml + row * 2 + 1, L);
      }
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

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

int max_parts_for(int max_blocks, int bs, int part_tokens) {
  const int64_t cap = (int64_t)max_blocks * bs;
  const int64_t p = (cap + part_tokens - 1) / part_tokens;
  return p < 1 ? 1 : (int)p;
}

// Workspace layout: [counters: units int32][partial acc: rows x D fp32][max,sum: rows x 2 fp32],
// each region 256-byte aligned.
struct WsLayout {
  int64_t counters_bytes, acc_bytes, ml_bytes;
  int64_t total() const { return counters_bytes + acc_bytes + ml_bytes; }
};

WsLayout ws_layout(int num_seqs, int num_q_heads, int num_kv_heads, int head_dim, int max_parts) {
  const int n_hg = (num_q_heads / num_kv_heads + 15) / 16;
  const int64_t units = (int64_t)num_seqs * num_kv_heads * n_hg;
  const int64_t rows = (int64_t)num_seqs * num_q_heads * max_parts;
  return WsLayout{align256(units * 4), align256(rows * head_dim * 4), align256(rows * 2 * 4)};
}

// Launch shape knobs, read once from the environment for tuning runs:
// IR_DECODE_WAVES (4 or 8 wavefronts per workgroup, default 4),
// IR_DECODE_MERGE ("kernel" (default): a second launch merges split-KV
// partials; "fused": the last-arriving workgroup merges them) and
// IR_DECODE_DEPTH (tiles in flight per wavefront, 2 (default) or 3).
struct LaunchKnobs {
  int waves = 4;
  bool fused = false;
  int depth = 2;
  LaunchKnobs() {
    if (const char* e = getenv("IR_DECODE_WAVES")) waves = atoi(e) == 8 ? 8 : 4;
    if (const char* e = getenv("IR_DECODE_MERGE")) fused = strcmp(e, "fused") == 0;
    if (const char* e = getenv("IR_DECODE_DEPTH")) depth = atoi(e) == 3 ? 3 : 2;
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
void launch_depth(const DecodeArgs& a, const LaunchKnobs& k, hipStream_t s) {
  if (k.depth == 3) launch_main<DT, D, BS16, NW, 3>(a, k.fused, s);
  else launch_main<DT, D, BS16, NW, 2>(a, k.fused, s);
}

template <int DT, int D>
int launch_decode(const DecodeArgs& a, bool bs16, hipStream_t s) {
  const LaunchKnobs& k = knobs();
  if (bs16) {
    if (k.waves == 8) launch_depth<DT, D, true, 8>(a, k, s);
    else launch_depth<DT, D, true, 4>(a, k, s);
  } else {
    if (k.waves == 8) launch_depth<DT, D, false, 8>(a, k, s);
    else launch_depth<DT, D, false, 4>(a, k, s);
  }
  if (!k.fused && a.max_parts > 1)
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
  // 256 CUs: no split-KV merge, fewest per-workgroup prologues. Otherwise
  // 1024-token partitions spread the keys over enough workgroups.
  (void)block_size;
  (void)max_blocks_per_seq;
  const int64_t units = (int64_t)num_seqs * num_kv_heads;
  return units >= 256 ? kMaxPartition : 1024;
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
  return ws_layout(num_seqs, num_q_heads, num_kv_heads, head_dim, mp).total();
}

extern "C" int ir_paged_decode(const void* q, int64_t q_seq_stride, int64_t q_head_stride,
                               const void* k_cache, const void* v_cache, int64_t cache_slot_stride,
                               int64_t cache_head_stride, int64_t num_blocks, int block_size,
                               const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                               const int32_t* context_lens, void* out, int64_t out_seq_stride,
                               int64_t out_head_stride, int num_seqs, int num_q_heads, int num_kv_heads,
                               int head_dim, float scale, int dtype, int partition_tokens,
                               void* workspace, int64_t workspace_bytes, int32_t* err_flags,
                               ir_stream_t stream) {
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
  a.max_parts = max_parts_for(max_blocks_per_seq, block_size, partition_tokens);
  a.counters = nullptr;
  a.ws_o = nullptr;
  a.ws_ml = nullptr;
  a.err = err_flags;
  IR_REQUIRE(a.max_parts <= 65535, "ir_paged_decode: %d partitions exceed the grid limit", a.max_parts);
  if (a.max_parts > 1) {
    const int64_t need = ir_paged_decode_workspace_size(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                                        max_blocks_per_seq, block_size, partition_tokens);
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u))
      return fail(IR_EWORKSPACE, "ir_paged_decode: workspace of %lld bytes (256-byte aligned) required, got %lld",
                  (long long)need, (long long)workspace_bytes);
    const WsLayout ly = ws_layout(num_seqs, num_q_heads, num_kv_heads, head_dim, a.max_parts);
    a.counters = (int32_t*)workspace;
    a.ws_o = (float*)((uint8_t*)workspace + ly.counters_bytes);
    a.ws_ml = (float*)((uint8_t*)workspace + ly.counters_bytes + ly.acc_bytes);
  }
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case IR_DTYPE_BF16:
      return head_dim == 128 ? launch_decode<IR_DTYPE_BF16, 128>(a, bs16, s)
                             : launch_decode<IR_DTYPE_BF16, 64>(a, bs16, s);
    case IR_DTYPE_F16:
      return head_dim == 128 ? launch_decode<IR_DTYPE_F16, 128>(a, bs16, s)
                             : launch_decode<IR_DTYPE_F16, 64>(a, bs16, s);
    default:
      return head_dim == 128 ? launch_decode<IR_DTYPE_F32, 128>(a, bs16, s)
                             : launch_decode<IR_DTYPE_F32, 64>(a, bs16, s);
  }
}
