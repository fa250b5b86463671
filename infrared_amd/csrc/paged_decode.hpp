// Device building blocks of the GQA paged decode kernel (one query token per
// sequence, paged_decode.hip).
//
// A "unit" is (sequence, KV head, group of <= 16 query heads of that KV head):
// the K/V rows of one KV head serve every query head of the group, so a unit
// reads each of its keys exactly once. A unit's keys are cut into 16-token
// tiles; the wavefronts of a workgroup take a run of tiles round-robin. Per
// tile a wavefront
//   1. loads the 16 K rows and 16 V rows of its KV head straight from the pool
//      with 16-byte loads (each row of one head is head_dim contiguous
//      elements),
//   2. scores S^T[token][head] = K . Q^T with MFMA (rows = 16 tokens, columns =
//      the group's query heads, padded to 16),
//   3. runs the online softmax in base 2 on the MFMA accumulator,
//   4. accumulates O^T[d][head] += V^T . P^T with MFMA (the P^T operand is the
//      lane's own four probabilities, V^T a register-level transpose).
// Loads run DEPTH-1 tiles ahead of the math (a register ring), and the block
// ids of a wavefront's tiles are fetched up front, one per lane, so no tile
// load waits on a block-table read.
//
// Algorithm parity: the one-shot softmax of infrared/model/layers.py:102-118
// over the gathered history (infrared/model/triton_attention.py:110-129), with
// the streaming max/sum update of infrared/model/triton_attention.py:135-177 and
// the exp2 fold of infrared/model/triton_attention.py:249. For 16-bit dtypes
// the probabilities are rounded to the input dtype before the PV product, as
// `softmax(scores.float()).to(q.dtype)` does in the reference.
#pragma once

#include "attn_tile.hpp"

namespace ir {

constexpr int kMaxWaveTiles = 64;  // tiles per wavefront and run (one block id per lane)
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
  int n_ups;          // units per sequence: num_kv_heads * n_hg (planned schedule)
  int32_t* counters;  // [seq][kv_head][head group], zero at rest
  float* ws_o;        // [seq][q_head][part][D]
  float* ws_ml;       // [seq][q_head][part][2]
  int32_t* err;
};

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

// Issues the loads of the tile starting at key t0 and returns a 4-bit mask of
// which of this lane's keys 4r+g (r = 0..3) may be used (the keys whose scores
// and V rows this lane holds, see staged_token). Every load is issued
// unconditionally and nothing else touches memory here: an unusable key (bad
// block id, past the context) reads row 0 of the pool instead and is masked in
// the math, and a bad block id only sets `bad` (reported once after the loop).
// That keeps the hardware wait counts exact, with no load-free or
// extra-memory-op path.
// BS16: `bid` is the tile's wave-uniform block id; otherwise every lane
// resolves its own keys through the block table.
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
// all usable in every lane takes the unmasked path. col_on: whether this
// lane's query column attends the tile at all (a unit shared by two sequences
// runs each one's private tiles with the other's columns off). An off column
// gets -inf scores, so zero probabilities; the V rows stay, since a lane's V
// operand serves every column of the PV product.
template <int DT, int D>
__device__ __forceinline__ void compute_tile(const Tile<DT, D>& tl, const uint32_t (&qr)[TileShape<DT, D>::KDW],
                                             uint32_t kmask, float scale_log2, uint8_t* kst, int lane, State<D>& st,
                                             bool col_on = true) {
  uint32_t kop[TileShape<DT, D>::KDW];
  kstage_transpose<DT, D>(kst, lane, tl.k, kop);
  const f32x4 s = qk_tile<DT, D>(kop, qr);
  float sv[4];
  bool vok[4];
  if (__all(kmask == 0xfu)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      vok[r] = true;
      sv[r] = col_on ? s[r] * scale_log2 : kNegInf;
    }
    softmax_pv<DT, D, true>(sv, tl.v, vok, st);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      vok[r] = (kmask >> r) & 1u;
      sv[r] = vok[r] && col_on ? s[r] * scale_log2 : kNegInf;
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

// Accumulates this wavefront's share of the unit's tiles [tile_lo, tile_hi)
// (wavefront w takes tiles tile_lo + w, tile_lo + w + NW, ...) into st. Keys
// at or past t_end are masked. Runs of up to NW * kMaxWaveTiles tiles: each
// run fetches its block ids once, one per lane.
template <int DT, int D, bool BS16, int NW, int DEPTH>
__device__ __forceinline__ void attend_tiles(const DecodeArgs& a, const int32_t* bt_row, const uint8_t* kc,
                                             const uint8_t* vc, const LaneOffsets<DT, D>& lo,
                                             const uint32_t (&qr)[TileShape<DT, D>::KDW], int tile_lo, int tile_hi,
                                             int t_end, uint8_t* kst, int lane, int w, State<D>& st, bool& bad) {
  constexpr int RUN = NW * kMaxWaveTiles;
  for (int r0 = tile_lo; r0 < tile_hi; r0 += RUN) {
    const int ntiles = min(tile_hi - r0, RUN);
    const int my_tiles = ntiles > w ? (ntiles - w + NW - 1) / NW : 0;
    if (my_tiles <= 0) break;
    const int t_begin = 16 * r0;
    int32_t bid_lane = 0;
    if constexpr (BS16) {
      if (lane < my_tiles) bid_lane = bt_row[(t_begin + 16 * (w + NW * lane)) / a.bs];
    }
    auto issue = [&](int i, Tile<DT, D>& tl) -> uint32_t {
      const int32_t bid = BS16 ? __builtin_amdgcn_readlane(bid_lane, i) : 0;
      return load_tile<DT, D, BS16>(a, bt_row, bid, kc, vc, lo, t_begin + 16 * (w + NW * i), t_end, lane, tl, bad);
    };
    // Register ring of DEPTH tiles: while one tile is in the math, the next
    // DEPTH-1 tiles' loads are in flight.
    const int last = my_tiles - 1;
    Tile<DT, D> ring[DEPTH];
    uint32_t mk[DEPTH];
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) mk[r] = issue(min(r, last), ring[r]);
    int i = 0;
    // Steady state: every issue is a real tile, so the body is straight-line
    // and the loads' wait counts are exact (a conditional issue here makes the
    // compiler drain the ring every tile: 59 -> 67 us on 64 sequences).
    for (; i + 2 * DEPTH <= my_tiles; i += DEPTH) {
#pragma unroll
      for (int r = 0; r < DEPTH; ++r) {
        compute_tile<DT, D>(ring[r], qr, mk[r], a.scale_log2, kst, lane, st);
        mk[r] = issue(i + r + DEPTH, ring[r]);
      }
    }
    // The last tiles: nothing is issued past the end (the merge after the loop
    // reuses the ring's registers and would wait for such loads); a slot past
    // the end is computed with an empty key mask, which changes nothing.
    for (; i < my_tiles; i += DEPTH) {
#pragma unroll
      for (int r = 0; r < DEPTH; ++r) {
        compute_tile<DT, D>(ring[r], qr, i + r < my_tiles ? mk[r] : 0u, a.scale_log2, kst, lane, st);
        if (i + r + DEPTH <= last) mk[r] = issue(i + r + DEPTH, ring[r]);
      }
    }
  }
}

// Q^T operand of (seq, query head qh), same k-slot assignment as the K loads;
// padded heads are zero.
template <int DT, int D>
__device__ __forceinline__ void load_query(const DecodeArgs& a, int seq, int qh, bool head_ok, int g,
                                           uint32_t (&qr)[TileShape<DT, D>::KDW]) {
  if (head_ok)
    load_k<DT, D>((const uint8_t*)a.q + ((int64_t)seq * a.q_seq + (int64_t)qh * a.q_head) * TileShape<DT, D>::EB, g,
                  qr);
  else
    zero_dwords(qr);
}

// Writes the workgroup's merged (normalised) result for heads head0..head0+nh.
template <int DT, int D, int NW>
__device__ __forceinline__ void store_merged(const DecodeArgs& a, const MergeSmem<NW, D>& sm, int seq, int head0,
                                             int nh) {
  constexpr int EB = TileShape<DT, D>::EB;
  for (int it = threadIdx.x; it < nh * (D / 4); it += NW * 64) {
    const int hc = it / (D / 4);
    const int d0 = (it - hc * (D / 4)) * 4;
    float M, L, o[4];
    merge_column<NW, D>(sm, hc, d0, M, L, o);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    store4<DT>((uint8_t*)a.out + ((int64_t)seq * a.o_seq + (int64_t)(head0 + hc) * a.o_head + d0) * EB, o, inv);
  }
}

// Log-sum-exp merge of n partial rows (acc at o[k * o_step], (max, sum) at
// ml[k * ml_step]) for 4 outputs d0..d0+3; `ld` reads one fp32.
template <typename Ld>
__device__ __forceinline__ void lse_merge(const float* o, int64_t o_step, const float* ml, int64_t ml_step, int n,
                                          Ld ld, float (&acc)[4], float& L) {
  float M = kNegInf;
  for (int p = 0; p < n; ++p) M = fmaxf(M, ld(ml + p * ml_step));
  L = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) acc[k] = 0.f;
  for (int p = 0; p < n; ++p) {
    const float mp = ld(ml + p * ml_step);
    const float lp = ld(ml + p * ml_step + 1);
    const float wt = mp == kNegInf ? 0.f : fast_exp2(mp - M);
    L += wt * lp;
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] += wt * ld(o + p * o_step + k);
  }
}

}  // namespace ir
