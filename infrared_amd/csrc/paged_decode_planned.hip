// Planned GQA paged decode: a work-balanced schedule computed once per batch
// of decode metadata (ir_paged_decode_plan) and run by every layer
// (ir_paged_decode_planned).
//
// Why balance: context lengths in a decode batch vary several-fold, and a CU
// streams at most ~36 GB/s however many workgroups it holds. With one
// workgroup per (sequence, KV head) the longest sequences set the call time
// while most CUs idle; splitting each sequence into fixed partitions does not
// help either, because the dispatcher places workgroup i and i + #CUs on the
// same CU. Here the call's 16-key tiles, ordered (sequence, unit, tile), form
// one list of
//   T = n_ups * sum_b ceil(context_b / 16)
// tiles (unit = KV head x group of <= 16 query heads; n_ups units per
// sequence), and workgroup g of a grid of one workgroup per CU takes the slice
// [g R, min((g + 1) R, T)), R = max(ceil(T / grid), 16), so every CU reads the
// same number of keys to within a tile.
//
// Why plan: a slice needs the prefix sums of all context lengths and every
// tile's block id. All layers of a decode step share block_tables and
// context_lens, so the plan kernel computes them once -- for each tile its
// pool offset (16-byte units, KV head included) and (unit << 5 | valid keys),
// for each wavefront a header at a fixed address -- and the per-layer kernel
// starts streaming one round trip after launch.
//
// The run: wavefront w of a workgroup takes the w-th contiguous quarter of its
// slice and streams it through a register ring that runs straight across unit
// boundaries (the tile math is paged_decode.hpp's, the next unit's query is
// prefetched). A unit inside the wavefront's quarter is normalised and written
// straight from registers. A unit that continues into later quarters stays in
// the registers of the wavefront that began it (its owner); the others leave
// their state in an LDS slot, and after the loop the owner folds them in. A
// unit cut by the slice's ends is staged in LDS; the workgroup writes it as an
// fp32 partial row (device scope), counts its arrival on the unit's counter,
// and the last of the unit's slices merges the rows with log-sum-exp weights
// and resets the counter, so a call is one launch and the counters are zero
// again after it.
#include <stdlib.h>
#include <string.h>

#include "paged_decode.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kPlanMaxSeqs = 1024;  // sequences per plan (prefix sums held in LDS)
constexpr int kPlanWaves = 4;       // streaming wavefronts per workgroup
constexpr int kPlanRun = 64;        // tile facts per wavefront and run (one per lane)
constexpr int kPlanMinTiles = 16;   // smallest slice

// Plan regions (byte offsets, 256-byte aligned):
//   hdr[8]             T, R, number of sequences with no usable key, number of pairs
//   seq_pre[B + 1]     list tiles before sequence b, per unit
//   empty[B]           sequences with no usable key
//   share[B]           shared 16-key tiles of sequences b, b + 1 (ir_paged_decode_plan's pair scan)
//   pair[B]            shared tiles of a pair's first sequence, -1 for its second, 0 alone
//   whdr[G][NW][8]     per wavefront: wlo, count, first unit, last unit, slice lo, hi,
//                      the slice's first and last unit
//   first[G][NW][64]   the first 64 tile facts of each wavefront
//   facts[T_cap]       every tile's facts in list order: (pool offset / 16 B,
//                      unit << 7 | column mask << 5 | valid keys)
struct PlanLayout {
  int64_t hdr, seq_pre, empty, share, pair, whdr, first, facts, total;
};

PlanLayout plan_layout(int64_t num_seqs, int64_t grid, int64_t t_cap) {
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  PlanLayout p;
  p.hdr = 0;
  p.seq_pre = al(p.hdr + 8 * 4);
  p.empty = al(p.seq_pre + (num_seqs + 1) * 4);
  p.share = al(p.empty + num_seqs * 4);
  p.pair = al(p.share + num_seqs * 4);
  p.whdr = al(p.pair + num_seqs * 4);
  p.first = al(p.whdr + grid * kPlanWaves * 8 * 4);
  p.facts = al(p.first + grid * kPlanWaves * kPlanRun * 8);
  p.total = al(p.facts + t_cap * 8);
  return p;
}

struct PlanArgs {
  const int32_t* bt;
  int64_t bt_stride;
  int max_blocks;
  const int32_t* ctx;
  int num_seqs, n_ups, n_hg, bs;
  int64_t num_blocks, c_slot16, c_head16;
  int min_tiles;
  int pairs;  // pair sequences that share prefix blocks into one unit
  uint8_t* plan;
  PlanLayout ly;
  int32_t* err;
};

// Workspace of the run: the partial rows [(grid + units) x 16 heads] of D fp32
// accumulators and (max, sum) pairs. A slice g writes unit u's partial at row
// g + u: rows are unique because slices and units are both increasing runs of
// the tile list, so a later slice never meets an earlier unit. The arrival
// counters ([units] int32, zero at rest) are a separate buffer.
struct PlannedWs {
  int64_t acc_bytes, ml_bytes;
  int64_t total() const { return acc_bytes + ml_bytes; }
};

PlannedWs planned_ws(int64_t units, int grid, int head_dim) {
  auto al = [](int64_t x) { return (x + 255) & ~(int64_t)255; };
  const int64_t rows = ((int64_t)grid + units) * 16;
  return PlannedWs{al(rows * head_dim * 4), al(rows * 2 * 4)};
}

// floor(x / d) for 0 <= x < 2^30 and quotients below 2^22: a float
// reciprocal estimate within one of the quotient, then an exact fix-up.
__device__ __forceinline__ int fdiv(int x, int d) {
  int q = (int)((float)x * __builtin_amdgcn_rcpf((float)d));
  int r = x - q * d;
  if (r < 0) {
    --q;
    r += d;
  }
  if (r >= d) ++q;
  return q;
}

// Issues the K and V loads of one tile whose first row sits `off16` 16-byte
// units past the pool bases.
template <int DT, int D>
__device__ __forceinline__ void issue_tile(const uint8_t* kc, const uint8_t* vc, uint32_t off16,
                                           const LaneOffsets<DT, D>& lo, Tile<DT, D>& tl) {
  typedef TileShape<DT, D> Sh;
  const uint64_t base = (uint64_t)off16 << 4;
  const uint8_t* tk = kc + base;
  const uint8_t* tv = vc + base;
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
}

// Writes the TILES consecutive outputs acc[0..TILES)[r] (one O^T register row
// of this lane) times `inv` to dst (non-temporal, as store4).
template <int DT, int D>
__device__ __forceinline__ void store_acc_run(uint8_t* dst, const State<D>& st, int r, float inv) {
  constexpr int TILES = D / 16;
  if constexpr (DT == IR_DTYPE_F32) {
#pragma unroll
    for (int n = 0; n < TILES; n += 4)
      *(f32x4*)(dst + 4 * n) = f32x4{st.acc[n][r] * inv, st.acc[n + 1][r] * inv, st.acc[n + 2][r] * inv,
                                     st.acc[n + 3][r] * inv};
  } else {
    using E = Elem<DT>;
    uint32_t wv[TILES / 2];
#pragma unroll
    for (int n = 0; n < TILES; n += 2) wv[n / 2] = E::pack2(st.acc[n][r] * inv, st.acc[n + 1][r] * inv);
    if constexpr (TILES == 8)
      __builtin_nontemporal_store(u32x4{wv[0], wv[1], wv[2], wv[3]}, (u32x4*)dst);
    else
      __builtin_nontemporal_store(u32x2{wv[0], wv[1]}, (u32x2*)dst);
  }
}

// Folds the state (m2, l2, acc2) into st (log-sum-exp weights).
template <int D>
__device__ __forceinline__ void fold_state(State<D>& st, float m2, float l2, const f32x4 (&acc2)[D / 16]) {
  const float M = fmaxf(st.m, m2);
  const float a = fast_exp2(st.m - M), b = fast_exp2(m2 - M);
  st.l = a * st.l + b * l2;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.acc[n] = a * st.acc[n] + b * acc2[n];
  st.m = M;
}

// One LDS state slot per wavefront, in the lane layout of State (column c,
// d = TILES * (4g + r) + n).
template <int NW, int D>
struct WaveSlots {
  float acc[NW][16][D + 4];
  float m[NW][16];
  float l[NW][16];
};

// Shared-prefix pairs. The prefix cache hands sequences with a common prompt
// prefix the same blocks for it (infrared/cache/block_manager.py:209-234,
// match_prefix), and a unit's query heads fill only n_rep of the 16 MFMA
// columns. So with pairs on (and 2 n_rep <= 16, one head group per KV head),
// sequence b and b + 1 whose tables begin with the same block ids become one
// unit per KV head: columns 0..n_rep-1 are b's query heads, n_rep..2 n_rep-1
// b + 1's, and the unit's tiles are the S shared tiles (both halves on), then
// b's private tiles (b's half on), then b + 1's (b + 1's half on). The shared
// prefix is read once instead of twice, each column still sees exactly its
// own sequence's keys in ascending order, and no extra merge is needed. Runs
// of consecutive sharing sequences pair from the run's start: (r, r+1),
// (r+2, r+3), ...; the second sequence of a pair has no tiles of its own.
// S counts the leading blocks equal in both tables that lie wholly inside
// both contexts (found by comparing every such block, all candidates at once).

// Inclusive max / sum over the block's threads in thread order, through
// per-wavefront totals in `wsum` (NW entries); every thread gets its prefix.
template <int NW, bool MAX>
__device__ __forceinline__ int block_scan_incl(int x, int* wsum) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(x, off);
    if (lane >= off) x = MAX ? max(x, v) : x + v;
  }
  __syncthreads();
  if (lane == 63) wsum[w] = x;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NW; ++i)
    if (i < w) x = MAX ? max(x, wsum[i]) : x + wsum[i];
  __syncthreads();
  return x;
}

// The pair scan (before the plan, when pairs are on): workgroup b compares
// the tables of sequences b and b + 1 over the blocks wholly inside both
// contexts and writes share[b], the 16-key tiles of their common leading
// blocks (0 unless both begin with the same valid block id).
constexpr int kPairThreads = 256;

__global__ __launch_bounds__(kPairThreads) void paged_decode_pair_kernel(PlanArgs p) {
  __shared__ int s_mis;
  const int b = blockIdx.x, tid = threadIdx.x;
  int32_t* share = (int32_t*)(p.plan + p.ly.share);
  const int cap = p.max_blocks * p.bs;
  auto ctx_of = [&](int q) { return max(0, min(p.ctx[q], cap)); };
  int nbm = 0;
  if (b + 1 < p.num_seqs) nbm = min(ctx_of(b), ctx_of(b + 1)) / p.bs;
  const int32_t* r0 = p.bt + (int64_t)b * p.bt_stride;
  const int32_t* r1 = r0 + p.bt_stride;
  const bool cand = nbm >= 1 && r0[0] >= 0 && (int64_t)r0[0] < p.num_blocks && r0[0] == r1[0];
  if (!cand) {  // uniform over the workgroup
    if (tid == 0) share[b] = 0;
    return;
  }
  if (tid == 0) s_mis = nbm;
  __syncthreads();
  for (int j = 1 + tid; j < nbm; j += kPairThreads)
    if (r0[j] != r1[j]) atomicMin(&s_mis, j);
  __syncthreads();
  if (tid == 0) share[b] = s_mis * p.bs / 16;
}

// Builds the plan: every workgroup scans the context lengths (block-wide
// prefix sum, one int32 per sequence), finds its slice, and writes its
// wavefronts' headers and tile facts; workgroup 0 also writes the header, the
// prefix sums, the list of sequences with no usable key and the pairs.
template <int NW>
__global__ __launch_bounds__(NW * 64) void paged_decode_plan_kernel(PlanArgs p) {
  constexpr int NT = NW * 64;
  __shared__ int s_pre[kPlanMaxSeqs + 1];
  __shared__ int s_ctx[kPlanMaxSeqs];
  __shared__ int s_share[kPlanMaxSeqs];  // shared tiles of pair (b, b + 1) / of a pair's first sequence
  __shared__ int s_lead[kPlanMaxSeqs];   // 1: first of a pair, -1: second, 0: alone
  __shared__ int s_wsum[NW];
  __shared__ int s_seq[2];
  __shared__ int s_nempty, s_npairs;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int grp = blockIdx.x;
  const int B = p.num_seqs, n_ups = p.n_ups;
  int32_t* hdr = (int32_t*)(p.plan + p.ly.hdr);
  if (tid == 0) {
    s_nempty = 0;
    s_npairs = 0;
  }

  const int per = (B + NT - 1) / NT;
  const int b_lo = min(B, tid * per);
  const int b_hi = min(B, b_lo + per);
  const int cap = p.max_blocks * p.bs;
  for (int b = b_lo; b < b_hi; ++b) {
    int ctx = p.ctx[b];
    if (ctx < 0 || ctx > cap) {
      if (grp == 0) flag_error(p.err, IR_ERR_CONTEXT_RANGE);
      ctx = ctx < 0 ? 0 : cap;
    }
    s_ctx[b] = ctx;
    s_share[b] = 0;
    s_lead[b] = 0;
  }
  __syncthreads();
  auto tiles0 = [&](int b) { return p.num_blocks > 0 ? (s_ctx[b] + 15) >> 4 : 0; };
  if (p.pairs) {
    // s_share[b]: shared tiles of (b, b + 1), from the pair scan that ran
    // before this launch; pairs from the start of each run of consecutive
    // sharing sequences (the run start before this thread's sequences is an
    // exclusive prefix max)
    const int32_t* sh = (const int32_t*)(p.plan + p.ly.share);
    for (int b = b_lo; b < b_hi; ++b) s_share[b] = sh[b];
    __syncthreads();
    int rmax = -1;
    for (int b = b_lo; b < b_hi; ++b)
      if (b == 0 || s_share[b - 1] == 0) rmax = b;
    const int r_incl = block_scan_incl<NW, true>(rmax, s_wsum);
    int rs = __shfl_up(r_incl, 1);
    if (lane == 0) {
      rs = -1;
      for (int i = 0; i < w; ++i) rs = max(rs, s_wsum[i]);
    }
    for (int b = b_lo; b < b_hi; ++b) {
      if (b == 0 || s_share[b - 1] == 0) rs = b;
      if (s_share[b] > 0 && ((b - rs) & 1) == 0) s_lead[b] = 1;
    }
    __syncthreads();
    for (int b = b_lo; b < b_hi; ++b)
      if (b > 0 && s_lead[b - 1] == 1) s_lead[b] = -1;
    __syncthreads();
    for (int b = b_lo; b < b_hi; ++b)
      if (s_lead[b] != 1) s_share[b] = 0;
    __syncthreads();
  }
  // tiles of each sequence's units: a pair's first sequence carries both
  // sequences' tiles less the shared ones, its second none
  auto tiles = [&](int b) {
    const int l = s_lead[b];
    return l < 0 ? 0 : l > 0 ? tiles0(b) + tiles0(b + 1) - s_share[b] : tiles0(b);
  };
  int mine = 0;
  for (int b = b_lo; b < b_hi; ++b) mine += tiles(b);
  int incl = mine;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int v = __shfl_up(incl, off);
    if (lane >= off) incl += v;
  }
  if (lane == 63) s_wsum[w] = incl;
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int v = s_wsum[i];
    incl += i < w ? v : 0;
    total += v;
  }
  const int T = total * n_ups;
  const int R = max((T + (int)gridDim.x - 1) / (int)gridDim.x, p.min_tiles);
  const int lo = (int)min((int64_t)grp * R, (int64_t)T);
  const int hi = min(T, lo + R);
  {
    int pre = incl - mine;
    for (int b = b_lo; b < b_hi; ++b) {
      s_pre[b] = pre;
      const int nxt = pre + tiles(b);
      if (lo < hi) {
        if (pre * n_ups <= lo && lo < nxt * n_ups) s_seq[0] = b;
        if (pre * n_ups <= hi - 1 && hi - 1 < nxt * n_ups) s_seq[1] = b;
      }
      if (grp == 0) {
        ((int32_t*)(p.plan + p.ly.seq_pre))[b] = pre;
        ((int32_t*)(p.plan + p.ly.pair))[b] = s_lead[b] > 0 ? s_share[b] : s_lead[b];
        if (nxt == pre && s_lead[b] == 0) ((int32_t*)(p.plan + p.ly.empty))[atomicAdd(&s_nempty, 1)] = b;
        if (s_lead[b] > 0) atomicAdd(&s_npairs, 1);
      }
      pre = nxt;
    }
    if (tid == 0) s_pre[B] = total;
  }
  __syncthreads();
  if (grp == 0 && tid == 0) {
    ((int32_t*)(p.plan + p.ly.seq_pre))[B] = total;
    hdr[0] = T;
    hdr[1] = R;
    hdr[2] = s_nempty;
    hdr[3] = s_npairs;
  }
  int32_t* wh = (int32_t*)(p.plan + p.ly.whdr) + ((int64_t)grp * NW + w) * 8;
  if (lo >= hi) {
    if (lane < 8) wh[lane] = lane == 1 ? 0 : (lane == 2 || lane == 3) ? -1 : lo;
    return;
  }
  const int seq0 = s_seq[0], seqN = s_seq[1];
  auto seq_of = [&](int t) {
    int b0 = seq0, b1 = seqN + 1;
    while (b1 - b0 > 1) {
      const int mid = (b0 + b1) >> 1;
      if (s_pre[mid] * n_ups <= t) b0 = mid;
      else b1 = mid;
    }
    return b0;
  };
  auto unit_of = [&](int t, int b) {
    return b * n_ups + fdiv(t - s_pre[b] * n_ups, s_pre[b + 1] - s_pre[b]);
  };
  const int n = hi - lo;
  const int wlo = lo + (int)((int64_t)n * w / NW);
  const int whi = lo + (int)((int64_t)n * (w + 1) / NW);
  const int cnt_w = whi - wlo;
  const int fl = cnt_w > 0 ? unit_of(wlo, seq_of(wlo)) : -1;
  const int ll = cnt_w > 0 ? unit_of(whi - 1, seq_of(whi - 1)) : -1;
  const int u_first = unit_of(lo, seq0);
  const int u_last = unit_of(hi - 1, seqN);
  if (lane < 8) {
    const int v[8] = {wlo, cnt_w, fl, ll, lo, hi, u_first, u_last};
    int x = v[0];
#pragma unroll
    for (int k = 1; k < 8; ++k) x = lane == k ? v[k] : x;
    wh[lane] = x;
  }
  bool bad = false;
  u32x2* facts = (u32x2*)(p.plan + p.ly.facts);
  u32x2* first = (u32x2*)(p.plan + p.ly.first) + ((int64_t)grp * NW + w) * kPlanRun;
  for (int r0 = 0; r0 < cnt_w; r0 += kPlanRun) {
    const int i = r0 + lane;
    if (i < cnt_w) {
      const int t = wlo + i;
      const int b = seq_of(t);
      const int ts = s_pre[b + 1] - s_pre[b];
      const int rel = t - s_pre[b] * n_ups;
      const int j = fdiv(rel, ts);
      const int ti = rel - j * ts;  // tile of the unit
      const int kvh = p.n_hg == 1 ? j : fdiv(j, p.n_hg);
      // which sequence's keys the tile holds, and which column halves see it
      int sq = b, tok0 = ti * 16;
      uint32_t cm = 1u;
      if (s_lead[b] > 0) {
        const int S = s_share[b], ta = tiles0(b);
        if (ti < S) cm = 3u;
        else if (ti >= ta) {
          sq = b + 1;
          tok0 = (ti - ta + S) * 16;
          cm = 2u;
        }
      }
      const int32_t bid = p.bt[(int64_t)sq * p.bt_stride + tok0 / p.bs];
      const bool ok = bid >= 0 && (int64_t)bid < p.num_blocks;
      bad |= !ok;
      const int64_t slot = ok ? (int64_t)bid * p.bs + (tok0 % p.bs) : 0;
      const uint32_t off16 = (uint32_t)(slot * p.c_slot16 + kvh * p.c_head16);
      const int valid = ok ? min(16, s_ctx[sq] - tok0) : 0;
      const u32x2 f = {off16, ((uint32_t)(b * n_ups + j) << 7) | (cm << 5) | (uint32_t)valid};
      facts[t] = f;
      if (r0 == 0) first[lane] = f;
    }
  }
  if (bad) flag_error(p.err, IR_ERR_BLOCK_RANGE);
}

// Lane-layout state slot I/O (column c, d = TILES * (4g + r) + n): TILES
// consecutive floats per (lane, r), moved as 16-byte LDS accesses.
template <int D>
__device__ __forceinline__ void slot_write(float* row, float* m, float* l, const State<D>& st, int g, int c) {
  constexpr int TILES = D / 16;
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int n = 0; n < TILES; n += 4)
      *(f32x4*)(row + TILES * (4 * g + r) + n) =
          f32x4{st.acc[n][r], st.acc[n + 1][r], st.acc[n + 2][r], st.acc[n + 3][r]};
  if (g == 0) {
    m[c] = st.m;
    l[c] = st.l;
  }
}
template <int D>
__device__ __forceinline__ void slot_read(const float* row, int g, f32x4 (&acc)[D / 16]) {
  constexpr int TILES = D / 16;
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int n = 0; n < TILES; n += 4) {
      const f32x4 x = *(const f32x4*)(row + TILES * (4 * g + r) + n);
      acc[n][r] = x[0];
      acc[n + 1][r] = x[1];
      acc[n + 2][r] = x[2];
      acc[n + 3][r] = x[3];
    }
}

// The decode over a plan: no scan, no block-table reads. A wavefront's header
// and its first 64 tile facts sit at fixed addresses, so its first tile loads
// go out one round trip after launch. The addresses those first reads need
// lead the argument list as plain scalars (the plan header sits at the plan's
// start; the other offsets precede the facts, so they fit 32 bits): this file
// is built with kernel-argument preloading, which hands the leading scalar
// arguments over in SGPRs at wave start, so the plan reads do not wait for a
// kernel-argument load.
template <int DT, int D, int NW, int DEPTH, bool PAIRS>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(DT == IR_DTYPE_F32 ? 1 : 2)))
void paged_decode_planned_kernel(const uint8_t* plan, uint32_t o_seq_pre, uint32_t o_pair, uint32_t o_whdr,
                                 uint32_t o_first, int B, DecodeArgs a, PlanLayout ly) {
  typedef TileShape<DT, D> Sh;
  constexpr int EB = Sh::EB;
  constexpr int NT = NW * 64;
  constexpr int TILES = D / 16;
  __shared__ WaveSlots<NW, D> sl;
  __shared__ WaveSlots<2, D> stg;  // this slice's cross-workgroup partials: [0] first unit, [1] last unit
  __shared__ __attribute__((aligned(16))) uint8_t kstage[NW][KStage<DT, D>::BYTES];
  __shared__ int s_pre[kPlanMaxSeqs + 1];
  __shared__ int s_pair[PAIRS ? kPlanMaxSeqs : 1];
  __shared__ int s_fl[NW];
  __shared__ int s_stg[2];
  __shared__ int s_last[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, g = lane >> 4, c = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = blockIdx.x;
  const int n_ups = a.n_ups;

  // ---- 1. everything the wavefront needs, requested at once
  // (a plan with pairs needs the pair kernel: its flag empties this
  // workgroup's slice rather than branching, so no read waits on it)
  const int32_t* hdr = (const int32_t*)plan;
  const int32_t* wh = (const int32_t*)(plan + o_whdr) + ((int64_t)grp * NW + w) * 8;
  const u32x2* facts = (const u32x2*)(plan + ly.facts);
  const int32_t* sp = (const int32_t*)(plan + o_seq_pre);
  const int32_t* pp = (const int32_t*)(plan + o_pair);
  const int pre0 = tid <= B ? sp[tid] : 0;  // every sequence's when B < NT
  const int pair0 = PAIRS && tid < B ? pp[tid] : 0;
  const u32x4 h4 = *(const u32x4*)hdr;
  const int R = (int)h4[1], hdr_pairs = (int)h4[3];
  // the wavefront's header in two 16-byte reads (the plan is 256-byte
  // aligned), so the select below cannot become a skipped load
  const u32x4 wh0 = *(const u32x4*)wh, wh1 = *(const u32x4*)(wh + 4);
  u32x2 f0 = ((const u32x2*)(plan + o_first))[((int64_t)grp * NW + w) * kPlanRun + lane];
  // every read above is used here, so they all go out before the first wait
  // (one round trip) instead of each behind the last one's use
  asm volatile("" ::"s"(R), "s"(hdr_pairs), "s"(wh0[0]), "s"(wh0[1]), "s"(wh0[2]), "s"(wh0[3]), "s"(wh1[0]),
               "s"(wh1[1]), "s"(wh1[2]), "v"(f0[0]), "v"(f0[1]), "v"(pre0), "v"(pair0));
  const bool wrong_plan = !PAIRS && hdr_pairs != 0;
  const int wlo = (int)wh0[0], cnt_w = (int)wh0[1], fl = (int)wh0[2], ll = (int)wh0[3];
  const int lo = (int)wh1[0], u_first = (int)wh1[2];
  const int hi = wrong_plan ? lo : (int)wh1[1];
  if (tid <= B) s_pre[tid] = pre0;
  for (int b = tid + NT; b <= B; b += NT) s_pre[b] = sp[b];
  if constexpr (PAIRS) {
    if (tid < B) s_pair[tid] = pair0;
    for (int b = tid + NT; b < B; b += NT) s_pair[b] = pp[b];
  }
  if (tid < NW) s_fl[tid] = -1;
  if (tid < 2) s_stg[tid] = -1;

  // sequences with no usable key get a zero output row (workgroup 0)
  if (grp == 0 && !wrong_plan) {
    const int n_empty = hdr[2];
    const int32_t* empty = (const int32_t*)(plan + ly.empty);
    constexpr int C8 = D / 8;
    for (int e = 0; e < n_empty; ++e) {
      const int b = empty[e];
      for (int it = tid; it < a.num_q_heads * C8; it += NT) {
        const int h = it / C8;
        const int d0 = (it - h * C8) * 8;
        const float z[4] = {0.f, 0.f, 0.f, 0.f};
        uint8_t* dst = (uint8_t*)a.out + ((int64_t)b * a.o_seq + (int64_t)h * a.o_head + d0) * EB;
        store4<DT>(dst, z, 0.f);
        store4<DT>(dst + 4 * EB, z, 0.f);
      }
    }
  }
  __syncthreads();
  if (wrong_plan && grp == 0 && tid == 0) flag_error(a.err, IR_ERR_PLAN);
  if (lo >= hi) return;  // uniform: past the end of the list (or a plan with pairs)

  struct Lbl {
    int u, b, j, us, ue;
  };
  auto label = [&](int u) {
    Lbl x;
    x.u = u;
    x.b = fdiv(u, n_ups);
    x.j = u - x.b * n_ups;
    const int ts = s_pre[x.b + 1] - s_pre[x.b];
    x.us = s_pre[x.b] * n_ups + x.j * ts;
    x.ue = x.us + ts;
    return x;
  };
  auto paired = [&](int b) { return PAIRS && s_pair[b] > 0; };
  auto q_of = [&](int u, uint32_t (&dst)[Sh::KDW]) {
    const int b = fdiv(u, n_ups);
    const int j = u - b * n_ups;
    const int hg = a.n_hg == 1 ? 0 : j - fdiv(j, a.n_hg) * a.n_hg;
    const int kvh = a.n_hg == 1 ? j : fdiv(j, a.n_hg);
    if (paired(b)) {  // columns 0..n_rep-1: sequence b, n_rep..2 n_rep-1: b + 1
      const int second = c >= a.n_rep;
      load_query<DT, D>(a, b + second, kvh * a.n_rep + c - second * a.n_rep, c < 2 * a.n_rep, g, dst);
      return;
    }
    const int hl = hg * 16 + c;
    load_query<DT, D>(a, b, kvh * a.n_rep + hl, hl < a.n_rep, g, dst);
  };
  uint32_t qr[Sh::KDW], qn[Sh::KDW];
  int q_lbl = -1, qn_lbl = -1;
  if (cnt_w > 0) {
    q_of(fl, qr);
    q_lbl = fl;
    if (fl < ll) {
      q_of(fl + 1, qn);
      qn_lbl = fl + 1;
    }
  }

  // ---- 2. the tile loop
  const uint8_t* kc = (const uint8_t*)a.kc;
  const uint8_t* vc = (const uint8_t*)a.vc;
  const LaneOffsets<DT, D> lo_off = lane_offsets<DT, D>(lane, a.c_slot * EB);
  const int whi = wlo + cnt_w;
  State<D> st;
  state_init(st);
  // pend: a unit finished at the loop's end whose output is written last, so
  // that no barrier of the end phase waits for its stores
  int cur = -1, keep = -1, pend = -1;

  // Columns of unit x that are outputs, and column col's (sequence, head).
  auto n_cols = [&](const Lbl& x) {
    const int hg = a.n_hg == 1 ? 0 : x.j - fdiv(x.j, a.n_hg) * a.n_hg;
    return paired(x.b) ? 2 * a.n_rep : min(16, a.n_rep - hg * 16);
  };
  auto out_of = [&](const Lbl& x, int col, int& sq, int& h) {
    const int hg = a.n_hg == 1 ? 0 : x.j - fdiv(x.j, a.n_hg) * a.n_hg;
    const int kvh = a.n_hg == 1 ? x.j : fdiv(x.j, a.n_hg);
    const int second = paired(x.b) && col >= a.n_rep;
    sq = x.b + second;
    h = kvh * a.n_rep + hg * 16 + col - second * a.n_rep;
  };
  auto write_out = [&](const Lbl& x) {
    if (c < n_cols(x)) {
      int sq, h;
      out_of(x, c, sq, h);
      const float inv = st.l > 0.f ? 1.f / st.l : 0.f;
      uint8_t* row = (uint8_t*)a.out + ((int64_t)sq * a.o_seq + (int64_t)h * a.o_head) * EB;
#pragma unroll
      for (int r = 0; r < 4; ++r) store_acc_run<DT, D>(row + TILES * (4 * g + r) * EB, st, r, inv);
    }
  };
  auto stage_partial = [&](int u, int k) {
    slot_write<D>(stg.acc[k][c], stg.m[k], stg.l[k], st, g, c);
    if (lane == 0) s_stg[k] = u;
  };
  auto wave_finish = [&](int u, bool at_end) {
    st.l = wave_sum_groups(st.l);
    const Lbl x = label(u);
    if (x.us >= wlo && x.ue <= whi) {
      if (at_end) {
        pend = u;
        return;
      }
      write_out(x);
    } else if (max(x.us, lo) < wlo) {
      slot_write<D>(sl.acc[w][c], sl.m[w], sl.l[w], st, g, c);
      if (lane == 0) s_fl[w] = u;
    } else if (x.ue > whi) {
      keep = u;
      return;
    } else {
      stage_partial(u, 0);
    }
    if (!at_end) state_init(st);
  };

  uint32_t info_off = f0[0], info_meta = f0[1];
  for (int r0 = 0; r0 < cnt_w; r0 += kPlanRun) {
    if (r0 > 0) {
      const u32x2 f = r0 + lane < cnt_w ? facts[wlo + r0 + lane] : u32x2{0u, 0u};
      info_off = f[0];
      info_meta = f[1];
    }
    const int cnt = min(kPlanRun, cnt_w - r0);
    const int last = cnt - 1;
    // Issues the loads of tile i of the run (`real`: i is known to be a tile of
    // the run). Past the run's end (the ring's last DEPTH issues, never
    // computed) it issues nothing: the end phase reuses the ring's registers,
    // and a load still in flight into them would hold it up (padding loads
    // cost 0.7 us per call this way).
    auto issue = [&](int i, Tile<DT, D>& tl, int& lb, bool& con, bool real) -> uint32_t {
      const int ii = real || i <= last ? i : last;
      const uint32_t off = (uint32_t)__builtin_amdgcn_readlane((int)info_off, ii);
      const uint32_t meta = (uint32_t)__builtin_amdgcn_readlane((int)info_meta, ii);
      if (real || i <= last) issue_tile<DT, D>(kc, vc, off, lo_off, tl);
      lb = (int)(meta >> 7);
      // this lane's column half sees the tile (column mask bits 5, 6)
      con = !PAIRS || ((meta >> (c >= a.n_rep ? 6 : 5)) & 1u);
      const int valid = (int)(meta & 31u);
      uint32_t m = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) m |= (4 * r + g < valid) ? (1u << r) : 0u;
      return m;
    };
    Tile<DT, D> ring[DEPTH];
    uint32_t mk[DEPTH];
    int lb[DEPTH];
    bool con[DEPTH];
    // Computes ring slot r, switching units (and queries) at a label change.
    auto step = [&](int r) {
      if (lb[r] != cur) {
        if (cur >= 0) wave_finish(cur, false);
        cur = lb[r];
        if (q_lbl != cur) {
          if (qn_lbl == cur) {
#pragma unroll
            for (int k = 0; k < Sh::KDW; ++k) qr[k] = qn[k];
          } else {
            q_of(cur, qr);
          }
          q_lbl = cur;
        }
        if (cur + 1 <= ll && qn_lbl != cur + 1) {
          q_of(cur + 1, qn);
          qn_lbl = cur + 1;
        }
      }
      compute_tile<DT, D>(ring[r], qr, mk[r], a.scale_log2, kstage[w], lane, st, con[r]);
    };
#pragma unroll
    for (int r = 0; r < DEPTH; ++r) mk[r] = issue(r, ring[r], lb[r], con[r], false);
    int i = 0;
    // Steady state: every issue is a real tile and the body has no branch
    // around it (the branch cost 0.9 us per call on 64 sequences, even with
    // one tile in flight); then the last DEPTH..2 DEPTH - 1 tiles.
    for (; i + 2 * DEPTH <= cnt; i += DEPTH) {
#pragma unroll
      for (int r = 0; r < DEPTH; ++r) {
        step(r);
        mk[r] = issue(i + r + DEPTH, ring[r], lb[r], con[r], true);
      }
    }
    for (; i < cnt; i += DEPTH) {
#pragma unroll
      for (int r = 0; r < DEPTH; ++r) {
        if (i + r < cnt) step(r);
        mk[r] = issue(i + r + DEPTH, ring[r], lb[r], con[r], false);
      }
    }
  }
  if (cur >= 0) wave_finish(cur, true);
  __syncthreads();

  // ---- 3. owners of units that run on into later quarters fold their slots in
  if (keep >= 0) {
    const Lbl x = label(keep);
#pragma unroll
    for (int w2 = 1; w2 < NW; ++w2) {
      if (w2 <= w || s_fl[w2] != keep) continue;
      f32x4 acc2[TILES];
      slot_read<D>(sl.acc[w2][c], g, acc2);
      fold_state(st, sl.m[w2][c], sl.l[w2][c], acc2);
    }
    if (x.us >= lo && x.ue <= hi) pend = keep;
    else stage_partial(keep, keep == u_first ? 0 : 1);
  }
  __syncthreads();

  // ---- 4. cross-workgroup partials (16-byte device-scope stores), arrivals and
  // the last arrival's merge
  const int U0 = s_stg[0], U1 = s_stg[1];
  if (U0 < 0 && U1 < 0) {
    if (pend >= 0) write_out(label(pend));
    return;
  }
  const __amdgpu_buffer_rsrc_t r_o = dev_rsrc(a.ws_o), r_ml = dev_rsrc(a.ws_ml);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int u = k == 0 ? U0 : U1;
    if (u < 0) continue;
    const Lbl x = label(u);
    const int nh = n_cols(x);
    for (int it = tid; it < nh * (D / 4); it += NT) {
      const int hc = it / (D / 4);
      const int d0 = (it - hc * (D / 4)) * 4;
      const int rr = (grp + u) * 16 + hc;  // < 2^22 rows (plannable), so byte offsets fit int
      store_dev4(r_o, (rr * D + d0) * 4, *(const f32x4*)&stg.acc[k][hc][d0]);
      if (d0 == 0) store_dev2(r_ml, rr * 8, f32x2{stg.m[k][hc], stg.l[k][hc]});
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid < 2) {
    const int u = tid == 0 ? U0 : U1;
    int lst = 0;
    if (u >= 0) {
      const Lbl x = label(u);
      const int np = (x.ue - 1) / R - x.us / R + 1;
      lst = __hip_atomic_fetch_add(a.counters + u, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == np - 1;
    }
    s_last[tid] = lst;
  }
  __syncthreads();
  // Both units' merges in one pass, so their loads are in flight together (one
  // after the other, the slices that end last -- which merge both -- took 2.15
  // instead of 1.17 us): items of 8 columns of one head, U0's first.
  constexpr int C8 = D / 8;
  int n0 = 0, n1 = 0, f0r = 0, f1r = 0, np0 = 0, np1 = 0;
  Lbl x0 = {}, x1 = {};
  if (U0 >= 0 && s_last[0]) {
    x0 = label(U0);
    n0 = n_cols(x0) * C8;
    f0r = (x0.us / R + U0) * 16;
    np0 = (x0.ue - 1) / R - x0.us / R + 1;
  }
  if (U1 >= 0 && s_last[1]) {
    x1 = label(U1);
    n1 = n_cols(x1) * C8;
    f1r = (x1.us / R + U1) * 16;
    np1 = (x1.ue - 1) / R - x1.us / R + 1;
  }
  for (int it = tid; it < n0 + n1; it += NT) {
    const bool k1 = it >= n0;
    const int j = k1 ? it - n0 : it;
    const int hc = j / C8;
    const int d0 = (j - hc * C8) * 8;
    float o[8], Ls;
    lse_merge_dev<D, 8, 8>(r_o, r_ml, (k1 ? f1r : f0r) + hc, 16, k1 ? np1 : np0, d0, o, Ls);
    const float inv = Ls > 0.f ? 1.f / Ls : 0.f;
    int sq, h;
    out_of(k1 ? x1 : x0, hc, sq, h);
    uint8_t* dst = (uint8_t*)a.out + ((int64_t)sq * a.o_seq + (int64_t)h * a.o_head + d0) * EB;
    const float lo4[4] = {o[0], o[1], o[2], o[3]}, hi4[4] = {o[4], o[5], o[6], o[7]};
    store4<DT>(dst, lo4, inv);
    store4<DT>(dst + 4 * EB, hi4, inv);
  }
  if (tid == 0 && n0) __hip_atomic_store(a.counters + U0, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (tid == 1 && n1) __hip_atomic_store(a.counters + U1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (pend >= 0) write_out(label(pend));
}

template <int DT, int D>
void launch_planned_dt_d(const DecodeArgs& a, const uint8_t* plan, const PlanLayout& ly, int grid, bool pairs,
                         hipStream_t s) {
  // One tile in flight per wavefront: at ~6.6 TB/s four wavefronts per CU keep
  // HBM saturated with one tile each, and the shorter queues halve the latency
  // of the end phase's round trips (two tiles in flight: 0.4 us slower per call
  // on 64 sequences x 28/4 heads, contexts 512..4096).
  // plan_layout: the header is at 0, and sequence, pair, wavefront-header and
  // first-fact regions are sized by the sequence count and grid only
  const uint32_t o_sp = (uint32_t)ly.seq_pre, o_pr = (uint32_t)ly.pair, o_wh = (uint32_t)ly.whdr,
                 o_fi = (uint32_t)ly.first;
  if (pairs)
    hipLaunchKernelGGL((paged_decode_planned_kernel<DT, D, kPlanWaves, 1, true>), dim3(grid), dim3(kPlanWaves * 64), 0,
                       s, plan, o_sp, o_pr, o_wh, o_fi, a.num_seqs, a, ly);
  else
    hipLaunchKernelGGL((paged_decode_planned_kernel<DT, D, kPlanWaves, 1, false>), dim3(grid), dim3(kPlanWaves * 64),
                       0, s, plan, o_sp, o_pr, o_wh, o_fi, a.num_seqs, a, ly);
}

// Pairs fit one unit's 16 MFMA columns when a KV head has at most 8 query
// heads (one head group).
bool pairs_fit(int num_q_heads, int num_kv_heads) { return 2 * (num_q_heads / num_kv_heads) <= 16; }

int n_hg_of(int num_q_heads, int num_kv_heads) { return (num_q_heads / num_kv_heads + 15) / 16; }

// Upper bound on the tile list for a table capacity.
int64_t t_cap_of(int num_seqs, int n_ups, int max_blocks, int bs) {
  return (int64_t)num_seqs * (((int64_t)max_blocks * bs + 15) / 16) * n_ups;
}

// Shapes the plan takes: 16-token tiles inside one block, the prefix sums in
// LDS, tile-list indices (and (unit << 7)) in int32, and fewer than 2^17 units,
// so the partial rows ((#CUs + units) x 16 x head_dim fp32) sit below the 2 GiB
// the device-scope buffer accesses address.
bool plannable(int num_seqs, int num_q_heads, int num_kv_heads, int max_blocks, int bs) {
  if (num_seqs <= 0 || num_seqs > kPlanMaxSeqs || num_kv_heads <= 0 || num_q_heads <= 0 ||
      num_q_heads % num_kv_heads || bs <= 0 || bs % 16 != 0 || max_blocks < 0)
    return false;
  const int n_ups = num_kv_heads * n_hg_of(num_q_heads, num_kv_heads);
  return t_cap_of(num_seqs, n_ups, max_blocks, bs) < ((int64_t)1 << 30) &&
         (int64_t)num_seqs * n_ups < ((int64_t)1 << 17);
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int64_t ir_paged_decode_plan_bytes(int num_seqs, int num_q_heads, int num_kv_heads, int max_blocks_per_seq,
                                              int block_size) {
  if (!plannable(num_seqs, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size)) return 0;
  const int n_ups = num_kv_heads * n_hg_of(num_q_heads, num_kv_heads);
  return plan_layout(num_seqs, device_cus(), t_cap_of(num_seqs, n_ups, max_blocks_per_seq, block_size)).total;
}

extern "C" int64_t ir_paged_decode_planned_workspace_bytes(int num_seqs, int num_q_heads, int num_kv_heads,
                                                           int head_dim) {
  if (num_seqs <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads || head_dim <= 0) return 0;
  const int64_t units = (int64_t)num_seqs * num_kv_heads * n_hg_of(num_q_heads, num_kv_heads);
  return planned_ws(units, device_cus(), head_dim).total();
}

extern "C" int ir_paged_decode_plan(const int32_t* block_tables, int64_t bt_stride, int max_blocks_per_seq,
                                    const int32_t* context_lens, int num_seqs, int num_q_heads, int num_kv_heads,
                                    int block_size, int64_t num_blocks, int64_t cache_slot_stride,
                                    int64_t cache_head_stride, int dtype, int flags, void* plan, int64_t plan_bytes,
                                    int32_t* err_flags, ir_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  IR_REQUIRE(eb > 0, "ir_paged_decode_plan: unknown dtype %d", dtype);
  IR_REQUIRE((flags & ~IR_PLAN_SHARE_GROUPS) == 0, "ir_paged_decode_plan: unknown flags 0x%x", flags);
  IR_REQUIRE(plannable(num_seqs, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size),
             "ir_paged_decode_plan: shape not plannable (1 <= batch <= %d, block size a multiple of 16)",
             kPlanMaxSeqs);
  IR_REQUIRE(num_blocks >= 0 && bt_stride >= max_blocks_per_seq, "ir_paged_decode_plan: bad sizes");
  const int64_t need = ir_paged_decode_plan_bytes(num_seqs, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size);
  IR_REQUIRE(plan && plan_bytes >= need && ((uintptr_t)plan & 255u) == 0,
             "ir_paged_decode_plan: plan of %lld bytes (256-byte aligned) required, got %lld", (long long)need,
             (long long)plan_bytes);
  IR_REQUIRE(block_tables && context_lens, "ir_paged_decode_plan: null pointer");
  IR_REQUIRE((cache_slot_stride * eb) % 16 == 0 && (cache_head_stride * eb) % 16 == 0,
             "ir_paged_decode_plan: cache strides must be multiples of 16 bytes");
  const int64_t slot16 = cache_slot_stride * eb / 16, head16 = cache_head_stride * eb / 16;
  IR_REQUIRE(num_blocks * block_size * slot16 + (int64_t)num_kv_heads * head16 < ((int64_t)1 << 32),
             "ir_paged_decode_plan: a pool of %lld blocks exceeds 32-bit tile offsets (64 GiB per layer)",
             (long long)num_blocks);
  PlanArgs p;
  p.bt = block_tables;
  p.bt_stride = bt_stride;
  p.max_blocks = max_blocks_per_seq;
  p.ctx = context_lens;
  p.num_seqs = num_seqs;
  p.n_hg = n_hg_of(num_q_heads, num_kv_heads);
  p.n_ups = num_kv_heads * p.n_hg;
  p.bs = block_size;
  p.num_blocks = num_blocks;
  p.c_slot16 = slot16;
  p.c_head16 = head16;
  p.min_tiles = kPlanMinTiles;
  p.pairs = (flags & IR_PLAN_SHARE_GROUPS) && pairs_fit(num_q_heads, num_kv_heads);
  p.plan = (uint8_t*)plan;
  const int grid = device_cus();
  p.ly = plan_layout(num_seqs, grid, t_cap_of(num_seqs, p.n_ups, max_blocks_per_seq, block_size));
  p.err = err_flags;
  if (p.pairs)
    hipLaunchKernelGGL(paged_decode_pair_kernel, dim3(num_seqs), dim3(kPairThreads), 0, (hipStream_t)stream, p);
  hipLaunchKernelGGL((paged_decode_plan_kernel<kPlanWaves>), dim3(grid), dim3(kPlanWaves * 64), 0,
                     (hipStream_t)stream, p);
  return check_launch("ir_paged_decode_plan");
}

extern "C" int ir_paged_decode_planned(const void* q, int64_t q_seq_stride, int64_t q_head_stride, const void* k_cache,
                                       const void* v_cache, int64_t cache_slot_stride, void* out,
                                       int64_t out_seq_stride, int64_t out_head_stride, int num_seqs,
                                       int num_q_heads, int num_kv_heads, int head_dim, int max_blocks_per_seq,
                                       int block_size, float scale, int dtype, int flags, const void* plan,
                                       int32_t* counters, int64_t num_counters, void* workspace,
                                       int64_t workspace_bytes, int32_t* err_flags, ir_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  IR_REQUIRE(eb > 0, "ir_paged_decode_planned: unknown dtype %d", dtype);
  IR_REQUIRE((flags & ~IR_PLAN_SHARE_GROUPS) == 0, "ir_paged_decode_planned: unknown flags 0x%x", flags);
  if (head_dim != 64 && head_dim != 128)
    return fail(IR_EUNSUPPORTED, "ir_paged_decode_planned: head_dim %d not supported (64, 128)", head_dim);
  IR_REQUIRE(plannable(num_seqs, num_q_heads, num_kv_heads, max_blocks_per_seq, block_size),
             "ir_paged_decode_planned: shape not plannable");
  IR_REQUIRE(plan && ((uintptr_t)plan & 255u) == 0, "ir_paged_decode_planned: plan missing or not 256-byte aligned");
  IR_REQUIRE(q && k_cache && v_cache && out, "ir_paged_decode_planned: null pointer");
  IR_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
             "ir_paged_decode_planned: q, caches and out must be 16-byte aligned");
  IR_REQUIRE((q_seq_stride * eb) % 16 == 0 && (q_head_stride * eb) % 16 == 0 && (cache_slot_stride * eb) % 16 == 0 &&
                 (out_seq_stride * eb) % 16 == 0 && (out_head_stride * eb) % 16 == 0,
             "ir_paged_decode_planned: strides must be multiples of 16 bytes");
  const int grid = device_cus();
  const int n_hg = n_hg_of(num_q_heads, num_kv_heads);
  const PlannedWs ws = planned_ws((int64_t)num_seqs * num_kv_heads * n_hg, grid, head_dim);
  if (!workspace || workspace_bytes < ws.total() || ((uintptr_t)workspace & 255u))
    return fail(IR_EWORKSPACE, "ir_paged_decode_planned: workspace of %lld bytes (256-byte aligned) required, got %lld",
                (long long)ws.total(), (long long)workspace_bytes);
  const int64_t units = (int64_t)num_seqs * num_kv_heads * n_hg;
  if (!counters || num_counters < units)
    return fail(IR_EWORKSPACE, "ir_paged_decode_planned: %lld arrival counters required, got %lld",
                (long long)units, (long long)num_counters);
  DecodeArgs a;
  memset(&a, 0, sizeof(a));
  a.q = q;
  a.q_seq = q_seq_stride;
  a.q_head = q_head_stride;
  a.kc = k_cache;
  a.vc = v_cache;
  a.c_slot = cache_slot_stride;
  a.out = out;
  a.o_seq = out_seq_stride;
  a.o_head = out_head_stride;
  a.num_seqs = num_seqs;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.n_rep = num_q_heads / num_kv_heads;
  a.n_hg = n_hg;
  a.n_ups = num_kv_heads * n_hg;
  a.scale_log2 = scale * kLog2e;
  a.err = err_flags;
  a.counters = counters;
  a.ws_o = (float*)workspace;
  a.ws_ml = (float*)((uint8_t*)workspace + ws.acc_bytes);
  const PlanLayout ly =
      plan_layout(num_seqs, grid, t_cap_of(num_seqs, a.n_ups, max_blocks_per_seq, block_size));
  const uint8_t* pl = (const uint8_t*)plan;
  hipStream_t s = (hipStream_t)stream;
  const bool pairs = (flags & IR_PLAN_SHARE_GROUPS) && pairs_fit(num_q_heads, num_kv_heads);
  switch (dtype) {
    case IR_DTYPE_BF16:
      head_dim == 128 ? launch_planned_dt_d<IR_DTYPE_BF16, 128>(a, pl, ly, grid, pairs, s)
                      : launch_planned_dt_d<IR_DTYPE_BF16, 64>(a, pl, ly, grid, pairs, s);
      break;
    case IR_DTYPE_F16:
      head_dim == 128 ? launch_planned_dt_d<IR_DTYPE_F16, 128>(a, pl, ly, grid, pairs, s)
                      : launch_planned_dt_d<IR_DTYPE_F16, 64>(a, pl, ly, grid, pairs, s);
      break;
    default:
      head_dim == 128 ? launch_planned_dt_d<IR_DTYPE_F32, 128>(a, pl, ly, grid, pairs, s)
                      : launch_planned_dt_d<IR_DTYPE_F32, 64>(a, pl, ly, grid, pairs, s);
  }
  return check_launch("ir_paged_decode_planned");
}
