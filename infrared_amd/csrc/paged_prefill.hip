// Chunked-prefill / prefix-hit / packed varlen paged attention for gfx950
// (16-bit dtypes, bf16/f16 MFMA).
//
// Query token i of sequence b (packed rows cu_seqlens_q[b] + i) sits at
// absolute position q_start[b] + i and attends keys t in [0, q_start[b] + i]
// of its own sequence, read through block_tables[b]. That is the additive
// mask of infrared/model/inputs.py:33-54 (causal, key column <= query column,
// no left padding) used by the prefix-hit prefill of
// infrared/engine/paged_engine.py:194-207, and, per sequence, the varlen mask
// of infrared/model/inputs.py:57-85 used by the packed mixed step of
// infrared/engine/paged_engine.py:461-516 (a decode row is a sequence with one
// query token at position context - 1).
//
// Work decomposition: an item is a (sequence, query block); each runs as one
// workgroup of NW wavefronts per KV head. A query block is TQ = 32 NW / n_rep
// tokens, so the block's (token, query head) pairs of the GQA group -- column
// j = token-in-block * n_rep + head -- fill 32 NW columns almost exactly (4
// wavefronts, 7 heads: 18 tokens, 126 columns); wavefront w owns columns
// 32w .. 32w+31 (two 16-column tiles). Every column of a workgroup reads the
// same KV head, so each K/V element staged in LDS feeds 32 columns per
// wavefront read. The workgroup walks the keys in 64-key tiles staged in an
// LDS ring, one barrier per tile.
//
// Shapes (host choice): 4-wavefront workgroups on a 2-deep ring, one tile at
// a time (~78 KB of LDS, <= 256 registers): two share a CU, and their waves,
// bound by no common barrier, fill each other's MFMA and VALU gaps -- the
// default for batches that fill the CUs twice over. Smaller batches take
// 4-wavefront workgroups on a 3-deep ring whose next tile's scores run beside
// the current tile's exponentials (one per CU, up to 512 registers: the
// shortest critical path when the CUs are not full). 8-wavefront workgroups
// (256 columns, 2-deep ring) serve GQA groups wider than 128 query heads and
// IR_PREFILL_WAVES=8; on 8 x 512-token chunks they measured 197 us against
// 181 us for two 4-wavefront workgroups per CU, although each staged tile
// feeds twice the columns.
//
// Plan (ir_paged_prefill_plan, built on the device once per step, shared by
// every layer): one entry per workgroup, (item, KV head, piece). The pieces
// run heaviest first -- the dispatcher places workgroups in index order, so
// that is the longest-processing-time rule -- with the key range of any item
// heavier than the mean load of a workgroup slot cut into pieces, each its own
// workgroup. A piece attends its share of the item's key tiles and writes fp32
// partial rows (max, sum, unnormalised output) into the plan; the last piece of
// the item to arrive (an arrival counter in the plan) merges them with
// log-sum-exp weights in part order and writes the output. The plan also
// places the work of each (shared-prefix group, KV head) on one XCD where the
// balance allows, so its K/V tiles -- a shared prefix included -- are fetched
// into one L2 (see the plan section). Without a plan, a sequence's last query
// blocks go first and nothing is cut.
//   K and V tiles: row-major [64 keys][D] (+32 bytes a row against bank
//   conflicts), loaded and stored alike (a thread's K and V pieces share the
//   key's slot); the PV product reads V^T with gfx950's transpose read.
// Per tile a wavefront computes S^T = K . Q^T with 16x16x32 MFMA (rows = keys,
// columns = its (token, head) pairs; Q^T stays in registers for the whole
// walk), the online softmax in base 2 down each column (a lane owns one
// column per column tile, so the running max/sum and the rescale are
// lane-local), and O^T += V^T . P^T where P^T is exactly the lane's own
// probabilities of the S^T tiles. Only tiles that cross the causal diagonal
// or the last key are masked.
//
// Parity: the one-shot softmax of infrared/model/layers.py:102-118 over the
// gathered history (infrared/model/triton_attention.py:110-129), streaming as
// in infrared/model/triton_attention.py:135-177; probabilities are rounded to
// the input dtype before the PV product, as softmax(...).to(q.dtype) does.
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include <type_traits>

#include "attn_tile.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kBtCache = 1024;  // block ids staged in LDS per workgroup
#ifndef IR_PREFILL_AHEAD
#define IR_PREFILL_AHEAD 1
#endif
// MFMA steps between an LDS operand read and its use (2 measured the same as
// 1 on the 8 x 512-token workload, with more register pressure)
constexpr int kOperandAhead = IR_PREFILL_AHEAD;

struct PrefillArgs {
  const void* q;
  int64_t q_tok, q_head;  // elements
  const void* kc;
  const void* vc;
  int64_t c_slot, c_head;  // elements
  int64_t num_blocks;
  int bs, bs_shift;  // bs_shift = log2(bs) for a power-of-two block size, else -1
  int c_slot32;      // c_slot when the fast addressing path applies
  const int32_t* bt;
  int64_t bt_stride;
  int max_blocks;
  const int32_t* cu_q;     // [num_seqs + 1]
  const int32_t* q_start;  // [num_seqs]
  int num_seqs, total_q, n_qblocks;
  void* out;
  int64_t o_tok, o_head;  // elements
  int num_q_heads, num_kv_heads, n_rep, tq;  // tq: query tokens per workgroup
  int nw;                                    // wavefronts per workgroup (4 or 8)
  float scale_log2;
  int32_t* err;
  // plan (or nulls): items[workgroup] = (item * H_kv + KV head, piece), item =
  // seq * n_qblocks + block (-1: no work), piece = nparts | part << 8 | first
  // piece index << 16
  const int2* items;
  int32_t* counters;  // one per (cut item, KV head), zero at rest
  float* ws_o;        // partial rows [piece][kv head][column][D]
  float* ws_ml;       // (max, sum) of each partial row
  int64_t n_items_grid;  // workgroups of a planned call (plan entries)
  // Fused K/V write (k_new null: none). Workgroups n_work, n_work + 1, ... of
  // the grid copy rows [0, n_write) of k_new / v_new ([rows, H_kv, D], strides
  // in elements) to the pool at write_slots[row]; the attending workgroups read
  // a sequence's own new keys (positions >= q_start[b]) from row src_row0 +
  // cu_q[b] + (position - q_start[b]) of k_new / v_new instead of the pool.
  const void* k_new;
  const void* v_new;
  int64_t kn_tok, kn_head, vn_tok, vn_head;
  const int64_t* write_slots;
  int64_t n_write, src_row0;
  int64_t n_work;  // attending workgroups (the grid less the writers)
};

// 16-byte pieces a writer lane moves, all loads in flight before any store.
constexpr int kWritePieces = 4;

// A writer workgroup of a fused call: its share of the rows x KV heads x
// 16-byte pieces, copied from k_new / v_new to the pool (kv_scatter's rules:
// a negative slot is skipped, a slot past the pool is flagged and skipped).
template <int D, int NT>
__device__ __forceinline__ void prefill_write_rows(const PrefillArgs& a, int64_t wg) {
  constexpr int P = D / 8;  // 16-byte pieces of one (row, head) of 16-bit elements
  const int64_t per_row = (int64_t)a.num_kv_heads * P;
  const int64_t total = a.n_write * per_row;
  const int64_t num_slots = a.num_blocks * a.bs;
  const int64_t first = wg * (NT * kWritePieces) + threadIdx.x;
  int64_t slot[kWritePieces], coff[kWritePieces];
  u32x4 kx[kWritePieces], vx[kWritePieces];
#pragma unroll
  for (int u = 0; u < kWritePieces; ++u) {
    const int64_t i = first + (int64_t)u * NT;
    const bool in = i < total;
    const int64_t ii = in ? i : 0;  // row 0 exists (n_write >= 1): loaded, never stored
    const int64_t row = ii / per_row;
    const int rem = (int)(ii - row * per_row);
    const int h = rem / P, part = rem - h * P;
    slot[u] = in ? a.write_slots[row] : -1;
    kx[u] = *(const u32x4*)((const uint16_t*)a.k_new + row * a.kn_tok + h * a.kn_head + part * 8);
    vx[u] = *(const u32x4*)((const uint16_t*)a.v_new + row * a.vn_tok + h * a.vn_head + part * 8);
    coff[u] = h * a.c_head + part * 8;
  }
#pragma unroll
  for (int u = 0; u < kWritePieces; ++u) {
    if (slot[u] < 0) continue;  // padding sentinel
    if (slot[u] >= num_slots) {
      flag_error(a.err, IR_ERR_SLOT_RANGE);
      continue;
    }
    *(u32x4*)((uint16_t*)a.kc + slot[u] * a.c_slot + coff[u]) = kx[u];
    *(u32x4*)((uint16_t*)a.vc + slot[u] * a.c_slot + coff[u]) = vx[u];
  }
}

template <int D, int NW_ = 8, int CT_ = 2>
struct PShape {
  static constexpr int NW = NW_;  // wavefronts per workgroup (8: two per SIMD; 4: one)
  static constexpr int CT = CT_;  // 16-column tiles per wavefront
  static constexpr int COLS = NW * CT * 16;  // (token, head) columns per workgroup
  static constexpr int BN = 64;   // keys per tile
  static constexpr int NT = NW * 64;
  // LDS row pitches: gfx950 serves the 16-row MFMA operand reads without bank
  // conflicts only with 32 extra bytes per K row and 16 per V^T row (8 and 16
  // bytes still conflict two ways, measured with SQ_LDS_BANK_CONFLICT)
  static constexpr int KROW = D + 16;  // elements per K row in LDS
  static constexpr int KCH = BN * D / 8;       // 16-byte K chunks per tile
  static constexpr int KPT = (KCH + NT - 1) / NT;
  static constexpr int KS = D / 32;   // k-steps of S^T = K . Q^T
  static constexpr int DTL = D / 16;  // d tiles of O^T
};

// FAST: power-of-two block size and a pool layer small enough for 24-bit slot
// and stride products (32-bit element offsets).
// SCHED: kLockstep (3-deep ring, next tile's scores beside this tile's
// exponentials) or kRing2 (2-deep ring, one tile at a time: ~78 KB of LDS
// and <= 256 registers, so two 4-wavefront workgroups share a CU).
constexpr int kLockstep = 0, kRing2 = 2;

template <int DT, int D, bool FAST, int NW, int CTW, int SCHED, bool FUSED = false>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW == 8 || SCHED == kRing2 ? 2 : 1)))
void paged_prefill_kernel(PrefillArgs a) {
  typedef PShape<D, NW, CTW> S;
  constexpr int EB = 2;
  constexpr int CT = S::CT, BN = S::BN, NT = S::NT;
  constexpr int RING = SCHED == kRing2 ? 2 : 3;
  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[RING][BN * S::KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vs_lds[RING][BN * S::KROW];
  __shared__ int32_t bt_lds[kBtCache];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int TQ = a.tq;

  if (FUSED && blockIdx.x >= a.n_work) {  // a writer of a fused call
    prefill_write_rows<D, NT>(a, blockIdx.x - a.n_work);
    return;
  }

  // ---- which (query block, KV head, sequence) and which piece of its keys:
  // plan entry i when a plan is given, else the last query blocks (most keys
  // within a sequence) first, uncut
  int tb, seq, kvh, nparts = 1, part = 0, pbase = 0;
  if (a.items) {
    const int2 e = a.items[blockIdx.x];
    const int item = e.x < 0 ? -1 : e.x / a.num_kv_heads;
    if (item < 0 || item >= a.num_seqs * a.n_qblocks) return;
    kvh = e.x - item * a.num_kv_heads;
    seq = item / a.n_qblocks;
    tb = item - seq * a.n_qblocks;
    nparts = max(e.y & 0xff, 1);
    part = min((e.y >> 8) & 0xff, nparts - 1);
    pbase = (int)((uint32_t)e.y >> 16);
  } else {
    const int per_tb = a.num_kv_heads * a.num_seqs;
    tb = a.n_qblocks - 1 - (int)(blockIdx.x / per_tb);
    const int rest = (int)(blockIdx.x % per_tb);
    seq = rest % a.num_seqs;
    kvh = rest / a.num_seqs;
  }

  int q_lo = a.cu_q[seq];
  int q_len = a.cu_q[seq + 1] - q_lo;
  if (q_lo < 0 || q_len < 0 || (int64_t)q_lo + q_len > a.total_q) {
    if (tid == 0 && tb == 0 && kvh == 0) flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    return;
  }
  const int tq0 = tb * TQ;
  // a chunk longer than the host's max_q_len has rows no workgroup covers
  if (tb == a.n_qblocks - 1 && kvh == 0 && tid == 0 && q_len > a.n_qblocks * TQ)
    flag_error(a.err, IR_ERR_CONTEXT_RANGE);
  if (tq0 >= q_len) return;
  int p0 = a.q_start[seq];
  const int cap = a.max_blocks * a.bs;
  if (p0 < 0 || (int64_t)p0 + q_len > cap) {
    if (tid == 0 && tb == 0 && kvh == 0) flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    p0 = p0 < 0 ? 0 : min(p0, cap);  // keeps p0 + q_len within int range
  }
  // keys this block needs: up to its last query's position, within the table;
  // this piece walks key tiles [t_lo, t_hi) of them
  const int kmax = min(cap, p0 + min(q_len, tq0 + TQ));
  const int nkb = kmax > 0 && a.num_blocks > 0 ? (kmax + BN - 1) / BN : 0;
  const int t_lo = (int)((int64_t)part * nkb / nparts);
  const int t_hi = (int)((int64_t)(part + 1) * nkb / nparts);

  // columns of this lane: tile ct holds column j = 32 w + 16 ct + c, i.e.
  // token tq0 + j / n_rep, query head kvh * n_rep + j % n_rep (recomputed for
  // the output store rather than kept live through the key walk)
  struct Col {
    int tok, head;
    bool ok;
  };
  auto column = [&](int ct) {
    const int j = w * (CT * 16) + ct * 16 + c;
    const int t = j / a.n_rep;
    return Col{tq0 + t, kvh * a.n_rep + (j - t * a.n_rep), t < TQ && tq0 + t < q_len};
  };
  const int32_t* bt_row = a.bt + (int64_t)seq * a.bt_stride;
  const uint16_t* kc = (const uint16_t*)a.kc + (int64_t)kvh * a.c_head;
  const uint16_t* vc = (const uint16_t*)a.vc + (int64_t)kvh * a.c_head;

  // ---- Q^T operands: lane (g, c) holds d = 32 ks + 8 g .. +7 of its column,
  // multiplied by scale * log2(e) and rounded back to the input dtype, so the
  // score MFMA yields base-2 exponents directly. The small-grid shape (every
  // workgroup alone on its CU: each one's latency is the call's) loads Q raw
  // and scales it once its first key tile is staged, so Q's round trip
  // overlaps the block ids' and the first tile's instead of preceding them.
  constexpr bool EARLY = NW == 8 && CT == 1 && SCHED == kRing2;
  u32x4 qreg[CT][S::KS];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const Col col = column(ct);
    const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)(q_lo + (col.ok ? col.tok : 0)) * a.q_tok +
                           (int64_t)(col.ok ? col.head : 0) * a.q_head;
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      if constexpr (EARLY) {
        const u32x4 x = *(const u32x4*)(qrow + ks * 32 + 8 * g);  // (a valid row when !col.ok)
        qreg[ct][ks] = col.ok ? x : u32x4{0u, 0u, 0u, 0u};
      } else {
        const u32x4 x = col.ok ? *(const u32x4*)(qrow + ks * 32 + 8 * g) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          qreg[ct][ks][e] = Elem<DT>::pack2(Elem<DT>::lo(x[e]) * a.scale_log2, Elem<DT>::hi(x[e]) * a.scale_log2);
      }
    }
  }

  // ---- block-id cache: ids [bt_base, bt_base + kBtCache) of this sequence
  const int nblk_needed = (kmax + a.bs - 1) / a.bs;
  int bt_base = 0;
  auto fill_bt = [&](int base) {
    __syncthreads();
    for (int i = tid; i < kBtCache && base + i < nblk_needed; i += NT) bt_lds[i] = bt_row[base + i];
    __syncthreads();
    bt_base = base;
  };
  bool bad = false;
  // Slot of absolute key k and whether it may be used: keys at or past kmax are
  // masked out; a bad block id is flagged and its K and V read as zeros. Every
  // load is issued (from slot 0 when unusable) and zeroed afterwards.
  auto slot_of = [&](int k, bool& use) -> int64_t {
    const bool in = k < kmax;
    // an unusable key looks up the cache's first id, inside the staged
    // window (key 0 would index below it once the window has moved)
    const int kk = in ? k : bt_base * a.bs;
    if constexpr (FAST) {
      const int blk = kk >> a.bs_shift;
      const int32_t bid = bt_lds[blk - bt_base];
      use = in && (uint32_t)bid < (uint32_t)a.num_blocks;
      bad |= in && !use;
      const int sl = use ? (bid << a.bs_shift) | (kk & (a.bs - 1)) : 0;
      return (int64_t)(uint32_t)__mul24(sl, a.c_slot32);  // element offset
    } else {
      const int blk = kk / a.bs;
      const int32_t bid = bt_lds[blk - bt_base];
      use = in && bid >= 0 && (int64_t)bid < a.num_blocks;
      bad |= in && !use;
      return use ? ((int64_t)bid * a.bs + (kk - blk * a.bs)) * a.c_slot : 0;
    }
  };
  auto zero_unless = [](u32x4 x, bool keep) {
    return u32x4{keep ? x[0] : 0u, keep ? x[1] : 0u, keep ? x[2] : 0u, keep ? x[3] : 0u};
  };

  // K and V of a key share its slot: each thread loads the same 16-byte
  // piece of both
  u32x4 kreg[S::KPT], vreg[S::KPT];
  // whether each load in flight reads a usable key: applied when the tile is
  // stored (zero_unless), not when it is loaded, so the loads stay in flight
  // through the next tile's math instead of being waited for at once
  bool kuse[S::KPT];
  // Global loads of key tile kb into registers (whole workgroup, uniform call).
  // In a fused call, a tile holding the sequence's new keys reads those keys
  // from the call's new rows (the writers fill their slots concurrently).
  const uint16_t* kn = a.k_new ? (const uint16_t*)a.k_new + (int64_t)kvh * a.kn_head : nullptr;
  const uint16_t* vn = a.v_new ? (const uint16_t*)a.v_new + (int64_t)kvh * a.vn_head : nullptr;
  const int64_t new_row0 = a.src_row0 + q_lo - p0;  // row of new key k: new_row0 + k
  auto load_into = [&](int kb, u32x4 (&kr)[S::KPT], u32x4 (&vr)[S::KPT], bool (&ku)[S::KPT]) {
    const int k0 = kb * BN;
    const int k_last = min(k0 + BN, kmax) - 1;
    const int last_blk = FAST ? k_last >> a.bs_shift : k_last / a.bs;
    if (last_blk >= bt_base + kBtCache) fill_bt(FAST ? k0 >> a.bs_shift : k0 / a.bs);
    if (FUSED && k0 + BN > p0) {  // uniform: new keys in this tile
#pragma unroll
      for (int i = 0; i < S::KPT; ++i) {
        const int q = tid + NT * i;
        if (S::KCH % NT == 0 || q < S::KCH) {
          const int key = q / (D / 8), part = q % (D / 8);
          const int kk = k0 + key;
          // a new key is read from the call's rows and needs no block id (the
          // check after the walk flags a bad one): a tile of new keys only
          // may be loaded before the block ids are
          const bool fresh = kk >= p0 && kk < kmax;
          bool use = fresh;
          int64_t sl = 0;
          if (!fresh) sl = slot_of(kk, use);
          const int64_t row = new_row0 + kk;
          const uint16_t* kp = fresh ? kn + row * a.kn_tok + part * 8 : kc + sl + part * 8;
          const uint16_t* vp = fresh ? vn + row * a.vn_tok + part * 8 : vc + sl + part * 8;
          kr[i] = *(const u32x4*)kp;
          vr[i] = *(const u32x4*)vp;
          ku[i] = use;
        }
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const int q = tid + NT * i;
      if (S::KCH % NT == 0 || q < S::KCH) {
        const int key = q / (D / 8), part = q % (D / 8);
        bool use;
        const int64_t sl = slot_of(k0 + key, use);
        kr[i] = *(const u32x4*)(kc + sl + part * 8);
        vr[i] = *(const u32x4*)(vc + sl + part * 8);
        ku[i] = use;
      }
    }
  };
  auto load_regs = [&](int kb) { load_into(kb, kreg, vreg, kuse); };
  // Registers -> LDS buffer `buf`: K and V tiles both row-major [64 keys][D]
  // (+32 bytes a row).
  auto store_from = [&](int buf, const u32x4 (&kr)[S::KPT], const u32x4 (&vr)[S::KPT], const bool (&ku)[S::KPT]) {
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const int q = tid + NT * i;
      if (q < S::KCH) {
        const int key = q / (D / 8), part = q % (D / 8);
        *(u32x4*)&ks_lds[buf][key * S::KROW + part * 8] = zero_unless(kr[i], ku[i]);
        *(u32x4*)&vs_lds[buf][key * S::KROW + part * 8] = zero_unless(vr[i], ku[i]);
      }
    }
  };
  auto store_regs = [&](int buf) { store_from(buf, kreg, vreg, kuse); };
  // V^T operand of PV step t (d tile t % DTL, 32-key step t / DTL) from the
  // row-major V tile at vb: lane (g, c) needs V[32 st + 4 g + e][16 dt + c]
  // (k-slots 0..3) and V[32 st + 16 + 4 g + e][..] (4..7), e = 0..3: the
  // columns of 4 consecutive rows. gfx950's transpose read returns, to lane
  // 4a + b of each 16-lane group, element b of the 4-element pieces that lanes
  // a, a + 4, a + 8, a + 12 address, so lane c points at row key0 + c / 4,
  // columns 16 dt + 4 (c % 4) .. +3, and gets its column of rows key0 .. +3.
  auto v_operand_tr = [&](const uint16_t* vb, int t) {
    const int dt = t % S::DTL, st = t / S::DTL;
    const int v_lane = (4 * g + (c >> 2)) * S::KROW + 4 * (c & 3);
    lds_u16* p = (lds_u16*)vb + v_lane + 32 * st * S::KROW + 16 * dt;
    const u32x2 lo = lds_read_tr16(p);
    const u32x2 hi = lds_read_tr16(p + 16 * S::KROW);
    return u32x4{lo[0], lo[1], hi[0], hi[1]};
  };

  // ---- online softmax state, per column tile: lane owns column c of it.
  // negm[ct] holds -m (the running base-2 max, 0 before the first tile) in
  // all four slots: it is the accumulator a tile's score MFMAs start from, so
  // the scores arrive as s - m and need only the exponential.
  f32x4 acc[CT][S::DTL], negm[CT];
  float l[CT];
#pragma unroll
  for (int qt = 0; qt < CT; ++qt) {
    negm[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    l[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < S::DTL; ++dt) acc[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int qpos0 = p0 + tq0;  // position of the block's first query
  int col_lim[CT];             // last key each column may see
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) col_lim[ct] = min(p0 + column(ct).tok, kmax - 1);

  // S^T += K . Q^T for key tile kt (< 4), k-step ks (< KS) of the tile staged
  // at kb_lds.
  auto qk_step = [&](const uint16_t* kb_lds, int kt, int ks, f32x4 (&x)[CT][4]) {
    const u32x4 ka = *(const u32x4*)&kb_lds[(kt * 16 + c) * S::KROW + ks * 32 + 8 * g];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) x[ct][kt] = mfma_k32<DT>(ka, qreg[ct][ks], x[ct][kt]);
  };
  auto zero_s = [](f32x4 (&x)[CT][4]) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) x[ct][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // One key tile kb, software pipelined: the scores `cur` of tile kb (base 2,
  // less the max m they were started from) are ready; while their
  // exponentials run on the VALU, the scores `nxt` of tile kb + 1 (already
  // staged) are computed on the MFMA pipe (NX), then O^T += V^T . P^T for tile
  // kb. The first tile sets m to its own max; later ones move it only when
  // their max exceeds it by more than kRescaleSlack, and only those tiles
  // subtract the change from their scores.
  auto step = [&](auto nx_tag, int kb, f32x4 (&cur)[CT][4], f32x4 (&nxt)[CT][4]) {
    constexpr bool NX = decltype(nx_tag)::value;
    using E = Elem<DT>;
    const int k0 = kb * BN;
    const bool first = kb == t_lo;
    // only tiles that cross the causal diagonal or the last key are masked
    if (!(k0 + BN - 1 <= qpos0 && k0 + BN <= kmax)) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k0 + kt * 16 + 4 * g + r > col_lim[ct]) cur[ct][kt][r] = kNegInf;
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float mx = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        mx = fmaxf(mx, fmaxf(fmaxf(cur[ct][kt][0], cur[ct][kt][1]), fmaxf(cur[ct][kt][2], cur[ct][kt][3])));
      mx = wave_max_groups_swap(mx);  // relative to m; finite on the first tile (key 0 is always visible)
      const bool grow = first || mx > kRescaleSlack;
      if (__any(grow)) {
        const float d = grow ? mx : 0.f;  // the max moves up by d
        if (!first) {
          const float alpha = fast_exp2(-d);
          l[ct] *= alpha;
#pragma unroll
          for (int dt = 0; dt < S::DTL; ++dt) acc[ct][dt] *= alpha;
        }
        negm[ct] -= d;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) cur[ct][kt] -= d;
      }
    }
    // next tile's scores (MFMA) interleaved with this tile's exponentials (VALU)
    const uint16_t* kn = ks_lds[(kb + 1) % RING];
    if constexpr (NX) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) nxt[ct][kt] = negm[ct];
    }
    // NQK = 4 * KS score MFMA steps, SPS of this lane's CT * 16 scores each.
    // Program order is kept step by step (sched_barrier): each step's K operand
    // was read one step earlier, its MFMAs go to the matrix pipe and the
    // exponentials of SPS scores fill the VALU meanwhile.
    constexpr int NQK = 4 * S::KS, SPS = CT * 16 / NQK;
    auto k_operand = [&](int t) {
      return *(const u32x4*)&kn[((t % 4) * 16 + c) * S::KROW + (t / 4) * 32 + 8 * g];
    };
    u32x4 kring[kOperandAhead];
#pragma unroll
    for (int t = 0; t < kOperandAhead; ++t) kring[t] = NX ? k_operand(t) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int t = 0; t < NQK; ++t) {
      if constexpr (NX) {
        const u32x4 ka = kring[t % kOperandAhead];
        if (t + kOperandAhead < NQK) kring[t % kOperandAhead] = k_operand(t + kOperandAhead);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) nxt[ct][t % 4] = mfma_k32<DT>(ka, qreg[ct][t / 4], nxt[ct][t % 4]);
      }
#pragma unroll
      for (int j = 0; j < SPS; ++j) {
        const int i = t * SPS + j;
        const int ct = i / 16, kt = (i % 16) / 4, r = i % 4;
        cur[ct][kt][r] = fast_exp2(cur[ct][kt][r]);
      }
      // (no scheduling barrier)
    }
    // P^T operands of the two 32-key steps: k-slots 0..3 = keys 4g..4g+3 of
    // tile 2st, k-slots 4..7 = keys 4g..4g+3 of tile 2st+1
    u32x4 pb[CT][2];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        pb[ct][st] = u32x4{E::pack2(cur[ct][2 * st][0], cur[ct][2 * st][1]),
                           E::pack2(cur[ct][2 * st][2], cur[ct][2 * st][3]),
                           E::pack2(cur[ct][2 * st + 1][0], cur[ct][2 * st + 1][1]),
                           E::pack2(cur[ct][2 * st + 1][2], cur[ct][2 * st + 1][3])};
        // the running sum adds the rounded probabilities the PV product uses,
        // two per instruction
#pragma unroll
        for (int e = 0; e < 4; ++e) l[ct] = sum2<DT>(pb[ct][st][e], l[ct]);
      }
    }
    // O^T += V^T . P^T; V^T operand: d row c of the tile, the same key slots
    // (operands read one step ahead)
    const uint16_t* vb_lds = vs_lds[kb % RING];
    auto v_operand = [&](int t) {
      return v_operand_tr(vb_lds, t);
    };
    u32x4 vring[kOperandAhead];
#pragma unroll
    for (int t = 0; t < kOperandAhead; ++t) vring[t] = v_operand(t);
#pragma unroll
    for (int t = 0; t < 2 * S::DTL; ++t) {
      const u32x4 va = vring[t % kOperandAhead];
      if (t + kOperandAhead < 2 * S::DTL) vring[t % kOperandAhead] = v_operand(t + kOperandAhead);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        acc[ct][t % S::DTL] = mfma_k32<DT>(va, pb[ct][t / S::DTL], acc[ct][t % S::DTL]);
    }
  };

  // ---- walk key tiles [t_lo, t_hi)
  if constexpr (EARLY) {
    // The small-grid shape: a workgroup alone on its CU has no other one to
    // cover its loads' latency, so a register ring of R tiles keeps R - 1
    // tiles' loads in flight behind the one being staged (all of a short
    // walk's at once); LDS stays a 2-deep ring. Tile t_lo + i
    // lives in ring slot i % R, the walk unrolled by R so every slot index is
    // fixed. The first tile, when it holds new keys only, is loaded before the
    // block ids are, with Q's loads.
    constexpr int R = 4;
    if (t_lo < t_hi) {
      u32x4 kr[R][S::KPT], vr[R][S::KPT];
      bool ku[R][S::KPT];
      const int bt0 = FAST ? (t_lo * BN) >> a.bs_shift : (t_lo * BN) / a.bs;
      if (FUSED && t_lo * BN >= p0) {  // uniform
        load_into(t_lo, kr[0], vr[0], ku[0]);
        fill_bt(bt0);
      } else {
        fill_bt(bt0);
        load_into(t_lo, kr[0], vr[0], ku[0]);
      }
#pragma unroll
      for (int j = 1; j < R; ++j)
        if (t_lo + j < t_hi) load_into(t_lo + j, kr[j], vr[j], ku[j]);
      store_from(t_lo & 1, kr[0], vr[0], ku[0]);
      __syncthreads();
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int ks = 0; ks < S::KS; ++ks) {
          const u32x4 x = qreg[ct][ks];
          u32x4 y;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            y[e] = Elem<DT>::pack2(Elem<DT>::lo(x[e]) * a.scale_log2, Elem<DT>::hi(x[e]) * a.scale_log2);
          qreg[ct][ks] = y;
        }
      f32x4 sc[CT][4];
      // tile kb (slot J): its scores, softmax and PV product from LDS buffer
      // kb % 2; tile kb + 1 staged from slot J + 1; tile kb + R's loads into slot J
      auto sub = [&](auto slot, int kb) {
        constexpr int J = decltype(slot)::value;
        if (kb >= t_hi) return;  // uniform
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) sc[ct][kt] = negm[ct];
#pragma unroll
        for (int t = 0; t < 4 * S::KS; ++t) qk_step(ks_lds[kb & 1], t % 4, t / 4, sc);
        step(std::false_type{}, kb, sc, sc);
        if (kb + 1 < t_hi) store_from((kb + 1) & 1, kr[(J + 1) % R], vr[(J + 1) % R], ku[(J + 1) % R]);
        if (kb + R < t_hi) load_into(kb + R, kr[J], vr[J], ku[J]);
        __syncthreads();
      };
      for (int kb = t_lo; kb < t_hi; kb += R) {
        sub(std::integral_constant<int, 0>{}, kb);
        sub(std::integral_constant<int, 1>{}, kb + 1);
        sub(std::integral_constant<int, 2>{}, kb + 2);
        sub(std::integral_constant<int, 3>{}, kb + 3);
      }
    }
  } else if constexpr (SCHED == kRing2) {
    // one tile per step: its scores (from -m), softmax and PV product read
    // buffer kb % 2 while tile kb + 1 is written to the other buffer from the
    // registers its loads filled a step earlier and tile kb + 2's loads go
    // out
    if (t_lo < t_hi) {
      fill_bt(FAST ? (t_lo * BN) >> a.bs_shift : (t_lo * BN) / a.bs);
      load_regs(t_lo);
      store_regs(t_lo & 1);
      if (t_lo + 1 < t_hi) load_regs(t_lo + 1);
      __syncthreads();
      f32x4 sc[CT][4];
      for (int kb = t_lo; kb < t_hi; ++kb) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) sc[ct][kt] = negm[ct];
#pragma unroll
        for (int t = 0; t < 4 * S::KS; ++t) qk_step(ks_lds[kb & 1], t % 4, t / 4, sc);
        step(std::false_type{}, kb, sc, sc);
        if (kb + 1 < t_hi) store_regs((kb + 1) & 1);
        if (kb + 2 < t_hi) load_regs(kb + 2);
        __syncthreads();
      }
    }
  } else if (t_lo < t_hi) {
    // 3-deep ring: tile kb (V) and tile kb + 1 (K) are read while tile kb + 2
    // is written from registers and tile kb + 3 is in flight
    auto tail = [&](int kb) {
      if (kb + 2 < t_hi) store_regs((kb + 2) % 3);
      if (kb + 3 < t_hi) load_regs(kb + 3);
      __syncthreads();
    };
    fill_bt(FAST ? (t_lo * BN) >> a.bs_shift : (t_lo * BN) / a.bs);
    load_regs(t_lo);
    store_regs(t_lo % 3);
    if (t_lo + 1 < t_hi) {
      load_regs(t_lo + 1);
      store_regs((t_lo + 1) % 3);
    }
    if (t_lo + 2 < t_hi) load_regs(t_lo + 2);
    __syncthreads();
    f32x4 sa[CT][4], sb[CT][4];
    zero_s(sa);
#pragma unroll
    for (int t = 0; t < 4 * S::KS; ++t) qk_step(ks_lds[t_lo % 3], t % 4, t / 4, sa);
    int kb = t_lo;
    // two tiles per trip so the score buffers swap roles without copies
    for (; kb + 2 < t_hi; kb += 2) {
      step(std::true_type{}, kb, sa, sb);
      tail(kb);
      step(std::true_type{}, kb + 1, sb, sa);
      tail(kb + 1);
    }
    if (kb + 1 < t_hi) {
      step(std::true_type{}, kb, sa, sb);
      tail(kb);
      step(std::false_type{}, kb + 1, sb, sa);
    } else {
      step(std::false_type{}, kb, sa, sb);
    }
  }
  if (bad) flag_error(a.err, IR_ERR_BLOCK_RANGE);
  if (FUSED && kvh == 0 && part == 0 && tid < TQ && tq0 + tid < q_len) {
    // this block's new tokens (checked once, by the KV head 0 workgroups):
    // each one's write slot must be the slot its block table gives it, which
    // the workgroups that read it as a key took it to be (a check after the
    // walk, off its loads' path)
    const int pos = p0 + tq0 + tid;
    const int blk = pos / a.bs;
    const int32_t bid = blk < a.max_blocks ? bt_row[blk] : -1;
    const int64_t ws = a.write_slots[a.src_row0 + q_lo + tq0 + tid];
    if (bid < 0 || (int64_t)bid >= a.num_blocks) {
      if (blk < a.max_blocks) flag_error(a.err, IR_ERR_BLOCK_RANGE);  // (read from its row all the same)
    } else if (ws != (int64_t)bid * a.bs + (pos - blk * a.bs)) {
      flag_error(a.err, IR_ERR_WRITE_SLOT);
    }
  }

  if (nparts == 1) {
    // ---- normalise and store: lane (g, c) register r of d tile dt = output
    // d = 16 dt + 4 g + r of column c
#pragma unroll
    for (int qt = 0; qt < CT; ++qt) {
      const float lsum = wave_sum_groups_swap(l[qt]);
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      const Col col = column(qt);
      if (!col.ok) continue;
      uint8_t* orow = (uint8_t*)a.out + ((int64_t)(q_lo + col.tok) * a.o_tok + (int64_t)col.head * a.o_head) * EB;
#pragma unroll
      for (int dt = 0; dt < S::DTL; ++dt) {
        const float o[4] = {acc[qt][dt][0], acc[qt][dt][1], acc[qt][dt][2], acc[qt][dt][3]};
        store4<DT>(orow + (dt * 16 + 4 * g) * EB, o, inv);
      }
    }
    return;
  }

  // ---- a piece of a cut item: publish this piece's partial rows (device
  // scope), count its arrival; the last piece to arrive merges them all in
  // part order (the same arithmetic whichever piece arrives last), its own
  // part from registers and the others loaded for exactly the (column, d)
  // elements each lane holds, every load of a part in flight together
  constexpr int COLS = S::COLS;
  const __amdgpu_buffer_rsrc_t r_o = dev_rsrc(a.ws_o), r_ml = dev_rsrc(a.ws_ml);
  const int row_step = a.num_kv_heads * COLS;  // rows between parts of one item
  const int row_base = (pbase * a.num_kv_heads + kvh) * COLS;  // part 0, column 0
  float lsum[CT];
#pragma unroll
  for (int qt = 0; qt < CT; ++qt) {
    lsum[qt] = wave_sum_groups_swap(l[qt]);
    const int row = row_base + part * row_step + w * (CT * 16) + qt * 16 + c;
#pragma unroll
    for (int dt = 0; dt < S::DTL; ++dt) store_dev4(r_o, (row * D + dt * 16 + 4 * g) * 4, acc[qt][dt]);
    if (g == 0) store_dev2(r_ml, row * 8, f32x2{-negm[qt][0], lsum[qt]});
  }
  __shared__ int s_last;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int32_t* ctr = a.counters + pbase * a.num_kv_heads + kvh;
  if (tid == 0) {
    const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == nparts - 1;
  }
  __syncthreads();
  if (!s_last) return;
  f32x4 o_run[CT][S::DTL];
  float m_run[CT], l_run[CT];
#pragma unroll
  for (int qt = 0; qt < CT; ++qt) {
    m_run[qt] = kNegInf;
    l_run[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < S::DTL; ++dt) o_run[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int p = 0; p < nparts; ++p) {
    f32x4 op[CT][S::DTL];
    float mp[CT], lp[CT];
    if (p == part) {
#pragma unroll
      for (int qt = 0; qt < CT; ++qt) {
        mp[qt] = -negm[qt][0];
        lp[qt] = lsum[qt];
#pragma unroll
        for (int dt = 0; dt < S::DTL; ++dt) op[qt][dt] = acc[qt][dt];
      }
    } else {
#pragma unroll
      for (int qt = 0; qt < CT; ++qt) {
        const int row = row_base + p * row_step + w * (CT * 16) + qt * 16 + c;
        const f32x2 ml = load_dev2(r_ml, row * 8);
        mp[qt] = ml[0];
        lp[qt] = ml[1];
#pragma unroll
        for (int dt = 0; dt < S::DTL; ++dt) op[qt][dt] = load_dev4(r_o, (row * D + dt * 16 + 4 * g) * 4);
      }
    }
#pragma unroll
    for (int qt = 0; qt < CT; ++qt) {
      // a part without keys has max -inf: its weight is exp2(-inf) = 0, and
      // fmaxf keeps an (-inf) - (-inf) exponent from becoming NaN
      const float mn = fmaxf(m_run[qt], mp[qt]);
      const float wa = fast_exp2(fmaxf(m_run[qt] - mn, -1e30f)), wb = fast_exp2(fmaxf(mp[qt] - mn, -1e30f));
      l_run[qt] = wa * l_run[qt] + wb * lp[qt];
#pragma unroll
      for (int dt = 0; dt < S::DTL; ++dt) o_run[qt][dt] = wa * o_run[qt][dt] + wb * op[qt][dt];
      m_run[qt] = mn;
    }
  }
#pragma unroll
  for (int qt = 0; qt < CT; ++qt) {
    const float inv = l_run[qt] > 0.f ? 1.f / l_run[qt] : 0.f;
    const Col col = column(qt);
    if (!col.ok) continue;
    uint8_t* orow = (uint8_t*)a.out + ((int64_t)(q_lo + col.tok) * a.o_tok + (int64_t)col.head * a.o_head) * EB;
#pragma unroll
    for (int dt = 0; dt < S::DTL; ++dt) {
      const float o[4] = {o_run[qt][dt][0], o_run[qt][dt][1], o_run[qt][dt][2], o_run[qt][dt][3]};
      store4<DT>(orow + (dt * 16 + 4 * g) * EB, o, inv);
    }
  }
  if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- fp32
//
// fp32 chunked prefill, the reference's fp32 path (fp32 scores, softmax and
// PV product), with 16x16x4 fp32 MFMAs: lane (g, c) of a product supplies
// element (row c, k-slot g) of A and (k-slot g, column c) of B and receives
// rows 4g..4g+3 of column c. A workgroup is 4 wavefronts of one 16-column
// tile: 64 columns, tq = 64 / n_rep tokens of one KV head's query heads, in
// the order of a plan built with IR_PLAN_F32 (heaviest first, the heaviest
// items cut into key-range pieces merged like the 16-bit kernel's), else the
// last query blocks first. Keys walk in 64-key tiles through LDS -- K
// row-major, V transposed, so both operands are 16-byte reads -- with the next
// tile's loads in flight in registers. The
// score product's k-slot g of step (m, r) is d = 16 m + 4 g + r (a lane's K
// read covers its four steps); the PV product's k-slot g of step (kt, r) is
// key 16 kt + 4 g + r, the lane's own probability of that key. Same masking,
// lazy rescale and flags as the 16-bit kernel.
constexpr int kF32Threads = 256;
constexpr int kF32Cols = 64;

template <int D, bool FAST>
__global__ __launch_bounds__(kF32Threads) __attribute__((amdgpu_waves_per_eu(2)))
void paged_prefill_f32_kernel(PrefillArgs a) {
  constexpr int NT = kF32Threads, BN = 64, MT = D / 16, DT4 = D / 4;
  constexpr int KROW = D + 4;           // floats per K row in LDS
  constexpr int VROW = BN + 4;          // floats per V^T row (one d, 64 keys)
  constexpr int BPT = (BN / 4) * DT4 / NT;  // 4-key x 4-d blocks of a tile per thread
  static_assert((BN / 4) * DT4 % NT == 0 && BPT >= 1, "a tile's blocks must divide among the threads");
  __shared__ __attribute__((aligned(16))) float ks[BN * KROW];
  __shared__ __attribute__((aligned(16))) float vt[D * VROW];
  __shared__ int32_t bt_lds[kBtCache];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int TQ = a.tq;
  // which (query block, KV head, sequence) and which piece of its keys: plan
  // entry i when a plan is given, else the last query blocks first, uncut
  int tb, seq, kvh, nparts = 1, part = 0, pbase = 0;
  if (a.items) {
    const int2 e = a.items[blockIdx.x];
    const int item = e.x < 0 ? -1 : e.x / a.num_kv_heads;
    if (item < 0 || item >= a.num_seqs * a.n_qblocks) return;
    kvh = e.x - item * a.num_kv_heads;
    seq = item / a.n_qblocks;
    tb = item - seq * a.n_qblocks;
    nparts = max(e.y & 0xff, 1);
    part = min((e.y >> 8) & 0xff, nparts - 1);
    pbase = (int)((uint32_t)e.y >> 16);
  } else {
    const int per_tb = a.num_kv_heads * a.num_seqs;
    tb = a.n_qblocks - 1 - (int)(blockIdx.x / per_tb);
    const int rest = (int)(blockIdx.x % per_tb);
    seq = rest % a.num_seqs;
    kvh = rest / a.num_seqs;
  }
  const int q_lo = a.cu_q[seq];
  const int q_len = a.cu_q[seq + 1] - q_lo;
  if (q_lo < 0 || q_len < 0 || (int64_t)q_lo + q_len > a.total_q) {
    if (tid == 0 && tb == 0 && kvh == 0) flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    return;
  }
  const int tq0 = tb * TQ;
  if (tb == a.n_qblocks - 1 && kvh == 0 && tid == 0 && q_len > a.n_qblocks * TQ)
    flag_error(a.err, IR_ERR_CONTEXT_RANGE);
  if (tq0 >= q_len) return;
  int p0 = a.q_start[seq];
  const int cap = a.max_blocks * a.bs;
  if (p0 < 0 || (int64_t)p0 + q_len > cap) {
    if (tid == 0 && tb == 0 && kvh == 0) flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    p0 = p0 < 0 ? 0 : min(p0, cap);
  }
  const int kmax = min(cap, p0 + min(q_len, tq0 + TQ));
  const int nkb = kmax > 0 && a.num_blocks > 0 ? (kmax + BN - 1) / BN : 0;
  // this piece walks key tiles [t_lo, t_hi); a cut item's pieces are at
  // least four tiles (the plan cuts only items of more than eight), so a
  // piece's first tile lies before every column's causal limit
  const int t_lo = (int)((int64_t)part * nkb / nparts);
  const int t_hi = (int)((int64_t)(part + 1) * nkb / nparts);

  // this lane's column j = 16 w + c: token tq0 + j / n_rep, query head
  // kvh * n_rep + j % n_rep
  const int j = w * 16 + c, jt = j / a.n_rep;
  const bool col_ok = jt < TQ && tq0 + jt < q_len;
  const int col_tok = tq0 + jt, col_head = kvh * a.n_rep + (j - jt * a.n_rep);
  // Q^T operand of score step (m, r): q[16 m + 4 g + r] of the column, times
  // scale * log2(e), so the scores come out as base-2 exponents
  float qreg[MT][4];
  {
    const float* qrow = (const float*)a.q + (int64_t)(q_lo + (col_ok ? col_tok : tq0)) * a.q_tok +
                        (int64_t)(col_ok ? col_head : kvh * a.n_rep) * a.q_head;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const f32x4 x = *(const f32x4*)(qrow + 16 * m + 4 * g);
#pragma unroll
      for (int r = 0; r < 4; ++r) qreg[m][r] = col_ok ? x[r] * a.scale_log2 : 0.f;
    }
  }

  const int32_t* bt_row = a.bt + (int64_t)seq * a.bt_stride;
  const float* kc = (const float*)a.kc + (int64_t)kvh * a.c_head;
  const float* vc = (const float*)a.vc + (int64_t)kvh * a.c_head;
  const int nblk_needed = (kmax + a.bs - 1) / a.bs;
  int bt_base = 0;
  auto fill_bt = [&](int base) {
    __syncthreads();
    for (int i = tid; i < kBtCache && base + i < nblk_needed; i += NT) bt_lds[i] = bt_row[base + i];
    __syncthreads();
    bt_base = base;
  };
  bool bad = false;
  // element offset of key k's row in the pool and whether it may be used
  // (keys past kmax are masked; a bad block id is flagged and reads as zeros)
  auto slot_of = [&](int k, bool& use) -> int64_t {
    const bool in = k < kmax;
    const int kk = in ? k : bt_base * a.bs;
    if constexpr (FAST) {
      const int blk = kk >> a.bs_shift;
      const int32_t bid = bt_lds[blk - bt_base];
      use = in && (uint32_t)bid < (uint32_t)a.num_blocks;
      bad |= in && !use;
      const int sl = use ? (bid << a.bs_shift) | (kk & (a.bs - 1)) : 0;
      return (int64_t)(uint32_t)__mul24(sl, a.c_slot32);
    } else {
      const int blk = kk / a.bs;
      const int32_t bid = bt_lds[blk - bt_base];
      use = in && bid >= 0 && (int64_t)bid < a.num_blocks;
      bad |= in && !use;
      return use ? ((int64_t)bid * a.bs + (kk - blk * a.bs)) * a.c_slot : 0;
    }
  };
  // a tile's 4-key x 4-d blocks: block b = tid + NT i holds keys 4 (b / DT4)
  // .. +3 at d = 4 (b % DT4) .. +3
  f32x4 kr[BPT][4], vr[BPT][4];
  bool ku[BPT][4];
  auto load_tile = [&](int kb) {
    const int k0 = kb * BN;
    const int k_last = min(k0 + BN, kmax) - 1;
    const int last_blk = FAST ? k_last >> a.bs_shift : k_last / a.bs;
    if (last_blk >= bt_base + kBtCache) fill_bt(FAST ? k0 >> a.bs_shift : k0 / a.bs);
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int b = tid + NT * i, key4 = b / DT4, d4 = b - key4 * DT4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        bool use;
        const int64_t sl = slot_of(k0 + 4 * key4 + e, use);
        kr[i][e] = *(const f32x4*)(kc + sl + 4 * d4);
        vr[i][e] = *(const f32x4*)(vc + sl + 4 * d4);
        ku[i][e] = use;
      }
    }
  };
  auto store_tile = [&]() {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int b = tid + NT * i, key4 = b / DT4, d4 = b - key4 * DT4;
#pragma unroll
      for (int e = 0; e < 4; ++e) *(f32x4*)&ks[(4 * key4 + e) * KROW + 4 * d4] = ku[i][e] ? kr[i][e] : zero;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        *(f32x4*)&vt[(4 * d4 + r) * VROW + 4 * key4] =
            f32x4{ku[i][0] ? vr[i][0][r] : 0.f, ku[i][1] ? vr[i][1][r] : 0.f, ku[i][2] ? vr[i][2][r] : 0.f,
                  ku[i][3] ? vr[i][3][r] : 0.f};
    }
  };

  // online softmax of this lane's column: -m (running base-2 max, 0 before
  // the first tile), the lane's share of the sum, O^T rows 16 dt + 4 g + i
  float negm = 0.f, l = 0.f;
  f32x4 acc[MT];
#pragma unroll
  for (int dt = 0; dt < MT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int qpos0 = p0 + tq0;
  const int col_lim = min(p0 + col_tok, kmax - 1);  // last key the column may see

  if (t_lo < t_hi) {
    fill_bt(FAST ? (t_lo * BN) >> a.bs_shift : (t_lo * BN) / a.bs);
    load_tile(t_lo);
    store_tile();
    if (t_lo + 1 < t_hi) load_tile(t_lo + 1);
    __syncthreads();
    for (int kb = t_lo; kb < t_hi; ++kb) {
      const int k0 = kb * BN;
      f32x4 s[4];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[kt] = f32x4{negm, negm, negm, negm};
#pragma unroll
      for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const f32x4 k4 = *(const f32x4*)&ks[(16 * kt + c) * KROW + 16 * m + 4 * g];
#pragma unroll
          for (int r = 0; r < 4; ++r) s[kt] = mfma_f32_k4(k4[r], qreg[m][r], s[kt]);
        }
      // only tiles that cross the causal diagonal or the last key are masked
      if (!(k0 + BN - 1 <= qpos0 && k0 + BN <= kmax)) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k0 + 16 * kt + 4 * g + r > col_lim) s[kt][r] = kNegInf;
      }
      float mx = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) mx = fmaxf(mx, fmaxf(fmaxf(s[kt][0], s[kt][1]), fmaxf(s[kt][2], s[kt][3])));
      mx = wave_max_groups_swap(mx);  // relative to m; finite on the piece's first tile
      const bool first = kb == t_lo;
      const bool grow = first || mx > kRescaleSlack;
      if (__any(grow)) {
        const float d = grow ? mx : 0.f;  // the max moves up by d
        if (!first) {
          const float alpha = fast_exp2(-d);
          l *= alpha;
#pragma unroll
          for (int dt = 0; dt < MT; ++dt) acc[dt] *= alpha;
        }
        negm -= d;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) s[kt] -= d;
      }
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s[kt][r] = fast_exp2(s[kt][r]);
          l += s[kt][r];
        }
#pragma unroll
      for (int dt = 0; dt < MT; ++dt)
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) {
          const f32x4 v4 = *(const f32x4*)&vt[(16 * dt + c) * VROW + 16 * kt + 4 * g];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[dt] = mfma_f32_k4(v4[r], s[kt][r], acc[dt]);
        }
      __syncthreads();  // every wavefront is done with tile kb
      if (kb + 1 < t_hi) {
        store_tile();
        if (kb + 2 < t_hi) load_tile(kb + 2);
      }
      __syncthreads();
    }
  }
  if (bad) flag_error(a.err, IR_ERR_BLOCK_RANGE);
  const float lsum = wave_sum_groups_swap(l);
  float* orow = (float*)a.out + (int64_t)(q_lo + col_tok) * a.o_tok + (int64_t)col_head * a.o_head;
  if (nparts == 1) {
    if (!col_ok) return;
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
    for (int dt = 0; dt < MT; ++dt) *(f32x4*)(orow + 16 * dt + 4 * g) = acc[dt] * inv;
    return;
  }

  // ---- a piece of a cut item: its partial rows (device scope) and arrival;
  // the last piece to arrive merges all of them in part order, its own from
  // registers (the same arithmetic whichever piece arrives last)
  const __amdgpu_buffer_rsrc_t r_o = dev_rsrc(a.ws_o), r_ml = dev_rsrc(a.ws_ml);
  const int row_step = a.num_kv_heads * kF32Cols;               // rows between parts of one item
  const int row_col = (pbase * a.num_kv_heads + kvh) * kF32Cols + j;  // part 0, this column
  {
    const int row = row_col + part * row_step;
#pragma unroll
    for (int dt = 0; dt < MT; ++dt) store_dev4(r_o, (row * D + 16 * dt + 4 * g) * 4, acc[dt]);
    if (g == 0) store_dev2(r_ml, row * 8, f32x2{-negm, lsum});
  }
  __shared__ int s_last;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int32_t* ctr = a.counters + pbase * a.num_kv_heads + kvh;
  if (tid == 0) s_last = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nparts - 1;
  __syncthreads();
  if (!s_last) return;
  f32x4 o_run[MT];
  float m_run = kNegInf, l_run = 0.f;
#pragma unroll
  for (int dt = 0; dt < MT; ++dt) o_run[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int p = 0; p < nparts; ++p) {
    f32x4 op[MT];
    float mp, lp;
    if (p == part) {
      mp = -negm;
      lp = lsum;
#pragma unroll
      for (int dt = 0; dt < MT; ++dt) op[dt] = acc[dt];
    } else {
      const int row = row_col + p * row_step;
      const f32x2 ml = load_dev2(r_ml, row * 8);
      mp = ml[0];
      lp = ml[1];
#pragma unroll
      for (int dt = 0; dt < MT; ++dt) op[dt] = load_dev4(r_o, (row * D + 16 * dt + 4 * g) * 4);
    }
    // a part without keys has max -inf: its weight is exp2(-inf) = 0, and
    // fmaxf keeps an (-inf) - (-inf) exponent from becoming NaN
    const float mn = fmaxf(m_run, mp);
    const float wa = fast_exp2(fmaxf(m_run - mn, -1e30f)), wb = fast_exp2(fmaxf(mp - mn, -1e30f));
    l_run = wa * l_run + wb * lp;
#pragma unroll
    for (int dt = 0; dt < MT; ++dt) o_run[dt] = wa * o_run[dt] + wb * op[dt];
    m_run = mn;
  }
  if (col_ok) {
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
    for (int dt = 0; dt < MT; ++dt) *(f32x4*)(orow + 16 * dt + 4 * g) = o_run[dt] * inv;
  }
  if (tid == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The fp32 launch: the step's K/V write (when given) as its own launch first,
// then one workgroup per plan entry, or per (query block, KV head, sequence)
// unplanned.
template <int D>
int launch_prefill_f32(PrefillArgs a, hipStream_t s) {
  if (a.k_new != nullptr) {
    const int rc = ir_kv_scatter(a.k_new, a.kn_tok, a.kn_head, a.v_new, a.vn_tok, a.vn_head, (void*)a.kc,
                                 (void*)a.vc, a.c_slot, a.c_head, a.num_blocks * a.bs, a.write_slots, a.n_write,
                                 a.num_kv_heads, D, IR_DTYPE_F32, a.err, (ir_stream_t)s);
    if (rc != IR_OK) return rc;
  }
  const int64_t grid = a.items ? a.n_items_grid : (int64_t)a.n_qblocks * a.num_kv_heads * a.num_seqs;
  if (grid <= 0) return ok();
  if (grid > 0x7fffffff) return fail(IR_EINVAL, "ir_paged_prefill: grid of %lld workgroups too large", (long long)grid);
  const int64_t slots = a.num_blocks * a.bs;
  const bool fast = a.bs_shift >= 0 && slots < (1 << 23) && a.c_slot < (1 << 23) &&
                    (slots * a.c_slot + a.c_head * a.num_kv_heads) < ((int64_t)1 << 31);
  if (fast)
    hipLaunchKernelGGL((paged_prefill_f32_kernel<D, true>), dim3((unsigned)grid), dim3(kF32Threads), 0, s, a);
  else
    hipLaunchKernelGGL((paged_prefill_f32_kernel<D, false>), dim3((unsigned)grid), dim3(kF32Threads), 0, s, a);
  return check_launch("ir_paged_prefill");
}

// ---------------------------------------------------------------- plan
//
// The dispatcher hands workgroup i to the first CU with room, in index order,
// so issuing the heaviest work first is the longest-processing-time rule. But
// an order cannot shorten the heaviest item itself, which bounds the call when
// one sequence's prefix is much longer than the rest. The plan therefore cuts
// every item heavier than 1.5x the mean load of a workgroup slot (and than
// kMinPieceTiles) into pieces of at most that threshold, at most kMaxParts per
// item and at most the plan's piece capacity in all (the smallest threshold
// that fits it, found by bisection). Measured on 8 chunks of 512 tokens after
// prefixes of U{0..8192} keys (per-workgroup timestamps): a workgroup costs ~7
// us plus ~2.2 us per 64-key tile while sharing its CU, and cutting at the
// mean (the longest item, 99 tiles, against a mean of 75) made the call 10%
// slower -- the pieces' fixed costs and merges outweighed a tail the
// heaviest-first order had mostly filled -- so only items well above the mean
// are cut.
//
// Placement. The dispatcher hands workgroup i to XCD i mod X, and each XCD
// has its own L2. It also dispatches in index order: an XCD without room for
// its next workgroup holds up the workgroups behind it for every XCD, so each
// run of X consecutive workgroups must carry similar work (placing each
// (sequence, KV head) on one XCD by cutting a cost line into X segments cut
// the fetched bytes of 8 x 512-token chunks by 27% but made the call 17%
// slower). Within that constraint the plan keeps a shared prefix in one L2:
// every query block of a sequence walks the same K/V tiles of its KV head,
// and sequences whose block tables begin with the same block share a cached
// prefix (the prefix cache hands each of them the same blocks for it). Share
// groups are runs of consecutive sequences whose first block ids are equal
// (each with at least one cached block). When the KV heads H divide X, a
// piece's H workgroups fill one of S = X / H slots of H consecutive XCDs in a
// row of X workgroups; every group keeps one slot (groups ranked by cost --
// tiles + kPieceFixed per workgroup -- and dealt to slots in snake order), each
// slot's pieces run heaviest first (counting sort over kXcdBuckets weight
// ranges), and row r holds the r-th piece of every slot, so head h of a group
// always runs on the same XCD. When the slots' costs differ by more than 10%,
// a slot would overflow the grid, there is one group, or the call is too
// large for the placement's LDS tables, the pieces keep one global
// heaviest-first order (kPlanBuckets weight ranges), a piece's heads on
// consecutive workgroups -- which already keeps head h on XCD h mod X when X
// divides H.
//
// One workgroup builds it once per step (every layer shares the metadata) and
// clears the arrival counters. Each thread owns a contiguous run of items, so
// the pieces' partial-row indices come from a deterministic scan; only the
// position of equal-weight pieces in the order varies, which changes the
// schedule, never a result bit.

constexpr int kPlanThreads = 1024;
constexpr int kPlanBuckets = 2048;  // weight ranges of the global order
constexpr int kXcdBuckets = 256;    // weight ranges of each XCD's order
constexpr int kMaxXcds = 16;
constexpr int kStartSize = kMaxXcds * kXcdBuckets + 1;
static_assert(kStartSize >= kPlanBuckets + 1, "bucket table too small for the global order");
constexpr int kMaxParts = 16;      // pieces per item (8-bit field)
constexpr int kMinPieceTiles = 8;  // items of at most this many key tiles are never cut
constexpr int kPlanWeightCache = 8192;  // items whose weights the plan keeps in LDS
constexpr int kPlaceSeqs = kPlanThreads;  // sequences the placement handles (one per thread)
constexpr int kPieceFixed = 3;  // a workgroup's fixed cost in key tiles (~7 us against ~2.2 us a tile)

struct PlanArgs {
  const int32_t* cu_q;
  const int32_t* q_start;
  const int32_t* bt;  // block tables: the first id of each row groups shared prefixes
  int64_t bt_stride;
  int num_seqs, total_q, n_qblocks, tq, cap, bs;  // cap: keys the block tables hold
  int num_kv_heads, slots, cap_pieces, xcds;      // slots: workgroups resident on the device at once
  int share_groups;   // place share groups on slots of XCDs (else one global order)
  int entries;        // workgroups of a planned call
  int2* items;        // [entries]
  int32_t* counters;  // [cap_pieces * num_kv_heads]
};

// 64-key tiles the workgroups of item (seq * n_qblocks + block) walk, following
// paged_prefill_kernel's bounds; -1 when they return without work (an item
// that only flags bad metadata weighs 0).
__device__ int prefill_item_weight(const PlanArgs& a, int item) {
  const int seq = item / a.n_qblocks, tb = item - seq * a.n_qblocks;
  const int q_lo = a.cu_q[seq], q_len = a.cu_q[seq + 1] - q_lo;
  if (q_lo < 0 || q_len < 0 || (int64_t)q_lo + q_len > a.total_q) return tb == 0 ? 0 : -1;
  const int tq0 = tb * a.tq;
  if (tq0 >= q_len) return -1;
  const int p0 = max(0, min(a.q_start[seq], a.cap));
  const int64_t kmax = min((int64_t)a.cap, (int64_t)p0 + min(q_len, tq0 + a.tq));
  return (int)((kmax + 63) / 64);
}

__device__ __forceinline__ int pieces_of(int w, int T) {
  return w > T ? min(kMaxParts, (w + T - 1) / T) : (w >= 0 ? 1 : 0);
}

// Block-wide sum / max over kPlanThreads threads (every thread gets the result).
__device__ int64_t plan_sum(int64_t x, int64_t* red) {
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  int64_t t = 0;
  for (int i = 0; i < kPlanThreads / 64; ++i) t += red[i];
  return t;
}

__device__ int64_t plan_max(int64_t x, int64_t* red) {
  for (int o = 32; o > 0; o >>= 1) x = max(x, (int64_t)__shfl_xor(x, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  int64_t t = red[0];
  for (int i = 1; i < kPlanThreads / 64; ++i) t = max(t, red[i]);
  return t;
}

// Exclusive prefix sum of x over the block's threads in thread order (buf:
// kPlanThreads + 1 entries); *total receives the sum. One wavefront scans runs
// of kPlanThreads / 64 values per lane.
__device__ int64_t plan_scan(int64_t x, int64_t* buf, int64_t* total) {
  const int tid = threadIdx.x, lane = tid & 63;
  buf[tid] = x;
  __syncthreads();
  if (tid < 64) {
    constexpr int kRun = kPlanThreads / 64;
    int64_t sum = 0;
    for (int k = 0; k < kRun; ++k) sum += buf[lane * kRun + k];
    int64_t incl = sum;
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    int64_t r = incl - sum;
    for (int k = 0; k < kRun; ++k) {
      const int64_t v = buf[lane * kRun + k];
      buf[lane * kRun + k] = r;
      r += v;
    }
    if (lane == 63) buf[kPlanThreads] = incl;
  }
  __syncthreads();
  const int64_t r = buf[tid];
  *total = buf[kPlanThreads];
  __syncthreads();
  return r;
}

// In-place exclusive scan of counts[0 .. len) by one wavefront (len <= 64 *
// runs); the caller synchronises around it.
__device__ void plan_scan_counts(int* counts, int len) {
  const int lane = threadIdx.x & 63;
  const int run = (len + 63) / 64;
  const int b_lo = min(len, lane * run), b_hi = min(len, b_lo + run);
  int sum = 0;
  for (int i = b_lo; i < b_hi; ++i) sum += counts[i];
  int incl = sum;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o);
    if (lane >= o) incl += y;
  }
  int r = incl - sum;
  for (int i = b_lo; i < b_hi; ++i) {
    const int cnt = counts[i];
    counts[i] = r;
    r += cnt;
  }
}

__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(PlanArgs a) {
  __shared__ int start[kStartSize];
  __shared__ int64_t red[kPlanThreads / 64];
  __shared__ int64_t scan[kPlanThreads + 1];
  __shared__ int w_cache[kPlanWeightCache];
  __shared__ int64_t seq_cost[kPlaceSeqs + 1];  // cost before each sequence's first item
  __shared__ int seq_gid[kPlaceSeqs];           // share group of each sequence
  __shared__ int glead[kPlaceSeqs + 1];         // first sequence of each group, then num_seqs
  __shared__ int64_t gcost[kPlaceSeqs];         // cost of each group
  __shared__ int gslot[kPlaceSeqs];             // slot of each group
  __shared__ unsigned long long slot_cost[kMaxXcds];
  __shared__ int slot_base[kMaxXcds + 1];
  __shared__ int s_place;
  const int tid = threadIdx.x;
  const int H = a.num_kv_heads;
  const int n = a.num_seqs * a.n_qblocks;
  const int per = (n + kPlanThreads - 1) / kPlanThreads;
  const int i_lo = min(n, tid * per), i_hi = min(n, i_lo + per);
  // the items' weights are read from global metadata once when they fit LDS
  const bool cached = n <= kPlanWeightCache;
  auto weight = [&](int i) { return cached ? w_cache[i] : prefill_item_weight(a, i); };

  int64_t tot = 0, wm = 0;
  for (int i = i_lo; i < i_hi; ++i) {
    const int w = prefill_item_weight(a, i);
    if (cached) w_cache[i] = w;
    tot += max(w, 0);
    wm = max(wm, (int64_t)w);
  }
  const int64_t total = plan_sum(tot, red);
  const int wmax = (int)plan_max(wm, red);
  // the cut threshold: the mean load of a workgroup slot, raised until the
  // pieces of the cut items fit the plan's capacity
  int lo = (int)max((int64_t)kMinPieceTiles, (total * H * 3 + 2 * a.slots - 1) / (2 * a.slots));
  int hi = max(lo, wmax);
  while (lo < hi) {
    const int mid = lo + (hi - lo) / 2;
    int64_t cnt = 0;
    for (int i = i_lo; i < i_hi; ++i) {
      const int w = weight(i);
      if (w > mid) cnt += pieces_of(w, mid);
    }
    if (plan_sum(cnt, red) <= a.cap_pieces) hi = mid;
    else lo = mid + 1;
  }
  const int T = lo;
  auto piece_info = [](int np, int p, int pb) { return np > 1 ? np | (p << 8) | (pb << 16) : 1; };

  // first partial-row piece of each cut item: exclusive scan over the runs
  int64_t mine = 0, all = 0;
  for (int i = i_lo; i < i_hi; ++i) {
    const int np = pieces_of(weight(i), T);
    if (np > 1) mine += np;
  }
  const int pb_run = (int)plan_scan(mine, scan, &all);

  // ---- slots: share groups and their costs
  const int X = a.xcds;
  const int S = H < X && X % H == 0 ? X / H : 1;
  // uniform over the block: every input of this test is
  const bool may_place =
      a.share_groups && S > 1 && S <= kMaxXcds && cached && a.num_seqs <= kPlaceSeqs && a.bt != nullptr;
  if (may_place) {
    int64_t cost_run = 0;
    for (int i = i_lo; i < i_hi; ++i) {
      const int w = weight(i), np = pieces_of(w, T);
      if (np > 0) cost_run += w + kPieceFixed * np;
    }
    int64_t line_total = 0;
    int64_t c = plan_scan(cost_run, scan, &line_total);
    for (int i = i_lo; i < i_hi; ++i) {
      if (i % a.n_qblocks == 0) seq_cost[i / a.n_qblocks] = c;
      const int w = weight(i), np = pieces_of(w, T);
      if (np > 0) c += w + kPieceFixed * np;
    }
    if (tid == 0) seq_cost[a.num_seqs] = line_total;
    // sequence tid starts a group unless its first block is the previous one's
    int flag = 0;
    if (tid < a.num_seqs) {
      auto first_block = [&](int q) {
        return a.q_start[q] >= a.bs && a.cap >= a.bs ? a.bt[(int64_t)q * a.bt_stride] : -1;
      };
      const int f = first_block(tid);
      flag = tid == 0 || f < 0 || f != first_block(tid - 1);
    }
    int64_t ngroups = 0;
    const int gid = (int)plan_scan(flag, scan, &ngroups) + flag - 1;
    if (tid < a.num_seqs) {
      seq_gid[tid] = gid;
      if (flag) glead[gid] = tid;
    }
    if (tid == 0) glead[ngroups] = a.num_seqs;
    if (tid < kMaxXcds) slot_cost[tid] = 0;
    __syncthreads();
    if (tid < ngroups) gcost[tid] = seq_cost[glead[tid + 1]] - seq_cost[glead[tid]];
    __syncthreads();
    // rank of group tid (heavier first, ties by index), dealt to the slots in
    // snake order: 0, 1, .., S-1, S-1, .., 0, 0, ..
    if (tid < ngroups) {
      const int64_t mine_c = gcost[tid];
      int rank = 0;
      for (int o = 0; o < ngroups; ++o) rank += gcost[o] > mine_c || (gcost[o] == mine_c && o < tid);
      const int k = rank % S;
      const int sl = (rank / S) & 1 ? S - 1 - k : k;
      gslot[tid] = sl;
      atomicAdd(&slot_cost[sl], (unsigned long long)mine_c);
    }
    for (int k = tid; k < kStartSize; k += kPlanThreads) start[k] = 0;
    if (tid == 0) s_place = ngroups > 1;
    __syncthreads();
    // the slots' costs within 10% of their mean
    if (tid < S && (int64_t)slot_cost[tid] * 10 * S > line_total * 11) s_place = 0;
    __syncthreads();
  }
  auto xbucket = [&](int pw) { return (int)((int64_t)(wmax - pw) * kXcdBuckets / ((int64_t)wmax + 1)); };
  if (may_place && s_place) {
    for (int i = i_lo; i < i_hi; ++i) {
      const int w = weight(i), np = pieces_of(w, T);
      if (np > 0) atomicAdd(&start[gslot[seq_gid[i / a.n_qblocks]] * kXcdBuckets + xbucket((w + np - 1) / np)], np);
    }
    __syncthreads();
    if (tid < 64) plan_scan_counts(start, S * kXcdBuckets + 1);
    __syncthreads();
    if (tid <= S) slot_base[tid] = start[tid * kXcdBuckets];
    __syncthreads();
    // every slot's pieces must fit the grid's rows
    if (tid < S && slot_base[tid + 1] - slot_base[tid] > a.entries / X) s_place = 0;
    __syncthreads();
  }
  const bool place = may_place && s_place;

  if (place) {
    // row r, slot sl: the r-th heaviest piece of the slot, KV head h on XCD
    // sl * H + h; entries past a slot's pieces are empty
    for (int k = tid; k < a.entries; k += kPlanThreads) {
      const int sl = (k % X) / H;
      if (k / X >= slot_base[sl + 1] - slot_base[sl]) a.items[k] = make_int2(-1, 0);
    }
    int pb = pb_run;
    for (int i = i_lo; i < i_hi; ++i) {
      const int w = weight(i), np = pieces_of(w, T);
      if (np == 0) continue;
      const int sl = gslot[seq_gid[i / a.n_qblocks]];
      const int r0 = atomicAdd(&start[sl * kXcdBuckets + xbucket((w + np - 1) / np)], np) - slot_base[sl];
      for (int p = 0; p < np; ++p)
        for (int h = 0; h < H; ++h) a.items[(r0 + p) * X + sl * H + h] = make_int2(i * H + h, piece_info(np, p, pb));
      if (np > 1) pb += np;
    }
  } else {
    // one global heaviest-first order of the pieces; bucket 0 holds the heaviest
    for (int k = tid; k <= kPlanBuckets; k += kPlanThreads) start[k] = 0;
    __syncthreads();
    auto bucket = [&](int pw) { return (int)((int64_t)(wmax - pw) * kPlanBuckets / ((int64_t)wmax + 1)); };
    for (int i = i_lo; i < i_hi; ++i) {
      const int w = weight(i);
      const int np = pieces_of(w, T);
      if (np > 0) atomicAdd(&start[bucket((w + np - 1) / np)], np);
    }
    __syncthreads();
    if (tid < 64) plan_scan_counts(start, kPlanBuckets + 1);  // start[kPlanBuckets] = pieces in all
    __syncthreads();
    const int used = start[kPlanBuckets];
    __syncthreads();
    int pb = pb_run;
    for (int i = i_lo; i < i_hi; ++i) {
      const int w = weight(i);
      const int np = pieces_of(w, T);
      if (np == 0) continue;
      const int pos = atomicAdd(&start[bucket((w + np - 1) / np)], np);
      for (int p = 0; p < np; ++p)
        for (int h = 0; h < H; ++h) a.items[(pos + p) * H + h] = make_int2(i * H + h, piece_info(np, p, pb));
      if (np > 1) pb += np;
    }
    for (int k = used * H + tid; k < a.entries; k += kPlanThreads) a.items[k] = make_int2(-1, 0);
  }
  for (int k = tid; k < a.cap_pieces * H; k += kPlanThreads) a.counters[k] = 0;
}

// Tuning knobs, read once per process: IR_PREFILL_WAVES (4 or 8) forces the
// workgroup size, IR_PREFILL_RING2 (1 or 0) forces or forbids the 2-deep ring,
// IR_PREFILL_CUTS=0 keeps the plan from cutting items (order only).
struct PrefillKnobs {
  int waves = 0;   // 0: 4, or 8 when 4 cannot hold a token's query heads
  int ring2 = -1;  // -1: the default (2-deep)
  bool cuts = true;
  bool split = true;  // a grid no larger than the CUs: 8 wavefronts of one column tile
  PrefillKnobs() {
    if (const char* e = getenv("IR_PREFILL_WAVES")) waves = atoi(e) == 8 ? 8 : 4;
    if (const char* e = getenv("IR_PREFILL_RING2")) ring2 = atoi(e) == 1 ? 1 : 0;
    if (const char* e = getenv("IR_PREFILL_CUTS")) cuts = atoi(e) != 0;
    if (const char* e = getenv("IR_PREFILL_SPLIT")) split = atoi(e) != 0;
  }
};

const PrefillKnobs& prefill_knobs() {
  static const PrefillKnobs k;
  return k;
}

// XCDs the plan lays its grid out for (1: the device has one, or more than
// the placement's tables hold).
int plan_xcds() {
  const int x = device_xcds();
  return x > 1 && x <= kMaxXcds ? x : 1;
}

// Workgroup shape and schedule of a prefill call, from its shapes alone (the
// plan and every layer's call agree on it): 4 wavefronts (128 query columns)
// on the 2-deep ring (the 3-deep ring only on request: it measured slower for
// every call shape, 9-21% on grids of fewer than two workgroups per CU); 8
// wavefronts (256 columns) when a token's query heads need more than 128
// columns or on request. `slots`: workgroups resident at once.
struct PrefillGeometry {
  int nw, tq, n_qblocks, sched, slots, cols;  // cols: query columns (token x head) of a work item
};

PrefillGeometry prefill_geometry(int max_q_len, int n_rep) {
  const PrefillKnobs& k = prefill_knobs();
  PrefillGeometry g;
  g.nw = (n_rep > PShape<128, 4>::COLS || k.waves == 8) ? 8 : 4;
  g.tq = (g.nw == 4 ? PShape<128, 4>::COLS : PShape<128, 8>::COLS) / n_rep;
  g.n_qblocks = (max_q_len + g.tq - 1) / g.tq;
  const int cus = device_cus();
  // 8 wavefronts always take the 2-deep ring (224 registers; their 3-deep
  // lockstep form needs more than 256 and spilled)
  const bool ring2 = g.nw == 8 || k.ring2 != 0;
  g.sched = ring2 ? kRing2 : kLockstep;
  g.slots = ring2 && g.nw == 4 ? 2 * cus : cus;
  g.cols = 32 * g.nw;
  return g;
}

// The fp32 kernel's items: 64 columns, two workgroups resident per CU
// (n_rep <= kF32Cols).
PrefillGeometry prefill_geometry_f32(int max_q_len, int n_rep) {
  PrefillGeometry g;
  g.nw = 4;
  g.tq = kF32Cols / n_rep;
  g.n_qblocks = (max_q_len + g.tq - 1) / g.tq;
  g.sched = kRing2;
  g.slots = 2 * device_cus();
  g.cols = kF32Cols;
  return g;
}

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

// Plan layout: items [entries] int2 (one per workgroup of a planned call),
// counters [cap_pieces * H_kv] int32, (max, sum) [cap_pieces * H_kv * cols]
// fp32 x 2, partial outputs [.. * D] fp32. At most items + cap_pieces pieces
// exist, each on H_kv workgroups; with X > 1 XCDs the grid holds 1.5x that,
// rounded to X, so an XCD may take more pieces than the mean.
struct PlanLayout {
  int64_t entries, cap_pieces, cols;
  int64_t off_ctr, off_ml, off_o, total;
};

PlanLayout plan_layout(const PrefillGeometry& g, int num_seqs, int num_kv_heads, int head_dim) {
  PlanLayout l;
  l.cols = g.cols;
  l.cap_pieces = (g.slots + num_kv_heads - 1) / num_kv_heads;
  const int64_t wgs = ((int64_t)num_seqs * g.n_qblocks + l.cap_pieces) * num_kv_heads;
  const int x = plan_xcds();
  l.entries = x > 1 ? x * ((wgs * 3 / 2 + x - 1) / x) : wgs;
  l.off_ctr = align256(l.entries * 8);
  const int64_t rows = l.cap_pieces * num_kv_heads * l.cols;
  l.off_ml = l.off_ctr + align256(l.cap_pieces * num_kv_heads * 4);
  l.off_o = l.off_ml + align256(rows * 8);
  l.total = l.off_o + align256(rows * head_dim * 4);
  return l;
}

template <int DT, int D>
int launch_prefill(PrefillArgs a, int sched, hipStream_t s) {
  const int64_t grid = a.items ? a.n_items_grid : (int64_t)a.n_qblocks * a.num_kv_heads * a.num_seqs;
  if (grid <= 0) return ok();
  if (grid > 0x7fffffff) return fail(IR_EINVAL, "ir_paged_prefill: grid of %lld workgroups too large", (long long)grid);
  a.n_work = grid;
  // a fused call's writers follow the attending workgroups (so the plan's
  // placement of those is unchanged): enough for every row x head x piece
  auto writers = [&](int nt) -> int64_t {
    if (a.k_new == nullptr) return 0;
    const int64_t pieces = a.n_write * a.num_kv_heads * (D / 8);
    return (pieces + (int64_t)nt * kWritePieces - 1) / ((int64_t)nt * kWritePieces);
  };
  // fast addressing: slot and stride below 2^23 (24-bit products) and every
  // element offset of the layer below 2^31
  const int64_t slots = a.num_blocks * a.bs;
  const bool fast = a.bs_shift >= 0 && slots < (1 << 23) && a.c_slot < (1 << 23) &&
                    (slots * a.c_slot + a.c_head * a.num_kv_heads) < ((int64_t)1 << 31);
  if (grid + writers(256) > 0x7fffffff) return fail(IR_EINVAL, "ir_paged_prefill: too many rows to write");
  const bool split = a.nw == 4 && !a.items && grid <= device_cus() && prefill_knobs().split;
  if (a.k_new != nullptr && !split) {
    // The write as its own launch first: a fused instance of the 4- and
    // 8-wavefront loops needs more registers than they have to spare (the
    // 4-wavefront one measured 10% slower, its spilling variant more).
    const int rc = ir_kv_scatter(a.k_new, a.kn_tok, a.kn_head, a.v_new, a.vn_tok, a.vn_head, (void*)a.kc,
                                 (void*)a.vc, a.c_slot, a.c_head, a.num_blocks * a.bs, a.write_slots, a.n_write,
                                 a.num_kv_heads, D, DT, a.err, (ir_stream_t)s);
    if (rc != IR_OK) return rc;
    a.k_new = a.v_new = nullptr;
  }
  const bool fused = a.k_new != nullptr;
#define IR_PREFILL_LAUNCH(NW_, CT_, SCHED_, NT_)                                                            \
  do {                                                                                                     \
    const dim3 block(NT_), g((unsigned)(grid + writers(NT_)));                                              \
    if (fast) hipLaunchKernelGGL((paged_prefill_kernel<DT, D, true, NW_, CT_, SCHED_>), g, block, 0, s, a);  \
    else hipLaunchKernelGGL((paged_prefill_kernel<DT, D, false, NW_, CT_, SCHED_>), g, block, 0, s, a);      \
  } while (0)
  if (split) {
    // every workgroup alone on its CU: its 128 columns on 8 wavefronts of one
    // 16-column tile (two per SIMD) rather than 4 of two, so each walks its
    // keys with half the per-wavefront work (the same arithmetic per column);
    // a fused call's writers and new-key loads fit its registers
    const dim3 block(PShape<D, 8, 1>::NT), g((unsigned)(grid + writers(PShape<D, 8, 1>::NT)));
    if (fused) {
      if (fast) hipLaunchKernelGGL((paged_prefill_kernel<DT, D, true, 8, 1, kRing2, true>), g, block, 0, s, a);
      else hipLaunchKernelGGL((paged_prefill_kernel<DT, D, false, 8, 1, kRing2, true>), g, block, 0, s, a);
    } else {
      if (fast) hipLaunchKernelGGL((paged_prefill_kernel<DT, D, true, 8, 1, kRing2>), g, block, 0, s, a);
      else hipLaunchKernelGGL((paged_prefill_kernel<DT, D, false, 8, 1, kRing2>), g, block, 0, s, a);
    }
  } else if (a.nw == 4 && sched == kRing2) {
    IR_PREFILL_LAUNCH(4, 2, kRing2, (PShape<D, 4>::NT));
  } else if (a.nw == 4) {
    IR_PREFILL_LAUNCH(4, 2, kLockstep, (PShape<D, 4>::NT));
  } else {
    IR_PREFILL_LAUNCH(8, 2, kRing2, (PShape<D, 8>::NT));
  }
#undef IR_PREFILL_LAUNCH
  return check_launch("ir_paged_prefill");
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int64_t ir_paged_prefill_plan_bytes(int num_seqs, int max_q_len, int num_q_heads, int num_kv_heads,
                                               int head_dim) {
  if (num_seqs <= 0 || max_q_len <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads ||
      num_q_heads / num_kv_heads > 256 || (head_dim != 64 && head_dim != 128))
    return 0;
  const int n_rep = num_q_heads / num_kv_heads;
  const int64_t b16 = plan_layout(prefill_geometry(max_q_len, n_rep), num_seqs, num_kv_heads, head_dim).total;
  if (n_rep > kF32Cols) return b16;
  return std::max(b16, plan_layout(prefill_geometry_f32(max_q_len, n_rep), num_seqs, num_kv_heads, head_dim).total);
}

extern "C" int ir_paged_prefill_plan_xcds(void) { return plan_xcds(); }

extern "C" int ir_paged_prefill(const void* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k_cache,
                                const void* v_cache, int64_t cache_slot_stride, int64_t cache_head_stride,
                                int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                                int max_blocks_per_seq, const int32_t* cu_seqlens_q, const int32_t* q_start,
                                int num_seqs, int total_q, int max_q_len, void* out, int64_t out_tok_stride,
                                int64_t out_head_stride, int num_q_heads, int num_kv_heads, int head_dim, float scale,
                                int dtype, void* plan, int64_t plan_bytes, const void* k_new,
                                int64_t k_new_tok_stride, int64_t k_new_head_stride, const void* v_new,
                                int64_t v_new_tok_stride, int64_t v_new_head_stride, const int64_t* write_slots,
                                int64_t n_write, int64_t src_row0, int32_t* err_flags, ir_stream_t stream) {
  IR_REQUIRE(dtype == IR_DTYPE_BF16 || dtype == IR_DTYPE_F16 || dtype == IR_DTYPE_F32,
             "ir_paged_prefill: unknown dtype %d", dtype);
  const bool f32 = dtype == IR_DTYPE_F32;
  const int eb = f32 ? 4 : 2;
  IR_REQUIRE(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_q_heads > 0 && num_kv_heads > 0 &&
                 block_size > 0 && max_blocks_per_seq >= 0 && num_blocks >= 0,
             "ir_paged_prefill: bad sizes");
  IR_REQUIRE(num_q_heads % num_kv_heads == 0, "ir_paged_prefill: num_q_heads %d not a multiple of num_kv_heads %d",
             num_q_heads, num_kv_heads);
  IR_REQUIRE(num_q_heads / num_kv_heads <= 256, "ir_paged_prefill: more than 256 query heads per KV head");
  if (f32 && num_q_heads / num_kv_heads > kF32Cols)
    return fail(IR_EUNSUPPORTED, "ir_paged_prefill: fp32 with more than %d query heads per KV head", kF32Cols);
  if (head_dim != 64 && head_dim != 128)
    return fail(IR_EUNSUPPORTED, "ir_paged_prefill: head_dim %d not supported (64, 128)", head_dim);
  IR_REQUIRE((int64_t)max_blocks_per_seq * block_size <= (int64_t)1 << 30,
             "ir_paged_prefill: block tables of %d x %d tokens exceed 2^30 keys", max_blocks_per_seq, block_size);
  IR_REQUIRE(scale > 0.f, "ir_paged_prefill: scale must be positive");
  if (num_seqs == 0 || total_q == 0 || max_q_len == 0) return ok();
  IR_REQUIRE(q && k_cache && v_cache && block_tables && cu_seqlens_q && q_start && out,
             "ir_paged_prefill: null pointer");
  // each output store is 4 elements: 8 bytes in 16-bit dtypes, 16 in fp32
  IR_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && ((uintptr_t)out % (4 * eb)) == 0,
             "ir_paged_prefill: q and caches must be 16-byte aligned, out %d-byte aligned", 4 * eb);
  IR_REQUIRE((q_tok_stride * eb) % 16 == 0 && (q_head_stride * eb) % 16 == 0 && (cache_slot_stride * eb) % 16 == 0 &&
                 (cache_head_stride * eb) % 16 == 0 && (out_tok_stride * eb) % (4 * eb) == 0 &&
                 (out_head_stride * eb) % (4 * eb) == 0,
             "ir_paged_prefill: q/cache strides must be multiples of 16 bytes, out strides of %d bytes", 4 * eb);
  PrefillArgs a;
  memset(&a, 0, sizeof(a));
  a.q = q;
  a.q_tok = q_tok_stride;
  a.q_head = q_head_stride;
  a.kc = k_cache;
  a.vc = v_cache;
  a.c_slot = cache_slot_stride;
  a.c_head = cache_head_stride;
  a.num_blocks = num_blocks;
  a.bs = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.c_slot32 = (int)(cache_slot_stride < (1 << 23) ? cache_slot_stride : 0);
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks_per_seq;
  a.cu_q = cu_seqlens_q;
  a.q_start = q_start;
  a.num_seqs = num_seqs;
  a.total_q = total_q;
  a.n_rep = num_q_heads / num_kv_heads;
  const PrefillGeometry geo = f32 ? prefill_geometry_f32(max_q_len, a.n_rep) : prefill_geometry(max_q_len, a.n_rep);
  a.nw = geo.nw;
  a.tq = geo.tq;
  a.n_qblocks = geo.n_qblocks;
  const int64_t n_items = (int64_t)num_seqs * a.n_qblocks;
  IR_REQUIRE(n_items * num_kv_heads <= 0x7fffffff, "ir_paged_prefill: %lld work items x %d KV heads",
             (long long)n_items, num_kv_heads);
  if (plan) {
    const PlanLayout ly = plan_layout(geo, num_seqs, num_kv_heads, head_dim);
    IR_REQUIRE(plan_bytes >= ly.total && ((uintptr_t)plan & 255u) == 0,
               "ir_paged_prefill: plan of %lld bytes (256-byte aligned) required, got %lld (build it with "
               "ir_paged_prefill_plan for the same metadata and shapes)",
               (long long)ly.total, (long long)plan_bytes);
    uint8_t* pl = (uint8_t*)plan;
    a.items = (const int2*)pl;
    a.counters = (int32_t*)(pl + ly.off_ctr);
    a.ws_ml = (float*)(pl + ly.off_ml);
    a.ws_o = (float*)(pl + ly.off_o);
    a.n_items_grid = ly.entries;
  }
  if (k_new != nullptr) {
    IR_REQUIRE(v_new && write_slots, "ir_paged_prefill: k_new given without v_new or write_slots");
    IR_REQUIRE(n_write >= 1 && src_row0 >= 0 && src_row0 + total_q <= n_write,
               "ir_paged_prefill: the new rows [%lld, %lld) must lie within the %lld rows written",
               (long long)src_row0, (long long)src_row0 + total_q, (long long)n_write);
    IR_REQUIRE(aligned16(k_new) && aligned16(v_new) && (k_new_tok_stride * eb) % 16 == 0 &&
                   (k_new_head_stride * eb) % 16 == 0 && (v_new_tok_stride * eb) % 16 == 0 &&
                   (v_new_head_stride * eb) % 16 == 0,
               "ir_paged_prefill: k_new / v_new must be 16-byte aligned with 16-byte strides");
    a.k_new = k_new;
    a.v_new = v_new;
    a.kn_tok = k_new_tok_stride;
    a.kn_head = k_new_head_stride;
    a.vn_tok = v_new_tok_stride;
    a.vn_head = v_new_head_stride;
    a.write_slots = write_slots;
    a.n_write = n_write;
    a.src_row0 = src_row0;
  }
  a.out = out;
  a.o_tok = out_tok_stride;
  a.o_head = out_head_stride;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.err = err_flags;
  hipStream_t s = (hipStream_t)stream;
  if (f32) return head_dim == 128 ? launch_prefill_f32<128>(a, s) : launch_prefill_f32<64>(a, s);
  if (dtype == IR_DTYPE_BF16)
    return head_dim == 128 ? launch_prefill<IR_DTYPE_BF16, 128>(a, geo.sched, s)
                           : launch_prefill<IR_DTYPE_BF16, 64>(a, geo.sched, s);
  return head_dim == 128 ? launch_prefill<IR_DTYPE_F16, 128>(a, geo.sched, s)
                         : launch_prefill<IR_DTYPE_F16, 64>(a, geo.sched, s);
}

extern "C" int ir_paged_prefill_plan(const int32_t* cu_seqlens_q, const int32_t* q_start, const int32_t* block_tables,
                                     int64_t bt_stride, int num_seqs, int total_q, int max_q_len,
                                     int max_blocks_per_seq, int block_size, int num_q_heads, int num_kv_heads,
                                     int head_dim, int flags, void* plan, int64_t plan_bytes, ir_stream_t stream) {
  IR_REQUIRE(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_q_heads > 0 && num_kv_heads > 0 &&
                 block_size > 0 && max_blocks_per_seq >= 0,
             "ir_paged_prefill_plan: bad sizes");
  IR_REQUIRE(num_q_heads % num_kv_heads == 0, "ir_paged_prefill_plan: num_q_heads %d not a multiple of num_kv_heads %d",
             num_q_heads, num_kv_heads);
  IR_REQUIRE((flags & ~(IR_PLAN_SHARE_GROUPS | IR_PLAN_F32)) == 0, "ir_paged_prefill_plan: unknown flags 0x%x",
             flags);
  const bool f32 = (flags & IR_PLAN_F32) != 0;
  if (f32 && num_q_heads / num_kv_heads > kF32Cols)
    return fail(IR_EUNSUPPORTED, "ir_paged_prefill_plan: fp32 with more than %d query heads per KV head", kF32Cols);
  IR_REQUIRE((int64_t)max_blocks_per_seq * block_size <= (int64_t)1 << 30,
             "ir_paged_prefill_plan: block tables of %d x %d tokens exceed 2^30 keys", max_blocks_per_seq,
             block_size);
  const int64_t need = ir_paged_prefill_plan_bytes(num_seqs, max_q_len, num_q_heads, num_kv_heads, head_dim);
  if (need == 0) return ok();  // nothing to plan
  IR_REQUIRE(plan && plan_bytes >= need && ((uintptr_t)plan & 255u) == 0,
             "ir_paged_prefill_plan: plan of %lld bytes (256-byte aligned) required, got %lld", (long long)need,
             (long long)plan_bytes);
  IR_REQUIRE(cu_seqlens_q && q_start && (block_tables || max_blocks_per_seq == 0),
             "ir_paged_prefill_plan: null pointer");
  IR_REQUIRE(bt_stride >= max_blocks_per_seq, "ir_paged_prefill_plan: bt_stride %lld below max_blocks_per_seq %d",
             (long long)bt_stride, max_blocks_per_seq);
  const int n_rep = num_q_heads / num_kv_heads;
  const PrefillGeometry geo = f32 ? prefill_geometry_f32(max_q_len, n_rep) : prefill_geometry(max_q_len, n_rep);
  const PlanLayout ly = plan_layout(geo, num_seqs, num_kv_heads, head_dim);
  IR_REQUIRE(ly.entries <= 0x7fffffff && ly.cap_pieces < 65536 &&
                 (int64_t)num_seqs * geo.n_qblocks * num_kv_heads <= 0x7fffffff &&
                 ly.cap_pieces * num_kv_heads * ly.cols * head_dim * 4 < ((int64_t)1 << 31),
             "ir_paged_prefill_plan: plan too large for this shape");
  PlanArgs p;
  p.cu_q = cu_seqlens_q;
  p.q_start = q_start;
  p.bt = max_blocks_per_seq > 0 ? block_tables : nullptr;
  p.bt_stride = bt_stride;
  p.num_seqs = num_seqs;
  p.total_q = total_q;
  p.n_qblocks = geo.n_qblocks;
  p.tq = geo.tq;
  p.cap = max_blocks_per_seq * block_size;
  p.bs = block_size;
  p.num_kv_heads = num_kv_heads;
  p.slots = geo.slots;
  p.cap_pieces = prefill_knobs().cuts ? (int)ly.cap_pieces : 0;
  p.xcds = plan_xcds();
  p.share_groups = (flags & IR_PLAN_SHARE_GROUPS) != 0;
  p.entries = (int)ly.entries;
  uint8_t* pl = (uint8_t*)plan;
  p.items = (int2*)pl;
  p.counters = (int32_t*)(pl + ly.off_ctr);
  hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, p);
  return check_launch("ir_paged_prefill_plan");
}
