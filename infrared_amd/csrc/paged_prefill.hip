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
// Work decomposition: one workgroup of NW wavefronts per (query block, KV
// head, sequence), dispatched heaviest first: in the order
// ir_paged_prefill_order builds once per step (all sequences' items by key
// tiles), or else a sequence's last query blocks first. NW
// is 8 (two per SIMD) unless that gives fewer workgroups than CUs; then 4 (one
// per SIMD, up to 512 registers), twice the workgroups with half the columns
// each, which shortens a small batch's critical path (4 x 256-token chunks:
// 19.0 -> 16.6 us; a large one runs twice as long with 4). A query block is
// TQ = 32 NW / n_rep tokens, so the block's (token, query head) pairs of the
// GQA group -- column j = token-in-block * n_rep + head -- fill 32 NW columns
// almost exactly (8 wavefronts, 7 heads: 36 tokens, 252 columns); wavefront w
// owns columns 32w .. 32w+31 (two 16-column tiles). Every column
// of a workgroup reads the same KV head, so each K/V element staged in LDS
// feeds 32 columns per wavefront read. The workgroup walks the keys in
// 64-key tiles staged in a 3-deep LDS ring: a later tile's global loads are
// in flight (in registers) while the current one is in the math, and are
// written to its LDS buffer a tile later. The workgroup runs in lockstep,
// one barrier per tile; 8-wavefront workgroups can instead run a ping-pong
// schedule (waves 4..7 half an iteration behind 0..3, so each SIMD overlaps
// one wave's MFMAs with the other's softmax), selected by
// IR_PREFILL_PINGPONG=1.
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
  const int32_t* order;  // [num_seqs * n_qblocks] items (seq * n_qblocks + block), or null
};

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
template <int DT, int D, bool FAST, int NW, int CTW, bool PP>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW == 8 ? 2 : 1)))
void paged_prefill_kernel(PrefillArgs a) {
  typedef PShape<D, NW, CTW> S;
  constexpr int EB = 2;
  constexpr int CT = S::CT, BN = S::BN, NT = S::NT;
  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[3][BN * S::KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vs_lds[3][BN * S::KROW];
  __shared__ int32_t bt_lds[kBtCache];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;
  const int TQ = a.tq;

  // ---- which (query block, KV head, sequence): item order[i / H_kv] of the
  // heaviest-first order when one is given, else the last query blocks (most
  // keys within a sequence) first
  int tb, seq, kvh;
  if (a.order) {
    const int k = (int)(blockIdx.x / a.num_kv_heads);
    kvh = (int)(blockIdx.x - (unsigned)k * a.num_kv_heads);
    const int item = a.order[k];
    if (item < 0 || item >= a.num_seqs * a.n_qblocks) return;
    seq = item / a.n_qblocks;
    tb = item - seq * a.n_qblocks;
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
  // keys this block needs: up to its last query's position, within the table
  const int kmax = min(cap, p0 + min(q_len, tq0 + TQ));
  const int nkb = kmax > 0 && a.num_blocks > 0 ? (kmax + BN - 1) / BN : 0;

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
  // score MFMA yields base-2 exponents directly
  u32x4 qreg[CT][S::KS];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const Col col = column(ct);
    const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)(q_lo + (col.ok ? col.tok : 0)) * a.q_tok +
                           (int64_t)(col.ok ? col.head : 0) * a.q_head;
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks) {
      const u32x4 x = col.ok ? *(const u32x4*)(qrow + ks * 32 + 8 * g) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        qreg[ct][ks][e] = Elem<DT>::pack2(Elem<DT>::lo(x[e]) * a.scale_log2, Elem<DT>::hi(x[e]) * a.scale_log2);
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
    const int kk = in ? k : 0;
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
  auto load_regs = [&](int kb) {
    const int k0 = kb * BN;
    const int k_last = min(k0 + BN, kmax) - 1;
    const int last_blk = FAST ? k_last >> a.bs_shift : k_last / a.bs;
    // (the ping-pong schedule runs only on tables the cache holds whole: its
    // wave groups never meet at the same barrier for a refill)
    if constexpr (!PP)
      if (last_blk >= bt_base + kBtCache) fill_bt(FAST ? k0 >> a.bs_shift : k0 / a.bs);
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const int q = tid + NT * i;
      if (S::KCH % NT == 0 || q < S::KCH) {
        const int key = q / (D / 8), part = q % (D / 8);
        bool use;
        const int64_t sl = slot_of(k0 + key, use);
        kreg[i] = *(const u32x4*)(kc + sl + part * 8);
        vreg[i] = *(const u32x4*)(vc + sl + part * 8);
        kuse[i] = use;
      }
    }
  };
  // Registers -> LDS buffer `buf`: K and V tiles both row-major [64 keys][D]
  // (+32 bytes a row).
  auto store_regs = [&](int buf) {
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const int q = tid + NT * i;
      if (q < S::KCH) {
        const int key = q / (D / 8), part = q % (D / 8);
        *(u32x4*)&ks_lds[buf][key * S::KROW + part * 8] = zero_unless(kreg[i], kuse[i]);
        *(u32x4*)&vs_lds[buf][key * S::KROW + part * 8] = zero_unless(vreg[i], kuse[i]);
      }
    }
  };
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
    const bool first = kb == 0;
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
    const uint16_t* kn = ks_lds[(kb + 1) % 3];
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
    const uint16_t* vb_lds = vs_lds[kb % 3];
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

  // ---- walk the key tiles through a 3-deep LDS ring: tile kb (V) and tile
  // kb + 1 (K) are read while tile kb + 2 is written from registers and tile
  // kb + 3 is in flight from global memory
  auto tail = [&](int kb) {
    if (kb + 2 < nkb) store_regs((kb + 2) % 3);
    if (kb + 3 < nkb) load_regs(kb + 3);
    __syncthreads();
  };
  if constexpr (PP) {
    // ---- ping-pong schedule (8 wavefronts, two per SIMD). Each wavefront's
    // iteration i is a matrix half -- the scores of tile i and the PV product
    // of tile i - 1, 64 MFMAs -- and a vector half -- tile i's softmax, one
    // tile's LDS store and the next tile's global loads. Waves 4..7 start one
    // barrier later than waves 0..3, so on every SIMD one wavefront runs its
    // matrix half while the other runs its vector half (in lockstep the two
    // pipes mostly took turns). Barrier intervals: the leading group's halves
    // of iteration i are intervals 2i and 2i + 1, the following group's
    // 2i + 1 and 2i + 2. Tile t is read (K) in intervals 2t, 2t + 1 and (V)
    // 2t + 2, 2t + 3, so the leaders store their part of it in interval
    // 2t - 1 (iteration t - 1) and the followers in 2t - 2 (iteration t - 2);
    // the next tile for its buffer (t + 3) is first stored in interval
    // 2t + 4: a 3-deep ring suffices. Each wavefront keeps one tile's global
    // loads in flight, issued an iteration before their store.
    const bool lead = w < NW / 2;
    const int ahead = lead ? 1 : 2;  // the tile a wavefront stores in iteration i is i + ahead
    f32x4 sc[CT][4];                 // scores of the tile in flight through the iteration
    u32x4 pb[CT][2];                 // probabilities of the previous tile (PV operand)
    using E = Elem<DT>;
    constexpr int NQK = 4 * S::KS, NPV = 2 * S::DTL;
    // matrix half: S(i) = K(i) . Q^T starting from -m (QK), O^T += V^T(i-1) . P^T(i-1) (PV)
    auto matrix_half = [&](auto qk_tag, auto pv_tag, int i) {
      constexpr bool QK = decltype(qk_tag)::value, PVH = decltype(pv_tag)::value;
      const uint16_t* kb_lds = ks_lds[i % 3];
      const uint16_t* vb_lds = vs_lds[(i + 2) % 3];
      auto k_operand = [&](int t) {
        return *(const u32x4*)&kb_lds[((t % 4) * 16 + c) * S::KROW + (t / 4) * 32 + 8 * g];
      };
      auto v_operand = [&](int t) {
        return v_operand_tr(vb_lds, t);
      };
      if constexpr (QK) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) sc[ct][kt] = negm[ct];
      }
      constexpr int NT_ = NQK > NPV ? NQK : NPV;
      u32x4 kring[kOperandAhead], vring[kOperandAhead];
#pragma unroll
      for (int t = 0; t < kOperandAhead; ++t) {
        if constexpr (QK) kring[t] = k_operand(t);
        if constexpr (PVH) vring[t] = v_operand(t);
      }
#pragma unroll
      for (int t = 0; t < NT_; ++t) {
        if constexpr (QK) {
          if (t < NQK) {
            const u32x4 ka = kring[t % kOperandAhead];
            if (t + kOperandAhead < NQK) kring[t % kOperandAhead] = k_operand(t + kOperandAhead);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) sc[ct][t % 4] = mfma_k32<DT>(ka, qreg[ct][t / 4], sc[ct][t % 4]);
          }
        }
        if constexpr (PVH) {
          if (t < NPV) {
            const u32x4 va = vring[t % kOperandAhead];
            if (t + kOperandAhead < NPV) vring[t % kOperandAhead] = v_operand(t + kOperandAhead);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
              acc[ct][t % S::DTL] = mfma_k32<DT>(va, pb[ct][t / S::DTL], acc[ct][t % S::DTL]);
          }
        }
        // keep the steps in program order: hoisting every operand read to
        // the top would hold all of them in registers at once
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // vector half: tile i's mask, running max (the first tile sets it; later
    // ones move it past kRescaleSlack only), exponentials, P^T and the sums
    auto vector_half = [&](int i) {
      const int k0 = i * BN;
      if (!(k0 + BN - 1 <= qpos0 && k0 + BN <= kmax)) {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int kt = 0; kt < 4; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (k0 + kt * 16 + 4 * g + r > col_lim[ct]) sc[ct][kt][r] = kNegInf;
      }
      const bool first = i == 0;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        float mx = kNegInf;
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          mx = fmaxf(mx, fmaxf(fmaxf(sc[ct][kt][0], sc[ct][kt][1]), fmaxf(sc[ct][kt][2], sc[ct][kt][3])));
        mx = wave_max_groups_swap(mx);
        const bool grow = first || mx > kRescaleSlack;
        if (__any(grow)) {
          const float d = grow ? mx : 0.f;
          if (!first) {
            const float alpha = fast_exp2(-d);
            l[ct] *= alpha;
#pragma unroll
            for (int dt = 0; dt < S::DTL; ++dt) acc[ct][dt] *= alpha;
          }
          negm[ct] -= d;
#pragma unroll
          for (int kt = 0; kt < 4; ++kt) sc[ct][kt] -= d;
        }
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) sc[ct][kt][r] = fast_exp2(sc[ct][kt][r]);
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          pb[ct][st] = u32x4{E::pack2(sc[ct][2 * st][0], sc[ct][2 * st][1]),
                             E::pack2(sc[ct][2 * st][2], sc[ct][2 * st][3]),
                             E::pack2(sc[ct][2 * st + 1][0], sc[ct][2 * st + 1][1]),
                             E::pack2(sc[ct][2 * st + 1][2], sc[ct][2 * st + 1][3])};
#pragma unroll
          for (int e = 0; e < 4; ++e) l[ct] = sum2<DT>(pb[ct][st][e], l[ct]);
        }
      }
    };
    if (nkb > 0) {
      fill_bt(0);
      load_regs(0);
      store_regs(0);
      if (!lead && nkb > 1) {
        load_regs(1);
        store_regs(1);
      }
      if (ahead < nkb) load_regs(ahead);
      __syncthreads();
      if (!lead) __syncthreads();  // the followers start half an iteration later
      auto vector_and_memory = [&](int i) {
        const int st = i + ahead;
        if (st < nkb) store_regs(st % 3);
        if (st + 1 < nkb) load_regs(st + 1);
        vector_half(i);
      };
      // iteration 0 has no PV product, iteration nkb no scores: peeled
      matrix_half(std::true_type{}, std::false_type{}, 0);
      __syncthreads();
      vector_and_memory(0);
      __syncthreads();
      for (int i = 1; i < nkb; ++i) {
        matrix_half(std::true_type{}, std::true_type{}, i);
        __syncthreads();
        vector_and_memory(i);
        __syncthreads();
      }
      matrix_half(std::false_type{}, std::true_type{}, nkb);
      __syncthreads();
      __syncthreads();
      if (lead) __syncthreads();  // as many barriers as the followers
    }
  } else if (nkb > 0) {
    fill_bt(0);
    load_regs(0);
    store_regs(0);
    if (nkb > 1) {
      load_regs(1);
      store_regs(1);
    }
    if (nkb > 2) load_regs(2);
    __syncthreads();
    f32x4 sa[CT][4], sb[CT][4];
    zero_s(sa);
#pragma unroll
    for (int t = 0; t < 4 * S::KS; ++t) qk_step(ks_lds[0], t % 4, t / 4, sa);
    int kb = 0;
    // two tiles per trip so the score buffers swap roles without copies
    for (; kb + 2 < nkb; kb += 2) {
      step(std::true_type{}, kb, sa, sb);
      tail(kb);
      step(std::true_type{}, kb + 1, sb, sa);
      tail(kb + 1);
    }
    if (kb + 1 < nkb) {
      step(std::true_type{}, kb, sa, sb);
      tail(kb);
      step(std::false_type{}, kb + 1, sb, sa);
    } else {
      step(std::false_type{}, kb, sa, sb);
    }
  }
  if (bad) flag_error(a.err, IR_ERR_BLOCK_RANGE);

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
}

// ---------------------------------------------------------------- work order
//
// The dispatcher hands workgroup i to the first CU with room, in index order,
// so issuing the heaviest items first is the longest-processing-time rule: on
// a chunked prefill whose items outnumber the CUs (8 chunks of 512 tokens
// after prefixes of 2.5k-4k keys: 480 workgroups, 1 per CU) the busiest CU's
// share drops from 1.26x to 1.06x of the mean (tile counts, simulated). The
// order is built once per step (all layers share the metadata) by one
// workgroup: every (sequence, query block) item is weighed by the 64-key tiles
// its workgroup walks, and a counting sort over kOrderBuckets equal-width
// weight ranges writes the items heaviest range first; items with no query
// rows go last as -1. Workgroups write disjoint outputs, so the order (ties
// land in any order) never changes a result bit.

constexpr int kOrderThreads = 1024;
constexpr int kOrderBuckets = 2048;

struct OrderArgs {
  const int32_t* cu_q;
  const int32_t* q_start;
  int num_seqs, total_q, n_qblocks, tq, cap;  // cap: keys the block tables hold
  int32_t* order;                             // [num_seqs * n_qblocks]
};

// 64-key tiles the workgroups of item (seq * n_qblocks + block) walk, following
// paged_prefill_kernel's bounds; -1 when they return without work (an item
// that only flags bad metadata weighs 0).
__device__ int prefill_item_weight(const OrderArgs& a, int item) {
  const int seq = item / a.n_qblocks, tb = item - seq * a.n_qblocks;
  const int q_lo = a.cu_q[seq], q_len = a.cu_q[seq + 1] - q_lo;
  if (q_lo < 0 || q_len < 0 || (int64_t)q_lo + q_len > a.total_q) return tb == 0 ? 0 : -1;
  const int tq0 = tb * a.tq;
  if (tq0 >= q_len) return -1;
  const int p0 = max(0, min(a.q_start[seq], a.cap));
  const int64_t kmax = min((int64_t)a.cap, (int64_t)p0 + min(q_len, tq0 + a.tq));
  return (int)((kmax + 63) / 64);
}

__global__ __launch_bounds__(kOrderThreads) void prefill_order_kernel(OrderArgs a) {
  __shared__ int start[kOrderBuckets + 1];  // bucket kOrderBuckets: items without work
  __shared__ int wave_max[kOrderThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int n = a.num_seqs * a.n_qblocks;

  int wmax = 0;
  for (int i = tid; i < n; i += kOrderThreads) wmax = max(wmax, prefill_item_weight(a, i));
  for (int o = 32; o > 0; o >>= 1) wmax = max(wmax, __shfl_xor(wmax, o));
  if (lane == 0) wave_max[tid >> 6] = wmax;
  for (int i = tid; i <= kOrderBuckets; i += kOrderThreads) start[i] = 0;
  __syncthreads();
  wmax = 0;
  for (int i = 0; i < kOrderThreads / 64; ++i) wmax = max(wmax, wave_max[i]);
  // bucket 0 holds the heaviest weights
  auto bucket = [&](int wt) {
    return wt < 0 ? kOrderBuckets : (int)((int64_t)(wmax - wt) * kOrderBuckets / ((int64_t)wmax + 1));
  };
  for (int i = tid; i < n; i += kOrderThreads) atomicAdd(&start[bucket(prefill_item_weight(a, i))], 1);
  __syncthreads();
  // exclusive scan of the counts by the first wavefront: lane l owns a run of
  // consecutive buckets
  if (tid < 64) {
    constexpr int kRun = (kOrderBuckets + 1 + 63) / 64;
    const int lo = lane * kRun, hi = min(lo + kRun, kOrderBuckets + 1);
    int sum = 0;
    for (int i = lo; i < hi; ++i) sum += start[i];
    int incl = sum;
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    int run = incl - sum;
    for (int i = lo; i < hi; ++i) {
      const int cnt = start[i];
      start[i] = run;
      run += cnt;
    }
  }
  __syncthreads();
  for (int i = tid; i < n; i += kOrderThreads) {
    const int wt = prefill_item_weight(a, i);
    const int pos = atomicAdd(&start[bucket(wt)], 1);
    a.order[pos] = wt < 0 ? -1 : i;
  }
}

// Tuning knobs, read once per process: IR_PREFILL_WAVES (4 or 8) forces the
// workgroup shape, IR_PREFILL_PINGPONG=1 selects the ping-pong schedule.
struct PrefillKnobs {
  int waves = 0;  // 0: by grid size
  bool pingpong = false;
  PrefillKnobs() {
    if (const char* e = getenv("IR_PREFILL_WAVES")) waves = atoi(e) == 4 ? 4 : 8;
    if (const char* e = getenv("IR_PREFILL_PINGPONG")) pingpong = atoi(e) == 1;
  }
};

const PrefillKnobs& prefill_knobs() {
  static const PrefillKnobs k;
  return k;
}

// Workgroup shape of a prefill call: 8 wavefronts (256 query columns) unless
// that leaves CUs idle, then 4 (128 columns), twice the workgroups with half
// the work each.
struct PrefillGeometry {
  int nw, tq, n_qblocks;
};

PrefillGeometry prefill_geometry(int max_q_len, int n_rep, int num_kv_heads, int num_seqs) {
  const int tq8 = PShape<128, 8>::COLS / n_rep;
  const int64_t wgs8 = (int64_t)((max_q_len + tq8 - 1) / tq8) * num_kv_heads * num_seqs;
  const int forced = prefill_knobs().waves;
  // (4 wavefronts hold at most 128 query heads per KV head)
  const bool four = n_rep <= PShape<128, 4>::COLS && (forced ? forced == 4 : wgs8 < device_cus());
  PrefillGeometry g;
  g.nw = four ? 4 : 8;
  g.tq = (four ? PShape<128, 4>::COLS : PShape<128, 8>::COLS) / n_rep;
  g.n_qblocks = (max_q_len + g.tq - 1) / g.tq;
  return g;
}

template <int DT, int D>
int launch_prefill(const PrefillArgs& a, hipStream_t s) {
  const int64_t grid = (int64_t)a.n_qblocks * a.num_kv_heads * a.num_seqs;
  if (grid <= 0) return ok();
  if (grid > 0x7fffffff) return fail(IR_EINVAL, "ir_paged_prefill: grid of %lld workgroups too large", (long long)grid);
  // fast addressing: slot and stride below 2^23 (24-bit products) and every
  // element offset of the layer below 2^31
  const int64_t slots = a.num_blocks * a.bs;
  const bool fast = a.bs_shift >= 0 && slots < (1 << 23) && a.c_slot < (1 << 23) &&
                    (slots * a.c_slot + a.c_head * a.num_kv_heads) < ((int64_t)1 << 31);
  // ping-pong schedule on request (IR_PREFILL_PINGPONG=1), for 8-wavefront
  // workgroups whose block tables fit the block-id cache whole. Measured on
  // the 8 x 512-token workload: ahead of lockstep while V went through a
  // register transpose (235 vs 257 us), behind it with row-major V and
  // transpose reads (242 vs 225 us), so lockstep is the default.
  const bool pp = a.nw == 8 && a.max_blocks <= kBtCache && prefill_knobs().pingpong;
  if (a.nw == 4) {
    const dim3 block(PShape<D, 4>::NT);
    if (fast)
      hipLaunchKernelGGL((paged_prefill_kernel<DT, D, true, 4, 2, false>), dim3((unsigned)grid), block, 0, s, a);
    else
      hipLaunchKernelGGL((paged_prefill_kernel<DT, D, false, 4, 2, false>), dim3((unsigned)grid), block, 0, s, a);
  } else if (pp) {
    const dim3 block(PShape<D, 8>::NT);
    if (fast)
      hipLaunchKernelGGL((paged_prefill_kernel<DT, D, true, 8, 2, true>), dim3((unsigned)grid), block, 0, s, a);
    else
      hipLaunchKernelGGL((paged_prefill_kernel<DT, D, false, 8, 2, true>), dim3((unsigned)grid), block, 0, s, a);
  } else {
    const dim3 block(PShape<D, 8>::NT);
    if (fast)
      hipLaunchKernelGGL((paged_prefill_kernel<DT, D, true, 8, 2, false>), dim3((unsigned)grid), block, 0, s, a);
    else
      hipLaunchKernelGGL((paged_prefill_kernel<DT, D, false, 8, 2, false>), dim3((unsigned)grid), block, 0, s, a);
  }
  return check_launch("ir_paged_prefill");
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_paged_prefill(const void* q, int64_t q_tok_stride, int64_t q_head_stride, const void* k_cache,
                                const void* v_cache, int64_t cache_slot_stride, int64_t cache_head_stride,
                                int64_t num_blocks, int block_size, const int32_t* block_tables, int64_t bt_stride,
                                int max_blocks_per_seq, const int32_t* cu_seqlens_q, const int32_t* q_start,
                                int num_seqs, int total_q, int max_q_len, void* out, int64_t out_tok_stride,
                                int64_t out_head_stride, int num_q_heads, int num_kv_heads, int head_dim, float scale,
                                int dtype, const int32_t* order, int64_t order_len, int32_t* err_flags,
                                ir_stream_t stream) {
  IR_REQUIRE(dtype == IR_DTYPE_BF16 || dtype == IR_DTYPE_F16 || dtype == IR_DTYPE_F32,
             "ir_paged_prefill: unknown dtype %d", dtype);
  if (dtype == IR_DTYPE_F32)
    return fail(IR_EUNSUPPORTED, "ir_paged_prefill: fp32 is not supported (bf16, f16); use ir_paged_attention_masked");
  IR_REQUIRE(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_q_heads > 0 && num_kv_heads > 0 &&
                 block_size > 0 && max_blocks_per_seq >= 0 && num_blocks >= 0,
             "ir_paged_prefill: bad sizes");
  IR_REQUIRE(num_q_heads % num_kv_heads == 0, "ir_paged_prefill: num_q_heads %d not a multiple of num_kv_heads %d",
             num_q_heads, num_kv_heads);
  IR_REQUIRE(num_q_heads / num_kv_heads <= 256, "ir_paged_prefill: more than 256 query heads per KV head");
  if (head_dim != 64 && head_dim != 128)
    return fail(IR_EUNSUPPORTED, "ir_paged_prefill: head_dim %d not supported (64, 128)", head_dim);
  IR_REQUIRE((int64_t)max_blocks_per_seq * block_size <= (int64_t)1 << 30,
             "ir_paged_prefill: block tables of %d x %d tokens exceed 2^30 keys", max_blocks_per_seq, block_size);
  IR_REQUIRE(scale > 0.f, "ir_paged_prefill: scale must be positive");
  if (num_seqs == 0 || total_q == 0 || max_q_len == 0) return ok();
  IR_REQUIRE(q && k_cache && v_cache && block_tables && cu_seqlens_q && q_start && out,
             "ir_paged_prefill: null pointer");
  IR_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && ((uintptr_t)out & 7u) == 0,
             "ir_paged_prefill: q and caches must be 16-byte aligned, out 8-byte aligned");
  IR_REQUIRE((q_tok_stride * 2) % 16 == 0 && (q_head_stride * 2) % 16 == 0 && (cache_slot_stride * 2) % 16 == 0 &&
                 (cache_head_stride * 2) % 16 == 0 && (out_tok_stride * 2) % 8 == 0 && (out_head_stride * 2) % 8 == 0,
             "ir_paged_prefill: q/cache strides must be multiples of 16 bytes, out strides of 8 bytes");
  PrefillArgs a;
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
  const PrefillGeometry geo = prefill_geometry(max_q_len, a.n_rep, num_kv_heads, num_seqs);
  a.nw = geo.nw;
  a.tq = geo.tq;
  a.n_qblocks = geo.n_qblocks;
  const int64_t n_items = (int64_t)num_seqs * a.n_qblocks;
  IR_REQUIRE(n_items <= 0x7fffffff, "ir_paged_prefill: %lld work items", (long long)n_items);
  IR_REQUIRE(!order || order_len == n_items,
             "ir_paged_prefill: order holds %lld items, this call has %lld (build it with ir_paged_prefill_order "
             "for the same metadata and shapes)",
             (long long)order_len, (long long)n_items);
  a.order = order;
  a.out = out;
  a.o_tok = out_tok_stride;
  a.o_head = out_head_stride;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.err = err_flags;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == IR_DTYPE_BF16)
    return head_dim == 128 ? launch_prefill<IR_DTYPE_BF16, 128>(a, s) : launch_prefill<IR_DTYPE_BF16, 64>(a, s);
  return head_dim == 128 ? launch_prefill<IR_DTYPE_F16, 128>(a, s) : launch_prefill<IR_DTYPE_F16, 64>(a, s);
}

extern "C" int64_t ir_paged_prefill_order_len(int num_seqs, int max_q_len, int num_q_heads, int num_kv_heads) {
  if (num_seqs <= 0 || max_q_len <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads)
    return 0;
  const PrefillGeometry geo = prefill_geometry(max_q_len, num_q_heads / num_kv_heads, num_kv_heads, num_seqs);
  return (int64_t)num_seqs * geo.n_qblocks;
}

extern "C" int ir_paged_prefill_order(const int32_t* cu_seqlens_q, const int32_t* q_start, int num_seqs,
                                      int total_q, int max_q_len, int max_blocks_per_seq, int block_size,
                                      int num_q_heads, int num_kv_heads, int32_t* order, int64_t order_len,
                                      ir_stream_t stream) {
  IR_REQUIRE(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_q_heads > 0 && num_kv_heads > 0 &&
                 block_size > 0 && max_blocks_per_seq >= 0,
             "ir_paged_prefill_order: bad sizes");
  IR_REQUIRE(num_q_heads % num_kv_heads == 0, "ir_paged_prefill_order: num_q_heads %d not a multiple of num_kv_heads %d",
             num_q_heads, num_kv_heads);
  IR_REQUIRE((int64_t)max_blocks_per_seq * block_size <= (int64_t)1 << 30,
             "ir_paged_prefill_order: block tables of %d x %d tokens exceed 2^30 keys", max_blocks_per_seq,
             block_size);
  const int64_t need = ir_paged_prefill_order_len(num_seqs, max_q_len, num_q_heads, num_kv_heads);
  IR_REQUIRE(order_len == need, "ir_paged_prefill_order: order holds %lld items, this call has %lld",
             (long long)order_len, (long long)need);
  IR_REQUIRE(need <= 0x7fffffff, "ir_paged_prefill_order: %lld work items", (long long)need);
  if (need == 0) return ok();
  IR_REQUIRE(cu_seqlens_q && q_start && order, "ir_paged_prefill_order: null pointer");
  const PrefillGeometry geo = prefill_geometry(max_q_len, num_q_heads / num_kv_heads, num_kv_heads, num_seqs);
  OrderArgs a;
  a.cu_q = cu_seqlens_q;
  a.q_start = q_start;
  a.num_seqs = num_seqs;
  a.total_q = total_q;
  a.n_qblocks = geo.n_qblocks;
  a.tq = geo.tq;
  a.cap = max_blocks_per_seq * block_size;
  a.order = order;
  hipLaunchKernelGGL(prefill_order_kernel, dim3(1), dim3(kOrderThreads), 0, (hipStream_t)stream, a);
  return check_launch("ir_paged_prefill_order");
}
