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
// Work decomposition: one workgroup per (32-token query block, KV head, group
// of NW query heads of that KV head, sequence); heaviest query blocks (most
// keys) are dispatched first. Wavefront w owns query head w of the group and
// the block's 32 query tokens (two 16-token column tiles). The workgroup walks
// the keys in 64-key tiles staged in LDS, double buffered: the next tile's
// global loads are in flight (in registers) while the current one is in the
// math, and they are written to the other LDS buffer afterwards.
//   K tile : row-major [64 keys][D] (+16 bytes a row against bank conflicts);
//   V tile : transposed [D][64 keys] (+8 bytes a row), written from pairs of
//            keys, so one d column of 4 consecutive keys is one 8-byte read.
// Per tile a wavefront computes S^T = K . Q^T with 16x16x32 MFMA (rows = keys,
// columns = its query tokens; Q^T stays in registers for the whole walk), the
// online softmax in base 2 down each column (a lane owns one query column, so
// the running max/sum and the rescale are lane-local), and O^T += V^T . P^T
// where P^T is exactly the lane's own probabilities of the S^T tiles.
// Only tiles that cross the causal diagonal or the last key are masked.
//
// Parity: the one-shot softmax of infrared/model/layers.py:102-118 over the
// gathered history (infrared/model/triton_attention.py:110-129), streaming as
// in infrared/model/triton_attention.py:135-177; probabilities are rounded to
// the input dtype before the PV product, as softmax(...).to(q.dtype) does.
#include "attn_tile.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kBtCache = 1024;  // block ids staged in LDS per workgroup

struct PrefillArgs {
  const void* q;
  int64_t q_tok, q_head;  // elements
  const void* kc;
  const void* vc;
  int64_t c_slot, c_head;  // elements
  int64_t num_blocks;
  int bs;
  const int32_t* bt;
  int64_t bt_stride;
  int max_blocks;
  const int32_t* cu_q;     // [num_seqs + 1]
  const int32_t* q_start;  // [num_seqs]
  int num_seqs, total_q, n_qblocks;
  void* out;
  int64_t o_tok, o_head;  // elements
  int num_q_heads, num_kv_heads, n_rep, n_hgp;
  float scale_log2;
  int32_t* err;
};

template <int D, int NW>
struct PShape {
  static constexpr int TQ = 32;   // query tokens per workgroup (2 column tiles)
  static constexpr int BN = 64;   // keys per tile
  static constexpr int NT = NW * 64;
  static constexpr int KROW = D + 8;   // elements per K row in LDS
  static constexpr int VROW = BN + 4;  // elements per V^T row in LDS
  static constexpr int KCH = BN * D / 8;       // 16-byte K chunks per tile
  static constexpr int VPR = BN / 2 * D / 8;   // (key pair, 8 d) V chunks per tile
  static constexpr int KPT = (KCH + NT - 1) / NT;
  static constexpr int VPT = (VPR + NT - 1) / NT;
  static constexpr int KS = D / 32;   // k-steps of S^T = K . Q^T
  static constexpr int DTL = D / 16;  // d tiles of O^T
};

template <int DT, int D, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(1)))
void paged_prefill_kernel(PrefillArgs a) {
  typedef PShape<D, NW> S;
  constexpr int EB = 2;
  constexpr int TQ = S::TQ, BN = S::BN, NT = S::NT;
  __shared__ __attribute__((aligned(16))) uint16_t ks_lds[2][BN * S::KROW];
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[2][D * S::VROW];
  __shared__ int32_t bt_lds[kBtCache];

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6, g = lane >> 4, c = lane & 15;

  // ---- which (query block, KV head, head group, sequence): heaviest first
  const int per_tb = a.num_kv_heads * a.n_hgp * a.num_seqs;
  const int tb = a.n_qblocks - 1 - (int)(blockIdx.x / per_tb);
  int rest = (int)(blockIdx.x % per_tb);
  const int seq = rest % a.num_seqs;
  rest /= a.num_seqs;
  const int hgp = rest % a.n_hgp;
  const int kvh = rest / a.n_hgp;

  int q_lo = a.cu_q[seq];
  int q_len = a.cu_q[seq + 1] - q_lo;
  if (q_lo < 0 || q_len < 0 || q_lo + q_len > a.total_q) {
    if (tid == 0 && tb == 0 && kvh == 0 && hgp == 0) flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    return;
  }
  const int tq0 = tb * TQ;
  if (tq0 >= q_len) return;
  int p0 = a.q_start[seq];
  const int cap = a.max_blocks * a.bs;
  if (p0 < 0 || (int64_t)p0 + q_len > cap) {
    if (tid == 0 && tb == 0 && kvh == 0 && hgp == 0) flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    p0 = p0 < 0 ? 0 : p0;
  }
  // keys this block needs: up to its last query's position, within the table
  const int kmax = min(cap, p0 + min(q_len, tq0 + TQ));
  const int nkb = kmax > 0 && a.num_blocks > 0 ? (kmax + BN - 1) / BN : 0;

  const int h_local = hgp * NW + w;
  const bool active = h_local < a.n_rep;
  const int head = kvh * a.n_rep + h_local;
  const int32_t* bt_row = a.bt + (int64_t)seq * a.bt_stride;
  const uint16_t* kc = (const uint16_t*)a.kc + (int64_t)kvh * a.c_head;
  const uint16_t* vc = (const uint16_t*)a.vc + (int64_t)kvh * a.c_head;

  // ---- Q^T operands: lane (g, c) holds d = 32 ks + 8 g .. +7 of query column c
  u32x4 qreg[2][S::KS];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int t = tq0 + qt * 16 + c;
    const bool ok = active && t < q_len;
    const uint16_t* qrow = (const uint16_t*)a.q + (int64_t)(q_lo + (ok ? t : 0)) * a.q_tok + (int64_t)head * a.q_head;
#pragma unroll
    for (int ks = 0; ks < S::KS; ++ks)
      qreg[qt][ks] = ok ? *(const u32x4*)(qrow + ks * 32 + 8 * g) : u32x4{0u, 0u, 0u, 0u};
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
  // slot of absolute key k (< kmax), or -1 (then masked out, V zeroed)
  auto slot_of = [&](int k) -> int64_t {
    if (k >= kmax) return -1;
    const int blk = k / a.bs;
    const int32_t bid = bt_lds[blk - bt_base];
    if (bid < 0 || (int64_t)bid >= a.num_blocks) {
      bad = true;
      return -1;
    }
    return (int64_t)bid * a.bs + (k - blk * a.bs);
  };

  u32x4 kreg[S::KPT];
  u32x4 vreg[S::VPT][2];
  // Global loads of key tile kb into registers (whole workgroup, uniform call).
  auto load_regs = [&](int kb) {
    const int k0 = kb * BN;
    const int last_blk = (min(k0 + BN, kmax) - 1) / a.bs;
    if (last_blk >= bt_base + kBtCache) fill_bt(k0 / a.bs);
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const int q = tid + NT * i;
      kreg[i] = u32x4{0u, 0u, 0u, 0u};
      if (q < S::KCH) {
        const int key = q / (D / 8), part = q % (D / 8);
        const int64_t s = slot_of(k0 + key);
        if (s >= 0) kreg[i] = *(const u32x4*)(kc + s * a.c_slot + part * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < S::VPT; ++i) {
      const int v = tid + NT * i;
      vreg[i][0] = vreg[i][1] = u32x4{0u, 0u, 0u, 0u};
      if (v < S::VPR) {
        const int pr = v % (BN / 2), part = v / (BN / 2);
        const int64_t s0 = slot_of(k0 + 2 * pr), s1 = slot_of(k0 + 2 * pr + 1);
        if (s0 >= 0) vreg[i][0] = *(const u32x4*)(vc + s0 * a.c_slot + part * 8);
        if (s1 >= 0) vreg[i][1] = *(const u32x4*)(vc + s1 * a.c_slot + part * 8);
      }
    }
  };
  // Registers -> LDS buffer `buf` (K row-major, V transposed).
  auto store_regs = [&](int buf) {
#pragma unroll
    for (int i = 0; i < S::KPT; ++i) {
      const int q = tid + NT * i;
      if (q < S::KCH) {
        const int key = q / (D / 8), part = q % (D / 8);
        *(u32x4*)&ks_lds[buf][key * S::KROW + part * 8] = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < S::VPT; ++i) {
      const int v = tid + NT * i;
      if (v < S::VPR) {
        const int pr = v % (BN / 2), part = v / (BN / 2);
        const u32x4 x0 = vreg[i][0], x1 = vreg[i][1];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t lo = (x0[e >> 1] >> (16 * (e & 1))) & 0xffffu;
          const uint32_t hi = (x1[e >> 1] >> (16 * (e & 1))) & 0xffffu;
          *(uint32_t*)&vt_lds[buf][(part * 8 + e) * S::VROW + 2 * pr] = lo | (hi << 16);
        }
      }
    }
  };

  // ---- online softmax state, per column tile: lane owns query column c
  f32x4 acc[2][S::DTL];
  float m[2], l[2];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    m[qt] = -__FLT_MAX__;
    l[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < S::DTL; ++dt) acc[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int qpos0 = p0 + tq0;  // position of the block's first query

  auto compute = [&](int buf, int k0) {
    const uint16_t* kb_lds = ks_lds[buf];
    const uint16_t* vb_lds = vt_lds[buf];
    f32x4 s[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) s[qt][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int ks = 0; ks < S::KS; ++ks) {
        const u32x4 ka = *(const u32x4*)&kb_lds[(kt * 16 + c) * S::KROW + ks * 32 + 8 * g];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) s[qt][kt] = mfma_k32<DT>(ka, qreg[qt][ks], s[qt][kt]);
      }
    // masking is needed only where the tile crosses the diagonal or the end
    const bool full = k0 + BN - 1 <= qpos0 && k0 + BN <= kmax;
    using E = Elem<DT>;
    u32x4 pb[2][2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float sv[4][4];
      const int lim = min(qpos0 + qt * 16 + c, kmax - 1);  // last key this column may see
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = s[qt][kt][r] * a.scale_log2;
          sv[kt][r] = (full || k0 + kt * 16 + 4 * g + r <= lim) ? x : kNegInf;
        }
      float mx = kNegInf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        mx = fmaxf(mx, fmaxf(fmaxf(sv[kt][0], sv[kt][1]), fmaxf(sv[kt][2], sv[kt][3])));
      mx = wave_max_groups(mx);
      const bool grow = mx > m[qt] + kRescaleSlack;
      if (__any(grow)) {
        const float m_new = grow ? mx : m[qt];
        const float alpha = fast_exp2(m[qt] - m_new);
        l[qt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < S::DTL; ++dt) acc[qt][dt] *= alpha;
        m[qt] = m_new;
      }
      float p[4][4];
      float ls = 0.f;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p[kt][r] = fast_exp2(sv[kt][r] - m[qt]);
          ls += p[kt][r];
        }
      l[qt] += ls;
      // P^T operands of the two 32-key steps: k-slots 0..3 = keys 4g..4g+3 of
      // tile 2st, k-slots 4..7 = keys 4g..4g+3 of tile 2st+1
#pragma unroll
      for (int st = 0; st < 2; ++st)
        pb[qt][st] = u32x4{E::pack2(p[2 * st][0], p[2 * st][1]), E::pack2(p[2 * st][2], p[2 * st][3]),
                           E::pack2(p[2 * st + 1][0], p[2 * st + 1][1]), E::pack2(p[2 * st + 1][2], p[2 * st + 1][3])};
    }
    // O^T += V^T . P^T; V^T operand: d row c of the tile, the same key slots
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int dt = 0; dt < S::DTL; ++dt) {
        const uint16_t* row = vb_lds + (dt * 16 + c) * S::VROW + st * 32;
        const u32x2 lo = *(const u32x2*)(row + 4 * g);
        const u32x2 hi = *(const u32x2*)(row + 16 + 4 * g);
        const u32x4 va = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) acc[qt][dt] = mfma_k32<DT>(va, pb[qt][st], acc[qt][dt]);
      }
  };

  // ---- walk the key tiles: tile kb in the math while kb + 1 sits in LDS
  // (written after kb's math) and kb + 2 is in flight in registers
  if (nkb > 0) {
    fill_bt(0);
    load_regs(0);
    store_regs(0);
    if (nkb > 1) load_regs(1);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
      if (active) compute(kb & 1, kb * BN);
      if (kb + 1 < nkb) store_regs((kb + 1) & 1);
      if (kb + 2 < nkb) load_regs(kb + 2);
      __syncthreads();
    }
  }
  if (bad) flag_error(a.err, IR_ERR_BLOCK_RANGE);
  if (!active) return;

  // ---- normalise and store: lane (g, c) register r of d tile dt = output
  // d = 16 dt + 4 g + r of query column c
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float lsum = wave_sum_groups(l[qt]);
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    const int t = tq0 + qt * 16 + c;
    if (t >= q_len) continue;
    uint8_t* orow = (uint8_t*)a.out + ((int64_t)(q_lo + t) * a.o_tok + (int64_t)head * a.o_head) * EB;
#pragma unroll
    for (int dt = 0; dt < S::DTL; ++dt) {
      const float o[4] = {acc[qt][dt][0], acc[qt][dt][1], acc[qt][dt][2], acc[qt][dt][3]};
      store4<DT>(orow + (dt * 16 + 4 * g) * EB, o, inv);
    }
  }
}

template <int DT, int D>
int launch_prefill(const PrefillArgs& a0, hipStream_t s) {
  PrefillArgs a = a0;
  const int nw = a.n_rep <= 4 ? 4 : 8;
  a.n_hgp = (a.n_rep + nw - 1) / nw;
  const int64_t grid = (int64_t)a.n_qblocks * a.num_kv_heads * a.n_hgp * a.num_seqs;
  if (grid <= 0) return ok();
  if (grid > 0x7fffffff) return fail(IR_EINVAL, "ir_paged_prefill: grid of %lld workgroups too large", (long long)grid);
  if (nw == 4)
    hipLaunchKernelGGL((paged_prefill_kernel<DT, D, 4>), dim3((unsigned)grid), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((paged_prefill_kernel<DT, D, 8>), dim3((unsigned)grid), dim3(512), 0, s, a);
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
                                int dtype, int32_t* err_flags, ir_stream_t stream) {
  IR_REQUIRE(dtype == IR_DTYPE_BF16 || dtype == IR_DTYPE_F16 || dtype == IR_DTYPE_F32,
             "ir_paged_prefill: unknown dtype %d", dtype);
  if (dtype == IR_DTYPE_F32)
    return fail(IR_EUNSUPPORTED, "ir_paged_prefill: fp32 is not supported (bf16, f16); use ir_paged_attention_masked");
  IR_REQUIRE(num_seqs >= 0 && total_q >= 0 && max_q_len >= 0 && num_q_heads > 0 && num_kv_heads > 0 &&
                 block_size > 0 && max_blocks_per_seq >= 0 && num_blocks >= 0,
             "ir_paged_prefill: bad sizes");
  IR_REQUIRE(num_q_heads % num_kv_heads == 0, "ir_paged_prefill: num_q_heads %d not a multiple of num_kv_heads %d",
             num_q_heads, num_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return fail(IR_EUNSUPPORTED, "ir_paged_prefill: head_dim %d not supported (64, 128)", head_dim);
  IR_REQUIRE((int64_t)max_blocks_per_seq * block_size <= (int64_t)1 << 30,
             "ir_paged_prefill: block tables of %d x %d tokens exceed 2^30 keys", max_blocks_per_seq, block_size);
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
  a.bt = block_tables;
  a.bt_stride = bt_stride;
  a.max_blocks = max_blocks_per_seq;
  a.cu_q = cu_seqlens_q;
  a.q_start = q_start;
  a.num_seqs = num_seqs;
  a.total_q = total_q;
  a.n_qblocks = (max_q_len + 31) / 32;
  a.out = out;
  a.o_tok = out_tok_stride;
  a.o_head = out_head_stride;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.n_rep = num_q_heads / num_kv_heads;
  a.n_hgp = 1;
  a.scale_log2 = scale * kLog2e;
  a.err = err_flags;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == IR_DTYPE_BF16)
    return head_dim == 128 ? launch_prefill<IR_DTYPE_BF16, 128>(a, s) : launch_prefill<IR_DTYPE_BF16, 64>(a, s);
  return head_dim == 128 ? launch_prefill<IR_DTYPE_F16, 128>(a, s) : launch_prefill<IR_DTYPE_F16, 64>(a, s);
}
