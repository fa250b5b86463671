// GQA paged decode attention for gfx950 (one query token per sequence).
//
// Work decomposition: one workgroup per (sequence, KV head, head group of <=16
// query heads, partition of `part_tokens` keys). Its NW wavefronts take the
// partition's 16-token tiles round-robin. Per tile a wavefront
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
// The wavefronts' (max, sum, acc) states merge through LDS; a sequence that
// needs one partition writes its output directly, longer ones write fp32
// partials that paged_decode_reduce merges with a log-sum-exp weighting.
//
// Algorithm parity: the one-shot softmax of infrared/model/layers.py:102-118
// over the gathered history (infrared/model/triton_attention.py:110-129), with
// the streaming max/sum update of infrared/model/triton_attention.py:135-177 and
// the exp2 fold of infrared/model/triton_attention.py:249. For 16-bit dtypes
// the probabilities are rounded to the input dtype before the PV product, as
// `softmax(scores.float()).to(q.dtype)` does in the reference.
#include "attn_tile.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kWaves = 4;  // wavefronts per workgroup

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
  float* ws_o;   // [seq][q_head][part][D]
  float* ws_ml;  // [seq][q_head][part][2]
  int32_t* err;
};

template <int DT, int D, bool BS16>
__device__ __forceinline__ bool load_tile(const DecodeArgs& a, const int32_t* bt_row, int kvh, int t0,
                                          int t_end, int g, int c, Tile<DT, D>& tl) {
  typedef TileShape<DT, D> Sh;
  const uint8_t* kc = (const uint8_t*)a.kc + (int64_t)kvh * a.c_head * Sh::EB;
  const uint8_t* vc = (const uint8_t*)a.vc + (int64_t)kvh * a.c_head * Sh::EB;
  const int64_t slot_bytes = a.c_slot * Sh::EB;
  if constexpr (BS16) {
    // The whole tile lies in one block: the block id is wave-uniform, and every
    // row of the block is inside the pool even past the context end.
    const int blk = t0 / a.bs;
    const int32_t bid = bt_row[blk];
    if (bid < 0 || (int64_t)bid >= a.num_blocks) {
      flag_error(a.err, IR_ERR_BLOCK_RANGE);
      zero_dwords(tl.k);
#pragma unroll
      for (int r = 0; r < 4; ++r) zero_dwords(tl.v[r]);
      return false;
    }
    const int64_t base = (int64_t)bid * a.bs + (t0 - blk * a.bs);
    load_k<DT, D>(kc + (base + c) * slot_bytes, g, tl.k);
#pragma unroll
    for (int r = 0; r < 4; ++r) load_v<DT, D>(vc + (base + 4 * g + r) * slot_bytes, c, tl.v[r]);
    return true;
  } else {
    // Any block size: every lane resolves its own keys' slots; keys past the
    // context are not read (their block-table entries may not exist).
    const int tk = t0 + c;
    const int64_t ks = tk < t_end ? token_slot(bt_row, tk, a.bs, a.num_blocks, a.err) : -1;
    if (ks >= 0)
      load_k<DT, D>(kc + ks * slot_bytes, g, tl.k);
    else
      zero_dwords(tl.k);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tv = t0 + 4 * g + r;
      const int64_t vs = tv < t_end ? token_slot(bt_row, tv, a.bs, a.num_blocks, a.err) : -1;
      if (vs >= 0)
        load_v<DT, D>(vc + vs * slot_bytes, c, tl.v[r]);
      else
        zero_dwords(tl.v[r]);
    }
    return true;
  }
}

template <int DT, int D>
__device__ __forceinline__ void compute_tile(const Tile<DT, D>& tl, const uint32_t (&qr)[TileShape<DT, D>::KDW],
                                             int t0, int t_end, bool tile_ok, float scale_log2, int g,
                                             State<D>& st) {
  const f32x4 s = qk_tile<DT, D>(tl.k, qr);
  float sv[4];
  bool vok[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    vok[r] = tile_ok && (t0 + 4 * g + r < t_end);
    sv[r] = vok[r] ? s[r] * scale_log2 : kNegInf;
  }
  softmax_pv<DT, D>(sv, tl.v, vok, st);
}

__device__ __forceinline__ int clamp_ctx(const DecodeArgs& a, int seq, bool report) {
  int ctx = a.ctx[seq];
  const int cap = a.max_blocks * a.bs;
  if (ctx < 0 || ctx > cap) {
    if (report) flag_error(a.err, IR_ERR_CONTEXT_RANGE);
    ctx = ctx < 0 ? 0 : cap;
  }
  return ctx;
}

template <int DT, int D, bool BS16>
__global__ __launch_bounds__(kWaves * 64) void paged_decode_kernel(DecodeArgs a) {
  typedef TileShape<DT, D> Sh;
  constexpr int EB = Sh::EB;
  __shared__ MergeSmem<kWaves, D> sm;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;

  int idx = blockIdx.x;
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
  const int ntiles = t_end > t_begin ? (t_end - t_begin + 15) >> 4 : 0;

  const int h_local = hg * 16 + c;
  const bool head_ok = h_local < a.n_rep;
  const int qh = kvh * a.n_rep + h_local;

  // Q^T operand, same k-slot assignment as the K loads; padded heads are zero.
  uint32_t qr[Sh::KDW];
  if (head_ok) {
    load_k<DT, D>((const uint8_t*)a.q + ((int64_t)seq * a.q_seq + (int64_t)qh * a.q_head) * EB, g, qr);
  } else {
#pragma unroll
    for (int i = 0; i < Sh::KDW; ++i) qr[i] = 0;
  }

  State<D> st;
  state_init(st);

  const int32_t* bt_row = a.bt + (int64_t)seq * a.bt_stride;
  // Two tiles in flight per wavefront: loads for both are issued before either
  // is consumed.
  for (int ti = w; ti < ntiles; ti += 2 * kWaves) {
    Tile<DT, D> t_a, t_b;
    const int t0a = t_begin + 16 * ti;
    const int t0b = t0a + 16 * kWaves;
    const bool has_b = ti + kWaves < ntiles;
    const bool ok_a = load_tile<DT, D, BS16>(a, bt_row, kvh, t0a, t_end, g, c, t_a);
    bool ok_b = false;
    if (has_b) ok_b = load_tile<DT, D, BS16>(a, bt_row, kvh, t0b, t_end, g, c, t_b);
    compute_tile<DT, D>(t_a, qr, t0a, t_end, ok_a, a.scale_log2, g, st);
    if (has_b) compute_tile<DT, D>(t_b, qr, t0b, t_end, ok_b, a.scale_log2, g, st);
  }
  st.l = wave_sum_groups(st.l);

  // ---- merge the wavefronts of this workgroup through LDS
  merge_publish<kWaves, D>(sm, st, w, g, c);
  __syncthreads();

  const int nh = min(16, a.n_rep - hg * 16);
  for (int it = threadIdx.x; it < nh * (D / 4); it += kWaves * 64) {
    const int hc = it / (D / 4);
    const int d0 = (it - hc * (D / 4)) * 4;
    float M, L, o[4];
    merge_column<kWaves, D>(sm, hc, d0, M, L, o);
    const int oh = kvh * a.n_rep + hg * 16 + hc;
    if (nparts == 1) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      store4<DT>((uint8_t*)a.out + ((int64_t)seq * a.o_seq + (int64_t)oh * a.o_head + d0) * EB, o, inv);
    } else {
      const int64_t row = ((int64_t)seq * a.num_q_heads + oh) * a.max_parts + part;
      const f32x4 ov = {o[0], o[1], o[2], o[3]};
      *(f32x4*)(a.ws_o + row * D + d0) = ov;
      if (d0 == 0) {
        a.ws_ml[row * 2 + 0] = M;
        a.ws_ml[row * 2 + 1] = L;
      }
    }
  }
}

// Log-sum-exp merge of a sequence's partitions: one wavefront per (seq, q head).
template <int DT, int D>
__global__ __launch_bounds__(64) void paged_decode_reduce(DecodeArgs a) {
  constexpr int EB = DT == IR_DTYPE_F32 ? 4 : 2;
  constexpr int PER = D / 64;  // d values per lane
  const int lane = threadIdx.x;
  const int qh = blockIdx.x % a.num_q_heads;
  const int seq = blockIdx.x / a.num_q_heads;
  const int ctx = clamp_ctx(a, seq, false);
  const int nparts = ctx > 0 ? (ctx + a.part_tokens - 1) / a.part_tokens : 1;
  if (nparts <= 1) return;
  const int64_t row0 = ((int64_t)seq * a.num_q_heads + qh) * a.max_parts;
  const float* ml = a.ws_ml + row0 * 2;
  float M = kNegInf;
  for (int p = lane; p < nparts; p += 64) M = fmaxf(M, ml[2 * p]);
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) M = fmaxf(M, __shfl_xor(M, off));
  float L = 0.f;
  float o[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) o[k] = 0.f;
  for (int p = 0; p < nparts; ++p) {
    const float mp = ml[2 * p];
    const float wt = mp == kNegInf ? 0.f : fast_exp2(mp - M);
    L += wt * ml[2 * p + 1];
    const float* src = a.ws_o + (row0 + p) * D + lane * PER;
#pragma unroll
    for (int k = 0; k < PER; ++k) o[k] += wt * src[k];
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  uint8_t* dst = (uint8_t*)a.out + ((int64_t)seq * a.o_seq + (int64_t)qh * a.o_head + lane * PER) * EB;
  using E = Elem<DT>;
#pragma unroll
  for (int k = 0; k < PER; ++k) ((typename E::storage*)dst)[k] = E::from_f32(o[k] * inv);
}

int64_t align256(int64_t x) { return (x + 255) & ~(int64_t)255; }

int max_parts_for(int max_blocks, int bs, int part_tokens) {
  const int64_t cap = (int64_t)max_blocks * bs;
  const int64_t p = (cap + part_tokens - 1) / part_tokens;
  return p < 1 ? 1 : (int)p;
}

template <int DT, int D>
int launch_decode(const DecodeArgs& a, bool bs16, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)a.num_seqs * a.num_kv_heads * a.n_hg), (unsigned)a.max_parts);
  if (bs16)
    hipLaunchKernelGGL((paged_decode_kernel<DT, D, true>), grid, dim3(kWaves * 64), 0, s, a);
  else
    hipLaunchKernelGGL((paged_decode_kernel<DT, D, false>), grid, dim3(kWaves * 64), 0, s, a);
  if (a.max_parts > 1)
    hipLaunchKernelGGL((paged_decode_reduce<DT, D>), dim3((unsigned)((int64_t)a.num_seqs * a.num_q_heads)),
                       dim3(64), 0, s, a);
  return check_launch("ir_paged_decode");
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_paged_decode_default_partition(int num_seqs, int num_kv_heads, int max_blocks_per_seq,
                                                 int block_size) {
  // Aim for about 2048 busy workgroups if contexts average half the table width.
  const int64_t max_ctx = (int64_t)max_blocks_per_seq * block_size;
  int64_t p = (int64_t)num_seqs * num_kv_heads * max_ctx / 4096;
  p = (p + 255) / 256 * 256;
  if (p < 256) p = 256;
  if (p > 8192) p = 8192;
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
  const int mp = max_parts_for(max_blocks_per_seq, block_size, partition_tokens);
  if (mp <= 1) return 0;
  const int64_t rows = (int64_t)num_seqs * num_q_heads * mp;
  return align256(rows * head_dim * 4) + align256(rows * 2 * 4);
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
  IR_REQUIRE(partition_tokens % 16 == 0, "ir_paged_decode: partition_tokens %d not a multiple of 16",
             partition_tokens);
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
    const int64_t rows = (int64_t)num_seqs * num_q_heads * a.max_parts;
    a.ws_o = (float*)workspace;
    a.ws_ml = (float*)((uint8_t*)workspace + align256(rows * head_dim * 4));
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
