// Paged attention over per-key flat slot ids and an additive mask: the metadata
// contract of the reference seam (PagedContext.gather_slots + mask,
// infrared/cache/paged_kv_cache.py:75-91, infrared/model/triton_attention.py:81-129).
//
// Works for every mask the reference builds: the decode mask of
// infrared/engine/paged_engine.py:630-638, the causal prefix-hit mask of
// infrared/model/inputs.py:33-54 and the packed varlen mask of
// infrared/model/inputs.py:57-85. Query "columns" are (query token, head)
// pairs of one GQA group, 16 per wavefront tile, so a decode step puts the
// group's heads on the MFMA columns exactly like the block-table kernel.
//
// Softmax semantics follow infrared/model/layers.py:116-117: scores are
// q.k*scale + mask and the softmax runs in fp32. Base-2 scores are clamped at
// -FLT_MAX instead of overflowing to -inf, so a row masked entirely with
// finfo.min averages V uniformly over its keys, as the reference softmax does.
#include "attn_tile.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kWaves = 4;

struct MaskedArgs {
  const uint8_t* q;
  int64_t q_b, q_s, q_h;  // elements
  const uint8_t* kc;
  const uint8_t* vc;
  int64_t c_slot, c_head;  // elements
  int64_t num_slots;
  const int64_t* gs;
  int64_t gs_b, gs_t;
  const uint8_t* mask;
  int64_t m_b, m_s, m_t;  // elements
  int mask_dtype;
  uint8_t* out;
  int64_t o_b, o_s, o_h;  // elements
  int batch, seq_q, seq_k, num_q_heads, num_kv_heads, n_rep, n_rt;
  float scale;
  int32_t* err;
  const int32_t* run_if;  // null, or run only when *run_if != 0
};

__device__ __forceinline__ float mask_at(const MaskedArgs& a, int64_t off) {
  switch (a.mask_dtype) {
    case IR_DTYPE_F32: return ((const float*)a.mask)[off];
    case IR_DTYPE_BF16: return bf16_to_f32(((const uint16_t*)a.mask)[off]);
    default: return f16_to_f32(((const uint16_t*)a.mask)[off]);
  }
}

__device__ __forceinline__ int64_t key_slot(const MaskedArgs& a, int b, int t) {
  if (t >= a.seq_k) return -1;
  const int64_t s = a.gs[(int64_t)b * a.gs_b + (int64_t)t * a.gs_t];
  if (s < 0 || s >= a.num_slots) {
    flag_error(a.err, IR_ERR_GATHER_RANGE);
    return -1;
  }
  return s;
}

template <int DT, int D>
__global__ __launch_bounds__(kWaves * 64) void paged_masked_kernel(MaskedArgs a) {
  typedef TileShape<DT, D> Sh;
  constexpr int EB = Sh::EB;
  __shared__ MergeSmem<kWaves, D> sm;
  // a gated call (the fallback half of a graph-captured decode-form check)
  // does nothing unless the check failed
  if (a.run_if && *a.run_if == 0) return;

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int g = lane >> 4;
  const int c = lane & 15;

  int idx = blockIdx.x;
  const int rt = idx % a.n_rt;
  idx /= a.n_rt;
  const int kvh = idx % a.num_kv_heads;
  const int b = idx / a.num_kv_heads;

  const int rows = a.seq_q * a.n_rep;
  const int row = rt * 16 + c;
  const bool col_ok = row < rows;
  const int sq = col_ok ? row / a.n_rep : 0;
  const int qh = kvh * a.n_rep + (col_ok ? row - sq * a.n_rep : 0);

  uint32_t qr[Sh::KDW];
  if (col_ok)
    load_k<DT, D>(a.q + ((int64_t)b * a.q_b + (int64_t)sq * a.q_s + (int64_t)qh * a.q_h) * EB, g, qr);
  else
    zero_dwords(qr);

  State<D> st;
  state_init(st);

  const uint8_t* kc = a.kc + (int64_t)kvh * a.c_head * EB;
  const uint8_t* vc = a.vc + (int64_t)kvh * a.c_head * EB;
  const int64_t slot_bytes = a.c_slot * EB;
  const int64_t mrow = (int64_t)b * a.m_b + (int64_t)sq * a.m_s;
  const int ntiles = (a.seq_k + 15) >> 4;

  for (int ti = w; ti < ntiles; ti += kWaves) {
    const int t0 = ti * 16;
    Tile<DT, D> tl;
    const int64_t ks = key_slot(a, b, t0 + c);
    if (ks >= 0)
      load_k<DT, D>(kc + ks * slot_bytes, g, tl.k);
    else
      zero_dwords(tl.k);
    bool vok[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t vs = key_slot(a, b, t0 + 4 * g + r);
      vok[r] = vs >= 0;
      if (vok[r])
        load_v<DT, D>(vc + vs * slot_bytes, c, tl.v[r]);
      else
        zero_dwords(tl.v[r]);
    }
    const f32x4 s = qk_tile<DT, D>(tl.k, qr);
    float sv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (vok[r]) {
        const float mv = col_ok ? mask_at(a, mrow + (int64_t)(t0 + 4 * g + r) * a.m_t) : 0.f;
        sv[r] = fmaxf((s[r] * a.scale + mv) * kLog2e, -__FLT_MAX__);
      } else {
        sv[r] = kNegInf;
      }
    }
    softmax_pv<DT, D, false>(sv, tl.v, vok, st);
  }
  st.l = wave_sum_groups(st.l);

  merge_publish<kWaves, D>(sm, st, w, g, c);
  __syncthreads();

  const int ncol = min(16, rows - rt * 16);
  for (int it = threadIdx.x; it < ncol * (D / 4); it += kWaves * 64) {
    const int hc = it / (D / 4);
    const int d0 = (it - hc * (D / 4)) * 4;
    float M, L, o[4];
    merge_column<kWaves, D>(sm, hc, d0, M, L, o);
    const int r = rt * 16 + hc;
    const int osq = r / a.n_rep;
    const int oh = kvh * a.n_rep + (r - osq * a.n_rep);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    store4<DT>(a.out + ((int64_t)b * a.o_b + (int64_t)osq * a.o_s + (int64_t)oh * a.o_h + d0) * EB, o, inv);
  }
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_paged_attention_masked(const void* q, int64_t q_b_stride, int64_t q_s_stride,
                                         int64_t q_h_stride, const void* k_cache, const void* v_cache,
                                         int64_t cache_slot_stride, int64_t cache_head_stride,
                                         int64_t num_slots, const int64_t* gather_slots, int64_t gs_b_stride,
                                         int64_t gs_t_stride, const void* mask, int64_t mask_b_stride,
                                         int64_t mask_s_stride, int64_t mask_t_stride, int mask_dtype,
                                         void* out, int64_t out_b_stride, int64_t out_s_stride,
                                         int64_t out_h_stride, int batch, int seq_q, int seq_k,
                                         int num_q_heads, int num_kv_heads, int head_dim, float scale,
                                         int dtype, int32_t* err_flags, const int32_t* run_if,
                                         ir_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  IR_REQUIRE(eb > 0, "ir_paged_attention_masked: unknown dtype %d", dtype);
  IR_REQUIRE(dtype_bytes(mask_dtype) > 0, "ir_paged_attention_masked: unknown mask dtype %d", mask_dtype);
  IR_REQUIRE(batch >= 0 && seq_q >= 0 && seq_k >= 0 && num_q_heads > 0 && num_kv_heads > 0 && num_slots >= 0,
             "ir_paged_attention_masked: bad sizes");
  IR_REQUIRE(num_q_heads % num_kv_heads == 0,
             "ir_paged_attention_masked: num_q_heads %d not a multiple of num_kv_heads %d", num_q_heads,
             num_kv_heads);
  if (head_dim != 64 && head_dim != 128)
    return fail(IR_EUNSUPPORTED, "ir_paged_attention_masked: head_dim %d not supported (64, 128)", head_dim);
  if ((int64_t)batch * seq_q == 0) return ok();
  IR_REQUIRE(q && k_cache && v_cache && out && (seq_k == 0 || (gather_slots && mask)),
             "ir_paged_attention_masked: null pointer");
  IR_REQUIRE(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out),
             "ir_paged_attention_masked: q, caches and out must be 16-byte aligned");
  IR_REQUIRE((q_b_stride * eb) % 16 == 0 && (q_s_stride * eb) % 16 == 0 && (q_h_stride * eb) % 16 == 0 &&
                 (cache_slot_stride * eb) % 16 == 0 && (cache_head_stride * eb) % 16 == 0 &&
                 (out_b_stride * eb) % 16 == 0 && (out_s_stride * eb) % 16 == 0 &&
                 (out_h_stride * eb) % 16 == 0,
             "ir_paged_attention_masked: strides must be multiples of 16 bytes");
  MaskedArgs a;
  a.q = (const uint8_t*)q;
  a.q_b = q_b_stride;
  a.q_s = q_s_stride;
  a.q_h = q_h_stride;
  a.kc = (const uint8_t*)k_cache;
  a.vc = (const uint8_t*)v_cache;
  a.c_slot = cache_slot_stride;
  a.c_head = cache_head_stride;
  a.num_slots = num_slots;
  a.gs = gather_slots;
  a.gs_b = gs_b_stride;
  a.gs_t = gs_t_stride;
  a.mask = (const uint8_t*)mask;
  a.m_b = mask_b_stride;
  a.m_s = mask_s_stride;
  a.m_t = mask_t_stride;
  a.mask_dtype = mask_dtype;
  a.out = (uint8_t*)out;
  a.o_b = out_b_stride;
  a.o_s = out_s_stride;
  a.o_h = out_h_stride;
  a.batch = batch;
  a.seq_q = seq_q;
  a.seq_k = seq_k;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.n_rep = num_q_heads / num_kv_heads;
  a.n_rt = (seq_q * a.n_rep + 15) / 16;
  a.scale = scale;
  a.err = err_flags;
  a.run_if = run_if;
  const int64_t nwg = (int64_t)batch * num_kv_heads * a.n_rt;
  IR_REQUIRE(nwg < (1ll << 31), "ir_paged_attention_masked: grid too large");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)nwg), block(kWaves * 64);
  switch (dtype) {
    case IR_DTYPE_BF16:
      if (head_dim == 128)
        hipLaunchKernelGGL((paged_masked_kernel<IR_DTYPE_BF16, 128>), grid, block, 0, s, a);
      else
        hipLaunchKernelGGL((paged_masked_kernel<IR_DTYPE_BF16, 64>), grid, block, 0, s, a);
      break;
    case IR_DTYPE_F16:
      if (head_dim == 128)
        hipLaunchKernelGGL((paged_masked_kernel<IR_DTYPE_F16, 128>), grid, block, 0, s, a);
      else
        hipLaunchKernelGGL((paged_masked_kernel<IR_DTYPE_F16, 64>), grid, block, 0, s, a);
      break;
    default:
      if (head_dim == 128)
        hipLaunchKernelGGL((paged_masked_kernel<IR_DTYPE_F32, 128>), grid, block, 0, s, a);
      else
        hipLaunchKernelGGL((paged_masked_kernel<IR_DTYPE_F32, 64>), grid, block, 0, s, a);
      break;
  }
  return check_launch("ir_paged_attention_masked");
}
