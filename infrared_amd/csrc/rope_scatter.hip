// Fused rotary position embedding + KV-slot scatter for gfx950.
//
// Replaces, per layer, the pair
//   q, k = apply_rotary_pos_emb(q, k, cos, sin)   (infrared/model/layers.py:79-89, :164)
//   PagedKVPool.write(layer, k, v, write_slots)   (infrared/cache/paged_kv_cache.py:48-57,
//                                                  infrared/model/triton_attention.py:101-104)
// with one launch: q is rotated into q_out, k is rotated and written straight
// into its pool slot, v is copied into its slot. The rotated K never makes a
// round trip through memory before the scatter.
//
// Numerics follow the reference's tensor ops exactly: the fp32 cos/sin tables
// are first rounded to the activation dtype (`cos.to(q.dtype)`), then
//   out = round(round(x * cos) + round(rotate_half(x) * sin)),
// rotate_half(x) = (-x2, x1) over the two halves of head_dim, every product and
// the sum rounded to the dtype as torch does for 16-bit tensors (fp32 math,
// round to nearest even). In fp32 the same three operations run unfused (no
// multiply-add contraction), so results are bit-identical to the reference.
//
// Work: one lane per (token, row, 8-element chunk of the first half); it also
// handles the matching 8 elements of the second half, which is what rotate_half
// pairs them with. Rows of a token: num_q_heads q rows, then num_kv_heads k
// rows, then num_kv_heads v rows.
#include "common.hpp"
#include "status.hpp"

namespace ir {
namespace {

struct RopeArgs {
  const uint8_t* q;
  int64_t q_tok, q_head;  // bytes
  uint8_t* qo;
  int64_t qo_tok, qo_head;
  const uint8_t* k;
  int64_t k_tok, k_head;
  const uint8_t* v;
  int64_t v_tok, v_head;
  const float* cos;
  const float* sin;
  int64_t cs_tok;  // elements
  uint8_t* kc;
  uint8_t* vc;
  int64_t c_slot, c_head;  // bytes
  int64_t num_slots;
  const int64_t* slots;
  int64_t n_tokens;
  int num_q_heads, num_kv_heads, head_dim;
  int32_t* err;
};

template <int DT>
struct Chunk8 {
  // 8 elements in fp32 plus their raw storage
  static constexpr int EB = DT == IR_DTYPE_F32 ? 4 : 2;
  __device__ __forceinline__ static void load(const uint8_t* p, float (&x)[8]) {
    if constexpr (DT == IR_DTYPE_F32) {
      const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = a[i];
        x[4 + i] = b[i];
      }
    } else {
      using E = Elem<DT>;
      const u32x4 w = *(const u32x4*)p;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[2 * i] = E::lo(w[i]);
        x[2 * i + 1] = E::hi(w[i]);
      }
    }
  }
  __device__ __forceinline__ static void copy(const uint8_t* src, uint8_t* dst) {
    *(u32x4*)dst = *(const u32x4*)src;
    if constexpr (DT == IR_DTYPE_F32) *(u32x4*)(dst + 16) = *(const u32x4*)(src + 16);
  }
  __device__ __forceinline__ static void store(uint8_t* p, const float (&x)[8]) {
    if constexpr (DT == IR_DTYPE_F32) {
      *(f32x4*)p = f32x4{x[0], x[1], x[2], x[3]};
      *(f32x4*)(p + 16) = f32x4{x[4], x[5], x[6], x[7]};
    } else {
      using E = Elem<DT>;
      *(u32x4*)p = u32x4{E::pack2(x[0], x[1]), E::pack2(x[2], x[3]), E::pack2(x[4], x[5]), E::pack2(x[6], x[7])};
    }
  }
  // value rounded to the dtype (identity for fp32)
  __device__ __forceinline__ static float round(float f) {
    if constexpr (DT == IR_DTYPE_F32) return f;
    else return Elem<DT>::to_f32(Elem<DT>::from_f32(f));
  }
};

template <int DT>
__global__ __launch_bounds__(256) void rope_kv_scatter_kernel(RopeArgs a) {
#pragma clang fp contract(off)
  typedef Chunk8<DT> C;
  const int half = a.head_dim / 2;
  const int chunks = half / 8;
  const int rows = a.num_q_heads + 2 * a.num_kv_heads;
  const int64_t per_tok = (int64_t)rows * chunks;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.n_tokens * per_tok) return;
  const int64_t tok = idx / per_tok;
  const int rem = (int)(idx - tok * per_tok);
  const int row = rem / chunks;
  const int i0 = (rem - row * chunks) * 8;  // first-half element index
  const int64_t off1 = (int64_t)i0 * C::EB, off2 = (int64_t)(i0 + half) * C::EB;

  const bool is_q = row < a.num_q_heads;
  const bool is_k = !is_q && row < a.num_q_heads + a.num_kv_heads;
  int64_t slot = 0;
  if (!is_q) {
    slot = a.slots[tok];
    if (slot < 0) return;  // padding sentinel
    if (slot >= a.num_slots) {
      flag_error(a.err, IR_ERR_SLOT_RANGE);
      return;
    }
  }
  if (!is_q && !is_k) {  // v row: plain copy into the slot
    const int h = row - a.num_q_heads - a.num_kv_heads;
    const uint8_t* src = a.v + tok * a.v_tok + h * a.v_head;
    uint8_t* dst = a.vc + slot * a.c_slot + h * a.c_head;
    C::copy(src + off1, dst + off1);
    C::copy(src + off2, dst + off2);
    return;
  }
  const uint8_t* src;
  uint8_t* dst;
  if (is_q) {
    src = a.q + tok * a.q_tok + row * a.q_head;
    dst = a.qo + tok * a.qo_tok + row * a.qo_head;
  } else {
    const int h = row - a.num_q_heads;
    src = a.k + tok * a.k_tok + h * a.k_head;
    dst = a.kc + slot * a.c_slot + h * a.c_head;
  }
  float x1[8], x2[8];
  C::load(src + off1, x1);
  C::load(src + off2, x2);
  // the 8 cos / sin values of each half, 16-byte loads
  float cv1[8], cv2[8], sv1[8], sv2[8];
  Chunk8<IR_DTYPE_F32>::load((const uint8_t*)(a.cos + tok * a.cs_tok + i0), cv1);
  Chunk8<IR_DTYPE_F32>::load((const uint8_t*)(a.cos + tok * a.cs_tok + i0 + half), cv2);
  Chunk8<IR_DTYPE_F32>::load((const uint8_t*)(a.sin + tok * a.cs_tok + i0), sv1);
  Chunk8<IR_DTYPE_F32>::load((const uint8_t*)(a.sin + tok * a.cs_tok + i0 + half), sv2);
  float o1[8], o2[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float c1 = C::round(cv1[e]), s1 = C::round(sv1[e]);
    const float c2 = C::round(cv2[e]), s2 = C::round(sv2[e]);
    // first half: x1 * cos + (-x2) * sin; second half: x2 * cos + x1 * sin
    const float a1 = C::round(x1[e] * c1), b1 = C::round(-x2[e] * s1);
    const float a2 = C::round(x2[e] * c2), b2 = C::round(x1[e] * s2);
    o1[e] = C::round(a1 + b1);
    o2[e] = C::round(a2 + b2);
  }
  C::store(dst + off1, o1);
  C::store(dst + off2, o2);
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_rope_kv_scatter(const void* q, int64_t q_tok_stride, int64_t q_head_stride, void* q_out,
                                  int64_t qo_tok_stride, int64_t qo_head_stride, const void* k, int64_t k_tok_stride,
                                  int64_t k_head_stride, const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                                  const float* cos, const float* sin, int64_t cs_tok_stride, void* k_cache,
                                  void* v_cache, int64_t cache_slot_stride, int64_t cache_head_stride,
                                  int64_t num_slots, const int64_t* slot_mapping, int64_t n_tokens, int num_q_heads,
                                  int num_kv_heads, int head_dim, int dtype, int32_t* err_flags,
                                  ir_stream_t stream) {
  const int eb = dtype_bytes(dtype);
  IR_REQUIRE(eb > 0, "ir_rope_kv_scatter: unknown dtype %d", dtype);
  IR_REQUIRE(n_tokens >= 0 && num_q_heads >= 0 && num_kv_heads > 0 && head_dim > 0 && num_slots >= 0,
             "ir_rope_kv_scatter: bad sizes");
  if (head_dim % 16 != 0)
    return fail(IR_EUNSUPPORTED, "ir_rope_kv_scatter: head_dim %d must be a multiple of 16", head_dim);
  if (n_tokens == 0) return ok();
  IR_REQUIRE(k && v && cos && sin && k_cache && v_cache && slot_mapping && (num_q_heads == 0 || (q && q_out)),
             "ir_rope_kv_scatter: null pointer");
  IR_REQUIRE(aligned16(k) && aligned16(v) && aligned16(k_cache) && aligned16(v_cache) && aligned16(cos) &&
                 aligned16(sin) && (num_q_heads == 0 || (aligned16(q) && aligned16(q_out))),
             "ir_rope_kv_scatter: tensors must be 16-byte aligned");
  IR_REQUIRE(cs_tok_stride % 4 == 0, "ir_rope_kv_scatter: cos/sin row stride must be a multiple of 4 elements");
  IR_REQUIRE((q_tok_stride * eb) % 16 == 0 && (q_head_stride * eb) % 16 == 0 && (qo_tok_stride * eb) % 16 == 0 &&
                 (qo_head_stride * eb) % 16 == 0 && (k_tok_stride * eb) % 16 == 0 && (k_head_stride * eb) % 16 == 0 &&
                 (v_tok_stride * eb) % 16 == 0 && (v_head_stride * eb) % 16 == 0 &&
                 (cache_slot_stride * eb) % 16 == 0 && (cache_head_stride * eb) % 16 == 0,
             "ir_rope_kv_scatter: strides must be multiples of 16 bytes");
  RopeArgs a;
  a.q = (const uint8_t*)q;
  a.q_tok = q_tok_stride * eb;
  a.q_head = q_head_stride * eb;
  a.qo = (uint8_t*)q_out;
  a.qo_tok = qo_tok_stride * eb;
  a.qo_head = qo_head_stride * eb;
  a.k = (const uint8_t*)k;
  a.k_tok = k_tok_stride * eb;
  a.k_head = k_head_stride * eb;
  a.v = (const uint8_t*)v;
  a.v_tok = v_tok_stride * eb;
  a.v_head = v_head_stride * eb;
  a.cos = cos;
  a.sin = sin;
  a.cs_tok = cs_tok_stride;
  a.kc = (uint8_t*)k_cache;
  a.vc = (uint8_t*)v_cache;
  a.c_slot = cache_slot_stride * eb;
  a.c_head = cache_head_stride * eb;
  a.num_slots = num_slots;
  a.slots = slot_mapping;
  a.n_tokens = n_tokens;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.err = err_flags;
  const int64_t total = n_tokens * (int64_t)(num_q_heads + 2 * num_kv_heads) * (head_dim / 16);
  IR_REQUIRE((total + 255) / 256 <= 0x7fffffff, "ir_rope_kv_scatter: too many tokens");
  const dim3 grid((unsigned)((total + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == IR_DTYPE_BF16)
    hipLaunchKernelGGL(rope_kv_scatter_kernel<IR_DTYPE_BF16>, grid, dim3(256), 0, s, a);
  else if (dtype == IR_DTYPE_F16)
    hipLaunchKernelGGL(rope_kv_scatter_kernel<IR_DTYPE_F16>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(rope_kv_scatter_kernel<IR_DTYPE_F32>, grid, dim3(256), 0, s, a);
  return check_launch("ir_rope_kv_scatter");
}
