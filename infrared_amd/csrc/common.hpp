// Shared device helpers for the gfx950 paged-attention kernels: element types,
// conversions, MFMA wrappers and the token -> slot address function.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "infrared_amd.h"

namespace ir {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even float -> bf16 bits (NaN stays NaN), the rounding torch
// applies in `.to(torch.bfloat16)`.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float f16_to_f32(uint32_t h) {
  _Float16 x = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)x;
}

__device__ __forceinline__ uint32_t f32_to_f16(float f) {
  _Float16 x = (_Float16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, x);
}

// Element-type traits. Storage is raw bits; arithmetic is always fp32.
template <int DT>
struct Elem;

template <>
struct Elem<IR_DTYPE_F32> {
  typedef float storage;
  static constexpr int bytes = 4;
  __device__ __forceinline__ static float load(const storage* p) { return *p; }
  __device__ __forceinline__ static storage from_f32(float f) { return f; }
  __device__ __forceinline__ static float to_f32(storage s) { return s; }
};

template <>
struct Elem<IR_DTYPE_BF16> {
  typedef uint16_t storage;
  static constexpr int bytes = 2;
  __device__ __forceinline__ static float to_f32(storage s) { return bf16_to_f32(s); }
  __device__ __forceinline__ static storage from_f32(float f) { return (storage)f32_to_bf16(f); }
  // packs two fp32 values into one dword of two elements (lo first), rounding
  // to nearest even (one v_cvt_pk_bf16_f32)
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  __device__ __forceinline__ static float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ __forceinline__ static float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
};

template <>
struct Elem<IR_DTYPE_F16> {
  typedef uint16_t storage;
  static constexpr int bytes = 2;
  __device__ __forceinline__ static float to_f32(storage s) { return f16_to_f32(s); }
  __device__ __forceinline__ static storage from_f32(float f) { return (storage)f32_to_f16(f); }
  __device__ __forceinline__ static uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  __device__ __forceinline__ static float lo(uint32_t w) { return f16_to_f32(w & 0xffffu); }
  __device__ __forceinline__ static float hi(uint32_t w) { return f16_to_f32(w >> 16); }
};

// ---------------------------------------------------------------- MFMA wrappers
//
// 16x16 fp32-accumulator layout (all three shapes below): lane l, register r
// holds D[row = 4*(l/16) + r][col = l%16]. Operand A (M x K) lane l holds
// A[row = l%16][k-slots of lane group l/16]; operand B (K x N) lane l holds
// B[k-slots of lane group l/16][col = l%16]. The kernels only rely on A and B
// sharing the same k-slot assignment, which is what makes the contraction a
// plain dot product over whatever element order the loads chose.

// 16x16x32, 16-bit inputs: 8 elements (4 dwords) of A and B per lane.
template <int DT>
__device__ __forceinline__ f32x4 mfma_k32(u32x4 a, u32x4 b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma_k32<IR_DTYPE_BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma_k32<IR_DTYPE_F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// gfx950 LDS transpose read of 16-bit elements (ds_read_b64_tr_b16): within
// each group of 16 lanes, lane 4a + b receives element b of the 4-element
// (8-byte) pieces addressed by lanes a, a + 4, a + 8 and a + 12, in that order
// (measured lane layout). p must point into LDS, 8-byte aligned.
// Takes an LDS-address-space pointer: offsets computed in that space fold
// into the instruction (a generic pointer costs a cast per read).
typedef __attribute__((address_space(3))) const uint16_t lds_u16;
__device__ __forceinline__ u32x2 lds_read_tr16(lds_u16* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  return __builtin_bit_cast(u32x2, v);
}

// acc + lo + hi of a dword holding two 16-bit elements (one v_dot2c against
// packed 1.0s, fp32 accumulation).
template <int DT>
__device__ __forceinline__ float sum2(uint32_t w, float acc);

template <>
__device__ __forceinline__ float sum2<IR_DTYPE_BF16>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, 0x3f803f80u),
                                         acc, false);
}

template <>
__device__ __forceinline__ float sum2<IR_DTYPE_F16>(uint32_t w, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), __builtin_bit_cast(f16x2, 0x3c003c00u), acc, false);
}

// 16x16x16, 16-bit inputs: 4 elements (2 dwords) of A and B per lane.
template <int DT>
__device__ __forceinline__ f32x4 mfma_k16(u32x2 a, u32x2 b, f32x4 c);

template <>
__device__ __forceinline__ f32x4 mfma_k16<IR_DTYPE_BF16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                    __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma_k16<IR_DTYPE_F16>(u32x2 a, u32x2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
}

// 16x16x4 fp32: one element of A and B per lane (k-slot = lane group).
__device__ __forceinline__ f32x4 mfma_f32_k4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- misc

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float wave_max_groups(float x) {
  // max over lanes l, l^16, l^32, l^48 (the four 16-lane groups)
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float wave_sum_groups(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

// The same two reductions with gfx950's lane-swap instructions (no LDS
// round trip): permlane32_swap pairs lane l with l^32, permlane16_swap pairs
// 16-lane rows 0<->1 and 2<->3. Both outputs of a swap are combined, so which
// one carries which half does not matter for a symmetric operation.
__device__ __forceinline__ float wave_max_groups_swap(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float wave_sum_groups_swap(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ void flag_error(int32_t* err, int32_t bit) {
  if (err) atomicOr(err, bit);
}

template <typename T>
__device__ __forceinline__ T load_nt(const T* p) {
  return __builtin_nontemporal_load(p);
}

// Flat slot of logical token `t` of a sequence whose block table row is `bt`:
// bt[t / bs] * bs + t % bs (infrared/engine/paged_engine.py:621-625), or -1 for
// a block id outside [0, num_blocks). Does not report; see token_slot.
__device__ __forceinline__ int64_t token_slot_or_neg(const int32_t* bt, int t, int bs, int64_t num_blocks) {
  const int blk = t / bs;
  const int32_t bid = bt[blk];
  if (bid < 0 || (int64_t)bid >= num_blocks) return -1;
  return (int64_t)bid * bs + (t - blk * bs);
}

// token_slot_or_neg that also flags IR_ERR_BLOCK_RANGE for a bad block id.
__device__ __forceinline__ int64_t token_slot(const int32_t* bt, int t, int bs, int64_t num_blocks,
                                              int32_t* err) {
  const int64_t s = token_slot_or_neg(bt, t, bs, num_blocks);
  if (s < 0) flag_error(err, IR_ERR_BLOCK_RANGE);
  return s;
}

}  // namespace ir
