// Register-tile attention building blocks shared by the decode and the
// gather_slots+mask kernels.
//
// A wavefront processes 16 keys at a time against up to 16 query "columns"
// (the query heads of one GQA group, or (query token, head) pairs).
// Lane l = 16*g + c (g = lane group 0..3, c = column 0..15):
//   K operand : the 16 K rows, lane (g,c) holds pieces of key row c;
//   Q operand : lane (g,c) holds the same pieces of column c's query row;
//   S^T       : MFMA result, lane (g,c) register r = score of key 4g+r, column c;
//   V operand : lane (g,c) holds head_dim/16 consecutive elements (from d =
//               (head_dim/16)*c) of key rows 4g..4g+3;
//   O^T acc   : lane (g,c) tile n register r = output d = (head_dim/16)*(4g+r) + n
//               of column c, i.e. one lane owns 4*head_dim/16 consecutive d.
#pragma once

#include "common.hpp"

namespace ir {

template <int DT, int D>
struct TileShape {
  static constexpr bool k16 = DT != IR_DTYPE_F32;
  static constexpr int EB = k16 ? 2 : 4;  // element bytes
  static constexpr int TILES = D / 16;    // PV output tiles of 16 d-rows
  // dwords of K one lane loads from its key row (16-bit: D/32 pieces of 8
  // elements; f32: D/16 pieces of 4 elements)
  static constexpr int KDW = k16 ? D / 8 : D / 4;
  // dwords of V one lane loads from each of its 4 key rows
  static constexpr int VDW = k16 ? TILES / 2 : TILES;
};

template <int DT, int D>
struct Tile {
  uint32_t k[TileShape<DT, D>::KDW];
  uint32_t v[4][TileShape<DT, D>::VDW];
};

template <int D>
struct State {
  float m, l;
  f32x4 acc[D / 16];
};

// Running max starts at -FLT_MAX (finite): a column that has seen no key yet
// then gets exp2(-inf - m) = 0 for absent keys instead of a NaN, and its first
// real tile always raises the max.
template <int D>
__device__ __forceinline__ void state_init(State<D>& st) {
  st.m = -__FLT_MAX__;
  st.l = 0.f;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) st.acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
}

template <int N>
__device__ __forceinline__ void load_dwords(const uint8_t* p, uint32_t (&r)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x4 x = ((const u32x4*)p)[i];
      r[4 * i + 0] = x[0];
      r[4 * i + 1] = x[1];
      r[4 * i + 2] = x[2];
      r[4 * i + 3] = x[3];
    }
  } else {
    static_assert(N == 2, "row piece must be 8 or 16*k bytes");
    const u32x2 x = *(const u32x2*)p;
    r[0] = x[0];
    r[1] = x[1];
  }
}

template <int N>
__device__ __forceinline__ void zero_dwords(uint32_t (&r)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) r[i] = 0u;
}

// K (or Q) pieces of one head row for lane group g. The element order is the
// MFMA k-slot order; K and Q use the same function so the contraction over
// head_dim is exact whatever order that is.
//   16-bit: piece j = elements [8*(4j+g), +8); f32: piece j = [16j+4g, +4).
template <int DT, int D>
__device__ __forceinline__ void load_k(const uint8_t* row, int g, uint32_t (&k)[TileShape<DT, D>::KDW]) {
  typedef TileShape<DT, D> Sh;
#pragma unroll
  for (int j = 0; j < Sh::KDW / 4; ++j) {
    const int d = Sh::k16 ? 8 * (4 * j + g) : 16 * j + 4 * g;
    const u32x4 x = *(const u32x4*)(row + d * Sh::EB);
    k[4 * j + 0] = x[0];
    k[4 * j + 1] = x[1];
    k[4 * j + 2] = x[2];
    k[4 * j + 3] = x[3];
  }
}

// V elements of one key row this lane needs: [TILES*c, TILES*c + TILES).
template <int DT, int D>
__device__ __forceinline__ void load_v(const uint8_t* row, int c, uint32_t (&v)[TileShape<DT, D>::VDW]) {
  typedef TileShape<DT, D> Sh;
  load_dwords<Sh::VDW>(row + Sh::TILES * c * Sh::EB, v);
}

// ---------------------------------------------------------------- K staged through LDS
//
// The QK MFMA wants lane (g,c) to own a head_dim run of key row c, but loading
// it that way makes every load instruction touch 16 rows x 64 B. Instead the
// K tile is loaded like V -- each instruction reads RPI whole rows, 1 KiB
// contiguous in a head-major pool -- written to a per-wavefront LDS tile and
// read back in operand layout. 16-byte chunk k of row t lives at LDS offset
// t * ROWB + 16 * (k ^ (t % CPR)): the XOR swizzle keeps both the row-wise
// writes and the column-wise operand reads free of bank conflicts.
template <int DT, int D>
struct KStage {
  static constexpr int ROWB = D * TileShape<DT, D>::EB;  // bytes of one K row of one head
  static constexpr int CPR = ROWB / 16;                  // 16-byte chunks per row
  static constexpr int RPI = 64 / CPR;                   // rows per load instruction
  static constexpr int NI = 16 / RPI;                    // load instructions per 16-row tile
  static constexpr int BYTES = 16 * ROWB;                // LDS bytes of one tile
  static_assert(NI * 4 == TileShape<DT, D>::KDW, "K staging and operand sizes differ");
};

// Row of the tile that lane `lane` loads in instruction i, and its chunk.
template <int DT, int D>
__device__ __forceinline__ int kstage_row(int i, int lane) {
  typedef KStage<DT, D> KS;
  return i * KS::RPI + lane / KS::CPR;
}

template <int DT, int D>
__device__ __forceinline__ int kstage_chunk(int lane) {
  return lane % KStage<DT, D>::CPR;
}

// Loads this lane's pieces of the K tile; row_ptr(t) is the byte address of
// key row t (0..15) of the tile for this lane.
template <int DT, int D, bool NT, typename RowPtr>
__device__ __forceinline__ void kstage_load(RowPtr row_ptr, int lane, uint32_t (&k)[TileShape<DT, D>::KDW]) {
  typedef KStage<DT, D> KS;
#pragma unroll
  for (int i = 0; i < KS::NI; ++i) {
    const u32x4* p = (const u32x4*)(row_ptr(kstage_row<DT, D>(i, lane)) + 16 * kstage_chunk<DT, D>(lane));
    const u32x4 x = NT ? __builtin_nontemporal_load(p) : *p;
    k[4 * i + 0] = x[0];
    k[4 * i + 1] = x[1];
    k[4 * i + 2] = x[2];
    k[4 * i + 3] = x[3];
  }
}

// Token held by MFMA row c of the staged-K operand: tok(c) = 4*(c%4) + c/4.
// The QK result then gives lane group g, register r the score of token
// 4r + g, so the four V rows a lane group needs for register r are tokens
// 4r..4r+3 -- one contiguous 1 KiB load across the lane groups.
__device__ __forceinline__ int staged_token(int c) { return 4 * (c & 3) + (c >> 2); }

// Writes the loaded pieces to the wavefront's LDS tile and reads back the QK
// operand (lane (g,c): token staged_token(c), chunks 4j+g), same element order
// as load_k.
template <int DT, int D>
__device__ __forceinline__ void kstage_transpose(uint8_t* lds, int lane, const uint32_t (&kin)[TileShape<DT, D>::KDW],
                                                 uint32_t (&kout)[TileShape<DT, D>::KDW]) {
  typedef KStage<DT, D> KS;
  const int ch = kstage_chunk<DT, D>(lane);
#pragma unroll
  for (int i = 0; i < KS::NI; ++i) {
    const int t = kstage_row<DT, D>(i, lane);
    *(u32x4*)(lds + t * KS::ROWB + 16 * (ch ^ (t % KS::CPR))) =
        u32x4{kin[4 * i], kin[4 * i + 1], kin[4 * i + 2], kin[4 * i + 3]};
  }
  // the operand reads below take rows other lanes wrote: keep them after the
  // writes (LDS executes one wavefront's accesses in order)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int g = lane >> 4, t = staged_token(lane & 15);
#pragma unroll
  for (int j = 0; j < KS::NI; ++j) {
    const u32x4 x = *(const u32x4*)(lds + t * KS::ROWB + 16 * ((4 * j + g) ^ (t % KS::CPR)));
    kout[4 * j + 0] = x[0];
    kout[4 * j + 1] = x[1];
    kout[4 * j + 2] = x[2];
    kout[4 * j + 3] = x[3];
  }
  // the next tile's writes must follow these reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// N dwords from p (16- or 8-byte loads), optionally non-temporal.
template <int N, bool NT>
__device__ __forceinline__ void load_dwords_nt(const uint8_t* p, uint32_t (&v)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x4 x = NT ? __builtin_nontemporal_load((const u32x4*)p + i) : ((const u32x4*)p)[i];
      v[4 * i + 0] = x[0];
      v[4 * i + 1] = x[1];
      v[4 * i + 2] = x[2];
      v[4 * i + 3] = x[3];
    }
  } else {
    static_assert(N == 2, "row piece must be 8 or 16*k bytes");
    const u32x2 x = NT ? __builtin_nontemporal_load((const u32x2*)p) : *(const u32x2*)p;
    v[0] = x[0];
    v[1] = x[1];
  }
}

// V elements of one key row this lane needs, optionally non-temporal.
template <int DT, int D, bool NT>
__device__ __forceinline__ void load_v_nt(const uint8_t* row, int c, uint32_t (&v)[TileShape<DT, D>::VDW]) {
  typedef TileShape<DT, D> Sh;
  load_dwords_nt<Sh::VDW, NT>(row + Sh::TILES * c * Sh::EB, v);
}

// S^T = K . Q^T for one 16-key tile; lane (g,c) register r = key 4g+r, column c.
template <int DT, int D>
__device__ __forceinline__ f32x4 qk_tile(const uint32_t (&k)[TileShape<DT, D>::KDW],
                                         const uint32_t (&qr)[TileShape<DT, D>::KDW]) {
  typedef TileShape<DT, D> Sh;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if constexpr (Sh::k16) {
#pragma unroll
    for (int j = 0; j < Sh::KDW / 4; ++j) {
      const u32x4 ka = {k[4 * j], k[4 * j + 1], k[4 * j + 2], k[4 * j + 3]};
      const u32x4 qb = {qr[4 * j], qr[4 * j + 1], qr[4 * j + 2], qr[4 * j + 3]};
      s = mfma_k32<DT>(ka, qb, s);
    }
  } else {
#pragma unroll
    for (int j = 0; j < Sh::KDW; ++j) s = mfma_f32_k4(__uint_as_float(k[j]), __uint_as_float(qr[j]), s);
  }
  return s;
}

// Lazy rescale: the running max of a column only moves when a tile's max
// exceeds it by more than kRescaleSlack (log2 units). The result is the same
// softmax -- numerator and denominator use the same max -- with unnormalised
// probabilities bounded by 2^kRescaleSlack, and the accumulator rescale (a
// pass over every output register) runs only on the rare tiles that raise a
// max (a wave-uniform branch).
constexpr float kRescaleSlack = 8.f;

// Online-softmax update with base-2 scores sv (-inf = key absent) followed by
// O^T += V^T . P^T. Unless FULL, `vok[r]` says whether key row 4g+r may be
// read; rows that may not are zeroed so 0 * V never meets a NaN pattern in
// stale pool memory. FULL tiles (every key present) skip that masking.
template <int DT, int D, bool FULL>
__device__ __forceinline__ void softmax_pv(const float (&sv)[4], const uint32_t (&vin)[4][TileShape<DT, D>::VDW],
                                           const bool (&vok)[4], State<D>& st) {
  typedef TileShape<DT, D> Sh;
  constexpr int TILES = Sh::TILES;
  float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
  mx = wave_max_groups(mx);
  const bool grow = mx > st.m + kRescaleSlack;
  if (__any(grow)) {
    const float m_new = grow ? mx : st.m;
    const float alpha = fast_exp2(st.m - m_new);  // 1 if unchanged, 0 from the start value
    st.l *= alpha;
#pragma unroll
    for (int n = 0; n < TILES; ++n) st.acc[n] *= alpha;
    st.m = m_new;
  }
  float p[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) p[r] = fast_exp2(sv[r] - st.m);
  st.l += (p[0] + p[1]) + (p[2] + p[3]);
  uint32_t v[4][Sh::VDW];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int i = 0; i < Sh::VDW; ++i) v[r][i] = (FULL || vok[r]) ? vin[r][i] : 0u;
  if constexpr (Sh::k16) {
    // P rounded to the input dtype, as softmax(...).to(q.dtype) does.
    using E = Elem<DT>;
    const u32x2 pb = {E::pack2(p[0], p[1]), E::pack2(p[2], p[3])};
#pragma unroll
    for (int n = 0; n < TILES; ++n) {
      // element n of rows 4g..4g+3 -> the 4 k-slots of this lane (transpose)
      const int wdw = n >> 1;
      uint32_t lo, hi;
      if ((n & 1) == 0) {
        lo = (v[0][wdw] & 0xffffu) | (v[1][wdw] << 16);
        hi = (v[2][wdw] & 0xffffu) | (v[3][wdw] << 16);
      } else {
        lo = (v[0][wdw] >> 16) | (v[1][wdw] & 0xffff0000u);
        hi = (v[2][wdw] >> 16) | (v[3][wdw] & 0xffff0000u);
      }
      const u32x2 va = {lo, hi};
      st.acc[n] = mfma_k16<DT>(va, pb, st.acc[n]);
    }
  } else {
    // fp32: one 16x16x4 product per key row; k-slot = lane group.
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int n = 0; n < TILES; ++n) st.acc[n] = mfma_f32_k4(__uint_as_float(v[r][n]), p[r], st.acc[n]);
  }
}

// LDS scratch for merging NW wavefronts' states of 16 columns.
template <int NW, int D>
struct MergeSmem {
  float acc[NW][16][D + 4];
  float m[NW][16];
  float l[NW][16];
};

// Publishes this wavefront's state (after its cross-group sum of l).
template <int NW, int D>
__device__ __forceinline__ void merge_publish(MergeSmem<NW, D>& sm, const State<D>& st, int w, int g, int c) {
  constexpr int TILES = D / 16;
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int n = 0; n < TILES; ++n) sm.acc[w][c][TILES * (4 * g + r) + n] = st.acc[n][r];
  if (g == 0) {
    sm.m[w][c] = st.m;
    sm.l[w][c] = st.l;
  }
}

// Combined (M, L, o[d0..d0+3]) of column hc over the NW published states.
template <int NW, int D>
__device__ __forceinline__ void merge_column(const MergeSmem<NW, D>& sm, int hc, int d0, float& M, float& L,
                                             float (&o)[4]) {
  M = kNegInf;
#pragma unroll
  for (int w = 0; w < NW; ++w) M = fmaxf(M, sm.m[w][hc]);
  L = 0.f;
  o[0] = o[1] = o[2] = o[3] = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float mw = sm.m[w][hc];
    const float wt = mw == kNegInf ? 0.f : fast_exp2(mw - M);
    L += wt * sm.l[w][hc];
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] += wt * sm.acc[w][hc][d0 + k];
  }
}

// ---------------------------------------------------------------- device-scope partial rows
//
// Device-scope accesses for split-KV partials: written through to the device
// coherence point and read back from it, so one workgroup can merge what
// workgroups on other XCDs wrote without a cache-wide fence. They are buffer
// loads/stores with the sc1 cache policy (the bits an agent-scope relaxed
// atomic load/store carries), 8 or 16 bytes wide, through a resource over
// `base` at byte offsets below 2 GiB: a partial row moves in a quarter of the
// requests 4-byte atomics would take, and under a saturated memory system each
// request is a long round trip (16-byte accesses took the planned decode's end
// phase from 5.9 to ~4 us).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void* base) {
  // dword3 0x00020000: DATA_FORMAT 32, the raw-buffer setting of this family
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, 0x7fffffff, 0x00020000);
}
constexpr int kCacheSc1 = 16;  // cache-policy operand of the buffer builtins: sc1
__device__ __forceinline__ void store_dev4(__amdgpu_buffer_rsrc_t r, int off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCacheSc1);
}
__device__ __forceinline__ void store_dev2(__amdgpu_buffer_rsrc_t r, int off, f32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, kCacheSc1);
}
__device__ __forceinline__ f32x4 load_dev4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCacheSc1);
}
__device__ __forceinline__ f32x2 load_dev2(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kCacheSc1);
}

// Log-sum-exp merge of n partial rows read at device scope, up to NB rows'
// loads in flight at a time (only rows that exist are read): row p is row0 +
// p * step, its D fp32 accumulators at byte (row * D) * 4 of r_o and its
// (max, sum) pair at byte row * 8 of r_ml. Gives the unnormalised
// o[d0..d0+W) (W = 4 or 8) and the sum L. The arithmetic order depends on n
// alone, so merges of the same rows are bit-identical whoever runs them. Rows
// with no key (max -inf) add nothing: an exponent of -inf - -inf is NaN, which
// fmaxf turns into -1e30 (weight 0) without a branch (branches here measured
// 0.5 us per call slower).
template <int D, int W = 4, int NB = 4>
__device__ __forceinline__ void lse_merge_dev(__amdgpu_buffer_rsrc_t r_o, __amdgpu_buffer_rsrc_t r_ml, int row0,
                                              int step, int n, int d0, float (&o)[W], float& L) {
  static_assert(W == 4 || W == 8, "4 or 8 columns");
  float M = kNegInf;
  L = 0.f;
#pragma unroll
  for (int e = 0; e < W; ++e) o[e] = 0.f;
#pragma unroll 1
  for (int p0 = 0; p0 < n; p0 += NB) {
    f32x2 ml[NB];
    float po[NB][W];
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      if (q > 0 && p0 + q >= n) continue;  // the batch's first row always exists
      const int row = row0 + (p0 + q) * step;
      ml[q] = load_dev2(r_ml, row * 8);
#pragma unroll
      for (int h = 0; h < W; h += 4) {
        const f32x4 v = load_dev4(r_o, (row * D + d0 + h) * 4);
        po[q][h] = v[0];
        po[q][h + 1] = v[1];
        po[q][h + 2] = v[2];
        po[q][h + 3] = v[3];
      }
    }
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      if (p0 + q >= n) continue;
      const float Mn = fmaxf(M, ml[q][0]);
      const float wa = fast_exp2(fmaxf(M - Mn, -1e30f)), wb = fast_exp2(fmaxf(ml[q][0] - Mn, -1e30f));
      L = wa * L + wb * ml[q][1];
#pragma unroll
      for (int e = 0; e < W; ++e) o[e] = wa * o[e] + wb * po[q][e];
      M = Mn;
    }
  }
}

// Output stores are non-temporal: the next kernel reads them, so nothing is
// gained by leaving them dirty in this XCD's L2 for the end of the kernel to
// write back (measured neutral to 0.3 us faster per planned 64-sequence
// decode, neutral for the prefill).
template <int DT>
__device__ __forceinline__ void store4(uint8_t* dst, const float (&o)[4], float scale) {
  if constexpr (DT == IR_DTYPE_F32) {
    const f32x4 x = {o[0] * scale, o[1] * scale, o[2] * scale, o[3] * scale};
    __builtin_nontemporal_store(x, (f32x4*)dst);
  } else {
    using E = Elem<DT>;
    const u32x2 x = {E::pack2(o[0] * scale, o[1] * scale), E::pack2(o[2] * scale, o[3] * scale)};
    __builtin_nontemporal_store(x, (u32x2*)dst);
  }
}

}  // namespace ir
