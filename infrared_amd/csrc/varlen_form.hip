// Prefill metadata from the reference engine's packed (varlen) form.
//
// The reference's prefill paths hand the attention seam one packed frame
// (batch 1): Q query tokens, a key axis K that concatenates each scheduled
// sequence's whole history [0, start + q) in order, per-key slots and an
// additive mask (infrared/engine/paged_engine.py:461-516 with
// infrared/model/inputs.py:57-85 for a mixed step; :194-206 with
// inputs.py:33-54 for a one-sequence prefix-hit prefill):
//   gather_slots[k_off_i + p] = bt_i[p / bs] * bs + p % bs   (p < start_i + q_i)
//   mask[r, k] = 0 iff key k belongs to query r's sequence and lies at or
//                before its position, finfo(dtype).min otherwise.
// Pass 1 (ir_varlen_form_scan) reads every mask row once: row r's visible
// keys must be one contiguous range [lo_r, hi_r] and every other value at
// most -6e4 (masked in any dtype). A sequence starts where lo moves; inside
// one, each row sees one key more than the row before; the sequences' key
// ranges tile [0, K) in order. That yields cu_seqlens_q, q_start (= the first
// row's hi - lo) and each sequence's key offset, and the sizes the host needs
// (sequence count, longest chunk, widest block table); the same call then
// verifies every slot of every sequence against the closed form and the pool,
// on the device, before the host reads anything. Any violation sets
// info[0]; the host then keeps the mask kernel, which reads the metadata as
// given. With info[0] clear, the same call writes the block tables
// bt_i[j] = gather_slots[k_off_i + j bs] / bs into a buffer of the caller's
// (stride: the widest table, read on the device) when they fit, and writes
// the verdict, the sizes, cu_seqlens_q and q_start into pinned host memory
// from the device, a caller's tag last; the chunked-prefill kernel over the
// tables attends exactly the keys the mask allows. Two launches for frames of
// up to 4,096 rows (the pass over the mask, then one that segments and checks),
// three beyond; the host waits once, for the tag, and launches nothing after
// it (ir_varlen_form_tables writes tables that did not fit).
#include <algorithm>

#include "common.hpp"
#include "status.hpp"

namespace ir {
namespace {

constexpr int kScanThreads = 256;
constexpr int kSegThreads = 1024;

__device__ __forceinline__ float mask_value(const void* m, int dtype, int64_t off) {
  if (dtype == IR_DTYPE_F32) return ((const float*)m)[off];
  const uint32_t h = ((const uint16_t*)m)[off];
  return dtype == IR_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
}

// finfo(dtype).min in every element of a 32-bit word (two for 16-bit masks).
template <int DT>
constexpr uint32_t kMinWord = DT == IR_DTYPE_F32 ? 0xff7fffffu : DT == IR_DTYPE_BF16 ? 0xff7fff7fu : 0xfbfffbffu;

// Bit e of `zero`: element e of a 16-byte piece is 0 (visible); bit e of
// `bad`: it is neither 0 nor masked (at most -6e4; NaN fails both).
template <int DT>
__device__ __forceinline__ void piece_bits(u32x4 x, uint32_t& zero, uint32_t& bad) {
  constexpr int PER = DT == IR_DTYPE_F32 ? 4 : 8;
  zero = 0;
  bad = 0;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    float v;
    if constexpr (DT == IR_DTYPE_F32) {
      v = __uint_as_float(x[e]);
    } else {
      const uint32_t h = (x[e >> 1] >> (16 * (e & 1))) & 0xffffu;
      v = DT == IR_DTYPE_BF16 ? bf16_to_f32(h) : f16_to_f32(h);
    }
    zero |= (uint32_t)(v == 0.f) << e;
    bad |= (uint32_t)(v != 0.f && !(v <= -6e4f)) << e;
  }
}

// Per-row record of the scan, zero at rest (every scan leaves it zero):
// INT_MAX - first visible key, last visible key + 1, their count, and whether
// any value is neither visible nor masked -- encoded so that the empty record
// is all zeros and every update is an atomic max, max, add or or.
struct RowRec {
  int first_c, last1, count, wrong;
};
constexpr int kFirstBias = 0x7fffffff;

// Wavefront reduction with no LDS round trip: DPP permutations inside each
// 16-lane row (lane ^ 1, lane ^ 2, then each 8-lane half mirrored, then the
// row mirrored), then gfx950's row swaps (rows 0<->1 and 2<->3, then the two
// 32-lane halves; both outputs of a swap are combined, so which carries which
// does not matter for a symmetric op). Every lane ends with the result; all
// 64 lanes must be active.
template <typename Op>
__device__ __forceinline__ int wave_fold(int x, Op op) {
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0xb1, 0xf, 0xf, false));   // quad_perm [1, 0, 3, 2]
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x4e, 0xf, 0xf, false));   // quad_perm [2, 3, 0, 1]
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x141, 0xf, 0xf, false));  // row_half_mirror
  x = op(x, __builtin_amdgcn_update_dpp(0, x, 0x140, 0xf, 0xf, false));  // row_mirror
  const auto b = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
  x = op((int)b[0], (int)b[1]);
  const auto a = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
  return op((int)a[0], (int)a[1]);
}

// A row's share of a run of visible keys [k_lo, k_hi] (count keys) and of
// wrong values, added to its record.
__device__ __forceinline__ void rec_add(RowRec* rec, int r, int k_lo, int k_hi, int count, int wrong) {
  if (count) {
    atomicMax(&rec[r].first_c, kFirstBias - k_lo);
    atomicMax(&rec[r].last1, k_hi + 1);
    atomicAdd(&rec[r].count, count);
  }
  if (wrong) atomicOr(&rec[r].wrong, 1);
}

// One row's part of a wavefront's pieces, folded over the wavefront and added
// to the row's record by lane 0.
__device__ __forceinline__ void wave_rec_add(RowRec* rec, int r, int f, int l, int n, int wr) {
  f = wave_fold(f, [](int a, int b) { return min(a, b); });
  l = wave_fold(l, [](int a, int b) { return max(a, b); });
  n = wave_fold(n, [](int a, int b) { return a + b; });
  const int any_wrong = __ballot(wr != 0) != 0ull;
  if ((threadIdx.x & 63) == 0) rec_add(rec, r, f, l, n, any_wrong);
}

// The scan's first kernel clears the verdict word and the workgroup ticket
// the verification counts on (the kernels after it read them).
__device__ __forceinline__ void clear_verdict(int32_t* info) {
  info[0] = 0;
  info[5] = 0;
}

// Contiguous masks: the flat [Q * K] array as 16-byte pieces, grid-stride.
// A wavefront takes 64 * kFlatPieces consecutive pieces per pass (each load
// instruction 1 KiB contiguous), all in flight before any is inspected. A
// piece that is all finfo.min -- nearly all of them -- costs an OR and an
// AND of its words; a wavefront whose pieces hold no visible key and no bad
// value moves on without any reduction. Otherwise each lane describes its
// piece as a run of visible keys in at most two rows (a piece straddles a row
// end when K is not a multiple of its elements), and the wavefront folds the
// lanes of the first two rows it touches into one atomic update per row
// (rows shorter than 64 pieces fall back to an update per lane). NARROW: the
// element index fits 31 bits.
constexpr int kFlatThreads = 256;
constexpr int kFlatPieces = 8;

template <int DT, bool NARROW>
__global__ __launch_bounds__(kFlatThreads) void varlen_flat_kernel(const u32x4* pieces, int64_t whole, int K, RowRec* rec,
                                                                  int32_t* info) {
  constexpr int PER = DT == IR_DTYPE_F32 ? 4 : 8;
  if (blockIdx.x == 0 && threadIdx.x == 0) clear_verdict(info);
  constexpr uint32_t M = kMinWord<DT>;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (kFlatThreads / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * (kFlatThreads / 64);
  constexpr int64_t kSpan = 64 * kFlatPieces;
  auto row_of = [&](int64_t e) -> int { return NARROW ? (int)((uint32_t)e / (uint32_t)K) : (int)(e / K); };
  for (int64_t base = wave * kSpan; base < whole; base += nwaves * kSpan) {
    const bool full = base + kSpan <= whole;  // uniform: every piece of the span exists
    const char* p = (const char*)(pieces + base);  // uniform base, unsigned 32-bit lane offsets
    u32x4 x[kFlatPieces];
    if (full) {
#pragma unroll
      for (int i = 0; i < kFlatPieces; ++i) x[i] = load_nt((const u32x4*)(p + (uint32_t)(i * 64 + lane) * 16u));
    } else {
      const int last = (int)(whole - 1 - base);
#pragma unroll
      for (int i = 0; i < kFlatPieces; ++i)
        x[i] = load_nt((const u32x4*)(p + (uint32_t)min(i * 64 + lane, last) * 16u));
    }
    // the common case: every piece of the span all finfo(dtype).min
    uint32_t special = 0;
#pragma unroll
    for (int i = 0; i < kFlatPieces; ++i)
      special |= ((x[i][0] | x[i][1] | x[i][2] | x[i][3]) ^ M) | ((x[i][0] & x[i][1] & x[i][2] & x[i][3]) ^ M);
    if (full && __ballot(special != 0u) == 0ull) continue;  // uniform
    // rows the span touches: with rows at least a span long, at most two, and
    // each lane folds its pieces into both before one wavefront reduction
    const int r0 = row_of(base * PER);
    const int r1 = row_of(min(base + kSpan, whole) * PER - 1);
    if (r1 - r0 <= 1) {  // uniform
      const int64_t b1 = (int64_t)(r0 + 1) * K;  // first element of row r0 + 1
      int f[2] = {K, K}, l[2] = {-1, -1}, n[2] = {0, 0}, wr[2] = {0, 0};
#pragma unroll
      for (int i = 0; i < kFlatPieces; ++i) {
        const int64_t c = base + i * 64 + lane;
        const uint32_t any = x[i][0] | x[i][1] | x[i][2] | x[i][3];
        const uint32_t all = x[i][0] & x[i][1] & x[i][2] & x[i][3];
        if (c >= whole || (any == M && all == M)) continue;
        uint32_t zero = (1u << PER) - 1u, bad = 0;
        if (any != 0u) piece_bits<DT>(x[i], zero, bad);
        const int64_t e0 = c * PER;
        const int split = (int)max((int64_t)0, min((int64_t)PER, b1 - e0));  // elements in row r0
        const uint32_t in_a = (1u << split) - 1u;
        const uint32_t za = zero & in_a, zb = zero & ~in_a;
        if (za) {
          const int k0 = (int)(e0 - (b1 - K));
          f[0] = min(f[0], k0 + __builtin_ctz(za));
          l[0] = max(l[0], k0 + 31 - __builtin_clz(za));
          n[0] += __builtin_popcount(za);
        }
        if (zb) {
          const int k0 = (int)(e0 - b1);
          f[1] = min(f[1], k0 + __builtin_ctz(zb));
          l[1] = max(l[1], k0 + 31 - __builtin_clz(zb));
          n[1] += __builtin_popcount(zb);
        }
        wr[0] |= (bad & in_a) != 0u;
        wr[1] |= (bad & ~in_a) != 0u;
      }
      wave_rec_add(rec, r0, f[0], l[0], n[0], wr[0]);
      if (r1 > r0) wave_rec_add(rec, r1, f[1], l[1], n[1], wr[1]);  // uniform
      continue;
    }
    // rows shorter than a span: each load instruction's 64 pieces on their own
#pragma unroll
    for (int i = 0; i < kFlatPieces; ++i) {
      const int64_t c = base + i * 64 + lane;
      const bool in = c < whole;
      const uint32_t any = x[i][0] | x[i][1] | x[i][2] | x[i][3];
      const uint32_t all = x[i][0] & x[i][1] & x[i][2] & x[i][3];
      uint32_t zero = 0, bad = 0;
      if (in && !(any == M && all == M)) {
        if (any == 0u) zero = (1u << PER) - 1u;
        else piece_bits<DT>(x[i], zero, bad);
      }
      if (__ballot((zero | bad) != 0u) == 0ull) continue;  // uniform
      // the wavefront's first row and the row of its last element
      const int64_t c_first = base + i * 64;
      const int r0 = row_of(c_first * PER);
      const int64_t c_last = min(c_first + 63, whole - 1);
      const int r_end = row_of(c_last * PER + PER - 1);
      // this lane's piece: elements e0 .. e0 + PER - 1, row ra up to key
      // K - 1, then (rows of at least 64 pieces) row ra + 1; split = its
      // elements in row ra
      const int64_t e0 = c * PER;
      const int ra = row_of(e0);
      const int k0 = (int)(e0 - (int64_t)ra * K);
      const int split = min(PER, K - k0);
      const uint32_t in_a = (1u << split) - 1u;
      const uint32_t za = zero & in_a, zb = zero & ~in_a;
      const int wa = (bad & in_a) != 0u, wb = (bad & ~in_a) != 0u;
      if (r_end - r0 > 1) {  // short rows (a piece may span several): one update per element
        for (uint32_t bits = zero | bad; bits; bits &= bits - 1u) {
          const int e = __builtin_ctz(bits);
          const int r = row_of(e0 + e), k = (int)(e0 + e - (int64_t)r * K);
          if ((zero >> e) & 1u) rec_add(rec, r, k, k, 1, 0);
          else rec_add(rec, r, 0, 0, 0, 1);
        }
        continue;
      }
      // fold into rows r0 (slot 0) and r0 + 1 (slot 1)
      int f[2] = {K, K}, l[2] = {-1, -1}, n[2] = {0, 0}, wr[2] = {0, 0};
      const int sa = ra - r0;  // 0 or 1
      if (za) {
        f[sa] = k0 + __builtin_ctz(za);
        l[sa] = k0 + 31 - __builtin_clz(za);
        n[sa] = __builtin_popcount(za);
      }
      wr[sa] |= wa;
      if (sa == 0) {  // the second part of a straddling piece belongs to r0 + 1
        if (zb) {
          f[1] = __builtin_ctz(zb) - split;
          l[1] = 31 - __builtin_clz(zb) - split;
          n[1] = __builtin_popcount(zb);
        }
        wr[1] |= wb;
      }
      wave_rec_add(rec, r0, f[0], l[0], n[0], wr[0]);
      if (r_end > r0) wave_rec_add(rec, r0 + 1, f[1], l[1], n[1], wr[1]);  // uniform
    }
  }
}

// The array's last partial piece (Q * K not a multiple of a piece), element by
// element, and strided masks: one workgroup per row.
__global__ __launch_bounds__(64) void varlen_tail_kernel(const void* mask, int dtype, int64_t e_from, int64_t e_to,
                                                          int K, RowRec* rec, int32_t* info) {
  if (threadIdx.x == 0) clear_verdict(info);
  for (int64_t e = e_from + threadIdx.x; e < e_to; e += 64) {
    const float x = mask_value(mask, dtype, e);
    const int r = (int)(e / K), k = (int)(e - (int64_t)r * K);
    if (x == 0.f) rec_add(rec, r, k, k, 1, 0);
    else if (!(x <= -6e4f)) rec_add(rec, r, 0, 0, 0, 1);
  }
}

__global__ __launch_bounds__(kScanThreads) void varlen_rows_strided_kernel(const void* mask, int dtype, int64_t m_q,
                                                                          int64_t m_k, int K, RowRec* rec,
                                                                          int32_t* info) {
  __shared__ int s_first, s_last, s_count, s_wrong;
  const int r = blockIdx.x, tid = threadIdx.x;
  if (r == 0 && tid == 0) clear_verdict(info);
  if (tid == 0) {
    s_first = K;
    s_last = -1;
    s_count = 0;
    s_wrong = 0;
  }
  __syncthreads();
  int first = K, last = -1, count = 0, wrong = 0;
  const int64_t row = (int64_t)r * m_q;
  for (int k = tid; k < K; k += kScanThreads) {
    const float x = mask_value(mask, dtype, row + (int64_t)k * m_k);
    if (x == 0.f) {
      first = min(first, k);
      last = max(last, k);
      ++count;
    } else {
      wrong |= !(x <= -6e4f);
    }
  }
  if (count) {
    atomicMin(&s_first, first);
    atomicMax(&s_last, last);
    atomicAdd(&s_count, count);
  }
  if (wrong) s_wrong = 1;
  __syncthreads();
  if (tid == 0) rec[r] = s_count ? RowRec{kFirstBias - s_first, s_last + 1, s_count, s_wrong} : RowRec{0, 0, 0, s_wrong};
}

// One workgroup: rows -> sequences, then the longest chunk and the widest
// table; info[0..3] written whole (no clearing before the pass). A row is
// usable when its visible keys are one contiguous range; a sequence starts
// where that range's first key moves. A thread takes kSegRows consecutive
// rows per pass (their records and the one before requested together), and
// the sequences a pass starts are numbered with a block-wide scan of the
// threads' counts (wavefront prefix sums, then the wavefronts' totals): two
// barriers per pass of kSegThreads * kSegRows rows.
constexpr int kSegRows = 4;
__global__ __launch_bounds__(kSegThreads) void varlen_segments_kernel(RowRec* rec, int Q, int K, int bs,
                                                                     int32_t* cu, int32_t* q_start, int32_t* seq_lo,
                                                                     int32_t* info) {
  constexpr int NWV = kSegThreads / 64;
  __shared__ int s_wave[NWV];
  __shared__ int s_base, s_bad, s_maxq, s_maxb;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid == 0) {
    s_base = 0;
    s_bad = 0;
    s_maxq = 0;
    s_maxb = 0;
  }
  __syncthreads();
  auto range = [](const RowRec& x, int& lo, int& hi) {
    const int first = kFirstBias - x.first_c, last = x.last1 - 1;
    const bool bad = x.wrong || x.count == 0 || last - first + 1 != x.count;
    lo = bad ? -1 : first;
    hi = bad ? -1 : last;
  };
  for (int c0 = 0; c0 < Q; c0 += kSegThreads * kSegRows) {
    const int r0 = c0 + tid * kSegRows;
    RowRec x[kSegRows + 1];  // the row before this thread's first, then its rows
#pragma unroll
    for (int j = 0; j <= kSegRows; ++j) {
      const int r = r0 - 1 + j;
      const RowRec y = rec[min(max(r, 0), Q - 1)];  // unconditional: the loads stay in flight together
      x[j] = r >= 0 && r < Q ? y : RowRec{0, 0, 0, 0};
    }
    int lo[kSegRows + 1], hi[kSegRows + 1], start[kSegRows];
    range(x[0], lo[0], hi[0]);
    if (r0 == 0) lo[0] = hi[0] = -1;
    int mine = 0;
#pragma unroll
    for (int j = 0; j < kSegRows; ++j) {
      const int r = r0 + j;
      range(x[j + 1], lo[j + 1], hi[j + 1]);
      start[j] = 0;
      if (r < Q) {
        start[j] = r == 0 || lo[j + 1] != lo[j];
        // a row whose own scan failed; a new sequence's keys follow the last
        // one's; a row of the same sequence sees one key more than the row before
        if (lo[j + 1] < 0 || (start[j] ? lo[j + 1] != hi[j] + 1 : hi[j + 1] != hi[j] + 1)) s_bad = 1;
        if (r == Q - 1 && hi[j + 1] != K - 1) s_bad = 1;  // the key axis ends with the last sequence
        mine += start[j];
      }
    }
    // exclusive prefix of `mine` over the block
    int incl = mine;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (lane >= o) incl += y;
    }
    if (lane == 63) s_wave[wv] = incl;
    __syncthreads();
    int i = s_base + incl - mine;
    for (int v = 0; v < wv; ++v) i += s_wave[v];
#pragma unroll
    for (int j = 0; j < kSegRows; ++j) {
      if (start[j]) {
        cu[i] = r0 + j;
        seq_lo[i] = lo[j + 1];
        q_start[i] = hi[j + 1] - lo[j + 1];
        ++i;
      }
    }
    __syncthreads();
    if (tid == 0) {
      int t = 0;
      for (int v = 0; v < NWV; ++v) t += s_wave[v];
      s_base += t;
    }
    __syncthreads();
  }
  const int nseq = s_base;
  if (tid == 0) cu[nseq] = Q;
  // every record read: leave them zero for the next scan
  for (int r = tid; r < Q; r += kSegThreads) rec[r] = RowRec{0, 0, 0, 0};
  __syncthreads();
  for (int i = tid; i < nseq; i += kSegThreads) {
    const int q = cu[i + 1] - cu[i];
    const int t = q_start[i] + q;
    atomicMax(&s_maxq, q);
    atomicMax(&s_maxb, (t + bs - 1) / bs);
  }
  __syncthreads();
  if (tid == 0) {
    info[0] = s_bad;
    info[1] = nseq;
    info[2] = s_maxq;
    info[3] = s_maxb;
    info[5] = 0;  // the check's workgroup ticket
  }
}

// Every key of the axis against the closed form: key k of sequence i (found
// by binary search of the sequences' first keys, staged in LDS when they fit)
// at position p = k - k_off_i must hold bt_i[p / bs] * bs + p % bs, where
// bt_i[j] = gather_slots[k_off_i + j * bs] / bs is a block id in the pool.
// ORs 1 into info[0] on any violation. The sequence count comes from info[1].
// The same grid writes the block tables, entry e = i * W + j of [info[1], W]
// (W = max(info[3], 1); zero past the sequence's keys), when they fit in
// `cap`. The last workgroup to finish (a ticket in info[5], which the
// segmentation zeroes) publishes info[4] (tables written) and, into the host
// record, the verdict, the sizes, cu_seqlens_q and q_start, then, after a
// system-scope fence, the caller's tag, so a host that polls the tag reads a
// whole record without synchronising the stream.
constexpr int kCheckStage = 4096;

// The host record, by the first wavefront of the (last) workgroup: the
// verdict and the sizes at [0..4], cu_seqlens_q at [8..8+n] and q_start at
// [9+n..9+2n) when the form holds, then, after a system-scope fence (the
// wavefront's stores all complete before it goes on), `tag` at [7], so a host
// that polls the tag reads a whole record. cu / q_start may point at LDS. The
// other wavefronts return at once.
__device__ void publish_record(int32_t* host, int bad, int nseq, int maxq, int width, bool written, const int32_t* cu,
                               const int32_t* q_start, int32_t tag) {
  const int lane = threadIdx.x;
  if (lane >= 64) return;
  if (lane < 7)
    host[lane] = lane == 0 ? bad : lane == 1 ? nseq : lane == 2 ? maxq : lane == 3 ? width : lane == 4 ? (int)written : 0;
  if (bad == 0 && nseq > 0) {
    for (int i = lane; i <= nseq; i += 64) host[8 + i] = cu[i];
    for (int i = lane; i < nseq; i += 64) host[9 + nseq + i] = q_start[i];
  }
  __threadfence_system();
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) *(volatile int32_t*)&host[7] = tag;
}

__global__ __launch_bounds__(kScanThreads) void varlen_check_kernel(const int64_t* gs, int64_t gs_k,
                                                                   const int32_t* seq_lo, const int32_t* cu,
                                                                   const int32_t* q_start, int K, int bs,
                                                                   int64_t num_blocks, int32_t* info, int32_t* bt,
                                                                   int cap, int32_t* host, int32_t tag) {
  __shared__ int s_lo[kCheckStage];
  __shared__ int s_bad, s_last;
  const int tid = threadIdx.x;
  const int nseq = info[1], maxq = info[2], width = info[3];
  const bool go = info[0] == 0 && nseq > 0;  // uniform: otherwise the scan already failed
  const int w = max(width, 1);
  const bool fits = go && bt != nullptr && (int64_t)nseq * w <= cap;
  const bool staged = nseq <= kCheckStage;
  if (tid == 0) s_bad = 0;
  if (go && staged)
    for (int i = tid; i < nseq; i += kScanThreads) s_lo[i] = seq_lo[i];
  __syncthreads();
  if (go) {
    const int k = blockIdx.x * kScanThreads + tid;
    if (k < K) {
      int lo = 0, hi = nseq - 1;  // the last sequence whose first key is <= k
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((staged ? s_lo[mid] : seq_lo[mid]) <= k) lo = mid;
        else hi = mid - 1;
      }
      const int64_t off = staged ? s_lo[lo] : seq_lo[lo];
      const int p = (int)(k - off);
      const int64_t head = gs[(off + (int64_t)(p / bs) * bs) * gs_k];
      const int64_t id = head / bs;
      if (p < 0 || head < 0 || head % bs != 0 || id >= num_blocks || gs[(int64_t)k * gs_k] != id * bs + p % bs)
        s_bad = 1;
    }
    if (fits) {
      // the segmentation found the sequences' key ranges tiling [0, K): sequence
      // i's keys are [k_off_i, k_off_{i+1}), the last one's end at K
      const unsigned n = (unsigned)(nseq * w);
      for (unsigned e = blockIdx.x * kScanThreads + tid; e < n; e += gridDim.x * kScanThreads) {
        const int i = (int)(e / (unsigned)w), j = (int)(e - (unsigned)i * w);
        const int lo = staged ? s_lo[i] : seq_lo[i];
        const int end = i + 1 < nseq ? (staged ? s_lo[i + 1] : seq_lo[i + 1]) : K;
        const int p = j * bs;
        bt[e] = p < end - lo ? (int32_t)(gs[(int64_t)(lo + p) * gs_k] / bs) : 0;
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    if (s_bad) atomicOr(&info[0], 1);
    __threadfence();
    s_last = atomicAdd(&info[5], 1) == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int bad = atomicOr(&info[0], 0);  // every workgroup's verdict is in
  const bool ok = bad == 0 && nseq > 0;
  if (tid == 0) info[4] = ok && fits;
  if (host != nullptr) publish_record(host, bad, nseq, maxq, width, ok && fits, cu, q_start, tag);
}

// Frames of at most kVerifyRows rows: the segmentation and the slot check in
// one launch. Every workgroup segments the rows itself, in LDS, from the row
// records (64 KiB at most, read by each), so no workgroup waits for another:
// workgroup 0 writes cu_seqlens_q, q_start, the sequences' first keys and
// info[1..3]; each workgroup checks its keys (grid-stride, at most one
// workgroup per CU) and writes their block-table entries. The workgroups
// count themselves, and the failed ones, in one ticket word (info[5], cleared
// by the scan): the last to arrive knows the verdict from its ticket, writes
// info[0] and info[4], zeroes the row records for the next call and publishes
// the host record.
//
// The rules are the segmentation kernel's, and the check kernel's closed form
// stated key by key, so that every slot a thread needs is loaded before the
// segmentation is known: key k at position p of its sequence holds a block
// head (>= 0, a multiple of bs, block id < num_blocks) when p % bs == 0 and
// gather_slots[k - 1] + 1 otherwise -- by induction over each block, the same
// as gather_slots[k] = bt[p / bs] * bs + p % bs with bt[j] the block id of the
// sequence's key j * bs. A key at a block head writes that table entry.
// Loads and LDS reads are issued unconditionally (indices clamped into range,
// results selected after): a load under a per-lane condition ends in a wait for
// it, which would serialise the record reads.
constexpr int kVerifyThreads = 1024;
constexpr int kVerifyRowsPer = 4;
constexpr int kVerifyRows = kVerifyThreads * kVerifyRowsPer;
constexpr int kTicketBad = 1 << 16;  // a failed workgroup's share of the ticket (grids of < 2^16)

// slot / bs and slot % bs, in 32 bits when the slot allows
__device__ __forceinline__ void slot_divmod(int64_t g, int bs, int64_t& q, int& r) {
  if ((uint64_t)g < 0x80000000ull) {
    const uint32_t u = (uint32_t)g, d = u / (uint32_t)bs;
    q = d;
    r = (int)(u - d * (uint32_t)bs);
  } else {
    q = g / bs;
    r = (int)(g - q * bs);
  }
}

__global__ __launch_bounds__(kVerifyThreads) void varlen_verify_kernel(RowRec* rec, int Q, const int64_t* gs,
                                                                    int64_t gs_k, int K, int bs, int64_t num_blocks,
                                                                    int32_t* cu, int32_t* q_start, int32_t* seq_lo,
                                                                    int32_t* info, int32_t* bt, int cap,
                                                                    int32_t* host, int32_t tag) {
  constexpr int NW = kVerifyThreads / 64;
  // rows' visible ranges (-1 when unusable), then the sequences' first rows and keys
  __shared__ int32_t s_rlo[kVerifyRows], s_rhi[kVerifyRows], s_cu[kVerifyRows + 1], s_lo[kVerifyRows];
  __shared__ int32_t s_qs[kVerifyRows];
  __shared__ __align__(16) int s_cnt[kVerifyRowsPer * NW];
  __shared__ int s_rows_bad, s_keys_bad, s_maxq, s_maxb, s_ticket;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // every load first: rows c * kVerifyThreads + tid, and this thread's first key and the one before it
  RowRec x[kVerifyRowsPer];
#pragma unroll
  for (int c = 0; c < kVerifyRowsPer; ++c) x[c] = rec[min(c * kVerifyThreads + tid, Q - 1)];
  const int k_first = blockIdx.x * kVerifyThreads + tid;
  int64_t g_here = -1, g_prev = -1;
  if (K > 0) {  // uniform
    const int kc = min(k_first, K - 1);
    g_here = gs[(int64_t)kc * gs_k];
    g_prev = gs[(int64_t)max(kc - 1, 0) * gs_k];
  }
  if (tid == 0) {
    s_rows_bad = 0;
    s_keys_bad = 0;
    s_maxq = 0;
    s_maxb = 0;
  }
#pragma unroll
  for (int c = 0; c < kVerifyRowsPer; ++c) {
    const int r = c * kVerifyThreads + tid;
    const int first = kFirstBias - x[c].first_c, last = x[c].last1 - 1;
    const bool unusable = x[c].wrong || x[c].count == 0 || last - first + 1 != x[c].count;
    if (r < Q) {
      s_rlo[r] = unusable ? -1 : first;
      s_rhi[r] = unusable ? -1 : last;
    }
  }
  __syncthreads();
  // sequence starts, row by row against the row before; numbered in row order.
  // Every range is read first and the rules are evaluated without branches.
  int lo[kVerifyRowsPer], hi[kVerifyRowsPer];
  uint32_t starts = 0;
  int bad = 0, rank[kVerifyRowsPer];
  {
    int lo_p[kVerifyRowsPer], hi_p[kVerifyRowsPer];
#pragma unroll
    for (int c = 0; c < kVerifyRowsPer; ++c) {
      const int rc = min(c * kVerifyThreads + tid, Q - 1), rp = max(rc - 1, 0);
      lo[c] = s_rlo[rc];
      hi[c] = s_rhi[rc];
      lo_p[c] = s_rlo[rp];
      hi_p[c] = s_rhi[rp];
    }
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int c = 0; c < kVerifyRowsPer; ++c) {
      const int r = c * kVerifyThreads + tid;
      const int in = r < Q, first = r == 0;
      const int lp = first ? -1 : lo_p[c], hp = first ? -1 : hi_p[c];
      const int st = in & (first | (lo[c] != lp));
      // a row whose own scan failed; a new sequence's keys follow the last
      // one's; a row of the same sequence sees one key more than the row before;
      // the key axis ends with the last sequence
      const int broken = st ? lo[c] != hp + 1 : hi[c] != hp + 1;
      bad |= in & ((lo[c] < 0) | broken | ((r == Q - 1) & (hi[c] != K - 1)));
      const uint64_t m = __ballot(st);
      rank[c] = __popcll(m & below);
      starts |= (uint32_t)st << c;
      if (lane == 0) s_cnt[c * NW + wv] = __popcll(m);
    }
  }
  if (bad) s_rows_bad = 1;
  __syncthreads();
  int cnt[kVerifyRowsPer * NW];
#pragma unroll
  for (int e = 0; e < kVerifyRowsPer * NW; e += 4) {
    const int4 v = *(const int4*)&s_cnt[e];
    cnt[e] = v.x;
    cnt[e + 1] = v.y;
    cnt[e + 2] = v.z;
    cnt[e + 3] = v.w;
  }
  int nseq = 0;
#pragma unroll
  for (int c = 0; c < kVerifyRowsPer; ++c) {
    int before = 0;
#pragma unroll
    for (int v = 0; v < NW; ++v) before += v < wv ? cnt[c * NW + v] : 0;
    if ((starts >> c) & 1u) {
      const int i = nseq + before + rank[c];
      s_cu[i] = c * kVerifyThreads + tid;
      s_lo[i] = lo[c];
      s_qs[i] = hi[c] - lo[c];
    }
#pragma unroll
    for (int v = 0; v < NW; ++v) nseq += cnt[c * NW + v];
  }
  if (tid == 0) s_cu[nseq] = Q;
  __syncthreads();
  // the longest chunk and the widest table
  int mq = 0, mb = 0;
  for (int e = tid; e < nseq; e += kVerifyThreads) {
    const int q = s_cu[e + 1] - s_cu[e];
    mq = max(mq, q);
    mb = max(mb, (s_qs[e] + q + bs - 1) / bs);
  }
  mq = wave_fold(mq, [](int a, int b) { return max(a, b); });
  mb = wave_fold(mb, [](int a, int b) { return max(a, b); });
  if (lane == 0) {
    atomicMax(&s_maxq, mq);
    atomicMax(&s_maxb, mb);
  }
  __syncthreads();
  const int maxq = s_maxq, width = s_maxb;
  const bool rows_ok = s_rows_bad == 0;  // uniform
  if (blockIdx.x == 0) {
    for (int e = tid; e <= nseq; e += kVerifyThreads) cu[e] = s_cu[e];
    for (int e = tid; e < nseq; e += kVerifyThreads) {
      q_start[e] = s_qs[e];
      seq_lo[e] = s_lo[e];
    }
    if (tid == 0) {
      info[1] = nseq;
      info[2] = maxq;
      info[3] = width;
    }
  }
  const int w = max(width, 1);
  const bool fits = rows_ok && bt != nullptr && (int64_t)nseq * w <= cap;
  if (rows_ok) {
    int keys_bad = 0;
    for (int k = k_first; k < K; k += gridDim.x * kVerifyThreads) {
      if (k != k_first) {
        g_here = gs[(int64_t)k * gs_k];
        g_prev = gs[(int64_t)(k - 1) * gs_k];
      }
      int a = 0, b = nseq - 1;  // the last sequence whose first key is <= k
      while (a < b) {
        const int mid = (a + b + 1) >> 1;
        if (s_lo[mid] <= k) a = mid;
        else b = mid - 1;
      }
      const int p = k - s_lo[a];
      if (p < 0) {
        keys_bad = 1;
      } else if (p % bs == 0) {
        int64_t id;
        int off;
        slot_divmod(g_here, bs, id, off);
        if (g_here < 0 || off != 0 || id >= num_blocks) keys_bad = 1;
        if (fits) bt[a * w + p / bs] = (int32_t)id;
      } else if (g_here != g_prev + 1) {
        keys_bad = 1;
      }
    }
    if (keys_bad) s_keys_bad = 1;
    if (fits) {
      // entries past each sequence's last block
      const unsigned n = (unsigned)(nseq * w);
      for (unsigned e = blockIdx.x * kVerifyThreads + tid; e < n; e += gridDim.x * kVerifyThreads) {
        const int sq = (int)(e / (unsigned)w), j = (int)(e - (unsigned)sq * w);
        const int end = sq + 1 < nseq ? s_lo[sq + 1] : K;
        if (j * bs >= end - s_lo[sq]) bt[e] = 0;
      }
    }
  }
  __syncthreads();
  const bool failed = !rows_ok || s_keys_bad != 0;  // uniform
  if (tid == 0) {
    __threadfence();
    s_ticket = atomicAdd(&info[5], 1 + (failed ? kTicketBad : 0)) + 1 + (failed ? kTicketBad : 0);
  }
  __syncthreads();
  const int ticket = s_ticket;
  if ((ticket & (kTicketBad - 1)) != (int)gridDim.x) return;
  __threadfence();
  const int verdict = ticket >= kTicketBad;  // some workgroup failed
  const bool ok = verdict == 0 && nseq > 0;
  if (tid == 0) {
    info[0] = verdict;
    info[4] = ok && fits;
  }
  if (host != nullptr) publish_record(host, verdict, nseq, maxq, width, ok && fits, s_cu, s_qs, tag);
  // every workgroup has read the row records: leave them zero for the next
  // scan (after the record, which the host may be waiting for)
  for (int r = tid; r < Q; r += kVerifyThreads) rec[r] = RowRec{0, 0, 0, 0};
}

// Workgroup (i, y): entries of sequence i's table whose first key lies in
// keys [y * kTableKeys, (y + 1) * kTableKeys).
constexpr int kTableKeys = 2048;
__global__ __launch_bounds__(kScanThreads) void varlen_tables_kernel(const int64_t* gs, int64_t gs_k,
                                                                    const int32_t* seq_lo, const int32_t* cu,
                                                                    const int32_t* q_start, int bs, int32_t* bt,
                                                                    int64_t bt_stride, int width) {
  const int i = blockIdx.x, tid = threadIdx.x;
  const int64_t lo = seq_lo[i];
  const int t_len = q_start[i] + (cu[i + 1] - cu[i]);
  const int t0 = blockIdx.y * kTableKeys;
  const int j0 = (t0 + bs - 1) / bs, j1 = min((t0 + kTableKeys + bs - 1) / bs, width);
  for (int j = j0 + tid; j < j1; j += kScanThreads) {
    const int p = j * bs;
    bt[(int64_t)i * bt_stride + j] = p < t_len ? (int32_t)(gs[(lo + p) * gs_k] / bs) : 0;
  }
}

// The flat scan with no more workgroups than stay resident on the device at
// once (occupancy queried once per instance): its grid-stride loop then never
// waits for a second round of workgroups to start after the first.
template <int DT, bool NARROW>
void launch_flat(const u32x4* pc, int64_t whole, int K, RowRec* rec, int32_t* info, hipStream_t s) {
  static const int per_cu = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void*>(&varlen_flat_kernel<DT, NARROW>),
                                                     kFlatThreads, 0) != hipSuccess || n < 1)
      n = 1;
    return n;
  }();
  constexpr int kWaves = kFlatThreads / 64;
  const int64_t spans = (whole + 64 * kFlatPieces - 1) / (64 * kFlatPieces);
  const int64_t wgs = std::min<int64_t>((spans + kWaves - 1) / kWaves, (int64_t)device_cus() * per_cu);
  hipLaunchKernelGGL((varlen_flat_kernel<DT, NARROW>), dim3((unsigned)wgs), dim3(kFlatThreads), 0, s, pc, whole, K,
                     rec, info);
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_varlen_form_scan(const void* mask, int64_t mask_q_stride, int64_t mask_k_stride, int mask_dtype,
                                   int num_q, int num_k, const int64_t* gather_slots, int64_t gs_k_stride,
                                   int block_size, int64_t num_blocks, int32_t* row_records, int32_t* cu_seqlens_q,
                                   int32_t* q_start, int32_t* seq_k_offsets, int32_t* info, int32_t* block_tables,
                                   int64_t tables_capacity, int32_t* host_record, int64_t host_capacity,
                                   int32_t tag, ir_stream_t stream) {
  IR_REQUIRE(dtype_bytes(mask_dtype) > 0, "ir_varlen_form_scan: unknown mask dtype %d", mask_dtype);
  IR_REQUIRE(num_q >= 0 && num_k >= 0 && block_size > 0 && num_blocks >= 0 && tables_capacity >= 0,
             "ir_varlen_form_scan: bad sizes");
  if (num_q == 0) return ok();
  IR_REQUIRE(mask && gather_slots && row_records && cu_seqlens_q && q_start && seq_k_offsets && info,
             "ir_varlen_form_scan: null pointer");
  IR_REQUIRE(((uintptr_t)row_records & 15) == 0, "ir_varlen_form_scan: row_records must be 16-byte aligned");
  IR_REQUIRE(host_record == nullptr || host_capacity >= 2 * (int64_t)num_q + 9,
             "ir_varlen_form_scan: host_record holds %lld int32, needs %lld", (long long)host_capacity,
             2 * (long long)num_q + 9);
  int32_t* host_dev = nullptr;
  if (host_record != nullptr) {
    const hipError_t e = hipHostGetDevicePointer((void**)&host_dev, host_record, 0);
    if (e != hipSuccess) {
      (void)hipGetLastError();  // not left for the next launch check to report
      return fail(IR_EINVAL, "ir_varlen_form_scan: host_record is not pinned host memory: %s", hipGetErrorString(e));
    }
  }
  hipStream_t s = (hipStream_t)stream;
  RowRec* rec = (RowRec*)row_records;
  const int per = 16 / dtype_bytes(mask_dtype);
  // contiguous rows from a 16-byte-aligned start: the flat array as 16-byte pieces
  const bool flat = num_k > 0 && mask_k_stride == 1 && mask_q_stride == num_k && ((uintptr_t)mask & 15) == 0;
  if (flat) {
    const int64_t elems = (int64_t)num_q * num_k, whole = elems / per;
    if (whole > 0) {
      const bool narrow = elems + 64 * kFlatPieces * per < ((int64_t)1 << 31);
      const u32x4* pc = (const u32x4*)mask;
      if (mask_dtype == IR_DTYPE_F32) {
        if (narrow) launch_flat<IR_DTYPE_F32, true>(pc, whole, num_k, rec, info, s);
        else launch_flat<IR_DTYPE_F32, false>(pc, whole, num_k, rec, info, s);
      } else if (mask_dtype == IR_DTYPE_BF16) {
        if (narrow) launch_flat<IR_DTYPE_BF16, true>(pc, whole, num_k, rec, info, s);
        else launch_flat<IR_DTYPE_BF16, false>(pc, whole, num_k, rec, info, s);
      } else {
        if (narrow) launch_flat<IR_DTYPE_F16, true>(pc, whole, num_k, rec, info, s);
        else launch_flat<IR_DTYPE_F16, false>(pc, whole, num_k, rec, info, s);
      }
    }
    if (whole * per < elems)
      hipLaunchKernelGGL(varlen_tail_kernel, dim3(1), dim3(64), 0, s, mask, mask_dtype, whole * per, elems, num_k,
                         rec, info);
  } else {
    hipLaunchKernelGGL(varlen_rows_strided_kernel, dim3(num_q), dim3(kScanThreads), 0, s, mask, mask_dtype,
                       mask_q_stride, mask_k_stride, num_k, rec, info);
  }
  int32_t* tables = tables_capacity > 0 ? block_tables : nullptr;
  const int cap = (int)std::min<int64_t>(tables_capacity, INT32_MAX);
  if (num_q <= kVerifyRows) {
    const int wgs = std::min(std::max((num_k + kVerifyThreads - 1) / kVerifyThreads, 1), device_cus());
    hipLaunchKernelGGL(varlen_verify_kernel, dim3((unsigned)wgs), dim3(kVerifyThreads), 0, s, rec, num_q,
                       gather_slots, gs_k_stride, num_k, block_size, num_blocks, cu_seqlens_q, q_start, seq_k_offsets,
                       info, tables, cap, host_dev, tag);
  } else {
    const int key_wgs = std::max((num_k + kScanThreads - 1) / kScanThreads, 1);
    hipLaunchKernelGGL(varlen_segments_kernel, dim3(1), dim3(kSegThreads), 0, s, rec, num_q, num_k, block_size,
                       cu_seqlens_q, q_start, seq_k_offsets, info);
    hipLaunchKernelGGL(varlen_check_kernel, dim3((unsigned)key_wgs), dim3(kScanThreads), 0, s, gather_slots,
                       gs_k_stride, seq_k_offsets, cu_seqlens_q, q_start, num_k, block_size, num_blocks, info, tables,
                       cap, host_dev, tag);
  }
  return check_launch("ir_varlen_form_scan");
}

extern "C" int ir_varlen_form_tables(const int64_t* gather_slots, int64_t gs_k_stride, const int32_t* seq_k_offsets,
                                     const int32_t* cu_seqlens_q, const int32_t* q_start, int num_seqs,
                                     int block_size, int32_t* block_tables, int64_t bt_stride,
                                     int max_blocks_per_seq, ir_stream_t stream) {
  IR_REQUIRE(num_seqs >= 0 && block_size > 0 && max_blocks_per_seq >= 1 && bt_stride >= max_blocks_per_seq,
             "ir_varlen_form_tables: bad sizes");
  if (num_seqs == 0) return ok();
  IR_REQUIRE(gather_slots && seq_k_offsets && cu_seqlens_q && q_start && block_tables,
             "ir_varlen_form_tables: null pointer");
  const int64_t slices = ((int64_t)max_blocks_per_seq * block_size + kTableKeys - 1) / kTableKeys;
  IR_REQUIRE(slices <= 65535, "ir_varlen_form_tables: %d blocks of %d keys per sequence is too many",
             max_blocks_per_seq, block_size);
  hipLaunchKernelGGL(varlen_tables_kernel, dim3(num_seqs, (unsigned)slices), dim3(kScanThreads), 0,
                     (hipStream_t)stream, gather_slots, gs_k_stride, seq_k_offsets, cu_seqlens_q, q_start,
                     block_size, block_tables, bt_stride, max_blocks_per_seq);
  return check_launch("ir_varlen_form_tables");
}
