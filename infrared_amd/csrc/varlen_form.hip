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
// (sequence count, longest chunk, widest block table). Pass 2
// (ir_varlen_form_tables) recovers bt_i[j] = gather_slots[k_off_i + j bs] / bs
// and verifies every slot of every sequence against the closed form and the
// pool. Any violation sets info[0]; the host then keeps the mask kernel, which
// reads the metadata as given. When both passes hold, the chunked-prefill
// kernel over these block tables attends exactly the keys the mask allows.
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

// Two wavefronts per row and four 16-byte pieces per lane and pass: of
// 64-1024 threads x 3-12 pieces, the fastest on a 4096 x 22819 bf16 mask.
constexpr int kRowThreads = 128;
constexpr int kRowPieces = 4;  // 16-byte pieces a lane has in flight per pass

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

// One workgroup per mask row: the first and last visible key, their count and
// whether any other value fails to mask. A contiguous mask is read as 16-byte
// pieces of the flat [Q * K] array, a lane's pieces of a pass all in flight
// before any is inspected; rows need not start on a piece, so the first
// and last piece of a row keep only the row's elements, and the array's last
// piece, when partial, is read element by element. Strided masks are read
// element by element.
template <int DT>
__global__ __launch_bounds__(kRowThreads) void varlen_rows_kernel(const void* mask, int64_t m_q, int64_t m_k, int Q,
                                                                  int K, bool flat, int32_t* range) {
  constexpr int PER = DT == IR_DTYPE_F32 ? 4 : 8;  // elements per 16-byte piece
  __shared__ int s_first, s_last, s_count, s_wrong;
  const int r = blockIdx.x, tid = threadIdx.x;
  if (tid == 0) {
    s_first = K;
    s_last = -1;
    s_count = 0;
    s_wrong = 0;
  }
  __syncthreads();
  int first = K, last = -1, count = 0, wrong = 0;
  auto visit = [&](int k, float x) {
    if (x == 0.f) {
      first = min(first, k);
      last = max(last, k);
      ++count;
    } else {
      wrong |= !(x <= -6e4f);
    }
  };
  if (flat) {
    const int64_t e0 = (int64_t)r * K, e1 = e0 + K;
    const int64_t c0 = e0 / PER, c1 = (e1 + PER - 1) / PER;
    const int64_t whole = (int64_t)Q * K / PER;  // pieces wholly inside the array
    // every lane loads every pass, past the row's last whole piece from that
    // piece again (a row with no whole piece of its own loads nothing and
    // inspects its elements one by one)
    const int64_t c_end = min(c1, whole) - 1;
    const u32x4* pieces = (const u32x4*)mask;
    auto inspect = [&](const u32x4& v, int64_t c) {
      const int k0 = (int)(c * PER - e0);  // key of the piece's element 0 (negative in a row's first piece)
      if (c >= whole) {
        for (int e = max(0, -k0); e < PER && k0 + e < K; ++e) visit(k0 + e, mask_value(mask, DT, e0 + k0 + e));
        return;
      }
      const int lo = max(0, -k0), hi = min(PER, K - k0);  // the row's elements of this piece
      const uint32_t keep = ((1u << hi) - 1u) & ~((1u << lo) - 1u);
      // a piece wholly in the row that is all +0 or all finfo(dtype).min --
      // nearly every piece of the reference's mask -- is settled from its
      // four words; anything else is inspected element by element
      const uint32_t any = v[0] | v[1] | v[2] | v[3];
      const uint32_t all = v[0] & v[1] & v[2] & v[3];
      const bool whole_piece = keep == (1u << PER) - 1u;
      if (whole_piece && any == 0u) {
        first = min(first, k0);
        last = max(last, k0 + PER - 1);
        count += PER;
        return;
      }
      if (whole_piece && any == kMinWord<DT> && all == kMinWord<DT>) return;
      uint32_t zero, bad;
      piece_bits<DT>(v, zero, bad);
      zero &= keep;
      wrong |= (bad & keep) != 0u;
      if (zero) {
        first = min(first, k0 + __builtin_ctz(zero));
        last = max(last, k0 + 31 - __builtin_clz(zero));
        count += __builtin_popcount(zero);
      }
    };
    for (int64_t base = c0; base < c1; base += (int64_t)kRowThreads * kRowPieces) {
      u32x4 x[kRowPieces];
      if (c_end >= c0) {  // uniform: the row holds a whole piece
#pragma unroll
        for (int i = 0; i < kRowPieces; ++i) x[i] = load_nt(pieces + min(base + i * kRowThreads + tid, c_end));
      }
#pragma unroll
      for (int i = 0; i < kRowPieces; ++i) {
        const int64_t c = base + i * kRowThreads + tid;
        if (c >= c1) break;
        inspect(x[i], c);
      }
    }
  } else {
    const int64_t row = (int64_t)r * m_q;
    for (int k = tid; k < K; k += kRowThreads) visit(k, mask_value(mask, DT, row + (int64_t)k * m_k));
  }
  if (count) {
    atomicMin(&s_first, first);
    atomicMax(&s_last, last);
    atomicAdd(&s_count, count);
  }
  if (wrong) s_wrong = 1;
  __syncthreads();
  if (tid == 0) {
    // no visible key, or a masked key between two visible ones: the row's
    // range is (-1, -1), which the segment pass reports
    const bool bad = s_wrong || s_count == 0 || s_last - s_first + 1 != s_count;
    range[2 * r] = bad ? -1 : s_first;
    range[2 * r + 1] = bad ? -1 : s_last;
  }
}

// One workgroup: rows -> sequences (block-wide scan of the rows where lo
// moves), then the longest chunk and the widest table; info[0..3] written
// whole (no clearing before the pass).
__global__ __launch_bounds__(kSegThreads) void varlen_segments_kernel(const int32_t* range, int Q, int K, int bs,
                                                                     int32_t* cu, int32_t* q_start, int32_t* seq_lo,
                                                                     int32_t* info) {
  __shared__ int s_scan[kSegThreads];
  __shared__ int s_base, s_bad, s_maxq, s_maxb;
  const int tid = threadIdx.x;
  if (tid == 0) {
    s_base = 0;
    s_bad = 0;
    s_maxq = 0;
    s_maxb = 0;
  }
  __syncthreads();
  for (int c0 = 0; c0 < Q; c0 += kSegThreads) {
    const int r = c0 + tid;
    int start = 0;
    if (r < Q) {
      const int lo = range[2 * r], hi = range[2 * r + 1];
      const int plo = r > 0 ? range[2 * r - 2] : -1, phi = r > 0 ? range[2 * r - 1] : -1;
      start = r == 0 || lo != plo;
      // a row whose own scan failed; a new sequence's keys follow the last
      // one's; a row of the same sequence sees one key more than the row before
      if (lo < 0 || (start ? lo != phi + 1 : hi != phi + 1)) s_bad = 1;
      if (r == Q - 1 && hi != K - 1) s_bad = 1;  // the key axis ends with the last sequence
    }
    s_scan[tid] = start;
    __syncthreads();
    // inclusive Hillis-Steele scan of the start flags
    for (int off = 1; off < kSegThreads; off <<= 1) {
      const int add = tid >= off ? s_scan[tid - off] : 0;
      __syncthreads();
      s_scan[tid] += add;
      __syncthreads();
    }
    if (r < Q && start) {
      const int i = s_base + s_scan[tid] - 1;
      const int lo = range[2 * r], hi = range[2 * r + 1];
      cu[i] = r;
      seq_lo[i] = lo;
      q_start[i] = hi - lo;
    }
    __syncthreads();
    if (tid == 0) s_base += s_scan[kSegThreads - 1];
    __syncthreads();
  }
  const int nseq = s_base;
  if (tid == 0) cu[nseq] = Q;
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
  }
}

// Workgroup (i, y): keys [y * kTableKeys, (y + 1) * kTableKeys) of sequence
// i -- its block-table entries written, every slot checked.
constexpr int kTableKeys = 2048;
__global__ __launch_bounds__(kScanThreads) void varlen_tables_kernel(const int64_t* gs, int64_t gs_k,
                                                                    const int32_t* seq_lo, const int32_t* cu,
                                                                    const int32_t* q_start, int bs,
                                                                    int64_t num_blocks, int32_t* bt,
                                                                    int64_t bt_stride, int width, int32_t* info) {
  __shared__ int s_bad;
  const int i = blockIdx.x, tid = threadIdx.x;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  const int64_t lo = seq_lo[i];
  const int t_len = q_start[i] + (cu[i + 1] - cu[i]);
  if ((t_len + bs - 1) / bs > width) s_bad = 1;
  const int t0 = blockIdx.y * kTableKeys, t1 = min(t0 + kTableKeys, t_len);
  for (int t = t0 + tid; t < t1; t += kScanThreads) {
    const int64_t head = gs[(lo + (int64_t)(t / bs) * bs) * gs_k];
    const int64_t id = head / bs;
    if (head < 0 || head % bs != 0 || id >= num_blocks || gs[(lo + t) * gs_k] != id * bs + t % bs) s_bad = 1;
  }
  // entry j belongs to the slice holding its first key, j * bs
  const int j0 = (t0 + bs - 1) / bs, j1 = min((t0 + kTableKeys + bs - 1) / bs, width);
  for (int j = j0 + tid; j < j1; j += kScanThreads) {
    const int p = j * bs;
    bt[(int64_t)i * bt_stride + j] = p < t_len ? (int32_t)(gs[(lo + p) * gs_k] / bs) : 0;
  }
  __syncthreads();
  if (tid == 0 && s_bad) atomicOr(&info[0], 1);
}

}  // namespace
}  // namespace ir

using namespace ir;

extern "C" int ir_varlen_form_scan(const void* mask, int64_t mask_q_stride, int64_t mask_k_stride, int mask_dtype,
                                   int num_q, int num_k, int block_size, int32_t* row_ranges, int32_t* cu_seqlens_q,
                                   int32_t* q_start, int32_t* seq_k_offsets, int32_t* info, ir_stream_t stream) {
  IR_REQUIRE(dtype_bytes(mask_dtype) > 0, "ir_varlen_form_scan: unknown mask dtype %d", mask_dtype);
  IR_REQUIRE(num_q >= 0 && num_k >= 0 && block_size > 0, "ir_varlen_form_scan: bad sizes");
  if (num_q == 0) return ok();
  IR_REQUIRE(mask && row_ranges && cu_seqlens_q && q_start && seq_k_offsets && info,
             "ir_varlen_form_scan: null pointer");
  hipStream_t s = (hipStream_t)stream;
  // contiguous rows from a 16-byte-aligned start: read as 16-byte pieces
  const bool flat = mask_k_stride == 1 && mask_q_stride == num_k && ((uintptr_t)mask & 15) == 0;
  if (mask_dtype == IR_DTYPE_F32)
    hipLaunchKernelGGL(varlen_rows_kernel<IR_DTYPE_F32>, dim3(num_q), dim3(kRowThreads), 0, s, mask, mask_q_stride,
                       mask_k_stride, num_q, num_k, flat, row_ranges);
  else if (mask_dtype == IR_DTYPE_BF16)
    hipLaunchKernelGGL(varlen_rows_kernel<IR_DTYPE_BF16>, dim3(num_q), dim3(kRowThreads), 0, s, mask, mask_q_stride,
                       mask_k_stride, num_q, num_k, flat, row_ranges);
  else
    hipLaunchKernelGGL(varlen_rows_kernel<IR_DTYPE_F16>, dim3(num_q), dim3(kRowThreads), 0, s, mask, mask_q_stride,
                       mask_k_stride, num_q, num_k, flat, row_ranges);
  hipLaunchKernelGGL(varlen_segments_kernel, dim3(1), dim3(kSegThreads), 0, s, row_ranges, num_q, num_k, block_size,
                     cu_seqlens_q, q_start, seq_k_offsets, info);
  return check_launch("ir_varlen_form_scan");
}

extern "C" int ir_varlen_form_tables(const int64_t* gather_slots, int64_t gs_k_stride, const int32_t* seq_k_offsets,
                                     const int32_t* cu_seqlens_q, const int32_t* q_start, int num_seqs,
                                     int block_size, int64_t num_blocks, int32_t* block_tables, int64_t bt_stride,
                                     int max_blocks_per_seq, int32_t* info, ir_stream_t stream) {
  IR_REQUIRE(num_seqs >= 0 && block_size > 0 && num_blocks >= 0 && max_blocks_per_seq >= 1 &&
                 bt_stride >= max_blocks_per_seq,
             "ir_varlen_form_tables: bad sizes");
  if (num_seqs == 0) return ok();
  IR_REQUIRE(gather_slots && seq_k_offsets && cu_seqlens_q && q_start && block_tables && info,
             "ir_varlen_form_tables: null pointer");
  const int64_t slices = ((int64_t)max_blocks_per_seq * block_size + kTableKeys - 1) / kTableKeys;
  IR_REQUIRE(slices <= 65535, "ir_varlen_form_tables: %d blocks of %d keys per sequence is too many",
             max_blocks_per_seq, block_size);
  hipLaunchKernelGGL(varlen_tables_kernel, dim3(num_seqs, (unsigned)slices), dim3(kScanThreads), 0,
                     (hipStream_t)stream, gather_slots, gs_k_stride, seq_k_offsets, cu_seqlens_q, q_start,
                     block_size, num_blocks, block_tables, bt_stride, max_blocks_per_seq, info);
  return check_launch("ir_varlen_form_tables");
}
