// Paged-KV verify attention for gfx950 (piece 1 of the verification path).
//
// Replaces FlashInfer's BatchPrefillWithPagedKVCacheWrapper.run() as called at
// batchspec/models/modules/attention/standard.py:69:
//   o[t, hq] = softmax_j(q[t, hq] . k[j, hq/g] * sm_scale + mask) . v[j, hq/g]
// over the kv tokens j of the request, gathered through the CSR page table.
//
// Work decomposition (one wave = one kv head x one block of query rows):
//   * the query rows of a kv head are (token t, head-in-group hh) -> row t*g+hh;
//     a wave owns 16*NT of them (NT = 1 or 2 MFMA column tiles);
//   * kv tokens are consumed in tiles of 32 (two 16-token subtiles); a subtile of a
//     page_size >= 16 cache lies inside one page, so its page id is wave-uniform;
//   * scores are computed transposed, S^T = K Q^T, with v_mfma_f32_16x16x32 (A = K
//     rows from the cache, loaded as whole 128-byte lines and rotated into the A
//     layout in registers; B = Q^T from LDS).  In the accumulator layout
//     each lane then holds one query row, so the softmax statistics are lane-local
//     up to a 4-lane reduction;
//   * the output is accumulated transposed as well, O^T = V^T P^T.  P^T is already in
//     B-operand layout (the kv-token order inside the 32-wide contraction is permuted
//     consistently for P and V).  V^T is formed from 16-byte row loads by an 8x8
//     transpose of 16-bit values in registers (v_perm_b32);
//   * the softmax reference maximum is only raised when a score exceeds it by more
//     than 2^8 (exp2 domain), so the O rescale runs on a handful of tiles instead of
//     every tile; every probability stays below 2^8, exact in the final O / l;
//   * workgroups are persistent: the host plan cuts the kv work of the whole batch
//     into equal shares (segments of consecutive tiles of one request).  The loop
//     over a workgroup's segments is flat: the K/V tile after the last tile of a
//     segment is the first tile of the next segment, prefetched like any other, so a
//     segment switch costs one Q load;
//   * a request split over several segments writes its partial results, normalised
//     and rounded to the input dtype (bf16 or fp16), with their fp32 log2-sum-exp; a
//     second kernel merges them in fp32.  (Merging inside the main kernel,
//     by the wave that completes the last part, needs device-scope coherence for
//     the partials across XCDs, whose L2 caches are not coherent with each other:
//     measured on MI355X, the device-scope stores, loads and counter round trips
//     cost more than the separate launch.)
#include <type_traits>

#include "attn_shape.h"
#include "common.h"

namespace bsx {
namespace attn {

constexpr int kTile = attn_shape::kTileTokens;
// Raise the softmax reference maximum only past this margin (log2 units).
constexpr float kRescaleMargin = 8.0f;

struct Params {
  const int32_t* blob;
  int off_seq, off_seg_indptr, off_segments, off_merge_seqs, off_part_indptr;
  int safe_pos;  // a valid position in kv_indices (used for loads of empty requests)
  int off_dyn;   // device plans: blob offset of {split requests, ...}; -1 otherwise
  const uint16_t* q;
  int64_t q_stride;  // elements between tokens
  const char* k_cache;
  const char* v_cache;
  int64_t page_stride_bytes;
  const int32_t* kv_indices;
  // BSX_MASK_TREE: one word per query token.  BSX_MASK_CUSTOM: [batch] bit offsets of
  // the requests' masks, then the packed bits (bit f at word bits_base + f / 32).
  const uint32_t* mask_words;
  int bits_base;
  uint16_t* out;
  int64_t out_stride;
  float* lse_out;
  // Rows appended at the tail of each request (token i of request b at position
  // kv_len_b - qo_len_b + i), or null: [total_qo][H_kv][D] with the token strides below.
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t knew_stride, vnew_stride;  // elements between tokens
  uint16_t* part_o;  // partial outputs (normalised, input dtype), [slot][kv head][row][D]
  float* part_lse;   // their log2-sum-exp, [slot][kv head][row]
  int num_qo_heads, num_kv_heads, group;
  int page_shift, page_mask;
  int mask_mode, sink, window;
  float scale_log2;  // sm_scale * log2(e)
  int heads_per_cta, qblocks_per_cta, n_qgroups, qrows_total, qrow_blocks;
};

// One segment of a workgroup's schedule, with its request's metadata.
struct Seg {
  int b, t0, t1, slot, qo_start, qo_len, kv_len, page_start;
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Wave-uniform read of read-only int32 metadata (plan blob, page ids) through the
// scalar unit: those loads are tracked by lgkmcnt, so they never wait behind the
// vector loads of the K/V tiles in flight.
typedef const int32_t __attribute__((address_space(4)))* const_i32_ptr;
__device__ __forceinline__ int ld_uniform(const int32_t* base, int64_t i) {
  return ((const_i32_ptr)base)[i];
}

__device__ __forceinline__ Seg load_seg(const Params& p, int si) {
  Seg s;
  const int32_t* sg = p.blob + p.off_segments + 4 * si;
  s.b = ld_uniform(sg, 0);
  s.t0 = ld_uniform(sg, 1);
  s.t1 = ld_uniform(sg, 2);
  s.slot = ld_uniform(sg, 3);
  const int32_t* sq = p.blob + p.off_seq + 4 * s.b;
  s.qo_start = ld_uniform(sq, 0);
  s.qo_len = ld_uniform(sq, 1);
  s.kv_len = ld_uniform(sq, 2);
  s.page_start = ld_uniform(sq, 3);
  return s;
}

// K and V tiles are streamed once: non-temporal loads keep them from displacing
// reusable lines in the caches.
__device__ __forceinline__ u32x4 ld_stream(const char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld_stream2(const char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}

__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) {
  // (a.lo16, b.lo16)
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) {
  // (a.hi16, b.hi16)
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == BSX_DTYPE_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Two fp32 values to packed 16-bit (round to nearest even): one v_cvt_pk_* each.
template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  if constexpr (DT == BSX_DTYPE_BF16) {
    typedef __bf16 h2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, h2_t));
  } else {
    typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, h2_t));
  }
}

// NaN-propagating maximum (v_maximum3_f32): unlike fmaxf it needs no quieting of
// its inputs.
__device__ __forceinline__ float max3f(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// Per-row visibility rule of the masked tiles, in a form that is the same for every
// mask mode (no branches in the tile loop).  Token j of the request is visible iff
//   j <= lim  and  (d < 0 or bit min(d, 31) of word)  and  (j < sink_end or j >= win_beg)
// with d = j - (kv_len - qo_len):
//   none:       lim = kv_len - 1,  word = ~0,          sink_end = kv_len
//   causal:     lim = diag + t,    word = ~0,          sink_end = kv_len
//   tree:       lim = kv_len - 1,  word = tree word,   sink_end = kv_len
//   streaming:  lim = diag + t,    word = ~0,          sink_end = sink, win_beg = kv_len - window
struct RowMask {
  int lim;
  uint32_t word;
};

// Applies the RowMask rule to the transposed scores of one tile: lane (c16, g4) holds
// query row c16 of tile nt against kv tokens j0 + 16 st + 4 g4 + e.
template <int NT>
__device__ __forceinline__ void mask_tile(f32x4 (&sacc)[2][NT], const RowMask (&rm)[NT], int j0,
                                          int g4, int diag, int sink_end, int win_beg) {
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = j0 + 16 * st + 4 * g4 + e;
      const int d = j - diag;
      const bool in_view = (j < sink_end) | (j >= win_beg);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const uint32_t bit = (rm[nt].word >> (uint32_t)min(max(d, 0), 31)) & 1u;
        const bool vis = (j <= rm[nt].lim) & ((d < 0) | (bit != 0u)) & in_view;
        sacc[st][nt][e] = vis ? sacc[st][nt][e] : -INFINITY;
      }
    }
}

// Online softmax of one tile against the reference maximum m_ref (exp2 domain, scores
// scaled by scale_log2).  The reference is raised, and O and l rescaled, only when some
// row's scaled maximum exceeds it by more than the margin (always on the first visible
// tile).  Returns the probabilities packed as the B operand of O^T += V^T P^T.  The row
// sums go to l_run (this lane's share).
template <int DT, int NJ, int NT>
__device__ __forceinline__ void softmax_tile(const f32x4 (&sacc)[2][NT], float scale_log2,
                                             float (&m_ref)[NT], float (&l_run)[NT],
                                             f32x4 (&o)[NJ][NT], uint32_t (&pb)[NT][4]) {
  bool need = false;
  float tmax[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float mx = max3f(max3f(sacc[0][nt][0], sacc[0][nt][1], sacc[0][nt][2]),
                           max3f(sacc[0][nt][3], sacc[1][nt][0], sacc[1][nt][1]),
                           __builtin_elementwise_maximum(sacc[1][nt][2], sacc[1][nt][3]));
    tmax[nt] = mx * scale_log2;
    need |= tmax[nt] > m_ref[nt] + kRescaleMargin;
  }
  if (__builtin_amdgcn_ballot_w64(need) != 0) {
    // wave-uniform and rare: row maxima over the 4 lane groups, then rescale
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float mx = tmax[nt];
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_ref[nt], mx);
      const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_ref[nt] - m_new);
      l_run[nt] *= alpha;
#pragma unroll
      for (int jm = 0; jm < NJ; ++jm) o[jm][nt] *= alpha;
      m_ref[nt] = m_new;
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float neg_m = m_ref[nt] == -INFINITY ? 0.f : -m_ref[nt];
    float pv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[e >> 2][nt][e & 3], scale_log2, neg_m));
      l_run[nt] += pv[e];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) pb[nt][r] = pack2<DT>(pv[2 * r], pv[2 * r + 1]);
  }
}

// V rows of tokens at or past kv_len hold unrelated data: zero them (their
// probabilities are 0, but 0 * Inf/NaN would not be).
template <int VW>
__device__ __forceinline__ void zero_rows_past_end(uint32_t (&vraw)[8][VW], int j0, int g4,
                                                   int kv_len) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const bool ok = j0 + 16 * (e >> 2) + 4 * g4 + (e & 3) < kv_len;
#pragma unroll
    for (int w = 0; w < VW; ++w) vraw[e][w] = ok ? vraw[e][w] : 0u;
  }
}

// V^T operands from 8 token rows per lane: A_jm[e] = V[tau(g4, e)][NJ*c16 + jm]
// (8x8 transpose of 16-bit values with v_perm_b32).
template <int NJ, int VW>
__device__ __forceinline__ void transpose_v(const uint32_t (&vraw)[8][VW], u32x4 (&va)[NJ]) {
#pragma unroll
  for (int jm = 0; jm < NJ; ++jm) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t w0 = vraw[2 * r][jm >> 1];
      const uint32_t w1 = vraw[2 * r + 1][jm >> 1];
      va[jm][r] = (jm & 1) ? perm_hi(w0, w1) : perm_lo(w0, w1);
    }
  }
}

template <int DT, int NJ, int NT>
__device__ __forceinline__ void pv_tile(const u32x4 (&va)[NJ], const uint32_t (&pb)[NT][4],
                                        f32x4 (&o)[NJ][NT]) {
#pragma unroll
  for (int jm = 0; jm < NJ; ++jm)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      u32x4 bop = {pb[nt][0], pb[nt][1], pb[nt][2], pb[nt][3]};
      o[jm][nt] = mfma16x16x32<DT>(va[jm], bop, o[jm][nt]);
    }
}

// End of a segment: normalise and store the wave's rows as the request's output, or,
// for a split request, as a partial in the input dtype with its log2-sum-exp for the
// merge kernel.
// Lane (c16, g4) holds row c16 of tile nt at d = NJ*(4 g4 + e) + jm (INTERLEAVED,
// 4 NJ consecutive values per lane) or at d = 16 jm + 4 g4 + e (runs of 4).
template <int DT, int D, int NT, bool INTERLEAVED>
__device__ __forceinline__ void store_row(uint16_t* dst, int g4, const f32x4 (&o)[D / 16][NT],
                                          int nt) {
  constexpr int NJ = D / 16;
  if constexpr (INTERLEAVED) {
    uint32_t packed[2 * NJ];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int jm = 0; jm < NJ; jm += 2)
        packed[(NJ * e + jm) / 2] = pack2<DT>(o[jm][nt][e], o[jm + 1][nt][e]);
    uint16_t* d0 = dst + NJ * 4 * g4;
#pragma unroll
    for (int w = 0; w < 2 * NJ; w += 4) {
      u32x4 v = {packed[w], packed[w + 1], packed[w + 2], packed[w + 3]};
      *reinterpret_cast<u32x4*>(d0 + 2 * w) = v;
    }
  } else {
#pragma unroll
    for (int jm = 0; jm < NJ; ++jm) {
      u32x2 v = {pack2<DT>(o[jm][nt][0], o[jm][nt][1]), pack2<DT>(o[jm][nt][2], o[jm][nt][3])};
      *reinterpret_cast<u32x2*>(dst + 16 * jm + 4 * g4) = v;
    }
  }
}

// l_run: this lane's share of the row sums (summed over the 4 lane groups here).
template <int DT, int D, int NT, bool INTERLEAVED = true>
__device__ __forceinline__ void finish_segment(const Params& p, const Seg& cur, int h, int row0,
                                               int c16, int g4, f32x4 (&o)[D / 16][NT],
                                               const float (&m_ref)[NT],
                                               const float (&l_run)[NT]) {
  constexpr int NJ = D / 16;
  const int g = p.group;
  const int nrows = cur.qo_len * g;
  float lse2[NT];
  bool rowv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float l = l_run[nt];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
    for (int jm = 0; jm < NJ; ++jm) o[jm][nt] *= inv;
    lse2[nt] = l > 0.f ? m_ref[nt] + __log2f(l) : -INFINITY;
    rowv[nt] = row0 + nt * 16 + c16 < nrows;
  }

  if (cur.slot >= 0) {
    // Split request: publish this part for the merge kernel.  The normalised partial
    // output is a convex combination of V rows, so the input dtype holds it; it is
    // stored in that dtype (one extra rounding at the output's own precision, 2^-9
    // relative for bf16 and 2^-12 for fp16), halving the partial traffic against
    // fp32, which is written, flushed from L2 at kernel end and read back by the
    // merge.  Plain stores: the pieces of a row combine into full lines in L2
    // (non-temporal stores measured 2.3x the write traffic).
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (!rowv[nt]) continue;
      const int row = row0 + nt * 16 + c16;
      const int64_t prow = ((int64_t)cur.slot * p.num_kv_heads + h) * p.qrows_total + row;
      store_row<DT, D, NT, INTERLEAVED>(p.part_o + prow * D, g4, o, nt);
      if (g4 == 0) p.part_lse[prow] = lse2[nt];
    }
  } else {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (!rowv[nt]) continue;
      const int row = row0 + nt * 16 + c16;
      const int tq = row / g;
      const int hh = row - tq * g;
      uint16_t* op =
          p.out + (int64_t)(cur.qo_start + tq) * p.out_stride + (int64_t)(h * g + hh) * D;
      store_row<DT, D, NT, INTERLEAVED>(op, g4, o, nt);
      if (p.lse_out != nullptr && g4 == 0)
        p.lse_out[(int64_t)(cur.qo_start + tq) * p.num_qo_heads + h * g + hh] =
            lse2[nt] * 0.69314718055994531f;
    }
  }
}

// Row masks of the wave's query rows for request `cur` (padded rows take the last
// query token's rule; their results are never stored).
template <int NT>
__device__ __forceinline__ void row_masks(const Params& p, const Seg& cur, int row0, int c16,
                                          RowMask (&rm)[NT]) {
  const bool causal_like = p.mask_mode == BSX_MASK_CAUSAL || p.mask_mode == BSX_MASK_STREAMING;
  const int nrows = cur.qo_len * p.group;
  const int diag = cur.kv_len - cur.qo_len;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = row0 + nt * 16 + c16;
    const bool rv = row < nrows;
    const int tq = rv ? row / p.group : 0;
    const int tq_m = rv ? tq : cur.qo_len - 1;
    rm[nt].lim = causal_like ? diag + tq_m : cur.kv_len - 1;
    rm[nt].word = ~0u;
    if (p.mask_mode == BSX_MASK_TREE && rv) rm[nt].word = p.mask_words[cur.qo_start + tq];
  }
}

// The layer's KV update fused into the attention launch (p.k_new != null).  Every
// workgroup whose segments reach a request's appended rows (tiles past kv_len - qo_len)
// first writes those rows, for its own kv heads, from p.k_new / p.v_new into their page
// slots and meets its waves at a barrier, which waits for the stores; its tile loads after
// that read the rows from the cache like any other.  Workgroups that share a request write
// the same bytes into the same slots, and none reads an appended slot without having
// written it first, so no read sees a slot's old contents.  The result equals the append
// followed by the attention launch bit for bit.  Rows at negative positions (kv_len below
// qo_len) have no slot and are skipped, as the standalone append skips them.
template <int D>
__device__ void append_rows_of_segments(const Params& p, int seg_begin, int seg_end, int hgroup) {
  constexpr int PIECES = D * 2 / 16;  // 16-byte pieces of a row's head slice
  const int64_t tok_bytes = (int64_t)p.num_kv_heads * D * 2;
  const int per_row = p.heads_per_cta * PIECES;
  const int64_t col0 = (int64_t)hgroup * p.heads_per_cta * D * 2;
  for (int si = seg_begin; si < seg_end; ++si) {
    const Seg s = load_seg(p, si);
    const int diag = s.kv_len - s.qo_len;
    if (s.t0 >= s.t1 || s.t1 * kTile <= diag) continue;  // reads no appended row
    for (int idx = threadIdx.x; idx < s.qo_len * per_row; idx += blockDim.x) {
      const int i = idx / per_row;
      const int pos = diag + i;
      if (pos < 0) continue;
      const int64_t col = col0 + (int64_t)(idx - i * per_row) * 16;
      const int page = p.kv_indices[s.page_start + (pos >> p.page_shift)];
      const int64_t dst =
          (int64_t)page * p.page_stride_bytes + (int64_t)(pos & p.page_mask) * tok_bytes + col;
      const int64_t src = s.qo_start + i;
      const u32x4 kv = *reinterpret_cast<const u32x4*>(
          reinterpret_cast<const char*>(p.k_new + src * p.knew_stride) + col);
      const u32x4 vv = *reinterpret_cast<const u32x4*>(
          reinterpret_cast<const char*>(p.v_new + src * p.vnew_stride) + col);
      *reinterpret_cast<u32x4*>(const_cast<char*>(p.k_cache) + dst) = kv;
      *reinterpret_cast<u32x4*>(const_cast<char*>(p.v_cache) + dst) = vv;
    }
  }
  __syncthreads();
}

// Packed custom mask bits: the two words holding bits [f, f + 32) (the bits end with a
// padding word), from one 8-byte load (dword alignment is enough for it); the 32 bits
// are the pair shifted right by f mod 32.
typedef uint32_t u32x2_dw __attribute__((ext_vector_type(2), aligned(4)));
__device__ __forceinline__ u32x2 mask_pair_at(const uint32_t* bits, int64_t f) {
  const u32x2_dw v = *reinterpret_cast<const u32x2_dw*>(bits + (f >> 5));
  return u32x2{v[0], v[1]};
}
__device__ __forceinline__ uint32_t mask_bits_of(u32x2 pair, int shift) {
  return (uint32_t)((((uint64_t)pair[1] << 32) | pair[0]) >> shift);
}

// General custom mask: token j0 + 16 st + 4 g4 + e of a lane's query row is visible iff
// bit (16 st + 4 g4 + e) of the row's tile word tw[nt] is set (and j <= lim, the kv end).
template <int NT>
__device__ __forceinline__ void mask_tile_bits(f32x4 (&sacc)[2][NT], const RowMask (&rm)[NT],
                                               const uint32_t (&tw)[NT], int j0, int g4) {
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 16 * st + 4 * g4 + e;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const bool vis = (j0 + c <= rm[nt].lim) & (((tw[nt] >> c) & 1u) != 0u);
        sacc[st][nt][e] = vis ? sacc[st][nt][e] : -INFINITY;
      }
    }
}

// NT: query-row tiles of 16 per wave.  D: head dim (64 or 128).  CUSTOM: a general
// boolean mask (BSX_MASK_CUSTOM): every tile is masked, with the 32 bits of each query
// row's mask over the tile read at the start of its step.
template <int DT, int D, int NT, bool PS_GE16, bool CUSTOM = false>
__global__ void __launch_bounds__(512) verify_attn_kernel(Params p) {
  constexpr int KS = D / 32;  // k-steps of the QK^T contraction
  constexpr int NJ = D / 16;  // output d tiles (also d values per lane in V loads)
  constexpr int QT = 16 * NT;
  constexpr int VW = NJ / 2;  // dwords per lane per token of a V row

  // Q operands live in LDS (each lane re-reads only what it wrote), keeping the
  // registers for the pipelined K/V tiles and the output accumulators.
  __shared__ u32x4 q_lds[8][NT * KS][64];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;

  const int hgroup = blockIdx.y / p.n_qgroups;
  const int qgroup = blockIdx.y % p.n_qgroups;
  const int h = hgroup * p.heads_per_cta + wave / p.qblocks_per_cta;
  const int qb = qgroup * p.qblocks_per_cta + wave % p.qblocks_per_cta;
  // Every wave runs the same segment list (for its own kv head and query block) and
  // the same tiles, and meets the others at a barrier before each tile: without it
  // the older wave of each SIMD wins instruction arbitration and finishes far ahead,
  // leaving the younger one to stream the rest at half the memory parallelism.

  const int seg_begin = ld_uniform(p.blob, p.off_seg_indptr + blockIdx.x);
  const int seg_end = ld_uniform(p.blob, p.off_seg_indptr + blockIdx.x + 1);
  if (seg_begin >= seg_end) return;
  if (p.k_new != nullptr) append_rows_of_segments<D>(p, seg_begin, seg_end, hgroup);

  const int g = p.group;
  const int64_t tok_bytes = (int64_t)p.num_kv_heads * D * 2;  // one kv token row (all heads)
  const uint32_t head_off = (uint32_t)(h * D * 2);
  const int row0 = qb * QT;

  // ---- tile loaders (K straight into A-operand layout; V as 8 token rows per lane).
  // Loads are unconditional (no exec-masked or skipped loads, so the compiler's wait
  // counting stays exact across the pipelined loop).  Addresses of tokens past kv_len
  // are clamped into memory the request owns (or, for a request without pages, into
  // a page another request owns); their scores are masked and V rows zeroed.
  u32x4 kreg[2][KS];
  uint32_t vraw[8][VW];
  auto page_pos = [&](int jsc, int kv_len, int page_start) -> int {
    return kv_len > 0 ? page_start + (jsc >> p.page_shift) : p.safe_pos;
  };
  // K loads cover whole 128-byte lines: load j of a subtile reads, in lane (c16, g4),
  // token (c16 & 7) + 8 (j & 1), bytes 128 (j >> 1) + 16 (g4 + 4 (c16 >> 3)) of the head's
  // slice, so one load is 8 token rows x 128 bytes.  (The A-operand layout, 16 token rows
  // x 64 bytes per load, requested every line twice, in two half-line requests, which
  // doubles the memory requests per byte of K.)  kfix() moves the data into the A layout.
  const int ktok = c16 & 7;
  const uint32_t kbyte = (uint32_t)(16 * (g4 + 4 * (c16 >> 3)));
  auto load_tile_k = [&](int tile, int kv_len, int page_start) {
    const int j0 = tile * kTile;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int js = j0 + 16 * st;
#pragma unroll
      for (int h = 0; h < 2; ++h) {  // token rows ktok + 8 h
        const char* base;
        uint32_t off;
        if constexpr (PS_GE16) {
          const int jsc = js < kv_len ? js : 0;  // subtile start, clamped into the request
          const int page = ld_uniform(p.kv_indices, page_pos(jsc, kv_len, page_start));
          base = p.k_cache + (int64_t)page * p.page_stride_bytes;
          off = (uint32_t)(((jsc & p.page_mask) + ktok + 8 * h) * tok_bytes) + head_off + kbyte;
        } else {
          const int j = max(min(js + ktok + 8 * h, kv_len - 1), 0);
          const int page = p.kv_indices[page_pos(j, kv_len, page_start)];
          base = p.k_cache + (int64_t)page * p.page_stride_bytes;
          off = (uint32_t)((j & p.page_mask) * tok_bytes) + head_off + kbyte;
        }
#pragma unroll
        for (int q = 0; q < KS / 2; ++q) kreg[st][2 * q + h] = ld_stream(base + off + 128 * q);
      }
    }
  };
  // The A operand of k-step s (token c16, bytes 64 s + 16 g4): for s = 2q, lanes c16 < 8
  // hold it already in load 2q, the others find it in load 2q+1 eight lanes away; for
  // s = 2q+1 the other way round.  Eight lanes away = a row rotation by 8 (DPP).
  const bool klow = c16 < 8;
  auto kfix = [&](const u32x4 (&x)[2][KS], u32x4 (&a)[2][KS]) {
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int q = 0; q < KS / 2; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t x0 = x[st][2 * q][e], x1 = x[st][2 * q + 1][e];
          const uint32_t r0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)x0, 0x128, 0xf, 0xf, false);
          const uint32_t r1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)x1, 0x128, 0xf, 0xf, false);
          a[st][2 * q][e] = klow ? x0 : r1;
          a[st][2 * q + 1][e] = klow ? r0 : x1;
        }
  };
  auto load_tile_v = [&](int tile, int kv_len, int page_start) {
    const int j0 = tile * kTile;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int js = j0 + 16 * st;
      const char* sbase = p.v_cache;
      uint32_t soff = 0;
      if constexpr (PS_GE16) {
        const int jsc = js < kv_len ? js : 0;
        const int page = ld_uniform(p.kv_indices, page_pos(jsc, kv_len, page_start));
        sbase = p.v_cache + (int64_t)page * p.page_stride_bytes;
        soff = (uint32_t)((jsc & p.page_mask) * tok_bytes) + head_off;
      }
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int e = 4 * st + e4;
        const char* base;
        uint32_t off;
        if constexpr (PS_GE16) {
          base = sbase;
          off = soff + (uint32_t)((4 * g4 + e4) * tok_bytes);
        } else {
          const int j = max(min(js + 4 * g4 + e4, kv_len - 1), 0);
          const int page = p.kv_indices[page_pos(j, kv_len, page_start)];
          base = p.v_cache + (int64_t)page * p.page_stride_bytes;
          off = (uint32_t)((j & p.page_mask) * tok_bytes) + head_off;
        }
        off += (uint32_t)(NJ * c16 * 2);
        if constexpr (VW == 4) {
          const u32x4 v = ld_stream(base + off);
          vraw[e][0] = v[0];
          vraw[e][1] = v[1];
          vraw[e][2] = v[2];
          vraw[e][3] = v[3];
        } else {
          const u32x2 v = ld_stream2(base + off);
          vraw[e][0] = v[0];
          vraw[e][1] = v[1];
        }
      }
    }
  };

  Seg cur = load_seg(p, seg_begin);
  Seg nxt = load_seg(p, min(seg_begin + 1, seg_end - 1));
  load_tile_k(cur.t0, cur.kv_len, cur.page_start);
  load_tile_v(cur.t0, cur.kv_len, cur.page_start);

  for (int si = seg_begin; si < seg_end; ++si) {
    const bool has_next = si + 1 < seg_end;
    const int nrows = cur.qo_len * g;
    // A segment with tiles runs the tile loop in every wave of the workgroup (uniform
    // barrier count); a wave without query rows in this request computes on padding.
    const bool has_tiles = cur.t0 < cur.t1;
    const int diag = cur.kv_len - cur.qo_len;

    // ---- Q (B operand of S^T = K Q^T): lane holds query row c16 of tile nt, d chunk
    // (s, g4).  Padded rows read row 0 (finite data; their results are never stored).
    const int sink_end = p.mask_mode == BSX_MASK_STREAMING ? p.sink : cur.kv_len;
    const int win_beg = p.mask_mode == BSX_MASK_STREAMING ? cur.kv_len - p.window : cur.kv_len;
    RowMask rm[NT];
    row_masks<NT>(p, cur, row0, c16, rm);
    int64_t mrow[NT];  // CUSTOM: bit offset of each lane row's mask row
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int row = row0 + nt * 16 + c16;
      const bool rv = row < nrows;
      const int tq = rv ? row / g : 0;
      const int hh = rv ? row - tq * g : 0;
      if constexpr (CUSTOM)
        mrow[nt] = (int64_t)ld_uniform(reinterpret_cast<const int32_t*>(p.mask_words), cur.b) +
                   (int64_t)tq * cur.kv_len;
      if (has_tiles) {
        const uint16_t* qp =
            p.q + (int64_t)(cur.qo_start + tq) * p.q_stride + (int64_t)(h * g + hh) * D;
#pragma unroll
        for (int s = 0; s < KS; ++s)
          q_lds[wave][nt * KS + s][lane] = *reinterpret_cast<const u32x4*>(qp + 32 * s + 8 * g4);
      }
    }

    f32x4 o[NJ][NT];
#pragma unroll
    for (int jm = 0; jm < NJ; ++jm)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[jm][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_ref[NT], l_run[NT];  // l_run: this lane's share of the row sum
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      m_ref[nt] = -INFINITY;
      l_run[nt] = 0.f;
    }

    // CUSTOM: the mask words of the next tile to run, loaded one tile ahead (with the K
    // prefetch) and shifted into place only when the tile runs, so that a tile's masking
    // waits for nothing the tile does not wait for already (loads complete in order: a
    // use right after the load would wait for the K prefetch issued before it).  A
    // segment's first tile loads its own.  Tiles start at multiples of 32 tokens, so the
    // shift is the row's bit offset mod 32 for every tile.
    u32x2 tw_next[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) tw_next[nt] = u32x2{0u, 0u};

    // Prefetch target after the last tile of this segment: the first tile of the next
    // segment, or (at the end of the schedule) the last tile again.
    const int end_tile = has_next ? nxt.t0 : max(cur.t1 - 1, 0);
    const int end_kv = has_next ? nxt.kv_len : cur.kv_len;
    const int end_pages = has_next ? nxt.page_start : cur.page_start;

    // One tile: S^T = K Q^T, softmax, O^T += V^T P^T, with the next tile's K and V
    // loads issued as soon as their registers are free.  MASKED is a compile-time
    // flag: the body loop over tiles that need no per-element mask is branch-free
    // around its loads, which keeps the compiler's load-wait counting exact.
    auto tile_step = [&](int tile, auto masked_tag, auto prefetch_tag, auto first_tag) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      constexpr bool PREFETCH = decltype(prefetch_tag)::value;
      constexpr bool FIRST = decltype(first_tag)::value;  // CUSTOM: no bits loaded ahead
      const int j0 = tile * kTile;
      const bool last = tile + 1 >= cur.t1;
      const int pf_tile = last ? end_tile : tile + 1;
      const int pf_kv = last ? end_kv : cur.kv_len;
      const int pf_pages = last ? end_pages : cur.page_start;
      // Workgroup barrier without a memory fence (the tile loads in flight stay in
      // flight).  The asm also keeps the Q reads from LDS inside the loop instead of
      // letting them be hoisted into registers the pipelined tiles need.
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      // (CUSTOM: the tile's mask bits, loaded during the previous tile)
      uint32_t tw[NT];
      if constexpr (CUSTOM) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const u32x2 pair =
              FIRST ? mask_pair_at(p.mask_words + p.bits_base, mrow[nt] + j0) : tw_next[nt];
          tw[nt] = mask_bits_of(pair, (int)(mrow[nt] & 31));
        }
      }

      u32x4 kop[2][KS];
      kfix(kreg, kop);
      f32x4 sacc[2][NT];
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < KS; ++s)
            acc = mfma16x16x32<DT>(kop[st][s], q_lds[wave][nt * KS + s][lane], acc);
          sacc[st][nt] = acc;
        }
      // K registers are free: prefetch.  The scheduling barriers keep each prefetch
      // after the last read of the registers it refills, so the loaded tile lands in
      // place (a load hoisted above those reads would need fresh registers and a copy
      // at the loop back-edge that waits for the load to complete).
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PREFETCH) load_tile_k(pf_tile, pf_kv, pf_pages);
      if constexpr (CUSTOM && PREFETCH) {
        // the next tile of this segment (its last tile again at the segment's end: the
        // next segment loads its own first bits)
        const int64_t jn = (int64_t)min(tile + 1, cur.t1 - 1) * kTile;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          tw_next[nt] = mask_pair_at(p.mask_words + p.bits_base, mrow[nt] + jn);
      }

      // CUSTOM: a tile inside the kv range whose 32 bits are set in every row of the wave
      // needs no mask and no zeroed V rows (uniform branches around register work only).
      const bool past_end = j0 + kTile > cur.kv_len;
      if constexpr (CUSTOM) {
        bool partial = past_end;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) partial |= tw[nt] != ~0u;
        if (__builtin_amdgcn_ballot_w64(partial) != 0) mask_tile_bits<NT>(sacc, rm, tw, j0, g4);
      } else if constexpr (MASKED) {
        mask_tile<NT>(sacc, rm, j0, g4, diag, sink_end, win_beg);
      }

      uint32_t pb[NT][4];
      softmax_tile<DT, NJ, NT>(sacc, p.scale_log2, m_ref, l_run, o, pb);

      if constexpr (CUSTOM) {
        if (past_end) zero_rows_past_end<VW>(vraw, j0, g4, cur.kv_len);
      } else if constexpr (MASKED) {
        zero_rows_past_end<VW>(vraw, j0, g4, cur.kv_len);
      }
      u32x4 va[NJ];
      transpose_v<NJ, VW>(vraw, va);
      // The transposed operands must be complete before the V registers are refilled:
      // an empty asm that reads them (and orders memory) pins the transposes above the
      // prefetch so the loads land in place.
#pragma unroll
      for (int jm = 0; jm < NJ; ++jm) asm volatile("" ::"v"(va[jm]) : "memory");
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (PREFETCH) load_tile_v(pf_tile, pf_kv, pf_pages);  // V registers are free
      pv_tile<DT, NJ, NT>(va, pb, o);
    };

    if (has_tiles) {
      // Tiles [t0, t_split) lie entirely inside the visible prefix (no mask needed);
      // [t_split, t1) touch the draft block, the kv end, or the sink/window view.
      int limit = p.mask_mode == BSX_MASK_NONE ? cur.kv_len : diag;
      if (p.mask_mode == BSX_MASK_STREAMING || CUSTOM) limit = 0;
      // The last tile of the workgroup's schedule has nothing to prefetch: it runs
      // after the loops (masked form, valid for any tile).
      const int t_end = has_next ? cur.t1 : cur.t1 - 1;
      const int t_split = max(cur.t0, min(t_end, limit / kTile));
      const std::true_type yes;
      const std::false_type no;
      if constexpr (CUSTOM) {
        // the segment's first tile loads its own mask bits; every later tile's come
        // from the step before it (the same load order on every path into the loop)
        if (t_end > cur.t0) {
          tile_step(cur.t0, yes, yes, yes);
          for (int tile = cur.t0 + 1; tile < t_end; ++tile) tile_step(tile, yes, yes, no);
          if (!has_next) tile_step(cur.t1 - 1, yes, no, no);
        } else {
          tile_step(cur.t1 - 1, yes, no, yes);  // the schedule's last tile, alone
        }
      } else {
        for (int tile = cur.t0; tile < t_split; ++tile) tile_step(tile, no, yes, no);
        for (int tile = t_split; tile < t_end; ++tile) tile_step(tile, yes, yes, no);
        if (!has_next) tile_step(cur.t1 - 1, yes, no, no);
      }
    } else if (has_next) {
      // No tile ran, so the prefetched tile was not consumed: load the next
      // segment's first tile now.
      load_tile_k(end_tile, end_kv, end_pages);
      load_tile_v(end_tile, end_kv, end_pages);
    }

    finish_segment<DT, D, NT>(p, cur, h, row0, c16, g4, o, m_ref, l_run);

    cur = nxt;
    nxt = load_seg(p, min(si + 2, seg_end - 1));
  }
}

// ---- Shared K/V tiles -----------------------------------------------------------
//
// When a kv head has more query rows than one wave holds (long drafts, token trees,
// large GQA groups), QB waves work on the same kv head.  Streaming its K/V tiles into
// each of those waves' registers would multiply the vector-memory requests per byte by
// QB, and the address/data path of the compute units, not HBM, would set the pace.
// Instead every K/V tile is copied once into LDS by direct global->LDS loads, split
// between the QB waves of the head, through a ring of tile stages; every wave then
// reads its MFMA operands from LDS.  Ring protocol, per tile n (stage n mod S):
//   wait until this wave's loads of tile n landed (at most (S-2) tiles of its loads
//   younger than them are in flight), barrier (every wave's loads of tile n landed and
//   every wave finished reading tile n-1), issue the loads of tile n+S-1 into the stage
//   of tile n-1, compute tile n from LDS.
// The direct loads are issued from inline assembly, invisible to the compiler's wait
// counting (it would otherwise wait for every load in flight before any LDS read); the
// wait above is explicit.  Loads return in issue order, so a count of younger loads
// is exact, and any other load issued later only makes the wait stricter.
template <int D>
struct SharedTile {
  static constexpr int kRowGranules = D / 8;        // 16-byte granules per token row
  static constexpr int kHalfBytes = kTile * D * 2;  // K (or V) part of one head's tile
  static constexpr int kHeadBytes = 2 * kHalfBytes;
  static constexpr int kChunks = kHeadBytes / 1024;  // 1 KB direct loads per head tile
  // Column swizzle (XOR of the 16-byte column with a function of the token), chosen so
  // that both operand reads run without LDS bank conflicts: the K reads (16-byte reads,
  // one column of 16 consecutive tokens per 16 lanes) and the transposing V reads
  // (8-byte reads, two columns of 4 consecutive tokens per 16 lanes).  For D = 128,
  // measured with the LDS conflict counter on gfx950: t ^ 12 (t & 1) gives both reads
  // their conflict-free time (4 and 2 cycles per instruction); t ^ 8 (t & 1) doubled the
  // K reads' (a 2-way conflict), and t alone doubled the V reads'.  For D = 64 (8
  // columns), t mod 8 gives both their conflict-free time.
  __device__ static __forceinline__ int swz(int t) {
    if constexpr (D == 128) return (t & 15) ^ ((t & 1) * 12);
    return t & 7;
  }
  // granule index of (token t, column c) inside a K or V half
  __device__ static __forceinline__ int at(int t, int c) {
    return t * kRowGranules + (c ^ swz(t));
  }
};

// 64 lanes x 16 bytes from sbase + voff (per lane) into LDS bytes [lds, lds + 1024),
// lane i at lds + 16 i.  M0 carries the LDS address (one wait state before its use).
// Non-temporal: the tiles are read once (measured on MI355X: 7.3 TB/s streaming
// through a 4-stage LDS ring, against 5.9 TB/s with the default policy).
__device__ __forceinline__ void dma_1k(const char* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt"
               ::"s"(lds), "v"(voff), "s"(sbase)
               : "memory");
}

template <int DT, int D, int QB>
__global__ void __launch_bounds__(512) verify_attn_shared_kernel(Params p) {
  using L = SharedTile<D>;
  constexpr int NT = 2;       // 32 query rows per wave
  constexpr int KS = D / 32;  // k-steps of the QK^T contraction
  constexpr int NJ = D / 16;  // output d tiles
  constexpr int VW = NJ / 2;  // dwords per lane per token of a V row
  constexpr int QT = 16 * NT;
  constexpr int S = attn_shape::shared_stages(D, QB);
  constexpr int NPER = L::kChunks / QB;  // direct loads per wave per tile
  constexpr int WAIT = (S - 2) * NPER;
  constexpr int HALF_CHUNKS = L::kChunks / 2;
  static_assert(L::kChunks % QB == 0 && (S & (S - 1)) == 0 && S <= 4, "bad shared-tile shape");

  __shared__ __attribute__((aligned(1024))) u32x4 smem[attn_shape::shared_lds_bytes(D, QB) / 16];

  const int lane = threadIdx.x & 63;
  const int wave = uni(threadIdx.x >> 6);  // scalar: the load addresses derive from it
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int hs = wave / QB;  // head slot of the workgroup
  const int qi = wave % QB;  // query block of the head
  const int hgroup = blockIdx.y / p.n_qgroups;
  const int qgroup = blockIdx.y % p.n_qgroups;
  const int h = hgroup * p.heads_per_cta + hs;
  const int row0 = (qgroup * QB + qi) * QT;

  const int seg_begin = ld_uniform(p.blob, p.off_seg_indptr + blockIdx.x);
  const int seg_end = ld_uniform(p.blob, p.off_seg_indptr + blockIdx.x + 1);
  if (seg_begin >= seg_end) return;
  if (p.k_new != nullptr) append_rows_of_segments<D>(p, seg_begin, seg_end, hgroup);

  const int g = p.group;
  const uint32_t tok_bytes = (uint32_t)(p.num_kv_heads * D * 2);
  const uint32_t head_off = (uint32_t)(h * D * 2);
  const int stage_granules = p.heads_per_cta * (L::kHeadBytes / 16);
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)smem;

  // ---- producer: this wave loads chunks [qi*NPER, (qi+1)*NPER) of its head's tile.
  // Chunk c is 64 consecutive granules (slots) of the K (c < HALF_CHUNKS) or V half;
  // slot s holds token s / kRowGranules, column (s % kRowGranules) ^ swz(token).
  uint32_t lane_off[NPER];
#pragma unroll
  for (int r = 0; r < NPER; ++r) {
    const int cc = (qi * NPER + r) % HALF_CHUNKS;
    const int s = 64 * cc + lane;
    const int t = s / L::kRowGranules;
    const int col = (s % L::kRowGranules) ^ L::swz(t);
    lane_off[r] = (uint32_t)(t & 15) * tok_bytes + head_off + (uint32_t)col * 16u;
  }
  // Schedule position of the next tile to load (segments without tiles are skipped;
  // past the end, nothing is loaded), with the page ids of its two 16-token subtiles.
  // The page ids are read when the cursor moves, one tile before the loads that use
  // them: a scalar read issued right before the loads would put its latency (long
  // under full memory load) on every tile's critical path.
  int pr_count = 0;  // tiles whose loads were issued
  int pr_si = seg_begin, pr_tile = 0, pr_t1 = 0, pr_kv = 0, pr_pages = 0;
  int pr_page0 = 0, pr_page1 = 0;  // (scalars, not an array indexed by a
  int pr_pofs0 = 0, pr_pofs1 = 0;  //  wave-dependent subtile: no dynamic indexing)
  bool pr_valid = false;
  auto pr_pages_of_tile = [&]() {
    const int j0 = pr_tile * kTile;
    const int js1 = j0 + 16;
    const int jsc0 = j0 < pr_kv ? j0 : 0;  // subtile starts, clamped into the request
    const int jsc1 = js1 < pr_kv ? js1 : 0;
    pr_page0 = ld_uniform(p.kv_indices, pr_pages + (jsc0 >> p.page_shift));
    pr_page1 = ld_uniform(p.kv_indices, pr_pages + (jsc1 >> p.page_shift));
    pr_pofs0 = (int)((uint32_t)(jsc0 & p.page_mask) * tok_bytes);
    pr_pofs1 = (int)((uint32_t)(jsc1 & p.page_mask) * tok_bytes);
  };
  auto pr_seek = [&](int si) {  // first segment >= si with tiles
    pr_valid = false;
    for (; si < seg_end; ++si) {
      const Seg s = load_seg(p, si);
      if (s.t0 < s.t1) {
        pr_si = si;
        pr_tile = s.t0;
        pr_t1 = s.t1;
        pr_kv = s.kv_len;
        pr_pages = s.page_start;
        pr_valid = true;
        pr_pages_of_tile();
        return;
      }
    }
  };
  auto pr_advance = [&]() {
    if (!pr_valid) return;
    if (++pr_tile >= pr_t1)
      pr_seek(pr_si + 1);
    else
      pr_pages_of_tile();
  };
  auto pr_issue = [&](int stage) {
    if (!pr_valid) return;
    ++pr_count;
    const uint32_t lds_stage =
        lds_base + (uint32_t)((stage * stage_granules) * 16 + hs * L::kHeadBytes);
#pragma unroll
    for (int r = 0; r < NPER; ++r) {
      const int c = qi * NPER + r;
      const int half = c / HALF_CHUNKS;
      const int cc = c % HALF_CHUNKS;
      const int sub = (cc * 64 / L::kRowGranules) >> 4;  // subtile of the chunk's tokens
      const int page = sub ? pr_page1 : pr_page0;
      const uint32_t pofs = (uint32_t)(sub ? pr_pofs1 : pr_pofs0);
      const char* base = (half ? p.v_cache : p.k_cache) + (int64_t)page * p.page_stride_bytes;
      dma_1k(base, pofs + lane_off[r],
             lds_stage + (uint32_t)(half * L::kHalfBytes + cc * 1024));
    }
  };

  pr_seek(seg_begin);
#pragma unroll
  for (int k = 0; k < S - 1; ++k) {
    pr_issue(k);
    pr_advance();
  }

  // Lane parts of the LDS operand indices.  K: column chunk s of token c16 (the second
  // 16-token subtile adds a constant); V: row 4 g4 + e4 (the second subtile likewise).
  constexpr int SUBTILE = 16 * L::kRowGranules;  // granules of 16 token rows
  int koff[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) koff[s] = L::at(c16, 4 * s + g4);
  // V^T operands come from transposing LDS reads (ds_read_b64_tr_b16): in each group of
  // 16 lanes, lane i receives element i & 3 of the 8 bytes addressed by lanes
  // (i >> 2) + 4 k, k = 0..3.  Lane (c16, g4) therefore addresses token
  // 16 h + 4 g4 + (c16 >> 2), columns 16 jm + 4 (c16 & 3) .. + 3, and receives
  // V[16 h + 4 g4 + k][16 jm + c16]: A[m = c16][8 g4 + 4 h + k] of O^T += V^T P^T for
  // output rows d = 16 jm + m (the token order of P^T, tau(g4, e) = 16 (e >> 2) +
  // 4 g4 + (e & 3), matches).  vtr[jm]: 8-byte index; the second subtile (h = 1) adds
  // a constant.
  int vtr[NJ];
#pragma unroll
  for (int jm = 0; jm < NJ; ++jm)
    vtr[jm] = 2 * L::at(4 * g4 + (c16 >> 2), 2 * jm + ((c16 & 3) >> 1)) + (c16 & 1);

  int n = 0;  // tiles consumed so far (stage n mod S)
  // Wait until this wave's loads of tile n landed: loads return in issue order, so it
  // is enough that no more than the loads of the tiles issued after it are still in
  // flight (S-2 tiles in the steady state; fewer at the end of the schedule, where no
  // tile follows).
  auto wait_tile = [&]() {
    const int younger = pr_count - n - 1;
    if (younger >= S - 2) {
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(WAIT) : "memory");
    } else if (S >= 4 && younger == 1) {
      asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(NPER) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    }
  };
  for (int si = seg_begin; si < seg_end; ++si) {
    const Seg cur = load_seg(p, si);
    const int nrows = cur.qo_len * g;
    const bool has_tiles = cur.t0 < cur.t1;
    const int diag = cur.kv_len - cur.qo_len;
    const int sink_end = p.mask_mode == BSX_MASK_STREAMING ? p.sink : cur.kv_len;
    const int win_beg = p.mask_mode == BSX_MASK_STREAMING ? cur.kv_len - p.window : cur.kv_len;
    RowMask rm[NT];
    row_masks<NT>(p, cur, row0, c16, rm);

    // Q (B operand of S^T = K Q^T) in registers; padded rows read row 0.
    u32x4 qr[NT * KS];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int row = row0 + nt * 16 + c16;
      const bool rv = row < nrows;
      const int tq = rv ? row / g : 0;
      const int hh = rv ? row - tq * g : 0;
      const uint16_t* qp =
          p.q + (int64_t)(cur.qo_start + tq) * p.q_stride + (int64_t)(h * g + hh) * D;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        qr[nt * KS + s] = has_tiles ? *reinterpret_cast<const u32x4*>(qp + 32 * s + 8 * g4)
                                    : u32x4{0u, 0u, 0u, 0u};
    }
    // Wait for Q and the mask words here, once per segment: a wait the compiler placed
    // at their first use inside the tile loop would run on every tile and drain the
    // direct loads in flight.
#pragma unroll
    for (int i = 0; i < NT * KS; ++i) asm volatile("" ::"v"(qr[i]));
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) asm volatile("" ::"v"(rm[nt].word));

    f32x4 o[NJ][NT];
#pragma unroll
    for (int jm = 0; jm < NJ; ++jm)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[jm][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_ref[NT], l_run[NT];  // l_run: this lane's share of the row sum
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      m_ref[nt] = -INFINITY;
      l_run[nt] = 0.f;
    }

    auto tile_step = [&](int tile, auto masked_tag) {
      constexpr bool MASKED = decltype(masked_tag)::value;
      const int j0 = tile * kTile;
      const int stage = n & (S - 1);
      wait_tile();
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      pr_issue((stage + S - 1) & (S - 1));
      pr_advance();

      const u32x4* tk = smem + stage * stage_granules + hs * (L::kHeadBytes / 16);
      const u32x4* tv = tk + L::kHalfBytes / 16;
      f32x4 sacc[2][NT];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        u32x4 ka[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) ka[s] = tk[koff[s] + SUBTILE * st];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int s = 0; s < KS; ++s) acc = mfma16x16x32<DT>(ka[s], qr[nt * KS + s], acc);
          sacc[st][nt] = acc;
        }
      }
      // V^T operands (issued before the softmax to hide the LDS latency)
      u32x4 va[NJ];
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
      const lds_s16x4* tv8 = reinterpret_cast<const lds_s16x4*>(
          reinterpret_cast<const __attribute__((address_space(3))) char*>(
              (const __attribute__((address_space(3))) u32x4*)tv));
#pragma unroll
      for (int jm = 0; jm < NJ; ++jm) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            const_cast<lds_s16x4*>(tv8 + vtr[jm]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            const_cast<lds_s16x4*>(tv8 + vtr[jm] + 2 * SUBTILE));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo);
        const u32x2 h2 = __builtin_bit_cast(u32x2, hi);
        va[jm] = u32x4{l2[0], l2[1], h2[0], h2[1]};
      }
      if constexpr (MASKED) mask_tile<NT>(sacc, rm, j0, g4, diag, sink_end, win_beg);
      uint32_t pb[NT][4];
      softmax_tile<DT, NJ, NT>(sacc, p.scale_log2, m_ref, l_run, o, pb);
      if constexpr (MASKED) {
        // V rows of tokens at or past kv_len hold unrelated data: zero them (element
        // e of va[jm] is token tau(g4, e))
        uint32_t keep[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t0 = j0 + 16 * (r >> 1) + 4 * g4 + 2 * (r & 1);
          keep[r] = (t0 < cur.kv_len ? 0x0000FFFFu : 0u) | (t0 + 1 < cur.kv_len ? 0xFFFF0000u : 0u);
        }
#pragma unroll
        for (int jm = 0; jm < NJ; ++jm)
#pragma unroll
          for (int r = 0; r < 4; ++r) va[jm][r] &= keep[r];
      }
      pv_tile<DT, NJ, NT>(va, pb, o);
      ++n;
    };

    if (has_tiles) {
      int limit = p.mask_mode == BSX_MASK_NONE ? cur.kv_len : diag;
      if (p.mask_mode == BSX_MASK_STREAMING) limit = 0;
      const int t_split = max(cur.t0, min(cur.t1, limit / kTile));
      for (int tile = cur.t0; tile < t_split; ++tile) tile_step(tile, std::false_type());
      for (int tile = t_split; tile < cur.t1; ++tile) tile_step(tile, std::true_type());
    }
    finish_segment<DT, D, NT, false>(p, cur, h, row0, c16, g4, o, m_ref, l_run);
  }
  // No direct load may still target this workgroup's LDS when it exits.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ---- Wave-split tiles -----------------------------------------------------------------
//
// For batches of short views with at most 16 query rows per kv head (a draft token over a
// sink + window view, say) and enough (request, kv head) pairs to fill the device: one
// workgroup per pair, whose kSplitWaves waves split the request's visible tiles into
// contiguous runs, each with its own online softmax, and combine them in LDS:
//   o = sum_w 2^(m_w - M) o_w / sum_w 2^(m_w - M) l_w,  lse = M + log2(sum_w ...),
// with M the largest reference maximum of the waves that saw a visible token.  No partial
// leaves the workgroup, so no merge launch follows.  The tile step is the per-wave
// kernel's (whole-line K loads, V rows transposed in registers, the next tile's loads
// issued as soon as its registers are free); every tile is masked (causal, sink +
// window, kv end).
using attn_shape::kSplitWaves;

template <int DT, int D>
__global__ void __launch_bounds__(64 * kSplitWaves) verify_attn_wsplit_kernel(Params p) {
  constexpr int NT = 1;
  constexpr int KS = D / 32;  // k-steps of the QK^T contraction
  constexpr int NJ = D / 16;  // output d tiles
  constexpr int VW = NJ / 2;  // dwords per lane per token of a V row
  constexpr int W = kSplitWaves;
  constexpr int FR = 4 * NJ;  // output floats per lane
  // [wave][fragment element][lane]: each store and read covers 64 consecutive floats
  __shared__ float o_lds[W][FR][64];
  __shared__ float m_lds[W][64], l_lds[W][64];
  __shared__ float oc_lds[FR][64];  // the combined, normalised output

  const int lane = threadIdx.x & 63;
  const int wave = uni(threadIdx.x >> 6);
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const int h = blockIdx.y;
  Seg cur;
  {
    const int32_t* sq = p.blob + p.off_seq + 4 * blockIdx.x;
    cur.b = blockIdx.x;
    cur.qo_start = ld_uniform(sq, 0);
    cur.qo_len = ld_uniform(sq, 1);
    cur.kv_len = ld_uniform(sq, 2);
    cur.page_start = ld_uniform(sq, 3);
    cur.slot = -1;
    cur.t0 = 0;
    cur.t1 = 0;
  }
  if (cur.qo_len == 0) return;  // (the whole workgroup)
  const int g = p.group;
  const uint32_t tok_bytes = (uint32_t)(p.num_kv_heads * D * 2);
  const uint32_t head_off = (uint32_t)(h * D * 2);

  // The layer's appended rows of this request and kv head, written before any load
  // (the stores complete before the barrier).
  if (p.k_new != nullptr) {
    constexpr int PIECES = D * 2 / 16;  // 16-byte pieces of a row's head slice
    const int diag0 = cur.kv_len - cur.qo_len;
    for (int idx = threadIdx.x; idx < cur.qo_len * PIECES; idx += blockDim.x) {
      const int i = idx / PIECES;
      const int pos = diag0 + i;
      if (pos < 0) continue;
      const int64_t col = (int64_t)head_off + (int64_t)(idx - i * PIECES) * 16;
      const int page = p.kv_indices[cur.page_start + (pos >> p.page_shift)];
      const int64_t dst = (int64_t)page * p.page_stride_bytes +
                          (int64_t)(pos & p.page_mask) * tok_bytes + col;
      const int64_t src = cur.qo_start + i;
      const u32x4 kv = *reinterpret_cast<const u32x4*>(
          reinterpret_cast<const char*>(p.k_new + src * p.knew_stride) + col);
      const u32x4 vv = *reinterpret_cast<const u32x4*>(
          reinterpret_cast<const char*>(p.v_new + src * p.vnew_stride) + col);
      *reinterpret_cast<u32x4*>(const_cast<char*>(p.k_cache) + dst) = kv;
      *reinterpret_cast<u32x4*>(const_cast<char*>(p.v_cache) + dst) = vv;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  // The visible tiles [0, a_end) and [w_beg, ntiles) (one run unless a sink + window view
  // leaves a gap), and this wave's run of them.
  const int ntiles = (cur.kv_len + kTile - 1) / kTile;
  int a_end = ntiles, w_beg = ntiles;
  if (p.mask_mode == BSX_MASK_STREAMING && cur.kv_len > p.sink + p.window) {
    const int ae = (p.sink + kTile - 1) / kTile;
    const int wb = max(0, cur.kv_len - p.window) / kTile;
    if (wb > ae) {
      a_end = ae;
      w_beg = wb;
    }
  }
  const int T = a_end + (ntiles - w_beg);
  const int i0 = (int)((int64_t)T * wave / W);
  const int i1 = (int)((int64_t)T * (wave + 1) / W);
  auto tile_of = [&](int i) { return i < a_end ? i : w_beg + (i - a_end); };

  const int nrows = cur.qo_len * g;  // <= 16 (the planner's condition)
  const int diag = cur.kv_len - cur.qo_len;
  const int sink_end = p.mask_mode == BSX_MASK_STREAMING ? p.sink : cur.kv_len;
  const int win_beg = p.mask_mode == BSX_MASK_STREAMING ? cur.kv_len - p.window : cur.kv_len;
  RowMask rm[NT];
  row_masks<NT>(p, cur, 0, c16, rm);
  // Q (B operand of S^T = K Q^T): lane holds query row c16, d chunk (s, g4); padded rows
  // read row 0 (finite data; their results are never stored)
  u32x4 qr[KS];
  {
    const bool rv = c16 < nrows;
    const int tq = rv ? c16 / g : 0;
    const int hh = rv ? c16 - tq * g : 0;
    const uint16_t* qp =
        p.q + (int64_t)(cur.qo_start + tq) * p.q_stride + (int64_t)(h * g + hh) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) qr[s] = *reinterpret_cast<const u32x4*>(qp + 32 * s + 8 * g4);
  }

  // Tile loads (page size >= 16: a 16-token subtile lies in one page).  K: whole
  // 128-byte lines (token (c16 & 7) + 8 h, bytes 128 q + 16 (g4 + 4 (c16 >> 3))), moved
  // into the A layout by a row rotation; V: 8 token rows per lane.
  u32x4 kreg[2][KS];
  uint32_t vraw[8][VW];
  const int ktok = c16 & 7;
  const uint32_t kbyte = (uint32_t)(16 * (g4 + 4 * (c16 >> 3)));
  auto page_of = [&](int js) {
    const int jsc = js < cur.kv_len ? js : 0;
    return ld_uniform(p.kv_indices, cur.page_start + (jsc >> p.page_shift));
  };
  auto load_tile_k = [&](int tile) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int js = tile * kTile + 16 * st;
      const int jsc = js < cur.kv_len ? js : 0;
      const char* base = p.k_cache + (int64_t)page_of(js) * p.page_stride_bytes;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const uint32_t off =
            (uint32_t)(((jsc & p.page_mask) + ktok + 8 * hh) * tok_bytes) + head_off + kbyte;
#pragma unroll
        for (int q = 0; q < KS / 2; ++q) kreg[st][2 * q + hh] = ld_stream(base + off + 128 * q);
      }
    }
  };
  const bool klow = c16 < 8;
  auto kfix = [&](u32x4 (&a)[2][KS]) {
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int q = 0; q < KS / 2; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t x0 = kreg[st][2 * q][e], x1 = kreg[st][2 * q + 1][e];
          const uint32_t r0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)x0, 0x128, 0xf, 0xf, false);
          const uint32_t r1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)x1, 0x128, 0xf, 0xf, false);
          a[st][2 * q][e] = klow ? x0 : r1;
          a[st][2 * q + 1][e] = klow ? r0 : x1;
        }
  };
  auto load_tile_v = [&](int tile) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int js = tile * kTile + 16 * st;
      const int jsc = js < cur.kv_len ? js : 0;
      const char* base = p.v_cache + (int64_t)page_of(js) * p.page_stride_bytes;
      const uint32_t soff = (uint32_t)((jsc & p.page_mask) * tok_bytes) + head_off;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int e = 4 * st + e4;
        const uint32_t off = soff + (uint32_t)((4 * g4 + e4) * tok_bytes) + (uint32_t)(NJ * c16 * 2);
        if constexpr (VW == 4) {
          const u32x4 v = ld_stream(base + off);
#pragma unroll
          for (int w = 0; w < 4; ++w) vraw[e][w] = v[w];
        } else {
          const u32x2 v = ld_stream2(base + off);
          vraw[e][0] = v[0];
          vraw[e][1] = v[1];
        }
      }
    }
  };

  f32x4 o[NJ][NT];
#pragma unroll
  for (int jm = 0; jm < NJ; ++jm) o[jm][0] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_ref[NT] = {-INFINITY};
  float l_run[NT] = {0.f};
  auto tile_step = [&](int i, auto prefetch_tag) {
    constexpr bool PREFETCH = decltype(prefetch_tag)::value;
    const int j0 = tile_of(i) * kTile;
    const int nxt = tile_of(i + 1);
    u32x4 kop[2][KS];
    kfix(kop);
    f32x4 sacc[2][NT];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = mfma16x16x32<DT>(kop[st][s], qr[s], acc);
      sacc[st][0] = acc;
    }
    // K registers are free: the next tile's K (kept after their last reads, so the
    // loaded tile lands in place)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PREFETCH) load_tile_k(nxt);
    mask_tile<NT>(sacc, rm, j0, g4, diag, sink_end, win_beg);
    uint32_t pb[NT][4];
    softmax_tile<DT, NJ, NT>(sacc, p.scale_log2, m_ref, l_run, o, pb);
    zero_rows_past_end<VW>(vraw, j0, g4, cur.kv_len);
    u32x4 va[NJ];
    transpose_v<NJ, VW>(vraw, va);
#pragma unroll
    for (int jm = 0; jm < NJ; ++jm) asm volatile("" ::"v"(va[jm]) : "memory");
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PREFETCH) load_tile_v(nxt);  // V registers are free
    pv_tile<DT, NJ, NT>(va, pb, o);
  };
  if (i0 < i1) {
    load_tile_k(tile_of(i0));
    load_tile_v(tile_of(i0));
    for (int i = i0; i + 1 < i1; ++i) tile_step(i, std::true_type());
    tile_step(i1 - 1, std::false_type());  // the run's last tile: nothing to prefetch
  }

  // Combine the waves' runs in LDS: wave w combines and normalises output d-tiles w,
  // w + W, ... of every run into oc_lds, then the first wave stores the rows.
  float l = l_run[0];
  l += __shfl_xor(l, 16);
  l += __shfl_xor(l, 32);
#pragma unroll
  for (int jm = 0; jm < NJ; ++jm)
#pragma unroll
    for (int e = 0; e < 4; ++e) o_lds[wave][4 * jm + e][lane] = o[jm][0][e];
  m_lds[wave][lane] = m_ref[0];
  l_lds[wave][lane] = l;
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < W; ++w)
    if (l_lds[w][lane] > 0.f) M = fmaxf(M, m_lds[w][lane]);
  float f[W];
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float lw = l_lds[w][lane];
    f[w] = lw > 0.f ? __builtin_amdgcn_exp2f(m_lds[w][lane] - M) : 0.f;
    L += f[w] * lw;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  for (int jm = wave; jm < NJ; jm += W)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) acc += f[w] * o_lds[w][4 * jm + e][lane];
      oc_lds[4 * jm + e][lane] = acc * inv;
    }
  __syncthreads();
  if (wave != 0) return;
  f32x4 oc[NJ][NT];
#pragma unroll
  for (int jm = 0; jm < NJ; ++jm)
#pragma unroll
    for (int e = 0; e < 4; ++e) oc[jm][0][e] = oc_lds[4 * jm + e][lane];
  if (c16 < nrows) {
    const int tq = c16 / g;
    const int hh = c16 - tq * g;
    uint16_t* op = p.out + (int64_t)(cur.qo_start + tq) * p.out_stride + (int64_t)(h * g + hh) * D;
    store_row<DT, D, NT, true>(op, g4, oc, 0);
    if (p.lse_out != nullptr && g4 == 0)
      p.lse_out[(int64_t)(cur.qo_start + tq) * p.num_qo_heads + h * g + hh] =
          (L > 0.f ? M + __log2f(L) : -INFINITY) * 0.69314718055994531f;
  }
}

// Combine the partial results of split requests: o = sum_p w_p o_p / sum_p w_p with
// w_p = 2^(lse_p - max lse), parts in slot order.  grid (split request, kv head, row
// chunk); one thread per (query row, 4 output columns).  The lse and o of up to U
// parts are loaded together (one memory round trip for most requests); longer part
// lists are folded in with a running maximum.
template <int DT, int D>
__global__ void __launch_bounds__(256) merge_kernel(Params p) {
  constexpr int TPR = D / 8;  // threads per row (8 columns each)
  constexpr int RPB = 256 / TPR;
  constexpr int U = 8;        // parts loaded per round
  // the request's merge record {first part, end of parts, first query token, query
  // tokens}: one scalar load
  typedef const u32x4 __attribute__((address_space(4)))* const_u4_ptr;
  // (a device plan's grid covers every request; its record count is in the blob)
  if (p.off_dyn >= 0 && (int)blockIdx.x >= ld_uniform(p.blob, p.off_dyn)) return;
  const u32x4 rec = ((const_u4_ptr)(p.blob + p.off_merge_seqs))[blockIdx.x];
  const int h = blockIdx.y;
  const int pbeg = (int)rec[0];
  const int pend = (int)rec[1];
  const int qo_start = (int)rec[2];
  const int qo_len = (int)rec[3];
  const int g = p.group;
  const int row = blockIdx.z * RPB + threadIdx.x / TPR;
  if (row >= qo_len * g) return;
  const int d8 = (threadIdx.x % TPR) * 8;
  const int64_t stride = (int64_t)p.num_kv_heads * p.qrows_total;  // rows between parts
  const int64_t base0 = (int64_t)h * p.qrows_total + row;
  float mx = -INFINITY;
  float wsum = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int q0 = pbeg; q0 < pend; q0 += U) {
    float l[U];
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int q = min(q0 + u, pend - 1);
      l[u] = q0 + u < pend ? p.part_lse[q * stride + base0] : -INFINITY;
      v[u] = *reinterpret_cast<const u32x4*>(p.part_o + (q * stride + base0) * D + d8);
    }
    float m_new = mx;
#pragma unroll
    for (int u = 0; u < U; ++u) m_new = fmaxf(m_new, l[u]);
    if (m_new == -INFINITY) continue;  // no visible token so far
    const float alpha = __builtin_amdgcn_exp2f(mx - m_new);  // 0 when mx is -inf
    wsum *= alpha;
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float w = __builtin_amdgcn_exp2f(l[u] - m_new);  // 0 for padded parts
      wsum += w;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[2 * c] += w * lo_f32<DT>(v[u][c]);
        acc[2 * c + 1] += w * hi_f32<DT>(v[u][c]);
      }
    }
    mx = m_new;
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const int tq = row / g;
  const int hh = row - tq * g;
  uint16_t* op = p.out + (int64_t)(qo_start + tq) * p.out_stride + (int64_t)(h * g + hh) * D + d8;
  u32x4 pk = {pack2<DT>(acc[0] * inv, acc[1] * inv), pack2<DT>(acc[2] * inv, acc[3] * inv),
              pack2<DT>(acc[4] * inv, acc[5] * inv), pack2<DT>(acc[6] * inv, acc[7] * inv)};
  *reinterpret_cast<u32x4*>(op) = pk;
  if (p.lse_out != nullptr && d8 == 0)
    p.lse_out[(int64_t)(qo_start + tq) * p.num_qo_heads + h * g + hh] =
        (wsum > 0.f ? mx + __log2f(wsum) : -INFINITY) * 0.69314718055994531f;
}

// Output of a batch whose page table holds no page at all: zeros (lse -inf).
template <int D>
__global__ void __launch_bounds__(256) empty_kernel(Params p, int total_qo) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_tok = (int64_t)p.num_qo_heads * D / 8;
  if (i >= (int64_t)total_qo * per_tok) return;
  const int64_t t = i / per_tok;
  const int64_t c = i - t * per_tok;
  *reinterpret_cast<u32x4*>(p.out + t * p.out_stride + c * 8) = u32x4{0u, 0u, 0u, 0u};
  if (p.lse_out != nullptr && c < p.num_qo_heads) p.lse_out[t * p.num_qo_heads + c] = -INFINITY;
}

template <int DT, int D, int NT, bool PS16>
static int launch_main(const bsx_attn_plan_t* plan, const Params& prm, int waves, hipStream_t st) {
  dim3 grid(plan->num_ctas, (plan->num_kv_heads / plan->heads_per_cta) * prm.n_qgroups);
  if (plan->mask_mode == BSX_MASK_CUSTOM)
    hipLaunchKernelGGL((verify_attn_kernel<DT, D, NT, PS16, true>), grid, dim3(64 * waves), 0, st,
                       prm);
  else
    hipLaunchKernelGGL((verify_attn_kernel<DT, D, NT, PS16>), grid, dim3(64 * waves), 0, st, prm);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

template <int DT, int D, int QB>
static int launch_shared(const bsx_attn_plan_t* plan, const Params& prm, hipStream_t st) {
  dim3 grid(plan->num_ctas, (plan->num_kv_heads / plan->heads_per_cta) * prm.n_qgroups);
  hipLaunchKernelGGL((verify_attn_shared_kernel<DT, D, QB>), grid,
                     dim3(64 * plan->heads_per_cta * QB), 0, st, prm);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

template <int DT, int D>
static int launch_all(const bsx_attn_plan_t* plan, const Params& prm, hipStream_t st) {
  if (prm.safe_pos < 0) {
    const int64_t n = (int64_t)plan->total_qo * plan->num_qo_heads * D / 8;
    if (n == 0) return BSX_OK;
    hipLaunchKernelGGL((empty_kernel<D>), dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, st, prm,
                       plan->total_qo);
    BSX_LAUNCH_CHECK();
    return BSX_OK;
  }
  if (plan->shared_kv_tiles == attn_shape::kPlanWaveSplit) {
    // one workgroup per (request, kv head); the waves merge in LDS: no merge launch
    hipLaunchKernelGGL((verify_attn_wsplit_kernel<DT, D>),
                       dim3(plan->batch, plan->num_kv_heads), dim3(64 * kSplitWaves), 0, st, prm);
    BSX_LAUNCH_CHECK();
    return BSX_OK;
  }
  const int waves = plan->heads_per_cta * prm.qblocks_per_cta;
  const bool ps16 = plan->page_size >= 16;
  int rc;
  if (plan->shared_kv_tiles) {
    rc = plan->qblocks_per_cta == 2   ? launch_shared<DT, D, 2>(plan, prm, st)
         : plan->qblocks_per_cta == 4 ? launch_shared<DT, D, 4>(plan, prm, st)
                                      : launch_shared<DT, D, 8>(plan, prm, st);
  } else if (plan->qrow_tile == 16) {
    rc = ps16 ? launch_main<DT, D, 1, true>(plan, prm, waves, st)
              : launch_main<DT, D, 1, false>(plan, prm, waves, st);
  } else {
    rc = ps16 ? launch_main<DT, D, 2, true>(plan, prm, waves, st)
              : launch_main<DT, D, 2, false>(plan, prm, waves, st);
  }
  if (rc != BSX_OK || plan->num_split_requests == 0) return rc;
  constexpr int RPB = 256 / (D / 8);
  const int max_rows = plan->max_qo_len * plan->group_size;
  dim3 grid(plan->num_split_requests, plan->num_kv_heads, (max_rows + RPB - 1) / RPB);
  hipLaunchKernelGGL((merge_kernel<DT, D>), grid, dim3(256), 0, st, prm);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

}  // namespace attn
}  // namespace bsx

using namespace bsx;

static int attn_run_impl(const bsx_attn_plan_t* plan, const int32_t* plan_blob_d, void* float_ws_d,
                         int dtype, const void* q_d, int64_t q_stride_tok,
                         const void* k_cache_d, const void* v_cache_d, int64_t page_stride,
                         const int32_t* kv_indices_d, const uint32_t* mask_words_d,
                         void* out_d, int64_t out_stride_tok, float* lse_d,
                         const void* k_new_d, int64_t k_new_stride, const void* v_new_d,
                         int64_t v_new_stride, void* stream) {
  BSX_REQUIRE(plan != nullptr && plan_blob_d != nullptr, BSX_ERR_INVALID, "null plan");
  BSX_REQUIRE(q_d && k_cache_d && v_cache_d && kv_indices_d && out_d, BSX_ERR_INVALID,
              "null tensor pointer");
  BSX_REQUIRE(dtype == BSX_DTYPE_BF16 || dtype == BSX_DTYPE_FP16, BSX_ERR_UNSUPPORTED,
              "verify attention supports bf16 and fp16 (got dtype %d)", dtype);
  BSX_REQUIRE(plan->head_dim == 64 || plan->head_dim == 128, BSX_ERR_UNSUPPORTED,
              "head_dim %d not supported (64 or 128)", plan->head_dim);
  BSX_REQUIRE((plan->mask_mode != BSX_MASK_TREE && plan->mask_mode != BSX_MASK_CUSTOM) ||
                  mask_words_d != nullptr,
              BSX_ERR_INVALID, "tree and custom mask modes need mask words");
  BSX_REQUIRE(plan->mask_mode != BSX_MASK_CUSTOM || !plan->shared_kv_tiles, BSX_ERR_INVALID,
              "inconsistent plan (custom masks run on the per-wave kernel)");
  BSX_REQUIRE(plan->num_partials == 0 || float_ws_d != nullptr, BSX_ERR_INVALID,
              "plan splits sequences but no float workspace given");
  BSX_REQUIRE(q_stride_tok >= (int64_t)plan->num_qo_heads * plan->head_dim &&
                  out_stride_tok >= (int64_t)plan->num_qo_heads * plan->head_dim,
              BSX_ERR_INVALID, "token stride smaller than heads*head_dim");
  BSX_REQUIRE(((uintptr_t)q_d % 16) == 0 && ((uintptr_t)out_d % 16) == 0 &&
                  ((uintptr_t)k_cache_d % 16) == 0 && ((uintptr_t)v_cache_d % 16) == 0 &&
                  (q_stride_tok % 8) == 0 && (out_stride_tok % 8) == 0 && (page_stride % 8) == 0,
              BSX_ERR_INVALID, "q/out/cache must be 16-byte aligned with strides multiple of 8");
  BSX_REQUIRE(plan->heads_per_cta > 0 && plan->num_kv_heads % plan->heads_per_cta == 0 &&
                  plan->qblocks_per_cta > 0 &&
                  plan->heads_per_cta * plan->qblocks_per_cta <= 8 &&
                  plan->num_qgroups * plan->qblocks_per_cta >= plan->qrow_blocks,
              BSX_ERR_INVALID, "inconsistent plan (workgroup shape)");
  if (plan->shared_kv_tiles == attn_shape::kPlanWaveSplit) {
    BSX_REQUIRE(plan->qrow_tile == 16 && plan->qrow_blocks == 1 && plan->page_size >= 16 &&
                    !plan->device_plan &&
                    (plan->mask_mode == BSX_MASK_NONE || plan->mask_mode == BSX_MASK_CAUSAL ||
                     plan->mask_mode == BSX_MASK_STREAMING),
                BSX_ERR_INVALID, "inconsistent plan (wave-split tiles)");
  } else if (plan->shared_kv_tiles) {
    const int qb = plan->qblocks_per_cta;
    BSX_REQUIRE((qb == 2 || qb == 4 || qb == 8) && plan->qrow_tile == 32 &&
                    plan->page_size >= 16 &&
                    plan->heads_per_cta <= attn_shape::shared_max_heads(plan->head_dim, qb),
                BSX_ERR_INVALID, "inconsistent plan (shared kv tiles)");
  }
  if (k_new_d || v_new_d) {
    BSX_REQUIRE(k_new_d && v_new_d, BSX_ERR_INVALID, "append needs both k_new and v_new");
    BSX_REQUIRE(((uintptr_t)k_new_d % 16) == 0 && ((uintptr_t)v_new_d % 16) == 0 &&
                    k_new_stride % 8 == 0 && v_new_stride % 8 == 0 &&
                    k_new_stride >= (int64_t)plan->num_kv_heads * plan->head_dim &&
                    v_new_stride >= (int64_t)plan->num_kv_heads * plan->head_dim,
                BSX_ERR_INVALID,
                "k_new/v_new must be 16-byte aligned with token strides >= H_kv*D, multiples of 8");
    BSX_REQUIRE(plan->safe_page_pos >= 0, BSX_ERR_INVALID,
                "the page table holds no page to append into");
  }
  if (plan->total_qo == 0) return BSX_OK;

  attn::Params prm;
  prm.k_new = static_cast<const uint16_t*>(k_new_d);
  prm.v_new = static_cast<const uint16_t*>(v_new_d);
  prm.knew_stride = k_new_stride;
  prm.vnew_stride = v_new_stride;
  prm.blob = plan_blob_d;
  prm.off_seq = plan->off_seq;
  prm.off_merge_seqs = plan->off_merge_seqs;
  prm.off_seg_indptr = plan->off_seg_indptr;
  prm.off_segments = plan->off_segments;
  prm.off_part_indptr = plan->off_part_indptr;
  prm.safe_pos = plan->safe_page_pos;
  prm.off_dyn = plan->device_plan ? plan->off_dyn : -1;
  prm.q = static_cast<const uint16_t*>(q_d);
  prm.q_stride = q_stride_tok;
  prm.k_cache = static_cast<const char*>(k_cache_d);
  prm.v_cache = static_cast<const char*>(v_cache_d);
  prm.page_stride_bytes = page_stride * 2;
  prm.kv_indices = kv_indices_d;
  prm.mask_words = mask_words_d;
  prm.bits_base = plan->batch;
  prm.out = static_cast<uint16_t*>(out_d);
  prm.out_stride = out_stride_tok;
  prm.lse_out = lse_d;
  // float workspace: [partial o (bf16)][partial lse (fp32)]
  const int64_t part_o_elems =
      (int64_t)plan->num_partials * plan->num_kv_heads * plan->qrow_tile * plan->qrow_blocks *
      plan->head_dim;
  prm.part_o = static_cast<uint16_t*>(float_ws_d);
  prm.part_lse = prm.part_o ? reinterpret_cast<float*>(prm.part_o + part_o_elems) : nullptr;
  prm.num_qo_heads = plan->num_qo_heads;
  prm.num_kv_heads = plan->num_kv_heads;
  prm.group = plan->group_size;
  int shift = 0;
  while ((1 << shift) < plan->page_size) ++shift;
  prm.page_shift = shift;
  prm.page_mask = plan->page_size - 1;
  prm.mask_mode = plan->mask_mode;
  prm.sink = plan->sink_tokens;
  prm.window = plan->window_tokens;
  prm.scale_log2 = plan->sm_scale * 1.4426950408889634f;
  prm.heads_per_cta = plan->heads_per_cta;
  prm.qblocks_per_cta = plan->qblocks_per_cta;
  prm.n_qgroups = plan->num_qgroups;
  prm.qrows_total = plan->qrow_tile * plan->qrow_blocks;
  prm.qrow_blocks = plan->qrow_blocks;

  hipStream_t st = as_stream(stream);
  if (dtype == BSX_DTYPE_BF16) {
    return plan->head_dim == 128 ? attn::launch_all<BSX_DTYPE_BF16, 128>(plan, prm, st)
                                 : attn::launch_all<BSX_DTYPE_BF16, 64>(plan, prm, st);
  }
  return plan->head_dim == 128 ? attn::launch_all<BSX_DTYPE_FP16, 128>(plan, prm, st)
                               : attn::launch_all<BSX_DTYPE_FP16, 64>(plan, prm, st);
}

extern "C" int bsx_attn_run(const bsx_attn_plan_t* plan, const int32_t* plan_blob_d, void* float_ws_d,
                            int dtype, const void* q_d, int64_t q_stride_tok,
                            const void* k_cache_d, const void* v_cache_d, int64_t page_stride,
                            const int32_t* kv_indices_d, const uint32_t* mask_words_d,
                            void* out_d, int64_t out_stride_tok, float* lse_d, void* stream) {
  return attn_run_impl(plan, plan_blob_d, float_ws_d, dtype, q_d, q_stride_tok, k_cache_d,
                       v_cache_d, page_stride, kv_indices_d, mask_words_d, out_d, out_stride_tok,
                       lse_d, nullptr, 0, nullptr, 0, stream);
}

extern "C" int bsx_attn_run_append(const bsx_attn_plan_t* plan, const int32_t* plan_blob_d,
                                   void* float_ws_d, int dtype, const void* q_d,
                                   int64_t q_stride_tok, const void* k_cache_d,
                                   const void* v_cache_d, int64_t page_stride,
                                   const int32_t* kv_indices_d, const uint32_t* mask_words_d,
                                   void* out_d, int64_t out_stride_tok, float* lse_d,
                                   const void* k_new_d, int64_t k_new_stride_tok,
                                   const void* v_new_d, int64_t v_new_stride_tok, void* stream) {
  BSX_REQUIRE(k_new_d && v_new_d, BSX_ERR_INVALID, "null k_new / v_new");
  return attn_run_impl(plan, plan_blob_d, float_ws_d, dtype, q_d, q_stride_tok, k_cache_d,
                       v_cache_d, page_stride, kv_indices_d, mask_words_d, out_d, out_stride_tok,
                       lse_d, k_new_d, k_new_stride_tok, v_new_d, v_new_stride_tok, stream);
}
