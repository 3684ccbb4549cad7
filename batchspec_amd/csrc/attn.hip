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
//     rows straight from the cache, B = Q^T).  In the accumulator layout each lane
//     then holds one query row, so the online-softmax row statistics are lane-local
//     up to a 4-lane reduction;
//   * the output is accumulated transposed as well, O^T = V^T P^T.  P^T is already in
//     B-operand layout (the kv-token order inside the 32-wide contraction is permuted
//     consistently for P and V).  V^T is formed from 16-byte row loads by an 8x8
//     transpose of 16-bit values in registers (v_perm_b32), so no LDS is used;
//   * workgroups are persistent: the host plan cuts the total tile count evenly over
//     the grid; a sequence split over several segments writes fp32 partials with their
//     log-sum-exp, and a merge kernel combines them.
#include <type_traits>

#include "common.h"

namespace bsx {
namespace attn {

constexpr int kTile = 32;

struct Params {
  const int32_t* blob;
  int off_seq, off_seg_indptr, off_segments, off_merge_seqs, off_part_indptr;
  const uint16_t* q;
  int64_t q_stride;  // elements between tokens
  const char* k_cache;
  const char* v_cache;
  int64_t page_stride_bytes;
  const int32_t* kv_indices;
  const uint32_t* mask_words;
  uint16_t* out;
  int64_t out_stride;
  float* lse_out;
  float* part_o;
  float* part_lse;
  int num_qo_heads, num_kv_heads, group;
  int page_shift, page_mask;
  int mask_mode, sink, window;
  float scale_log2;  // sm_scale * log2(e)
  int heads_per_cta, qblocks_per_cta, n_qgroups, qrows_total;
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Wave-uniform read of read-only int32 metadata (plan blob, page ids) through the
// scalar unit: s_load is tracked by lgkmcnt, so it never waits behind the vector
// loads of the K/V tiles in flight.
typedef const int32_t __attribute__((address_space(4)))* const_i32_ptr;
__device__ __forceinline__ int ld_uniform(const int32_t* base, int64_t i) {
  return ((const_i32_ptr)base)[i];
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

template <int DT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)f32_to_half_bits<DT>(lo) | ((uint32_t)f32_to_half_bits<DT>(hi) << 16);
}

// Visibility of kv token j for query token tq of a request (j < kv_len already known).
__device__ __forceinline__ bool visible(const Params& p, int mode, int j, int tq, int kv_len,
                                        int qo_len, uint32_t word) {
  const int diag = kv_len - qo_len;  // first kv column of the draft block
  if (mode == BSX_MASK_CAUSAL) return j <= diag + tq;
  if (mode == BSX_MASK_TREE) return j < diag || ((word >> (uint32_t)(j - diag)) & 1u);
  if (mode == BSX_MASK_STREAMING)
    return (j < p.sink || j >= kv_len - p.window) && j <= diag + tq;
  return true;
}

// Combine the partial results of split requests: o = sum_p w_p o_p / sum_p w_p with
// w_p = 2^(lse_p - max lse).  grid (merge request, kv head, row chunk); one thread
// per (query row, 4 output columns); the part loads are unrolled so they overlap.
template <int DT, int D>
__global__ void __launch_bounds__(256) merge_kernel(Params p) {
  constexpr int TPR = D / 4;    // threads per row
  constexpr int RPB = 256 / TPR;
  constexpr int U = 8;          // parts loaded per round
  const int b = ld_uniform(p.blob, p.off_merge_seqs + blockIdx.x);
  const int h = blockIdx.y;
  const int pbeg = ld_uniform(p.blob, p.off_part_indptr + b);
  const int pend = ld_uniform(p.blob, p.off_part_indptr + b + 1);
  const int qo_start = ld_uniform(p.blob, p.off_seq + b * 4 + 0);
  const int qo_len = ld_uniform(p.blob, p.off_seq + b * 4 + 1);
  const int g = p.group;
  const int row = blockIdx.z * RPB + threadIdx.x / TPR;
  if (row >= qo_len * g) return;
  const int d4 = (threadIdx.x % TPR) * 4;
  const int64_t stride = (int64_t)p.num_kv_heads * p.qrows_total;  // between parts
  const int64_t base0 = (int64_t)h * p.qrows_total + row;
  float mx = -INFINITY;
  for (int q0 = pbeg; q0 < pend; q0 += U) {
    float l[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      l[u] = q0 + u < pend ? p.part_lse[(q0 + u) * stride + base0] : -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u) mx = fmaxf(mx, l[u]);
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  float wsum = 0.f;
  if (mx != -INFINITY) {
    for (int q0 = pbeg; q0 < pend; q0 += U) {
      float l[U];
      f32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int q = min(q0 + u, pend - 1);
        l[u] = p.part_lse[q * stride + base0];
        v[u] = *reinterpret_cast<const f32x4*>(p.part_o + (q * stride + base0) * D + d4);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (q0 + u < pend) {
          const float w = __builtin_amdgcn_exp2f(l[u] - mx);
          acc += w * v[u];
          wsum += w;
        }
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const int tq = row / g;
  const int hh = row - tq * g;
  uint16_t* op = p.out + (int64_t)(qo_start + tq) * p.out_stride + (int64_t)(h * g + hh) * D + d4;
  u32x2 pk = {pack2<DT>(acc[0] * inv, acc[1] * inv), pack2<DT>(acc[2] * inv, acc[3] * inv)};
  *reinterpret_cast<u32x2*>(op) = pk;
  if (p.lse_out != nullptr && d4 == 0)
    p.lse_out[(int64_t)(qo_start + tq) * p.num_qo_heads + h * g + hh] =
        (wsum > 0.f ? mx + __log2f(wsum) : -INFINITY) * 0.69314718055994531f;
}

// NT: query-row tiles of 16 per wave.  D: head dim (64 or 128).
template <int DT, int D, int NT, bool PS_GE16>
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
  // The plan makes heads_per_cta divide num_kv_heads, so every wave has a head; all
  // waves take part in the block barriers of the partial-merge handshake.

  const int32_t* seq = p.blob + p.off_seq;
  const int32_t* segs = p.blob + p.off_segments;
  const int seg_begin = ld_uniform(p.blob, p.off_seg_indptr + blockIdx.x);
  const int seg_end = ld_uniform(p.blob, p.off_seg_indptr + blockIdx.x + 1);

  const int g = p.group;
  const int64_t tok_bytes = (int64_t)p.num_kv_heads * D * 2;  // one kv token row (all heads)
  const uint32_t head_off = (uint32_t)(h * D * 2);

  for (int si = seg_begin; si < seg_end; ++si) {
    const int b = ld_uniform(segs, si * 4 + 0);
    const int t0 = ld_uniform(segs, si * 4 + 1);
    const int t1 = ld_uniform(segs, si * 4 + 2);
    const int slot = ld_uniform(segs, si * 4 + 3);
    const int qo_start = ld_uniform(seq, b * 4 + 0);
    const int qo_len = ld_uniform(seq, b * 4 + 1);
    const int kv_len = ld_uniform(seq, b * 4 + 2);
    const int page_start = ld_uniform(seq, b * 4 + 3);
    const int nrows = qo_len * g;
    const int row0 = qb * QT;

    if (row0 < nrows) {
      // ---- Q (B operand of S^T = K Q^T): lane holds query row c16 of tile nt, d chunk (s, g4).
      int tq_of[NT];
      uint32_t word_of[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int row = row0 + nt * 16 + c16;
        const bool rv = row < nrows;
        const int tq = rv ? row / g : 0;
        const int hh = rv ? row - tq * g : 0;
        tq_of[nt] = rv ? tq : qo_len;  // padded rows: any in-range bound is harmless
        word_of[nt] = 0u;
        if (p.mask_mode == BSX_MASK_TREE && rv) word_of[nt] = p.mask_words[qo_start + tq];
        const uint16_t* qp =
            p.q + (int64_t)(qo_start + tq) * p.q_stride + (int64_t)(h * g + hh) * D;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          u32x4 v = {0u, 0u, 0u, 0u};
          if (rv) v = *reinterpret_cast<const u32x4*>(qp + 32 * s + 8 * g4);
          q_lds[wave][nt * KS + s][lane] = v;
        }
      }

      f32x4 o[NJ][NT];
#pragma unroll
      for (int jm = 0; jm < NJ; ++jm)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) o[jm][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      float m_run[NT], l_run[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        m_run[nt] = -INFINITY;
        l_run[nt] = 0.f;
      }

      // ---- tile loaders (K straight into A-operand layout; V as 8 token rows per lane)
      u32x4 kreg[2][KS];
      uint32_t vraw[8][VW];
      // Loads are unconditional (no exec-masked branches, so the compiler's wait
      // counting stays exact across the pipelined loop).  Addresses of tokens past
      // kv_len are clamped into memory the request owns; their scores are masked and
      // their V rows zeroed before use.
      auto load_tile_k = [&](int tile) {
        const int j0 = tile * kTile;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int js = j0 + 16 * st;
          const char* base;
          uint32_t off;
          if constexpr (PS_GE16) {
            const int jsc = js < kv_len ? js : 0;  // subtile start, clamped into the request
            const int page = ld_uniform(p.kv_indices, page_start + (jsc >> p.page_shift));
            base = p.k_cache + (int64_t)page * p.page_stride_bytes;
            off = (uint32_t)(((jsc & p.page_mask) + c16) * tok_bytes) + head_off;
          } else {
            const int j = min(js + c16, kv_len - 1);
            const int page = p.kv_indices[page_start + (j >> p.page_shift)];
            base = p.k_cache + (int64_t)page * p.page_stride_bytes;
            off = (uint32_t)((j & p.page_mask) * tok_bytes) + head_off;
          }
#pragma unroll
          for (int s = 0; s < KS; ++s)
            kreg[st][s] = *reinterpret_cast<const u32x4*>(base + off + (32 * s + 8 * g4) * 2);
        }
      };
      auto load_tile_v = [&](int tile) {
        const int j0 = tile * kTile;
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int js = j0 + 16 * st;
          const char* sbase = p.v_cache;
          uint32_t soff = 0;
          if constexpr (PS_GE16) {
            const int jsc = js < kv_len ? js : 0;
            const int page = ld_uniform(p.kv_indices, page_start + (jsc >> p.page_shift));
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
              const int j = min(js + 4 * g4 + e4, kv_len - 1);
              const int page = p.kv_indices[page_start + (j >> p.page_shift)];
              base = p.v_cache + (int64_t)page * p.page_stride_bytes;
              off = (uint32_t)((j & p.page_mask) * tok_bytes) + head_off;
            }
            off += (uint32_t)(NJ * c16 * 2);
            if constexpr (VW == 4) {
              const u32x4 v = *reinterpret_cast<const u32x4*>(base + off);
              vraw[e][0] = v[0];
              vraw[e][1] = v[1];
              vraw[e][2] = v[2];
              vraw[e][3] = v[3];
            } else {
              const u32x2 v = *reinterpret_cast<const u32x2*>(base + off);
              vraw[e][0] = v[0];
              vraw[e][1] = v[1];
            }
          }
        }
      };

      const int diag = kv_len - qo_len;
      // One tile: S^T = K Q^T, online softmax, O^T += V^T P^T, with the next tile's K
      // and V loads issued as soon as their registers are free.  MASKED is a
      // compile-time flag: the body loop over tiles that need no per-element mask is
      // branch-free, which keeps the compiler's load-wait counting exact.
      auto tile_step = [&](int tile, int t_end, auto masked_tag) {
        constexpr bool MASKED = decltype(masked_tag)::value;
        const int j0 = tile * kTile;
        // compiler-only barrier: keeps the Q reads from LDS inside the loop instead of
        // letting them be hoisted into registers the pipelined tiles need
        asm volatile("" ::: "memory");

        f32x4 sacc[2][NT];
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KS; ++s)
              acc = mfma16x16x32<DT>(kreg[st][s], q_lds[wave][nt * KS + s][lane], acc);
            sacc[st][nt] = acc;
          }
        if (tile + 1 < t_end) load_tile_k(tile + 1);  // K registers are free: prefetch

#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float sv = sacc[st][nt][e] * p.scale_log2;
              if constexpr (MASKED) {
                const int j = j0 + 16 * st + 4 * g4 + e;
                const bool vis = j < kv_len &&
                                 visible(p, p.mask_mode, j, tq_of[nt], kv_len, qo_len, word_of[nt]);
                sv = vis ? sv : -INFINITY;
              }
              sacc[st][nt][e] = sv;
            }

        // online softmax (rows are lane-local; 4 lane groups share a row)
        uint32_t pb[NT][4];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float mx = fmaxf(fmaxf(fmaxf(sacc[0][nt][0], sacc[0][nt][1]),
                                 fmaxf(sacc[0][nt][2], sacc[0][nt][3])),
                           fmaxf(fmaxf(sacc[1][nt][0], sacc[1][nt][1]),
                                 fmaxf(sacc[1][nt][2], sacc[1][nt][3])));
          mx = fmaxf(mx, __shfl_xor(mx, 16));
          mx = fmaxf(mx, __shfl_xor(mx, 32));
          const float m_new = fmaxf(m_run[nt], mx);
          const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
          const float alpha = __builtin_amdgcn_exp2f(m_run[nt] - m_use);
          float pv[8];
          float rs = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            pv[e] = __builtin_amdgcn_exp2f(sacc[e >> 2][nt][e & 3] - m_use);
            rs += pv[e];
          }
          l_run[nt] = l_run[nt] * alpha + rs;
          m_run[nt] = m_new;
#pragma unroll
          for (int jm = 0; jm < NJ; ++jm) o[jm][nt] *= alpha;
#pragma unroll
          for (int r = 0; r < 4; ++r) pb[nt][r] = pack2<DT>(pv[2 * r], pv[2 * r + 1]);
        }

        if constexpr (MASKED) {  // rows past kv_len hold unrelated data: zero them
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const bool ok = j0 + 16 * (e >> 2) + 4 * g4 + (e & 3) < kv_len;
#pragma unroll
            for (int w = 0; w < VW; ++w) vraw[e][w] = ok ? vraw[e][w] : 0u;
          }
        }
        // V^T operands: A_jm[e] = V[tau(g4, e)][NJ*c16 + jm]
        u32x4 va[NJ];
#pragma unroll
        for (int jm = 0; jm < NJ; ++jm) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t w0 = vraw[2 * r][jm >> 1];
            const uint32_t w1 = vraw[2 * r + 1][jm >> 1];
            va[jm][r] = (jm & 1) ? perm_hi(w0, w1) : perm_lo(w0, w1);
          }
        }
        if (tile + 1 < t_end) load_tile_v(tile + 1);  // V registers are free: prefetch
#pragma unroll
        for (int jm = 0; jm < NJ; ++jm)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            u32x4 bop = {pb[nt][0], pb[nt][1], pb[nt][2], pb[nt][3]};
            o[jm][nt] = mfma16x16x32<DT>(va[jm], bop, o[jm][nt]);
          }
      };

      // Tiles [t0, t_split) lie entirely inside the visible prefix (no mask needed);
      // [t_split, t1) touch the draft block, the kv end, or the sink/window view.
      int limit = p.mask_mode == BSX_MASK_NONE ? kv_len : diag;
      if (p.mask_mode == BSX_MASK_STREAMING) limit = 0;
      const int t_split = max(t0, min(t1, limit / kTile));
      if (t0 < t1) {
        load_tile_k(t0);
        load_tile_v(t0);
      }
      for (int tile = t0; tile < t_split; ++tile)
        tile_step(tile, t1, std::integral_constant<bool, false>());
      for (int tile = t_split; tile < t1; ++tile)
        tile_step(tile, t1, std::integral_constant<bool, true>());

      // ---- finalize: lane holds row c16 of tile nt, d = NJ*(4 g4 + e) + jm
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float l = l_run[nt];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        const int row = row0 + nt * 16 + c16;
        if (row >= nrows) continue;
        const int tq = row / g;
        const int hh = row - tq * g;
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const float lse2 = l > 0.f ? m_run[nt] + __log2f(l) : -INFINITY;
        if (slot < 0) {
          uint16_t* op = p.out + (int64_t)(qo_start + tq) * p.out_stride +
                         (int64_t)(h * g + hh) * D + NJ * 4 * g4;
          uint32_t packed[2 * NJ];
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int jm = 0; jm < NJ; jm += 2)
              packed[(NJ * e + jm) / 2] = pack2<DT>(o[jm][nt][e] * inv, o[jm + 1][nt][e] * inv);
#pragma unroll
          for (int w = 0; w < 2 * NJ; w += 4) {
            u32x4 v = {packed[w], packed[w + 1], packed[w + 2], packed[w + 3]};
            *reinterpret_cast<u32x4*>(op + 2 * w) = v;
          }
          if (p.lse_out != nullptr && g4 == 0)
            p.lse_out[(int64_t)(qo_start + tq) * p.num_qo_heads + h * g + hh] =
                lse2 * 0.69314718055994531f;
        } else {
          float* pp = p.part_o +
                      (((int64_t)slot * p.num_kv_heads + h) * p.qrows_total + row) * D +
                      NJ * 4 * g4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int jm = 0; jm < NJ; jm += 4) {
              f32x4 v = {o[jm][nt][e] * inv, o[jm + 1][nt][e] * inv, o[jm + 2][nt][e] * inv,
                         o[jm + 3][nt][e] * inv};
              *reinterpret_cast<f32x4*>(pp + NJ * e + jm) = v;
            }
          }
          if (g4 == 0)
            p.part_lse[((int64_t)slot * p.num_kv_heads + h) * p.qrows_total + row] = lse2;
        }
      }
    }

  }
}

template <int DT, int D, int NT, bool PS16>
static int launch_main(const bsx_attn_plan_t* plan, const Params& prm, int waves, hipStream_t st) {
  dim3 grid(plan->num_ctas, (plan->num_kv_heads / plan->heads_per_cta) * prm.n_qgroups);
  hipLaunchKernelGGL((verify_attn_kernel<DT, D, NT, PS16>), grid, dim3(64 * waves), 0, st, prm);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

template <int DT, int D>
static int launch_all(const bsx_attn_plan_t* plan, const Params& prm, hipStream_t st) {
  const int waves = plan->heads_per_cta * prm.qblocks_per_cta;
  const bool ps16 = plan->page_size >= 16;
  int rc;
  if (plan->qrow_tile == 16) {
    rc = ps16 ? launch_main<DT, D, 1, true>(plan, prm, waves, st)
              : launch_main<DT, D, 1, false>(plan, prm, waves, st);
  } else {
    rc = ps16 ? launch_main<DT, D, 2, true>(plan, prm, waves, st)
              : launch_main<DT, D, 2, false>(plan, prm, waves, st);
  }
  if (rc != BSX_OK || plan->num_merge_seqs == 0) return rc;
  constexpr int RPB = 256 / (D / 4);
  const int max_rows = plan->max_qo_len * plan->group_size;
  dim3 grid(plan->num_merge_seqs, plan->num_kv_heads, (max_rows + RPB - 1) / RPB);
  hipLaunchKernelGGL((merge_kernel<DT, D>), grid, dim3(256), 0, st, prm);
  BSX_LAUNCH_CHECK();
  return BSX_OK;
}

}  // namespace attn
}  // namespace bsx

using namespace bsx;

extern "C" int bsx_attn_run(const bsx_attn_plan_t* plan, const int32_t* plan_blob_d,
                            void* float_ws_d, int dtype, const void* q_d, int64_t q_stride_tok,
                            const void* k_cache_d, const void* v_cache_d, int64_t page_stride,
                            const int32_t* kv_indices_d, const uint32_t* mask_words_d,
                            void* out_d, int64_t out_stride_tok, float* lse_d, void* stream) {
  BSX_REQUIRE(plan != nullptr && plan_blob_d != nullptr, BSX_ERR_INVALID, "null plan");
  BSX_REQUIRE(q_d && k_cache_d && v_cache_d && kv_indices_d && out_d, BSX_ERR_INVALID,
              "null tensor pointer");
  BSX_REQUIRE(dtype == BSX_DTYPE_BF16 || dtype == BSX_DTYPE_FP16, BSX_ERR_UNSUPPORTED,
              "verify attention supports bf16 and fp16 (got dtype %d)", dtype);
  BSX_REQUIRE(plan->head_dim == 64 || plan->head_dim == 128, BSX_ERR_UNSUPPORTED,
              "head_dim %d not supported (64 or 128)", plan->head_dim);
  BSX_REQUIRE(plan->mask_mode != BSX_MASK_TREE || mask_words_d != nullptr, BSX_ERR_INVALID,
              "tree mask mode needs mask words");
  BSX_REQUIRE(plan->num_merge_seqs == 0 || float_ws_d != nullptr, BSX_ERR_INVALID,
              "plan splits sequences but no float workspace given");
  BSX_REQUIRE(q_stride_tok >= (int64_t)plan->num_qo_heads * plan->head_dim &&
                  out_stride_tok >= (int64_t)plan->num_qo_heads * plan->head_dim,
              BSX_ERR_INVALID, "token stride smaller than heads*head_dim");
  BSX_REQUIRE(((uintptr_t)q_d % 16) == 0 && ((uintptr_t)out_d % 16) == 0 &&
                  ((uintptr_t)k_cache_d % 16) == 0 && ((uintptr_t)v_cache_d % 16) == 0 &&
                  (q_stride_tok % 8) == 0 && (out_stride_tok % 8) == 0 && (page_stride % 8) == 0,
              BSX_ERR_INVALID, "q/out/cache must be 16-byte aligned with strides multiple of 8");
  if (plan->num_segments == 0) return BSX_OK;

  attn::Params prm;
  prm.blob = plan_blob_d;
  prm.off_seq = plan->off_seq;
  prm.off_seg_indptr = plan->off_seg_indptr;
  prm.off_segments = plan->off_segments;
  prm.off_merge_seqs = plan->off_merge_seqs;
  prm.off_part_indptr = plan->off_part_indptr;
  prm.q = static_cast<const uint16_t*>(q_d);
  prm.q_stride = q_stride_tok;
  prm.k_cache = static_cast<const char*>(k_cache_d);
  prm.v_cache = static_cast<const char*>(v_cache_d);
  prm.page_stride_bytes = page_stride * 2;
  prm.kv_indices = kv_indices_d;
  prm.mask_words = mask_words_d;
  prm.out = static_cast<uint16_t*>(out_d);
  prm.out_stride = out_stride_tok;
  prm.lse_out = lse_d;
  // float workspace: [partial o][partial lse]
  const int64_t part_o_floats =
      (int64_t)plan->num_partials * plan->num_kv_heads * plan->qrow_tile * plan->qrow_blocks *
      plan->head_dim;
  prm.part_o = static_cast<float*>(float_ws_d);
  prm.part_lse = prm.part_o ? prm.part_o + part_o_floats : nullptr;
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
  BSX_REQUIRE(plan->heads_per_cta > 0 && plan->num_kv_heads % plan->heads_per_cta == 0 &&
                  plan->qblocks_per_cta > 0 &&
                  plan->heads_per_cta * plan->qblocks_per_cta <= 8 &&
                  plan->num_qgroups * plan->qblocks_per_cta >= plan->qrow_blocks,
              BSX_ERR_INVALID, "inconsistent plan (workgroup shape)");
  prm.heads_per_cta = plan->heads_per_cta;
  prm.qblocks_per_cta = plan->qblocks_per_cta;
  prm.n_qgroups = plan->num_qgroups;
  prm.qrows_total = plan->qrow_tile * plan->qrow_blocks;

  hipStream_t st = as_stream(stream);
  if (dtype == BSX_DTYPE_BF16) {
    return plan->head_dim == 128 ? attn::launch_all<BSX_DTYPE_BF16, 128>(plan, prm, st)
                                 : attn::launch_all<BSX_DTYPE_BF16, 64>(plan, prm, st);
  }
  return plan->head_dim == 128 ? attn::launch_all<BSX_DTYPE_FP16, 128>(plan, prm, st)
                               : attn::launch_all<BSX_DTYPE_FP16, 64>(plan, prm, st);
}
