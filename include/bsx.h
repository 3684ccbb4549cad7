/*
 * bsx.h — C ABI of the MI355X (gfx950) speculative-verification hot path.
 *
 * Three pieces, each replacing one FlashInfer call site of BatchSpec:
 *   1. paged-KV verify attention  (BatchPrefillWithPagedKVCacheWrapper.plan/run)
 *   2. paged KV append            (get_seq_lens / get_batch_indices_positions /
 *                                   append_paged_kv_cache)
 *   3. speculative acceptance     (evaluate_posterior greedy branch,
 *                                   chain_speculative_sampling, sampling.softmax)
 *
 * Conventions
 *   - Every pointer named *_d is device memory; *_h is host memory.
 *   - The caller owns every buffer, including workspaces; the library never
 *     allocates device memory.
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *     Every device entry point is asynchronous, does no host synchronisation and
 *     may be captured into a hipGraph.
 *   - Every entry point returns a bsx_status; on failure bsx_last_error() gives a
 *     thread-local message. Nothing throws across the ABI.
 *   - Integer index tensors are int32 (CSR page tables) or int64 (token ids), as
 *     in the reference.
 *   - A row of logits (vocab x dtype size) must stay below 2^31 bytes in the softmax,
 *     sampling and acceptance-from-logits entry points (BSX_ERR_UNSUPPORTED otherwise).
 */
#ifndef BSX_H
#define BSX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  BSX_OK = 0,
  BSX_ERR_INVALID = -1,     /* bad argument (shape, dtype, null pointer)        */
  BSX_ERR_CAPACITY = -2,    /* caller buffer or workspace too small             */
  BSX_ERR_UNSUPPORTED = -3, /* valid request outside what the kernels implement */
  BSX_ERR_HIP = -4          /* a HIP runtime call failed                        */
} bsx_status;

enum { BSX_DTYPE_BF16 = 0, BSX_DTYPE_FP16 = 1, BSX_DTYPE_FP32 = 2 };

/* Attention mask modes (the reference's plan(causal=..., custom_mask=...)). */
enum {
  BSX_MASK_NONE = 0,   /* full attention to all kv_len tokens                   */
  BSX_MASK_CAUSAL = 1, /* bottom-right aligned causal: q row t sees
                          j <= kv_len - qo_len + t                             */
  BSX_MASK_TREE = 2,   /* full attention to the first kv_len - qo_len tokens,
                          then bit (j - (kv_len - qo_len)) of a per-query-token
                          uint32 word over the last qo_len tokens (qo_len <= 32) */
  BSX_MASK_STREAMING = 3, /* sink + recent window view: token j is visible iff
                          j < sink or j >= kv_len - window, combined with the
                          causal rule over the last qo_len tokens              */
  BSX_MASK_CUSTOM = 4  /* any boolean [qo_len x kv_len] mask per request, packed
                          by bsx_custom_mask_prepare (host plans, per-wave kernel) */
};

const char* bsx_last_error(void);
int bsx_version(void);

/* ------------------------------------------------------------------------- */
/* 1. Verify attention                                                        */
/* ------------------------------------------------------------------------- */

/* Host-side schedule produced by bsx_attn_plan; the device half of the plan is
 * an int32 blob of `plan_ints` entries that the caller copies to device memory
 * (any stream ordering that completes before bsx_attn_run reads it); the kernels
 * only read it, so one copied blob serves any number of runs. */
typedef struct {
  int32_t batch;
  int32_t num_qo_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t page_size;
  int32_t mask_mode;
  int32_t group_size;     /* num_qo_heads / num_kv_heads                      */
  int32_t qrow_tile;      /* query rows per wave (16 or 32)                   */
  int32_t qrow_blocks;    /* waves per kv head that split the query rows      */
  int32_t heads_per_cta;  /* kv heads handled by one workgroup                */
  int32_t qblocks_per_cta;/* query-row blocks handled by one workgroup        */
  int32_t num_qgroups;    /* ceil(qrow_blocks / qblocks_per_cta)              */
  int32_t num_ctas;       /* grid.x of the kernel; grid.y =
                             (num_kv_heads/heads_per_cta) * num_qgroups       */
  int32_t num_segments;
  int32_t num_partials;   /* partial-result slots of split requests           */
  int32_t num_split_requests; /* requests whose kv range spans several segments */
  int32_t max_qo_len;
  int32_t tile_tokens;    /* kv tokens per inner-loop tile (32)               */
  int32_t sink_tokens;    /* BSX_MASK_STREAMING only                          */
  int32_t window_tokens;  /* BSX_MASK_STREAMING only                          */
  int32_t off_seq;        /* int32 offsets of the sub-arrays inside the blob   */
  int32_t off_seg_indptr;
  int32_t off_segments;
  int32_t off_merge_seqs;
  int32_t off_part_indptr;
  int32_t plan_ints;      /* total int32 entries of the device blob           */
  int64_t float_ws_bytes; /* bytes of float workspace bsx_attn_run needs       */
  float sm_scale;
  int32_t total_qo;       /* qo_indptr[batch]                                 */
  int32_t safe_page_pos;  /* a kv_indices position owned by some request, or -1
                             when the page table holds no page               */
  int32_t shared_kv_tiles;/* 1: the qblocks_per_cta waves of a kv head share
                             each K/V tile through LDS (many query rows per
                             kv head); 0: every wave streams its own tiles;
                             2: one workgroup per (request, kv head), its
                             waves splitting the request's tiles and merging
                             in LDS (grid batch x num_kv_heads, no partials) */
  int64_t total_tiles;    /* kv tiles of the whole schedule                   */
  int32_t device_plan;    /* 1: the blob is written on the device by
                             bsx_attn_plan_device; counts above are bounds    */
  int32_t off_dyn;        /* device plan: int32 offset of {split requests,
                             error code, segments, reserved} in the blob      */
} bsx_attn_plan_t;

/* Size (int32 entries) of the host buffer bsx_attn_plan needs for its blob. */
int64_t bsx_attn_plan_ints_bound(int batch, int num_cus);

/* Replaces BatchPrefillWithPagedKVCacheWrapper.plan(...) as called by
 * batchspec/backends/standard_engine.py:132-143 (causal=True) and
 * batchspec/backends/mtp_engine.py:420-432 (custom mask): validates the page
 * table, derives kv lengths (reference formula of FlashInfer get_seq_lens used at
 * batchspec/models/modules/kv_cache.py:66-70), and splits the kv work evenly over
 * a persistent grid sized to fill `num_cus` compute units.  Host-only; no GPU
 * needed.
 *   qo_indptr_h[batch+1], kv_indptr_h[batch+1], kv_last_page_len_h[batch]
 *   kv_indices_len: entries of the paged_kv_indices tensor run() will read;
 *   kv_indptr_h[batch] beyond it is rejected (negative: not checked).
 *   sm_scale <= 0 means 1/sqrt(head_dim). */
int bsx_attn_plan(const int32_t* qo_indptr_h, const int32_t* kv_indptr_h,
                  const int32_t* kv_last_page_len_h, int batch, int num_qo_heads,
                  int num_kv_heads, int head_dim, int page_size, int mask_mode,
                  int sink_tokens, int window_tokens, float sm_scale, int num_cus,
                  int64_t kv_indices_len, int32_t* plan_blob_h, int64_t blob_capacity_ints,
                  bsx_attn_plan_t* plan_out);

/* The same host schedule written into the fixed, bound-sized blob layout of a shape
 * made by bsx_attn_plan_device_shape (below) for the wrapper's use_cuda_graph=True
 * mode (batchspec/backends/base/attn_wrapper.py:53-57): every launch argument of
 * bsx_attn_run (grid, blob offsets, workspace layout, merge grid) depends on the
 * shape only, so a graph that captured run() stays valid when plan() is called again
 * with other lengths, as FlashInfer's graph mode allows.  batch <= shape->batch
 * (requests past `batch` are empty); every query length <= shape->max_qo_len; the
 * table must hold a page.  plan_out = *shape with total_qo and total_tiles set. */
int bsx_attn_plan_fixed(const bsx_attn_plan_t* shape, const int32_t* qo_indptr_h,
                        const int32_t* kv_indptr_h, const int32_t* kv_last_page_len_h,
                        int batch, int64_t kv_indices_len, int32_t* plan_blob_h,
                        int64_t blob_capacity_ints, bsx_attn_plan_t* plan_out);

/* Device-side planning (no counterpart in the reference, whose plan() always
 * schedules on the host from host copies of the page table,
 * batchspec/backends/base/attn_wrapper.py:33-72 with the callers above): the
 * schedule is computed by one GPU workgroup from the device page table, so a verify
 * step (page-table update, plan, attention, acceptance) can be captured in one graph
 * and replayed with lengths that change between replays.
 *
 * bsx_attn_plan_device_shape (host only) fixes what a graph needs to know at
 * capture time: the workgroup shape for query lengths up to max_qo_len, the grid,
 * the blob layout and the float workspace, all sized by bounds for `batch`
 * requests.  bsx_attn_plan_device (stream-ordered, no host synchronisation) then
 * writes the blob from qo_indptr_d[batch+1], kv_indptr_d[batch+1] and
 * kv_last_page_len_d[batch].  The device schedule cuts the kv tiles into equal
 * cost shares of the fixed grid (a tile costs 1, a segment start 2, as in
 * bsx_attn_plan).  Requirements checked on the device: indptrs non-decreasing from
 * 0, last-page lengths in [0, page_size], query lengths at most max_qo_len (32 in
 * tree mode), at least one page in the table and kv_indptr[batch] <= kv_indices_len
 * (when kv_indices_len >= 0); a violation writes an error code
 * (BSX_ERR_*) into blob[off_dyn + 1] and an empty schedule (no output is written),
 * otherwise 0.  A device plan's total_qo is the bound batch * max_qo_len: q and out
 * passed to bsx_attn_run need that many token rows. */
int bsx_attn_plan_device_shape(int batch, int num_qo_heads, int num_kv_heads, int head_dim,
                               int page_size, int mask_mode, int sink_tokens,
                               int window_tokens, float sm_scale, int num_cus, int max_qo_len,
                               bsx_attn_plan_t* plan_out);
int bsx_attn_plan_device(const bsx_attn_plan_t* plan, const int32_t* qo_indptr_d,
                         const int32_t* kv_indptr_d, const int32_t* kv_last_page_len_d,
                         int64_t kv_indices_len, int32_t* plan_blob_d, void* stream);

/* Replaces BatchPrefillWithPagedKVCacheWrapper.run(q, paged_kv_cache) as called
 * at batchspec/models/modules/attention/standard.py:69.
 *   q_d        [total_qo, num_qo_heads, head_dim] (bf16 or fp16), row stride
 *              q_stride_tok elements between tokens
 *   k_cache_d  K of page p, slot s, head h at
 *              k_cache_d + p*page_stride + s*num_kv_heads*head_dim + h*head_dim
 *   v_cache_d  same addressing (for the reference layout [P,2,ps,H,D],
 *              v_cache_d = k_cache_d + ps*H*D and page_stride = 2*ps*H*D)
 *   kv_indices_d page ids in CSR order (paged_kv_indices)
 *   mask_words_d uint32 per query token for BSX_MASK_TREE; the descriptor of
 *              bsx_custom_mask_prepare for BSX_MASK_CUSTOM; else NULL
 *   out_d      [total_qo, num_qo_heads, head_dim], same dtype as q
 *   lse_d      optional float [total_qo, num_qo_heads] log-sum-exp (natural
 *              log, of the scaled scores), or NULL
 *   plan_blob_d the device copy of the plan blob
 *   float_ws_d at least plan->float_ws_bytes bytes (partial results of split
 *              requests); runs that share one workspace must not overlap in time.
 * Two kernel launches when the plan splits requests (attention, then the merge of
 * the partial results), one otherwise. */
int bsx_attn_run(const bsx_attn_plan_t* plan, const int32_t* plan_blob_d,
                 void* float_ws_d, int dtype, const void* q_d, int64_t q_stride_tok,
                 const void* k_cache_d, const void* v_cache_d, int64_t page_stride,
                 const int32_t* kv_indices_d, const uint32_t* mask_words_d,
                 void* out_d, int64_t out_stride_tok, float* lse_d, void* stream);

/* The layer's KV update and its attention in one call: StandardKVCache.update(k, v,
 * kv_append_indptr = qo_indptr, page_table) (batchspec/models/modules/kv_cache.py:47-84,
 * called at batchspec/models/modules/attention/standard.py:63-66) followed by run(q,
 * kv_cache) (standard.py:69).  Arguments of bsx_attn_run, plus the appended rows
 * k_new_d / v_new_d [total_qo, num_kv_heads, head_dim] (token strides in elements):
 * token i of request b goes to position kv_len_b - qo_len_b + i of the cache, where the
 * plan's page table already counts it.  One launch: each workgroup whose tiles reach a
 * request's appended rows first writes them (for its kv heads) into the cache, then reads
 * them back with the other rows.  Outputs and cache contents equal bsx_kv_append followed
 * by bsx_attn_run; rows at negative positions (kv_len < qo_len) are skipped, as there. */
int bsx_attn_run_append(const bsx_attn_plan_t* plan, const int32_t* plan_blob_d,
                        void* float_ws_d, int dtype, const void* q_d, int64_t q_stride_tok,
                        const void* k_cache_d, const void* v_cache_d, int64_t page_stride,
                        const int32_t* kv_indices_d, const uint32_t* mask_words_d,
                        void* out_d, int64_t out_stride_tok, float* lse_d,
                        const void* k_new_d, int64_t k_new_stride_tok, const void* v_new_d,
                        int64_t v_new_stride_tok, void* stream);

/* plan(custom_mask=...) as the MTP engine calls it (batchspec/backends/mtp_engine.py:
 * 399-432: the flattened boolean mask, per request cat(ones(qo_len, cachelen),
 * common_attn_mask), qo_len x kv_len entries), packed on the device as FlashInfer's
 * plan() packs it.  mask_d: n_bools bytes (0 = hidden).  req_d [batch][4] int32 =
 * (qo_start, qo_len, kv_len, offset of the request's first entry in mask_d).  Writes
 *   desc_d       batch + ceil(n_bools / 32) + 1 uint32: the bit offsets, then the
 *                packed bits (little bit order) and a padding word: the mask_words_d
 *                of a BSX_MASK_CUSTOM run;
 *   general_d    [batch] int32: 0 when the request's mask has the tree form (every row
 *                sees its first kv_len - qo_len tokens, qo_len <= 32), 1 otherwise, 2
 *                when its entries do not lie inside the mask;
 *   tree_words_d [total_qo] uint32, for the requests of the tree form: the
 *                mask_words_d of a BSX_MASK_TREE run (bit c of token i = entry
 *                (i, kv_len - qo_len + c)).
 * A batch whose requests all have the tree form runs as BSX_MASK_TREE (the fast
 * path); otherwise as BSX_MASK_CUSTOM.  Two launches, no host synchronisation. */
int bsx_custom_mask_prepare(const void* mask_d, int64_t n_bools, const int32_t* req_d,
                            int batch, uint32_t* desc_d, uint32_t* tree_words_d,
                            int32_t* general_d, void* stream);

/* ------------------------------------------------------------------------- */
/* 2. Paged KV append                                                         */
/* ------------------------------------------------------------------------- */

/* FlashInfer get_seq_lens as used at batchspec/models/modules/kv_cache.py:66-70:
 * seq_lens[b] = (kv_indptr[b+1]-kv_indptr[b]-1)*page_size + last_page_len[b]
 * (0 when the request holds no page). */
int bsx_get_seq_lens(const int32_t* kv_indptr_d, const int32_t* kv_last_page_len_d,
                     int batch, int page_size, int32_t* seq_lens_d, void* stream);

/* FlashInfer get_batch_indices_positions as used at
 * batchspec/models/modules/kv_cache.py:64-72: for token i of request b,
 * batch_indices[i] = b, positions[i] = seq_lens[b] - n_b + (i - append_indptr[b]). */
int bsx_get_batch_indices_positions(const int32_t* append_indptr_d,
                                    const int32_t* seq_lens_d, int batch, int nnz,
                                    int32_t* batch_indices_d, int32_t* positions_d,
                                    void* stream);

/* FlashInfer append_paged_kv_cache (kv_layout NHD) as used at
 * batchspec/models/modules/kv_cache.py:73-83: cache[page(pos), slot(pos)] = k[i]. */
int bsx_append_paged_kv_cache(const void* append_key_d, const void* append_value_d,
                              int64_t key_stride_tok, int64_t value_stride_tok,
                              const int32_t* batch_indices_d, const int32_t* positions_d,
                              int nnz, void* k_cache_d, void* v_cache_d,
                              int64_t page_stride, const int32_t* kv_indices_d,
                              const int32_t* kv_indptr_d, int num_kv_heads, int head_dim,
                              int page_size, int elem_bytes, void* stream);

/* Fused StandardKVCache.update (batchspec/models/modules/kv_cache.py:47-84): the
 * three calls above in one kernel, without the host read of append_indptr[-1]
 * (kv_cache.py:71); nnz comes from the shape of k. */
int bsx_kv_append(const void* k_d, const void* v_d, int64_t k_stride_tok,
                  int64_t v_stride_tok, const int32_t* append_indptr_d,
                  const int32_t* kv_indptr_d, const int32_t* kv_indices_d,
                  const int32_t* kv_last_page_len_d, int batch, int nnz, void* k_cache_d,
                  void* v_cache_d, int64_t page_stride, int num_kv_heads, int head_dim,
                  int page_size, int elem_bytes, void* stream);

/* MTPEngine.collate_accepted_kv_cache (batchspec/backends/mtp_engine.py:577-631)
 * without the per-layer whole-cache copy: for every layer and request b the KV rows
 * of the accepted regular tokens, at positions prev_cachelens[b] + i*(draft_length+1)
 * for 1 <= i < accept_nums[b], move in place to positions prev_cachelens[b] + i,
 * addressed through the page table (no contiguous-page assumption).  The page-table
 * trim that follows (delete_kv, mtp_engine.py:630-631) stays on the host.
 *   accept_nums_d [B] int64 (clamped to [0, draft_length+1]); prev_cachelens_d [B]
 *   int32; k_bases_d / v_bases_d: device arrays of num_layers 16-byte aligned base
 *   addresses of each layer's K and V views (same page stride and shape for all
 *   layers).  Positions beyond a request's pages are skipped. */
int bsx_collate_accepted_kv(const int64_t* accept_nums_d, const int32_t* prev_cachelens_d,
                            int batch, int draft_length, const int32_t* kv_indptr_d,
                            const int32_t* kv_indices_d, const int64_t* k_bases_d,
                            const int64_t* v_bases_d, int num_layers, int64_t page_stride,
                            int num_kv_heads, int head_dim, int page_size, int elem_bytes,
                            void* stream);

/* ------------------------------------------------------------------------- */
/* 3. Acceptance                                                              */
/* ------------------------------------------------------------------------- */

/* Row argmax (torch.argmax: first maximum, NaN counts as maximum) over
 * [rows, vocab] logits, as used by `target_logits.argmax(-1)` at
 * batchspec/backends/mtp_engine.py:747 and greedy `sample` at
 * batchspec/backends/utils/sampling.py:89-90.  ws_d: bsx_argmax_ws_bytes. */
int64_t bsx_argmax_ws_bytes(int64_t rows, int64_t vocab);
int bsx_argmax(const void* logits_d, int dtype, int64_t rows, int64_t vocab,
               int64_t row_stride, int64_t* out_d, void* ws_d, int64_t ws_bytes,
               void* stream);

/* Greedy branch of MTPEngine.evaluate_posterior
 * (batchspec/backends/mtp_engine.py:553-560).
 *   draft_d [B,k] int64; target ids: target_ids_d [B,k+1] int64, or (when
 *   target_ids_d is NULL) target_logits_d [B,k+1,V] whose argmax is fused.
 *   mode 0 = reference rule accept = (#matches)+1 (mtp_engine.py:556);
 *   mode 1 = longest-prefix rule.
 *   Outputs: bonus_d [B] int64, accept_d [B] int64, eos_acc_d [B] uint8. */
int64_t bsx_accept_greedy_ws_bytes(int B, int k, int64_t vocab);
int bsx_accept_greedy(const int64_t* draft_d, const int64_t* target_ids_d,
                      const void* target_logits_d, int dtype, int B, int k,
                      int64_t vocab, int64_t eos_id, int mode, int64_t* bonus_d,
                      int64_t* accept_d, uint8_t* eos_acc_d, void* ws_d,
                      int64_t ws_bytes, void* stream);

/* Allocation-free greedy acceptance: no counterpart in the reference.  For callers
 * that cannot allocate or pass a workspace (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results as
 * bsx_accept_greedy without ws_d / ws_bytes: the argmax partials go to a file-scope
 * device array of BSX_NOALLOC_SCRATCH_BYTES bytes per GPU, held until the process
 * ends.  Shapes whose partials exceed it (bsx_accept_greedy_ws_bytes(B, k, vocab) >
 * BSX_NOALLOC_SCRATCH_BYTES; at vocab 128256 in bf16 that is B*(k+1) > 32768 rows)
 * return BSX_ERR_CAPACITY.  The library allocates nothing here.  Every call on a GPU
 * shares that GPU's array: calls that overlap in time on one GPU race. */
#define BSX_NOALLOC_SCRATCH_BYTES (4 << 20)
int bsx_accept_greedy_noalloc(const int64_t* draft_d, const int64_t* target_ids_d,
                              const void* target_logits_d, int dtype, int B, int k,
                              int64_t vocab, int64_t eos_id, int mode, int64_t* bonus_d,
                              int64_t* accept_d, uint8_t* eos_acc_d, void* stream);

/* Chain speculative sampling (flashinfer.sampling.chain_speculative_sampling as
 * called at batchspec/backends/mtp_engine.py:569) with explicit uniforms.
 *   draft_probs_d [B,k,V] fp32 or NULL (NULL = one-hot at the draft token, the
 *   MTP case of mtp_engine.py:565-567); target_probs_d [B,k+1,V] fp32;
 *   draft_ids_d [B,k] int64; uniforms_d [B,k+1] fp32 in [0,1): u[:, i<k] for the
 *   ratio tests, u[:, k] for the residual / bonus draw.
 *   Outputs: out_ids_d [B,k+1] int32 (-1 padded), accepted_d [B] int32 (draft
 *   tokens accepted when each position is tested on its own), emitted_d [B] int32
 *   (length of the accepted prefix). */
int64_t bsx_chain_ws_bytes(int B, int k, int64_t vocab);
int bsx_chain_speculative_sampling(const float* draft_probs_d, const int64_t* draft_ids_d,
                                   const float* target_probs_d, const float* uniforms_d,
                                   int B, int k, int64_t vocab, int32_t* out_ids_d,
                                   int32_t* accepted_d, int32_t* emitted_d, void* ws_d,
                                   int64_t ws_bytes, void* stream);

/* Same test fused with the temperature softmax of both distributions
 * (get_sampling_probs, batchspec/backends/utils/sampling.py:47-48, with top-k
 * and top-p off): reads bf16/fp16/fp32 logits once instead of fp32 probs.
 *   draft_logits_d [B,k,V] or NULL (one-hot draft); target_logits_d [B,k+1,V]. */
int bsx_chain_speculative_sampling_logits(const void* draft_logits_d,
                                          const int64_t* draft_ids_d,
                                          const void* target_logits_d, int dtype,
                                          float temperature, const float* uniforms_d,
                                          int B, int k, int64_t vocab, int32_t* out_ids_d,
                                          int32_t* accepted_d, int32_t* emitted_d,
                                          void* ws_d, int64_t ws_bytes, void* stream);

/* flashinfer.sampling.softmax(logits, temperature) as called at
 * batchspec/backends/utils/sampling.py:48, with the deterministic reduction
 * order shared with the fused acceptance kernels. probs_d [rows, vocab] fp32. */
int64_t bsx_softmax_ws_bytes(int64_t rows);
int bsx_softmax(const void* logits_d, int dtype, float temperature, int64_t rows,
                int64_t vocab, float* probs_d, void* ws_d, int64_t ws_bytes,
                void* stream);

/* Sync-free page-table update: PageTable.insert_kv (sign +1) / delete_kv (sign -1)
 * (batchspec/backends/base/page_table.py:55-137) with PageManager.allocate / free
 * (batchspec/backends/utils/paging.py:155-277), in one kernel on fixed-size buffers.
 *   num_pages_d, last_len_d, cachelens_d (or NULL) [B] int32: updated in place;
 *   d_d [B] int32 lengths, or NULL to use d_scalar for every request;
 *   indptr_d [B+1], indices_d [B*max_pages]: the rebuilt CSR (page k of request r is
 *   r*max_pages + k, the reference allocator's ids).
 * No update happens when no length is positive (the reference returns early), or when
 * an insert would exceed max_pages for some request: then *errors_d (if given) is
 * incremented, where the reference raises RuntimeError. */
int bsx_page_table_update(int32_t* num_pages_d, int32_t* last_len_d, int32_t* cachelens_d,
                          const int32_t* d_d, int32_t d_scalar, int sign, int B,
                          int page_size, int max_pages, int32_t* indptr_d,
                          int32_t* indices_d, int32_t* errors_d, void* stream);

/* Greedy acceptance fused with the delete of the rejected tokens that follows it in the
 * verify step: MTPEngine.evaluate_posterior's greedy branch
 * (batchspec/backends/mtp_engine.py:553-560) and then PageTable.delete_kv(n_inserted -
 * accept_nums) (batchspec/backends/base/page_table.py:95-137).  The arguments of
 * bsx_accept_greedy (ids, or logits with the fused argmax and its workspace), then
 * those of bsx_page_table_update for a delete of n_inserted - accept_b tokens per
 * request (n_inserted >= k + 1: the tokens the step inserted).  One argmax launch (when
 * given logits) plus one kernel that evaluates every request and updates the table;
 * outputs and table state equal bsx_accept_greedy followed by bsx_page_table_update.
 * At most 8192 requests. */
int bsx_accept_greedy_delete(const int64_t* draft_d, const int64_t* target_ids_d,
                             const void* target_logits_d, int dtype, int B, int k,
                             int64_t vocab, int64_t eos_id, int mode, int64_t* bonus_d,
                             int64_t* accept_d, uint8_t* eos_acc_d, void* ws_d,
                             int64_t ws_bytes, int32_t n_inserted, int32_t* num_pages_d,
                             int32_t* last_len_d, int32_t* cachelens_d, int page_size,
                             int max_pages, int32_t* indptr_d, int32_t* indices_d,
                             void* stream);

/* Draft-tree masks on the device: replaces the MTP mask and position ids of
 * MTPEngine._setup_common_attn_mask_and_position_ids (batchspec/backends/mtp_engine.py:
 * 172-208) and the per-request ones/mask concatenation before plan() (:410-417), and
 * the EAGLE tree masks, from parent arrays.
 *   parents_d [B, parents_stride] int32 (parents_stride 0: one array [n] shared by
 *   every request); parent[i] < i, -1 for a node hanging off the cached prefix (a
 *   parent >= i or < -1 ends the chain there).  n <= 32.
 *   Outputs: words_d [B*n] uint32, bit j = token j is the token or an ancestor (the
 *   attention plan's tree_mask_words); positions_d [B*n] int64 (or NULL) =
 *   cachelens_d[b] (0 if NULL) + depth. */
int bsx_tree_masks(const int32_t* parents_d, int64_t parents_stride, int n,
                   const int32_t* cachelens_d, int B, uint32_t* words_d,
                   int64_t* positions_d, void* stream);

/* Top-k / top-p renormalisation (batchspec/backends/utils/sampling.py:50-56: top-p on
 * the full softmax(logits/T), then top-k on the renormalised distribution; top-k is on
 * iff 0 < top_k < vocab, top-p iff 0 < top_p < 1) fused into the stochastic acceptance
 * (mtp_engine.py:561-575 with get_sampling_probs(target_preds, top_p, top_k, T) at
 * :564).  The kept set is every value at or above a threshold (ties kept); threshold
 * masses and draws use 2^-40 fixed point, so the ids are bit-identical to the CPU
 * restatement given the same uniforms.  draft_logits_d (or NULL: one-hot draft) is
 * filtered the same way.  With both filters off this is
 * bsx_chain_speculative_sampling_logits.  ws_d: bsx_chain_filtered_ws_bytes. */
int64_t bsx_filter_ws_bytes(int64_t rows);
int64_t bsx_chain_filtered_ws_bytes(int B, int k, int64_t vocab);
int bsx_chain_speculative_sampling_filtered(const void* draft_logits_d,
                                            const int64_t* draft_ids_d,
                                            const void* target_logits_d, int dtype,
                                            float temperature, int top_k, float top_p,
                                            const float* uniforms_d, int B, int k,
                                            int64_t vocab, int32_t* out_ids_d,
                                            int32_t* accepted_d, int32_t* emitted_d,
                                            void* ws_d, int64_t ws_bytes, void* stream);

/* get_sampling_probs (batchspec/backends/utils/sampling.py:18-58): fp32 probabilities
 * [rows, vocab] of softmax(logits/T) after the top-p and top-k renormalisation above
 * (bsx_softmax when both are off).  ws_d: bsx_sampling_probs_ws_bytes. */
int64_t bsx_sampling_probs_ws_bytes(int64_t rows);
int bsx_sampling_probs(const void* logits_d, int dtype, float temperature, int top_k,
                       float top_p, int64_t rows, int64_t vocab, float* probs_d, void* ws_d,
                       int64_t ws_bytes, void* stream);

/* sample() (batchspec/backends/utils/sampling.py:61-115) for temperature > 0: one id
 * per row of [rows, vocab] logits drawn from the filtered distribution with
 * uniforms_d[row] (int32 ids, as FlashInfer's samplers return before the reference's
 * .long() at :114).  Temperature 0 is bsx_argmax.  ws_d: bsx_sample_ws_bytes. */
int64_t bsx_sample_ws_bytes(int64_t rows, int64_t vocab);
int bsx_sample(const void* logits_d, int dtype, float temperature, int top_k, float top_p,
               const float* uniforms_d, int64_t rows, int64_t vocab, int32_t* out_d,
               void* ws_d, int64_t ws_bytes, void* stream);

/* Streaming-read probe, a measurement kernel with no counterpart in the reference: reads
 * `bytes` (a multiple of 16) from src_d once with non-temporal 16-byte loads, every load
 * of a thread issued together, `threads` per workgroup and `loads_per_thread` loads per
 * thread (1..32, powers of two); writes nothing but (rarely) a word of sink_d [1].  Its
 * time is the floor of a kernel that reads the same bytes once. */
int bsx_read_probe(const void* src_d, int64_t bytes, int threads, int loads_per_thread,
                   uint32_t* sink_d, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* BSX_H */
