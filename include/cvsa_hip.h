/*
 * cvsa_hip.h - C ABI of libcvsa_hip.so, the MI355X (gfx950) implementation of
 * the CVSA decode-step attention path.
 *
 * Conventions shared by every entry point:
 *  - Pointers are device pointers unless stated otherwise.  bf16 tensors are
 *    passed as uint16_t (raw bfloat16 bits).
 *  - The paged cache layout is the reference's: k_cache / v_cache are
 *    [num_blocks, block_size, H_kv, D] bf16, fully contiguous
 *    (cvsa/runtime/kv_cache.py:40-47).  block_tables are [B, >=W] int32 with
 *    unit stride along pages; context_lens are [B] int32.  Buffer lengths
 *    are not passed: every per-sequence or per-(sequence, KV head) buffer
 *    must cover the call's whole batch (B rows, or B * H_kv), or the kernels
 *    read or write past its end; the caller checks this before the call.
 *  - `stream` is a hipStream_t (NULL = default stream).  Kernels are only
 *    enqueued; no entry point synchronises the host.
 *  - The library allocates no device memory.  Outputs and workspaces belong
 *    to the caller; a step plan (below) is a small host object.
 *  - Return value: CVSA_OK (0), or a negative CVSA_ERR_* code with nothing
 *    enqueued.  cvsa_last_error() then returns a thread-local message.
 *  - Supported geometry: D in {32, 64, 128, 256}, block_size in {8, 16, 32, 64,
 *    128},
 *    G = H_q / H_kv in 1..128 (decode launches serve 16 query heads per KV
 *    head; larger groups are enqueued as one launch per 16),
 *    any H_kv (B * H_kv <= 65535), W <= 262144 pages (top-p budgets:
 *    W <= 32768), and B * H_kv <= 4096 for dense and verified decode.
 *    Anything else returns CVSA_ERR_UNSUPPORTED.
 *  - Entry points are re-entrant.  Calls that share a decode workspace must
 *    be ordered on one stream.
 */
#ifndef CVSA_HIP_H
#define CVSA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CVSA_ABI_VERSION 14

enum {
  CVSA_OK = 0,
  CVSA_ERR_INVALID = -1,     /* bad pointer, shape, stride or alignment */
  CVSA_ERR_UNSUPPORTED = -2, /* geometry outside the supported set */
  CVSA_ERR_LAUNCH = -3,      /* the HIP runtime refused the launch */
  CVSA_ERR_WORKSPACE = -4    /* workspace missing or too small */
};

enum { CVSA_DTYPE_BF16 = 0, CVSA_DTYPE_FP16 = 1, CVSA_DTYPE_FP32 = 2 };

/* Thread-local description of the last failure on this thread. */
const char *cvsa_last_error(void);
int cvsa_abi_version(void);

/*
 * Page scoring.  Replaces triton_score_pages
 * (cvsa/kernels/page_scores.py:77-119, kernel :12-74).
 *   q_rep[b,h] = bf16(sum_g q[b, h*G+g] * (1/G))          (fp32 sum, RNE)
 *   page_scores[b,h,p] = max_{t < tokens(p)} fp32(q_rep . K[bt[b,p], t, h]) * D^-0.5
 *   page_scores[b,h,p] = -inf when p*block_size >= context_lens[b].
 * q: [B, H_q, D] bf16 with element strides (q_stride_b, q_stride_h, 1).
 * page_scores: [B, H_kv, W] fp32, contiguous.
 */
int cvsa_score_pages(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                     const uint16_t *k_cache, int64_t num_blocks,
                     const int32_t *block_tables, int64_t bt_stride_b,
                     const int32_t *context_lens, int32_t B, int32_t H_q,
                     int32_t H_kv, int32_t D, int32_t block_size, int32_t W,
                     float *page_scores, void *stream);

/*
 * Top-k page selection.  Replaces the uniform-budget branch of
 * CVSABackend._scoring_step (cvsa/backend.py:737-747: torch.topk(sorted=False)
 * then n_per_head = min(budget, n_valid)).
 *   page_indices[b,h,:budget] = the `budget` largest scores of row (b,h),
 *     ties broken by lower page index, written in ascending page order.
 *   n_per_head[b,h] = min(budget, n_valid(b)), n_valid = (ctx-1)/bs + 1.
 * When accept_out and coverage_out are non-NULL the coverage gate of the new
 * selection is fused in, with the semantics of cvsa_check_coverage
 * (cvsa/backend.py:757-761).
 */
int cvsa_select_topk(const float *page_scores, int32_t B, int32_t H_kv,
                     int32_t W, const int32_t *context_lens,
                     int32_t block_size, int32_t budget, int32_t *page_indices,
                     int32_t *n_per_head, float tau, uint8_t *accept_out,
                     float *coverage_out, void *stream);

/*
 * The lazy coverage decision taken on the device.  Replaces the branch of
 * CVSABackend._lazy_step (cvsa/backend.py:420-465) that reads the accept
 * mask of the cached selection on the host and then either reuses that
 * selection or runs a scoring step (backend.py:737-771).
 *   check_accept[B*H_kv]: coverage gate of the cached selection (the
 *     accept_out of cvsa_check_coverage); must not alias accept_out.
 *   all heads passed -> page_indices / n_per_head / coverage_out untouched,
 *     accept_out[:] = 1.
 *   otherwise        -> as cvsa_select_topk with the fused gate, writing
 *     the new selection over page_indices / n_per_head in place, and
 *     scores_cache (optional, [B,H_kv,W]) receives a copy of page_scores.
 *   stats (optional, int64[6], accumulated; [4], [5] are scratch that must
 *     start at zero and are left at zero): [0] += all passed, [1] += some
 *     head failed, [2] += scoring steps run (same as [1]), [3] += number
 *     of heads that passed.
 *   check_accept == NULL: a fresh selection (no cached one).  With
 *     count_gate == 0 the stats book a lazy scoring step without a cached
 *     selection ([1] += 1, [2] += 1); with count_gate != 0 they book a
 *     fixed-interval scoring step by the new selection's gate
 *     (backend.py:859-863: [2] += 1, [3] += heads accepted, [0] or [1] += 1
 *     by whether every head accepted).
 *   sel_scores (optional, [B,H_kv,W]): scores the new selection ranks while
 *     page_scores drive its coverage gate and scores_cache (the Quest
 *     selector with the exact gate, backend.py:723-727); NULL = page_scores.
 */
int cvsa_select_or_keep(const float *page_scores, const float *sel_scores,
                        const uint8_t *check_accept,
                        int32_t B, int32_t H_kv, int32_t W,
                        const int32_t *context_lens, int32_t block_size,
                        int32_t budget, int32_t *page_indices,
                        int32_t *n_per_head, float tau, uint8_t *accept_out,
                        float *coverage_out, float *scores_cache,
                        int64_t *stats, int32_t count_gate, void *stream);

/*
 * cvsa_select_or_keep with a budget per (b, kv-head) row: the lazy check
 * (and the fixed-interval scoring step's booking) of the static-table
 * branch of CVSABackend (_static_select, cvsa/backend.py:622-650, whose
 * budgets the host knows), or of any per-row budgets computed beforehand,
 * taken on the device.  The keep decision, counters, scores_cache and
 * sel_scores are those of cvsa_select_or_keep; a new selection is that of
 * cvsa_select_budgeted with these row_budgets ([B*H_kv] int32, each
 * clamped to [1, W]) and rows of `width` entries (the row stride of
 * page_indices; a budget above it is clamped to it), with its coverage
 * gate.  No counterpart of its own in the reference, whose lazy step reads
 * the accept mask on the host (backend.py:440-446).
 */
int cvsa_select_or_keep_budgeted(const float *page_scores, const float *sel_scores,
                                 const uint8_t *check_accept, int32_t B, int32_t H_kv,
                                 int32_t W, const int32_t *context_lens, int32_t block_size,
                                 const int32_t *row_budgets, int32_t width,
                                 int32_t *page_indices, int32_t *n_per_head, float tau,
                                 uint8_t *accept_out, float *coverage_out,
                                 float *scores_cache, int64_t *stats, int32_t count_gate,
                                 void *stream);

/*
 * Selection with a budget per (b, kv-head) row.  Replaces the top-p branch
 * of CVSABackend._scoring_step (_topp_select, cvsa/backend.py:652-681), the
 * static-table branch (_static_select, :622-650) and the selection of the
 * adaptive branch (_adaptive_select, :522-570, budgets from
 * cvsa_adaptive_budgets).
 *   top_p in (0, 1), row_budgets NULL: with p = softmax(sel row),
 *     need = 1 + #{k : sum of the k largest p < top_p}, k_row =
 *     clamp(need, 3, W).  The masses exp(s - max) are summed exactly as
 *     40-bit fixed point, in descending score order; the reference's fp32
 *     cumsum can put need one page off where the cumulative mass lies
 *     within rounding of top_p.  A row with +inf / NaN or no finite score
 *     (NaN softmax in the reference) gets need = 1.
 *   row_budgets [B*H_kv] int32 (top_p = 0): k_row = row_budgets[b*H_kv+h]
 *     (clamped to [1, W]; the static table's clamp(round(frac*P), 3, P) is
 *     applied by the caller).
 *   k_row is then clamped to `width`, the row stride of page_indices: the
 *     row's first k_row entries receive the pages of its k_row largest
 *     ranking scores (ties to the lower page) in ascending page order;
 *     entries past k_row are left unwritten.  width = W never clamps.
 *   n_per_head[b,h] = min(k_row, n_valid(b)).
 *   sel_scores (optional): the ranking scores (the Quest selector); NULL =
 *     page_scores.  accept_out / coverage_out (optional): the coverage
 *     gate of the new selection on page_scores, as cvsa_select_topk.
 */
int cvsa_select_budgeted(const float *page_scores, const float *sel_scores,
                         int32_t B, int32_t H_kv, int32_t W,
                         const int32_t *context_lens, int32_t block_size,
                         float top_p, const int32_t *row_budgets, int32_t width,
                         int32_t *page_indices, int32_t *n_per_head, float tau,
                         uint8_t *accept_out, float *coverage_out, void *stream);

/*
 * Per-head budgets of CVSABackend._adaptive_select (cvsa/backend.py:
 * 522-570): the kv-heads of each sequence compete for H_kv * base_budget
 * slots among all their page scores; raw[b,h] = head h's share of the
 * H_kv * base_budget largest scores of sequence b (ties at the last value
 * to the lower heads; the reference's torch.topk leaves them unspecified);
 * budgets[b*H_kv+h] = clamp(round(fp32(raw) * fp32(1 - floor_ratio) +
 * fp32(base_budget * floor_ratio)), 1, n_valid(b)), round half to even.
 * The selection itself is cvsa_select_budgeted with these row budgets.
 * H_kv <= 64.
 */
int cvsa_adaptive_budgets(const float *page_scores, int32_t B, int32_t H_kv, int32_t W,
                          const int32_t *context_lens, int32_t block_size,
                          int32_t base_budget, double floor_ratio, int32_t *budgets,
                          void *stream);

/*
 * Coverage gate.  Replaces triton_check_coverage
 * (cvsa/kernels/coverage.py:218-265, kernel :159-215).
 *   lse_all = M + log(sum exp(s - M) + 1e-30), M = max(max_p s, -1e20)
 *   lse_sel = same over the first n_per_head[b,h] selected pages
 *   coverage = exp(lse_sel - lse_all);  accept = coverage >= tau  (fp32)
 * selected: rows of `sel_stride` int32 per (b,h).
 */
int cvsa_check_coverage(const float *page_scores, int32_t B, int32_t H_kv,
                        int32_t W, const int32_t *selected, int64_t sel_stride,
                        const int32_t *n_per_head, float tau,
                        uint8_t *accept_out, float *coverage_out, void *stream);

/*
 * Workspace of the paged decode entry points, in bytes, for a call whose
 * heads visit at most `max_sel_pages` listed pages and, when `all_pages` is
 * non-zero, up to W pages (dense heads).  It holds per-head completion
 * counters and the split-K partial softmax states.  A workspace must be
 * zeroed once (cvsa_workspace_init) before its first use; every decode call
 * leaves its counters at zero again.  May be 0 bytes (then NULL is
 * accepted).
 */
size_t cvsa_decode_workspace_bytes(int32_t B, int32_t H_q, int32_t H_kv,
                                   int32_t D, int32_t max_sel_pages,
                                   int32_t W, int32_t all_pages);

/* Zero a workspace on `stream` with a fill kernel (once, before first use). */
int cvsa_workspace_init(void *workspace, size_t workspace_bytes, void *stream);

/*
 * Sparse paged decode over a per-KV-head page list.  Replaces
 * triton_sparse_decode_unnorm (cvsa/kernels/sparse_decode.py:537-573) when
 * the (o_unnorm, m_out, l_out) outputs are given, and triton_sparse_decode /
 * triton_sparse_decode_reuse (:286-350, :681-721) when `out` is given.
 * Either or both output forms may be requested.
 *   For q-head j of batch b (KV head h = j / G), over the first
 *   n_per_head[b*H_kv+h] entries of page_indices row (b,h) and the tokens
 *   t < min(bs, ctx - page*bs) of each:
 *     s = (q . K) * D^-0.5,  m = max s,  l = sum exp(s - m),
 *     o_unnorm = sum exp(s - m) * V,   out = o_unnorm / max(l, 1e-6).
 *   A head with no pages yields m = -inf, l = 0, o = 0 (out = 0).
 * page_indices: rows of idx_stride int32 per (b,h); max_selected bounds
 * n_per_head.  o_unnorm [B,H_q,D] fp32; m_out, l_out [B,H_q] fp32;
 * out [B,H_q,D] of out_dtype; out and o_unnorm contiguous, 16-byte aligned.
 * work (optional, int64[2]): the effective-budget counters of
 * CVSABackend._record_work (cvsa/backend.py:368-390); each head adds the
 * pages it attended to work[0] and n_valid(b) to work[1].
 */
int cvsa_sparse_decode(const uint16_t *q, int64_t q_stride_b,
                       int64_t q_stride_h, const uint16_t *k_cache,
                       const uint16_t *v_cache, int64_t num_blocks,
                       const int32_t *block_tables, int64_t bt_stride_b,
                       const int32_t *context_lens,
                       const int32_t *page_indices, int64_t idx_stride,
                       const int32_t *n_per_head, int32_t max_selected,
                       int32_t B, int32_t H_q, int32_t H_kv, int32_t D,
                       int32_t block_size, int32_t W, float *o_unnorm,
                       float *m_out, float *l_out, void *out,
                       int32_t out_dtype, int64_t *work, void *workspace,
                       size_t workspace_bytes, void *stream);

/*
 * cvsa_sparse_decode without a workspace argument: allocates nothing and
 * needs no caller-owned scratch.  No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The split-K
 * counters and partials live in a static 4.5 MiB device array of the
 * library (one per GPU, held until the process ends; every listed launch
 * needs at most 4.3 MB of it, at G = 16 and D = 256, and 1.1 MB at G = 8,
 * D = 128; a larger need returns CVSA_ERR_WORKSPACE).  Its first
 * call on a device looks the array up and zeroes its counters on `stream`.
 * All calls on one GPU share the array: calls that overlap in time on one
 * GPU (other streams, other threads) race and must be ordered by the
 * caller.  Arguments, outputs and errors as cvsa_sparse_decode.
 */
int cvsa_sparse_decode_noalloc(const uint16_t *q, int64_t q_stride_b,
                               int64_t q_stride_h, const uint16_t *k_cache,
                               const uint16_t *v_cache, int64_t num_blocks,
                               const int32_t *block_tables,
                               int64_t bt_stride_b,
                               const int32_t *context_lens,
                               const int32_t *page_indices,
                               int64_t idx_stride,
                               const int32_t *n_per_head,
                               int32_t max_selected, int32_t B, int32_t H_q,
                               int32_t H_kv, int32_t D, int32_t block_size,
                               int32_t W, float *o_unnorm, float *m_out,
                               float *l_out, void *out, int32_t out_dtype,
                               int64_t *work, void *stream);

/*
 * cvsa_sparse_decode with the step's token append folded in: for every
 * sequence b < B, the append of cvsa_append_kv (one token: rows b of
 * k_new / v_new, [H_kv, D] bf16, new_stride_b elements apart), then the
 * listed decode of cvsa_sparse_decode over the appended cache, as one launch
 * for 16-token pages, D = 128, H_q / H_kv <= 16 and B <= 256 (otherwise the
 * two entry points in order, with the same results).  No counterpart in the
 * reference, whose decode loops append (SequenceKVManager.append_token_kv,
 * cvsa/runtime/kv_cache.py:133-150) and then call the backend: it is for
 * decode drivers whose reuse steps would otherwise pay a second launch per
 * layer for the append.  The attention is that of the append followed by
 * cvsa_sparse_decode, bit for bit.
 * slots: HOST array of 2 * B int32 from the caller's mirror of the
 * allocation state: slots[2b] = context_lens[b] before the append,
 * slots[2b + 1] = the block the append allocates for b (its page
 * slots[2b] / block_size is new: slots[2b] % block_size == 0 and not yet
 * allocated; the r-th such sequence in increasing b takes next_free + r), or
 * -1.  Inconsistent slots return CVSA_ERR_INVALID before anything is
 * enqueued.  slots_dev: the same 2 * B int32 in device memory instead, for a
 * launch that a captured graph replays (the slots change every step, the
 * kernel arguments of a captured launch do not); only the one-launch shapes
 * take them (CVSA_ERR_UNSUPPORTED otherwise).  The launch checks each device
 * slot: a sequence whose slot is out of range (context length outside
 * [0, 16 W), a new block outside [-1, num_blocks) or not at a page start)
 * appends nothing, its output is undefined, and *slot_errors (an optional
 * device int32, accumulated) is incremented once for it.
 * Exactly one of slots and slots_dev is given.  block_tables, context_lens
 * and pages_allocated are updated as cvsa_append_kv does; the other
 * arguments, outputs and errors are those of cvsa_sparse_decode (normalised
 * output only).
 */
int cvsa_sparse_decode_append(const uint16_t *q, int64_t q_stride_b,
                              int64_t q_stride_h, uint16_t *k_cache,
                              uint16_t *v_cache, int64_t num_blocks,
                              int32_t *block_tables, int64_t bt_stride_b,
                              int32_t *context_lens,
                              const int32_t *page_indices, int64_t idx_stride,
                              const int32_t *n_per_head, int32_t max_selected,
                              int32_t B, int32_t H_q, int32_t H_kv, int32_t D,
                              int32_t block_size, int32_t W, void *out,
                              int32_t out_dtype, int64_t *work, void *workspace,
                              size_t workspace_bytes, const uint16_t *k_new,
                              const uint16_t *v_new, int64_t new_stride_b,
                              int32_t *pages_allocated, const int32_t *slots,
                              const int32_t *slots_dev, int32_t *slot_errors,
                              void *stream);

/*
 * Dense paged decode over every valid page.  Replaces
 * DenseAttentionBackend._triton_dense (cvsa/runtime/dense.py:40-68), i.e.
 * the sparse kernel with all pages selected.  Outputs as cvsa_sparse_decode.
 */
int cvsa_dense_decode(const uint16_t *q, int64_t q_stride_b,
                      int64_t q_stride_h, const uint16_t *k_cache,
                      const uint16_t *v_cache, int64_t num_blocks,
                      const int32_t *block_tables, int64_t bt_stride_b,
                      const int32_t *context_lens, int32_t B, int32_t H_q,
                      int32_t H_kv, int32_t D, int32_t block_size, int32_t W,
                      float *o_unnorm, float *m_out, float *l_out, void *out,
                      int32_t out_dtype, int64_t *work, void *workspace,
                      size_t workspace_bytes, void *stream);

/*
 * Verified decode: the draft/recovery branch of a scoring step in one pass.
 * Replaces cvsa/backend.py:775-779 (accept-all: o_d / l_d) and the exact
 * recovery branch :818-844 (triton_compute_complement, complement decode,
 * triton_lse_merge).  Heads with accept[b*H_kv+h] != 0 attend their selected
 * pages (the draft); rejected heads attend draft + complement = every valid
 * page in one pass, which is the LSE merge of the two partial softmaxes.
 * Outputs as cvsa_sparse_decode.
 */
int cvsa_verified_decode(const uint16_t *q, int64_t q_stride_b,
                         int64_t q_stride_h, const uint16_t *k_cache,
                         const uint16_t *v_cache, int64_t num_blocks,
                         const int32_t *block_tables, int64_t bt_stride_b,
                         const int32_t *context_lens,
                         const int32_t *page_indices, int64_t idx_stride,
                         const int32_t *n_per_head, int32_t max_selected,
                         const uint8_t *accept, int32_t B, int32_t H_q,
                         int32_t H_kv, int32_t D, int32_t block_size,
                         int32_t W, float *o_unnorm, float *m_out,
                         float *l_out, void *out, int32_t out_dtype,
                         int64_t *work, void *workspace,
                         size_t workspace_bytes, void *stream);

/*
 * Verified decode with approximate recovery: the draft/recovery branch of a
 * scoring step when CVSABackend.approx_recovery_pct is set.  Replaces
 * cvsa/backend.py:775-779 (accept-all: o_d / l_d) and :780-817 (expanded
 * top-k, its sparse decode, and the per-head select between the normalised
 * draft and the normalised expanded decode).  Accepted heads
 * (accept[b*H_kv+h] != 0) attend their selected pages; rejected heads attend
 * the first min(exp_budget, n_valid) pages of exp_indices[b,h,:] (the
 * exp_budget largest ranking scores, e.g. cvsa_select_topk with budget
 * exp_budget).  Effective-budget counters as the reference books them: when
 * some head is rejected every head adds n_per_head + min(exp_budget,
 * n_valid), else n_per_head.  exp_budget in [1, W], exp_stride >= exp_budget.
 * Outputs as cvsa_sparse_decode.
 */
int cvsa_verified_decode_approx(const uint16_t *q, int64_t q_stride_b,
                                int64_t q_stride_h, const uint16_t *k_cache,
                                const uint16_t *v_cache, int64_t num_blocks,
                                const int32_t *block_tables, int64_t bt_stride_b,
                                const int32_t *context_lens,
                                const int32_t *page_indices, int64_t idx_stride,
                                const int32_t *n_per_head, int32_t max_selected,
                                const uint8_t *accept, const int32_t *exp_indices,
                                int64_t exp_stride, int32_t exp_budget, int32_t B,
                                int32_t H_q, int32_t H_kv, int32_t D, int32_t block_size,
                                int32_t W, float *o_unnorm, float *m_out,
                                float *l_out, void *out, int32_t out_dtype,
                                int64_t *work, void *workspace,
                                size_t workspace_bytes, void *stream);

/*
 * Complement page lists.  Replaces triton_compute_complement
 * (cvsa/kernels/coverage.py:99-150, kernel :30-96).
 *   comp_indices[b,h,:] = ascending valid pages p < n_valid(b) that are not
 *   among the first n_per_head[b,h] selected pages, zero-filled to `width`;
 *   n_comp[b,h] = their count, 0 for heads with accept[b,h] != 0.
 * accept may be NULL (no head accepted).  width must be >= max_b n_valid(b).
 */
int cvsa_compute_complement(const int32_t *page_indices, int64_t idx_stride,
                            const int32_t *n_per_head,
                            const int32_t *context_lens, int32_t block_size,
                            const uint8_t *accept, int32_t B, int32_t H_kv,
                            int32_t width, int32_t *comp_indices,
                            int32_t *n_comp, void *stream);

/*
 * Selective LSE merge.  Replaces triton_lse_merge
 * (cvsa/kernels/coverage.py:329-367, kernel :273-326)
 * and selective_lse_merge (cvsa/lse_merge.py:11-54).
 *   accepted kv head: out = o_d / max(l_d, 1e-6)
 *   rejected: m = max(m_d, m_c), a = exp(m_d - m), c = exp(m_c - m),
 *             out = (o_d a + o_c c) / max(l_d a + l_c c, 1e-6)
 * o_*: [B,H_q,D] fp32; m_*, l_*: [B,H_q] fp32; accept [B,H_kv] uint8.
 */
int cvsa_lse_merge(const float *o_d, const float *m_d, const float *l_d,
                   const float *o_c, const float *m_c, const float *l_c,
                   const uint8_t *accept, int32_t B, int32_t H_q, int32_t H_kv,
                   int32_t D, void *out, int32_t out_dtype, void *stream);

/*
 * Batched token append.  Replaces SequenceKVManager.append_token_kv
 * (cvsa/runtime/kv_cache.py:133-150) for sequences
 * [seq_begin, seq_begin + n_seqs) in one launch, without host syncs:
 *   page = ctx / bs, off = ctx % bs;
 *   if off == 0 and page >= pages_allocated[b]: the r-th such sequence (in
 *     increasing b) gets block next_free_block + r, block_tables[b,page] is
 *     set to it and pages_allocated[b] += 1;
 *   K/V[block_tables[b,page], off] = k_new/v_new row;  context_lens[b] += 1.
 * k_new/v_new: n_seqs rows of [H_kv, D] bf16, new_stride_b elements apart.
 * The caller tracks how many blocks were taken (the host mirror of
 * context_lens / pages_allocated) and must ensure they exist.
 */
int cvsa_append_kv(const uint16_t *k_new, const uint16_t *v_new,
                   int64_t new_stride_b, uint16_t *k_cache, uint16_t *v_cache,
                   int64_t num_blocks, int32_t *block_tables,
                   int64_t bt_stride_b, int32_t W, int32_t *context_lens,
                   int32_t *pages_allocated, int32_t seq_begin, int32_t n_seqs,
                   int32_t next_free_block, int32_t H_kv, int32_t D,
                   int32_t block_size, void *stream);

/*
 * Quest page metadata.  CVSABackend._quest_page_scores
 * (cvsa/backend.py:572-620) needs, per page and KV head, the extremes of the
 * keys over the page's valid tokens (:593-603); the reference recomputes
 * them from the cache on every call, its Quest baseline keeps them per page
 * (eval/baselines.py:77-140).  This entry point brings them up to date:
 *   meta: [num_blocks, H_kv, 2, D] bf16; meta[blk][h][0] = kmin,
 *     meta[blk][h][1] = kmax over the first meta_ntok[blk][h] tokens of blk.
 *   meta_ntok: [num_blocks, H_kv] int32, zero before the first update.
 * Every page of every row whose valid-token count under context_lens
 * differs from meta_ntok is recomputed from k_cache (and its count
 * written).  Keys are assumed to change only by appends: a block whose
 * tokens are rewritten (reused for another sequence) needs its meta_ntok
 * entries cleared first.  A block listed by two rows must hold the same
 * number of valid tokens in both.  k_cache and meta 16-byte aligned.
 */
int cvsa_quest_meta_update(const uint16_t *k_cache, int64_t num_blocks,
                           const int32_t *block_tables, int64_t bt_stride_b,
                           const int32_t *context_lens, int32_t B, int32_t H_kv, int32_t D,
                           int32_t block_size, int32_t W, uint16_t *meta, int32_t *meta_ntok,
                           void *stream);

/*
 * Quest page scores from the metadata.  Replaces
 * CVSABackend._quest_page_scores (cvsa/backend.py:572-620):
 *   page_scores[b,h,p] = sum_d max(q_rep_d * kmin_d, q_rep_d * kmax_d) * D^-0.5
 *   (q_rep as in cvsa_score_pages; fp32 products and sum), -inf when
 *   p*block_size >= context_lens[b] or the block id lies outside the pool.
 * meta: as cvsa_quest_meta_update left it, 16-byte aligned.
 */
int cvsa_quest_scores(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                      const uint16_t *meta, int64_t num_blocks,
                      const int32_t *block_tables, int64_t bt_stride_b,
                      const int32_t *context_lens, int32_t B, int32_t H_q,
                      int32_t H_kv, int32_t D, int32_t block_size, int32_t W,
                      float *page_scores, void *stream);

/*
 * The Quest scores of CVSABackend._quest_page_scores (cvsa/backend.py:
 * 572-620) with the metadata refresh of cvsa_quest_meta_update in the same
 * launch: each page whose count is stale is recomputed, written back and
 * scored from the new values; the others are scored from meta.  Equal, bit
 * for bit, to cvsa_quest_meta_update followed by cvsa_quest_scores.
 * check_accept (may be NULL): B*H_kv flags of a lazy coverage check; when
 * every flag is set the call does nothing (the kept selection needs no
 * ranking scores, and the stale pages wait for the next scoring call).
 */
int cvsa_quest_refresh_scores(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                              const uint16_t *k_cache, int64_t num_blocks,
                              const int32_t *block_tables, int64_t bt_stride_b,
                              const int32_t *context_lens, const uint8_t *check_accept,
                              int32_t B, int32_t H_q, int32_t H_kv, int32_t D,
                              int32_t block_size, int32_t W, uint16_t *meta, int32_t *meta_ntok,
                              float *page_scores, void *stream);

/*
 * Step plans: one layer's decode steps, each enqueued by a single call.
 * The native form of the per-layer step sequences of CVSABackend
 * (cvsa/backend.py): the reuse step (_reuse_step, :866-881: sparse decode of
 * the kept selection), the lazy check (_lazy_step, :392-465: fresh scores,
 * coverage of the kept selection, keep it or reselect, decode with exact
 * recovery) and the fixed-interval scoring step (_scoring_step, :683-864,
 * counters booked by the new selection's gate), with the exact or the
 * Quest page scorer (selector).  The reference issues these
 * as separate Python-level kernel calls; a plan validates the layer's
 * buffers once so that a step costs one host call.
 *
 * The descriptor names the caller's device buffers; they must stay valid
 * while the plan is used.  The plan itself is host memory allocated by
 * cvsa_step_plan_create and released by cvsa_step_plan_destroy (no device
 * memory).  cvsa_step_plan_create checks everything the step's entry points
 * would check, so cvsa_step_plan_run fails only on a bad query pointer,
 * kind or output (nothing enqueued) or a refused launch (CVSA_ERR_LAUNCH;
 * the launches before it stay enqueued).
 */
typedef struct cvsa_step_desc {
  int32_t B, H_q, H_kv, D, block_size, W;
  int32_t budget;              /* selection width: pages per (b, kv-head) row */
  float tau;                   /* coverage threshold */
  int32_t out_dtype;           /* CVSA_DTYPE_* of the step output */
  int64_t q_stride_b, q_stride_h;
  const uint16_t *k_cache, *v_cache;
  int64_t num_blocks;
  const int32_t *block_tables;
  int64_t bt_stride_b;
  const int32_t *context_lens;
  int32_t *page_indices;       /* [B, H_kv, budget]: the layer's selection, updated in place */
  int32_t *n_per_head;         /* [B * H_kv] */
  float *page_scores;          /* [B, H_kv, W]: the step's page scores */
  float *scores_cache;         /* [B, H_kv, W] or NULL: scores of the last reselection */
  uint8_t *check_accept;       /* [B * H_kv]: gate of the kept selection (lazy check) */
  uint8_t *accept;             /* [B * H_kv]: heads accepted by the step */
  float *coverage;             /* [B * H_kv] */
  int64_t *stats;              /* int64[6] counters of cvsa_select_or_keep, or NULL */
  int64_t *work;               /* int64[2] effective-budget counters, or NULL */
  void *workspace;             /* decode workspace, zeroed once (cvsa_workspace_init) */
  size_t workspace_bytes;      /* >= cvsa_step_workspace_bytes(desc) */
  int32_t selector;            /* CVSA_SELECT_*: which scores rank and which gate */
  uint16_t *quest_meta;        /* Quest selectors: metadata of k_cache, as for */
  int32_t *quest_ntok;         /*   cvsa_quest_refresh_scores (else NULL) */
  float *sel_scores;           /* CVSA_SELECT_QUEST: [B, H_kv, W] ranking scores (else NULL) */
  int32_t *spec_state;         /* int32[2] or NULL: speculative lazy checks (below); [0] is
                                  initialised to 1, [1] to 0 */
  uint8_t *sel_map;            /* [B * H_kv, sel_map_stride] bytes, zeroed, or NULL: the map
                                  of the selection (below) */
  int64_t sel_map_stride;      /* >= W, a multiple of 16 (sel_map 16-byte aligned) */
  int32_t approx_budget;       /* > 0: approximate recovery (below); 0: exact recovery */
  int32_t *approx_indices;     /* [B, H_kv, approx_budget] when approx_budget > 0 */
} cvsa_step_desc;

/* Page scorers of a plan (CVSABackend selector / light_normalizer,
 * cvsa/backend.py:150-177, :697-727). */
enum {
  CVSA_SELECT_EXACT = 0,     /* exact page scores rank and gate (cvsa_score_pages) */
  CVSA_SELECT_QUEST = 1,     /* Quest scores rank (into sel_scores), exact scores gate; a
                                lazy check computes the Quest scores only if a head failed */
  CVSA_SELECT_QUEST_LN = 2   /* Quest scores rank and gate (light_normalizer) */
};

/*
 * Speculative lazy checks (spec_state non-NULL).  A lazy check that keeps
 * its selection outputs the sparse decode of that selection, which does not
 * depend on the step's new page scores.  The plan then decodes the cached
 * selection in the same launch as the page scoring (the decode's latency
 * hides under the scoring stream), and the verified decode only books the
 * effective-budget counters when the check kept the selection.  Whether to
 * speculate is predicted from the previous check of the same plan
 * (spec_state[0], written by the selection kernel); a wrong prediction costs
 * time, never results: the outputs, selections, masks and counters equal
 * those of the sequential chain bit for bit.  spec_state[0] = 1 predicts a
 * keep; 2 predicts that every head will be rejected (exact recovery then
 * attends every valid page of every head): with a selection map the launch
 * then decodes every valid page of every head in the identity partition
 * (the listed partition of the page list 0, 1, 2, ...), scoring every page
 * it walks from its keys, so the keys are read once, and a verified decode
 * whose heads are all rejected (which uses that partition itself) only
 * books the counters; the verified decode writes 2 when every head of its
 * launch was rejected.  spec_state[1] records which speculative decode ran
 * (0 none, 1 listed, 2 dense).  Plans whose gate scores are
 * Quest scores (CVSA_SELECT_QUEST_LN), whose H_kv is 1 or 2 or whose D is
 * not 128 run the sequential chain and leave spec_state unchanged.
 * With a selection map (sel_map; 16-token pages) the speculative decode
 * also scores the pages it walks, from the keys it reads for the decode,
 * and the page scoring skips them: the kept selection's keys are read once
 * per check instead of twice, with the same score bits.  The plan writes
 * the map with every selection it makes and maps a selection it adopted
 * (page_indices given at creation) before its first speculative check; a
 * caller that writes page_indices / n_per_head itself must then call
 * cvsa_step_plan_selection_changed.
 */
/*
 * Approximate recovery (approx_budget > 0; CVSABackend approx_recovery_pct,
 * cvsa/backend.py:780-817, with approx_budget = min(max(budget + 1,
 * int(W * approx_recovery_pct)), W)): a selection step writes, for every
 * row whose new selection fails its gate, that row's expanded selection
 * (the approx_budget largest ranking scores, ascending) into
 * approx_indices, and the step's decode is cvsa_verified_decode_approx:
 * rejected heads attend their expanded selection instead of every valid
 * page.  Rows whose gate passed keep stale approx_indices rows.  The
 * expanded selection ranks the selection's scores (sel_scores under
 * CVSA_SELECT_QUEST, else page_scores).
 */
enum {
  CVSA_STEP_REUSE = 0,      /* sparse decode of the kept selection */
  CVSA_STEP_LAZY_CHECK = 1, /* score, check, keep or reselect, verified decode */
  CVSA_STEP_SCORE = 2,      /* score, reselect (gate booked in stats), verified decode */
  CVSA_STEP_FRESH = 3       /* score, first selection of a lazy layer (booked as a lazy
                               scoring step), verified decode */
};

typedef struct cvsa_step_plan cvsa_step_plan;

/* Workspace a plan needs: the larger of its listed and verified decodes. */
size_t cvsa_step_workspace_bytes(const cvsa_step_desc *desc);
int cvsa_step_plan_create(const cvsa_step_desc *desc, cvsa_step_plan **plan);
/* The plan's page_indices / n_per_head were written by something other than
 * the plan: its selection map is rebuilt before the next speculative check.
 * No counterpart in the reference (its selection is a fresh tensor per
 * scoring step). */
int cvsa_step_plan_selection_changed(cvsa_step_plan *plan);
/* q: [B, H_q, D] bf16 with the descriptor's strides; out: [B, H_q, D]. */
int cvsa_step_plan_run(cvsa_step_plan *plan, int32_t kind, const uint16_t *q, void *out,
                       void *stream);
/* A reuse step (CVSA_STEP_REUSE) with the step's token append folded in:
 * cvsa_sparse_decode_append over the plan's buffers, whose k_cache,
 * v_cache, block_tables and context_lens it writes (see there for k_new,
 * v_new, new_stride_b, pages_allocated, slots, slots_dev and slot_errors).  No counterpart in the
 * reference (its loops append, then call the backend). */
int cvsa_step_plan_run_append(cvsa_step_plan *plan, const uint16_t *q, void *out,
                              const uint16_t *k_new, const uint16_t *v_new,
                              int64_t new_stride_b, int32_t *pages_allocated,
                              const int32_t *slots, const int32_t *slots_dev,
                              int32_t *slot_errors, void *stream);
void cvsa_step_plan_destroy(cvsa_step_plan *plan);

#ifdef __cplusplus
}
#endif

#endif /* CVSA_HIP_H */
