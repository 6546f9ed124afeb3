// Entry points internal to libcvsa_hip.so (not exported): a step plan's
// lazy check with its speculative decode (page scoring fused with the decode
// of the cached selection, the select-or-keep that records its decision,
// and the verified decode that skips what the speculation wrote).
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace cvsa_internal {

// Shapes for which score_and_speculate has a fused launch: H_kv 4, 8 or 16
// at D = 128, G = H_q / H_kv at most 16.
bool score_spec_fusable(int32_t H_kv, int32_t D, int32_t G);

int score_and_speculate(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                        const uint16_t *k_cache, const uint16_t *v_cache, int64_t num_blocks,
                        const int32_t *block_tables, int64_t bt_stride_b,
                        const int32_t *context_lens, const int32_t *page_indices,
                        int64_t idx_stride, const int32_t *n_per_head, int32_t max_selected,
                        int32_t B, int32_t H_q, int32_t H_kv, int32_t D, int32_t block_size,
                        int32_t W, float *page_scores, void *out, int32_t out_dtype,
                        int32_t *spec_state, const uint8_t *sel_map, int64_t sel_map_stride,
                        void *workspace, size_t workspace_bytes, void *stream);

// cvsa_verified_decode (exp_indices NULL) or cvsa_verified_decode_approx;
// with spec_state, a launch after a kept speculation only books counters.
int verified_decode_after_speculation(
    const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t *k_cache,
    const uint16_t *v_cache, int64_t num_blocks, const int32_t *block_tables,
    int64_t bt_stride_b, const int32_t *context_lens, const int32_t *page_indices,
    int64_t idx_stride, const int32_t *n_per_head, int32_t max_selected, const uint8_t *accept,
    const int32_t *exp_indices, int64_t exp_stride, int32_t exp_budget, int32_t B, int32_t H_q,
    int32_t H_kv, int32_t D, int32_t block_size, int32_t W, void *out, int32_t out_dtype,
    int64_t *work, int32_t *spec_state, void *workspace, size_t workspace_bytes,
    void *stream);

// cvsa_select_or_keep for a step plan: with check_accept, also writes the
// keep decision to *keep_flag (1: every head passed the check and the
// selection stayed, 0: reselected) -- the prediction the plan's next lazy
// check speculates on; with sel_map, every row it (re)selects also gets its
// selection map row (byte p = page p is among the row's first n_per_head
// entries; rows sel_map_stride bytes apart, the bytes past W stay 0); with
// keep_work, a kept selection whose speculative decode ran (keep_flag[1])
// gets that decode's effective-budget counters booked here instead of by
// the verified decode after it (verified_decode_after_speculation); with
// exp_indices ([rows, exp_budget]), a row whose new selection fails its
// gate also gets its expanded selection (the exp_budget largest ranking
// scores, ascending; approximate recovery, cvsa/backend.py:780-799).
int select_for_plan(const float *page_scores, const float *sel_scores,
                    const uint8_t *check_accept, int32_t B, int32_t H_kv, int32_t W,
                    const int32_t *context_lens, int32_t block_size, int32_t budget,
                    int32_t *page_indices, int32_t *n_per_head, float tau, uint8_t *accept_out,
                    float *coverage_out, float *scores_cache, int64_t *stats,
                    int32_t count_gate, int32_t *keep_flag, uint8_t *sel_map,
                    int64_t sel_map_stride, int64_t *keep_work, int32_t exp_budget,
                    int32_t *exp_indices, void *stream);

// The selection map of a selection made elsewhere: row r (of `rows`) of
// sel_map cleared over sel_map_stride bytes, then byte p set for each of the
// row's first n_per_head[r] entries p in [0, W).
int build_selection_map(const int32_t *page_indices, int64_t idx_stride,
                        const int32_t *n_per_head, int32_t rows, int32_t W, uint8_t *sel_map,
                        int64_t sel_map_stride, void *stream);

}  // namespace cvsa_internal
