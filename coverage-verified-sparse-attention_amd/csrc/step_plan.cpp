// Step plans: a layer's reuse, lazy-check and fixed-interval scoring steps,
// each enqueued by one host call.  The plan copies the caller's descriptor
// after checking everything the chained entry points check, then replays the
// chain (cvsa_score_pages or cvsa_quest_refresh_scores, cvsa_check_coverage,
// cvsa_select_or_keep, cvsa_verified_decode / cvsa_sparse_decode) with the
// stored arguments.
// This is host code only: the kernels are the entry points' own.
#include <hip/hip_runtime.h>
#include <new>
#include <stdint.h>

#include "../../include/cvsa_hip.h"
#include "internal.h"

namespace cvsa_host {
int fail(int code, const char *fmt, ...);
}

#define STEP_REQUIRE(cond, code, ...)                   \
  do {                                                  \
    if (!(cond)) return cvsa_host::fail(code, __VA_ARGS__); \
  } while (0)

struct cvsa_step_plan {
  cvsa_step_desc d;
  // d.sel_map holds the map of the selection in d.page_indices: the plan's
  // own selections write it; one made elsewhere (an adopted selection, or
  // cvsa_step_plan_selection_changed) is mapped before the next lazy check.
  bool map_valid;
};

namespace {

constexpr int kMaxPages = 1 << 18;  // pages per row (cvsa_common.h kMaxPagesWide)
constexpr int64_t kMaxDecodeHeads = 4096;

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

size_t workspace_need(const cvsa_step_desc &d) {
  const size_t listed =
      cvsa_decode_workspace_bytes(d.B, d.H_q, d.H_kv, d.D, d.budget, d.W, 0);
  const size_t verified =
      cvsa_decode_workspace_bytes(d.B, d.H_q, d.H_kv, d.D, d.budget, d.W, 1);
  return listed > verified ? listed : verified;
}

// The union of the checks of the entry points a plan chains.
int check_desc(const cvsa_step_desc &d) {
  STEP_REQUIRE(d.B > 0 && d.H_kv > 0 && d.H_q > 0 && d.H_q % d.H_kv == 0, CVSA_ERR_INVALID,
               "step_plan: bad head counts B=%d H_q=%d H_kv=%d", d.B, d.H_q, d.H_kv);
  const int G = d.H_q / d.H_kv;
  STEP_REQUIRE(G <= 128, CVSA_ERR_UNSUPPORTED, "step_plan: GQA group size %d not in 1..128",
               G);
  STEP_REQUIRE((int64_t)d.B * d.H_kv <= kMaxDecodeHeads, CVSA_ERR_UNSUPPORTED,
               "step_plan: B * H_kv = %lld exceeds %lld heads", (long long)d.B * d.H_kv,
               (long long)kMaxDecodeHeads);
  STEP_REQUIRE((d.D == 32 || d.D == 64 || d.D == 128 || d.D == 256) &&
                   (d.block_size == 8 || d.block_size == 16 || d.block_size == 32 ||
                    d.block_size == 64 || d.block_size == 128),
               CVSA_ERR_UNSUPPORTED,
               "step_plan: D=%d not in {32, 64, 128, 256} or block_size=%d not in {8, 16, 32, 64, 128}",
               d.D, d.block_size);
  STEP_REQUIRE(d.W > 0 && d.W <= kMaxPages, CVSA_ERR_UNSUPPORTED,
               "step_plan: W=%d not in 1..%d", d.W, kMaxPages);
  STEP_REQUIRE(d.budget >= 1 && d.budget <= d.W, CVSA_ERR_INVALID,
               "step_plan: budget=%d must be in [1, W=%d]", d.budget, d.W);
  STEP_REQUIRE(d.num_blocks > 0 && d.bt_stride_b >= d.W, CVSA_ERR_INVALID,
               "step_plan: num_blocks=%lld, block-table row stride %lld < W=%d",
               (long long)d.num_blocks, (long long)d.bt_stride_b, d.W);
  STEP_REQUIRE(d.q_stride_b % 8 == 0 && d.q_stride_h % 8 == 0, CVSA_ERR_INVALID,
               "step_plan: q strides must be multiples of 8 elements");
  STEP_REQUIRE(d.k_cache && d.v_cache && d.block_tables && d.context_lens && d.page_indices &&
                   d.n_per_head && d.page_scores && d.check_accept && d.accept && d.coverage,
               CVSA_ERR_INVALID, "step_plan: null buffer in the descriptor");
  STEP_REQUIRE(aligned16(d.k_cache) && aligned16(d.v_cache), CVSA_ERR_INVALID,
               "step_plan: k_cache / v_cache must be 16-byte aligned");
  STEP_REQUIRE(d.out_dtype >= CVSA_DTYPE_BF16 && d.out_dtype <= CVSA_DTYPE_FP32,
               CVSA_ERR_INVALID, "step_plan: bad output dtype %d", d.out_dtype);
  STEP_REQUIRE(d.selector >= CVSA_SELECT_EXACT && d.selector <= CVSA_SELECT_QUEST_LN,
               CVSA_ERR_INVALID, "step_plan: unknown selector %d", d.selector);
  if (d.selector != CVSA_SELECT_EXACT) {
    STEP_REQUIRE(d.quest_meta && d.quest_ntok && aligned16(d.quest_meta), CVSA_ERR_INVALID,
                 "step_plan: the Quest selectors need quest_meta (16-byte aligned) and "
                 "quest_ntok");
    STEP_REQUIRE((int64_t)d.B * d.H_kv <= 65535, CVSA_ERR_UNSUPPORTED,
                 "step_plan: B * H_kv exceeds 65535 rows for the Quest scorer");
  }
  STEP_REQUIRE(d.selector != CVSA_SELECT_QUEST || d.sel_scores != nullptr, CVSA_ERR_INVALID,
               "step_plan: CVSA_SELECT_QUEST needs a sel_scores buffer");
  STEP_REQUIRE(d.sel_map == nullptr || (d.sel_map_stride >= d.W && d.sel_map_stride % 16 == 0 &&
                                        aligned16(d.sel_map)),
               CVSA_ERR_INVALID,
               "step_plan: sel_map rows must be 16-byte aligned, a multiple of 16 bytes and "
               "at least W=%d bytes apart (got %lld)",
               d.W, (long long)d.sel_map_stride);
  if (d.approx_budget != 0) {
    STEP_REQUIRE(d.approx_budget >= 1 && d.approx_budget <= d.W && d.approx_indices != nullptr,
                 CVSA_ERR_INVALID,
                 "step_plan: approximate recovery needs approx_indices and an approx_budget in "
                 "[1, W=%d] (got %d)",
                 d.W, d.approx_budget);
  }
  const size_t need = workspace_need(d);
  STEP_REQUIRE(need < ((size_t)1 << 31), CVSA_ERR_UNSUPPORTED,
               "step_plan: a decode workspace of %zu bytes exceeds the 2 GiB buffer range",
               need);
  STEP_REQUIRE(need == 0 || (d.workspace != nullptr && d.workspace_bytes >= need &&
                                ((uintptr_t)d.workspace & 255) == 0),
               CVSA_ERR_WORKSPACE,
               "step_plan: workspace of %zu bytes (256-byte aligned) required, got %zu", need,
               d.workspace_bytes);
  return CVSA_OK;
}

int quest(const cvsa_step_desc &d, const uint16_t *q, const uint8_t *check, float *scores,
          void *stream) {
  return cvsa_quest_refresh_scores(q, d.q_stride_b, d.q_stride_h, d.k_cache, d.num_blocks,
                                   d.block_tables, d.bt_stride_b, d.context_lens, check, d.B,
                                   d.H_q, d.H_kv, d.D, d.block_size, d.W, d.quest_meta,
                                   d.quest_ntok, scores, stream);
}

// The gate's page scores (page_scores): the exact scan, or the Quest
// scores under light_normalizer.
int score(const cvsa_step_desc &d, const uint16_t *q, void *stream) {
  if (d.selector == CVSA_SELECT_QUEST_LN) return quest(d, q, nullptr, d.page_scores, stream);
  return cvsa_score_pages(q, d.q_stride_b, d.q_stride_h, d.k_cache, d.num_blocks,
                          d.block_tables, d.bt_stride_b, d.context_lens, d.B, d.H_q, d.H_kv,
                          d.D, d.block_size, d.W, d.page_scores, stream);
}

// Separate ranking scores (CVSA_SELECT_QUEST) into sel_scores; with a
// lazy check's flags they are computed only if a head failed.
int rank(const cvsa_step_desc &d, const uint16_t *q, const uint8_t *check, void *stream) {
  if (d.selector != CVSA_SELECT_QUEST) return CVSA_OK;
  return quest(d, q, check, d.sel_scores, stream);
}

// The step's verified decode (exact or approximate recovery); with
// spec_state, after a speculative check.
int verified(const cvsa_step_desc &d, const uint16_t *q, void *out, int32_t *spec_state,
             void *stream) {
  const bool ar = d.approx_budget > 0;
  return cvsa_internal::verified_decode_after_speculation(
      q, d.q_stride_b, d.q_stride_h, d.k_cache, d.v_cache, d.num_blocks, d.block_tables,
      d.bt_stride_b, d.context_lens, d.page_indices, d.budget, d.n_per_head, d.budget, d.accept,
      ar ? d.approx_indices : nullptr, d.approx_budget, d.approx_budget, d.B, d.H_q, d.H_kv,
      d.D, d.block_size, d.W, out, d.out_dtype, d.work, spec_state, d.workspace,
      d.workspace_bytes, stream);
}

}  // namespace

extern "C" size_t cvsa_step_workspace_bytes(const cvsa_step_desc *desc) {
  if (desc == nullptr) return 0;
  return workspace_need(*desc);
}

extern "C" int cvsa_step_plan_create(const cvsa_step_desc *desc, cvsa_step_plan **plan) {
  STEP_REQUIRE(desc && plan, CVSA_ERR_INVALID, "step_plan_create: null argument");
  *plan = nullptr;
  const int rc = check_desc(*desc);
  if (rc != CVSA_OK) return rc;
  cvsa_step_plan *p = new (std::nothrow) cvsa_step_plan;
  STEP_REQUIRE(p != nullptr, CVSA_ERR_INVALID, "step_plan_create: out of host memory");
  p->d = *desc;
  p->map_valid = false;
  *plan = p;
  return CVSA_OK;
}

extern "C" int cvsa_step_plan_selection_changed(cvsa_step_plan *plan) {
  STEP_REQUIRE(plan, CVSA_ERR_INVALID, "step_plan_selection_changed: null plan");
  plan->map_valid = false;
  return CVSA_OK;
}

extern "C" void cvsa_step_plan_destroy(cvsa_step_plan *plan) {
  if (plan == nullptr) return;
  delete plan;
}

namespace {

// Whether a lazy check of this plan speculates: spec_state given, gate
// scores from the exact scan, and a fused scoring + decode launch for H_kv.
bool speculates(const cvsa_step_desc &d) {
  return d.spec_state != nullptr && d.selector != CVSA_SELECT_QUEST_LN && d.block_size != 8 &&
         cvsa_internal::score_spec_fusable(d.H_kv, d.D, d.H_q / d.H_kv);
}

// The plan's selection map, when it has one (16-token pages).
uint8_t *plan_map(const cvsa_step_desc &d) { return d.block_size == 16 ? d.sel_map : nullptr; }

// The selection step of a plan: cvsa_select_or_keep writing the plan's
// selection map with the selection.
int plan_select(const cvsa_step_desc &d, const uint8_t *check, float *scores_cache,
                int32_t count_gate, int32_t *keep_flag, void *stream) {
  const float *sel = d.selector == CVSA_SELECT_QUEST ? d.sel_scores : nullptr;
  // With the keep flag (a speculative check), a kept speculation's counters
  // are booked by the select.
  return cvsa_internal::select_for_plan(
      d.page_scores, sel, check, d.B, d.H_kv, d.W, d.context_lens, d.block_size, d.budget,
      d.page_indices, d.n_per_head, d.tau, d.accept, d.coverage, scores_cache, d.stats,
      count_gate, keep_flag, plan_map(d), d.sel_map_stride,
      keep_flag != nullptr ? d.work : nullptr, d.approx_budget,
      d.approx_budget > 0 ? d.approx_indices : nullptr, stream);
}

// The lazy check with the speculative decode: one launch scores the pages
// and decodes the cached selection (if spec_state[0] predicts a keep), then
// the check, the select-or-keep that records its decision in spec_state[0],
// and the verified decode, which only books counters when the selection was
// kept and the speculative decode ran.  With a selection map the launch
// scores the selection's pages from the decode's keys; a selection the plan
// did not make is mapped first.
int speculative_check(cvsa_step_plan &p, const uint16_t *q, void *out, void *stream) {
  const cvsa_step_desc &d = p.d;
  int rc;
  uint8_t *map = plan_map(d);
  if (map != nullptr && !p.map_valid) {
    if ((rc = cvsa_internal::build_selection_map(d.page_indices, d.budget, d.n_per_head,
                                                 d.B * d.H_kv, d.W, map, d.sel_map_stride,
                                                 stream)) != CVSA_OK)
      return rc;
    p.map_valid = true;
  }
  if ((rc = cvsa_internal::score_and_speculate(
           q, d.q_stride_b, d.q_stride_h, d.k_cache, d.v_cache, d.num_blocks, d.block_tables,
           d.bt_stride_b, d.context_lens, d.page_indices, d.budget, d.n_per_head, d.budget, d.B,
           d.H_q, d.H_kv, d.D, d.block_size, d.W, d.page_scores, out, d.out_dtype,
           d.spec_state, map, d.sel_map_stride, d.workspace, d.workspace_bytes, stream)) !=
      CVSA_OK)
    return rc;
  if ((rc = cvsa_check_coverage(d.page_scores, d.B, d.H_kv, d.W, d.page_indices, d.budget,
                                d.n_per_head, d.tau, d.check_accept, d.coverage, stream)) !=
      CVSA_OK)
    return rc;
  if ((rc = rank(d, q, d.check_accept, stream)) != CVSA_OK) return rc;
  if ((rc = plan_select(d, d.check_accept, d.scores_cache, 0, d.spec_state, stream)) !=
      CVSA_OK)
    return rc;
  return verified(d, q, out, d.spec_state, stream);
}

}  // namespace

extern "C" int cvsa_step_plan_run_append(cvsa_step_plan *plan, const uint16_t *q, void *out,
                                         const uint16_t *k_new, const uint16_t *v_new,
                                         int64_t new_stride_b, int32_t *pages_allocated,
                                         const int32_t *slots, const int32_t *slots_dev,
                                         int32_t *slot_errors, void *stream) {
  STEP_REQUIRE(plan && q && out, CVSA_ERR_INVALID, "step_plan_run_append: null argument");
  STEP_REQUIRE(aligned16(q), CVSA_ERR_INVALID,
               "step_plan_run_append: q must be 16-byte aligned");
  const cvsa_step_desc &d = plan->d;
  // The descriptor's caches, page table and context lengths are the
  // caller's writable buffers; this step appends to them.
  return cvsa_sparse_decode_append(
      q, d.q_stride_b, d.q_stride_h, const_cast<uint16_t *>(d.k_cache),
      const_cast<uint16_t *>(d.v_cache), d.num_blocks, const_cast<int32_t *>(d.block_tables),
      d.bt_stride_b, const_cast<int32_t *>(d.context_lens), d.page_indices, d.budget,
      d.n_per_head, d.budget, d.B, d.H_q, d.H_kv, d.D, d.block_size, d.W, out, d.out_dtype,
      d.work, d.workspace, d.workspace_bytes, k_new, v_new, new_stride_b, pages_allocated,
      slots, slots_dev, slot_errors, stream);
}

extern "C" int cvsa_step_plan_run(cvsa_step_plan *plan, int32_t kind, const uint16_t *q,
                                  void *out, void *stream) {
  STEP_REQUIRE(plan && q && out, CVSA_ERR_INVALID, "step_plan_run: null argument");
  STEP_REQUIRE(aligned16(q), CVSA_ERR_INVALID, "step_plan_run: q must be 16-byte aligned");
  STEP_REQUIRE(kind == CVSA_STEP_REUSE || kind == CVSA_STEP_LAZY_CHECK ||
                   kind == CVSA_STEP_SCORE || kind == CVSA_STEP_FRESH,
               CVSA_ERR_INVALID, "step_plan_run: unknown step kind %d", kind);
  const cvsa_step_desc &d = plan->d;
  int rc;
  switch (kind) {
    case CVSA_STEP_REUSE:
      return cvsa_sparse_decode(q, d.q_stride_b, d.q_stride_h, d.k_cache, d.v_cache,
                                d.num_blocks, d.block_tables, d.bt_stride_b, d.context_lens,
                                d.page_indices, d.budget, d.n_per_head, d.budget, d.B, d.H_q,
                                d.H_kv, d.D, d.block_size, d.W, nullptr, nullptr, nullptr, out,
                                d.out_dtype, d.work, d.workspace, d.workspace_bytes, stream);
    case CVSA_STEP_LAZY_CHECK:
      if (speculates(d)) return speculative_check(*plan, q, out, stream);
      if ((rc = score(d, q, stream)) != CVSA_OK) return rc;
      if ((rc = cvsa_check_coverage(d.page_scores, d.B, d.H_kv, d.W, d.page_indices, d.budget,
                                    d.n_per_head, d.tau, d.check_accept, d.coverage,
                                    stream)) != CVSA_OK)
        return rc;
      if ((rc = rank(d, q, d.check_accept, stream)) != CVSA_OK) return rc;
      if ((rc = plan_select(d, d.check_accept, d.scores_cache, 0, nullptr, stream)) != CVSA_OK)
        return rc;
      return verified(d, q, out, nullptr, stream);
    case CVSA_STEP_FRESH:
      if ((rc = score(d, q, stream)) != CVSA_OK) return rc;
      if ((rc = rank(d, q, nullptr, stream)) != CVSA_OK) return rc;
      if ((rc = plan_select(d, nullptr, d.scores_cache, 0, nullptr, stream)) != CVSA_OK)
        return rc;
      plan->map_valid = true;  // every row selected anew
      return verified(d, q, out, nullptr, stream);
    default:  // CVSA_STEP_SCORE
      if ((rc = score(d, q, stream)) != CVSA_OK) return rc;
      if ((rc = rank(d, q, nullptr, stream)) != CVSA_OK) return rc;
      if ((rc = plan_select(d, nullptr, nullptr, 1, nullptr, stream)) != CVSA_OK) return rc;
      plan->map_valid = true;
      return verified(d, q, out, nullptr, stream);
  }
}
