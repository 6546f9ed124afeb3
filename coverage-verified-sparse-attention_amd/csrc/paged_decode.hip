// Host side of the paged decode: launch planning, argument checks,
// workspaces and the C-ABI entry points (cvsa_sparse_decode,
// cvsa_sparse_decode_noalloc, cvsa_verified_decode, cvsa_dense_decode and
// their workspace helpers).  The kernels and their semantics are in
// decode_kernels.h; decode_g*.hip instantiate them per GQA group size.
#include "decode_kernels.h"
#include "internal.h"

#include <mutex>

namespace cvsa {

CVSA_DECODE_EXTERN(1)
CVSA_DECODE_EXTERN(2)
CVSA_DECODE_EXTERN(3)
CVSA_DECODE_EXTERN(4)
CVSA_DECODE_EXTERN(5)
CVSA_DECODE_EXTERN(6)
CVSA_DECODE_EXTERN(7)
CVSA_DECODE_EXTERN(8)
CVSA_DECODE_EXTERN(9)
CVSA_DECODE_EXTERN(10)
CVSA_DECODE_EXTERN(11)
CVSA_DECODE_EXTERN(12)
CVSA_DECODE_EXTERN(13)
CVSA_DECODE_EXTERN(14)
CVSA_DECODE_EXTERN(15)
CVSA_DECODE_EXTERN(16)

__global__ void fill_zero_kernel(uint32_t *p, size_t n_words) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}


// Launch plan.  Listed launches (every head walks its page list) use the
// static split grid of listed_decode_kernel: ~target_workgroups()
// workgroups spread over the heads, at least kMinPagesPerWg pages per split,
// at most kMaxSplits splits per head.  Verified and dense launches use the
// stream-K grid of streamk_decode_kernel: target_workgroups(), fewer when
// even the largest possible page list (every head walking all W pages) would
// give a workgroup less than kMinPagesPerWg pages; the kernel narrows it to
// the pages actually walked.
struct DecodeLaunch {
  bool streamk;
  int grid_x, grid_y;
  int pps, n_splits;    // listed partition
  int pps_all, n_splits_all;  // identity partition (verified launches: every head rejected)
  int sk_grid;          // stream-K partition (<= kMaxSplits workgroups)
  size_t partial_rows;  // rows of G x part_stride(D) fp32 (0: no workspace)
};

static DecodeLaunch plan_launch(int B, int H_kv, int max_sel, int W, bool listed,
                                bool all_pages) {
  const int64_t heads = (int64_t)B * H_kv;
  const int target = kTargetWorkgroups;
  DecodeLaunch p{};
  if (listed && !all_pages) {
    int wg_per_head = heads >= target ? 1 : (int)(target / heads);
    if (wg_per_head > kMaxSplits) wg_per_head = kMaxSplits;
    int pps = (max_sel + wg_per_head - 1) / wg_per_head;
    if (pps < kMinPagesPerWg) pps = kMinPagesPerWg;
    pps = (pps + kWavesPerWg - 1) / kWavesPerWg * kWavesPerWg;
    while ((max_sel + pps - 1) / pps > kMaxSplits) pps += kWavesPerWg;
    p.streamk = false;
    p.pps = pps;
    p.n_splits = max_sel > pps ? (max_sel + pps - 1) / pps : 1;
    p.grid_x = p.n_splits;
    p.grid_y = (int)heads;
    p.partial_rows = p.n_splits > 1 ? (size_t)heads * p.n_splits : 0;
    return p;
  }
  int64_t per_head = listed ? max_sel : 0;
  if (W > per_head) per_head = W;
  int64_t g = (heads * per_head + kMinPagesPerWg - 1) / kMinPagesPerWg;
  if (g > target) g = target;
  if (g < 1) g = 1;
  p.streamk = true;
  p.sk_grid = (int)g;
  p.grid_x = (int)g;
  p.grid_y = 1;
  p.partial_rows = g > 1 ? (size_t)g + heads : 0;  // row w + h: workgroup w's partial of head h
  if (listed) {
    // Verified launches also carry the listed partition, which they run
    // when every head is accepted: at least one workgroup per (split, head).
    const DecodeLaunch lp = plan_launch(B, H_kv, max_sel, W, true, false);
    p.pps = lp.pps;
    p.n_splits = lp.n_splits;
    const int64_t n_listed = (int64_t)lp.grid_x * lp.grid_y;
    if (n_listed > p.grid_x) p.grid_x = (int)n_listed;
    if (lp.partial_rows > p.partial_rows) p.partial_rows = lp.partial_rows;
    // ... and the identity partition, which they run when every head is
    // rejected: the listed partition of a W-page list.
    const DecodeLaunch ip = plan_launch(B, H_kv, W, W, true, false);
    p.pps_all = ip.pps;
    p.n_splits_all = ip.n_splits;
    const int64_t n_ident = (int64_t)ip.grid_x * ip.grid_y;
    if (n_ident > p.grid_x) p.grid_x = (int)n_ident;
    if (ip.partial_rows > p.partial_rows) p.partial_rows = ip.partial_rows;
  }
  return p;
}

// Workspace: a fixed area of kMaxHeads completion counters and
// kGroupCounters group counters of the two-level merge (uint32), then the
// partial rows.  The counter area has the same size and place for every
// launch, so launches of different B * H_kv that share a workspace never
// read one another's partial rows as counters: counter h of every launch is
// word h, and every launch leaves the words it used at zero.  Launches with
// split partials have at most kMaxHeads heads (stream-K: checked at launch;
// listed: more than one split per head only below kMaxSplits heads).
constexpr size_t kCounterAreaBytes = (size_t)(kMaxHeads + kGroupCounters) * sizeof(unsigned);
static_assert(kTargetWorkgroups * 2 <= kGroupCounters, "a group counter per group start");
static_assert(kCounterAreaBytes % 256 == 0, "partial rows start 256-byte aligned");

static size_t workspace_bytes_for(int B, int H_q, int H_kv, int D, int max_sel, int W,
                                  bool listed, bool all_pages) {
  // One launch serves at most kMaxGroup query heads per KV head; larger
  // groups run as several launches over the same workspace.
  const int G = min(H_q / H_kv, kMaxGroup);
  const DecodeLaunch p = plan_launch(B, H_kv, max_sel, W, listed, all_pages);
  if (p.partial_rows == 0) return 0;
  return kCounterAreaBytes + p.partial_rows * G * part_stride(D) * sizeof(float);
}

// Head dimensions with decode kernels.
static bool decode_head_dim(int D) { return head_dim_supported(D); }

// Argument checks of a decode launch (everything but the workspace) and its
// launch plan; fills the launch-shape fields of `a`.  Returns a status.
static int validate_decode(const char *name, DecodeArgs &a, int B, int H_q, int H_kv, int D,
                           int block_size, int W, bool listed, bool all_pages,
                           DecodeLaunch &p, size_t &need) {
  CVSA_REQUIRE(a.q && a.k_cache && a.v_cache && a.block_tables && a.ctx_lens,
               CVSA_ERR_INVALID, "%s: null pointer argument", name);
  CVSA_REQUIRE(B > 0 && B * (int64_t)H_kv <= 65535 && W > 0 && a.num_blocks > 0,
               CVSA_ERR_INVALID, "%s: bad sizes B=%d H_kv=%d W=%d", name, B, H_kv, W);
  CVSA_REQUIRE(H_kv > 0 && H_q > 0 && H_q % H_kv == 0, CVSA_ERR_INVALID,
               "%s: H_q=%d is not a multiple of H_kv=%d", name, H_q, H_kv);
  const int G = H_q / H_kv;
  CVSA_REQUIRE(G >= 1 && G <= kMaxGroupTotal, CVSA_ERR_UNSUPPORTED,
               "%s: GQA group size %d not in 1..%d", name, G, kMaxGroupTotal);
  CVSA_REQUIRE(decode_head_dim(D) && block_size_supported(block_size), CVSA_ERR_UNSUPPORTED,
               "%s: D=%d, block_size=%d not supported (D in {32, 64, 128, 256}, block_size in "
               "{8, 16, 32, 64, 128})",
               name, D, block_size);
  const int ts = page_tile_shift(block_size);
  CVSA_REQUIRE(a.num_blocks <= (INT32_MAX >> ts), CVSA_ERR_UNSUPPORTED,
               "%s: %lld blocks exceed the tile index range", name, (long long)a.num_blocks);
  CVSA_REQUIRE(W <= kMaxPagesWide, CVSA_ERR_UNSUPPORTED, "%s: W=%d exceeds %d pages", name,
               W, kMaxPagesWide);
  CVSA_REQUIRE(a.bt_sb >= W, CVSA_ERR_INVALID, "%s: block-table row stride %lld < W=%d",
               name, (long long)a.bt_sb, W);
  CVSA_REQUIRE(((uintptr_t)a.q & 15) == 0 && a.q_sb % 8 == 0 && a.q_sh % 8 == 0 &&
                   ((uintptr_t)a.k_cache & 15) == 0 && ((uintptr_t)a.v_cache & 15) == 0,
               CVSA_ERR_INVALID,
               "%s: q / caches must be 16-byte aligned with strides that are multiples "
               "of 8 elements",
               name);
  if (listed) {
    CVSA_REQUIRE(a.page_idx && a.n_pages, CVSA_ERR_INVALID,
                 "%s: page_indices / n_per_head missing", name);
    CVSA_REQUIRE(a.max_sel >= 0 && a.max_sel <= kMaxPagesWide && a.idx_stride >= a.max_sel,
                 CVSA_ERR_INVALID, "%s: bad selection width %d (row stride %lld)", name,
                 a.max_sel, (long long)a.idx_stride);
  }
  if (a.alt_idx != nullptr) {
    CVSA_REQUIRE(listed && a.accept != nullptr, CVSA_ERR_INVALID,
                 "%s: an expanded selection needs accept flags", name);
    CVSA_REQUIRE(a.alt_budget >= 1 && a.alt_budget <= W && a.alt_stride >= a.alt_budget,
                 CVSA_ERR_INVALID,
                 "%s: expanded budget %d must be in [1, W=%d] with a row stride >= it (%lld)",
                 name, a.alt_budget, W, (long long)a.alt_stride);
  }
  const bool want_unnorm = a.o_unnorm || a.m_out || a.l_out;
  CVSA_REQUIRE(!want_unnorm || (a.o_unnorm && a.m_out && a.l_out), CVSA_ERR_INVALID,
               "%s: o_unnorm, m_out and l_out must be given together", name);
  CVSA_REQUIRE(want_unnorm || a.out, CVSA_ERR_INVALID, "%s: no output requested", name);
  CVSA_REQUIRE(((uintptr_t)a.out & 15) == 0 && ((uintptr_t)a.o_unnorm & 15) == 0,
               CVSA_ERR_INVALID, "%s: out / o_unnorm must be 16-byte aligned", name);
  CVSA_REQUIRE(a.out == nullptr || (a.out_dtype >= CVSA_DTYPE_BF16 &&
                                    a.out_dtype <= CVSA_DTYPE_FP32),
               CVSA_ERR_INVALID, "%s: bad output dtype %d", name, a.out_dtype);

  p = plan_launch(B, H_kv, listed ? a.max_sel : 0, W, listed, all_pages);
  CVSA_REQUIRE((!p.streamk && p.partial_rows == 0) || (int64_t)B * H_kv <= kMaxHeads,
               CVSA_ERR_UNSUPPORTED, "%s: B * H_kv = %lld exceeds %d heads per launch", name,
               (long long)B * H_kv, kMaxHeads);
  need = workspace_bytes_for(B, H_q, H_kv, D, listed ? a.max_sel : 0, W, listed, all_pages);
  CVSA_REQUIRE(need == 0 || need - kCounterAreaBytes < ((size_t)1 << 31),
               CVSA_ERR_UNSUPPORTED,
               "%s: %zu bytes of split partials exceed the 2 GiB buffer range", name,
               need - kCounterAreaBytes);
  a.W = W;
  a.H_kv = H_kv;
  a.heads = B * H_kv;
  a.pps = p.pps << ts;
  a.n_splits = p.n_splits;
  a.pps_all = p.pps_all << ts;
  a.n_splits_all = p.n_splits_all;
  a.sk_grid = p.sk_grid;
  a.D = D;
  a.ts = ts;
  a.tl = tile_rows_log2(block_size);
  a.q_group = G;
  a.q_off = 0;
  a.scale = (float)pow((double)D, -0.5);
  return CVSA_OK;
}

// Enqueue a validated launch with its workspace (need bytes, 0 = none).
static void bind_workspace(DecodeArgs &a, void *workspace, size_t need) {
  a.counters = reinterpret_cast<unsigned *>(workspace);
  a.part = need == 0 ? nullptr
                     : reinterpret_cast<float *>(reinterpret_cast<char *>(workspace) +
                                                 kCounterAreaBytes);
  a.part_bytes = need == 0 ? 0u : (uint32_t)(need - kCounterAreaBytes);
}

static int enqueue_decode(const char *name, DecodeArgs a, int G, bool listed,
                          const DecodeLaunch &p, void *workspace, size_t need, hipStream_t st) {
  bind_workspace(a, workspace, need);
  const dim3 grid(p.grid_x, p.grid_y), block(kWavesPerWg * kWave);
  const int kind = !p.streamk ? kLaunchListed
                   : !listed   ? kLaunchAll
                   : a.alt_idx != nullptr ? kLaunchApprox
                                          : kLaunchVerified;
  // Groups of more than kMaxGroup query heads: one launch per kMaxGroup of
  // them, in order on the stream (each leaves the workspace counters at
  // zero); the first books the effective-budget counters.
  unsigned long long *work = a.work;
  a.q_group = G;
  for (int off = 0; off < G; off += kMaxGroup) {
    a.q_off = off;
    a.work = off == 0 ? work : nullptr;
    switch (min(kMaxGroup, G - off)) {
#define CVSA_DEC_CASE(GG)                             \
  case GG:                                            \
    launch_decode_g<GG>(a, kind, grid, block, st);    \
    break;
      CVSA_DEC_CASE(1) CVSA_DEC_CASE(2) CVSA_DEC_CASE(3) CVSA_DEC_CASE(4)
      CVSA_DEC_CASE(5) CVSA_DEC_CASE(6) CVSA_DEC_CASE(7) CVSA_DEC_CASE(8)
      CVSA_DEC_CASE(9) CVSA_DEC_CASE(10) CVSA_DEC_CASE(11) CVSA_DEC_CASE(12)
      CVSA_DEC_CASE(13) CVSA_DEC_CASE(14) CVSA_DEC_CASE(15) CVSA_DEC_CASE(16)
#undef CVSA_DEC_CASE
      default:
        break;
    }
    const int rc = cvsa_host::check_launch(name);
    if (rc != CVSA_OK) return rc;
  }
  return CVSA_OK;
}

static int check_workspace(const char *name, void *workspace, size_t workspace_bytes,
                           size_t need) {
  CVSA_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need &&
                                ((uintptr_t)workspace & 255) == 0),
               CVSA_ERR_WORKSPACE,
               "%s: workspace of %zu bytes (256-byte aligned) required, got %zu", name,
               need, workspace_bytes);
  return CVSA_OK;
}

static int launch_decode(const char *name, DecodeArgs a, int B, int H_q, int H_kv, int D,
                         int block_size, int W, bool listed, bool all_pages,
                         void *workspace, size_t workspace_bytes, hipStream_t st) {
  DecodeLaunch p{};
  size_t need = 0;
  int rc = validate_decode(name, a, B, H_q, H_kv, D, block_size, W, listed, all_pages, p, need);
  if (rc != CVSA_OK) return rc;
  if ((rc = check_workspace(name, workspace, workspace_bytes, need)) != CVSA_OK) return rc;
  return enqueue_decode(name, a, H_q / H_kv, listed, p, workspace, need, st);
}

static DecodeArgs base_args(const uint16_t *q, int64_t q_sb, int64_t q_sh,
                            const uint16_t *k_cache, const uint16_t *v_cache,
                            int64_t num_blocks, const int32_t *block_tables, int64_t bt_sb,
                            const int32_t *context_lens, float *o_unnorm, float *m_out,
                            float *l_out, void *out, int32_t out_dtype, int64_t *work) {
  DecodeArgs a{};
  a.work = reinterpret_cast<unsigned long long *>(work);
  a.q = q;
  a.q_sb = q_sb;
  a.q_sh = q_sh;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.num_blocks = num_blocks;
  a.block_tables = block_tables;
  a.bt_sb = bt_sb;
  a.ctx_lens = context_lens;
  a.o_unnorm = o_unnorm;
  a.m_out = m_out;
  a.l_out = l_out;
  a.out = out;
  a.out_dtype = out_dtype;
  return a;
}

}  // namespace cvsa

using namespace cvsa;

extern "C" size_t cvsa_decode_workspace_bytes(int32_t B, int32_t H_q, int32_t H_kv,
                                              int32_t D, int32_t max_sel_pages, int32_t W,
                                              int32_t all_pages) {
  if (B <= 0 || H_kv <= 0 || H_q <= 0 || H_q % H_kv != 0 || W <= 0 || max_sel_pages < 0 ||
      !decode_head_dim(D))
    return 0;
  const bool listed = max_sel_pages > 0;
  return workspace_bytes_for(B, H_q, H_kv, D, max_sel_pages, W, listed, all_pages != 0);
}

extern "C" int cvsa_workspace_init(void *workspace, size_t workspace_bytes, void *stream) {
  CVSA_REQUIRE(workspace && ((uintptr_t)workspace & 3) == 0 && workspace_bytes % 4 == 0,
               CVSA_ERR_INVALID, "workspace_init: workspace must be 4-byte aligned and sized");
  const size_t words = workspace_bytes / 4;
  if (words == 0) return CVSA_OK;
  size_t blocks = (words + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<uint32_t *>(workspace), words);
  return cvsa_host::check_launch("workspace_init");
}

extern "C" int cvsa_sparse_decode(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                                  const uint16_t *k_cache, const uint16_t *v_cache,
                                  int64_t num_blocks, const int32_t *block_tables,
                                  int64_t bt_stride_b, const int32_t *context_lens,
                                  const int32_t *page_indices, int64_t idx_stride,
                                  const int32_t *n_per_head, int32_t max_selected,
                                  int32_t B, int32_t H_q, int32_t H_kv, int32_t D,
                                  int32_t block_size, int32_t W, float *o_unnorm,
                                  float *m_out, float *l_out, void *out, int32_t out_dtype,
                                  int64_t *work, void *workspace, size_t workspace_bytes,
                                  void *stream) {
  DecodeArgs a = base_args(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                           block_tables, bt_stride_b, context_lens, o_unnorm, m_out, l_out,
                           out, out_dtype, work);
  a.page_idx = page_indices;
  a.idx_stride = idx_stride;
  a.max_sel = max_selected;
  a.n_pages = n_per_head;
  if (page_indices == nullptr)
    return cvsa_host::fail(CVSA_ERR_INVALID, "sparse_decode: page_indices is NULL");
  return launch_decode("sparse_decode", a, B, H_q, H_kv, D, block_size, W, true, false,
                       workspace, workspace_bytes, (hipStream_t)stream);
}

// ------------------------------------------------ decode with the token append
// cvsa_sparse_decode_append: the append of cvsa_append_kv (one token per
// sequence, slots from the caller's host mirror) and the listed decode of
// cvsa_sparse_decode over the appended cache.  One launch
// (listed_append_kernel) for 16-token pages, D = 128, G <= 16 and
// B <= kMaxAppendSeqs; otherwise the two entry points in order.
static int check_append_slots(const char *name, const int32_t *slots, int B, int block_size,
                              int W, int64_t num_blocks, int &next_free) {
  CVSA_REQUIRE(slots != nullptr, CVSA_ERR_INVALID, "%s: slots is NULL", name);
  next_free = -1;
  int rank = 0;
  for (int b = 0; b < B; ++b) {
    const int ctx = slots[2 * b], blk = slots[2 * b + 1];
    CVSA_REQUIRE(ctx >= 0 && ctx / block_size < W, CVSA_ERR_INVALID,
                 "%s: sequence %d: context %d + 1 exceeds the block table (%d pages)", name, b,
                 ctx, W);
    if (blk < 0) {
      CVSA_REQUIRE(blk == -1, CVSA_ERR_INVALID, "%s: sequence %d: bad new block %d", name, b,
                   blk);
      continue;
    }
    if (next_free < 0) next_free = blk;
    CVSA_REQUIRE(ctx % block_size == 0 && blk == next_free + rank && blk < num_blocks,
                 CVSA_ERR_INVALID,
                 "%s: sequence %d: new block %d is not the next of the allocator (context %d, "
                 "%lld blocks)",
                 name, b, blk, ctx, (long long)num_blocks);
    ++rank;
  }
  if (next_free < 0) next_free = 0;
  return CVSA_OK;
}

extern "C" int cvsa_sparse_decode_append(
    const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h, uint16_t *k_cache,
    uint16_t *v_cache, int64_t num_blocks, int32_t *block_tables, int64_t bt_stride_b,
    int32_t *context_lens, const int32_t *page_indices, int64_t idx_stride,
    const int32_t *n_per_head, int32_t max_selected, int32_t B, int32_t H_q, int32_t H_kv,
    int32_t D, int32_t block_size, int32_t W, void *out, int32_t out_dtype, int64_t *work,
    void *workspace, size_t workspace_bytes, const uint16_t *k_new, const uint16_t *v_new,
    int64_t new_stride_b, int32_t *pages_allocated, const int32_t *slots,
    const int32_t *slots_dev, int32_t *slot_errors, void *stream) {
  const char *name = "sparse_decode_append";
  CVSA_REQUIRE((slots == nullptr) != (slots_dev == nullptr), CVSA_ERR_INVALID,
               "%s: exactly one of slots (host) and slots_dev (device) is required", name);
  CVSA_REQUIRE(k_new && v_new && pages_allocated && page_indices, CVSA_ERR_INVALID,
               "%s: null pointer argument", name);
  CVSA_REQUIRE(((uintptr_t)k_new & 15) == 0 && ((uintptr_t)v_new & 15) == 0 &&
                   new_stride_b % 8 == 0 && new_stride_b >= (int64_t)H_kv * D,
               CVSA_ERR_INVALID,
               "%s: new K/V rows must be 16-byte aligned, new_stride_b a multiple of 8 >= "
               "H_kv * D",
               name);
  DecodeArgs a = base_args(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                           block_tables, bt_stride_b, context_lens, nullptr, nullptr, nullptr,
                           out, out_dtype, work);
  a.page_idx = page_indices;
  a.idx_stride = idx_stride;
  a.max_sel = max_selected;
  a.n_pages = n_per_head;
  DecodeLaunch p{};
  size_t need = 0;
  int rc = validate_decode(name, a, B, H_q, H_kv, D, block_size, W, true, false, p, need);
  if (rc != CVSA_OK) return rc;
  if ((rc = check_workspace(name, workspace, workspace_bytes, need)) != CVSA_OK) return rc;
  int next_free = 0;
  if (slots != nullptr &&
      (rc = check_append_slots(name, slots, B, block_size, W, num_blocks, next_free)) !=
          CVSA_OK)
    return rc;
  const int G = H_q / H_kv;
  hipStream_t st = (hipStream_t)stream;
  const bool one_launch = D == 128 && block_size == kPageTokens && G <= kMaxGroup &&
                          B <= kMaxAppendSeqs && !p.streamk;
  CVSA_REQUIRE(one_launch || slots_dev == nullptr, CVSA_ERR_UNSUPPORTED,
               "%s: device slots need the one-launch form (D = 128, block_size 16, "
               "H_q / H_kv <= %d, B <= %d)",
               name, kMaxGroup, kMaxAppendSeqs);
  if (!one_launch) {
    if ((rc = cvsa_append_kv(k_new, v_new, new_stride_b, k_cache, v_cache, num_blocks,
                             block_tables, bt_stride_b, W, context_lens, pages_allocated, 0, B,
                             next_free, H_kv, D, block_size, stream)) != CVSA_OK)
      return rc;
    return enqueue_decode(name, a, G, true, p, workspace, need, st);
  }
  AppendArgs app{};
  app.k_new = k_new;
  app.v_new = v_new;
  app.new_sb = new_stride_b;
  app.block_tables = block_tables;
  app.ctx_lens = context_lens;
  app.pages_allocated = pages_allocated;
  app.max_pages = W;
  app.slot_dev = reinterpret_cast<const int2 *>(slots_dev);
  app.slot_errors = slots_dev != nullptr ? slot_errors : nullptr;
  if (slots != nullptr)
    for (int b = 0; b < B; ++b) app.slot[b] = make_int2(slots[2 * b], slots[2 * b + 1]);
  bind_workspace(a, workspace, need);
  a.q_group = G;
  a.q_off = 0;
  const dim3 grid(p.grid_x, p.grid_y);
  switch (G) {
#define CVSA_APP_CASE(GG)                     \
  case GG:                                    \
    launch_append_g<GG>(a, app, grid, st);    \
    break;
    CVSA_APP_CASE(1) CVSA_APP_CASE(2) CVSA_APP_CASE(3) CVSA_APP_CASE(4)
    CVSA_APP_CASE(5) CVSA_APP_CASE(6) CVSA_APP_CASE(7) CVSA_APP_CASE(8)
    CVSA_APP_CASE(9) CVSA_APP_CASE(10) CVSA_APP_CASE(11) CVSA_APP_CASE(12)
    CVSA_APP_CASE(13) CVSA_APP_CASE(14) CVSA_APP_CASE(15) CVSA_APP_CASE(16)
#undef CVSA_APP_CASE
    default:
      break;
  }
  return cvsa_host::check_launch(name);
}

// ------------------------------------------------ allocation-free variant
// cvsa_sparse_decode_noalloc keeps the decode workspace in this file-scope
// device array instead of a caller-owned buffer.  Each GPU the library runs
// on holds its own copy until the process ends.  A listed launch needs at
// most kCounterAreaBytes + kMaxSplits partials of G x (D + 4) fp32, G <= 16,
// D <= 256 (4.3 MB: plan_launch splits heads only when there are fewer than
// kMaxSplits of them, into at most kMaxSplits / heads splits each), so every
// call cvsa_sparse_decode accepts fits; a larger need is refused all the
// same.
constexpr size_t kScratchBytes = (size_t)9 << 19;  // 4.5 MiB
static_assert(kScratchBytes >= kCounterAreaBytes + (size_t)kMaxSplits * kMaxGroup *
                                                       part_stride(256) * sizeof(float),
              "scratch holds every listed launch");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch`, per device

// The device address of `scratch` on the stream's device, looked up once per
// device (with that device current).  The first lookup also zeroes the
// counter area on `st`, ahead of the call's own launch; every launch leaves
// the counters it used at zero again.  The partial rows need no clearing:
// each launch writes a row before any workgroup reads it.
static int scratch_for(hipStream_t st, void **out) {
  int dev = 0;
  hipError_t e = st != nullptr ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  CVSA_REQUIRE(e == hipSuccess, CVSA_ERR_INVALID,
               "sparse_decode_noalloc: cannot tell the stream's device: %s",
               hipGetErrorString(e));
  CVSA_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, CVSA_ERR_UNSUPPORTED,
               "sparse_decode_noalloc: device %d beyond the %d supported", dev,
               kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = 0;
    bool switched = false;
    e = hipGetDevice(&cur);
    if (e == hipSuccess && cur != dev) {
      e = hipSetDevice(dev);
      switched = e == hipSuccess;
    }
    void *ptr = nullptr;
    if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e == hipSuccess) {
      hipLaunchKernelGGL(fill_zero_kernel, dim3(16), dim3(256), 0, st,
                         reinterpret_cast<uint32_t *>(ptr), kCounterAreaBytes / 4);
      e = hipGetLastError();
    }
    if (switched) (void)hipSetDevice(cur);
    CVSA_REQUIRE(e == hipSuccess && ptr != nullptr, CVSA_ERR_LAUNCH,
                 "sparse_decode_noalloc: scratch set-up on device %d failed: %s", dev,
                 hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return CVSA_OK;
}

extern "C" int cvsa_sparse_decode_noalloc(
    const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t *k_cache,
    const uint16_t *v_cache, int64_t num_blocks, const int32_t *block_tables,
    int64_t bt_stride_b, const int32_t *context_lens, const int32_t *page_indices,
    int64_t idx_stride, const int32_t *n_per_head, int32_t max_selected, int32_t B,
    int32_t H_q, int32_t H_kv, int32_t D, int32_t block_size, int32_t W, float *o_unnorm,
    float *m_out, float *l_out, void *out, int32_t out_dtype, int64_t *work, void *stream) {
  const char *name = "sparse_decode_noalloc";
  DecodeArgs a = base_args(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                           block_tables, bt_stride_b, context_lens, o_unnorm, m_out, l_out,
                           out, out_dtype, work);
  a.page_idx = page_indices;
  a.idx_stride = idx_stride;
  a.max_sel = max_selected;
  a.n_pages = n_per_head;
  if (page_indices == nullptr)
    return cvsa_host::fail(CVSA_ERR_INVALID, "%s: page_indices is NULL", name);
  DecodeLaunch p{};
  size_t need = 0;
  const int rc = validate_decode(name, a, B, H_q, H_kv, D, block_size, W, true, false, p, need);
  if (rc != CVSA_OK) return rc;
  CVSA_REQUIRE(need <= kScratchBytes, CVSA_ERR_WORKSPACE,
               "%s: the launch needs %zu bytes of scratch, more than the %zu-byte static "
               "scratch; use cvsa_sparse_decode with a workspace",
               name, need, kScratchBytes);
  void *ws = nullptr;
  if (need > 0) {
    const int src = scratch_for((hipStream_t)stream, &ws);
    if (src != CVSA_OK) return src;
  }
  return enqueue_decode(name, a, H_q / H_kv, true, p, ws, need, (hipStream_t)stream);
}

namespace cvsa_internal {

bool score_spec_fusable(int32_t H_kv, int32_t D, int32_t G) {
  return D == 128 && H_kv >= 4 && H_kv % 4 == 0 && H_kv <= 16 && G >= 1 && G <= kMaxGroup;
}

// A lazy check's page scoring (cvsa_score_pages into page_scores) fused
// with the speculative decode of its cached selection (cvsa_sparse_decode
// into out, run only if spec_state[0] predicts that the check keeps the
// selection; spec_state[1] records whether it ran).  Effective-budget
// counters are left to the verified decode.  H_kv must be 4, 8 or 16.
// With sel_map (the selection's map, select_for_plan) and 16-token pages,
// a speculative decode also scores the pages it walks, from the keys it
// reads anyway, and the scoring part skips them: the selection's keys are
// read once instead of twice, and the scores keep their bits.
int score_and_speculate(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                        const uint16_t *k_cache, const uint16_t *v_cache, int64_t num_blocks,
                        const int32_t *block_tables, int64_t bt_stride_b,
                        const int32_t *context_lens, const int32_t *page_indices,
                        int64_t idx_stride, const int32_t *n_per_head, int32_t max_selected,
                        int32_t B, int32_t H_q, int32_t H_kv, int32_t D, int32_t block_size,
                        int32_t W, float *page_scores, void *out, int32_t out_dtype,
                        int32_t *spec_state, const uint8_t *sel_map, int64_t sel_map_stride,
                        void *workspace, size_t workspace_bytes, void *stream) {
  const char *name = "score_pages + speculative decode";
  DecodeArgs a = base_args(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                           block_tables, bt_stride_b, context_lens, nullptr, nullptr, nullptr,
                           out, out_dtype, nullptr);
  a.page_idx = page_indices;
  a.idx_stride = idx_stride;
  a.max_sel = max_selected;
  a.n_pages = n_per_head;
  a.spec_state = spec_state;
  CVSA_REQUIRE(page_indices && spec_state && page_scores, CVSA_ERR_INVALID,
               "%s: page_indices, spec_state and page_scores are required", name);
  CVSA_REQUIRE(H_kv > 0 && H_q % H_kv == 0 && score_spec_fusable(H_kv, D, H_q / H_kv) &&
                   block_size != 8,
               CVSA_ERR_UNSUPPORTED,
               "%s: H_kv=%d not in {4,8,16}, D=%d not 128, G > %d or 8-token pages", name,
               H_kv, D, kMaxGroup);
  DecodeLaunch p{};
  size_t need = 0;
  int rc = validate_decode(name, a, B, H_q, H_kv, D, block_size, W, true, false, p, need);
  if (rc != CVSA_OK) return rc;
  // The speculative dense decode walks the identity partition (a listed
  // walk of a W-page list), as a verified launch whose heads are all
  // rejected does.
  const DecodeLaunch ip = plan_launch(B, H_kv, W, W, true, false);
  a.pps_all = ip.pps << a.ts;
  a.n_splits_all = ip.n_splits;
  const size_t need_ident = workspace_bytes_for(B, H_q, H_kv, D, W, W, true, false);
  if (need_ident > need) need = need_ident;
  if ((rc = check_workspace(name, workspace, workspace_bytes, need)) != CVSA_OK) return rc;
  bind_workspace(a, workspace, need);
  const int G = H_q / H_kv;
  ScoreArgs sa{q, q_stride_b, q_stride_h, k_cache, num_blocks, block_tables,
               bt_stride_b, context_lens, page_scores, W, G, 1.0f / (float)G, a.scale,
               block_size, a.ts};
  if (sel_map != nullptr && a.ts == 0) {
    CVSA_REQUIRE(sel_map_stride >= W && sel_map_stride % 16 == 0 &&
                     ((uintptr_t)sel_map & 15) == 0,
                 CVSA_ERR_INVALID, "%s: selection map rows of %lld bytes", name,
                 (long long)sel_map_stride);
    sa.skip_map = sel_map;
    sa.skip_stride = sel_map_stride;
    a.spec_scores = page_scores;
    a.inv_g = sa.inv_g;
  }
  static_assert(kSpecScorePPW % 8 == 0, "a scoring wave holds whole pages of up to 8 tiles");
  // 16-token pages: a wave per head and kSpecHeadPPW pages; else a wave per
  // 4 heads and kSpecScorePPW tiles.
  const int64_t waves =
      a.ts == 0 ? (int64_t)((W + kSpecHeadPPW - 1) / kSpecHeadPPW) * H_kv
                : (int64_t)(((W << a.ts) + kSpecScorePPW - 1) / kSpecScorePPW) * (H_kv / 4);
  const int score_gx = (int)((waves + kWavesPerWg - 1) / kWavesPerWg);
  const int64_t n_dec = (int64_t)max(p.grid_x * p.grid_y, ip.grid_x * ip.grid_y);
  const int64_t grid = n_dec + (int64_t)score_gx * B;
  hipStream_t st = (hipStream_t)stream;
  switch (G) {
#define CVSA_SPEC_CASE(GG)                                                \
  case GG:                                                                \
    launch_spec_g<GG>(a, sa, score_gx, dim3((unsigned)grid), st);          \
    break;
    CVSA_SPEC_CASE(1) CVSA_SPEC_CASE(2) CVSA_SPEC_CASE(3) CVSA_SPEC_CASE(4)
    CVSA_SPEC_CASE(5) CVSA_SPEC_CASE(6) CVSA_SPEC_CASE(7) CVSA_SPEC_CASE(8)
    CVSA_SPEC_CASE(9) CVSA_SPEC_CASE(10) CVSA_SPEC_CASE(11) CVSA_SPEC_CASE(12)
    CVSA_SPEC_CASE(13) CVSA_SPEC_CASE(14) CVSA_SPEC_CASE(15) CVSA_SPEC_CASE(16)
#undef CVSA_SPEC_CASE
    default:
      break;
  }
  return cvsa_host::check_launch(name);
}

// cvsa_verified_decode after score_and_speculate and the check's
// select-or-keep: when the check kept its selection (spec_state[0]) and the
// speculative decode wrote the outputs (spec_state[1]), the launch only
// books the effective-budget counters.
int verified_decode_after_speculation(
    const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t *k_cache,
    const uint16_t *v_cache, int64_t num_blocks, const int32_t *block_tables,
    int64_t bt_stride_b, const int32_t *context_lens, const int32_t *page_indices,
    int64_t idx_stride, const int32_t *n_per_head, int32_t max_selected, const uint8_t *accept,
    const int32_t *exp_indices, int64_t exp_stride, int32_t exp_budget, int32_t B, int32_t H_q,
    int32_t H_kv, int32_t D, int32_t block_size, int32_t W, void *out, int32_t out_dtype,
    int64_t *work, int32_t *spec_state, void *workspace, size_t workspace_bytes,
    void *stream) {
  DecodeArgs a = base_args(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                           block_tables, bt_stride_b, context_lens, nullptr, nullptr, nullptr,
                           out, out_dtype, work);
  a.page_idx = page_indices;
  a.idx_stride = idx_stride;
  a.max_sel = max_selected;
  a.n_pages = n_per_head;
  a.accept = accept;
  a.spec_state = spec_state;
  a.alt_idx = exp_indices;
  a.alt_stride = exp_stride;
  a.alt_budget = exp_budget;
  CVSA_REQUIRE(page_indices && accept, CVSA_ERR_INVALID,
               "verified decode: page_indices and accept are required");
  return launch_decode("verified_decode", a, B, H_q, H_kv, D, block_size, W, true, true,
                       workspace, workspace_bytes, (hipStream_t)stream);
}

}  // namespace cvsa_internal

extern "C" int cvsa_dense_decode(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                                 const uint16_t *k_cache, const uint16_t *v_cache,
                                 int64_t num_blocks, const int32_t *block_tables,
                                 int64_t bt_stride_b, const int32_t *context_lens, int32_t B,
                                 int32_t H_q, int32_t H_kv, int32_t D, int32_t block_size,
                                 int32_t W, float *o_unnorm, float *m_out, float *l_out,
                                 void *out, int32_t out_dtype, int64_t *work,
                                 void *workspace, size_t workspace_bytes, void *stream) {
  DecodeArgs a = base_args(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                           block_tables, bt_stride_b, context_lens, o_unnorm, m_out, l_out,
                           out, out_dtype, work);
  return launch_decode("dense_decode", a, B, H_q, H_kv, D, block_size, W, false, true,
                       workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int cvsa_verified_decode(const uint16_t *q, int64_t q_stride_b,
                                    int64_t q_stride_h, const uint16_t *k_cache,
                                    const uint16_t *v_cache, int64_t num_blocks,
                                    const int32_t *block_tables, int64_t bt_stride_b,
                                    const int32_t *context_lens,
                                    const int32_t *page_indices, int64_t idx_stride,
                                    const int32_t *n_per_head, int32_t max_selected,
                                    const uint8_t *accept, int32_t B, int32_t H_q,
                                    int32_t H_kv, int32_t D, int32_t block_size, int32_t W,
                                    float *o_unnorm, float *m_out, float *l_out, void *out,
                                    int32_t out_dtype, int64_t *work, void *workspace,
                                    size_t workspace_bytes, void *stream) {
  DecodeArgs a = base_args(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                           block_tables, bt_stride_b, context_lens, o_unnorm, m_out, l_out,
                           out, out_dtype, work);
  a.page_idx = page_indices;
  a.idx_stride = idx_stride;
  a.max_sel = max_selected;
  a.n_pages = n_per_head;
  a.accept = accept;
  if (page_indices == nullptr || accept == nullptr)
    return cvsa_host::fail(CVSA_ERR_INVALID,
                           "verified_decode: page_indices and accept are required");
  return launch_decode("verified_decode", a, B, H_q, H_kv, D, block_size, W, true, true,
                       workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int cvsa_verified_decode_approx(
    const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h, const uint16_t *k_cache,
    const uint16_t *v_cache, int64_t num_blocks, const int32_t *block_tables,
    int64_t bt_stride_b, const int32_t *context_lens, const int32_t *page_indices,
    int64_t idx_stride, const int32_t *n_per_head, int32_t max_selected, const uint8_t *accept,
    const int32_t *exp_indices, int64_t exp_stride, int32_t exp_budget, int32_t B, int32_t H_q,
    int32_t H_kv, int32_t D, int32_t block_size, int32_t W, float *o_unnorm, float *m_out,
    float *l_out, void *out, int32_t out_dtype, int64_t *work, void *workspace,
    size_t workspace_bytes, void *stream) {
  DecodeArgs a = base_args(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                           block_tables, bt_stride_b, context_lens, o_unnorm, m_out, l_out,
                           out, out_dtype, work);
  a.page_idx = page_indices;
  a.idx_stride = idx_stride;
  a.max_sel = max_selected;
  a.n_pages = n_per_head;
  a.accept = accept;
  a.alt_idx = exp_indices;
  a.alt_stride = exp_stride;
  a.alt_budget = exp_budget;
  if (page_indices == nullptr || accept == nullptr || exp_indices == nullptr)
    return cvsa_host::fail(CVSA_ERR_INVALID,
                           "verified_decode_approx: page_indices, accept and exp_indices are "
                           "required");
  return launch_decode("verified_decode_approx", a, B, H_q, H_kv, D, block_size, W, true, true,
                       workspace, workspace_bytes, (hipStream_t)stream);
}
