// Quest page metadata and scores.
//
// CVSABackend._quest_page_scores (cvsa/backend.py:572-620) ranks pages by
// the Quest bound  sum_d max(q_d * kmin_d, q_d * kmax_d) * D^-0.5,  with
// kmin / kmax the per-dimension extremes of the page's keys over its valid
// tokens and q the bf16 group mean of the query heads; pages without a valid
// token score -inf.  The reference gathers every page's keys on every call.
// Here the extremes are kept as page metadata (as the reference's Quest
// baseline does, eval/baselines.py:77-140) and refreshed only for the pages
// that gained tokens, so a scoring pass reads 512 B per page and head
// instead of the 4 KiB of keys.
//
// Metadata layout: meta[block][h][0][d] = kmin, meta[block][h][1][d] = kmax,
// bf16 (exact: they are key values), indexed by physical block.
#include "cvsa_common.h"

namespace cvsa {

constexpr int kQuestPagesPerWave = 4;  // a wave scores 4 pages per step: 16 lanes each

// One wave per (page, kv-head): lane l owns dimensions 2l, 2l+1 of the
// page's valid token rows (each load instruction reads one whole 256-byte
// row), and writes their min and max.
__global__ __launch_bounds__(256) void quest_meta_kernel(
    const uint16_t *__restrict__ k_cache, int64_t num_blocks,
    const int32_t *__restrict__ block_tables, int64_t bt_sb,
    const int32_t *__restrict__ context_lens, const int32_t *__restrict__ seen_lens,
    int32_t *__restrict__ seen_out, int H_kv, int W, uint16_t *__restrict__ meta) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bh = blockIdx.y;
  const int b = bh / H_kv;
  const int h = bh - b * H_kv;
  const int ctx = __builtin_amdgcn_readfirstlane(context_lens[b]);
  const int seen = __builtin_amdgcn_readfirstlane(seen_lens[b]);
  if (seen_out != nullptr && h == 0 && blockIdx.x == 0 && threadIdx.x == 0) seen_out[b] = ctx;
  if (ctx <= 0 || ctx == seen) return;
  // Pages holding positions [seen, ctx); all pages when the context shrank.
  const int p_lo = ctx > seen ? seen / kPageTokens : 0;
  const int p_hi = min((ctx - 1) / kPageTokens, W - 1);
  const int stride = gridDim.x * 4;
  const int64_t row_stride = (int64_t)H_kv * kHeadDim;                 // between tokens
  const int64_t page_elems = (int64_t)kPageTokens * row_stride;       // between blocks
  for (int p = p_lo + blockIdx.x * 4 + wave; p <= p_hi; p += stride) {
    const int phys = __builtin_amdgcn_readfirstlane(block_tables[b * bt_sb + p]);
    if (phys < 0 || phys >= num_blocks) continue;  // uniform
    const int ntok = min(kPageTokens, ctx - p * kPageTokens);
    const uint32_t *src = reinterpret_cast<const uint32_t *>(
        k_cache + (int64_t)phys * page_elems + (int64_t)h * kHeadDim) + lane;
    uint32_t w[kPageTokens];
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t)
      w[t] = src[(int64_t)min(t, ntok - 1) * (row_stride / 2)];
    float lo0 = bf16_lo(w[0]), hi0 = lo0, lo1 = bf16_hi(w[0]), hi1 = lo1;
#pragma unroll
    for (int t = 1; t < kPageTokens; ++t) {
      const float x0 = bf16_lo(w[t]), x1 = bf16_hi(w[t]);
      lo0 = fminf(lo0, x0);
      hi0 = fmaxf(hi0, x0);
      lo1 = fminf(lo1, x1);
      hi1 = fmaxf(hi1, x1);
    }
    // The extremes are key values, so their top 16 bits are the bf16 bits.
    uint32_t *dst = reinterpret_cast<uint32_t *>(meta + ((int64_t)phys * H_kv + h) * 2 * kHeadDim);
    dst[lane] = (__float_as_uint(lo0) >> 16) | (__float_as_uint(lo1) & 0xffff0000u);
    dst[kHeadDim / 2 + lane] = (__float_as_uint(hi0) >> 16) | (__float_as_uint(hi1) & 0xffff0000u);
  }
}

// One wave per (b, kv-head, run of pages): lanes 16j .. 16j+15 take page j
// of each group of four, lane seg = l % 16 holds dimensions 8seg .. 8seg+7
// (16 bytes of kmin and 16 of kmax, read whole by the 16 lanes) and q_rep's
// matching segment; the 16-lane sum is formed with DPP.
__global__ __launch_bounds__(256) void quest_scores_kernel(
    const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh,
    const uint16_t *__restrict__ meta, int64_t num_blocks,
    const int32_t *__restrict__ block_tables, int64_t bt_sb,
    const int32_t *__restrict__ context_lens, int H_kv, int G, float inv_g, float scale,
    int W, int ppw, float *__restrict__ scores) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bh = blockIdx.y;
  const int b = bh / H_kv;
  const int h = bh - b * H_kv;
  const int p0 = (blockIdx.x * 4 + wave) * ppw;
  if (p0 >= W) return;
  const int seg = lane & 15;
  const int sub = lane >> 4;
  const int ctx = __builtin_amdgcn_readfirstlane(context_lens[b]);
  const uint4 qv = group_mean_q(q, q_sb, q_sh, b, h, G, seg, inv_g);
  float qf[8];
  qf[0] = bf16_lo(qv.x); qf[1] = bf16_hi(qv.x);
  qf[2] = bf16_lo(qv.y); qf[3] = bf16_hi(qv.y);
  qf[4] = bf16_lo(qv.z); qf[5] = bf16_hi(qv.z);
  qf[6] = bf16_lo(qv.w); qf[7] = bf16_hi(qv.w);
  float *out = scores + (int64_t)bh * W;
  const int p_end = min(W, p0 + ppw);
  for (int pb = p0; pb < p_end; pb += kQuestPagesPerWave) {
    const int p = pb + sub;
    const bool in_row = p < p_end;
    const int pc = in_row ? p : p_end - 1;
    const int phys = block_tables[b * bt_sb + pc];
    const bool valid = in_row && pc * kPageTokens < ctx && phys >= 0 && phys < num_blocks;
    const uint16_t *m = meta + ((int64_t)(valid ? phys : 0) * H_kv + h) * 2 * kHeadDim + 8 * seg;
    const uint4 mn = *reinterpret_cast<const uint4 *>(m);
    const uint4 mx = *reinterpret_cast<const uint4 *>(m + kHeadDim);
    const uint32_t lo[4] = {mn.x, mn.y, mn.z, mn.w};
    const uint32_t hi[4] = {mx.x, mx.y, mx.z, mx.w};
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc += fmaxf(qf[2 * i] * bf16_lo(lo[i]), qf[2 * i] * bf16_lo(hi[i]));
      acc += fmaxf(qf[2 * i + 1] * bf16_hi(lo[i]), qf[2 * i + 1] * bf16_hi(hi[i]));
    }
    acc = group_sum<16>(acc) * scale;
    if (seg == 0 && in_row) out[p] = valid ? acc : -INFINITY;
  }
}

}  // namespace cvsa

using namespace cvsa;

extern "C" int cvsa_quest_meta_update(const uint16_t *k_cache, int64_t num_blocks,
                                      const int32_t *block_tables, int64_t bt_stride_b,
                                      const int32_t *context_lens, const int32_t *seen_lens,
                                      int32_t *seen_out, int32_t B, int32_t H_kv, int32_t D,
                                      int32_t block_size, int32_t W, int32_t all_pages,
                                      uint16_t *meta, void *stream) {
  CVSA_REQUIRE(k_cache && block_tables && context_lens && seen_lens && meta, CVSA_ERR_INVALID,
               "quest_meta_update: null pointer argument");
  CVSA_REQUIRE((const void *)seen_out != (const void *)seen_lens, CVSA_ERR_INVALID,
               "quest_meta_update: seen_out must not alias seen_lens");
  CVSA_REQUIRE(B > 0 && B <= 65535 && H_kv > 0 && (int64_t)B * H_kv <= 65535 && W > 0 &&
                   num_blocks > 0,
               CVSA_ERR_INVALID, "quest_meta_update: bad sizes B=%d H_kv=%d W=%d", B, H_kv, W);
  CVSA_REQUIRE(D == kHeadDim && block_size == kPageTokens, CVSA_ERR_UNSUPPORTED,
               "quest_meta_update: only D=128, block_size=16 are supported (got D=%d, bs=%d)",
               D, block_size);
  CVSA_REQUIRE(bt_stride_b >= W, CVSA_ERR_INVALID,
               "quest_meta_update: block-table row stride %lld < W=%d", (long long)bt_stride_b,
               W);
  CVSA_REQUIRE(((uintptr_t)k_cache & 3) == 0 && ((uintptr_t)meta & 15) == 0, CVSA_ERR_INVALID,
               "quest_meta_update: k_cache must be 4-byte and meta 16-byte aligned");
  // all_pages: a workgroup (4 waves) per 4 pages of every row, for a first
  // build; otherwise one workgroup per (b, kv-head) walks its new pages.
  const int chunks = all_pages ? (W + 3) / 4 : 1;
  hipLaunchKernelGGL(quest_meta_kernel, dim3(chunks, B * H_kv), dim3(256), 0,
                     (hipStream_t)stream, k_cache, num_blocks, block_tables, bt_stride_b,
                     context_lens, seen_lens, seen_out, H_kv, W, meta);
  return cvsa_host::check_launch("quest_meta_update");
}

extern "C" int cvsa_quest_scores(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                                 const uint16_t *meta, int64_t num_blocks,
                                 const int32_t *block_tables, int64_t bt_stride_b,
                                 const int32_t *context_lens, int32_t B, int32_t H_q,
                                 int32_t H_kv, int32_t D, int32_t block_size, int32_t W,
                                 float *page_scores, void *stream) {
  CVSA_REQUIRE(q && meta && block_tables && context_lens && page_scores, CVSA_ERR_INVALID,
               "quest_scores: null pointer argument");
  CVSA_REQUIRE(B > 0 && H_kv > 0 && (int64_t)B * H_kv <= 65535 && W > 0 && num_blocks > 0,
               CVSA_ERR_INVALID, "quest_scores: bad sizes B=%d H_kv=%d W=%d", B, H_kv, W);
  CVSA_REQUIRE(H_q > 0 && H_q % H_kv == 0, CVSA_ERR_INVALID,
               "quest_scores: H_q=%d is not a multiple of H_kv=%d", H_q, H_kv);
  CVSA_REQUIRE(D == kHeadDim && block_size == kPageTokens, CVSA_ERR_UNSUPPORTED,
               "quest_scores: only D=128, block_size=16 are supported (got D=%d, bs=%d)", D,
               block_size);
  CVSA_REQUIRE(W <= kMaxPages, CVSA_ERR_UNSUPPORTED, "quest_scores: W=%d exceeds %d pages", W,
               kMaxPages);
  CVSA_REQUIRE(bt_stride_b >= W, CVSA_ERR_INVALID,
               "quest_scores: block-table row stride %lld < W=%d", (long long)bt_stride_b, W);
  CVSA_REQUIRE(((uintptr_t)q & 15) == 0 && q_stride_b % 8 == 0 && q_stride_h % 8 == 0 &&
                   ((uintptr_t)meta & 15) == 0,
               CVSA_ERR_INVALID,
               "quest_scores: q / meta must be 16-byte aligned with q strides that are "
               "multiples of 8 elements");
  const int G = H_q / H_kv;
  // Pages per wave: as many (up to 64) as keep >= ~2048 waves in the launch.
  const int64_t rows = (int64_t)B * H_kv;
  int ppw = kQuestPagesPerWave;
  while (ppw < 64 && rows * W / (2 * ppw) >= 2048) ppw *= 2;
  const int waves = (W + ppw - 1) / ppw;
  hipLaunchKernelGGL(quest_scores_kernel, dim3((waves + 3) / 4, B * H_kv), dim3(256), 0,
                     (hipStream_t)stream, q, q_stride_b, q_stride_h, meta, num_blocks,
                     block_tables, bt_stride_b, context_lens, H_kv, G, 1.0f / (float)G,
                     (float)pow((double)D, -0.5), W, ppw, page_scores);
  return cvsa_host::check_launch("quest_scores");
}
