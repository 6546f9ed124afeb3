// Quest page metadata and scores.
//
// CVSABackend._quest_page_scores (cvsa/backend.py:572-620) ranks pages by
// the Quest bound  sum_d max(q_d * kmin_d, q_d * kmax_d) * D^-0.5,  with
// kmin / kmax the per-dimension extremes of the page's keys over its valid
// tokens and q the bf16 group mean of the query heads; pages without a valid
// token score -inf.  The reference gathers every page's keys on every call.
// Here the extremes are kept as page metadata (as the reference's Quest
// baseline does, eval/baselines.py:77-140) and refreshed only for the pages
// whose valid-token count changed, so a scoring pass reads 4D bytes per page
// and head (512 B at D = 128) instead of the 32D bytes of keys.
//
// Metadata layout: meta[block][h][0][d] = kmin, meta[block][h][1][d] = kmax,
// bf16 (exact: they are key values), indexed by physical block;
// meta_ntok[block][h] int32 = the number of leading tokens of the block the
// extremes cover (0: none).  A page is recomputed when its valid-token count
// under the current context differs from meta_ntok, by the wave that scores
// it, which also writes the new count.
#include "cvsa_common.h"

namespace cvsa {

// Extremes of 8 dimensions (one 16-byte segment) of a page's ntok >= 1
// valid token rows, packed as bf16 like the metadata.  Rows are read 16 at a
// time (rows past the last valid one repeat it).
__device__ __forceinline__ void segment_minmax(const uint16_t *__restrict__ rows,
                                               int64_t row_stride, int ntok, uint4 &mn,
                                               uint4 &mx) {
  float lo[8], hi[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    lo[e] = INFINITY;
    hi[e] = -INFINITY;
  }
  for (int t0 = 0; t0 < ntok; t0 += kPageTokens) {
    uint4 r[kPageTokens];
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t)
      r[t] = *reinterpret_cast<const uint4 *>(rows + (int64_t)min(t0 + t, ntok - 1) * row_stride);
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t) {
      const uint32_t w[4] = {r[t].x, r[t].y, r[t].z, r[t].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        lo[2 * i] = fminf(lo[2 * i], bf16_lo(w[i]));
        hi[2 * i] = fmaxf(hi[2 * i], bf16_lo(w[i]));
        lo[2 * i + 1] = fminf(lo[2 * i + 1], bf16_hi(w[i]));
        hi[2 * i + 1] = fmaxf(hi[2 * i + 1], bf16_hi(w[i]));
      }
    }
  }
  // The extremes are key values, so their top 16 bits are the bf16 bits.
  auto pack = [](float a, float b) {
    return (__float_as_uint(a) >> 16) | (__float_as_uint(b) & 0xffff0000u);
  };
  mn = make_uint4(pack(lo[0], lo[1]), pack(lo[2], lo[3]), pack(lo[4], lo[5]), pack(lo[6], lo[7]));
  mx = make_uint4(pack(hi[0], hi[1]), pack(hi[2], hi[3]), pack(hi[4], hi[5]), pack(hi[6], hi[7]));
}

// One wave per (b, kv-head, run of ppw pages, a multiple of 16), LPR = D / 8
// lanes per page: lanes LPR*j .. LPR*j+LPR-1 take page j of each group of
// RPL = 64 / LPR pages (8, 4, 2 at D = 64, 128, 256); lane seg = l % LPR
// holds dimensions 8seg .. 8seg+7 (16 bytes of kmin and 16 of kmax, read
// whole by the LPR lanes) and q_rep's matching segment; the LPR-lane sum is
// formed with DPP (and a permlane swap at LPR = 32).  Sixteen pages are in
// flight per wave: their block-table entries are read first, then their
// metadata, so each run of 16 pays two load latencies.
//
// REFRESH: pages whose valid-token count differs from meta_ntok are
// recomputed from k_cache, written back (extremes and count) and scored
// from the new values.  SCORE: write the scores (else only refresh).
// check_accept (optional, n_heads flags): when every flag is set the
// launch does nothing; a lazy check that kept its selection needs no
// ranking scores.
template <int D, bool REFRESH, bool SCORE>
__global__ __launch_bounds__(256) void quest_scores_kernel(
    const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh, uint16_t *__restrict__ meta,
    int32_t *__restrict__ meta_ntok, int64_t num_blocks,
    const int32_t *__restrict__ block_tables, int64_t bt_sb,
    const int32_t *__restrict__ context_lens, const uint16_t *__restrict__ k_cache,
    const uint8_t *__restrict__ check_accept, int n_heads, int H_kv, int G, float inv_g,
    float scale, int W, int ppw, int bs, float *__restrict__ scores) {
  constexpr int LPR = D / 8;
  constexpr int RPL = kWave / LPR;  // pages per wave load
  constexpr int kIter = 16 / RPL;   // wave loads per run of sixteen pages
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bh = blockIdx.y;
  const int b = bh / H_kv;
  const int h = bh - b * H_kv;
  const int p0 = (blockIdx.x * 4 + wave) * ppw;
  if (p0 >= W) return;
  const int seg = lane % LPR;
  const int sub = lane / LPR;
  const int p_end = min(W, p0 + ppw);
  // Block-table entries of the next run of 16 pages: the first run's are
  // requested before the check flags and the query rows, so their
  // latencies overlap.
  int phys[kIter];
  auto load_phys = [&](int pb) {
#pragma unroll
    for (int i = 0; i < kIter; ++i)
      phys[i] = block_tables[b * bt_sb + min(pb + RPL * i + sub, p_end - 1)];
  };
  load_phys(p0);
  if (check_accept != nullptr) {
    int bad = 0;
    for (int i = lane; i < n_heads; i += 64) bad |= check_accept[i] == 0;
    if (__ballot(bad) == 0) return;
  }
  const int ctx = __builtin_amdgcn_readfirstlane(context_lens[b]);
  float qf[8];
  if (SCORE) {
    const uint4 qv = group_mean_q(q, q_sb, q_sh, b, h, G, seg, inv_g);
    qf[0] = bf16_lo(qv.x); qf[1] = bf16_hi(qv.x);
    qf[2] = bf16_lo(qv.y); qf[3] = bf16_hi(qv.y);
    qf[4] = bf16_lo(qv.z); qf[5] = bf16_hi(qv.z);
    qf[6] = bf16_lo(qv.w); qf[7] = bf16_hi(qv.w);
  }
  const int64_t row_stride = (int64_t)H_kv * D;  // between tokens of a block
  for (int pb = p0; pb < p_end; pb += kIter * RPL) {
    bool valid[kIter];
#pragma unroll
    for (int i = 0; i < kIter; ++i) {
      const int p = pb + RPL * i + sub;
      valid[i] = p < p_end && p * bs < ctx && phys[i] >= 0 && phys[i] < num_blocks;
    }
    uint4 mn[kIter], mx[kIter];
    int have[kIter];
#pragma unroll
    for (int i = 0; i < kIter; ++i) {
      const int64_t slot = (int64_t)(valid[i] ? phys[i] : 0) * H_kv + h;
      if (SCORE) {
        const uint16_t *m = meta + slot * 2 * D + 8 * seg;
        mn[i] = *reinterpret_cast<const uint4 *>(m);
        mx[i] = *reinterpret_cast<const uint4 *>(m + D);
      }
      if (REFRESH) have[i] = meta_ntok[slot];
    }
    int cur[kIter];
#pragma unroll
    for (int i = 0; i < kIter; ++i) cur[i] = phys[i];
    if (pb + kIter * RPL < p_end) load_phys(pb + kIter * RPL);
    if (REFRESH) {
#pragma unroll
      for (int i = 0; i < kIter; ++i) {
        const int p = pb + RPL * i + sub;
        const int ntok = min(bs, ctx - p * bs);
        if (valid[i] && have[i] != ntok) {
          const int64_t slot = (int64_t)cur[i] * H_kv + h;
          segment_minmax(k_cache + (int64_t)cur[i] * bs * row_stride +
                             (int64_t)h * D + 8 * seg,
                         row_stride, ntok, mn[i], mx[i]);
          uint16_t *m = meta + slot * 2 * D + 8 * seg;
          *reinterpret_cast<uint4 *>(m) = mn[i];
          *reinterpret_cast<uint4 *>(m + D) = mx[i];
          if (seg == 0) meta_ntok[slot] = ntok;
        }
      }
    }
    if (SCORE) {
      float *out = scores + (int64_t)bh * W;
#pragma unroll
      for (int i = 0; i < kIter; ++i) {
        const int p = pb + RPL * i + sub;
        const uint32_t lo[4] = {mn[i].x, mn[i].y, mn[i].z, mn[i].w};
        const uint32_t hi[4] = {mx[i].x, mx[i].y, mx[i].z, mx[i].w};
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc += fmaxf(qf[2 * e] * bf16_lo(lo[e]), qf[2 * e] * bf16_lo(hi[e]));
          acc += fmaxf(qf[2 * e + 1] * bf16_hi(lo[e]), qf[2 * e + 1] * bf16_hi(hi[e]));
        }
        acc = group_sum<LPR>(acc) * scale;
        if (seg == 0 && p < p_end) out[p] = valid[i] ? acc : -INFINITY;
      }
    }
  }
}

}  // namespace cvsa

using namespace cvsa;

namespace {

// Pages per wave: 16, or up to 64 while >= 4096 waves remain in the launch.
dim3 quest_grid(int B, int H_kv, int W, int &ppw) {
  const int64_t rows = (int64_t)B * H_kv;
  ppw = 16;
  while (ppw < 64 && rows * W / (2 * ppw) >= 4096) ppw *= 2;
  const int waves = (W + ppw - 1) / ppw;
  return dim3((waves + 3) / 4, B * H_kv);
}

int check_quest_sizes(const char *name, int32_t B, int32_t H_kv, int32_t D, int32_t block_size,
                      int32_t W, int64_t num_blocks, int64_t bt_stride_b, const void *meta) {
  CVSA_REQUIRE(B > 0 && H_kv > 0 && (int64_t)B * H_kv <= 65535 && W > 0 && num_blocks > 0,
               CVSA_ERR_INVALID, "%s: bad sizes B=%d H_kv=%d W=%d", name, B, H_kv, W);
  CVSA_REQUIRE(head_dim_supported(D) && block_size_supported(block_size), CVSA_ERR_UNSUPPORTED,
               "%s: D=%d not in {32, 64, 128, 256} or block_size=%d not in {8, 16, 32, 64, 128}", name, D,
               block_size);
  CVSA_REQUIRE(W <= kMaxPagesWide, CVSA_ERR_UNSUPPORTED, "%s: W=%d exceeds %d pages", name,
               W, kMaxPagesWide);
  CVSA_REQUIRE(bt_stride_b >= W, CVSA_ERR_INVALID, "%s: block-table row stride %lld < W=%d",
               name, (long long)bt_stride_b, W);
  CVSA_REQUIRE(((uintptr_t)meta & 15) == 0, CVSA_ERR_INVALID, "%s: meta must be 16-byte aligned",
               name);
  return CVSA_OK;
}

int check_quest_q(const char *name, const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                  int32_t H_q, int32_t H_kv) {
  CVSA_REQUIRE(H_q > 0 && H_q % H_kv == 0, CVSA_ERR_INVALID,
               "%s: H_q=%d is not a multiple of H_kv=%d", name, H_q, H_kv);
  CVSA_REQUIRE(((uintptr_t)q & 15) == 0 && q_stride_b % 8 == 0 && q_stride_h % 8 == 0,
               CVSA_ERR_INVALID,
               "%s: q must be 16-byte aligned with strides that are multiples of 8 elements",
               name);
  return CVSA_OK;
}

}  // namespace

extern "C" int cvsa_quest_meta_update(const uint16_t *k_cache, int64_t num_blocks,
                                      const int32_t *block_tables, int64_t bt_stride_b,
                                      const int32_t *context_lens, int32_t B, int32_t H_kv,
                                      int32_t D, int32_t block_size, int32_t W, uint16_t *meta,
                                      int32_t *meta_ntok, void *stream) {
  static const char *name = "quest_meta_update";
  CVSA_REQUIRE(k_cache && block_tables && context_lens && meta && meta_ntok, CVSA_ERR_INVALID,
               "%s: null pointer argument", name);
  int rc = check_quest_sizes(name, B, H_kv, D, block_size, W, num_blocks, bt_stride_b, meta);
  if (rc != CVSA_OK) return rc;
  CVSA_REQUIRE(((uintptr_t)k_cache & 15) == 0, CVSA_ERR_INVALID,
               "%s: k_cache must be 16-byte aligned", name);
  int ppw;
  const dim3 grid = quest_grid(B, H_kv, W, ppw);
#define CVSA_QUEST_REFRESH(DD)                                                               \
  hipLaunchKernelGGL((quest_scores_kernel<DD, true, false>), grid, dim3(256), 0,             \
                     (hipStream_t)stream, nullptr, 0, 0, meta, meta_ntok, num_blocks,        \
                     block_tables, bt_stride_b, context_lens, k_cache, nullptr, 0, H_kv, 1,  \
                     1.0f, 1.0f, W, ppw, block_size, nullptr)
  if (D == 32)
    CVSA_QUEST_REFRESH(32);
  else if (D == 64)
    CVSA_QUEST_REFRESH(64);
  else if (D == 256)
    CVSA_QUEST_REFRESH(256);
  else
    CVSA_QUEST_REFRESH(128);
#undef CVSA_QUEST_REFRESH
  return cvsa_host::check_launch(name);
}

extern "C" int cvsa_quest_scores(const uint16_t *q, int64_t q_stride_b, int64_t q_stride_h,
                                 const uint16_t *meta, int64_t num_blocks,
                                 const int32_t *block_tables, int64_t bt_stride_b,
                                 const int32_t *context_lens, int32_t B, int32_t H_q,
                                 int32_t H_kv, int32_t D, int32_t block_size, int32_t W,
                                 float *page_scores, void *stream) {
  static const char *name = "quest_scores";
  CVSA_REQUIRE(q && meta && block_tables && context_lens && page_scores, CVSA_ERR_INVALID,
               "%s: null pointer argument", name);
  int rc = check_quest_sizes(name, B, H_kv, D, block_size, W, num_blocks, bt_stride_b, meta);
  if (rc == CVSA_OK) rc = check_quest_q(name, q, q_stride_b, q_stride_h, H_q, H_kv);
  if (rc != CVSA_OK) return rc;
  const int G = H_q / H_kv;
  int ppw;
  const dim3 grid = quest_grid(B, H_kv, W, ppw);
  // Without refresh the kernel only reads the metadata.
  const float scale = (float)pow((double)D, -0.5);
#define CVSA_QUEST_SCORE(DD)                                                                 \
  hipLaunchKernelGGL((quest_scores_kernel<DD, false, true>), grid, dim3(256), 0,             \
                     (hipStream_t)stream, q, q_stride_b, q_stride_h,                         \
                     const_cast<uint16_t *>(meta), nullptr, num_blocks, block_tables,        \
                     bt_stride_b, context_lens, nullptr, nullptr, 0, H_kv, G,                \
                     1.0f / (float)G, scale, W, ppw, block_size, page_scores)
  if (D == 32)
    CVSA_QUEST_SCORE(32);
  else if (D == 64)
    CVSA_QUEST_SCORE(64);
  else if (D == 256)
    CVSA_QUEST_SCORE(256);
  else
    CVSA_QUEST_SCORE(128);
#undef CVSA_QUEST_SCORE
  return cvsa_host::check_launch(name);
}

extern "C" int cvsa_quest_refresh_scores(const uint16_t *q, int64_t q_stride_b,
                                         int64_t q_stride_h, const uint16_t *k_cache,
                                         int64_t num_blocks, const int32_t *block_tables,
                                         int64_t bt_stride_b, const int32_t *context_lens,
                                         const uint8_t *check_accept, int32_t B, int32_t H_q,
                                         int32_t H_kv, int32_t D, int32_t block_size, int32_t W,
                                         uint16_t *meta, int32_t *meta_ntok, float *page_scores,
                                         void *stream) {
  static const char *name = "quest_refresh_scores";
  CVSA_REQUIRE(q && k_cache && meta && meta_ntok && block_tables && context_lens && page_scores,
               CVSA_ERR_INVALID, "%s: null pointer argument", name);
  int rc = check_quest_sizes(name, B, H_kv, D, block_size, W, num_blocks, bt_stride_b, meta);
  if (rc == CVSA_OK) rc = check_quest_q(name, q, q_stride_b, q_stride_h, H_q, H_kv);
  if (rc != CVSA_OK) return rc;
  CVSA_REQUIRE(((uintptr_t)k_cache & 15) == 0, CVSA_ERR_INVALID,
               "%s: k_cache must be 16-byte aligned", name);
  const int G = H_q / H_kv;
  int ppw;
  const dim3 grid = quest_grid(B, H_kv, W, ppw);
  const float scale = (float)pow((double)D, -0.5);
#define CVSA_QUEST_BOTH(DD)                                                                   \
  hipLaunchKernelGGL((quest_scores_kernel<DD, true, true>), grid, dim3(256), 0,               \
                     (hipStream_t)stream, q, q_stride_b, q_stride_h, meta, meta_ntok,         \
                     num_blocks, block_tables, bt_stride_b, context_lens, k_cache,            \
                     check_accept, B * H_kv, H_kv, G, 1.0f / (float)G, scale, W, ppw,         \
                     block_size, page_scores)
  if (D == 32)
    CVSA_QUEST_BOTH(32);
  else if (D == 64)
    CVSA_QUEST_BOTH(64);
  else if (D == 256)
    CVSA_QUEST_BOTH(256);
  else
    CVSA_QUEST_BOTH(128);
#undef CVSA_QUEST_BOTH
  return cvsa_host::check_launch(name);
}
