// Page scoring: page_scores[b,h,p] = max over valid tokens of (q_rep . K) * D^-0.5.
//
// Follows triton_score_pages (cvsa/kernels/page_scores.py:77-119, kernel
// :12-74): q_rep is the bf16-rounded GQA group mean of q (:94-95), the dot is
// accumulated in fp32 and scaled after the sum (:67), masked tokens are -inf
// (:68) and pages starting at or beyond the context are -inf (:44-47).
//
// MI355X mapping: the reference runs one tiny program per (b, kv-head, page).
// Here a wave streams whole 1 KiB runs of a page: a page is block_size x H_kv
// rows of 2D bytes stored back to back (32 KiB for H_kv = 8, D = 128), so
// every 16-byte lane load is part of a fully coalesced 1 KiB wave load, and
// the D / 8 lanes that hold one (token, head) row reduce its dot product
// with DPP adds.
#include "cvsa_common.h"
#include "score_body.h"

namespace cvsa {

// Heads of one 1 KiB wave load at head dimension D: 64 / (D / 8).
constexpr int rows_per_load(int D) { return kWave / (D / 8); }

// H_kv a multiple of R = rows_per_load(D): a wave owns R KV heads of PPW
// pages (score_body.h).
template <int D, int HKV, int PPW>
__global__ __launch_bounds__(256) void score_pages_group_kernel(const ScoreArgs s) {
  static_assert(HKV % rows_per_load(D) == 0, "head-group layout");
  score_group_wave<D, PPW>(s, HKV, blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
                           blockIdx.y);
}

// H_kv < R: one wave streams a whole page; lane l covers row l / LPR of each
// group of R (token, head) rows and d-segment (l % LPR) * 8 (LPR = D / 8).
template <int D, int HKV>
__global__ __launch_bounds__(256) void score_pages_kernel(
    const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh,
    const uint16_t *__restrict__ k_cache, int64_t num_blocks,
    const int32_t *__restrict__ block_tables, int64_t bt_sb,
    const int32_t *__restrict__ context_lens, float *__restrict__ scores,
    int W, int G, float inv_g, float scale, int ppw, int bs, int ts) {
  constexpr int LPR = D / 8;
  constexpr int R = rows_per_load(D);
  static_assert(HKV < R && R % HKV == 0, "small-head layout");
  constexpr int NLOAD = kPageTokens * HKV / R;     // 16-byte loads per lane per tile
  constexpr int TILE_ELEMS = kPageTokens * HKV * D;
  constexpr int S = HKV * LPR;                     // lane distance between rows of one head

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rsub = lane / LPR;
  const int seg = lane % LPR;
  const int b = blockIdx.y;
  const int p_begin = (blockIdx.x * 4 + wave) * ppw;
  if (p_begin >= W) return;
  const int ctx = context_lens[b];
  const int h = rsub % HKV;
  const uint4 qr = group_mean_q(q, q_sb, q_sh, b, h, G, seg, inv_g);

  const int p_end = min(W, p_begin + ppw);
  for (int p = p_begin; p < p_end; ++p) {
    float *dst = scores + (int64_t)b * HKV * W + p;
    const int ntok = min(bs, ctx - p * bs);
    const int phys = ntok > 0 ? block_tables[b * bt_sb + p] : -1;
    if (phys < 0 || phys >= num_blocks) {
      // Beyond the context (or an out-of-range block id): no valid token.
      if (seg == 0 && rsub < HKV) dst[(int64_t)h * W] = -INFINITY;
      continue;
    }
    float mx = -INFINITY;
    for (int sub = 0; sub < (1 << ts); ++sub) {  // the page's 16-token tiles
      const uint16_t *src =
          k_cache + ((int64_t)phys << ts | sub) * TILE_ELEMS + lane * 8;
      uint4 kv[NLOAD];
#pragma unroll
      for (int i = 0; i < NLOAD; ++i) kv[i] = stream_load16(src + i * 64 * 8);
      const int tn = ntok - sub * kPageTokens;  // valid tokens of the tile (<= 0: none)
#pragma unroll
      for (int i = 0; i < NLOAD; ++i) {
        const int t = (i * R + rsub) / HKV;
        const float sc = group_sum<LPR>(dot8_bf16(kv[i], qr, 0.f)) * scale;
        if (t < tn) mx = fmaxf(mx, sc);
      }
    }
    // Rows of one head sit S lanes apart: combine them.
    float a, c;
    if constexpr (S <= 8) mx = fmaxf(mx, dpp_f<kDppRowRor8>(mx));
    if constexpr (S <= 16) {
      xchg16(mx, a, c);
      mx = fmaxf(a, c);
    }
    xchg32(mx, a, c);
    mx = fmaxf(a, c);
    // A zero score is written as +0, as by the group kernel.
    if (seg == 0 && rsub < HKV) dst[(int64_t)h * W] = mx + 0.f;
  }
}

}  // namespace cvsa

using namespace cvsa;

extern "C" int cvsa_score_pages(const uint16_t *q, int64_t q_stride_b,
                                int64_t q_stride_h, const uint16_t *k_cache,
                                int64_t num_blocks,
                                const int32_t *block_tables,
                                int64_t bt_stride_b,
                                const int32_t *context_lens, int32_t B,
                                int32_t H_q, int32_t H_kv, int32_t D,
                                int32_t block_size, int32_t W,
                                float *page_scores, void *stream) {
  CVSA_REQUIRE(q && k_cache && block_tables && context_lens && page_scores,
               CVSA_ERR_INVALID, "score_pages: null pointer argument");
  CVSA_REQUIRE(B > 0 && B <= 65535 && W > 0 && num_blocks > 0, CVSA_ERR_INVALID,
               "score_pages: bad sizes B=%d W=%d num_blocks=%lld", B, W,
               (long long)num_blocks);
  CVSA_REQUIRE(H_kv > 0 && H_q > 0 && H_q % H_kv == 0, CVSA_ERR_INVALID,
               "score_pages: H_q=%d is not a multiple of H_kv=%d", H_q, H_kv);
  const int ts = tile_shift(block_size);
  CVSA_REQUIRE(head_dim_supported(D) && ts >= 0, CVSA_ERR_UNSUPPORTED,
               "score_pages: D=%d not in {64, 128, 256} or block_size=%d not in {16, 32, 64}",
               D, block_size);
  CVSA_REQUIRE(num_blocks <= (INT32_MAX >> ts), CVSA_ERR_UNSUPPORTED,
               "score_pages: %lld blocks exceed the tile index range", (long long)num_blocks);
  CVSA_REQUIRE(H_kv == 1 || H_kv == 2 || H_kv == 4 || H_kv == 8 || H_kv == 16,
               CVSA_ERR_UNSUPPORTED, "score_pages: H_kv=%d not in {1,2,4,8,16}", H_kv);
  CVSA_REQUIRE(W <= kMaxPages, CVSA_ERR_UNSUPPORTED,
               "score_pages: W=%d exceeds %d pages", W, kMaxPages);
  CVSA_REQUIRE(bt_stride_b >= W, CVSA_ERR_INVALID,
               "score_pages: block-table row stride %lld < W=%d",
               (long long)bt_stride_b, W);
  CVSA_REQUIRE(((uintptr_t)q & 15) == 0 && q_stride_b % 8 == 0 && q_stride_h % 8 == 0 &&
                   ((uintptr_t)k_cache & 15) == 0,
               CVSA_ERR_INVALID,
               "score_pages: q / k_cache must be 16-byte aligned with strides that are "
               "multiples of 8 elements");
  const int G = H_q / H_kv;
  const float inv_g = 1.0f / (float)G;
  const float scale = (float)pow((double)D, -0.5);

  hipStream_t st = (hipStream_t)stream;
  const int R = kWave / (D / 8);
  if (H_kv % R == 0) {
    // Head-group layout: waves = tiles / PPW x H_kv / R.  As many 16-token
    // tiles per wave (up to 8, at least one page) as keep >= ~2048 waves
    // (8 per CU) in the launch: the setup (q_rep, block-table fetch) is
    // amortised over more tiles, and the last-wave tail stays short.
    const int Wt = W << ts;
    const int64_t group_tiles = (int64_t)B * Wt * (H_kv / R);
    int ppw = 1 << ts;
    while (ppw < 8 && group_tiles / (2 * ppw) >= 2048) ppw *= 2;
    const int64_t waves = ((Wt + ppw - 1) / ppw) * (int64_t)(H_kv / R);
    dim3 grid((unsigned)((waves + 3) / 4), B);
    const ScoreArgs sa{q, q_stride_b, q_stride_h, k_cache, (int64_t)num_blocks, block_tables,
                       bt_stride_b, context_lens, page_scores, W, G, inv_g, scale,
                       block_size, ts};
#define CVSA_GROUP_CASE(DD, HK, PP)                                                          \
  if (D == DD && H_kv == HK && ppw == PP) {                                                  \
    hipLaunchKernelGGL((score_pages_group_kernel<DD, HK, PP>), grid, dim3(256), 0, st, sa);  \
    return cvsa_host::check_launch("score_pages");                                           \
  }
#define CVSA_GROUP_PPW(DD, HK) \
  CVSA_GROUP_CASE(DD, HK, 1) CVSA_GROUP_CASE(DD, HK, 2) CVSA_GROUP_CASE(DD, HK, 4) \
  CVSA_GROUP_CASE(DD, HK, 8)
    CVSA_GROUP_PPW(64, 8) CVSA_GROUP_PPW(64, 16)
    CVSA_GROUP_PPW(128, 4) CVSA_GROUP_PPW(128, 8) CVSA_GROUP_PPW(128, 16)
    CVSA_GROUP_PPW(256, 2) CVSA_GROUP_PPW(256, 4) CVSA_GROUP_PPW(256, 8) CVSA_GROUP_PPW(256, 16)
#undef CVSA_GROUP_PPW
#undef CVSA_GROUP_CASE
    return cvsa_host::fail(CVSA_ERR_UNSUPPORTED, "score_pages: H_kv=%d, D=%d has no launch",
                           H_kv, D);
  }
  const int64_t total = (int64_t)B * W;
  int ppw = (int)((total + 8191) / 8192);
  ppw = ppw < 1 ? 1 : (ppw > 8 ? 8 : ppw);
  dim3 grid((W + 4 * ppw - 1) / (4 * ppw), B);
#define CVSA_SCORE_CASE(DD, HK)                                                          \
  if (D == DD && H_kv == HK) {                                                           \
    hipLaunchKernelGGL((score_pages_kernel<DD, HK>), grid, dim3(256), 0, st, q,          \
                       q_stride_b, q_stride_h, k_cache, (int64_t)num_blocks,             \
                       block_tables, bt_stride_b, context_lens, page_scores, W, G,       \
                       inv_g, scale, ppw, block_size, ts);                               \
    return cvsa_host::check_launch("score_pages");                                       \
  }
  CVSA_SCORE_CASE(64, 1) CVSA_SCORE_CASE(64, 2) CVSA_SCORE_CASE(64, 4)
  CVSA_SCORE_CASE(128, 1) CVSA_SCORE_CASE(128, 2)
  CVSA_SCORE_CASE(256, 1)
#undef CVSA_SCORE_CASE
  return cvsa_host::fail(CVSA_ERR_UNSUPPORTED, "score_pages: H_kv=%d, D=%d has no launch", H_kv,
                         D);
}
