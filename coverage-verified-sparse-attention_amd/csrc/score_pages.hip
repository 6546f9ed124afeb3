// Page scoring: page_scores[b,h,p] = max over valid tokens of (q_rep . K) * D^-0.5.
//
// Follows triton_score_pages (cvsa/kernels/page_scores.py:77-119, kernel
// :12-74): q_rep is the bf16-rounded GQA group mean of q (:94-95), the dot is
// accumulated in fp32 and scaled after the sum (:67), masked tokens are -inf
// (:68) and pages starting at or beyond the context are -inf (:44-47).
//
// MI355X mapping: the reference runs one tiny program per (b, kv-head, page).
// Here a wave streams whole 1 KiB runs of a page: a page is block_size x H_kv
// rows of 256 B stored back to back (32 KiB for H_kv = 8), so every 16-byte
// lane load is part of a fully coalesced 1 KiB wave load, and the 16 lanes of
// a DPP row hold one (token, head) row and reduce its dot product with four
// fused DPP adds.
#include "cvsa_common.h"
#include "score_body.h"

namespace cvsa {

// H_kv >= 4: a wave owns four KV heads ("quad") of PPW pages (score_body.h).
template <int HKV, int PPW>
__global__ __launch_bounds__(256) void score_pages_quad_kernel(const ScoreArgs s) {
  static_assert(HKV >= 4 && HKV % 4 == 0, "quad layout");
  score_quad_wave<PPW>(s, HKV, blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
                       blockIdx.y);
}

// H_kv < 4: one wave streams a whole page; lane l covers row (l >> 4) of
// each group of four (token, head) rows and d-segment (l & 15) * 8.
template <int HKV>
__global__ __launch_bounds__(256) void score_pages_kernel(
    const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh,
    const uint16_t *__restrict__ k_cache, int64_t num_blocks,
    const int32_t *__restrict__ block_tables, int64_t bt_sb,
    const int32_t *__restrict__ context_lens, float *__restrict__ scores,
    int W, int G, float inv_g, float scale, int ppw) {
  static_assert(HKV < 4, "small-head layout");
  constexpr int NLOAD = kPageTokens * HKV / 4;     // 16-byte loads per lane per page
  constexpr int PAGE_ELEMS = kPageTokens * HKV * kHeadDim;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rsub = lane >> 4;
  const int seg = lane & 15;
  const int b = blockIdx.y;
  const int p_begin = (blockIdx.x * 4 + wave) * ppw;
  if (p_begin >= W) return;
  const int ctx = context_lens[b];
  const int h = rsub % HKV;
  const uint4 qr = group_mean_q(q, q_sb, q_sh, b, h, G, seg, inv_g);

  const int p_end = min(W, p_begin + ppw);
  for (int p = p_begin; p < p_end; ++p) {
    float *dst = scores + (int64_t)b * HKV * W + p;
    const int ntok = min(kPageTokens, ctx - p * kPageTokens);
    const int phys = ntok > 0 ? block_tables[b * bt_sb + p] : -1;
    if (phys < 0 || phys >= num_blocks) {
      // Beyond the context (or an out-of-range block id): no valid token.
      if (seg == 0 && rsub < HKV) dst[(int64_t)h * W] = -INFINITY;
      continue;
    }
    const uint16_t *src = k_cache + (int64_t)phys * PAGE_ELEMS + lane * 8;
    uint4 kv[NLOAD];
#pragma unroll
    for (int i = 0; i < NLOAD; ++i) kv[i] = stream_load16(src + i * 64 * 8);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NLOAD; ++i) {
      const int t = (i * 4 + rsub) / HKV;
      const float s = group_sum<16>(dot8_bf16(kv[i], qr, 0.f)) * scale;
      if (t < ntok) mx = fmaxf(mx, s);
    }
    // Several row groups share a head: combine them.
    float a, c;
    if constexpr (HKV == 1) {
      xchg16(mx, a, c); mx = fmaxf(a, c);
      xchg32(mx, a, c); mx = fmaxf(a, c);
    } else {
      xchg32(mx, a, c); mx = fmaxf(a, c);
    }
    if (seg == 0 && rsub < HKV) dst[(int64_t)h * W] = mx;
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
  CVSA_REQUIRE(D == kHeadDim && block_size == kPageTokens, CVSA_ERR_UNSUPPORTED,
               "score_pages: only D=128, block_size=16 are supported (got D=%d, bs=%d)",
               D, block_size);
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
  if (H_kv >= 4) {
    // Quad layout: waves = pages / PPW x H_kv / 4.  As many pages per wave
    // (up to 8) as keep >= ~2048 waves (8 per CU) in the launch: the setup
    // (q_rep, block-table fetch) is amortised over more pages, and the
    // last-wave tail stays short.
    const int64_t quad_pages = (int64_t)B * W * (H_kv / 4);
    int ppw = 1;
    while (ppw < 8 && quad_pages / (2 * ppw) >= 2048) ppw *= 2;
    const int64_t waves = ((W + ppw - 1) / ppw) * (int64_t)(H_kv / 4);
    dim3 grid((unsigned)((waves + 3) / 4), B);
    const ScoreArgs sa{q, q_stride_b, q_stride_h, k_cache, (int64_t)num_blocks, block_tables,
                       bt_stride_b, context_lens, page_scores, W, G, inv_g, scale};
#define CVSA_QUAD_CASE(HK, PP)                                                          \
  if (H_kv == HK && ppw == PP) {                                                        \
    hipLaunchKernelGGL((score_pages_quad_kernel<HK, PP>), grid, dim3(256), 0, st, sa);  \
    return cvsa_host::check_launch("score_pages");                                      \
  }
    CVSA_QUAD_CASE(4, 1) CVSA_QUAD_CASE(4, 2) CVSA_QUAD_CASE(4, 4) CVSA_QUAD_CASE(4, 8)
    CVSA_QUAD_CASE(8, 1) CVSA_QUAD_CASE(8, 2) CVSA_QUAD_CASE(8, 4) CVSA_QUAD_CASE(8, 8)
    CVSA_QUAD_CASE(16, 1) CVSA_QUAD_CASE(16, 2) CVSA_QUAD_CASE(16, 4) CVSA_QUAD_CASE(16, 8)
#undef CVSA_QUAD_CASE
    return cvsa_host::fail(CVSA_ERR_UNSUPPORTED, "score_pages: H_kv=%d not in {1,2,4,8,16}",
                           H_kv);
  }
  const int64_t total = (int64_t)B * W;
  int ppw = (int)((total + 8191) / 8192);
  ppw = ppw < 1 ? 1 : (ppw > 8 ? 8 : ppw);
  dim3 grid((W + 4 * ppw - 1) / (4 * ppw), B);
  switch (H_kv) {
#define CVSA_SCORE_CASE(HK)                                                     \
  case HK:                                                                      \
    hipLaunchKernelGGL(score_pages_kernel<HK>, grid, dim3(256), 0, st, q,       \
                       q_stride_b, q_stride_h, k_cache, (int64_t)num_blocks,    \
                       block_tables, bt_stride_b, context_lens, page_scores, W, \
                       G, inv_g, scale, ppw);                                   \
    break;
    CVSA_SCORE_CASE(1)
    CVSA_SCORE_CASE(2)
#undef CVSA_SCORE_CASE
    default:
      return cvsa_host::fail(CVSA_ERR_UNSUPPORTED,
                             "score_pages: H_kv=%d not in {1,2,4,8,16}", H_kv);
  }
  return cvsa_host::check_launch("score_pages");
}
