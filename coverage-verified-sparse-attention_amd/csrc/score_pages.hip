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

namespace cvsa {

// H_kv >= 4: a wave owns four KV heads ("quad" hq) of PPW pages.  For each
// token of a page, the quad's four 256-byte rows are contiguous (1 KiB), so
// one 16-byte load per lane reads them whole: lane l holds head 4*hq + (l >> 4),
// d-segment (l & 15) * 8.  The 16 lanes of a DPP row finish the dot product
// with four fused DPP adds, and each lane keeps the running max of its head.
// The wave's block-table entries are fetched once (lane j: page j) and the
// next page's keys are requested before the current page is reduced.
template <int HKV, int PPW>
__global__ __launch_bounds__(256) void score_pages_quad_kernel(
    const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh,
    const uint16_t *__restrict__ k_cache, int64_t num_blocks,
    const int32_t *__restrict__ block_tables, int64_t bt_sb,
    const int32_t *__restrict__ context_lens, float *__restrict__ scores, int W, int G,
    float inv_g, float scale) {
  static_assert(HKV >= 4 && HKV % 4 == 0, "quad layout");
  constexpr int NQ = HKV / 4;  // quads per page
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hq = gw % NQ;
  const int p_begin = (gw / NQ) * PPW;
  const int b = blockIdx.y;
  if (p_begin >= W) return;
  const int h = 4 * hq + (lane >> 4);
  const int seg = lane & 15;
  const int ctx = __builtin_amdgcn_readfirstlane(context_lens[b]);
  const int n = min(PPW, W - p_begin);

  // Page j of this wave: block id in lane j (-1 when the page holds no
  // valid token or the id is outside the pool).
  int my_phys = -1;
  if (lane < n) {
    const int p = p_begin + lane;
    if (p * kPageTokens < ctx) {
      const int id = block_tables[b * bt_sb + p];
      if (id >= 0 && id < num_blocks) my_phys = id;
    }
  }
  const uint4 qr = group_mean_q(q, q_sb, q_sh, b, h, G, seg, inv_g);
  const int64_t lane_off = (int64_t)hq * 4 * kHeadDim + lane * 8;
  const int64_t row_stride = (int64_t)HKV * kHeadDim;
  const int64_t page_elems = kPageTokens * row_stride;

  // Unconditional loads (block 0 for pages without valid tokens) keep the
  // prefetch free of branches.
  auto fetch = [&](int j, uint4 (&kv)[kPageTokens]) {
    const int phys = max(__builtin_amdgcn_readlane(my_phys, j), 0);
    const uint16_t *src = k_cache + (int64_t)phys * page_elems + lane_off;
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t) kv[t] = stream_load16(src + t * row_stride);
  };
  auto consume = [&](int j, const uint4 (&kv)[kPageTokens]) {
    const int p = p_begin + j;
    const int ntok = __builtin_amdgcn_readlane(my_phys, j) < 0
                         ? 0
                         : min(kPageTokens, ctx - p * kPageTokens);
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t) {
      const float s = group_sum<16>(dot8_bf16(kv[t], qr, 0.f)) * scale;
      if (t < ntok) mx = fmaxf(mx, s);
    }
    if (seg == 0) scores[((int64_t)b * HKV + h) * W + p] = mx;
  };
  uint4 buf[2][kPageTokens];
  fetch(0, buf[0]);
#pragma unroll
  for (int j = 0; j < PPW; ++j) {
    if (j + 1 < PPW) fetch(min(j + 1, n - 1), buf[(j + 1) & 1]);
    if (j < n) consume(j, buf[j & 1]);
  }
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
#define CVSA_QUAD_CASE(HK, PP)                                                          \
  if (H_kv == HK && ppw == PP) {                                                        \
    hipLaunchKernelGGL((score_pages_quad_kernel<HK, PP>), grid, dim3(256), 0, st, q,    \
                       q_stride_b, q_stride_h, k_cache, (int64_t)num_blocks,            \
                       block_tables, bt_stride_b, context_lens, page_scores, W, G,      \
                       inv_g, scale);                                                   \
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
