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

// H_kv a multiple of R known only at run time (e.g. 12, 24, 32, 40 KV heads
// at D = 128): the head-group layout with the head count as an argument.
template <int D, int PPW>
__global__ __launch_bounds__(256) void score_pages_group_any_kernel(const ScoreArgs s, int hkv) {
  score_group_wave<D, PPW>(s, hkv, blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
                           blockIdx.y);
}

// Any other H_kv (neither a multiple of R nor a divisor of it, e.g. 3, 5, 6
// at D = 128): a wave scores one KV head, wave gw of sequence b head
// gw % H_kv over pages [(gw / H_kv) * PPW, +PPW).  Lane l holds key row
// l / LPR of each group of RPL = 64 / LPR rows of a 16-token tile and
// d-segment (l % LPR) * 8 (LPR = D / 8), so a tile is NL = 16 / RPL loads of
// RPL rows of 2D bytes (H_kv * 2D bytes apart).  A row's dot product is
// finished by the LPR lanes that hold it with score_group_wave's DPP tree
// (same bits); each lane keeps the maximum of its rows over the page's
// tiles, and the RPL row groups are combined when the page ends.  The next
// tile's keys are requested before the current one is reduced.
template <int D, int PPW>
__global__ __launch_bounds__(256) void score_pages_head_kernel(const ScoreArgs s, int hkv) {
  constexpr int LPR = D / 8;
  constexpr int RPL = kWave / LPR;
  constexpr int NL = kPageTokens / RPL;
  static_assert(PPW <= kWave, "a lane per page for the block ids");
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.y;
  const int h = gw % hkv;
  const int p_begin = (gw / hkv) * PPW;
  if (p_begin >= s.W) return;
  const int row = lane / LPR, seg = lane % LPR;
  const int ctx = __builtin_amdgcn_readfirstlane(s.context_lens[b]);
  const int n = min(PPW, s.W - p_begin);
  // Page j of this wave: block id in lane j (-1 when the page holds no valid
  // token or its id is outside the pool).
  int my_phys = -1;
  if (lane < n) {
    const int p = p_begin + lane;
    if (p * s.bs < ctx) {
      const int id = s.block_tables[b * s.bt_sb + p];
      if (id >= 0 && id < s.num_blocks) my_phys = id;
    }
  }
  const uint4 qr = group_mean_q(s.q, s.q_sb, s.q_sh, b, h, s.G, seg, s.inv_g);
  // Rows of a tile: 16, or 8 at 8-token pages, whose loads of rows 8..15
  // read rows 0..7 of the same block again (masked out below).
  const int tr = min(s.bs, kPageTokens);
  const int rmask = tr - 1;
  const int64_t row_stride = (int64_t)hkv * D;
  const int64_t tile_elems = tr * row_stride;
  const int64_t lane_off = (row & rmask) * row_stride + (int64_t)h * D + seg * 8;
  const int tm = (1 << s.ts) - 1;
  const int nt = n << s.ts;  // tiles of this wave
  // Unconditional loads (block 0 for pages without valid tokens) keep the
  // prefetch free of branches.
  auto fetch = [&](int t, uint4 (&kv)[NL]) {
    const int phys = max(__builtin_amdgcn_readlane(my_phys, t >> s.ts), 0);
    const uint16_t *src = s.k_cache + (((int64_t)phys << s.ts) | (t & tm)) * tile_elems + lane_off;
#pragma unroll
    for (int i = 0; i < NL; ++i) kv[i] = stream_load16(src + (int64_t)((i * RPL) & rmask) * row_stride);
  };
  float pm = -INFINITY;  // this lane's rows, over the tiles of the current page
  auto consume = [&](int t, const uint4 (&kv)[NL]) {
    const int j = t >> s.ts, sub = t & tm;
    const int p = p_begin + j;
    const int tn = __builtin_amdgcn_readlane(my_phys, j) < 0
                       ? 0
                       : min(tr, ctx - p * s.bs - sub * tr);
    float mx = sub == 0 ? -INFINITY : pm;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const float sc = group_sum<LPR>(dot8_bf16(kv[i], qr, 0.f)) * s.scale;
      if (row + RPL * i < tn) mx = fmaxf(mx, sc);
    }
    pm = mx;
    if (sub == tm) {
      mx = wave_max_from_groups<LPR>(mx);
      // A zero score is written as +0, as by the other layouts.
      if (lane == 0) s.scores[((int64_t)b * hkv + h) * s.W + p] = mx + 0.f;
    }
  };
  uint4 buf[2][NL];
  fetch(0, buf[0]);
  for (int t = 0; t < nt; ++t) {
    if (t + 1 < nt) fetch(t + 1, buf[(t + 1) & 1]);
    consume(t, buf[t & 1]);
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
  CVSA_REQUIRE(head_dim_supported(D) && block_size_supported(block_size), CVSA_ERR_UNSUPPORTED,
               "score_pages: D=%d not in {32, 64, 128, 256} or block_size=%d not in {8, 16, 32, "
               "64, 128}",
               D, block_size);
  const int ts = page_tile_shift(block_size);
  CVSA_REQUIRE(num_blocks <= (INT32_MAX >> ts), CVSA_ERR_UNSUPPORTED,
               "score_pages: %lld blocks exceed the tile index range", (long long)num_blocks);
  CVSA_REQUIRE(W <= kMaxPagesWide, CVSA_ERR_UNSUPPORTED,
               "score_pages: W=%d exceeds %d pages", W, kMaxPagesWide);
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
  if (H_kv % R == 0 && block_size != 8) {
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
#undef CVSA_GROUP_CASE
#define CVSA_GROUP_CASE(DD, HK, PP)                                                      \
  if (D == DD && ppw == PP) {                                                            \
    hipLaunchKernelGGL((score_pages_group_any_kernel<DD, PP>), grid, dim3(256), 0, st, sa, \
                       H_kv);                                                            \
    return cvsa_host::check_launch("score_pages");                                       \
  }
    CVSA_GROUP_PPW(32, 0) CVSA_GROUP_PPW(64, 0) CVSA_GROUP_PPW(128, 0) CVSA_GROUP_PPW(256, 0)
#undef CVSA_GROUP_PPW
#undef CVSA_GROUP_CASE
    return cvsa_host::fail(CVSA_ERR_UNSUPPORTED, "score_pages: H_kv=%d, D=%d has no launch",
                           H_kv, D);
  }
  if (R % H_kv != 0 || D == 32 || block_size == 8) {
    // One KV head per wave (also every H_kv below 16 at D = 32, and every
    // H_kv at 8-token pages): as many pages per wave (up to 16) as keep
    // >= ~2048 waves in the launch.
    const int64_t head_pages = (int64_t)B * W * H_kv;
    int ppw = 1;
    while (ppw < 16 && head_pages / (2 * ppw) >= 2048) ppw *= 2;
    const int64_t waves = ((W + ppw - 1) / ppw) * (int64_t)H_kv;
    dim3 grid((unsigned)((waves + 3) / 4), B);
    const ScoreArgs sa{q, q_stride_b, q_stride_h, k_cache, (int64_t)num_blocks, block_tables,
                       bt_stride_b, context_lens, page_scores, W, G, inv_g, scale,
                       block_size, ts};
#define CVSA_HEAD_CASE(DD, PP)                                                             \
  if (D == DD && ppw == PP) {                                                              \
    hipLaunchKernelGGL((score_pages_head_kernel<DD, PP>), grid, dim3(256), 0, st, sa, H_kv); \
    return cvsa_host::check_launch("score_pages");                                         \
  }
#define CVSA_HEAD_PPW(DD) \
  CVSA_HEAD_CASE(DD, 1) CVSA_HEAD_CASE(DD, 2) CVSA_HEAD_CASE(DD, 4) CVSA_HEAD_CASE(DD, 8) \
  CVSA_HEAD_CASE(DD, 16)
    CVSA_HEAD_PPW(32) CVSA_HEAD_PPW(64) CVSA_HEAD_PPW(128) CVSA_HEAD_PPW(256)
#undef CVSA_HEAD_PPW
#undef CVSA_HEAD_CASE
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
