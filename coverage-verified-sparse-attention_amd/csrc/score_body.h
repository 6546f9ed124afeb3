// Page scoring of one wave in the head-group layout (H_kv a multiple of the
// heads one wave load covers), shared by the scoring kernel and the lazy
// check's fused scoring + speculative decode launch.
//
// page_scores[b,h,p] = max over valid tokens of (q_rep . K) * D^-0.5, as
// triton_score_pages (cvsa/kernels/page_scores.py:77-119, kernel :12-74):
// q_rep is the bf16-rounded GQA group mean of q (:94-95), the dot is
// accumulated in fp32 and scaled after the sum (:67), masked tokens are -inf
// (:68) and pages starting at or beyond the context are -inf (:44-47).
// A page's score does not depend on which wave computes it, so launches with
// different pages per wave write the same bits.
#pragma once
#include "cvsa_common.h"

namespace cvsa {

struct ScoreArgs {
  const uint16_t *q;
  int64_t q_sb, q_sh;
  const uint16_t *k_cache;
  int64_t num_blocks;
  const int32_t *block_tables;
  int64_t bt_sb;
  const int32_t *context_lens;
  float *scores;
  int W, G;
  float inv_g, scale;
  int bs, ts;  // block size, tiles per page = 1 << ts
};

// Wave gw of sequence b owns head group hg = gw % (hkv / R) of 16-token
// tiles [(gw / (hkv / R)) * PPW, +PPW) (whole pages: PPW is a multiple of
// the tiles per page), where LPR = D / 8 lanes hold one 2D-byte
// key row and R = 64 / LPR rows make one wave load (R = 8, 4, 2 heads at
// D = 64, 128, 256).  For each token of a page, the group's R rows are
// contiguous (1 KiB), so one 16-byte load per lane reads them whole: lane l
// holds head R*hg + l / LPR, d-segment (l % LPR) * 8.  The LPR lanes of a
// row finish the dot product with DPP adds (and a permlane swap at LPR = 32),
// and each lane keeps the running max of its head over the tiles of a page.
// The wave's block-table entries are fetched once (lane j: tile j) and the
// next tile's keys are requested before the current tile is reduced.  hkv
// is a compile-time constant where the caller's is.
template <int D, int PPW>
__device__ __forceinline__ void score_group_wave(const ScoreArgs &s, int hkv, int gw, int b) {
  constexpr int LPR = D / 8;
  constexpr int R = kWave / LPR;
  const int ng = hkv / R;  // head groups per page
  const int lane = threadIdx.x & 63;
  const int hg = gw % ng;
  const int t_begin = (gw / ng) * PPW;
  const int W = s.W;
  const int tm = (1 << s.ts) - 1;
  if (t_begin >= (W << s.ts)) return;
  const int h = R * hg + lane / LPR;
  const int seg = lane % LPR;
  const int ctx = __builtin_amdgcn_readfirstlane(s.context_lens[b]);
  const int n = min(PPW, (W << s.ts) - t_begin);

  // Tile j of this wave: physical tile in lane j (-1 when its page holds no
  // valid token or the page's block id is outside the pool).
  int my_phys = -1;
  if (lane < n) {
    const int lt = t_begin + lane;
    const int p = lt >> s.ts;
    if (p * s.bs < ctx) {
      const int id = s.block_tables[b * s.bt_sb + p];
      if (id >= 0 && id < s.num_blocks) my_phys = (id << s.ts) | (lt & tm);
    }
  }
  const uint4 qr = group_mean_q(s.q, s.q_sb, s.q_sh, b, h, s.G, seg, s.inv_g);
  const int64_t lane_off = (int64_t)hg * R * D + lane * 8;
  const int64_t row_stride = (int64_t)hkv * D;
  const int64_t page_elems = kPageTokens * row_stride;

  // Unconditional loads (block 0 for pages without valid tokens) keep the
  // prefetch free of branches.
  auto fetch = [&](int j, uint4 (&kv)[kPageTokens]) {
    const int phys = max(__builtin_amdgcn_readlane(my_phys, j), 0);
    const uint16_t *src = s.k_cache + (int64_t)phys * page_elems + lane_off;
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t) kv[t] = stream_load16(src + t * row_stride);
  };
  float pm = -INFINITY;  // running max over the tiles of the current page
  auto consume = [&](int j, const uint4 (&kv)[kPageTokens]) {
    const int lt = t_begin + j;
    const int ntok = __builtin_amdgcn_readlane(my_phys, j) < 0
                         ? 0
                         : min(kPageTokens, ctx - lt * kPageTokens);
    float mx = (j & tm) == 0 ? -INFINITY : pm;
#pragma unroll
    for (int t = 0; t < kPageTokens; ++t) {
      const float sc = group_sum<LPR>(dot8_bf16(kv[t], qr, 0.f)) * s.scale;
      if (t < ntok) mx = fmaxf(mx, sc);
    }
    pm = mx;
    if (seg == 0 && (j & tm) == tm) s.scores[((int64_t)b * hkv + h) * W + (lt >> s.ts)] = mx;
  };
  uint4 buf[2][kPageTokens];
  fetch(0, buf[0]);
#pragma unroll
  for (int j = 0; j < PPW; ++j) {
    if (j + 1 < PPW) fetch(min(j + 1, n - 1), buf[(j + 1) & 1]);
    if (j < n) consume(j, buf[j & 1]);
  }
}

}  // namespace cvsa
