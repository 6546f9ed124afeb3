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
// different pages per wave write the same bits; a zero score is written as
// +0 (the sign of a zero maximum would otherwise depend on the order in which
// the maximum is taken, which differs between the waves below and the lazy
// check's decode part).
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
  // Pages another part of the launch scores (or NULL; score_head_wave):
  // byte p of row b * H_kv + h (rows skip_stride bytes apart) is nonzero
  // when page p of that row is scored elsewhere.
  const uint8_t *skip_map;
  int64_t skip_stride;
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
    if (seg == 0 && (j & tm) == tm) s.scores[((int64_t)b * hkv + h) * W + (lt >> s.ts)] = mx + 0.f;
  };
  uint4 buf[2][kPageTokens];
  fetch(0, buf[0]);
#pragma unroll
  for (int j = 0; j < PPW; ++j) {
    if (j + 1 < PPW) fetch(min(j + 1, n - 1), buf[(j + 1) & 1]);
    if (j < n) consume(j, buf[j & 1]);
  }
}

// Page scoring of one wave and one KV head (D = 128, 16-token pages), the
// lazy check's fused launch: wave gw of sequence b scores head h = gw % hkv
// over pages [(gw / hkv) * PPW, +PPW).  A page's 16 key rows of head h are
// 256 bytes each, H_kv * 256 bytes apart; one 16-byte load per lane reads
// four of them (lane l: row l / 16 + 4 i of load i, d-segment l % 16), so
// four loads read the page, and PD pages are in flight.  Each token's dot
// product is score_group_wave's (segment s in lane s of a 16-lane row, the
// same DPP tree), so the scores have the same bits.  With `skip` and
// s.skip_map, the pages the map marks are neither read nor written, and so
// are pages below `skip_below`: their loads are moved past the page and
// dropped by the buffer bounds check, a choice the whole wave shares.
template <int PPW, int PD>
__device__ __forceinline__ void score_head_wave(const ScoreArgs &s, int hkv, int gw, int b,
                                                bool skip, int skip_below = 0) {
  constexpr int D = 128, LPR = 16, NL = kPageTokens / (kWave / LPR);  // 4 loads per page
  static_assert(PPW <= kWave, "a lane per page for the block ids");
  const int lane = threadIdx.x & 63;
  const int h = gw % hkv;
  const int p_begin = (gw / hkv) * PPW;
  const int W = s.W;
  if (p_begin >= W) return;
  const int n = min(PPW, W - p_begin);
  if (p_begin + n <= skip_below) return;  // every page of the wave is scored elsewhere
  const int seg = lane % LPR, row = lane / LPR;
  const int ctx = __builtin_amdgcn_readfirstlane(s.context_lens[b]);
  const int64_t rowi = (int64_t)b * hkv + h;
  // Page j of this wave: block id in lane j (-1 when the page holds no valid
  // token or its id is outside the pool), skip flag in bit j of `skipped`.
  int my_phys = -1;
  bool mark = false;
  if (lane < n) {
    const int p = p_begin + lane;
    if (p * kPageTokens < ctx) {
      const int id = s.block_tables[b * s.bt_sb + p];
      if (id >= 0 && id < s.num_blocks) my_phys = id;
    }
    if (skip && s.skip_map != nullptr) mark = s.skip_map[rowi * s.skip_stride + p] != 0;
    mark = mark || p < skip_below;
  }
  const uint64_t skipped = __ballot(mark);
  const uint4 qr = group_mean_q(s.q, s.q_sb, s.q_sh, b, h, s.G, seg, s.inv_g);
  const int64_t row_stride = (int64_t)hkv * D;
  const uint32_t page_bytes = (uint32_t)(kPageTokens * row_stride * 2);
  const uint32_t voff = (uint32_t)((row * row_stride + (int64_t)h * D + seg * 8) * 2);
  const uint32_t load_step = (uint32_t)(kWave / LPR * row_stride * 2);  // 4 rows

  auto fetch = [&](int j, uint4 (&kv)[NL]) {
    const int phys = max(__builtin_amdgcn_readlane(my_phys, j), 0);
    const uint16_t *page = s.k_cache + (int64_t)phys * kPageTokens * row_stride;
    const uint32_t off = voff + (((skipped >> j) & 1) != 0 ? kRegionSkip : 0u);
#pragma unroll
    for (int i = 0; i < NL; ++i) kv[i] = region_load16(page, page_bytes, off, i * load_step);
  };
  auto consume = [&](int j, const uint4 (&kv)[NL]) {
    const int ntok =
        __builtin_amdgcn_readlane(my_phys, j) < 0 ? 0 : min(kPageTokens, ctx - (p_begin + j) * kPageTokens);
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const float sc = group_sum<LPR>(dot8_bf16(kv[i], qr, 0.f)) * s.scale;
      if (row + (kWave / LPR) * i < ntok) mx = fmaxf(mx, sc);
    }
    float x, y;
    xchg16(mx, x, y);
    mx = fmaxf(x, y);
    xchg32(mx, x, y);
    mx = fmaxf(x, y);
    if (lane == 0 && ((skipped >> j) & 1) == 0) s.scores[rowi * W + p_begin + j] = mx + 0.f;
  };
  uint4 buf[PD][NL];
#pragma unroll
  for (int u = 0; u < PD - 1; ++u) fetch(min(u, n - 1), buf[u]);
#pragma unroll
  for (int j = 0; j < PPW; j += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      // Page j + u + PD - 1 into slot (u + PD - 1) % PD, then page j + u.
      if (j + u + PD - 1 < PPW) fetch(min(j + u + PD - 1, n - 1), buf[(u + PD - 1) % PD]);
      if (j + u < n) consume(j + u, buf[u]);
    }
  }
}

}  // namespace cvsa
