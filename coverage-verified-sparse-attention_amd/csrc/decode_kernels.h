// Paged decode attention over a per-KV-head page list, emitting the
// un-normalised softmax state (o, m, l) and/or the normalised output.
//
// Semantics follow the reference's sparse decode kernels
// (cvsa/kernels/sparse_decode.py:14-132, :136-234, :423-500): for each
// q-head, over the first n_sel listed pages of its KV head and the tokens
// t < min(bs, ctx - page*bs) of each page (:76-80), s = (q . K) * D^-0.5,
// m = max s, l = sum exp(s - m), o = sum exp(s - m) V (:101-124); the
// normalised output is o / max(l, 1e-6) (:127, :271).  Split-K partial
// states are combined with the log-sum-exp rule of _reduce_tiles_kernel
// (:237-276, :576-606).
//
// MI355X mapping.  The reference launches one program per q-head, so each
// K/V page tile is fetched G times.  Here a workgroup owns one KV head and a
// contiguous range of its page list; each of its four waves takes every
// fourth page, loads the page's 16 K rows and 16 V rows once (256 B per row,
// 16-byte lane loads) and applies them to all G query heads of the group as
// two small matrix-core tiles (S = K Q^T, O += P V; see MfmaEngine).  The
// four waves merge in LDS.  When a head's pages span several workgroups
// (splits), each stores its partial (o, m, l) and bumps the head's
// completion counter; the last one to arrive merges the partials and writes
// the outputs, so one launch does the whole decode.  The last workgroup
// resets the counter to zero for the next launch.
//
// Ordering of the split hand-off.  Partials are written and read through a
// raw buffer resource with the sc1 cache policy: on gfx950 such stores are
// written through the issuing XCD's L2 to the device coherence point and
// such loads miss in the reading XCD's L2, so no L2 writeback or invalidate
// (an agent-scope release / acquire fence) is needed.  A workgroup waits
// for its partial stores to complete (s_waitcnt vmcnt(0) and a barrier)
// before its relaxed agent-scope atomic increment of the head's counter; the
// last arriver issues its partial loads only after that atomic has
// returned.  This rests on the gfx950 cache policy described, not on the
// HIP memory model's release / acquire pairing.  Building with
// -DCVSA_FORMAL_HANDOFF=1 replaces it with that pairing (an agent-scope
// release fence in every thread before the counter, an acq_rel counter
// increment, an agent-scope acquire fence in the last arriver): the same
// bits, but the L2 writeback and invalidate those fences compile to cost
// the cfg3 listed decode 31.5 us against 19.3 us (one rejected head 67 vs
// 37 us, dense 135 vs 96 us), so the default build keeps the cache-policy
// protocol.
//
// Head modes: a listed head walks page_indices[b,h,:n_per_head]; an
// all-pages head walks pages 0..n_valid-1 (dense decode).  In verified mode
// accepted heads are listed and rejected heads walk every valid page: the
// draft pages plus the complement pages in one pass, which equals the LSE
// merge of the draft and complement partial softmaxes.  In approximate
// mode rejected heads walk their expanded selection instead
// (cvsa/backend.py:780-812: an expanded top-k at approx_recovery_pct of the
// pages, decoded and normalised on its own).
//
// Tiles: the kernels walk 16-token tiles.  A page (block) of block_size =
// 16 * 2^ts tokens is 2^ts consecutive tiles of its block, so tile sub of
// logical page lp is logical tile (lp << ts) | sub, stored at physical tile
// (block << ts) | sub, 16 * H_kv * D elements apart.  Head walks, splits and
// stream-K ranges count tiles; the effective-budget counters count pages.
#pragma once

#include "cvsa_common.h"
#include "score_body.h"
#include <hip/hip_fp16.h>

namespace cvsa {

// Split partials of head dimension D are rows of part_stride(D) floats:
// o[D], m, l and two pad words, so every row starts on a 16-byte boundary.
// A q-head's o is D / 4 float4 chunks.
__host__ __device__ constexpr int part_stride(int D) { return D + 4; }
constexpr int kMaxSplits = 256;            // partials per head (and workgroups per launch)
constexpr int kMinPagesPerWave = 2;        // pages per wave of a split, at least

struct DecodeArgs {
  const uint16_t *q;
  int64_t q_sb, q_sh;
  const uint16_t *k_cache;
  const uint16_t *v_cache;
  int64_t num_blocks;
  const int32_t *block_tables;
  int64_t bt_sb;
  const int32_t *ctx_lens;
  const int32_t *page_idx;  // NULL: every head walks all valid pages
  int64_t idx_stride;
  int max_sel;
  const int32_t *n_pages;
  const uint8_t *accept;  // non-NULL: verified mode
  int H_kv, W;
  int D;      // head dimension (the launch's engine is compiled for it)
  int ts;     // tiles per page = 1 << ts
  int tl;     // rows of a tile = 1 << tl: 4, or 3 for 8-token pages
  // Query heads: the launch serves heads q_off .. q_off + G - 1 (G the
  // kernel's group, at most 16) of each KV head's group of q_group; a larger
  // group runs as one launch per 16 of its heads.
  int q_group, q_off;
  int heads;  // B * H_kv
  int pps, n_splits;  // listed partition: tiles per split, splits per head
  // Identity partition (every valid page of every head, in page order, as
  // a listed walk of the list 0, 1, 2, ...): tiles per split, splits per
  // head.  Verified launches whose heads are all rejected use it, and so
  // does the lazy check's speculative dense decode, so the two write the
  // same bits.
  int pps_all, n_splits_all;
  int sk_grid;        // stream-K partition: workgroups (<= kMaxSplits)
  float scale;
  float *o_unnorm, *m_out, *l_out;
  void *out;
  int out_dtype;
  float *part;               // split partials (see PartBuf)
  uint32_t part_bytes;
  unsigned *counters;        // per head, zero between launches
  unsigned long long *work;  // optional effective-budget counters
  // A lazy check's speculation (or NULL).  [0]: the prediction, 1 = the
  // check keeps its selection (speculative listed decode of the cached
  // selection), 2 = every head is rejected (speculative dense decode, the
  // identity partition), else none; the check's select-or-keep overwrites
  // it with its keep flag (0 / 1), and a verified launch whose heads are
  // all rejected sets it to 2.  [1]: which speculative decode ran and wrote
  // the outputs (0 none, 1 listed, 2 dense).
  int32_t *spec_state;
  // The speculative decode also writes the page scores of the pages it
  // walks into spec_scores [B * H_kv, W] (or NULL), as the page scoring
  // would (q_rep the group mean of q_group heads times inv_g).
  float *spec_scores;
  float inv_g;
  // Approximate recovery (kModeApprox): a rejected head walks the first
  // min(alt_budget, n_valid) pages of its expanded selection alt_idx[bh]
  // instead of every valid page.
  const int32_t *alt_idx;
  int64_t alt_stride;
  int alt_budget;
};

// A reuse step's token append folded into its listed decode
// (cvsa_sparse_decode_append): sequence b's new K/V rows go to token
// slot[b].x % 16 of logical page slot[b].x / 16 (16-token pages), into block
// slot[b].y when that page is allocated by this append, else the block its
// table entry names; the context length becomes slot[b].x + 1.  The
// workgroups that attend that page take the new token's rows from k_new /
// v_new, so no workgroup reads the cache slot being written.
constexpr int kMaxAppendSeqs = 256;
struct AppendArgs {
  const uint16_t *k_new, *v_new;  // [B, H_kv, D] rows, new_sb elements apart
  int64_t new_sb;
  int32_t *block_tables, *ctx_lens, *pages_allocated;  // updated by the append
  int max_pages;  // block-table width W
  // The slots in device memory (written before the launch, e.g. by a copy
  // that a captured graph replays), or NULL: the slots are slot[].  The host
  // checks slot[] before the launch; device slots are checked here: one out
  // of range (context length outside [0, 16 W), a new block outside
  // [-1, num_blocks), or a new block not at a page start) appends nothing,
  // leaves that sequence's outputs undefined and adds 1 to *slot_errors
  // (when given).
  const int2 *slot_dev;
  int32_t *slot_errors;
  int2 slot[kMaxAppendSeqs];  // (context length before the append, new block or -1)
};

// The new token of a walk's sequence: its logical page and row, its block
// when the append allocates it (else -1), and its K/V rows for this KV head.
struct NewToken {
  int page = -1, off = 0, new_blk = -1;
  const uint16_t *k = nullptr, *v = nullptr;
};

__device__ __forceinline__ void store_out(void *out, int dtype, int64_t i, float y) {
  if (dtype == CVSA_DTYPE_BF16) {
    reinterpret_cast<uint16_t *>(out)[i] = (uint16_t)f32_to_bf16_bits(y);
  } else if (dtype == CVSA_DTYPE_FP16) {
    reinterpret_cast<__half *>(out)[i] = __float2half_rn(y);
  } else {
    reinterpret_cast<float *>(out)[i] = y;
  }
}


template <int D>
__device__ __forceinline__ void write_outputs(const DecodeArgs &a, int64_t qrow, int d, float O,
                                              float M, float L) {
  if (a.o_unnorm != nullptr) {
    a.o_unnorm[qrow * D + d] = O;
    if (d == 0) {
      a.m_out[qrow] = M;
      a.l_out[qrow] = L;
    }
  }
  if (a.out != nullptr) store_out(a.out, a.out_dtype, qrow * D + d, O / fmaxf(L, 1e-6f));
}

// Effective-budget counters: pages attended by this head (n) and the valid
// pages of its sequence (nv).
__device__ __forceinline__ void add_work(const DecodeArgs &a, int n, int nv) {
  atomicAdd(&a.work[0], (unsigned long long)n);
  atomicAdd(&a.work[1], (unsigned long long)max(0, nv));
}

// n_valid_pages(ctx, 1 << sh) for pages of 1 << sh tokens (sh = tl + ts),
// the division a shift where ctx > 0.
__device__ __forceinline__ int valid_pages_sh(int ctx, int sh) {
  return ctx > 0 ? ((ctx - 1) >> sh) + 1 : n_valid_pages(ctx, 1 << sh);
}

// Logical tile of entry e of a head's listed walk: tile e & (2^ts - 1) of
// page idx_row[e >> ts].  ts is the engine's tile shift, a compile-time 0
// for 16-token pages; the result is valid iff it lies in [0, W << ts) (with
// ts > 0 a page outside [0, W) gives -1, so no shift can wrap into range).
__device__ __forceinline__ int listed_tile(const DecodeArgs &a, const int32_t *idx_row, int e,
                                           int ts) {
  const int lp = idx_row[e >> ts];
  if (ts == 0) return lp;
  return lp >= 0 && lp < a.W ? (lp << ts) | (e & ((1 << ts) - 1)) : -1;
}

// Physical tile of logical tile lt of sequence b: valid iff lt is valid and
// the result lies in [0, num_blocks << ts).  The block-table load is
// unconditional (index clamped).
__device__ __forceinline__ int tile_block(const DecodeArgs &a, int b, int lt, int ts) {
  const int phys = a.block_tables[b * a.bt_sb + min(max(lt, 0) >> ts, a.W - 1)];
  if (ts == 0) return phys;
  return lt >= 0 && phys >= 0 && phys < a.num_blocks ? (phys << ts) | (lt & ((1 << ts) - 1))
                                                     : -1;
}


// Tiles walked by head bh: those of its listed pages (page_indices[bh,
// :n_per_head]), or of every valid page (dense heads, rejected heads of a
// verified launch).
// MODE is a template parameter and verified mode loads accept[bh] and
// n_per_head[bh] unconditionally and picks with selects: an earlier form
// that branched on null pointers was miscompiled (a live scalar register was
// reused across the branch).
enum { kModeAll = 0, kModeListed = 1, kModeVerified = 2, kModeApprox = 3 };
// Page lists of a head's walk: every valid page, page_indices, alt_idx.
enum { kWalkAll = 0, kWalkListed = 1, kWalkAlt = 2 };

template <int MODE>
__device__ __forceinline__ int head_pages(const DecodeArgs &a, int bh, int &walk, int ts,
                                          int tl) {
  int n_all = 0, n_list = 0;
  if constexpr (MODE != kModeListed)
    n_all = max(0, min(valid_pages_sh(a.ctx_lens[bh / a.H_kv], tl + ts), a.W)) << ts;
  if constexpr (MODE != kModeAll) n_list = min(max(a.n_pages[bh], 0), a.max_sel) << ts;
  if constexpr (MODE == kModeAll) {
    walk = kWalkAll;
    return n_all;
  } else if constexpr (MODE == kModeListed) {
    walk = kWalkListed;
    return n_list;
  } else if constexpr (MODE == kModeVerified) {
    const bool acc = a.accept[bh] != 0;
    walk = acc ? kWalkListed : kWalkAll;
    return acc ? n_list : n_all;
  } else {
    const bool acc = a.accept[bh] != 0;
    const int n_alt = min(a.alt_budget << ts, n_all);
    walk = acc ? kWalkListed : kWalkAlt;
    return acc ? n_list : n_alt;
  }
}

// Pages booked in the effective-budget counters for head bh of an
// approximate-recovery launch in which some head was rejected
// (backend.py:812-850: the draft's n_per_head plus the expanded
// selection's min(exp_budget, n_valid) on every head).
__device__ __forceinline__ int approx_booked_pages(const DecodeArgs &a, int bh, int nv) {
  return min(max(a.n_pages[bh], 0), a.max_sel) + min(a.alt_budget, max(0, nv));
}

// Stream-K partition.  The heads' page walks are concatenated (head-major)
// into one list of T pages and cut into n_wg equal ranges; workgroup w owns
// pages [start(w), start(w + 1)), start(w) = floor(w * T / n_wg).  n_wg is the
// launch size, reduced so that a workgroup gets at least kMinPagesPerWg
// pages.  T < 2^31 and n_wg <= kMaxSplits, so every quantity is computed in
// 32 bits (64-bit division is a long instruction sequence on the GPU).
constexpr int kMaxHeads = 4096;  // B * H_kv of one launch
// Two-level merge of a stream-K head with more than kTwoLevelMin partials:
// groups of kMergeGroup consecutive contributors, each merged by its last
// arriver into the group's first partial row, then the groups by the last
// group merger.  Group counters follow the kMaxHeads head counters: word
// 2 w0 + (group > 0) for a group whose first contributor is workgroup w0 (a
// workgroup starts at most one head's first group and one head's later
// group, since a head with more than kTwoLevelMin partials covers every
// workgroup between its first and last entirely).
constexpr int kMergeGroup = 16;
constexpr int kTwoLevelMin = 48;
constexpr int kGroupCounters = 2 * 256;  // 2 x the largest stream-K grid
constexpr int kMinPagesPerWg = kMinPagesPerWave * 4;

struct Partition {
  int T, n, q, r;  // pages, workgroups, T / n, T % n
  __device__ __forceinline__ Partition(int T_, int grid) : T(T_) {
    n = max(1, min(grid, (T + kMinPagesPerWg - 1) / kMinPagesPerWg));
    q = T / n;
    r = T - q * n;
  }
  // floor(w * T / n) = w * q + floor(w * r / n), with w * r < n^2 < 2^31.
  __device__ __forceinline__ int start(int w) const { return w * q + (w * r) / n; }
  // The workgroup whose range holds page p (the largest w with start(w) <= p):
  // a float estimate of (p + 1) * n / T, off by at most one, then corrected.
  __device__ __forceinline__ int owner(int p) const {
    int w = min(n - 1, (int)((float)(p + 1) * (float)n / (float)T));
    if (start(w) > p) --w;
    else if (w + 1 < n && start(w + 1) <= p) ++w;
    return w;
  }
};

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// The split partials of one launch, accessed through a raw buffer resource
// with the agent-scope cache policy (sc1) at 16 (or 8) bytes per access:
// stores reach the device coherence point before the split's completion
// counter moves, and loads never return a line that another XCD's L2 still
// holds.  Offsets are in floats; accesses past the range read 0 / are
// dropped by the buffer bounds check.
struct PartBuf {
  static constexpr int kCpolAgent = 16;         // sc1
  static constexpr int kRsrcWord3 = 0x00020000;  // 32-bit data format, raw
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ PartBuf(float *base, uint32_t bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, kRsrcWord3)) {}
  __device__ __forceinline__ void store4(uint32_t off, f32x4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, (int)(off * 4), 0,
                                           kCpolAgent);
  }
  __device__ __forceinline__ void store2(uint32_t off, f32x2 v) const {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, (int)(off * 4), 0,
                                          kCpolAgent);
  }
  __device__ __forceinline__ f32x4 load4(uint32_t off) const {
    return __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off * 4), 0, kCpolAgent));
  }
  __device__ __forceinline__ f32x2 load2(uint32_t off) const {
    return __builtin_bit_cast(
        f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)(off * 4), 0, kCpolAgent));
  }
};

// Outputs for q-row qrow, elements d0 .. d0+3 (one float4 chunk, d0 % 4 == 0):
// one 16-byte store of o_unnorm and one 8- or 16-byte store of out.  The
// outputs are the last stores of a launch, which cannot end before they
// complete, so they are written as few, wide stores.
template <int D>
__device__ __forceinline__ void write_outputs4(const DecodeArgs &a, int64_t qrow, int d0,
                                               f32x4 O, float M, float L) {
  const int64_t i = qrow * D + d0;
  if (a.o_unnorm != nullptr) {
    *reinterpret_cast<f32x4 *>(a.o_unnorm + i) = O;
    if (d0 == 0) {
      a.m_out[qrow] = M;
      a.l_out[qrow] = L;
    }
  }
  if (a.out == nullptr) return;
  if (a.out_dtype == CVSA_DTYPE_FP32) {
    f32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = O[e] / fmaxf(L, 1e-6f);
    *reinterpret_cast<f32x4 *>(reinterpret_cast<float *>(a.out) + i) = y;
    return;
  }
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float y = O[e] / fmaxf(L, 1e-6f);
    w[e] = a.out_dtype == CVSA_DTYPE_BF16 ? f32_to_bf16_bits(y)
                                          : (uint32_t)__half_as_ushort(__float2half_rn(y));
  }
  *reinterpret_cast<uint2 *>(reinterpret_cast<uint16_t *>(a.out) + i) =
      make_uint2(w[0] | (w[1] << 16), w[2] | (w[3] << 16));
}

// LDS of the merge: (m, l) of every (split, g), rewritten in place as
// (weight, l); the head's totals; per-thread sums of the split lanes.
template <int G, int NT>
struct MergeLds {
  f32x2 ml[kMaxSplits * G];
  float M[G], L[G];
  f32x4 acc[NT];
};

// o chunks of one merging thread requested together (KB of merge_partials):
// 16 in the listed decode, whose merge ends the kernel, so a cfg3-sized head
// (32 splits) is read in one memory round trip; 8 in the stream-K kernel,
// whose merge sits inside its segment loop, where 16 would cost it an
// occupancy step.
constexpr int kMergeBatchListed = 16;
constexpr int kMergeBatchStreamK = 8;

// Merge of a head's n_act split partials by the last of its workgroups
// (partial sp at row offset head_off + sp * row_step rows).  TO_PART: the
// merged (o, m, l) of the rows go to the partial row at part_off instead of
// the outputs (the first level of a two-level merge; no counters booked).
// Thread t owns float4 chunk c = t % NC of the head's G x D outputs and the
// splits j, j + J, ... (j = t / NC); their o chunks are loaded KB at a time,
// the first KB together with the (m, l) pairs.  When the
// outputs hold more chunks than the workgroup has threads (G x D > 4 NT) each
// thread takes chunks t, t + NT, ... in turn, every split of each.  The
// (m, l) pairs go to LDS first; one wave per q-head turns them into the
// weights exp(m_sp - M) and the totals (M, L).
template <int G, int D, int NT, int KB, bool TO_PART = false>
__device__ __forceinline__ void merge_partials(const DecodeArgs &a, const PartBuf &pb,
                                               uint32_t head_off, int n_act, int bh, int n,
                                               int nv, MergeLds<G, NT> &s, int row_step = 1,
                                               uint32_t part_off = 0) {
  constexpr int kChunksPerRow = D / 4;
  constexpr int kPartStride = part_stride(D);
  const uint32_t row_elems = (uint32_t)row_step * (uint32_t)(G * kPartStride);
  constexpr int NC = G * kChunksPerRow;
  constexpr int J = NT / NC > 0 ? NT / NC : 1;
  constexpr int NPASS = (NC + NT - 1) / NT;
  constexpr int NW = NT / kWave;
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int j = NPASS == 1 ? t / NC : 0;
  const bool active = t < NC * J;

  for (int e = t; e < n_act * G; e += NT)
    s.ml[e] = pb.load2(head_off + (uint32_t)(e / G) * row_elems + (e % G) * kPartStride + D);
  const int per_lane = active ? (n_act - j + J - 1) / J : 0;  // splits of this thread
  auto load_batch = [&](int g, int d0, int b0, f32x4 (&v)[KB]) {
#pragma unroll
    for (int k = 0; k < KB; ++k) {
      const int sp = min(j + (b0 + k) * J, n_act - 1);
      v[k] = pb.load4(head_off + (uint32_t)sp * row_elems + g * kPartStride + d0);
    }
  };
  f32x4 cur[KB];
  {
    const int c = NPASS == 1 ? t % NC : t;  // NPASS > 1: t < NT < NC
    load_batch(c / kChunksPerRow, 4 * (c % kChunksPerRow), 0, cur);
  }
  __syncthreads();
  for (int gg = wave; gg < G; gg += NW) {  // wave-uniform
    float mx = -INFINITY;
    for (int sp = lane; sp < n_act; sp += kWave) mx = fmaxf(mx, s.ml[sp * G + gg].x);
    mx = wave_max_from_groups<1>(mx);
    float ls = 0.f;
    for (int sp = lane; sp < n_act; sp += kWave) {
      const f32x2 v = s.ml[sp * G + gg];
      const float w = (mx == -INFINITY || v.x == -INFINITY) ? 0.f : fast_exp(v.x - mx);
      ls += w * v.y;
      s.ml[sp * G + gg].x = w;
    }
    ls = wave_sum_from_groups<1>(ls);
    if (lane == 0) {
      s.M[gg] = mx;
      s.L[gg] = ls;
    }
  }
  __syncthreads();
#pragma unroll 1
  for (int pass = 0; pass < NPASS; ++pass) {
    const int c = NPASS == 1 ? t % NC : min(t + pass * NT, NC - 1);
    const bool live = NPASS == 1 ? active : t + pass * NT < NC;
    const int g = c / kChunksPerRow;
    const int d0 = 4 * (c % kChunksPerRow);
    if (pass > 0) load_batch(g, d0, 0, cur);
    f32x4 O = {0.f, 0.f, 0.f, 0.f};
    // A thread's first KB splits were requested with the (m, l) pairs, so a
    // head of up to KB * J splits costs one memory round trip; more splits
    // are read KB at a time.
    for (int b0 = 0;;) {
#pragma unroll
      for (int k = 0; k < KB; ++k) {
        const int sp = min(j + (b0 + k) * J, n_act - 1);
        const float w = b0 + k < per_lane ? s.ml[sp * G + g].x : 0.f;
        O += w * cur[k];
      }
      b0 += KB;
      if (b0 >= per_lane) break;
      load_batch(g, d0, b0, cur);
    }
    if constexpr (J > 1) {
      s.acc[t] = O;
      __syncthreads();
      if (active && j == 0) {
#pragma unroll
        for (int jj = 1; jj < J; ++jj) O += s.acc[t + jj * NC];
      }
    }
    if (live && j == 0) {
      if constexpr (TO_PART) {
        pb.store4(part_off + g * kPartStride + d0, O);
        if (d0 == 0) pb.store2(part_off + g * kPartStride + D, f32x2{s.M[g], s.L[g]});
      } else {
        write_outputs4<D>(a, (int64_t)bh * a.q_group + a.q_off + g, d0, O, s.M[g], s.L[g]);
      }
    }
  }
  if (!TO_PART && t == 0 && a.work != nullptr) add_work(a, n, nv);
}

// ---------------------------------------------------------------- engines
// A page engine owns one wave's softmax state for the G query heads of a KV
// head and applies pages to it.  Page = the K and V rows of one page held in
// registers (fetched PD pages ahead); consume() applies one page; finish()
// leaves the wave's (o, m, l) in LDS.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// MFMA engine: the G query heads (padded to 16) of a KV head against a page
// of 16 tokens are two small dense tiles for the matrix cores.
//   S = K Q^T: v_mfma_f32_16x16x32_bf16, four d-chunks of 32.  A operand =
//     K rows (lane l: token l%16, d 32kk + 8(l/16) .. +8, one 16-byte load),
//     B operand = Q^T (loaded once), result lane l: head l%16, tokens
//     4(l/16) .. +4.
//   O += P V: v_mfma_f32_16x16x16_bf16, eight 16-column blocks of d.  The S
//     result layout is exactly the A operand layout of P (head l%16, tokens
//     4(l/16) .. +4), so P needs no data movement; it is split into a bf16
//     high part and a bf16 remainder (two MFMAs) to keep ~16 mantissa bits.
//     The B operand wants 4 tokens of one d column per lane: the V page goes
//     through a wave-private LDS tile (rows padded to 272 bytes so the four
//     lane groups read disjoint banks).  Result lane l: heads 4(l/16) .. +4,
//     d column 16 blk + l%16.
// Softmax state: m and the running l of head l%16 live in the four lanes of
// that head; a rescale of O rows goes through LDS (16 factors per wave).
template <int G, int D, int TS>
struct MfmaEngine {
  static_assert(G <= 16, "GQA group larger than the MFMA tile");
  static_assert(D == 32 || D == 64 || D == 128 || D == 256, "head dimension");
  static_assert(TS == 0 || TS == -1, "tile shift: 0 (16-token pages) or -1 (from the args)");
  static constexpr int kD = D;
  static constexpr int kTileShift = TS;  // -1: from the args
  // Tiles per page = 1 << tshift(a), rows per tile = 1 << tlog(a): compiled
  // in for 16-token pages.
  static __device__ __forceinline__ int tshift(const DecodeArgs &a) { return TS >= 0 ? TS : a.ts; }
  static __device__ __forceinline__ int tlog(const DecodeArgs &a) { return TS >= 0 ? 4 : a.tl; }
  static constexpr int NK = D / 32;         // S = K Q^T MFMAs (32 dimensions each)
  static constexpr int NB = D / 16;         // O column blocks (16 dimensions each)
  static constexpr int LPR = D / 8;         // lanes per V row (16 bytes each)
  static constexpr int RPL = kWave / LPR;   // V rows per wave load
  static constexpr int NV = kPageTokens / RPL;  // V loads per page
  static constexpr int kVRow = D + 8;       // LDS row of the V tile, in bf16
  struct Page {
    uint4 k[NK], v[NV];
  };
  struct Lds {
    uint16_t v[kPageTokens * kVRow];
    float alpha[16];
  };

  float4_t o[NB];
  bf16x8_t qb[NK];
  float m_g, l_g;
  int lane;
  int rmask;  // rows of a tile - 1: a load of row r reads row r & rmask
  int64_t koff, voff, row_stride;
  float scale;

  __device__ __forceinline__ void init(const DecodeArgs &a, int b, int h, int lane_, Lds &) {
    lane = lane_;
    scale = a.scale;
    rmask = (1 << tlog(a)) - 1;
    row_stride = (int64_t)a.H_kv * D;
    const int c16 = lane & 15, grp = lane >> 4;
    koff = (int64_t)h * D + (c16 & rmask) * row_stride + 8 * grp;
    voff = (int64_t)h * D + ((lane / LPR) & rmask) * row_stride + 8 * (lane % LPR);
    // Rows past the group repeat head G-1: MFMA output rows are independent
    // and those rows are never written out.  No select on the loaded value,
    // so nothing waits for q before the first page is consumed.
    const uint16_t *qrow =
        a.q + b * a.q_sb + (int64_t)(h * a.q_group + a.q_off + min(c16, G - 1)) * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      qb[kk] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(qrow + 32 * kk + 8 * grp));
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) o[blk] = float4_t{0.f, 0.f, 0.f, 0.f};
    m_g = -INFINITY;
    l_g = 0.f;
  }

  // K loads are plain: one instruction reads 64 bytes of each of 16 rows, so
  // every 128-byte line is requested by two instructions, and with the
  // nontemporal hint the line could leave the cache in between (measured:
  // more HBM fetches, slower).  V loads read whole rows and keep the hint.
  __device__ __forceinline__ void fetch(const uint16_t *kp, const uint16_t *vp, Page &pg) const {
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      pg.k[kk] = *reinterpret_cast<const uint4 *>(kp + koff + 32 * kk);
    // Load i reads rows RPL i + lane / LPR: with 8-row tiles those past row
    // 7 fold onto rows 0..7 (RPL is a power of two, so the mask splits).
#pragma unroll
    for (int i = 0; i < NV; ++i)
      pg.v[i] = stream_load16(vp + voff + ((RPL * i) & rmask) * row_stride);
  }

  // fetch() for a walk whose sequence appends a token in this launch: the
  // lanes of row `newrow` of the page (-1: none) read the new token's K/V
  // (k_row / v_row, this KV head's D elements) instead of the cache.
  __device__ __forceinline__ void fetch_new(const uint16_t *kp, const uint16_t *vp, Page &pg,
                                            int newrow, const uint16_t *k_row,
                                            const uint16_t *v_row) const {
    const int grp = lane >> 4;
    const uint16_t *kb = (lane & 15) == newrow ? k_row + 8 * grp : kp + koff;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      pg.k[kk] = *reinterpret_cast<const uint4 *>(kb + 32 * kk);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int t = RPL * i + lane / LPR;
      pg.v[i] = stream_load16(t == newrow ? v_row + 8 * (lane % LPR)
                                          : vp + voff + RPL * i * row_stride);
    }
  }

  // Page score of the walk's KV head from the page's keys, bit for bit the
  // page scoring's (score_group_wave): lane (c16, grp) holds dimensions
  // 32 kk + 8 grp .. +8 of token c16, the scorer's segment s = 4 kk + grp,
  // so the scorer's pairwise sum over s (bit 0, 1, 2, 3 of s in turn) is
  // the partner at lane ^ 16, at lane ^ 32, then the kk pairs; the maximum
  // over the ntok valid tokens follows.  qrep: the 16 segments of q_rep.
  __device__ __forceinline__ float page_score(const Page &pg, int ntok,
                                              const uint4 *qrep) const {
    static_assert(NK == 4, "segment mapping of the 128-dimension rows");
    const int grp = lane >> 4;
    float x[NK];
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) x[kk] = dot8_bf16(pg.k[kk], qrep[4 * kk + grp], 0.f);
    float a, b;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      xchg16(x[kk], a, b);
      x[kk] = a + b;
    }
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      xchg32(x[kk], a, b);
      x[kk] = a + b;
    }
    const float sc = ((x[0] + x[1]) + (x[2] + x[3])) * scale;
    float m = (lane & 15) < ntok ? sc : -INFINITY;
    m = fmaxf(m, dpp_f<kDppQuadXor1>(m));
    m = fmaxf(m, dpp_f<kDppQuadXor2>(m));
    m = fmaxf(m, dpp_f<kDppRowHalfMirror>(m));
    m = fmaxf(m, dpp_f<kDppRowMirror>(m));
    return m + 0.f;
  }

  __device__ __forceinline__ void consume(Page &pg, int ntok, Lds &lds) {
    const int c16 = lane & 15, grp = lane >> 4;
    const int t0 = 4 * grp;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < NK; ++kk)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, pg.k[kk]),
                                                    qb[kk], acc, 0, 0, 0);
    float sv[4];
    float pm = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sv[j] = t0 + j < ntok ? acc[j] * scale : -INFINITY;
      pm = fmaxf(pm, sv[j]);
    }
    float x, y;
    xchg16(pm, x, y);
    pm = fmaxf(x, y);
    xchg32(pm, x, y);
    pm = fmaxf(x, y);  // page max of head c16, in all four of its lanes
    const float m_new = fmaxf(m_g, pm);
    if (__ballot(m_new > m_g) != 0) {  // some head of the wave rescales
      const float alpha = m_new > m_g ? (m_g == -INFINITY ? 0.f : fast_exp(m_g - m_new)) : 1.f;
      l_g *= alpha;
      m_g = m_new;
      if (lane < 16) lds.alpha[lane] = alpha;
      const float4 ar = *reinterpret_cast<const float4 *>(&lds.alpha[t0]);  // rows 4grp .. +4
#pragma unroll
      for (int blk = 0; blk < NB; ++blk) {
        o[blk][0] *= ar.x;
        o[blk][1] *= ar.y;
        o[blk][2] *= ar.z;
        o[blk][3] *= ar.w;
      }
    }
    // P (head c16, tokens t0 .. t0+3) as bf16 high part + bf16 remainder.
    short4_t ph, pl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float p = sv[j] == -INFINITY ? 0.f : fast_exp(sv[j] - m_g);
      l_g += p;
      const uint32_t hi = f32_to_bf16_bits(p);
      const float rem = p - __uint_as_float(hi << 16);
      ph[j] = (short)hi;
      pl[j] = (short)f32_to_bf16_bits(rem);
    }
    // V page -> LDS tile (rows past the context are stored as zeros: the
    // reference never reads them).
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int t = RPL * i + lane / LPR;
      const uint4 w = t < ntok ? pg.v[i] : make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4 *>(&lds.v[t * kVRow + 8 * (lane % LPR)]) = w;
    }
#pragma unroll
    for (int blk = 0; blk < NB; ++blk) {
      short4_t vb;
#pragma unroll
      for (int j = 0; j < 4; ++j) vb[j] = (short)lds.v[(t0 + j) * kVRow + 16 * blk + c16];
      o[blk] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ph, vb, o[blk], 0, 0, 0);
      o[blk] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pl, vb, o[blk], 0, 0, 0);
    }
  }

  template <int NW>
  __device__ __forceinline__ void finish(int wave, int lane_, float (*s_o)[G][D],
                                         float (*s_m)[G], float (*s_l)[G]) {
    const int c16 = lane & 15, grp = lane >> 4;
    float x, y;
    xchg16(l_g, x, y);
    l_g = x + y;
    xchg32(l_g, x, y);
    l_g = x + y;  // head c16's l over all 16 token rows
    if (lane < G) {
      s_m[wave][lane] = m_g;
      s_l[wave][lane] = l_g;
    }
#pragma unroll
    for (int blk = 0; blk < NB; ++blk)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int g = 4 * grp + j;
        if (g < G) s_o[wave][g][16 * blk + c16] = o[blk][j];
      }
  }
};

// The split hand-off's three steps.  publish_partials: every thread's
// partial-row stores complete before the workgroup's counter moves;
// handoff_count: thread 0 bumps the counter and returns its old value;
// acquire_partials: the last arriver's partial loads come after it.
#ifndef CVSA_FORMAL_HANDOFF
#define CVSA_FORMAL_HANDOFF 0
#endif
__device__ __forceinline__ void publish_partials() {
#if CVSA_FORMAL_HANDOFF
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
#else
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
  __syncthreads();
}
__device__ __forceinline__ unsigned handoff_count(unsigned *ctr) {
#if CVSA_FORMAL_HANDOFF
  return __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
#else
  return __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#endif
}
__device__ __forceinline__ void acquire_partials() {
#if CVSA_FORMAL_HANDOFF
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#endif
}

template <class L, int NW>
__device__ __forceinline__ L &s_eng_of(L (&eng)[NW], int wave) { return eng[wave]; }

// End of one workgroup's walk over pages of head h (the waves' states are in
// s_o / s_m / s_l, behind a barrier).  If the workgroup is the head's only
// contributor (n_act == 1) it writes the outputs.  Otherwise it stores its
// partial (o, m, l) in partial row my_row, bumps the head's counter, and the
// last of the n_act contributors merges rows first_row .. first_row+n_act-1.
// TWO (stream-K): a head with more than kTwoLevelMin contributors (rows
// consecutive, contributor i = my_row - first_row) merges in two levels:
// the last arriver of each group of kMergeGroup contributors merges the
// group into the group's first row (after loading every row of the group)
// and bumps the head's counter; the last of the groups merges the group
// rows and writes the outputs.  One workgroup merging ~140 partials takes
// ~9 dependent batches of loads; two levels take one batch each and one more
// store-wait-counter.
template <int G, int D, int NW, int KB, bool TWO = false>
__device__ __forceinline__ void segment_epilogue(const DecodeArgs &a, const PartBuf &pb, int h,
                                                 int n, int nv, int n_act, uint32_t my_row,
                                                 uint32_t first_row,
                                                 const float (&s_o)[NW][G][D],
                                                 const float (&s_m)[NW][G],
                                                 const float (&s_l)[NW][G], int &s_last,
                                                 MergeLds<G, NW * kWave> &s_merge) {
  constexpr int NT = NW * kWave;
  constexpr int kChunksPerRow = D / 4;
  constexpr int kPartStride = part_stride(D);
  // Workgroup state of float4 chunk c (q-head g = c / (D/4), elements d0 .. d0+3):
  // the waves' (o, m, l) rescaled to the workgroup maximum.
  auto wg_state4 = [&](int c, f32x4 &O, float &M, float &L) {
    const int g = c / kChunksPerRow, d0 = 4 * (c % kChunksPerRow);
    M = s_m[0][g];
#pragma unroll
    for (int wv = 1; wv < NW; ++wv) M = fmaxf(M, s_m[wv][g]);
    O = f32x4{0.f, 0.f, 0.f, 0.f};
    L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int wv = 0; wv < NW; ++wv) {
        const float mw = s_m[wv][g];
        if (mw != -INFINITY) {
          const float f = fast_exp(mw - M);
          O += f * *reinterpret_cast<const f32x4 *>(&s_o[wv][g][d0]);
          L += s_l[wv][g] * f;
        }
      }
    }
  };
  if (n_act <= 1) {
    for (int c = threadIdx.x; c < G * kChunksPerRow; c += NT) {
      f32x4 O;
      float M, L;
      wg_state4(c, O, M, L);
      write_outputs4<D>(a, (int64_t)h * a.q_group + a.q_off + c / kChunksPerRow,
                        4 * (c % kChunksPerRow), O, M, L);
    }
    if (threadIdx.x == 0 && a.work != nullptr) add_work(a, n, nv);
    return;
  }
  const uint32_t my_off = my_row * (uint32_t)(G * kPartStride);
  for (int c = threadIdx.x; c < G * kChunksPerRow; c += NT) {
    f32x4 O;
    float M, L;
    wg_state4(c, O, M, L);
    const int g = c / kChunksPerRow, d0 = 4 * (c % kChunksPerRow);
    pb.store4(my_off + g * kPartStride + d0, O);
    if (d0 == 0) pb.store2(my_off + g * kPartStride + D, f32x2{M, L});
  }
  publish_partials();
  constexpr uint32_t kRowElems = (uint32_t)(G * kPartStride);
  if (TWO && n_act > kTwoLevelMin) {  // uniform
    const int i = (int)(my_row - first_row);
    const int gi = i / kMergeGroup;
    const int g0 = gi * kMergeGroup;
    const int gsize = min(kMergeGroup, n_act - g0);
    const int ng = (n_act + kMergeGroup - 1) / kMergeGroup;
    const uint32_t w0 = first_row - (uint32_t)h + (uint32_t)g0;  // the group's first workgroup
    unsigned *gc = a.counters + kMaxHeads + 2 * w0 + (gi != 0 ? 1 : 0);
    if (threadIdx.x == 0) s_last = handoff_count(gc) == (unsigned)(gsize - 1);
    __syncthreads();
    if (!s_last) return;  // uniform
    acquire_partials();
    if (threadIdx.x == 0)
      __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t grow = (first_row + (uint32_t)g0) * kRowElems;
    merge_partials<G, D, NT, KB, true>(a, pb, grow, gsize, h, 0, 0, s_merge, 1, grow);
    publish_partials();
    if (threadIdx.x == 0) s_last = handoff_count(&a.counters[h]) == (unsigned)(ng - 1);
    __syncthreads();
    if (s_last) {
      acquire_partials();
      if (threadIdx.x == 0)
        __hip_atomic_store(&a.counters[h], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      merge_partials<G, D, NT, KB>(a, pb, first_row * kRowElems, ng, h, n, nv, s_merge,
                                   kMergeGroup);
    }
    return;
  }
  if (threadIdx.x == 0) s_last = handoff_count(&a.counters[h]) == (unsigned)(n_act - 1);
  __syncthreads();
  if (s_last) {
    acquire_partials();
    // Last contributor of the head: merge its partials, write the outputs.
    if (threadIdx.x == 0)
      __hip_atomic_store(&a.counters[h], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    merge_partials<G, D, NT, KB>(a, pb, first_row * kRowElems, n_act, h, n, nv, s_merge);
  }
}

// LDS of a workgroup's page walk and epilogue: the waves' (o, m, l), the
// last-arriver flag, and the engines' LDS, which is dead once a walk ends and
// is reused by the merge.
template <int G, class Engine, int NW>
struct WalkLds {
  union Tail {
    typename Engine::Lds eng[NW];
    MergeLds<G, NW * kWave> merge;
  };
  float o[NW][G][Engine::kD] __attribute__((aligned(16)));
  float m[NW][G];
  float l[NW][G];
  int last;
  Tail tail __attribute__((aligned(16)));
};

// The first page-list entries of split `split` of head bh (lane j of wave
// w: entry r0 + w + NW j) and their block-table entries, requested as early
// as possible: their position only needs r0 = split * pps.  Lanes past the
// head's pages are discarded by the walk.
template <int NW>
__device__ __forceinline__ int listed_first_entry(const DecodeArgs &a, int split, int bh,
                                                  int wave, int lane, int ts) {
  if (a.max_sel <= 0) return 0;
  return listed_tile(a, a.page_idx + (int64_t)bh * a.idx_stride,
                     min(split * a.pps + wave + NW * lane, (a.max_sel << ts) - 1), ts);
}

__device__ __forceinline__ int listed_first_block(const DecodeArgs &a, int bh, int lt, int ts) {
  if (a.max_sel <= 0) return 0;
  return tile_block(a, bh / a.H_kv, lt, ts);
}

template <int NW>
__device__ __forceinline__ void listed_first_pages(const DecodeArgs &a, int split, int bh,
                                                   int wave, int lane, int ts, int &lp,
                                                   int &phys) {
  lp = listed_first_entry<NW>(a, split, bh, wave, lane, ts);
  phys = listed_first_block(a, bh, lp, ts);
}

// The first tiles of split `split` of a head's identity walk (lane j of wave
// w: entry r0 + w + NW j, the tile of the same index) and their blocks.
template <int NW>
__device__ __forceinline__ void ident_first_pages(const DecodeArgs &a, int split, int bh,
                                                  int wave, int lane, int ts, int &lp,
                                                  int &phys) {
  lp = split * a.pps_all + wave + NW * lane;
  phys = tile_block(a, bh / a.H_kv, lp, ts);
}

// Tiles per split of a listed walk over n tiles: the launch's a.pps (sized
// on the host by its largest head, max_sel pages) for a head of max_sel
// pages, whose first entries were requested at split * a.pps before its
// count arrived; a shorter head (a per-head budget, a short context) sizes
// its splits by its own count over the launch's n_splits (a multiple of NW,
// at least kMinPagesPerWg pages), so its pages spread over every split
// instead of the first n / a.pps.  ceil(n / pps) <= n_splits either way.
template <int NW>
__device__ __forceinline__ int listed_pps(const DecodeArgs &a, int n, int ts) {
  if (n >= (a.max_sel << ts)) return a.pps;
  const int per = (n + a.n_splits - 1) / a.n_splits;
  return max((per + NW - 1) / NW * NW, kMinPagesPerWg << ts);
}

// Listed pages of a head (the sparse decode of reuse steps, and verified
// launches whose heads are all accepted): split s of head bh walks listed
// pages [s * pps, (s + 1) * pps) of bh (pps: listed_pps); splits past a
// head's pages only take part when the head is empty (split 0 writes its
// outputs).  Partial row of (split, head) = head * n_splits + split.
// With APP, the walk's sequence appends token nt in this launch: the
// context length is nt's page * 16 + row + 1 (16-token pages), and nt's page
// reads that row from nt's rows (Engine::fetch_new) and, when the append
// allocates the page, its block from nt.
// With SCORE and a.spec_scores, the walk also writes the page score of
// every page it walks (Engine::page_score; qrep: this wave's LDS copy of the
// 16 q_rep segments, 16-token pages).
template <int G, class Engine, int NW, int PD, bool APP = false, bool SCORE = false,
          bool IDENT = false>
__device__ __forceinline__ void listed_walk(const DecodeArgs &a, int split, int bh, int spec_lp,
                                            int spec_phys, WalkLds<G, Engine, NW> &L,
                                            const NewToken &nt = NewToken(),
                                            uint4 *qrep = nullptr) {
  using Page = typename Engine::Page;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = bh / a.H_kv;
  const int h = bh - b * a.H_kv;
  const int ctx = APP ? nt.page * kPageTokens + nt.off + 1
                      : __builtin_amdgcn_readfirstlane(a.ctx_lens[b]);
  const int n_spl = IDENT ? a.n_splits_all : a.n_splits;
  const int32_t *idx_row = a.page_idx + (int64_t)bh * a.idx_stride;
  const int ts = Engine::tshift(a);
  const int tl = Engine::tlog(a);
  // IDENT: entry e is tile e of the head's valid pages (n_valid as the
  // reference computes it, at most W).
  const int n = IDENT ? max(0, min(valid_pages_sh(ctx, tl + ts), a.W)) << ts
                      : min(max(__builtin_amdgcn_readfirstlane(a.n_pages[bh]), 0), a.max_sel)
                            << ts;
  const int pps = IDENT ? a.pps_all : listed_pps<NW>(a, n, ts);
  // The first entries (spec_lp, spec_phys) were requested at split * a.pps:
  // a head with splits of its own size requests them again.
  const bool refetch = !IDENT && pps != a.pps;  // uniform
  const int r0 = split * pps;
  const int r1 = min(n, r0 + pps);
  const int n_act = (n + pps - 1) / pps;  // splits holding pages of this head
  if (r0 >= r1 && !(split == 0 && n_act == 0)) return;  // uniform

  Engine eng;
  eng.init(a, b, h, lane, s_eng_of(L.tail.eng, wave));
  // Wave-private q_rep: lane < 16 computes segment `lane` (its loads go out
  // ahead of the first pages') and stores it to LDS just before the first
  // page score, so no wait for q holds up the first page requests; the LDS
  // store and the later reads are the same wave's, in order.
  const bool scoring = SCORE && a.spec_scores != nullptr;  // uniform
  uint4 qr_own = make_uint4(0u, 0u, 0u, 0u);
  bool qr_stored = false;
  if constexpr (SCORE) {
    if (scoring)
      qr_own = group_mean_q(a.q, a.q_sb, a.q_sh, b, h, a.q_group, min(lane, 15), a.inv_g);
  }
  const int64_t page_elems = ((int64_t)a.H_kv * Engine::kD) << tl;  // between tiles
  const int npw = max(0, (r1 - r0 - wave + NW - 1) / NW);
  for (int c0 = 0; c0 < npw; c0 += kWave) {
    const int cn = min(kWave, npw - c0);
    int my_phys = 0, my_ntok = 0, my_new = -1, my_lt = -1;
    if (lane < cn) {
      const bool spec = c0 == 0 && !refetch;
      const int lt = spec ? spec_lp
                     : IDENT ? r0 + wave + NW * (c0 + lane)
                             : listed_tile(a, idx_row, r0 + wave + NW * (c0 + lane), ts);
      if (lt >= 0 && lt < (a.W << ts)) {
        my_lt = lt;
        int pt = spec ? spec_phys : tile_block(a, b, lt, ts);
        if (APP && lt == nt.page && nt.new_blk >= 0) pt = nt.new_blk;
        if (pt >= 0 && pt < (a.num_blocks << ts)) {
          my_phys = pt;
          my_ntok = max(0, min(1 << tl, ctx - (lt << tl)));
          if (APP && lt == nt.page) my_new = nt.off;
        }
      }
    }
    // Loads are unconditional so that no branch separates a prefetch from
    // the page being consumed: a page without valid tokens reads block 0 (in
    // bounds) and is masked out by consume(); prefetches past the end re-read
    // the wave's last page (already cached) and are never consumed.
    auto fetch = [&](int j, Page &pg) {
      const int64_t base = (int64_t)__builtin_amdgcn_readlane(my_phys, j) * page_elems;
      if constexpr (APP)
        eng.fetch_new(a.k_cache + base, a.v_cache + base, pg,
                      __builtin_amdgcn_readlane(my_new, j), nt.k, nt.v);
      else
        eng.fetch(a.k_cache + base, a.v_cache + base, pg);
      return __builtin_amdgcn_readlane(my_ntok, j);
    };
    Page pbuf[PD];
    int nt[PD];
    // The first trip fetches pages 0..PD-1 and consumes page 0; every fetch
    // of a slot uses the same registers and the wait counts see PD-1 pages
    // outstanding.
    for (int j = 1 - PD; j < cn; j += PD) {
#pragma unroll
      for (int u = 0; u < PD; ++u) {
        const int slot = (u + PD - 1) % PD;  // slot of page j+u+PD-1
        nt[slot] = fetch(min(j + u + PD - 1, cn - 1), pbuf[slot]);
        if (j + u >= 0 && j + u < cn) {
          if constexpr (SCORE) {
            if (scoring) {
              if (!qr_stored) {
                if (lane < 16) qrep[lane] = qr_own;
                qr_stored = true;
              }
              const float sc = eng.page_score(pbuf[u], nt[u], qrep);
              const int lt = __builtin_amdgcn_readlane(my_lt, j + u);
              if (lane == 0 && lt >= 0) a.spec_scores[(int64_t)bh * a.W + lt] = sc;
            }
          }
          eng.consume(pbuf[u], nt[u], s_eng_of(L.tail.eng, wave));
        }
      }
    }
  }
  eng.template finish<NW>(wave, lane, L.o, L.m, L.l);
  __syncthreads();
  const PartBuf pb(a.part, a.part_bytes);
  segment_epilogue<G, Engine::kD, NW, kMergeBatchListed>(
      a, pb, bh, n >> ts, valid_pages_sh(ctx, tl + ts), n_act, (uint32_t)(bh * n_spl + split),
      (uint32_t)(bh * n_spl), L.o, L.m, L.l, L.last, L.tail.merge);
}

// The listed decode: a static grid of (split, head) workgroups.
template <int G, class Engine, int NW, int PD>
__global__ __launch_bounds__(NW * kWave) void listed_decode_kernel(const DecodeArgs a) {
  __shared__ WalkLds<G, Engine, NW> L;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int lp, phys;
  listed_first_pages<NW>(a, blockIdx.x, blockIdx.y, wave, lane, Engine::tshift(a), lp, phys);
  listed_walk<G, Engine, NW, PD>(a, blockIdx.x, blockIdx.y, lp, phys, L);
}

// The listed decode of a reuse step with the step's token append folded in
// (16-token pages, D = 128): workgroup (split, bh) walks as
// listed_decode_kernel with its sequence's new token taken from k_new / v_new
// (NewToken), and split 0 of each head writes that head's new K/V rows to
// the cache slot, which no workgroup of the launch reads; split 0 of a
// sequence's first head also moves its context length, page-table entry
// and allocation count as cvsa_append_kv does.  Later launches see the
// appended cache.
template <int G, class Engine, int NW, int PD>
__global__ __launch_bounds__(NW * kWave) void listed_append_kernel(const DecodeArgs a,
                                                                   const AppendArgs app) {
  static_assert(Engine::kD == 128, "the fused append is built for D = 128");
  __shared__ WalkLds<G, Engine, NW> L;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int split = blockIdx.x, bh = blockIdx.y;
  const int b = bh / a.H_kv;
  const int h = bh - b * a.H_kv;
  const int2 sl = app.slot_dev != nullptr ? app.slot_dev[b] : app.slot[b];  // uniform
  const bool ok = sl.x >= 0 && sl.x < app.max_pages * kPageTokens && sl.y >= -1 &&
                  sl.y < a.num_blocks && (sl.y < 0 || (sl.x & 15) == 0);
  NewToken nt;
  nt.page = ok ? sl.x >> 4 : -1;
  nt.off = ok ? sl.x & 15 : kPageTokens - 1;  // not ok: context length 0
  nt.new_blk = ok ? sl.y : -1;
  const int64_t row = (int64_t)b * app.new_sb + (int64_t)h * Engine::kD;
  nt.k = app.k_new + row;
  nt.v = app.v_new + row;
  int lp, phys;
  listed_first_pages<NW>(a, split, bh, wave, lane, 0, lp, phys);
  if (lp == nt.page && nt.new_blk >= 0) phys = nt.new_blk;
  // Split 0's wave 0 appends: lanes 0-15 copy the head's K row, lanes 16-31
  // its V row, 16 bytes each.  Their loads are requested with the walk's
  // first ones and the stores wait until the walk is done.
  const bool writer = ok && split == 0 && wave == 0;  // uniform
  int blk = -1;
  uint4 x = make_uint4(0u, 0u, 0u, 0u);
  if (writer) {
    blk = nt.new_blk >= 0 ? nt.new_blk : a.block_tables[(int64_t)b * a.bt_sb + nt.page];
    x = *reinterpret_cast<const uint4 *>((lane >= 16 ? nt.v : nt.k) + 8 * (lane & 15));
  }
  if (!ok && split == 0 && h == 0 && threadIdx.x == 0 && app.slot_errors != nullptr)
    atomicAdd(app.slot_errors, 1);  // a rejected device slot is reported, not dropped silently
  listed_walk<G, Engine, NW, PD, true>(a, split, bh, lp, phys, L, nt);
  if (!writer) return;
  if (lane < 32 && blk >= 0 && blk < a.num_blocks) {
    const int64_t dst =
        (((int64_t)blk * kPageTokens + nt.off) * a.H_kv + h) * Engine::kD + 8 * (lane & 15);
    *reinterpret_cast<uint4 *>(const_cast<uint16_t *>(lane >= 16 ? a.v_cache : a.k_cache) +
                               dst) = x;
  }
  if (h == 0 && lane == 0) {
    app.ctx_lens[b] = sl.x + 1;
    if (nt.new_blk >= 0) {
      app.block_tables[(int64_t)b * a.bt_sb + nt.page] = nt.new_blk;
      app.pages_allocated[b] += 1;
    }
  }
}

// 16-token tiles per scoring wave of the fused launch below.
constexpr int kSpecScorePPW = 8;
// Pages per scoring wave of the fused launch at 16-token pages (one head per
// wave, score_head_wave).
constexpr int kSpecHeadPPW = 16;

// A lazy check's page scoring and the speculative listed decode of its
// cached selection in one launch.  Workgroups [0, n_splits * heads) are the
// listed decode's (split, head) workgroups, w -> (w % n_splits, w /
// n_splits), bit for bit listed_decode_kernel; they run only if
// spec_state[0] predicts that the check keeps its selection, and workgroup 0
// records in spec_state[1] whether they ran.  The other workgroups score
// pages (workgroup x of sequence b at index n_dec + b * score_gx + x): at
// 16-token pages one head and kSpecHeadPPW pages per wave (score_head_wave),
// else as score_pages_group_kernel<128, ...> (kSpecScorePPW tiles of 4 heads
// per wave).  With a selection map (s.skip_map) the decode part also writes
// the page scores of the pages it walks, from the keys it reads anyway, and
// the scoring part skips them when the decode runs: every page is scored
// once, with the same bits (the per-token arithmetic is the same).
// The parts share no memory otherwise: the decode reads the cached
// selection, which only the check's select-or-keep, launched after this
// kernel, rewrites.
// One launch lets the decode's dependent metadata loads and split hand-off
// overlap the scoring stream without a second stream and its events.
// Three waves per SIMD (the register budget that allows, 168 VGPRs, holds
// the decode without spills): 768 workgroups resident instead of 512, so the
// decode and scoring workgroups of a cfg3 launch all run at once (check
// step 68.4 -> 64.5 us at cfg3, 82.2 -> 75.5 us at cfg4).  Reading the kept
// selection's keys once: kept check 64.0 -> 61.1 us at cfg3 (16 pages per
// scoring wave; 8 and 32 measured 61.2 and 62.0).
template <int G, class Engine, int NW, int PD>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(3)))
void score_spec_kernel(const DecodeArgs a,
                                                                const ScoreArgs s,
                                                                int score_gx) {
  static_assert(NW == 4, "the scoring part runs four waves per workgroup");
  __shared__ WalkLds<G, Engine, NW> L;
  __shared__ uint4 s_qrep[NW][16];  // decode part: q_rep per wave
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n_dec = max(a.n_splits, a.n_splits_all) * a.heads;
  const int w = blockIdx.x;
  // The speculation that runs: 1 = listed decode of the cached selection
  // (predicted keep), 2 = dense decode, which needs the scoring from its
  // keys (16-token pages and a selection map), else 0.
  const int pred = __builtin_amdgcn_readfirstlane(a.spec_state[0]);
  const int go = pred == 1 ? 1
                 : pred == 2 && Engine::kTileShift == 0 && a.spec_scores != nullptr ? 2
                                                                                    : 0;
  if (w >= n_dec) {  // uniform
    const int sw = w - n_dec;
    const int gw = (sw % score_gx) * NW + wave, b = sw / score_gx;
    if constexpr (Engine::kTileShift == 0) {
      // With a skip map, the pages the speculative decode walks (when it
      // runs) are scored there: the selection's, or every valid page.
      const int ctx = __builtin_amdgcn_readfirstlane(s.context_lens[b]);
      score_head_wave<kSpecHeadPPW, 4>(s, a.H_kv, gw, b, s.skip_map != nullptr && go == 1,
                                       go == 2 ? n_valid_pages(ctx, kPageTokens) : 0);
    } else {
      score_group_wave<128, kSpecScorePPW>(s, a.H_kv, gw, b);
    }
    return;
  }
  if (w == 0 && threadIdx.x == 0) a.spec_state[1] = go;
  if (go == 1) {  // uniform
    if (w >= a.n_splits * a.heads) return;
    const int split = w % a.n_splits;
    const int bh = w / a.n_splits;
    int lp, phys;
    listed_first_pages<NW>(a, split, bh, wave, lane, Engine::tshift(a), lp, phys);
    listed_walk<G, Engine, NW, PD, false, Engine::kTileShift == 0>(a, split, bh, lp, phys, L,
                                                                   NewToken(), s_qrep[wave]);
  } else if constexpr (Engine::kTileShift == 0) {
    if (go != 2 || w >= a.n_splits_all * a.heads) return;  // uniform
    const int split = w % a.n_splits_all;
    const int bh = w / a.n_splits_all;
    int lp, phys;
    ident_first_pages<NW>(a, split, bh, wave, lane, 0, lp, phys);
    listed_walk<G, Engine, NW, PD, false, true, true>(a, split, bh, lp, phys, L, NewToken(),
                                                      s_qrep[wave]);
  }
}

// NW waves per workgroup, PD pages of K/V in flight per wave.
//
// Every workgroup first computes the pages each head walks and their prefix
// (the same partition in every workgroup), then walks the segments of its
// range: (head h, pages s0..s1 of h's walk).  A segment that is a whole head
// writes the outputs; otherwise it stores a partial (o, m, l) in row w + h of
// the partial buffer (unique: a later workgroup never starts at an earlier
// head, so (w, h) -> w + h is one-to-one, and head h's partials are the
// consecutive rows owner(first page) + h .. owner(last page) + h), bumps the
// head's counter, and the last contributor merges.  Heads that walk no pages
// are written by workgroup h mod n_wg.
template <int G, class Engine, int NW, int PD, int MODE>
__global__ __launch_bounds__(NW * kWave) void streamk_decode_kernel(const DecodeArgs a) {
  constexpr int NT = NW * kWave;         // threads per workgroup
  static_assert(NW == 4, "kMinPagesPerWg assumes four waves");
  using Page = typename Engine::Page;

  __shared__ WalkLds<G, Engine, NW> L;
  __shared__ int s_wsum[NW];
  __shared__ int s_odd[NW];               // a head of the wave's pass walks != max_sel pages
  __shared__ int s_start[kMaxHeads + 1];  // exclusive prefix of pages per head
  __shared__ uint8_t s_listed[kMaxHeads];  // kWalk* of each head
  auto &s_o = L.o;
  auto &s_m = L.m;
  auto &s_l = L.l;
  auto &s_last = L.last;
  auto &s_tail = L.tail;
  auto &s_eng = s_tail.eng;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = blockIdx.x;
  const int heads = a.heads;
  constexpr int D = Engine::kD;
  const int ts = Engine::tshift(a);
  const int tl = Engine::tlog(a);
  const int64_t page_elems = ((int64_t)a.H_kv * D) << tl;  // between tiles

  // Verified launches whose heads are all accepted (a lazy check that keeps
  // its selection, or a scoring step whose gate passes everywhere) run the
  // listed decode's static partition: workgroup w takes split w % n_splits
  // of head w / n_splits, exactly as listed_decode_kernel, so the outputs
  // are bit for bit those of the listed decode.  Its first page-list
  // entries are requested together with the accept flags and spec_state,
  // their block-table entries once the launch is known to walk.  When the
  // check kept its selection (spec_state[0], written by the check's
  // select-or-keep) and a speculative listed decode of that selection
  // already wrote the outputs (spec_state[1]), there is nothing left: the
  // select-or-keep booked that decode's effective-budget counters.  Every
  // head accepted does not imply a kept selection: a rejected head is
  // reselected and accepted when the new selection passes its gate.
  if constexpr (MODE == kModeVerified || MODE == kModeApprox) {
    const int n_listed = a.n_splits * heads;
    const int split = w % max(a.n_splits, 1);
    const int bh = min(w / max(a.n_splits, 1), heads - 1);
    const int lp = listed_first_entry<NW>(a, split, bh, wave, lane, Engine::tshift(a));
    int spec_done = 0;
    if (a.spec_state != nullptr)
      spec_done = __builtin_amdgcn_readfirstlane(a.spec_state[0] == 1 && a.spec_state[1] == 1);
    if (spec_done != 0) return;  // uniform; every head was accepted (kept)
    int rejected = 0, accepted = 0;
    for (int i = threadIdx.x; i < heads; i += NT) {
      rejected |= a.accept[i] == 0;
      accepted |= a.accept[i] != 0;
    }
    rejected = __syncthreads_or(rejected);
    accepted = __syncthreads_or(accepted);
    if (rejected == 0) {  // uniform
      if (w < n_listed)
        listed_walk<G, Engine, NW, PD>(a, split, bh, lp,
                                       listed_first_block(a, bh, lp, Engine::tshift(a)), L);
      return;
    }
    // Every head rejected (exact recovery: each attends all its valid
    // pages): the identity partition, whose outputs a speculative dense
    // decode of the lazy check (spec_state[1] == 2) already wrote with the
    // same bits; then only its effective-budget counters are booked.  The
    // next check of the layer is told to speculate that way again.
    if (MODE == kModeVerified && accepted == 0) {  // uniform
      const bool dense_done =
          a.spec_state != nullptr && __builtin_amdgcn_readfirstlane(a.spec_state[1]) == 2;
      if (w == 0 && threadIdx.x == 0 && a.spec_state != nullptr) a.spec_state[0] = 2;
      if (dense_done) {
        if (w == 0 && a.work != nullptr) {
          for (int i = threadIdx.x; i < heads; i += NT) {
            const int nv = valid_pages_sh(a.ctx_lens[i / a.H_kv], tl + ts);
            add_work(a, max(0, min(nv, a.W)), nv);
          }
        }
        return;
      }
      if (w >= a.n_splits_all * heads) return;
      const int isplit = w % a.n_splits_all;
      const int ibh = w / a.n_splits_all;
      int ilp, iphys;
      ident_first_pages<NW>(a, isplit, ibh, wave, lane, ts, ilp, iphys);
      listed_walk<G, Engine, NW, PD, false, false, true>(a, isplit, ibh, ilp, iphys, L);
      return;
    }
  }

  // Speculative page lookups for the common case in which every head walks
  // max_sel listed pages: the range start is then known without the scan.
  // The first page-list entries, the head's context length and q and the
  // head counts of the scan are requested at entry, the pages' block-table
  // entries as soon as the page-list entries arrive, and the first PD pages
  // of K/V before the scan: two memory round trips fewer before the first
  // K/V load.  Used only if the scan confirms the case.  The loads are
  // issued without branches (indices clamped; a WG without a speculated
  // range reads harmless in-bounds entries and discards them), so the
  // compiler never has to drain them at a join.
  Engine eng;
  const int max_sel_t = a.max_sel << ts;  // tiles of a full selection
  const int T_spec = heads * max_sel_t;
  const Partition spec_part(T_spec, a.sk_grid);
  int spec_lp = 0, spec_phys = 0, h_spec = -1, r_spec = 0, ctx_spec = 0, g1_spec = 0;
  int b_spec = 0, h_c = 0;  // clamped speculated head and its sequence
  if constexpr (MODE != kModeAll) {
    const int ms = max(max_sel_t, 1);
    const int wc = min(w, spec_part.n - 1);
    const int g0 = spec_part.start(wc);
    g1_spec = spec_part.start(wc + 1);
    const int hs = min(g0 / ms, heads - 1);
    r_spec = g0 - hs * ms;
    h_c = hs;
    b_spec = hs / a.H_kv;
    const int rs = max(0, min(r_spec + wave + NW * lane, max_sel_t - 1));
    const int32_t *src =
        a.max_sel > 0 ? a.page_idx + (int64_t)hs * a.idx_stride + (rs >> ts) : a.block_tables;
    const int lp0 = *src;
    spec_lp = ts == 0 ? lp0 : lp0 >= 0 && lp0 < a.W ? (lp0 << ts) | (rs & ((1 << ts) - 1)) : -1;
    ctx_spec = __builtin_amdgcn_readfirstlane(a.ctx_lens[b_spec]);
    eng.init(a, b_spec, hs - b_spec * a.H_kv, lane, s_eng[wave]);
    if (a.max_sel > 0 && w < spec_part.n) h_spec = hs;
  }

  // Pages per head, one head per thread and pass of NT heads (loads issued
  // without a branch, index clamped), scanned into their exclusive prefix
  // in s_start.
  auto wave_incl_scan = [&](int c) { return (int)wave_incl_scan_u32((uint32_t)c); };
  // A head walking its expanded selection never takes the speculated
  // partition, whose first pages come from page_indices.
  int l_first = kWalkAll;
  int c_first = head_pages<MODE>(a, min((int)threadIdx.x, heads - 1), l_first, ts, tl);
  if constexpr (MODE != kModeAll)
    spec_phys = tile_block(a, b_spec, spec_lp, ts);
  if ((int)threadIdx.x >= heads) c_first = 0;
  const int incl_first = wave_incl_scan(c_first);
  if (lane == kWave - 1) s_wsum[wave] = incl_first;
  const bool odd_first =
      __ballot((int)threadIdx.x < heads && (c_first != max_sel_t || l_first == kWalkAlt)) != 0;
  if (lane == 0) s_odd[wave] = odd_first ? 1 : 0;

  // One wave's walk over its pages s0 + wave + NW*j of a segment, in chunks
  // of up to 64 pages: lane j of a chunk looks up page j's block id and
  // valid-token count; the loop reads them with readlane and keeps PD pages
  // of K/V loads in flight (slot (u + PD - 1) % PD holds page u after the
  // prologue).  Loads are unconditional so that no branch separates a
  // prefetch from the page being consumed: a page without valid tokens reads
  // block 0 (in bounds) and is masked out by consume(); prefetches past the
  // end re-read the wave's last page (already cached) and are never consumed.
  Page pbuf[PD];
  int nt[PD];                 // logical page of each slot (kNoPage: none)
  int my_phys = 0, my_lp = 0;
  int cur_ctx = 0;            // context length of the segment being walked
  constexpr int kNoPage = 1 << 26;  // ctx - kNoPage * 16 < 0: no valid token
  auto lookup = [&](int s0, int c0, int cn, bool listed, const int32_t *idx_row, int b,
                    bool spec) {
    const int r = s0 + wave + NW * (c0 + lane);
    int lp = r, phys = 0;
    if (spec) {  // the speculative entries of the chunk (tile of entry r), consumed by every lane
      lp = spec_lp;
      phys = spec_phys;
    } else if (lane < cn) {
      if (listed) lp = listed_tile(a, idx_row, r, ts);
      phys = tile_block(a, b, lp, ts);
    }
    const bool ok = lane < cn && lp >= 0 && lp < (a.W << ts) && phys >= 0 &&
                    phys < (a.num_blocks << ts);
    my_phys = ok ? phys : 0;
    my_lp = ok ? lp : kNoPage;
  };
  // Page j of the chunk into pg; returns its logical page (the valid-token
  // count needs the context length only when the page is consumed).
  auto fetch = [&](int j, Page &pg) {
    const int64_t base = (int64_t)__builtin_amdgcn_readlane(my_phys, j) * page_elems;
    eng.fetch(a.k_cache + base, a.v_cache + base, pg);
    return __builtin_amdgcn_readlane(my_lp, j);
  };
  auto ntok = [&](int lp) { return min(1 << tl, max(0, cur_ctx - (lp << tl))); };
  auto prologue = [&](int cn) {
#pragma unroll
    for (int u = 0; u < PD; ++u)
      nt[(u + PD - 1) % PD] = fetch(max(0, min(u, cn - 1)), pbuf[(u + PD - 1) % PD]);
  };
  auto steady = [&](int cn) {
    eng.consume(pbuf[PD - 1], ntok(nt[PD - 1]), s_eng[wave]);  // page 0
    for (int j = 1; j < cn; j += PD) {
#pragma unroll
      for (int u = 0; u < PD; ++u) {
        const int slot = (u + PD - 1) % PD;  // slot of page j+u+PD-1
        nt[slot] = fetch(min(j + u + PD - 1, cn - 1), pbuf[slot]);
        if (j + u < cn) eng.consume(pbuf[u], ntok(nt[u]), s_eng[wave]);
      }
    }
  };

  // First PD pages of the speculated segment (a WG without one fetches block
  // 0 and never consumes it).
  if constexpr (MODE != kModeAll) {
    const int s1 = min(g1_spec, (h_c + 1) * max_sel_t) - h_c * max_sel_t;
    const int npw = h_spec >= 0 ? max(0, (s1 - r_spec - wave + NW - 1) / NW) : 0;
    lookup(r_spec, 0, min(kWave, npw), true, nullptr, b_spec, true);
    prologue(min(kWave, npw));
  }
  // Pass 0 (peeled: a loop header here makes the compiler wait for the
  // speculative loads), then the passes of launches with more than NT heads.
  int uneven = 0;  // some head walks a number of pages other than max_sel
  auto finish_pass = [&](int hh, int c, int incl, int lst, int &carry) {
    lds_barrier();
    int excl = incl - c, total = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      if (i < wave) excl += s_wsum[i];
      total += s_wsum[i];
      uneven |= s_odd[i];
    }
    if (hh < heads) {
      s_start[hh] = carry + excl;
      s_listed[hh] = (uint8_t)lst;
    }
    carry += total;
    lds_barrier();  // s_wsum is rewritten by the next pass
  };
  int carry = 0;
  finish_pass(threadIdx.x, c_first, incl_first, l_first, carry);
  if (heads > NT) {  // uniform
    for (int base = NT; base < heads; base += NT) {
      const int hh = base + threadIdx.x;
      int lst = kWalkAll;
      int c = head_pages<MODE>(a, min(hh, heads - 1), lst, ts, tl);
      if (hh >= heads) c = 0;
      const int incl = wave_incl_scan(c);
      if (lane == kWave - 1) s_wsum[wave] = incl;
      const bool odd = __ballot(hh < heads && (c != max_sel_t || lst == kWalkAlt)) != 0;
      if (lane == 0) s_odd[wave] = odd ? 1 : 0;
      finish_pass(hh, c, incl, lst, carry);
    }
  }
  int T = carry;
  if (threadIdx.x == 0) s_start[heads] = T;
  lds_barrier();
  T = __builtin_amdgcn_readfirstlane(T);

  // Every head walks max_sel pages (a matching total is not enough: one
  // head's extra pages can make up for another's missing ones).
  const bool spec_ok = uneven == 0 && T == T_spec && h_spec >= 0;
  const Partition part = spec_ok ? spec_part : Partition(max(T, 1), a.sk_grid);
  const int n_wg = T > 0 ? part.n : a.sk_grid;
  if (w >= n_wg) return;  // uniform

  // Heads without pages: (o, m, l) = (0, -inf, 0), zero output.
  for (int hh = w; hh < heads; hh += n_wg) {
    if (s_start[hh + 1] != s_start[hh]) continue;  // uniform
    const int64_t row0 = (int64_t)hh * a.q_group + a.q_off;
    for (int i = threadIdx.x; i < G * D; i += NT)
      write_outputs<D>(a, row0 + i / D, i % D, 0.f, -INFINITY, 0.f);
    if (threadIdx.x == 0 && a.work != nullptr) {
      const int nv = valid_pages_sh(a.ctx_lens[hh / a.H_kv], tl + ts);
      add_work(a, MODE == kModeApprox ? approx_booked_pages(a, hh, nv) : 0, nv);
    }
  }
  if (T == 0) return;

  const int g0 = part.start(w);
  const int g1 = part.start(w + 1);
  // First head of the range: the last head that starts at or before g0 (it
  // holds page g0, so it is not empty).
  int lo = h_spec;
  if (!spec_ok) {
    lo = 0;
    int hi = heads - 1;
    while (lo < hi) {  // uniform binary search
      const int mid = (lo + hi + 1) >> 1;
      if (s_start[mid] <= g0) lo = mid;
      else hi = mid - 1;
    }
  }
  const PartBuf pb(a.part, a.part_bytes);

  for (int h = lo; h < heads; ++h) {
    const int P = __builtin_amdgcn_readfirstlane(s_start[h]);
    if (P >= g1) break;  // uniform
    const int n = __builtin_amdgcn_readfirstlane(s_start[h + 1]) - P;
    if (n == 0) continue;
    const int s0 = max(g0, P) - P, s1 = min(g1, P + n) - P;
    const int b = h / a.H_kv;
    const int hk = h - b * a.H_kv;
    const int walk = s_listed[h];
    const bool listed = walk != kWalkAll;
    const bool on_spec = h == h_spec;  // eng, ctx_spec already belong to this head
    const int ctx = on_spec ? ctx_spec : __builtin_amdgcn_readfirstlane(a.ctx_lens[b]);
    const int32_t *idx_row = MODE == kModeApprox && walk == kWalkAlt
                                 ? a.alt_idx + (int64_t)h * a.alt_stride
                                 : a.page_idx + (int64_t)h * a.idx_stride;
    const bool use_spec = spec_ok && on_spec && s0 == r_spec && walk == kWalkListed;

    if (!on_spec || h != lo) eng.init(a, b, hk, lane, s_eng[wave]);
    cur_ctx = ctx;
    const int npw = max(0, (s1 - s0 - wave + NW - 1) / NW);
    for (int c0 = 0; c0 < npw; c0 += kWave) {
      const int cn = min(kWave, npw - c0);
      if (!(use_spec && c0 == 0)) {  // the speculated chunk is already in flight
        lookup(s0, c0, cn, listed, idx_row, b, false);
        prologue(cn);
      }
      steady(cn);
    }
    eng.template finish<NW>(wave, lane, s_o, s_m, s_l);
    __syncthreads();

    const int first = part.owner(P);
    const int nv = valid_pages_sh(ctx, tl + ts);
    const int booked = MODE == kModeApprox ? approx_booked_pages(a, h, nv) : n >> ts;
    segment_epilogue<G, D, NW, kMergeBatchStreamK, true>(a, pb, h, booked, nv,
                               part.owner(P + n - 1) - first + 1, (uint32_t)(w + h),
                               (uint32_t)(first + h), s_o, s_m, s_l, s_last, s_tail.merge);
    __syncthreads();  // LDS is reused by the next segment
  }
}

// Workgroups per launch, at most kMaxSplits (a head's partials are merged
// in one workgroup's LDS): one per CU of the 256-CU part.
constexpr int kTargetWorkgroups = 256;
static_assert(kTargetWorkgroups <= kMaxSplits, "one merge per head fits the merge LDS");
constexpr int kWavesPerWg = 4;

// Launches of a validated decode for GQA group size G, explicitly
// instantiated per G in the decode_g*.hip files (one translation unit per
// four group sizes, so the library's objects compile in parallel).  Pages of
// K/V in flight per wave: 2, or 1 at D = 256, whose pages hold twice the
// registers.
enum { kLaunchListed = 0, kLaunchVerified = 1, kLaunchAll = 2, kLaunchApprox = 3 };

template <int G, int D, int TS>
void launch_decode_gdt(const DecodeArgs &a, int kind, dim3 grid, dim3 block, hipStream_t st) {
  constexpr int PD = D > 128 ? 1 : 2;
  using E = MfmaEngine<G, D, TS>;
  if (kind == kLaunchListed)
    hipLaunchKernelGGL((listed_decode_kernel<G, E, kWavesPerWg, PD>), grid, block, 0, st, a);
  else if (kind == kLaunchVerified)
    hipLaunchKernelGGL((streamk_decode_kernel<G, E, kWavesPerWg, PD, kModeVerified>), grid,
                       block, 0, st, a);
  else if (kind == kLaunchApprox)
    hipLaunchKernelGGL((streamk_decode_kernel<G, E, kWavesPerWg, PD, kModeApprox>), grid,
                       block, 0, st, a);
  else
    hipLaunchKernelGGL((streamk_decode_kernel<G, E, kWavesPerWg, PD, kModeAll>), grid, block, 0,
                       st, a);
}

// 16-token pages run engines with the tile shift compiled in (0).
template <int G, int D>
void launch_decode_gd(const DecodeArgs &a, int kind, dim3 grid, dim3 block, hipStream_t st) {
  if (a.ts == 0 && a.tl == 4)
    launch_decode_gdt<G, D, 0>(a, kind, grid, block, st);
  else
    launch_decode_gdt<G, D, -1>(a, kind, grid, block, st);
}

template <int G>
void launch_decode_g(const DecodeArgs &a, int kind, dim3 grid, dim3 block, hipStream_t st) {
  if (a.D == 32)
    launch_decode_gd<G, 32>(a, kind, grid, block, st);
  else if (a.D == 64)
    launch_decode_gd<G, 64>(a, kind, grid, block, st);
  else if (a.D == 256)
    launch_decode_gd<G, 256>(a, kind, grid, block, st);
  else
    launch_decode_gd<G, 128>(a, kind, grid, block, st);
}

// The reuse step's listed decode with the token append (D = 128, 16-token
// pages).
template <int G>
void launch_append_g(const DecodeArgs &a, const AppendArgs &app, dim3 grid, hipStream_t st) {
  hipLaunchKernelGGL((listed_append_kernel<G, MfmaEngine<G, 128, 0>, kWavesPerWg, 2>), grid,
                     dim3(kWavesPerWg * kWave), 0, st, a, app);
}

// The lazy check's fused scoring + speculative decode (D = 128).
template <int G>
void launch_spec_g(const DecodeArgs &a, const ScoreArgs &s, int score_gx, dim3 grid,
                   hipStream_t st) {
  if (a.ts == 0 && a.tl == 4)
    hipLaunchKernelGGL((score_spec_kernel<G, MfmaEngine<G, 128, 0>, kWavesPerWg, 2>), grid,
                       dim3(kWavesPerWg * kWave), 0, st, a, s, score_gx);
  else
    hipLaunchKernelGGL((score_spec_kernel<G, MfmaEngine<G, 128, -1>, kWavesPerWg, 2>), grid,
                       dim3(kWavesPerWg * kWave), 0, st, a, s, score_gx);
}

#define CVSA_DECODE_LAUNCHERS(PREFIX, GG)                                                    \
  PREFIX template void launch_decode_g<GG>(const DecodeArgs &, int, dim3, dim3, hipStream_t); \
  PREFIX template void launch_spec_g<GG>(const DecodeArgs &, const ScoreArgs &, int, dim3,   \
                                         hipStream_t);                                         \
  PREFIX template void launch_append_g<GG>(const DecodeArgs &, const AppendArgs &, dim3,      \
                                           hipStream_t);
#define CVSA_DECODE_EXTERN(GG) CVSA_DECODE_LAUNCHERS(extern, GG)
#define CVSA_DECODE_INSTANTIATE(GG) CVSA_DECODE_LAUNCHERS(, GG)

constexpr int kMaxGroup = 16;       // query heads of one launch: one MFMA tile
constexpr int kMaxGroupTotal = 128;  // query heads per KV head (launches of 16)

}  // namespace cvsa
