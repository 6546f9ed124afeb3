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
// 16-byte lane loads) and applies them to all G query heads of the group.
// Lane l holds d-segment (l % LPT) of token slot (l / LPT); the q.K dot is
// finished with an LPT-lane DPP reduction, the page max with DPP and
// permlane swaps, and P.V accumulates in registers.  The four waves merge in
// LDS.  When a head's pages span several workgroups (splits), each stores its
// partial (o, m, l) and bumps the head's completion counter; the last one to
// arrive merges the partials and writes the outputs, so one launch does the
// whole decode.  Partials move through agent-coherent accesses (relaxed
// agent-scope atomic stores and loads, which bypass the per-XCD L2s) and the
// counter increment is issued only after the stores have completed, so no
// L2 writeback or invalidate is needed inside the kernel.  The last
// workgroup resets the counter to zero for the next launch.
//
// Head modes: a listed head walks page_indices[b,h,:n_per_head]; an
// all-pages head walks pages 0..n_valid-1 (dense decode).  In verified mode
// accepted heads are listed and rejected heads walk every valid page: the
// draft pages plus the complement pages in one pass, which equals the LSE
// merge of the draft and complement partial softmaxes.
#include "cvsa_common.h"
#include <hip/hip_fp16.h>
#include <stdlib.h>

namespace cvsa {

constexpr int kPartStride = kHeadDim + 2;  // o[D], m, l
constexpr int kMaxSplits = 32;             // partials per head
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
  float scale;
  int pps_sel, pps_all, n_splits;
  float *o_unnorm, *m_out, *l_out;
  void *out;
  int out_dtype;
  float *part;
  unsigned *counters;        // per head, zero between launches
  unsigned long long *work;  // optional effective-budget counters
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


__device__ __forceinline__ void write_outputs(const DecodeArgs &a, int64_t qrow, int d, float O,
                                              float M, float L) {
  if (a.o_unnorm != nullptr) {
    a.o_unnorm[qrow * kHeadDim + d] = O;
    if (d == 0) {
      a.m_out[qrow] = M;
      a.l_out[qrow] = L;
    }
  }
  if (a.out != nullptr) store_out(a.out, a.out_dtype, qrow * kHeadDim + d, O / fmaxf(L, 1e-6f));
}

// Effective-budget counters: pages attended by this head and n_valid(b).
__device__ __forceinline__ void add_work(const DecodeArgs &a, int n, int ctx) {
  atomicAdd(&a.work[0], (unsigned long long)n);
  atomicAdd(&a.work[1], (unsigned long long)max(0, n_valid_pages(ctx, kPageTokens)));
}


// Page walk of one head.  MODE is a template parameter so that verified mode
// loads accept[bh] and n_per_head[bh] unconditionally and picks (n, pages
// per split) with selects: an earlier form that branched on null pointers
// was miscompiled (a live scalar register was reused across the branch).
enum { kModeAll = 0, kModeListed = 1, kModeVerified = 2 };

template <int MODE>
struct HeadWalk {
  bool listed;
  int n, pps;
  __device__ __forceinline__ HeadWalk(const DecodeArgs &a, int bh, int ctx) {
    const int n_all = max(0, min(n_valid_pages(ctx, kPageTokens), a.W));
    if constexpr (MODE == kModeAll) {
      listed = false;
      n = n_all;
      pps = a.pps_all;
    } else {
      const int n_list = min(max(__builtin_amdgcn_readfirstlane(a.n_pages[bh]), 0), a.max_sel);
      if constexpr (MODE == kModeListed) {
        listed = true;
        n = n_list;
        pps = a.pps_sel;
      } else {
        listed = __builtin_amdgcn_readfirstlane((int)a.accept[bh]) != 0;
        n = listed ? n_list : n_all;
        pps = listed ? a.pps_sel : a.pps_all;
      }
    }
  }
};

__device__ __forceinline__ float coherent_load(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void coherent_store(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Merge of a head's n_act split partials by its last workgroup.  Every load
// is issued up front (o values of this thread's elements into registers,
// (m, l) pairs into LDS; indices clamped to the last active split), so the
// merge costs a single memory round trip.  Each wave then works on one
// q-head g at a time (its 64 elements share g): lane sp holds split sp's
// weight exp(m_sp - M), the wave reduces M and L with lane moves, and the
// weighted sum over splits reads the weights back with readlane.
template <int G, int NT, int NS>
__device__ __forceinline__ void merge_partials(const DecodeArgs &a, const float *head_part,
                                               int n_act, int bh, int n, int ctx,
                                               float (*s_pm)[kMaxSplits],
                                               float (*s_pl)[kMaxSplits]) {
  static_assert(NS <= kWave && (NT % kHeadDim) == 0, "merge layout");
  constexpr int EPT = (G * kHeadDim + NT - 1) / NT;
  constexpr int stride = G * kPartStride;  // between splits
  const int lane = threadIdx.x & 63;
  float ov[EPT][NS];
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int i = min((int)threadIdx.x + k * NT, G * kHeadDim - 1);
    const float *pe = head_part + (i / kHeadDim) * kPartStride + (i % kHeadDim);
#pragma unroll
    for (int sp = 0; sp < NS; ++sp) ov[k][sp] = coherent_load(pe + min(sp, n_act - 1) * stride);
  }
  for (int t = threadIdx.x; t < G * n_act; t += NT) {
    const int g = t / n_act, sp = t - g * n_act;
    const float *pg = head_part + (int64_t)sp * stride + g * kPartStride;
    s_pm[g][sp] = coherent_load(pg + kHeadDim);
    s_pl[g][sp] = coherent_load(pg + kHeadDim + 1);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < EPT; ++k) {
    const int i0 = (int)(threadIdx.x & ~63) + k * NT;  // first element of this wave
    if (i0 >= G * kHeadDim) break;                     // wave-uniform
    const int g = i0 / kHeadDim;
    const float mv = lane < n_act ? s_pm[g][lane] : -INFINITY;
    const float lv = lane < n_act ? s_pl[g][lane] : 0.f;
    const float M = wave_max_from_groups<1>(mv);
    const float w = (M == -INFINITY || mv == -INFINITY) ? 0.f : fast_exp(mv - M);
    const float L = wave_sum_from_groups<1>(w * lv);
    float O = 0.f;
#pragma unroll
    for (int sp = 0; sp < NS; ++sp)
      O += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), sp)) *
           ov[k][sp];
    const int i = i0 + lane;
    write_outputs(a, (int64_t)bh * G + g, i % kHeadDim, O, M, L);
  }
  if (threadIdx.x == 0 && a.work != nullptr) add_work(a, n, ctx);
}

// ---------------------------------------------------------------- engines
// A page engine owns one wave's softmax state for the G query heads of a KV
// head and applies pages to it.  Page = the K and V rows of one page held in
// registers (fetched PD pages ahead); consume() applies one page; finish()
// leaves the wave's (o, m, l) in LDS.

// VALU engine: lane l holds d-segment (l % LPT) of token slot (l / LPT);
// q.K uses packed bf16 dot products with an LPT-lane DPP reduction, P.V is
// fp32 FMA.  Lane vector v covers elements v*LPT*8 + seg*8 .. +8, so each
// load instruction reads whole 128-byte lines of every row it touches.
template <int G, int LPT>
struct ValuEngine {
  static constexpr int E = kHeadDim / LPT;      // d-elements per lane
  static constexpr int NV = E / 8;              // 16-byte vectors per lane per row
  static constexpr int VSTRIDE = LPT * 8;       // elements between a lane's vectors
  static constexpr int TPP = kWave / LPT;       // token slots per pass
  static constexpr int NPASS = kPageTokens / TPP;
  static_assert(NPASS >= 1 && NV >= 1, "bad lane layout");
  struct Page {
    uint4 k[NPASS][NV], v[NPASS][NV];
  };
  struct Lds {};

  float m[G], l[G], o[G][E];
  uint4 qv[G][NV];
  int tg, seg;
  int64_t lane_off, row_stride;
  float scale;

  __device__ __forceinline__ void init(const DecodeArgs &a, int b, int h, int lane, Lds &) {
    tg = lane / LPT;
    seg = lane % LPT;
    scale = a.scale;
    row_stride = (int64_t)a.H_kv * kHeadDim;
    lane_off = (int64_t)h * kHeadDim + seg * 8 + (int64_t)tg * row_stride;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = -INFINITY;
      l[g] = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) o[g][e] = 0.f;
#pragma unroll
      for (int v = 0; v < NV; ++v)
        qv[g][v] = *reinterpret_cast<const uint4 *>(
            a.q + b * a.q_sb + (int64_t)(h * G + g) * a.q_sh + v * VSTRIDE + seg * 8);
    }
  }

  __device__ __forceinline__ void fetch(const uint16_t *kp, const uint16_t *vp, Page &pg) const {
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int64_t off = lane_off + (int64_t)(ps * TPP) * row_stride;
#pragma unroll
      for (int v = 0; v < NV; ++v)
        pg.k[ps][v] = stream_load16(kp + off + v * VSTRIDE);
#pragma unroll
      for (int v = 0; v < NV; ++v)
        pg.v[ps][v] = stream_load16(vp + off + v * VSTRIDE);
    }
  }

  __device__ __forceinline__ void consume(Page &pg, int ntok, Lds &) {
    float s[NPASS][G];
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const bool valid = ps * TPP + tg < ntok;
      // Tokens past the context contribute nothing, whatever their V rows
      // hold (the reference masks those loads); zeroed in place.
#pragma unroll
      for (int v = 0; v < NV; ++v)
        if (!valid) pg.v[ps][v] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = 0.f;
#pragma unroll
        for (int v = 0; v < NV; ++v) acc = dot8_bf16(pg.k[ps][v], qv[g][v], acc);
        acc = group_sum<LPT>(acc) * scale;
        s[ps][g] = valid ? acc : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float pm = s[0][g];
#pragma unroll
      for (int ps = 1; ps < NPASS; ++ps) pm = fmaxf(pm, s[ps][g]);
      pm = wave_max_from_groups<LPT>(pm);
      if (pm > m[g]) {  // wave-uniform
        const float alpha = fast_exp(m[g] - pm);
        l[g] *= alpha;
#pragma unroll
        for (int e = 0; e < E; ++e) o[g][e] *= alpha;
        m[g] = pm;
      }
#pragma unroll
      for (int ps = 0; ps < NPASS; ++ps) {
        const bool valid = s[ps][g] != -INFINITY;
        const float p = valid ? fast_exp(s[ps][g] - m[g]) : 0.f;
        l[g] += p;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          const uint4 w = pg.v[ps][v];
          o[g][v * 8 + 0] += p * bf16_lo(w.x);
          o[g][v * 8 + 1] += p * bf16_hi(w.x);
          o[g][v * 8 + 2] += p * bf16_lo(w.y);
          o[g][v * 8 + 3] += p * bf16_hi(w.y);
          o[g][v * 8 + 4] += p * bf16_lo(w.z);
          o[g][v * 8 + 5] += p * bf16_hi(w.z);
          o[g][v * 8 + 6] += p * bf16_lo(w.w);
          o[g][v * 8 + 7] += p * bf16_hi(w.w);
        }
      }
    }
  }

  template <int NW>
  __device__ __forceinline__ void finish(int wave, int lane, float (*s_o)[G][kHeadDim],
                                         float (*s_m)[G], float (*s_l)[G]) {
    // Sum the token slots of the wave (lanes that share a d-segment).
#pragma unroll
    for (int g = 0; g < G; ++g) {
      l[g] = sum_across_groups<LPT>(l[g]);
#pragma unroll
      for (int e = 0; e < E; ++e) o[g][e] = sum_across_groups<LPT>(o[g][e]);
    }
    if (tg == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int v = 0; v < NV; ++v)
#pragma unroll
          for (int e = 0; e < 8; ++e) s_o[wave][g][v * VSTRIDE + seg * 8 + e] = o[g][v * 8 + e];
    }
    if (lane == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s_m[wave][g] = m[g];
        s_l[wave][g] = l[g];
      }
    }
  }
};

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
template <int G>
struct MfmaEngine {
  static_assert(G <= 16, "GQA group larger than the MFMA tile");
  static constexpr int kVRow = kHeadDim + 8;  // LDS row of the V tile, in bf16
  struct Page {
    uint4 k[4], v[4];
  };
  struct Lds {
    uint16_t v[kPageTokens * kVRow];
    float alpha[16];
  };

  float4_t o[8];
  bf16x8_t qb[4];
  float m_g, l_g;
  int lane;
  int64_t koff, voff, row_stride;
  float scale;

  __device__ __forceinline__ void init(const DecodeArgs &a, int b, int h, int lane_, Lds &) {
    lane = lane_;
    scale = a.scale;
    row_stride = (int64_t)a.H_kv * kHeadDim;
    const int c16 = lane & 15, grp = lane >> 4;
    koff = (int64_t)h * kHeadDim + c16 * row_stride + 8 * grp;
    voff = (int64_t)h * kHeadDim + grp * row_stride + 8 * c16;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (c16 < G)
        w = *reinterpret_cast<const uint4 *>(a.q + b * a.q_sb + (int64_t)(h * G + c16) * a.q_sh +
                                             32 * kk + 8 * grp);
      qb[kk] = __builtin_bit_cast(bf16x8_t, w);
    }
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) o[blk] = float4_t{0.f, 0.f, 0.f, 0.f};
    m_g = -INFINITY;
    l_g = 0.f;
  }

  __device__ __forceinline__ void fetch(const uint16_t *kp, const uint16_t *vp, Page &pg) const {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      pg.k[kk] = stream_load16(kp + koff + 32 * kk);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pg.v[i] = stream_load16(vp + voff + 4 * i * row_stride);
  }

  __device__ __forceinline__ void consume(Page &pg, int ntok, Lds &lds) {
    const int c16 = lane & 15, grp = lane >> 4;
    const int t0 = 4 * grp;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
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
      for (int blk = 0; blk < 8; ++blk) {
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
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * i + grp;
      const uint4 w = t < ntok ? pg.v[i] : make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4 *>(&lds.v[t * kVRow + 8 * c16]) = w;
    }
#pragma unroll
    for (int blk = 0; blk < 8; ++blk) {
      short4_t vb;
#pragma unroll
      for (int j = 0; j < 4; ++j) vb[j] = (short)lds.v[(t0 + j) * kVRow + 16 * blk + c16];
      o[blk] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ph, vb, o[blk], 0, 0, 0);
      o[blk] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pl, vb, o[blk], 0, 0, 0);
    }
  }

  template <int NW>
  __device__ __forceinline__ void finish(int wave, int lane_, float (*s_o)[G][kHeadDim],
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
    for (int blk = 0; blk < 8; ++blk)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int g = 4 * grp + j;
        if (g < G) s_o[wave][g][16 * blk + c16] = o[blk][j];
      }
  }
};

// NW waves per workgroup, PD pages of K/V in flight per wave.
template <int G, class Engine, int NW, int PD, int MODE>
__global__ __launch_bounds__(NW * kWave) void paged_decode_kernel(const DecodeArgs a) {
  constexpr int NT = NW * kWave;         // threads per workgroup
  using Page = typename Engine::Page;

  __shared__ float s_o[NW][G][kHeadDim];
  __shared__ float s_m[NW][G];
  __shared__ float s_l[NW][G];
  __shared__ int s_last;
  __shared__ float s_pm[G][kMaxSplits], s_pl[G][kMaxSplits];
  __shared__ __attribute__((aligned(16))) typename Engine::Lds s_eng[NW];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int bh = blockIdx.y;
  const int split = blockIdx.x;
  const int b = bh / a.H_kv;
  const int h = bh - b * a.H_kv;
  const int ctx = __builtin_amdgcn_readfirstlane(a.ctx_lens[b]);
  // The first page-list entries of a listed head are requested together with
  // the head's scalar state (their position only needs the split's start,
  // split * pps_sel), which takes one memory round trip off the page-table
  // lookups.  Lanes past the head's pages are never consumed.
  // The block-table entries of those pages are requested as soon as the
  // entries arrive (clamped into the table; lanes past the head's pages
  // are discarded later), so the table lookup does not wait for the head's
  // page count either.
  int spec_lp = 0, spec_phys = 0;
  if constexpr (MODE != kModeAll) {
    if (a.max_sel > 0) {
      const int rs = min(split * a.pps_sel + wave + NW * lane, a.max_sel - 1);
      spec_lp = a.page_idx[(int64_t)bh * a.idx_stride + rs];
      spec_phys = a.block_tables[b * a.bt_sb + min(max(spec_lp, 0), a.W - 1)];
    }
  } else {
    spec_lp = min(split * a.pps_all + wave + NW * lane, a.W - 1);
    spec_phys = a.block_tables[b * a.bt_sb + spec_lp];
  }

  const HeadWalk<MODE> hw(a, bh, ctx);
  const bool listed = hw.listed;
  const int n = hw.n, pps = hw.pps;
  const int r0 = split * pps;
  const int r1 = min(n, r0 + pps);

  if (r0 < r1) {
    Engine eng;
    eng.init(a, b, h, lane, s_eng[wave]);
    const int64_t page_elems = (int64_t)kPageTokens * a.H_kv * kHeadDim;  // between blocks
    const int32_t *idx_row = listed ? a.page_idx + (int64_t)bh * a.idx_stride : nullptr;

    // This wave's pages are r0 + wave + NW*j.  Lane j looks up page j's block
    // id and valid-token count up front; the page loop reads them with
    // readlane and keeps PD pages of K/V loads in flight.
    const int npw = (r1 - r0 - wave + NW - 1) / NW;
    for (int c0 = 0; c0 < npw; c0 += kWave) {
      const int cn = min(kWave, npw - c0);
      int my_phys = 0, my_ntok = 0;
      if (lane < cn) {
        const int r = r0 + wave + NW * (c0 + lane);
        // Chunk 0 of a listed head (or of an all-pages launch) uses the
        // entries requested up front; the spec index equals r there.
        const bool spec = c0 == 0 && (MODE == kModeAll || listed);
        const int lp = spec ? spec_lp : (listed ? idx_row[r] : r);
        if (lp >= 0 && lp < a.W) {
          const int phys = spec ? spec_phys : a.block_tables[b * a.bt_sb + lp];
          if (phys >= 0 && phys < a.num_blocks) {
            my_phys = phys;
            my_ntok = min(kPageTokens, ctx - lp * kPageTokens);
          }
        }
      }
      // Loads are unconditional so that no branch separates a prefetch from
      // the page being consumed: a page without valid tokens reads block 0
      // (in bounds) and is masked out by consume(); prefetches past the end
      // re-read the wave's last page (already cached) and are never consumed.
      auto fetch = [&](int j, Page &pg) {
        const int64_t base = (int64_t)__builtin_amdgcn_readlane(my_phys, j) * page_elems;
        eng.fetch(a.k_cache + base, a.v_cache + base, pg);
        return __builtin_amdgcn_readlane(my_ntok, j);
      };
      Page pb[PD];
      int nt[PD];
      // No separate prologue: the first trip fetches pages 0..PD-1 and
      // consumes only page 0, so every fetch of a slot uses the same
      // registers and the wait counts see PD-1 pages outstanding.
      for (int j = 1 - PD; j < cn; j += PD) {
#pragma unroll
        for (int u = 0; u < PD; ++u) {
          const int slot = (u + PD - 1) % PD;  // slot of page j+u+PD-1
          nt[slot] = fetch(min(j + u + PD - 1, cn - 1), pb[slot]);
          if (j + u >= 0 && j + u < cn) eng.consume(pb[u], nt[u], s_eng[wave]);
        }
      }
    }
    eng.template finish<NW>(wave, lane, s_o, s_m, s_l);
  }
  __syncthreads();

  // Merge the waves: wave-partial (o, m, l) -> workgroup (O, M, L) for
  // element i = g * D + d.
  auto wg_state = [&](int i, float &O, float &M, float &L) {
    const int g = i / kHeadDim, d = i - g * kHeadDim;
    M = -INFINITY;
    O = 0.f;
    L = 0.f;
    if (r0 < r1) {
      M = s_m[0][g];
#pragma unroll
      for (int w = 1; w < NW; ++w) M = fmaxf(M, s_m[w][g]);
      if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float mw = s_m[w][g];
          if (mw != -INFINITY) {
            const float f = fast_exp(mw - M);
            O += s_o[w][g][d] * f;
            L += s_l[w][g] * f;
          }
        }
      }
    }
  };

  const int n_act = (n + pps - 1) / pps;  // splits holding pages of this head
  if (n_act <= 1) {
    // Split 0 owns the whole head (or the head is empty): write the outputs.
    if (split == 0) {
      for (int i = threadIdx.x; i < G * kHeadDim; i += NT) {
        float O, M, L;
        wg_state(i, O, M, L);
        write_outputs(a, (int64_t)bh * G + i / kHeadDim, i % kHeadDim, O, M, L);
      }
      if (threadIdx.x == 0 && a.work != nullptr) add_work(a, n, ctx);
    }
    return;
  }
  if (r0 >= r1) return;  // no pages for this split (uniform)

  float *head_part = a.part + (int64_t)bh * a.n_splits * G * kPartStride;
  float *my_part = head_part + (int64_t)split * G * kPartStride;
  for (int i = threadIdx.x; i < G * kHeadDim; i += NT) {
    const int g = i / kHeadDim, d = i - g * kHeadDim;
    float O, M, L;
    wg_state(i, O, M, L);
    coherent_store(my_part + g * kPartStride + d, O);
    if (d == 0) {
      coherent_store(my_part + g * kPartStride + kHeadDim, M);
      coherent_store(my_part + g * kPartStride + kHeadDim + 1, L);
    }
  }
  // Every wave's partial stores have completed before the counter moves.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&a.counters[bh], 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == (unsigned)(n_act - 1);
  }
  __syncthreads();
  if (!s_last) return;

  // Last split of the head: merge all partials and write the outputs.
  if (threadIdx.x == 0)
    __hip_atomic_store(&a.counters[bh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (n_act <= 8)
    merge_partials<G, NT, 8>(a, head_part, n_act, bh, n, ctx, s_pm, s_pl);
  else if (n_act <= 16)
    merge_partials<G, NT, 16>(a, head_part, n_act, bh, n, ctx, s_pm, s_pl);
  else
    merge_partials<G, NT, kMaxSplits>(a, head_part, n_act, bh, n, ctx, s_pm, s_pl);
}

__global__ void fill_zero_kernel(uint32_t *p, size_t n_words) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_words;
       i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

struct DecodePlan {
  int pps_sel, pps_all, n_splits;
};

static int env_int(const char *name, int dflt) {
  const char *e = getenv(name);
  const int x = e ? atoi(e) : 0;
  return x > 0 ? x : dflt;
}

// Page engine: 1 = matrix cores (MfmaEngine), 0 = VALU (ValuEngine);
// CVSA_DECODE_ENGINE overrides the default (read once).
static int decode_engine() {
  static const int v = getenv("CVSA_DECODE_ENGINE") ? atoi(getenv("CVSA_DECODE_ENGINE")) : 1;
  return v;
}

// Workgroups per launch (tuning knob CVSA_DECODE_TARGET_WGS, read once).
static int target_workgroups() {
  static const int v = env_int("CVSA_DECODE_TARGET_WGS", 256);
  return v;
}
constexpr int kWavesPerWg = 4;

// Pages per split: spread the heads over ~target_workgroups() workgroups,
// at least two pages per wave and at most kMaxSplits splits per head.
static DecodePlan plan_decode(int B, int H_kv, int max_sel, int W, bool listed,
                              bool all_pages) {
  const int heads = B * H_kv;
  const int target = target_workgroups();
  const int waves = kWavesPerWg;
  const int min_pps = kMinPagesPerWave * waves;
  int wg_per_head = heads >= target ? 1 : target / heads;
  if (wg_per_head > kMaxSplits) wg_per_head = kMaxSplits;
  auto pps_for = [&](int pages) {
    int pps = (pages + wg_per_head - 1) / wg_per_head;
    if (pps < min_pps) pps = min_pps;
    pps = (pps + waves - 1) / waves * waves;
    while ((pages + pps - 1) / pps > kMaxSplits) pps += waves;
    return pps;
  };
  DecodePlan p;
  p.pps_sel = pps_for(listed ? max_sel : 0);
  p.pps_all = pps_for(all_pages ? W : 0);
  const int s1 = listed ? (max_sel + p.pps_sel - 1) / p.pps_sel : 0;
  const int s2 = all_pages ? (W + p.pps_all - 1) / p.pps_all : 0;
  p.n_splits = s1 > s2 ? s1 : s2;
  if (p.n_splits < 1) p.n_splits = 1;
  return p;
}

// Workspace: per-head completion counters (uint32, padded to 256 bytes),
// then split partials [B*H_kv][n_splits][G][D + 2] fp32; none with a single
// split.
static size_t counter_bytes(int heads) { return ((size_t)heads * 4 + 255) / 256 * 256; }

static size_t workspace_bytes_for(int B, int H_q, int H_kv, int max_sel, int W, bool listed,
                                  bool all_pages) {
  const int heads = B * H_kv;
  const int G = H_q / H_kv;
  const DecodePlan p = plan_decode(B, H_kv, max_sel, W, listed, all_pages);
  if (p.n_splits == 1) return 0;
  return counter_bytes(heads) + (size_t)heads * p.n_splits * G * kPartStride * sizeof(float);
}

// Lanes per token row, chosen so that the o accumulators stay at <= 64
// VGPRs for every group size.
template <int G>
struct LanesPerRow {
  static constexpr int value = G <= 2 ? 4 : (G <= 4 ? 8 : 16);
};

static int launch_decode(const char *name, DecodeArgs a, int B, int H_q, int H_kv, int D,
                         int block_size, int W, bool listed, bool all_pages,
                         void *workspace, size_t workspace_bytes, hipStream_t st) {
  CVSA_REQUIRE(a.q && a.k_cache && a.v_cache && a.block_tables && a.ctx_lens,
               CVSA_ERR_INVALID, "%s: null pointer argument", name);
  CVSA_REQUIRE(B > 0 && B * (int64_t)H_kv <= 65535 && W > 0 && a.num_blocks > 0,
               CVSA_ERR_INVALID, "%s: bad sizes B=%d H_kv=%d W=%d", name, B, H_kv, W);
  CVSA_REQUIRE(H_kv > 0 && H_q > 0 && H_q % H_kv == 0, CVSA_ERR_INVALID,
               "%s: H_q=%d is not a multiple of H_kv=%d", name, H_q, H_kv);
  const int G = H_q / H_kv;
  CVSA_REQUIRE(G >= 1 && G <= 8, CVSA_ERR_UNSUPPORTED,
               "%s: GQA group size %d not in 1..8", name, G);
  CVSA_REQUIRE(D == kHeadDim && block_size == kPageTokens, CVSA_ERR_UNSUPPORTED,
               "%s: only D=128, block_size=16 are supported (got D=%d, bs=%d)", name, D,
               block_size);
  CVSA_REQUIRE(W <= kMaxPages, CVSA_ERR_UNSUPPORTED, "%s: W=%d exceeds %d pages", name, W,
               kMaxPages);
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
    CVSA_REQUIRE(a.max_sel >= 0 && a.max_sel <= kMaxPages && a.idx_stride >= a.max_sel,
                 CVSA_ERR_INVALID, "%s: bad selection width %d (row stride %lld)", name,
                 a.max_sel, (long long)a.idx_stride);
  }
  const bool want_unnorm = a.o_unnorm || a.m_out || a.l_out;
  CVSA_REQUIRE(!want_unnorm || (a.o_unnorm && a.m_out && a.l_out), CVSA_ERR_INVALID,
               "%s: o_unnorm, m_out and l_out must be given together", name);
  CVSA_REQUIRE(want_unnorm || a.out, CVSA_ERR_INVALID, "%s: no output requested", name);
  CVSA_REQUIRE(a.out == nullptr || (a.out_dtype >= CVSA_DTYPE_BF16 &&
                                    a.out_dtype <= CVSA_DTYPE_FP32),
               CVSA_ERR_INVALID, "%s: bad output dtype %d", name, a.out_dtype);

  const DecodePlan p = plan_decode(B, H_kv, listed ? a.max_sel : 0, W, listed, all_pages);
  const size_t need = workspace_bytes_for(B, H_q, H_kv, listed ? a.max_sel : 0, W, listed,
                                          all_pages);
  CVSA_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need &&
                                ((uintptr_t)workspace & 255) == 0),
               CVSA_ERR_WORKSPACE,
               "%s: workspace of %zu bytes (256-byte aligned) required, got %zu", name,
               need, workspace_bytes);
  a.pps_sel = p.pps_sel;
  a.pps_all = p.pps_all;
  a.n_splits = p.n_splits;

  a.W = W;
  a.H_kv = H_kv;
  a.scale = (float)pow((double)D, -0.5);
  a.counters = reinterpret_cast<unsigned *>(workspace);
  a.part = need == 0 ? nullptr
                     : reinterpret_cast<float *>(reinterpret_cast<char *>(workspace) +
                                                 counter_bytes(B * H_kv));
  const dim3 grid(p.n_splits, B * H_kv);
  const int mode = !listed ? kModeAll : (all_pages ? kModeVerified : kModeListed);
  const bool use_mfma = decode_engine() == 1;
#define CVSA_DEC_LAUNCH(GG, MM)                                                              \
  do {                                                                                       \
    if (use_mfma)                                                                            \
      hipLaunchKernelGGL((paged_decode_kernel<GG, MfmaEngine<GG>, kWavesPerWg, 2, MM>),      \
                         grid, dim3(kWavesPerWg * kWave), 0, st, a);                         \
    else                                                                                     \
      hipLaunchKernelGGL((paged_decode_kernel<GG, ValuEngine<GG, LanesPerRow<GG>::value>,    \
                                              kWavesPerWg, 2, MM>),                          \
                         grid, dim3(kWavesPerWg * kWave), 0, st, a);                         \
  } while (0)
#define CVSA_DEC_CASE(GG)                                                                    \
  case GG:                                                                                   \
    if (mode == kModeAll) CVSA_DEC_LAUNCH(GG, kModeAll);                                     \
    else if (mode == kModeListed) CVSA_DEC_LAUNCH(GG, kModeListed);                          \
    else CVSA_DEC_LAUNCH(GG, kModeVerified);                                                 \
    break;
  switch (G) {
    CVSA_DEC_CASE(1)
    CVSA_DEC_CASE(2)
    CVSA_DEC_CASE(3)
    CVSA_DEC_CASE(4)
    CVSA_DEC_CASE(5)
    CVSA_DEC_CASE(6)
    CVSA_DEC_CASE(7)
    CVSA_DEC_CASE(8)
    default:
      break;
  }
#undef CVSA_DEC_CASE
#undef CVSA_DEC_LAUNCH
  return cvsa_host::check_launch(name);
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
  (void)D;
  if (B <= 0 || H_kv <= 0 || H_q <= 0 || H_q % H_kv != 0 || W <= 0 || max_sel_pages < 0)
    return 0;
  const bool listed = max_sel_pages > 0;
  return workspace_bytes_for(B, H_q, H_kv, max_sel_pages, W, listed, all_pages != 0);
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
