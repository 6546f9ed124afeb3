// Top-k page selection and the coverage gate.
//
// Selection replaces the uniform-budget branch of CVSABackend._scoring_step
// (cvsa/backend.py:737-747): the `budget` largest page scores of each
// (b, kv-head) row.  torch.topk(sorted=False) leaves the order of its result
// unspecified; this kernel fixes it: the set is ordered by (score desc,
// page asc), and written in ascending page order.  Because invalid pages
// (-inf) are exactly the pages >= n_valid, the first n_per_head =
// min(budget, n_valid) entries are then always valid pages.
//
// The coverage gate follows _coverage_kernel (cvsa/kernels/coverage.py:
// 159-215): lse_all over every page score with the -1e20 floor and the
// +1e-30 inside the log (:183-195), lse_sel over the first n_sel selected
// scores (:198-208), coverage = exp(lse_sel - lse_all) and accept =
// coverage >= tau compared in fp32 (:211-212).
//
// One 1024-thread workgroup per (b, kv-head); thread t owns the R
// consecutive pages [t*R, t*R + R).  The k-th largest score is found in two
// steps: a 4096-bucket histogram over the row's finite value range [min, max]
// (the bucket of a value is a non-decreasing function of it, so the k-th
// largest lies in the bucket where the count from the top reaches k), then
// one wave ranks the few scores of that bucket against each other.  Rows
// where that bucket holds more than 64 scores (heavy ties, extreme
// outliers) or that hold +inf / NaN fall back to a 4-pass, 8-bit MSB radix
// select over order-preserving integer keys.  A block scan then places the
// selected pages in ascending order.
//
// A workgroup per row makes these kernels a chain of short dependent steps
// on one CU, so latency is what counts: every barrier in this file orders
// LDS only (lds_barrier), which keeps global loads in flight across it and
// never waits for earlier global stores, and loads are issued as early as
// the step that needs them allows.
#include "cvsa_common.h"
#include "internal.h"

namespace cvsa {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;
constexpr int kHistCopies = 16;
constexpr int kHistStride = 257;
constexpr int kBuckets = 4096;                          // value buckets of the first step
constexpr int kBucketsPerThread = kBuckets / kSelThreads;
constexpr int kRankCands = kWave;                       // scores one wave ranks directly

// Unsigned key in the order of the float, with -0 and +0 one key (they
// compare equal, so the lower page wins between them).
__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  u = u == 0x80000000u ? 0u : u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Bucket of a finite score in [vmin, vmin + kBuckets / inv]: a composition of
// correctly rounded, monotone operations, so it never decreases as v grows,
// and every evaluation gives the same bits (no fast-math in this library).
__device__ __forceinline__ int value_bucket(float v, float vmin, float inv) {
  return (int)fminf((v - vmin) * inv, (float)(kBuckets - 1));
}

// Block-wide max of two keys and sum of one counter, one barrier.  `red`
// holds 3 x kSelWaves words and is not reused by another reduction.
__device__ __forceinline__ void block_range(uint32_t &kmax, uint32_t &kneg, uint32_t &cnt,
                                            uint32_t (*red)[3]) {
  kmax = wave_max_u32(kmax);
  kneg = wave_max_u32(kneg);
  cnt = wave_sum_u32(cnt);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red[wave][0] = kmax;
    red[wave][1] = kneg;
    red[wave][2] = cnt;
  }
  lds_barrier();
  kmax = red[0][0];
  kneg = red[0][1];
  cnt = red[0][2];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) {
    kmax = max(kmax, red[w][0]);
    kneg = max(kneg, red[w][1]);
    cnt += red[w][2];
  }
}

// Counter update whose result is not waited for (a no-return atomic).
__device__ __forceinline__ void stat_add(long long *p, long long v) {
  __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exclusive prefix sum of one uint32 per thread over the block, plus total.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *wsum,
                                                         uint32_t &total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t incl = wave_incl_scan_u32(v);
  lds_barrier();
  if (lane == 63) wsum[wave] = incl;
  lds_barrier();
  uint32_t before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const uint32_t s = wsum[w];
    before += (w < wave) ? s : 0u;
    tot += s;
  }
  total = tot;
  return before + incl - v;
}

// Exclusive prefix sum of one uint64 per thread over the block, plus total.
__device__ __forceinline__ unsigned long long block_exclusive_scan_u64(
    unsigned long long v, unsigned long long *wsum64, unsigned long long &total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  unsigned long long incl = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const unsigned long long o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  lds_barrier();
  if (lane == 63) wsum64[wave] = incl;
  lds_barrier();
  unsigned long long before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kSelWaves; ++w) {
    const unsigned long long x = wsum64[w];
    before += (w < wave) ? x : 0ull;
    tot += x;
  }
  total = tot;
  return before + incl - v;
}

// lse over a set given its fp32 maximum `mx` and sum of exp(s - M); the
// reference floors the running max at -1e20 (coverage.py:183, :207).
__device__ __forceinline__ float lse_from(float mx_floor, float sum) {
  return mx_floor + logf(sum + 1e-30f);
}

// Max (first) and sum (second) of two values over the block; `red` holds
// 2 x kSelWaves floats and is not reused by the other.
__device__ __forceinline__ void block_max2(float &a, float &b, float (*red)[2]) {
  a = wave_max_from_groups<1>(a);
  b = wave_max_from_groups<1>(b);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red[wave][0] = a;
    red[wave][1] = b;
  }
  lds_barrier();
  a = red[0][0];
  b = red[0][1];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) {
    a = fmaxf(a, red[w][0]);
    b = fmaxf(b, red[w][1]);
  }
}

// Sums of a and b and the max of c over the block in one barrier; `red`
// holds 3 x kSelWaves floats and is not reused by another reduction.
__device__ __forceinline__ void block_sum2_max1(float &a, float &b, float &c, float (*red)[3]) {
  a = wave_sum_from_groups<1>(a);
  b = wave_sum_from_groups<1>(b);
  c = wave_max_from_groups<1>(c);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red[wave][0] = a;
    red[wave][1] = b;
    red[wave][2] = c;
  }
  lds_barrier();
  a = red[0][0];
  b = red[0][1];
  c = red[0][2];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) {
    a += red[w][0];
    b += red[w][1];
    c = fmaxf(c, red[w][2]);
  }
}

__device__ __forceinline__ void block_sum1(float &a, float *red) {
  a = wave_sum_from_groups<1>(a);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = a;
  lds_barrier();
  a = red[0];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) a += red[w];
}

__device__ __forceinline__ void block_sum2(float &a, float &b, float (*red)[2]) {
  a = wave_sum_from_groups<1>(a);
  b = wave_sum_from_groups<1>(b);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red[wave][0] = a;
    red[wave][1] = b;
  }
  lds_barrier();
  a = red[0][0];
  b = red[0][1];
#pragma unroll
  for (int w = 1; w < kSelWaves; ++w) {
    a += red[w][0];
    b += red[w][1];
  }
}

// One pass of the MSB radix select: hist_c holds kHistCopies copies of the
// histogram of the pass's 8-bit digit over the keys still in the running
// (behind an LDS barrier); returns the digit holding the krem-th largest of
// them and krem minus the number of those keys with a higher digit.  Ends
// with the histograms free for the next pass.
__device__ __forceinline__ void radix_digit(const uint32_t *hist_c, uint32_t *hist,
                                            uint32_t krem, uint32_t *s_digit, uint32_t *s_krem,
                                            uint32_t &digit, uint32_t &krem_out) {
  const int t = threadIdx.x, lane = t & 63;
  if (t < 256) {
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < kHistCopies; ++j) c += hist_c[j * kHistStride + t];
    hist[t] = c;
  }
  lds_barrier();
  if (t < 64) {
    // Lane l holds digits 4l..4l+3; count the candidates above each digit.
    const uint32_t c0 = hist[4 * lane], c1 = hist[4 * lane + 1];
    const uint32_t c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
    const uint32_t local = c0 + c1 + c2 + c3;
    uint32_t suffix = local;  // inclusive sum over lanes >= l
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t o = __shfl_down(suffix, off, 64);
      if (lane + off < 64) suffix += o;
    }
    uint32_t above = suffix - local;  // candidates with a higher digit
    const uint32_t cs[4] = {c3, c2, c1, c0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (above < krem && above + cs[j] >= krem) {
        *s_digit = (uint32_t)(4 * lane + 3 - j);
        *s_krem = krem - above;
      }
      above += cs[j];
    }
  }
  lds_barrier();
  digit = *s_digit;
  krem_out = *s_krem;
  lds_barrier();
}

// 4-pass, 8-bit MSB radix select of the k-th largest key among the keys
// with alive(r) set: returns that key T and k - #(alive keys > T), the
// number of keys equal to T that the selection takes.  Every lane adds
// into copy (lane % kHistCopies) of the histogram, rows padded by one word so
// that the copies of a bin sit in different LDS banks: scores cluster in a
// few leading digits, so lanes of one instruction often hit the same bin.
template <int R, typename Alive>
__device__ __forceinline__ void radix_select(const float (&val)[R], Alive alive, uint32_t k,
                                             uint32_t *hist, uint32_t *hist_c,
                                             uint32_t *s_digit, uint32_t *s_krem,
                                             uint32_t &T, uint32_t &krem) {
  const int t = threadIdx.x, lane = t & 63;
  uint32_t prefix = 0, pmask = 0;
  krem = k;
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = t; i < kHistCopies * kHistStride; i += kSelThreads) hist_c[i] = 0;
    lds_barrier();
    uint32_t *my_hist = hist_c + (lane % kHistCopies) * kHistStride;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t key = order_key(val[r]);
      if (alive(r) && (key & pmask) == prefix) atomicAdd(&my_hist[(key >> shift) & 255u], 1u);
    }
    lds_barrier();
    uint32_t digit;
    radix_digit(hist_c, hist, krem, s_digit, s_krem, digit, krem);
    prefix |= digit << shift;
    pmask |= 0xFFu << shift;
  }
  T = prefix;
}

// The lazy coverage check decided on the device (CVSABackend._lazy_step,
// cvsa/backend.py:420-465), shared by the select kernels: when every head of
// the layer kept its coverage on the cached selection (check_accept), that
// selection stays and all heads are accepted (returns true: the workgroup
// has nothing left to do); otherwise a fresh selection replaces it in place.
// Counters: stats[0] accept-all checks, [1] rejections, [2] scoring steps,
// [3] heads that passed the check.  All barriers here order LDS only.
__device__ __forceinline__ bool lazy_decision(
    const uint8_t *__restrict__ check_accept, int n_heads, int bh, int b, int width,
    int block_size, const int32_t *__restrict__ n_per_head,
    const int32_t *__restrict__ context_lens, uint8_t *__restrict__ accept_out,
    long long *__restrict__ stats, int count_gate, int32_t *__restrict__ keep_flag,
    unsigned long long *__restrict__ keep_work, int &s_nok, int &s_nbad) {
  const int t = threadIdx.x;
  if (check_accept != nullptr) {
    // A kept speculation's booking (below) needs these: requested with the
    // flags, in the same round trip.
    int spec_ran = 0, n_row = 0, ctx_row = 0;
    if (keep_work != nullptr && t == 0) {
      spec_ran = keep_flag[1];
      n_row = n_per_head[bh];
      ctx_row = context_lens[b];
    }
    int nok;
    bool all_ok;
    if (n_heads <= kWave) {  // uniform
      // Every wave reads the flags itself (one per lane): no barrier.
      const int lane = t & 63;
      nok = __popcll(__ballot(lane < n_heads && check_accept[lane] != 0));
      all_ok = nok == n_heads;
    } else {
      if (t == 0) {
        s_nok = 0;
        s_nbad = 0;
      }
      lds_barrier();
      int cnt = 0, bad = 0;
      for (int i = t; i < n_heads; i += kSelThreads) {
        const int v = check_accept[i] != 0;
        cnt += v;
        bad |= !v;
      }
      if (cnt) atomicAdd(&s_nok, cnt);
      if (bad) s_nbad = 1;
      lds_barrier();
      nok = s_nok;
      all_ok = s_nbad == 0;
    }
    if (stats != nullptr && bh == 0 && t == 0) {
      stat_add(&stats[0], all_ok ? 1 : 0);
      stat_add(&stats[1], all_ok ? 0 : 1);
      stat_add(&stats[2], all_ok ? 0 : 1);
      stat_add(&stats[3], nok);
    }
    // The decision, for the next check's speculative decode (a step plan's
    // prediction that the check keeps its selection).
    if (keep_flag != nullptr && bh == 0 && t == 0) *keep_flag = all_ok ? 1 : 0;
    if (all_ok) {
      if (t == 0) {
        accept_out[bh] = 1;
        // A kept selection whose speculative listed decode already ran
        // (keep_flag[1] == 1; 2 is the dense speculation, whose outputs the
        // verified decode replaces): the effective-budget counters of that
        // decode's walk of this row (what the verified decode would book),
        // so the verified decode after it has nothing left to do.
        if (keep_work != nullptr && spec_ran == 1) {
          atomicAdd(&keep_work[0], (unsigned long long)min(max(n_row, 0), width));
          atomicAdd(&keep_work[1], (unsigned long long)max(0, n_valid_pages(ctx_row, block_size)));
        }
      }
      return true;
    }
  } else if (stats != nullptr && !count_gate && bh == 0 && t == 0) {
    stat_add(&stats[1], 1);  // a lazy scoring step without a cached selection
    stat_add(&stats[2], 1);
  }
  return false;
}

// Row budgets (MODE): kUniform, the same `budget` for every row;
// kTopP, the smallest prefix of the row's pages by score whose softmax mass
// reaches top_p (CVSABackend._topp_select, backend.py:652-681), at least 3;
// kTable, row_budgets[b * H_kv + h] (_static_select, :622-650, and the
// budgets of _adaptive_select, :522-570).  `width` is the row stride of
// page_indices: k is clamped to it.
enum { kUniform = 0, kTopP = 1, kTable = 2 };
static_assert(kHistCopies * kHistStride >= kBuckets, "hist_c holds a second-level histogram");

// SEP: the selection ranks sel_scores while the coverage gate (and
// scores_cache) use scores (CVSABackend._scoring_step, backend.py:723-727:
// the Quest selector proposes, the exact scan verifies).
template <int R, bool SEP, int MODE>
__global__ __launch_bounds__(kSelThreads) void select_topk_kernel(
    const float *__restrict__ scores, const float *__restrict__ sel_scores, int W, int H_kv,
    const int32_t *__restrict__ context_lens, int block_size, int budget, int width,
    float top_p, const int32_t *__restrict__ row_budgets,
    int32_t *__restrict__ page_indices, int32_t *__restrict__ n_per_head, float tau,
    uint8_t *__restrict__ accept_out, float *__restrict__ coverage_out,
    const uint8_t *__restrict__ check_accept, int n_heads, float *__restrict__ scores_cache,
    long long *__restrict__ stats, int count_gate, int32_t *__restrict__ keep_flag,
    uint8_t *__restrict__ sel_map, int64_t map_stride,
    unsigned long long *__restrict__ keep_work, int exp_budget,
    int32_t *__restrict__ exp_indices) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t hist_c[kHistCopies * kHistStride];
  __shared__ uint32_t hist_b[kBuckets];
  __shared__ uint32_t s_cand[kRankCands];
  __shared__ uint32_t wsum[kSelWaves];
  __shared__ uint32_t red_rng[kSelWaves][3];
  __shared__ float red_max[kSelWaves][2], red_sum[kSelWaves][2], red_s3[kSelWaves][3];
  __shared__ float red_s1[kSelWaves];
  __shared__ uint32_t s_digit, s_krem, s_T, s_bucket, s_kb, s_nb, s_ncand;
  __shared__ int s_nok, s_nbad, s_acc;
  // Top-p only: softmax mass per value bucket (64-bit fixed point, so the
  // sums do not depend on the order of the atomic adds).
  __shared__ unsigned long long mass_b[MODE == kTopP ? kBuckets : 1];
  __shared__ unsigned long long s_candm[MODE == kTopP ? kRankCands : 1];
  __shared__ uint32_t s_candi[MODE == kTopP ? kRankCands : 1];
  __shared__ unsigned long long wsum64[MODE == kTopP ? kSelWaves : 1];
  __shared__ unsigned long long s_mass;

  const int bh = blockIdx.x;
  const int b = bh / H_kv;
  const int t = threadIdx.x;
  const float *row = (SEP ? sel_scores : scores) + (int64_t)bh * W;
  const int i0 = t * R;
  // 16-byte loads when W % 4 == 0 (row starts are then 16-byte aligned and
  // each group of 4 lies wholly inside or outside the row).  The choice is
  // uniform and the loads are unconditional (clamped into the row, values
  // past it replaced by -inf): per-lane branches around loads would make the
  // compiler wait for all of them at the first later use of any.
  const bool vec = R >= 4 && (W & 3) == 0;

  // The lazy check's keep decision (lazy_decision).  The scores are
  // requested only once a reselection is certain: a wave cannot retire
  // before its loads return, so loads issued ahead would hold up the
  // (common) keep path.
  // All barriers below order LDS only: loads stay in flight across them and
  // stores issued before them are not waited for.  (Scalar loads count
  // with LDS operations, so even a context-length load here would hold up
  // the check's barriers.)
  if (lazy_decision(check_accept, n_heads, bh, b, width, block_size, n_per_head, context_lens,
                    accept_out, stats, count_gate, keep_flag, keep_work, s_nok, s_nbad))
    return;

  const int ctx = context_lens[b];
  auto load_row = [&](const float *src, float (&dst)[R]) {
    if (vec) {
#pragma unroll
      for (int r = 0; r < R; r += 4) {
        const float4 v4 = *reinterpret_cast<const float4 *>(src + min(i0 + r, W - 4));
        dst[r] = v4.x;
        dst[r + 1 < R ? r + 1 : r] = v4.y;
        dst[r + 2 < R ? r + 2 : r] = v4.z;
        dst[r + 3 < R ? r + 3 : r] = v4.w;
      }
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r) dst[r] = src[min(i0 + r, W - 1)];
    }
#pragma unroll
    for (int r = 0; r < R; ++r) dst[r] = i0 + r < W ? dst[r] : -INFINITY;
  };
  float val[R];  // scores the selection ranks
  load_row(row, val);
  float gv[SEP ? R : 1];  // scores of the coverage gate when they differ
  if constexpr (SEP) load_row(scores + (int64_t)bh * W, gv);
  auto gate = [&](int r) -> float {
    if constexpr (SEP) return gv[r];
    else return val[r];
  };

  if (scores_cache != nullptr) {
    float *dst = scores_cache + (int64_t)bh * W + i0;
    if (vec) {
#pragma unroll
      for (int r = 0; r < R; r += 4)
        if (i0 + r < W)
          *reinterpret_cast<float4 *>(dst + r) = make_float4(
              gate(r), gate(r + 1 < R ? r + 1 : r), gate(r + 2 < R ? r + 2 : r),
              gate(r + 3 < R ? r + 3 : r));
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (i0 + r < W) dst[r] = gate(r);
    }
  }

  // ---- the budget-th largest key T and krem = budget - #(keys > T)
  // Range of the finite scores (as keys) and their count; +inf / NaN
  // entries are counted in the high half of `cnt`.  -inf (pages past the
  // context) lies below every finite score.
  for (int i = t; i < kBuckets; i += kSelThreads) hist_b[i] = 0;
  if (t == 0) s_ncand = 0;
  uint32_t kmax = 0, kneg = 0, cnt = 0;
  const auto finite = [&](int r) { return i0 + r < W && fabsf(val[r]) <= 3.402823466e38f; };
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (finite(r)) {
      const uint32_t key = order_key(val[r]);
      kmax = max(kmax, key);
      kneg = max(kneg, ~key);
      cnt += 1;
    } else if (i0 + r < W && val[r] != -INFINITY) {
      cnt += 1u << 16;
    }
  }
  block_range(kmax, kneg, cnt, red_rng);
  const uint32_t kmin = ~kneg, n_fin = cnt & 0xFFFFu, n_odd = cnt >> 16;
  float vmin = 0.f, inv = 0.f;
  const auto bucket = [&](int r) { return finite(r) ? value_bucket(val[r], vmin, inv) : -1; };

  // Top-p budget: 1 + the number of pages, in descending score order, whose
  // inclusive cumulative softmax mass is below top_p, clamped to [3, W]
  // (backend.py:672-678).  exp(s - max) is summed as 40-bit fixed point.
  // The page where the mass crosses top_p * total is found by the same value
  // buckets as the top-k (mass per bucket, scanned from the top), then among
  // that bucket's scores: ranked exactly when they are at most 64, else
  // through a second 4096-bucket level inside the bucket, whose crossing
  // bucket is then walked in page order (its scores differ by at most
  // 2^-24 of the row's range, or are equal).
  const auto find_cross = [&](const uint32_t *cnts, const unsigned long long *ms,
                              unsigned long long base, unsigned long long target)
                              __attribute__((always_inline)) {
    uint32_t c[kBucketsPerThread], lc = 0;
    unsigned long long m[kBucketsPerThread], lm = 0;
#pragma unroll
    for (int j = 0; j < kBucketsPerThread; ++j) {
      const int idx = kBuckets - 1 - (kBucketsPerThread * t + j);
      c[j] = cnts[idx];
      m[j] = ms[idx];
      lc += c[j];
      lm += m[j];
    }
    if (t == 0) s_bucket = 0xFFFFFFFFu;
    uint32_t ctot;
    unsigned long long mtot;
    uint32_t cab = block_exclusive_scan(lc, wsum, ctot);
    unsigned long long mab = base + block_exclusive_scan_u64(lm, wsum64, mtot);
#pragma unroll
    for (int j = 0; j < kBucketsPerThread; ++j) {
      if (mab < target && mab + m[j] >= target) {
        s_bucket = (uint32_t)(kBuckets - 1 - (kBucketsPerThread * t + j));
        s_kb = cab;
        s_nb = c[j];
        s_mass = mab;
      }
      cab += c[j];
      mab += m[j];
    }
    lds_barrier();
  };
  const auto topp_budget = [&](bool &hist_ready) __attribute__((always_inline)) -> int {
    // A row holding +inf / NaN, or no finite score, has a NaN softmax in
    // the reference: no prefix counts as below top_p, need = 1.
    if (n_odd != 0 || n_fin == 0) return min(3, W);
    const float M = key_value(kmax);
    const auto mass = [&](int r) __attribute__((always_inline)) -> unsigned long long {
      return finite(r) ? (unsigned long long)(expf(val[r] - M) * 1099511627776.0f) : 0ull;
    };
    unsigned long long part = 0, total = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) part += mass(r);
    (void)block_exclusive_scan_u64(part, wsum64, total);
    const unsigned long long target =
        (unsigned long long)ceil((double)top_p * (double)total);
    uint32_t before = 0;          // pages ranked above the range still to walk
    unsigned long long base = 0;  // their mass
    int lvl = 0, b1 = -1, b2 = -1;
    float vmin2 = 0.f, inv2 = 0.f;
    const float lo = key_value(kmin);
    const float inv1 = (float)kBuckets / (M - lo);
    if (kmin != kmax && inv1 > 0.f && inv1 <= 3.402823466e38f) {
      vmin = lo;  // the buckets of the top-k below
      inv = inv1;
      for (int i = t; i < kBuckets; i += kSelThreads) mass_b[i] = 0ull;
      lds_barrier();
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int bk = bucket(r);
        if (bk >= 0) {
          atomicAdd(&hist_b[bk], 1u);
          atomicAdd(&mass_b[bk], mass(r));
        }
      }
      lds_barrier();
      hist_ready = true;
      find_cross(hist_b, mass_b, 0ull, target);
      if (s_bucket == 0xFFFFFFFFu) return min(max((int)n_fin, 3), W);  // not reached
      b1 = (int)s_bucket;
      before = s_kb;
      base = s_mass;
      const uint32_t nb = s_nb;
      lvl = 1;
      if (nb <= (uint32_t)kRankCands) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (bucket(r) == b1) {
            const uint32_t slot = atomicAdd(&s_ncand, 1u);
            s_cand[slot] = order_key(val[r]);
            s_candm[slot] = mass(r);
            s_candi[slot] = (uint32_t)(i0 + r);
          }
        }
        lds_barrier();
        if (t < kWave) {
          uint32_t lt = 0;
          if (t < (int)nb) {
            const uint32_t key = s_cand[t], idx = s_candi[t];
            unsigned long long prefix = 0;
            for (uint32_t j = 0; j < nb; ++j) {
              const uint32_t kj = s_cand[j];
              prefix += (kj > key || (kj == key && s_candi[j] < idx)) ? s_candm[j] : 0ull;
            }
            lt = base + prefix + s_candm[t] < target ? 1u : 0u;
          }
          lt = wave_sum_u32(lt);
          if (t == 0) {
            s_kb = lt;
            s_ncand = 0;  // the top-k gathers its own candidates
          }
        }
        lds_barrier();
        return min(max((int)(before + s_kb + 1), 3), W);
      }
      // Second level: the key range of bucket b1's scores.
      uint32_t kx = 0, kn = 0, cn = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        if (bucket(r) == b1) {
          const uint32_t key = order_key(val[r]);
          kx = max(kx, key);
          kn = max(kn, ~key);
        }
      }
      block_range(kx, kn, cn, red_rng);
      if (kx != ~kn) {
        vmin2 = key_value(~kn);
        inv2 = (float)kBuckets / (key_value(kx) - vmin2);
        if (inv2 > 0.f && inv2 <= 3.402823466e38f) {
          for (int i = t; i < kBuckets; i += kSelThreads) {
            hist_c[i] = 0u;
            mass_b[i] = 0ull;
          }
          lds_barrier();
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (bucket(r) == b1) {
              const int bk = value_bucket(val[r], vmin2, inv2);
              atomicAdd(&hist_c[bk], 1u);
              atomicAdd(&mass_b[bk], mass(r));
            }
          }
          lds_barrier();
          find_cross(hist_c, mass_b, base, target);
          if (s_bucket != 0xFFFFFFFFu) {
            b2 = (int)s_bucket;
            before += s_kb;
            base = s_mass;
            lvl = 2;
          }
        }
      }
    }
    // The remaining range in page order.
    const auto in_range = [&](int r) __attribute__((always_inline)) {
      if (!finite(r)) return false;
      if (lvl == 0) return true;
      if (bucket(r) != b1) return false;
      return lvl == 1 || value_bucket(val[r], vmin2, inv2) == b2;
    };
    unsigned long long mine = 0, tot = 0;
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (in_range(r)) mine += mass(r);
    unsigned long long run = base + block_exclusive_scan_u64(mine, wsum64, tot);
    uint32_t lt = 0, lt_total = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (in_range(r)) {
        run += mass(r);
        lt += run < target ? 1u : 0u;
      }
    }
    (void)block_exclusive_scan(lt, wsum, lt_total);
    return min(max((int)(before + lt_total + 1), 3), W);
  };

  // The row's budget k.
  int k = budget;
  bool hist_ready = false;  // hist_b already holds the bucket counts
  if constexpr (MODE == kTable) k = min(max(row_budgets[bh], 1), W);
  if constexpr (MODE == kTopP) k = topp_budget(hist_ready);
  k = min(k, width);  // a row holds at most `width` pages: the best ones

  // The kk-th largest key T and krem = kk - #(keys > T).  Plan 0: T and
  // krem found directly; 1: radix select over the row; 2: radix select of
  // the k_radix-th largest inside bucket bstar.  Called a second time for
  // the expanded selection of approximate recovery (its bucket counts are
  // those of the first call).
  const auto threshold = [&](int kk, uint32_t &T, uint32_t &krem) __attribute__((always_inline)) {
    uint32_t k_radix = (uint32_t)kk;
    int plan = 1, bstar = -1;
    if (n_odd == 0 && (uint32_t)kk > n_fin) {
      // Every finite page, then the lowest -inf pages.
      T = order_key(-INFINITY);
      krem = (uint32_t)kk - n_fin;
      plan = 0;
    } else if (n_odd == 0 && kmin == kmax) {
      T = kmax;
      krem = (uint32_t)kk;
      plan = 0;
    } else if (n_odd == 0) {
      vmin = key_value(kmin);
      inv = (float)kBuckets / (key_value(kmax) - vmin);
      // Otherwise max - min overflows.
      if (inv > 0.f && inv <= 3.402823466e38f) {
        if (!hist_ready) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int bk = bucket(r);
            if (bk >= 0) atomicAdd(&hist_b[bk], 1u);
          }
          hist_ready = true;
        }
        lds_barrier();
        // Thread t holds buckets kBuckets-1-(4t+j), j = 0..3: the exclusive
        // scan over threads counts the scores in higher buckets.
        uint32_t c[kBucketsPerThread], local = 0;
#pragma unroll
        for (int j = 0; j < kBucketsPerThread; ++j) {
          c[j] = hist_b[kBuckets - 1 - (kBucketsPerThread * t + j)];
          local += c[j];
        }
        uint32_t total_b;
        uint32_t above = block_exclusive_scan(local, wsum, total_b);
#pragma unroll
        for (int j = 0; j < kBucketsPerThread; ++j) {
          if (above < (uint32_t)kk && above + c[j] >= (uint32_t)kk) {
            s_bucket = (uint32_t)(kBuckets - 1 - (kBucketsPerThread * t + j));
            s_kb = (uint32_t)kk - above;
            s_nb = c[j];
          }
          above += c[j];
        }
        lds_barrier();
        bstar = (int)s_bucket;
        const uint32_t kb = s_kb, nb = s_nb;
        // The buckets are recomputed below rather than kept live across the
        // scan (same operands, same bits).
        asm volatile("" : "+v"(vmin), "+v"(inv));
        if (nb <= (uint32_t)kRankCands) {
          // Rank the bucket's scores: T is the key with gt < kb <= gt + eq.
#pragma unroll
          for (int r = 0; r < R; ++r)
            if (bucket(r) == bstar) s_cand[atomicAdd(&s_ncand, 1u)] = order_key(val[r]);
          lds_barrier();
          if (t < kWave) {
            const uint32_t mine = t < (int)nb ? s_cand[t] : 0u;
            uint32_t gt = 0, eq = 0;
            for (uint32_t j = 0; j < nb; ++j) {
              const uint32_t o = s_cand[j];
              gt += o > mine;
              eq += o == mine;
            }
            if (t < (int)nb && gt < kb && kb <= gt + eq) {
              s_T = mine;
              s_krem = kb - gt;
            }
            if (t == 0) s_ncand = 0;  // every lane has read nb candidates
          }
          lds_barrier();
          T = s_T;
          krem = s_krem;
          plan = 0;
        } else {
          plan = 2;
          k_radix = kb;
        }
      }
    }
    if (plan != 0) {
      const auto alive = [&](int r) { return i0 + r < W && (plan == 1 || bucket(r) == bstar); };
      radix_select<R>(val, alive, k_radix, hist, hist_c, &s_digit, &s_krem, T, krem);
    }
  };

  // Ascending-order compaction of the selection (T, krem): the first
  // n_write entries into out_row; ties at T go to the lowest pages.  Sets
  // in[r] for this thread's pages among the first n_sel entries.
  const auto compact = [&](uint32_t T, uint32_t krem, int n_write, int n_sel, int32_t *out_row,
                           bool (&in)[R]) __attribute__((always_inline)) {
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (i0 + r < W) {
        const uint32_t key = order_key(val[r]);
        gt += key > T;
        eq += key == T;
      }
    }
    uint32_t total;
    const uint32_t excl = block_exclusive_scan(gt | (eq << 16), wsum, total);
    const uint32_t gt_before = excl & 0xFFFFu, eq_before = excl >> 16;
    uint32_t eq_seen = eq_before;
    uint32_t pos = gt_before + min(eq_before, krem);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      bool sel = false;
      const uint32_t key = order_key(val[r]);
      if (i0 + r < W) {
        if (key > T) {
          sel = true;
        } else if (key == T) {
          sel = eq_seen < krem;
          ++eq_seen;
        }
      }
      in[r] = sel && (int)pos < n_sel;
      if (sel) {
        if ((int)pos < n_write) out_row[pos] = i0 + r;  // pos < kk for a correct select
        ++pos;
      }
    }
  };

  uint32_t T = 0, krem = 0;
  threshold(k, T, krem);
  const int n_sel = min(k, n_valid_pages(ctx, block_size));
  bool counted[R];
  compact(T, krem, k, n_sel, page_indices + (int64_t)bh * width, counted);
  if (t == 0) n_per_head[bh] = n_sel;
  if (sel_map != nullptr) {
    // The row's selection map: this thread's pages i0 .. i0 + R - 1.
    uint8_t *mrow = sel_map + (int64_t)bh * map_stride;
    if constexpr (R % 4 == 0) {
#pragma unroll
      for (int r = 0; r < R; r += 4)
        if (i0 + r < W)
          *reinterpret_cast<uint32_t *>(mrow + i0 + r) =
              (uint32_t)counted[r] | (uint32_t)counted[r + 1] << 8 |
              (uint32_t)counted[r + 2] << 16 | (uint32_t)counted[r + 3] << 24;
    } else {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (i0 + r < W) mrow[i0 + r] = counted[r] ? 1 : 0;
    }
  }

  if (accept_out == nullptr) return;
  // ---- coverage of the new selection
  // When the selection ranks the gate's scores and the row holds no +inf /
  // NaN, the maximum over every page is the row's largest finite score
  // (found with the value range above), and so, in all but odd cases (a
  // finite score past the valid pages), is the maximum over the counted
  // pages: that guess saves a block-wide max; the counted maximum is reduced
  // with the sums, and a wrong guess recomputes the selection's sum.
  const bool fast_max = !SEP && n_odd == 0;  // uniform
  float mx = -INFINITY, ms = -INFINITY;
  if (fast_max) {
    mx = n_fin > 0 ? key_value(kmax) : -INFINITY;
    ms = mx;
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      mx = fmaxf(mx, gate(r));
      if (counted[r]) ms = fmaxf(ms, gate(r));
    }
    block_max2(mx, ms, red_max);
  }
  const float m_all = fmaxf(mx, -1e20f);
  // Padding lanes of the reference's power-of-two selection block carry
  // -1e20 into the max whenever n_sel is below that block (coverage.py:205).
  int msel_block = 1;
  while (msel_block < width) msel_block <<= 1;
  float m_sel = n_sel < msel_block ? fmaxf(ms, -1e20f) : ms;
  float se = 0.f, ss = 0.f, ms_true = -INFINITY;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    se += fast_exp(gate(r) - m_all);
    if (counted[r]) {
      ss += fast_exp(gate(r) - m_sel);
      ms_true = fmaxf(ms_true, gate(r));
    }
  }
  if (fast_max) {
    block_sum2_max1(se, ss, ms_true, red_s3);
    if (ms_true != ms) {  // uniform; the counted pages miss the row's maximum
      m_sel = n_sel < msel_block ? fmaxf(ms_true, -1e20f) : ms_true;
      ss = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (counted[r]) ss += fast_exp(gate(r) - m_sel);
      block_sum1(ss, red_s1);
    }
  } else {
    block_sum2(se, ss, red_sum);
  }
  if (t == 0) {
    const float cov = expf(lse_from(m_sel, ss) - lse_from(m_all, se));
    const int acc = cov >= tau ? 1 : 0;
    coverage_out[bh] = cov;
    accept_out[bh] = (uint8_t)acc;
    s_acc = acc;
    if (stats != nullptr && count_gate) {
      // Fixed-interval scoring step (backend.py:859-863): tally this head,
      // then the last head of the call books the step as all-accepted or
      // not.  stats[4] (rejected heads of this call) and stats[5] (heads
      // done) are scratch that the last head clears again.  Ordering: every
      // atomic here is performed at the device's coherence point (agent
      // scope, no cached copy), and the s_waitcnt below makes this head's
      // stats[4] add complete before its stats[5] add is issued, so the
      // head that sees done == n_heads - 1 reads every head's stats[4]
      // add.  This rests on that gfx950 behaviour of atomics, not on a
      // release / acquire pairing of the HIP memory model.
      __hip_atomic_fetch_add(&stats[3], (long long)acc, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(&stats[4], (long long)(1 - acc), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      const long long done = __hip_atomic_fetch_add(&stats[5], 1LL, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
      if (done == (long long)n_heads - 1) {
        const long long rej = __hip_atomic_fetch_add(&stats[4], 0LL, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        stats[0] += rej == 0 ? 1 : 0;
        stats[1] += rej != 0 ? 1 : 0;
        stats[2] += 1;
        __hip_atomic_store(&stats[4], 0LL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&stats[5], 0LL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }

  // Approximate recovery (cvsa/backend.py:780-799): a row whose new
  // selection failed its gate also gets the exp_budget largest ranking
  // scores, in ascending page order, as its expanded selection (the
  // reference ranks every row; only rejected rows attend theirs).
  if constexpr (MODE == kUniform) {
    if (exp_indices == nullptr) return;  // uniform
    lds_barrier();
    if (s_acc != 0) return;  // uniform
    const int k2 = min(exp_budget, W);
    uint32_t T2 = 0, krem2 = 0;
    threshold(k2, T2, krem2);
    bool in2[R];
    compact(T2, krem2, k2, k2, exp_indices + (int64_t)bh * exp_budget, in2);
  }
}

// Rows wider than the register-resident kernel holds (W > kMaxPages, up to
// kMaxPagesWide pages): the same selection and gate (uniform or per-row
// table budgets), streaming the row from memory.  The k-th largest key T
// and krem come from the 4-pass 8-bit MSB radix select over the row's
// order keys (the register kernel's bucket step finds the same T and krem
// faster; here each pass reads the row), the ascending compaction walks
// the row in tiles of kWideTile pages (a block scan per tile, running
// counts between tiles), and the gate's two log-sum-exps take a pass of
// their own once the counted pages are known (a bit per page in LDS).
// Same outputs as select_topk_kernel: selection, n_per_head, selection
// map, scores cache, coverage and accept, the lazy check's decision and
// counters; the expanded selection of approximate recovery comes from
// expand_wide_kernel, launched after it.
constexpr int kWidePerThread = 4;  // pages per thread of a compaction tile
constexpr int kWideTile = kSelThreads * kWidePerThread;
// One workgroup streams its row, so the loads in flight bound the rate:
// strips of kStrip coalesced loads per thread (32 KiB per workgroup) in two
// buffers that alternate, so that one strip's loads are in flight while
// the other is used.  The loads are unconditional (addresses clamped into
// the row): loads under a branch make the compiler wait for every
// outstanding load at the join.
constexpr int kStrip = 8;

// f(i, row[i]) for every i in [0, n), in strips of kStrip coalesced loads
// per thread (element e of thread t at strip base + e * kSelThreads + t).
template <typename F>
__device__ __forceinline__ void stream_row(const float *__restrict__ row, int n, F &&f) {
  const int t = threadIdx.x;
  constexpr int kLen = kStrip * kSelThreads;
  const auto load = [&](float (&x)[kStrip], int base) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < kStrip; ++e) x[e] = row[min(base + e * kSelThreads + t, n - 1)];
  };
  const auto use = [&](const float (&x)[kStrip], int base) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < kStrip; ++e) {
      const int i = base + e * kSelThreads + t;
      if (i < n) f(i, x[e]);
    }
  };
  // The scheduling barriers keep the loads in program order (the compiler
  // would otherwise move one buffer's use, or its first loads, past the
  // other's loads and then wait for both).
  float a[kStrip], b[kStrip];
  load(a, 0);
  __builtin_amdgcn_sched_barrier(0);
  load(b, kLen);
  __builtin_amdgcn_sched_barrier(0);
  for (int base = 0; base < n; base += 2 * kLen) {
    use(a, base);
    load(a, base + 2 * kLen);
    __builtin_amdgcn_sched_barrier(0);
    use(b, base + kLen);
    load(b, base + 3 * kLen);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// LDS of the wide-row threshold: the radix histograms, the value-bucket
// histogram (in hist_c), the block reductions and the candidates of the
// k-th value bucket.
constexpr int kWideCands = 4 * kSelThreads;
struct WideLds {
  uint32_t hist[256];
  uint32_t hist_c[kHistCopies * kHistStride];
  uint32_t wsum[kSelWaves];
  uint32_t red_rng[kSelWaves][3];
  float cand[kWideCands];
  uint32_t digit, krem, bucket, kb, nb, ncand;
  int odd;
};

// 8-bit MSB radix select over a row in memory (four passes over it) of the
// k-th largest key among the pages with alive(v), as radix_select.
template <typename Alive>
__device__ __forceinline__ void wide_radix(const float *__restrict__ row, int W, uint32_t k,
                                           Alive alive, WideLds &L, uint32_t &T,
                                           uint32_t &krem) {
  const int t = threadIdx.x, lane = t & 63;
  uint32_t prefix = 0, pmask = 0;
  krem = k;
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = t; i < kHistCopies * kHistStride; i += kSelThreads) L.hist_c[i] = 0;
    lds_barrier();
    uint32_t *my_hist = L.hist_c + (lane % kHistCopies) * kHistStride;
    stream_row(row, W, [&](int, float v) {
      const uint32_t key = order_key(v);
      if ((key & pmask) == prefix && alive(v)) atomicAdd(&my_hist[(key >> shift) & 255u], 1u);
    });
    lds_barrier();
    uint32_t digit;
    radix_digit(L.hist_c, L.hist, krem, &L.digit, &L.krem, digit, krem);
    prefix |= digit << shift;
    pmask |= 0xFFu << shift;
  }
  T = prefix;
}

// The k-th largest key T of a row of W scores in memory and krem = k -
// #(keys > T), with the register kernel's plan: the range of the finite
// scores (one pass), their counts in kBuckets value buckets (one pass),
// then the bucket holding the k-th largest, whose scores (at most
// kWideCands: one more pass gathers them) are ranked in LDS; a larger
// bucket, or a row with +inf / NaN scores or too wide a range, takes the
// radix select over the row (restricted to that bucket when there is one).
__device__ __forceinline__ void wide_threshold(const float *__restrict__ row, int W, uint32_t k,
                                               WideLds &L, uint32_t &T, uint32_t &krem) {
  const int t = threadIdx.x, lane = t & 63;
  if (t == 0) {
    L.odd = 0;
    L.ncand = 0;
  }
  lds_barrier();
  // Range of the finite scores (as keys) and their count; any +inf / NaN
  // sets L.odd.  -inf lies below every finite score.
  uint32_t kmax = 0, kneg = 0, cnt = 0;
  stream_row(row, W, [&](int, float v) {
    if (fabsf(v) <= 3.402823466e38f) {
      const uint32_t key = order_key(v);
      kmax = max(kmax, key);
      kneg = max(kneg, ~key);
      cnt += 1;
    } else if (v != -INFINITY) {
      L.odd = 1;
    }
  });
  block_range(kmax, kneg, cnt, L.red_rng);  // its barrier also orders L.odd
  const uint32_t kmin = ~kneg, n_fin = cnt;
  const auto everything = [](float) { return true; };
  if (L.odd != 0) {  // uniform
    wide_radix(row, W, k, everything, L, T, krem);
    return;
  }
  if (k > n_fin) {  // every finite page, then the lowest -inf pages
    T = order_key(-INFINITY);
    krem = k - n_fin;
    return;
  }
  if (kmin == kmax) {
    T = kmax;
    krem = k;
    return;
  }
  const float vmin = key_value(kmin);
  const float inv = (float)kBuckets / (key_value(kmax) - vmin);
  if (!(inv > 0.f && inv <= 3.402823466e38f)) {  // max - min overflows
    wide_radix(row, W, k, everything, L, T, krem);
    return;
  }
  uint32_t *hist_b = L.hist_c;
  for (int i = t; i < kBuckets; i += kSelThreads) hist_b[i] = 0;
  lds_barrier();
  stream_row(row, W, [&](int, float v) {
    if (fabsf(v) <= 3.402823466e38f) atomicAdd(&hist_b[value_bucket(v, vmin, inv)], 1u);
  });
  lds_barrier();
  // Thread t holds buckets kBuckets-1-(4t+j), j = 0..3: the exclusive scan
  // over threads counts the scores in higher buckets.
  uint32_t c[kBucketsPerThread], local = 0;
#pragma unroll
  for (int j = 0; j < kBucketsPerThread; ++j) {
    c[j] = hist_b[kBuckets - 1 - (kBucketsPerThread * t + j)];
    local += c[j];
  }
  uint32_t total_b;
  uint32_t above = block_exclusive_scan(local, L.wsum, total_b);
#pragma unroll
  for (int j = 0; j < kBucketsPerThread; ++j) {
    if (above < k && above + c[j] >= k) {
      L.bucket = (uint32_t)(kBuckets - 1 - (kBucketsPerThread * t + j));
      L.kb = k - above;
      L.nb = c[j];
    }
    above += c[j];
  }
  lds_barrier();
  const int bstar = (int)L.bucket;
  const uint32_t kb = L.kb, nb = L.nb;
  const auto in_bucket = [&](float v) {
    return fabsf(v) <= 3.402823466e38f && value_bucket(v, vmin, inv) == bstar;
  };
  if (nb > (uint32_t)kWideCands) {  // uniform
    wide_radix(row, W, kb, in_bucket, L, T, krem);
    return;
  }
  // Gather the bucket's scores (a wave-aggregated append: exactly nb of
  // them, the same bucket function as the counts), then rank them.
  stream_row(row, W, [&](int, float v) {
    const bool take = in_bucket(v);
    const unsigned long long m = __ballot(take);
    if (m == 0ull) return;
    const int leader = __ffsll((long long)m) - 1;
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(&L.ncand, (uint32_t)__popcll(m));
    base = __shfl(base, leader, 64);
    if (take) L.cand[base + __popcll(m & ((1ull << lane) - 1ull))] = v;
  });
  lds_barrier();
  constexpr int RC = kWideCands / kSelThreads;
  float cv[RC];
#pragma unroll
  for (int r = 0; r < RC; ++r) cv[r] = L.cand[min(t + r * kSelThreads, kWideCands - 1)];
  const auto alive = [&](int r) { return (uint32_t)(t + r * kSelThreads) < nb; };
  radix_select<RC>(cv, alive, kb, L.hist, L.hist_c, &L.digit, &L.krem, T, krem);
}

// Ascending compaction of a wide row's selection (T, krem) into out_row
// (its first n_write entries; ties at T go to the lowest pages), in tiles of
// kWideTile pages: a block scan per tile, running counts between tiles.
// MAIN (the selection, not an expanded one) also writes the counted bits
// (pages among the first n_sel selected) into s_bits, the selection map row
// and the scores cache row (either may be null), and takes the gate maxima
// of `grow` over every page (mx) and over the counted pages (ms).
template <bool MAIN, bool SEP>
__device__ __forceinline__ void wide_compact(const float *__restrict__ row,
                                             const float *__restrict__ grow, int W, uint32_t T,
                                             uint32_t krem, int n_write, int n_sel,
                                             int32_t *__restrict__ out_row, uint32_t *wsum,
                                             uint32_t *s_bits, uint8_t *__restrict__ map_row,
                                             float *__restrict__ cache_row, float &mx,
                                             float &ms) {
  const int t = threadIdx.x;
  uint32_t gt_run = 0, eq_run = 0;  // keys > T and == T in the tiles before
  // Two tiles in alternating buffers: one tile's loads are in flight while
  // the other is compacted (unconditional loads at clamped addresses).
  constexpr bool G = SEP && MAIN;  // separate gate scores
  const auto fetch = [&](float (&v)[kWidePerThread], float (&g)[G ? kWidePerThread : 1],
                         int base) __attribute__((always_inline)) {
    const int p0 = base + t * kWidePerThread;
#pragma unroll
    for (int e = 0; e < kWidePerThread; ++e) v[e] = row[min(p0 + e, W - 1)];
    if constexpr (G) {
#pragma unroll
      for (int e = 0; e < kWidePerThread; ++e) g[e] = grow[min(p0 + e, W - 1)];
    }
  };
  const auto tile = [&](const float (&v)[kWidePerThread],
                        const float (&gs)[G ? kWidePerThread : 1], int base)
                        __attribute__((always_inline)) {
    const int p0 = base + t * kWidePerThread;
    const auto g = [&](int e) {
      if constexpr (G) return gs[e];
      else return v[e];
    };
    uint32_t gt = 0, eq = 0;
#pragma unroll
    for (int e = 0; e < kWidePerThread; ++e) {
      if (p0 + e < W) {
        const uint32_t key = order_key(v[e]);
        gt += key > T;
        eq += key == T;
      }
    }
    uint32_t total;
    const uint32_t excl = block_exclusive_scan(gt | (eq << 16), wsum, total);
    uint32_t eq_seen = eq_run + (excl >> 16);
    uint32_t pos = gt_run + (excl & 0xFFFFu) + min(eq_seen, krem);
    uint32_t bits = 0;
#pragma unroll
    for (int e = 0; e < kWidePerThread; ++e) {
      bool sel = false;
      if (p0 + e < W) {
        const uint32_t key = order_key(v[e]);
        if (key > T) {
          sel = true;
        } else if (key == T) {
          sel = eq_seen < krem;
          ++eq_seen;
        }
      }
      const bool counted = sel && (int)pos < n_sel;
      bits |= counted ? 1u << e : 0u;
      if (sel) {
        if ((int)pos < n_write) out_row[pos] = p0 + e;
        ++pos;
      }
      if (MAIN && p0 + e < W) {
        mx = fmaxf(mx, g(e));
        if (counted) ms = fmaxf(ms, g(e));
      }
    }
    if (MAIN && p0 < W) {
      atomicOr(&s_bits[p0 >> 5], bits << (p0 & 31));
      if (map_row != nullptr) {
#pragma unroll
        for (int e = 0; e < kWidePerThread; ++e)
          if (p0 + e < W) map_row[p0 + e] = (bits >> e) & 1u;
      }
      if (cache_row != nullptr) {
#pragma unroll
        for (int e = 0; e < kWidePerThread; ++e)
          if (p0 + e < W) cache_row[p0 + e] = g(e);
      }
    }
    gt_run += total & 0xFFFFu;
    eq_run += total >> 16;
  };
  float va[kWidePerThread], vb[kWidePerThread];
  float ga[G ? kWidePerThread : 1], gb[G ? kWidePerThread : 1];
  fetch(va, ga, 0);
  __builtin_amdgcn_sched_barrier(0);
  fetch(vb, gb, kWideTile);
  __builtin_amdgcn_sched_barrier(0);
  for (int base = 0; base < W; base += 2 * kWideTile) {
    tile(va, ga, base);
    fetch(va, ga, base + 2 * kWideTile);
    __builtin_amdgcn_sched_barrier(0);
    if (base + kWideTile < W) tile(vb, gb, base + kWideTile);  // uniform
    fetch(vb, gb, base + 3 * kWideTile);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <bool SEP, int MODE>
__global__ __launch_bounds__(kSelThreads) void select_topk_wide_kernel(
    const float *__restrict__ scores, const float *__restrict__ sel_scores, int W, int H_kv,
    const int32_t *__restrict__ context_lens, int block_size, int budget, int width,
    const int32_t *__restrict__ row_budgets, int32_t *__restrict__ page_indices,
    int32_t *__restrict__ n_per_head, float tau, uint8_t *__restrict__ accept_out,
    float *__restrict__ coverage_out, const uint8_t *__restrict__ check_accept, int n_heads,
    float *__restrict__ scores_cache, long long *__restrict__ stats, int count_gate,
    int32_t *__restrict__ keep_flag, uint8_t *__restrict__ sel_map, int64_t map_stride,
    unsigned long long *__restrict__ keep_work) {
  static_assert(MODE == kUniform || MODE == kTable, "wide rows: uniform or table budgets");
  __shared__ WideLds L;
  __shared__ uint32_t s_bits[kMaxPagesWide / 32];  // the counted pages
  __shared__ float red_max[kSelWaves][2], red_sum[kSelWaves][2];
  __shared__ int s_nok, s_nbad;

  const int bh = blockIdx.x;
  const int b = bh / H_kv;
  const int t = threadIdx.x;
  const float *row = (SEP ? sel_scores : scores) + (int64_t)bh * W;
  const float *grow = scores + (int64_t)bh * W;
  if (lazy_decision(check_accept, n_heads, bh, b, width, block_size, n_per_head, context_lens,
                    accept_out, stats, count_gate, keep_flag, keep_work, s_nok, s_nbad))
    return;
  const int ctx = context_lens[b];
  int k = budget;
  if constexpr (MODE == kTable) k = min(max(row_budgets[bh], 1), W);
  k = min(k, width);

  float mx = -INFINITY, ms = -INFINITY;  // gate maxima: every page, counted pages
  for (int i = t; i < (W + 31) / 32; i += kSelThreads) s_bits[i] = 0u;
  const int n_sel = min(k, n_valid_pages(ctx, block_size));
  uint32_t T = 0, krem = 0;
  wide_threshold(row, W, (uint32_t)k, L, T, krem);
  wide_compact<true, SEP>(row, grow, W, T, krem, k, n_sel, page_indices + (int64_t)bh * width,
                          L.wsum, s_bits,
                          sel_map != nullptr ? sel_map + (int64_t)bh * map_stride : nullptr,
                          scores_cache != nullptr ? scores_cache + (int64_t)bh * W : nullptr,
                          mx, ms);
  if (t == 0) n_per_head[bh] = n_sel;
  if (accept_out == nullptr) return;

  // ---- coverage of the new selection (the register kernel's rules)
  block_max2(mx, ms, red_max);  // also orders the counted bits before their reads
  const float m_all = fmaxf(mx, -1e20f);
  int msel_block = 1;
  while (msel_block < width) msel_block <<= 1;
  const float m_sel = n_sel < msel_block ? fmaxf(ms, -1e20f) : ms;
  float se = 0.f, ss = 0.f;
  stream_row(grow, W, [&](int p, float g) {
    se += fast_exp(g - m_all);
    if ((s_bits[p >> 5] >> (p & 31)) & 1u) ss += fast_exp(g - m_sel);
  });
  block_sum2(se, ss, red_sum);
  if (t == 0) {
    const float cov = expf(lse_from(m_sel, ss) - lse_from(m_all, se));
    const int acc = cov >= tau ? 1 : 0;
    coverage_out[bh] = cov;
    accept_out[bh] = (uint8_t)acc;
    if (stats != nullptr && count_gate) {
      // As in select_topk_kernel: the last head of a fixed-interval scoring
      // step books it (the same gfx950 ordering of agent-scope atomics).
      __hip_atomic_fetch_add(&stats[3], (long long)acc, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(&stats[4], (long long)(1 - acc), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      const long long done = __hip_atomic_fetch_add(&stats[5], 1LL, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
      if (done == (long long)n_heads - 1) {
        const long long rej = __hip_atomic_fetch_add(&stats[4], 0LL, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        stats[0] += rej == 0 ? 1 : 0;
        stats[1] += rej != 0 ? 1 : 0;
        stats[2] += 1;
        __hip_atomic_store(&stats[4], 0LL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&stats[5], 0LL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
}

// Approximate recovery of wide rows: a rejected row's expanded selection
// (the exp_budget largest ranking scores in ascending page order), after
// select_topk_wide_kernel on the same stream wrote the row's accept flag.
// A launch of its own keeps both kernels within their registers.
template <bool SEP>
__global__ __launch_bounds__(kSelThreads) void expand_wide_kernel(
    const float *__restrict__ scores, const float *__restrict__ sel_scores, int W,
    const uint8_t *__restrict__ accept, int exp_budget, int32_t *__restrict__ exp_indices) {
  __shared__ WideLds L;
  const int bh = blockIdx.x;
  if (accept[bh] != 0) return;  // uniform
  const float *row = (SEP ? sel_scores : scores) + (int64_t)bh * W;
  const int k2 = min(exp_budget, W);
  uint32_t T = 0, krem = 0;
  wide_threshold(row, W, (uint32_t)k2, L, T, krem);
  float mx = -INFINITY, ms = -INFINITY;
  wide_compact<false, SEP>(row, row, W, T, krem, k2, k2, exp_indices + (int64_t)bh * exp_budget,
                           L.wsum, nullptr, nullptr, nullptr, mx, ms);
}

// Budgets of CVSABackend._adaptive_select (cvsa/backend.py:522-570): the
// kv-heads of sequence b compete for K = H_kv * base slots.  raw[h] counts
// head h's scores among the K largest of all H_kv * W scores of b (ties at
// the K-th value go to the lower heads; the reference's torch.topk leaves
// them unspecified), then budget = round(fp32(raw) * keep + floor_cap)
// (round half to even, keep = 1 - floor_ratio and floor_cap = base *
// floor_ratio as fp32, :550-552), clamped to [1, n_valid] (:554-557).
// One workgroup per sequence: an 8-bit MSB radix select of the K-th largest
// key over the row's scores (four passes over them), then per-head counts.
// Each thread requests eight scores before it updates the histogram with
// any of them.
constexpr int kMaxAdaptiveHeads = 64;
constexpr int kAdaptiveBatch = 8;

__global__ __launch_bounds__(kSelThreads) void adaptive_budget_kernel(
    const float *__restrict__ scores, int H_kv, int W,
    const int32_t *__restrict__ context_lens, int block_size, int base, float keep,
    float floor_cap, int32_t *__restrict__ budgets) {
  __shared__ uint32_t hist_c[kHistCopies * kHistStride];
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_digit, s_krem;
  __shared__ uint32_t s_gt[kMaxAdaptiveHeads], s_eq[kMaxAdaptiveHeads];
  const int b = blockIdx.x, t = threadIdx.x, lane = t & 63;
  const float *row = scores + (int64_t)b * H_kv * W;
  const int N = H_kv * W;
  uint32_t prefix = 0, pmask = 0, krem = (uint32_t)min(H_kv * base, N);
#pragma unroll 1
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int i = t; i < kHistCopies * kHistStride; i += kSelThreads) hist_c[i] = 0;
    lds_barrier();
    uint32_t *my_hist = hist_c + (lane % kHistCopies) * kHistStride;
    for (int i0 = t; i0 < N; i0 += kAdaptiveBatch * kSelThreads) {
      float v[kAdaptiveBatch];
#pragma unroll
      for (int j = 0; j < kAdaptiveBatch; ++j) v[j] = row[min(i0 + j * kSelThreads, N - 1)];
#pragma unroll
      for (int j = 0; j < kAdaptiveBatch; ++j) {
        const uint32_t key = order_key(v[j]);
        if (i0 + j * kSelThreads < N && (key & pmask) == prefix)
          atomicAdd(&my_hist[(key >> shift) & 255u], 1u);
      }
    }
    lds_barrier();
    if (t < 256) {
      uint32_t c = 0;
#pragma unroll
      for (int j = 0; j < kHistCopies; ++j) c += hist_c[j * kHistStride + t];
      hist[t] = c;
    }
    lds_barrier();
    if (t < 64) {
      // Lane l holds digits 4l..4l+3; count the keys above each digit.
      const uint32_t c0 = hist[4 * lane], c1 = hist[4 * lane + 1];
      const uint32_t c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
      const uint32_t local = c0 + c1 + c2 + c3;
      uint32_t suffix = local;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_down(suffix, off, 64);
        if (lane + off < 64) suffix += o;
      }
      uint32_t above = suffix - local;
      const uint32_t cs[4] = {c3, c2, c1, c0};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (above < krem && above + cs[j] >= krem) {
          s_digit = (uint32_t)(4 * lane + 3 - j);
          s_krem = krem - above;
        }
        above += cs[j];
      }
    }
    lds_barrier();
    prefix |= s_digit << shift;
    pmask |= 0xFFu << shift;
    krem = s_krem;
    lds_barrier();
  }
  const uint32_t T = prefix;
  if (t < H_kv) {
    s_gt[t] = 0;
    s_eq[t] = 0;
  }
  lds_barrier();
  for (int h = 0; h < H_kv; ++h) {
    uint32_t gt = 0, eq = 0;
    const float *hrow = row + (int64_t)h * W;
    for (int p0 = t; p0 < W; p0 += kAdaptiveBatch * kSelThreads) {
      float v[kAdaptiveBatch];
#pragma unroll
      for (int j = 0; j < kAdaptiveBatch; ++j) v[j] = hrow[min(p0 + j * kSelThreads, W - 1)];
#pragma unroll
      for (int j = 0; j < kAdaptiveBatch; ++j) {
        const uint32_t key = order_key(v[j]);
        const bool in = p0 + j * kSelThreads < W;
        gt += in && key > T;
        eq += in && key == T;
      }
    }
    gt = wave_sum_u32(gt);
    eq = wave_sum_u32(eq);
    if (lane == 0 && (gt | eq) != 0) {
      atomicAdd(&s_gt[h], gt);
      atomicAdd(&s_eq[h], eq);
    }
  }
  lds_barrier();
  if (t == 0) {
    const int nv = n_valid_pages(context_lens[b], block_size);
    uint32_t ties = krem;  // keys equal to T among the K largest
    for (int h = 0; h < H_kv; ++h) {
      const uint32_t take = min(ties, s_eq[h]);
      ties -= take;
      const float raw = (float)(s_gt[h] + take);
      const float mixed = __fadd_rn(__fmul_rn(raw, keep), floor_cap);
      const int fb = (int)rintf(mixed);
      budgets[b * H_kv + h] = min(max(fb, 1), nv);
    }
  }
}

// Coverage gate of a given selection, one workgroup per (b, kv-head).  All
// global loads are issued at once (the row strided by the block so each
// load instruction is coalesced, the selection list, n_per_head); for rows
// of up to 8192 pages the row is staged in LDS and the selected scores are
// gathered from there.  The two maxima and the two sums each take one block
// reduction.
template <int R>
__global__ __launch_bounds__(kSelThreads) void check_coverage_kernel(
    const float *__restrict__ scores, int W, const int32_t *__restrict__ selected,
    int sel_width, int sel_block, const int32_t *__restrict__ n_per_head,
    float tau, uint8_t *__restrict__ accept_out, float *__restrict__ coverage_out) {
  constexpr bool kStage = R <= 8;
  __shared__ float s_row[kStage ? R * kSelThreads : 1];
  __shared__ float red_max[kSelWaves][2], red_sum[kSelWaves][2];
  const int bh = blockIdx.x;
  const int t = threadIdx.x;
  const float *row = scores + (int64_t)bh * W;
  const int32_t *sel = selected + (int64_t)bh * sel_width;

  const int n_raw = n_per_head[bh];
  float v[R];
  int pidx[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int i = t + r * kSelThreads;
    v[r] = i < W ? row[i] : -INFINITY;
    pidx[r] = i < sel_width ? sel[i] : -1;
  }
  // Selected scores: entries j < n_sel of the row (coverage.py:198-208).
  // n_sel is clamped to the row width and indices outside [0, W) read as
  // -inf, so a malformed selection cannot read out of bounds.
  const int n_sel = max(0, min(n_raw, sel_width));
  float sv[R];
  if constexpr (kStage) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = t + r * kSelThreads;
      if (i < W) s_row[i] = v[r];
    }
    lds_barrier();
  }
  float mx_all = -INFINITY, mx_sel = -INFINITY;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int j = t + r * kSelThreads;
    const int p = pidx[r];
    float x = -INFINITY;
    if (j < n_sel && p >= 0 && p < W) x = kStage ? s_row[p] : row[p];
    sv[r] = x;
    mx_all = fmaxf(mx_all, v[r]);
    mx_sel = fmaxf(mx_sel, x);
  }
  block_max2(mx_all, mx_sel, red_max);
  // lse_all floors its running max at -1e20 (coverage.py:180); lse_sel has
  // -1e20 padding lanes whenever n_sel is short of the power-of-two block.
  const float m_all = fmaxf(mx_all, -1e20f);
  const float m_sel = n_sel < sel_block ? fmaxf(mx_sel, -1e20f) : mx_sel;
  float se_all = 0.f, se_sel = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    se_all += fast_exp(v[r] - m_all);
    if (t + r * kSelThreads < n_sel) se_sel += fast_exp(sv[r] - m_sel);
  }
  block_sum2(se_all, se_sel, red_sum);
  if (t == 0) {
    const float cov = expf(lse_from(m_sel, se_sel) - lse_from(m_all, se_all));
    coverage_out[bh] = cov;
    accept_out[bh] = cov >= tau ? 1 : 0;
  }
}

// check_coverage_kernel for rows wider than it holds in registers (W or
// the selection width above kMaxPages): the same two log-sum-exps and
// rules, streaming the row and gathering the selected scores from memory.
__global__ __launch_bounds__(kSelThreads) void check_coverage_wide_kernel(
    const float *__restrict__ scores, int W, const int32_t *__restrict__ selected,
    int sel_width, int sel_block, const int32_t *__restrict__ n_per_head,
    float tau, uint8_t *__restrict__ accept_out, float *__restrict__ coverage_out) {
  __shared__ float red_max[kSelWaves][2], red_sum[kSelWaves][2];
  const int bh = blockIdx.x;
  const int t = threadIdx.x;
  const float *row = scores + (int64_t)bh * W;
  const int32_t *sel = selected + (int64_t)bh * sel_width;
  const int n_sel = max(0, min(n_per_head[bh], sel_width));
  // f(score) for every selected j < n_sel (-inf for an id outside
  // [0, W)): kStrip ids, then kStrip scores in flight (unconditional loads
  // at clamped addresses).
  const auto for_selected = [&](auto &&f) {
    for (int j0 = 0; j0 < n_sel; j0 += kStrip * kSelThreads) {
      int p[kStrip];
      float v[kStrip];
#pragma unroll
      for (int e = 0; e < kStrip; ++e) p[e] = sel[min(j0 + e * kSelThreads + t, n_sel - 1)];
#pragma unroll
      for (int e = 0; e < kStrip; ++e) v[e] = row[min(max(p[e], 0), W - 1)];
#pragma unroll
      for (int e = 0; e < kStrip; ++e)
        if (j0 + e * kSelThreads + t < n_sel) f(p[e] >= 0 && p[e] < W ? v[e] : -INFINITY);
    }
  };
  float mx_all = -INFINITY, mx_sel = -INFINITY;
  stream_row(row, W, [&](int, float v) { mx_all = fmaxf(mx_all, v); });
  for_selected([&](float v) { mx_sel = fmaxf(mx_sel, v); });
  block_max2(mx_all, mx_sel, red_max);
  const float m_all = fmaxf(mx_all, -1e20f);
  const float m_sel = n_sel < sel_block ? fmaxf(mx_sel, -1e20f) : mx_sel;
  float se_all = 0.f, se_sel = 0.f;
  stream_row(row, W, [&](int, float v) { se_all += fast_exp(v - m_all); });
  for_selected([&](float v) { se_sel += fast_exp(v - m_sel); });
  block_sum2(se_all, se_sel, red_sum);
  if (t == 0) {
    const float cov = expf(lse_from(m_sel, se_sel) - lse_from(m_all, se_all));
    coverage_out[bh] = cov;
    accept_out[bh] = cov >= tau ? 1 : 0;
  }
}

static int keys_per_thread(int n) {
  int r = 1;
  while (r * kSelThreads < n) r <<= 1;
  return r;
}


static int launch_select(const char *name, const float *page_scores, const float *sel_scores,
                         int32_t B, int32_t H_kv,
                         int32_t W, const int32_t *context_lens, int32_t block_size,
                         int32_t budget, int32_t *page_indices, int32_t *n_per_head, float tau,
                         uint8_t *accept_out, float *coverage_out, const uint8_t *check_accept,
                         float *scores_cache, int64_t *stats, int count_gate,
                         void *stream, int mode = kUniform, float top_p = 0.f,
                         const int32_t *row_budgets = nullptr, int32_t *keep_flag = nullptr,
                         uint8_t *sel_map = nullptr, int64_t map_stride = 0,
                         int64_t *keep_work = nullptr, int32_t exp_budget = 0,
                         int32_t *exp_indices = nullptr) {
  CVSA_REQUIRE(page_scores && context_lens && page_indices && n_per_head, CVSA_ERR_INVALID,
               "%s: null pointer argument", name);
  CVSA_REQUIRE((accept_out == nullptr) == (coverage_out == nullptr), CVSA_ERR_INVALID,
               "%s: accept_out and coverage_out must both be set or both NULL", name);
  CVSA_REQUIRE(check_accept == nullptr || accept_out != nullptr, CVSA_ERR_INVALID,
               "%s: a device-side check needs accept_out", name);
  CVSA_REQUIRE(!count_gate || (check_accept == nullptr && accept_out != nullptr),
               CVSA_ERR_INVALID, "%s: count_gate needs a fresh selection with its gate", name);
  CVSA_REQUIRE(B > 0 && H_kv > 0 && W > 0 && block_size > 0, CVSA_ERR_INVALID,
               "%s: bad sizes B=%d H_kv=%d W=%d bs=%d", name, B, H_kv, W, block_size);
  CVSA_REQUIRE(budget >= 1 && budget <= W, CVSA_ERR_INVALID,
               "%s: budget=%d must be in [1, W=%d]", name, budget, W);
  CVSA_REQUIRE(W <= kMaxPagesWide, CVSA_ERR_UNSUPPORTED, "%s: W=%d exceeds %d pages", name, W,
               kMaxPagesWide);
  CVSA_REQUIRE(W <= kMaxPages || mode != kTopP, CVSA_ERR_UNSUPPORTED,
               "%s: top-p budgets take rows of at most %d pages (W=%d)", name, kMaxPages, W);
  CVSA_REQUIRE(sel_map == nullptr || (map_stride >= W && map_stride % 16 == 0 &&
                                      ((uintptr_t)sel_map & 15) == 0),
               CVSA_ERR_INVALID,
               "%s: selection map rows of %lld bytes (16-byte aligned, >= W=%d) required",
               name, (long long)map_stride, W);
  CVSA_REQUIRE(exp_indices == nullptr || (mode == kUniform && accept_out != nullptr &&
                                          exp_budget >= 1 && exp_budget <= W),
               CVSA_ERR_INVALID,
               "%s: an expanded selection needs the uniform budget, the gate and an expanded "
               "budget in [1, W=%d] (got %d)",
               name, W, exp_budget);
  const int R = keys_per_thread(W);
  const dim3 grid(B * H_kv);
  hipStream_t st = (hipStream_t)stream;
  long long *st64 = reinterpret_cast<long long *>(stats);
  // In the variable-budget modes `budget` is the row stride of page_indices.
  const int width = budget;
  if (W > kMaxPages) {
#define CVSA_WIDE_LAUNCH(SEP, MODE)                                                          \
  hipLaunchKernelGGL((select_topk_wide_kernel<SEP, MODE>), grid, dim3(kSelThreads), 0, st,   \
                     page_scores, sel_scores, W, H_kv, context_lens, block_size, budget,     \
                     width, row_budgets, page_indices, n_per_head, tau, accept_out,          \
                     coverage_out, check_accept, B * H_kv, scores_cache, st64, count_gate,   \
                     keep_flag, sel_map, map_stride,                                          \
                     reinterpret_cast<unsigned long long *>(keep_work))
    if (sel_scores != nullptr) {
      if (mode == kTable) CVSA_WIDE_LAUNCH(true, kTable);
      else CVSA_WIDE_LAUNCH(true, kUniform);
    } else {
      if (mode == kTable) CVSA_WIDE_LAUNCH(false, kTable);
      else CVSA_WIDE_LAUNCH(false, kUniform);
    }
#undef CVSA_WIDE_LAUNCH
    // Approximate recovery: the expanded selection of every rejected row.
    if (mode == kUniform && exp_indices != nullptr && accept_out != nullptr) {
      if (sel_scores != nullptr)
        hipLaunchKernelGGL(expand_wide_kernel<true>, grid, dim3(kSelThreads), 0, st,
                           page_scores, sel_scores, W, accept_out, exp_budget, exp_indices);
      else
        hipLaunchKernelGGL(expand_wide_kernel<false>, grid, dim3(kSelThreads), 0, st,
                           page_scores, sel_scores, W, accept_out, exp_budget, exp_indices);
    }
    return cvsa_host::check_launch(name);
  }
  switch (R) {
#define CVSA_SEL_LAUNCH(RR, SEP, MODE)                                                      \
  hipLaunchKernelGGL((select_topk_kernel<RR, SEP, MODE>), grid, dim3(kSelThreads), 0, st,   \
                     page_scores, sel_scores, W, H_kv, context_lens, block_size, budget,    \
                     width, top_p, row_budgets, page_indices, n_per_head, tau, accept_out,  \
                     coverage_out, check_accept, B * H_kv, scores_cache, st64, count_gate,    \
                     keep_flag, sel_map, map_stride,                                         \
                     reinterpret_cast<unsigned long long *>(keep_work), exp_budget, exp_indices)
#define CVSA_SEL_MODES(RR, SEP)                                    \
  if (mode == kTopP) CVSA_SEL_LAUNCH(RR, SEP, kTopP);              \
  else if (mode == kTable) CVSA_SEL_LAUNCH(RR, SEP, kTable);       \
  else CVSA_SEL_LAUNCH(RR, SEP, kUniform);
#define CVSA_SEL_CASE(RR)                                       \
  case RR:                                                      \
    if (sel_scores != nullptr) {                                \
      CVSA_SEL_MODES(RR, true)                                  \
    } else {                                                    \
      CVSA_SEL_MODES(RR, false)                                 \
    }                                                           \
    break;
    CVSA_SEL_CASE(1)
    CVSA_SEL_CASE(2)
    CVSA_SEL_CASE(4)
    CVSA_SEL_CASE(8)
    CVSA_SEL_CASE(16)
    CVSA_SEL_CASE(32)
#undef CVSA_SEL_CASE
#undef CVSA_SEL_MODES
#undef CVSA_SEL_LAUNCH
    default:
      return cvsa_host::fail(CVSA_ERR_UNSUPPORTED, "%s: W=%d too large", name, W);
  }
  return cvsa_host::check_launch(name);
}

}  // namespace cvsa

using namespace cvsa;

extern "C" int cvsa_select_topk(const float *page_scores, int32_t B, int32_t H_kv, int32_t W,
                                const int32_t *context_lens, int32_t block_size,
                                int32_t budget, int32_t *page_indices, int32_t *n_per_head,
                                float tau, uint8_t *accept_out, float *coverage_out,
                                void *stream) {
  return launch_select("select_topk", page_scores, nullptr, B, H_kv, W, context_lens,
                       block_size, budget, page_indices, n_per_head, tau, accept_out,
                       coverage_out, nullptr, nullptr, nullptr, 0, stream);
}

extern "C" int cvsa_select_or_keep(const float *page_scores, const float *sel_scores,
                                   const uint8_t *check_accept,
                                   int32_t B, int32_t H_kv, int32_t W,
                                   const int32_t *context_lens, int32_t block_size,
                                   int32_t budget, int32_t *page_indices, int32_t *n_per_head,
                                   float tau, uint8_t *accept_out, float *coverage_out,
                                   float *scores_cache, int64_t *stats, int32_t count_gate,
                                   void *stream) {
  CVSA_REQUIRE(accept_out && coverage_out, CVSA_ERR_INVALID,
               "select_or_keep: accept_out and coverage_out are required");
  return launch_select("select_or_keep", page_scores, sel_scores, B, H_kv, W, context_lens,
                       block_size, budget, page_indices, n_per_head, tau, accept_out,
                       coverage_out, check_accept, scores_cache, stats, count_gate, stream);
}

extern "C" int cvsa_select_or_keep_budgeted(
    const float *page_scores, const float *sel_scores, const uint8_t *check_accept, int32_t B,
    int32_t H_kv, int32_t W, const int32_t *context_lens, int32_t block_size,
    const int32_t *row_budgets, int32_t width, int32_t *page_indices, int32_t *n_per_head,
    float tau, uint8_t *accept_out, float *coverage_out, float *scores_cache, int64_t *stats,
    int32_t count_gate, void *stream) {
  CVSA_REQUIRE(accept_out && coverage_out && row_budgets, CVSA_ERR_INVALID,
               "select_or_keep_budgeted: row_budgets, accept_out and coverage_out are "
               "required");
  return launch_select("select_or_keep_budgeted", page_scores, sel_scores, B, H_kv, W,
                       context_lens, block_size, width, page_indices, n_per_head, tau,
                       accept_out, coverage_out, check_accept, scores_cache, stats, count_gate,
                       stream, kTable, 0.f, row_budgets);
}

namespace cvsa_internal {

int select_for_plan(const float *page_scores, const float *sel_scores,
                    const uint8_t *check_accept, int32_t B, int32_t H_kv, int32_t W,
                    const int32_t *context_lens, int32_t block_size, int32_t budget,
                    int32_t *page_indices, int32_t *n_per_head, float tau, uint8_t *accept_out,
                    float *coverage_out, float *scores_cache, int64_t *stats,
                    int32_t count_gate, int32_t *keep_flag, uint8_t *sel_map,
                    int64_t sel_map_stride, int64_t *keep_work, int32_t exp_budget,
                    int32_t *exp_indices, void *stream) {
  CVSA_REQUIRE(accept_out && coverage_out, CVSA_ERR_INVALID,
               "select_or_keep: accept_out and coverage_out are required");
  CVSA_REQUIRE(keep_flag == nullptr || check_accept != nullptr, CVSA_ERR_INVALID,
               "select_or_keep: a keep flag needs check_accept");
  CVSA_REQUIRE(keep_work == nullptr || keep_flag != nullptr, CVSA_ERR_INVALID,
               "select_or_keep: booking a kept speculation needs the keep flag");
  return launch_select("select_or_keep", page_scores, sel_scores, B, H_kv, W, context_lens,
                       block_size, budget, page_indices, n_per_head, tau, accept_out,
                       coverage_out, check_accept, scores_cache, stats, count_gate, stream,
                       kUniform, 0.f, nullptr, keep_flag, sel_map, sel_map_stride, keep_work,
                       exp_budget, exp_indices);
}

__global__ __launch_bounds__(kSelThreads) void selection_map_kernel(
    const int32_t *__restrict__ page_indices, int64_t idx_stride,
    const int32_t *__restrict__ n_per_head, int W, uint8_t *__restrict__ sel_map,
    int64_t map_stride) {
  const int row = blockIdx.x;
  uint8_t *mrow = sel_map + (int64_t)row * map_stride;
  for (int64_t i = threadIdx.x * 16; i < map_stride; i += kSelThreads * 16)
    *reinterpret_cast<uint4 *>(mrow + i) = make_uint4(0u, 0u, 0u, 0u);
  __syncthreads();  // the clearing stores before the marking ones
  const int n = max(0, min(n_per_head[row], (int)idx_stride));
  const int32_t *idx = page_indices + (int64_t)row * idx_stride;
  for (int i = threadIdx.x; i < n; i += kSelThreads) {
    const int p = idx[i];
    if (p >= 0 && p < W) mrow[p] = 1;
  }
}

int build_selection_map(const int32_t *page_indices, int64_t idx_stride,
                        const int32_t *n_per_head, int32_t rows, int32_t W, uint8_t *sel_map,
                        int64_t sel_map_stride, void *stream) {
  CVSA_REQUIRE(page_indices && n_per_head && sel_map, CVSA_ERR_INVALID,
               "selection map: null pointer argument");
  CVSA_REQUIRE(rows > 0 && W > 0 && idx_stride > 0 && sel_map_stride >= W &&
                   sel_map_stride % 16 == 0 && ((uintptr_t)sel_map & 15) == 0,
               CVSA_ERR_INVALID, "selection map: bad sizes rows=%d W=%d stride=%lld", rows, W,
               (long long)sel_map_stride);
  hipLaunchKernelGGL(selection_map_kernel, dim3(rows), dim3(kSelThreads), 0,
                     (hipStream_t)stream, page_indices, idx_stride, n_per_head, W, sel_map,
                     sel_map_stride);
  return cvsa_host::check_launch("selection map");
}

}  // namespace cvsa_internal

extern "C" int cvsa_select_budgeted(const float *page_scores, const float *sel_scores,
                                    int32_t B, int32_t H_kv, int32_t W,
                                    const int32_t *context_lens, int32_t block_size,
                                    float top_p, const int32_t *row_budgets, int32_t width,
                                    int32_t *page_indices, int32_t *n_per_head, float tau,
                                    uint8_t *accept_out, float *coverage_out, void *stream) {
  CVSA_REQUIRE((top_p > 0.f) != (row_budgets != nullptr), CVSA_ERR_INVALID,
               "select_budgeted: give exactly one of top_p and row_budgets");
  CVSA_REQUIRE(row_budgets != nullptr || top_p < 1.f, CVSA_ERR_INVALID,
               "select_budgeted: top_p=%g must be in (0, 1)", (double)top_p);
  return launch_select("select_budgeted", page_scores, sel_scores, B, H_kv, W, context_lens,
                       block_size, width, page_indices, n_per_head, tau, accept_out,
                       coverage_out, nullptr, nullptr, nullptr, 0, stream,
                       top_p > 0.f ? kTopP : kTable, top_p, row_budgets);
}

extern "C" int cvsa_adaptive_budgets(const float *page_scores, int32_t B, int32_t H_kv,
                                     int32_t W, const int32_t *context_lens,
                                     int32_t block_size, int32_t base_budget,
                                     double floor_ratio, int32_t *budgets, void *stream) {
  CVSA_REQUIRE(page_scores && context_lens && budgets, CVSA_ERR_INVALID,
               "adaptive_budgets: null pointer argument");
  CVSA_REQUIRE(B > 0 && H_kv > 0 && W > 0 && block_size > 0 && base_budget > 0,
               CVSA_ERR_INVALID, "adaptive_budgets: bad sizes B=%d H_kv=%d W=%d base=%d", B,
               H_kv, W, base_budget);
  CVSA_REQUIRE(H_kv <= kMaxAdaptiveHeads && (int64_t)H_kv * W <= (int64_t)1 << 24,
               CVSA_ERR_UNSUPPORTED,
               "adaptive_budgets: H_kv=%d (max %d) or H_kv*W=%lld (max 2^24) too large", H_kv,
               kMaxAdaptiveHeads, (long long)H_kv * W);
  // The reference forms these in Python (double) and torch applies them to
  // an fp32 tensor.
  const float keep = (float)(1.0 - floor_ratio);
  const float floor_cap = (float)((double)base_budget * floor_ratio);
  hipLaunchKernelGGL(adaptive_budget_kernel, dim3(B), dim3(kSelThreads), 0,
                     (hipStream_t)stream, page_scores, H_kv, W, context_lens, block_size,
                     base_budget, keep, floor_cap, budgets);
  return cvsa_host::check_launch("adaptive_budgets");
}

extern "C" int cvsa_check_coverage(const float *page_scores, int32_t B,
                                   int32_t H_kv, int32_t W,
                                   const int32_t *selected, int64_t sel_stride,
                                   const int32_t *n_per_head, float tau,
                                   uint8_t *accept_out, float *coverage_out,
                                   void *stream) {
  CVSA_REQUIRE(page_scores && selected && n_per_head && accept_out && coverage_out,
               CVSA_ERR_INVALID, "check_coverage: null pointer argument");
  CVSA_REQUIRE(B > 0 && H_kv > 0 && W > 0 && sel_stride > 0, CVSA_ERR_INVALID,
               "check_coverage: bad sizes B=%d H_kv=%d W=%d sel_stride=%lld", B, H_kv,
               W, (long long)sel_stride);
  CVSA_REQUIRE(W <= kMaxPagesWide && sel_stride <= kMaxPagesWide, CVSA_ERR_UNSUPPORTED,
               "check_coverage: W=%d / selection width %lld exceed %d", W,
               (long long)sel_stride, kMaxPagesWide);
  // The reference pads the selection to a power of two (coverage.py:234-237).
  int sel_block = 1;
  while (sel_block < sel_stride) sel_block <<= 1;
  const dim3 grid(B * H_kv);
  hipStream_t st = (hipStream_t)stream;
  const int width = (int)sel_stride;
  if (W > kMaxPages || sel_block > kMaxPages) {
    hipLaunchKernelGGL(check_coverage_wide_kernel, grid, dim3(kSelThreads), 0, st, page_scores,
                       W, selected, width, sel_block, n_per_head, tau, accept_out,
                       coverage_out);
    return cvsa_host::check_launch("check_coverage");
  }
  const int R = keys_per_thread(W > sel_block ? W : sel_block);
  switch (R) {
#define CVSA_COV_CASE(RR)                                                       \
  case RR:                                                                      \
    hipLaunchKernelGGL(check_coverage_kernel<RR>, grid, dim3(kSelThreads), 0, st, \
                       page_scores, W, selected, width, sel_block,               \
                       n_per_head, tau, accept_out, coverage_out);               \
    break;
    CVSA_COV_CASE(1)
    CVSA_COV_CASE(2)
    CVSA_COV_CASE(4)
    CVSA_COV_CASE(8)
    CVSA_COV_CASE(16)
    CVSA_COV_CASE(32)
#undef CVSA_COV_CASE
    default:
      return cvsa_host::fail(CVSA_ERR_UNSUPPORTED, "check_coverage: W=%d too large", W);
  }
  return cvsa_host::check_launch("check_coverage");
}
