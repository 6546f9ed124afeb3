// Shared device helpers and host-side error plumbing for libcvsa_hip.so.
// Target: gfx950 (CDNA4), wave64.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <math.h>

#include "../../include/cvsa_hip.h"

namespace cvsa {

constexpr int kWave = 64;
constexpr int kHeadDim = 128;   // the head dimension of the fused lazy-check launch
constexpr int kPageTokens = 16; // tokens of a tile (a page is 1, 2 or 4 tiles)

// Head dimensions the kernels are compiled for.
__host__ __device__ constexpr bool head_dim_supported(int D) {
  return D == 32 || D == 64 || D == 128 || D == 256;
}

// The kernels walk pages as 16-token tiles: a page of block_size tokens is
// 1 << tile_shift(block_size) consecutive tiles of its block.  -1: the block
// size is not supported.
__host__ __device__ constexpr int tile_shift(int block_size) {
  return block_size == 16 ? 0 : block_size == 32 ? 1 : block_size == 64 ? 2
         : block_size == 128 ? 3 : -1;
}
// 8-token pages: a page is one tile of which only rows 0..7 exist; the
// kernels read row r & 7 in place of row r (in the page's own block, so no
// load leaves the pool) and mask rows 8..15 out as tokens past the page.
// Block sizes with kernels: 8, 16, 32, 64, 128.
__host__ __device__ constexpr bool block_size_supported(int block_size) {
  return block_size == 8 || tile_shift(block_size) >= 0;
}
// Tiles per page as a shift (0 for 8-token pages) and log2 of the rows of
// a tile (3 for 8-token pages, else 4).
__host__ __device__ constexpr int page_tile_shift(int block_size) {
  return block_size == 8 ? 0 : tile_shift(block_size);
}
__host__ __device__ constexpr int tile_rows_log2(int block_size) {
  return block_size == 8 ? 3 : 4;
}
// Pages per row: the register-resident select and coverage kernels hold
// rows of up to kMaxPages; wider rows, up to kMaxPagesWide pages, stream
// from memory (select_topk_wide_kernel, check_coverage_wide_kernel).
constexpr int kMaxPages = 32768;
constexpr int kMaxPagesWide = 1 << 18;

// ---------------------------------------------------------------- numerics

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// acc + a.lo*b.lo + a.hi*b.hi on packed bf16 pairs (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc,
                                         false);
}

// 16-byte load of data read once per launch (K/V pages): the nontemporal hint
// keeps it from displacing reusable lines in the caches.
__device__ __forceinline__ uint4 stream_load16(const uint16_t *p) {
  typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
  const v4u_t v = __builtin_nontemporal_load(reinterpret_cast<const v4u_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// stream_load16 of byte voff + soff of the `bytes`-byte region at `base`
// (base and soff the same in every lane of the wave).  A lane whose voff is
// at or past `bytes` (kRegionSkip added to an in-region offset) gets 16 zero
// bytes and makes no memory access: the buffer bounds check drops it.
constexpr uint32_t kRegionSkip = 0x40000000u;
__device__ __forceinline__ uint4 region_load16(const void *base, uint32_t bytes, uint32_t voff,
                                               uint32_t soff) {
  constexpr int kRsrcWord3 = 0x00020000;  // 32-bit data format, raw
  constexpr int kCpolNontemporal = 2;     // nt
  typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, kRsrcWord3);
  const v4u_t v = __builtin_bit_cast(
      v4u_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, kCpolNontemporal));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Sum of the 8 products of two 16-byte bf16 vectors, accumulated onto acc.
__device__ __forceinline__ float dot8_bf16(const uint4 &a, const uint4 &b, float acc) {
  acc = dot2_bf16(a.x, b.x, acc);
  acc = dot2_bf16(a.y, b.y, acc);
  acc = dot2_bf16(a.z, b.z, acc);
  acc = dot2_bf16(a.w, b.w, acc);
  return acc;
}

// q_rep[h][seg*8 .. seg*8+8): fp32 sum over the group, times 1/G, rounded
// to bf16 (the bf16 result of q.view(B,H_kv,G,D).mean(2)).
__device__ __forceinline__ uint4 group_mean_q(const uint16_t *__restrict__ q, int64_t q_sb,
                                              int64_t q_sh, int b, int h, int G, int seg,
                                              float inv_g) {
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  // Four rows per batch are loaded before any is summed (one load latency
  // per batch); the sum still runs over g in order.  The first batch is
  // outside the loop, so loads the caller issued earlier are not waited for
  // at a loop entry.
  const uint16_t *base = q + b * q_sb + (int64_t)h * G * q_sh + seg * 8;
  auto batch = [&](int g0) {
    uint4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[j] = *reinterpret_cast<const uint4 *>(base + (int64_t)min(g0 + j, G - 1) * q_sh);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (g0 + j < G) {
        acc[0] += bf16_lo(v[j].x); acc[1] += bf16_hi(v[j].x);
        acc[2] += bf16_lo(v[j].y); acc[3] += bf16_hi(v[j].y);
        acc[4] += bf16_lo(v[j].z); acc[5] += bf16_hi(v[j].z);
        acc[6] += bf16_lo(v[j].w); acc[7] += bf16_hi(v[j].w);
      }
    }
  };
  batch(0);
  for (int g0 = 4; g0 < G; g0 += 4) batch(g0);
  uint4 r;
  r.x = pack_bf16x2(acc[0] * inv_g, acc[1] * inv_g);
  r.y = pack_bf16x2(acc[2] * inv_g, acc[3] * inv_g);
  r.z = pack_bf16x2(acc[4] * inv_g, acc[5] * inv_g);
  r.w = pack_bf16x2(acc[6] * inv_g, acc[7] * inv_g);
  return r;
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// waits for every outstanding global load of the wave; with this one, loads
// issued before the barrier stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// exp(x) through the hardware base-2 exponential.
__device__ __forceinline__ float fast_exp(float x) { return exp2f(x * 1.4426950408889634f); }

// ------------------------------------------------------------- lane moves
// DPP controls (gfx9 encoding).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xF, 0xF, true));
}

// Value of lane (l ^ 16) and of lane (l ^ 32): the two halves of each
// permlane swap pair hold {v[l], v[l^16]} (resp. {v[l], v[l^32]}).
__device__ __forceinline__ void xchg16(float v, float &a, float &b) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                            false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void xchg32(float v, float &a, float &b) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                            false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// All-reduce over aligned groups of W lanes (W in 1,2,4,8,16,32); every
// lane of a group ends with the same bits.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W >= 2) v += dpp_f<kDppQuadXor1>(v);
  if constexpr (W >= 4) v += dpp_f<kDppQuadXor2>(v);
  if constexpr (W >= 8) v += dpp_f<kDppRowHalfMirror>(v);
  if constexpr (W >= 16) v += dpp_f<kDppRowMirror>(v);
  if constexpr (W >= 32) {
    float a, b;
    xchg16(v, a, b);
    v = a + b;
  }
  return v;
}

// Max over the whole wave of a value that is uniform inside aligned groups
// of W lanes (W in 1,2,4,8,16).  Returns a wave-uniform value.
template <int W>
__device__ __forceinline__ float wave_max_from_groups(float v) {
  if constexpr (W < 2) v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  if constexpr (W < 4) v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  if constexpr (W < 8) v = fmaxf(v, dpp_f<kDppRowHalfMirror>(v));
  if constexpr (W < 16) v = fmaxf(v, dpp_f<kDppRowMirror>(v));
  float a, b;
  xchg16(v, a, b);
  v = fmaxf(a, b);
  xchg32(v, a, b);
  v = fmaxf(a, b);
  return v;
}

template <int W>
__device__ __forceinline__ float wave_sum_from_groups(float v) {
  if constexpr (W < 2) v += dpp_f<kDppQuadXor1>(v);
  if constexpr (W < 4) v += dpp_f<kDppQuadXor2>(v);
  if constexpr (W < 8) v += dpp_f<kDppRowHalfMirror>(v);
  if constexpr (W < 16) v += dpp_f<kDppRowMirror>(v);
  float a, b;
  xchg16(v, a, b);
  v = a + b;
  xchg32(v, a, b);
  v = a + b;
  return v;
}

// ------------------------------------------------ integer wave reductions
// DPP and permlane moves instead of __shfl_* (an LDS permute per step).

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

__device__ __forceinline__ uint32_t xchg_max16_32(uint32_t v) {
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max(r[0], r[1]);
  r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max(r[0], r[1]);
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u<kDppQuadXor1>(v));
  v = max(v, dpp_u<kDppQuadXor2>(v));
  v = max(v, dpp_u<kDppRowHalfMirror>(v));
  v = max(v, dpp_u<kDppRowMirror>(v));
  return xchg_max16_32(v);
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  v += dpp_u<kDppQuadXor1>(v);
  v += dpp_u<kDppQuadXor2>(v);
  v += dpp_u<kDppRowHalfMirror>(v);
  v += dpp_u<kDppRowMirror>(v);
  auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = r[0] + r[1];
  r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return r[0] + r[1];
}

// Inclusive prefix sum over the wave: row_shr steps inside each row of 16
// lanes (lanes shifted in from outside the row read 0), then the totals of
// the lower rows, read from lanes 15, 31 and 47.
constexpr int kDppRowShr1 = 0x111;
constexpr int kDppRowShr2 = 0x112;
constexpr int kDppRowShr4 = 0x114;
constexpr int kDppRowShr8 = 0x118;

__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  v += dpp_u<kDppRowShr1>(v);
  v += dpp_u<kDppRowShr2>(v);
  v += dpp_u<kDppRowShr4>(v);
  v += dpp_u<kDppRowShr8>(v);
  const uint32_t t0 = __builtin_amdgcn_readlane(v, 15);
  const uint32_t t1 = __builtin_amdgcn_readlane(v, 31);
  const uint32_t t2 = __builtin_amdgcn_readlane(v, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return v + (row >= 1 ? t0 : 0u) + (row >= 2 ? t1 : 0u) + (row >= 3 ? t2 : 0u);
}

// Sum over lanes that share (lane mod W): adds the 64/W lanes
// {l, l+W, l+2W, ...}.  All those lanes end with the same value.
template <int W>
__device__ __forceinline__ float sum_across_groups(float v) {
  if constexpr (W <= 4) v += dpp_f<kDppRowRor4>(v);
  if constexpr (W <= 8) v += dpp_f<kDppRowRor8>(v);
  float a, b;
  xchg16(v, a, b);
  v = a + b;
  xchg32(v, a, b);
  v = a + b;
  return v;
}

// Pages of a sequence that hold at least one position below ctx, following
// the reference's ((ctx - 1) / bs) + 1 with truncating division, so ctx = 0
// still counts one page (cvsa/backend.py:687, coverage.py:60).
__device__ __host__ __forceinline__ int n_valid_pages(int ctx, int bs) {
  return (ctx - 1) / bs + 1;
}

}  // namespace cvsa

// ------------------------------------------------------------ host helpers
namespace cvsa_host {

void set_error(const char *fmt, ...);
int fail(int code, const char *fmt, ...);
int check_launch(const char *what);

}  // namespace cvsa_host

#define CVSA_REQUIRE(cond, code, ...)                 \
  do {                                                \
    if (!(cond)) return cvsa_host::fail(code, __VA_ARGS__); \
  } while (0)
