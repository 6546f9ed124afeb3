// Recovery building blocks: complement page lists and the selective LSE merge.
//
// compute_complement follows _complement_idx_kernel / triton_compute_complement
// (cvsa/kernels/coverage.py:30-96, :99-150): for each rejected (b, kv-head)
// the ascending list of valid pages p < n_valid that are not among the first
// n_sel selected pages, zero-filled to the output width; accepted heads get
// an empty list (:54-58).  The reference tests membership with an O(P*k)
// loop (:72-80); here the selection is first marked in an LDS bitmap and a
// block scan compacts the unmarked pages in O(P + k).
//
// lse_merge follows _lse_merge_kernel (cvsa/kernels/coverage.py:273-326) and
// selective_lse_merge (cvsa/lse_merge.py:11-54).
#include "cvsa_common.h"
#include <hip/hip_fp16.h>

namespace cvsa {

constexpr int kCompThreads = 256;

__global__ __launch_bounds__(kCompThreads) void complement_kernel(
    const int32_t *__restrict__ page_indices, int64_t idx_stride, int sel_width,
    const int32_t *__restrict__ n_per_head, const int32_t *__restrict__ context_lens,
    int block_size, const uint8_t *__restrict__ accept, int H_kv, int width,
    int32_t *__restrict__ comp, int32_t *__restrict__ n_comp) {
  __shared__ uint32_t bitmap[kMaxPagesWide / 32];
  __shared__ uint32_t wsum[kCompThreads / kWave];
  const int bh = blockIdx.x;
  const int b = bh / H_kv;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  int32_t *out = comp + (int64_t)bh * width;

  if (accept != nullptr && accept[bh] != 0) {
    for (int i = t; i < width; i += kCompThreads) out[i] = 0;
    if (t == 0) n_comp[bh] = 0;
    return;
  }
  const int nv = max(0, min(n_valid_pages(context_lens[b], block_size), width));
  const int ns = max(0, min(n_per_head[bh], sel_width));
  const int words = (nv + 31) / 32;
  for (int w = t; w < words; w += kCompThreads) bitmap[w] = 0u;
  __syncthreads();
  const int32_t *sel = page_indices + (int64_t)bh * idx_stride;
  for (int j = t; j < ns; j += kCompThreads) {
    const int p = sel[j];
    if (p >= 0 && p < nv) atomicOr(&bitmap[p >> 5], 1u << (p & 31));
  }
  __syncthreads();

  // Thread t owns pages [t*C, t*C + C).
  const int C = (nv + kCompThreads - 1) / kCompThreads;
  const int p0 = t * C, p1 = min(nv, p0 + C);
  uint32_t cnt = 0;
  for (int p = p0; p < p1; ++p) cnt += ((bitmap[p >> 5] >> (p & 31)) & 1u) ? 0u : 1u;
  // Block exclusive scan of cnt.
  uint32_t incl = cnt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t o = __shfl_up(incl, off, 64);
    if (lane >= off) incl += o;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t before = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kCompThreads / kWave; ++w) {
    before += (w < wave) ? wsum[w] : 0u;
    total += wsum[w];
  }
  uint32_t pos = before + incl - cnt;
  for (int p = p0; p < p1; ++p)
    if (!((bitmap[p >> 5] >> (p & 31)) & 1u)) out[pos++] = p;
  for (int i = (int)total + t; i < width; i += kCompThreads) out[i] = 0;
  if (t == 0) n_comp[bh] = (int32_t)total;
}

__global__ __launch_bounds__(256) void lse_merge_kernel(
    const float *__restrict__ o_d, const float *__restrict__ m_d,
    const float *__restrict__ l_d, const float *__restrict__ o_c,
    const float *__restrict__ m_c, const float *__restrict__ l_c,
    const uint8_t *__restrict__ accept, int H_q, int H_kv, int D, int64_t total,
    void *out, int dtype) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t row = i / D;  // b * H_q + qh
  const int b = (int)(row / H_q);
  const int qh = (int)(row - (int64_t)b * H_q);
  const int G = H_q / H_kv;
  const bool acc = accept[(int64_t)b * H_kv + qh / G] != 0;
  float y;
  if (acc) {
    y = o_d[i] / fmaxf(l_d[row], 1e-6f);
  } else {
    const float md = m_d[row], mc = m_c[row];
    const float mm = fmaxf(md, mc);
    const float sd = expf(md - mm), sc = expf(mc - mm);
    const float lm = l_d[row] * sd + l_c[row] * sc;
    y = (o_d[i] * sd + o_c[i] * sc) / fmaxf(lm, 1e-6f);
  }
  if (dtype == CVSA_DTYPE_BF16)
    reinterpret_cast<uint16_t *>(out)[i] = (uint16_t)f32_to_bf16_bits(y);
  else if (dtype == CVSA_DTYPE_FP16)
    reinterpret_cast<__half *>(out)[i] = __float2half_rn(y);
  else
    reinterpret_cast<float *>(out)[i] = y;
}

}  // namespace cvsa

using namespace cvsa;

extern "C" int cvsa_compute_complement(const int32_t *page_indices, int64_t idx_stride,
                                       const int32_t *n_per_head,
                                       const int32_t *context_lens, int32_t block_size,
                                       const uint8_t *accept, int32_t B, int32_t H_kv,
                                       int32_t width, int32_t *comp_indices,
                                       int32_t *n_comp, void *stream) {
  CVSA_REQUIRE(page_indices && n_per_head && context_lens && comp_indices && n_comp,
               CVSA_ERR_INVALID, "compute_complement: null pointer argument");
  CVSA_REQUIRE(B > 0 && H_kv > 0 && block_size > 0 && width > 0 && idx_stride >= 0,
               CVSA_ERR_INVALID, "compute_complement: bad sizes B=%d H_kv=%d width=%d", B,
               H_kv, width);
  CVSA_REQUIRE(width <= kMaxPagesWide, CVSA_ERR_UNSUPPORTED,
               "compute_complement: width=%d exceeds %d pages", width, kMaxPagesWide);
  // Selection rows are idx_stride wide; all of a row is candidate selection.
  const int sel_width = (int)(idx_stride > kMaxPagesWide ? kMaxPagesWide : idx_stride);
  hipLaunchKernelGGL(complement_kernel, dim3(B * H_kv), dim3(kCompThreads), 0,
                     (hipStream_t)stream, page_indices, idx_stride, sel_width, n_per_head,
                     context_lens, block_size, accept, H_kv, width, comp_indices, n_comp);
  return cvsa_host::check_launch("compute_complement");
}

extern "C" int cvsa_lse_merge(const float *o_d, const float *m_d, const float *l_d,
                              const float *o_c, const float *m_c, const float *l_c,
                              const uint8_t *accept, int32_t B, int32_t H_q, int32_t H_kv,
                              int32_t D, void *out, int32_t out_dtype, void *stream) {
  CVSA_REQUIRE(o_d && m_d && l_d && o_c && m_c && l_c && accept && out, CVSA_ERR_INVALID,
               "lse_merge: null pointer argument");
  CVSA_REQUIRE(B > 0 && H_kv > 0 && H_q > 0 && H_q % H_kv == 0 && D > 0, CVSA_ERR_INVALID,
               "lse_merge: bad sizes B=%d H_q=%d H_kv=%d D=%d", B, H_q, H_kv, D);
  CVSA_REQUIRE(out_dtype >= CVSA_DTYPE_BF16 && out_dtype <= CVSA_DTYPE_FP32,
               CVSA_ERR_INVALID, "lse_merge: bad output dtype %d", out_dtype);
  const int64_t total = (int64_t)B * H_q * D;
  const int64_t blocks = (total + 255) / 256;
  hipLaunchKernelGGL(lse_merge_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, o_d, m_d, l_d, o_c, m_c, l_c, accept, H_q, H_kv, D,
                     total, out, out_dtype);
  return cvsa_host::check_launch("lse_merge");
}
