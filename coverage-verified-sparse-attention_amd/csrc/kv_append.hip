// Batched decode-token append into the paged KV cache.
//
// Follows SequenceKVManager.append_token_kv (cvsa/runtime/kv_cache.py:133-150)
// for a range of sequences at once: page = ctx // bs, offset = ctx % bs; a
// sequence at offset 0 whose page is not allocated yet takes the next block
// of the bump allocator (:142-146, PagedKVCache.allocate_blocks :53-62); the
// token's K and V rows are written (:148-149, write_kv :64-70) and ctx grows
// by one (:150).  The reference does this one sequence at a time with two
// host syncs each; here one workgroup handles up to 1024 sequences: a block
// scan numbers the sequences that need a block (in increasing b, the order
// the reference's loop allocates in), then all threads copy the rows.
#include "cvsa_common.h"

namespace cvsa {

constexpr int kAppendThreads = 1024;

__global__ __launch_bounds__(kAppendThreads) void append_kv_kernel(
    const uint16_t *__restrict__ k_new, const uint16_t *__restrict__ v_new,
    int64_t new_sb, uint16_t *__restrict__ k_cache, uint16_t *__restrict__ v_cache,
    int64_t num_blocks, int32_t *__restrict__ block_tables, int64_t bt_sb, int W,
    int32_t *__restrict__ context_lens, int32_t *__restrict__ pages_allocated,
    int seq_begin, int n_seqs, int next_free, int H_kv, int D, int block_size) {
  __shared__ int s_blk[kAppendThreads];
  __shared__ int s_off[kAppendThreads];
  __shared__ uint32_t wsum[kAppendThreads / kWave];
  const int i = threadIdx.x;
  const int lane = i & 63, wave = i >> 6;
  const int b = seq_begin + i;
  const int vec_per_row = H_kv * D / 8;
  const int total = n_seqs * vec_per_row;

  // The new rows do not depend on the slot: up to kPre 16-byte vectors per
  // thread are requested with the context lengths, so the copy below waits
  // for no load of its own (a batch of more rows loads them in the loop).
  constexpr int kPre = 4;
  const bool pre = total <= kPre * kAppendThreads;  // uniform
  uint4 pk[kPre], pv[kPre];
  if (pre) {
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
      const int v = min(i + k * kAppendThreads, total - 1);
      const int s = v / vec_per_row;
      const int64_t src = s * new_sb + (v - s * vec_per_row) * 8;
      pk[k] = *reinterpret_cast<const uint4 *>(k_new + src);
      pv[k] = *reinterpret_cast<const uint4 *>(v_new + src);
    }
  }

  int ctx = 0, page = 0, off = 0;
  uint32_t need = 0;
  if (i < n_seqs) {
    ctx = context_lens[b];
    page = ctx / block_size;
    off = ctx - page * block_size;
    need = (off == 0 && page >= pages_allocated[b]) ? 1u : 0u;
  }
  uint32_t incl = need;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t x = __shfl_up(incl, o, 64);
    if (lane >= o) incl += x;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t before = 0;
#pragma unroll
  for (int w = 0; w < kAppendThreads / kWave; ++w) before += (w < wave) ? wsum[w] : 0u;
  const uint32_t rank = before + incl - need;

  if (i < n_seqs) {
    int blk = -1;
    if (page >= 0 && page < W) {
      if (need) {
        blk = next_free + (int)rank;
        block_tables[b * bt_sb + page] = blk;
        pages_allocated[b] += 1;
      } else {
        blk = block_tables[b * bt_sb + page];
      }
    }
    s_blk[i] = (blk >= 0 && blk < num_blocks) ? blk : -1;
    s_off[i] = off;
  }
  __syncthreads();

  // Copy the K and V rows: [H_kv, D] bf16 per sequence, as 16-byte vectors.
  auto dst_of = [&](int v, int &s) {
    s = v / vec_per_row;
    const int blk = s_blk[s];
    return blk < 0 ? (int64_t)-1
                   : ((int64_t)blk * block_size + s_off[s]) * H_kv * D + (v - s * vec_per_row) * 8;
  };
  if (pre) {
#pragma unroll
    for (int k = 0; k < kPre; ++k) {
      const int v = i + k * kAppendThreads;
      int s;
      const int64_t dst = v < total ? dst_of(v, s) : (int64_t)-1;
      if (dst < 0) continue;
      *reinterpret_cast<uint4 *>(k_cache + dst) = pk[k];
      *reinterpret_cast<uint4 *>(v_cache + dst) = pv[k];
    }
  } else {
    for (int v = i; v < total; v += kAppendThreads) {
      int s;
      const int64_t dst = dst_of(v, s);
      if (dst < 0) continue;
      const int64_t src = s * new_sb + (v - s * vec_per_row) * 8;
      *reinterpret_cast<uint4 *>(k_cache + dst) = *reinterpret_cast<const uint4 *>(k_new + src);
      *reinterpret_cast<uint4 *>(v_cache + dst) = *reinterpret_cast<const uint4 *>(v_new + src);
    }
  }
  if (i < n_seqs) context_lens[b] = ctx + 1;
}

}  // namespace cvsa

using namespace cvsa;

extern "C" int cvsa_append_kv(const uint16_t *k_new, const uint16_t *v_new,
                              int64_t new_stride_b, uint16_t *k_cache, uint16_t *v_cache,
                              int64_t num_blocks, int32_t *block_tables, int64_t bt_stride_b,
                              int32_t W, int32_t *context_lens, int32_t *pages_allocated,
                              int32_t seq_begin, int32_t n_seqs, int32_t next_free_block,
                              int32_t H_kv, int32_t D, int32_t block_size, void *stream) {
  CVSA_REQUIRE(k_new && v_new && k_cache && v_cache && block_tables && context_lens &&
                   pages_allocated,
               CVSA_ERR_INVALID, "append_kv: null pointer argument");
  CVSA_REQUIRE(n_seqs > 0 && n_seqs <= kAppendThreads && seq_begin >= 0 && H_kv > 0 &&
                   W > 0 && num_blocks > 0 && block_size > 0 && bt_stride_b >= W,
               CVSA_ERR_INVALID, "append_kv: bad sizes n_seqs=%d H_kv=%d W=%d", n_seqs,
               H_kv, W);
  CVSA_REQUIRE(head_dim_supported(D), CVSA_ERR_UNSUPPORTED,
               "append_kv: D=%d not in {32, 64, 128, 256}", D);
  CVSA_REQUIRE(((uintptr_t)k_new & 15) == 0 && ((uintptr_t)v_new & 15) == 0 &&
                   new_stride_b % 8 == 0 && ((uintptr_t)k_cache & 15) == 0 &&
                   ((uintptr_t)v_cache & 15) == 0,
               CVSA_ERR_INVALID, "append_kv: rows must be 16-byte aligned");
  hipLaunchKernelGGL(append_kv_kernel, dim3(1), dim3(kAppendThreads), 0, (hipStream_t)stream,
                     k_new, v_new, new_stride_b, k_cache, v_cache, num_blocks, block_tables,
                     bt_stride_b, W, context_lens, pages_allocated, seq_begin, n_seqs,
                     next_free_block, H_kv, D, block_size);
  return cvsa_host::check_launch("append_kv");
}
