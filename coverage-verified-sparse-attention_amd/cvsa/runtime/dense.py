"""Dense paged decode attention over every valid page.

API of the reference's DenseAttentionBackend (cvsa/runtime/dense.py:16-111).
The reference tries FlashInfer and falls back to its sparse kernel with all
pages selected (:40-68); here the HIP paged-decode kernel walks every valid
page directly (no index list), for every GQA ratio in 1..128.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import ops


class DenseAttentionBackend:
    """Backend protocol: __call__(q, k_cache, v_cache, block_tables, context_lens,
    layer_idx) -> [B, H_q, D] in q.dtype."""

    def __init__(self, num_kv_heads, num_q_heads, head_dim, block_size):
        self.num_kv_heads = num_kv_heads
        self.num_q_heads = num_q_heads
        self.num_q_per_kv = num_q_heads // num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size

    def reset(self):
        pass

    def step_done(self, layer_idx, num_layers):
        pass

    def __call__(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                 work: Optional[torch.Tensor] = None):
        return ops.dense_decode(q, k_cache, v_cache, block_tables, context_lens,
                                self.num_kv_heads, self.num_q_per_kv, self.block_size,
                                work=work)
