"""Selective log-sum-exp merge of draft and complement attention.

Same signature and semantics as the reference's cvsa/lse_merge.py:11-54:
accepted KV heads return the normalised draft, rejected heads the online
softmax merge of draft and complement (the exact dense result).  Runs the
HIP merge kernel; tensors must be on the GPU.
"""
from __future__ import annotations

import torch

from . import ops


def selective_lse_merge(o_draft: torch.Tensor, m_draft: torch.Tensor, l_draft: torch.Tensor,
                        o_comp: torch.Tensor, m_comp: torch.Tensor, l_comp: torch.Tensor,
                        accept_mask: torch.Tensor, num_q_per_kv: int,
                        output_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """[B, H_q, D] in output_dtype (cvsa/lse_merge.py:11-54)."""
    return ops.lse_merge(o_draft, m_draft, l_draft, o_comp, m_comp, l_comp, accept_mask,
                         accept_mask.shape[1], num_q_per_kv, output_dtype)
