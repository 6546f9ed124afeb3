"""Complement page sets for CVSA verification.

Same signature and return contract as the reference's cvsa/complement.py:11-69:
(complement_indices [B, H_kv, max_complement] int32, n_complement [B, H_kv]
int32), with max_complement the largest count, or a [B, H_kv, 1] zero dummy
when every head is empty (:60-63).  The reference orders pages through an
unstable sort (:66-67); here they are ascending.  Runs the HIP complement
kernel; the output width needs two host reads, as in the reference (:32, :60).
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import ops


def compute_complement_pages(page_indices: torch.Tensor, n_per_head: torch.Tensor,
                             context_lens: torch.Tensor, block_size: int,
                             accept_mask: Optional[torch.Tensor] = None
                             ) -> Tuple[torch.Tensor, torch.Tensor]:
    comp, ncomp = ops.compute_complement(page_indices, n_per_head, context_lens, block_size,
                                         accept_mask)
    max_comp = int(ncomp.max().item()) if ncomp.numel() else 0
    if max_comp == 0:
        B, H = ncomp.shape
        return torch.zeros(B, H, 1, dtype=torch.int32, device=comp.device), ncomp
    return comp[..., :max_comp].contiguous(), ncomp
