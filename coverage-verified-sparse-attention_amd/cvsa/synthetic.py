"""Seeded synthetic paged-KV inputs for the decode-path configurations.

q, K and V are drawn i.i.d. N(0, 1) in fp32 and rounded to bf16.  Physical
pages are a random permutation of the pool, so block tables are never the
identity.  A "hot" page of KV head h in sequence b has every key shifted by
``shift * qhat`` before rounding, where qhat is the unit vector of the fp32
GQA group mean of q[b]: the page-scoring statistic q_rep . k then rises by
``shift`` of its own standard deviation (std(q_rep . k) = |q_rep| for
k ~ N(0, I)).  Sink pages (the first ``sink_pages`` logical pages) get the
same kind of shift on every head.

The pool holds B * P used blocks (P = pages of the context) plus
``spare_blocks`` free ones; the free ones are the ids >= B * P, which is
where PagedKVCache's bump allocator continues for appended tokens.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import torch


@dataclass
class PagedInputs:
    q: torch.Tensor              # [B, H_q, D] bf16
    k_cache: torch.Tensor        # [num_blocks, bs, H_kv, D] bf16
    v_cache: torch.Tensor
    block_tables: torch.Tensor   # [B, W] int32
    context_lens: torch.Tensor   # [B] int32
    num_kv_heads: int
    num_q_per_kv: int
    block_size: int
    used_blocks: int             # first free block id
    hot_pages: List[List[List[int]]] = field(default_factory=list)  # [b][h] -> logical pages


def _generator(device: torch.device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_paged_inputs(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                      context_len, block_size: int = 16, seed: int = 0,
                      device="cpu", max_pages: Optional[int] = None, spare_blocks: int = 16,
                      hot_heads: Optional[Sequence[int]] = None, n_hot: int = 8,
                      n_hot_range: Optional[Sequence[int]] = None, hot_shift: float = 3.0,
                      sink_pages: int = 0, sink_shift: float = 0.0,
                      random_hot_heads: int = 0) -> PagedInputs:
    """Build one layer's decode inputs.

    context_len: int, or a per-sequence list.
    hot_heads:   KV heads that get hot pages (default: every other head);
                 ignored when ``n_hot_range`` is given.
    n_hot_range: (lo, hi): every (b, h) draws its hot-page count from U{lo..hi}.
    random_hot_heads: if > 0, each sequence draws this many hot heads at
                 random (instead of ``hot_heads``).
    """
    device = torch.device(device)
    g = _generator(device, seed)
    B, H, D, bs = batch, num_kv_heads, head_dim, block_size
    G = num_q_heads // num_kv_heads
    ctxs = [int(context_len)] * B if isinstance(context_len, int) else [int(c) for c in context_len]
    pages = [max(1, -(-c // bs)) for c in ctxs]
    P = max(pages)
    W = max_pages if max_pages is not None else P
    if W < P:
        raise ValueError(f"max_pages={W} < pages of the context {P}")
    used = sum(pages)
    num_blocks = used + spare_blocks

    q32 = torch.randn(B, num_q_heads, D, generator=g, device=device, dtype=torch.float32)
    q = q32.to(torch.bfloat16)
    K = torch.randn(num_blocks, bs, H, D, generator=g, device=device, dtype=torch.float32)
    V = torch.randn(num_blocks, bs, H, D, generator=g, device=device, dtype=torch.float32)
    perm = torch.randperm(used, generator=g, device=device).to(torch.int32)
    bt = torch.zeros(B, W, dtype=torch.int32, device=device)
    off = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]

    qrep = q.to(torch.float32).view(B, H, G, D).mean(dim=2)
    qhat = qrep / qrep.norm(dim=-1, keepdim=True).clamp(min=1e-12)       # [B, H, D]

    if hot_heads is None:
        hot_heads = list(range(0, H, 2))
    hot: List[List[List[int]]] = [[[] for _ in range(H)] for _ in range(B)]
    for b in range(B):
        nv = pages[b]
        cand = max(0, nv - sink_pages)
        if random_hot_heads:
            hot_heads = torch.randperm(H, generator=g, device=device)[:random_hot_heads].tolist()
        if sink_pages and sink_shift:
            phys = bt[b, :min(sink_pages, nv)].long()
            K[phys] += sink_shift * qhat[b].view(1, 1, H, D)
        for h in range(H):
            if n_hot_range is not None:
                lo, hi = n_hot_range
                cnt = int(torch.randint(lo, hi + 1, (1,), generator=g, device=device))
            else:
                cnt = n_hot if h in hot_heads else 0
            cnt = min(cnt, cand)
            if cnt == 0:
                continue
            sel = torch.randperm(cand, generator=g, device=device)[:cnt] + sink_pages
            hot[b][h] = sorted(int(x) for x in sel.tolist())
            phys = bt[b, sel].long()
            K[phys, :, h, :] += hot_shift * qhat[b, h]
    ctx_t = torch.tensor(ctxs, dtype=torch.int32, device=device)
    return PagedInputs(q=q, k_cache=K.to(torch.bfloat16), v_cache=V.to(torch.bfloat16),
                       block_tables=bt, context_lens=ctx_t, num_kv_heads=H, num_q_per_kv=G,
                       block_size=bs, used_blocks=used, hot_pages=hot)


def jitter_query(q: torch.Tensor, scale: float, seed: int) -> torch.Tensor:
    """q + scale * N(0, 1), rounded to bf16: the next decode step's query."""
    g = _generator(q.device, seed)
    noise = torch.randn(q.shape, generator=g, device=q.device, dtype=torch.float32)
    return (q.to(torch.float32) + scale * noise).to(torch.bfloat16)
