"""Seeded inputs of the golden backend traces (plain torch, CPU).

Shared by make_backend_trace.py, which runs the reference implementation on
them, and by the tests, which rebuild the same tensors and compare the
oracle and the HIP path with the recorded results.  Everything is drawn from
one torch.Generator; ``input_digest`` fingerprints the tensors so that a
change of generator behaviour is caught instead of silently comparing
different inputs.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import List

import torch

BLOCK = 16


@dataclass
class GoldenCase:
    q: List[torch.Tensor]            # per step [B, H_q, D] bf16
    k_new: List[torch.Tensor]        # per step [B, H_kv, D] bf16 (appended after the call)
    v_new: List[torch.Tensor]
    k_cache: torch.Tensor            # [num_blocks, 16, H_kv, D] bf16
    v_cache: torch.Tensor
    block_tables: torch.Tensor       # [B, W] int32
    context_lens: torch.Tensor       # [B] int32
    pages_allocated: List[int]
    next_free: int


def make_case(seed: int, batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
              context_lens: List[int], steps: int, hot_heads: List[int], n_hot: int,
              shift: float, spare_blocks: int = 8) -> GoldenCase:
    g = torch.Generator().manual_seed(seed)
    G = num_q_heads // num_kv_heads
    pages = [(c + BLOCK - 1) // BLOCK for c in context_lens]
    used = sum(pages)
    W = max((c + steps + BLOCK - 1) // BLOCK for c in context_lens) + 1
    nb = used + spare_blocks + batch * ((steps + BLOCK - 1) // BLOCK + 1)
    k = torch.randn(nb, BLOCK, num_kv_heads, head_dim, generator=g)
    v = torch.randn(nb, BLOCK, num_kv_heads, head_dim, generator=g)
    q0 = torch.randn(batch, num_q_heads, head_dim, generator=g).to(torch.bfloat16)
    perm = torch.randperm(used, generator=g).to(torch.int32)
    bt = torch.zeros(batch, W, dtype=torch.int32)
    off = 0
    for b in range(batch):
        bt[b, :pages[b]] = perm[off:off + pages[b]]
        off += pages[b]
    # Hot pages: keys shifted along the unit group-mean query of their head,
    # in fp32 before rounding to bf16.
    q_rep = q0.float().view(batch, num_kv_heads, G, head_dim).mean(2)
    q_hat = q_rep / q_rep.norm(dim=-1, keepdim=True)
    for b in range(batch):
        for h in hot_heads:
            sel = torch.randperm(pages[b], generator=g)[:n_hot]
            for p in sel.tolist():
                k[int(bt[b, p]), :, h, :] += shift * q_hat[b, h]
    q_steps, k_new, v_new = [], [], []
    for _ in range(steps):
        q_steps.append((q0.float() + 0.3 * torch.randn(q0.shape, generator=g)).to(torch.bfloat16))
        k_new.append(torch.randn(batch, num_kv_heads, head_dim, generator=g).to(torch.bfloat16))
        v_new.append(torch.randn(batch, num_kv_heads, head_dim, generator=g).to(torch.bfloat16))
    return GoldenCase(q_steps, k_new, v_new, k.to(torch.bfloat16), v.to(torch.bfloat16), bt,
                      torch.tensor(context_lens, dtype=torch.int32), pages, used)


def input_digest(case: GoldenCase) -> str:
    h = hashlib.sha256()
    for t in (case.k_cache, case.v_cache, case.block_tables, case.context_lens, *case.q,
              *case.k_new, *case.v_new):
        h.update(t.contiguous().view(torch.uint8).numpy().tobytes())
    return h.hexdigest()


# Scenarios: backend keyword arguments plus the input recipe.  Sizes are small
# enough for the reference's kernels under the Triton interpreter on a CPU.
SCENARIOS = {
    "lazy_m3": dict(
        inputs=dict(seed=1101, batch=2, num_q_heads=8, num_kv_heads=2, head_dim=128,
                    context_lens=[700, 512], steps=10, hot_heads=[0, 1], n_hot=4, shift=8.0),
        backend=dict(budget_pct=0.25, coverage_threshold=0.855, lazy=True, check_interval=3)),
    "fixed_r3": dict(
        inputs=dict(seed=1102, batch=1, num_q_heads=8, num_kv_heads=2, head_dim=128,
                    context_lens=[600], steps=7, hot_heads=[0, 1], n_hot=4, shift=7.0),
        backend=dict(budget_pct=0.25, coverage_threshold=0.87, lazy=False, reuse_interval=3)),
    "lazy_cov1_gqa7": dict(
        inputs=dict(seed=1103, batch=1, num_q_heads=14, num_kv_heads=2, head_dim=128,
                    context_lens=[640], steps=7, hot_heads=[0, 1], n_hot=4, shift=9.0),
        backend=dict(budget_pct=0.25, coverage_threshold=0.77, lazy=True, check_interval=3,
                     coverage_interval=1)),
    # cfg1 of BASELINE: 8B attention shapes, one sequence of 8192 tokens (512
    # pages), budget 1/4, tau 0.9, exact recovery; a scoring step then a reuse
    # step.  "cfg1": the literal recipe (+3 sigma hot pages on heads 0, 2, 4,
    # 6: every head's coverage falls below tau and is recovered); "cfg1_mixed":
    # +12 sigma, so the hot heads pass and the others are recovered.
    "cfg1": dict(
        inputs=dict(seed=1001, batch=1, num_q_heads=32, num_kv_heads=8, head_dim=128,
                    context_lens=[8192], steps=2, hot_heads=[0, 2, 4, 6], n_hot=8, shift=3.0),
        backend=dict(budget_pct=0.25, coverage_threshold=0.9, lazy=False, reuse_interval=2),
        record_state=True),
    "cfg1_mixed": dict(
        inputs=dict(seed=1011, batch=1, num_q_heads=32, num_kv_heads=8, head_dim=128,
                    context_lens=[8192], steps=2, hot_heads=[0, 2, 4, 6], n_hot=8,
                    shift=12.0),
        backend=dict(budget_pct=0.25, coverage_threshold=0.9, lazy=False, reuse_interval=2),
        record_state=True),
    "approx_lazy": dict(
        inputs=dict(seed=1104, batch=1, num_q_heads=8, num_kv_heads=2, head_dim=128,
                    context_lens=[512], steps=5, hot_heads=[0, 1], n_hot=3, shift=8.0),
        backend=dict(budget_pct=0.125, coverage_threshold=0.8, lazy=True, check_interval=2,
                     approx_recovery_pct=0.5)),
}
