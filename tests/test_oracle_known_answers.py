"""The reference's own known-answer tests, run against the CPU oracle.

Each test restates one test of the reference's tests/ directory (cited) with
the same inputs and expected values, so the oracle is pinned to the answers
the reference's authors fixed.
"""
import pytest
import torch

from oracle import cvsa_oracle as ref
from oracle.backend_oracle import OracleCVSABackend


# ---- tests/test_complement.py:10-100 (compute_complement_pages) ----------

def test_complement_basic():
    """tests/test_complement.py:10-40: 10 pages; {0,2,4} -> 7, {1,3} -> 8."""
    ctx = torch.tensor([160])
    pi = torch.zeros(1, 2, 3, dtype=torch.int32)
    pi[0, 0] = torch.tensor([0, 2, 4])
    pi[0, 1] = torch.tensor([1, 3, 0])
    nph = torch.tensor([[3, 2]], dtype=torch.int32)
    comp, n = ref.compute_complement_pages(pi, nph, ctx, 16)
    assert n[0, 0].item() == 7 and n[0, 1].item() == 8
    for h in range(2):
        sel = set(pi[0, h, :int(nph[0, h])].tolist())
        c = set(comp[0, h, :int(n[0, h])].tolist())
        assert not (sel & c)
        assert len(sel | c) == 10


def test_complement_accept_mask():
    """tests/test_complement.py:43-65: accepted heads -> 0, rejected -> 3."""
    ctx = torch.tensor([80])
    pi = torch.zeros(1, 4, 2, dtype=torch.int32)
    pi[0, :, 0] = torch.tensor([0, 1, 2, 3])
    pi[0, :, 1] = torch.tensor([1, 2, 3, 4])
    nph = torch.full((1, 4), 2, dtype=torch.int32)
    acc = torch.tensor([[True, False, True, False]])
    _, n = ref.compute_complement_pages(pi, nph, ctx, 16, acc)
    assert n[0].tolist() == [0, 3, 0, 3]


def test_complement_full_budget():
    """tests/test_complement.py:68-81: every page selected -> empty, dummy width 1."""
    comp, n = ref.compute_complement_pages(torch.tensor([[[0, 1, 2]]], dtype=torch.int32),
                                           torch.tensor([[3]], dtype=torch.int32),
                                           torch.tensor([48]), 16)
    assert n[0, 0].item() == 0
    assert comp.shape == (1, 1, 1)


def test_complement_batch():
    """tests/test_complement.py:84-100: contexts 80 and 48 -> 3 and 1."""
    pi = torch.zeros(2, 1, 2, dtype=torch.int32)
    pi[0, 0] = torch.tensor([0, 1])
    pi[1, 0] = torch.tensor([0, 1])
    _, n = ref.compute_complement_pages(pi, torch.tensor([[2], [2]], dtype=torch.int32),
                                        torch.tensor([80, 48]), 16)
    assert n[0, 0].item() == 3 and n[1, 0].item() == 1


# ---- tests/test_lse_merge.py:29-108 (selective_lse_merge) ----------------

def _dense(q, k, v):
    """tests/test_lse_merge.py:10-15"""
    s = torch.einsum("bhd,bhnd->bhn", q, k) / (q.shape[-1] ** 0.5)
    return torch.einsum("bhn,bhnd->bhd", torch.softmax(s, dim=-1), v)


def _unnorm(q, k, v):
    """tests/test_lse_merge.py:18-26"""
    s = torch.einsum("bhd,bhnd->bhn", q, k) / (q.shape[-1] ** 0.5)
    m = s.max(dim=-1).values
    e = (s - m.unsqueeze(-1)).exp()
    return torch.einsum("bhn,bhnd->bhd", e, v), m, e.sum(-1)


def test_merge_equals_dense():
    """tests/test_lse_merge.py:29-51: draft(first 5) + complement(rest) == dense."""
    torch.manual_seed(42)
    B, H_q, D, N, H_kv = 1, 4, 64, 20, 2
    q = torch.randn(B, H_q, D)
    k = torch.randn(B, H_q, N, D)
    v = torch.randn(B, H_q, N, D)
    od, md, ld = _unnorm(q, k[:, :, :5], v[:, :, :5])
    oc, mc, lc = _unnorm(q, k[:, :, 5:], v[:, :, 5:])
    merged = ref.lse_merge(od, md, ld, oc, mc, lc, torch.zeros(B, H_kv, dtype=torch.bool),
                           H_q // H_kv, torch.float32)
    assert (merged - _dense(q, k, v)).abs().max().item() < 1e-4


def test_accepted_heads_use_draft():
    """tests/test_lse_merge.py:54-85: accepted -> draft (<1e-6), rejected -> dense (<1e-4)."""
    torch.manual_seed(42)
    B, H_kv, D, N, G = 1, 2, 64, 20, 2
    k = torch.randn(B, H_kv, N, D).repeat_interleave(G, dim=1)
    v = torch.randn(B, H_kv, N, D).repeat_interleave(G, dim=1)
    q = torch.randn(B, H_kv * G, D)
    od, md, ld = _unnorm(q, k[:, :, :5], v[:, :, :5])
    oc, mc, lc = _unnorm(q, k[:, :, 5:], v[:, :, 5:])
    merged = ref.lse_merge(od, md, ld, oc, mc, lc, torch.tensor([[True, False]]), G,
                           torch.float32)
    draft = od / ld.clamp(min=1e-6).unsqueeze(-1)
    assert (merged[:, :G] - draft[:, :G]).abs().max().item() < 1e-6
    assert (merged[:, G:] - _dense(q, k, v)[:, G:]).abs().max().item() < 1e-4


def test_all_accepted():
    """tests/test_lse_merge.py:88-108: complement (0, -inf, 0) -> o_d / l_d."""
    torch.manual_seed(42)
    od = torch.randn(1, 4, 64)
    md = torch.randn(1, 4)
    ld = torch.rand(1, 4) + 0.1
    merged = ref.lse_merge(od, md, ld, torch.zeros_like(od), torch.full_like(md, float("-inf")),
                           torch.zeros_like(ld), torch.ones(1, 2, dtype=torch.bool), 2,
                           torch.float32)
    assert (merged - od / ld.unsqueeze(-1)).abs().max().item() < 1e-6


# ---- tests/test_effective_budget.py:34-95 (_record_work / get_stats) -----

def _oracle_backend(**kw):
    d = dict(num_kv_heads=4, num_q_heads=32, head_dim=128, block_size=16, num_layers=32,
             budget_pct=0.05, coverage_threshold=0.90)
    d.update(kw)
    return OracleCVSABackend(**d)


def test_record_work_accumulates():
    """tests/test_effective_budget.py:34-57: 10/48 then 15/96."""
    b = _oracle_backend()
    assert b._attn_work is None
    ctx = torch.tensor([64, 128], dtype=torch.int32)
    b._record_work(ctx, torch.tensor(10))
    assert int(b._attn_work) == 10 and int(b._attn_work_max) == 48
    b._record_work(ctx, torch.tensor(5))
    assert int(b._attn_work) == 15 and int(b._attn_work_max) == 96


def test_get_stats_effective_budget():
    """tests/test_effective_budget.py:60-77: 2 of 16 pages -> 12.5 %."""
    b = _oracle_backend()
    assert "effective_budget_pct" not in b.get_stats()
    b._record_work(torch.tensor([64], dtype=torch.int32), torch.tensor(2))
    st = b.get_stats()
    assert abs(st["effective_budget_pct"] - 12.5) < 1e-6
    assert st["total_pages_attended"] == 2 and st["total_pages_max"] == 16


def test_reset_clears_effective_budget():
    """tests/test_effective_budget.py:80-95."""
    b = _oracle_backend()
    b._record_work(torch.tensor([64], dtype=torch.int32), torch.tensor(5))
    b.reset()
    assert "effective_budget_pct" not in b.get_stats()


# ---- tests/test_triton_kernels.py:117-155 (coverage vs torch restatement) -

@pytest.mark.parametrize("B,n_ctx,tau", [(1, 256, 0.8), (4, 512, 0.9), (4, 1024, 0.95)])
def test_coverage_matches_logsumexp_restatement(B, n_ctx, tau):
    """tests/test_triton_kernels.py:117-155: the oracle's coverage equals the
    logsumexp restatement (:134-141) within 1e-4 with identical accept masks.
    Data as make_test_data (:22-68): random fp32 page scores, budget 10 %."""
    g = torch.Generator().manual_seed(B * 1000 + n_ctx)
    H_kv = 8
    n_pages = (n_ctx - 1) // 16 + 1
    budget = max(3, int(n_pages * 0.10))
    ps = torch.randn(B, H_kv, n_pages, generator=g)
    _, idx = torch.topk(ps, budget, dim=-1)
    idx = idx.to(torch.int32)
    nph = torch.full((B, H_kv), budget, dtype=torch.int32)
    lse_all = torch.logsumexp(ps, dim=-1)
    sel = torch.gather(ps, 2, idx.long())
    cov_ref = (torch.logsumexp(sel, dim=-1) - lse_all).exp()
    acc, cov = ref.check_coverage(ps, idx, nph, tau)
    assert (cov - cov_ref).abs().max().item() < 1e-4
    assert torch.equal(acc, cov_ref >= tau)
