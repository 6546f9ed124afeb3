"""Per-head budget selection (cvsa_select_budgeted, cvsa_adaptive_budgets)
against the oracle's restatements of CVSABackend._topp_select,
_static_select and _adaptive_select (cvsa/backend.py:522-681), and the
backend's top-p / static-table / adaptive schedules against the oracle
backend.

Top-p budgets depend on where the cumulative softmax mass crosses top_p.
The kernel sums the masses as 40-bit fixed point (cumulative error below
2e-8 of the total at W = 32768) and the oracle in fp64, so they agree
except where the oracle's cumulative mass at the boundary lies within 1e-7
of top_p; such rows may differ by one page and are checked against both
neighbours."""
import math

import pytest
import torch

from oracle import cvsa_oracle as ref
from cvsa import ops
from test_gpu_backend import _run

pytestmark = pytest.mark.gpu

BOUNDARY_EPS = 1e-7


def _ctx_for(W, valid):
    return torch.tensor([v * 16 - 5 for v in valid], dtype=torch.int32)


def _scores(B, H, W, valid, seed, temp):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn(B, H, W, generator=g) * temp
    for b, v in enumerate(valid):
        s[b, :, v:] = float("-inf")
    return s


def _check_topp(s, ctx, p, idx, nph, width=None):
    """Every row: n_per_head and the selected set agree with the oracle,
    allowing the neighbouring budget where the boundary is within eps."""
    B, H, W = s.shape
    width = W if width is None else width
    need, order = ref.topp_need(s, p)
    sd = s.double()
    probs = torch.softmax(sd, dim=-1)
    cum = torch.cumsum(probs.gather(-1, order), dim=-1)
    p32 = float(torch.tensor(p, dtype=torch.float32))
    nv = ref.n_valid_pages(ctx, 16)
    loose = 0
    for b in range(B):
        for h in range(H):
            k = int(need[b, h])
            cands = [k]
            if k >= 2 and abs(float(cum[b, h, k - 2]) - p32) < BOUNDARY_EPS:
                cands.append(k - 1)
            if k <= W - 1 and abs(float(cum[b, h, k - 1]) - p32) < BOUNDARY_EPS:
                cands.append(k + 1)
            cands = {min(max(c, 3), W) for c in cands}
            got_n = int(nph[b, h])
            ok = False
            for c in cands:
                c = min(c, width)
                n = min(c, int(nv[b]))
                if got_n != n:
                    continue
                want = sorted(order[b, h, :n].tolist())
                if idx[b, h, :n].tolist() == want:
                    ok = True
                    break
            assert ok, (b, h, k, got_n, sorted(cands))
            loose += len(cands) > 1
    return loose


@pytest.mark.parametrize("W,temp", [(100, 1.0), (1000, 2.0), (4096, 0.5), (8192, 3.0),
                                    (20000, 1.5)])
@pytest.mark.parametrize("p", [0.5, 0.9, 0.99])
def test_topp_matches_oracle(gpu, W, temp, p):
    B, H = 2, 4
    valid = [W, max(3, W // 3)]
    s = _scores(B, H, W, valid, seed=W + int(100 * p), temp=temp)
    ctx = _ctx_for(W, valid)
    idx, nph = ops.select_budgeted(s.to(gpu), ctx.to(gpu), 16, top_p=p)
    loose = _check_topp(s, ctx, p, idx.cpu(), nph.cpu())
    assert loose < B * H   # most rows are held to the exact budget


def test_topp_ties_and_clusters(gpu):
    """Rows that send the crossing bucket down the slow paths: heavy exact
    ties (> 64 equal scores, walked in page order), a tight cluster (second
    level), all-equal finite scores, +inf / NaN rows (need 1 -> 3) and a
    width below the budget."""
    W = 3000
    rows = []
    g = torch.Generator().manual_seed(9)
    t = torch.full((W,), -5.0)
    t[torch.randperm(W, generator=g)[:500]] = 1.0           # 500 equal top scores
    rows.append(t)
    c = torch.randn(W, generator=g) - 6.0
    c[:800] = 2.0 + torch.rand(800, generator=g) * 1e-3    # tight cluster of 800
    rows.append(c)
    rows.append(torch.full((W,), 0.25))                     # all equal
    i = torch.randn(W, generator=g)
    i[17] = float("inf")
    rows.append(i)
    n = torch.randn(W, generator=g)
    n[5] = float("nan")
    rows.append(n)
    rows.append(torch.randn(W, generator=g) * 0.01)         # nearly flat: large budgets
    s = torch.stack(rows).view(len(rows), 1, W)
    ctx = torch.full((len(rows),), W * 16, dtype=torch.int32)
    for p in (0.3, 0.9):
        idx, nph = ops.select_budgeted(s.to(gpu), ctx.to(gpu), 16, top_p=p)
        _check_topp(s, ctx, p, idx.cpu(), nph.cpu())
        assert int(nph[3]) == 3 and int(nph[4]) == 3
        idx, nph = ops.select_budgeted(s.to(gpu), ctx.to(gpu), 16, top_p=p, width=64)
        _check_topp(s, ctx, p, idx.cpu(), nph.cpu(), width=64)


def test_topp_gate_and_separate_ranking(gpu):
    B, H, W = 2, 8, 2048
    valid = [W, 700]
    gate = _scores(B, H, W, valid, seed=3, temp=2.0)
    rank = gate + 0.3 * torch.randn(B, H, W, generator=torch.Generator().manual_seed(4))
    ctx = _ctx_for(W, valid)
    idx, nph, acc, cov = ops.select_budgeted(gate.to(gpu), ctx.to(gpu), 16, top_p=0.8,
                                             tau=0.85, sel_scores=rank.to(gpu))
    _check_topp(rank, ctx, 0.8, idx.cpu(), nph.cpu())
    wacc, wcov = ref.check_coverage(gate, idx.cpu(), nph.cpu(), 0.85)
    assert (cov.cpu() - wcov).abs().max().item() < 1e-5
    margin = (wcov - 0.85).abs() > 1e-5
    assert torch.equal(acc.cpu()[margin], wacc[margin])


@pytest.mark.parametrize("W", [64, 5000])
def test_static_table_matches_oracle(gpu, W):
    B, H = 3, 4
    valid = [W, W // 2, 2]
    s = _scores(B, H, W, valid, seed=W, temp=1.0)
    ctx = _ctx_for(W, valid)
    fr = [0.05, 0.2, 0.5, 0.01]
    per_head = ref.static_budgets(fr, W)
    width = int(per_head.max())
    idx, nph, acc, cov = ops.select_budgeted(
        s.to(gpu), ctx.to(gpu), 16,
        row_budgets=per_head.to(torch.int32).view(1, H).expand(B, H).contiguous().to(gpu),
        width=width, tau=0.9)
    widx, wnph = ref.static_select(s, fr, ctx, 16)
    assert torch.equal(nph.cpu(), wnph)
    for b in range(B):
        for h in range(H):
            n = int(wnph[b, h])
            assert idx[b, h, :n].cpu().tolist() == widx[b, h, :n].tolist(), (b, h)
    wacc, wcov = ref.check_coverage(s, widx, wnph, 0.9)
    assert (cov.cpu() - wcov).abs().max().item() < 1e-5


@pytest.mark.parametrize("H,W,base,floor", [(4, 64, 10, 0.0), (8, 3000, 300, 0.5),
                                            (8, 2048, 200, 0.25), (2, 500, 499, 0.0),
                                            (8, 8192, 1024, 0.5), (16, 5000, 100, 0.5)])
def test_adaptive_budgets_match_oracle(gpu, H, W, base, floor):
    """Budgets exact (ties at the threshold to the lower head on both sides;
    rounded scores make many ties), then the selection by those budgets.
    The shapes take the register-resident kernels (H * W up to 64K scores)
    and the streaming one (16 x 5000)."""
    B = 3
    valid = [W, W // 2, 5]
    g = torch.Generator().manual_seed(W + H)
    s = (torch.randn(B, H, W, generator=g) * 3).round()
    for b, v in enumerate(valid):
        s[b, :, v:] = float("-inf")
    ctx = _ctx_for(W, valid)
    got = ops.adaptive_budgets(s.to(gpu), base, ctx.to(gpu), 16, floor)
    want = ref.adaptive_budgets(s, base, ctx, 16, floor)
    assert torch.equal(got.cpu(), want)
    width = int(want.max())
    idx, nph, acc, cov = ops.select_budgeted(s.to(gpu), ctx.to(gpu), 16, row_budgets=got,
                                             width=width, tau=0.9)
    widx, wnph = ref.adaptive_select(s, base, ctx, 16, floor)
    assert torch.equal(nph.cpu(), wnph)
    for b in range(B):
        for h in range(H):
            n = int(wnph[b, h])
            assert idx[b, h, :n].cpu().tolist() == widx[b, h, :n].tolist(), (b, h)


def test_select_budgeted_rejects_bad_arguments(gpu):
    s = torch.zeros(1, 2, 10, device=gpu)
    ctx = torch.tensor([160], dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError):
        ops.select_budgeted(s, ctx, 16)
    with pytest.raises(ValueError):
        ops.select_budgeted(s, ctx, 16, top_p=1.0)
    with pytest.raises(ValueError):
        ops.select_budgeted(s, ctx, 16, top_p=0.5, width=11)
    with pytest.raises(ValueError):
        ops.select_budgeted(s, ctx, 16, row_budgets=torch.ones(1, 3, dtype=torch.int32,
                                                                device=gpu))


@pytest.mark.parametrize("sep", [False, True])
def test_select_or_keep_row_budgets(gpu, sep):
    """cvsa_select_or_keep_budgeted: keep the cached selection when every
    head passed; else the selection of select_budgeted with the same row
    budgets and width (budgets above the width clamped), with its gate,
    the scores cache and the counters of select_or_keep; and a fresh
    selection booked by its own gate."""
    B, H, W, width = 2, 4, 3000, 800
    valid = [W, 1100]
    g = torch.Generator().manual_seed(31 + sep)
    ps = _scores(B, H, W, valid, seed=41 + sep, temp=2.0)
    rank = ps + 0.4 * torch.randn(B, H, W, generator=g) if sep else None
    if rank is not None:
        rank[ps == float("-inf")] = float("-inf")
    ctx = _ctx_for(W, valid)
    rows = torch.tensor([[3, 200, 700, 50], [1000, 3, 10, 3000]], dtype=torch.int32)
    d = dict(sel_scores=None if rank is None else rank.to(gpu))
    sel0 = torch.randint(0, W, (B, H, width), generator=g).to(torch.int32)
    nph0 = torch.randint(0, width, (B, H), generator=g).to(torch.int32)
    d_sel, d_nph = sel0.to(gpu), nph0.to(gpu)
    old = torch.randn(B, H, W, generator=g)
    d_cache = old.to(gpu)
    cov = torch.full((B, H), -7.0, device=gpu)
    stats = torch.zeros(6, dtype=torch.int64, device=gpu)
    check = torch.ones(B, H, dtype=torch.bool, device=gpu)
    acc = ops.select_or_keep(ps.to(gpu), check, width, ctx.to(gpu), 16, 0.9, d_sel, d_nph, cov,
                             d_cache, stats, row_budgets=rows.to(gpu), **d)
    assert bool(acc.all())
    assert torch.equal(d_sel.cpu(), sel0) and torch.equal(d_nph.cpu(), nph0)
    assert torch.equal(d_cache.cpu(), old) and stats.tolist() == [1, 0, 0, B * H, 0, 0]
    check[1, 2] = False
    acc = ops.select_or_keep(ps.to(gpu), check, width, ctx.to(gpu), 16, 0.9, d_sel, d_nph, cov,
                             d_cache, stats, row_budgets=rows.to(gpu), **d)
    widx, wnph, wacc, wcov = ops.select_budgeted(ps.to(gpu), ctx.to(gpu), 16,
                                                 row_budgets=rows.to(gpu), width=width, tau=0.9,
                                                 **d)
    assert torch.equal(d_nph.cpu(), wnph.cpu())
    for b in range(B):
        for h in range(H):
            n = int(wnph[b, h])
            assert n == min(int(rows[b, h]), width, valid[b])
            assert torch.equal(d_sel[b, h, :n].cpu(), widx[b, h, :n].cpu()), (b, h)
    assert torch.equal(acc, wacc) and torch.equal(cov, wcov)
    assert torch.equal(d_cache.cpu(), ps)
    assert stats.tolist() == [1, 1, 1, 2 * B * H - 1, 0, 0]
    sel3, nph3, cov3 = torch.empty_like(d_sel), torch.empty_like(d_nph), torch.empty_like(cov)
    acc3 = ops.select_or_keep(ps.to(gpu), None, width, ctx.to(gpu), 16, 0.9, sel3, nph3, cov3,
                              None, stats, count_gate=True, row_budgets=rows.to(gpu), **d)
    assert torch.equal(nph3, wnph) and torch.equal(acc3, wacc)
    n_acc = int(acc3.sum())
    all_acc = int(n_acc == B * H)
    assert stats.tolist() == [1 + all_acc, 2 - all_acc, 2, 2 * B * H - 1 + n_acc, 0, 0]
    with pytest.raises(ValueError):
        ops.select_or_keep(ps.to(gpu), check, width, ctx.to(gpu), 16, 0.9, d_sel, d_nph, cov,
                           row_budgets=rows.to(gpu).to(torch.int64))


CFG = dict(batch=2, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=[5000, 2600],
           hot_heads=[0, 3, 6], n_hot=8, hot_shift=10.0)


# With the exact selector a top-p set's coverage is its own softmax mass
# (>= top_p), so tau is kept away from top_p: the gate then decides clearly.
@pytest.mark.parametrize("kw", [
    dict(top_p=0.9, coverage_threshold=0.95, lazy=True, check_interval=3),
    dict(top_p=0.7, coverage_threshold=0.9, lazy=False, reuse_interval=2),
    dict(top_p=0.9, coverage_threshold=0.9, lazy=True, check_interval=2, selector="quest"),
    dict(top_p=0.8, coverage_threshold=0.9, lazy=False, reuse_interval=1,
         approx_recovery_pct=0.4),
    dict(static_budget_table={0: [0.1, 0.3, 0.2, 0.05, 0.15, 0.25, 0.1, 0.4]},
         coverage_threshold=0.9, lazy=True, check_interval=3),
    dict(static_budget_table={0: [0.2] * 4 + [0.1] * 4}, coverage_threshold=0.9, lazy=False,
         reuse_interval=2),
    dict(static_budget_table={0: [0.05, 0.3, 0.1, 0.2, 0.15, 0.1, 0.25, 0.05]},
         coverage_threshold=0.9, lazy=True, check_interval=2, selector="quest"),
    dict(adaptive_selection=True, coverage_threshold=0.9, lazy=True, check_interval=3),
    dict(adaptive_selection=True, adaptive_floor_ratio=0.2, coverage_threshold=0.8,
         lazy=False, reuse_interval=2, selector="quest"),
])
def test_backend_budgeted_schedules(gpu, kw):
    kw = dict(budget_pct=0.2, **kw)
    stats, trace, _ = _run(gpu, CFG, kw, steps=7, seed=777)
    assert any(t["kind"].startswith("score") for t in trace)
