"""Rows of more than 32768 pages (up to 262144) against the CPU oracle.

Rows up to 32768 pages are selected and gated by kernels that hold the row
in registers; wider rows go to select_topk_wide_kernel and
check_coverage_wide_kernel, which stream the row from memory (an 8-bit
radix select of the k-th key, a tiled ascending compaction, the gate's two
log-sum-exps over the counted pages).  Selections, n_per_head, complements
and accept masks are compared bit-exact (accept away from tau by 1e-5),
coverage within 1e-5, outputs within the north star's 2e-2.  The backend
runs (lockstep with the oracle backend, every selection, mask, output and
counter compared) cover the whole decode step at widths only these kernels
serve: block size 16 and 8, a draft wider than 32768 pages, exact and
approximate recovery, a kept listed speculation and the dense speculation
of an all-rejected check, and the Quest, adaptive and static-table
selectors.
"""
import pytest
import torch

from oracle import cvsa_oracle as ref
from cvsa import ops
from test_gpu_backend import _run

pytestmark = pytest.mark.gpu

COV_ATOL = 1e-5


def _rows(B, H, W, seed, tail_valid=None):
    g = torch.Generator().manual_seed(seed)
    ps = torch.randn(B, H, W, generator=g)
    ps[0, H - 1] = (ps[0, H - 1] * 2).round() / 2      # heavy ties
    ctx = torch.tensor([W * 16] + [max(1, (tail_valid or W // 3) * 16 - 5)] * (B - 1),
                       dtype=torch.int32)
    nv = ref.n_valid_pages(ctx, 16)
    for b in range(1, B):
        ps[b, :, int(nv[b]):] = float("-inf")
    return ps, ctx


def _gate_ok(acc, cov, wacc, wcov, tau):
    assert (cov - wcov).abs().max().item() < COV_ATOL
    margin = (wcov - tau).abs() > 1e-5
    assert torch.equal(acc[margin], wacc[margin])


@pytest.mark.parametrize("W,budget", [(32769, 4096), (65536, 8192), (131072 + 37, 1),
                                      (131072 + 37, 16385), (262144, 32768),
                                      (40000, 40000), (50000, 3)])
def test_select_topk_wide_bit_exact(gpu, W, budget):
    ps, ctx = _rows(2, 2, W, W + budget)
    idx, nph, acc, cov = ops.select_topk(ps.to(gpu), budget, ctx.to(gpu), 16, tau=0.9)
    widx, wnph = ref.select_topk(ps, budget, ctx, 16)
    assert torch.equal(idx.cpu(), widx)
    assert torch.equal(nph.cpu(), wnph)
    wacc, wcov = ref.check_coverage(ps, widx, wnph, 0.9)
    _gate_ok(acc.cpu(), cov.cpu(), wacc, wcov, 0.9)
    # Without the gate: the same selection.
    idx2, nph2 = ops.select_topk(ps.to(gpu), budget, ctx.to(gpu), 16)
    assert torch.equal(idx2.cpu(), widx) and torch.equal(nph2.cpu(), wnph)


def test_select_topk_wide_special_rows(gpu):
    """The register kernel's special rows at W = 40000: all equal, +0/-0,
    one huge outlier, an fp32-overflowing range, +inf and NaN entries,
    near-ties in one bucket, fewer finite scores than the budget; and a
    row whose k-th value bucket holds more scores than the kernel ranks in
    LDS (an outlier stretches the range, so the bulk shares one bucket)."""
    W, budget = 40000, 5000
    g = torch.Generator().manual_seed(W)
    rows = [torch.full((W,), 1.25)]
    z = torch.zeros(W)
    z[torch.randperm(W, generator=g)[: W // 2]] = -0.0
    rows.append(z)
    r = torch.randn(W, generator=g)
    r[7] = 1e30
    rows.append(r)
    r = torch.randn(W, generator=g)
    r[3], r[W - 2] = 3.0e38, -3.0e38
    rows.append(r)
    r = torch.randn(W, generator=g)
    r[torch.randperm(W, generator=g)[:40]] = float("inf")
    r[11] = float("nan")
    rows.append(r)
    rows.append(1.0 + torch.randint(0, 50, (W,), generator=g).float() * 2.0 ** -20)
    r = torch.randn(W, generator=g)
    r[torch.randperm(W, generator=g)[: W - budget // 2]] = float("-inf")
    rows.append(r)
    r = 1.0 + torch.randint(0, 3000, (W,), generator=g).float() * 2.0 ** -22
    r[123] = 1000.0
    rows.append(r)
    ps = torch.stack(rows).view(1, len(rows), W)
    ctx = torch.tensor([W * 16], dtype=torch.int32)
    idx, nph, acc, cov = ops.select_topk(ps.to(gpu), budget, ctx.to(gpu), 16, tau=0.9)
    widx, wnph = ref.select_topk(ps, budget, ctx, 16)
    for h in range(len(rows)):
        assert torch.equal(idx.cpu()[0, h], widx[0, h]), h
    assert torch.equal(nph.cpu(), wnph)
    finite_rows = [0, 1, 2, 5, 7]
    wacc, wcov = ref.check_coverage(ps, widx, wnph, 0.9)
    assert (cov.cpu()[0, finite_rows] - wcov[0, finite_rows]).abs().max().item() < COV_ATOL


def test_select_or_keep_wide(gpu):
    """Keep, reselect in place (scores cached, counters booked) and a
    fresh selection booked by its own gate, at W = 50000."""
    W, budget = 50000, 6000
    B, H = 2, 2
    g = torch.Generator().manual_seed(77)
    ctx = torch.tensor([W * 16 - 3, (W // 2) * 16], dtype=torch.int32)
    old_ps = torch.randn(B, H, W, generator=g)
    new_ps = torch.randn(B, H, W, generator=g)
    nv = ref.n_valid_pages(ctx, 16)
    new_ps[1, :, int(nv[1]):] = float("-inf")
    sel0, nph0 = ref.select_topk(old_ps, budget, ctx, 16)
    stats = torch.zeros(6, dtype=torch.int64, device=gpu)
    d_sel, d_nph = sel0.to(gpu), nph0.to(gpu)
    d_cache = old_ps.to(gpu)
    cov = torch.full((B, H), -7.0, device=gpu)
    check = torch.ones(B, H, dtype=torch.bool, device=gpu)
    acc = ops.select_or_keep(new_ps.to(gpu), check, budget, ctx.to(gpu), 16, 0.9, d_sel, d_nph,
                             cov, d_cache, stats)
    assert bool(acc.all())
    assert torch.equal(d_sel.cpu(), sel0) and torch.equal(d_nph.cpu(), nph0)
    assert torch.equal(d_cache.cpu(), old_ps) and bool((cov == -7.0).all())
    assert stats.tolist() == [1, 0, 0, B * H, 0, 0]
    check[1, 0] = False
    acc = ops.select_or_keep(new_ps.to(gpu), check, budget, ctx.to(gpu), 16, 0.9, d_sel, d_nph,
                             cov, d_cache, stats)
    widx, wnph = ref.select_topk(new_ps, budget, ctx, 16)
    assert torch.equal(d_sel.cpu(), widx) and torch.equal(d_nph.cpu(), wnph)
    assert torch.equal(d_cache.cpu(), new_ps)
    wacc, wcov = ref.check_coverage(new_ps, widx, wnph, 0.9)
    _gate_ok(acc.cpu(), cov.cpu(), wacc, wcov, 0.9)
    assert stats.tolist() == [1, 1, 1, 2 * B * H - 1, 0, 0]
    sel3, nph3, cov3 = torch.empty_like(d_sel), torch.empty_like(d_nph), torch.empty_like(cov)
    acc3 = ops.select_or_keep(new_ps.to(gpu), None, budget, ctx.to(gpu), 16, 0.9, sel3, nph3,
                              cov3, None, stats, count_gate=True)
    assert torch.equal(sel3.cpu(), widx) and torch.equal(acc3, acc)
    n_acc = int(acc3.sum())
    all_acc = int(n_acc == B * H)
    assert stats.tolist() == [1 + all_acc, 2 - all_acc, 2, 2 * B * H - 1 + n_acc, 0, 0]


@pytest.mark.parametrize("W,k", [(70000, 9000), (40000, 33000), (262144, 100)])
def test_check_coverage_wide(gpu, W, k):
    """Rows and selections wider than the register kernel's (W, or the
    selection's power-of-two block, above 32768), with out-of-range ids."""
    g = torch.Generator().manual_seed(W + k)
    B, H = 2, 2
    ps = torch.randn(B, H, W, generator=g) * 2
    sel = torch.stack([torch.stack([torch.randperm(W, generator=g)[:k] for _ in range(H)])
                       for _ in range(B)]).to(torch.int32)
    sel[0, 0, :5] = torch.tensor([-1, W, W + 7, -100, 3], dtype=torch.int32)
    nph = torch.tensor([[k, k - 1], [k // 2, 0]], dtype=torch.int32)
    for tau in (0.0, 0.5, 0.9):
        acc, cov = ops.check_coverage(ps.to(gpu), sel.to(gpu), nph.to(gpu), tau)
        wacc, wcov = ref.check_coverage(ps, sel, nph, tau)
        _gate_ok(acc.cpu(), cov.cpu(), wacc, wcov, tau)


def test_select_budgeted_table_wide(gpu):
    """Per-row budgets (the static-table / adaptive path) ranked by separate
    scores, gated on the page scores, at W = 65536 and a narrower width."""
    W, B, H = 65536, 2, 3
    ps, ctx = _rows(B, H, W, 5, tail_valid=20000)
    g = torch.Generator().manual_seed(6)
    rank = ps + 0.5 * torch.randn(B, H, W, generator=g)
    rank[ps == float("-inf")] = float("-inf")
    budgets = torch.tensor([[3, 40000, 8192], [1, 25000, 65536]], dtype=torch.int32)
    width = 40000
    idx, nph, acc, cov = ops.select_budgeted(ps.to(gpu), ctx.to(gpu), 16,
                                             row_budgets=budgets.to(gpu), width=width,
                                             tau=0.9, sel_scores=rank.to(gpu))
    idx, nph = idx.cpu(), nph.cpu()
    nv = ref.n_valid_pages(ctx, 16)
    want_sel = torch.zeros(B, H, width, dtype=torch.int32)
    want_n = torch.zeros(B, H, dtype=torch.int32)
    for b in range(B):
        for h in range(H):
            k = min(int(budgets[b, h]), width)
            wi, _ = ref.select_topk(rank[b:b + 1, h:h + 1], k, ctx[b:b + 1], 16)
            n = min(k, int(nv[b]))
            want_n[b, h] = n
            want_sel[b, h, :n] = wi[0, 0, :n]
            assert torch.equal(idx[b, h, :n], wi[0, 0, :n]), (b, h)
    assert torch.equal(nph, want_n)
    wacc, wcov = ref.check_coverage(ps, want_sel, want_n, 0.9)
    _gate_ok(acc.cpu(), cov.cpu(), wacc, wcov, 0.9)


def test_topp_wide_rows_refused(gpu):
    ps = torch.randn(1, 1, 40000, device=gpu)
    ctx = torch.tensor([40000 * 16], dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="top-p"):
        ops.select_budgeted(ps, ctx, 16, top_p=0.9)


def test_compute_complement_wide(gpu):
    g = torch.Generator().manual_seed(19)
    B, H, k = 2, 2, 30000
    ctx = torch.tensor([16 * 100000, 16 * 40000 - 3], dtype=torch.int32)
    idx = torch.randint(-2, 100005, (B, H, k), generator=g).to(torch.int32)
    nph = torch.tensor([[k, 17], [0, k - 5]], dtype=torch.int32)
    acc = torch.tensor([[False, False], [True, False]])
    comp, n = ops.compute_complement(idx.to(gpu), nph.to(gpu), ctx.to(gpu), 16, acc.to(gpu))
    wcomp, wn = ref.compute_complement(idx, nph, ctx, 16, acc)
    assert torch.equal(n.cpu(), wn) and torch.equal(comp.cpu(), wcomp)


_WIDE = dict(batch=1, num_q_heads=4, num_kv_heads=1, head_dim=32, n_hot=24, hot_heads=[0])
# The fused scoring + speculative decode of the lazy check serves D = 128
# with 4, 8 or 16 KV heads.
_SPEC = dict(batch=1, num_q_heads=16, num_kv_heads=4, head_dim=128, n_hot=24)


@pytest.mark.parametrize("case", [
    # block size 16, 33000 pages, every head hot (coverage 0.41-0.58 on
    # this seed, tau 0.3): the check keeps the selection its listed
    # speculation already decoded (spec_state [1, 1])
    dict(cfg=dict(_SPEC, context_len=33000 * 16 - 5, hot_heads=[0, 1, 2, 3], hot_shift=14.0),
         kw=dict(budget_pct=0.125, coverage_threshold=0.3, lazy=True, check_interval=3),
         expect="keep"),
    # block size 8, 37500 pages (one KV head of D = 32)
    dict(cfg=dict(_WIDE, context_len=37500 * 8 - 1, block_size=8, hot_shift=12.0),
         kw=dict(budget_pct=0.125, coverage_threshold=0.9, lazy=True, check_interval=3),
         expect="recover"),
    # a draft of 35000 pages (budget 1/2 of 70000) and two KV heads of D = 64
    dict(cfg=dict(batch=1, num_q_heads=8, num_kv_heads=2, head_dim=64, n_hot=16,
                  hot_heads=[1], context_len=70000 * 16, hot_shift=12.0),
         kw=dict(budget_pct=0.5, coverage_threshold=0.9, lazy=True, check_interval=3),
         expect="recover"),
    # approximate recovery (the expanded selection of the wide kernel)
    dict(cfg=dict(_WIDE, context_len=40000 * 16, hot_shift=6.0),
         kw=dict(budget_pct=0.1, coverage_threshold=0.95, lazy=True, check_interval=2,
                 approx_recovery_pct=0.3),
         expect="approx"),
    # every gate rejects: the second check speculates a dense decode over
    # the identity partition of 33000 pages (spec_state [2, 2])
    dict(cfg=dict(_SPEC, context_len=33000 * 16 + 7, hot_heads=[0], hot_shift=4.0),
         kw=dict(budget_pct=0.125, coverage_threshold=0.999, lazy=True, check_interval=2),
         expect="dense"),
    # the Quest selector: separate ranking scores with a uniform budget
    dict(cfg=dict(_SPEC, context_len=34000 * 16 - 3, hot_heads=[1, 2], hot_shift=12.0),
         kw=dict(budget_pct=0.125, coverage_threshold=0.9, lazy=True, check_interval=3,
                 selector="quest"),
         expect="recover"),
    # ... with approximate recovery (the expansion ranks the Quest scores)
    dict(cfg=dict(_SPEC, context_len=34000 * 16, hot_heads=[0], hot_shift=6.0),
         kw=dict(budget_pct=0.1, coverage_threshold=0.95, lazy=True, check_interval=2,
                 selector="quest", approx_recovery_pct=0.3),
         expect="approx", seed=8811),
    # adaptive per-head budgets (per-row budgets of the wide kernel)
    dict(cfg=dict(_WIDE, num_kv_heads=2, num_q_heads=8, hot_heads=[1],
                  context_len=36000 * 16, hot_shift=10.0),
         kw=dict(budget_pct=0.125, coverage_threshold=0.9, lazy=True, check_interval=3,
                 adaptive_selection=True),
         expect="recover"),
    # a static budget table (per-row budgets, fixed-interval schedule)
    dict(cfg=dict(_WIDE, num_kv_heads=2, num_q_heads=8, hot_heads=[0],
                  context_len=36000 * 16, hot_shift=10.0),
         kw=dict(static_budget_table={0: [0.05, 0.2]}, coverage_threshold=0.9, lazy=False,
                 reuse_interval=2),
         expect="recover"),
], ids=["bs16_keep", "bs8", "wide_draft", "approx", "dense_spec", "quest", "quest_approx",
        "adaptive", "static_table"])
def test_backend_wide_rows_lockstep(gpu, case):
    # Seeds with no head within the fp64 margins (the lockstep harness
    # counts them; the BASELINE bar is zero).
    stats, trace, lock = _run(gpu, case["cfg"], case["kw"], steps=6,
                              seed=case.get("seed", 8800), gen_on_gpu=True)
    kinds = [t["kind"] for t in trace]
    assert kinds[0].startswith("score"), kinds
    assert "reuse" in kinds, kinds
    rejected = [not bool(t["accept"].all()) for t in trace if "accept" in t]
    plan = lock.gpu_b._step_plans.get(0)
    expect = case["expect"]
    if expect == "keep":
        assert not any(rejected) and "lazy_accept" in kinds, kinds
        assert plan.spec_state.tolist() == [1, 1]
    elif expect == "recover":
        assert any(rejected), kinds
    elif expect == "approx":
        assert "score_approx" in kinds, kinds
    else:
        assert all(rejected), kinds
        assert plan.spec_state.tolist() == [2, 2]
    print(lock.summary())
