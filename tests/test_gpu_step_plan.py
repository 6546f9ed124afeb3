"""Step plans (cvsa_step_plan_*): each step kind equals the same kernels
called one by one, bit for bit, and the backend gives identical outputs and
statistics with plans and on its per-kernel path (timing enabled)."""
import pytest
import torch

from cvsa import ops
from cvsa.ops import _lib
from cvsa.backend import CVSABackend
from cvsa.synthetic import make_paged_inputs, jitter_query
from test_gpu_backend import _Runtime

pytestmark = pytest.mark.gpu

H, G = 8, 4


def _inputs(dev, seed=11, h=H, g=G):
    inp = make_paged_inputs(batch=2, num_q_heads=h * g, num_kv_heads=h, head_dim=128,
                            context_len=[5000, 2300], hot_heads=[x for x in (0, 3, 5) if x < h],
                            n_hot=6, hot_shift=10.0, seed=seed, device=dev)
    W = inp.block_tables.shape[1]
    return inp, W, max(3, int(W * 0.25))


@pytest.mark.parametrize("tau", [0.0, 0.995])
def test_plan_kinds_equal_separate_kernels(gpu, tau):
    inp, W, budget = _inputs(gpu)
    ctx, bt = inp.context_lens, inp.block_tables
    ps0 = ops.score_pages(jitter_query(inp.q, 0.5, 3), inp.k_cache, bt, ctx, H, G, 16)
    sel0, nph0 = ops.select_topk(ps0, budget, ctx, 16)
    stats_p = torch.zeros(6, dtype=torch.int64, device=gpu)
    stats_r = torch.zeros(6, dtype=torch.int64, device=gpu)
    work_p = torch.zeros(2, dtype=torch.int64, device=gpu)
    work_r = torch.zeros(2, dtype=torch.int64, device=gpu)
    cache_p, cache_r = ps0.clone(), ps0.clone()
    plan = ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, bt, ctx, H, G, 16, budget, tau,
                        sel0.clone(), nph0.clone(), cache_p, stats_p, work_p)
    sel_r, nph_r = sel0.clone(), nph0.clone()

    # reuse step
    got = plan.run(_lib.STEP_REUSE, inp.q)
    want = ops.sparse_decode_reuse(inp.q, inp.k_cache, inp.v_cache, bt, ctx,
                                   sel_r.view(2 * H, -1), nph_r.view(2 * H),
                                   ops.next_power_of_2(budget), H, G, 16, work=work_r)
    assert torch.equal(got, want)

    # lazy check: keep (tau 0: every head passes) or reselect (tau 0.995)
    q1 = jitter_query(inp.q, 0.5, 4)
    got = plan.run(_lib.STEP_LAZY_CHECK, q1)
    ps = ops.score_pages(q1, inp.k_cache, bt, ctx, H, G, 16)
    chk, cov = ops.check_coverage(ps, sel_r, nph_r, tau)
    acc = ops.select_or_keep(ps, chk, budget, ctx, 16, tau, sel_r, nph_r, cov, cache_r, stats_r)
    want = ops.verified_decode(q1, inp.k_cache, inp.v_cache, bt, ctx, sel_r, nph_r, acc, H, G,
                               16, output_dtype=q1.dtype, work=work_r)
    assert torch.equal(got, want)
    assert torch.equal(plan.page_scores, ps)
    assert torch.equal(plan.check_accept.view(torch.bool), chk)
    assert torch.equal(plan.accept.view(torch.bool), acc)
    assert torch.equal(plan.coverage, cov)
    assert torch.equal(plan.page_indices, sel_r) and torch.equal(plan.n_per_head, nph_r)
    assert torch.equal(cache_p, cache_r)
    assert torch.equal(stats_p, stats_r) and torch.equal(work_p, work_r)
    assert bool(chk.all()) == (tau == 0.0)

    # fixed-interval scoring step (gate booked in the counters)
    q2 = jitter_query(inp.q, 0.5, 5)
    got = plan.run(_lib.STEP_SCORE, q2)
    ps = ops.score_pages(q2, inp.k_cache, bt, ctx, H, G, 16)
    acc = ops.select_or_keep(ps, None, budget, ctx, 16, tau, sel_r, nph_r, cov, None, stats_r,
                             count_gate=True)
    want = ops.verified_decode(q2, inp.k_cache, inp.v_cache, bt, ctx, sel_r, nph_r, acc, H, G,
                               16, output_dtype=q2.dtype, work=work_r)
    assert torch.equal(got, want)
    assert torch.equal(plan.accept.view(torch.bool), acc)
    assert torch.equal(plan.page_indices, sel_r) and torch.equal(plan.n_per_head, nph_r)
    assert torch.equal(stats_p, stats_r) and torch.equal(work_p, work_r)


@pytest.mark.parametrize("tau", [0.0, 0.6, 0.995])
@pytest.mark.parametrize("predict_keep", [1, 0])
@pytest.mark.parametrize("shape", [(8, 4), (2, 4)])
def test_approx_plan_equals_separate_kernels(gpu, tau, predict_keep, shape):
    """A plan with approximate recovery (approx_budget): the first selection,
    a lazy check (kept at tau 0, reselected otherwise, with either
    speculative prediction) and a fixed-interval scoring step equal the
    separate kernels bit for bit -- select, the expanded top-k of the
    rejected rows (select_topk at approx_budget), verified_decode_approx --
    and the rows the plan's selection kernel expanded are those of the
    separate top-k.  Shapes (H_kv, G): the fused check launch at H_kv 8,
    the sequential chain at H_kv 2."""
    H, G = shape
    inp, W, budget = _inputs(gpu, h=H, g=G)
    ctx, bt = inp.context_lens, inp.block_tables
    exp_budget = min(max(budget + 1, int(W * 0.5)), W)
    stats_p = torch.zeros(6, dtype=torch.int64, device=gpu)
    stats_r = torch.zeros(6, dtype=torch.int64, device=gpu)
    work_p = torch.zeros(2, dtype=torch.int64, device=gpu)
    work_r = torch.zeros(2, dtype=torch.int64, device=gpu)
    plan = ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, bt, ctx, H, G, 16, budget, tau,
                        stats=stats_p, work=work_p, own_scores_cache=True,
                        approx_budget=exp_budget)
    sel_r = torch.empty(2, H, budget, dtype=torch.int32, device=gpu)
    nph_r = torch.empty(2, H, dtype=torch.int32, device=gpu)
    cov_r = torch.empty(2, H, dtype=torch.float32, device=gpu)
    cache_r = torch.empty(2, H, W, dtype=torch.float32, device=gpu)

    def expanded_tail(q, ps, acc):
        exp, _ = ops.select_topk(ps, exp_budget, ctx, 16)
        out = ops.verified_decode_approx(q, inp.k_cache, inp.v_cache, bt, ctx, sel_r, nph_r,
                                         acc, exp, H, G, 16, output_dtype=q.dtype, work=work_r)
        rej = ~acc
        assert torch.equal(plan.approx_indices[rej], exp[rej])
        return out

    # the first selection of a lazy layer
    q0 = jitter_query(inp.q, 0.5, 3)
    got = plan.run(_lib.STEP_FRESH, q0)
    ps = ops.score_pages(q0, inp.k_cache, bt, ctx, H, G, 16)
    acc = ops.select_or_keep(ps, None, budget, ctx, 16, tau, sel_r, nph_r, cov_r, cache_r,
                             stats_r)
    assert torch.equal(got, expanded_tail(q0, ps, acc))
    assert torch.equal(plan.page_indices, sel_r) and torch.equal(plan.n_per_head, nph_r)

    # a lazy check, with the prediction given
    if plan.spec_state is not None:
        plan.spec_state[0] = predict_keep
    q1 = jitter_query(inp.q, 0.5, 4)
    got = plan.run(_lib.STEP_LAZY_CHECK, q1)
    ps = ops.score_pages(q1, inp.k_cache, bt, ctx, H, G, 16)
    chk, cov = ops.check_coverage(ps, sel_r, nph_r, tau)
    acc = ops.select_or_keep(ps, chk, budget, ctx, 16, tau, sel_r, nph_r, cov, cache_r, stats_r)
    assert torch.equal(got, expanded_tail(q1, ps, acc))
    assert torch.equal(plan.accept.view(torch.bool), acc)
    assert torch.equal(plan.page_indices, sel_r) and torch.equal(plan.n_per_head, nph_r)
    assert bool(chk.all()) == (tau == 0.0)

    # a fixed-interval scoring step
    q2 = jitter_query(inp.q, 0.5, 5)
    got = plan.run(_lib.STEP_SCORE, q2)
    ps = ops.score_pages(q2, inp.k_cache, bt, ctx, H, G, 16)
    acc = ops.select_or_keep(ps, None, budget, ctx, 16, tau, sel_r, nph_r, cov, None, stats_r,
                             count_gate=True)
    assert torch.equal(got, expanded_tail(q2, ps, acc))
    assert torch.equal(stats_p, stats_r) and torch.equal(work_p, work_r)
    if tau == 0.995:
        assert not bool(acc.all())


def _worst_pages(ps, budget, nph):
    """The `budget` lowest-scoring valid pages of every row (ascending page
    order): a selection whose coverage any top-k selection exceeds."""
    key = torch.where(torch.isfinite(ps), ps, torch.full_like(ps, float("inf")))
    worst = torch.sort(torch.argsort(key, dim=2)[:, :, :budget], dim=2).values.to(torch.int32)
    cols = torch.arange(budget, device=ps.device).view(1, 1, -1)
    return torch.where(cols < nph.unsqueeze(2), worst, torch.zeros_like(worst))


@pytest.mark.parametrize("case", ["keep", "reselect", "reselect_passes", "reject_all"])
@pytest.mark.parametrize("predict_keep", [1, 0, 2])
@pytest.mark.parametrize("shape", [(8, 4), (4, 7), (16, 2), (2, 4)])
def test_speculative_check_every_prediction(gpu, case, predict_keep, shape):
    """A lazy check whose speculative decode is predicted right or wrong
    equals the separate kernels and a plan without speculation bit for bit:
    output, selection, gate, counters, page scores.  Predictions: 1 = keep
    (listed decode of the cached selection), 2 = every head rejected (dense
    decode over the identity partition, which also scores every valid
    page), 0 = none.  "keep": tau 0, the check keeps its selection;
    "reselect": tau 0.995, it reselects and the new gate rejects;
    "reselect_passes": the cached selection is every row's worst page and
    tau lies between its coverage and the fresh selection's, so the check
    rejects every head and the new gate accepts every head; "reject_all":
    tau above 1, every gate rejects every head.  spec_state records which
    speculative decode ran and, afterwards, the check's own decision (2 when
    the new gate rejected every head).  Shapes (H_kv, G): the fused launch
    for H_kv 8, 4 and 16; H_kv 2 runs the sequential chain and leaves
    spec_state as it was."""
    H, G = shape
    inp, W, budget = _inputs(gpu, h=H, g=G)
    ctx, bt = inp.context_lens, inp.block_tables
    ps0 = ops.score_pages(jitter_query(inp.q, 0.5, 3), inp.k_cache, bt, ctx, H, G, 16)
    sel0, nph0 = ops.select_topk(ps0, budget, ctx, 16)
    q1 = jitter_query(inp.q, 0.5, 4)
    tau = {"keep": 0.0, "reselect": 0.995, "reject_all": 1.5}.get(case)
    if case == "reselect_passes":
        ps1 = ops.score_pages(q1, inp.k_cache, bt, ctx, H, G, 16)
        nph0 = torch.ones_like(nph0)
        sel0 = _worst_pages(ps1, budget, nph0)
        cov_old = ops.check_coverage(ps1, sel0, nph0, 0.5)[1]
        cov_new = ops.check_coverage(ps1, *ops.select_topk(ps1, budget, ctx, 16), 0.5)[1]
        assert float(cov_old.max()) < float(cov_new.min())
        tau = 0.5 * (float(cov_old.max()) + float(cov_new.min()))
    plans, bufs = [], []
    for speculate in (True, False):
        b = dict(stats=torch.zeros(6, dtype=torch.int64, device=gpu),
                 work=torch.zeros(2, dtype=torch.int64, device=gpu), cache=ps0.clone())
        plans.append(ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, bt, ctx, H, G, 16, budget,
                                  tau, sel0.clone(), nph0.clone(), b["cache"], b["stats"],
                                  b["work"], speculate=speculate))
        bufs.append(b)
    assert plans[1].spec_state is None
    plans[0].spec_state[0] = predict_keep
    got = plans[0].run(_lib.STEP_LAZY_CHECK, q1)
    plain = plans[1].run(_lib.STEP_LAZY_CHECK, q1)
    stats_r = torch.zeros(6, dtype=torch.int64, device=gpu)
    work_r = torch.zeros(2, dtype=torch.int64, device=gpu)
    sel_r, nph_r, cache_r = sel0.clone(), nph0.clone(), ps0.clone()
    ps = ops.score_pages(q1, inp.k_cache, bt, ctx, H, G, 16)
    chk, cov = ops.check_coverage(ps, sel_r, nph_r, tau)
    acc = ops.select_or_keep(ps, chk, budget, ctx, 16, tau, sel_r, nph_r, cov, cache_r, stats_r)
    want = ops.verified_decode(q1, inp.k_cache, inp.v_cache, bt, ctx, sel_r, nph_r, acc, H, G,
                               16, output_dtype=q1.dtype, work=work_r)
    for plan, b, out in ((plans[0], bufs[0], got), (plans[1], bufs[1], plain)):
        assert torch.equal(out, want)
        assert torch.equal(plan.page_scores, ps)  # also where the decode part scored
        assert torch.equal(plan.accept.view(torch.bool), acc)
        assert torch.equal(plan.page_indices, sel_r) and torch.equal(plan.n_per_head, nph_r)
        assert torch.equal(b["cache"], cache_r)
        assert torch.equal(b["stats"], stats_r) and torch.equal(b["work"], work_r)
    keep = bool(chk.all())
    assert keep == (case == "keep")
    assert bool(acc.all()) == (case not in ("reselect", "reject_all"))
    assert case not in ("reselect_passes", "reject_all") or not bool(chk.any())
    assert case != "reject_all" or not bool(acc.any())
    fused = H in (4, 8, 16)
    decision = 1 if keep else (2 if not bool(acc.any()) else 0)
    assert plans[0].spec_state.tolist() == ([decision, predict_keep] if fused
                                            else [predict_keep, 0])
    # the next check speculates on this one's decision: a reuse step between
    # them reads the (possibly reselected) selection and still matches
    got = plans[0].run(_lib.STEP_REUSE, q1)
    want = ops.sparse_decode_reuse(q1, inp.k_cache, inp.v_cache, bt, ctx,
                                   sel_r.view(2 * H, -1), nph_r.view(2 * H),
                                   ops.next_power_of_2(budget), H, G, 16)
    assert torch.equal(got, want)


@pytest.mark.parametrize("tau", [0.0, 0.995])
def test_fresh_kind_equals_separate_kernels(gpu, tau):
    """A plan that owns its selection and scores cache: the first selection
    of a lazy layer (score, fresh select booked as a scoring step, verified
    decode), twice in a row in the same buffers."""
    inp, W, budget = _inputs(gpu)
    ctx, bt = inp.context_lens, inp.block_tables
    stats_p = torch.zeros(6, dtype=torch.int64, device=gpu)
    stats_r = torch.zeros(6, dtype=torch.int64, device=gpu)
    work_p = torch.zeros(2, dtype=torch.int64, device=gpu)
    work_r = torch.zeros(2, dtype=torch.int64, device=gpu)
    plan = ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, bt, ctx, H, G, 16, budget, tau,
                        stats=stats_p, work=work_p, own_scores_cache=True)
    assert plan.owns_selection and plan.scores_cache is not None
    for seed in (6, 7):
        q1 = jitter_query(inp.q, 0.5, seed)
        got = plan.run(_lib.STEP_FRESH, q1)
        ps = ops.score_pages(q1, inp.k_cache, bt, ctx, H, G, 16)
        sel_r = torch.empty(2, H, budget, dtype=torch.int32, device=gpu)
        nph_r = torch.empty(2, H, dtype=torch.int32, device=gpu)
        cov = torch.empty(2, H, dtype=torch.float32, device=gpu)
        cache_r = torch.empty_like(ps)
        acc = ops.select_or_keep(ps, None, budget, ctx, 16, tau, sel_r, nph_r, cov, cache_r,
                                 stats_r)
        want = ops.verified_decode(q1, inp.k_cache, inp.v_cache, bt, ctx, sel_r, nph_r, acc,
                                   H, G, 16, output_dtype=q1.dtype, work=work_r)
        assert torch.equal(got, want), seed
        assert torch.equal(plan.page_scores, ps)
        assert torch.equal(plan.scores_cache, cache_r)
        assert torch.equal(plan.accept.view(torch.bool), acc)
        assert torch.equal(plan.coverage, cov)
        assert torch.equal(plan.page_indices, sel_r) and torch.equal(plan.n_per_head, nph_r)
        assert torch.equal(stats_p, stats_r) and torch.equal(work_p, work_r)
    # each call booked as one rejection and one scoring step
    assert stats_p[1].item() == 2 and stats_p[2].item() == 2


@pytest.mark.parametrize("selector", [_lib.SELECT_QUEST, _lib.SELECT_QUEST_LN])
@pytest.mark.parametrize("tau", [0.0, 0.995])
def test_plan_quest_kinds_equal_separate_kernels(gpu, selector, tau):
    """Quest-ranked plans (exact gate, or the light normalizer's Quest gate):
    first selection, lazy check and fixed-interval step equal the separate
    kernels, metadata included."""
    inp, W, budget = _inputs(gpu)
    ctx, bt = inp.context_lens, inp.block_tables
    ln = selector == _lib.SELECT_QUEST_LN
    qm_p, qm_r = ops.QuestPageMeta(inp.k_cache), ops.QuestPageMeta(inp.k_cache)
    stats_p = torch.zeros(6, dtype=torch.int64, device=gpu)
    stats_r = torch.zeros(6, dtype=torch.int64, device=gpu)
    work_p = torch.zeros(2, dtype=torch.int64, device=gpu)
    work_r = torch.zeros(2, dtype=torch.int64, device=gpu)
    plan = ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, bt, ctx, H, G, 16, budget, tau,
                        stats=stats_p, work=work_p, own_scores_cache=True, selector=selector,
                        quest=qm_p)
    assert (plan.sel_scores is None) == ln

    def gate(q):
        return qm_r.scores(q, bt, ctx, H, G, 16) if ln else ops.score_pages(q, inp.k_cache, bt,
                                                                            ctx, H, G, 16)

    sel_r = torch.empty(2, H, budget, dtype=torch.int32, device=gpu)
    nph_r = torch.empty(2, H, dtype=torch.int32, device=gpu)
    cov_r = torch.empty(2, H, dtype=torch.float32, device=gpu)
    cache_r = torch.empty(2, H, W, dtype=torch.float32, device=gpu)
    rank_r = None if ln else torch.empty(2, H, W, dtype=torch.float32, device=gpu)

    def rank(q, check=None):
        return None if ln else qm_r.scores(q, bt, ctx, H, G, 16, check, rank_r)

    def compare(got, want, ps, acc):
        assert torch.equal(got, want)
        assert torch.equal(plan.page_scores, ps)
        assert torch.equal(plan.accept.view(torch.bool), acc)
        assert torch.equal(plan.page_indices, sel_r) and torch.equal(plan.n_per_head, nph_r)
        assert torch.equal(stats_p, stats_r) and torch.equal(work_p, work_r)
        used = qm_r.ntok > 0   # blocks no row lists hold no metadata
        assert torch.equal(qm_p.ntok, qm_r.ntok)
        assert torch.equal(qm_p.meta[used], qm_r.meta[used])
        if not ln:
            assert torch.equal(plan.sel_scores, rank_r)

    # first selection of a lazy layer
    q1 = jitter_query(inp.q, 0.5, 6)
    got = plan.run(_lib.STEP_FRESH, q1)
    ps = gate(q1)
    acc = ops.select_or_keep(ps, None, budget, ctx, 16, tau, sel_r, nph_r, cov_r, cache_r,
                             stats_r, sel_scores=rank(q1))
    want = ops.verified_decode(q1, inp.k_cache, inp.v_cache, bt, ctx, sel_r, nph_r, acc, H, G,
                               16, output_dtype=q1.dtype, work=work_r)
    compare(got, want, ps, acc)
    assert torch.equal(plan.scores_cache, cache_r)

    # lazy check (the ranking scores are computed only if a head failed)
    q2 = jitter_query(inp.q, 0.5, 7)
    got = plan.run(_lib.STEP_LAZY_CHECK, q2)
    ps = gate(q2)
    chk, cov = ops.check_coverage(ps, sel_r, nph_r, tau)
    acc = ops.select_or_keep(ps, chk, budget, ctx, 16, tau, sel_r, nph_r, cov, cache_r,
                             stats_r, sel_scores=rank(q2, chk))
    want = ops.verified_decode(q2, inp.k_cache, inp.v_cache, bt, ctx, sel_r, nph_r, acc, H, G,
                               16, output_dtype=q2.dtype, work=work_r)
    compare(got, want, ps, acc)
    assert torch.equal(plan.check_accept.view(torch.bool), chk)
    assert torch.equal(plan.scores_cache, cache_r)
    assert bool(chk.all()) == (tau == 0.0)

    # fixed-interval scoring step
    q3 = jitter_query(inp.q, 0.5, 8)
    got = plan.run(_lib.STEP_SCORE, q3)
    ps = gate(q3)
    acc = ops.select_or_keep(ps, None, budget, ctx, 16, tau, sel_r, nph_r, cov, None, stats_r,
                             count_gate=True, sel_scores=rank(q3))
    want = ops.verified_decode(q3, inp.k_cache, inp.v_cache, bt, ctx, sel_r, nph_r, acc, H, G,
                               16, output_dtype=q3.dtype, work=work_r)
    compare(got, want, ps, acc)


def test_plan_rejects_buffers_it_cannot_use(gpu):
    inp, W, budget = _inputs(gpu)
    args = (inp.q, inp.k_cache, inp.v_cache, inp.block_tables, inp.context_lens, H, G, 16)
    with pytest.raises(ValueError):
        ops.StepPlan(*args, budget, 0.9, torch.zeros(2, H, budget + 1, dtype=torch.int32,
                                                     device=gpu),
                     torch.zeros(2, H, dtype=torch.int32, device=gpu))
    with pytest.raises(ValueError):  # int64 block tables would need a converted copy
        ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, inp.block_tables.long(), inp.context_lens,
                     H, G, 16, budget, 0.9)
    with pytest.raises(ValueError):  # budget outside [1, W]
        ops.StepPlan(*args, W + 1, 0.9)
    with pytest.raises(ValueError):  # a Quest selector without metadata
        ops.StepPlan(*args, budget, 0.9, selector=_lib.SELECT_QUEST)
    with pytest.raises(ValueError):  # metadata of another cache
        ops.StepPlan(*args, budget, 0.9, selector=_lib.SELECT_QUEST_LN,
                     quest=ops.QuestPageMeta(inp.k_cache.clone()))


@pytest.mark.parametrize("kw", [
    dict(lazy=True, check_interval=5),
    dict(lazy=True, check_interval=2),
    dict(lazy=False, reuse_interval=1),
    dict(lazy=False, reuse_interval=3),
    dict(lazy=True, check_interval=2, selector="quest"),
    dict(lazy=True, check_interval=3, selector="quest", light_normalizer=True),
    dict(lazy=False, reuse_interval=2, selector="quest"),
    dict(lazy=False, reuse_interval=1, selector="quest", light_normalizer=True),
])
def test_backend_plans_equal_kernel_path(gpu, kw):
    """Same decode loop (appends included) through step plans and through
    the per-kernel path: identical outputs and counters."""
    inp, W, budget = _inputs(gpu, seed=21)
    steps = 10
    bt = torch.zeros(2, W + 2, dtype=torch.int32)
    bt[:, :W] = inp.block_tables.cpu()
    inp.block_tables = bt
    for name in ("q", "k_cache", "v_cache", "context_lens"):
        setattr(inp, name, getattr(inp, name).cpu())
    rt_a, rt_b = _Runtime(inp, gpu, 16), _Runtime(inp, gpu, 16)
    mk = dict(num_kv_heads=H, num_q_heads=H * G, head_dim=128, block_size=16,
              budget_pct=0.25, coverage_threshold=0.9, **kw)
    plan_b, kern_b = CVSABackend(**mk), CVSABackend(**mk)
    kern_b.enable_timing(True)
    g = torch.Generator().manual_seed(5)
    for step in range(steps):
        if step == 6:
            # plans that own their selection outlive a reset
            kept = plan_b._step_plans.get(0)
            plan_b.reset()
            kern_b.reset()
        q = jitter_query(inp.q, 0.3, 700 + step).to(gpu)
        a = plan_b(q, rt_a.cache.k_cache, rt_a.cache.v_cache, rt_a.mgr.block_tables,
                   rt_a.mgr.context_lens, 0)
        b = kern_b(q, rt_b.cache.k_cache, rt_b.cache.v_cache, rt_b.mgr.block_tables,
                   rt_b.mgr.context_lens, 0)
        assert torch.equal(a, b), step
        ma, mb = plan_b._last_accept_mask.get(0), kern_b._last_accept_mask.get(0)
        assert (ma is None) == (mb is None) and (ma is None or torch.equal(ma, mb)), step
        plan_b.step_done(0, 1)
        kern_b.step_done(0, 1)
        kn = torch.randn(2, H, 128, generator=g).to(torch.bfloat16).to(gpu)
        vn = torch.randn(2, H, 128, generator=g).to(torch.bfloat16).to(gpu)
        rt_a.mgr.append_tokens_kv(kn, vn)
        rt_b.mgr.append_tokens_kv(kn, vn)
    assert 0 in plan_b._step_plans and not kern_b._step_plans
    assert kept is not None and plan_b._step_plans[0] is kept
    sa, sb = plan_b.get_stats(), kern_b.get_stats()
    for k in sa:
        assert sa[k] == sb[k], (k, sa[k], sb[k])


@pytest.mark.parametrize("seed", range(8))
def test_random_shapes_plan_equals_separate_kernels(gpu, seed):
    """Random B, H_kv, G, ragged contexts, budget and tau: a plan (with and
    without speculation) runs a first selection, two lazy checks, a reuse
    step and a fixed-interval scoring step; every output, selection, gate and
    counter equals the same kernels called one by one, bit for bit."""
    _plan_equals_separate_kernels(gpu, seed, 128)


@pytest.mark.parametrize("D", [32, 64, 256])
@pytest.mark.parametrize("seed", range(3))
def test_random_shapes_plan_head_dims(gpu, seed, D):
    """The same at head dimensions 32, 64 and 256 (no speculation there: the
    fused lazy-check launch is compiled for D = 128, so the plan runs the
    plain chain whether or not it was asked to speculate)."""
    _plan_equals_separate_kernels(gpu, seed, D)


@pytest.mark.parametrize("BS", [8, 32, 64, 128])
@pytest.mark.parametrize("seed", range(3))
def test_random_shapes_plan_block_sizes(gpu, seed, BS):
    """The same at block sizes 8, 32, 64 and 128 (speculation included at D = 128,
    except at 8-token pages, where the plan runs the plain chain)."""
    _plan_equals_separate_kernels(gpu, seed, [128, 64, 128][seed], BS)


@pytest.mark.parametrize("seed", range(4))
def test_random_shapes_plan_wide_groups(gpu, seed):
    """The same with 9..16 query heads per KV head."""
    _plan_equals_separate_kernels(gpu, seed, 128, [16, 32, 16, 64][seed], (9, 16))


@pytest.mark.parametrize("seed", range(3))
def test_random_shapes_plan_large_groups(gpu, seed):
    """The same with 17..40 query heads per KV head (no speculation: the
    decode runs as one launch per 16 query heads)."""
    _plan_equals_separate_kernels(gpu, 10 + seed, 128, [16, 32, 16][seed], (17, 40))


def _plan_equals_separate_kernels(gpu, seed, D, BS=16, G_range=(1, 8)):
    g = torch.Generator().manual_seed(100 + seed)
    rnd = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))  # noqa: E731
    H = [1, 2, 4, 8, 16][rnd(0, 4)]
    G = rnd(*G_range)
    B = rnd(1, 3)
    ctx = [rnd(40, 6000) for _ in range(B)]
    inp = make_paged_inputs(B, H * G, H, D, ctx, block_size=BS, seed=seed, device=gpu,
                            max_pages=max((c - 1) // BS + 1 for c in ctx) + rnd(0, 3),
                            hot_heads=list(range(0, H, 2)), n_hot=4, hot_shift=8.0)
    W = inp.block_tables.shape[1]
    budget = max(3, int(W * [0.125, 0.25, 0.5][rnd(0, 2)]))
    tau = [0.0, 0.5, 0.9, 0.995][rnd(0, 3)]
    ctx_t, bt = inp.context_lens, inp.block_tables
    runs = []
    for speculate in (True, False):
        stats = torch.zeros(6, dtype=torch.int64, device=gpu)
        work = torch.zeros(2, dtype=torch.int64, device=gpu)
        plan = ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, bt, ctx_t, H, G, BS, budget, tau,
                            stats=stats, work=work, own_scores_cache=True, speculate=speculate)
        outs = []
        for step, kind in enumerate((_lib.STEP_FRESH, _lib.STEP_LAZY_CHECK, _lib.STEP_LAZY_CHECK,
                                     _lib.STEP_REUSE, _lib.STEP_SCORE)):
            q = jitter_query(inp.q, 0.4, 300 + 10 * seed + step)
            outs.append(plan.run(kind, q).clone())
        runs.append((plan, stats, work, outs))
    # the separate kernels
    stats = torch.zeros(6, dtype=torch.int64, device=gpu)
    work = torch.zeros(2, dtype=torch.int64, device=gpu)
    sel = torch.empty(B, H, budget, dtype=torch.int32, device=gpu)
    nph = torch.empty(B, H, dtype=torch.int32, device=gpu)
    cov = torch.empty(B, H, dtype=torch.float32, device=gpu)
    cache = torch.empty(B, H, W, dtype=torch.float32, device=gpu)
    want = []
    for step, kind in enumerate(("fresh", "check", "check", "reuse", "score")):
        q = jitter_query(inp.q, 0.4, 300 + 10 * seed + step)
        if kind == "reuse":
            want.append(ops.sparse_decode_reuse(q, inp.k_cache, inp.v_cache, bt, ctx_t,
                                                sel.view(B * H, -1), nph.view(B * H),
                                                ops.next_power_of_2(budget), H, G, BS,
                                                work=work))
            continue
        ps = ops.score_pages(q, inp.k_cache, bt, ctx_t, H, G, BS)
        if kind == "fresh":
            acc = ops.select_or_keep(ps, None, budget, ctx_t, BS, tau, sel, nph, cov, cache,
                                     stats)
        elif kind == "check":
            chk, cov = ops.check_coverage(ps, sel, nph, tau)
            acc = ops.select_or_keep(ps, chk, budget, ctx_t, BS, tau, sel, nph, cov, cache,
                                     stats)
        else:
            acc = ops.select_or_keep(ps, None, budget, ctx_t, BS, tau, sel, nph, cov, None,
                                     stats, count_gate=True)
        want.append(ops.verified_decode(q, inp.k_cache, inp.v_cache, bt, ctx_t, sel, nph, acc,
                                        H, G, BS, output_dtype=q.dtype, work=work))
    for plan, p_stats, p_work, outs in runs:
        for step, (got, ref_out) in enumerate(zip(outs, want)):
            assert torch.equal(got, ref_out), (seed, step, plan.spec_state is not None)
        assert torch.equal(plan.page_indices, sel) and torch.equal(plan.n_per_head, nph)
        assert torch.equal(p_stats, stats) and torch.equal(p_work, work), seed


def _map_of(sel, nph, W, stride):
    """The selection map a plan keeps: byte p of row r set for the row's
    first n_per_head entries."""
    rows = sel.reshape(-1, sel.shape[-1]).long().cpu()
    n = nph.reshape(-1).cpu()
    m = torch.zeros(rows.shape[0], stride, dtype=torch.uint8)
    for r in range(rows.shape[0]):
        m[r, rows[r, :int(n[r])]] = 1
    return m


@pytest.mark.parametrize("shape", [(8, 4), (4, 7), (16, 16), (8, 1)])
def test_selection_map_and_scores_over_a_schedule(gpu, shape):
    """A plan's selection map follows every selection it makes (fresh,
    reselect, keep) and an adopted or externally written one
    (selection_changed); the page scores of every lazy check, part of them
    computed by the speculative decode from the keys it walks, equal
    cvsa_score_pages bit for bit, whatever the prediction.  Two plans share
    the selection buffers (tau 0: keeps; tau 0.999: reselects), each told
    when the other may have rewritten the selection."""
    H, G = shape
    inp, W, budget = _inputs(gpu, h=H, g=G)
    ctx, bt = inp.context_lens, inp.block_tables
    stats = torch.zeros(6, dtype=torch.int64, device=gpu)
    work = torch.zeros(2, dtype=torch.int64, device=gpu)
    fresh = ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, bt, ctx, H, G, 16, budget, 0.9,
                         stats=stats, work=work, own_scores_cache=True)
    stride = fresh.sel_map.shape[1]
    assert stride % 16 == 0 and stride >= W
    fresh.run(_lib.STEP_FRESH, jitter_query(inp.q, 0.5, 10))
    torch.cuda.synchronize()
    assert torch.equal(fresh.sel_map.cpu(),
                       _map_of(fresh.page_indices, fresh.n_per_head, W, stride))
    plans = {tau: ops.StepPlan(inp.q, inp.k_cache, inp.v_cache, bt, ctx, H, G, 16, budget, tau,
                               fresh.page_indices, fresh.n_per_head, fresh.scores_cache, stats,
                               work) for tau in (0.0, 0.999)}
    schedule = [(11, 1, 0.0), (12, 0, 0.0), (13, 1, 0.999), (14, 1, 0.0), (15, 0, 0.999),
                (16, 1, 0.0), (17, 1, 0.0), (18, 0, 0.999), (19, 0, 0.0)]
    for step, (seed, predict, tau) in enumerate(schedule):
        q = jitter_query(inp.q, 0.5, seed)
        if step == 4:
            # a selection written outside the plans: the worst pages
            ps_prev = ops.score_pages(q, inp.k_cache, bt, ctx, H, G, 16)
            nph = fresh.n_per_head
            nph.copy_(torch.minimum(nph, torch.full_like(nph, budget // 2)))
            fresh.page_indices.copy_(_worst_pages(ps_prev, budget, nph))
            for p in plans.values():
                p.selection_changed()
        p = plans[tau]
        p.spec_state[0] = predict
        p.run(_lib.STEP_LAZY_CHECK, q)
        for other in plans.values():
            if other is not p:
                other.selection_changed()
        ps = ops.score_pages(q, inp.k_cache, bt, ctx, H, G, 16)
        assert torch.equal(p.page_scores, ps), (step, predict, tau)
        torch.cuda.synchronize()
        assert torch.equal(p.sel_map.cpu(), _map_of(p.page_indices, p.n_per_head, W, stride)), \
            (step, predict, tau)
