"""Multi-step decode parity of the GPU CVSABackend against the oracle state machine.

Both backends run the same decode loop (query jittered per step, one token
appended per sequence per step through the paged-KV runtime) on identical
inputs.  Every selection and every coverage gate is compared where the
oracle makes it (``_Lockstep``, hooked into the oracle backend):

* exactly, on every head, against the oracle's selector and gate applied to
  the GPU's own fp32 ranking / gate scores (the integer work of the kernels:
  top-k, budgets, accept bits); the only exception is a gate whose coverage
  lies within 1e-6 of tau (or a top-p row whose cumulative mass lies within
  1e-6 of top_p), where fp32 and fp64 arithmetic on the same scores may
  disagree -- those are counted ("own-margin heads");
* the GPU's fp32 scores against the oracle's fp64 scores, 1e-4 relative;
* the oracle's own fp64 selection and gate against the GPU's: equal on every
  head except where the fp64 answer is decided within the realised fp32
  score error (k-th / (k+1)-th gap <= 2 x the row's largest score error, or
  |coverage - tau| <= 1e-5); those "fp64-margin heads" are counted, checked
  to be a top-k set of the oracle's scores within that error, and the oracle
  then takes the GPU's answer so that both keep one state.
Per call the outputs agree to 2e-2 max-abs, the cached selections and accept
masks are identical, and at the end get_stats() is identical.  Each test
asserts its margin-head counts (zero for the seeds chosen here) and reports
them in the message.  The BASELINE configurations run at full size (128K
context, B=32, G=8 ...), including the literal BASELINE recipes (+3 sigma
hot pages, +2 sigma sink) and cfg4's tau sweep.
"""
import pytest
import torch

from oracle import cvsa_oracle as ref
from oracle.backend_oracle import OracleCVSABackend
from cvsa.backend import CVSABackend
from cvsa.runtime.kv_cache import PagedKVCache, SequenceKVManager
from cvsa.synthetic import make_paged_inputs, jitter_query

pytestmark = pytest.mark.gpu

OUT_ATOL = 2e-2
SCORE_RTOL = 1e-4       # GPU fp32 scores vs oracle fp64 scores
COV_ATOL = 1e-5         # coverage from GPU scores vs from oracle scores
OWN_MARGIN = 1e-6       # fp32 vs fp64 gate / top-p decision on the same scores


class _Runtime:
    """A GPU cache + manager and a CPU oracle copy of the same state."""

    def __init__(self, inp, dev, extra_tokens):
        B = inp.q.shape[0]
        nb = inp.k_cache.shape[0]
        bs, H, D = inp.k_cache.shape[1], inp.k_cache.shape[2], inp.k_cache.shape[3]
        W = inp.block_tables.shape[1]
        self.bs = bs
        self.cache = PagedKVCache(nb, bs, H, D, device=str(dev))
        self.cache.k_cache.copy_(inp.k_cache)
        self.cache.v_cache.copy_(inp.v_cache)
        self.cache._next_free = inp.used_blocks
        self.mgr = SequenceKVManager(self.cache, B, W * bs)
        self.mgr.block_tables.copy_(inp.block_tables)
        self.mgr.context_lens.copy_(inp.context_lens)
        pages = [-(-int(c) // bs) for c in inp.context_lens.tolist()]
        self.mgr._pages_allocated = list(pages)
        self.mgr.sync_host_state()
        self.K = inp.k_cache.clone()
        self.V = inp.v_cache.clone()
        self.bt = inp.block_tables.clone()
        self.ctx = inp.context_lens.clone()
        self.alloc = torch.tensor(pages, dtype=torch.int32)
        self.nf = inp.used_blocks

    def append(self, k, v, dev):
        self.mgr.append_tokens_kv(k.to(dev), v.to(dev))
        for b in range(k.shape[0]):
            self.nf = ref.append_token_kv(self.K, self.V, self.bt, self.ctx, self.alloc, self.nf,
                                          b, k[b], v[b], self.bs)


def _cpu(t):
    return None if t is None else t.detach().cpu().clone()


def _topp_boundary(scores, top_p, tol):
    """Rows whose top-p budget is decided within `tol` of top_p: the fp64
    cumulative softmax mass at the crossing (or the entry before it) lies
    within tol of fp32(top_p)."""
    need, order = ref.topp_need(scores, top_p)
    cum = torch.cumsum(torch.softmax(scores.double(), -1).gather(-1, order), -1)
    p32 = float(torch.tensor(top_p, dtype=torch.float32))
    B, H, P = scores.shape
    near = torch.zeros(B, H, dtype=torch.bool)
    for b in range(B):
        for h in range(H):
            k = int(need[b, h])
            for j in (k - 2, k - 1):
                if 0 <= j < P and abs(float(cum[b, h, j]) - p32) < tol:
                    near[b, h] = True
    return near


class _Lockstep:
    """The comparisons of the module docstring, run from the oracle's hooks.

    Call ``before_gpu`` before and ``after_gpu`` after each GPU backend call,
    then call the oracle backend (which invokes ``on_select`` / ``on_gate``)."""

    def __init__(self, gpu_b, ora_b, kw, ctx_cpu):
        self.gpu_b = gpu_b
        self.kw = kw
        self.tau = float(kw.get("coverage_threshold", 0.9))
        self.bs = gpu_b.block_size
        self.ctx = ctx_cpu                   # the oracle runtime's context lengths (live)
        self.own_margin = 0                  # fp32-vs-fp64 on the GPU's own scores
        self.margin_sel = 0                  # fp64 selection decided within the score error
        self.margin_gate = 0                 # fp64 accept decided within the coverage error
        self.heads_checked = 0
        self.g = {}
        self.expanded_checked = 0
        ora_b.on_select = self.on_select
        ora_b.on_gate = self.on_gate
        ora_b.on_expand = self.on_expand

    # ------------------------------------------------------------ snapshots
    def before_gpu(self, layer=0):
        sel = self.gpu_b._cached_selection.get(layer)
        self.prev_sel = None if sel is None else (_cpu(sel[0]), _cpu(sel[1]))
        self.prev_scoring = self.gpu_b._counters()[2]

    def after_gpu(self, layer=0):
        b = self.gpu_b
        g = {"new": b._counters()[2] > self.prev_scoring}
        chk = b._last_check.get(layer)
        g["check"] = None if chk is None else (_cpu(chk[0]), _cpu(chk[1]))
        acc = b._last_accept_mask.get(layer)
        g["accept"] = _cpu(acc)
        if g["new"]:
            pi, nph = b._cached_selection[layer]
            g["idx"], g["nph"] = _cpu(pi), _cpu(nph)
            g["gate"] = _cpu(b._cached_page_scores[layer])
            rank = b._last_rank_scores.get(layer)
            g["ranked"] = g["gate"] if rank is None else _cpu(rank)
            # Approximate recovery: the expanded selection the tracing
            # attribute reports, and the rows the step plan's selection
            # kernel wrote for the rejected heads (when a plan ran the step).
            exp = b._last_expanded_selection.get(layer) if b.approx_recovery_pct else None
            g["exp"] = None if exp is None else (_cpu(exp[0]), _cpu(exp[1]))
            plan = b._step_plans.get(layer)
            g["plan_exp"] = None
            if (plan is not None and plan.approx_budget > 0
                    and b._cached_selection[layer][0] is plan.page_indices):
                g["plan_exp"] = _cpu(plan.approx_indices)
        self.g = g

    # ------------------------------------------------------------ helpers
    def _select(self, scores, layer):
        kw = self.kw
        if kw.get("top_p") is not None:
            return ref.topp_select(scores, kw["top_p"], self.ctx, self.bs)
        if kw.get("static_budget_table") is not None:
            return ref.static_select(scores, torch.as_tensor(kw["static_budget_table"][layer]),
                                     self.ctx, self.bs)
        W = scores.shape[-1]
        budget = max(3, int(W * kw.get("budget_pct", 0.10)))
        if kw.get("adaptive_selection"):
            return ref.adaptive_select(scores, budget, self.ctx, self.bs,
                                       kw.get("adaptive_floor_ratio", 0.5))
        return ref.select_topk(scores, budget, self.ctx, self.bs)

    @staticmethod
    def _score_error(gpu, ora, what):
        """fp32 vs fp64 scores: same -inf pattern, 1e-4 relative; returns the
        largest absolute error of each row [B, H]."""
        fin = torch.isfinite(ora)
        assert torch.equal(torch.isfinite(gpu), fin), what
        zero = torch.zeros((), dtype=torch.float64)
        diff = torch.where(fin, (gpu.double() - ora.double()).abs(), zero)
        rel = diff / ora.double().abs().clamp(min=1.0)
        assert float(rel.max()) < SCORE_RTOL, (what, float(rel.max()))
        return diff.amax(dim=-1)

    # ------------------------------------------------------------ hooks
    def on_select(self, layer, ranked_o, idx_o, nph_o):
        g = self.g
        assert g.get("new"), "the oracle made a new selection where the GPU kept its own"
        R, gi, gn = g["ranked"], g["idx"], g["nph"]
        err = self._score_error(R, ranked_o, "ranking scores")
        # Exact on the GPU's own scores.
        ri, rn = self._select(R, layer)
        own = torch.zeros(gn.shape, dtype=torch.bool)
        if self.kw.get("top_p") is not None:
            own = _topp_boundary(R, self.kw["top_p"], OWN_MARGIN)
        B, H = gn.shape
        for b in range(B):
            for h in range(H):
                if own[b, h]:
                    continue
                n = int(gn[b, h])
                assert n == int(rn[b, h]), ("n_per_head", b, h, n, int(rn[b, h]))
                assert torch.equal(gi[b, h, :n], ri[b, h, :n]), ("selection", b, h)
        self.own_margin += int(own.sum())
        self.heads_checked += B * H
        # The oracle's fp64 selection: equal outside the score-error margin.
        S = ranked_o.double()
        for b in range(B):
            for h in range(H):
                n, no = int(gn[b, h]), int(nph_o[b, h])
                same = n == no and torch.equal(gi[b, h, :n], idx_o[b, h, :no])
                if same:
                    continue
                self.margin_sel += 1
                tol = 2.0 * float(err[b, h]) + 1e-9
                assert abs(n - no) <= 1, ("budget", b, h, n, no)
                sel = gi[b, h, :n].long()
                assert torch.all(sel[1:] > sel[:-1]), (b, h)
                srt = torch.sort(S[b, h], descending=True).values
                kth = float(srt[n - 1])
                assert float(S[b, h, sel].min()) >= kth - tol, ("near-tie set", b, h, tol)
                rest = S[b, h].clone()
                rest[sel] = float("-inf")
                assert float(rest.max()) <= kth + tol, ("near-tie set", b, h, tol)
        return gi, gn

    def on_expand(self, layer, ranked_o, exp_o, exp_budget):
        """The expanded selection of approximate recovery: the GPU's (the
        tracing attribute's rows, and the step plan's rows for rejected
        heads) exactly equals the oracle's selector on the GPU's own ranking
        scores, and the oracle's fp64 choice outside the score-error margin."""
        g = self.g
        assert g.get("exp") is not None, "the oracle expanded where the GPU did not"
        gi, gn = g["exp"]
        R = g["ranked"]
        err = self._score_error(R, ranked_o, "ranking scores (expansion)")
        ri, rn = ref.select_topk(R, exp_budget, self.ctx, self.bs)
        assert gi.shape[-1] == exp_budget and torch.equal(gn, rn), ("expanded counts", gn, rn)
        B, H = gn.shape
        rejected = ~g["accept"]
        pe = g["plan_exp"]
        for b in range(B):
            for h in range(H):
                n = int(gn[b, h])
                assert torch.equal(gi[b, h, :n], ri[b, h, :n]), ("expanded", b, h)
                if pe is not None and bool(rejected[b, h]):
                    assert torch.equal(pe[b, h, :n], ri[b, h, :n]), ("plan expanded", b, h)
                same = torch.equal(gi[b, h, :n], exp_o[b, h, :n])
                if not same:
                    self.margin_sel += 1
                    tol = 2.0 * float(err[b, h]) + 1e-9
                    S = ranked_o.double()
                    kth = float(torch.sort(S[b, h], descending=True).values[n - 1])
                    sel = gi[b, h, :n].long()
                    assert float(S[b, h, sel].min()) >= kth - tol, ("near-tie set", b, h)
        self.expanded_checked += int(rejected.sum())
        return gi

    def on_gate(self, layer, where, scores_o, idx, nph, accept_o, cov_o):
        g = self.g
        rr = self.kw.get("random_reject_prob")
        if where == "new" and rr is not None:
            # The new selection's gate is overridden on both sides (rr in
            # {0, 1}: every head accepted or every head rejected); its
            # coverage is still checked.
            assert rr in (0.0, 1.0), rr
            assert g.get("new")
            assert bool((g["accept"] == (rr == 0.0)).all()), g["accept"]
            acc_r, cov_r = ref.check_coverage(g["gate"], idx, nph, self.tau)
            assert float((cov_r - cov_o).abs().max()) < COV_ATOL, (where, cov_r, cov_o)
            self.heads_checked += acc_r.numel()
            return g["accept"].clone()
        if where == "new":
            assert g.get("new"), "the oracle gated a new selection the GPU did not make"
            G, A = g["gate"], g["accept"]
        else:
            assert g.get("check") is not None, f"the GPU ran no {where} check"
            G, A = g["check"]
            assert self.prev_sel is not None
            pi, pn = self.prev_sel
            assert torch.equal(pn, nph), "cached selections differ before the check"
            assert torch.equal(pi[..., :idx.shape[-1]], idx), "cached selections differ"
        assert A is not None and A.dtype == torch.bool
        self._score_error(G, scores_o, f"gate scores ({where})")
        # Exact on the GPU's own scores.
        acc_r, cov_r = ref.check_coverage(G, idx, nph, self.tau)
        own = (cov_r - self.tau).abs() <= OWN_MARGIN
        assert torch.equal(A[~own], acc_r[~own]), (where, A, acc_r)
        self.own_margin += int(own.sum())
        self.heads_checked += A.numel()
        # Against the oracle's fp64 gate.
        assert float((cov_r - cov_o).abs().max()) < COV_ATOL, (where, cov_r, cov_o)
        diff = A != accept_o
        if bool(diff.any()):
            assert bool(((cov_o - self.tau).abs()[diff] <= COV_ATOL).all()), (where, cov_o)
            self.margin_gate += int(diff.sum())
        return A.clone()

    def summary(self):
        return (f"heads checked {self.heads_checked}: fp64-margin selection "
                f"{self.margin_sel}, fp64-margin gate {self.margin_gate}, own-margin "
                f"{self.own_margin}")


def _make_runtime(dev, cfg, seed, steps, extra, gen_on_gpu):
    if gen_on_gpu:
        # Long contexts: draw the inputs on the GPU, then give the oracle host copies.
        inp = make_paged_inputs(**cfg, seed=seed, max_pages=None, spare_blocks=extra,
                                device=dev)
        for name in ("q", "k_cache", "v_cache", "block_tables", "context_lens"):
            setattr(inp, name, getattr(inp, name).cpu())
    else:
        inp = make_paged_inputs(**cfg, seed=seed, max_pages=None, spare_blocks=extra)
    B = inp.q.shape[0]
    bs = inp.k_cache.shape[1]
    W = inp.block_tables.shape[1]
    # leave room in the block table for the appended tokens
    W2 = W + (steps + bs - 1) // bs + 1
    bt = torch.zeros(B, W2, dtype=torch.int32)
    bt[:, :W] = inp.block_tables
    inp.block_tables = bt
    return inp, _Runtime(inp, dev, extra)


def _run(dev, cfg, kw, steps, seed, extra=32, gen_on_gpu=False, expect_margin=0, layers=1,
         own_caches=False):
    """Run both backends for ``steps`` decode steps of ``layers`` layers in
    lockstep and compare them.  The layers share one cache, or with
    ``own_caches`` each has its own (independent inputs and hot pages per
    layer, as a model's layers).  ``expect_margin`` is the number of margin
    heads (of every kind) the seed gives; the BASELINE bar is zero."""
    runs = [_make_runtime(dev, cfg, seed + 17 * l, steps, extra, gen_on_gpu)
            for l in range(layers if own_caches else 1)]
    inp, rt = runs[0]
    B, H_q, D = inp.q.shape
    H = inp.num_kv_heads
    bs = inp.k_cache.shape[1]
    gpu_b = CVSABackend(num_kv_heads=H, num_q_heads=H_q, head_dim=D, block_size=bs, **kw)
    ora_b = OracleCVSABackend(num_kv_heads=H, num_q_heads=H_q, head_dim=D, block_size=bs, **kw)
    lock = _Lockstep(gpu_b, ora_b, kw, rt.ctx)
    g = torch.Generator().manual_seed(seed + 1)
    for step in range(steps):
        for layer in range(layers):
            inp, rt = runs[layer if own_caches else 0]
            lock.ctx = rt.ctx
            q = jitter_query(inp.q, 0.3, seed + 100 + step * layers + layer)
            lock.before_gpu(layer)
            out = gpu_b(q.to(dev), rt.cache.k_cache, rt.cache.v_cache, rt.mgr.block_tables,
                        rt.mgr.context_lens, layer).cpu()
            lock.after_gpu(layer)
            n_tr = len(ora_b.trace)
            want = ora_b(q, rt.K, rt.V, rt.bt, rt.ctx, layer)
            kinds = [t["kind"] for t in ora_b.trace[n_tr:]]
            new_sel = any(k.startswith("score") for k in kinds)
            assert new_sel == lock.g["new"], (step, layer, kinds)
            err = (out.float() - want.float()).abs().max().item()
            assert err < OUT_ATOL, (step, layer, err, kinds)
            ga, oa = gpu_b._last_accept_mask.get(layer), ora_b._last_accept_mask.get(layer)
            assert (ga is None) == (oa is None), (step, layer)
            if ga is not None:
                assert torch.equal(ga.cpu(), oa), (step, layer)
            ge = gpu_b._last_expanded_selection.get(layer)
            oe = ora_b._last_expanded_selection.get(layer)
            assert (ge is None) == (oe is None), (step, layer)
            gs, os_ = gpu_b._cached_selection.get(layer), ora_b._cached_selection.get(layer)
            assert (gs is None) == (os_ is None), (step, layer)   # none on a dense layer
            if gs is not None:
                assert torch.equal(gs[1].cpu(), os_[1]), (step, layer)
                for b in range(B):
                    for h in range(H):
                        n = int(os_[1][b, h])
                        assert torch.equal(gs[0][b, h, :n].cpu(), os_[0][b, h, :n]), (
                            step, layer, b, h)
            gpu_b.step_done(layer, layers)
            ora_b.step_done(layer, layers)
        for inp_l, rt_l in runs:
            kn = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
            vn = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
            rt_l.append(kn, vn, dev)
    sg, so = gpu_b.get_stats(), ora_b.get_stats()
    assert sg == so, (sg, so)
    total = lock.margin_sel + lock.margin_gate + lock.own_margin
    assert total == expect_margin, lock.summary()
    return sg, ora_b.trace, lock


CFG1 = dict(batch=1, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=8192,
            hot_heads=[0, 2, 4, 6], n_hot=8, hot_shift=12.0)


def test_lazy_schedule_cfg1(gpu):
    """cfg1 shapes, lazy M=5, budget 1/4, tau 0.9, exact recovery."""
    stats, trace, _ = _run(gpu, CFG1, dict(budget_pct=0.25, coverage_threshold=0.9, lazy=True,
                                        check_interval=5), steps=12, seed=1000)
    kinds = {t["kind"] for t in trace}
    assert "reuse" in kinds and any(k.startswith("score") for k in kinds)


def test_fixed_interval_schedule_ragged_batch(gpu):
    cfg = dict(batch=3, num_q_heads=32, num_kv_heads=8, head_dim=128,
               context_len=[3000, 1500, 4100], hot_heads=[1, 3], n_hot=6, hot_shift=10.0)
    _run(gpu, cfg, dict(budget_pct=0.25, coverage_threshold=0.8, lazy=False,
                        reuse_interval=3), steps=7, seed=2000)


def test_lazy_gqa7_every_step_check(gpu):
    cfg = dict(batch=2, num_q_heads=28, num_kv_heads=4, head_dim=128, context_len=2048,
               n_hot_range=(0, 16), hot_shift=11.0)
    _run(gpu, cfg, dict(budget_pct=0.25, coverage_threshold=0.9, lazy=True), steps=6,
         seed=3000)


def test_approx_recovery_and_dense_layer(gpu):
    cfg = dict(batch=2, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=2048,
               hot_heads=[0, 1, 2, 3], n_hot=4, hot_shift=9.0)
    _run(gpu, cfg, dict(budget_pct=0.10, coverage_threshold=0.9, lazy=True, check_interval=2,
                        approx_recovery_pct=0.3), steps=5, seed=4000)
    _run(gpu, cfg, dict(budget_pct=0.10, dense_layers=[0], lazy=True, check_interval=2),
         steps=3, seed=4001)


def test_coverage_interval_variant(gpu):
    cfg = dict(batch=1, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=4096,
               hot_heads=[0, 2, 4, 6], n_hot=8, hot_shift=12.0)
    _run(gpu, cfg, dict(budget_pct=0.25, coverage_threshold=0.9, lazy=True, check_interval=4,
                        coverage_interval=1), steps=9, seed=5000)


def test_tracing_attributes(gpu):
    """_last_expanded_selection holds complement pages only when a head rejected."""
    inp = make_paged_inputs(1, 32, 8, 128, 2048, seed=6000, hot_heads=[0, 2, 4, 6], n_hot=8,
                            hot_shift=12.0)
    q, K, V, bt, cl = (t.to(gpu) for t in (inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                            inp.context_lens))
    b = CVSABackend(8, 32, 128, 16, budget_pct=0.25, coverage_threshold=0.9)
    b(q, K, V, bt, cl, 3)
    acc = b._last_accept_mask[3].cpu()
    exp = b._last_expanded_selection.get(3)
    if bool(acc.all()):
        assert exp is None
    else:
        comp, n = exp
        pi, nph = b._cached_selection[3]
        wc, wn = ref.compute_complement(pi.cpu(), nph.cpu(), inp.context_lens, 16, acc)
        assert torch.equal(n.cpu(), wn) and torch.equal(comp.cpu(), wc)


# The BASELINE configurations at full size (one layer; lazy M=5, exact
# recovery): a scoring step, four reuse steps and a lazy check, with one
# token appended per sequence per step.  Key shifts as in bench.py.
# The BASELINE configurations at full size (one layer): a scoring step,
# reuse steps and lazy checks, one token appended per sequence per step.
# name -> (inputs, budget_pct, seed, backend keywords).  The "_recipe" cases
# use the literal BASELINE recipe (+3 sigma hot pages, +2 sigma sink: every
# head's coverage lands far below tau, so every check recovers every head);
# the others use the shifts bench.py measures with (most heads above tau).
_LAZY5 = dict(lazy=True, check_interval=5, coverage_threshold=0.9)
_CFG3_SHAPE = dict(batch=1, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=131072)
_CFG4_SHAPE = dict(batch=8, num_q_heads=28, num_kv_heads=4, head_dim=128, context_len=32768,
                   n_hot_range=(0, 64), hot_shift=17.0)
FULL_SIZE = {
    "cfg1_recipe": (dict(batch=1, num_q_heads=32, num_kv_heads=8, head_dim=128,
                         context_len=8192, hot_heads=[0, 2, 4, 6], n_hot=8, hot_shift=3.0),
                    0.25, 1001, dict(lazy=False, reuse_interval=1, coverage_threshold=0.9)),
    "cfg2": (dict(batch=32, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=8192,
                  random_hot_heads=4, n_hot=8, hot_shift=12.0), 0.25, 7002, _LAZY5),
    "cfg3": (dict(_CFG3_SHAPE, hot_heads=list(range(8)), n_hot=32, hot_shift=14.0,
                  sink_pages=128, sink_shift=14.0), 0.125, 7003, _LAZY5),
    "cfg3_recipe": (dict(_CFG3_SHAPE, hot_heads=list(range(8)), n_hot=32, hot_shift=3.0,
                         sink_pages=128, sink_shift=2.0), 0.125, 1003, _LAZY5),
    "cfg4": (_CFG4_SHAPE, 0.25, 7004, _LAZY5),
    "cfg4_tau080": (_CFG4_SHAPE, 0.25, 7014, dict(_LAZY5, coverage_threshold=0.80)),
    "cfg4_tau095": (_CFG4_SHAPE, 0.25, 7024, dict(_LAZY5, coverage_threshold=0.95)),
    "cfg5": (dict(batch=4, num_q_heads=64, num_kv_heads=8, head_dim=128, context_len=65536,
                  hot_heads=list(range(8)), n_hot=32, hot_shift=14.0, sink_pages=128,
                  sink_shift=14.0), 0.25, 7005, _LAZY5),
}


@pytest.mark.parametrize("name", sorted(FULL_SIZE))
def test_baseline_configuration_full_size(gpu, name):
    cfg, budget, seed, kw = FULL_SIZE[name]
    stats, trace, lock = _run(gpu, cfg, dict(kw, budget_pct=budget), steps=6, seed=seed,
                              gen_on_gpu=True)
    kinds = [t["kind"] for t in trace]
    assert kinds[0].startswith("score"), kinds
    if kw.get("lazy"):
        assert "reuse" in kinds, kinds
    if name.endswith("_recipe"):
        # Coverage far below tau on every head: every check recovers every head.
        assert all(not bool(t["accept"].any()) for t in trace if "accept" in t), kinds
    print(f"{name}: {lock.summary()}")


def test_dense_speculation_literal_cfg3_full_size(gpu):
    """The literal cfg3 recipe at full size (128K context) over 16 steps:
    the first check rejects every head, so the checks after it speculate a
    dense decode (spec_state [2, 2] after each) and their verified launches
    only book counters.  Selections, masks, outputs and statistics in
    lockstep with the oracle backend at every step."""
    cfg, budget, seed, kw = FULL_SIZE["cfg3_recipe"]
    stats, trace, lock = _run(gpu, cfg, dict(kw, budget_pct=budget), steps=16,
                              seed=seed + 5, gen_on_gpu=True)
    kinds = [t["kind"] for t in trace]
    assert sum(k.startswith("score") for k in kinds) == 4, kinds  # fresh + three checks
    assert all(not bool(t["accept"].any()) for t in trace if "accept" in t), kinds
    plan = lock.gpu_b._step_plans[0]
    assert plan.spec_state is not None and plan.spec_state.tolist() == [2, 2]
    print(lock.summary())


@pytest.mark.parametrize("seed", [0, 1])
def test_dense_speculation_ragged_batch(gpu, seed):
    """Ragged contexts (B = 3), tau 0.999 so every gate rejects every head,
    lazy M = 3 over 14 steps with appends crossing pages: the checks after
    the first speculate a dense decode over the identity partition of each
    sequence's own context; in lockstep with the oracle backend."""
    cfg = dict(batch=3, num_q_heads=32, num_kv_heads=8, head_dim=128,
               context_len=[3001 + 97 * seed, 777, 5000 - 13 * seed], hot_heads=[0, 3],
               n_hot=4, hot_shift=8.0)
    kw = dict(budget_pct=0.125, coverage_threshold=0.999, lazy=True, check_interval=3)
    stats, trace, lock = _run(gpu, cfg, kw, steps=14, seed=950 + seed)
    assert all(not bool(t["accept"].any()) for t in trace if "accept" in t)
    plan = lock.gpu_b._step_plans[0]
    assert plan.spec_state is not None and plan.spec_state.tolist() == [2, 2]
    print(lock.summary())


@pytest.mark.parametrize("kw", [
    dict(selector="quest"),
    dict(selector="quest", light_normalizer=True),
    dict(top_p=0.9, coverage_threshold=0.95),
    dict(adaptive_selection=True),
])
def test_selectors_at_cfg3_full_size(gpu, kw):
    """The Quest, light-normalizer, top-p and adaptive schedules at cfg3's
    full size (128K context, 8192 pages) against the oracle backend."""
    cfg, budget, seed, lazy = FULL_SIZE["cfg3"]
    kw = dict(dict(lazy, budget_pct=budget), **kw)
    stats, trace, lock = _run(gpu, cfg, kw, steps=6, seed=seed + 11, gen_on_gpu=True)
    kinds = [t["kind"] for t in trace]
    assert "reuse" in kinds and kinds[0].startswith("score"), kinds
    print(f"{kw}: {lock.summary()}")


def test_timing_buckets(gpu):
    """enable_timing: get_stats adds the reference's per-kernel buckets
    (backend.py:217-223, :300-310) with the same keys; the scoring, coverage
    and draft buckets are filled, complement and LSE merge stay at zero (they
    are folded into the verified decode), and the counters leave the
    schedule statistics unchanged."""
    inp = make_paged_inputs(1, 32, 8, 128, 3000, seed=6100, hot_heads=[0, 2, 4, 6], n_hot=8,
                            hot_shift=12.0)
    q, K, V, bt, cl = (t.to(gpu) for t in (inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                            inp.context_lens))
    timed = CVSABackend(8, 32, 128, 16, num_layers=2, budget_pct=0.25, lazy=True,
                        check_interval=3)
    plain = CVSABackend(8, 32, 128, 16, num_layers=2, budget_pct=0.25, lazy=True,
                        check_interval=3)
    timed.enable_timing(True)
    for step in range(7):
        qs = jitter_query(q, 0.3, 40 + step)
        for layer in range(2):
            a = timed(qs, K, V, bt, cl, layer)
            b = plain(qs, K, V, bt, cl, layer)
            assert torch.equal(a, b)
            timed.step_done(layer, 2)
            plain.step_done(layer, 2)
    st, sp = timed.get_stats(), plain.get_stats()
    keys = {"scoring", "coverage", "sparse_draft", "ar_recovery", "lse_merge", "complement"}
    assert set(st["kernel_times_ms_total"]) == keys
    assert set(st["kernel_counts"]) == keys and set(st["kernel_ms_per_decode_step"]) == keys
    for k in ("scoring", "coverage", "sparse_draft"):
        assert st["kernel_counts"][k] > 0 and st["kernel_times_ms_total"][k] > 0, k
    assert st["kernel_counts"]["complement"] == 0 and st["kernel_counts"]["lse_merge"] == 0
    n = st["total_decode_steps"]
    assert n == 7
    for k in keys:
        assert st["kernel_ms_per_decode_step"][k] == pytest.approx(
            st["kernel_times_ms_total"][k] / n)
    assert {k: v for k, v in st.items() if not k.startswith("kernel_")} == sp


def _random_schedule(seed):
    """A random shape and schedule: B, H_kv, G, ragged contexts, budget, tau,
    lazy (M, coverage interval) or fixed interval, approximate recovery or a
    dense layer now and then."""
    g = torch.Generator().manual_seed(5000 + seed)
    rnd = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))  # noqa: E731
    H = [1, 2, 4, 8][rnd(0, 3)]
    G = rnd(1, 8)
    B = rnd(1, 3)
    cfg = dict(batch=B, num_q_heads=H * G, num_kv_heads=H, head_dim=128,
               context_len=[rnd(200, 5000) for _ in range(B)],
               hot_heads=list(range(0, H, 2)), n_hot=rnd(2, 8), hot_shift=float(rnd(6, 12)))
    kw = dict(budget_pct=[0.125, 0.25, 0.5][rnd(0, 2)],
              coverage_threshold=[0.5, 0.8, 0.9, 0.95][rnd(0, 3)])
    if rnd(0, 1):
        kw.update(lazy=True, check_interval=rnd(2, 5))
        if rnd(0, 2) == 0:
            kw["coverage_interval"] = 1
    else:
        kw.update(lazy=False, reuse_interval=rnd(1, 4))
    if rnd(0, 3) == 0:
        kw["approx_recovery_pct"] = 0.25
    return cfg, kw


@pytest.mark.parametrize("seed", range(8))
def test_random_schedules_against_oracle(gpu, seed):
    """Eight random shapes and schedules, ten steps with appends, in lockstep
    with the oracle backend: selections, masks, outputs and statistics."""
    cfg, kw = _random_schedule(seed)
    stats, trace, lock = _run(gpu, cfg, kw, steps=10, seed=600 + seed)
    print(f"seed {seed} {cfg} {kw}: {lock.summary()}")


# The reference's deployed setting cvsa_5_90_c4_ar20_dL0 (the method-name
# parser, eval/longbench_cvsa.py:190-236: budget 5%, tau 0.90, lazy checks
# every 4 steps, approximate recovery at 20% of the pages, layer 0 dense;
# every latency it publishes, eval/plot_pareto.py:141-150).
DEPLOYED = dict(budget_pct=0.05, coverage_threshold=0.9, lazy=True, check_interval=4,
                approx_recovery_pct=0.2, dense_layers=[0])


_CFG2_ALL_HOT = dict(FULL_SIZE["cfg2"][0], random_hot_heads=0, hot_heads=list(range(8)),
                     n_hot=8, hot_shift=16.0)


@pytest.mark.parametrize("recipe", ["cfg2", "cfg2_all_hot"])
def test_deployed_setting_cfg2_full_size(gpu, recipe):
    """cvsa_5_90_c4_ar20_dL0 at cfg2's full size (B=32, 32/8/128, 8192
    tokens, one token appended per sequence per step) over a dense layer 0
    and a CVSA layer 1, nine decode steps, in lockstep with the oracle
    backend: outputs, selections, accept masks, the expanded selections of
    rejected heads (also the rows the step plan's selection kernel wrote)
    and statistics; zero margin heads.  With cfg2's recipe (hot pages on
    half of the heads) most heads are recovered and every check reselects;
    with every head hot most heads pass and checks can keep."""
    cfg = FULL_SIZE["cfg2"][0] if recipe == "cfg2" else _CFG2_ALL_HOT
    stats, trace, lock = _run(gpu, cfg, DEPLOYED, steps=9, seed=7102, gen_on_gpu=True,
                              layers=2)
    kinds = [t["kind"] for t in trace]
    assert "dense" in kinds and "reuse" in kinds, kinds
    if recipe == "cfg2":
        assert "score_approx" in kinds and lock.expanded_checked > 0, kinds
    print(f"deployed {recipe}: {kinds}: {lock.summary()}, expanded rows checked "
          f"{lock.expanded_checked}")


@pytest.mark.parametrize("shift", [3.0, 12.0])
def test_approx_recovery_cfg1(gpu, shift):
    """Approximate recovery (20%) at cfg1's shape (B=1, 32/8/128, 8192
    tokens, budget 1/4, tau 0.9, scoring every step): with the literal +3
    sigma recipe every head is recovered through its expanded selection,
    at +12 sigma the hot heads pass."""
    cfg = dict(FULL_SIZE["cfg1_recipe"][0], hot_shift=shift)
    kw = dict(budget_pct=0.25, coverage_threshold=0.9, lazy=False, reuse_interval=1,
              approx_recovery_pct=0.2)
    stats, trace, lock = _run(gpu, cfg, kw, steps=4, seed=1011, gen_on_gpu=True)
    assert lock.expanded_checked > 0
    if shift == 3.0:
        assert all(not bool(t["accept"].any()) for t in trace if "accept" in t)
    print(f"cfg1 approx {shift}: {lock.summary()}")


def test_random_reject_every_gate(gpu):
    """random_reject_prob=1.0 (backend.py:433-441, :762-767): every gate
    rejects every head, so every lazy check rescores and recovers every
    head; lockstep with the oracle backend."""
    kw = dict(budget_pct=0.25, coverage_threshold=0.9, lazy=True, check_interval=3,
              random_reject_prob=1.0)
    stats, trace, lock = _run(gpu, CFG1, kw, steps=7, seed=1021)
    assert all(not bool(t["accept"].any()) for t in trace if "accept" in t)
    assert stats["all_accepted_pct"] == 0.0 and stats["rescore_rate"] == 100.0


def test_random_reject_never(gpu):
    """random_reject_prob=0.0: every gate accepts every head.  Lockstep
    with the oracle, and bit for bit the backend that accepts every head by
    its threshold (coverage_threshold=0): outputs, selections and
    statistics."""
    kw = dict(budget_pct=0.25, coverage_threshold=0.9, lazy=True, check_interval=3,
              random_reject_prob=0.0)
    _run(gpu, CFG1, kw, steps=7, seed=1031)
    inp = make_paged_inputs(**CFG1, seed=1032)
    q, K, V, bt, cl = (t.to(gpu) for t in (inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                            inp.context_lens))
    never = CVSABackend(8, 32, 128, 16, **kw)
    base = CVSABackend(8, 32, 128, 16, **dict(kw, coverage_threshold=0.0,
                                              random_reject_prob=None))
    for step in range(7):
        qs = jitter_query(q, 0.3, 1040 + step)
        a = never(qs, K, V, bt, cl, 0)
        b = base(qs, K, V, bt, cl, 0)
        assert torch.equal(a, b), step
        assert torch.equal(never._cached_selection[0][0], base._cached_selection[0][0])
        assert torch.equal(never._cached_selection[0][1], base._cached_selection[0][1])
        never.step_done(0, 1)
        base.step_done(0, 1)
    assert never.get_stats() == base.get_stats()


def test_cfg2_baseline_schedule_20_steps(gpu):
    """cfg2 as BASELINE states it: B=32, 8B shapes, 8192-token contexts, 20
    consecutive decode steps each appending one token per sequence, lazy
    M=5, budget 1/4, tau 0.9 -- the whole schedule (4 checks, 16 reuse
    steps) in lockstep with the oracle backend."""
    cfg, budget, seed, kw = FULL_SIZE["cfg2"]
    # 20 appended tokens from a page boundary: two new pages per sequence.
    stats, trace, lock = _run(gpu, cfg, dict(kw, budget_pct=budget), steps=20, seed=seed,
                              gen_on_gpu=True, extra=cfg["batch"] * 3)
    kinds = [t["kind"] for t in trace]
    assert kinds.count("reuse") == 16 and stats["total_decode_steps"] == 20, kinds
    print(f"cfg2 x 20 steps: {kinds}: {lock.summary()}")


def test_cfg5_layers_with_own_caches(gpu):
    """cfg5's shapes (Llama-3.1-70B attention 64q/8kv/d128, B=4, 65536-token
    contexts) over four layers, each with its own cache and hot-page
    clusters (as BASELINE's per-layer independent caches), ten decode steps
    with appends, lazy M=5, in lockstep with the oracle backend."""
    cfg, budget, seed, kw = FULL_SIZE["cfg5"]
    stats, trace, lock = _run(gpu, cfg, dict(kw, budget_pct=budget), steps=10, seed=seed,
                              gen_on_gpu=True, layers=4, own_caches=True)
    kinds = [t["kind"] for t in trace]
    assert kinds.count("reuse") == 32, kinds
    print(f"cfg5 x 4 layers x 10 steps: {lock.summary()}")
