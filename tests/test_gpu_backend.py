"""Multi-step decode parity of the GPU CVSABackend against the oracle state machine.

Both backends run the same decode loop (query jittered per step, one token
appended per sequence per step through the paged-KV runtime) on identical
inputs.  Checked per call: output max-abs, the accept mask (exact outside the
|coverage - tau| margin), the cached page selection (exact outside the
k-th/(k+1)-th score-gap margin, a top-k set of the oracle scores inside it),
the append state; at the end get_stats() must be identical.  The BASELINE
configurations run at full size (128K context, B=32, G=8 ...).
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
GAP_MARGIN = 1e-5
COV_MARGIN = 1e-5


class _Runtime:
    """A GPU cache + manager and a CPU oracle copy of the same state."""

    def __init__(self, inp, dev, extra_tokens):
        B = inp.q.shape[0]
        nb = inp.k_cache.shape[0]
        H, D = inp.k_cache.shape[2], inp.k_cache.shape[3]
        W = inp.block_tables.shape[1]
        self.cache = PagedKVCache(nb, 16, H, D, device=str(dev))
        self.cache.k_cache.copy_(inp.k_cache)
        self.cache.v_cache.copy_(inp.v_cache)
        self.cache._next_free = inp.used_blocks
        self.mgr = SequenceKVManager(self.cache, B, W * 16)
        self.mgr.block_tables.copy_(inp.block_tables)
        self.mgr.context_lens.copy_(inp.context_lens)
        pages = [-(-int(c) // 16) for c in inp.context_lens.tolist()]
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
                                          b, k[b], v[b], 16)


def _margins(ps, budget, cov, tau):
    """Heads where selection / acceptance is numerically undecidable."""
    srt = torch.sort(ps, dim=-1, descending=True).values
    if budget < ps.shape[-1]:
        gap = (srt[..., budget - 1] - srt[..., budget]).abs()
        bad_sel = gap <= GAP_MARGIN * srt[..., budget - 1].abs().clamp(min=1.0)
    else:
        bad_sel = torch.zeros(ps.shape[:2], dtype=torch.bool)
    bad_acc = (cov - tau).abs() <= COV_MARGIN
    return bad_sel, bad_acc


def _check_near_tie_selection(pi, nph, ps, budget, bad_sel):
    """Heads whose k-th/(k+1)-th gap is within the margin: the GPU's set must
    still be a top-``budget`` set of the oracle scores up to that margin."""
    srt = torch.sort(ps, dim=-1, descending=True).values
    for b, h in bad_sel.nonzero().tolist():
        n = int(nph[b, h])
        sel = pi[b, h, :n].long()
        assert torch.all(sel[1:] > sel[:-1]), (b, h)
        kth = float(srt[b, h, budget - 1])
        tol = GAP_MARGIN * max(abs(kth), 1.0)
        assert float(ps[b, h, sel].min()) >= kth - tol, (b, h)
        rest = ps[b, h].clone()
        rest[sel] = float("-inf")
        assert float(rest.max()) <= kth + tol, (b, h)


def _check_budgeted_selection(pi, nph, t, kw, tau):
    """Per-head budgets (top_p / static_budget_table / adaptive_selection):
    each row's first
    n_per_head pages equal the oracle's, except rows whose budget or k-th
    page is numerically undecidable (top-p boundary within 1e-4 of top_p:
    the GPU ranks its fp32 page scores, the oracle fp64 ones; or the score
    gap after the k-th page within the margin), which are counted and not
    compared.  Returns (undecidable rows, accept-margin mask)."""
    ranked = t.get("sel_scores", t["page_scores"])
    wi, wn = t["page_indices"], t["n_per_head"]
    B, H, W = ranked.shape
    srt = torch.sort(ranked, dim=-1, descending=True).values
    loose = torch.zeros(B, H, dtype=torch.bool)
    if kw.get("top_p") is not None:
        need, order = ref.topp_need(ranked, kw["top_p"])
        cum = torch.cumsum(torch.softmax(ranked.double(), -1).gather(-1, order), -1)
        p32 = float(torch.tensor(kw["top_p"], dtype=torch.float32))
        for b in range(B):
            for h in range(H):
                k = int(need[b, h])
                near = abs(float(cum[b, h, k - 1]) - p32) < 1e-4
                near |= k >= 2 and abs(float(cum[b, h, k - 2]) - p32) < 1e-4
                loose[b, h] = bool(near)
    for b in range(B):
        for h in range(H):
            n = int(wn[b, h])
            if n < W:
                gap = float(srt[b, h, n - 1] - srt[b, h, n])
                if abs(gap) <= GAP_MARGIN * max(abs(float(srt[b, h, n - 1])), 1.0):
                    loose[b, h] = True
            if loose[b, h]:
                continue
            assert int(nph[b, h]) == n, (b, h)
            assert pi[b, h, :n].tolist() == wi[b, h, :n].tolist(), (b, h)
    return loose, (t["coverage"] - tau).abs() <= COV_MARGIN


def _run(dev, cfg, kw, steps, seed, extra=32, gen_on_gpu=False, max_margin_frac=0.0):
    """Run both backends for ``steps`` calls and compare them.

    Heads whose selection is a near-tie are held to the tolerant top-k check;
    ``max_margin_frac`` bounds the share of (b, h) head-checks whose coverage
    lies within the margin of tau (their accept bit is not compared).  Large
    shapes draw a few such heads; small shapes must have none.
    """
    if gen_on_gpu:
        # Long contexts: draw the inputs on the GPU, then give the oracle host copies.
        inp = make_paged_inputs(**cfg, seed=seed, max_pages=None, spare_blocks=extra,
                                device=dev)
        for name in ("q", "k_cache", "v_cache", "block_tables", "context_lens"):
            setattr(inp, name, getattr(inp, name).cpu())
    else:
        inp = make_paged_inputs(**cfg, seed=seed, max_pages=None, spare_blocks=extra)
    B, H_q, D = inp.q.shape
    H = inp.num_kv_heads
    W = inp.block_tables.shape[1]
    # leave room in the block table for the appended tokens
    W2 = W + (steps + 15) // 16 + 1
    bt = torch.zeros(B, W2, dtype=torch.int32)
    bt[:, :W] = inp.block_tables
    inp.block_tables = bt
    rt = _Runtime(inp, dev, extra)
    gpu_b = CVSABackend(num_kv_heads=H, num_q_heads=H_q, head_dim=D, block_size=16, **kw)
    ora_b = OracleCVSABackend(num_kv_heads=H, num_q_heads=H_q, head_dim=D, block_size=16, **kw)
    g = torch.Generator().manual_seed(seed + 1)
    margin_sel = margin_acc = checks = 0
    for step in range(steps):
        q = jitter_query(inp.q, 0.3, seed + 100 + step)
        out = gpu_b(q.to(dev), rt.cache.k_cache, rt.cache.v_cache, rt.mgr.block_tables,
                    rt.mgr.context_lens, 0).cpu()
        n_tr = len(ora_b.trace)
        want = ora_b(q, rt.K, rt.V, rt.bt, rt.ctx, 0)
        tr = ora_b.trace[n_tr:]
        err = (out.float() - want.float()).abs().max().item()
        scoring = [t for t in tr if t["kind"].startswith("score")]
        budgeted = (kw.get("top_p") is not None or kw.get("static_budget_table") is not None
                    or kw.get("adaptive_selection", False))
        if scoring and budgeted:
            t = scoring[-1]
            pi, nph = gpu_b._cached_selection[0]
            bad_sel, bad_acc = _check_budgeted_selection(
                pi.cpu(), nph.cpu(), t, kw, kw.get("coverage_threshold", 0.9))
            margin_sel += int(bad_sel.sum())
            margin_acc += int(bad_acc.sum())
            checks += bad_sel.numel()
            acc = gpu_b._last_accept_mask[0].cpu()
            ok = ~(bad_acc | bad_sel)
            assert torch.equal(acc[ok], t["accept"][ok]), step
        elif scoring:
            t = scoring[-1]
            budget = t["page_indices"].shape[-1]
            ranked = t.get("sel_scores", t["page_scores"])   # what the selection ranks
            bad_sel, bad_acc = _margins(ranked, budget, t["coverage"], kw.get(
                "coverage_threshold", 0.9))
            margin_sel += int(bad_sel.sum())
            margin_acc += int(bad_acc.sum())
            checks += bad_sel.numel()
            pi, nph = gpu_b._cached_selection[0]
            ok = ~bad_sel
            assert torch.equal(pi.cpu()[ok], t["page_indices"][ok]), step
            _check_near_tie_selection(pi.cpu(), nph.cpu(), ranked, budget, bad_sel)
            assert torch.equal(nph.cpu(), t["n_per_head"])
            acc = gpu_b._last_accept_mask[0].cpu()
            ok = ~bad_acc
            assert torch.equal(acc[ok], t["accept"][ok]), step
        assert err < OUT_ATOL, (step, err, [t["kind"] for t in tr])
        gpu_b.step_done(0, 1)
        ora_b.step_done(0, 1)
        kn = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
        vn = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
        rt.append(kn, vn, dev)
    assert margin_acc <= max_margin_frac * checks, (margin_sel, margin_acc, checks)
    sg, so = gpu_b.get_stats(), ora_b.get_stats()
    if margin_acc == 0 and not (budgeted and margin_sel):
        assert sg == so, (sg, so)
    return sg, ora_b.trace


CFG1 = dict(batch=1, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=8192,
            hot_heads=[0, 2, 4, 6], n_hot=8, hot_shift=12.0)


def test_lazy_schedule_cfg1(gpu):
    """cfg1 shapes, lazy M=5, budget 1/4, tau 0.9, exact recovery."""
    stats, trace = _run(gpu, CFG1, dict(budget_pct=0.25, coverage_threshold=0.9, lazy=True,
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
FULL_SIZE = {
    "cfg3": (dict(batch=1, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=131072,
                  hot_heads=list(range(8)), n_hot=32, hot_shift=14.0, sink_pages=128,
                  sink_shift=14.0), 0.125, 7003),
    "cfg4": (dict(batch=8, num_q_heads=28, num_kv_heads=4, head_dim=128, context_len=32768,
                  n_hot_range=(0, 64), hot_shift=17.0), 0.25, 7004),
    "cfg5": (dict(batch=4, num_q_heads=64, num_kv_heads=8, head_dim=128, context_len=65536,
                  hot_heads=list(range(8)), n_hot=32, hot_shift=14.0, sink_pages=128,
                  sink_shift=14.0), 0.25, 7005),
    "cfg2": (dict(batch=32, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=8192,
                  random_hot_heads=4, n_hot=8, hot_shift=12.0), 0.25, 7002),
}


@pytest.mark.parametrize("name", sorted(FULL_SIZE))
def test_baseline_configuration_full_size(gpu, name):
    cfg, budget, seed = FULL_SIZE[name]
    stats, trace = _run(gpu, cfg, dict(budget_pct=budget, coverage_threshold=0.9, lazy=True,
                                       check_interval=5), steps=6, seed=seed, gen_on_gpu=True,
                        max_margin_frac=0.02)
    kinds = [t["kind"] for t in trace]
    assert "reuse" in kinds and kinds[0].startswith("score"), kinds


@pytest.mark.parametrize("kw", [
    dict(selector="quest"),
    dict(selector="quest", light_normalizer=True),
    dict(top_p=0.9, coverage_threshold=0.95),
    dict(adaptive_selection=True),
])
def test_selectors_at_cfg3_full_size(gpu, kw):
    """The Quest, light-normalizer, top-p and adaptive schedules at cfg3's
    full size (128K context, 8192 pages) against the oracle backend."""
    cfg, budget, seed = FULL_SIZE["cfg3"]
    kw = dict(dict(budget_pct=budget, coverage_threshold=0.9, lazy=True, check_interval=5),
              **kw)
    stats, trace = _run(gpu, cfg, kw, steps=6, seed=seed + 11, gen_on_gpu=True,
                        max_margin_frac=0.02)
    kinds = [t["kind"] for t in trace]
    assert "reuse" in kinds and kinds[0].startswith("score"), kinds


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
