"""The multi-layer decode driver (cvsa.runtime.decode_driver).

* Against the oracle: the driver's per-layer protocol (append, backend call,
  step_done for every layer of a step; eager and with graph-replayed reuse
  steps) over several layers and steps gives the oracle backend's outputs,
  selections, accept masks, complement pages and statistics, the oracle
  running the same protocol on CPU copies of every layer's cache with the
  reference's append rule.
* Graph-replayed reuse steps are bit-identical to the eager per-layer
  protocol, step after step with appends and scoring steps in between (each
  replay is checked against the eager run), and leave the same schedule,
  statistics and tracing state.
* Appends folded into the reuse steps' decode launches
  (``DecodeDriver(fuse_append=True)``, cvsa_step_plan_run_append) give the
  outputs, caches, page tables, context lengths, allocation counts and
  statistics of the separate append followed by the call, bit for bit, with
  sequences crossing page boundaries, in the one-launch form (16-token
  pages, D = 128, G <= 16) and in the two-launch form of other shapes.
"""
import pytest
import torch

from oracle import cvsa_oracle as ref
from oracle.backend_oracle import OracleCVSABackend
from cvsa.backend import CVSABackend
from cvsa.runtime.decode_driver import DecodeDriver, SyntheticDecodeLayers

pytestmark = pytest.mark.gpu

SHAPE = dict(num_layers=4, batch=2, num_q_heads=32, num_kv_heads=8, head_dim=128,
             context_len=[3000, 1700], max_new_tokens=24, seed=5, hot_heads=[0, 3, 6],
             n_hot=6, hot_shift=10.0)


class _OracleLayers:
    """CPU copies of every layer's cache, table, lengths and allocator."""

    def __init__(self, layers):
        self.K = [c.k_cache.cpu() for c in layers.caches]
        self.V = [c.v_cache.cpu() for c in layers.caches]
        self.bt = [m.block_tables.cpu() for m in layers.managers]
        self.ctx = [m.context_lens.cpu() for m in layers.managers]
        self.alloc = [torch.tensor(m._pages_allocated, dtype=torch.int32)
                      for m in layers.managers]
        self.nf = [c._next_free for c in layers.caches]

    def append(self, l, k, v):
        for b in range(k.shape[0]):
            self.nf[l] = ref.append_token_kv(self.K[l], self.V[l], self.bt[l], self.ctx[l],
                                             self.alloc[l], self.nf[l], b, k[b], v[b], 16)


ORACLE_SHAPE = dict(num_layers=3, batch=2, num_q_heads=32, num_kv_heads=8, head_dim=128,
                    context_len=[2600, 1900], max_new_tokens=16, seed=11,
                    hot_heads=[0, 2, 5, 7], n_hot=6, hot_shift=9.0)


@pytest.mark.parametrize("mode", ["eager", "graphs", "fused", "fused_graphs"])
@pytest.mark.parametrize("kw", [dict(lazy=True, check_interval=3),
                                dict(lazy=False, reuse_interval=2)])
def test_driver_matches_oracle_backend(gpu, mode, kw):
    """3 layers x 12 steps with one token appended per sequence per layer and
    step: every layer's output, cached selection, accept mask and complement
    pages after every step, and the final statistics, against the oracle
    backend driven through the same protocol."""
    L = ORACLE_SHAPE["num_layers"]
    layers = SyntheticDecodeLayers(device=gpu, **ORACLE_SHAPE)
    cfg = dict(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16, num_layers=L,
               budget_pct=0.2, coverage_threshold=0.9, **kw)
    backend = CVSABackend(**cfg)
    oracle = OracleCVSABackend(**cfg)
    state = _OracleLayers(layers)
    graphs = mode in ("graphs", "fused_graphs")
    driver = DecodeDriver(backend, layers, graphs=graphs, fuse_append=mode.startswith("fused"))
    kinds = set()
    for step in range(12):
        q, k, v = layers.step_inputs(step)
        outs = [o.float().cpu() for o in driver.step(q, k, v)]
        qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
        for l in range(L):
            state.append(l, kc[l], vc[l])
            n_tr = len(oracle.trace)
            want = oracle(qc[l], state.K[l], state.V[l], state.bt[l], state.ctx[l], l)
            oracle.step_done(l, L)
            kinds.update(t["kind"] for t in oracle.trace[n_tr:])
            err = (outs[l] - want.float()).abs().max().item()
            assert err < 2e-2, (step, l, err)
            gs, os_ = backend._cached_selection[l], oracle._cached_selection[l]
            assert torch.equal(gs[1].cpu(), os_[1]), (step, l)
            for b in range(2):
                for h in range(8):
                    n = int(os_[1][b, h])
                    assert torch.equal(gs[0][b, h, :n].cpu(), os_[0][b, h, :n]), (step, l, b, h)
            ga, oa = backend._last_accept_mask.get(l), oracle._last_accept_mask.get(l)
            assert (ga is None) == (oa is None), (step, l)
            if ga is not None:
                assert torch.equal(ga.cpu(), oa), (step, l)
            ge = backend._last_expanded_selection.get(l)
            oe = oracle._last_expanded_selection.get(l)
            assert (ge is None) == (oe is None), (step, l)
            if ge is not None:
                assert torch.equal(ge[1].cpu(), oe[1]), (step, l)
                for b in range(2):
                    for h in range(8):
                        n = int(oe[1][b, h])
                        assert torch.equal(ge[0][b, h, :n].cpu(), oe[0][b, h, :n])
        for l in range(L):
            assert torch.equal(layers.managers[l].context_lens.cpu(), state.ctx[l])
            assert torch.equal(layers.managers[l].block_tables.cpu(), state.bt[l])
    assert backend.get_stats() == oracle.get_stats()
    assert {"reuse"} < kinds and any(k.startswith("score") for k in kinds), kinds
    if graphs:
        assert driver.replays >= 1, driver.replays


def _pair(gpu, kw):
    runs = []
    for graphs in (False, True):
        layers = SyntheticDecodeLayers(device=gpu, **SHAPE)
        backend = CVSABackend(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                              num_layers=SHAPE["num_layers"], budget_pct=0.2,
                              coverage_threshold=0.9, **kw)
        # chunks of 2 layers: several graphs per step, appends between them
        runs.append((layers, backend, DecodeDriver(backend, layers, graphs=graphs,
                                                   graph_chunk=2)))
    return runs


@pytest.mark.parametrize("kw", [dict(lazy=True, check_interval=3),
                                dict(lazy=False, reuse_interval=2),
                                dict(lazy=True, check_interval=4, selector="quest")])
def test_graph_replay_equals_eager(gpu, kw):
    (la, ba, da), (lb, bb, db) = _pair(gpu, kw)
    for step in range(12):
        q, k, v = la.step_inputs(step)
        out_a = [o.clone() for o in da.step(q, k, v)]
        out_b = [o.clone() for o in db.step(q, k, v)]
        for layer, (a, b) in enumerate(zip(out_a, out_b)):
            assert torch.equal(a, b), (step, layer)
        for layer in range(SHAPE["num_layers"]):
            ma, mb = ba._last_accept_mask.get(layer), bb._last_accept_mask.get(layer)
            assert (ma is None) == (mb is None), (step, layer)
            if ma is not None:
                assert torch.equal(ma, mb), (step, layer)
        for ma, mb in zip(la.managers, lb.managers):
            assert torch.equal(ma.context_lens, mb.context_lens)
            assert torch.equal(ma.block_tables, mb.block_tables)
    assert db.captures >= 1 and db.replays >= 3, (db.captures, db.replays)
    assert ba._step == bb._step
    assert ba.get_stats() == bb.get_stats()


def test_driver_run_reports_latency(gpu):
    layers = SyntheticDecodeLayers(device=gpu, **dict(SHAPE, max_new_tokens=16))
    backend = CVSABackend(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                          num_layers=SHAPE["num_layers"], budget_pct=0.2, lazy=True,
                          check_interval=5)
    res = DecodeDriver(backend, layers, graphs=True).run(steps=8, warmup=3)
    assert res["steps"] == 8 and len(res["per_step_ms"]) == 8
    assert 0 < res["median_ms"] <= res["p99_ms"]
    assert res["graph_replays"] >= 4


def _count_fused(monkeypatch):
    """Counts folded reuse calls: the checked entry (StepPlan.run_reuse_append)
    and the backend's prepared call (_FusedReuse.run)."""
    from cvsa import ops
    from cvsa import backend as backend_mod
    calls = []
    orig = ops.StepPlan.run_reuse_append
    orig_fast = backend_mod._FusedReuse.run

    def counted(self, *a, **k):
        calls.append(1)
        return orig(self, *a, **k)

    def counted_fast(self, *a, **k):
        out = orig_fast(self, *a, **k)
        if out is not None:
            calls.append(1)
        return out

    monkeypatch.setattr(ops.StepPlan, "run_reuse_append", counted)
    monkeypatch.setattr(backend_mod._FusedReuse, "run", counted_fast)
    return calls


@pytest.mark.parametrize("shape", [
    # one launch: 16-token pages, D = 128, G = 4; sequences cross pages at
    # steps 8, 12 and 0 / 16
    dict(num_q_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
         context_len=[3000, 1700, 1792]),
    # two launches inside the entry point: D = 64; 32-token pages; G = 20
    dict(num_q_heads=16, num_kv_heads=4, head_dim=64, block_size=16,
         context_len=[2040, 1000]),
    dict(num_q_heads=32, num_kv_heads=8, head_dim=128, block_size=32,
         context_len=[2016, 990]),
    dict(num_q_heads=40, num_kv_heads=2, head_dim=128, block_size=16,
         context_len=[1600, 2047]),
], ids=["one_launch", "d64", "bs32", "g20"])
def test_fused_append_equals_separate(gpu, monkeypatch, shape):
    calls = _count_fused(monkeypatch)
    L, steps = 3, 20
    runs = []
    for fuse in (False, True):
        layers = SyntheticDecodeLayers(num_layers=L, batch=len(shape["context_len"]),
                                       max_new_tokens=steps, seed=21, device=gpu,
                                       hot_heads=[0, 1], n_hot=6, hot_shift=9.0, **shape)
        backend = CVSABackend(num_kv_heads=shape["num_kv_heads"],
                              num_q_heads=shape["num_q_heads"], head_dim=shape["head_dim"],
                              block_size=shape["block_size"], num_layers=L, budget_pct=0.25,
                              coverage_threshold=0.9, lazy=True, check_interval=4)
        runs.append((layers, backend, DecodeDriver(backend, layers, fuse_append=fuse)))
    (la, ba, da), (lb, bb, db) = runs
    for step in range(steps):
        q, k, v = la.step_inputs(step)
        n0 = len(calls)
        out_a = [o.clone() for o in da.step(q, k, v)]
        assert len(calls) == n0, "the separate run took the fused path"
        out_b = [o.clone() for o in db.step(q, k, v)]
        for layer, (a, b) in enumerate(zip(out_a, out_b)):
            assert torch.equal(a, b), (step, layer)
    torch.cuda.synchronize()
    for l in range(L):
        ca, cb = la.caches[l], lb.caches[l]
        ma, mb = la.managers[l], lb.managers[l]
        assert torch.equal(ca.k_cache, cb.k_cache) and torch.equal(ca.v_cache, cb.v_cache), l
        assert torch.equal(ma.block_tables, mb.block_tables), l
        assert torch.equal(ma.context_lens, mb.context_lens), l
        assert torch.equal(ma._pages_allocated_dev, mb._pages_allocated_dev), l
        assert ma._pages_allocated == mb._pages_allocated and ma._ctx_host == mb._ctx_host, l
        assert ca._next_free == cb._next_free, l
        assert ma._ctx_host == [int(x) for x in mb.context_lens.tolist()], l
        assert ma._pages_allocated == [int(x) for x in mb._pages_allocated_dev.tolist()], l
    assert ba.get_stats() == bb.get_stats()
    # every reuse call of the fused run (3 of every 4 steps per layer) was fused
    assert len(calls) == L * (steps - steps // 4), len(calls)


def test_fused_fast_path_falls_back(gpu, monkeypatch):
    """The prepared folded call (after a layer's first checked one) hands a
    call back to the checked path when what it was checked for changes: a
    non-contiguous row tensor, another stream, a reset backend, a cache
    swapped under the manager.  Outputs, caches and statistics equal the
    separate append and call throughout."""
    from cvsa import backend as backend_mod
    fast = []
    orig_fast = backend_mod._FusedReuse.run

    def counted_fast(self, *a, **k):
        fast.append(1)
        return orig_fast(self, *a, **k)

    monkeypatch.setattr(backend_mod._FusedReuse, "run", counted_fast)
    runs = []
    for fuse in (False, True):
        layers = SyntheticDecodeLayers(num_layers=1, batch=2, num_q_heads=32, num_kv_heads=8,
                                       head_dim=128, context_len=[1500, 2100],
                                       max_new_tokens=40, seed=31, device=gpu,
                                       hot_heads=[0, 1], n_hot=6, hot_shift=9.0)
        backend = CVSABackend(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                              num_layers=1, budget_pct=0.25, coverage_threshold=0.9,
                              lazy=True, check_interval=5)
        runs.append((layers, backend))
    (la, ba), (lb, bb) = runs
    side = torch.cuda.Stream(gpu)

    def step(i, variant):
        q, k, v = la.step_inputs(i)
        ma, mb = la.managers[0], lb.managers[0]
        ma.append_tokens_kv(k[0], v[0])
        ca = la.caches[0]
        a = ba(q[0], ca.k_cache, ca.v_cache, ma.block_tables, ma.context_lens, 0)
        kb, vb = k[0], v[0]
        if variant == "strided":
            kb = torch.empty(kb.shape[0], kb.shape[1], 2 * kb.shape[2], dtype=kb.dtype,
                             device=gpu)[:, :, ::2].copy_(kb)
            assert not kb.is_contiguous()
        n0 = len(fast)
        if variant == "stream":
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                b = bb.call_with_append(q[0], kb, vb, mb, 0)
            torch.cuda.current_stream().wait_stream(side)
        else:
            b = bb.call_with_append(q[0], kb, vb, mb, 0)
        ba.step_done(0, 1)
        bb.step_done(0, 1)
        torch.cuda.synchronize()
        assert torch.equal(a, b), (i, variant)
        return len(fast) > n0

    took = [step(i, "plain") for i in range(8)]
    assert any(took[2:5]) and any(took[6:8]), took  # reuse steps after the first
    assert not step(8, "strided") and not step(9, "stream")
    ba.reset()
    bb.reset()
    assert not step(10, "plain")          # a scoring step after reset
    took = [step(i, "plain") for i in range(11, 16)]  # backend steps 1-5 (5: a check)
    assert took[1] and took[2] and not took[4], took
    for (layers, _b) in runs:             # the same blocks under a new tensor object
        c = layers.caches[0]
        c.k_cache = c.k_cache.clone()
    assert not step(16, "plain")          # a reuse step over the new cache: checked path
    torch.cuda.synchronize()
    ca, cb = la.caches[0], lb.caches[0]
    assert torch.equal(ca.k_cache, cb.k_cache) and torch.equal(ca.v_cache, cb.v_cache)
    assert torch.equal(la.managers[0].context_lens, lb.managers[0].context_lens)
    assert ba.get_stats() == bb.get_stats()


def test_fused_append_rejects_inconsistent_slots(gpu):
    """A slot table that does not follow the allocator is refused before any
    launch: the cache, tables and lengths stay as they were."""
    import ctypes
    from cvsa import ops
    layers = SyntheticDecodeLayers(num_layers=1, batch=2, num_q_heads=32, num_kv_heads=8,
                                   head_dim=128, context_len=[1601, 1700], max_new_tokens=4,
                                   seed=3, device=gpu)
    backend = CVSABackend(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                          num_layers=1, budget_pct=0.25, lazy=True, check_interval=4)
    mgr, cache = layers.managers[0], layers.caches[0]
    q, k, v = layers.step_inputs(0)
    backend(q[0], cache.k_cache, cache.v_cache, mgr.block_tables, mgr.context_lens, 0)
    backend.step_done(0, 1)
    plan = backend.reuse_plan_for(q[0], cache.k_cache, cache.v_cache, mgr.block_tables,
                                  mgr.context_lens, 0)
    assert plan is not None
    before = (mgr.context_lens.clone(), mgr.block_tables.clone(), cache.k_cache[:4].clone())
    slots, _ = mgr.fused_append_slots()
    bad = (ctypes.c_int32 * 4)(*slots)
    bad[1] = 7  # sequence 0 is mid-page (1601 % 16 == 1): it takes no new block
    with pytest.raises(ValueError):
        plan.run_reuse_append(q[0], k[0], v[0], mgr._pages_allocated_dev, bad)
    torch.cuda.synchronize()
    assert torch.equal(mgr.context_lens, before[0]) and torch.equal(mgr.block_tables, before[1])
    assert torch.equal(cache.k_cache[:4], before[2])


@pytest.mark.parametrize("kw,in_place", [(dict(lazy=True, check_interval=3), False),
                                         (dict(lazy=False, reuse_interval=2), False),
                                         (dict(lazy=True, check_interval=4), True)])
def test_fused_graph_replay_equals_eager(gpu, kw, in_place):
    """Graph replay of chunks of folded append-and-decode launches (device
    slots staged before each replay) against the eager separate append and
    call, step after step, with sequences crossing page boundaries: outputs,
    masks, caches, tables, lengths, allocation counts and statistics equal.
    With in_place the graph driver's inputs are made in its static buffers."""
    shape = dict(SHAPE, context_len=[3000, 1792], max_new_tokens=30)
    runs = []
    for graphs, fuse in ((False, False), (True, True)):
        layers = SyntheticDecodeLayers(device=gpu, **shape)
        backend = CVSABackend(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                              num_layers=SHAPE["num_layers"], budget_pct=0.2,
                              coverage_threshold=0.9, **kw)
        runs.append((layers, backend, DecodeDriver(backend, layers, graphs=graphs,
                                                   graph_chunk=3 if in_place else 2,
                                                   fuse_append=fuse)))
    (la, ba, da), (lb, bb, db) = runs
    for step in range(24):
        q, k, v = la.step_inputs(step)
        out_a = [o.clone() for o in da.step(q, k, v)]
        if in_place:
            qs, ks, vs = db.static_inputs()
            qs.copy_(q), ks.copy_(k), vs.copy_(v)
            out_b = [o.clone() for o in db.step(qs, ks, vs)]
        else:
            out_b = [o.clone() for o in db.step(q, k, v)]
        for layer, (a, b) in enumerate(zip(out_a, out_b)):
            assert torch.equal(a, b), (step, layer)
        for layer in range(SHAPE["num_layers"]):
            ma, mb = ba._last_accept_mask.get(layer), bb._last_accept_mask.get(layer)
            assert (ma is None) == (mb is None), (step, layer)
            if ma is not None:
                assert torch.equal(ma, mb), (step, layer)
        for ma, mb in zip(la.managers, lb.managers):
            assert torch.equal(ma.context_lens, mb.context_lens), step
            assert torch.equal(ma.block_tables, mb.block_tables), step
            assert torch.equal(ma._pages_allocated_dev, mb._pages_allocated_dev), step
            assert ma._ctx_host == mb._ctx_host and ma._pages_allocated == mb._pages_allocated
    torch.cuda.synchronize()
    for ca, cb in zip(la.caches, lb.caches):
        assert torch.equal(ca.k_cache, cb.k_cache) and torch.equal(ca.v_cache, cb.v_cache)
        assert ca._next_free == cb._next_free
    assert db.captures >= 1 and db.replays >= 6, (db.captures, db.replays)
    assert ba._step == bb._step
    assert ba.get_stats() == bb.get_stats()
