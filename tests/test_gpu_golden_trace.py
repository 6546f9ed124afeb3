"""The HIP path against the reference implementation's recorded multi-step
behaviour (golden traces written by tests/golden/make_backend_trace.py):
outputs, accept masks, selected / complement / expanded page sets, schedule
counters, statistics and the paged-KV append state; for the two cfg1-shaped
traces (8B attention, one 8192-token sequence) also the coverage and the
merged result's log-sum-exp of the scoring step."""
import pytest
import torch

from golden_trace_check import SCENARIOS, replay
from cvsa.backend import CVSABackend
from cvsa.runtime.kv_cache import PagedKVCache, SequenceKVManager

pytestmark = pytest.mark.gpu


def _runtime(dev):
    def make(case):
        nb, _, H, D = case.k_cache.shape
        W = case.block_tables.shape[1]
        B = case.block_tables.shape[0]
        cache = PagedKVCache(nb, 16, H, D, device=str(dev))
        cache.k_cache.copy_(case.k_cache)
        cache.v_cache.copy_(case.v_cache)
        cache._next_free = case.next_free
        mgr = SequenceKVManager(cache, B, W * 16)
        mgr.block_tables.copy_(case.block_tables)
        mgr.context_lens.copy_(case.context_lens)
        mgr._pages_allocated = list(case.pages_allocated)
        mgr.sync_host_state()

        def call_args(q):
            return q.to(dev), cache.k_cache, cache.v_cache, mgr.block_tables, mgr.context_lens

        def append(b, k, v):
            mgr.append_token_kv(b, k.to(dev), v.to(dev))

        def state():
            return mgr.block_tables.cpu().numpy(), mgr.context_lens.cpu().numpy()

        runtimes.append((dev, mgr))
        return call_args, append, state
    runtimes = []
    make.runtimes = runtimes
    return make


def _counters(b):
    return dict(scoring=b._total_scoring_steps, checks=b._total_coverage_checks,
                accepts=b._accept_counts, rejects=b._reject_counts)


def _hip_state(b, args):
    """Coverage of the last selection on its gate scores and the merged
    result's LSE per q-head, through the HIP ops (the verified decode's
    (m, l): draft pages on accepted heads, every valid page on rejected)."""
    from cvsa import ops
    q, K, V, bt, ctx = args
    idx, nph = b._cached_selection[0]
    _, cov = ops.check_coverage(b._cached_page_scores[0], idx, nph, b.tau)
    acc = b._last_accept_mask[0]
    _, (_, m, l) = ops.verified_decode(q, K, V, bt, ctx, idx, nph, acc, b.num_kv_heads,
                                       b.num_q_per_kv, 16, return_state=True)
    return cov, m + torch.log(l)


@pytest.mark.parametrize("name", sorted(SCENARIOS))
def test_hip_backend_matches_reference_trace(gpu, name):
    replay(name, lambda inp, kw: CVSABackend(inp["num_kv_heads"], inp["num_q_heads"],
                                             inp["head_dim"], 16, **kw),
           _runtime(gpu), _counters, _hip_state)


@pytest.mark.parametrize("name", sorted(SCENARIOS))
def test_hip_backend_matches_reference_trace_folded_appends(gpu, monkeypatch, name):
    """The same traces with each step's appends folded into the next call
    (CVSABackend.call_with_append, the decode loops' append-then-call order):
    a reuse step through a step plan appends in its decode launch, every
    other call appends first; all recorded quantities as above."""
    from cvsa import ops
    calls = []
    orig = ops.StepPlan.run_reuse_append

    def counted(self, *a, **k):
        calls.append(1)
        return orig(self, *a, **k)

    monkeypatch.setattr(ops.StepPlan, "run_reuse_append", counted)
    make = _runtime(gpu)

    def fused(backend, q, k_rows, v_rows):
        dev, mgr = make.runtimes[-1]
        return backend.call_with_append(q.to(dev), k_rows.to(dev).contiguous(),
                                        v_rows.to(dev).contiguous(), mgr, 0)

    replay(name, lambda inp, kw: CVSABackend(inp["num_kv_heads"], inp["num_q_heads"],
                                             inp["head_dim"], 16, **kw),
           make, _counters, _hip_state, fused_call=fused)
    if name in ("lazy_m3", "fixed_r3", "cfg1", "cfg1_mixed"):
        assert calls, (name, "no reuse step took the folded path")
