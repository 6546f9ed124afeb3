"""The CPU oracle against the reference implementation's own multi-step
behaviour: golden traces of the reference CVSABackend (schedule, counters,
accept masks, selected and complement page sets, outputs, append state)."""
import pytest
import torch

from golden_trace_check import SCENARIOS, replay
from oracle import cvsa_oracle as ref
from oracle.backend_oracle import OracleCVSABackend


def _oracle_backend(inp, kw):
    return OracleCVSABackend(inp["num_kv_heads"], inp["num_q_heads"], inp["head_dim"], 16, **kw)


def _oracle_runtime(case):
    K, V = case.k_cache.clone(), case.v_cache.clone()
    bt, ctx = case.block_tables.clone(), case.context_lens.clone()
    alloc = torch.tensor(case.pages_allocated, dtype=torch.int32)
    nf = [case.next_free]

    def call_args(q):
        return q, K, V, bt, ctx

    def append(b, k, v):
        nf[0] = ref.append_token_kv(K, V, bt, ctx, alloc, nf[0], b, k, v, 16)

    def state():
        return bt.numpy(), ctx.numpy()

    return call_args, append, state


def _counters(b):
    return dict(scoring=b._total_scoring_steps, checks=b._total_coverage_checks,
                accepts=b._accept_counts, rejects=b._reject_counts)


def _oracle_state(b, args):
    """Coverage of the last selection on its gate scores, and the merged
    result's LSE per q-head: the draft's on accepted heads, attention over
    every valid page (draft + complement) on rejected heads."""
    q, K, V, bt, ctx = args
    idx, nph = b._cached_selection[0]
    _, cov = ref.check_coverage(b._cached_page_scores[0], idx, nph, b.tau)
    acc = b._last_accept_mask[0]
    H, G = b.num_kv_heads, b.num_q_per_kv
    _, md, ld = ref.sparse_decode_unnorm(q, K, V, bt, idx, nph, ctx, H, G, 16)
    _, (_, ma, la) = ref.dense_decode(q, K, V, bt, ctx, H, G, 16, return_state=True)
    rej = ~acc.repeat_interleave(G, dim=1)
    lse = torch.where(rej, ma + torch.log(la), md + torch.log(ld))
    return cov, lse


@pytest.mark.parametrize("name", sorted(SCENARIOS))
def test_oracle_matches_reference_trace(name):
    replay(name, _oracle_backend, _oracle_runtime, _counters, _oracle_state)
