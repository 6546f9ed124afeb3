"""Quest page metadata and scores (cvsa_quest_meta_update, cvsa_quest_scores,
cvsa_quest_refresh_scores) against the oracle's restatement of CVSABackend._quest_page_scores
(cvsa/backend.py:572-620), the selection with separate ranking and gate
scores, and the backend's selector="quest" / light_normalizer schedules
against the oracle backend."""
import pytest
import torch

from oracle import cvsa_oracle as ref
from cvsa import ops
from cvsa.runtime.kv_cache import PagedKVCache, SequenceKVManager
from cvsa.synthetic import make_paged_inputs, jitter_query
from test_gpu_backend import _run

pytestmark = pytest.mark.gpu

SCORE_RTOL = 1e-5


def _close(got, want):
    fin = torch.isfinite(want)
    assert torch.equal(torch.isfinite(got), fin)
    assert torch.equal(got[~fin], want[~fin])
    err = ((got[fin] - want[fin]).abs() / want[fin].abs().clamp(min=1.0)).max().item()
    assert err < SCORE_RTOL, err


@pytest.mark.parametrize("B,H_q,H,ctx", [(2, 32, 8, [3000, 1501]), (1, 28, 4, [8191]),
                                         (3, 16, 2, [17, 530, 16]), (1, 8, 1, [5000])])
def test_quest_scores_first_build(gpu, B, H_q, H, ctx):
    inp = make_paged_inputs(B, H_q, H, 128, ctx, seed=B * 100 + H, device=gpu,
                            hot_heads=[0], n_hot=4, hot_shift=6.0)
    qm = ops.QuestPageMeta(inp.k_cache)
    got = qm.scores(inp.q, inp.block_tables, inp.context_lens, H, H_q // H, 16)
    want = ref.quest_page_scores(inp.q.cpu(), inp.k_cache.cpu(), inp.block_tables.cpu(),
                                 inp.context_lens.cpu(), H, H_q // H, 16)
    _close(got.cpu(), want)


def test_quest_meta_follows_appends(gpu):
    """Appends of 1, 3 and 17 tokens between refreshes (crossing pages), and
    a shrunken context: metadata and scores stay equal to the oracle's."""
    B, H, D = 2, 4, 128
    inp = make_paged_inputs(B, 16, H, D, [470, 33], seed=7, hot_heads=[1], n_hot=3,
                            hot_shift=5.0, spare_blocks=8, max_pages=40)
    cache = PagedKVCache(inp.k_cache.shape[0], 16, H, D, device=str(gpu))
    cache.k_cache.copy_(inp.k_cache)
    cache.v_cache.copy_(inp.v_cache)
    cache._next_free = inp.used_blocks
    mgr = SequenceKVManager(cache, B, 40 * 16)
    mgr.block_tables.copy_(inp.block_tables)
    mgr.context_lens.copy_(inp.context_lens)
    mgr._pages_allocated = [-(-int(c) // 16) for c in inp.context_lens.tolist()]
    mgr.sync_host_state()
    qm = ops.QuestPageMeta(cache.k_cache)
    # the same updates through the two separate entry points
    meta2 = torch.empty_like(qm.meta)
    ntok2 = torch.zeros_like(qm.ntok)
    g = torch.Generator().manual_seed(3)

    def check():
        q = jitter_query(inp.q, 0.5, int(mgr.context_lens.sum())).to(gpu)
        got = qm.scores(q, mgr.block_tables, mgr.context_lens, H, 4, 16).cpu()
        ops.quest_meta_update(cache.k_cache, mgr.block_tables, mgr.context_lens, meta2, ntok2)
        sep = ops.quest_scores(q, meta2, mgr.block_tables, mgr.context_lens, H, 4, 16).cpu()
        assert torch.equal(got, sep)
        assert torch.equal(ntok2, qm.ntok)
        K, bt, cl = cache.k_cache.cpu(), mgr.block_tables.cpu(), mgr.context_lens.cpu()
        _close(got, ref.quest_page_scores(q.cpu(), K, bt, cl, H, 4, 16))
        kmin, kmax = ref.page_key_minmax(K, bt, cl, 16)
        meta = qm.meta.cpu().float()
        for b in range(B):
            for p in range(-(-int(cl[b]) // 16)):
                blk = int(bt[b, p])
                assert torch.equal(meta[blk, :, 0], kmin[b, p]), (b, p)
                assert torch.equal(meta[blk, :, 1], kmax[b, p]), (b, p)
                assert torch.equal(meta2[blk].cpu(), qm.meta[blk].cpu()), (b, p)
                n = min(16, int(cl[b]) - 16 * p)
                assert bool((qm.ntok[blk] == n).all()), (b, p)

    check()
    for n in (1, 3, 17, 1, 16):
        for _ in range(n):
            mgr.append_tokens_kv(torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(gpu),
                                 torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(gpu))
        check()
    # shrink: every page up to the new length is rebuilt
    mgr.context_lens.copy_(torch.tensor([100, 20], dtype=torch.int32))
    check()


def test_quest_refresh_skips_when_every_head_passed(gpu):
    """With a lazy check's flags: nothing is written when every head passed
    (scores and metadata stay as they were); one failing head computes all."""
    B, H_q, H = 2, 32, 8
    inp = make_paged_inputs(B, H_q, H, 128, [3000, 1501], seed=12, device=gpu)
    qm = ops.QuestPageMeta(inp.k_cache)
    args = (inp.q, inp.block_tables, inp.context_lens, H, H_q // H, 16)
    W = inp.block_tables.shape[1]
    out = torch.full((B, H, W), 7.0, device=gpu)
    flags = torch.ones(B, H, dtype=torch.bool, device=gpu)
    qm.scores(*args, check_accept=flags, out=out)
    assert bool((out == 7.0).all()) and not bool(qm.ntok.any())
    flags[1, 3] = False
    got = qm.scores(*args, check_accept=flags, out=out)
    assert got is out
    want = ref.quest_page_scores(inp.q.cpu(), inp.k_cache.cpu(), inp.block_tables.cpu(),
                                 inp.context_lens.cpu(), H, H_q // H, 16)
    _close(out.cpu(), want)
    assert torch.equal(qm.scores(*args).cpu(), out.cpu())


def test_select_or_keep_with_separate_ranking_scores(gpu):
    g = torch.Generator().manual_seed(11)
    B, H, W, budget = 2, 8, 2048, 256
    ctx = torch.tensor([W * 16 - 9, 1000 * 16], dtype=torch.int32)
    gate = torch.randn(B, H, W, generator=g)
    rank = gate + 0.5 * torch.randn(B, H, W, generator=g)
    nv = ref.n_valid_pages(ctx, 16)
    gate[1, :, int(nv[1]):] = float("-inf")
    rank[1, :, int(nv[1]):] = float("-inf")
    pi = torch.empty(B, H, budget, dtype=torch.int32, device=gpu)
    nph = torch.empty(B, H, dtype=torch.int32, device=gpu)
    cov = torch.empty(B, H, device=gpu)
    cache = torch.empty(B, H, W, device=gpu)
    bad = torch.zeros(B, H, dtype=torch.bool, device=gpu)   # force a reselection
    acc = ops.select_or_keep(gate.to(gpu), bad, budget, ctx.to(gpu), 16, 0.9, pi, nph, cov,
                             cache, None, sel_scores=rank.to(gpu))
    widx, wnph = ref.select_topk(rank, budget, ctx, 16)
    wacc, wcov = ref.check_coverage(gate, widx, wnph, 0.9)
    assert torch.equal(pi.cpu(), widx) and torch.equal(nph.cpu(), wnph)
    assert (cov.cpu() - wcov).abs().max().item() < 1e-5
    margin = (wcov - 0.9).abs() > 1e-5
    assert torch.equal(acc.cpu()[margin], wacc[margin])
    assert torch.equal(cache.cpu(), gate)


CFG = dict(batch=2, num_q_heads=32, num_kv_heads=8, head_dim=128, context_len=[6000, 3500],
           hot_heads=[0, 2, 5], n_hot=8, hot_shift=9.0)


@pytest.mark.parametrize("kw", [
    dict(selector="quest", lazy=True, check_interval=3),
    dict(selector="quest", light_normalizer=True, lazy=True, check_interval=3),
    dict(selector="quest", lazy=False, reuse_interval=2),
    dict(selector="quest", light_normalizer=True, lazy=False, reuse_interval=1),
])
def test_backend_quest_schedules(gpu, kw):
    kw = dict(budget_pct=0.25, coverage_threshold=0.9, **kw)
    stats, trace, _ = _run(gpu, CFG, kw, steps=8, seed=4242)
    assert any(t["kind"].startswith("score") for t in trace)
