"""GPU parity of every HIP op (through the C ABI) against the CPU oracle.

Tolerances: page scores 1e-4 relative, coverage 1e-5,
normalised bf16 outputs max-abs 2e-2 (observed ~1e-2 or below), LSE
(m + ln l) 1e-3 relative.  Integer work (selection, complement, block
tables, append) is compared bit-exact.  Selection and accept masks are
exact on the same page scores; when compared through independently
computed scores, heads whose k-th / (k+1)-th score gap or |coverage - tau|
is below a margin are excluded and counted (the seeds keep that count 0).
"""
import pytest
import torch

from oracle import cvsa_oracle as ref
from cvsa import ops
from cvsa.synthetic import make_paged_inputs

pytestmark = pytest.mark.gpu

SCORE_RTOL = 1e-4
OUT_ATOL = 2e-2
LSE_RTOL = 1e-3
COV_ATOL = 1e-5


def _inputs(seed, B=1, H_q=32, H_kv=8, ctx=2048, W=None, **kw):
    return make_paged_inputs(B, H_q, H_kv, 128, ctx, seed=seed, max_pages=W, **kw)


def _dev(inp, d):
    return (inp.q.to(d), inp.k_cache.to(d), inp.v_cache.to(d), inp.block_tables.to(d),
            inp.context_lens.to(d))


GEOMS = [  # (B, H_q, H_kv, ctx)
    (1, 32, 8, 8192),                 # cfg1 shapes
    (3, 32, 8, [300, 1024, 17]),      # ragged batch, partial last pages
    (2, 28, 4, [2048, 1000]),         # Qwen GQA 7
    (2, 64, 8, 1500),                 # GQA 8
    (2, 8, 8, 999),                   # G = 1
    (2, 4, 2, 777),                   # G = 2, H_kv = 2
    (1, 4, 1, 640),                   # H_kv = 1
    (1, 32, 16, 512),                 # H_kv = 16
    (2, 12, 4, 321),                  # G = 3
]


@pytest.mark.parametrize("geom", GEOMS)
def test_score_pages(gpu, geom):
    B, H_q, H_kv, ctx = geom
    inp = _inputs(100, B, H_q, H_kv, ctx)
    q, K, V, bt, cl = _dev(inp, gpu)
    got = ops.score_pages(q, K, bt, cl, H_kv, H_q // H_kv, 16).cpu()
    want = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H_kv,
                           H_q // H_kv, 16)
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    err = ((got[fin] - want[fin]).abs() / want[fin].abs().clamp(min=1.0)).max().item()
    assert err < SCORE_RTOL, err


@pytest.mark.parametrize("B,H_q,H_kv,ctx", [(1, 32, 8, 65536 - 7), (1, 32, 8, 131072),
                                          (2, 28, 4, 32768 + 3)])
def test_score_pages_long_context(gpu, B, H_q, H_kv, ctx):
    """Launches with several pages per wave (2 and 8) against the oracle
    (inputs drawn on the GPU, copied to the host for the oracle)."""
    inp = make_paged_inputs(B, H_q, H_kv, 128, ctx, seed=110, device=gpu)
    q, K, bt, cl = inp.q, inp.k_cache, inp.block_tables, inp.context_lens
    got = ops.score_pages(q, K, bt, cl, H_kv, H_q // H_kv, 16).cpu()
    want = ref.score_pages(q.cpu(), K.cpu(), bt.cpu(), cl.cpu(), H_kv, H_q // H_kv, 16)
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    err = ((got[fin] - want[fin]).abs() / want[fin].abs().clamp(min=1.0)).max().item()
    assert err < SCORE_RTOL, err


def test_score_pages_block_table_wider_than_context(gpu):
    inp = _inputs(101, 2, 32, 8, [100, 5000], W=400)
    q, K, V, bt, cl = _dev(inp, gpu)
    got = ops.score_pages(q, K, bt, cl, 8, 4, 16).cpu()
    want = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, 8, 4, 16)
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    assert (got[fin] - want[fin]).abs().max().item() < 1e-4


@pytest.mark.parametrize("W,budget", [(512, 128), (8192, 1024), (37, 3), (1000, 1000),
                                      (5000, 1), (32768, 4096)])
def test_select_topk_bit_exact(gpu, W, budget):
    g = torch.Generator().manual_seed(W + budget)
    B, H = 2, 4
    ps = torch.randn(B, H, W, generator=g)
    ps[0, 1] = (ps[0, 1] * 2).round() / 2          # heavy ties
    ctx = torch.tensor([W * 16, max(1, (W // 3) * 16 - 5)], dtype=torch.int32)
    nv = ref.n_valid_pages(ctx, 16)
    ps[1, :, int(nv[1]):] = float("-inf")
    idx, nph, acc, cov = ops.select_topk(ps.to(gpu), budget, ctx.to(gpu), 16, tau=0.9)
    widx, wnph = ref.select_topk(ps, budget, ctx, 16)
    assert torch.equal(idx.cpu(), widx)
    assert torch.equal(nph.cpu(), wnph)
    wacc, wcov = ref.check_coverage(ps, widx, wnph, 0.9)
    assert (cov.cpu() - wcov).abs().max().item() < COV_ATOL
    margin = (wcov - 0.9).abs() > 1e-5
    assert torch.equal(acc.cpu()[margin], wacc[margin])


@pytest.mark.parametrize("W,budget", [(8192, 1024), (20000, 2500)])
def test_select_topk_special_rows(gpu, W, budget):
    """One row per path of the selection: all scores equal, +0/-0 mixed
    (equal scores), one huge outlier (the k-th bucket overflows the rank
    step), a value range whose width overflows fp32, +inf and NaN entries,
    near-ties packed into one bucket, and fewer finite scores than the
    budget."""
    g = torch.Generator().manual_seed(W)
    rows = []
    rows.append(torch.full((W,), 1.25))
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
    ps = torch.stack(rows).view(1, len(rows), W)
    ctx = torch.tensor([W * 16], dtype=torch.int32)
    idx, nph, acc, cov = ops.select_topk(ps.to(gpu), budget, ctx.to(gpu), 16, tau=0.9)
    widx, wnph = ref.select_topk(ps, budget, ctx, 16)
    for h in range(len(rows)):
        assert torch.equal(idx.cpu()[0, h], widx[0, h]), h
    assert torch.equal(nph.cpu(), wnph)
    finite_rows = [0, 1, 2, 5]
    wacc, wcov = ref.check_coverage(ps, widx, wnph, 0.9)
    assert (cov.cpu()[0, finite_rows] - wcov[0, finite_rows]).abs().max().item() < COV_ATOL


@pytest.mark.parametrize("W,budget", [(2048, 512), (8192, 1024), (100, 3)])
def test_select_or_keep(gpu, W, budget):
    """Keep the cached selection when every head passed, else refresh it in
    place exactly as select_topk; counters as the lazy schedule counts them."""
    g = torch.Generator().manual_seed(W * 3 + budget)
    B, H = 2, 8
    ctx = torch.tensor([W * 16 - 3, max(1, (W // 2) * 16)], dtype=torch.int32)
    old_ps = torch.randn(B, H, W, generator=g)
    new_ps = torch.randn(B, H, W, generator=g)
    nv = ref.n_valid_pages(ctx, 16)
    new_ps[1, :, int(nv[1]):] = float("-inf")
    sel0, nph0 = ref.select_topk(old_ps, budget, ctx, 16)
    stats = torch.zeros(6, dtype=torch.int64, device=gpu)
    d_sel, d_nph = sel0.to(gpu), nph0.to(gpu)
    d_cache = old_ps.to(gpu)
    cov = torch.full((B, H), -7.0, device=gpu)
    # 1) every head passed: nothing changes, all heads accepted
    check = torch.ones(B, H, dtype=torch.bool, device=gpu)
    acc = ops.select_or_keep(new_ps.to(gpu), check, budget, ctx.to(gpu), 16, 0.9, d_sel, d_nph,
                             cov, d_cache, stats)
    assert bool(acc.all())
    assert torch.equal(d_sel.cpu(), sel0) and torch.equal(d_nph.cpu(), nph0)
    assert torch.equal(d_cache.cpu(), old_ps) and bool((cov == -7.0).all())
    assert stats.tolist() == [1, 0, 0, B * H, 0, 0]
    # 2) one head failed: fresh top-k + gate for every head, scores cached
    check[1, 3] = False
    acc = ops.select_or_keep(new_ps.to(gpu), check, budget, ctx.to(gpu), 16, 0.9, d_sel, d_nph,
                             cov, d_cache, stats)
    widx, wnph = ref.select_topk(new_ps, budget, ctx, 16)
    assert torch.equal(d_sel.cpu(), widx) and torch.equal(d_nph.cpu(), wnph)
    assert torch.equal(d_cache.cpu(), new_ps)
    wacc, wcov = ref.check_coverage(new_ps, widx, wnph, 0.9)
    assert (cov.cpu() - wcov).abs().max().item() < COV_ATOL
    margin = (wcov - 0.9).abs() > 1e-5
    assert torch.equal(acc.cpu()[margin], wacc[margin])
    assert stats.tolist() == [1, 1, 1, 2 * B * H - 1, 0, 0]
    # 3) a fresh selection booked by its own gate (fixed-interval schedule)
    sel3 = torch.empty_like(d_sel)
    nph3 = torch.empty_like(d_nph)
    cov3 = torch.empty_like(cov)
    acc3 = ops.select_or_keep(new_ps.to(gpu), None, budget, ctx.to(gpu), 16, 0.9, sel3, nph3,
                              cov3, None, stats, count_gate=True)
    assert torch.equal(sel3.cpu(), widx) and torch.equal(acc3, acc)
    n_acc = int(acc3.sum())
    all_acc = int(n_acc == B * H)
    assert stats.tolist() == [1 + all_acc, 2 - all_acc, 2, 2 * B * H - 1 + n_acc, 0, 0]


@pytest.mark.parametrize("k,W", [(128, 512), (1000, 2048), (5, 9)])
def test_check_coverage(gpu, k, W):
    g = torch.Generator().manual_seed(k * 7 + W)
    B, H = 3, 8
    ps = torch.randn(B, H, W, generator=g) * 2
    sel = torch.stack([torch.stack([torch.randperm(W, generator=g)[:k] for _ in range(H)])
                       for _ in range(B)]).to(torch.int32)
    nph = torch.randint(0, k + 1, (B, H), generator=g).to(torch.int32)
    for tau in (0.0, 0.5, 0.9):
        acc, cov = ops.check_coverage(ps.to(gpu), sel.to(gpu), nph.to(gpu), tau)
        wacc, wcov = ref.check_coverage(ps, sel, nph, tau)
        assert (cov.cpu() - wcov).abs().max().item() < COV_ATOL
        margin = (wcov - tau).abs() > 1e-5
        assert torch.equal(acc.cpu()[margin], wacc[margin])


def _check_state(o, m, l, wo, wm, wl):
    fin = torch.isfinite(wm)
    assert torch.equal(torch.isfinite(m), fin)
    if fin.any():
        lse = m[fin] + torch.log(l[fin])
        wlse = wm[fin] + torch.log(wl[fin])
        assert ((lse - wlse).abs() / wlse.abs().clamp(min=1.0)).max().item() < LSE_RTOL
        on = o / l.clamp(min=1e-30).unsqueeze(-1)
        won = wo / wl.clamp(min=1e-30).unsqueeze(-1)
        assert (on[fin] - won[fin]).abs().max().item() < 1e-3
    assert float(l[~fin].abs().max()) == 0.0 if (~fin).any() else True


@pytest.mark.parametrize("geom", GEOMS)
def test_sparse_decode_unnorm_and_norm(gpu, geom):
    B, H_q, H_kv, ctx = geom
    G = H_q // H_kv
    inp = _inputs(200, B, H_q, H_kv, ctx)
    q, K, V, bt, cl = _dev(inp, gpu)
    ps = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H_kv, G, 16)
    W = inp.block_tables.shape[1]
    budget = max(3, W // 4)
    idx, nph = ref.select_topk(ps, min(budget, W), inp.context_lens, 16)
    o, m, l = ops.sparse_decode_unnorm(q, K, V, bt, idx.to(gpu), nph.to(gpu), cl, H_kv, G, 16)
    wo, wm, wl = ref.sparse_decode_unnorm(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                          idx, nph, inp.context_lens, H_kv, G, 16)
    _check_state(o.cpu(), m.cpu(), l.cpu(), wo, wm, wl)
    out = ops.sparse_decode(q, K, V, bt, idx.to(gpu), nph.to(gpu), cl, H_kv, G, 16)
    wout = ref.normalise(wo, wl, torch.bfloat16)
    assert out.dtype == torch.bfloat16
    assert (out.cpu().float() - wout.float()).abs().max().item() < OUT_ATOL


def test_sparse_decode_edge_cases(gpu):
    """Empty selections, out-of-range ids, pages past the context, duplicates."""
    inp = _inputs(201, 2, 32, 8, [700, 40], W=64)
    q, K, V, bt, cl = _dev(inp, gpu)
    idx = torch.zeros(2, 8, 6, dtype=torch.int32)
    idx[:, :, :] = torch.tensor([0, 3, 63, 2, 2, -5], dtype=torch.int32)
    nph = torch.tensor([[0, 1, 2, 3, 4, 5, 6, 6], [6, 5, 4, 3, 2, 1, 0, 6]], dtype=torch.int32)
    o, m, l = ops.sparse_decode_unnorm(q, K, V, bt, idx.to(gpu), nph.to(gpu), cl, 8, 4, 16)
    wo, wm, wl = ref.sparse_decode_unnorm(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                          idx, nph, inp.context_lens, 8, 4, 16)
    _check_state(o.cpu(), m.cpu(), l.cpu(), wo, wm, wl)
    out = ops.sparse_decode(q, K, V, bt, idx.to(gpu), nph.to(gpu), cl, 8, 4, 16).cpu()
    empty = ~torch.isfinite(wm)
    assert float(out.float()[empty].abs().max()) == 0.0


@pytest.mark.parametrize("geom", GEOMS[:6])
def test_dense_decode(gpu, geom):
    B, H_q, H_kv, ctx = geom
    G = H_q // H_kv
    inp = _inputs(300, B, H_q, H_kv, ctx)
    q, K, V, bt, cl = _dev(inp, gpu)
    out, (o, m, l) = ops.dense_decode(q, K, V, bt, cl, H_kv, G, 16, return_state=True)
    wout, (wo, wm, wl) = ref.dense_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                          inp.context_lens, H_kv, G, 16, return_state=True)
    _check_state(o.cpu(), m.cpu(), l.cpu(), wo, wm, wl)
    assert (out.cpu().float() - wout.float()).abs().max().item() < OUT_ATOL


@pytest.mark.parametrize("geom", GEOMS[:5])
def test_verified_decode_matches_reference_recovery(gpu, geom):
    """Fused verified decode vs the reference's draft + complement + merge."""
    B, H_q, H_kv, ctx = geom
    G = H_q // H_kv
    inp = _inputs(400, B, H_q, H_kv, ctx)
    q, K, V, bt, cl = _dev(inp, gpu)
    ps = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H_kv, G, 16)
    W = inp.block_tables.shape[1]
    idx, nph = ref.select_topk(ps, max(3, W // 8), inp.context_lens, 16)
    g = torch.Generator().manual_seed(1)
    accept = torch.rand(B, H_kv, generator=g) > 0.5
    out = ops.verified_decode(q, K, V, bt, cl, idx.to(gpu), nph.to(gpu), accept.to(gpu), H_kv,
                              G, 16)
    want = ref.verified_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                               inp.context_lens, idx, nph, accept, H_kv, G, 16)
    assert (out.cpu().float() - want.float()).abs().max().item() < OUT_ATOL


@pytest.mark.parametrize("geom", GEOMS[:5] + [GEOMS[6]])
@pytest.mark.parametrize("pattern", ["mixed", "all_rejected", "all_accepted"])
def test_verified_decode_approx_matches_reference(gpu, geom, pattern):
    """Approximate recovery in one launch (cvsa_verified_decode_approx) vs
    the reference's branch (backend.py:775-817) restated with the oracle:
    accepted heads = normalised draft over the selection, rejected heads =
    normalised sparse decode of the expanded top-k's first min(exp_budget,
    n_valid) pages; (o, m, l) of every head, and the effective-budget
    counters as the reference books them (n_per_head, plus min(exp_budget,
    n_valid) on every head when some head is rejected)."""
    B, H_q, H_kv, ctx = geom
    G = H_q // H_kv
    inp = _inputs(410, B, H_q, H_kv, ctx, hot_heads=list(range(0, H_kv, 2)), n_hot=6,
                  hot_shift=9.0)
    q, K, V, bt, cl = _dev(inp, gpu)
    ps = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H_kv, G, 16)
    W = inp.block_tables.shape[1]
    budget = max(3, W // 8)
    exp_budget = min(max(budget + 1, int(W * 0.3)), W)
    idx, nph = ref.select_topk(ps, budget, inp.context_lens, 16)
    exp, exp_n = ref.select_topk(ps, exp_budget, inp.context_lens, 16)
    g = torch.Generator().manual_seed(2)
    accept = {"mixed": torch.rand(B, H_kv, generator=g) > 0.5,
              "all_rejected": torch.zeros(B, H_kv, dtype=torch.bool),
              "all_accepted": torch.ones(B, H_kv, dtype=torch.bool)}[pattern]
    work = torch.zeros(2, dtype=torch.int64, device=gpu)
    out, (o, m, l) = ops.verified_decode_approx(
        q, K, V, bt, cl, idx.to(gpu), nph.to(gpu), accept.to(gpu), exp.to(gpu), H_kv, G, 16,
        return_state=True, work=work)
    wd = ref.sparse_decode_unnorm(inp.q, inp.k_cache, inp.v_cache, inp.block_tables, idx, nph,
                                  inp.context_lens, H_kv, G, 16)
    we = ref.sparse_decode_unnorm(inp.q, inp.k_cache, inp.v_cache, inp.block_tables, exp,
                                  exp_n, inp.context_lens, H_kv, G, 16)
    acc_q = accept.repeat_interleave(G, dim=1)
    wo = torch.where(acc_q.unsqueeze(-1), wd[0], we[0])
    wm = torch.where(acc_q, wd[1], we[1])
    wl = torch.where(acc_q, wd[2], we[2])
    _check_state(o.cpu(), m.cpu(), l.cpu(), wo, wm, wl)
    want = torch.where(acc_q.unsqueeze(-1), ref.normalise(wd[0], wd[2], torch.float64),
                       ref.normalise(we[0], we[2], torch.float64)).to(torch.bfloat16)
    assert (out.cpu().float() - want.float()).abs().max().item() < OUT_ATOL
    nv = ref.n_valid_pages(inp.context_lens, 16)
    booked = int(nph.sum())
    if not bool(accept.all()):
        booked += int(exp_n.sum())
    assert work.tolist() == [booked, int(nv.sum()) * H_kv]


def test_compute_complement_exact(gpu):
    g = torch.Generator().manual_seed(9)
    B, H, k = 3, 8, 20
    ctx = torch.tensor([16 * 64, 16 * 10 + 3, 16 * 64 - 1], dtype=torch.int32)
    idx = torch.randint(-2, 70, (B, H, k), generator=g).to(torch.int32)
    nph = torch.randint(0, k + 1, (B, H), generator=g).to(torch.int32)
    acc = torch.rand(B, H, generator=g) > 0.6
    comp, n = ops.compute_complement(idx.to(gpu), nph.to(gpu), ctx.to(gpu), 16, acc.to(gpu))
    wcomp, wn = ref.compute_complement(idx, nph, ctx, 16, acc)
    assert torch.equal(n.cpu(), wn) and torch.equal(comp.cpu(), wcomp)
    from cvsa.complement import compute_complement_pages
    c2, n2 = compute_complement_pages(idx.to(gpu), nph.to(gpu), ctx.to(gpu), 16, acc.to(gpu))
    wc2, wn2 = ref.compute_complement_pages(idx, nph, ctx, 16, acc)
    assert torch.equal(n2.cpu(), wn2) and torch.equal(c2.cpu(), wc2)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_lse_merge(gpu, out_dtype):
    g = torch.Generator().manual_seed(4)
    B, H_kv, G, D = 3, 8, 4, 128
    od, oc = torch.randn(B, H_kv * G, D, generator=g), torch.randn(B, H_kv * G, D, generator=g)
    md, mc = torch.randn(B, H_kv * G, generator=g), torch.randn(B, H_kv * G, generator=g)
    ld, lc = torch.rand(B, H_kv * G, generator=g) + .1, torch.rand(B, H_kv * G, generator=g) + .1
    mc[0, :4] = float("-inf")
    lc[0, :4] = 0.0
    acc = torch.rand(B, H_kv, generator=g) > 0.5
    args = [t.to(gpu) for t in (od, md, ld, oc, mc, lc, acc)]
    got = ops.lse_merge(*args, H_kv, G, out_dtype).cpu()
    want = ref.lse_merge(od, md, ld, oc, mc, lc, acc, G, out_dtype)
    tol = 1e-5 if out_dtype == torch.float32 else 1e-2
    assert (got.float() - want.float()).abs().max().item() < tol
    from cvsa.lse_merge import selective_lse_merge
    got2 = selective_lse_merge(*args, G, out_dtype).cpu()
    assert torch.equal(got2, got)


@pytest.mark.parametrize("D,bs", [(128, 16), (64, 16), (256, 16), (128, 32), (64, 64)])
def test_append_kv_matches_reference_loop(gpu, D, bs):
    from cvsa.runtime.kv_cache import PagedKVCache, SequenceKVManager
    B, H = 5, 8
    cache = PagedKVCache(64, bs, H, D, device=str(gpu))
    mgr = SequenceKVManager(cache, B, bs * 8)
    g = torch.Generator().manual_seed(2)
    lens = [15, 16, 0, 33, 47]
    for b, n in enumerate(lens):
        if n:
            kv = torch.randn(n, H, D, generator=g).to(torch.bfloat16)
            mgr.prefill_kv(b, kv.to(gpu), (-kv).to(gpu))
    # CPU oracle copy of the state
    K = cache.k_cache.cpu().clone()
    V = cache.v_cache.cpu().clone()
    bt = mgr.block_tables.cpu().clone()
    ctx = mgr.context_lens.cpu().clone()
    alloc = torch.tensor(mgr._pages_allocated, dtype=torch.int32)
    nf = cache._next_free
    for step in range(20):
        kn = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
        vn = torch.randn(B, H, D, generator=g).to(torch.bfloat16)
        if step % 3 == 0:
            mgr.append_token_kv(1, kn[1].to(gpu), vn[1].to(gpu))
            nf = ref.append_token_kv(K, V, bt, ctx, alloc, nf, 1, kn[1], vn[1], bs)
        else:
            mgr.append_tokens_kv(kn.to(gpu), vn.to(gpu))
            for b in range(B):
                nf = ref.append_token_kv(K, V, bt, ctx, alloc, nf, b, kn[b], vn[b], bs)
    assert cache._next_free == nf
    assert torch.equal(mgr.block_tables.cpu(), bt)
    assert torch.equal(mgr.context_lens.cpu(), ctx)
    assert mgr._ctx_host == ctx.tolist()
    assert torch.equal(cache.k_cache.cpu(), K) and torch.equal(cache.v_cache.cpu(), V)


def test_ops_reject_bad_input(gpu):
    inp = _inputs(500, 1, 32, 8, 256)
    q, K, V, bt, cl = _dev(inp, gpu)
    with pytest.raises(ValueError):
        ops.score_pages(q.cpu(), K, bt, cl, 8, 4, 16)
    with pytest.raises(NotImplementedError):
        ops.score_pages(q[:, :, :96].contiguous(), K[..., :96].contiguous(), bt, cl, 8, 4, 16)
    with pytest.raises(ValueError):
        ops.select_topk(torch.zeros(1, 8, 16, device=gpu), 17, cl, 16)


@pytest.mark.parametrize("extra", [2, 16])
def test_verified_decode_block_table_wider_than_context(gpu, extra):
    """Rejected heads walk n_valid pages with their own split size even when
    the block table is wider than the context (regression: a miscompiled
    branch once gave rejected heads the listed heads' split size)."""
    inp = _inputs(410, 1, 32, 8, 8192, W=512 + extra)
    q, K, V, bt, cl = _dev(inp, gpu)
    ps = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, 8, 4, 16)
    idx, nph = ref.select_topk(ps, 64, inp.context_lens, 16)
    accept = torch.tensor([[False, False, True, False, True, False, True, False]])
    out = ops.verified_decode(q, K, V, bt, cl, idx.to(gpu), nph.to(gpu), accept.to(gpu), 8, 4,
                              16).cpu()
    want = ref.verified_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                               inp.context_lens, idx, nph, accept, 8, 4, 16)
    assert (out.float() - want.float()).abs().max().item() < OUT_ATOL
    dense = ops.dense_decode(q, K, V, bt, cl, 8, 4, 16).cpu()
    rej = ~accept.repeat_interleave(4, dim=1)[0]
    # Same pages, possibly other split sizes: equal up to fp32 summation order.
    assert (out[0][rej].float() - dense[0][rej].float()).abs().max().item() < 8e-3


def _torch_attention(q, K, V, bt, cl, pages, h, G):
    """fp32 softmax attention of the G q-heads of KV head h of sequence 0 over
    logical `pages` (torch on the GPU; reference for long contexts)."""
    phys = bt[0, pages].long()
    k = K[phys, :, h].float().reshape(-1, 128)
    v = V[phys, :, h].float().reshape(-1, 128)
    tok = (pages[:, None] * 16 + torch.arange(16, device=q.device)[None]).reshape(-1)
    s = q[0, h * G:(h + 1) * G].float() @ k.T * 128 ** -0.5
    s[:, tok >= cl[0]] = -float("inf")
    m = s.max(dim=1).values
    p = torch.exp(s - m[:, None])
    l = p.sum(dim=1)
    return (p @ v) / l[:, None], m + torch.log(l)


@pytest.mark.parametrize("ctx,budget", [(65536 - 5, 512), (131072, 1024)])
def test_decode_many_splits(gpu, ctx, budget):
    """Long contexts: rejected heads of a verified launch and every head of a
    dense launch spread over up to 256 splits (merged from as many partials)."""
    H, G = 8, 4
    inp = make_paged_inputs(1, 32, H, 128, ctx, seed=420, device=gpu, hot_heads=[0, 3],
                            n_hot=16, hot_shift=8.0)
    q, K, V, bt, cl = inp.q, inp.k_cache, inp.v_cache, inp.block_tables, inp.context_lens
    ps = ops.score_pages(q, K, bt, cl, H, G, 16)
    idx, nph = ops.select_topk(ps, budget, cl, 16)
    accept = torch.tensor([[True, False, True, True, False, True, False, True]], device=gpu)
    out, (o, m, l) = ops.verified_decode(q, K, V, bt, cl, idx, nph, accept, H, G, 16,
                                         return_state=True, output_dtype=torch.float32)
    dense, (do, dm, dl) = ops.dense_decode(q, K, V, bt, cl, H, G, 16, return_state=True)
    n_valid = (ctx - 1) // 16 + 1
    every = torch.arange(n_valid, device=gpu)
    for h in range(H):
        pages = idx[0, h, :nph[0, h]].long() if bool(accept[0, h]) else every
        want, want_lse = _torch_attention(q, K, V, bt, cl, pages, h, G)
        rows = slice(h * G, (h + 1) * G)
        assert (out[0, rows] - want).abs().max().item() < 1e-3, h
        lse = m[0, rows] + torch.log(l[0, rows])
        assert ((lse - want_lse).abs() / want_lse.abs().clamp(min=1.0)).max().item() < LSE_RTOL
        dwant, dwant_lse = _torch_attention(q, K, V, bt, cl, every, h, G)
        assert (dense[0, rows].float() - dwant).abs().max().item() < OUT_ATOL, h
        dlse = dm[0, rows] + torch.log(dl[0, rows])
        assert ((dlse - dwant_lse).abs() / dwant_lse.abs().clamp(min=1.0)).max().item() < LSE_RTOL


@pytest.mark.parametrize("rejected", [0, 3, 7])
def test_verified_decode_uneven_walks_with_the_uniform_total(gpu, rejected):
    """A verified launch whose heads walk max_sel pages in total on average
    but not each: one rejected head walks all 1024 valid pages, the seven
    accepted heads walk none, and 8 x max_sel = 1024 as well.  Regression:
    the stream-K kernel took a matching total for "every head walks max_sel
    pages", started workgroups at the wrong head and skipped pages of the
    rejected head (which pages depended on the head's index).  Every head is
    compared with torch attention over its pages."""
    H, G, ctx, budget = 8, 4, 16 * 1024, 128
    inp = make_paged_inputs(1, 32, H, 128, ctx, seed=431, device=gpu, hot_heads=[rejected],
                            n_hot=8, hot_shift=6.0)
    q, K, V, bt, cl = inp.q, inp.k_cache, inp.v_cache, inp.block_tables, inp.context_lens
    idx = torch.zeros(1, H, budget, dtype=torch.int32, device=gpu)
    nph = torch.zeros(1, H, dtype=torch.int32, device=gpu)
    accept = torch.ones(1, H, dtype=torch.bool, device=gpu)
    accept[0, rejected] = False
    out, (o, m, l) = ops.verified_decode(q, K, V, bt, cl, idx, nph, accept, H, G, 16,
                                         return_state=True, output_dtype=torch.float32)
    every = torch.arange(1024, device=gpu)
    for h in range(H):
        rows = slice(h * G, (h + 1) * G)
        if h != rejected:
            assert bool((out[0, rows] == 0).all()) and bool((l[0, rows] == 0).all()), h
            continue
        want, want_lse = _torch_attention(q, K, V, bt, cl, every, h, G)
        assert (out[0, rows] - want).abs().max().item() < 1e-3, h
        lse = m[0, rows] + torch.log(l[0, rows])
        assert ((lse - want_lse).abs() / want_lse.abs().clamp(min=1.0)).max().item() < LSE_RTOL


def test_prepare_reuse_state_then_reuse_decode(gpu):
    """prepare_reuse_state (sparse_decode.py:664-678) pads a width-100
    selection to 128 with page 0; sparse_decode_reuse (:681-721) on that
    state attends only each row's first n_per_head pages.  Some heads have
    n_per_head below the budget (one is empty); both steps are compared with
    the oracle (the state exactly, the output to the bf16 tolerance)."""
    B, H, G = 2, 8, 4
    inp = _inputs(440, B, 32, H, [4000, 2500], W=256)
    q, K, V, bt, cl = _dev(inp, gpu)
    ps = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H, G, 16)
    idx, nph = ref.select_topk(ps, 100, inp.context_lens, 16)
    nph[0, 3] = 37
    nph[1, 5] = 0
    nph[1, 6] = 99
    pi, n, padded = ops.prepare_reuse_state(idx.to(gpu), nph.to(gpu), H, B)
    wpi, wn, wpadded = ref.prepare_reuse_state(idx, nph, H, B)
    assert padded == wpadded == 128
    assert torch.equal(pi.cpu(), wpi) and torch.equal(n.cpu(), wn)
    out = ops.sparse_decode_reuse(q, K, V, bt, cl, pi, n, padded, H, G, 16).cpu()
    want = ref.sparse_decode_reuse(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                   inp.context_lens, wpi, wn, wpadded, H, G, 16)
    assert out.dtype == torch.bfloat16
    assert (out.float() - want.float()).abs().max().item() < OUT_ATOL
    assert float(out[1, 5 * G:6 * G].float().abs().max()) == 0.0   # empty head


def test_group_mean_matches_torch_gpu_mean(gpu):
    """The reference forms q_rep with torch's mean on the GPU
    (page_scores.py:94-95); the oracle's bf16(fp32 sum x fp32(1/G)) equals it
    bit for bit for every group size, G = 7 included (torch's CPU mean
    divides instead, and differs there)."""
    g = torch.Generator().manual_seed(441)
    for G in range(1, 9):
        q = torch.randn(16, 8 * G, 128, generator=g).to(torch.bfloat16)
        got = q.to(gpu).view(16, 8, G, 128).mean(dim=2).cpu()
        assert torch.equal(ref.group_mean_bf16(q, 8, G), got), G


def test_workspace_shared_across_head_counts(gpu):
    """Decode launches of different B * H_kv share one workspace on one
    stream: a split listed decode at B=1, H_kv=8, W=8192 (256 partial rows)
    followed by a verified decode at B=16, H_kv=8, 8K context (128 heads,
    stream-K), and then the listed decode again.  Regression: the counter
    area was sized per launch, so the second launch read the first one's
    partial rows as the counters of heads 64..127, skipped their merges and
    left their outputs unwritten.  Both launches are compared with the
    oracle."""
    ops._WORKSPACES.clear()       # the first launch below sizes the workspace
    H, G = 8, 4
    big = make_paged_inputs(1, 32, H, 128, 131072, seed=430, device=gpu, hot_heads=[1, 5],
                            n_hot=16, hot_shift=8.0)
    ps = ops.score_pages(big.q, big.k_cache, big.block_tables, big.context_lens, H, G, 16)
    idx, nph = ops.select_topk(ps, 1024, big.context_lens, 16)
    small = _inputs(431, 16, 32, H, 8192)
    sq, sK, sV, sbt, scl = _dev(small, gpu)
    sps = ref.score_pages(small.q, small.k_cache, small.block_tables, small.context_lens, H, G,
                          16)
    sidx, snph = ref.select_topk(sps, 128, small.context_lens, 16)
    g = torch.Generator().manual_seed(432)
    sacc = torch.rand(16, H, generator=g) > 0.3
    swant = ref.verified_decode(small.q, small.k_cache, small.v_cache, small.block_tables,
                                small.context_lens, sidx, snph, sacc, H, G, 16)
    bq, bK, bV, bbt, bcl = (t.cpu() for t in (big.q, big.k_cache, big.v_cache,
                                              big.block_tables, big.context_lens))
    bwant = ref.sparse_decode(bq, bK, bV, bbt, idx.cpu(), nph.cpu(), bcl, H, G, 16)

    def listed():
        return ops.sparse_decode(big.q, big.k_cache, big.v_cache, big.block_tables, idx, nph,
                                 big.context_lens, H, G, 16).cpu()

    def verified():
        return ops.verified_decode(sq, sK, sV, sbt, scl, sidx.to(gpu), snph.to(gpu),
                                   sacc.to(gpu), H, G, 16).cpu()

    first = listed()
    ws = ops._WORKSPACES[(gpu.index, ops._stream(gpu))]
    second = verified()
    assert ops._WORKSPACES[(gpu.index, ops._stream(gpu))] is ws   # the same workspace
    third = listed()
    for got, want in ((first, bwant), (second, swant), (third, bwant)):
        assert (got.float() - want.float()).abs().max().item() < OUT_ATOL
    assert torch.equal(first, third)


def test_append_prepared_and_converting_paths_agree(gpu):
    """SequenceKVManager appends bf16 rows through a prepared launch
    (ops.AppendCall) and other dtypes through ops.append_kv: the same
    tokens give the same caches, tables and lengths either way, across page
    boundaries; the prepared call rejects rows that do not fit it."""
    from cvsa.runtime.kv_cache import PagedKVCache, SequenceKVManager
    B, H, D = 3, 8, 128
    caches, mgrs = [], []
    for _ in range(2):
        c = PagedKVCache(32, 16, H, D, device=str(gpu))
        m = SequenceKVManager(c, B, 16 * 6)
        caches.append(c)
        mgrs.append(m)
    g = torch.Generator().manual_seed(8)
    for step in range(40):
        k = torch.randn(B, H, D, generator=g).to(gpu)
        v = torch.randn(B, H, D, generator=g).to(gpu)
        mgrs[0].append_tokens_kv(k.to(torch.bfloat16), v.to(torch.bfloat16))   # prepared
        mgrs[1].append_tokens_kv(k, v)                                         # converting
        if step % 7 == 3:   # a single sequence through the prepared call
            kb = torch.randn(H, D, generator=g).to(torch.bfloat16).to(gpu)
            mgrs[0].append_token_kv(1, kb, kb)
            mgrs[1].append_token_kv(1, kb.float(), kb.float())
    assert mgrs[0]._append_call is not None and mgrs[1]._append_call is None
    for a, b in ((caches[0].k_cache, caches[1].k_cache), (caches[0].v_cache, caches[1].v_cache),
                 (mgrs[0].block_tables, mgrs[1].block_tables),
                 (mgrs[0].context_lens, mgrs[1].context_lens)):
        assert torch.equal(a, b)
    call = mgrs[0]._append_call
    bad = torch.zeros(B, H, D - 1, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        call.run(bad, bad, 0, caches[0]._next_free)
    ok = torch.zeros(2, H, D, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):   # rows past the batch
        call.run(ok, ok, 2, caches[0]._next_free)
