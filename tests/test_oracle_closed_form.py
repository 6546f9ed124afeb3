"""Pin the CPU oracle with what the mathematics fixes.

Brute force on tiny inputs, closed forms (all pages selected = textbook
softmax attention), invariants (draft + complement = dense, coverage = 1 for
a full selection) and the rounding rule of the bf16 group mean, at head
dimensions 32, 64, 128, 256 and block sizes 8, 16, 32, 64, 128 where they
depend on them.  A few tests
plant a plausible mistake in a copy of the oracle and show the checks fail.
"""
import math

import pytest
import torch

from oracle import cvsa_oracle as ref
from cvsa.synthetic import make_paged_inputs


# (head dimension, block size): the kernels' geometries.  Contexts scale with
# the block size so that every geometry has full, partial and missing pages.
GEOMETRIES = [(128, 16), (64, 32), (256, 64), (32, 8), (128, 128)]


def _tiny(seed=0, B=2, H_q=8, H_kv=2, ctx=(70, 33), W=6, D=128, bs=16):
    ctx = [c * bs // 16 for c in ctx]
    return make_paged_inputs(B, H_q, H_kv, D, ctx, block_size=bs, seed=seed, max_pages=W,
                             hot_heads=[0], n_hot=1, hot_shift=2.0)


def _brute_scores(inp):
    """Per (b, h, p, t) loops in float64."""
    q, K, bt, ctx = inp.q, inp.k_cache, inp.block_tables, inp.context_lens
    B, H_q, D = q.shape
    H, G, bs = inp.num_kv_heads, inp.num_q_per_kv, inp.block_size
    W = bt.shape[1]
    scale = ref.fp32_scale(D)
    out = torch.full((B, H, W), float("-inf"))
    for b in range(B):
        for h in range(H):
            qr = torch.zeros(D)
            for g in range(G):
                qr += q[b, h * G + g].float()
            qr = (qr * torch.tensor(1.0 / G, dtype=torch.float32)).to(torch.bfloat16).double()
            for p in range(W):
                if p * bs >= int(ctx[b]):
                    continue
                best = -math.inf
                for t in range(bs):
                    if p * bs + t >= int(ctx[b]):
                        break
                    s = float(torch.dot(K[int(bt[b, p]), t, h].double(), qr))
                    best = max(best, float(torch.tensor(s, dtype=torch.float32) * scale))
                out[b, h, p] = best
    return out


@pytest.mark.parametrize("D,bs", GEOMETRIES)
def test_score_pages_brute_force(D, bs):
    inp = _tiny(D=D, bs=bs)
    got = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens,
                          inp.num_kv_heads, inp.num_q_per_kv, inp.block_size)
    want = _brute_scores(inp)
    assert torch.equal(torch.isinf(got), torch.isinf(want))
    fin = torch.isfinite(want)
    assert (got[fin] - want[fin]).abs().max().item() < 1e-6


def test_group_mean_matches_torch_mean_for_power_of_two_groups():
    g = torch.Generator().manual_seed(3)
    for G in (1, 2, 4, 8):
        q = torch.randn(3, 4 * G, 128, generator=g).to(torch.bfloat16)
        a = ref.group_mean_bf16(q, 4, G)
        b = q.view(3, 4, G, 128).mean(dim=2)
        assert torch.equal(a, b), G


def test_prepare_reuse_state_pads_to_a_power_of_two_with_page_zero():
    """sparse_decode.py:664-678: width 100 pads to 128 with page 0; a width
    that is already a power of two is kept; rows flatten head-major."""
    g = torch.Generator().manual_seed(11)
    for k, want in ((100, 128), (128, 128), (3, 4), (1, 1)):
        idx = torch.randint(1, 50, (2, 3, k), generator=g).to(torch.int32)
        nph = torch.randint(0, k + 1, (2, 3), generator=g).to(torch.int32)
        pi, n, padded = ref.prepare_reuse_state(idx, nph, 3, 2)
        assert padded == want and pi.shape == (6, want) and pi.dtype == torch.int32
        for b in range(2):
            for h in range(3):
                assert pi[b * 3 + h, :k].tolist() == idx[b, h].tolist()
                assert pi[b * 3 + h, k:].tolist() == [0] * (want - k)
                assert int(n[b * 3 + h]) == int(nph[b, h])


@pytest.mark.parametrize("D,bs", GEOMETRIES)
def test_reuse_decode_of_padded_state_equals_unpadded_decode(D, bs):
    """The padding is never read: decoding a prepared state gives exactly the
    decode of the unpadded selection, on rows with n_per_head below the
    width, an empty row and a full row."""
    inp = _tiny(seed=12, ctx=(90, 60), W=6, D=D, bs=bs)
    idx = torch.tensor([[[5, 0, 2], [1, 3, 4]], [[2, 1, 0], [3, 0, 1]]], dtype=torch.int32)
    nph = torch.tensor([[1, 3], [0, 2]], dtype=torch.int32)
    want = ref.sparse_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables, idx, nph,
                             inp.context_lens, 2, 4, bs)
    pi, n, padded = ref.prepare_reuse_state(idx, nph, 2, 2)
    assert padded == 4
    got = ref.sparse_decode_reuse(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                  inp.context_lens, pi, n, padded, 2, 4, bs)
    assert torch.equal(got, want)
    # a padded page would change the result if it were read
    n_all = torch.full((4,), 4, dtype=torch.int32)
    other = ref.sparse_decode_reuse(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                    inp.context_lens, pi, n_all, padded, 2, 4, bs)
    assert not torch.equal(other, want)


def test_select_topk_brute_force_with_ties_and_invalid_pages():
    g = torch.Generator().manual_seed(5)
    B, H, W, bs = 3, 2, 40, 16
    # quantised scores produce many exact ties
    ps = (torch.randint(0, 6, (B, H, W), generator=g).float() * 0.5)
    ctx = torch.tensor([16 * 40, 16 * 25 - 3, 16 * 2])
    nv = ref.n_valid_pages(ctx, bs)
    for b in range(B):
        ps[b, :, int(nv[b]):] = float("-inf")
    for budget in (1, 3, 10, 25, 40):
        idx, nph = ref.select_topk(ps, budget, ctx, bs)
        for b in range(B):
            for h in range(H):
                order = sorted(range(W), key=lambda p: (-ps[b, h, p].item(), p))
                assert idx[b, h].tolist() == sorted(order[:budget])
                assert int(nph[b, h]) == min(budget, int(nv[b]))
                # the first n_per_head entries are valid pages
                assert all(p < int(nv[b]) for p in idx[b, h, :int(nph[b, h])].tolist())


def test_n_valid_pages_formula():
    ctx = torch.tensor([0, 1, 15, 16, 17, 32, 131072])
    assert ref.n_valid_pages(ctx, 16).tolist() == [1, 1, 1, 1, 2, 2, 8192]
    assert ref.n_valid_pages(ctx, 32).tolist() == [1, 1, 1, 1, 1, 1, 4096]
    ctx = torch.tensor([0, 1, 63, 64, 65, 131072])
    assert ref.n_valid_pages(ctx, 64).tolist() == [1, 1, 1, 1, 2, 2048]


def test_coverage_special_cases():
    g = torch.Generator().manual_seed(7)
    ps = torch.randn(2, 3, 20, generator=g)
    full = torch.arange(20, dtype=torch.int32).view(1, 1, 20).expand(2, 3, 20).contiguous()
    acc, cov = ref.check_coverage(ps, full, torch.full((2, 3), 20, dtype=torch.int32), 0.999)
    assert torch.allclose(cov, torch.ones_like(cov), atol=1e-6) and bool(acc.all())
    some = full[..., :4].contiguous()
    acc0, cov0 = ref.check_coverage(ps, some, torch.full((2, 3), 4, dtype=torch.int32), 0.0)
    assert bool(acc0.all())
    want = torch.exp(ps[..., :4]).sum(-1) / torch.exp(ps).sum(-1)
    assert torch.allclose(cov0, want, atol=1e-6)
    # no selected page: coverage 0
    _, covz = ref.check_coverage(ps, some, torch.zeros(2, 3, dtype=torch.int32), 0.5)
    assert float(covz.max()) == 0.0


@pytest.mark.parametrize("D,bs", GEOMETRIES)
def test_decode_all_pages_equals_textbook_softmax(D, bs):
    inp = _tiny(seed=11, D=D, bs=bs)
    out, (o, m, l) = ref.dense_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                      inp.context_lens, inp.num_kv_heads, inp.num_q_per_kv,
                                      inp.block_size, return_state=True)
    B, H_q, D = inp.q.shape
    G = inp.num_q_per_kv
    for b in range(B):
        c = int(inp.context_lens[b])
        pages = -(-c // bs)
        phys = inp.block_tables[b, :pages].long()
        for j in range(H_q):
            h = j // G
            keys = inp.k_cache[phys, :, h].reshape(-1, D)[:c]
            vals = inp.v_cache[phys, :, h].reshape(-1, D)[:c]
            want = ref.softmax_attention(inp.q[b, j], keys, vals)
            got = o[b, j].double() / l[b, j].double()
            assert (got - want).abs().max().item() < 1e-5
            s = (keys.double() @ inp.q[b, j].double()) / math.sqrt(D)
            assert abs(float(m[b, j]) - float(s.max())) < 1e-5


@pytest.mark.parametrize("D,bs", GEOMETRIES)
def test_draft_plus_complement_equals_dense(D, bs):
    inp = _tiny(seed=13, D=D, bs=bs)
    ps = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens,
                         inp.num_kv_heads, inp.num_q_per_kv, inp.block_size)
    idx, nph = ref.select_topk(ps, 2, inp.context_lens, bs)
    rejected = torch.zeros(idx.shape[0], idx.shape[1], dtype=torch.bool)
    got = ref.verified_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                              inp.context_lens, idx, nph, rejected, inp.num_kv_heads,
                              inp.num_q_per_kv, bs, acc_dtype=torch.float64)
    dense = ref.dense_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                             inp.context_lens, inp.num_kv_heads, inp.num_q_per_kv, bs)
    assert (got.float() - dense.float()).abs().max().item() <= 1e-2  # bf16 outputs
    # accepted heads return the normalised draft
    accepted = torch.ones_like(rejected)
    got_a = ref.verified_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables,
                                inp.context_lens, idx, nph, accepted, inp.num_kv_heads,
                                inp.num_q_per_kv, bs)
    draft = ref.sparse_decode(inp.q, inp.k_cache, inp.v_cache, inp.block_tables, idx, nph,
                              inp.context_lens, inp.num_kv_heads, inp.num_q_per_kv, bs)
    assert torch.equal(got_a, draft)


def test_empty_selection_contract():
    inp = _tiny(seed=17)
    idx = torch.zeros(2, 2, 3, dtype=torch.int32)
    o, m, l = ref.sparse_decode_unnorm(inp.q, inp.k_cache, inp.v_cache, inp.block_tables, idx,
                                       torch.zeros(2, 2, dtype=torch.int32), inp.context_lens,
                                       2, 4, 16)
    assert float(o.abs().max()) == 0.0 and float(l.max()) == 0.0
    assert bool(torch.isinf(m).all()) and bool((m < 0).all())


@pytest.mark.parametrize("bs", [8, 16, 32, 64, 128])
def test_append_token_allocation_rule(bs):
    """kv_cache.py:133-150: a block is taken only at offset 0 of a new page."""
    K = torch.zeros(8, bs, 1, 4)
    V = torch.zeros(8, bs, 1, 4)
    bt = torch.zeros(1, 4, dtype=torch.int32)
    ctx = torch.tensor([bs - 1], dtype=torch.int32)
    alloc = torch.tensor([1], dtype=torch.int32)
    nf = 5
    for i in range(3):
        nf = ref.append_token_kv(K, V, bt, ctx, alloc, nf, 0, torch.full((1, 4), float(i + 1)),
                                 torch.full((1, 4), -float(i + 1)), bs)
    assert ctx.tolist() == [bs + 2] and alloc.tolist() == [2] and nf == 6
    assert bt[0, 1].item() == 5
    assert K[int(bt[0, 0]), bs - 1, 0, 0].item() == 1.0
    assert K[5, 0, 0, 0].item() == 2.0 and K[5, 1, 0, 0].item() == 3.0


# ---- planted mistakes: a wrong oracle must fail the checks above ----------

def test_planted_mistake_wrong_scale_is_caught(monkeypatch):
    inp = _tiny(seed=19)
    monkeypatch.setattr(ref, "fp32_scale", lambda D: 1.0 / D)   # dropped sqrt
    got = ref.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens,
                          inp.num_kv_heads, inp.num_q_per_kv, inp.block_size)
    monkeypatch.undo()
    want = _brute_scores(inp)
    fin = torch.isfinite(want)
    assert (got[fin] - want[fin]).abs().max().item() > 1e-3


def test_planted_mistake_wrong_head_grouping_is_caught():
    """Interleaved instead of contiguous GQA groups changes q_rep."""
    inp = _tiny(seed=23)
    q = inp.q
    B, H_q, D = q.shape
    H, G = inp.num_kv_heads, inp.num_q_per_kv
    wrong = q.view(B, G, H, D).transpose(1, 2).float().mean(2).to(torch.bfloat16)
    right = ref.group_mean_bf16(q, H, G)
    assert not torch.equal(wrong, right)


def test_planted_mistake_merge_without_rescale_is_caught():
    torch.manual_seed(0)
    od, oc = torch.randn(1, 2, 8), torch.randn(1, 2, 8)
    md, mc = torch.tensor([[0.0, 3.0]]), torch.tensor([[2.0, -1.0]])
    ld, lc = torch.rand(1, 2) + 0.5, torch.rand(1, 2) + 0.5
    good = ref.lse_merge(od, md, ld, oc, mc, lc, torch.zeros(1, 1, dtype=torch.bool), 2,
                         torch.float64)
    naive = (od + oc) / (ld + lc).unsqueeze(-1)   # forgets exp(m - M)
    assert (good - naive).abs().max().item() > 1e-2
