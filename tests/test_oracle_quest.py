"""Pins of the Quest page scorer of the oracle (ref.quest_page_scores), which
restates CVSABackend._quest_page_scores (cvsa/backend.py:572-620).  The
reference's tests do not cover this scorer, so it is pinned by what the
mathematics fixes: the Quest bound is an upper bound of the page's exact max
score, it equals that score on one-token pages, it is a plain sum over
dimensions (brute force), it ignores slots past the context, and for a
non-negative query it is q . kmax."""
import math

import pytest
import torch

from oracle import cvsa_oracle as ref


def _inputs(seed, B=2, H=2, G=2, W=6, ctx=(85, 50), nb=20, D=128, bs=16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H * G, D, generator=g).to(torch.bfloat16)
    k = torch.randn(nb, bs, H, D, generator=g).to(torch.bfloat16)
    bt = torch.randperm(nb, generator=g)[: B * W].view(B, W).to(torch.int32)
    cl = torch.tensor(ctx, dtype=torch.int32)
    return q, k, bt, cl, H, G


@pytest.mark.parametrize("D,bs", [(128, 16), (64, 32), (256, 64)])
def test_quest_bounds_the_exact_page_score(D, bs):
    for seed in range(4):
        q, k, bt, cl, H, G = _inputs(seed, ctx=(85 * bs // 16, 50 * bs // 16), D=D, bs=bs)
        quest = ref.quest_page_scores(q, k, bt, cl, H, G, bs)
        exact = ref.score_pages(q, k, bt, cl, H, G, bs)
        fin = torch.isfinite(exact)
        assert torch.equal(fin, torch.isfinite(quest))
        assert bool((quest[fin] >= exact[fin] - 1e-5).all())
        # and it is not the same function
        assert float((quest[fin] - exact[fin]).max()) > 0.5


def test_quest_equals_exact_on_one_token_pages():
    q, k, bt, cl, H, G = _inputs(7, ctx=(81, 49))   # last pages hold one token
    quest = ref.quest_page_scores(q, k, bt, cl, H, G, 16)
    exact = ref.score_pages(q, k, bt, cl, H, G, 16)
    for b, p in ((0, 5), (1, 3)):
        assert torch.allclose(quest[b, :, p], exact[b, :, p], rtol=0, atol=1e-5)


@pytest.mark.parametrize("D,bs", [(128, 16), (64, 32), (256, 64)])
def test_quest_brute_force(D, bs):
    c = 40 * bs // 16
    q, k, bt, cl, H, G = _inputs(3, B=1, W=3, ctx=(c,), D=D, bs=bs)
    got = ref.quest_page_scores(q, k, bt, cl, H, G, bs)
    qf = q.float()
    scale = D ** -0.5
    for h in range(H):
        qr = [float(torch.tensor(sum(float(qf[0, h * G + j, d]) for j in range(G)) / G)
                    .to(torch.bfloat16)) for d in range(D)]
        for p in range(3):
            n = min(bs, c - bs * p)
            rows = k[int(bt[0, p]), :n, h].float()
            total = 0.0
            for d in range(D):
                lo = min(float(rows[t, d]) for t in range(n))
                hi = max(float(rows[t, d]) for t in range(n))
                total += max(qr[d] * lo, qr[d] * hi)
            assert math.isclose(float(got[0, h, p]), total * scale, rel_tol=1e-5, abs_tol=1e-5)


def test_quest_ignores_slots_past_the_context_and_empty_pages():
    q, k, bt, cl, H, G = _inputs(5)
    want = ref.quest_page_scores(q, k, bt, cl, H, G, 16)
    k2 = k.clone()
    k2[int(bt[0, 5]), 85 - 80:] = 1e4        # garbage after the last valid token of b=0
    k2[int(bt[1, 3]), 50 - 48:] = -1e4
    assert torch.equal(ref.quest_page_scores(q, k2, bt, cl, H, G, 16), want)
    assert bool(torch.isinf(want[1, :, 4:]).all()) and bool((want[1, :, 4:] < 0).all())


def test_quest_nonnegative_query_is_q_dot_kmax():
    q, k, bt, cl, H, G = _inputs(9)
    q = q.abs()
    got = ref.quest_page_scores(q, k, bt, cl, H, G, 16)
    _, kmax = ref.page_key_minmax(k, bt, cl, 16)
    qr = ref.group_mean_bf16(q, H, G).double()
    want = torch.einsum("bhd,bphd->bhp", qr, kmax.nan_to_num(neginf=0.0).double()) * 128 ** -0.5
    fin = torch.isfinite(got)
    assert torch.allclose(got[fin].double(), want[fin], rtol=1e-6, atol=1e-6)
