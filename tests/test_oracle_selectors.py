"""Pins of the oracle's per-head budget selections: ref.topp_need /
ref.topp_select (restating CVSABackend._topp_select, cvsa/backend.py:652-681),
ref.static_select (_static_select, :622-650) and ref.adaptive_budgets /
ref.adaptive_select (_adaptive_select, :522-570).  The reference's tests do
not cover these selectors, so they are pinned by closed forms (uniform and
geometric page masses, a dominating head, floor ratios 0 and 1), the strict
"< top_p" boundary, the clamps and rounding, the NaN rows, and scalar brute
forces on small rows."""
import math

import torch

from oracle import cvsa_oracle as ref


def _row(scores):
    return torch.tensor(scores, dtype=torch.float32).view(1, 1, -1)


def test_topp_uniform_mass_is_ceil_p_n():
    # n equal finite scores, the rest -inf: need = ceil(p * n) (p * n not integral)
    for n, p in ((20, 0.37), (50, 0.9), (7, 0.95), (100, 0.123)):
        s = [0.5] * n + [float("-inf")] * 9
        need, _ = ref.topp_need(_row(s), p)
        assert int(need) == max(3, math.ceil(p * n)), (n, p)


def test_topp_boundary_is_strict():
    # eight pages of mass 1/8: the cumulative mass reaches 0.5 exactly at the
    # fourth page, which is then the last one taken ("cum < p" counts three)
    need, _ = ref.topp_need(_row([1.0] * 8), 0.5)
    assert int(need) == 4
    need, _ = ref.topp_need(_row([1.0] * 8), 0.5000001)
    assert int(need) == 5


def test_topp_geometric_closed_form():
    # masses proportional to 2^-j: cum_k = (1 - 2^-k) / (1 - 2^-n)
    n = 30
    g = torch.Generator().manual_seed(3)
    perm = torch.randperm(n, generator=g)
    s = torch.empty(n)
    s[perm] = -torch.arange(n, dtype=torch.float32) * math.log(2.0)
    for p in (0.5, 0.8, 0.97, 0.999):
        need, order = ref.topp_need(s.view(1, 1, -1), p)
        pf = float(torch.tensor(p, dtype=torch.float32))
        want = next(k for k in range(1, n + 1)
                    if (1 - 2.0 ** -k) / (1 - 2.0 ** -n) >= pf)
        assert int(need) == max(3, want), p
        assert torch.equal(order[0, 0, :5], perm[:5])   # ranked by score


def test_topp_clamps_and_nan_rows():
    # one page dominates: need = 1, clamped up to 3; P = 2 clamps down to 2
    need, _ = ref.topp_need(_row([30.0, 0.0, 0.0, 0.0, 0.0]), 0.9)
    assert int(need) == 3
    need, _ = ref.topp_need(_row([1.0, 1.0]), 0.9)
    assert int(need) == 2
    for bad in ([float("inf"), 0.0, 1.0, 2.0], [float("nan")] * 4,
                [float("-inf")] * 4):
        need, _ = ref.topp_need(_row(bad), 0.9)
        assert int(need) == 3


def test_topp_brute_force():
    g = torch.Generator().manual_seed(7)
    for trial in range(20):
        P = int(torch.randint(4, 40, (1,), generator=g))
        temp = float(torch.rand(1, generator=g)) * 4 + 0.1
        s = (torch.randn(P, generator=g) * temp).tolist()
        p = float(torch.rand(1, generator=g)) * 0.9 + 0.05
        pf = float(torch.tensor(p, dtype=torch.float32))
        mx = max(s)
        e = [math.exp(x - mx) for x in s]
        tot = sum(e)
        ranked = sorted(range(P), key=lambda i: (-s[i], i))
        cum, below = 0.0, 0
        for i in ranked:
            cum += e[i] / tot
            below += cum < pf
        need, order = ref.topp_need(torch.tensor(s).view(1, 1, -1), p)
        assert int(need) == min(max(below + 1, 3), P), trial
        assert order[0, 0].tolist() == ranked


def test_topp_select_sets_and_valid_pages():
    # b=0: four valid pages, all needed at p=0.999; b=1: two valid pages,
    # need clamped up to 3 takes the lowest -inf page too, and n_per_head =
    # n_valid keeps the valid ones, which come first in ascending order
    s = torch.full((2, 1, 10), float("-inf"))
    s[0, 0, :4] = torch.tensor([0.0, 2.0, 1.0, 0.5])
    s[1, 0, :2] = torch.tensor([1.0, 2.0])
    ctx = torch.tensor([56, 20], dtype=torch.int32)
    idx, nph = ref.topp_select(s, 0.999, ctx, 16)
    assert nph.tolist() == [[4], [2]]
    assert idx.shape[-1] == 4
    assert idx[0, 0].tolist() == [0, 1, 2, 3]
    assert idx[1, 0, :3].tolist() == [0, 1, 2]


def test_static_select_budgets_and_sets():
    # clamp(round(frac * P), 3, P) with round half to even
    assert ref.static_budgets([0.5, 0.25, 0.9, 0.01, 2.0], 10).tolist() == [5, 3, 9, 3, 10]
    assert ref.static_budgets([0.25], 10).tolist() == [3]      # 2.5 -> 2 -> clamp 3
    assert ref.static_budgets([0.45], 10).tolist() == [4]      # 4.5 -> 4 (half to even)
    g = torch.Generator().manual_seed(5)
    B, H, P = 2, 3, 24
    s = torch.randn(B, H, P, generator=g)
    ctx = torch.tensor([24 * 16, 10 * 16 - 3], dtype=torch.int32)
    s[1, :, 10:] = float("-inf")
    fr = [0.2, 0.5, 0.75]
    idx, nph = ref.static_select(s, fr, ctx, 16)
    k = ref.static_budgets(fr, P).tolist()
    assert idx.shape[-1] == max(min(x, 24) for x in k)
    for b in range(B):
        for h in range(H):
            n = min(k[h], 24 if b == 0 else 10)
            assert int(nph[b, h]) == n
            want = sorted(sorted(range(P), key=lambda i: (-float(s[b, h, i]), i))[:n])
            assert idx[b, h, :n].tolist() == want


def _adaptive_brute(s, base, floor, nv):
    """Scalar restatement: count heads among the H*base largest (value desc,
    head asc), blend in fp32, round half to even, clamp."""
    H, P = len(s), len(s[0])
    cells = sorted(((-s[h][p], h) for h in range(H) for p in range(P)))
    raw = [0] * H
    for _, h in cells[:min(H * base, H * P)]:
        raw[h] += 1
    keep = torch.tensor(1.0 - floor, dtype=torch.float32)
    cap = torch.tensor(base * floor, dtype=torch.float32)
    out = []
    for r in raw:
        m = float(torch.tensor(float(r), dtype=torch.float32) * keep + cap)
        out.append(min(max(int(round(m)), 1), nv))   # Python round is half to even
    return out


def test_adaptive_floor_ratio_limits():
    g = torch.Generator().manual_seed(11)
    s = torch.randn(2, 4, 50, generator=g)
    ctx = torch.tensor([50 * 16, 20 * 16], dtype=torch.int32)
    # floor 1: every head gets the base budget (clamped to n_valid)
    assert ref.adaptive_budgets(s, 12, ctx, 16, 1.0).tolist() == [[12] * 4, [12] * 4]
    assert ref.adaptive_budgets(s, 30, ctx, 16, 1.0).tolist() == [[30] * 4, [20] * 4]
    # floor 0: the raw shares, which add up to H * base
    b0 = ref.adaptive_budgets(s, 12, torch.tensor([800, 800], dtype=torch.int32), 16, 0.0)
    assert b0.sum(dim=1).tolist() == [48, 48]


def test_adaptive_dominating_head_and_rounding():
    # head 0 above everything: it takes min(P, H * base) slots, the rest
    # compete for what is left
    s = torch.zeros(1, 3, 10)
    s[0, 0] = 10.0 + torch.arange(10, dtype=torch.float32)
    s[0, 1] = torch.arange(10, dtype=torch.float32) * 0.1
    s[0, 2] = torch.arange(10, dtype=torch.float32) * 0.1 + 0.05
    ctx = torch.tensor([160], dtype=torch.int32)
    assert ref.adaptive_budgets(s, 4, ctx, 16, 0.0).tolist() == [[10, 1, 1]]
    # raw (10, 1, 1) at floor 0.5, base 3: 10*0.5+1.5 = 6.5 -> 6; 1*0.5+1.5 = 2
    assert ref.adaptive_budgets(s, 3, ctx, 16, 0.5).tolist() == [[6, 2, 2]]


def test_adaptive_brute_force_and_ties():
    g = torch.Generator().manual_seed(13)
    for trial in range(12):
        H = int(torch.randint(1, 6, (1,), generator=g))
        P = int(torch.randint(3, 25, (1,), generator=g))
        base = int(torch.randint(1, P + 1, (1,), generator=g))
        floor = [0.0, 0.25, 0.5, 0.9][trial % 4]
        s = torch.randn(1, H, P, generator=g).round()     # many exact ties
        nv = int(torch.randint(1, P + 1, (1,), generator=g))
        s[0, :, nv:] = float("-inf")
        ctx = torch.tensor([nv * 16], dtype=torch.int32)
        got = ref.adaptive_budgets(s, base, ctx, 16, floor)[0].tolist()
        assert got == _adaptive_brute(s[0].tolist(), base, floor, nv), trial
        idx, nph = ref.adaptive_select(s, base, ctx, 16, floor)
        for h in range(H):
            n = int(nph[0, h])
            want = sorted(sorted(range(P), key=lambda p: (-float(s[0, h, p]), p))[:n])
            assert idx[0, h, :n].tolist() == want
