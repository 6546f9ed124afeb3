"""Seeded random decode launches against fp32 torch attention.

Each case draws a batch of ragged contexts (partial last pages, block tables
wider than the context), G in 1..8 (and 9..48), H_kv in {1, 2, 4, 8, 16}, a selection
width (budget) and per-head selections of any length from 0 to the width
(ascending pages, garbage past n_per_head), and an accept mask.  The listed
decode (every head walks its selection), the verified decode (accepted heads
their selection, rejected heads every valid page, stream-K partition) and
the dense decode are compared per (sequence, KV head) with softmax attention
over those pages in fp32.  Cases 0..3 make the verified walk total equal to
B * H_kv * width with uneven per-head walks (the situation of the
"every head walks max_sel pages" regression), the others are free draws.
The same draws run at head dimensions 64 and 256 (engines compiled per D,
split partials of G x (D + 4) floats, merges over several chunk passes when
G x D / 4 exceeds the workgroup) and at block sizes 32 and 64 (pages walked
as 2 or 4 tiles of 16 tokens).
"""
import pytest
import torch

from cvsa import ops
from cvsa.synthetic import make_paged_inputs

pytestmark = pytest.mark.gpu

OUT_ATOL = 2e-3        # fp32 outputs against fp32 attention
LSE_RTOL = 1e-3
def _attention(q, K, V, bt, b, ctx, h, G, pages):
    """Softmax attention of q-heads h*G..h*G+G-1 of sequence b over logical
    `pages` (fp32, torch); (zeros, -inf) when no token is valid."""
    D = q.shape[-1]
    BS = K.shape[1]
    rows = q[b, h * G:(h + 1) * G].float()
    if pages.numel() == 0:
        return torch.zeros_like(rows), torch.full((G,), -float("inf"), device=q.device)
    phys = bt[b, pages].long()
    k = K[phys, :, h].float().reshape(-1, D)
    v = V[phys, :, h].float().reshape(-1, D)
    tok = (pages[:, None] * BS + torch.arange(BS, device=q.device)[None]).reshape(-1)
    s = rows @ k.T * D ** -0.5
    s[:, tok >= ctx] = -float("inf")
    m = s.max(dim=1).values
    p = torch.exp(s - m[:, None])
    l = p.sum(dim=1)
    return (p @ v) / l[:, None], m + torch.log(l)


def _case(seed, dev, D=128, BS=16, G_range=(1, 8)):
    g = torch.Generator().manual_seed(seed)
    rnd = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))  # noqa: E731
    H = [1, 2, 4, 8, 16][rnd(0, 4)]
    G = rnd(*G_range)
    B = rnd(1, 4)
    uneven = seed < 4
    if uneven:   # one sequence, pages enough for every head's walk to coincide
        B, H = 1, [4, 8][seed % 2]
    ctx = [rnd(1, 9000) for _ in range(B)]
    if uneven:
        ctx = [BS * H * 64]                       # n_valid = 64 * H pages
    n_valid = [(c - 1) // BS + 1 for c in ctx]
    W = max(n_valid) + rnd(0, 6)
    budget = 64 if uneven else rnd(1, W)
    inp = make_paged_inputs(B, H * G, H, D, ctx, block_size=BS, seed=seed, device=dev,
                            max_pages=W,
                            hot_heads=list(range(0, H, 2)), n_hot=4, hot_shift=4.0)
    idx = torch.randint(-3, W + 3, (B, H, budget), generator=g).to(torch.int32)
    nph = torch.zeros(B, H, dtype=torch.int32)
    accept = torch.rand(B, H, generator=g) < 0.6
    for b in range(B):
        for h in range(H):
            top = min(budget, n_valid[b])
            r = float(torch.rand(1, generator=g))
            n = 0 if r < 0.1 else top if r < 0.4 else rnd(0, top)
            sel = torch.randperm(n_valid[b], generator=g)[:n].sort().values
            idx[b, h, :n] = sel.to(torch.int32)
            nph[b, h] = n
    if uneven:
        # verified walk: one rejected head walks all 64 * H pages, the others
        # nothing -- the total equals H * budget
        nph.zero_()
        accept.fill_(True)
        accept[0, seed % H] = False
    return inp, W, budget, idx.to(dev), nph.to(dev), accept.to(dev), H, G, B, ctx, n_valid


def _check(gpu, seed, D, BS=16, G_range=(1, 8)):
    inp, W, budget, idx, nph, accept, H, G, B, ctx, n_valid = _case(seed, gpu, D, BS, G_range)
    q, K, V, bt, cl = inp.q, inp.k_cache, inp.v_cache, inp.block_tables, inp.context_lens
    lo, lm, ll = ops.sparse_decode_unnorm(q, K, V, bt, idx, nph, cl, H, G, BS)
    ver, (vo, vm, vl) = ops.verified_decode(q, K, V, bt, cl, idx, nph, accept, H, G, BS,
                                            return_state=True, output_dtype=torch.float32)
    dense = ops.dense_decode(q, K, V, bt, cl, H, G, BS)
    o_listed = lo / torch.clamp(ll, min=1e-6)[..., None]
    for b in range(B):
        every = torch.arange(n_valid[b], device=gpu)
        for h in range(H):
            rows = slice(h * G, (h + 1) * G)
            sel = idx[b, h, :int(nph[b, h])].long()
            want, want_lse = _attention(q, K, V, bt, b, ctx[b], h, G, sel)
            assert (o_listed[b, rows] - want).abs().max().item() < OUT_ATOL, (seed, b, h)
            pages = sel if bool(accept[b, h]) else every
            want_v, want_vlse = _attention(q, K, V, bt, b, ctx[b], h, G, pages)
            assert (ver[b, rows] - want_v).abs().max().item() < OUT_ATOL, (seed, b, h)
            if pages.numel():
                lse = vm[b, rows] + torch.log(vl[b, rows])
                rel = (lse - want_vlse).abs() / want_vlse.abs().clamp(min=1.0)
                assert rel.max().item() < LSE_RTOL, (seed, b, h)
            want_d, _ = _attention(q, K, V, bt, b, ctx[b], h, G, every)
            assert (dense[b, rows].float() - want_d).abs().max().item() < 2e-2, (seed, b, h)


@pytest.mark.parametrize("seed", range(16))
def test_random_decode_launches(gpu, seed):
    _check(gpu, seed, 128)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("seed", range(8))
def test_random_decode_launches_head_dims(gpu, seed, D):
    _check(gpu, seed, D)


@pytest.mark.parametrize("BS", [32, 64])
@pytest.mark.parametrize("seed", range(8))
def test_random_decode_launches_block_sizes(gpu, seed, BS):
    _check(gpu, seed, [128, 64, 256][seed % 3], BS)


@pytest.mark.parametrize("seed", range(8))
def test_random_decode_launches_wide_groups(gpu, seed):
    """G = 9..16 query heads per KV head (one MFMA tile of 16 columns)."""
    _check(gpu, seed, [128, 64, 256, 128][seed % 4], [16, 16, 16, 32][seed % 4], (9, 16))


@pytest.mark.parametrize("seed", range(4))
def test_random_decode_launches_large_groups(gpu, seed):
    """G = 17..48 query heads per KV head: one launch per 16 of them."""
    _check(gpu, 20 + seed, [128, 64, 256, 128][seed], [16, 16, 16, 32][seed], (17, 48))
