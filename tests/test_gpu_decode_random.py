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
The decode with the token append folded in (cvsa_sparse_decode_append) is
drawn the same way, with sequences at page offsets 0, mid-page and last
slot, and compared with the append followed by the decode, bit for bit.
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


@pytest.mark.parametrize("D", [32, 64, 256])
@pytest.mark.parametrize("seed", range(8))
def test_random_decode_launches_head_dims(gpu, seed, D):
    _check(gpu, seed, D)


@pytest.mark.parametrize("BS", [8, 32, 64, 128])
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


def _append_case(seed, dev, D, BS, G):
    """A batch whose sequences sit at random page offsets (0, mid, last),
    the next free blocks after the used ones, and selections that hold the
    new token's page on about half of the heads (its page before the append
    when the token is mid-page, the page the append allocates otherwise)."""
    g = torch.Generator().manual_seed(1000 + seed)
    rnd = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))  # noqa: E731
    H = [1, 2, 4, 8][rnd(0, 3)]
    B = rnd(1, 5)
    ctx = []
    for _ in range(B):
        pages = rnd(1, 300)
        off = [0, rnd(1, BS - 2), BS - 1][rnd(0, 2)]
        ctx.append(pages * BS + off)
    inp = make_paged_inputs(B, H * G, H, D, ctx, block_size=BS, seed=seed, device=dev,
                            spare_blocks=B + 4)
    W = inp.block_tables.shape[1] + 1
    bt = torch.zeros(B, W, dtype=torch.int32, device=dev)
    bt[:, :W - 1] = inp.block_tables
    alloc = torch.tensor([-(-c // BS) for c in ctx], dtype=torch.int32, device=dev)
    width = rnd(1, 64)
    pi = torch.zeros(B, H, width, dtype=torch.int32)
    nph = torch.zeros(B, H, dtype=torch.int32)
    for b in range(B):
        n_valid = ctx[b] // BS + 1          # pages after the append
        new_page = ctx[b] // BS
        for h in range(H):
            n = rnd(0, min(width, n_valid))
            pages = torch.randperm(n_valid, generator=g)[:n]
            if n and rnd(0, 1) and new_page not in pages.tolist():
                pages[0] = new_page
            pi[b, h, :n] = pages.sort().values.to(torch.int32)
            nph[b, h] = n
    kn = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(dev)
    vn = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(dev)
    return inp, bt, alloc, pi.to(dev), nph.to(dev), kn, vn, ctx


def _slots(ctx, alloc, next_free, BS):
    slots, r = [], 0
    for c, a in zip(ctx, alloc.tolist()):
        new = c % BS == 0 and c // BS >= a
        slots += [c, next_free + r if new else -1]
        r += int(new)
    return slots


@pytest.mark.parametrize("shape", [(128, 16, 4), (128, 16, 1), (128, 16, 16), (128, 16, 7),
                                   (64, 16, 4), (256, 16, 4), (128, 32, 4), (128, 16, 20)],
                         ids=lambda s: f"D{s[0]}_bs{s[1]}_G{s[2]}")
@pytest.mark.parametrize("seed", range(3))
def test_random_decode_append(gpu, seed, shape):
    """cvsa_sparse_decode_append (one launch at D = 128, 16-token pages,
    G <= 16; two launches otherwise) against cvsa_append_kv followed by
    cvsa_sparse_decode on a copy of the same state: outputs bit-identical,
    caches, tables, lengths, allocation counts and work counters equal; the
    new token is on a selected page for about half of the heads."""
    D, BS, G = shape
    inp, bt, alloc, pi, nph, kn, vn, ctx = _append_case(seed, gpu, D, BS, G)
    H = inp.k_cache.shape[2]
    next_free = inp.used_blocks
    state = [inp.k_cache.clone(), inp.v_cache.clone(), bt.clone(),
             inp.context_lens.clone(), alloc.clone()]
    ref = [t.clone() for t in state]
    work_a = torch.zeros(2, dtype=torch.int64, device=gpu)
    work_b = torch.zeros(2, dtype=torch.int64, device=gpu)
    out = ops.sparse_decode_append(inp.q, state[0], state[1], state[2], state[3], pi, nph,
                                   kn, vn, state[4], _slots(ctx, alloc, next_free, BS), H, G,
                                   BS, work=work_a)
    ops.append_kv(kn, vn, ref[0], ref[1], ref[2], ref[3], ref[4], 0, next_free, BS)
    want = ops.sparse_decode(inp.q, ref[0], ref[1], ref[2], pi, nph, ref[3], H, G, BS)
    pif, nphf = pi.reshape(-1, pi.shape[2]), nph.reshape(-1)
    ops.sparse_decode_reuse(inp.q, ref[0], ref[1], ref[2], ref[3], pif, nphf, pi.shape[2], H,
                            G, BS, work=work_b)
    torch.cuda.synchronize()
    assert torch.equal(out, want), (seed, shape)
    for a, b in zip(state, ref):
        assert torch.equal(a, b), (seed, shape)
    assert torch.equal(work_a, work_b), (work_a.tolist(), work_b.tolist())
    # and against attention over the appended cache in fp32
    for b in range(len(ctx)):
        for h in range(H):
            n = int(nph[b, h])
            o, _ = _attention(inp.q, ref[0], ref[1], ref[2], b, ctx[b] + 1, h, G,
                              pi[b, h, :n].long())
            err = (out[b, h * G:(h + 1) * G].float() - o).abs().max().item()
            assert err < 2e-2, (seed, shape, b, h, err)


@pytest.mark.parametrize("seed", range(4))
def test_decode_append_device_slots(gpu, seed):
    """The slots of cvsa_sparse_decode_append read from device memory (the
    form a captured graph replays) against the same slots from the host:
    outputs, caches, tables, lengths and allocation counts identical."""
    inp, bt, alloc, pi, nph, kn, vn, ctx = _append_case(seed, gpu, 128, 16, [4, 1, 16, 7][seed])
    H, G = inp.k_cache.shape[2], inp.q.shape[1] // inp.k_cache.shape[2]
    slots = _slots(ctx, alloc, inp.used_blocks, 16)
    runs = []
    errors = torch.zeros(1, dtype=torch.int32, device=gpu)
    for sl in (slots, torch.tensor(slots, dtype=torch.int32, device=gpu).view(-1, 2)):
        st = [inp.k_cache.clone(), inp.v_cache.clone(), bt.clone(), inp.context_lens.clone(),
              alloc.clone()]
        out = ops.sparse_decode_append(inp.q, *st[:4], pi, nph, kn, vn, st[4], sl, H, G, 16,
                                       slot_errors=errors)
        runs.append([out] + st)
    torch.cuda.synchronize()
    assert int(errors.item()) == 0
    for a, b in zip(*runs):
        assert torch.equal(a, b), seed


def test_decode_append_device_slots_out_of_range(gpu):
    """Device slots the launch cannot take (context length past the table,
    a new block past the cache or not at a page start, a negative length)
    append nothing for their sequence; the other sequences are unaffected."""
    inp, bt, alloc, pi, nph, kn, vn, ctx = _append_case(5, gpu, 128, 16, 4)
    B, H, G = len(ctx), inp.k_cache.shape[2], 4
    slots = _slots(ctx, alloc, inp.used_blocks, 16)
    good = [inp.k_cache.clone(), inp.v_cache.clone(), bt.clone(), inp.context_lens.clone(),
            alloc.clone()]
    want = ops.sparse_decode_append(inp.q, *good[:4], pi, nph, kn, vn, good[4], slots, H, G, 16)
    W, nb = bt.shape[1], inp.k_cache.shape[0]
    bad_forms = [(W * 16, -1), (-1, -1), (ctx[0] // 16 * 16, nb), (ctx[0] // 16 * 16 + 1, 0)]
    errors = torch.zeros(1, dtype=torch.int32, device=gpu)
    for i, bad in enumerate(bad_forms):
        sl = list(slots)
        sl[0], sl[1] = bad
        st = [inp.k_cache.clone(), inp.v_cache.clone(), bt.clone(), inp.context_lens.clone(),
              alloc.clone()]
        out = ops.sparse_decode_append(inp.q, *st[:4], pi, nph, kn, vn, st[4],
                                       torch.tensor(sl, dtype=torch.int32,
                                                    device=gpu).view(-1, 2), H, G, 16,
                                       slot_errors=errors)
        torch.cuda.synchronize()
        assert int(errors.item()) == i + 1, bad   # the refused slot is reported
        assert torch.equal(st[3][0], inp.context_lens[0]), bad
        assert torch.equal(st[4][0], alloc[0]) and torch.equal(st[2][0], bt[0]), bad
        if B > 1:
            assert torch.equal(out[1:], want[1:]), bad
            assert torch.equal(st[3][1:], good[3][1:]) and torch.equal(st[2][1:], good[2][1:])
        # sequence 0's rows of the cache are those before the append
        blocks = bt[0, :-(-ctx[0] // 16)].long()
        assert torch.equal(st[0][blocks], inp.k_cache[blocks]), bad
        assert torch.equal(st[1][blocks], inp.v_cache[blocks]), bad


def test_decode_append_large_batch(gpu):
    """More sequences than the one-launch form takes (B = 260 > 256): the
    entry point appends and decodes in two launches with the same results."""
    B, H, G, D, BS = 260, 2, 4, 128, 16
    g = torch.Generator().manual_seed(77)
    ctx = [int(x) for x in torch.randint(1, 80, (B,), generator=g)]
    inp = make_paged_inputs(B, H * G, H, D, ctx, block_size=BS, seed=77, device=gpu,
                            spare_blocks=B + 4)
    W = inp.block_tables.shape[1] + 1
    bt = torch.zeros(B, W, dtype=torch.int32, device=gpu)
    bt[:, :W - 1] = inp.block_tables
    alloc = torch.tensor([-(-c // BS) for c in ctx], dtype=torch.int32, device=gpu)
    width = 4
    pi = torch.zeros(B, H, width, dtype=torch.int32)
    nph = torch.zeros(B, H, dtype=torch.int32)
    for b in range(B):
        n_valid = ctx[b] // BS + 1
        n = min(width, n_valid)
        pi[b, :, :n] = torch.arange(n_valid - n, n_valid, dtype=torch.int32)
        nph[b] = n
    pi, nph = pi.to(gpu), nph.to(gpu)
    kn = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(gpu)
    vn = torch.randn(B, H, D, generator=g).to(torch.bfloat16).to(gpu)
    state = [inp.k_cache.clone(), inp.v_cache.clone(), bt.clone(), inp.context_lens.clone(),
             alloc.clone()]
    ref = [t.clone() for t in state]
    out = ops.sparse_decode_append(inp.q, *state[:4], pi, nph, kn, vn, state[4],
                                   _slots(ctx, alloc, inp.used_blocks, BS), H, G, BS)
    ops.append_kv(kn, vn, *ref, 0, inp.used_blocks, BS)
    want = ops.sparse_decode(inp.q, ref[0], ref[1], ref[2], pi, nph, ref[3], H, G, BS)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    for a, b in zip(state, ref):
        assert torch.equal(a, b)
