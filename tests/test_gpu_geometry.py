"""Head dimensions 32, 64 and 256, block sizes 8, 32, 64 and 128 and GQA groups of 9 to
40 query heads through the entry points that take them, against the
oracle: page scoring in both of its layouts (a wave load holds 64 / (D/8)
key rows, so the head-group layout needs H_kv a multiple of 8, 4, 2 at
D = 64, 128, 256 and smaller H_kv take the whole-page layout) and with
several tiles per wave, Quest metadata and scores, and the backend's
schedules in lockstep with the oracle backend.  Decode launches and step
plans at these geometries run with the random draws of
test_gpu_decode_random.py and test_gpu_step_plan.py, the KV append in
test_gpu_ops.py.
"""
import pytest
import torch

from oracle import cvsa_oracle as ref
from cvsa import ops
from cvsa.synthetic import make_paged_inputs
from test_gpu_backend import _random_schedule, _run

pytestmark = pytest.mark.gpu

SCORE_RTOL = 1e-4      # page scores, relative (as at D = 128)
QUEST_RTOL = 1e-5

GEOMS = [  # (B, H_q, H_kv, ctx)
    (2, 32, 8, [3000, 517]),
    (1, 28, 4, 2048),
    (3, 12, 4, [17, 300, 1024]),
    (2, 4, 2, 777),
    (1, 4, 1, 640),
    (1, 32, 16, 512),
]


def _close(got, want, rtol):
    fin = torch.isfinite(want)
    assert torch.equal(torch.isfinite(got), fin)
    assert torch.equal(got[~fin], want[~fin])
    err = ((got[fin] - want[fin]).abs() / want[fin].abs().clamp(min=1.0)).max().item()
    assert err < rtol, err


GEOMETRIES = [(64, 16), (256, 16), (128, 32), (128, 64), (64, 32), (256, 64),
              (32, 16), (32, 64), (128, 8), (64, 8), (256, 8), (32, 8), (128, 128),
              (64, 128)]  # (D, bs)


@pytest.mark.parametrize("D,bs", GEOMETRIES)
@pytest.mark.parametrize("geom", GEOMS)
def test_score_pages_geometry(gpu, geom, D, bs):
    B, H_q, H_kv, ctx = geom
    inp = make_paged_inputs(B, H_q, H_kv, D, ctx, block_size=bs, seed=200 + H_kv, device=gpu,
                            hot_heads=[0], n_hot=4, hot_shift=4.0)
    got = ops.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H_kv,
                          H_q // H_kv, bs).cpu()
    want = ref.score_pages(inp.q.cpu(), inp.k_cache.cpu(), inp.block_tables.cpu(),
                           inp.context_lens.cpu(), H_kv, H_q // H_kv, bs)
    _close(got, want, SCORE_RTOL)


@pytest.mark.parametrize("D,bs,H_kv,ctx", [(64, 16, 16, 131072), (256, 16, 16, 65536),
                                           (256, 16, 2, 65539), (64, 16, 2, 40000),
                                           (128, 32, 8, 131072), (128, 64, 8, 65536 - 5),
                                           (256, 64, 4, 65536)])
def test_score_pages_geometry_long_context(gpu, D, bs, H_kv, ctx):
    """Launches with 2 to 8 tiles per wave (and the whole-page layout over
    many pages) against the oracle."""
    inp = make_paged_inputs(1, 4 * H_kv, H_kv, D, ctx, block_size=bs, seed=210, device=gpu)
    got = ops.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H_kv, 4,
                          bs).cpu()
    want = ref.score_pages(inp.q.cpu(), inp.k_cache.cpu(), inp.block_tables.cpu(),
                           inp.context_lens.cpu(), H_kv, 4, bs)
    _close(got, want, SCORE_RTOL)


@pytest.mark.parametrize("D,bs", GEOMETRIES)
@pytest.mark.parametrize("B,H_q,H,ctx", [(2, 32, 8, [3000, 1501]), (1, 28, 4, [8191]),
                                         (3, 16, 2, [17, 530, 16]), (1, 8, 1, [5000])])
def test_quest_geometry(gpu, B, H_q, H, ctx, D, bs):
    """Quest scores of a first build and the page extremes it stores."""
    inp = make_paged_inputs(B, H_q, H, D, ctx, block_size=bs, seed=B * 100 + H, device=gpu,
                            hot_heads=[0], n_hot=4, hot_shift=6.0)
    qm = ops.QuestPageMeta(inp.k_cache)
    got = qm.scores(inp.q, inp.block_tables, inp.context_lens, H, H_q // H, bs)
    K, bt, cl = inp.k_cache.cpu(), inp.block_tables.cpu(), inp.context_lens.cpu()
    _close(got.cpu(), ref.quest_page_scores(inp.q.cpu(), K, bt, cl, H, H_q // H, bs),
           QUEST_RTOL)
    kmin, kmax = ref.page_key_minmax(K, bt, cl, bs)
    meta = qm.meta.cpu().float()
    for b in range(B):
        for p in range(-(-int(cl[b]) // bs)):
            blk = int(bt[b, p])
            assert torch.equal(meta[blk, :, 0], kmin[b, p]), (b, p)
            assert torch.equal(meta[blk, :, 1], kmax[b, p]), (b, p)


@pytest.mark.parametrize("D,bs", GEOMETRIES)
@pytest.mark.parametrize("seed", [0, 3, 5])
def test_random_schedules_geometry(gpu, seed, D, bs):
    """Random shapes and schedules of the backend at other head dimensions
    and block sizes, ten steps with appends (crossing pages), in lockstep
    with the oracle backend."""
    cfg, kw = _random_schedule(seed)
    cfg["head_dim"] = D
    cfg["block_size"] = bs
    stats, trace, lock = _run(gpu, cfg, kw, steps=10, seed=700 + seed)
    print(f"seed {seed} D {D} bs {bs} {cfg} {kw}: {lock.summary()}")


@pytest.mark.parametrize("G,H,bs", [(12, 8, 16), (16, 4, 16), (10, 2, 32), (16, 1, 64),
                                    (32, 1, 16), (24, 4, 16), (40, 2, 32)])
def test_random_schedules_wide_groups(gpu, G, H, bs):
    """Backend schedules with 9..40 query heads per KV head (above 16: one
    decode launch per 16 of them)."""
    cfg, kw = _random_schedule(G + H)
    cfg.update(num_q_heads=H * G, num_kv_heads=H, block_size=bs,
               hot_heads=list(range(0, H, 2)))
    stats, trace, lock = _run(gpu, cfg, kw, steps=10, seed=800 + G)
    print(f"G {G} H {H} bs {bs} {cfg} {kw}: {lock.summary()}")


# KV-head counts outside the compiled-in set: a multiple of the rows of one
# wave load (64 / (D/8)) takes the head-group layout with the count as an
# argument, any other count the one-head-per-wave layout.
ANY_HKV = [  # (B, H_q, H_kv, ctx)
    (1, 96, 32, 3000),          # MHA-sized head count (G = 3)
    (2, 32, 32, [517, 2049]),   # G = 1, H_kv = 32
    (1, 36, 12, 1500),          # a multiple of 4 not compiled in
    (2, 18, 6, [800, 33]),      # neither a multiple nor a divisor of 4
    (1, 15, 3, 4096 + 5),
    (3, 35, 5, [17, 640, 2000]),
    (1, 7, 7, 999),
]


@pytest.mark.parametrize("D,bs", GEOMETRIES + [(128, 16)])
@pytest.mark.parametrize("geom", ANY_HKV)
def test_score_pages_any_kv_heads(gpu, geom, D, bs):
    B, H_q, H_kv, ctx = geom
    inp = make_paged_inputs(B, H_q, H_kv, D, ctx, block_size=bs, seed=300 + H_kv, device=gpu,
                            hot_heads=[0, H_kv - 1], n_hot=4, hot_shift=4.0)
    got = ops.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H_kv,
                          H_q // H_kv, bs).cpu()
    want = ref.score_pages(inp.q.cpu(), inp.k_cache.cpu(), inp.block_tables.cpu(),
                           inp.context_lens.cpu(), H_kv, H_q // H_kv, bs)
    _close(got, want, SCORE_RTOL)


@pytest.mark.parametrize("D,bs,H_kv,ctx", [(128, 16, 32, 65536), (128, 16, 6, 131072 - 3),
                                           (64, 32, 5, 65536), (256, 16, 3, 40000)])
def test_score_pages_any_kv_heads_long_context(gpu, D, bs, H_kv, ctx):
    """Several pages per wave in the layouts for any head count."""
    inp = make_paged_inputs(1, 2 * H_kv, H_kv, D, ctx, block_size=bs, seed=310 + H_kv,
                            device=gpu)
    got = ops.score_pages(inp.q, inp.k_cache, inp.block_tables, inp.context_lens, H_kv, 2,
                          bs).cpu()
    want = ref.score_pages(inp.q.cpu(), inp.k_cache.cpu(), inp.block_tables.cpu(),
                           inp.context_lens.cpu(), H_kv, 2, bs)
    _close(got, want, SCORE_RTOL)


@pytest.mark.parametrize("G,H,bs", [(1, 32, 16), (4, 6, 16), (2, 12, 32), (7, 3, 16),
                                    (1, 5, 64)])
def test_random_schedules_any_kv_heads(gpu, G, H, bs):
    """Backend schedules (step plans and the per-kernel path) at KV-head
    counts outside {1, 2, 4, 8, 16}, ten steps with appends, in lockstep
    with the oracle backend."""
    cfg, kw = _random_schedule(G * 7 + H)
    cfg.update(num_q_heads=H * G, num_kv_heads=H, block_size=bs,
               hot_heads=list(range(0, H, 2)))
    stats, trace, lock = _run(gpu, cfg, kw, steps=10, seed=900 + H)
    print(f"G {G} H {H} bs {bs} {cfg} {kw}: {lock.summary()}")
