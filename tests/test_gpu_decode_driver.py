"""The multi-layer decode driver (cvsa.runtime.decode_driver): graph-replayed
reuse steps are bit-identical to the eager per-layer protocol, step after
step with appends and scoring steps in between (each replay is checked
against the eager run), and leave the same schedule, statistics and tracing
state."""
import pytest
import torch

from cvsa.backend import CVSABackend
from cvsa.runtime.decode_driver import DecodeDriver, SyntheticDecodeLayers

pytestmark = pytest.mark.gpu

SHAPE = dict(num_layers=4, batch=2, num_q_heads=32, num_kv_heads=8, head_dim=128,
             context_len=[3000, 1700], max_new_tokens=24, seed=5, hot_heads=[0, 3, 6],
             n_hot=6, hot_shift=10.0)


def _pair(gpu, kw):
    runs = []
    for graphs in (False, True):
        layers = SyntheticDecodeLayers(device=gpu, **SHAPE)
        backend = CVSABackend(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                              num_layers=SHAPE["num_layers"], budget_pct=0.2,
                              coverage_threshold=0.9, **kw)
        runs.append((layers, backend, DecodeDriver(backend, layers, graphs=graphs)))
    return runs


@pytest.mark.parametrize("kw", [dict(lazy=True, check_interval=3),
                                dict(lazy=False, reuse_interval=2),
                                dict(lazy=True, check_interval=4, selector="quest")])
def test_graph_replay_equals_eager(gpu, kw):
    (la, ba, da), (lb, bb, db) = _pair(gpu, kw)
    for step in range(12):
        q, k, v = la.step_inputs(step)
        out_a = [o.clone() for o in da.step(q, k, v)]
        out_b = [o.clone() for o in db.step(q, k, v)]
        for layer, (a, b) in enumerate(zip(out_a, out_b)):
            assert torch.equal(a, b), (step, layer)
        for layer in range(SHAPE["num_layers"]):
            ma, mb = ba._last_accept_mask.get(layer), bb._last_accept_mask.get(layer)
            assert (ma is None) == (mb is None), (step, layer)
            if ma is not None:
                assert torch.equal(ma, mb), (step, layer)
        for ma, mb in zip(la.managers, lb.managers):
            assert torch.equal(ma.context_lens, mb.context_lens)
            assert torch.equal(ma.block_tables, mb.block_tables)
    assert db.captures >= 1 and db.replays >= 3, (db.captures, db.replays)
    assert ba._step == bb._step
    assert ba.get_stats() == bb.get_stats()


def test_driver_run_reports_latency(gpu):
    layers = SyntheticDecodeLayers(device=gpu, **dict(SHAPE, max_new_tokens=16))
    backend = CVSABackend(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16,
                          num_layers=SHAPE["num_layers"], budget_pct=0.2, lazy=True,
                          check_interval=5)
    res = DecodeDriver(backend, layers, graphs=True).run(steps=8, warmup=3)
    assert res["steps"] == 8 and len(res["per_step_ms"]) == 8
    assert 0 < res["median_ms"] <= res["p99_ms"]
    assert res["graph_replays"] >= 4
