"""Page-access traces (cvsa.tracing) in the reference's format
(scripts/collect_page_traces.py:49-156, :433-476).

CPU: the wrapper over the oracle backend, checked against what the trace
must be -- every valid page on a dense layer; the selection's pages where
every head of sequence 0 passed the gate; every valid page where one of its
heads was rejected under exact recovery (selection + complement); the rich
accept metadata equal to the backend's gate -- and a JSON round trip of the
reference's result layout.
GPU: the wrapper over the HIP backend records the same traces as over the
oracle backend run in lockstep.
"""
import pytest
import torch

from oracle import cvsa_oracle as ref
from oracle.backend_oracle import OracleCVSABackend
from cvsa.synthetic import jitter_query, make_paged_inputs
from cvsa.tracing import TracingWrapper, load_traces_json, save_traces_json, trace_result

L, STEPS = 3, 7
KW = dict(num_kv_heads=8, num_q_heads=32, head_dim=128, block_size=16, num_layers=L,
          budget_pct=0.25, coverage_threshold=0.9, lazy=True, check_interval=3,
          dense_layers=[2])


def _layer_inputs(device="cpu"):
    """Layer 0: hot pages on every head (gates pass); layer 1: on half the
    heads (gates reject some); layer 2 is dense."""
    heads = [list(range(8)), [0, 1, 2, 5], [0]]
    shift = [12.0, 7.0, 7.0]
    return [make_paged_inputs(2, 32, 8, 128, [1100, 700], seed=50 + l, device=device,
                              hot_heads=heads[l], n_hot=4, hot_shift=shift[l])
            for l in range(L)]


def _drive(backend, inps, device="cpu", after_call=None):
    tr = TracingWrapper(backend, 16, L, rich=True)
    for step in range(STEPS):
        for l, inp in enumerate(inps):
            q = jitter_query(inp.q, 0.3, 900 + 10 * step + l)
            args = [t.to(device) for t in (q, inp.k_cache, inp.v_cache, inp.block_tables,
                                           inp.context_lens)]
            tr(*args, l)
            if after_call is not None:
                after_call(step, l)
            tr.step_done(l, L)
    return tr


def test_traces_of_oracle_backend_follow_the_gate():
    inps = _layer_inputs()
    oracle = OracleCVSABackend(**KW)
    n_valid = int(ref.n_valid_pages(inps[0].context_lens, 16)[0])
    expected, counts = [], {"rejected": 0, "accepted": 0}

    def after_call(step, l):
        """What the trace of this call must be, from the oracle's state now."""
        rec = oracle.trace[-1]
        if rec["kind"] == "dense":
            expected.append((step, l, list(range(n_valid)), None))
            return
        idx, nph = oracle._cached_selection[l]
        sel = sorted({int(p) for h in range(8) for p in idx[0, h, :int(nph[0, h])]})
        rich = None
        if "accept" in rec:                    # a call that ran the coverage gate
            acc = rec["accept"][0]
            rich = {"accept_mask": acc.tolist(), "n_rejected": int((~acc).sum()),
                    "has_expanded": rec["kind"] == "score_exact"}
        if rec["kind"] == "score_exact" and not bool(rec["accept"][0].all()):
            expected.append((step, l, list(range(n_valid)), rich))   # selection + complement
            counts["rejected"] += 1
        else:
            expected.append((step, l, sel, rich))
            counts["accepted"] += rec["kind"] != "reuse"

    tr = _drive(oracle, inps, after_call=after_call)
    assert len(tr.traces) == STEPS and len(tr.rich_traces) == STEPS
    for step, l, pages, rich in expected:
        assert tr.traces[step][l] == pages, (step, l)
        assert tr.rich_traces[step].get(l) == rich, (step, l)
    assert counts["rejected"] and counts["accepted"], counts


def test_trace_file_round_trip(tmp_path):
    inps = _layer_inputs()
    tr = _drive(OracleCVSABackend(**KW), inps)
    sample = {"sample_idx": 0, "seq_len": 1100 + STEPS, "n_pages": 69,
              "n_steps": len(tr.traces), "traces": tr.traces, "rich_traces": tr.rich_traces}
    res = trace_result("cvsa_25_90_c3", [sample], model="synthetic", block_size=16,
                       num_layers=L, num_kv_heads=8, task="synthetic", max_steps=STEPS)
    path = tmp_path / "cvsa_25_90_c3.json"
    save_traces_json(str(path), {"cvsa_25_90_c3": res})
    back = load_traces_json(str(path))["cvsa_25_90_c3"]
    assert back == res
    assert set(back) == {"method", "model", "block_size", "num_layers", "num_kv_heads",
                         "task", "max_steps", "samples"}
    assert isinstance(next(iter(back["samples"][0]["traces"][0])), int)


@pytest.mark.gpu
def test_traces_of_hip_backend_equal_oracle_traces(gpu):
    from cvsa.backend import CVSABackend
    inps = _layer_inputs()
    gpu_tr = _drive(CVSABackend(**KW), inps, gpu)
    ora_tr = _drive(OracleCVSABackend(**KW), inps)
    assert gpu_tr.traces == ora_tr.traces
    assert gpu_tr.rich_traces == ora_tr.rich_traces
    assert any(r for step in gpu_tr.rich_traces for r in step.values()
               if r and r["n_rejected"])
