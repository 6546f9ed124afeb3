"""Page-access traces (cvsa.tracing) in the reference's format
(scripts/collect_page_traces.py:49-156, :433-476).

CPU: the wrapper over the oracle backend, checked against what the trace
must be -- every valid page on a dense layer; the selection's pages where
every head of sequence 0 passed the gate; every valid page where one of its
heads was rejected under exact recovery (selection + complement); the rich
accept metadata equal to the backend's gate -- a JSON round trip of the
reference's result layout, and the reference's pickle files ({method}.pkl,
all_traces.pkl) read back by a restatement of the reference's consumer
(eval/plot_recovery_heatmap.py:97-141) through an unpickler that refuses
every global.
GPU: the wrapper over the HIP backend records the same traces as over the
oracle backend run in lockstep, and its pickle files equal the oracle's.
"""
import io
import math
import os
import pickle

import pytest
import torch

from oracle import cvsa_oracle as ref
from oracle.backend_oracle import OracleCVSABackend
from cvsa.synthetic import jitter_query, make_paged_inputs
from cvsa.tracing import (TracingWrapper, load_traces_json, load_traces_pickle,
                          save_traces_json, save_traces_pickle, trace_result)

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


def _result(tr, method):
    sample = {"sample_idx": 0, "seq_len": 1100 + STEPS, "n_pages": 69,
              "n_steps": len(tr.traces), "traces": tr.traces, "rich_traces": tr.rich_traces}
    return trace_result(method, [sample], model="synthetic", block_size=16, num_layers=L,
                        num_kv_heads=8, task="synthetic", max_steps=STEPS)


def _recovery_by_consumer(out_dir, method):
    """What eval/plot_recovery_heatmap.py:97-141 computes from the files: it
    opens {method}.pkl, else all_traces.pkl (then indexes it by the method
    key when the payload has no num_layers), and per sample, step and layer
    takes n_rejected / num_kv_heads (NaN where a layer has no entry)."""
    path = os.path.join(out_dir, f"{method}.pkl")
    if not os.path.exists(path):
        path = os.path.join(out_dir, "all_traces.pkl")
    payload = load_traces_pickle(path)
    if "num_layers" not in payload:
        payload = payload[method]
    n_layers, n_heads = int(payload["num_layers"]), int(payload["num_kv_heads"])
    out = []
    for sample in payload["samples"]:
        rich = sample.get("rich_traces", [])
        assert rich, "the consumer requires rich_traces"
        out.append([[float(step[l]["n_rejected"]) / n_heads if step.get(l) is not None
                     else math.nan for l in range(n_layers)] for step in rich])
    return out


def _same(a, b):
    return all(x == y or (math.isnan(x) and math.isnan(y))
               for ra, rb in zip(a, b) for sa, sb in zip(ra, rb) for x, y in zip(sa, sb))


def test_trace_pickles_read_by_the_reference_consumer(tmp_path):
    inps = _layer_inputs()
    tr = _drive(OracleCVSABackend(**KW), inps)
    method = "cvsa_ar20_c4_dL0"
    res = _result(tr, method)
    other = dict(res, method="dense", samples=[dict(res["samples"][0], rich_traces=[])])
    paths = save_traces_pickle(str(tmp_path), {method: res, "dense": other})
    assert sorted(os.path.basename(p) for p in paths) == ["all_traces.pkl", "cvsa_ar20_c4_dL0.pkl",
                                                          "dense.pkl"]
    # Both files load back unchanged, with int layer keys, through the
    # global-refusing unpickler and through plain pickle alike.
    assert load_traces_pickle(str(tmp_path / f"{method}.pkl")) == res
    both = load_traces_pickle(str(tmp_path / "all_traces.pkl"))
    assert both == {method: res, "dense": other}
    with open(tmp_path / "all_traces.pkl", "rb") as f:
        assert pickle.load(f) == both
    assert isinstance(next(iter(both[method]["samples"][0]["traces"][0])), int)
    # The consumer's recovery fractions equal the gate's rejections.
    want = [[[r[l]["n_rejected"] / 8 if r.get(l) is not None else math.nan
              for l in range(L)] for r in tr.rich_traces]]
    got = _recovery_by_consumer(str(tmp_path), method)
    assert _same(got, want)
    assert any(x > 0 for row in got[0] for x in row if not math.isnan(x))
    # The combined file alone serves the consumer too.
    os.remove(tmp_path / f"{method}.pkl")
    assert _same(_recovery_by_consumer(str(tmp_path), method), want)


def test_trace_pickles_hold_plain_values_only(tmp_path):
    inps = _layer_inputs()
    res = _result(_drive(OracleCVSABackend(**KW), inps), "m")
    bad = dict(res, samples=[dict(res["samples"][0], n_pages=torch.tensor(69))])
    with pytest.raises(TypeError):
        save_traces_pickle(str(tmp_path), {"m": bad})
    with pytest.raises(TypeError):
        save_traces_pickle(str(tmp_path), {"m": dict(res, max_steps=(STEPS,))})
    with pytest.raises(ValueError):
        save_traces_pickle(str(tmp_path), {"other": res})   # method key != result's method
    assert not os.listdir(tmp_path)                        # nothing written on refusal
    # A file naming any global is refused by the loader without running it.
    path = tmp_path / "evil.pkl"
    with open(path, "wb") as f:
        pickle.dump({"samples": [io.BytesIO]}, f)
    with pytest.raises(pickle.UnpicklingError):
        load_traces_pickle(str(path))


@pytest.mark.gpu
def test_traces_of_hip_backend_equal_oracle_traces(gpu, tmp_path):
    from cvsa.backend import CVSABackend
    inps = _layer_inputs()
    gpu_tr = _drive(CVSABackend(**KW), inps, gpu)
    ora_tr = _drive(OracleCVSABackend(**KW), inps)
    assert gpu_tr.traces == ora_tr.traces
    assert gpu_tr.rich_traces == ora_tr.rich_traces
    save_traces_pickle(str(tmp_path / "gpu"), {"m": _result(gpu_tr, "m")})
    save_traces_pickle(str(tmp_path / "ora"), {"m": _result(ora_tr, "m")})
    for name in ("m.pkl", "all_traces.pkl"):
        assert (load_traces_pickle(str(tmp_path / "gpu" / name))
                == load_traces_pickle(str(tmp_path / "ora" / name)))
    assert any(r for step in gpu_tr.rich_traces for r in step.values()
               if r and r["n_rejected"])
