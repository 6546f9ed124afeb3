"""Replay of a golden backend trace (see tests/golden/make_backend_trace.py)
against a backend under test: the CPU oracle or the HIP path."""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
if GOLDEN not in sys.path:
    sys.path.insert(0, GOLDEN)

from golden_inputs import SCENARIOS, input_digest, make_case  # noqa: E402

OUT_ATOL = 2e-2


def load(name):
    with open(os.path.join(GOLDEN, "backend_trace.json")) as f:
        meta = json.load(f)[name]
    arrays = dict(np.load(os.path.join(GOLDEN, f"backend_trace_{name}.npz")))
    return meta, arrays


def _sorted_sets(idx, n):
    idx, n = idx.cpu().to(torch.int64), n.cpu()
    out = torch.full_like(idx, -1)
    for b in range(idx.shape[0]):
        for h in range(idx.shape[1]):
            k = int(n[b, h])
            out[b, h, :k] = torch.sort(idx[b, h, :k]).values
    return out.to(torch.int32).numpy()


COV_ATOL = 1e-3      # coverage (BASELINE north-star tolerance)
LSE_RTOL = 1e-3      # log-sum-exp of the merged result, relative


def replay(name, make_backend, make_runtime, counters_of, state_of=None, fused_call=None):
    """make_backend(kwargs) -> backend; make_runtime(case) -> (call_args_fn,
    append_fn, state_fn); counters_of(backend) -> dict like the recorded one.
    state_of(backend, call_args) -> (coverage [B, H_kv], lse [B, H_q]) of the
    backend's last scoring step, for scenarios that recorded them.
    fused_call(backend, q, k_rows, v_rows) -> output: when given, the append of
    step s's tokens (every sequence) and the call of step s + 1 are made by
    this one call (the order the reference takes, append then call), and the
    last step's append by append_fn."""
    sc = SCENARIOS[name]
    meta, arr = load(name)
    case = make_case(**sc["inputs"])
    assert input_digest(case) == meta["digest"], "golden inputs changed"
    inp = sc["inputs"]
    backend = make_backend(inp, sc["backend"])
    call_args, append, state = make_runtime(case)
    for s in range(inp["steps"]):
        if fused_call is not None and s > 0:
            out = fused_call(backend, case.q[s], case.k_new[s - 1], case.v_new[s - 1])
        else:
            out = backend(*call_args(case.q[s]), 0)
        want = torch.from_numpy(arr[f"out_{s}"]).view(torch.bfloat16).float()
        err = (out.detach().cpu().float() - want).abs().max().item()
        assert err <= OUT_ATOL, (name, s, err)
        acc = backend._last_accept_mask.get(0)
        assert (acc is None) == (f"accept_{s}" not in arr), (name, s, "accept presence")
        if acc is not None:
            assert np.array_equal(acc.cpu().to(torch.uint8).numpy(), arr[f"accept_{s}"]), \
                (name, s, "accept mask")
        if f"sel_{s}" in arr:
            pi, nph = backend._cached_selection[0]
            assert np.array_equal(nph.cpu().to(torch.int32).numpy(), arr[f"nph_{s}"]), (name, s)
            assert np.array_equal(_sorted_sets(pi, nph), arr[f"sel_{s}"]), (name, s, "selection")
        exp = backend._last_expanded_selection.get(0)
        assert (exp is None) == (f"exp_{s}" not in arr), (name, s, "expanded presence")
        if exp is not None:
            ei, en = exp
            assert np.array_equal(en.cpu().to(torch.int32).numpy(), arr[f"expn_{s}"]), (name, s)
            assert np.array_equal(_sorted_sets(ei, en), arr[f"exp_{s}"]), (name, s, "expanded")
        assert counters_of(backend) == meta["counters"][s], (name, s, "counters")
        if state_of is not None and f"cov_{s}" in arr:
            cov, lse = state_of(backend, call_args(case.q[s]))
            want_cov = torch.from_numpy(arr[f"cov_{s}"])
            want_lse = torch.from_numpy(arr[f"lse_{s}"])
            assert (cov.cpu().float() - want_cov).abs().max().item() < COV_ATOL, (name, s)
            rel = ((lse.cpu().float() - want_lse).abs() / want_lse.abs().clamp(min=1.0))
            assert rel.max().item() < LSE_RTOL, (name, s, "lse")
        backend.step_done(0, 1)
        if fused_call is None or s == inp["steps"] - 1:
            for b in range(inp["batch"]):
                append(b, case.k_new[s][b], case.v_new[s][b])
    bt, ctx = state()
    assert np.array_equal(bt, arr["block_tables"]) and np.array_equal(ctx, arr["context_lens"])
    stats = backend.get_stats()
    want = meta["stats"]
    assert set(stats) >= set(want), (name, sorted(stats), sorted(want))
    for k, v in want.items():
        assert stats[k] == v, (name, k, stats[k], v)
