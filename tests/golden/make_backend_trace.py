"""Write the golden backend traces: the reference CVSABackend run step by step.

Run in the build container only (needs /root/reference and its Triton
kernels, executed by the Triton interpreter on the CPU):

    python tests/golden/make_backend_trace.py

For every scenario of golden_inputs.SCENARIOS it drives the reference's
decode loop (backend call, step_done, one appended token per sequence via the
reference SequenceKVManager) and records, per call: the output bits, the
accept mask, the cached selection (as sorted sets: torch.topk(sorted=False)
leaves the order open), the expanded/complement selection, and the schedule
counters; at the end get_stats(), the block tables and context lengths.
Scenarios with ``record_state`` also keep, per scoring step, the coverage the
reference's coverage kernel returned and the log-sum-exp of the merged
result per query head (from the draft's and the complement's (m, l), as the
reference's LSE merge combines them), captured by wrapping the kernel
functions the reference backend calls.
Outputs: backend_trace_<scenario>.npz (arrays) and backend_trace.json
(stats, counters, input digests).  Nothing from the reference is stored
except these numbers.
"""
from __future__ import annotations

import json
import os
import sys

os.environ["TRITON_INTERPRET"] = "1"
HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = os.environ.get("CVSA_REFERENCE", "/root/reference")
sys.path.insert(0, HERE)
sys.path.insert(0, REFERENCE)

import numpy as np  # noqa: E402
import torch  # noqa: E402

from golden_inputs import SCENARIOS, input_digest, make_case  # noqa: E402
import cvsa.backend as reference_backend  # noqa: E402  (the reference package)
from cvsa.backend import CVSABackend  # noqa: E402
from cvsa.runtime.kv_cache import PagedKVCache, SequenceKVManager  # noqa: E402


def sorted_rows(t, n):
    """Per-(b,h) rows of t sorted ascending over the first n entries, -1 after."""
    t = t.to(torch.int64).clone()
    out = torch.full_like(t, -1)
    for b in range(t.shape[0]):
        for h in range(t.shape[1]):
            k = int(n[b, h])
            out[b, h, :k] = torch.sort(t[b, h, :k]).values
    return out.to(torch.int32).numpy()


class _Capture:
    """Wraps the reference backend's kernel entry points to keep what one
    call computed: the coverage and the (m, l) of the draft and complement
    sparse decodes."""

    def __init__(self, module):
        self.module = module
        self.calls = {}
        self.saved = {}
        for name in ("triton_check_coverage", "triton_sparse_decode_unnorm"):
            fn = getattr(module, name)
            self.saved[name] = fn
            setattr(module, name, self._wrap(name, fn))

    def _wrap(self, name, fn):
        def inner(*args, **kwargs):
            out = fn(*args, **kwargs)
            self.calls.setdefault(name, []).append(out)
            return out
        return inner

    def take(self):
        calls, self.calls = self.calls, {}
        return calls

    def restore(self):
        for name, fn in self.saved.items():
            setattr(self.module, name, fn)


def merged_lse(decodes, accept, G):
    """LSE per q-head: the draft's m + ln l on accepted heads, the
    log-add of the draft's and the complement's on rejected ones."""
    _, m_d, l_d = decodes[0]
    lse = m_d + torch.log(l_d)
    if len(decodes) > 1:
        _, m_c, l_c = decodes[1]
        lse_c = m_c + torch.log(l_c)
        lse_c = torch.where(torch.isnan(lse_c), torch.full_like(lse_c, -float("inf")), lse_c)
        both = torch.logaddexp(lse, lse_c)
        rej = ~accept.repeat_interleave(G, dim=1)
        lse = torch.where(rej, both, lse)
    return lse.to(torch.float32).numpy()


def run(name, sc):
    inp = sc["inputs"]
    case = make_case(**inp)
    B, H_q, H_kv, D = inp["batch"], inp["num_q_heads"], inp["num_kv_heads"], inp["head_dim"]
    nb = case.k_cache.shape[0]
    cache = PagedKVCache(nb, 16, H_kv, D, device="cpu")
    cache.k_cache.copy_(case.k_cache)
    cache.v_cache.copy_(case.v_cache)
    cache._next_free = case.next_free
    W = case.block_tables.shape[1]
    mgr = SequenceKVManager(cache, B, W * 16)
    mgr.block_tables.copy_(case.block_tables)
    mgr.context_lens.copy_(case.context_lens)
    mgr._pages_allocated = list(case.pages_allocated)
    backend = CVSABackend(H_kv, H_q, D, 16, **sc["backend"])
    capture = _Capture(reference_backend) if sc.get("record_state") else None
    arrays, counters = {}, []
    for s in range(inp["steps"]):
        out = backend(case.q[s], cache.k_cache, cache.v_cache, mgr.block_tables,
                      mgr.context_lens, 0)
        arrays[f"out_{s}"] = out.contiguous().view(torch.int16).numpy()
        if capture is not None:
            calls = capture.take()
            if "triton_check_coverage" in calls:
                acc, cov = calls["triton_check_coverage"][-1]
                arrays[f"cov_{s}"] = cov.to(torch.float32).numpy()
                arrays[f"lse_{s}"] = merged_lse(calls["triton_sparse_decode_unnorm"], acc,
                                                H_q // H_kv)
        acc = backend._last_accept_mask.get(0)
        if acc is not None:
            arrays[f"accept_{s}"] = acc.to(torch.uint8).numpy()
        if 0 in backend._cached_selection:
            pi, nph = backend._cached_selection[0]
            arrays[f"sel_{s}"] = sorted_rows(pi, nph)
            arrays[f"nph_{s}"] = nph.to(torch.int32).numpy()
        exp = backend._last_expanded_selection.get(0)
        if exp is not None:
            ei, en = exp
            if ei.dim() == 3:
                arrays[f"exp_{s}"] = sorted_rows(ei, en)
                arrays[f"expn_{s}"] = en.to(torch.int32).numpy()
        counters.append(dict(scoring=backend._total_scoring_steps,
                             checks=backend._total_coverage_checks,
                             accepts=backend._accept_counts, rejects=backend._reject_counts))
        backend.step_done(0, 1)
        for b in range(B):
            mgr.append_token_kv(b, case.k_new[s][b], case.v_new[s][b])
    if capture is not None:
        capture.restore()
    arrays["block_tables"] = mgr.block_tables.numpy()
    arrays["context_lens"] = mgr.context_lens.numpy()
    np.savez_compressed(os.path.join(HERE, f"backend_trace_{name}.npz"), **arrays)
    stats = {k: v for k, v in backend.get_stats().items()}
    return dict(digest=input_digest(case), stats=stats, counters=counters)


def main():
    """Regenerates every scenario, or only those named on the command line
    (the others keep their recorded entries)."""
    path = os.path.join(HERE, "backend_trace.json")
    meta = {}
    if os.path.exists(path):
        with open(path) as f:
            meta = json.load(f)
    names = sys.argv[1:] or list(SCENARIOS)
    for name in names:
        meta[name] = run(name, SCENARIOS[name])
        print(name, meta[name]["stats"], flush=True)
    with open(path, "w") as f:
        json.dump(meta, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
