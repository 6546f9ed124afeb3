"""Page-access traces of a decode run, in the reference's trace format.

``TracingWrapper`` wraps an attention backend the way the reference's
wrapper does (scripts/collect_page_traces.py:49-156): it is called like the
backend, forwards ``step_done`` / ``reset`` / any other attribute, and after
every decode step (all layers done) appends ``{layer: sorted pages}`` to
``traces`` -- the logical pages of sequence 0 the backend attended at that
layer: every valid page for a dense backend or dense layer; for a CVSA
backend the union over KV heads of the cached selection, plus the expanded
(approximate recovery) or complement (exact recovery) pages of the heads the
coverage gate rejected at that call; every valid page before a layer's first
selection.  With ``rich=True`` it also appends, per step, ``{layer:
{"accept_mask": [H_kv bools], "n_rejected": int, "has_expanded": bool}}``
for the layers whose call ran a coverage gate.

The reference collects the pages with one host read per KV head; here each
layer call gathers them on the device and reads them once.

``trace_result`` builds one method's result in the reference's layout
(collect_page_traces.py:433-476: method, model, block_size, num_layers,
num_kv_heads, task, max_steps and a list of samples with sample_idx,
seq_len, n_pages, n_steps, traces and optional rich_traces).
``save_traces_pickle`` writes a run's results the way the reference's
collector does (collect_page_traces.py:466-478): ``{method}.pkl`` per method
and ``all_traces.pkl`` with every method, so the reference's readers
(eval/plot_recovery_heatmap.py:97-114) open them unchanged.  The files hold
only dicts, lists, ints, floats, strs, bools and None; ``save_traces_pickle``
refuses anything else, and ``load_traces_pickle`` reads them back with an
unpickler that refuses every global, so loading one executes nothing.
``save_traces_json`` / ``load_traces_json`` keep the same layout as JSON;
layer keys, which JSON stores as strings, are turned back into ints on
loading.
"""
from __future__ import annotations

import io
import json
import os
import pickle
from typing import Dict, List, Optional

import torch

from .runtime.dense import DenseAttentionBackend

__all__ = ["TracingWrapper", "trace_result", "save_traces_json", "load_traces_json",
           "save_traces_pickle", "load_traces_pickle"]


def _n_valid(context_lens: torch.Tensor, block_size: int) -> int:
    """n_valid of sequence 0 (collect_page_traces.py:73)."""
    return int(((context_lens[0].float() - 1) / block_size).long() + 1)


class TracingWrapper:
    """Records the pages a backend attends, per decode step and layer."""

    def __init__(self, backend, block_size: int, num_layers: int, rich: bool = False):
        self.backend = backend
        self.block_size = block_size
        self.num_layers = num_layers
        self.rich = rich
        self.traces: List[Dict[int, List[int]]] = []
        self.rich_traces: Optional[List[dict]] = [] if rich else None
        self._current_step: Dict[int, List[int]] = {}
        self._current_rich: Optional[dict] = {} if rich else None

    def __call__(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        n_valid = _n_valid(context_lens, self.block_size)
        output = self.backend(q, k_cache, v_cache, block_tables, context_lens, layer_idx)
        self._current_step[layer_idx] = self._extract_pages(layer_idx, n_valid)
        if self.rich:
            self._current_rich[layer_idx] = self._extract_rich(layer_idx)
        return output

    def _extract_pages(self, layer_idx: int, n_valid: int) -> List[int]:
        """Sorted logical pages of sequence 0 attended at this call."""
        b = self.backend
        if isinstance(b, DenseAttentionBackend) or not hasattr(b, "_cached_selection"):
            return list(range(n_valid))
        if layer_idx in getattr(b, "_dense_layers", ()):
            return list(range(n_valid))
        sel = b._cached_selection.get(layer_idx)
        if sel is None:
            return list(range(n_valid))   # before the layer's first selection
        page_indices, n_per_head = sel
        parts = [self._head_pages(page_indices[0], n_per_head[0])]
        exp = b._last_expanded_selection.get(layer_idx)
        accept = b._last_accept_mask.get(layer_idx)
        if exp is not None and accept is not None:
            exp_pi, exp_nph = exp
            rejected = ~accept[0].to(torch.bool).to(exp_nph.device)
            parts.append(self._head_pages(exp_pi[0], torch.where(
                rejected, exp_nph[0], torch.zeros_like(exp_nph[0]))))
        pages = torch.unique(torch.cat(parts))   # sorted
        return [int(p) for p in pages.cpu().tolist()]

    @staticmethod
    def _head_pages(idx: torch.Tensor, n: torch.Tensor) -> torch.Tensor:
        """The first n[h] entries of every row h of idx [H, k], flattened."""
        cols = torch.arange(idx.shape[1], device=idx.device).view(1, -1)
        keep = cols < n.to(idx.device).view(-1, 1).to(torch.long)
        return idx[keep].to(torch.long)

    def _extract_rich(self, layer_idx: int) -> Optional[dict]:
        """Accept metadata of sequence 0 (collect_page_traces.py:114-131)."""
        b = self.backend
        if not hasattr(b, "_last_accept_mask"):
            return None
        accept = b._last_accept_mask.get(layer_idx)
        if accept is None:
            return None
        mask = [bool(v) for v in accept[0].cpu().tolist()]
        has_exp = b._last_expanded_selection.get(layer_idx) is not None
        return {"accept_mask": mask, "n_rejected": sum(1 for v in mask if not v),
                "has_expanded": has_exp}

    def step_done(self, layer_idx: int, num_layers: int):
        self.backend.step_done(layer_idx, num_layers)
        if layer_idx == num_layers - 1:
            self.traces.append(dict(self._current_step))
            self._current_step = {}
            if self.rich:
                self.rich_traces.append(dict(self._current_rich))
                self._current_rich = {}

    def reset(self):
        self.backend.reset()
        self.traces = []
        self._current_step = {}
        if self.rich:
            self.rich_traces = []
            self._current_rich = {}

    def get_traces(self) -> List[Dict[int, List[int]]]:
        return self.traces

    def __getattr__(self, name):
        return getattr(self.backend, name)


def trace_result(method: str, samples: List[dict], *, model: str, block_size: int,
                 num_layers: int, num_kv_heads: int, task: str, max_steps: int) -> dict:
    """One method's result in the reference's layout; ``samples`` are dicts
    with sample_idx, seq_len, n_pages, n_steps, traces (and rich_traces)."""
    return {"method": method, "model": model, "block_size": block_size,
            "num_layers": num_layers, "num_kv_heads": num_kv_heads, "task": task,
            "max_steps": max_steps, "samples": samples}


def save_traces_json(path: str, results) -> None:
    """Write one result (or a {method: result} dict) as JSON."""
    with open(path, "w") as f:
        json.dump(results, f)


def _int_keys(steps):
    return [{int(k): v for k, v in step.items()} for step in steps]


def load_traces_json(path: str):
    """Read what save_traces_json wrote, with int layer keys again."""
    with open(path) as f:
        data = json.load(f)
    results = [data] if "samples" in data else list(data.values())
    for res in results:
        for s in res["samples"]:
            s["traces"] = _int_keys(s["traces"])
            if "rich_traces" in s:
                s["rich_traces"] = _int_keys(s["rich_traces"])
    return data


_PLAIN_SCALARS = (bool, int, float, str, type(None))


def _check_plain(obj, where: str = "result") -> None:
    """Raise TypeError unless obj is built from dicts, lists and scalars only
    (tuples and torch/numpy values would pickle as globals)."""
    if type(obj) in _PLAIN_SCALARS:
        return
    if type(obj) is list:
        for i, v in enumerate(obj):
            _check_plain(v, f"{where}[{i}]")
        return
    if type(obj) is dict:
        for k, v in obj.items():
            if type(k) not in _PLAIN_SCALARS:
                raise TypeError(f"{where}: key {k!r} of type {type(k).__name__}")
            _check_plain(v, f"{where}[{k!r}]")
        return
    raise TypeError(f"{where}: value of type {type(obj).__name__} is not a plain "
                    "dict/list/int/float/str/bool/None")


def save_traces_pickle(out_dir: str, results: Dict[str, dict]) -> List[str]:
    """Write ``{method}.pkl`` for every ``{method: result}`` entry and
    ``all_traces.pkl`` with all of them into out_dir (created if missing),
    as collect_page_traces.py:466-478 does; returns the paths written."""
    if not isinstance(results, dict) or not results:
        raise ValueError("results must be a non-empty {method: result} dict")
    for method, res in results.items():
        if not isinstance(method, str) or not method or os.sep in method:
            raise ValueError(f"method name {method!r} is not a file name")
        if not isinstance(res, dict) or res.get("method") != method:
            raise ValueError(f"result of {method!r} must be a trace_result dict "
                             "whose 'method' is that name")
        _check_plain(res, method)
    os.makedirs(out_dir, exist_ok=True)
    paths = []
    for method, res in results.items():
        path = os.path.join(out_dir, f"{method}.pkl")
        with open(path, "wb") as f:
            pickle.dump(res, f)
        paths.append(path)
    path = os.path.join(out_dir, "all_traces.pkl")
    with open(path, "wb") as f:
        pickle.dump(dict(results), f)
    paths.append(path)
    return paths


class _PlainUnpickler(pickle.Unpickler):
    """An unpickler that loads no class or function at all."""

    def find_class(self, module, name):
        raise pickle.UnpicklingError(f"trace files hold no globals ({module}.{name})")


def load_traces_pickle(path: str):
    """Read a ``{method}.pkl`` or ``all_traces.pkl``; refuses any file that
    names a global (class, function), so nothing in it is executed."""
    with open(path, "rb") as f:
        data = f.read()
    return _PlainUnpickler(io.BytesIO(data)).load()
