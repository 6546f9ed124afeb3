"""Multi-layer decode driver with the reference harnesses' per-layer protocol.

The reference decode loops (eval/latency_benchmark.py:361-562,
eval/longbench_harness.py:323-391) run, for every generated token and every
layer: project q/k/v, append the token's K/V to the layer's paged cache
(SequenceKVManager.append_token_kv), call the attention backend on the
layer's cache, then ``step_done(layer, num_layers)``; a step's latency is
taken end to end with a synchronisation before it.  This driver runs the
same protocol over synthetic per-step q/k/v (no model weights: the layer's
output is not fed to the next layer, whose projections are synthetic too),
so it measures the attention path as the harness drives it: the batched
append, the backend's schedule and its host cost per layer call.

With ``graphs=True`` the layers run in chunks of ``graph_chunk``
consecutive layers: a chunk whose every layer call is a reuse step through
a step plan (``CVSABackend.reuse_plan_for``) is captured once as a HIP graph
and replayed for later such steps while each of its layers still maps to
the same plan: one launch per chunk instead of one validated host call per
layer.  The appends stay eager (their block ids come from the host
allocator); each layer's cache is its own, so only a layer's own append has
to precede its call: a chunk's appends are issued, then its replay, and the
host prepares the next chunk while the GPU runs this one (one graph for
every layer would leave the GPU idle while the host issues every append and
checks every plan first).  Replays repeat the calls' host bookkeeping
(``note_replayed_reuse``, ``step_done``), so schedule, counters and tracing
state match an eager run; outputs are bit-identical to it.

With ``fuse_append=True`` eager steps hand each layer's append to
``CVSABackend.call_with_append``, which folds it into a reuse step's decode
launch; with ``graphs=True`` as well, a chunk of such reuse steps is one
replay of its fused launches, which read the step's new rows from static
buffers and its append slots (block ids from the host allocator) from a
device buffer written just before the replay.
"""
from __future__ import annotations

import statistics
import time
from typing import List, Optional

import numpy as np
import torch

from ..synthetic import jitter_query, make_paged_inputs
from .kv_cache import PagedKVCache, SequenceKVManager


class SyntheticDecodeLayers:
    """Per-layer paged caches prefilled with synthetic K/V (independent seeds
    per layer, hot pages as in the benchmark inputs) and a generator of the
    per-step q / k / v of every layer."""

    def __init__(self, num_layers: int, batch: int, num_q_heads: int, num_kv_heads: int,
                 head_dim: int, context_len, max_new_tokens: int, block_size: int = 16,
                 seed: int = 0, device="cuda", **hot):
        self.num_layers = num_layers
        self.batch = batch
        self.num_q_heads = num_q_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.seed = seed
        self.device = torch.device(device)
        ctxs = [int(context_len)] * batch if isinstance(context_len, int) else list(context_len)
        extra_pages = -(-max_new_tokens // block_size) + 1
        self.caches: List[PagedKVCache] = []
        self.managers: List[SequenceKVManager] = []
        self.base_q: List[torch.Tensor] = []
        for layer in range(num_layers):
            inp = make_paged_inputs(batch, num_q_heads, num_kv_heads, head_dim, ctxs,
                                    block_size=block_size, seed=seed + 7919 * layer,
                                    device=self.device, spare_blocks=batch * extra_pages,
                                    **hot)
            nb = inp.k_cache.shape[0]
            cache = PagedKVCache(nb, block_size, num_kv_heads, head_dim, device=str(self.device))
            cache.k_cache.copy_(inp.k_cache)
            cache.v_cache.copy_(inp.v_cache)
            mgr = SequenceKVManager(cache, batch, max(ctxs) + max_new_tokens + block_size)
            mgr.adopt(inp.block_tables, inp.context_lens, inp.used_blocks)
            self.caches.append(cache)
            self.managers.append(mgr)
            self.base_q.append(inp.q)
            del inp

    def step_inputs(self, step: int):
        """q [L, B, H_q, D] and the new token's k, v [L, B, H_kv, D] of a step
        (bf16, deterministic in (seed, step))."""
        L, B = self.num_layers, self.batch
        q = torch.stack([jitter_query(self.base_q[l], 0.3, self.seed + 1000 * step + l)
                         for l in range(L)])
        g = torch.Generator(device=self.device).manual_seed(self.seed * 31 + step)
        kv = torch.randn(2, L, B, self.num_kv_heads, self.head_dim, generator=g,
                         device=self.device).to(torch.bfloat16)
        return q, kv[0], kv[1]


class DecodeDriver:
    """Runs decode steps of ``layers`` through ``backend`` with the
    reference per-layer protocol; see the module docstring."""

    def __init__(self, backend, layers: SyntheticDecodeLayers, graphs: bool = False,
                 stream: Optional[torch.cuda.Stream] = None, graph_chunk: int = 8,
                 fuse_append: bool = False):
        self.backend = backend
        self.layers = layers
        self.graphs = graphs
        # Eager steps hand each layer's append to the backend
        # (CVSABackend.call_with_append), which folds it into the decode
        # launch of a reuse step.
        self.fuse_append = bool(fuse_append) and hasattr(backend, "call_with_append")
        self.graph_chunk = max(1, int(graph_chunk))
        # Graph capture needs a stream other than the legacy default one, and
        # the step plans are bound to the stream they were made on: every
        # step of the driver runs on this one.
        self.stream = stream if stream is not None else torch.cuda.Stream(layers.device)
        L, B = layers.num_layers, layers.batch
        self.q_static = torch.empty(L, B, layers.num_q_heads, layers.head_dim,
                                    dtype=torch.bfloat16, device=layers.device)
        self._graphs = {}   # chunk index -> (graph, plans, output buffers)
        self.replays = 0
        self.captures = 0
        # Graphs with folded appends: the new rows in static buffers and each
        # chunk's append slots copied to the device before its replay (the
        # slots change every step; a captured launch's arguments do not).
        # Only the one-launch shapes of cvsa_sparse_decode_append take device
        # slots; other chunks run eagerly.
        self._fold_graphs = (self.graphs and self.fuse_append and layers.head_dim == 128
                             and layers.block_size == 16 and B <= 256
                             and layers.num_q_heads // layers.num_kv_heads <= 16)
        # Eager steps with folded appends read their inputs from static
        # buffers too, through per-layer views made once: a view made per
        # layer and step (indexing or unbind) costs the host more than the
        # folded call itself.
        self._static_eager = self.fuse_append and not self.graphs
        if self._fold_graphs or self._static_eager:
            shape = (L, B, layers.num_kv_heads, layers.head_dim)
            self.k_static = torch.empty(shape, dtype=torch.bfloat16, device=layers.device)
            self.v_static = torch.empty(shape, dtype=torch.bfloat16, device=layers.device)
            self._views = tuple(t.unbind(0) for t in (self.q_static, self.k_static,
                                                      self.v_static))
        if self._fold_graphs:
            self._slots = {}  # chunk index -> [device slots, pinned slots, event]
            # Sequences whose device slot a replayed launch refused (none
            # while the slots follow the managers); checked by run().
            self.slot_errors = torch.zeros(1, dtype=torch.int32, device=layers.device)

    # ------------------------------------------------------------ one step
    def _append(self, k, v, layers):
        for l in layers:
            self.layers.managers[l].append_tokens_kv(k[l], v[l])

    def _chunks(self):
        L, c = self.layers.num_layers, self.graph_chunk
        return [range(i, min(L, i + c)) for i in range(0, L, c)]

    def static_inputs(self):
        """The input buffers of the graph modes and of eager steps with
        folded appends (q [L, B, H_q, D], and with folded appends k / v [L,
        B, H_kv, D]; None where the mode has none).  A step given these
        tensors themselves reads them in place: a caller that makes its
        inputs there (as a captured model's projections would) saves the
        per-step copies into them."""
        if self._static_eager or self._fold_graphs:
            return self.q_static, self.k_static, self.v_static
        if not self.graphs:
            return None, None, None
        return self.q_static, None, None

    def _eager(self, q, k=None, v=None, layers=None) -> List[torch.Tensor]:
        """Per layer: the append of the new token (when k / v are given), the
        backend call, step_done -- the reference's order."""
        outs = []
        L = self.layers.num_layers
        if k is not None and self.fuse_append:
            call, done = self.backend.call_with_append, self.backend.step_done
            managers = self.layers.managers
            if self._static_eager or k is self.k_static:
                # The static buffers' per-layer views (inputs copied in
                # unless they were made there).
                for t, buf in zip((q, k, v), (self.q_static, self.k_static, self.v_static)):
                    if t is not buf:
                        buf.copy_(t)
                qs, ks, vs = self._views
            else:
                qs, ks, vs = q, k, v
            for l in (range(L) if layers is None else layers):
                outs.append(call(qs[l], ks[l], vs[l], managers[l], l))
                done(l, L)
            return outs
        for l in (range(L) if layers is None else layers):
            cache, mgr = self.layers.caches[l], self.layers.managers[l]
            if k is not None:
                mgr.append_tokens_kv(k[l], v[l])
            outs.append(self.backend(q[l], cache.k_cache, cache.v_cache, mgr.block_tables,
                                     mgr.context_lens, l))
            self.backend.step_done(l, L)
        return outs

    def _plans_now(self, layers):
        """The reuse plan of every layer in ``layers`` at the current step
        (None if one of them would not run a plan-driven reuse step)."""
        plans = []
        for l in layers:
            cache, mgr = self.layers.caches[l], self.layers.managers[l]
            p = self.backend.reuse_plan_for(self.q_static[l], cache.k_cache, cache.v_cache,
                                            mgr.block_tables, mgr.context_lens, l)
            if p is None:
                return None
            plans.append(p)
        return plans

    def step(self, q, k, v) -> List[torch.Tensor]:
        """One decode step: q [L, B, H_q, D], k / v [L, B, H_kv, D], made on
        the caller's current stream.  Returns the per-layer outputs, ready on
        that stream; in graph mode they may be the graph's output buffers,
        valid until the next step."""
        caller = torch.cuda.current_stream(self.layers.device)
        self.stream.wait_stream(caller)
        outs = self._step(q, k, v)
        caller.wait_stream(self.stream)
        return outs

    def _stage_slots(self, ci, chunk):
        """The append slots of every layer of a chunk (host mirrors) into the
        chunk's pinned slot buffer, which the chunk's graph copies to the
        device as its first node; the buffer is rewritten only once the
        previous replay of the chunk is done with it.  Returns the slot
        buffers and the mirrors' commit functions."""
        B = self.layers.batch
        st = self._slots.get(ci)
        if st is None:
            dev = torch.empty(len(chunk), B, 2, dtype=torch.int32, device=self.layers.device)
            pin = torch.empty(len(chunk), B, 2, dtype=torch.int32, pin_memory=True)
            st = self._slots[ci] = [dev, pin, torch.cuda.Event(), False]
        dev, pin, done, used = st
        if used:
            done.synchronize()
        host = pin.numpy()
        commits = []
        for j, l in enumerate(chunk):
            slots, commit = self.layers.managers[l].fused_append_slots()
            host[j] = np.frombuffer(slots, dtype=np.int32).reshape(B, 2)
            commits.append(commit)
        return dev, pin, done, commits

    def _fold_graph_step(self, k, v) -> List[torch.Tensor]:
        """Graph mode with folded appends: a chunk whose every layer is a
        plan-driven reuse step with appendable rows replays (or captures) its
        fused append-and-decode launches, which read the slots staged for
        this step; other chunks run eagerly through call_with_append."""
        if k is not self.k_static:
            self.k_static.copy_(k)
        if v is not self.v_static:
            self.v_static.copy_(v)
        L = self.layers.num_layers
        managers = self.layers.managers
        outs = []
        for ci, chunk in enumerate(self._chunks()):
            plans = self._plans_now(chunk)
            if plans is not None and not all(
                    managers[l].fusable_rows(self.k_static[l], self.v_static[l]) for l in chunk):
                plans = None
            if plans is None:
                outs += self._eager(self.q_static, self.k_static, self.v_static, layers=chunk)
                continue
            slots_dev, slots_pin, done, commits = self._stage_slots(ci, chunk)
            cached = self._graphs.get(ci)
            if cached is None or any(a is not b for a, b in zip(plans, cached[1])):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=self.stream):
                    slots_dev.copy_(slots_pin, non_blocking=True)
                    chunk_outs = [
                        p.run_reuse_append(self.q_static[l], self.k_static[l], self.v_static[l],
                                           managers[l]._pages_allocated_dev,
                                           slots_dev=slots_dev[j],
                                           slot_errors=self.slot_errors)
                        for j, (p, l) in enumerate(zip(plans, chunk))]
                graph.replay()
                self._graphs[ci] = (graph, plans, chunk_outs)
                self.captures += 1
            else:
                cached[0].replay()
                self.replays += 1
                chunk_outs = cached[2]
            done.record(self.stream)
            self._slots[ci][3] = True
            for commit in commits:
                commit()
            for l in chunk:
                self.backend.note_replayed_reuse(l)
                self.backend.step_done(l, L)
            outs += chunk_outs
        return outs

    def _step(self, q, k, v) -> List[torch.Tensor]:
        with torch.cuda.stream(self.stream):
            if not self.graphs:
                return self._eager(q, k, v)
            if q is not self.q_static:
                self.q_static.copy_(q)
            if self._fold_graphs:
                return self._fold_graph_step(k, v)
            # Graph mode, chunk by chunk: the chunk's appends, then its
            # calls -- replayed when every layer of the chunk maps to the
            # plans its graph was captured with, else captured (host
            # bookkeeping now, kernels at the replay) or, when a layer takes
            # another path, made eagerly.
            L = self.layers.num_layers
            outs = []
            for ci, chunk in enumerate(self._chunks()):
                self._append(k, v, chunk)
                plans = self._plans_now(chunk)
                if plans is None:
                    outs += self._eager(self.q_static, layers=chunk)
                    continue
                cached = self._graphs.get(ci)
                if cached is None or any(a is not b for a, b in zip(plans, cached[1])):
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph, stream=self.stream):
                        chunk_outs = self._eager(self.q_static, layers=chunk)
                    graph.replay()
                    self._graphs[ci] = (graph, plans, chunk_outs)
                    self.captures += 1
                    outs += chunk_outs
                    continue
                cached[0].replay()
                self.replays += 1
                for l in chunk:
                    self.backend.note_replayed_reuse(l)
                    self.backend.step_done(l, L)
                outs += cached[2]
            return outs

    # ------------------------------------------------------------ timing
    def run(self, steps: int, warmup: int = 5, first_step: int = 0):
        """The reference's timed decode (latency_benchmark.py:478-520):
        warmup steps, a counter reset, then per-step end-to-end latency with
        a synchronisation before each step.  Inputs of every step are made
        before its timing starts."""
        times, host = [], []
        static = self.static_inputs()
        for i in range(warmup + steps):
            s = first_step + i
            q, k, v = self.layers.step_inputs(s)
            # Graph modes read their inputs from fixed buffers: the inputs
            # are made there, as a captured model's projections would.
            q, k, v = [t if buf is None else buf.copy_(t) for t, buf in zip((q, k, v), static)]
            torch.cuda.synchronize()
            if i == warmup and hasattr(self.backend, "_accept_counts"):
                self.backend._accept_counts = 0
                self.backend._reject_counts = 0
                self.backend._total_scoring_steps = 0
                self.backend._per_head_accept_sum = 0
                self.backend._per_head_total = 0
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record(self.stream)
            t0 = time.perf_counter()
            self.step(q, k, v)
            t1 = time.perf_counter()
            end.record(self.stream)
            torch.cuda.synchronize()
            if i >= warmup:
                times.append(start.elapsed_time(end))
                host.append((t1 - t0) * 1e3)
        if self._fold_graphs:
            bad = int(self.slot_errors.item())
            if bad:
                raise RuntimeError(f"decode driver: {bad} device append slots were refused "
                                   "(the slots no longer follow the managers)")
        ms = sorted(times)
        B = self.layers.batch
        return {
            "steps": steps, "warmup": warmup,
            "mean_ms": statistics.mean(times), "median_ms": statistics.median(times),
            "p95_ms": ms[min(len(ms) - 1, int(0.95 * len(ms)))],
            "p99_ms": ms[min(len(ms) - 1, int(0.99 * len(ms)))],
            "tokens_per_sec": B * 1000.0 / statistics.mean(times),
            "per_step_ms": times,
            "host_ms_mean": statistics.mean(host),   # time to issue a step
            "graph_replays": self.replays, "graph_captures": self.captures,
        }
