"""Coverage-Verified Sparse Attention (CVSA) backend on MI355X.

Sparse attention as draft, coverage as acceptance criterion, and recovery on
low-coverage heads.  Drop-in for the reference's cvsa/backend.py
(CVSABackend :45-881): same constructor keywords and defaults, the same
backend protocol (``__call__``, ``reset``, ``step_done``, ``get_stats``,
``enable_timing``), the same scheduling (fixed interval R, lazy check every
M steps, optional coverage-only steps), the same statistics keys and the
tracing attributes ``_cached_selection``, ``_last_accept_mask``,
``_last_expanded_selection`` and ``_dense_layers``.

What runs per layer call (HIP kernels from cvsa.ops):
  scoring step  score_pages -> select_topk (+ coverage gate) -> verified_decode
  lazy check    score_pages -> check_coverage -> select_or_keep -> verified_decode
  reuse step    sparse decode over the cached selection
These sequences run from a native step plan (ops.StepPlan), the first
selection of a layer included: one host call per step instead of one
validated call per kernel, while the caches, tables, counters and stream
stay the same.
The reference's draft decode, complement, complement decode and LSE merge
collapse into verified_decode: accepted heads attend their selected pages,
rejected heads attend every valid page in one pass, which equals the LSE
merge of draft and complement.  The lazy accept-all decision is taken on
the device (select_or_keep keeps the cached selection or refreshes it in
place), and the statistics counters and effective-budget counters are
accumulated there too, so a lazy decode step never waits for the host.
Approximate recovery (approx_recovery_pct) runs through the step plans as
well: the selection kernel writes each rejected row's expanded selection
and the verified decode attends it (ops.verified_decode_approx), so the
reference's deployed setting (budget 5%, tau 0.9, M=4, ar20, dense layer 0)
takes no host read either.  Host reads remain where the reference's result
needs one: the random-rejection counterfactual, coverage-only steps, the
per-head budget selectors and the per-kernel path (timing enabled).

The Quest selector (selector="quest", cvsa/backend.py:572-620) ranks pages
by per-page key min/max metadata that is recomputed only for the pages
whose valid-token count changed (ops.QuestPageMeta) rather than gathered
from the whole cache; with light_normalizer its scores also drive the
coverage gate, so no step reads all keys.  A lazy check on the device asks
for the ranking scores with its flags: they are computed only when some
head failed.

Per-head budgets: ``top_p`` (the smallest page set per head whose softmax
mass over the ranking scores reaches top_p, backend.py:652-681),
``static_budget_table`` (offline per-head fractions, :622-650) and
``adaptive_selection`` (heads compete for H_kv * budget slots, :522-570)
select through ops.select_budgeted with the new selection's gate fused;
like the reference they read the largest budget on the host (top-p,
adaptive) and take the per-kernel path.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Set, Tuple

import ctypes
import weakref

import torch

from . import ops
from .runtime.dense import DenseAttentionBackend


class _PendingComplement:
    """Complement pages of a scoring step, computed only if someone reads
    ``_last_expanded_selection`` (the reference builds them eagerly)."""

    __slots__ = ("accept", "page_indices", "n_per_head", "context_lens", "block_size")

    def __init__(self, accept, page_indices, n_per_head, context_lens, block_size):
        self.accept = accept
        self.page_indices = page_indices
        self.n_per_head = n_per_head
        self.context_lens = context_lens
        self.block_size = block_size

    def resolve(self):
        if bool(self.accept.all()):
            return None
        return ops.compute_complement(self.page_indices, self.n_per_head, self.context_lens,
                                      self.block_size, self.accept)


class _PendingExpanded:
    """Expanded selection of an approximate-recovery step, computed only if
    someone reads ``_last_expanded_selection`` (backend.py:780-815: the
    top exp_budget pages of every row by the ranking scores, present when a
    head was rejected)."""

    __slots__ = ("accept", "scores", "exp_budget", "context_lens", "block_size")

    def __init__(self, accept, scores, exp_budget, context_lens, block_size):
        self.accept = accept
        self.scores = scores
        self.exp_budget = exp_budget
        self.context_lens = context_lens
        self.block_size = block_size

    def resolve(self):
        if bool(self.accept.all()):
            return None
        return ops.select_topk(self.scores, self.exp_budget, self.context_lens,
                               self.block_size)


class _FusedReuse:
    """A layer's reuse step with the token append folded in
    (cvsa_step_plan_run_append), checked in full once by call_with_append.
    A later call only compares identities (the layer's plan, selection,
    scores, counters, the manager's buffers, the stream) and the layout of
    q and the new rows with the ones checked; any difference sends the call
    back to the checked path.  The slots go through one ctypes array."""

    __slots__ = ("plan", "manager", "pages_dev", "kv_shape", "dev_index", "out_args",
                 "slots", "fn", "handle", "stream", "new_stride")

    def __init__(self, plan, manager, k_new):
        self.plan = plan
        self.manager = manager
        self.pages_dev = manager._pages_allocated_dev
        self.kv_shape = k_new.shape
        self.dev_index = plan.dev.index
        self.out_args = (plan.out_shape, plan.dev, plan.out_dtype)
        self.slots = (ctypes.c_int32 * (2 * manager.batch_size))()
        self.fn = plan._run_append
        self.handle = plan._h
        self.stream = plan.stream
        self.new_stride = k_new.stride(0)

    def fits(self, backend, q, k_new, v_new, layer_idx) -> bool:
        plan = self.plan
        m = self.manager
        cache = m.cache
        r = plan.refs
        if (backend._step_plans.get(layer_idx) is not plan or backend._track_timing
                or r[0] is not cache.k_cache or r[1] is not cache.v_cache
                or r[2] is not m.block_tables or r[3] is not m.context_lens
                or r[4] is not backend._work_buf or r[5] is not backend._dev_stats
                or m._pages_allocated_dev is not self.pages_dev):
            return False
        sel = backend._cached_selection.get(layer_idx)
        cached = backend._cached_page_scores.get(layer_idx)
        if (sel is None or sel[0] is not plan.page_indices
                or not (cached is plan.scores_cache or cached is plan.page_scores)):
            return False
        if r[7] is not None and backend._plan_selector(cache.k_cache)[1] is not r[7]:
            return False
        bf16 = torch.bfloat16
        idx = self.dev_index
        return (q.dtype is plan.out_dtype and (q.shape, q.stride()) == plan.q_meta
                and q.get_device() == idx and k_new.dtype is bf16 and v_new.dtype is bf16
                and k_new.shape == self.kv_shape and v_new.shape == self.kv_shape
                and k_new.get_device() == idx and v_new.get_device() == idx
                and k_new.is_contiguous() and v_new.is_contiguous()
                and torch._C._cuda_getCurrentRawStream(idx) == self.stream)

    def run(self, q, k_new, v_new):
        """The launch, or None when a pointer is not 16-byte aligned."""
        qp, kp, vp = q.data_ptr(), k_new.data_ptr(), v_new.data_ptr()
        if (qp | kp | vp) & 15:
            return None
        m = self.manager
        need = m.fill_fused_slots(self.slots)
        shape, dev, dtype = self.out_args
        out = torch.empty(shape, device=dev, dtype=dtype)
        rc = self.fn(self.handle, qp, out.data_ptr(), kp, vp, self.new_stride,
                     self.pages_dev.data_ptr(), self.slots, None, None, self.stream)
        if rc != 0:
            ops.check(rc, "step_plan_run_append")
        m.commit_fused(need)
        return out


def _device_counter(slot: int, host_name: str):
    """A statistics counter kept partly on the host and partly in slot `slot`
    of the device counter block (accumulated by the lazy decision kernel).
    Reading it synchronises; assigning it (as evaluation harnesses do to
    reset the counters) sets the host part and clears the device part."""

    def fget(self):
        value = getattr(self, host_name)
        if self._dev_stats is not None:
            value += int(self._dev_stats[slot].item())
        return value

    def fset(self, value):
        setattr(self, host_name, value)
        if self._dev_stats is not None:
            self._dev_stats[slot].zero_()

    return property(fget, fset)


class CVSABackend:
    """Draft with sparse attention, verify with coverage, recover rejected heads."""

    _accept_counts = _device_counter(0, "_h_accept_counts")
    _reject_counts = _device_counter(1, "_h_reject_counts")
    _total_scoring_steps = _device_counter(2, "_h_total_scoring_steps")
    _per_head_accept_sum = _device_counter(3, "_h_per_head_accept_sum")

    def __init__(
        self,
        num_kv_heads: int,
        num_q_heads: int,
        head_dim: int,
        block_size: int,
        num_layers: int = 32,
        budget_pct: float = 0.10,
        reuse_interval: int = 16,
        coverage_threshold: float = 0.90,
        dense_layers: Optional[List[int]] = None,
        lazy: bool = False,
        check_interval: Optional[int] = None,
        coverage_interval: Optional[int] = None,
        approx_recovery_pct: Optional[float] = None,
        adaptive_selection: bool = False,
        adaptive_floor_ratio: float = 0.5,
        random_reject_prob: Optional[float] = None,
        static_budget_table: Optional[Dict[int, List[float]]] = None,
        selector: str = "exact",
        top_p: Optional[float] = None,
        light_normalizer: bool = False,
    ):
        self.num_kv_heads = num_kv_heads
        self.num_q_heads = num_q_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.num_layers = num_layers
        self.num_q_per_kv = num_q_heads // num_kv_heads
        self.budget_pct = budget_pct
        self.reuse_interval = reuse_interval
        self.tau = coverage_threshold

        self._dense_layers: Set[int] = set(dense_layers or [])
        self._dense_backend = None
        if self._dense_layers:
            self._dense_backend = DenseAttentionBackend(num_kv_heads, num_q_heads, head_dim,
                                                        block_size)
        self.approx_recovery_pct = approx_recovery_pct
        self.lazy = lazy
        self.check_interval = check_interval or 1
        self.coverage_interval = coverage_interval or self.check_interval
        self.adaptive_selection = adaptive_selection
        self.adaptive_floor_ratio = adaptive_floor_ratio
        self.random_reject_prob = random_reject_prob
        self.static_budget_table = None
        if static_budget_table is not None:
            self.static_budget_table = {int(layer): torch.as_tensor(f, dtype=torch.float32)
                                        for layer, f in static_budget_table.items()}
        # Validation in the reference's order (backend.py:150-151, 163-166, 176-177).
        if selector not in ("exact", "quest"):
            raise ValueError(f"Unknown selector: {selector!r}")
        self.selector = selector
        if light_normalizer and selector != "quest":
            raise ValueError(
                "light_normalizer=True requires selector='quest' "
                "(the sketch supplies both selection and normalizer)")
        self.light_normalizer = light_normalizer
        if top_p is not None and not (0.0 < top_p < 1.0):
            raise ValueError(f"top_p must be in (0, 1), got {top_p}")
        self.top_p = top_p
        # Row budgets of the static table on the device, per (layer, B, W).
        self._table_budgets: Dict[tuple, Tuple[torch.Tensor, int]] = {}
        # Quest metadata per key cache (keyed by id, with a weak reference to
        # tell a reused id from the cache it was built for).
        self._quest_meta: Dict[int, Tuple[weakref.ref, ops.QuestPageMeta]] = {}

        self._last_accept_mask: Dict[int, Optional[torch.Tensor]] = {}
        # (gate scores, per-head accept) of the coverage check of a layer's
        # cached selection in its last call, when that call ran one (lazy
        # check or coverage-only step); views of live buffers, read them
        # before the layer's next call.
        self._last_check: Dict[int, Tuple[torch.Tensor, torch.Tensor]] = {}
        # Ranking scores of a layer's new selection in its last call, when
        # they differ from the gate's (the Quest selector with the exact gate).
        self._last_rank_scores: Dict[int, torch.Tensor] = {}
        self._expanded_store: Dict[int, object] = {}
        self._attn_work: Optional[torch.Tensor] = None
        self._attn_work_max: Optional[torch.Tensor] = None
        self._work_buf: Optional[torch.Tensor] = None
        self._dev_stats: Optional[torch.Tensor] = None

        self._step = 0
        self._reuse_state: Dict[int, Tuple[torch.Tensor, torch.Tensor, int]] = {}
        self._reuse_plans: Dict[int, ops.DecodeCall] = {}
        self._step_plans: Dict[int, ops.StepPlan] = {}
        self._fused: Dict[int, _FusedReuse] = {}
        self._cached_selection: Dict[int, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._cached_page_scores: Dict[int, torch.Tensor] = {}

        self._accept_counts = 0
        self._reject_counts = 0
        self._total_scoring_steps = 0
        self._total_coverage_checks = 0
        self._per_head_accept_sum = 0
        self._per_head_total = 0
        self._dense_layer_steps = 0

        self._track_timing = False
        self._kernel_times_ms: Dict[str, float] = {
            "scoring": 0.0, "coverage": 0.0, "sparse_draft": 0.0,
            "ar_recovery": 0.0, "lse_merge": 0.0, "complement": 0.0,
        }
        self._kernel_counts: Dict[str, int] = {k: 0 for k in self._kernel_times_ms}
        self._pending_events: list = []

    # ------------------------------------------------------------ tracing
    @property
    def _last_expanded_selection(self) -> Dict[int, Optional[Tuple[torch.Tensor, torch.Tensor]]]:
        """Expanded (approximate recovery) or complement (exact recovery) pages
        of the last scoring step per layer, present only when a head was
        rejected (backend.py:815, :842).  Complements are built on first read."""
        for layer in list(self._expanded_store):
            v = self._expanded_store[layer]
            if isinstance(v, (_PendingComplement, _PendingExpanded)):
                v = v.resolve()
                if v is None:
                    del self._expanded_store[layer]
                    continue
                self._expanded_store[layer] = v
        return dict(self._expanded_store)

    # ------------------------------------------------------------ timing
    def enable_timing(self, track: bool = True):
        """Per-kernel event timing on/off (backend.py:225-228)."""
        self._track_timing = track

    def _time_kernel(self, name: str, fn, *args, **kwargs):
        if not self._track_timing:
            return fn(*args, **kwargs)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        result = fn(*args, **kwargs)
        end.record()
        self._pending_events.append((name, start, end))
        return result

    def _flush_timing(self):
        if not self._track_timing or not self._pending_events:
            return
        torch.cuda.synchronize()
        for name, start, end in self._pending_events:
            self._kernel_times_ms[name] += start.elapsed_time(end)
            self._kernel_counts[name] += 1
        self._pending_events.clear()

    # ------------------------------------------------------------ protocol
    def reset(self):
        """backend.py:252-272"""
        self._step = 0
        self._reuse_state = {}
        self._reuse_plans = {}
        self._fused = {}
        # Step plans that own their selection stay: the next first selection
        # of their layer is made in their buffers again.
        self._step_plans = {k: p for k, p in self._step_plans.items() if p.owns_selection}
        # Quest metadata objects (and the plans that use them) stay, but
        # forget every block: a new sequence may rewrite the cache.
        for ref, meta in list(self._quest_meta.values()):
            if ref() is None:
                continue
            meta.invalidate()
        self._quest_meta = {k: e for k, e in self._quest_meta.items() if e[0]() is not None}
        self._cached_selection = {}
        self._cached_page_scores = {}
        self._last_accept_mask = {}
        self._last_check = {}
        self._last_rank_scores = {}
        self._expanded_store = {}
        if self._attn_work is not None:
            self._attn_work.zero_()
            self._attn_work_max.zero_()
        self._accept_counts = 0
        self._reject_counts = 0
        self._total_scoring_steps = 0
        self._total_coverage_checks = 0
        self._per_head_accept_sum = 0
        self._per_head_total = 0
        self._dense_layer_steps = 0
        for k in self._kernel_times_ms:
            self._kernel_times_ms[k] = 0.0
            self._kernel_counts[k] = 0
        self._pending_events.clear()

    @property
    def is_scoring_step(self):
        return self._step % self.reuse_interval == 0

    def step_done(self, layer_idx: int, num_layers: int):
        if layer_idx == num_layers - 1:
            self._step += 1

    def get_stats(self) -> dict:
        """Same keys and formulas as backend.py:282-311."""
        accepts, rejects, scoring, head_accepts = self._counters()
        total_checks = max(self._total_coverage_checks, scoring, 1)
        stats = {
            "total_scoring_steps": scoring,
            "total_coverage_checks": self._total_coverage_checks,
            "all_accepted_pct": accepts / max(total_checks, 1) * 100,
            "some_rejected_pct": rejects / max(total_checks, 1) * 100,
            "per_head_accept_rate": head_accepts / max(self._per_head_total, 1) * 100,
            "total_decode_steps": self._step,
            "lazy": self.lazy,
            "check_interval": self.check_interval if self.lazy else None,
            "rescore_rate": (scoring / max(self._total_coverage_checks, 1) * 100
                             if self.lazy else 100.0),
        }
        if self._attn_work is not None:
            pages_attended = int(self._attn_work.item())
            pages_max = int(self._attn_work_max.item())
            if pages_max > 0:
                stats["effective_budget_pct"] = pages_attended / pages_max * 100
                stats["total_pages_attended"] = pages_attended
                stats["total_pages_max"] = pages_max
        if self._track_timing:
            self._flush_timing()
            n_decode = max(self._step, 1)
            stats["kernel_times_ms_total"] = dict(self._kernel_times_ms)
            stats["kernel_counts"] = dict(self._kernel_counts)
            stats["kernel_ms_per_decode_step"] = {
                k: self._kernel_times_ms[k] / n_decode for k in self._kernel_times_ms}
        return stats

    def __call__(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """backend.py:313-366"""
        self._last_accept_mask.pop(layer_idx, None)
        self._last_check.pop(layer_idx, None)
        self._last_rank_scores.pop(layer_idx, None)
        self._expanded_store.pop(layer_idx, None)

        if layer_idx in self._dense_layers:
            # Dense attends every valid page on every head (:327-333).
            self._dense_layer_steps += 1
            work = self._decode_work(context_lens)
            out = self._dense_backend(q, k_cache, v_cache, block_tables, context_lens,
                                      layer_idx, work=work)
            if work is None:
                n_valid = ((context_lens.float() - 1) / self.block_size).long() + 1
                self._record_work(context_lens, n_valid.sum() * self.num_kv_heads)
            return out

        if self.lazy:
            is_scoring_step = self._step % self.check_interval == 0
            is_coverage_step = self._step % self.coverage_interval == 0
            has_cache = layer_idx in self._reuse_state
            has_scores = layer_idx in self._cached_page_scores
            if is_scoring_step:
                return self._lazy_step(q, k_cache, v_cache, block_tables, context_lens,
                                       layer_idx)
            elif is_coverage_step and has_cache and has_scores:
                return self._coverage_only_step(q, k_cache, v_cache, block_tables,
                                                context_lens, layer_idx)
            elif has_cache:
                return self._reuse_step(q, k_cache, v_cache, block_tables, context_lens,
                                        layer_idx)
            else:
                return self._lazy_step(q, k_cache, v_cache, block_tables, context_lens,
                                       layer_idx)
        elif self.is_scoring_step:
            return self._scoring_step(q, k_cache, v_cache, block_tables, context_lens,
                                      layer_idx)
        else:
            return self._reuse_step(q, k_cache, v_cache, block_tables, context_lens, layer_idx)

    # ------------------------------------------------------------ graph replay
    def reuse_plan_for(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """The step plan this call would run as a reuse step at the current
        step, or None when the call would score, check, or take another
        path.  A reuse step through a plan is device work only (its counters
        accumulate on the device), so a caller may capture it in a graph and
        replay it for later reuse steps while this keeps returning the same
        plan, calling ``note_replayed_reuse`` and ``step_done`` per replayed
        call."""
        if layer_idx in self._dense_layers or layer_idx not in self._reuse_state:
            return None
        if self.lazy:
            if self._step % self.check_interval == 0:
                return None
            if (self._step % self.coverage_interval == 0
                    and layer_idx in self._cached_page_scores):
                return None
        elif self.is_scoring_step:
            return None
        return self._matching_plan(layer_idx, q, k_cache, v_cache, block_tables, context_lens)

    def _plain_reuse_step(self, layer_idx) -> bool:
        """Whether a call of this layer at the current step is a reuse step
        (the schedule of __call__, backend.py:313-366)."""
        if layer_idx in self._dense_layers or layer_idx not in self._reuse_state:
            return False
        step = self._step
        if self.lazy:
            return not (step % self.check_interval == 0
                        or (step % self.coverage_interval == 0
                            and layer_idx in self._cached_page_scores))
        return step % self.reuse_interval != 0

    def call_with_append(self, q, k_new, v_new, manager, layer_idx):
        """The decode loops' append then call (``manager.append_tokens_kv(k_new,
        v_new)``, then this backend on the manager's cache, tables and context
        lengths), with the append folded into the decode launch when the call
        is a reuse step through a step plan (cvsa_step_plan_run_append);
        otherwise the two in turn.  Same outputs, cache, tables, context
        lengths and statistics either way; no counterpart in the reference.
        The first folded call of a layer is checked in full; later ones reuse
        that check while the plan, buffers, stream and layouts stay the same
        (a decode loop's per-layer host cost)."""
        fc = self._fused.get(layer_idx)
        if (fc is not None and fc.manager is manager and self._plain_reuse_step(layer_idx)
                and fc.fits(self, q, k_new, v_new, layer_idx)):
            out = fc.run(q, k_new, v_new)
            if out is not None:
                self.note_replayed_reuse(layer_idx)
                return out
        cache = manager.cache
        args = (cache.k_cache, cache.v_cache, manager.block_tables, manager.context_lens)
        plan = None
        if manager.fusable_rows(k_new, v_new):
            plan = self.reuse_plan_for(q, *args, layer_idx)
        if plan is None:
            manager.append_tokens_kv(k_new, v_new)
            return self(q, *args, layer_idx)
        slots, commit = manager.fused_append_slots()
        out = plan.run_reuse_append(q, k_new, v_new, manager._pages_allocated_dev, slots)
        commit()
        self._fused[layer_idx] = _FusedReuse(plan, manager, k_new)
        self.note_replayed_reuse(layer_idx)
        return out

    def note_replayed_reuse(self, layer_idx: int) -> None:
        """Host bookkeeping of a reuse call that was replayed from a graph
        instead of made (backend.py:313-321: the call clears the layer's
        accept mask and expanded selection)."""
        self._last_accept_mask.pop(layer_idx, None)
        self._last_check.pop(layer_idx, None)
        self._last_rank_scores.pop(layer_idx, None)
        self._expanded_store.pop(layer_idx, None)

    # ------------------------------------------------------------ accounting
    def _ensure_work(self, device) -> torch.Tensor:
        if self._work_buf is None:
            self._work_buf = torch.zeros(2, dtype=torch.long, device=device)
            self._attn_work = self._work_buf[0]
            self._attn_work_max = self._work_buf[1]
        return self._work_buf

    def _work(self, device) -> Optional[torch.Tensor]:
        """The [attended, max] counter pair when it lives on `device`; the
        decode kernels add to it directly."""
        buf = self._ensure_work(device)
        return buf if buf.device == torch.device(device) else None

    def _record_work(self, context_lens: torch.Tensor, pages_attended: torch.Tensor):
        """backend.py:368-390: pages_attended is summed over batch x KV heads;
        the maximum is n_valid x H_kv per sequence."""
        self._ensure_work(context_lens.device)
        n_valid = ((context_lens.float() - 1) / self.block_size).long() + 1
        dense_max = n_valid.sum() * self.num_kv_heads
        self._attn_work += pages_attended.to(torch.long).to(self._attn_work.device)
        self._attn_work_max += dense_max.to(torch.long).to(self._attn_work_max.device)

    def _counters(self) -> Tuple[int, int, int, int]:
        """(accept-all checks, rejections, scoring steps, heads accepted)."""
        host = [self._h_accept_counts, self._h_reject_counts, self._h_total_scoring_steps,
                self._h_per_head_accept_sum]
        if self._dev_stats is not None:
            host = [h + d for h, d in zip(host, self._dev_stats[:4].tolist())]
        return tuple(host)

    def _ensure_dev_stats(self, device) -> Optional[torch.Tensor]:
        if self._dev_stats is None:
            self._dev_stats = torch.zeros(6, dtype=torch.long, device=device)
        return self._dev_stats if self._dev_stats.device == torch.device(device) else None

    def _decode_work(self, context_lens):
        """Counter pair for a kernel launch, or None after recording on the host."""
        return self._work(context_lens.device)

    # ------------------------------------------------------------ steps
    def _reuse_decode(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        work = self._decode_work(context_lens)
        plan = self._matching_plan(layer_idx, q, k_cache, v_cache, block_tables, context_lens)
        if plan is not None:
            return plan.run(ops._lib.STEP_REUSE, q)
        # The launch of a layer's reuse decode is validated once and replayed
        # while the caches, tables, selection and stream stay the same.
        plan = self._reuse_plans.get(layer_idx)
        if plan is None or not plan.matches(q, k_cache, v_cache, block_tables, context_lens,
                                            work):
            pi_flat, nph_flat, padded = self._reuse_state[layer_idx]
            plan = ops.prepare_sparse_decode_reuse(
                q, k_cache, v_cache, block_tables, context_lens, pi_flat, nph_flat, padded,
                self.num_kv_heads, self.num_q_per_kv, self.block_size, work)
            self._reuse_plans[layer_idx] = plan
        out = self._time_kernel("sparse_draft", plan.run, q)[3]
        if work is None:
            self._record_work(context_lens, self._cached_selection[layer_idx][1].sum())
        return out

    def _apply_random_reject(self, accept_mask):
        if self.random_reject_prob is None:
            return accept_mask
        if torch.rand(1, device=accept_mask.device).item() < self.random_reject_prob:
            return torch.zeros_like(accept_mask)
        return torch.ones_like(accept_mask)

    def _lazy_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """backend.py:392-465"""
        if layer_idx in self._cached_selection:
            plan = self._lazy_plan(layer_idx, q, k_cache, v_cache, block_tables, context_lens)
            if plan is not None:
                output = plan.run(ops._lib.STEP_LAZY_CHECK, q)
                self._last_check[layer_idx] = (plan.page_scores,
                                               plan.check_accept.view(torch.bool))
                self._total_coverage_checks += 1
                self._book_plan_gate(plan, layer_idx, context_lens)
                return output
        else:
            # The layer's first selection (a lazy scoring step without a
            # cached selection, :427-465), made in the plan's own buffers.
            plan = self._fresh_plan(layer_idx, q, k_cache, v_cache, block_tables, context_lens,
                                    own_scores_cache=True)
            if plan is not None:
                output = plan.run(ops._lib.STEP_FRESH, q)
                self._total_coverage_checks += 1
                self._adopt_plan_selection(plan, layer_idx, context_lens, plan.scores_cache)
                return output
        page_scores = self._time_kernel("scoring", self._gate_scores, q, k_cache, block_tables,
                                        context_lens)
        self._total_coverage_checks += 1
        if layer_idx in self._cached_selection:
            page_indices, n_per_head = self._cached_selection[layer_idx]
            accept_mask, coverage = self._time_kernel(
                "coverage", ops.check_coverage, page_scores, page_indices, n_per_head,
                self.tau)
            self._last_check[layer_idx] = (page_scores, accept_mask)
            if self._device_decision_ok(layer_idx, page_scores, context_lens):
                return self._lazy_device_step(q, k_cache, v_cache, block_tables,
                                              context_lens, layer_idx, page_scores,
                                              accept_mask, coverage)
            accept_mask = self._apply_random_reject(accept_mask)
            n_acc = int(accept_mask.sum().item())  # one host read decides the branch
            self._h_per_head_accept_sum += n_acc
            self._per_head_total += accept_mask.numel()
            if n_acc == accept_mask.numel():
                self._h_accept_counts += 1
                self._last_accept_mask[layer_idx] = accept_mask
                return self._reuse_decode(q, k_cache, v_cache, block_tables, context_lens,
                                          layer_idx)
        self._h_reject_counts += 1
        return self._scoring_step(q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                                  page_scores=page_scores)

    # ------------------------------------------------------------ scorers
    def _quest_page_scores(self, q, k_cache, block_tables, context_lens, check_accept=None):
        """backend.py:572-620: Quest ranking scores [B, H_kv, W] fp32, from
        page metadata of this key cache that is recomputed for the pages
        whose valid-token count changed.  With a lazy check's flags, nothing
        is computed when every head passed (the scores are then unused)."""
        return self._quest_state(k_cache).scores(q, block_tables, context_lens,
                                                 self.num_kv_heads, self.num_q_per_kv,
                                                 self.block_size, check_accept)

    def _quest_state(self, k_cache):
        """The Quest metadata of this key cache (created on first use)."""
        entry = self._quest_meta.get(id(k_cache))
        if entry is None or entry[0]() is not k_cache:
            entry = (weakref.ref(k_cache), ops.QuestPageMeta(k_cache))
            self._quest_meta[id(k_cache)] = entry
        return entry[1]

    def _plan_selector(self, k_cache):
        """The step-plan scorer code and Quest metadata of this backend."""
        if self.selector != "quest":
            return ops._lib.SELECT_EXACT, None
        code = ops._lib.SELECT_QUEST_LN if self.light_normalizer else ops._lib.SELECT_QUEST
        return code, self._quest_state(k_cache)

    def _gate_scores(self, q, k_cache, block_tables, context_lens):
        """Scores of the coverage gate (and the cache): the Quest sketch with
        light_normalizer, else the exact scan (backend.py:407-418, :697-709)."""
        if self.light_normalizer:
            return self._quest_page_scores(q, k_cache, block_tables, context_lens)
        return ops.score_pages(q, k_cache, block_tables, context_lens, self.num_kv_heads,
                               self.num_q_per_kv, self.block_size)

    def _sel_scores(self, q, k_cache, block_tables, context_lens, check_accept=None):
        """Scores the selection ranks when they differ from the gate's
        (selector="quest" without light_normalizer, backend.py:723-727), else
        None."""
        if self.selector != "quest" or self.light_normalizer:
            return None
        return self._time_kernel("scoring", self._quest_page_scores, q, k_cache, block_tables,
                                 context_lens, check_accept)

    # ------------------------------------------------------------ step plans
    def _matching_plan(self, layer_idx, q, k_cache, v_cache, block_tables, context_lens):
        """The layer's step plan if it fits this call and still holds the
        layer's selection and cached scores (the lazy check's scores cache,
        or the plan's own scores after a fixed-interval scoring step)."""
        plan = self._step_plans.get(layer_idx)
        if plan is None or self._track_timing:
            return None
        sel = self._cached_selection.get(layer_idx)
        cached = self._cached_page_scores.get(layer_idx)
        if (sel is None or sel[0] is not plan.page_indices
                or not (cached is plan.scores_cache or cached is plan.page_scores)
                or not plan.matches(q, k_cache, v_cache, block_tables, context_lens,
                                    self._work(q.device), self._dev_stats,
                                    self._plan_selector(k_cache)[1])):
            return None
        return plan

    def _new_plan(self, layer_idx, q, k_cache, v_cache, block_tables, context_lens,
                  page_indices=None, n_per_head=None, scores_cache=None,
                  own_scores_cache=False):
        """Build the layer's step plan, or None where a step needs the
        per-kernel path (timing, host-side decisions, unsupported buffers)."""
        if (self._track_timing or self.random_reject_prob is not None
                or self.top_p is not None or self.static_budget_table is not None
                or self.adaptive_selection):
            return None
        dev = q.device
        work = self._work(dev)
        stats = self._ensure_dev_stats(dev)
        if work is None or stats is None:
            return None
        W = block_tables.shape[1]
        budget = max(3, int(W * self.budget_pct))
        selector, quest = self._plan_selector(k_cache)
        try:
            plan = ops.StepPlan(q, k_cache, v_cache, block_tables, context_lens,
                                self.num_kv_heads, self.num_q_per_kv, self.block_size, budget,
                                self.tau, page_indices, n_per_head, scores_cache, stats, work,
                                own_scores_cache=own_scores_cache, selector=selector,
                                quest=quest, approx_budget=self._approx_budget(budget, W))
        except (ValueError, NotImplementedError):
            return None
        self._step_plans[layer_idx] = plan
        return plan

    def _approx_budget(self, budget: int, n_pages: int) -> int:
        """Expanded budget of approximate recovery (backend.py:782-783), 0
        under exact recovery."""
        if self.approx_recovery_pct is None:
            return 0
        return min(max(budget + 1, int(n_pages * self.approx_recovery_pct)), n_pages)

    def _plan_expanded(self, plan, accept_mask, context_lens):
        """What a plan step leaves for ``_last_expanded_selection``: the
        complement (exact recovery) or the expanded selection (approximate),
        each built on first read."""
        if plan.approx_budget > 0:
            ranked = plan.sel_scores if plan.sel_scores is not None else plan.page_scores
            return _PendingExpanded(accept_mask, ranked, plan.approx_budget, context_lens,
                                    self.block_size)
        return _PendingComplement(accept_mask, plan.page_indices, plan.n_per_head,
                                  context_lens, self.block_size)

    def _fresh_plan(self, layer_idx, q, k_cache, v_cache, block_tables, context_lens,
                    own_scores_cache=False):
        """The layer's plan for a step that makes a new selection in the
        plan's own buffers: the existing one if it owns its selection and fits
        this call, else a new one (None where the per-kernel path is needed)."""
        plan = self._step_plans.get(layer_idx)
        if (plan is not None and not self._track_timing and plan.owns_selection
                and (plan.scores_cache is not None) == own_scores_cache
                and plan.matches(q, k_cache, v_cache, block_tables, context_lens,
                                 self._work(q.device), self._dev_stats,
                                 self._plan_selector(k_cache)[1])):
            return plan
        if self._track_timing:
            return None
        return self._new_plan(layer_idx, q, k_cache, v_cache, block_tables, context_lens,
                              own_scores_cache=own_scores_cache)

    def _adopt_plan_selection(self, plan, layer_idx, context_lens, cached_scores):
        """Bookkeeping after a plan made a new selection: it becomes the
        layer's cached selection (and reuse state), with its gate outputs."""
        B = plan.page_indices.shape[0]
        accept_mask = plan.accept.view(torch.bool)
        self._last_accept_mask[layer_idx] = accept_mask
        self._expanded_store[layer_idx] = self._plan_expanded(plan, accept_mask, context_lens)
        self._cached_page_scores[layer_idx] = cached_scores
        self._reuse_state[layer_idx] = (plan.page_indices.view(B * self.num_kv_heads, -1),
                                        plan.n_per_head.view(B * self.num_kv_heads),
                                        ops.next_power_of_2(plan.budget))
        self._reuse_plans.pop(layer_idx, None)
        self._cached_selection[layer_idx] = (plan.page_indices, plan.n_per_head)
        if plan.sel_scores is not None:
            self._last_rank_scores[layer_idx] = plan.sel_scores

    def _lazy_plan(self, layer_idx, q, k_cache, v_cache, block_tables, context_lens):
        plan = self._matching_plan(layer_idx, q, k_cache, v_cache, block_tables, context_lens)
        if plan is not None:
            return plan
        page_indices, n_per_head = self._cached_selection[layer_idx]
        return self._new_plan(layer_idx, q, k_cache, v_cache, block_tables, context_lens,
                              page_indices, n_per_head,
                              self._cached_page_scores.get(layer_idx))

    def _book_plan_gate(self, plan, layer_idx, context_lens):
        """Host-side bookkeeping of a plan's check or scoring step."""
        if plan.sel_scores is not None:
            self._last_rank_scores[layer_idx] = plan.sel_scores
        accept_mask = plan.accept.view(torch.bool)
        self._per_head_total += accept_mask.numel()
        self._last_accept_mask[layer_idx] = accept_mask
        self._expanded_store[layer_idx] = self._plan_expanded(plan, accept_mask, context_lens)

    def _device_decision_ok(self, layer_idx, page_scores, context_lens) -> bool:
        """Whether the lazy accept-all decision can stay on the device: exact
        recovery, no counterfactual rejections, the cached selection and
        scores match this call's shape, counters live on this device."""
        if (self.random_reject_prob is not None or self.approx_recovery_pct is not None
                or self.top_p is not None
                or (self.adaptive_selection and self.static_budget_table is None)):
            return False
        page_indices, n_per_head = self._cached_selection[layer_idx]
        B, H_kv, W = page_scores.shape
        if self._static_only():
            budget = self._static_rows(layer_idx, B, W, page_scores.device)[1]
        else:
            budget = max(3, int(W * self.budget_pct))
        if (tuple(page_indices.shape) != (B, H_kv, budget) or not page_indices.is_contiguous()
                or tuple(n_per_head.shape) != (B, H_kv) or not n_per_head.is_contiguous()):
            return False
        cached = self._cached_page_scores.get(layer_idx)
        if cached is not None and (cached.shape != page_scores.shape
                                   or not cached.is_contiguous()):
            return False
        dev = page_scores.device
        return self._work(dev) is not None and self._ensure_dev_stats(dev) is not None

    def _lazy_device_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                          page_scores, check_accept, coverage):
        """_lazy_step with the accept-all branch (backend.py:440-465) taken on
        the device: select_or_keep keeps the cached selection when every head
        passed, or refreshes it in place (the scoring step's top-k and
        coverage gate, :737-771); verified_decode then attends the selection
        on accepted heads and every valid page on rejected heads.  The
        counters of both branches accumulate on the device."""
        page_indices, n_per_head = self._cached_selection[layer_idx]
        budget = page_indices.shape[2]
        plan = self._step_plans.get(layer_idx)
        if plan is not None and plan.page_indices is page_indices:
            plan.selection_changed()  # select_or_keep below may rewrite it in place
        self._per_head_total += check_accept.numel()
        sel_scores = self._sel_scores(q, k_cache, block_tables, context_lens, check_accept)
        if sel_scores is not None:
            self._last_rank_scores[layer_idx] = sel_scores
        rows = None
        if self._static_only():  # a new selection takes the table's budgets
            rows = self._static_rows(layer_idx, page_scores.shape[0], page_scores.shape[2],
                                     page_scores.device)[0]
        accept_mask = self._time_kernel(
            "coverage", ops.select_or_keep, page_scores, check_accept, budget, context_lens,
            self.block_size, self.tau, page_indices, n_per_head, coverage,
            self._cached_page_scores.get(layer_idx), self._dev_stats, sel_scores=sel_scores,
            row_budgets=rows)
        self._last_accept_mask[layer_idx] = accept_mask
        output = self._time_kernel(
            "sparse_draft", ops.verified_decode, q, k_cache, v_cache, block_tables,
            context_lens, page_indices, n_per_head, accept_mask, self.num_kv_heads,
            self.num_q_per_kv, self.block_size, output_dtype=q.dtype,
            work=self._work(context_lens.device))
        # Present only when a head was rejected, as after a scoring step.
        self._expanded_store[layer_idx] = _PendingComplement(
            accept_mask, page_indices, n_per_head, context_lens, self.block_size)
        return output

    def _coverage_only_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """backend.py:467-520"""
        page_scores = self._cached_page_scores[layer_idx]
        page_indices, n_per_head = self._cached_selection[layer_idx]
        accept_mask, _coverage = self._time_kernel(
            "coverage", ops.check_coverage, page_scores, page_indices, n_per_head, self.tau)
        self._last_check[layer_idx] = (page_scores, accept_mask)
        accept_mask = self._apply_random_reject(accept_mask)
        n_acc = int(accept_mask.sum().item())
        self._h_per_head_accept_sum += n_acc
        self._per_head_total += accept_mask.numel()
        self._total_coverage_checks += 1
        if n_acc == accept_mask.numel():
            self._h_accept_counts += 1
            self._last_accept_mask[layer_idx] = accept_mask
            return self._reuse_decode(q, k_cache, v_cache, block_tables, context_lens,
                                      layer_idx)
        self._h_reject_counts += 1
        return self._scoring_step(q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                                  page_scores=None)

    def _scoring_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                      page_scores=None):
        """backend.py:683-864 (uniform, top-p, static-table or adaptive budgets;
        exact or approximate recovery)."""
        B = q.shape[0]
        n_pages = block_tables.shape[1]
        budget = max(3, int(n_pages * self.budget_pct))                           # :690

        if page_scores is None and not self.lazy:
            # Fixed-interval scoring step from the layer's step plan: the
            # selection and scores live in the plan's buffers.
            plan = self._fresh_plan(layer_idx, q, k_cache, v_cache, block_tables, context_lens)
            if plan is not None:
                output = plan.run(ops._lib.STEP_SCORE, q)
                self._per_head_total += plan.accept.numel()
                self._adopt_plan_selection(plan, layer_idx, context_lens, plan.page_scores)
                return output

        if page_scores is None:
            page_scores = self._time_kernel("scoring", self._gate_scores, q, k_cache,
                                            block_tables, context_lens)
        self._cached_page_scores[layer_idx] = page_scores                         # :713
        sel_scores = self._sel_scores(q, k_cache, block_tables, context_lens)      # :723-727
        if sel_scores is not None:
            self._last_rank_scores[layer_idx] = sel_scores

        # Top-k selection fused with the coverage gate of the new selection.
        # In the fixed-interval schedule the gate's counters (:859-863) are
        # booked on the device, so the step needs no host read.
        dev = page_scores.device
        budgeted = (self.top_p is not None or self.static_budget_table is not None
                    or self.adaptive_selection)
        # A static table's budgets are known on the host, so its selection
        # needs no host read either.
        device_book = ((not budgeted or self._static_only()) and not self.lazy
                       and self.random_reject_prob is None
                       and self.approx_recovery_pct is None
                       and self._ensure_dev_stats(dev) is not None)
        if device_book:
            H = self.num_kv_heads
            rows = None
            if budgeted:
                rows, budget = self._static_rows(layer_idx, B, n_pages, dev)
            page_indices = torch.empty(B, H, budget, dtype=torch.int32, device=dev)
            n_per_head = torch.empty(B, H, dtype=torch.int32, device=dev)
            coverage = torch.empty(B, H, dtype=torch.float32, device=dev)
            accept_mask = self._time_kernel(
                "coverage", ops.select_or_keep, page_scores, None, budget, context_lens,
                self.block_size, self.tau, page_indices, n_per_head, coverage, None,
                self._dev_stats, count_gate=True, sel_scores=sel_scores, row_budgets=rows)
            self._per_head_total += B * H
        elif budgeted:
            # Per-head budgets (:727-732), gate fused; budget becomes the
            # largest one, as in the reference.
            page_indices, n_per_head, accept_mask, budget = self._time_kernel(
                "coverage", self._budgeted_select, page_scores, sel_scores, layer_idx,
                context_lens, budget)
        elif sel_scores is None:
            page_indices, n_per_head, accept_mask, _coverage = self._time_kernel(
                "coverage", ops.select_topk, page_scores, budget, context_lens,
                self.block_size, self.tau)
        else:
            # The selector proposes, the gate scores verify (:723-761).
            page_indices, n_per_head = self._time_kernel(
                "coverage", ops.select_topk, sel_scores, budget, context_lens,
                self.block_size)
            accept_mask, _coverage = self._time_kernel(
                "coverage", ops.check_coverage, page_scores, page_indices, n_per_head,
                self.tau)
        accept_mask = self._apply_random_reject(accept_mask)
        self._last_accept_mask[layer_idx] = accept_mask                           # :771

        if self.approx_recovery_pct is None:
            # Accepted heads: normalised draft (:775-779); rejected heads:
            # complement + LSE merge == every valid page (:818-844).
            work = self._decode_work(context_lens)
            output = self._time_kernel(
                "sparse_draft", ops.verified_decode, q, k_cache, v_cache, block_tables,
                context_lens, page_indices, n_per_head, accept_mask, self.num_kv_heads,
                self.num_q_per_kv, self.block_size, output_dtype=q.dtype, work=work)
            if work is None:
                n_valid = ((context_lens.float() - 1) / self.block_size).long() + 1
                pages = torch.where(accept_mask, n_per_head.long(),
                                    n_valid.unsqueeze(1).expand_as(n_per_head)).sum()
                self._record_work(context_lens, pages)
            self._expanded_store[layer_idx] = _PendingComplement(
                accept_mask, page_indices, n_per_head, context_lens, self.block_size)
            if not self.lazy and not device_book:
                n_acc = int(accept_mask.sum().item())
                if n_acc == accept_mask.numel():
                    self._h_accept_counts += 1
                else:
                    self._h_reject_counts += 1
                self._h_per_head_accept_sum += n_acc
                self._per_head_total += accept_mask.numel()
        else:
            output = self._approx_recovery(q, k_cache, v_cache, block_tables, context_lens,
                                           layer_idx,
                                           page_scores if sel_scores is None else sel_scores,
                                           page_indices, n_per_head,
                                           accept_mask, budget, n_pages)

        # Reuse state and cached selection (:852-856).  The selection is
        # used in place; the kernels need no power-of-two padding.
        self._reuse_state[layer_idx] = (page_indices.view(B * self.num_kv_heads, -1),
                                        n_per_head.view(B * self.num_kv_heads),
                                        ops.next_power_of_2(page_indices.shape[2]))
        self._reuse_plans.pop(layer_idx, None)
        self._cached_selection[layer_idx] = (page_indices, n_per_head)
        if not device_book:
            self._h_total_scoring_steps += 1                                      # :859
        return output

    def _static_only(self) -> bool:
        """Per-head budgets from the static table alone (top-p takes
        precedence over it, backend.py:727-736): budgets the host knows."""
        return self.top_p is None and self.static_budget_table is not None

    def _static_rows(self, layer_idx, B, W, device):
        """The static table's budgets of this layer, [B, H_kv] int32 on the
        device, and the largest (the selection's row width): clamp(round(
        frac * P), 3, P) (backend.py:638), made once per shape."""
        key = (layer_idx, B, W, device)
        entry = self._table_budgets.get(key)
        if entry is None:
            fracs = self.static_budget_table[layer_idx]
            per_head = torch.clamp((fracs * W).round().long(), min=3, max=W)      # :638
            rows = per_head.to(torch.int32).view(1, -1).expand(B, -1).contiguous()
            entry = (rows.to(device), int(per_head.max()))
            self._table_budgets[key] = entry
        return entry

    def _budgeted_select(self, page_scores, sel_scores, layer_idx, context_lens, base_budget):
        """_topp_select / _static_select / _adaptive_select (backend.py:
        522-681, in the reference's order of precedence, :727-736) with the
        coverage gate of the new selection: (page_indices [B, H_kv,
        max_budget], n_per_head, accept_mask, max_budget)."""
        W = page_scores.shape[2]
        if self.top_p is None and self.static_budget_table is None:
            ranked = page_scores if sel_scores is None else sel_scores
            budgets = ops.adaptive_budgets(ranked, base_budget, context_lens, self.block_size,
                                           self.adaptive_floor_ratio)
            max_budget = int(budgets.max().item())   # :559, a host read as in the reference
            idx, nph, acc, _cov = ops.select_budgeted(
                page_scores, context_lens, self.block_size, row_budgets=budgets,
                width=max_budget, tau=self.tau, sel_scores=sel_scores)
            return idx, nph, acc, max_budget
        if self.top_p is not None:
            idx, nph, acc, _cov = ops.select_budgeted(
                page_scores, context_lens, self.block_size, top_p=self.top_p, tau=self.tau,
                sel_scores=sel_scores)
            max_budget = int(nph.max().item())   # :679, a host read as in the reference
            return idx[:, :, :max_budget].contiguous(), nph, acc, max_budget
        budgets, max_budget = self._static_rows(layer_idx, page_scores.shape[0], W,
                                                page_scores.device)
        idx, nph, acc, _cov = ops.select_budgeted(
            page_scores, context_lens, self.block_size, row_budgets=budgets, width=max_budget,
            tau=self.tau, sel_scores=sel_scores)
        return idx, nph, acc, max_budget

    def _approx_recovery(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                         page_scores, page_indices, n_per_head, accept_mask, budget, n_pages):
        """Approximate recovery branch (backend.py:775-817): rejected heads use
        an expanded top-k at approx_recovery_pct of the pages, ranked by the
        selection scores (``page_scores`` here)."""
        B = q.shape[0]
        n_acc = int(accept_mask.sum().item())
        all_acc = n_acc == accept_mask.numel()
        draft = self._time_kernel(
            "sparse_draft", ops.sparse_decode, q, k_cache, v_cache, block_tables, page_indices,
            n_per_head, context_lens, self.num_kv_heads, self.num_q_per_kv, self.block_size)
        pages = n_per_head.sum()
        if all_acc:
            output = draft
            if not self.lazy:
                self._h_accept_counts += 1
        else:
            exp_budget = self._approx_budget(budget, n_pages)
            exp_indices, exp_nph = ops.select_topk(page_scores, exp_budget, context_lens,
                                                   self.block_size)
            expanded = self._time_kernel(
                "ar_recovery", ops.sparse_decode, q, k_cache, v_cache, block_tables,
                exp_indices, exp_nph, context_lens, self.num_kv_heads, self.num_q_per_kv,
                self.block_size)
            pages = pages + exp_nph.sum()
            accept_q = accept_mask.repeat_interleave(self.num_q_per_kv, dim=1)
            output = torch.where(accept_q.unsqueeze(-1), draft, expanded)
            self._expanded_store[layer_idx] = (exp_indices, exp_nph)
            if not self.lazy:
                self._h_reject_counts += 1
        self._record_work(context_lens, pages)
        if not self.lazy:
            self._h_per_head_accept_sum += n_acc
            self._per_head_total += accept_mask.numel()
        return output

    def _reuse_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """backend.py:866-881, including the step-decrement fallback (:868-872)."""
        if layer_idx not in self._reuse_state:
            self._step -= 1
            return self(q, k_cache, v_cache, block_tables, context_lens, layer_idx)
        return self._reuse_decode(q, k_cache, v_cache, block_tables, context_lens, layer_idx)
