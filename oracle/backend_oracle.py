"""CPU restatement of CVSABackend's scheduling -- TEST INFRASTRUCTURE ONLY.

Follows cvsa/backend.py of DJ-Melvin/coverage-verified-sparse-attention
(line numbers below) for the configurations this build covers: the exact
page scorer or the Quest min/max scorer (selector="quest", for selection
only or, with light_normalizer, for the coverage gate too) with a uniform
budget, top-p budgets (``top_p``), a static per-head budget table
(``static_budget_table``) or adaptive budgets (``adaptive_selection``),
exact recovery (complement + LSE merge)
or approximate recovery (``approx_recovery_pct``), dense layers, the fixed
interval (``reuse_interval``) and lazy (``check_interval`` /
``coverage_interval``) schedules, and the statistics of get_stats().
All kernels are the oracle ops of :mod:`oracle.cvsa_oracle`.
"""
from __future__ import annotations

from typing import Dict, List, Optional

import torch

from . import cvsa_oracle as ref


class OracleCVSABackend:
    """cvsa/backend.py:45-881 restated on CPU tensors."""

    def __init__(self, num_kv_heads, num_q_heads, head_dim, block_size, num_layers=32,
                 budget_pct=0.10, reuse_interval=16, coverage_threshold=0.90,
                 dense_layers: Optional[List[int]] = None, lazy=False,
                 check_interval=None, coverage_interval=None, approx_recovery_pct=None,
                 selector="exact", light_normalizer=False, top_p=None,
                 static_budget_table=None, adaptive_selection=False, adaptive_floor_ratio=0.5,
                 random_reject_prob=None, acc_dtype=torch.float64):
        # :80-115
        self.num_kv_heads = num_kv_heads
        self.num_q_heads = num_q_heads
        self.head_dim = head_dim
        self.block_size = block_size
        self.num_layers = num_layers
        self.num_q_per_kv = num_q_heads // num_kv_heads
        self.budget_pct = budget_pct
        self.reuse_interval = reuse_interval
        self.tau = coverage_threshold
        self._dense_layers = set(dense_layers or [])
        self.approx_recovery_pct = approx_recovery_pct
        self.lazy = lazy
        self.check_interval = check_interval or 1
        self.coverage_interval = coverage_interval or self.check_interval
        self.selector = selector
        self.light_normalizer = light_normalizer
        self.top_p = top_p
        self.static_budget_table = None if static_budget_table is None else {
            int(layer): torch.as_tensor(f, dtype=torch.float32)
            for layer, f in static_budget_table.items()}
        self.adaptive_selection = adaptive_selection
        self.adaptive_floor_ratio = adaptive_floor_ratio
        self.random_reject_prob = random_reject_prob
        self.acc_dtype = acc_dtype
        # Optional test hooks (None: the reference behaviour).  A parity test
        # that runs this oracle beside another implementation uses them to
        # compare every selection and gate where it is made, and to adopt the
        # other side's answer on heads whose fp64 and fp32 answers may
        # legitimately differ (near ties), so both sides keep one state.
        #   on_select(layer, ranked, idx, nph) -> (idx, nph)
        #   on_gate(layer, where, gate_scores, idx, nph, accept, cov) -> accept
        #     where: "check" (lazy check of the cached selection),
        #     "coverage_only", or "new" (gate of a new selection).
        #   on_expand(layer, ranked, exp_idx, exp_budget) -> exp_idx
        #     (the expanded selection of approximate recovery)
        self.on_select = None
        self.on_gate = None
        self.on_expand = None
        self.reset()

    def reset(self):
        """:252-272"""
        self._step = 0
        self._reuse_state: Dict[int, tuple] = {}
        self._cached_selection: Dict[int, tuple] = {}
        self._cached_page_scores: Dict[int, torch.Tensor] = {}
        self._last_accept_mask: Dict[int, torch.Tensor] = {}
        self._last_expanded_selection: Dict[int, tuple] = {}
        self._attn_work = None
        self._attn_work_max = None
        self._accept_counts = 0
        self._reject_counts = 0
        self._total_scoring_steps = 0
        self._total_coverage_checks = 0
        self._per_head_accept_sum = 0
        self._per_head_total = 0
        self._dense_layer_steps = 0
        self.trace: List[dict] = []   # one record per call, for parity tests

    def step_done(self, layer_idx, num_layers):
        """:278-280"""
        if layer_idx == num_layers - 1:
            self._step += 1

    def get_stats(self) -> dict:
        """:282-311 (without the optional timing block)."""
        total_checks = max(self._total_coverage_checks, self._total_scoring_steps, 1)
        stats = {
            "total_scoring_steps": self._total_scoring_steps,
            "total_coverage_checks": self._total_coverage_checks,
            "all_accepted_pct": self._accept_counts / max(total_checks, 1) * 100,
            "some_rejected_pct": self._reject_counts / max(total_checks, 1) * 100,
            "per_head_accept_rate": self._per_head_accept_sum / max(self._per_head_total, 1) * 100,
            "total_decode_steps": self._step,
            "lazy": self.lazy,
            "check_interval": self.check_interval if self.lazy else None,
            "rescore_rate": (self._total_scoring_steps / max(self._total_coverage_checks, 1) * 100
                             if self.lazy else 100.0),
        }
        if self._attn_work is not None:
            pages_attended = int(self._attn_work)
            pages_max = int(self._attn_work_max)
            if pages_max > 0:
                stats["effective_budget_pct"] = pages_attended / pages_max * 100
                stats["total_pages_attended"] = pages_attended
                stats["total_pages_max"] = pages_max
        return stats

    # ---------------------------------------------------------------- calls
    def __call__(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """:313-366"""
        self._last_accept_mask.pop(layer_idx, None)
        self._last_expanded_selection.pop(layer_idx, None)
        if layer_idx in self._dense_layers:
            self._dense_layer_steps += 1
            nv = ref.n_valid_pages(context_lens, self.block_size)
            self._record_work(context_lens, nv.sum() * self.num_kv_heads)
            self.trace.append({"layer": layer_idx, "kind": "dense"})
            return ref.dense_decode(q, k_cache, v_cache, block_tables, context_lens,
                                    self.num_kv_heads, self.num_q_per_kv, self.block_size,
                                    self.acc_dtype)
        if self.lazy:
            is_scoring = self._step % self.check_interval == 0
            is_cov = self._step % self.coverage_interval == 0
            has_cache = layer_idx in self._reuse_state
            has_scores = layer_idx in self._cached_page_scores
            if is_scoring:
                return self._lazy_step(q, k_cache, v_cache, block_tables, context_lens, layer_idx)
            if is_cov and has_cache and has_scores:
                return self._coverage_only_step(q, k_cache, v_cache, block_tables,
                                                context_lens, layer_idx)
            if has_cache:
                return self._reuse_step(q, k_cache, v_cache, block_tables, context_lens,
                                        layer_idx)
            return self._lazy_step(q, k_cache, v_cache, block_tables, context_lens, layer_idx)
        if self._step % self.reuse_interval == 0:
            return self._scoring_step(q, k_cache, v_cache, block_tables, context_lens,
                                      layer_idx)
        return self._reuse_step(q, k_cache, v_cache, block_tables, context_lens, layer_idx)

    def _record_work(self, context_lens, pages_attended):
        """:368-390"""
        if self._attn_work is None:
            self._attn_work = torch.zeros((), dtype=torch.long)
            self._attn_work_max = torch.zeros((), dtype=torch.long)
        nv = ref.n_valid_pages(context_lens, self.block_size)
        self._attn_work += torch.as_tensor(pages_attended).to(torch.long)
        self._attn_work_max += (nv.sum() * self.num_kv_heads).to(torch.long)

    def _random_reject(self, accept):
        """The counterfactual override of :433-441 / :762-767: one Bernoulli
        draw per gate; every head of the layer is rejected or accepted."""
        if self.random_reject_prob is None:
            return accept
        if torch.rand(1).item() < self.random_reject_prob:
            return torch.zeros_like(accept)
        return torch.ones_like(accept)

    def _reuse_decode(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        idx, nph = self._cached_selection[layer_idx]
        self._record_work(context_lens, nph.sum())
        return ref.sparse_decode(q, k_cache, v_cache, block_tables, idx, nph, context_lens,
                                 self.num_kv_heads, self.num_q_per_kv, self.block_size,
                                 self.acc_dtype)

    def _gate_scores(self, q, k_cache, block_tables, context_lens):
        """Scores of the coverage gate: the Quest sketch with
        light_normalizer, else the exact scan (:407-418, :697-709)."""
        fn = ref.quest_page_scores if self.light_normalizer else ref.score_pages
        return fn(q, k_cache, block_tables, context_lens, self.num_kv_heads, self.num_q_per_kv,
                  self.block_size, self.acc_dtype)

    def _lazy_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """:392-465"""
        page_scores = self._gate_scores(q, k_cache, block_tables, context_lens)
        self._total_coverage_checks += 1
        if layer_idx in self._cached_selection:
            idx, nph = self._cached_selection[layer_idx]
            accept, cov = ref.check_coverage(page_scores, idx, nph, self.tau, self.acc_dtype)
            if self.on_gate is not None:
                accept = self.on_gate(layer_idx, "check", page_scores, idx, nph, accept, cov)
            accept = self._random_reject(accept)
            self._per_head_accept_sum += int(accept.sum())
            self._per_head_total += accept.numel()
            if bool(accept.all()):
                self._accept_counts += 1
                self._last_accept_mask[layer_idx] = accept
                self.trace.append({"layer": layer_idx, "kind": "lazy_accept",
                                   "accept": accept.clone(), "coverage": cov.clone()})
                return self._reuse_decode(q, k_cache, v_cache, block_tables, context_lens,
                                          layer_idx)
        self._reject_counts += 1
        return self._scoring_step(q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                                  page_scores=page_scores)

    def _coverage_only_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """:467-520"""
        page_scores = self._cached_page_scores[layer_idx]
        idx, nph = self._cached_selection[layer_idx]
        accept, cov = ref.check_coverage(page_scores, idx, nph, self.tau, self.acc_dtype)
        if self.on_gate is not None:
            accept = self.on_gate(layer_idx, "coverage_only", page_scores, idx, nph, accept, cov)
        accept = self._random_reject(accept)
        self._per_head_accept_sum += int(accept.sum())
        self._per_head_total += accept.numel()
        self._total_coverage_checks += 1
        if bool(accept.all()):
            self._accept_counts += 1
            self._last_accept_mask[layer_idx] = accept
            self.trace.append({"layer": layer_idx, "kind": "coverage_only_accept",
                               "accept": accept.clone(), "coverage": cov.clone()})
            return self._reuse_decode(q, k_cache, v_cache, block_tables, context_lens,
                                      layer_idx)
        self._reject_counts += 1
        return self._scoring_step(q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                                  page_scores=None)

    def _scoring_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx,
                      page_scores=None):
        """:683-864 (uniform budget, exact or approximate recovery)."""
        B = q.shape[0]
        n_pages = block_tables.shape[1]
        nv = ref.n_valid_pages(context_lens, self.block_size)
        budget = max(3, int(n_pages * self.budget_pct))                          # :690
        if page_scores is None:
            page_scores = self._gate_scores(q, k_cache, block_tables, context_lens)
        self._cached_page_scores[layer_idx] = page_scores                        # :713
        sel_scores = page_scores                                                 # :723-727
        if self.selector == "quest" and not self.light_normalizer:
            sel_scores = ref.quest_page_scores(q, k_cache, block_tables, context_lens,
                                               self.num_kv_heads, self.num_q_per_kv,
                                               self.block_size, self.acc_dtype)
        if self.top_p is not None:                                               # :727-729
            idx, nph = ref.topp_select(sel_scores, self.top_p, context_lens, self.block_size)
            budget = idx.shape[-1]
        elif self.static_budget_table is not None:                               # :730-732
            idx, nph = ref.static_select(sel_scores, self.static_budget_table[layer_idx],
                                         context_lens, self.block_size)
            budget = idx.shape[-1]
        elif self.adaptive_selection:                                            # :733-735
            idx, nph = ref.adaptive_select(sel_scores, budget, context_lens, self.block_size,
                                           self.adaptive_floor_ratio)
            budget = idx.shape[-1]
        else:
            idx, nph = ref.select_topk(sel_scores, budget, context_lens, self.block_size)
        if self.on_select is not None:
            idx, nph = self.on_select(layer_idx, sel_scores, idx, nph)
        o_d, m_d, l_d = ref.sparse_decode_unnorm(q, k_cache, v_cache, block_tables, idx, nph,
                                                 context_lens, self.num_kv_heads,
                                                 self.num_q_per_kv, self.block_size,
                                                 self.acc_dtype)
        accept, cov = ref.check_coverage(page_scores, idx, nph, self.tau, self.acc_dtype)
        if self.on_gate is not None:
            accept = self.on_gate(layer_idx, "new", page_scores, idx, nph, accept, cov)
        accept = self._random_reject(accept)                                     # :762-767
        self._last_accept_mask[layer_idx] = accept
        recovery_pages = None
        if bool(accept.all()):                                                   # :775-779
            out = ref.normalise(o_d, l_d, q.dtype)
            if not self.lazy:
                self._accept_counts += 1
            kind = "score_accept"
        elif self.approx_recovery_pct is not None:                               # :780-817
            exp_budget = max(budget + 1, int(n_pages * self.approx_recovery_pct))
            exp_budget = min(exp_budget, n_pages)
            exp_idx, _ = ref.select_topk(sel_scores, exp_budget, context_lens, self.block_size)
            if self.on_expand is not None:
                exp_idx = self.on_expand(layer_idx, sel_scores, exp_idx, exp_budget)
            exp_nph = torch.clamp(nv, max=exp_budget).to(torch.int32).unsqueeze(1).expand(
                B, self.num_kv_heads).contiguous()
            o_e, m_e, l_e = ref.sparse_decode_unnorm(q, k_cache, v_cache, block_tables, exp_idx,
                                                     exp_nph, context_lens, self.num_kv_heads,
                                                     self.num_q_per_kv, self.block_size,
                                                     self.acc_dtype)
            recovery_pages = exp_nph.sum()
            acc_q = accept.repeat_interleave(self.num_q_per_kv, dim=1)
            out = torch.where(acc_q.unsqueeze(-1), ref.normalise(o_d, l_d, torch.float64),
                              ref.normalise(o_e, l_e, torch.float64)).to(q.dtype)
            self._last_expanded_selection[layer_idx] = (exp_idx, exp_nph)
            if not self.lazy:
                self._reject_counts += 1
            kind = "score_approx"
        else:                                                                    # :818-844
            comp, ncomp = ref.compute_complement(idx, nph, context_lens, self.block_size, accept)
            o_c, m_c, l_c = ref.sparse_decode_unnorm(q, k_cache, v_cache, block_tables, comp,
                                                     ncomp, context_lens, self.num_kv_heads,
                                                     self.num_q_per_kv, self.block_size,
                                                     self.acc_dtype)
            recovery_pages = ncomp.sum()
            out = ref.lse_merge(o_d, m_d, l_d, o_c, m_c, l_c, accept, self.num_q_per_kv,
                                q.dtype, self.acc_dtype)
            self._last_expanded_selection[layer_idx] = (comp, ncomp)
            if not self.lazy:
                self._reject_counts += 1
            kind = "score_exact"
        pages = nph.sum()
        if recovery_pages is not None:
            pages = pages + recovery_pages
        self._record_work(context_lens, pages)                                   # :846-850
        self._reuse_state[layer_idx] = True                                      # :852-855
        self._cached_selection[layer_idx] = (idx, nph)                           # :856
        self._total_scoring_steps += 1                                           # :859
        if not self.lazy:
            self._per_head_accept_sum += int(accept.sum())
            self._per_head_total += accept.numel()
        self.trace.append({"layer": layer_idx, "kind": kind, "accept": accept.clone(),
                           "coverage": cov.clone(), "page_indices": idx.clone(),
                           "n_per_head": nph.clone(), "page_scores": page_scores,
                           "sel_scores": sel_scores})
        return out

    def _reuse_step(self, q, k_cache, v_cache, block_tables, context_lens, layer_idx):
        """:866-881, including the step-decrement fallback (:868-872)."""
        if layer_idx not in self._reuse_state:
            self._step -= 1
            return self(q, k_cache, v_cache, block_tables, context_lens, layer_idx)
        self.trace.append({"layer": layer_idx, "kind": "reuse"})
        return self._reuse_decode(q, k_cache, v_cache, block_tables, context_lens, layer_idx)
