"""HIP operators of the CVSA decode path, with the reference's argument lists.

Each function mirrors one entry of the reference's kernel API (the
``triton_*`` functions of ``cvsa/kernels``) with the same arguments and
return tuple, allocates its outputs with the torch caching allocator and
launches the gfx950 kernels of ``libcvsa_hip.so`` on the current stream.
All tensors must live on one ROCm GPU; there is no CPU path.

Workspaces of the paged decode kernels (split-K partial states) are cached
per (device, stream) and grown on demand; they need no initialisation.
"""
from __future__ import annotations

import ctypes
import weakref
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import CVSAError, check

__all__ = [
    "CVSAError",
    "score_pages",
    "select_topk",
    "select_budgeted",
    "adaptive_budgets",
    "check_coverage",
    "sparse_decode_unnorm",
    "sparse_decode",
    "prepare_reuse_state",
    "sparse_decode_reuse",
    "dense_decode",
    "verified_decode",
    "verified_decode_approx",
    "compute_complement",
    "lse_merge",
    "append_kv",
    "AppendCall",
    "next_power_of_2",
    "StepPlan",
    "quest_meta_update",
    "quest_scores",
    "quest_refresh_scores",
    "QuestPageMeta",
]

_DTYPE_CODE = {
    torch.bfloat16: _lib.DTYPE_BF16,
    torch.float16: _lib.DTYPE_FP16,
    torch.float32: _lib.DTYPE_FP32,
}


def next_power_of_2(n: int) -> int:
    """Round up to a power of two, minimum 1 (sparse_decode.py:279-283)."""
    if n <= 1:
        return 1
    return 1 << (n - 1).bit_length()


# ---------------------------------------------------------------- helpers

def _device_of(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(
                f"CVSA ops run on the GPU only; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor argument")
    return dev


def _stream(dev: torch.device) -> int:
    return torch._C._cuda_getCurrentRawStream(dev.index)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _i32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def _check_cache(k_cache: torch.Tensor, name: str = "k_cache") -> None:
    if k_cache.dim() != 4:
        raise ValueError(f"{name} must be [num_blocks, block_size, H_kv, D], got {tuple(k_cache.shape)}")
    if k_cache.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {k_cache.dtype}")
    if not k_cache.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_q(q: torch.Tensor) -> torch.Tensor:
    if q.dim() != 3:
        raise ValueError(f"q must be [B, H_q, D], got {tuple(q.shape)}")
    if q.dtype != torch.bfloat16:
        raise ValueError(f"q must be bfloat16, got {q.dtype}")
    if q.stride(2) != 1 or q.stride(0) % 8 or q.stride(1) % 8 or q.data_ptr() % 16:
        q = q.contiguous()
    return q


def _block_tables(bt: torch.Tensor) -> torch.Tensor:
    bt = bt if bt.dtype == torch.int32 else bt.to(torch.int32)
    if bt.dim() != 2 or bt.stride(1) != 1:
        bt = bt.contiguous()
    return bt


def _check_seqs(who: str, B: int, block_tables=None, context_lens=None) -> None:
    """The per-sequence inputs of a call over B sequences: block_tables
    [B, W] and context_lens [B].  The kernels index them by sequence, so a
    shorter tensor would be read past its end on the device."""
    if block_tables is not None and (block_tables.dim() != 2 or block_tables.shape[0] != B):
        raise ValueError(f"{who}: block_tables must be [{B}, W], got "
                         f"{tuple(block_tables.shape)}")
    if context_lens is not None and (context_lens.dim() != 1 or context_lens.shape[0] != B):
        raise ValueError(f"{who}: context_lens must be [{B}], got {tuple(context_lens.shape)}")


def _check_count(who: str, name: str, t, n: int) -> None:
    """t (if given) holds exactly n entries: one per row the kernel reads."""
    if t is not None and t.numel() != n:
        raise ValueError(f"{who}: {name} must hold {n} entries, got {t.numel()}")


def _check_rows(who: str, name: str, t, rows: int, min_cols: int) -> None:
    """t (if given) is [rows, >= min_cols]: one row per (sequence, KV head)."""
    if t is not None and (t.dim() != 2 or t.shape[0] != rows or t.shape[1] < min_cols):
        raise ValueError(f"{who}: {name} must be [{rows}, >= {min_cols}], got "
                         f"{tuple(t.shape)}")


_WORKSPACES: dict = {}


def _workspace(dev: torch.device, nbytes: int) -> Optional[torch.Tensor]:
    """Per-(device, stream) decode workspace of at least nbytes (None for 0)."""
    if nbytes == 0:
        return None
    stream = _stream(dev)
    key = (dev.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        # Zeroed once: the decode kernels keep their completion counters at
        # zero between calls.
        size = (nbytes + (1 << 20) - 1) // (1 << 20) * (1 << 20)
        ws = torch.empty(size, dtype=torch.uint8, device=dev)
        check(_lib.load().cvsa_workspace_init(ws.data_ptr(), size, stream), "workspace_init")
        _WORKSPACES[key] = ws
    return ws


# ---------------------------------------------------------------- scoring

def score_pages(q: torch.Tensor, k_cache: torch.Tensor, block_tables: torch.Tensor,
                context_lens: torch.Tensor, num_kv_heads: int, num_q_per_kv: int,
                block_size: int) -> torch.Tensor:
    """max(q_rep . K) * D^-0.5 per page and KV head -> [B, H_kv, W] fp32.

    Mirrors triton_score_pages (cvsa/kernels/page_scores.py:77-119).
    """
    dev = _device_of(q, k_cache, block_tables, context_lens)
    q = _check_q(q)
    _check_cache(k_cache)
    bt = _block_tables(block_tables)
    ctx = _i32(context_lens)
    B, H_q, D = q.shape
    _check_seqs("score_pages", B, bt, ctx)
    if num_kv_heads * num_q_per_kv != H_q or k_cache.shape[2] != num_kv_heads:
        raise ValueError("score_pages: head counts do not match q / k_cache")
    if k_cache.shape[1] != block_size or k_cache.shape[3] != D:
        raise ValueError("score_pages: k_cache block_size / head_dim mismatch")
    W = bt.shape[1]
    out = torch.empty(B, num_kv_heads, W, device=dev, dtype=torch.float32)
    check(_lib.load().cvsa_score_pages(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), k_cache.shape[0],
        bt.data_ptr(), bt.stride(0), ctx.data_ptr(), B, H_q, num_kv_heads, D,
        block_size, W, out.data_ptr(), _stream(dev)), "score_pages")
    return out


def select_topk(page_scores: torch.Tensor, budget: int, context_lens: torch.Tensor,
                block_size: int, tau: Optional[float] = None):
    """Top-`budget` pages per (b, kv-head) and n_per_head = min(budget, n_valid).

    Replaces ``torch.topk(page_scores, budget, sorted=False)`` plus the
    n_per_head computation of CVSABackend._scoring_step
    (cvsa/backend.py:737-747).  The set is the `budget` largest scores with
    ties to the lower page index, returned in ascending page order.
    With ``tau`` the coverage gate of the new selection is fused in and
    (page_indices, n_per_head, accept_mask, coverage) is returned.
    """
    dev = _device_of(page_scores, context_lens)
    if page_scores.dtype != torch.float32 or page_scores.dim() != 3:
        raise ValueError("page_scores must be [B, H_kv, W] float32")
    ps = page_scores.contiguous()
    ctx = _i32(context_lens)
    B, H_kv, W = ps.shape
    _check_seqs("select_topk", B, None, ctx)
    if not 1 <= budget <= W:
        raise ValueError(f"select_topk: budget {budget} must be in [1, {W}]")
    idx = torch.empty(B, H_kv, budget, device=dev, dtype=torch.int32)
    nph = torch.empty(B, H_kv, device=dev, dtype=torch.int32)
    acc = cov = None
    if tau is not None:
        acc = torch.empty(B, H_kv, device=dev, dtype=torch.uint8)
        cov = torch.empty(B, H_kv, device=dev, dtype=torch.float32)
    check(_lib.load().cvsa_select_topk(
        ps.data_ptr(), B, H_kv, W, ctx.data_ptr(), block_size, budget, idx.data_ptr(),
        nph.data_ptr(), float(tau) if tau is not None else 0.0, _ptr(acc), _ptr(cov),
        _stream(dev)), "select_topk")
    if tau is None:
        return idx, nph
    return idx, nph, acc.view(torch.bool), cov


def select_budgeted(page_scores: torch.Tensor, context_lens: torch.Tensor, block_size: int, *,
                    top_p: Optional[float] = None, row_budgets: Optional[torch.Tensor] = None,
                    width: Optional[int] = None, tau: Optional[float] = None,
                    sel_scores: Optional[torch.Tensor] = None):
    """Selection with a budget per (b, kv-head) row (cvsa_select_budgeted).

    ``top_p``: each row takes the smallest prefix of its pages by score whose
    softmax mass reaches top_p, at least 3 (CVSABackend._topp_select,
    cvsa/backend.py:652-681).  ``row_budgets`` ([B, H_kv] int32 on the
    device): row (b, h) takes row_budgets[b, h] pages (_static_select,
    :622-650, or the budgets of adaptive_budgets).  The
    pages are ranked by ``sel_scores`` when given, else by ``page_scores``.
    Returns ``page_indices`` [B, H_kv, width] (default width W; each row's
    first n_per_head entries are its selected valid pages, in ascending page
    order; entries past the row's budget are unspecified) and
    ``n_per_head``; with ``tau`` also the accept mask and coverage of the
    selection's gate on ``page_scores``.
    """
    dev = _device_of(page_scores, context_lens, row_budgets, sel_scores)
    if page_scores.dtype != torch.float32 or page_scores.dim() != 3:
        raise ValueError("page_scores must be [B, H_kv, W] float32")
    ps = page_scores.contiguous()
    B, H_kv, W = ps.shape
    if (top_p is None) == (row_budgets is None):
        raise ValueError("select_budgeted: give exactly one of top_p and row_budgets")
    if top_p is not None and not 0.0 < top_p < 1.0:
        raise ValueError(f"select_budgeted: top_p must be in (0, 1), got {top_p}")
    if row_budgets is not None and (row_budgets.dtype != torch.int32
                                    or row_budgets.shape != (B, H_kv)
                                    or not row_budgets.is_contiguous()):
        raise ValueError(f"select_budgeted: row_budgets must be a contiguous int32 [{B}, {H_kv}]")
    if sel_scores is not None:
        if sel_scores.shape != ps.shape or sel_scores.dtype != torch.float32:
            raise ValueError("select_budgeted: sel_scores must match page_scores")
        sel_scores = sel_scores.contiguous()
    width = W if width is None else int(width)
    if not 1 <= width <= W:
        raise ValueError(f"select_budgeted: width {width} must be in [1, {W}]")
    ctx = _i32(context_lens)
    _check_seqs("select_budgeted", B, None, ctx)
    idx = torch.empty(B, H_kv, width, device=dev, dtype=torch.int32)
    nph = torch.empty(B, H_kv, device=dev, dtype=torch.int32)
    acc = cov = None
    if tau is not None:
        acc = torch.empty(B, H_kv, device=dev, dtype=torch.uint8)
        cov = torch.empty(B, H_kv, device=dev, dtype=torch.float32)
    check(_lib.load().cvsa_select_budgeted(
        ps.data_ptr(), _ptr(sel_scores), B, H_kv, W, ctx.data_ptr(), block_size,
        float(top_p) if top_p is not None else 0.0, _ptr(row_budgets), width, idx.data_ptr(),
        nph.data_ptr(), float(tau) if tau is not None else 0.0, _ptr(acc), _ptr(cov),
        _stream(dev)), "select_budgeted")
    if tau is None:
        return idx, nph
    return idx, nph, acc.view(torch.bool), cov


def adaptive_budgets(sel_scores: torch.Tensor, base_budget: int, context_lens: torch.Tensor,
                     block_size: int, floor_ratio: float) -> torch.Tensor:
    """Per-head budgets [B, H_kv] int32 of CVSABackend._adaptive_select
    (cvsa/backend.py:522-570), computed on the device
    (cvsa_adaptive_budgets): the heads of a sequence compete for
    H_kv * base_budget of their largest scores, blended toward base_budget by
    floor_ratio and clamped to [1, n_valid]."""
    dev = _device_of(sel_scores, context_lens)
    if sel_scores.dtype != torch.float32 or sel_scores.dim() != 3:
        raise ValueError("sel_scores must be [B, H_kv, W] float32")
    ss = sel_scores.contiguous()
    B, H_kv, W = ss.shape
    if base_budget < 1:
        raise ValueError("adaptive_budgets: base_budget must be >= 1")
    ctx = _i32(context_lens)
    _check_seqs("adaptive_budgets", B, None, ctx)
    out = torch.empty(B, H_kv, device=dev, dtype=torch.int32)
    check(_lib.load().cvsa_adaptive_budgets(
        ss.data_ptr(), B, H_kv, W, ctx.data_ptr(), block_size, int(base_budget),
        float(floor_ratio), out.data_ptr(), _stream(dev)), "adaptive_budgets")
    return out


def select_or_keep(page_scores: torch.Tensor, check_accept: Optional[torch.Tensor],
                   budget: int, context_lens: torch.Tensor, block_size: int, tau: float,
                   page_indices: torch.Tensor, n_per_head: torch.Tensor,
                   coverage: torch.Tensor, scores_cache: Optional[torch.Tensor] = None,
                   stats: Optional[torch.Tensor] = None,
                   count_gate: bool = False, *,
                   sel_scores: Optional[torch.Tensor] = None,
                   row_budgets: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The selection decisions of CVSABackend taken on the device.

    With ``check_accept`` (the coverage gate of the cached selection) this is
    the lazy check of _lazy_step (cvsa/backend.py:420-465): when every head
    passed, the cached selection in ``page_indices`` / ``n_per_head`` stays
    and every head is accepted; otherwise the top-``budget`` selection of
    ``page_scores`` replaces it in place, ``coverage`` receives its coverage
    and ``scores_cache`` a copy of ``page_scores``.  Without it, a fresh
    selection is written.  ``stats`` (int64[6], slots 4-5 scratch)
    accumulates accept-all checks, rejections, scoring steps and heads that
    passed; with ``count_gate`` a fresh selection is booked as a
    fixed-interval scoring step by its own gate (backend.py:859-863).
    With ``sel_scores`` a new selection ranks those scores while
    ``page_scores`` drive its gate and the cache (the Quest selector with the
    exact gate, backend.py:723-727).
    With ``row_budgets`` ([B, H_kv] int32, e.g. a static table's,
    backend.py:622-650) a new selection takes row (b, h)'s own budget, at
    most ``budget``, the row width of ``page_indices``
    (cvsa_select_or_keep_budgeted).
    Returns the accept mask [B, H_kv] bool of the heads for this step.
    """
    dev = _device_of(page_scores, check_accept, page_indices, n_per_head, coverage)
    if page_scores.dtype != torch.float32 or page_scores.dim() != 3:
        raise ValueError("page_scores must be [B, H_kv, W] float32")
    ps = page_scores.contiguous()
    B, H_kv, W = ps.shape
    if not 1 <= budget <= W:
        raise ValueError(f"select_or_keep: budget {budget} must be in [1, {W}]")
    checks = [("page_indices", page_indices, (B, H_kv, budget), torch.int32),
              ("n_per_head", n_per_head, (B, H_kv), torch.int32),
              ("coverage", coverage, (B, H_kv), torch.float32)]
    if check_accept is not None:
        checks.append(("check_accept", check_accept, (B, H_kv), torch.bool))
    for name, t, shape, dt in checks:
        if tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"select_or_keep: {name} must be a contiguous {dt} {shape}")
    if scores_cache is not None and (scores_cache.shape != ps.shape or not
                                     scores_cache.is_contiguous() or
                                     scores_cache.dtype != torch.float32):
        raise ValueError("select_or_keep: scores_cache must be a contiguous float32 [B, H_kv, W]")
    if stats is not None and (stats.dtype != torch.int64 or stats.numel() < 6 or
                              not stats.is_contiguous()):
        raise ValueError("select_or_keep: stats must be a contiguous int64 tensor of >= 6")
    if count_gate and (check_accept is not None or stats is None):
        raise ValueError("select_or_keep: count_gate books a fresh selection into stats")
    if sel_scores is not None:
        if (sel_scores.shape != ps.shape or sel_scores.dtype != torch.float32
                or sel_scores.device != dev):
            raise ValueError("select_or_keep: sel_scores must be float32 like page_scores")
        sel_scores = sel_scores.contiguous()
    ctx = _i32(context_lens)
    _check_seqs("select_or_keep", B, None, ctx)
    acc = torch.empty(B, H_kv, device=dev, dtype=torch.uint8)
    if row_budgets is not None:
        if (row_budgets.dtype != torch.int32 or tuple(row_budgets.shape) != (B, H_kv)
                or not row_budgets.is_contiguous() or row_budgets.device != dev):
            raise ValueError(f"select_or_keep: row_budgets must be a contiguous int32 "
                             f"[{B}, {H_kv}] on {dev}")
        check(_lib.load().cvsa_select_or_keep_budgeted(
            ps.data_ptr(), _ptr(sel_scores), _ptr(check_accept), B, H_kv, W, ctx.data_ptr(),
            block_size, row_budgets.data_ptr(), budget, page_indices.data_ptr(),
            n_per_head.data_ptr(), float(tau), acc.data_ptr(), coverage.data_ptr(),
            _ptr(scores_cache), _ptr(stats), 1 if count_gate else 0, _stream(dev)),
            "select_or_keep")
        return acc.view(torch.bool)
    check(_lib.load().cvsa_select_or_keep(
        ps.data_ptr(), _ptr(sel_scores), _ptr(check_accept), B, H_kv, W, ctx.data_ptr(),
        block_size, budget,
        page_indices.data_ptr(), n_per_head.data_ptr(), float(tau), acc.data_ptr(),
        coverage.data_ptr(), _ptr(scores_cache), _ptr(stats), 1 if count_gate else 0,
        _stream(dev)), "select_or_keep")
    return acc.view(torch.bool)


def check_coverage(page_scores: torch.Tensor, selected_indices: torch.Tensor,
                   n_per_head: torch.Tensor, tau: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """coverage = exp(lse(selected) - lse(all)); accept = coverage >= tau.

    Mirrors triton_check_coverage (cvsa/kernels/coverage.py:218-265).
    Returns (accept_mask [B, H_kv] bool, coverage [B, H_kv] float32).
    """
    dev = _device_of(page_scores, selected_indices, n_per_head)
    if page_scores.dtype != torch.float32 or page_scores.dim() != 3:
        raise ValueError("page_scores must be [B, H_kv, W] float32")
    ps = page_scores.contiguous()
    B, H_kv, W = ps.shape
    sel = _i32(selected_indices)
    if sel.dim() != 3 or sel.shape[:2] != (B, H_kv):
        raise ValueError("selected_indices must be [B, H_kv, budget]")
    nph = _i32(n_per_head).reshape(B * H_kv)
    acc = torch.empty(B, H_kv, device=dev, dtype=torch.uint8)
    cov = torch.empty(B, H_kv, device=dev, dtype=torch.float32)
    check(_lib.load().cvsa_check_coverage(
        ps.data_ptr(), B, H_kv, W, sel.data_ptr(), sel.shape[2], nph.data_ptr(),
        float(tau), acc.data_ptr(), cov.data_ptr(), _stream(dev)), "check_coverage")
    return acc.view(torch.bool), cov


# ---------------------------------------------------------------- Quest

def _check_quest_state(meta, meta_ntok, k_cache):
    nb, _, H, D = k_cache.shape
    if meta.shape != (nb, H, 2, D) or meta.dtype != torch.bfloat16 or not meta.is_contiguous():
        raise ValueError(f"meta must be a contiguous bfloat16 [{nb}, {H}, 2, {D}]")
    if (meta_ntok.shape != (nb, H) or meta_ntok.dtype != torch.int32
            or not meta_ntok.is_contiguous()):
        raise ValueError(f"meta_ntok must be a contiguous int32 [{nb}, {H}]")


def quest_meta_update(k_cache: torch.Tensor, block_tables: torch.Tensor,
                      context_lens: torch.Tensor, meta: torch.Tensor,
                      meta_ntok: torch.Tensor) -> None:
    """Refresh the Quest page metadata (per block and KV head: key min and
    max over the page's valid tokens) of every page whose valid-token count
    differs from ``meta_ntok``; see cvsa_quest_meta_update.  ``meta`` is
    [num_blocks, H_kv, 2, D] bf16, ``meta_ntok`` [num_blocks, H_kv] int32
    (zero before the first update)."""
    dev = _device_of(k_cache, block_tables, context_lens, meta, meta_ntok)
    _check_cache(k_cache)
    _check_quest_state(meta, meta_ntok, k_cache)
    nb, bs, H, D = k_cache.shape
    bt = _block_tables(block_tables)
    ctx = _i32(context_lens)
    if bt.dim() != 2:
        raise ValueError(f"quest_meta_update: block_tables must be [B, W], got {tuple(bt.shape)}")
    B, W = bt.shape
    _check_seqs("quest_meta_update", B, bt, ctx)
    check(_lib.load().cvsa_quest_meta_update(
        k_cache.data_ptr(), nb, bt.data_ptr(), bt.stride(0), ctx.data_ptr(), B, H, D, bs, W,
        meta.data_ptr(), meta_ntok.data_ptr(), _stream(dev)), "quest_meta_update")


def quest_scores(q: torch.Tensor, meta: torch.Tensor, block_tables: torch.Tensor,
                 context_lens: torch.Tensor, num_kv_heads: int, num_q_per_kv: int,
                 block_size: int) -> torch.Tensor:
    """Quest page scores [B, H_kv, W] fp32 from the page metadata: the
    ranking of CVSABackend._quest_page_scores (cvsa/backend.py:572-620)."""
    dev = _device_of(q, meta, block_tables, context_lens)
    q = _check_q(q)
    B, H_q, D = q.shape
    if num_kv_heads * num_q_per_kv != H_q:
        raise ValueError("quest_scores: head counts do not match q")
    _check_meta(meta, num_kv_heads, D)
    bt = _block_tables(block_tables)
    ctx = _i32(context_lens)
    _check_seqs("quest_scores", B, bt, ctx)
    W = bt.shape[1]
    out = torch.empty(B, num_kv_heads, W, device=dev, dtype=torch.float32)
    check(_lib.load().cvsa_quest_scores(
        q.data_ptr(), q.stride(0), q.stride(1), meta.data_ptr(), meta.shape[0], bt.data_ptr(),
        bt.stride(0), ctx.data_ptr(), B, H_q, num_kv_heads, D, block_size, W, out.data_ptr(),
        _stream(dev)), "quest_scores")
    return out


def _check_meta(meta, num_kv_heads, D):
    if (meta.dim() != 4 or meta.shape[1:] != (num_kv_heads, 2, D)
            or meta.dtype != torch.bfloat16 or not meta.is_contiguous()):
        raise ValueError(f"meta must be a contiguous bfloat16 [num_blocks, {num_kv_heads}, 2, {D}]")


def quest_refresh_scores(q: torch.Tensor, k_cache: torch.Tensor, block_tables: torch.Tensor,
                         context_lens: torch.Tensor, meta: torch.Tensor, meta_ntok: torch.Tensor,
                         num_kv_heads: int, num_q_per_kv: int, block_size: int,
                         check_accept: Optional[torch.Tensor] = None,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """quest_meta_update followed by quest_scores, in one launch
    (cvsa_quest_refresh_scores).  With ``check_accept`` (a lazy check's
    [B, H_kv] flags) nothing is computed when every head passed: ``out``
    then keeps its previous contents."""
    dev = _device_of(q, k_cache, meta, meta_ntok, block_tables, context_lens, check_accept, out)
    q = _check_q(q)
    _check_cache(k_cache)
    _check_quest_state(meta, meta_ntok, k_cache)
    nb, bs, H, D = k_cache.shape
    B, H_q, _ = q.shape
    if num_kv_heads * num_q_per_kv != H_q or H != num_kv_heads:
        raise ValueError("quest_refresh_scores: head counts do not match q / k_cache")
    bt = _block_tables(block_tables)
    ctx = _i32(context_lens)
    _check_seqs("quest_refresh_scores", B, bt, ctx)
    W = bt.shape[1]
    if check_accept is not None and (check_accept.shape != (B, num_kv_heads)
                                     or check_accept.dtype != torch.bool
                                     or not check_accept.is_contiguous()):
        raise ValueError(f"check_accept must be a contiguous bool [{B}, {num_kv_heads}]")
    if out is None:
        out = torch.empty(B, num_kv_heads, W, device=dev, dtype=torch.float32)
    elif out.shape != (B, num_kv_heads, W) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous float32 [{B}, {num_kv_heads}, {W}]")
    check(_lib.load().cvsa_quest_refresh_scores(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), nb, bt.data_ptr(),
        bt.stride(0), ctx.data_ptr(), _ptr(check_accept), B, H_q, num_kv_heads, D, block_size, W,
        meta.data_ptr(), meta_ntok.data_ptr(), out.data_ptr(), _stream(dev)),
        "quest_refresh_scores")
    return out


class QuestPageMeta:
    """The Quest metadata of one paged key cache, kept current across calls.

    ``meta`` [num_blocks, H_kv, 2, D] bf16 holds each block's key extremes
    and ``ntok`` [num_blocks, H_kv] int32 the number of tokens they cover.
    ``scores(...)`` recomputes the pages whose valid-token count changed
    and scores every page, in one launch.  Valid while keys are only
    appended; ``invalidate()`` forgets every block (needed when blocks are
    rewritten, e.g. reused for another sequence).
    """

    def __init__(self, k_cache: torch.Tensor):
        _check_cache(k_cache)
        nb, _, H, D = k_cache.shape
        self.k_cache = k_cache
        self.meta = torch.empty(nb, H, 2, D, device=k_cache.device, dtype=torch.bfloat16)
        self.ntok = torch.zeros(nb, H, device=k_cache.device, dtype=torch.int32)

    def invalidate(self) -> None:
        self.ntok.zero_()

    def scores(self, q, block_tables, context_lens, num_kv_heads, num_q_per_kv, block_size,
               check_accept=None, out=None):
        return quest_refresh_scores(q, self.k_cache, block_tables, context_lens, self.meta,
                                    self.ntok, num_kv_heads, num_q_per_kv, block_size,
                                    check_accept, out)


# ---------------------------------------------------------------- decode

class DecodeCall:
    """A validated decode launch whose buffers stay fixed between calls.

    Built by :func:`prepare_decode`; ``run(q)`` launches it for a new query
    of the same shape and strides, allocating only the outputs.  ``matches``
    tells whether the call can be reused for a given set of buffers (same
    tensor objects, same stream); callers that hold a DecodeCall across
    steps check it before every use.
    """

    __slots__ = ("fn", "args", "kind", "dev", "stream", "q_meta", "out_shape", "out_dtype",
                 "want_state", "refs", "reusable", "_out_i", "_state_i")

    def matches(self, q, k_cache, v_cache, block_tables, context_lens, work) -> bool:
        r = self.refs
        return (self.reusable and r[0] is k_cache and r[1] is v_cache and r[2] is block_tables
                and r[3] is context_lens and r[4] is work
                and torch._C._cuda_getCurrentRawStream(self.dev.index) == self.stream
                and q.device == self.dev and q.dtype == torch.bfloat16
                and (q.shape, q.stride()) == self.q_meta and q.data_ptr() % 16 == 0)

    def run(self, q):
        args = self.args
        args[0] = q.data_ptr()
        o = m = l = out = None
        if self.want_state:
            B, H_q, D = self.out_shape
            o = torch.empty(B, H_q, D, device=self.dev, dtype=torch.float32)
            m = torch.empty(B, H_q, device=self.dev, dtype=torch.float32)
            l = torch.empty(B, H_q, device=self.dev, dtype=torch.float32)
            i = self._state_i
            args[i], args[i + 1], args[i + 2] = o.data_ptr(), m.data_ptr(), l.data_ptr()
        if self.out_dtype is not None:
            out = torch.empty(self.out_shape, device=self.dev, dtype=self.out_dtype)
            args[self._out_i] = out.data_ptr()
        check(self.fn(*args), self.kind)
        return o, m, l, out


def prepare_decode(kind: str, q, k_cache, v_cache, block_tables, context_lens, num_kv_heads,
                   num_q_per_kv, block_size, pi_flat=None, nph_flat=None, max_sel=0,
                   accept=None, want_state=False, want_out=True, out_dtype=None,
                   work=None, exp_flat=None, exp_budget=0) -> DecodeCall:
    """Validate a decode launch and build its argument list (see DecodeCall)."""
    dev = _device_of(q, k_cache, v_cache, block_tables, context_lens, pi_flat, nph_flat,
                     accept, work, exp_flat)
    if work is not None and (work.dtype != torch.int64 or work.numel() < 2
                             or not work.is_contiguous()):
        raise ValueError(f"{kind}: work must be a contiguous int64 tensor of 2 counters")
    q = _check_q(q)
    _check_cache(k_cache)
    _check_cache(v_cache, "v_cache")
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache shapes differ")
    bt = _block_tables(block_tables)
    ctx = _i32(context_lens)
    B, H_q, D = q.shape
    _check_seqs(kind, B, bt, ctx)
    rows = B * num_kv_heads
    if pi_flat is not None:
        _check_rows(kind, "page_indices", pi_flat, rows, max_sel)
        _check_count(kind, "n_per_head", nph_flat, rows)
    _check_count(kind, "accept_mask", accept, rows)
    if exp_flat is not None:
        _check_rows(kind, "exp_indices", exp_flat, rows, exp_budget)
    if num_kv_heads * num_q_per_kv != H_q or k_cache.shape[2] != num_kv_heads:
        raise ValueError(f"{kind}: head counts do not match q / caches")
    if k_cache.shape[1] != block_size or k_cache.shape[3] != D:
        raise ValueError(f"{kind}: cache block_size / head_dim mismatch")
    W = bt.shape[1]
    L = _lib.load()
    listed = pi_flat is not None
    all_pages = kind in ("dense_decode", "verified_decode", "verified_decode_approx")
    need = L.cvsa_decode_workspace_bytes(B, H_q, num_kv_heads, D, max_sel if listed else 0,
                                         W, 1 if all_pages else 0)
    ws = _workspace(dev, need)
    od = None
    code = 0
    if want_out:
        od = out_dtype or q.dtype
        if od not in _DTYPE_CODE:
            raise ValueError(f"unsupported output dtype {od}")
        code = _DTYPE_CODE[od]
    stream = torch._C._cuda_getCurrentRawStream(dev.index)
    head = [q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.shape[0], bt.data_ptr(), bt.stride(0), ctx.data_ptr()]
    if kind == "sparse_decode":
        fn = L.cvsa_sparse_decode
        mid = [pi_flat.data_ptr(), pi_flat.stride(0), nph_flat.data_ptr(), max_sel]
    elif kind == "dense_decode":
        fn = L.cvsa_dense_decode
        mid = []
    elif kind == "verified_decode":
        fn = L.cvsa_verified_decode
        mid = [pi_flat.data_ptr(), pi_flat.stride(0), nph_flat.data_ptr(), max_sel,
               accept.data_ptr()]
    else:
        fn = L.cvsa_verified_decode_approx
        mid = [pi_flat.data_ptr(), pi_flat.stride(0), nph_flat.data_ptr(), max_sel,
               accept.data_ptr(), exp_flat.data_ptr(), exp_flat.stride(0), exp_budget]
    sizes = [B, H_q, num_kv_heads, D, block_size, W]
    tail = [None, None, None, None, code, _ptr(work), _ptr(ws),
            0 if ws is None else ws.numel(), stream]
    c = DecodeCall()
    c.fn = fn
    c.args = head + mid + sizes + tail
    c._state_i = len(head) + len(mid) + len(sizes)
    c._out_i = c._state_i + 3
    c.kind = kind
    c.dev = dev
    c.stream = stream
    c.q_meta = (q.shape, q.stride())
    c.out_shape = (B, H_q, D)
    c.out_dtype = od
    c.want_state = want_state
    # The tensors the launch reads; the converted ones (if any) are kept
    # alive here but make the call non-reusable, since their content is a
    # snapshot of the caller's tensors.
    c.refs = (k_cache, v_cache, block_tables, context_lens, work, bt, ctx, pi_flat, nph_flat,
              accept, ws, exp_flat)
    c.reusable = bt is block_tables and ctx is context_lens
    return c


def _decode(kind: str, q, k_cache, v_cache, block_tables, context_lens, num_kv_heads,
            num_q_per_kv, block_size, pi_flat=None, nph_flat=None, max_sel=0,
            accept=None, want_state=False, want_out=True, out_dtype=None, work=None,
            exp_flat=None, exp_budget=0):
    c = prepare_decode(kind, q, k_cache, v_cache, block_tables, context_lens, num_kv_heads,
                       num_q_per_kv, block_size, pi_flat, nph_flat, max_sel, accept, want_state,
                       want_out, out_dtype, work, exp_flat, exp_budget)
    return c.run(_check_q(q))


class StepPlan:
    """One layer's decode steps, each enqueued by one native call.

    Wraps cvsa_step_plan_* (include/cvsa_hip.h): ``run(kind, q)`` enqueues a
    reuse step (sparse decode of the layer's selection), a lazy check (fresh
    scores, coverage of the kept selection, keep it or reselect in place,
    decode with exact recovery) or a fixed-interval scoring step (reselect,
    gate booked in ``stats``, decode) for a new query and returns the
    [B, H_q, D] output in q's dtype.  The sequences are those of
    CVSABackend._reuse_step, _lazy_step and _scoring_step
    (cvsa/backend.py:866-881, :392-465, :683-864).

    The plan keeps the layer's selection (``page_indices`` [B, H_kv, budget],
    ``n_per_head`` [B, H_kv], updated in place; allocated by the plan when
    not given, ``owns_selection``), the step's ``page_scores`` [B, H_kv, W],
    an optional ``scores_cache`` (the scores of the last reselection, given
    or allocated with ``own_scores_cache``) and gate buffers ``check_accept``
    / ``accept`` / ``coverage`` [B, H_kv]; every check or scoring step
    rewrites the latter.  Kind STEP_FRESH makes a lazy layer's first
    selection in the plan's buffers.
    ``selector`` (_lib.SELECT_*) picks the page scorer: exact scores rank
    and gate; SELECT_QUEST ranks by the Quest scores of ``quest`` (a
    QuestPageMeta of k_cache) into ``sel_scores`` while exact scores gate;
    SELECT_QUEST_LN ranks and gates by the Quest scores.
    ``matches`` tells whether a call's buffers, query layout and stream are
    the ones the plan was built for.
    With ``approx_budget`` > 0 the plan's checks and scoring steps recover
    rejected heads approximately (CVSABackend approx_recovery_pct,
    cvsa/backend.py:780-817): the selection step writes each rejected
    row's expanded selection into ``approx_indices`` [B, H_kv,
    approx_budget] and the decode attends it (cvsa_verified_decode_approx).
    With ``speculate`` (default) a lazy check decodes the cached selection
    in the same launch as the page scoring, and the verified decode skips
    its work when the check kept that selection (see
    cvsa_step_desc.spec_state; exact gate scores, H_kv in 4, 8, 16 and D = 128
    only); with 16-token pages that decode also scores the selection's pages
    from the keys it reads, which the page scoring then skips (``sel_map``,
    the selection's page map).  Results are bit-identical either way.  A caller that writes
    ``page_indices`` / ``n_per_head`` itself calls ``selection_changed()``.
    """

    __slots__ = ("dev", "stream", "q_meta", "out_shape", "out_dtype", "refs", "page_indices",
                 "n_per_head", "page_scores", "scores_cache", "check_accept", "accept",
                 "coverage", "budget", "owns_selection", "selector", "sel_scores", "spec_state",
                 "sel_map", "approx_budget", "approx_indices", "h_kv", "_h", "_run",
                 "_run_append", "_pa_ok", "_slots_ok", "_fin", "__weakref__")

    def __init__(self, q, k_cache, v_cache, block_tables, context_lens, num_kv_heads,
                 num_q_per_kv, block_size, budget, tau, page_indices=None, n_per_head=None,
                 scores_cache=None, stats=None, work=None, own_scores_cache=False,
                 selector=_lib.SELECT_EXACT, quest=None, speculate=True, approx_budget=0):
        dev = _device_of(q, k_cache, v_cache, block_tables, context_lens, page_indices,
                         n_per_head, scores_cache, stats, work)
        if selector not in (_lib.SELECT_EXACT, _lib.SELECT_QUEST, _lib.SELECT_QUEST_LN):
            raise ValueError(f"step plan: unknown selector {selector}")
        if (selector != _lib.SELECT_EXACT) != (quest is not None):
            raise ValueError("step plan: the Quest selectors need quest metadata, the exact "
                             "one none")
        if quest is not None and (quest.k_cache is not k_cache or quest.meta.device != dev):
            raise ValueError("step plan: quest metadata belongs to another key cache")
        q = _check_q(q)
        _check_cache(k_cache)
        _check_cache(v_cache, "v_cache")
        if k_cache.shape != v_cache.shape:
            raise ValueError("k_cache and v_cache shapes differ")
        if (block_tables.dtype != torch.int32 or block_tables.dim() != 2
                or block_tables.stride(1) != 1 or context_lens.dtype != torch.int32
                or not context_lens.is_contiguous()):
            raise ValueError("step plan: block_tables must be int32 [B, W] with unit page "
                             "stride and context_lens contiguous int32")
        B, H_q, D = q.shape
        _check_seqs("step plan", B, block_tables, context_lens)
        H = num_kv_heads
        if H * num_q_per_kv != H_q or k_cache.shape[2] != H:
            raise ValueError("step plan: head counts do not match q / caches")
        if k_cache.shape[1] != block_size or k_cache.shape[3] != D:
            raise ValueError("step plan: cache block_size / head_dim mismatch")
        W = block_tables.shape[1]
        self.owns_selection = page_indices is None
        if page_indices is None:
            page_indices = torch.empty(B, H, budget, dtype=torch.int32, device=dev)
            n_per_head = torch.empty(B, H, dtype=torch.int32, device=dev)
        if own_scores_cache:
            scores_cache = torch.empty(B, H, W, dtype=torch.float32, device=dev)
        for name, t, shape, dt in (("page_indices", page_indices, (B, H, budget), torch.int32),
                                   ("n_per_head", n_per_head, (B, H), torch.int32)):
            if tuple(t.shape) != shape or t.dtype != dt or not t.is_contiguous():
                raise ValueError(f"step plan: {name} must be a contiguous {dt} {shape}")
        if scores_cache is not None and (tuple(scores_cache.shape) != (B, H, W)
                                         or scores_cache.dtype != torch.float32
                                         or not scores_cache.is_contiguous()):
            raise ValueError("step plan: scores_cache must be a contiguous float32 [B, H_kv, W]")
        for name, t, n in (("stats", stats, 6), ("work", work, 2)):
            if t is not None and (t.dtype != torch.int64 or t.numel() < n
                                  or not t.is_contiguous()):
                raise ValueError(f"step plan: {name} must be a contiguous int64[>= {n}]")
        if q.dtype not in _DTYPE_CODE:
            raise ValueError(f"unsupported output dtype {q.dtype}")
        self.page_scores = torch.empty(B, H, W, dtype=torch.float32, device=dev)
        self.check_accept = torch.empty(B, H, dtype=torch.uint8, device=dev)
        self.accept = torch.empty(B, H, dtype=torch.uint8, device=dev)
        self.coverage = torch.empty(B, H, dtype=torch.float32, device=dev)
        self.selector = selector
        self.sel_scores = (torch.empty(B, H, W, dtype=torch.float32, device=dev)
                           if selector == _lib.SELECT_QUEST else None)
        # [0]: the previous check kept its selection (predicted for the first
        # check), [1]: the speculative decode ran.
        self.spec_state = (torch.tensor([1, 0], dtype=torch.int32, device=dev)
                           if speculate else None)
        # Byte p of row b * H_kv + h: page p is in the selection (rows of W
        # rounded up to 16 bytes; zero past W).
        map_stride = (W + 15) // 16 * 16
        self.sel_map = (torch.zeros(B * H, map_stride, dtype=torch.uint8, device=dev)
                        if speculate and block_size == 16 else None)
        # Approximate recovery: the expanded selections of the rows that a
        # selection step rejected (rows of accepted heads are stale).
        if not 0 <= approx_budget <= W:
            raise ValueError(f"step plan: approx_budget={approx_budget} not in [0, W={W}]")
        self.approx_budget = approx_budget
        self.approx_indices = (torch.zeros(B, H, approx_budget, dtype=torch.int32, device=dev)
                               if approx_budget > 0 else None)
        d = _lib.StepDesc(
            B=B, H_q=H_q, H_kv=H, D=D, block_size=block_size, W=W, budget=budget,
            tau=float(tau), out_dtype=_DTYPE_CODE[q.dtype], q_stride_b=q.stride(0),
            q_stride_h=q.stride(1), k_cache=k_cache.data_ptr(), v_cache=v_cache.data_ptr(),
            num_blocks=k_cache.shape[0], block_tables=block_tables.data_ptr(),
            bt_stride_b=block_tables.stride(0), context_lens=context_lens.data_ptr(),
            page_indices=page_indices.data_ptr(), n_per_head=n_per_head.data_ptr(),
            page_scores=self.page_scores.data_ptr(), scores_cache=_ptr(scores_cache),
            check_accept=self.check_accept.data_ptr(), accept=self.accept.data_ptr(),
            coverage=self.coverage.data_ptr(), stats=_ptr(stats), work=_ptr(work),
            selector=selector, quest_meta=None if quest is None else quest.meta.data_ptr(),
            quest_ntok=None if quest is None else quest.ntok.data_ptr(),
            sel_scores=_ptr(self.sel_scores), spec_state=_ptr(self.spec_state),
            sel_map=_ptr(self.sel_map), sel_map_stride=map_stride,
            approx_budget=approx_budget, approx_indices=_ptr(self.approx_indices))
        L = _lib.load()
        ws = _workspace(dev, L.cvsa_step_workspace_bytes(ctypes.byref(d)))
        d.workspace = _ptr(ws)
        d.workspace_bytes = 0 if ws is None else ws.numel()
        h = ctypes.c_void_p()
        check(L.cvsa_step_plan_create(ctypes.byref(d), ctypes.byref(h)), "step_plan_create")
        self._h = h.value
        self._run = L.cvsa_step_plan_run
        self._run_append = L.cvsa_step_plan_run_append
        self._pa_ok = self._slots_ok = None     # append buffers already checked
        self.h_kv = H
        self._fin = weakref.finalize(self, L.cvsa_step_plan_destroy, h.value)
        self.dev = dev
        self.stream = _stream(dev)
        self.q_meta = (q.shape, q.stride())
        self.out_shape = (B, H_q, D)
        self.out_dtype = q.dtype
        self.page_indices = page_indices
        self.n_per_head = n_per_head
        self.scores_cache = scores_cache
        self.budget = budget
        # Every buffer the plan's launches touch stays alive with the plan.
        self.refs = (k_cache, v_cache, block_tables, context_lens, work, stats, ws, quest)

    def matches(self, q, k_cache, v_cache, block_tables, context_lens, work, stats,
                quest=None) -> bool:
        r = self.refs
        return (r[0] is k_cache and r[1] is v_cache and r[2] is block_tables
                and r[3] is context_lens and r[4] is work and r[5] is stats and r[7] is quest
                and torch._C._cuda_getCurrentRawStream(self.dev.index) == self.stream
                and q.device == self.dev and q.dtype == self.out_dtype
                and (q.shape, q.stride()) == self.q_meta and q.data_ptr() % 16 == 0)

    def selection_changed(self) -> None:
        """page_indices / n_per_head were written outside the plan
        (cvsa_step_plan_selection_changed)."""
        check(_lib.load().cvsa_step_plan_selection_changed(self._h), "step_plan_selection_changed")

    def run(self, kind: int, q: torch.Tensor) -> torch.Tensor:
        out = torch.empty(self.out_shape, device=self.dev, dtype=self.out_dtype)
        check(self._run(self._h, kind, q.data_ptr(), out.data_ptr(), self.stream),
              "step_plan_run")
        return out

    def run_reuse_append(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                         pages_allocated: torch.Tensor, slots=None,
                         slots_dev: Optional[torch.Tensor] = None,
                         slot_errors: Optional[torch.Tensor] = None) -> torch.Tensor:
        """A reuse step with the step's token append folded in
        (cvsa_step_plan_run_append): k_new / v_new [B, H_kv, D] contiguous
        bf16, pages_allocated the int32 [B] allocation counts on the device,
        slots the host int32 array of SequenceKVManager.fused_append_slots,
        or slots_dev the same values in a contiguous int32 [B, 2] device
        tensor (for a launch a captured graph replays; a sequence whose
        device slot is out of range appends nothing and adds 1 to
        ``slot_errors``, an optional int32 device counter).  Writes the
        plan's caches, block table and context lengths."""
        who = "run_reuse_append"
        if (slots is None) == (slots_dev is None):
            raise ValueError(f"{who}: give exactly one of slots and slots_dev")
        B, H_q, D = self.out_shape
        if (q.device != self.dev or q.dtype != self.out_dtype
                or (q.shape, q.stride()) != self.q_meta):
            raise ValueError(f"{who}: q must have the plan's device, dtype, shape and strides")
        _check_new_rows(who, k_new, v_new, (B, self.h_kv, D), self.dev)
        if pages_allocated is not self._pa_ok:
            _check_pages_allocated(who, pages_allocated, B, self.dev)
            self._pa_ok = pages_allocated
        if slots_dev is not None:
            if slots_dev is not self._slots_ok:
                _append_slots(who, slots_dev, B, self.dev)
                self._slots_ok = slots_dev
            slot_arr = None
            _check_slot_errors(who, slot_errors, self.dev)
        else:
            slot_arr, _ = _append_slots(who, slots, B, self.dev)
        out = torch.empty(self.out_shape, device=self.dev, dtype=self.out_dtype)
        check(self._run_append(
            self._h, q.data_ptr(), out.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
            k_new.stride(0), pages_allocated.data_ptr(), slot_arr, _ptr(slots_dev),
            _ptr(slot_errors), self.stream), "step_plan_run_append")
        return out


def _check_new_rows(who: str, k_new, v_new, shape, dev) -> None:
    """k_new / v_new: the appended token's rows, contiguous bf16 ``shape`` on dev."""
    for t in (k_new, v_new):
        if (not isinstance(t, torch.Tensor) or t.dtype != torch.bfloat16
                or t.shape != shape or t.device != dev or not t.is_contiguous()):
            raise ValueError(f"{who}: k_new / v_new must be contiguous bfloat16 "
                             f"{tuple(shape)} on {dev}")


def _append_slots(who: str, slots, B: int, dev):
    """(host ctypes array, device tensor) of an append's 2 * B slot entries:
    a host sequence of (context length before the append, block to allocate
    or -1) per sequence, or the same in a contiguous int32 [B, 2] tensor on
    dev; exactly one of the two is returned non-None."""
    if isinstance(slots, torch.Tensor):
        if (slots.dtype != torch.int32 or slots.shape != (B, 2)
                or not slots.is_contiguous() or slots.device != dev):
            raise ValueError(f"{who}: device slots must be a contiguous int32 "
                             f"({B}, 2) tensor on {dev}")
        return None, slots
    if slots is None or len(slots) != 2 * B:
        raise ValueError(f"{who}: {2 * B} slot entries expected")
    if isinstance(slots, ctypes.Array) and slots._type_ is ctypes.c_int32:
        return slots, None
    return (ctypes.c_int32 * (2 * B))(*slots), None


def _check_slot_errors(who: str, slot_errors, dev) -> None:
    if slot_errors is not None and (
            not isinstance(slot_errors, torch.Tensor) or slot_errors.dtype != torch.int32
            or slot_errors.numel() < 1 or slot_errors.device != dev):
        raise ValueError(f"{who}: slot_errors must be an int32 device tensor on {dev}")


def _check_pages_allocated(who: str, pages_allocated, B: int, dev) -> None:
    if (not isinstance(pages_allocated, torch.Tensor) or pages_allocated.dtype != torch.int32
            or pages_allocated.shape != (B,) or pages_allocated.device != dev
            or not pages_allocated.is_contiguous()):
        raise ValueError(f"{who}: pages_allocated must be a contiguous int32 ({B},) tensor "
                         f"on {dev}")


def _flat_selection(page_indices: torch.Tensor, n_per_head: torch.Tensor, num_kv_heads: int):
    if page_indices.dim() != 3:
        raise ValueError("page_indices must be [B, H_kv, max_selected]")
    B, H, k = page_indices.shape
    if H != num_kv_heads:
        raise ValueError("page_indices head dimension does not match num_kv_heads")
    pi = _i32(page_indices).reshape(B * H, k)
    nph = _i32(n_per_head).reshape(B * H)
    return pi, nph, k


def sparse_decode_unnorm(q, k_cache, v_cache, block_tables, page_indices, n_per_head,
                         context_lens, num_kv_heads, num_q_per_kv, block_size=64):
    """Un-normalised sparse attention (O_unnorm [B,H_q,D], M [B,H_q], L [B,H_q]).

    Mirrors triton_sparse_decode_unnorm (cvsa/kernels/sparse_decode.py:537-573).
    A head with n_per_head = 0 gives (0, -inf, 0) where the reference gives
    NaN (the identity of the LSE merge instead of an undefined value).
    """
    pi, nph, k = _flat_selection(page_indices, n_per_head, num_kv_heads)
    o, m, l, _ = _decode("sparse_decode", q, k_cache, v_cache, block_tables, context_lens,
                         num_kv_heads, num_q_per_kv, block_size, pi, nph, k,
                         want_state=True, want_out=False)
    return o, m, l


def sparse_decode(q, k_cache, v_cache, block_tables, page_indices, n_per_head,
                  context_lens, num_kv_heads, num_q_per_kv, block_size=64):
    """Normalised sparse attention -> [B, H_q, D] in q.dtype.

    Mirrors triton_sparse_decode (cvsa/kernels/sparse_decode.py:286-350).
    Unlike the reference's tiled path (:371-383) the result never aliases
    a cached buffer.
    """
    pi, nph, k = _flat_selection(page_indices, n_per_head, num_kv_heads)
    return _decode("sparse_decode", q, k_cache, v_cache, block_tables, context_lens,
                   num_kv_heads, num_q_per_kv, block_size, pi, nph, k)[3]


def sparse_decode_append(q, k_cache, v_cache, block_tables, context_lens, page_indices,
                         n_per_head, k_new, v_new, pages_allocated, slots, num_kv_heads,
                         num_q_per_kv, block_size, work: Optional[torch.Tensor] = None,
                         slot_errors: Optional[torch.Tensor] = None):
    """append_kv of one token per sequence, then sparse_decode over the
    appended cache, in one launch where the shapes allow
    (cvsa_sparse_decode_append; no reference counterpart).

    ``slots``: a host sequence of 2 * B int32, (context length before the
    append, block the append allocates or -1) per sequence, as
    SequenceKVManager.fused_append_slots builds them, or the same values in a
    contiguous int32 [B, 2] tensor on the device (the one-launch shapes
    only: D = 128, 16-token pages, at most 16 query heads per KV head and
    256 sequences; the launch checks them, and a sequence whose slot is out
    of range appends nothing, gets an undefined output and adds 1 to
    ``slot_errors``, an optional int32 [1] device counter).  block_tables,
    context_lens and pages_allocated (contiguous int32) and the caches are
    updated in place.  Returns the normalised output [B, H_q, D] in q.dtype.
    """
    pi, nph, k = _flat_selection(page_indices, n_per_head, num_kv_heads)
    dev = _device_of(q, k_cache, v_cache, block_tables, context_lens, pi, nph, k_new, v_new,
                     pages_allocated, work)
    q = _check_q(q)
    _check_cache(k_cache)
    _check_cache(v_cache, "v_cache")
    for name, t in (("block_tables", block_tables), ("context_lens", context_lens),
                    ("pages_allocated", pages_allocated)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"sparse_decode_append: {name} must be contiguous int32")
    B, H_q, D = q.shape
    who = "sparse_decode_append"
    _check_seqs(who, B, block_tables, context_lens)
    _check_pages_allocated(who, pages_allocated, B, dev)
    _check_rows(who, "page_indices", pi, B * num_kv_heads, k)
    _check_count(who, "n_per_head", nph, B * num_kv_heads)
    if num_kv_heads * num_q_per_kv != H_q or k_cache.shape[2] != num_kv_heads:
        raise ValueError(f"{who}: head counts do not match q / caches")
    if k_cache.shape[1] != block_size or k_cache.shape[3] != D:
        raise ValueError("sparse_decode_append: cache block_size / head_dim mismatch")
    _check_new_rows("sparse_decode_append", k_new, v_new, (B, num_kv_heads, D), dev)
    slot_arr, slot_dev = _append_slots("sparse_decode_append", slots, B, dev)
    _check_slot_errors("sparse_decode_append", slot_errors, dev)
    W = block_tables.shape[1]
    L = _lib.load()
    need = L.cvsa_decode_workspace_bytes(B, H_q, num_kv_heads, D, k, W, 0)
    ws = _workspace(dev, need)
    out = torch.empty(B, H_q, D, device=dev, dtype=q.dtype)
    if q.dtype not in _DTYPE_CODE:
        raise ValueError(f"unsupported output dtype {q.dtype}")
    check(L.cvsa_sparse_decode_append(
        q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.shape[0], block_tables.data_ptr(), block_tables.stride(0),
        context_lens.data_ptr(), pi.data_ptr(), pi.stride(0), nph.data_ptr(), k, B, H_q,
        num_kv_heads, D, block_size, W, out.data_ptr(), _DTYPE_CODE[q.dtype], _ptr(work),
        _ptr(ws), 0 if ws is None else ws.numel(), k_new.data_ptr(), v_new.data_ptr(),
        k_new.stride(0), pages_allocated.data_ptr(), slot_arr, _ptr(slot_dev),
        _ptr(slot_errors), _stream(dev)), "sparse_decode_append")
    return out


def prepare_reuse_state(page_indices, n_per_head, num_kv_heads, B):
    """(pi_flat, nph_flat, padded_max_selected) for sparse_decode_reuse.

    Same contract as the reference (cvsa/kernels/sparse_decode.py:664-678):
    indices padded with 0 to a power of two, flattened to [B*H_kv, padded].
    """
    actual = page_indices.shape[2]
    padded = next_power_of_2(actual)
    pi = page_indices
    if padded > actual:
        pi = torch.nn.functional.pad(page_indices, (0, padded - actual), value=0)
    pi_flat = _i32(pi).reshape(B * num_kv_heads, padded).contiguous()
    nph_flat = _i32(n_per_head).reshape(B * num_kv_heads).contiguous()
    return pi_flat, nph_flat, padded


def sparse_decode_reuse(q, k_cache, v_cache, block_tables, context_lens, pi_flat, nph_flat,
                        padded_max_selected, num_kv_heads, num_q_per_kv, block_size,
                        work: Optional[torch.Tensor] = None):
    """Normalised sparse attention on a prepared selection -> [B, H_q, D].

    Mirrors triton_sparse_decode_reuse (cvsa/kernels/sparse_decode.py:681-721).
    ``work`` (int64[2]) accumulates the effective-budget counters.
    """
    return prepare_sparse_decode_reuse(q, k_cache, v_cache, block_tables, context_lens,
                                       pi_flat, nph_flat, padded_max_selected, num_kv_heads,
                                       num_q_per_kv, block_size, work).run(_check_q(q))[3]


def prepare_sparse_decode_reuse(q, k_cache, v_cache, block_tables, context_lens, pi_flat,
                                nph_flat, padded_max_selected, num_kv_heads, num_q_per_kv,
                                block_size, work: Optional[torch.Tensor] = None) -> DecodeCall:
    """The launch of sparse_decode_reuse as a reusable DecodeCall."""
    width = min(int(padded_max_selected), pi_flat.shape[1])
    return prepare_decode("sparse_decode", q, k_cache, v_cache, block_tables, context_lens,
                          num_kv_heads, num_q_per_kv, block_size, pi_flat, nph_flat, width,
                          work=work)


def dense_decode(q, k_cache, v_cache, block_tables, context_lens, num_kv_heads,
                 num_q_per_kv, block_size, return_state: bool = False,
                 work: Optional[torch.Tensor] = None):
    """Attention over every valid page -> [B, H_q, D] in q.dtype.

    The reference's dense fallback (cvsa/runtime/dense.py:40-68) selects all
    pages; here no index list is built at all.  With ``return_state`` also
    returns the un-normalised (o, m, l).
    """
    o, m, l, out = _decode("dense_decode", q, k_cache, v_cache, block_tables, context_lens,
                           num_kv_heads, num_q_per_kv, block_size, want_state=return_state,
                           work=work)
    return (out, (o, m, l)) if return_state else out


def verified_decode(q, k_cache, v_cache, block_tables, context_lens, page_indices, n_per_head,
                    accept_mask, num_kv_heads, num_q_per_kv, block_size,
                    return_state: bool = False, output_dtype=None,
                    work: Optional[torch.Tensor] = None):
    """Draft for accepted heads, exact recovery for rejected heads, one launch.

    Equivalent to the exact-recovery branch of CVSABackend._scoring_step
    (cvsa/backend.py:775-779, :818-844): accepted heads return the
    normalised draft over their selected pages; rejected heads return the
    LSE merge of draft and complement, which is attention over every valid
    page, computed here in a single pass over those pages.
    """
    pi, nph, k = _flat_selection(page_indices, n_per_head, num_kv_heads)
    acc = accept_mask
    if acc.dtype == torch.bool:
        acc = acc.view(torch.uint8)
    acc = acc.to(torch.uint8).contiguous().reshape(-1)
    o, m, l, out = _decode("verified_decode", q, k_cache, v_cache, block_tables, context_lens,
                           num_kv_heads, num_q_per_kv, block_size, pi, nph, k, accept=acc,
                           want_state=return_state, out_dtype=output_dtype, work=work)
    return (out, (o, m, l)) if return_state else out


def verified_decode_approx(q, k_cache, v_cache, block_tables, context_lens, page_indices,
                           n_per_head, accept_mask, exp_indices, num_kv_heads, num_q_per_kv,
                           block_size, return_state: bool = False, output_dtype=None,
                           work: Optional[torch.Tensor] = None):
    """Draft for accepted heads, approximate recovery for rejected heads.

    Equivalent to the approximate-recovery branch of
    CVSABackend._scoring_step (cvsa/backend.py:775-817): accepted heads
    return the normalised draft over their selected pages, rejected heads
    the normalised sparse decode of the first min(exp_budget, n_valid)
    pages of their row of ``exp_indices`` [B, H_kv, exp_budget] (the
    expanded top-k, e.g. ``select_topk(scores, exp_budget, ...)``).  The
    effective-budget counters book what the reference books: when a head
    is rejected, n_per_head + min(exp_budget, n_valid) on every head.
    """
    pi, nph, k = _flat_selection(page_indices, n_per_head, num_kv_heads)
    if exp_indices.dim() != 3 or exp_indices.shape[:2] != page_indices.shape[:2]:
        raise ValueError("exp_indices must be [B, H_kv, exp_budget]")
    exp_budget = exp_indices.shape[2]
    ex = _i32(exp_indices).reshape(-1, exp_budget)
    acc = accept_mask
    if acc.dtype == torch.bool:
        acc = acc.view(torch.uint8)
    acc = acc.to(torch.uint8).contiguous().reshape(-1)
    o, m, l, out = _decode("verified_decode_approx", q, k_cache, v_cache, block_tables,
                           context_lens, num_kv_heads, num_q_per_kv, block_size, pi, nph, k,
                           accept=acc, want_state=return_state, out_dtype=output_dtype,
                           work=work, exp_flat=ex, exp_budget=exp_budget)
    return (out, (o, m, l)) if return_state else out


# ---------------------------------------------------------------- recovery

def compute_complement(page_indices, n_per_head, context_lens, block_size, accept_mask,
                       width: Optional[int] = None):
    """Valid pages not selected, ascending, per (b, kv-head); 0 for accepted heads.

    Mirrors triton_compute_complement (cvsa/kernels/coverage.py:99-150):
    returns (complement [B, H_kv, width] int32,
    n_complement [B, H_kv] int32).  ``width`` defaults to max_b n_valid(b),
    which costs one host sync as in the reference (coverage.py:121); pass
    it (e.g. the block-table width) to avoid the sync.
    """
    dev = _device_of(page_indices, n_per_head, context_lens, accept_mask)
    B, H, k = page_indices.shape
    pi = _i32(page_indices).reshape(B * H, k)
    nph = _i32(n_per_head).reshape(B * H)
    ctx = _i32(context_lens)
    _check_seqs("compute_complement", B, None, ctx)
    _check_count("compute_complement", "accept_mask", accept_mask, B * H)
    if width is None:
        width = int(((ctx.max().item() - 1) // block_size) + 1)
        width = max(width, 1)
    acc = None
    if accept_mask is not None:
        acc = accept_mask.view(torch.uint8) if accept_mask.dtype == torch.bool else accept_mask
        acc = acc.to(torch.uint8).contiguous().reshape(-1)
    comp = torch.empty(B, H, width, device=dev, dtype=torch.int32)
    ncomp = torch.empty(B, H, device=dev, dtype=torch.int32)
    check(_lib.load().cvsa_compute_complement(
        pi.data_ptr(), pi.stride(0), nph.data_ptr(), ctx.data_ptr(), block_size, _ptr(acc),
        B, H, width, comp.data_ptr(), ncomp.data_ptr(), _stream(dev)), "compute_complement")
    return comp, ncomp


def lse_merge(o_draft, m_draft, l_draft, o_comp, m_comp, l_comp, accept_mask, num_kv_heads,
              num_q_per_kv, output_dtype=torch.bfloat16):
    """Per-head merge: accepted -> normalised draft, rejected -> LSE merge.

    Mirrors triton_lse_merge (cvsa/kernels/coverage.py:329-367).
    """
    dev = _device_of(o_draft, m_draft, l_draft, o_comp, m_comp, l_comp, accept_mask)
    B, H_q, D = o_draft.shape
    if num_kv_heads * num_q_per_kv != H_q:
        raise ValueError("lse_merge: head counts do not match")
    _check_count("lse_merge", "o_comp", o_comp, B * H_q * D)
    for name, t in (("m_draft", m_draft), ("l_draft", l_draft), ("m_comp", m_comp),
                    ("l_comp", l_comp)):
        _check_count("lse_merge", name, t, B * H_q)
    _check_count("lse_merge", "accept_mask", accept_mask, B * num_kv_heads)
    f32 = lambda t: t.to(torch.float32).contiguous()
    od, md, ld, oc, mc, lc = map(f32, (o_draft, m_draft, l_draft, o_comp, m_comp, l_comp))
    acc = accept_mask.view(torch.uint8) if accept_mask.dtype == torch.bool else accept_mask
    acc = acc.to(torch.uint8).contiguous()
    if output_dtype not in _DTYPE_CODE:
        raise ValueError(f"unsupported output dtype {output_dtype}")
    out = torch.empty(B, H_q, D, device=dev, dtype=output_dtype)
    check(_lib.load().cvsa_lse_merge(
        od.data_ptr(), md.data_ptr(), ld.data_ptr(), oc.data_ptr(), mc.data_ptr(), lc.data_ptr(),
        acc.data_ptr(), B, H_q, num_kv_heads, D, out.data_ptr(), _DTYPE_CODE[output_dtype],
        _stream(dev)), "lse_merge")
    return out


# ---------------------------------------------------------------- KV append

def append_kv(k_new, v_new, k_cache, v_cache, block_tables, context_lens, pages_allocated,
              seq_begin: int, next_free_block: int, block_size: int) -> None:
    """Append one token per sequence [seq_begin, seq_begin + k_new.shape[0]).

    Device-side form of SequenceKVManager.append_token_kv
    (cvsa/runtime/kv_cache.py:133-150); see cvsa_append_kv in the C header.
    block_tables, context_lens and pages_allocated are updated in place and
    must be contiguous int32.
    """
    dev = _device_of(k_new, v_new, k_cache, v_cache, block_tables, context_lens,
                     pages_allocated)
    _check_cache(k_cache)
    _check_cache(v_cache, "v_cache")
    for name, t in (("block_tables", block_tables), ("context_lens", context_lens),
                    ("pages_allocated", pages_allocated)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"append_kv: {name} must be contiguous int32")
    n = k_new.shape[0]
    if not 1 <= n <= 1024:
        raise ValueError(f"append_kv: {n} sequences per call (1..1024 supported)")
    batch = block_tables.shape[0] if block_tables.dim() == 2 else -1
    _check_seqs("append_kv", batch, block_tables, context_lens)
    _check_count("append_kv", "pages_allocated", pages_allocated, batch)
    if not (0 <= seq_begin and seq_begin + n <= batch):
        raise ValueError(f"append_kv: sequences [{seq_begin}, {seq_begin + n}) outside the "
                         f"batch of {batch}")
    H_kv, D = k_cache.shape[2], k_cache.shape[3]
    kn = k_new.to(torch.bfloat16).reshape(n, H_kv * D).contiguous()
    vn = v_new.to(torch.bfloat16).reshape(n, H_kv * D).contiguous()
    check(_lib.load().cvsa_append_kv(
        kn.data_ptr(), vn.data_ptr(), kn.stride(0), k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.shape[0], block_tables.data_ptr(), block_tables.stride(0),
        block_tables.shape[1], context_lens.data_ptr(), pages_allocated.data_ptr(), seq_begin,
        n, next_free_block, H_kv, D, block_size, _stream(dev)), "append_kv")


class AppendCall:
    """A validated cvsa_append_kv launch over fixed cache and table buffers.

    Built once per set of buffers (and stream); ``run(k, v, seq_begin,
    next_free_block)`` appends one token per sequence with only the per-call
    arguments set, for the host cost of a decode loop that appends every
    layer of every step.  ``k`` / ``v`` must be contiguous bfloat16
    [n, H_kv, D] on the cache's device.
    """

    __slots__ = ("fn", "args", "dev", "stream", "refs", "H_kv", "D", "batch")

    def __init__(self, k_cache, v_cache, block_tables, context_lens, pages_allocated,
                 block_size: int):
        dev = _device_of(k_cache, v_cache, block_tables, context_lens, pages_allocated)
        _check_cache(k_cache)
        _check_cache(v_cache, "v_cache")
        if k_cache.shape != v_cache.shape:
            raise ValueError("append_kv: k_cache and v_cache shapes differ")
        for name, t in (("block_tables", block_tables), ("context_lens", context_lens),
                        ("pages_allocated", pages_allocated)):
            if t.dtype != torch.int32 or not t.is_contiguous():
                raise ValueError(f"append_kv: {name} must be contiguous int32")
        self.H_kv, self.D = k_cache.shape[2], k_cache.shape[3]
        self.batch = block_tables.shape[0] if block_tables.dim() == 2 else -1
        _check_seqs("append_kv", self.batch, block_tables, context_lens)
        _check_count("append_kv", "pages_allocated", pages_allocated, self.batch)
        self.fn = _lib.load().cvsa_append_kv
        self.args = [0, 0, self.H_kv * self.D, k_cache.data_ptr(), v_cache.data_ptr(),
                     k_cache.shape[0], block_tables.data_ptr(), block_tables.stride(0),
                     block_tables.shape[1], context_lens.data_ptr(), pages_allocated.data_ptr(),
                     0, 0, 0, self.H_kv, self.D, block_size, _stream(dev)]
        self.dev = dev
        self.stream = self.args[-1]
        self.refs = (k_cache, v_cache, block_tables, context_lens, pages_allocated)

    def matches(self, k_cache, v_cache, block_tables, context_lens, pages_allocated) -> bool:
        r = self.refs
        return (r[0] is k_cache and r[1] is v_cache and r[2] is block_tables
                and r[3] is context_lens and r[4] is pages_allocated
                and torch._C._cuda_getCurrentRawStream(self.dev.index) == self.stream)

    def run(self, k_new, v_new, seq_begin: int, next_free_block: int) -> None:
        n = k_new.shape[0]
        shape = (n, self.H_kv, self.D)
        if (k_new.dtype != torch.bfloat16 or v_new.dtype != torch.bfloat16
                or k_new.shape != shape or v_new.shape != shape
                or not (k_new.is_contiguous() and v_new.is_contiguous())
                or k_new.device != self.dev or v_new.device != self.dev
                or not (0 <= seq_begin and seq_begin + n <= self.batch)):
            raise ValueError(f"append_kv: k / v must be contiguous bfloat16 {shape} on "
                             f"{self.dev} for sequences inside the batch of {self.batch}")
        args = self.args
        args[0] = k_new.data_ptr()
        args[1] = v_new.data_ptr()
        args[11] = seq_begin
        args[12] = n
        args[13] = next_free_block
        check(self.fn(*args), "append_kv")
