"""Per-op CPU restatement of the CVSA decode path -- TEST INFRASTRUCTURE ONLY.

Reference: DJ-Melvin/coverage-verified-sparse-attention.  Each function cites
the reference lines it restates.  Accumulation runs in ``acc_dtype``
(float64 by default, so the oracle is the exact value the fp32 GPU kernels
approximate; float32 for the timed CPU baseline).  Results are returned in
the reference's output dtypes.

Contract points where the HIP path is held to a fixed answer for a case the
reference leaves undefined or implementation-specific (all documented in the
C header):
  * top-k: the set of the ``budget`` largest scores, ties to the lower page
    index, listed in ascending page order (torch.topk(sorted=False) leaves
    the order unspecified, cvsa/backend.py:737-738);
  * empty page list: (o, m, l) = (0, -inf, 0) and a zero normalised output
    (the reference produces NaN, cvsa/kernels/sparse_decode.py:107,263);
  * listed pages outside [0, W) or mapping to a block outside the pool, and
    pages without a valid token, contribute nothing;
  * top-p, static-table and adaptive selections: ties to the lower page (and,
    for the adaptive head competition, to the lower head), where torch's
    sort / topk leave them open (cvsa/backend.py:537-541, :567, :647, :672).

How each function is pinned (tests/test_oracle_*.py unless noted):
  * prepare_reuse_state, sparse_decode_reuse: closed form (padding with page
    0 to a power of two) and invariance (a padded state decodes exactly as
    the unpadded selection), test_oracle_closed_form;
  * score_pages, check_coverage, select_topk, sparse_decode(_unnorm),
    dense_decode, compute_complement, lse_merge, append_token_kv: the
    reference backend's golden traces (tests/golden/), the reference tests'
    known answers, closed forms and brute force (test_oracle_known_answers,
    test_oracle_closed_form, test_golden_backend_trace);
  * page_key_minmax, quest_page_scores: the Quest bound's mathematics
    (upper bound of the exact page max, equality on one-token pages, brute
    force, masked slots, q . kmax for a non-negative query), test_oracle_quest;
  * topp_need, topp_select, static_budgets, static_select, adaptive_budgets,
    adaptive_select: closed forms (uniform and geometric masses, the strict
    boundary, clamps, half-even rounding, floor ratios 0 and 1, a dominating
    head) and scalar brute force, test_oracle_selectors.
Parity unpinned: the tie order at top-p / adaptive boundaries (implementation
defined in the reference) and the dense baseline's FlashInfer arithmetic.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

NEG_FLOOR = -1e20   # coverage.py:180, :205 (running-max floor / masked lanes)
LOG_EPS = 1e-30     # coverage.py:195, :208
NORM_EPS = 1e-6     # sparse_decode.py:127,271; coverage.py:305,321; lse_merge.py:36,48


def next_power_of_2(n: int) -> int:
    """cvsa/kernels/sparse_decode.py:279-283."""
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def fp32_scale(head_dim: int) -> float:
    """D ** -0.5 as the fp32 constant the kernels multiply by
    (cvsa/kernels/page_scores.py:106, sparse_decode.py:334)."""
    return float(torch.tensor(head_dim ** -0.5, dtype=torch.float32))


def n_valid_pages(context_lens: torch.Tensor, block_size: int) -> torch.Tensor:
    """((ctx.float() - 1) / bs).long() + 1  (cvsa/backend.py:687,
    cvsa/complement.py:31, cvsa/runtime/dense.py:47).  .long() truncates
    toward zero, so ctx = 0 gives one page."""
    return ((context_lens.to(torch.float32) - 1) / block_size).to(torch.int64) + 1


# ------------------------------------------------------------------ scoring

def group_mean_bf16(q: torch.Tensor, num_kv_heads: int, num_q_per_kv: int) -> torch.Tensor:
    """q.view(B, H_kv, G, D).mean(dim=2) on bf16 input
    (cvsa/kernels/page_scores.py:94-95): the fp32 sum over the group times
    fp32(1/G), rounded to bf16 -- the reduction torch applies on the GPU."""
    B, H_q, D = q.shape
    qg = q.to(torch.float32).reshape(B, num_kv_heads, num_q_per_kv, D)
    acc = qg[:, :, 0].clone()
    for g in range(1, num_q_per_kv):
        acc = acc + qg[:, :, g]
    inv = torch.tensor(1.0 / num_q_per_kv, dtype=torch.float32)
    return (acc * inv).to(torch.bfloat16)


def score_pages(q, k_cache, block_tables, context_lens, num_kv_heads, num_q_per_kv,
                block_size, acc_dtype=torch.float64, page_chunk: int = 2048) -> torch.Tensor:
    """triton_score_pages (cvsa/kernels/page_scores.py:77-119, kernel :12-74).

    page_scores[b,h,p] = max_{t < tokens(p)} (q_rep[b,h] . K[bt[b,p], t, h]) * scale,
    -inf for pages whose first position is >= ctx (:43-47) and for masked
    tokens (:68); output pre-filled with -inf (:97-100).
    """
    B, H_q, D = q.shape
    W = block_tables.shape[1]
    scale = fp32_scale(D)
    q_rep = group_mean_bf16(q, num_kv_heads, num_q_per_kv).to(acc_dtype)
    out = torch.full((B, num_kv_heads, W), float("-inf"), dtype=torch.float32)
    nb = k_cache.shape[0]
    for b in range(B):
        ctx = int(context_lens[b])
        n = max(0, min(W, -(-ctx // block_size)))
        for p0 in range(0, n, page_chunk):
            p1 = min(n, p0 + page_chunk)
            phys = block_tables[b, p0:p1].long()
            ok = (phys >= 0) & (phys < nb)
            K = k_cache[phys.clamp(0, nb - 1)].to(acc_dtype)          # [n, bs, H, D]
            dots = torch.einsum("pthd,hd->hpt", K, q_rep[b])          # [H, n, bs]
            s = dots.to(torch.float32) * scale
            pos = torch.arange(p0, p1).unsqueeze(1) * block_size + torch.arange(block_size)
            valid = (pos < ctx) & ok.unsqueeze(1)
            s = s.masked_fill(~valid.unsqueeze(0), float("-inf"))
            out[b, :, p0:p1] = s.amax(dim=-1)
    return out


def page_key_minmax(k_cache, block_tables, context_lens, block_size):
    """Per (b, page, kv-head) min and max of the keys over the page's valid
    tokens (positions < ctx), the metadata of CVSABackend._quest_page_scores
    (cvsa/backend.py:593-603) and of the Quest baseline
    (eval/baselines.py:77-117).  Returns (kmin, kmax) [B, W, H_kv, D] fp32,
    +inf / -inf where a page has no valid token."""
    B, W = block_tables.shape
    nb, bs, H, D = k_cache.shape
    kmin = torch.full((B, W, H, D), float("inf"), dtype=torch.float32)
    kmax = torch.full((B, W, H, D), float("-inf"), dtype=torch.float32)
    for b in range(B):
        ctx = int(context_lens[b])
        for p in range(W):
            n = min(block_size, ctx - p * block_size)
            phys = int(block_tables[b, p])
            if n <= 0 or not 0 <= phys < nb:
                continue
            keys = k_cache[phys, :n].to(torch.float32)            # [n, H, D]
            kmin[b, p] = keys.amin(dim=0)
            kmax[b, p] = keys.amax(dim=0)
    return kmin, kmax


def quest_page_scores(q, k_cache, block_tables, context_lens, num_kv_heads, num_q_per_kv,
                      block_size, acc_dtype=torch.float64) -> torch.Tensor:
    """CVSABackend._quest_page_scores (cvsa/backend.py:572-620).

    score[b,h,p] = sum_d max(q_rep_d * kmin_d, q_rep_d * kmax_d) * D^-0.5 over
    the page's valid tokens (the Quest upper bound of the page's max dot
    product), q_rep the bf16 group mean (:606-607), -inf for pages without a
    valid token (:616-618).  Block ids outside the pool give -inf (the
    reference would index its cache with them)."""
    B, H_q, D = q.shape
    W = block_tables.shape[1]
    q_rep = group_mean_bf16(q, num_kv_heads, num_q_per_kv).to(acc_dtype)   # [B, H, D]
    kmin, kmax = page_key_minmax(k_cache, block_tables, context_lens, block_size)
    qb = q_rep.unsqueeze(1)                                                # [B, 1, H, D]
    with torch.no_grad():
        lo = qb * kmin.to(acc_dtype).nan_to_num(posinf=0.0)
        hi = qb * kmax.to(acc_dtype).nan_to_num(neginf=0.0)
        upper = torch.maximum(lo, hi).sum(dim=-1) * fp32_scale(D)          # [B, W, H]
    out = upper.to(torch.float32).transpose(1, 2).contiguous()             # [B, H, W]
    valid = torch.isfinite(kmax[..., 0]).transpose(1, 2)                   # [B, H, W]
    return out.masked_fill(~valid, float("-inf"))


# ---------------------------------------------------------------- selection

def select_topk(page_scores: torch.Tensor, budget: int, context_lens: torch.Tensor,
                block_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Uniform-budget selection of CVSABackend._scoring_step
    (cvsa/backend.py:737-747) with the fixed order contract: the `budget`
    largest scores, ties to the lower page, listed in ascending page order;
    n_per_head = min(budget, n_valid)."""
    B, H, W = page_scores.shape
    order = torch.sort(page_scores, dim=-1, descending=True, stable=True).indices[..., :budget]
    idx = order.sort(dim=-1).values.to(torch.int32)
    nv = n_valid_pages(context_lens, block_size)
    nph = torch.clamp(nv, max=budget).to(torch.int32).unsqueeze(1).expand(B, H).contiguous()
    return idx, nph


def topp_need(sel_scores: torch.Tensor, top_p: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """The top-p budget of CVSABackend._topp_select (cvsa/backend.py:664-678)
    in fp64: p = softmax(row), sorted descending (ties to the lower page),
    need = 1 + #{k : cumsum_k < top_p}, clamped to [3, P].  top_p is compared
    as fp32, as torch compares a float32 tensor with a Python float.  Returns
    (need [B, H] int64, the descending order [B, H, P]).  A row whose
    softmax is NaN (+inf / NaN scores, or no finite one) gets need = 3."""
    B, H, P = sel_scores.shape
    s = sel_scores.to(torch.float64)
    order = torch.sort(s, dim=-1, descending=True, stable=True).indices
    with torch.no_grad():
        probs = torch.softmax(s, dim=-1)
    cum = torch.cumsum(probs.gather(-1, order), dim=-1)
    p32 = float(torch.tensor(top_p, dtype=torch.float32))
    need = (cum < p32).sum(dim=-1) + 1
    return need.clamp(min=3, max=P), order


def topp_select(sel_scores, top_p, context_lens, block_size):
    """CVSABackend._topp_select (cvsa/backend.py:652-681): the pages of each
    row's top-p set (see topp_need) in ascending page order, rows of
    max_budget = max n_per_head entries whose first n_per_head are the
    valid pages of the set; n_per_head = min(need, n_valid)."""
    B, H, P = sel_scores.shape
    need, order = topp_need(sel_scores, top_p)
    nv = n_valid_pages(context_lens, block_size).view(B, 1)
    nph = torch.minimum(need, nv.expand(B, H)).to(torch.int32)
    return _prefix_sets(order, need, nph)


def static_select(sel_scores, fractions, context_lens, block_size):
    """CVSABackend._static_select (cvsa/backend.py:622-650): per-head budgets
    clamp(round(frac * P), 3, P) from an offline table, n_per_head =
    min(budget_h, n_valid); the top budget_h pages of each row in ascending
    page order (ties to the lower page), rows of max budget entries."""
    B, H, P = sel_scores.shape
    per_head = static_budgets(fractions, P)
    order = torch.sort(sel_scores.to(torch.float64), dim=-1, descending=True,
                       stable=True).indices
    k = per_head.view(1, H).expand(B, H)
    nv = n_valid_pages(context_lens, block_size).view(B, 1)
    nph = torch.minimum(k, nv.expand(B, H)).to(torch.int32)
    return _prefix_sets(order, k, nph)


def static_budgets(fractions, P: int) -> torch.Tensor:
    """Per-head page budgets of a static table row (backend.py:638):
    clamp(round(frac * P), 3, P), round half to even as torch.round."""
    f = torch.as_tensor(fractions, dtype=torch.float32)
    return torch.clamp(torch.round(f * P).long(), min=3, max=P)


def adaptive_budgets(sel_scores, base_budget, context_lens, block_size, floor_ratio):
    """The budgets of CVSABackend._adaptive_select (cvsa/backend.py:522-559):
    raw[b,h] = head h's share of the H * base_budget largest scores of
    sequence b, ties at the last value to the lower heads (torch.topk leaves
    them unspecified); budget = round(fp32(raw) * fp32(1 - floor_ratio) +
    fp32(base * floor_ratio)) with round half to even, clamped to
    [1, n_valid]."""
    B, H, P = sel_scores.shape
    K = min(H * base_budget, H * P)
    keep = torch.tensor(1.0 - floor_ratio, dtype=torch.float32)
    cap = torch.tensor(base_budget * floor_ratio, dtype=torch.float32)
    nv = n_valid_pages(context_lens, block_size)
    out = torch.empty(B, H, dtype=torch.int32)
    for b in range(B):
        vals = sel_scores[b].to(torch.float64).reshape(-1)          # head-major
        heads = torch.arange(H).repeat_interleave(P)
        # order by (value desc, head asc): a stable sort of the head-major row
        order = torch.sort(vals, descending=True, stable=True).indices[:K]
        raw = torch.bincount(heads[order], minlength=H).to(torch.float32)
        mixed = raw * keep + cap          # two fp32 roundings, as torch
        fb = torch.round(mixed).to(torch.int32)
        out[b] = torch.clamp(fb, min=1).clamp(max=int(nv[b]))
    return out


def adaptive_select(sel_scores, base_budget, context_lens, block_size, floor_ratio):
    """CVSABackend._adaptive_select (cvsa/backend.py:522-570): the pages of
    each row's top budget[b,h] scores in ascending page order (ties to the
    lower page), rows of max budget entries; n_per_head = budget."""
    budgets = adaptive_budgets(sel_scores, base_budget, context_lens, block_size, floor_ratio)
    order = torch.sort(sel_scores.to(torch.float64), dim=-1, descending=True,
                       stable=True).indices
    return _prefix_sets(order, budgets, budgets)


def _prefix_sets(order, k_row, nph):
    """Rows of the k_row first pages of `order`, sorted ascending, truncated
    to max(nph) entries (the valid ones come first: invalid pages score -inf
    and have the highest indices)."""
    B, H, P = order.shape
    width = max(int(nph.max()), 1)
    out = torch.zeros(B, H, width, dtype=torch.int32)
    for b in range(B):
        for h in range(H):
            sel = torch.sort(order[b, h, :int(k_row[b, h])]).values[:width]
            out[b, h, :sel.numel()] = sel.to(torch.int32)
    return out, nph


def check_coverage(page_scores, selected_indices, n_per_head, tau,
                   acc_dtype=torch.float64) -> Tuple[torch.Tensor, torch.Tensor]:
    """triton_check_coverage (cvsa/kernels/coverage.py:218-265, kernel
    :159-215).

    lse_all: running max floored at -1e20 (:180), log(sum + 1e-30) (:195);
    lse_sel over the first n_sel selected scores, with -1e20 in the max for
    the padding lanes of the power-of-two block (:198-208);
    coverage = exp(lse_sel - lse_all), accept = coverage >= fp32(tau) (:211-212).
    """
    B, H, W = page_scores.shape
    k = selected_indices.shape[2]
    block = next_power_of_2(k)
    s = page_scores.to(acc_dtype)
    m_all = s.amax(dim=-1).clamp(min=NEG_FLOOR)
    lse_all = m_all + torch.log(torch.exp(s - m_all.unsqueeze(-1)).sum(-1) + LOG_EPS)
    sel_idx = selected_indices.long()
    in_range = (sel_idx >= 0) & (sel_idx < W)
    sel = torch.gather(s, 2, sel_idx.clamp(0, W - 1))
    sel = torch.where(in_range, sel, torch.full_like(sel, float("-inf")))
    nsel = n_per_head.long().clamp(0, k)
    mask = torch.arange(k).view(1, 1, k) < nsel.unsqueeze(-1)
    m_sel = torch.where(mask, sel, torch.full_like(sel, float("-inf"))).amax(dim=-1)
    m_sel = torch.where(nsel < block, m_sel.clamp(min=NEG_FLOOR), m_sel)
    e = torch.where(mask, torch.exp(sel - m_sel.unsqueeze(-1)), torch.zeros_like(sel))
    lse_sel = m_sel + torch.log(e.sum(-1) + LOG_EPS)
    cov = torch.exp(lse_sel - lse_all).to(torch.float32)
    accept = cov >= torch.tensor(tau, dtype=torch.float32)
    return accept, cov


# ------------------------------------------------------------------- decode

def _gather_tokens(k_cache, v_cache, block_tables, b, h, pages, ctx, block_size, W):
    """K/V rows of the valid tokens of `pages` for KV head h, in list order
    (masking rule of cvsa/kernels/sparse_decode.py:76-80)."""
    nb = k_cache.shape[0]
    ks, vs = [], []
    for lp in pages:
        lp = int(lp)
        if lp < 0 or lp >= W:
            continue
        phys = int(block_tables[b, lp])
        if phys < 0 or phys >= nb:
            continue
        ntok = min(block_size, ctx - lp * block_size)
        if ntok <= 0:
            continue
        ks.append(k_cache[phys, :ntok, h])
        vs.append(v_cache[phys, :ntok, h])
    if not ks:
        return None, None
    return torch.cat(ks), torch.cat(vs)


def sparse_decode_unnorm(q, k_cache, v_cache, block_tables, page_indices, n_per_head,
                         context_lens, num_kv_heads, num_q_per_kv, block_size,
                         acc_dtype=torch.float64):
    """triton_sparse_decode_unnorm (cvsa/kernels/sparse_decode.py:537-573,
    kernels :423-500, :136-234, :576-606) in closed form:
    s = (q . K) * scale, m = max s, l = sum exp(s - m), o = sum exp(s - m) V
    over the valid tokens of the first n_per_head listed pages.
    Returns (o [B,H_q,D], m [B,H_q], l [B,H_q]) float32."""
    B, H_q, D = q.shape
    G = num_q_per_kv
    W = block_tables.shape[1]
    k = page_indices.shape[2]
    scale = fp32_scale(D)
    o = torch.zeros(B, H_q, D, dtype=torch.float32)
    m = torch.full((B, H_q), float("-inf"), dtype=torch.float32)
    l = torch.zeros(B, H_q, dtype=torch.float32)
    for b in range(B):
        ctx = int(context_lens[b])
        for h in range(num_kv_heads):
            n = max(0, min(int(n_per_head[b, h]), k))
            K, V = _gather_tokens(k_cache, v_cache, block_tables, b, h,
                                  page_indices[b, h, :n].tolist(), ctx, block_size, W)
            if K is None:
                continue
            Q = q[b, h * G:(h + 1) * G].to(acc_dtype)                 # [G, D]
            s = (K.to(acc_dtype) @ Q.T) * scale                       # [T, G]
            mm = s.amax(dim=0)
            p = torch.exp(s - mm)
            o[b, h * G:(h + 1) * G] = (p.T @ V.to(acc_dtype)).to(torch.float32)
            m[b, h * G:(h + 1) * G] = mm.to(torch.float32)
            l[b, h * G:(h + 1) * G] = p.sum(dim=0).to(torch.float32)
    return o, m, l


def normalise(o, l, dtype):
    """o / max(l, 1e-6) cast to dtype (sparse_decode.py:127-131, :271-276)."""
    return (o.to(torch.float64) / l.to(torch.float64).clamp(min=NORM_EPS).unsqueeze(-1)).to(dtype)


def sparse_decode(q, k_cache, v_cache, block_tables, page_indices, n_per_head, context_lens,
                  num_kv_heads, num_q_per_kv, block_size, acc_dtype=torch.float64):
    """triton_sparse_decode / triton_sparse_decode_reuse
    (cvsa/kernels/sparse_decode.py:286-350, :681-721): normalised, q.dtype."""
    o, m, l = sparse_decode_unnorm(q, k_cache, v_cache, block_tables, page_indices,
                                   n_per_head, context_lens, num_kv_heads, num_q_per_kv,
                                   block_size, acc_dtype)
    return normalise(o, l, q.dtype)


def prepare_reuse_state(page_indices, n_per_head, num_kv_heads, B):
    """cvsa/kernels/sparse_decode.py:664-678: the selection padded with page 0
    to the next power of two of its width and flattened to [B * H_kv, padded],
    n_per_head to [B * H_kv]; returns (pi_flat, nph_flat, padded)."""
    k = page_indices.shape[2]
    padded = next_power_of_2(k)
    pi = torch.zeros(B, num_kv_heads, padded, dtype=torch.int32)
    pi[:, :, :k] = page_indices.to(torch.int32)
    return (pi.reshape(B * num_kv_heads, padded), n_per_head.to(torch.int32).reshape(-1),
            padded)


def sparse_decode_reuse(q, k_cache, v_cache, block_tables, context_lens, pi_flat, nph_flat,
                        padded_max_selected, num_kv_heads, num_q_per_kv, block_size,
                        acc_dtype=torch.float64):
    """triton_sparse_decode_reuse (cvsa/kernels/sparse_decode.py:681-721): the
    normalised sparse decode of a prepared state; each row's first
    n_per_head entries are its pages (the padding is never read)."""
    B = q.shape[0]
    idx = pi_flat[:, :padded_max_selected].reshape(B, num_kv_heads, padded_max_selected)
    nph = nph_flat.reshape(B, num_kv_heads)
    return sparse_decode(q, k_cache, v_cache, block_tables, idx, nph, context_lens,
                         num_kv_heads, num_q_per_kv, block_size, acc_dtype)


def all_pages_selection(context_lens, block_tables, num_kv_heads, block_size):
    """The dense fallback's selection: every page, n = n_valid
    (cvsa/runtime/dense.py:44-57)."""
    B, W = block_tables.shape
    idx = torch.arange(W, dtype=torch.int32).view(1, 1, W).expand(B, num_kv_heads, W)
    nv = n_valid_pages(context_lens, block_size).clamp(max=W).to(torch.int32)
    return idx.contiguous(), nv.unsqueeze(1).expand(B, num_kv_heads).contiguous()


def dense_decode(q, k_cache, v_cache, block_tables, context_lens, num_kv_heads, num_q_per_kv,
                 block_size, acc_dtype=torch.float64, return_state=False):
    """DenseAttentionBackend._triton_dense (cvsa/runtime/dense.py:40-68):
    sparse decode with every valid page selected."""
    idx, nph = all_pages_selection(context_lens, block_tables, num_kv_heads, block_size)
    o, m, l = sparse_decode_unnorm(q, k_cache, v_cache, block_tables, idx, nph, context_lens,
                                   num_kv_heads, num_q_per_kv, block_size, acc_dtype)
    out = normalise(o, l, q.dtype)
    return (out, (o, m, l)) if return_state else out


# ----------------------------------------------------------------- recovery

def compute_complement(page_indices, n_per_head, context_lens, block_size, accept_mask,
                       width: Optional[int] = None):
    """triton_compute_complement (cvsa/kernels/coverage.py:99-150, kernel
    :30-96): ascending valid pages not among the first n_sel selected,
    zero-filled to width = max_b n_valid(b); accepted heads -> n = 0."""
    B, H, k = page_indices.shape
    nv = n_valid_pages(context_lens, block_size)
    if width is None:
        width = max(1, int(nv.max()))
    comp = torch.zeros(B, H, width, dtype=torch.int32)
    ncomp = torch.zeros(B, H, dtype=torch.int32)
    for b in range(B):
        nvb = max(0, min(int(nv[b]), width))
        for h in range(H):
            if accept_mask is not None and bool(accept_mask[b, h]):
                continue
            n = max(0, min(int(n_per_head[b, h]), k))
            chosen = set(int(x) for x in page_indices[b, h, :n].tolist())
            rest = [p for p in range(nvb) if p not in chosen]
            comp[b, h, :len(rest)] = torch.tensor(rest, dtype=torch.int32)
            ncomp[b, h] = len(rest)
    return comp, ncomp


def compute_complement_pages(page_indices, n_per_head, context_lens, block_size,
                             accept_mask=None):
    """compute_complement_pages (cvsa/complement.py:11-69): the same sets,
    width = max complement count, or a [B, H, 1] zero dummy when every count
    is 0 (:60-63).  The reference's order comes from an unstable sort
    (:66-67); the oracle lists ascending pages."""
    comp, ncomp = compute_complement(page_indices, n_per_head, context_lens, block_size,
                                     accept_mask)
    mx = int(ncomp.max()) if ncomp.numel() else 0
    if mx == 0:
        return torch.zeros(comp.shape[0], comp.shape[1], 1, dtype=torch.int32), ncomp
    return comp[..., :mx].contiguous(), ncomp


def lse_merge(o_d, m_d, l_d, o_c, m_c, l_c, accept_mask, num_q_per_kv,
              output_dtype=torch.bfloat16, acc_dtype=torch.float64):
    """selective_lse_merge (cvsa/lse_merge.py:11-54) == triton_lse_merge
    (cvsa/kernels/coverage.py:273-326)."""
    acc_q = accept_mask.repeat_interleave(num_q_per_kv, dim=1)
    od, md, ld = o_d.to(acc_dtype), m_d.to(acc_dtype), l_d.to(acc_dtype)
    oc, mc, lc = o_c.to(acc_dtype), m_c.to(acc_dtype), l_c.to(acc_dtype)
    o_acc = od / ld.clamp(min=NORM_EPS).unsqueeze(-1)
    mm = torch.maximum(md, mc)
    sd, sc = torch.exp(md - mm), torch.exp(mc - mm)
    lm = ld * sd + lc * sc
    o_rej = (od * sd.unsqueeze(-1) + oc * sc.unsqueeze(-1)) / lm.clamp(min=NORM_EPS).unsqueeze(-1)
    return torch.where(acc_q.unsqueeze(-1), o_acc, o_rej).to(output_dtype)


def verified_decode(q, k_cache, v_cache, block_tables, context_lens, page_indices,
                    n_per_head, accept_mask, num_kv_heads, num_q_per_kv, block_size,
                    acc_dtype=torch.float64):
    """The exact-recovery branch of CVSABackend._scoring_step as the
    reference computes it (cvsa/backend.py:818-844): draft (o_d, m_d, l_d),
    complement pages, complement attention, LSE merge -> q.dtype."""
    o_d, m_d, l_d = sparse_decode_unnorm(q, k_cache, v_cache, block_tables, page_indices,
                                         n_per_head, context_lens, num_kv_heads,
                                         num_q_per_kv, block_size, acc_dtype)
    comp, ncomp = compute_complement(page_indices, n_per_head, context_lens, block_size,
                                     accept_mask)
    o_c, m_c, l_c = sparse_decode_unnorm(q, k_cache, v_cache, block_tables, comp, ncomp,
                                         context_lens, num_kv_heads, num_q_per_kv, block_size,
                                         acc_dtype)
    return lse_merge(o_d, m_d, l_d, o_c, m_c, l_c, accept_mask, num_q_per_kv, q.dtype, acc_dtype)


# ---------------------------------------------------------------- KV append

def append_token_kv(k_cache, v_cache, block_tables, context_lens, pages_allocated, next_free,
                    seq_idx, k, v, block_size) -> int:
    """SequenceKVManager.append_token_kv (cvsa/runtime/kv_cache.py:133-150)
    with PagedKVCache.allocate_blocks (:53-62): mutates the tensors in place
    and returns the new bump-allocator position."""
    ctx = int(context_lens[seq_idx])
    page = ctx // block_size
    off = ctx % block_size
    if off == 0 and page >= int(pages_allocated[seq_idx]):
        assert next_free + 1 <= k_cache.shape[0], "Out of blocks"
        block_tables[seq_idx, page] = next_free
        next_free += 1
        pages_allocated[seq_idx] += 1
    blk = int(block_tables[seq_idx, page])
    k_cache[blk, off] = k
    v_cache[blk, off] = v
    context_lens[seq_idx] += 1
    return next_free


def softmax_attention(q, keys, values, acc_dtype=torch.float64):
    """Textbook softmax(q K^T / sqrt(D)) V for one query: the closed form the
    page-level kernels reduce to when every page is selected
    (tests/test_lse_merge.py:10-15 of the reference uses the same form)."""
    D = q.shape[-1]
    s = (keys.to(acc_dtype) @ q.to(acc_dtype)) / math.sqrt(D)
    return torch.softmax(s, dim=0) @ values.to(acc_dtype)
