"""Host-side argument checks of the folded append entry points run before
anything reaches the C ABI (no GPU needed): StepPlan.run_reuse_append and
ops.sparse_decode_append refuse a bad k_new / v_new, pages_allocated or slot
argument with ValueError, and a good call reaches the native call with the
prepared arguments."""
import ctypes

import pytest
import torch

from cvsa import ops

B, H_KV, G, D = 3, 2, 4, 128


def _plan(calls):
    """A StepPlan shell on the CPU whose native append call only records."""
    p = object.__new__(ops.StepPlan)
    q = torch.zeros(B, H_KV * G, D, dtype=torch.bfloat16)
    p.dev = q.device
    p.stream = 0
    p.q_meta = (q.shape, q.stride())
    p.out_shape = (B, H_KV * G, D)
    p.out_dtype = q.dtype
    p.h_kv = H_KV
    p._h = 1
    p._pa_ok = p._slots_ok = None
    p._run_append = lambda *a: calls.append(a) or 0
    return p, q


def _good():
    rows = dict(k_new=torch.zeros(B, H_KV, D, dtype=torch.bfloat16),
                v_new=torch.zeros(B, H_KV, D, dtype=torch.bfloat16),
                pages_allocated=torch.zeros(B, dtype=torch.int32))
    return rows


def test_run_reuse_append_accepts_good_arguments():
    calls = []
    p, q = _plan(calls)
    out = p.run_reuse_append(q, slots=[0, -1] * B, **_good())
    assert out.shape == (B, H_KV * G, D) and len(calls) == 1
    slot_arr = calls[0][7]
    assert isinstance(slot_arr, ctypes.Array) and list(slot_arr) == [0, -1] * B
    p.run_reuse_append(q, slots_dev=torch.zeros(B, 2, dtype=torch.int32), **_good())
    assert len(calls) == 2 and calls[1][7] is None


BAD = [
    ("k_new", lambda g: g["k_new"].float()),                                  # dtype
    ("v_new", lambda g: torch.zeros(B, H_KV, D + 1, dtype=torch.bfloat16)),   # shape
    ("k_new", lambda g: torch.zeros(B, D, H_KV, dtype=torch.bfloat16).transpose(1, 2)),
    ("v_new", lambda g: torch.zeros(B, H_KV, 2 * D, dtype=torch.bfloat16)[..., ::2]),
    ("v_new", lambda g: [0] * D),                                             # not a tensor
    ("pages_allocated", lambda g: torch.zeros(B, dtype=torch.int64)),
    ("pages_allocated", lambda g: torch.zeros(B + 1, dtype=torch.int32)),
    ("pages_allocated", lambda g: torch.zeros(2 * B, dtype=torch.int32)[::2]),
]


@pytest.mark.parametrize("name,make", BAD)
def test_run_reuse_append_refuses_bad_rows(name, make):
    calls = []
    p, q = _plan(calls)
    args = _good()
    args[name] = make(args)
    with pytest.raises(ValueError):
        p.run_reuse_append(q, slots=[0, -1] * B, **args)
    assert not calls


@pytest.mark.parametrize("slots,slots_dev", [
    ([0, -1] * (B - 1), None),                                        # too few host slots
    ((ctypes.c_int32 * (2 * B - 2))(), None),                         # short ctypes array
    (None, None),                                                     # neither given
    ([0, -1] * B, torch.zeros(B, 2, dtype=torch.int32)),              # both given
    (None, torch.zeros(B, 2, dtype=torch.int64)),
    (None, torch.zeros(B, 3, dtype=torch.int32)),
    (None, torch.zeros(2, B, dtype=torch.int32).T),
])
def test_run_reuse_append_refuses_bad_slots(slots, slots_dev):
    calls = []
    p, q = _plan(calls)
    with pytest.raises(ValueError):
        p.run_reuse_append(q, slots=slots, slots_dev=slots_dev, **_good())
    assert not calls


def test_run_reuse_append_converts_other_ctypes_arrays():
    """A ctypes array of another element type is copied into int32 entries,
    never handed to the library as is."""
    calls = []
    p, q = _plan(calls)
    arr = (ctypes.c_int64 * (2 * B))(*([5, -1] * B))
    p.run_reuse_append(q, slots=arr, **_good())
    got = calls[0][7]
    assert got._type_ is ctypes.c_int32 and list(got) == [5, -1] * B


def test_run_reuse_append_refuses_a_different_query_layout():
    calls = []
    p, _ = _plan(calls)
    for q in (torch.zeros(B, H_KV * G, D, dtype=torch.float16),
              torch.zeros(B, D, H_KV * G, dtype=torch.bfloat16).transpose(1, 2),
              torch.zeros(B + 1, H_KV * G, D, dtype=torch.bfloat16)):
        with pytest.raises(ValueError):
            p.run_reuse_append(q, slots=[0, -1] * B, **_good())
    assert not calls


def test_checked_append_buffers_are_rechecked_when_they_change():
    calls = []
    p, q = _plan(calls)
    p.run_reuse_append(q, slots=[0, -1] * B, **_good())
    args = _good()
    args["pages_allocated"] = torch.zeros(B, dtype=torch.int64)
    with pytest.raises(ValueError):
        p.run_reuse_append(q, slots=[0, -1] * B, **args)
    assert len(calls) == 1


@pytest.mark.parametrize("errors", [torch.zeros(1, dtype=torch.int64), [0],
                                    torch.zeros(0, dtype=torch.int32)])
def test_run_reuse_append_refuses_bad_slot_errors(errors):
    """The refused-slot counter of a device-slot append must be an int32
    tensor on the plan's device."""
    calls = []
    p, q = _plan(calls)
    with pytest.raises(ValueError):
        p.run_reuse_append(q, slots_dev=torch.zeros(B, 2, dtype=torch.int32),
                           slot_errors=errors, **_good())
    assert not calls
    out = p.run_reuse_append(q, slots_dev=torch.zeros(B, 2, dtype=torch.int32),
                             slot_errors=torch.zeros(1, dtype=torch.int32), **_good())
    assert out.shape == (B, H_KV * G, D) and len(calls) == 1 and calls[0][9] is not None


# ---------------------------------------------------------------- batch shapes
#
# Every op's kernel indexes block_tables, context_lens, selections and masks
# by sequence and (sequence, KV head); a tensor shorter than the call's batch
# would be read or written past its end on the device.  Each op refuses such
# a call with ValueError before anything native runs: the fixture below
# lets the ops see CPU tensors and turns any native call into a failure.

NB, BS = 8, 16


@pytest.fixture
def host_only(monkeypatch):
    def no_native(*a, **k):
        raise AssertionError("reached the native library")
    monkeypatch.setattr(ops, "_device_of", lambda *t: torch.device("cpu"))
    monkeypatch.setattr(ops._lib, "load", no_native)
    monkeypatch.setattr(ops, "_stream", lambda dev: 0)
    monkeypatch.setattr(ops, "_workspace", lambda dev, n: None)


def _inp(b=B, w=6):
    q = torch.zeros(b, H_KV * G, D, dtype=torch.bfloat16)
    kc = torch.zeros(NB, BS, H_KV, D, dtype=torch.bfloat16)
    bt = torch.zeros(b, w, dtype=torch.int32)
    ctx = torch.full((b,), 40, dtype=torch.int32)
    sel = torch.zeros(b, H_KV, 3, dtype=torch.int32)
    nph = torch.full((b, H_KV), 3, dtype=torch.int32)
    acc = torch.ones(b, H_KV, dtype=torch.bool)
    ps = torch.zeros(b, H_KV, w, dtype=torch.float32)
    return q, kc, bt, ctx, sel, nph, acc, ps


def _short(t):
    return t[:-1]


BATCH_CASES = {
    "score_pages/block_tables": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.score_pages(
        q, kc, _short(bt), ctx, H_KV, G, BS),
    "score_pages/context_lens": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.score_pages(
        q, kc, bt, _short(ctx), H_KV, G, BS),
    "select_topk/context_lens": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.select_topk(
        ps, 3, _short(ctx), BS),
    "select_or_keep/context_lens": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.select_or_keep(
        ps, acc, 3, _short(ctx), BS, 0.9, sel, nph, torch.zeros(B, H_KV)),
    "select_budgeted/context_lens": lambda q, kc, bt, ctx, sel, nph, acc, ps:
        ops.select_budgeted(ps, _short(ctx), BS, top_p=0.5),
    "sparse_decode/page_indices": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.sparse_decode(
        q, kc, kc, bt, _short(sel), _short(nph), ctx, H_KV, G, BS),
    "dense_decode/context_lens": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.dense_decode(
        q, kc, kc, bt, _short(ctx), H_KV, G, BS),
    "verified_decode/accept_mask": lambda q, kc, bt, ctx, sel, nph, acc, ps:
        ops.verified_decode(q, kc, kc, bt, ctx, sel, nph, _short(acc), H_KV, G, BS),
    "verified_decode/block_tables": lambda q, kc, bt, ctx, sel, nph, acc, ps:
        ops.verified_decode(q, kc, kc, _short(bt), ctx, sel, nph, acc, H_KV, G, BS),
    "verified_decode_approx/exp_indices": lambda q, kc, bt, ctx, sel, nph, acc, ps:
        ops.prepare_decode("verified_decode_approx", q, kc, kc, bt, ctx, H_KV, G, BS,
                           sel.reshape(B * H_KV, 3), nph.reshape(-1), 3,
                           accept=acc.view(torch.uint8).reshape(-1),
                           exp_flat=torch.zeros(B * H_KV - 1, 4, dtype=torch.int32),
                           exp_budget=4),
    "sparse_decode_reuse/n_per_head": lambda q, kc, bt, ctx, sel, nph, acc, ps:
        ops.sparse_decode_reuse(q, kc, kc, bt, ctx, sel.reshape(B * H_KV, 3),
                                nph.reshape(-1)[:-1], 4, H_KV, G, BS),
    "compute_complement/context_lens": lambda q, kc, bt, ctx, sel, nph, acc, ps:
        ops.compute_complement(sel, nph, _short(ctx), BS, acc, width=6),
    "lse_merge/m_comp": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.lse_merge(
        torch.zeros(B, H_KV * G, D), torch.zeros(B, H_KV * G), torch.ones(B, H_KV * G),
        torch.zeros(B, H_KV * G, D), torch.zeros(B - 1, H_KV * G), torch.ones(B, H_KV * G),
        acc, H_KV, G),
    "append_kv/batch": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.append_kv(
        torch.zeros(2, H_KV, D, dtype=torch.bfloat16), torch.zeros(2, H_KV, D, dtype=torch.bfloat16),
        kc, kc, bt, ctx, torch.zeros(B, dtype=torch.int32), B - 1, NB, BS),
    "step_plan/block_tables": lambda q, kc, bt, ctx, sel, nph, acc, ps: ops.StepPlan(
        q, kc, kc, _short(bt), ctx, H_KV, G, BS, 3, 0.9),
}


@pytest.mark.parametrize("case", sorted(BATCH_CASES))
def test_ops_refuse_inputs_shorter_than_the_batch(host_only, case):
    """The refusal names the short argument (and not some other check)."""
    arg = case.split("/")[1]
    with pytest.raises(ValueError, match=arg):
        BATCH_CASES[case](*_inp())
