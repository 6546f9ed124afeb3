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
