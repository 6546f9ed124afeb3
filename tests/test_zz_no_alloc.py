"""cvsa_sparse_decode_noalloc (static device scratch, no workspace argument)
against cvsa_sparse_decode with a caller-owned workspace, through the C ABI.

The two entry points run the same kernels with the same launch plan, so their
outputs must agree bit for bit: a normalised bf16 output and the
un-normalised (o, m, l) state.  Two calls in a row, the second on a smaller
input (fewer splits and heads), so the second call runs on scratch that
still holds the first call's partial rows and counters.
"""

import pytest
import torch

from cvsa import ops
from cvsa.ops import _lib
from cvsa.synthetic import make_paged_inputs

pytestmark = pytest.mark.gpu


def _args(inp, idx, nph, dev):
    q, K, V, bt, cl = inp.q, inp.k_cache, inp.v_cache, inp.block_tables, inp.context_lens
    B, H_q, D = q.shape
    H = inp.num_kv_heads
    pi = idx.reshape(B * H, -1).contiguous()
    nh = nph.reshape(B * H).contiguous()
    head = [q.data_ptr(), q.stride(0), q.stride(1), K.data_ptr(), V.data_ptr(), K.shape[0],
            bt.data_ptr(), bt.stride(0), cl.data_ptr(), pi.data_ptr(), pi.stride(0),
            nh.data_ptr(), pi.shape[1], B, H_q, H, D, 16, bt.shape[1]]
    return head, (pi, nh)


def _outputs(B, H_q, dev):
    return (torch.empty(B, H_q, 128, device=dev, dtype=torch.float32),
            torch.empty(B, H_q, device=dev, dtype=torch.float32),
            torch.empty(B, H_q, device=dev, dtype=torch.float32),
            torch.empty(B, H_q, 128, device=dev, dtype=torch.bfloat16))


def _call_pair(lib, inp, budget, dev):
    """Both entry points on one input; returns (with workspace, no-alloc)."""
    q, K, bt, cl = inp.q, inp.k_cache, inp.block_tables, inp.context_lens
    B, H_q, D = q.shape
    H = inp.num_kv_heads
    ps = ops.score_pages(q, K, bt, cl, H, H_q // H, 16)
    idx, nph = ops.select_topk(ps, budget, cl, 16)
    head, keep = _args(inp, idx, nph, dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    need = lib.cvsa_decode_workspace_bytes(B, H_q, H, D, head[12], bt.shape[1], 0)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    _lib.check(lib.cvsa_workspace_init(ws.data_ptr(), ws.numel(), stream), "workspace_init")
    results = []
    for noalloc in (False, True):
        o, m, l, out = _outputs(B, H_q, dev)
        tail = [o.data_ptr(), m.data_ptr(), l.data_ptr(), out.data_ptr(), _lib.DTYPE_BF16, None]
        if noalloc:
            rc = lib.cvsa_sparse_decode_noalloc(*head, *tail, stream)
        else:
            rc = lib.cvsa_sparse_decode(*head, *tail, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "noalloc test decode")
        results.append((o, m, l, out))
    torch.cuda.synchronize(dev)
    del keep
    return results, need


def test_noalloc_matches_workspace_entry_point(gpu):
    lib = _lib.load()
    # First call: long context, one sequence -> 32 splits per KV head.
    big = make_paged_inputs(1, 32, 8, 128, 65536, seed=910, device=gpu, hot_heads=[2, 7],
                            n_hot=16, hot_shift=8.0)
    (ref_big, got_big), need_big = _call_pair(lib, big, 512, gpu)
    assert need_big > 0
    # Second call: smaller input (fewer heads in total, fewer splits each).
    small = make_paged_inputs(2, 28, 4, 128, [3000, 1777], seed=911, device=gpu,
                              n_hot_range=(0, 8), hot_shift=8.0)
    (ref_small, got_small), need_small = _call_pair(lib, small, 48, gpu)
    assert 0 < need_small < need_big
    for want, got in ((ref_big, got_big), (ref_small, got_small)):
        for a, b in zip(want, got):
            assert torch.equal(a, b)


def test_noalloc_rejects_bad_arguments_before_launch(gpu):
    lib = _lib.load()
    inp = make_paged_inputs(1, 32, 8, 128, 256, seed=912, device=gpu)
    idx = torch.zeros(1, 8, 4, dtype=torch.int32, device=gpu)
    nph = torch.full((1, 8), 4, dtype=torch.int32, device=gpu)
    head, keep = _args(inp, idx, nph, gpu)
    head[14] = 30                                       # H_q not a multiple of H_kv
    o, m, l, out = _outputs(1, 32, gpu)
    rc = lib.cvsa_sparse_decode_noalloc(*head, o.data_ptr(), m.data_ptr(), l.data_ptr(),
                                        out.data_ptr(), _lib.DTYPE_BF16, None,
                                        torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == _lib.CVSA_ERR_INVALID
    assert b"sparse_decode_noalloc" in lib.cvsa_last_error()
    rc = lib.cvsa_sparse_decode_noalloc(*head[:9], None, *head[10:], o.data_ptr(), m.data_ptr(),
                                        l.data_ptr(), out.data_ptr(), _lib.DTYPE_BF16, None, None)
    assert rc == _lib.CVSA_ERR_INVALID
    del keep
