"""Paged KV cache: a bf16 block pool plus per-sequence page tables.

Same classes, signatures, layout and allocation order as the reference's
cvsa/runtime/kv_cache.py (CacheConfig :14-21, PagedKVCache :24-84,
SequenceKVManager :87-150): the pool is ``[num_blocks, block_size, H_kv, D]``,
a bump allocator hands out consecutive block ids, ``block_tables`` is
``[B, max_pages]`` int32 and ``context_lens`` is ``[B]`` int32.

MI355X differences: the manager keeps a host mirror of every context length
and allocated-page count, so appending a decode token needs no device->host
read; ``append_token_kv`` / ``append_tokens_kv`` launch the HIP append kernel
(one launch for a whole batch) instead of per-sequence ``.item()`` calls.
Block tables accept any block ids, so randomly permuted physical pages work.
If ``block_tables`` / ``context_lens`` are edited directly, call
``sync_host_state()`` before the next append.
"""
from __future__ import annotations

import ctypes

from dataclasses import dataclass

import torch

from .. import ops


@dataclass
class CacheConfig:
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    device: torch.device


class PagedKVCache:
    """Block pool with a bump allocator (kv_cache.py:24-84)."""

    def __init__(self, num_blocks: int, block_size: int, num_kv_heads: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, device: str = "cuda"):
        self.config = CacheConfig(num_blocks=num_blocks, block_size=block_size,
                                  num_kv_heads=num_kv_heads, head_dim=head_dim, dtype=dtype,
                                  device=torch.device(device))
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.k_cache = torch.zeros(num_blocks, block_size, num_kv_heads, head_dim, dtype=dtype,
                                   device=device)
        self.v_cache = torch.zeros(num_blocks, block_size, num_kv_heads, head_dim, dtype=dtype,
                                   device=device)
        self._next_free = 0
        self._total_blocks = num_blocks

    def allocate_blocks(self, n: int) -> torch.Tensor:
        """n consecutive block ids as int32 (kv_cache.py:53-62)."""
        assert self._next_free + n <= self._total_blocks, \
            f"Out of blocks: need {n}, have {self._total_blocks - self._next_free}"
        ids = torch.arange(self._next_free, self._next_free + n, dtype=torch.int32,
                           device=self.config.device)
        self._next_free += n
        return ids

    def _reserve(self, n: int) -> int:
        """Advance the bump allocator by n without building an id tensor;
        returns the first id (the ids are first .. first + n - 1)."""
        assert self._next_free + n <= self._total_blocks, \
            f"Out of blocks: need {n}, have {self._total_blocks - self._next_free}"
        first = self._next_free
        self._next_free += n
        return first

    def write_kv(self, block_id: int, token_offset: int, k: torch.Tensor, v: torch.Tensor):
        """One token's [H_kv, D] K/V rows (kv_cache.py:64-70)."""
        self.k_cache[block_id, token_offset] = k
        self.v_cache[block_id, token_offset] = v

    def write_kv_block(self, block_id: int, k_block: torch.Tensor, v_block: torch.Tensor,
                       n_tokens: int):
        """The first n_tokens rows of a block (kv_cache.py:72-80)."""
        self.k_cache[block_id, :n_tokens] = k_block[:n_tokens]
        self.v_cache[block_id, :n_tokens] = v_block[:n_tokens]

    def reset(self):
        """Free all blocks without zeroing (kv_cache.py:82-84)."""
        self._next_free = 0


class SequenceKVManager:
    """Page tables and context lengths of a batch (kv_cache.py:87-150)."""

    def __init__(self, cache: PagedKVCache, batch_size: int, max_context_len: int):
        self.cache = cache
        self.batch_size = batch_size
        self.block_size = cache.block_size
        self.max_pages = (max_context_len + cache.block_size - 1) // cache.block_size
        dev = cache.config.device
        self.block_tables = torch.zeros(batch_size, self.max_pages, dtype=torch.int32, device=dev)
        self.context_lens = torch.zeros(batch_size, dtype=torch.int32, device=dev)
        self._pages_allocated = [0] * batch_size
        # Device copy of _pages_allocated read by the append kernel, and the
        # host mirror of context_lens.
        self._pages_allocated_dev = torch.zeros(batch_size, dtype=torch.int32, device=dev)
        self._ctx_host = [0] * batch_size
        self._append_call = None
        self._fuse_shape = None   # (row shape, cache, device) of fusable_rows

    def adopt(self, block_tables: torch.Tensor, context_lens: torch.Tensor,
              next_free_block: int) -> None:
        """Take over a prepared layout: page tables [B, <= max_pages] and
        context lengths [B] whose pages are already written to the cache,
        with blocks [0, next_free_block) in use."""
        B, W = block_tables.shape
        if B != self.batch_size or W > self.max_pages:
            raise ValueError(f"block tables {tuple(block_tables.shape)} do not fit "
                             f"[{self.batch_size}, {self.max_pages}]")
        self.block_tables.zero_()
        self.block_tables[:, :W].copy_(block_tables)
        self.context_lens.copy_(context_lens)
        bs = self.block_size
        self._pages_allocated = [-(-int(c) // bs) for c in context_lens.tolist()]
        self.cache._next_free = int(next_free_block)
        self.sync_host_state()

    def sync_host_state(self):
        """Re-read context lengths and allocation counts from the device."""
        self._ctx_host = [int(x) for x in self.context_lens.tolist()]
        self._pages_allocated_dev.copy_(torch.tensor(self._pages_allocated, dtype=torch.int32))

    def prefill_kv(self, seq_idx: int, k_all: torch.Tensor, v_all: torch.Tensor):
        """Store a prompt's [seq_len, H_kv, D] K/V (kv_cache.py:110-131)."""
        seq_len = k_all.shape[0]
        bs = self.block_size
        n_pages = (seq_len + bs - 1) // bs
        block_ids = self.cache.allocate_blocks(n_pages)
        self.block_tables[seq_idx, :n_pages] = block_ids
        full = seq_len // bs
        if full:
            ids = block_ids[:full].long()
            self.cache.k_cache[ids] = k_all[:full * bs].reshape(full, bs, *k_all.shape[1:]).to(
                self.cache.k_cache.dtype)
            self.cache.v_cache[ids] = v_all[:full * bs].reshape(full, bs, *v_all.shape[1:]).to(
                self.cache.v_cache.dtype)
        rem = seq_len - full * bs
        if rem:
            last = self.cache._next_free - 1  # id of the last block just allocated
            self.cache.write_kv_block(last, k_all[full * bs:], v_all[full * bs:], rem)
        self.context_lens[seq_idx] = seq_len
        self._pages_allocated[seq_idx] = n_pages
        self._pages_allocated_dev[seq_idx] = n_pages
        self._ctx_host[seq_idx] = seq_len

    def _plan_append(self, seqs) -> int:
        """Blocks the append of one token to each of `seqs` allocates."""
        bs = self.block_size
        need = 0
        for s in seqs:
            ctx = self._ctx_host[s]
            page = ctx // bs
            if page >= self.max_pages:
                raise IndexError(
                    f"sequence {s}: context {ctx} + 1 exceeds the block table ({self.max_pages} pages)")
            if ctx % bs == 0 and page >= self._pages_allocated[s]:
                need += 1
        return need

    def _commit_append(self, seqs) -> None:
        bs = self.block_size
        for s in seqs:
            ctx = self._ctx_host[s]
            if ctx % bs == 0 and ctx // bs >= self._pages_allocated[s]:
                self._pages_allocated[s] += 1
            self._ctx_host[s] = ctx + 1

    def append_token_kv(self, seq_idx: int, k: torch.Tensor, v: torch.Tensor):
        """Append one decode token's [H_kv, D] K/V (kv_cache.py:133-150)."""
        self._append(seq_idx, k.reshape(1, *k.shape[-2:]), v.reshape(1, *v.shape[-2:]))

    def append_tokens_kv(self, k: torch.Tensor, v: torch.Tensor):
        """Append one token to every sequence: k, v are [B, H_kv, D]; one launch."""
        if k.shape[0] != self.batch_size:
            raise ValueError(f"expected {self.batch_size} rows, got {k.shape[0]}")
        self._append(0, k, v)

    def fusable_rows(self, k: torch.Tensor, v: torch.Tensor) -> bool:
        """Whether [B, H_kv, D] rows k / v can be appended by a decode launch
        (cvsa_sparse_decode_append): contiguous bf16 on the cache's device,
        one row per sequence."""
        c = self.cache.k_cache
        want = self._fuse_shape
        if want is None or want[1] is not c:
            want = self._fuse_shape = (torch.Size((self.batch_size, c.shape[2], c.shape[3])),
                                       c, c.device)
        return (k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16
                and k.shape == want[0] and v.shape == want[0] and k.device == want[2]
                and v.device == want[2] and k.is_contiguous() and v.is_contiguous()
                and k.data_ptr() % 16 == 0 and v.data_ptr() % 16 == 0)

    def fused_append_slots(self):
        """The slots of one token appended to every sequence by a decode
        launch: a ctypes int32 array of (context length before the append,
        block the append allocates or -1) per sequence, the allocation rule
        of append_token_kv (kv_cache.py:133-150) applied to the host mirror.
        Returns (slots, commit); call commit() once the launch is enqueued
        (it reserves the blocks and advances the mirror)."""
        slots = (ctypes.c_int32 * (2 * self.batch_size))()
        need = self.fill_fused_slots(slots)

        def commit():
            self.commit_fused(need)

        return slots, commit

    def fill_fused_slots(self, slots) -> int:
        """fused_append_slots into an existing ctypes int32 array of 2 * B
        entries; returns the number of blocks the append allocates, to be
        reserved with commit_fused(n) once the launch is enqueued."""
        bs = self.block_size
        first = self.cache._next_free
        pages = self._pages_allocated
        ctxs = self._ctx_host
        r = 0
        for s in range(self.batch_size):
            ctx = ctxs[s]
            page = ctx // bs
            if page >= self.max_pages:
                raise IndexError(f"sequence {s}: context {ctx} + 1 exceeds the block table "
                                 f"({self.max_pages} pages)")
            slots[2 * s] = ctx
            if ctx % bs == 0 and page >= pages[s]:
                slots[2 * s + 1] = first + r
                r += 1
            else:
                slots[2 * s + 1] = -1
        if first + r > self.cache._total_blocks:
            raise AssertionError(f"Out of blocks: need {r}, have "
                                 f"{self.cache._total_blocks - first}")
        return r

    def commit_fused(self, need: int) -> None:
        """Reserve the blocks of a fused append and advance the host mirror."""
        self.cache._reserve(need)
        self._commit_append(range(self.batch_size))

    def _append(self, seq_begin: int, k: torch.Tensor, v: torch.Tensor):
        n = k.shape[0]
        seqs = range(seq_begin, seq_begin + n)
        need = self._plan_append(seqs)
        buffers = (self.cache.k_cache, self.cache.v_cache, self.block_tables, self.context_lens,
                   self._pages_allocated_dev)
        if (k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16 and k.is_contiguous()
                and v.is_contiguous() and k.device == buffers[0].device):
            # The launch over this manager's buffers is validated once.
            call = self._append_call
            if call is None or not call.matches(*buffers):
                call = self._append_call = ops.AppendCall(*buffers, self.block_size)
            call.run(k, v, seq_begin, self.cache._reserve(need))
        else:
            ops.append_kv(k, v, *buffers, seq_begin, self.cache._reserve(need),
                          self.block_size)
        self._commit_append(seqs)
