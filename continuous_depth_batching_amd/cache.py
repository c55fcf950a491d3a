"""Paged KV cache: FIFO block allocation on the host, one pool tensor in HBM.

Host side (bit-compatible with the reference's allocation order):
  * ``BlockManager`` hands out block ids FIFO and appends freed ids at the
    back (continuous_batching/cache_manager.py:33-90);
  * each request owns a block list; position t lives at pool row
    ``blocks[t // block_size] * block_size + t % block_size`` (:190-213).
Device side (MI355X layout):
  * one contiguous pool ``[num_cache_layers, 2, (num_blocks + 2) * block_size, Hkv, D]``
    -- keys and values of every cache layer -- so a row's cache layer is just an
    offset and one kernel launch can serve rows of different loop slots; the two
    trailing blocks are never allocated (the reference's sentinel/trash blocks);
  * a persistent device block table ``[table_rows, width]`` (int32, -1 padded):
    every active request owns one row, and allocations/frees are applied as a
    batch of (row, column, block) updates before the next launch instead of
    re-uploading whole tables.
"""

from __future__ import annotations

from collections import deque

import numpy as np
import torch

from . import _tick, ops
from .kv_cache_policy import LoopedKvLayout


class CacheFullError(RuntimeError):
    """The KV cache cannot place work and no preemption can relieve it."""


class PagedKVCache:
    """Paged KV pool plus block bookkeeping for one engine."""

    EXTRA_BLOCKS = 2

    def __init__(self, *, layout: LoopedKvLayout, num_blocks: int, block_size: int, num_kv_heads: int,
                 head_dim: int, max_model_len: int, max_num_batched_tokens: int, max_requests: int,
                 dtype: torch.dtype, device: torch.device) -> None:
        self.layout = layout
        self.kv_policy = layout.policy
        self.kv_slots_per_layer = layout.slots_per_layer
        self.num_layers = layout.num_cache_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_pages = num_blocks * block_size
        self.num_key_value_heads = num_kv_heads
        self.head_dim = head_dim
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_blocks_per_request = -(-max_model_len // block_size)
        self.dtype = dtype
        self.device = device
        rows = (num_blocks + self.EXTRA_BLOCKS) * block_size
        self.pool = torch.zeros((self.num_layers, 2, rows, num_kv_heads, head_dim), dtype=dtype, device=device)
        self.view = ops.KVPoolView(self.pool, block_size)
        # FIFO block ids, allocated map and peak (cb/cache_manager.py:72-90), in the tick core.
        self._block_manager = _tick.BlockPool(num_blocks, block_size)
        self.block_table: dict[str, list[int]] = {}
        # Device block table: one row per active request.
        self.table_rows = max_requests
        self.table_width = self.max_blocks_per_request
        self.host_table = np.full((self.table_rows, self.table_width), -1, dtype=np.int32)
        self.device_table = torch.full((self.table_rows, self.table_width), -1, dtype=torch.int32, device=device)
        self._free_table_rows: list[int] = list(range(self.table_rows - 1, -1, -1))
        self.table_row_of: dict[str, int] = {}
        # Flat indices of device-table cells whose host value changed since the last flush. A cell
        # may change several times (a freed row reused by a new request); only its final value is
        # uploaded, so one scatter never writes a cell twice.
        self._dirty: set[int] = set()
        cap = max(1024, 4 * max_requests)
        self._stage_index = torch.empty(cap, dtype=torch.int64, pin_memory=device.type == "cuda")
        self._stage_value = torch.empty(cap, dtype=torch.int32, pin_memory=device.type == "cuda")
        self._dev_index = torch.empty(cap, dtype=torch.int64, device=device)
        self._dev_value = torch.empty(cap, dtype=torch.int32, device=device)
        self._stage_event: torch.cuda.Event | None = None

    # -- allocation (host) ---------------------------------------------------------------------------------
    def get_num_free_blocks(self) -> int:
        return self._block_manager.num_free_blocks

    def get_num_allocated_blocks(self) -> int:
        return self._block_manager.num_allocated_blocks

    @property
    def peak_num_allocated_blocks(self) -> int:
        return self._block_manager.peak_num_allocated_blocks

    def reset_peak_usage(self) -> None:
        self._block_manager.reset_peak_usage()

    def will_allocation_be_successful(self, n_blocks: int, allocated_blocks: int) -> bool:
        del allocated_blocks
        return n_blocks <= self.get_num_free_blocks()

    def allocate_blocks(self, n_blocks: int, request_id: str, allocated_blocks: int) -> int | None:
        if not self.will_allocation_be_successful(n_blocks, allocated_blocks):
            return None
        if len(self.block_table.get(request_id, ())) + n_blocks > self.table_width:
            raise ValueError(f"Request {request_id} needs more than {self.table_width} blocks (max_model_len)")
        blocks = self._block_manager.get_free_blocks(n_blocks)
        if blocks is None:
            raise ValueError(f"Failed to allocate {n_blocks} blocks for request {request_id}")
        owned = self.block_table.setdefault(request_id, [])
        row = self.table_row_of.get(request_id)
        if row is None:
            if not self._free_table_rows:
                raise CacheFullError("no free block-table row: more active requests than max_num_seqs allows")
            row = self._free_table_rows.pop()
            self.table_row_of[request_id] = row
        start = len(owned)
        owned.extend(blocks)
        for j, b in enumerate(blocks):
            self._queue_table_update(row, start + j, b)
        return n_blocks

    def free_blocks(self, request_id: str) -> None:
        blocks = self.block_table.pop(request_id, None)
        if blocks is None:
            return
        self._block_manager.free_blocks(blocks)
        row = self.table_row_of.pop(request_id)
        for j in range(len(blocks)):
            self._queue_table_update(row, j, -1)
        self._free_table_rows.append(row)

    def free_all_requests(self) -> None:
        for request_id in list(self.block_table):
            self.free_blocks(request_id)

    def _queue_table_update(self, row: int, col: int, value: int) -> None:
        self.host_table[row, col] = value
        self._dirty.add(row * self.table_width + col)

    # -- slot mapping ----------------------------------------------------------------------------------------
    def write_rows(self, request_id: str, past_length: int, query_length: int) -> np.ndarray:
        """Pool rows of positions past..past+query-1 (cache_manager.py:190-213)."""

        blocks = self.block_table.get(request_id)
        if blocks is None:
            raise ValueError(f"No block table found for request {request_id}")
        total = past_length + query_length
        needed = -(-total // self.block_size)
        if needed > len(blocks):
            raise ValueError(f"Request {request_id} needs {needed} blocks for length {total}, "
                             f"but only has {len(blocks)} allocated")
        pos = np.arange(past_length, total, dtype=np.int64)
        return np.asarray(blocks, dtype=np.int64)[pos // self.block_size] * self.block_size + pos % self.block_size

    def token_row(self, request_id: str, position: int) -> int:
        blocks = self.block_table[request_id]
        return blocks[position // self.block_size] * self.block_size + position % self.block_size

    def kv_slot_for_recurrent_step(self, recurrent_step: int) -> int:
        return self.layout.slot_for_step(recurrent_step)

    @property
    def requires_slot_homogeneous_recurrent_batches(self) -> bool:
        return self.kv_slots_per_layer > 1

    # -- device table sync ----------------------------------------------------------------------------------
    def take_table_updates(self, idx_out: np.ndarray, val_out: np.ndarray) -> int | None:
        """Move the queued cell updates into a launch's own upload buffers: cell indices into
        ``idx_out`` (int64) and values into ``val_out`` (int32); returns their count, or None
        (and leaves them queued for flush_table_updates) when they do not fit."""

        n = len(self._dirty)
        if n > len(idx_out):
            return None
        if n:
            idx_out[:n] = np.fromiter(self._dirty, dtype=np.int64, count=n)
            val_out[:n] = self.host_table.reshape(-1)[idx_out[:n]]
            self._dirty.clear()
        return n

    def flush_table_updates(self) -> None:
        """Apply queued block-table updates on the current stream (one H2D pair + one scatter)."""

        n = len(self._dirty)
        if n == 0:
            return
        if self._stage_event is not None:
            self._stage_event.synchronize()  # the previous upload has left the pinned staging buffers
        if n > self._stage_index.numel():
            cap = 2 * n
            pin = self.device.type == "cuda"
            self._stage_index = torch.empty(cap, dtype=torch.int64, pin_memory=pin)
            self._stage_value = torch.empty(cap, dtype=torch.int32, pin_memory=pin)
            self._dev_index = torch.empty(cap, dtype=torch.int64, device=self.device)
            self._dev_value = torch.empty(cap, dtype=torch.int32, device=self.device)
        index = np.fromiter(self._dirty, dtype=np.int64, count=n)
        self._dirty.clear()
        self._stage_index.numpy()[:n] = index
        self._stage_value.numpy()[:n] = self.host_table.reshape(-1)[index]
        self._dev_index[:n].copy_(self._stage_index[:n], non_blocking=True)
        self._dev_value[:n].copy_(self._stage_value[:n], non_blocking=True)
        if self._stage_event is None:
            self._stage_event = torch.cuda.Event()
        self._stage_event.record()
        ops.copy_rows_raw(self._dev_value[:n].view(n, 1), None, self.device_table.view(-1, 1),
                          self._dev_index[:n], n)

    def snapshot_request_table(self, request_id: str) -> list[int]:
        """The kernel-visible block-table row of a request (for parity checks)."""

        row = self.table_row_of[request_id]
        return self.device_table[row].cpu().tolist()
