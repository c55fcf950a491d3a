"""KV-pressure preemption: soft reset (recompute) and swap to a pinned host pool (offload).

``OffloadingManager`` is the host bookkeeping of pkg/offloading_manager.py:27-348:
it picks between swapping a victim's KV blocks out and soft-resetting it, keeps
the host-block map of swapped requests, copies them back on restore and counts
both kinds of preemption. The victim is always a stalled decoder, at a clean
token boundary, chosen by the engine.

``KvSwapPool`` moves the blocks. The reference issues one ``copy_`` per block,
per layer, per K/V plane (2 * layers * blocks small copies). Here one host-pool
block holds one device block's slabs for every cache layer, K and V, so a block
is one contiguous host range:

    host pool: (num_host_blocks, 2 * num_cache_layers, block_size * Hkv * D)

A swap-out gathers the victim's slabs, block-major, into a staging buffer in
HBM with the row-copy kernel and hands each run of consecutive host blocks to
one DMA; a restore DMAs the runs into staging and scatters them with one
row-copy launch. Everything is ordered on the compute stream, so a block freed
after a swap-out is only rewritten by work queued behind the copy.
"""

from __future__ import annotations

import logging
import time
from collections import deque
from contextlib import nullcontext
from typing import Any, Callable

import numpy as np
import torch

from . import ops

logger = logging.getLogger("ContinuousBatchingLogger")


def host_block_runs(host_blocks: list[int]) -> list[tuple[int, int, int]]:
    """(first host block, offset in the list, length) of each run of consecutive host blocks."""

    runs: list[tuple[int, int, int]] = []
    k = 0
    n = len(host_blocks)
    while k < n:
        start = k
        while k + 1 < n and host_blocks[k + 1] == host_blocks[k] + 1:
            k += 1
        runs.append((host_blocks[start], start, k - start + 1))
        k += 1
    return runs


class KvSwapPool:
    """Pinned host pool for swapped-out KV blocks, and the device path that fills and drains it."""

    #: Device staging bytes; a victim larger than this moves in several chunks.
    STAGING_BYTES = 64 << 20

    def __init__(self, cache: Any, num_host_blocks: int, stream: torch.cuda.Stream | None = None) -> None:
        if cache.device.type != "cuda":
            raise RuntimeError("the KV swap pool moves blocks with the HIP row-copy kernel; the cache is on the CPU")
        self.cache = cache
        self.slabs = 2 * cache.num_layers
        # Block-rows per (layer, K/V) plane of the device pool, spare blocks included.
        self.plane_blocks = cache.pool.shape[2] // cache.block_size
        self.block_elems = cache.block_size * cache.num_key_value_heads * cache.head_dim
        self.device_rows = cache.pool.view(self.slabs * self.plane_blocks, self.block_elems)
        self.num_host_blocks = num_host_blocks
        self.host = torch.empty((num_host_blocks, self.slabs, self.block_elems), dtype=cache.dtype, pin_memory=True)
        block_bytes = self.slabs * self.block_elems * self.host.element_size()
        self.chunk_blocks = max(1, min(cache.max_blocks_per_request, self.STAGING_BYTES // block_bytes))
        self.staging = torch.empty((self.chunk_blocks * self.slabs, self.block_elems), dtype=cache.dtype,
                                   device=cache.device)
        cap = cache.max_blocks_per_request * self.slabs
        self._index_host = torch.empty(cap, dtype=torch.int64, pin_memory=True)
        self._index_dev = torch.empty(cap, dtype=torch.int64, device=cache.device)
        self._index_event: torch.cuda.Event | None = None
        self.stream = stream
        # Optional HIP-event timing of every move: (direction, bytes, start, end).
        self.record_timings = False
        self._timings: list[tuple[str, int, torch.cuda.Event, torch.cuda.Event]] = []

    def _scope(self):
        return torch.cuda.stream(self.stream) if self.stream is not None else nullcontext()

    def _timed(self, direction: str, blocks: int):
        if not self.record_timings:
            return None
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        self._timings.append((direction, blocks * self.slabs * self.block_elems * self.host.element_size(),
                              start, end))
        return end

    def transfer_summary(self) -> dict[str, float]:
        """Moves, bytes and device milliseconds per direction (call after a synchronize)."""

        out: dict[str, float] = {}
        for direction, nbytes, start, end in self._timings:
            out[f"{direction}_moves"] = out.get(f"{direction}_moves", 0) + 1
            out[f"{direction}_bytes"] = out.get(f"{direction}_bytes", 0) + nbytes
            out[f"{direction}_ms"] = round(out.get(f"{direction}_ms", 0.0) + start.elapsed_time(end), 3)
        return out

    def _upload_index(self, device_blocks: list[int]) -> torch.Tensor:
        """Device rows of every slab of ``device_blocks``, block-major, on the compute stream.

        A restore moves every request restored in a tick at once, so the index buffers grow
        past one request's blocks when needed."""

        blocks = np.asarray(device_blocks, dtype=np.int64)
        if blocks.min() < 0 or blocks.max() >= self.cache.num_blocks:
            raise ValueError(f"device blocks out of range for the KV pool: {device_blocks}")
        rows = (np.arange(self.slabs, dtype=np.int64)[None, :] * self.plane_blocks + blocks[:, None]).reshape(-1)
        if self._index_event is not None:
            self._index_event.synchronize()  # the previous upload has left the pinned buffer
        if rows.size > self._index_host.numel():
            self._index_host = torch.empty(rows.size, dtype=torch.int64, pin_memory=True)
            self._index_dev = torch.empty(rows.size, dtype=torch.int64, device=self.cache.device)
        self._index_host.numpy()[: rows.size] = rows
        dev = self._index_dev[: rows.size]
        dev.copy_(self._index_host[: rows.size], non_blocking=True)
        if self._index_event is None:
            self._index_event = torch.cuda.Event()
        self._index_event.record()
        return dev

    def _check(self, host_blocks: list[int], device_blocks: list[int]) -> None:
        if len(host_blocks) != len(device_blocks):
            raise ValueError(f"{len(host_blocks)} host blocks for {len(device_blocks)} device blocks")
        if host_blocks and (min(host_blocks) < 0 or max(host_blocks) >= self.num_host_blocks):
            raise ValueError(f"host blocks out of range for a {self.num_host_blocks}-block pool")

    def swap_out(self, device_blocks: list[int], host_blocks: list[int]) -> None:
        """host[host_blocks[j]] = device block device_blocks[j], over every cache layer, K and V."""

        self._check(host_blocks, device_blocks)
        if not device_blocks:
            return
        s, step = self.slabs, self.chunk_blocks
        with self._scope():
            end = self._timed("out", len(device_blocks))
            index = self._upload_index(device_blocks)
            for c0 in range(0, len(device_blocks), step):
                c1 = min(len(device_blocks), c0 + step)
                ops.copy_rows_raw(self.device_rows, index[c0 * s:c1 * s], self.staging, None, (c1 - c0) * s)
                for h0, k0, r in host_block_runs(host_blocks[c0:c1]):
                    self.host[h0:h0 + r].view(r * s, self.block_elems).copy_(
                        self.staging[k0 * s:(k0 + r) * s], non_blocking=True)
            if end is not None:
                end.record()

    def swap_in(self, host_blocks: list[int], device_blocks: list[int]) -> None:
        """Device block device_blocks[j] = host[host_blocks[j]], over every cache layer, K and V."""

        self._check(host_blocks, device_blocks)
        if not device_blocks:
            return
        s, step = self.slabs, self.chunk_blocks
        with self._scope():
            end = self._timed("in", len(device_blocks))
            index = self._upload_index(device_blocks)
            for c0 in range(0, len(device_blocks), step):
                c1 = min(len(device_blocks), c0 + step)
                for h0, k0, r in host_block_runs(host_blocks[c0:c1]):
                    self.staging[k0 * s:(k0 + r) * s].copy_(
                        self.host[h0:h0 + r].view(r * s, self.block_elems), non_blocking=True)
                ops.copy_rows_raw(self.staging, None, self.device_rows, index[c0 * s:c1 * s], (c1 - c0) * s)
            if end is not None:
                end.record()


class OffloadingManager:
    """Preemption of stalled decoders: swap out when the host pool has room, else soft reset
    (pkg/offloading_manager.py:27-348)."""

    def __init__(self, cache: Any, scheduler: Any, cpu_offload_space_gib: float | None, *,
                 allow_recompute_fallback: bool = True,
                 swap_factory: Callable[[int], Any] | None = None) -> None:
        self.cache = cache
        self.scheduler = scheduler
        # A soft reset re-prefills at full depth; under a policy that rewrites KV on early exit
        # that changes what the cache holds, so the fallback is disabled there.
        self._allow_recompute_fallback = allow_recompute_fallback
        self._request_id_to_cpu_blocks: dict[str, list[int]] = {}
        self.num_offload_preemptions = 0
        self.num_recompute_preemptions = 0
        self.num_restores = 0
        # (time, request_id, "offload" | "recompute") per preemption, and (time, request_id,
        # re-prefill length) per soft reset: a handful of entries per run, always recorded.
        self.preemption_events: list[tuple[float, str, str]] = []
        self.recompute_events: list[tuple[float, str, int]] = []
        self.restore_events: list[tuple[float, str]] = []
        self._num_cpu_blocks = self._compute_num_cpu_blocks(cpu_offload_space_gib)
        self.swap: Any = None
        self._free_cpu_blocks: deque[int] = deque()
        if self._num_cpu_blocks == 0:
            if cpu_offload_space_gib:
                logger.warning(f"cpu_offload_space={cpu_offload_space_gib} GiB holds no KV block; preemption "
                               "will use soft reset (recompute) only.")
            return
        if swap_factory is None:
            raise ValueError("a host swap pool needs a swap_factory")
        self.swap = swap_factory(self._num_cpu_blocks)
        self._free_cpu_blocks = deque(range(self._num_cpu_blocks))

    @property
    def offloading_enabled(self) -> bool:
        return self._num_cpu_blocks > 0

    @property
    def num_cpu_blocks(self) -> int:
        return self._num_cpu_blocks

    @property
    def num_preemptions(self) -> int:
        return self.num_offload_preemptions + self.num_recompute_preemptions

    def preemption_stats(self) -> dict[str, int]:
        return {"preemptions": self.num_preemptions, "offload_preemptions": self.num_offload_preemptions,
                "recompute_preemptions": self.num_recompute_preemptions, "restores": self.num_restores}

    def bytes_per_block(self) -> int:
        """Bytes of one KV block over every cache layer, K and V."""

        c = self.cache
        elem = torch.empty((), dtype=c.dtype).element_size()
        return 2 * c.num_layers * c.block_size * c.num_key_value_heads * c.head_dim * elem

    def _compute_num_cpu_blocks(self, cpu_offload_space_gib: float | None) -> int:
        if not cpu_offload_space_gib or cpu_offload_space_gib <= 0:
            return 0
        return int(cpu_offload_space_gib * 1024**3) // self.bytes_per_block()

    def preempt_request(self, request_id: str, state: Any) -> None:
        """Preempt a stalled decoder (pkg/offloading_manager.py:172-217): swap its KV out when the
        pool has room, else soft-reset it; free its blocks, re-queue it and hold new admissions
        until a request finishes."""

        logger.info(f"Preempting request {request_id}: {len(state.initial_tokens)} prompt + "
                    f"{len(state.generated_tokens)} generated tokens.")
        stamp = time.perf_counter()
        if self._offload_to_cpu(request_id, state):
            state.prepare_for_offload_requeue()
            new_state = state
            self.num_offload_preemptions += 1
            policy = "offload"
        else:
            if not self._allow_recompute_fallback:
                needed = len(self.cache.block_table.get(request_id, []))
                raise RuntimeError(
                    f"CPU swap pool cannot hold request {request_id} ({needed} blocks needed, "
                    f"{len(self._free_cpu_blocks)} free) and the soft-reset fallback is disabled: "
                    "re-prefilling at full depth would replace the KV this cache policy rewrote on "
                    "early exit. Increase cpu_offload_space or reduce load.")
            new_state = state.create_equivalent_initial_request()
            self.num_recompute_preemptions += 1
            policy = "recompute"
            self.recompute_events.append((stamp, request_id, len(new_state.remaining_prefill_tokens)))
        self.preemption_events.append((stamp, request_id, policy))
        self.scheduler.finish_request(request_id)
        self.scheduler.add_waiting_request(new_state)
        self.scheduler.block_new_requests = True

    def _offload_to_cpu(self, request_id: str, state: Any) -> bool:
        """Swap a request's blocks out (pkg/offloading_manager.py:276-314); False if the pool is full."""

        if state.is_cpu_offloaded:
            raise RuntimeError(f"Request {request_id} is already offloaded; refusing to offload it twice.")
        device_blocks = self.cache.block_table.get(request_id, [])
        total = len(device_blocks)
        if total == 0 or len(self._free_cpu_blocks) < total:
            return False
        host_blocks = [self._free_cpu_blocks.popleft() for _ in range(total)]
        self.swap.swap_out(list(device_blocks), host_blocks)
        self._request_id_to_cpu_blocks[request_id] = host_blocks
        state.is_cpu_offloaded = True
        return True

    def restore_scheduled_requests(self, states: list[Any]) -> None:
        """Copy the swapped-out KV of restored requests back (pkg/offloading_manager.py:219-274).

        A restored request may already hold one more block for its next token; only the blocks
        that were swapped out are filled, in device-block order."""

        host: list[int] = []
        device: list[int] = []
        for state in states:
            if not state.is_cpu_offloaded:
                continue
            cpu_blocks = self._request_id_to_cpu_blocks.pop(state.request_id)
            gpu_blocks = self.cache.block_table.get(state.request_id, [])
            if len(gpu_blocks) < len(cpu_blocks):
                raise RuntimeError(f"Request {state.request_id} restored with {len(gpu_blocks)} blocks for "
                                   f"{len(cpu_blocks)} swapped-out ones")
            host.extend(cpu_blocks)
            device.extend(gpu_blocks[: len(cpu_blocks)])
            state.is_cpu_offloaded = False
            state.allocated_blocks = len(gpu_blocks)
            self.num_restores += 1
            self.restore_events.append((time.perf_counter(), state.request_id))
        if not host:
            return
        self.swap.swap_in(host, device)
        # Stream-ordered: the host-to-device reads above run before any later swap-out rewrites
        # these host blocks.
        self._free_cpu_blocks.extend(host)

    def free_request_cpu_cache(self, state: Any) -> None:
        if state.is_cpu_offloaded:
            self._free_cpu_blocks.extend(self._request_id_to_cpu_blocks.pop(state.request_id, []))
            state.is_cpu_offloaded = False

    def free_all_waiting_cpu_caches(self) -> None:
        for state in self.scheduler.waiting_requests.values():
            self.free_request_cpu_cache(state)

    def reset(self) -> None:
        self._request_id_to_cpu_blocks.clear()
        self._free_cpu_blocks = deque(range(self._num_cpu_blocks))
        self.num_offload_preemptions = 0
        self.num_recompute_preemptions = 0
        self.num_restores = 0
        self.preemption_events.clear()
        self.recompute_events.clear()
        self.restore_events.clear()


__all__ = ["KvSwapPool", "OffloadingManager", "host_block_runs"]
