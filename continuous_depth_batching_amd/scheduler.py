"""CDB scheduler: prompt admission, the mixed-depth ready queue and the coda queue.

One tick schedules one homogeneous bucket, in priority order coda (once
``min_coda_batch_size`` tokens wait) > prefill (when admission allows) >
recurrent > an undersized coda flush (continuous_depth_batching/scheduler.py:101-140).
Recurrent work is a FIFO deque; a stepped batch's survivors and freshly
sampled successors return to its head in launch order, which keeps a bounded
working set advancing (:142-180). Under multi-slot KV layouts a recurrent
batch holds only items writing the same slot (:322-346). Admission, token
budgets and block allocation follow scheduler_base.py:171-545. ``mixed_slot_launches`` lifts the
slot rule (the kernels read a cache layer per row).

The per-tick decisions run in the C++ tick core (``_tick.schedule_next`` and the
admission functions beside it) over this object's attributes: the queues, the
request dicts and counters stay here, where the engine and its statistics read them.
"""

from __future__ import annotations

import time
from collections import deque
from dataclasses import dataclass
from typing import Literal

from . import _tick
from .cache import PagedKVCache
from .config import resolve_min_free_slots
from .requests import DepthWorkItem, FutureRequestState, RequestState, RequestStatus, logger

ScheduledKind = Literal["prefill", "coda", "recurrent"]


def reserved_peak_blocks(initial_len: int, max_new_tokens: int | None, max_model_len: int, block_size: int) -> int:
    """Worst-case blocks a request can hold (utils.py:107-129)."""

    total = max_model_len if max_new_tokens is None else min(initial_len + max_new_tokens, max_model_len)
    return -(-total // block_size)


@dataclass
class ScheduledCDBBatch:
    kind: ScheduledKind
    requests: list[FutureRequestState] | None = None
    depth_items: list[DepthWorkItem] | None = None
    num_q_tokens: int = 0
    max_kv_read: int = 0


class CDBScheduler:
    def __init__(self, cache: PagedKVCache, max_recurrent_steps: int, *, safety_margin: float = 0.2,
                 kv_pressure_mode: str = "recompute", max_model_len: int | None = None, max_num_seqs: int = 256,
                 min_free_slots: int | None = None, min_coda_batch_size: int = 1,
                 mixed_slot_launches: bool = False) -> None:
        if max_recurrent_steps <= 0:
            raise ValueError(f"max_recurrent_steps must be positive, got {max_recurrent_steps}")
        if min_coda_batch_size <= 0:
            raise ValueError(f"min_coda_batch_size must be positive, got {min_coda_batch_size}")
        if max_num_seqs <= 0:
            raise ValueError(f"max_num_seqs must be positive, got {max_num_seqs}")
        self.cache = cache
        self.max_num_seqs = min(max_num_seqs, cache.max_num_batched_tokens)
        self.safety_margin = 0.0 if kv_pressure_mode == "reserve" else safety_margin
        self.kv_pressure_mode = kv_pressure_mode
        self.max_model_len = max_model_len
        self.max_decode_fast_path_length = cache.max_blocks_per_request * cache.block_size
        self.min_free_slots = resolve_min_free_slots(min_free_slots, self.max_num_seqs)
        self.max_recurrent_steps = max_recurrent_steps
        self.min_coda_batch_size = min(min_coda_batch_size, self.max_num_seqs)
        self.slot_homogeneous = cache.requires_slot_homogeneous_recurrent_batches and not mixed_slot_launches
        self._slot_of_step = tuple(cache.kv_slot_for_recurrent_step(s) for s in range(max_recurrent_steps)) \
            if self.slot_homogeneous else None
        # Completions before the steady-state window opens (steady_state_summary); None leaves it off.
        self.steady_warmup_requests: int | None = None
        if kv_pressure_mode == "reserve":
            if max_model_len is None:
                raise ValueError("kv_pressure_mode='reserve' requires max_model_len")
            peak = reserved_peak_blocks(0, max_model_len, max_model_len, cache.block_size)
            if peak > cache.num_blocks:
                raise ValueError(f"kv_pressure_mode='reserve' cannot serve a max-length request: needs {peak} "
                                 f"blocks but the cache has {cache.num_blocks}")
        self.reset()

    def reset(self) -> None:
        self.active_requests: dict[str, RequestState] = {}
        self.waiting_requests: dict[str, RequestState] = {}
        self.waiting_requests_order: deque[str] = deque()
        self.block_new_requests = False
        # Deques of work items in the tick core; the per-tick head re-insertion and bucket
        # pops run there (enqueue_front, pop_batch, pop_front).
        self.ready_queue = _tick.ItemQueue()
        self.coda_queue = _tick.ItemQueue()
        self.mixed_batches_scheduled = 0
        self.refill_events = 0
        self.max_depth_queue_size = 0
        self.in_flight_request_ids: set[str] = set()
        self.max_in_flight_requests = 0
        self.max_live_requests = 0
        self.max_resident_requests = 0
        self.resident_samples = 0
        self.resident_sum = 0
        self.completed_requests = 0
        self.completed_generated_tokens = 0
        self._steady_start_time: float | None = None
        self._steady_end_time: float | None = None
        self._steady_start_progress = (0, 0)
        self._steady_end_progress = (0, 0)
        self._steady_ticks = 0
        self._steady_resident_sum = 0

    # -- bookkeeping -------------------------------------------------------------------------------------------
    def add_waiting_request(self, state: RequestState) -> None:
        self.waiting_requests[state.request_id] = state
        self.waiting_requests_order.append(state.request_id)

    def has_pending_work(self) -> bool:
        return bool(self.coda_queue or self.ready_queue or self.active_requests or self.waiting_requests)

    def record_resident_sample(self) -> None:
        """Resident-set peak and mean, and the steady-state window when one is tracked."""

        _tick.record_resident_sample(self)

    # -- steady-state window (scheduler_base.py:315-398) --------------------------------------------------------
    @property
    def steady_window_open(self) -> bool:
        return self._steady_start_time is not None and self._steady_end_time is None

    def _advance_steady_window(self, resident: int) -> None:
        """Open the window on the tick ``steady_warmup_requests`` requests have completed while prompts
        still wait; close it on the first tick after the last admission (which belongs to the drain)."""

        if self.steady_warmup_requests is None or self._steady_end_time is not None:
            return
        if self._steady_start_time is None:
            if self.completed_requests < self.steady_warmup_requests or not self.waiting_requests:
                return
            self._steady_start_time = time.perf_counter()
            self._steady_start_progress = self._progress_snapshot()
        elif not self.waiting_requests:
            self.close_steady_window()
            return
        self._steady_ticks += 1
        self._steady_resident_sum += resident

    def _progress_snapshot(self) -> tuple[int, int]:
        """Requests completed and tokens generated so far, resident and re-queued requests included."""

        generated = self.completed_generated_tokens
        generated += sum(state.total_generated_len() for state in self.active_requests.values())
        generated += sum(state.total_generated_len() for state in self.waiting_requests.values())
        return self.completed_requests, generated

    def close_steady_window(self) -> None:
        if self._steady_start_time is None or self._steady_end_time is not None:
            return
        self._steady_end_time = time.perf_counter()
        self._steady_end_progress = self._progress_snapshot()

    def steady_state_summary(self) -> dict | None:
        """Throughput inside the steady-state window, or None when the run held no such window
        (the warm-up count was never reached, or only while draining, or nothing completed)."""

        if self._steady_start_time is None or self._steady_end_time is None:
            return None
        window_s = self._steady_end_time - self._steady_start_time
        completed = self._steady_end_progress[0] - self._steady_start_progress[0]
        generated = self._steady_end_progress[1] - self._steady_start_progress[1]
        if window_s <= 0.0 or completed <= 0:
            return None
        return {"warmup_requests": self.steady_warmup_requests, "window_s": window_s, "ticks": self._steady_ticks,
                "completed_requests": completed, "generated_tokens": generated,
                "requests_per_second": completed / window_s, "generated_tokens_per_second": generated / window_s,
                "mean_resident_requests": self._steady_resident_sum / self._steady_ticks if self._steady_ticks else 0.0}

    def record_completion(self, state: RequestState) -> None:
        self.completed_requests += 1
        self.completed_generated_tokens += state.total_generated_len()

    def finish_request(self, request_id: str) -> None:
        self.cache.free_blocks(request_id)
        self.active_requests.pop(request_id, None)
        self.in_flight_request_ids.discard(request_id)
        if self.waiting_requests.pop(request_id, None) is not None:
            self.waiting_requests_order.remove(request_id)

    def free_unfinished_requests(self) -> None:
        for request_id in list(self.active_requests):
            self.finish_request(request_id)
        for request_id in list(self.waiting_requests):
            self.finish_request(request_id)

    def release_in_flight_request(self, request_id: str) -> None:
        self.in_flight_request_ids.discard(request_id)

    def _mark_request_in_flight(self, request_id: str) -> None:
        in_flight = self.in_flight_request_ids
        in_flight.add(request_id)
        if len(in_flight) > self.max_in_flight_requests:
            self.max_in_flight_requests = len(in_flight)
        live = len(self.active_requests) + len(self.waiting_requests)
        if live > self.max_live_requests:
            self.max_live_requests = live

    # -- admission (scheduler_base.py:171-201, 416-545) --------------------------------------------------------
    def prefill_admitted(self) -> bool:
        """Prefill may run: nothing decodes, or the free blocks exceed the safety margin."""

        return _tick.prefill_admitted(self)

    def free_residency_slots(self) -> int:
        return max(0, self.max_num_seqs - len(self.active_requests))

    def admit_offloaded_restores(self) -> list[RequestState]:
        """Move swapped-out waiting requests back to the active set with blocks for their restored
        length plus one token (scheduler_base.py:434-460).

        Restores go before fresh prompts, are held while draining after a preemption, are bounded
        by the open resident slots and stop at the first request whose blocks do not fit."""

        if self.block_new_requests or self.kv_pressure_mode != "offload":
            return []
        admitted: list[RequestState] = []
        for request_id in list(self.waiting_requests_order):
            state = self.waiting_requests[request_id]
            if not state.is_cpu_offloaded:
                continue
            if self.free_residency_slots() == 0 or not self._allocate_blocks_if_needed(state, 1):
                break
            self.active_requests[request_id] = state
            del self.waiting_requests[request_id]
            self.waiting_requests_order.remove(request_id)
            admitted.append(state)
        return admitted

    def get_prefill_bucket(self) -> list[RequestState]:
        """Requests mid-prefill with no token in flight, then admissible waiting prompts."""

        return _tick.prefill_bucket(self)

    def _allocate_blocks_if_needed(self, state: RequestState, len_next_tokens: int) -> bool:
        return _tick.allocate_if_needed(self, state, len_next_tokens)

    # -- bucket selection (continuous_depth_batching/scheduler.py:101-349) ------------------------------------
    def schedule_next(self, token_budget: int, cache_budget: int, *, allow_coda: bool = True) -> ScheduledCDBBatch | None:
        return _tick.schedule_next(self, token_budget, cache_budget, allow_coda)

    def enqueue_depth(self, item: DepthWorkItem, *, front: bool = False) -> None:
        if not 0 <= item.recurrent_step < self.max_recurrent_steps:
            raise ValueError(f"recurrent_step must be in [0, {self.max_recurrent_steps}), got {item.recurrent_step}")
        self._mark_request_in_flight(item.state.request_id)
        if item.recurrent_step == 0 and self.ready_queue:
            self.refill_events += 1
        if front:
            self.ready_queue.appendleft(item)
        else:
            self.ready_queue.append(item)
        self.max_depth_queue_size = max(self.max_depth_queue_size, len(self.ready_queue))

    def enqueue_depth_front(self, items: list[DepthWorkItem]) -> None:
        """Return items to the queue head preserving their order (enqueue_depth(front=True)
        applied from the last item to the first, in one pass)."""

        if not items:
            return
        queue = self.ready_queue
        self.refill_events += _tick.enqueue_front(queue, items, self.max_recurrent_steps, self.in_flight_request_ids)
        # The in-flight set only grew inside, so its peak is its size now.
        if len(self.in_flight_request_ids) > self.max_in_flight_requests:
            self.max_in_flight_requests = len(self.in_flight_request_ids)
        live = len(self.active_requests) + len(self.waiting_requests)
        if live > self.max_live_requests:
            self.max_live_requests = live
        if len(queue) > self.max_depth_queue_size:
            self.max_depth_queue_size = len(queue)

    def enqueue_coda(self, item: DepthWorkItem) -> None:
        self._mark_request_in_flight(item.state.request_id)
        self.coda_queue.append(item)

    def enqueue_coda_items(self, items: list[DepthWorkItem]) -> None:
        """enqueue_coda over ``items`` in order, with the in-flight peaks updated once."""

        if not items:
            return
        in_flight = self.in_flight_request_ids
        for item in items:
            in_flight.add(item.state.request_id)
        if len(in_flight) > self.max_in_flight_requests:
            self.max_in_flight_requests = len(in_flight)
        live = len(self.active_requests) + len(self.waiting_requests)
        if live > self.max_live_requests:
            self.max_live_requests = live
        self.coda_queue.extend(items)

    def schedule_prefill_batch(self, token_budget: int, cache_budget: int) -> ScheduledCDBBatch | None:
        return _tick.schedule_prefill(self, token_budget, cache_budget)


_tick.bind_batch_type(ScheduledCDBBatch)

__all__ = ["CDBScheduler", "ScheduledCDBBatch", "reserved_peak_blocks", "logger"]
