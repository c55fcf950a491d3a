"""ContinuousDepthBatchingEngine: the CDB decode loop on the MI355X kernels.

Public API and scheduling semantics follow continuous_depth_batching/continuous_api.py:
``from_model(model, cdb_config)`` / ``generate_batch(input_ids, max_new_tokens=...,
eos_token_id=..., exit_depths=...)``. One scheduler tick launches one bucket:

  * prefill -- a full-depth forward over admitted prompt chunks; on the async
    path each prompt's first decode token enters its prelude straight from the
    device tokens (eager entry) and queues at the tail;
  * recurrent -- one block application over up to ``max_num_seqs`` work items
    that may sit at different loop steps; exited items go to the coda queue,
    survivors advance a step and return to the queue head in launch order;
  * coda -- LM head + argmax for exited tokens; on the async path the
    successor token's prelude is staged from the device tokens before the host
    reads them (eager re-entry, queue head), with at most two codas in flight.

The exit decision of every row comes from the ``cdb_exit_gate`` kernel (live
gate, replayed synthetic depth, forced final step). On the synchronous horizon
the host waits for a launch's decisions before routing it, as the reference
does; on the delayed horizon a launch's routing uses the decisions of the
item's previous launch, which have long landed.
"""

from __future__ import annotations

import gc
import time
from collections import Counter, deque
from dataclasses import dataclass, field
from typing import Any, Callable

import torch

from .cache import CacheFullError, PagedKVCache
from .decode_staging import DecodeStaging
from .offloading import OffloadingManager
from .config import ContinuousDepthBatchingConfig, validate_cache_size_request
from .exit_policy import ExitPolicy
from .kv_cache_policy import LoopedKvLayout, copies_exit_kv, resolve_kv_slots_per_layer
from .model_adapter import CDBModelAdapter, resolve_cdb_model_adapter
from .model_runner import (
    CODA_PIPELINE_DEPTH,
    ModelRunner,
    PendingCodaResult,
    PendingFlags,
    PendingPrefillResult,
)
from .requests import TMP_TOKEN_ID, DepthWorkItem, GenerationOutput, RequestState, RequestStatus
from .scheduler import CDBScheduler, ScheduledCDBBatch
from . import _tick


@dataclass
class ContinuousDepthBatchingStats:
    """Runtime counters (continuous_api.py:114-228)."""

    prefill_batches: int = 0
    prefill_requests: int = 0
    recurrent_batches: int = 0
    coda_batches: int = 0
    recurrent_steps: int = 0
    coda_tokens: int = 0
    generated_tokens: int = 0
    prefill_recurrent_steps: int = 0
    prefill_coda_tokens: int = 0
    fixed_depth_recurrent_steps: int = 0
    exit_depth_histogram: Counter = field(default_factory=Counter)
    recurrent_step_histogram: Counter = field(default_factory=Counter)
    mixed_recurrent_batches: int = 0
    mixed_recurrent_depth_histogram: Counter = field(default_factory=Counter)
    max_mixed_depths_per_batch: int = 0
    scheduler_refills: int = 0
    max_depth_queue_size: int = 0
    recurrent_graph_hits: int = 0
    recurrent_graph_captures: int = 0
    max_in_flight_requests: int = 0
    max_live_requests: int = 0
    prelude_batches: Counter = field(default_factory=Counter)
    prelude_tokens: Counter = field(default_factory=Counter)
    prelude_gathered_tokens: Counter = field(default_factory=Counter)
    cancelled_depth_items: int = 0
    coda_suppressed_ticks: int = 0
    max_pending_coda_results: int = 0
    coda_pipeline_blocked_ticks: int = 0
    scheduler_ticks: int = 0
    exit_kv_copies: int = 0

    @property
    def skipped_recurrent_steps(self) -> int:
        return max(0, self.fixed_depth_recurrent_steps - self.recurrent_steps)

    @property
    def mean_recurrent_batch_size(self) -> float:
        return self.recurrent_steps / self.recurrent_batches if self.recurrent_batches else 0.0

    @property
    def mean_coda_batch_size(self) -> float:
        return self.coda_tokens / self.coda_batches if self.coda_batches else 0.0


def _prelude_event(site: str, items: list[DepthWorkItem]) -> tuple:
    return ("prelude", site, tuple((i.state.request_id, i.token_position, i.hidden_slot) for i in items))


@dataclass
class _WaveCarry:
    """What one no-refill iteration leaves for the next on the delayed horizon
    (cdb/continuous_api.py:80-110 keeps the same three parts).

    ``groups`` are successors built before their tokens are on the host, each group with the
    staged result whose device tokens its rows index; the next wave's one prelude gathers them.
    ``coda`` is the last wave's staged coda, read after the next wave's first launch.
    ``prefills`` are prompt readbacks, applied at the top of the next iteration."""

    groups: list[tuple[Any, list[DepthWorkItem], list[int]]] = field(default_factory=list)
    coda: PendingCodaResult | None = None
    prefills: list[PendingPrefillResult] = field(default_factory=list)

    def num_items(self) -> int:
        return sum(len(items) for _, items, _ in self.groups)

    def empty(self) -> bool:
        return not self.groups and self.coda is None and not self.prefills


DEFAULT_MEM_FRACTION_STATIC = 0.8


def resolve_num_blocks(num_blocks: int | None, mem_fraction: float | None, bytes_per_block: int,
                       device: torch.device | str) -> int:
    """Explicit num_blocks, or the usable blocks of the post-load budget
    ``free - total * (1 - fraction)`` (kv_cache_sizing.py:34-80, paged_cache_geometry.py:143-144).

    The model is loaded before the engine is built, so the reserve ``total * (1 - fraction)``
    covers graph captures, activations and every allocation outside the KV pool. On a 288 GB
    MI355X the default fraction leaves about 58 GB of that reserve."""

    validate_cache_size_request(num_blocks, mem_fraction)
    if num_blocks is not None:
        return num_blocks
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("Automatic KV cache sizing requires CUDA (torch's device for the GPU); set num_blocks "
                         "explicitly for other devices")
    gc.collect()
    torch.cuda.empty_cache()
    free, total = torch.cuda.mem_get_info(device)
    fraction = DEFAULT_MEM_FRACTION_STATIC if mem_fraction is None else mem_fraction
    budget = int(free - total * (1 - fraction))
    blocks = budget // bytes_per_block - PagedKVCache.EXTRA_BLOCKS
    if blocks <= 0:
        raise ValueError(f"No usable KV blocks fit: free={free} bytes, total={total} bytes, "
                         f"mem_fraction_static={fraction}, bytes_per_block={bytes_per_block}. "
                         "Increase mem_fraction_static or reduce the model/cache size.")
    return blocks


@dataclass
class ContinuousDepthBatchingEngine:
    model: Any
    cdb_config: ContinuousDepthBatchingConfig
    cache: PagedKVCache
    scheduler: CDBScheduler
    runner: ModelRunner
    model_adapter: CDBModelAdapter
    exit_policy: ExitPolicy
    exit_kv_layout: LoopedKvLayout | None = None
    offloading_manager: OffloadingManager | None = None
    last_stats: ContinuousDepthBatchingStats = field(default_factory=ContinuousDepthBatchingStats)
    pending_coda_results: deque = field(default_factory=deque)
    pending_prefill_results: deque = field(default_factory=deque)
    staging: DecodeStaging | None = None
    finished_outputs: dict = field(default_factory=dict)
    # Schedule-parity hooks. ``record_launches`` logs every launch with the state it reads:
    #   ("prefill",   ((request_id, start_position, query_length, has_new_token), ...))
    #   ("prelude",   site, ((request_id, token_position, hidden_slot), ...))
    #   ("recurrent", ((request_id, token_position, step, hidden_slot, block_ids), ...), exits, refills)
    #   ("coda",      ((request_id, token_position, hidden_slot), ...))
    # ``consume_all_results`` consumes every staged prefill/coda result at the next consume point
    # (waiting for it), so the schedule depends on the inputs alone, not on device timing.
    record_launches: bool = False
    launch_log: list = field(default_factory=list)
    consume_all_results: bool = False
    _exit_kv_backlog: list = field(default_factory=list)
    _pending_flags: dict = field(default_factory=dict)

    # -- construction (continuous_api.py:274-376) -------------------------------------------------------------
    @classmethod
    def from_model(cls, model: Any, cdb_config: ContinuousDepthBatchingConfig, *, dtype: torch.dtype | None = None,
                   model_adapter: CDBModelAdapter | None = None,
                   runner_factory: Callable[..., ModelRunner] | None = None) -> "ContinuousDepthBatchingEngine":
        """Build the engine for ``model`` (continuous_api.py:274-376).

        ``runner_factory`` replaces the device runner, with ModelRunner's keyword arguments and
        interface; the engine's scheduling does not depend on which runner executes the stages."""

        del dtype
        cfg = cdb_config.get_resolved(model.config)
        adapter = resolve_cdb_model_adapter(model, model_adapter)
        assert cfg.max_recurrent_steps is not None
        adapter.configure_recurrent_steps(cfg.max_recurrent_steps)
        adapter.configure_exit_signal(cfg.exit_threshold is not None or cfg.synthetic_exit_replay)
        exit_policy = ExitPolicy(spec=adapter.exit_policy_spec(), threshold=cfg.exit_threshold,
                                 min_recurrent_steps=cfg.min_recurrent_steps,
                                 max_recurrent_steps=cfg.max_recurrent_steps,
                                 delay_gate_consumption=cfg.delay_gate_consumption,
                                 use_async_batching=cfg.use_async_batching,
                                 synthetic_exit_replay=cfg.synthetic_exit_replay)
        adapter.configure_kv_policy(cfg.kv_policy, cfg.kv_slots_per_layer)
        layout = adapter.kv_cache_layout()
        num_kv_heads, head_dim = adapter.kv_geometry()
        elem = torch.empty((), dtype=adapter.dtype).element_size()
        bytes_per_block = 2 * layout.num_cache_layers * cfg.block_size * num_kv_heads * head_dim * elem
        cfg.num_blocks = resolve_num_blocks(cfg.num_blocks, cfg.mem_fraction_static, bytes_per_block, adapter.device)
        cfg.max_num_seqs = min(cfg.max_num_seqs, cfg.max_num_batched_tokens)
        cache = PagedKVCache(layout=layout, num_blocks=cfg.num_blocks, block_size=cfg.block_size,
                             num_kv_heads=num_kv_heads, head_dim=head_dim, max_model_len=cfg.max_model_len,
                             max_num_batched_tokens=cfg.max_num_batched_tokens, max_requests=cfg.max_num_seqs,
                             dtype=adapter.dtype, device=adapter.device)
        runner = (runner_factory or ModelRunner)(engine_config=cfg, cache=cache, model_adapter=adapter,
                                                  exit_policy=exit_policy)
        scheduler = CDBScheduler(cache, cfg.max_recurrent_steps, safety_margin=cfg.safety_margin,
                                 kv_pressure_mode=cfg.kv_pressure_mode, max_model_len=cfg.max_model_len,
                                 max_num_seqs=cfg.max_num_seqs, min_free_slots=cfg.min_free_slots,
                                 min_coda_batch_size=cfg.min_coda_batch_size,
                                 mixed_slot_launches=cfg.mixed_slot_recurrent_batches)
        exit_kv_layout = layout if copies_exit_kv(cfg.kv_policy) else None
        offloading_manager = OffloadingManager(cache, scheduler, cfg.cpu_offload_space,
                                               allow_recompute_fallback=not copies_exit_kv(cfg.kv_policy),
                                               swap_factory=runner.make_kv_swap_pool)
        staging = DecodeStaging(cache, cfg.kv_pressure_mode, offloading_manager.preempt_request)
        return cls(model=model, cdb_config=cfg, cache=cache, scheduler=scheduler, runner=runner,
                   model_adapter=adapter, exit_policy=exit_policy, exit_kv_layout=exit_kv_layout,
                   offloading_manager=offloading_manager, staging=staging)

    # -- public API (continuous_api.py:378-452) -----------------------------------------------------------------
    @torch.no_grad()
    def generate_batch(self, input_ids: list[list[int]], *, max_new_tokens: int | list[int],
                       eos_token_id: int | list[int] | None = None, stop_sequences: list[list[int]] | None = None,
                       warmup: bool = True, model_kwargs: dict | None = None,
                       exit_depths: list[list[int]] | None = None, arrival_offsets_s: list[float] | None = None,
                       record_token_times: bool = False, record_queue_samples: bool = False) -> list[GenerationOutput]:
        del warmup, record_token_times, record_queue_samples
        if arrival_offsets_s is not None:
            raise NotImplementedError("open-loop arrivals are not served by this engine")
        self._validate_generate_inputs(input_ids, max_new_tokens)
        mnt = list(max_new_tokens) if isinstance(max_new_tokens, list) else [max_new_tokens] * len(input_ids)
        mnt = self._cap_to_model_len(input_ids, mnt)
        self._validate_model_kwargs(model_kwargs)
        self.exit_policy.validate_serving_timing()
        self._validate_exit_depths(input_ids, mnt, exit_depths)
        self.reset()
        states = [RequestState(request_id=f"request-{i}", initial_tokens=list(p), max_new_tokens=mnt[i],
                               eos_token_id=eos_token_id,
                               stop_sequences=[list(s) for s in stop_sequences] if stop_sequences else [],
                               synthetic_exit_depths=list(exit_depths[i]) if exit_depths is not None else [],
                               replay_eos_finishes=self.cdb_config.replay_eos_finishes)
                  for i, p in enumerate(input_ids)]
        for s in states:
            self.scheduler.add_waiting_request(s)
        try:
            with self.runner.stream_scope():
                if self.cdb_config.refill:
                    self._run_scheduler_loop()
                else:
                    self._run_no_refill_loop()
        finally:
            self.runner.synchronize()
            self.scheduler.close_steady_window()
            self.scheduler.free_unfinished_requests()
        outputs = [self.finished_outputs[s.request_id] for s in states]
        self.last_stats.generated_tokens = sum(len(o.generated_tokens) for o in outputs)
        return outputs

    def reset(self) -> None:
        self.offloading_manager.free_all_waiting_cpu_caches()
        self.scheduler.reset()
        self.cache.free_all_requests()
        self.cache.reset_peak_usage()
        self.runner.reset_cdb_runtime_counters()
        self.offloading_manager.reset()
        self.last_stats = ContinuousDepthBatchingStats()
        self.pending_coda_results.clear()
        self.pending_prefill_results.clear()
        self.staging.clear()
        self.finished_outputs.clear()
        self._exit_kv_backlog.clear()
        self._pending_flags.clear()
        self.launch_log.clear()

    # -- refill loop (continuous_api.py:503-606) ----------------------------------------------------------------
    def _run_scheduler_loop(self) -> None:
        """Scheduler ticks until every request finished and every staged result was taken in.

        A tick takes in the results that have landed (waiting for them when nothing else is
        pending), puts restored and parked decoders back into the loop, then launches the one
        bucket ``schedule_next`` picks. A tick that gets no bucket instead waits for a staged
        result, takes a parked decoder's KV away, or reports a dead end."""

        sched = self.scheduler
        while sched.has_pending_work() or self.pending_coda_results or self.pending_prefill_results:
            self._take_landed_results()
            if not sched.has_pending_work():  # what landed finished the last request, or nothing is left
                continue
            self._resume_decoders()
            batch = self._pick_batch()
            if batch is None:
                self._unblock()
            else:
                self._launch(batch)
        self._take_landed_results(wait=True)
        self._finish_stats()

    def _take_landed_results(self, *, wait: bool = False) -> None:
        """Prefill results first: a request's first token (prefill) comes before its second (coda).
        Each kind is waited for when ``wait`` is set or the scheduler has nothing else pending."""

        idle = lambda: wait or not self.scheduler.has_pending_work()
        self._consume_ready_prefill_results(block=idle())
        self._consume_ready_coda_results(block=idle())

    def _resume_decoders(self) -> None:
        """Swapped-out requests whose KV came back, then parked decoders, share one prelude launch
        at the head of the depth queue. Restores run first so that the prefill gate of this tick
        sees them; they already hold the block of their pending token."""

        items = [item for state in self._restore_offloaded_requests()
                 if (item := self.staging.stage(state)) is not None]
        items += self.staging.retry_parked()
        self._prelude_and_enqueue_depth(items, site="resumed", front=True)

    def _pick_batch(self) -> ScheduledCDBBatch | None:
        stats, sched = self.last_stats, self.scheduler
        stats.scheduler_ticks += 1
        in_flight = len(self.pending_coda_results)
        stats.coda_suppressed_ticks += in_flight > 0
        coda_open = in_flight < CODA_PIPELINE_DEPTH
        batch = sched.schedule_next(token_budget=self.cache.max_num_batched_tokens,
                                    cache_budget=self.cache.num_pages, allow_coda=coda_open)
        # Count the ticks where the pipeline bound held back a coda that would have run.
        if not coda_open and sched.coda_queue and (batch is None
                                                    or len(sched.coda_queue) >= sched.min_coda_batch_size):
            stats.coda_pipeline_blocked_ticks += 1
        return batch

    def _unblock(self) -> None:
        if self.pending_prefill_results:
            self._consume_ready_prefill_results(block=True)
        elif self.pending_coda_results:
            self._consume_ready_coda_results(block=True)
        elif self.staging.parked:
            self.staging.yield_one(len(self.scheduler.active_requests))
        else:
            self._raise_scheduler_stall()

    def _launch(self, batch: ScheduledCDBBatch) -> None:
        if batch.kind == "prefill":
            self._run_prefill_batch(batch)
        elif batch.kind == "coda":
            self._stage_coda_batch(batch.depth_items or [])
        else:
            self._run_mixed_recurrent_batch(batch.depth_items or [])

    def _finish_stats(self) -> None:
        s = self.last_stats
        s.scheduler_refills = self.scheduler.refill_events
        s.max_depth_queue_size = self.scheduler.max_depth_queue_size
        s.recurrent_graph_hits = self.runner.recurrent_graph_hits
        s.recurrent_graph_captures = self.runner.recurrent_graph_captures
        s.max_in_flight_requests = self.scheduler.max_in_flight_requests
        s.max_live_requests = self.scheduler.max_live_requests
        assert self.cdb_config.max_recurrent_steps is not None
        s.fixed_depth_recurrent_steps = s.coda_tokens * self.cdb_config.max_recurrent_steps

    # -- prefill (continuous_api.py:995-1088) -------------------------------------------------------------------
    def _run_prefill_batch(self, scheduled: ScheduledCDBBatch) -> None:
        requests = scheduled.requests or []
        if not requests:
            raise RuntimeError("Prefill scheduler tick has no requests")
        stats = self.last_stats
        stats.prefill_batches += 1
        stats.prefill_requests += len(requests)
        stats.prefill_recurrent_steps += scheduled.num_q_tokens * (self.cdb_config.max_recurrent_steps or 0)
        pending = self.runner.stage_prefill_batch(requests, allow_async=self.cdb_config.use_async_batching)
        if self.record_launches:
            self.launch_log.append(self._prefill_event(requests))
        eager_flags: list[bool] = []
        eager_items: list[DepthWorkItem] = []
        eager_rows: list[int] = []
        for future in requests:
            state = future.state
            if not future.has_new_token:
                self.scheduler.release_in_flight_request(state.request_id)
                continue
            stats.prefill_coda_tokens += 1
            eager = False
            if (self.cdb_config.use_async_batching and not state.will_finish_on_pending_token()
                    and self.staging.reserve_row(state)):
                eager = True
                eager_rows.append(len(eager_flags))
                eager_items.append(self.staging.work_item(state, token_id=TMP_TOKEN_ID))
            eager_flags.append(eager)
        pending.eager_entries = eager_flags
        if eager_items:
            self._record_prelude("after_prefill_eager", len(eager_items), gathered=len(eager_items))
            self.runner.compute_prelude_batch(eager_items, device_groups=[(pending, eager_rows)])
            if self.record_launches:
                self.launch_log.append(_prelude_event("after_prefill_eager", eager_items))
            self._enqueue_prelude_items(eager_items, front=False)
        self.pending_prefill_results.append(pending)

    @staticmethod
    def _prefill_event(requests) -> tuple:
        return ("prefill", tuple((f.state.request_id, f.state.position_offset - f.query_length, f.query_length,
                                  f.has_new_token) for f in requests))

    def _recurrent_rows(self, items: list[DepthWorkItem]) -> tuple:
        table = self.cache.block_table
        return tuple((i.state.request_id, i.token_position, i.recurrent_step, i.hidden_slot,
                      tuple(table.get(i.state.request_id, ()))) for i in items)

    def _consume_ready_prefill_results(self, *, block: bool) -> None:
        block = block or self.consume_all_results
        while self.pending_prefill_results:
            pending = self.pending_prefill_results[0]
            if not block and not pending.is_ready():
                return
            self.pending_prefill_results.popleft()
            self._consume_prefill_result(pending)

    def _consume_prefill_result(self, pending: PendingPrefillResult) -> None:
        tokens = self.runner.consume_prefill_result(pending)
        eager = pending.eager_entries or [False] * len(tokens)
        new_items: list[DepthWorkItem] = []
        k = 0
        for future in pending.futures:
            if not future.has_new_token:
                continue
            state = future.state
            token, was_eager = tokens[k], eager[k]
            k += 1
            if state.status == RequestStatus.FINISHED:
                continue
            if was_eager:
                if state.update_and_check_completion(token):
                    self._retire_request(state)
                continue
            if self._advance_after_prefill(state, token):
                continue
            item = self.staging.stage(state)
            if item is not None:
                new_items.append(item)
        self._prelude_and_enqueue_depth(new_items, site="after_prefill")

    # -- recurrent (continuous_api.py:1090-1280) ----------------------------------------------------------------
    def _run_mixed_recurrent_batch(self, items: list[DepthWorkItem]) -> None:
        items = self._drop_cancelled_items(items)
        if not items:
            return
        stats = self.last_stats
        stats.mixed_recurrent_batches += 1
        launch_steps = [item.recurrent_step for item in items]
        depth_counts = Counter(launch_steps)
        stats.max_mixed_depths_per_batch = max(stats.max_mixed_depths_per_batch, len(depth_counts))
        for step, count in depth_counts.items():
            stats.mixed_recurrent_depth_histogram[step] += count
            stats.recurrent_step_histogram[step] += count
        rows = self._recurrent_rows(items) if self.record_launches else None
        flags = self.runner.compute_recurrent_batch(items)
        stats.recurrent_batches += 1
        stats.recurrent_steps += len(items)
        max_steps = self.cdb_config.max_recurrent_steps
        if not self.exit_policy.delayed():
            # Synchronous horizon: this launch's decisions route its rows. The device lists the
            # exiting and the staying rows in launch order; the tick core does the bookkeeping
            # (exit depths, coda list, step advance of the staying rows).
            backlog = self._exit_kv_backlog if self.exit_kv_layout is not None else None
            if flags.lists is not None:
                coda_items, refills, exits = _tick.route_lists(
                    items, flags.routing_lists(), max_steps, stats.exit_depth_histogram, backlog)
            else:
                coda_items, refills, exits = _tick.route_sync(
                    items, flags.wait(), max_steps, stats.exit_depth_histogram, backlog)
            self.scheduler.enqueue_coda_items(coda_items)
            if refills:
                self.scheduler.enqueue_depth_front(refills)
            self._flush_exit_kv_copies()
            if self.record_launches:
                self.launch_log.append(("recurrent", rows, tuple(map(bool, exits)), self.scheduler.refill_events))
            return
        # Delayed horizon: a launch's decisions route the item after its next launch (tick core:
        # the previous launch's flag per row, this launch's flags kept for the survivors).
        coda_items, refills, exits = _tick.route_delayed(
            items, flags, max_steps, self._pending_flags, stats.exit_depth_histogram,
            self._exit_kv_backlog if self.exit_kv_layout is not None else None)
        self.scheduler.enqueue_coda_items(coda_items)
        if refills:
            self.scheduler.enqueue_depth_front(refills)
        self._flush_exit_kv_copies()
        if self.record_launches:
            self.launch_log.append(("recurrent", rows, tuple(map(bool, exits)), self.scheduler.refill_events))

    def _record_exit(self, item: DepthWorkItem, step: int) -> None:
        if item.apply_exit_gate:
            item.state.current_token_exit_depth = step
            item.state.exit_depths.append(step)
            self.last_stats.exit_depth_histogram[step] += 1
        self._pending_flags.pop(id(item), None)
        max_steps = self.cdb_config.max_recurrent_steps or 0
        if self.exit_kv_layout is not None and step < max_steps - 1:
            self._exit_kv_backlog.append((item, step))

    def _flush_exit_kv_copies(self) -> None:
        """Copy each exited token's exit-step KV into its deeper slots before any deeper read."""

        if not self._exit_kv_backlog:
            return
        backlog, self._exit_kv_backlog = self._exit_kv_backlog, []
        rows = [self.cache.token_row(item.state.request_id, item.token_position) for item, _ in backlog]
        steps = [step for _, step in backlog]
        self.runner.copy_exit_kv(rows, steps)
        self.last_stats.exit_kv_copies += len(rows)

    # -- coda (continuous_api.py:1282-1406) ---------------------------------------------------------------------
    def _stage_coda_batch(self, items: list[DepthWorkItem]) -> None:
        items = self._drop_cancelled_items(items)
        if not items:
            return
        use_async = self.cdb_config.use_async_batching
        selected: list[tuple[list[DepthWorkItem], list[int], list[bool]]] = []

        def successors(coda_items: list[DepthWorkItem]) -> tuple[list[DepthWorkItem], list[int]]:
            # Runs once the coda's tokens count as in flight, before the coda launch,
            # so the runner can fuse the successors' prelude into it.
            eager_items, eager_rows, flags = self._select_eager_reentries(coda_items)
            selected.append((eager_items, eager_rows, flags))
            if eager_items:
                self._record_prelude("after_coda_eager", len(eager_items), gathered=len(eager_items))
            return eager_items, eager_rows

        pending = self.runner.stage_coda_batch(items, allow_async=use_async,
                                               successors=successors if use_async else None)
        if self.record_launches:
            self.launch_log.append(("coda", tuple((i.state.request_id, i.token_position, i.hidden_slot)
                                                  for i in items)))
        if use_async:
            eager_items, _, flags = selected[0]
            pending.eager_reentries = flags
            if self.record_launches and eager_items:
                self.launch_log.append(_prelude_event("after_coda_eager", eager_items))
            self._enqueue_prelude_items(eager_items, front=True)
        self.pending_coda_results.append(pending)
        self.last_stats.max_pending_coda_results = max(self.last_stats.max_pending_coda_results,
                                                       len(self.pending_coda_results))

    def _select_eager_reentries(self, coda_items: list[DepthWorkItem]
                                ) -> tuple[list[DepthWorkItem], list[int], list[bool]]:
        """Successors staged ahead of their token (cdb/continuous_api.py:1304-1327): every coda
        row whose request will not finish on the pending token and gets a KV slot."""

        # Per row: skip a request that finishes on its pending token, else advance its position
        # and keep a KV slot for it (its last block, or a new one), then build its successor.
        return _tick.select_eager(coda_items, self.cache.block_size, self.staging.reserve_row,
                                  DepthWorkItem, TMP_TOKEN_ID)

    def _consume_ready_coda_results(self, *, block: bool) -> None:
        block = block or self.consume_all_results
        while self.pending_coda_results:
            pending = self.pending_coda_results[0]
            if not block and not pending.is_ready():
                return
            self.pending_coda_results.popleft()
            self._consume_coda_result(pending)

    def _consume_coda_result(self, pending: PendingCodaResult) -> None:
        """Sampled tokens of a coda batch (cdb/continuous_api.py:1378-1406).

        The tick core walks the rows: finished requests are skipped, eager rows only record
        their token, other rows advance their position first. What is left here is the
        requests that finished (retired) and the non-eager survivors (next token staged),
        in row order."""

        tokens = self.runner.consume_coda_result(pending)
        self.last_stats.coda_batches += 1
        self.last_stats.coda_tokens += len(pending.items)
        new_items: list[DepthWorkItem] = []
        for state, stage in _tick.consume_coda(pending.items, tokens, pending.eager_reentries):
            if not stage:
                self._retire_request(state)
                continue
            new = self.staging.stage(state)
            if new is not None:
                new_items.append(new)
        self._prelude_and_enqueue_depth(new_items, site="after_coda_staged", front=True)

    def _advance_after_coda(self, item: DepthWorkItem, token: int) -> bool:
        state = item.state
        state.position_offset += 1
        finished = state.update_and_check_completion(token)
        if finished:
            self._retire_request(state)
        return finished

    def _advance_after_prefill(self, state: RequestState, token: int) -> bool:
        finished = state.update_and_check_completion(token)
        if finished:
            self._retire_request(state)
        return finished

    def _retire_request(self, state: RequestState) -> None:
        self.scheduler.record_completion(state)
        self.scheduler.finish_request(state.request_id)
        self.staging.forget(state.request_id)
        self.finished_outputs[state.request_id] = state.to_generation_output()
        self.scheduler.block_new_requests = False

    def _drop_cancelled_items(self, items: list[DepthWorkItem]) -> list[DepthWorkItem]:
        live, dead = _tick.split_live(items, RequestStatus.FINISHED)
        if dead:
            self.runner.release_hidden_slots(dead)
            for i in dead:
                self._pending_flags.pop(id(i), None)
            self.last_stats.cancelled_depth_items += len(dead)
        return live

    # -- decode-token staging (continuous_api.py:1530-1669) -----------------------------------------------------
    def _record_prelude(self, site: str, count: int, *, gathered: int = 0) -> None:
        self.last_stats.prelude_batches[site] += 1
        self.last_stats.prelude_tokens[site] += count
        if gathered:
            self.last_stats.prelude_gathered_tokens[site] += gathered

    def _prelude_and_enqueue_depth(self, items: list[DepthWorkItem], *, site: str, front: bool = False) -> None:
        if items:
            self._record_prelude(site, len(items))
            self.runner.compute_prelude_batch(items)
            if self.record_launches:
                self.launch_log.append(_prelude_event(site, items))
        self._enqueue_prelude_items(items, front=front)

    def _enqueue_prelude_items(self, items: list[DepthWorkItem], *, front: bool) -> None:
        if front:
            self.scheduler.enqueue_depth_front(items)
        else:
            for item in items:
                self.scheduler.enqueue_depth(item)

    def _restore_offloaded_requests(self) -> list[RequestState]:
        """Re-admit swapped-out requests and copy their KV back before any launch reads it
        (continuous_api.py:1490-1505)."""

        if not self.offloading_manager.offloading_enabled:
            return []
        restored = self.scheduler.admit_offloaded_restores()
        if restored:
            self.offloading_manager.restore_scheduled_requests(restored)
        return restored

    def _raise_scheduler_stall(self) -> None:
        """A tick with no bucket, no staged result and no parked decoder: nothing will change, so
        the leading prefill candidate names the cause (cdb/continuous_api.py:1450-1488)."""

        waiting = self.scheduler.get_prefill_bucket()
        if not waiting:
            raise CacheFullError("scheduler dead end: no bucket, nothing in flight and no prompt waiting")
        head = waiting[0]
        chunk = min(len(head.remaining_prefill_tokens), self.cache.max_num_batched_tokens)
        blocks = self.cache.block_size
        missing = (head.current_len() + chunk + blocks - 1) // blocks - head.allocated_blocks
        if not self.cache.will_allocation_be_successful(missing, head.allocated_blocks):
            raise CacheFullError(f"prompt chunk of request {head.request_id} does not fit: it needs {missing} more "
                                 f"KV blocks and {self.cache.get_num_free_blocks()} are free, with no decoding "
                                 "request left to free any")
        raise RuntimeError(f"request {head.request_id} cannot be scheduled: its {head.current_len()} KV tokens "
                           f"exceed the cache budget of {self.cache.num_pages} tokens")

    # -- no-refill baseline (continuous_api.py:608-944) ---------------------------------------------------------
    def _run_no_refill_loop(self) -> None:
        """Sequence-level baseline: each iteration prefills while admission allows, then runs one
        lockstep wave over every decoder whose token is sampled; rows that exit are not refilled.

        On the delayed horizon nothing in the loop waits for a readback: a prefill's first tokens
        and a wave's coda stay staged, their successors are built ahead of the tokens, and the next
        wave's one prelude gathers those tokens on the device. The coda is read after that wave's
        first launch, so a finish it reveals cancels the successor then."""

        sched = self.scheduler
        carry = _WaveCarry()
        while sched.has_pending_work():
            prefills, carry.prefills = carry.prefills, []
            for pending in prefills:
                self._apply_wave_prefill(pending)
            # Restored requests decode again, so they join this wave's cohort scan.
            self._restore_offloaded_requests()
            sched.record_resident_sample()
            did_prefill = False
            while sched.prefill_admitted():
                scheduled = sched.schedule_prefill_batch(token_budget=self.cache.max_num_batched_tokens,
                                                         cache_budget=self.cache.num_pages)
                if scheduled is None or not scheduled.requests:
                    break
                self._run_no_refill_prefill(scheduled, carry)
                did_prefill = True
            if self._run_wave(carry) or did_prefill:
                continue
            if self.staging.parked:
                # No wave can run and no parked decoder can allocate: take one's KV away.
                self.staging.yield_one(len(sched.active_requests))
                continue
            if sched.has_pending_work():
                raise CacheFullError("no-refill wave dead end: no waiting prompt fits the KV cache "
                                     "and no decode token is ready")
        if not carry.empty():
            raise RuntimeError("no-refill loop ended with staged work still carried: its requests would "
                               "have counted as pending")
        self._finish_stats()

    def _run_no_refill_prefill(self, scheduled: ScheduledCDBBatch, carry: _WaveCarry) -> None:
        requests = scheduled.requests or []
        stats = self.last_stats
        stats.prefill_batches += 1
        stats.prefill_requests += len(requests)
        stats.prefill_recurrent_steps += scheduled.num_q_tokens * (self.cdb_config.max_recurrent_steps or 0)
        delayed = self.exit_policy.delayed()
        pending = self.runner.stage_prefill_batch(requests, allow_async=self.cdb_config.use_async_batching)
        if self.record_launches:
            self.launch_log.append(self._prefill_event(requests))
        # Successors that enter this iteration's wave ahead of their token, within the launch
        # width the carried successors leave.
        room = max(0, self.cdb_config.max_num_seqs - carry.num_items())
        flags: list[bool] = []
        ahead: list[DepthWorkItem] = []
        rows: list[int] = []
        for future in requests:
            state = future.state
            if future.has_new_token:
                stats.prefill_coda_tokens += 1
                enter = (delayed and len(ahead) < room and not state.will_finish_on_pending_token()
                         and self.staging.reserve_row(state))
                if enter:
                    rows.append(len(flags))
                    ahead.append(self.staging.work_item(state, token_id=TMP_TOKEN_ID))
                flags.append(enter)
            self.scheduler.release_in_flight_request(state.request_id)
        pending.eager_entries = flags
        if not delayed:
            self._apply_wave_prefill(pending)
            return
        if ahead:
            carry.groups.append((pending, ahead, rows))
        carry.prefills.append(pending)

    def _apply_wave_prefill(self, pending: PendingPrefillResult) -> None:
        """A prefill's first tokens. The wave's cohort scan stages the next token, so this only
        records each token; a successor that already entered a wave is cancelled by a finish."""

        tokens = self.runner.consume_prefill_result(pending)
        entered = pending.eager_entries or [False] * len(tokens)
        sampled = (f.state for f in pending.futures if f.has_new_token)
        for state, token, _ in zip(sampled, tokens, entered, strict=True):
            if state.status != RequestStatus.FINISHED and state.update_and_check_completion(token):
                self._retire_request(state)

    def _apply_wave_coda(self, pending: PendingCodaResult) -> None:
        tokens = self.runner.consume_coda_result(pending)
        self.last_stats.coda_batches += 1
        self.last_stats.coda_tokens += len(pending.items)
        ahead = pending.eager_reentries or [False] * len(tokens)
        for item, token, entered in zip(pending.items, tokens, ahead, strict=True):
            state = item.state
            if state.status == RequestStatus.FINISHED:
                continue
            if not entered:
                self._advance_after_coda(item, token)
            elif state.update_and_check_completion(token):
                self._retire_request(state)

    def _run_wave(self, carry: _WaveCarry) -> bool:
        """One lockstep wave; returns whether it did any work (a launch, or reading a carried coda)."""

        sched = self.scheduler
        stats = self.last_stats
        groups, coda = carry.groups, carry.coda
        carry.groups, carry.coda = [], None
        # A request retired since its successor was built (a first token read at the top of this
        # iteration) loses that successor; it never took a hidden slot.
        live_groups = []
        for result, items, rows in groups:
            keep = [(i, r) for i, r in zip(items, rows) if i.state.status != RequestStatus.FINISHED]
            stats.cancelled_depth_items += len(items) - len(keep)
            if keep:
                live_groups.append((result, [i for i, _ in keep], [r for _, r in keep]))
        carried = [item for _, items, _ in live_groups for item in items]
        # Requests whose coda is still unread hold a token one wave behind: not scanned now.
        behind = {i.state.request_id for i in coda.items} if coda is not None else set()
        cohort = [s for s in sched.active_requests.values()
                  if s.status == RequestStatus.DECODING and s.tokens_to_process and s.tokens_to_process[0] >= 0
                  and s.request_id not in behind]
        cohort = cohort[: max(0, self.cdb_config.max_num_seqs - len(carried))]
        items = carried + [item for s in cohort if (item := self.staging.stage(s)) is not None]
        if not items:
            if coda is None:
                return False
            self._apply_wave_coda(coda)
            return True
        self._record_prelude("wave_cohort", len(items), gathered=len(carried))
        self.runner.compute_prelude_batch(items, device_groups=[(result, rows) for result, _, rows in live_groups])
        if self.record_launches:
            self.launch_log.append(_prelude_event("wave_cohort", items))
        max_steps = self.cdb_config.max_recurrent_steps or 0
        # On the delayed horizon a launch's decisions route the item after its next launch,
        # exactly as in the refill loop.
        delayed = self.exit_policy.delayed()
        previous: dict[int, tuple[PendingFlags, int]] = {}
        survivors = items
        exited: list[DepthWorkItem] = []
        for step in range(max_steps):
            for item in survivors:
                item.recurrent_step = step
            rows = self._recurrent_rows(survivors) if self.record_launches else None
            flags = self.runner.compute_recurrent_batch(survivors)
            stats.recurrent_batches += 1
            stats.recurrent_steps += len(survivors)
            stats.recurrent_step_histogram[step] += len(survivors)
            if coda is not None:
                # Read while the wave's first launch runs; a finish it reveals cancels below.
                self._apply_wave_coda(coda)
                coda = None
            continuing, cancelled, exits = [], [], []
            for idx, item in enumerate(survivors):
                if item.state.status == RequestStatus.FINISHED:
                    cancelled.append(item)
                    previous.pop(id(item), None)
                    exits.append(False)
                    continue
                if delayed:
                    prev = previous.pop(id(item), None)
                    gate_exit = item.apply_exit_gate and prev is not None and prev[0].get(prev[1])
                else:
                    gate_exit = item.apply_exit_gate and flags.get(idx)
                leave = step == max_steps - 1 or bool(gate_exit)
                exits.append(leave)
                if leave:
                    self._record_exit(item, step)
                    exited.append(item)
                else:
                    continuing.append(item)
                    if delayed:
                        previous[id(item)] = (flags, idx)
            if cancelled:
                self.runner.release_hidden_slots(cancelled)
                stats.cancelled_depth_items += len(cancelled)
            self._flush_exit_kv_copies()
            if self.record_launches:
                self.launch_log.append(("recurrent", rows, tuple(map(bool, exits)), sched.refill_events))
            survivors = continuing
            if not survivors:
                break
        if not exited:
            return True
        pending = self.runner.stage_coda_batch(exited, allow_async=delayed)
        if self.record_launches:
            self.launch_log.append(("coda", tuple((i.state.request_id, i.token_position, i.hidden_slot)
                                                  for i in exited)))
        if not delayed:
            self._apply_wave_coda(pending)
            return True
        # Successors of the exited rows enter the next wave ahead of their tokens.
        ahead, rows, flags = self._select_eager_reentries(exited)
        pending.eager_reentries = flags
        if ahead:
            carry.groups.append((pending, ahead, rows))
        carry.coda = pending
        return True

    # -- validation (continuous_api.py:1746-1833) ---------------------------------------------------------------
    @staticmethod
    def _validate_generate_inputs(input_ids: list[list[int]], max_new_tokens: int | list[int]) -> None:
        if not input_ids:
            raise ValueError("input_ids must contain at least one prompt")
        if isinstance(max_new_tokens, list):
            if len(max_new_tokens) != len(input_ids):
                raise ValueError(f"max_new_tokens has {len(max_new_tokens)} entries but there are "
                                 f"{len(input_ids)} prompts")
            bad = [i for i, v in enumerate(max_new_tokens) if v < 1]
            if bad:
                raise ValueError(f"max_new_tokens must be >= 1 for every request, but got <1 at indices {bad}")
        elif max_new_tokens <= 0:
            raise ValueError(f"max_new_tokens must be positive, but got {max_new_tokens}")
        empty = [i for i, p in enumerate(input_ids) if not p]
        if empty:
            raise ValueError(f"input_ids contains empty prompts at indices {empty}")

    def _cap_to_model_len(self, input_ids: list[list[int]], mnt: list[int]) -> list[int]:
        limit = self.cdb_config.max_model_len
        too_long = [i for i, p in enumerate(input_ids) if len(p) >= limit]
        if too_long:
            raise ValueError(f"{len(too_long)} prompt(s) have length >= max_model_len ({limit}) and leave no room "
                             f"for a generated token: requests {too_long[:5]}")
        return [min(m, limit - len(p)) for m, p in zip(mnt, input_ids)]

    def _validate_model_kwargs(self, model_kwargs: dict | None) -> None:
        if (self.cdb_config.exit_threshold is not None and model_kwargs is not None
                and model_kwargs.get("use_early_exit_gate") is False):
            raise ValueError("exit_threshold CDB requires use_early_exit_gate to stay enabled")

    def _validate_exit_depths(self, input_ids: list[list[int]], mnt: list[int],
                              exit_depths: list[list[int]] | None) -> None:
        if exit_depths is None:
            return
        cfg = self.cdb_config
        if not cfg.synthetic_exit_replay:
            raise ValueError("exit_depths requires cdb_config.synthetic_exit_replay=True")
        if cfg.exit_threshold is not None:
            raise ValueError("exit_depths cannot be combined with exit_threshold")
        if len(exit_depths) != len(input_ids):
            raise ValueError(f"exit_depths has {len(exit_depths)} entries but there are {len(input_ids)} requests")
        max_steps = cfg.max_recurrent_steps or 0
        for i, depths in enumerate(exit_depths):
            if len(depths) != mnt[i] - 1:
                raise ValueError(f"exit_depths[{i}] has {len(depths)} entries but the request stages "
                                 f"{mnt[i] - 1} decode tokens (max_new_tokens - 1)")
            for d in depths:
                if not 0 <= d < max_steps:
                    raise ValueError(f"exit_depths[{i}] value {d} is out of range [0, {max_steps}); values are "
                                     "0-based recurrent steps")
        if copies_exit_kv(cfg.kv_policy):
            return
        slots = resolve_kv_slots_per_layer(cfg.kv_policy, total_recurrent_steps=max_steps,
                                           requested_slots=cfg.kv_slots_per_layer)
        extra = int(cfg.delay_gate_consumption and cfg.use_async_batching)
        for depths in exit_depths:
            for d in depths:
                if d + 1 + extra < slots:
                    raise ValueError("Every replay exit depth must write all static KV slots before exit: "
                                     f"kv_slots_per_layer={slots}, exit step {d + 1 + extra}")


__all__ = ["ContinuousDepthBatchingEngine", "ContinuousDepthBatchingStats", "CacheFullError",
           "PendingFlags", "time"]
