"""The scheduler's per-tick decisions in the tick core against the Python they replace.

``_tick.schedule_next`` and the admission functions beside it (csrc/tick.cpp)
take over ``CDBScheduler``'s bucket choice, prompt admission, chunking and
block allocation (continuous_depth_batching/scheduler.py:101-140, 205-296;
continuous_batching/scheduler_base.py:171-201, 416-545). ``PythonScheduler``
below keeps the per-request Python those functions replace. Twin schedulers over
twin caches run the same seeded sequence of arrivals, depth and coda work,
ticks, prefill completions, decode-token allocations and finishes; every
returned batch and every piece of scheduler, request and cache state must agree
after every operation, under each pressure mode.
"""

from __future__ import annotations

import random
from collections import deque
from itertools import islice

import pytest

from continuous_depth_batching_amd.requests import DepthWorkItem, FutureRequestState, RequestState, RequestStatus
from continuous_depth_batching_amd.scheduler import CDBScheduler, ScheduledCDBBatch, reserved_peak_blocks
from tests.host_runner import make_engine


class PythonScheduler(CDBScheduler):
    """CDBScheduler with the tick-core calls replaced by the per-request Python."""

    def record_resident_sample(self) -> None:
        resident = len(self.active_requests)
        self.max_resident_requests = max(self.max_resident_requests, resident)
        self.resident_samples += 1
        self.resident_sum += resident
        self._advance_steady_window(resident)

    def has_decode_work(self) -> bool:
        return any(s.status == RequestStatus.DECODING for s in self.active_requests.values())

    def has_prefill_headroom(self) -> bool:
        return self.cache.get_num_free_blocks() > self.safety_margin * self.cache.num_blocks

    def prefill_admitted(self) -> bool:
        return not self.has_decode_work() or self.has_prefill_headroom()

    def admit_prefill_batch(self, candidates: list[RequestState]) -> bool:
        if not candidates:
            return False
        if any(s.status == RequestStatus.PREFILLING for s in candidates):
            return True
        return self.free_residency_slots() >= self.min_free_slots

    def _get_waiting_candidates(self, limit: int) -> list[RequestState]:
        fresh = (self.waiting_requests[r] for r in self.waiting_requests_order
                 if not self.waiting_requests[r].is_cpu_offloaded)
        return list(islice(fresh, limit))

    def get_prefill_bucket(self) -> list[RequestState]:
        prefilling = [s for s in self.active_requests.values()
                      if s.status == RequestStatus.PREFILLING and s.request_id not in self.in_flight_request_ids]
        if self.block_new_requests:
            return prefilling
        admissible = self._get_waiting_candidates(limit=self.free_residency_slots())
        if self.kv_pressure_mode == "reserve":
            committed = sum(reserved_peak_blocks(len(s.initial_tokens), s.max_new_tokens, self.max_model_len,
                                                 self.cache.block_size) for s in self.active_requests.values())
            fitting = []
            for s in admissible:
                need = reserved_peak_blocks(len(s.initial_tokens), s.max_new_tokens, self.max_model_len,
                                            self.cache.block_size)
                if committed + need > self.cache.num_blocks:
                    break
                committed += need
                fitting.append(s)
            admissible = fitting
        return prefilling + admissible

    def _cleanup_waiting_queue(self, ids: set[str]) -> None:
        remaining = set(ids)
        order = self.waiting_requests_order
        while remaining and order and order[0] in remaining:
            remaining.discard(order.popleft())
        if remaining:
            self.waiting_requests_order = deque(r for r in order if r not in remaining)

    def _allocate_blocks_if_needed(self, state: RequestState, len_next_tokens: int) -> bool:
        current = state.current_len()
        if state.allocated_blocks * self.cache.block_size - current < len_next_tokens:
            needed = -(-(current + len_next_tokens) // self.cache.block_size) - state.allocated_blocks
            got = self.cache.allocate_blocks(needed, state.request_id, state.allocated_blocks)
            if got is None:
                return False
            state.allocated_blocks += got
        return True

    def schedule_next(self, token_budget: int, cache_budget: int, *, allow_coda: bool = True):
        self.record_resident_sample()
        if allow_coda and len(self.coda_queue) >= self.min_coda_batch_size:
            batch = self._pop_coda()
            if batch:
                return ScheduledCDBBatch(kind="coda", depth_items=batch)
        if self.prefill_admitted():
            prefill = self.schedule_prefill_batch(token_budget, cache_budget)
            if prefill is not None:
                return prefill
        size = min(self.max_num_seqs, len(self.ready_queue))
        if size:
            from continuous_depth_batching_amd import _tick

            recurrent = _tick.pop_batch(self.ready_queue, size, self._slot_of_step)
            self.mixed_batches_scheduled += 1
            if recurrent:
                return ScheduledCDBBatch(kind="recurrent", depth_items=recurrent)
        if allow_coda:
            batch = self._pop_coda()
            if batch:
                return ScheduledCDBBatch(kind="coda", depth_items=batch)
        return None

    def _pop_coda(self) -> list[DepthWorkItem]:
        n = min(self.max_num_seqs, len(self.coda_queue))
        return [self.coda_queue.popleft() for _ in range(n)]

    def schedule_prefill_batch(self, token_budget: int, cache_budget: int):
        candidates = self.get_prefill_bucket()
        if not self.admit_prefill_batch(candidates):
            return None
        to_remove: set[str] = set()
        scheduled, num_q_tokens, max_kv_read = self._process_prefill_candidates(candidates, token_budget,
                                                                                cache_budget, to_remove)
        self._cleanup_waiting_queue(to_remove)
        if not scheduled:
            return None
        return ScheduledCDBBatch(kind="prefill", requests=scheduled, num_q_tokens=num_q_tokens,
                                 max_kv_read=max_kv_read)

    def _process_prefill_candidates(self, candidates, token_budget, cache_budget, to_remove):
        scheduled = []
        decode_fast_path = True
        margin_blocks = self.safety_margin * self.cache.num_blocks
        original_tokens, original_cache = token_budget, cache_budget
        for state in candidates:
            free = self.cache.get_num_free_blocks()
            if free < margin_blocks and scheduled:
                break
            tokens = state.remaining_prefill_tokens
            request_len = min(len(tokens), token_budget)
            if request_len == 0:
                continue
            eligible = request_len == 1 and state.position_offset < self.max_decode_fast_path_length
            read_needed = state.current_len()
            if not (decode_fast_path and eligible) and cache_budget < read_needed:
                continue
            if not self._allocate_blocks_if_needed(state, request_len):
                if free == 0 and state.request_id in self.waiting_requests:
                    break
                continue
            self._schedule_prefill_request(state, tokens, request_len, to_remove)
            self._mark_request_in_flight(state.request_id)
            request_len = len(state.tokens_to_process)
            decode_fast_path &= request_len == 1 and state.position_offset < self.max_decode_fast_path_length
            token_budget -= request_len
            cache_budget -= read_needed
            scheduled.append(FutureRequestState(state, not state.remaining_prefill_tokens, request_len))
            if self.waiting_requests.pop(state.request_id, None) is not None:
                to_remove.add(state.request_id)
            if token_budget == 0 or (cache_budget <= 0 and not decode_fast_path):
                break
        return scheduled, original_tokens - token_budget, original_cache - cache_budget

    def _schedule_prefill_request(self, state, tokens, request_len, to_remove) -> None:
        if len(tokens) <= request_len:
            if state.status == RequestStatus.PENDING:
                self.active_requests[state.request_id] = state
                to_remove.add(state.request_id)
            if state.status <= RequestStatus.PREFILLING:
                state.tokens_to_process = state.remaining_prefill_tokens
                state.remaining_prefill_tokens = []
                state.status = RequestStatus.DECODING
            return
        if state.status == RequestStatus.PENDING:
            self.active_requests[state.request_id] = state
            state.status = RequestStatus.PREFILLING
            to_remove.add(state.request_id)
        state.remaining_prefill_tokens = tokens[request_len:]
        state.tokens_to_process = tokens[:request_len]


def _batch_view(batch):
    if batch is None:
        return None
    return (batch.kind, batch.num_q_tokens, batch.max_kv_read,
            None if batch.requests is None else [(f.state.request_id, f.has_new_token, f.query_length)
                                                 for f in batch.requests],
            None if batch.depth_items is None else [(i.state.request_id, i.token_id, i.recurrent_step)
                                                    for i in batch.depth_items])


def _state_view(s: RequestState):
    return (s.request_id, int(s.status), list(s.tokens_to_process), list(s.remaining_prefill_tokens),
            s.position_offset, s.allocated_blocks, s.lifespan[0] >= 0, s.is_cpu_offloaded)


def _scheduler_view(sched: CDBScheduler):
    counters = ("mixed_batches_scheduled", "refill_events", "max_depth_queue_size", "max_in_flight_requests",
                "max_live_requests", "max_resident_requests", "resident_samples", "resident_sum",
                "completed_requests", "_steady_ticks", "_steady_resident_sum", "block_new_requests")
    cache = sched.cache
    return ([_state_view(s) for s in sched.active_requests.values()],
            [_state_view(s) for s in sched.waiting_requests.values()],
            list(sched.waiting_requests_order), sorted(sched.in_flight_request_ids),
            [(i.state.request_id, i.token_id, i.recurrent_step) for i in sched.ready_queue],
            [(i.state.request_id, i.token_id, i.recurrent_step) for i in sched.coda_queue],
            [getattr(sched, c) for c in counters], sched._steady_start_time is None,
            cache._block_manager.free_list(), {k: list(v) for k, v in cache.block_table.items()},
            dict(cache.table_row_of))


class Twin:
    """The same operation applied to the tick-core scheduler and to the Python one."""

    def __init__(self, rng: random.Random, mode: str, margin: float, max_num_seqs: int, min_coda: int,
                 num_blocks: int) -> None:
        self.rng = rng
        self.pair = []
        for cls in (CDBScheduler, PythonScheduler):
            engine = make_engine(num_blocks=num_blocks, block_size=4, max_num_batched_tokens=16, max_model_len=64,
                                 max_num_seqs=max_num_seqs)
            self.pair.append(cls(engine.cache, 3, safety_margin=margin, kv_pressure_mode=mode,
                                 max_model_len=64, max_num_seqs=max_num_seqs, min_coda_batch_size=min_coda))
        self.states: list[dict[str, RequestState]] = [{}, {}]
        self.next_id = 0

    def check(self, what: str) -> None:
        a, b = (_scheduler_view(s) for s in self.pair)
        assert a == b, what

    def arrive(self, offloaded: bool) -> None:
        rid = f"r{self.next_id}"
        self.next_id += 1
        prompt = [self.rng.randrange(100) for _ in range(self.rng.randint(1, 20))]
        mnt = self.rng.choice([None, 1, 4, 12, 40])
        for sched, states in zip(self.pair, self.states):
            state = RequestState(request_id=rid, initial_tokens=list(prompt), max_new_tokens=mnt)
            state.is_cpu_offloaded = offloaded
            states[rid] = state
            sched.add_waiting_request(state)

    def tick(self) -> None:
        budget = self.rng.choice([1, 3, 8, 16, 1000])
        reads = self.rng.choice([0, 2, 10, 40, 10_000])
        allow = self.rng.random() < 0.8
        got = [_batch_view(s.schedule_next(budget, reads, allow_coda=allow)) for s in self.pair]
        assert got[0] == got[1], (budget, reads, allow)
        view = got[0]
        if view is not None and view[0] == "prefill":
            # What the engine does once a prefill launch is consumed: the chunk is in the KV cache.
            for sched, states in zip(self.pair, self.states):
                for rid, _, q_len in view[3]:
                    states[rid].position_offset += q_len
                    sched.release_in_flight_request(rid)

    def decode_token(self) -> None:
        decoding = sorted(r for r, s in self.states[0].items() if s.status == RequestStatus.DECODING
                          and r in self.pair[0].active_requests)
        if not decoding:
            return
        rid = self.rng.choice(decoding)
        got = []
        for sched, states in zip(self.pair, self.states):
            ok = sched._allocate_blocks_if_needed(states[rid], 1)
            if ok:
                states[rid].position_offset += 1
            got.append(ok)
        assert got[0] == got[1]

    def enqueue(self, coda: bool) -> None:
        active = sorted(self.pair[0].active_requests)
        if not active:
            return
        rid = self.rng.choice(active)
        step, token = self.rng.randrange(3), self.rng.randrange(100)
        for sched, states in zip(self.pair, self.states):
            item = DepthWorkItem(state=states[rid], token_id=token, token_position=0, recurrent_step=step)
            if coda:
                sched.enqueue_coda(item)
            else:
                sched.enqueue_depth(item)

    def finish(self) -> None:
        live = sorted(set(self.pair[0].active_requests) | set(self.pair[0].waiting_requests))
        if not live:
            return
        rid = self.rng.choice(live)
        for sched, states in zip(self.pair, self.states):
            sched.record_completion(states[rid])
            sched.finish_request(rid)

    def release(self) -> None:
        ids = sorted(self.pair[0].in_flight_request_ids)
        if ids:
            rid = self.rng.choice(ids)
            for sched in self.pair:
                sched.release_in_flight_request(rid)

    def toggle_block(self) -> None:
        flag = self.rng.random() < 0.3
        for sched in self.pair:
            sched.block_new_requests = flag


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("mode", ["recompute", "reserve", "offload"])
def test_schedule_next_matches_the_python_scheduler(seed: int, mode: str) -> None:
    rng = random.Random(1000 * seed + len(mode))
    twin = Twin(rng, mode, margin=rng.choice([0.0, 0.2, 0.5]), max_num_seqs=rng.choice([1, 2, 3, 5]),
                min_coda=rng.choice([1, 2, 3]), num_blocks=rng.choice([16, 24, 64] if mode == "reserve" else [8, 24, 64]))
    if seed % 3 == 0:
        for sched in twin.pair:
            sched.steady_warmup_requests = 2
    ops = ["arrive"] * 3 + ["tick"] * 6 + ["decode"] * 3 + ["depth", "coda", "coda", "finish", "release", "block"]
    for step in range(300):
        op = rng.choice(ops)
        if op == "arrive":
            twin.arrive(offloaded=mode == "offload" and rng.random() < 0.25)
        elif op == "tick":
            twin.tick()
        elif op == "decode":
            twin.decode_token()
        elif op in ("depth", "coda"):
            twin.enqueue(coda=op == "coda")
        elif op == "finish":
            twin.finish()
        elif op == "release":
            twin.release()
        else:
            twin.toggle_block()
        twin.check(f"step {step}: {op}")
        if op != "tick":
            continue
        for a, b in ((twin.pair[0].get_prefill_bucket(), twin.pair[1].get_prefill_bucket()),):
            assert [s.request_id for s in a] == [s.request_id for s in b]
        assert twin.pair[0].prefill_admitted() == twin.pair[1].prefill_admitted()


def test_tick_core_scheduler_errors() -> None:
    from continuous_depth_batching_amd import _tick

    engine = make_engine()
    sched = CDBScheduler(engine.cache, 3, max_num_seqs=2)
    sched.waiting_requests_order.append("ghost")  # an id with no waiting request
    with pytest.raises(KeyError):
        sched.get_prefill_bucket()
    sched.waiting_requests_order.clear()
    sched.ready_queue = deque()  # the queues must be the tick core's ItemQueue
    with pytest.raises(TypeError):
        sched.schedule_next(4, 4)
    with pytest.raises(AttributeError):
        _tick.schedule_next(object(), 4, 4, True)
