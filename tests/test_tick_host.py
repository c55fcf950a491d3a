"""The host tick core (``_tick``, csrc/tick.cpp) against the per-row Python it replaces.

``route_sync`` must route a launch's rows exactly as the engine's synchronous
horizon does (cdb/continuous_api.py:1090-1223): exits in row order to the coda
list with their exit bookkeeping, the rest stepped on in row order.
``fill_recurrent`` must write the launch metadata the runner documents
(cdb/model_runner.py:704-754), padding rows included.
"""

from __future__ import annotations

import random
from collections import Counter

import numpy as np
import pytest

from continuous_depth_batching_amd import _tick
from continuous_depth_batching_amd.model_runner import ModelRunner
from continuous_depth_batching_amd.requests import DepthWorkItem, RequestState, RequestStatus

M = ModelRunner


def _items(rng: random.Random, n: int, max_steps: int) -> list[DepthWorkItem]:
    items = []
    for i in range(n):
        state = RequestState(request_id=f"r{i}", initial_tokens=[1])
        items.append(DepthWorkItem(state=state, token_id=rng.randrange(100), token_position=rng.randrange(5000),
                                   recurrent_step=rng.randrange(max_steps),
                                   synthetic_exit_depth=rng.choice([None, 0, 1, 2, 3]),
                                   apply_exit_gate=rng.random() < 0.8, hidden_slot=rng.randrange(1000)))
    return items


def _route_python(items, flags, max_steps, hist, backlog):
    coda, refills, exits = [], [], []
    for idx, item in enumerate(items):
        step = item.recurrent_step
        leave = bool(flags[idx]) if item.apply_exit_gate else step == max_steps - 1
        exits.append(leave)
        if leave:
            if item.apply_exit_gate:
                item.state.current_token_exit_depth = step
                item.state.exit_depths.append(step)
                hist[step] += 1
            if backlog is not None and step < max_steps - 1:
                backlog.append((item, step))
            coda.append(item)
        else:
            item.recurrent_step = step + 1
            refills.append(item)
    return coda, refills, exits


def _snapshot(items):
    return [(i.recurrent_step, i.state.current_token_exit_depth, list(i.state.exit_depths)) for i in items]


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("with_backlog", [False, True])
def test_route_sync_matches_the_per_row_routing(seed: int, with_backlog: bool) -> None:
    rng = random.Random(seed)
    max_steps = 4
    n = rng.randrange(1, 60)
    items_a = _items(random.Random(seed + 100), n, max_steps)
    items_b = _items(random.Random(seed + 100), n, max_steps)
    flags = np.zeros(n + 7, dtype=np.uint8)  # padding rows past n are ignored
    flags[:n] = [rng.random() < 0.4 for _ in range(n)]
    flags[n:] = 1
    hist_a, hist_b = Counter({1: 5}), Counter({1: 5})
    back_a = [] if with_backlog else None
    back_b = [] if with_backlog else None
    coda_a, refills_a, exits_a = _tick.route_sync(items_a, flags, max_steps, hist_a, back_a)
    coda_b, refills_b, exits_b = _route_python(items_b, flags, max_steps, hist_b, back_b)
    idx = {id(it): k for k, it in enumerate(items_a)}
    idx_b = {id(it): k for k, it in enumerate(items_b)}
    assert [idx[id(i)] for i in coda_a] == [idx_b[id(i)] for i in coda_b]
    assert [idx[id(i)] for i in refills_a] == [idx_b[id(i)] for i in refills_b]
    assert exits_a == exits_b and all(type(e) is bool for e in exits_a)
    assert hist_a == hist_b
    assert _snapshot(items_a) == _snapshot(items_b)
    if with_backlog:
        assert [(idx[id(i)], s) for i, s in back_a] == [(idx_b[id(i)], s) for i, s in back_b]


def _compact_python(flags: np.ndarray, slots: np.ndarray) -> np.ndarray:
    """cdb_route_compact restated: [n_exit, n_stay, exiting rows, staying rows], padding skipped."""

    live = np.nonzero(slots >= 0)[0]
    exit_rows = [int(r) for r in live if flags[r]]
    stay_rows = [int(r) for r in live if not flags[r]]
    return np.array([len(exit_rows), len(stay_rows)] + exit_rows + stay_rows, dtype=np.int32)


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("with_backlog", [False, True])
def test_route_lists_equals_route_sync(seed: int, with_backlog: bool) -> None:
    """Routing from the device's lists (exiting rows, then staying rows, each in launch order)
    gives route_sync's coda list, refills, exit flags, histogram, backlog and item state."""

    rng = random.Random(seed)
    max_steps = 4
    n = rng.randrange(1, 60)
    items_a = _items(random.Random(seed + 200), n, max_steps)
    items_b = _items(random.Random(seed + 200), n, max_steps)
    for it in items_a + items_b:
        it.apply_exit_gate = True  # the device lists carry the gate's decisions
    rows = n + rng.randrange(0, 9)
    flags = np.zeros(rows, dtype=np.uint8)
    flags[:n] = [rng.random() < 0.4 for _ in range(n)]
    flags[n:] = 1  # padding rows, skipped by their negative bank slot
    slots = np.full(rows, -1, np.int64)
    slots[:n] = np.arange(n)
    lists = _compact_python(flags, slots)
    hist_a, hist_b = Counter({2: 1}), Counter({2: 1})
    back_a = [] if with_backlog else None
    back_b = [] if with_backlog else None
    got = _tick.route_lists(items_a, lists, max_steps, hist_a, back_a)
    want = _tick.route_sync(items_b, flags, max_steps, hist_b, back_b)
    idx = {id(it): k for k, it in enumerate(items_a)}
    idx_b = {id(it): k for k, it in enumerate(items_b)}
    for a, b in zip(got[:2], want[:2]):
        assert [idx[id(i)] for i in a] == [idx_b[id(i)] for i in b]
    assert got[2] == want[2] and all(type(e) is bool for e in got[2])
    assert hist_a == hist_b and _snapshot(items_a) == _snapshot(items_b)
    if with_backlog:
        assert [(idx[id(i)], s) for i, s in back_a] == [(idx_b[id(i)], s) for i, s in back_b]


def test_route_lists_rejects_lists_that_are_not_a_launch_order_partition() -> None:
    items = _items(random.Random(1), 5, 4)
    for it in items:
        it.apply_exit_gate = True
    # wrong total, an exit list out of order, a repeated stay, a row in both lists, a row past the launch
    for bad in ([2, 2, 0, 3, 1, 2], [2, 3, 3, 0, 1, 2, 4], [1, 4, 0, 1, 2, 3, 3], [2, 3, 0, 1, 1, 3, 4],
                [2, 3, 0, 5, 1, 2, 3]):
        with pytest.raises(ValueError, match="partition"):
            _tick.route_lists(items, np.array(bad, np.int32), 4, Counter(), None)
    items[3].apply_exit_gate = False
    with pytest.raises(ValueError, match="apply the exit gate"):
        _tick.route_lists(items, np.array([2, 3, 1, 3, 0, 2, 4], np.int32), 4, Counter(), None)


def test_route_sync_rejects_short_flags_and_bad_backlog() -> None:
    items = _items(random.Random(0), 4, 4)
    with pytest.raises(ValueError, match="fewer exit flags"):
        _tick.route_sync(items, np.zeros(3, np.uint8), 4, Counter(), None)
    with pytest.raises(TypeError):
        _tick.route_sync(items, np.zeros(4, np.uint8), 4, Counter(), ())


def _fill_python(items, i64, i32, row_of, base, core, slot_of_step):
    n = len(items)
    i64[:n] = [it.hidden_slot for it in items]
    i32[M.META_POSITIONS, :n] = [it.token_position for it in items]
    i32[M.META_TABLE_ROWS, :n] = [row_of[it.state.request_id] for it in items]
    i32[M.META_STEPS, :n] = [it.recurrent_step for it in items]
    i32[M.META_LAYER_OFFSET, :n] = [base + slot_of_step[it.recurrent_step] * core for it in items]
    i32[M.META_SYNTHETIC, :n] = [-1 if it.synthetic_exit_depth is None or not it.apply_exit_gate
                                 else it.synthetic_exit_depth for it in items]
    i64[n:] = -1
    i32[M.META_POSITIONS, n:] = -1
    i32[M.META_TABLE_ROWS, n:] = 0
    i32[M.META_LAYER_OFFSET, n:] = base
    i32[M.META_STEPS, n:] = 0
    i32[M.META_SYNTHETIC, n:] = -1


@pytest.mark.parametrize("seed", range(4))
def test_fill_recurrent_matches_the_documented_metadata(seed: int) -> None:
    rng = random.Random(seed)
    n = rng.randrange(1, 40)
    rows = n + rng.randrange(0, 9)
    items = _items(rng, n, 4)
    row_of = {it.state.request_id: rng.randrange(256) for it in items}
    slot_of_step = (0, 1, 2, 3) if seed % 2 else (0, 0, 0, 0)
    got64, got32 = np.full(rows, 77, np.int64), np.full((5, rows), 77, np.int32)
    want64, want32 = np.full(rows, 77, np.int64), np.full((5, rows), 77, np.int32)
    _tick.fill_recurrent(items, got64, got32, row_of, 2, 24, slot_of_step)
    _fill_python(items, want64, want32, row_of, 2, 24, slot_of_step)
    assert np.array_equal(got64, want64) and np.array_equal(got32, want32)


def test_fill_recurrent_errors() -> None:
    items = _items(random.Random(1), 3, 4)
    row_of = {it.state.request_id: 0 for it in items}
    with pytest.raises(KeyError):
        _tick.fill_recurrent(items, np.empty(4, np.int64), np.empty((5, 4), np.int32), {}, 0, 1, (0, 1, 2, 3))
    with pytest.raises(ValueError, match="metadata buffers"):
        _tick.fill_recurrent(items, np.empty(2, np.int64), np.empty((5, 2), np.int32), row_of, 0, 1, (0, 1, 2, 3))
    with pytest.raises(ValueError, match="out of range"):
        _tick.fill_recurrent(items, np.empty(4, np.int64), np.empty((5, 4), np.int32), row_of, 0, 1, (0,))
    with pytest.raises(ValueError):
        _tick.fill_recurrent(items, np.empty(4, np.int64)[::-1], np.empty((5, 4), np.int32), row_of, 0, 1,
                             (0, 1, 2, 3))


# -- block manager, queues and eager successors -------------------------------------------------------------
def test_block_pool_is_fifo_with_a_peak_and_rejects_double_frees() -> None:
    # cb/cache_manager.py:72-90: popleft on allocate, append on free.
    pool = _tick.BlockPool(8, 16)
    assert (pool.num_blocks, pool.block_size, pool.num_free_blocks) == (8, 16, 8)
    assert pool.get_free_blocks(3) == [0, 1, 2]
    assert pool.get_free_blocks(6) is None and pool.num_free_blocks == 5
    assert pool.get_free_blocks(2) == [3, 4]
    assert pool.num_allocated_blocks == 5 and pool.peak_num_allocated_blocks == 5
    pool.free_blocks([1, 3])
    assert pool.free_list() == [5, 6, 7, 1, 3]
    assert pool.get_free_blocks(4) == [5, 6, 7, 1]
    assert pool.peak_num_allocated_blocks == 7
    pool.free_blocks([0, 2, 4, 5, 6, 7, 1])
    assert pool.num_allocated_blocks == 0 and pool.peak_num_allocated_blocks == 7
    pool.reset_peak_usage()
    assert pool.peak_num_allocated_blocks == 0
    with pytest.raises(ValueError, match="Cannot free block 2"):
        pool.free_blocks([2])
    with pytest.raises(ValueError, match="Cannot free block 99"):
        pool.free_blocks([99])
    with pytest.raises(ValueError):
        pool.get_free_blocks(-1)
    assert pool.get_free_blocks(0) == []


def test_item_queue_behaves_as_a_deque() -> None:
    q = _tick.ItemQueue()
    assert len(q) == 0 and not q
    a, b, c = object(), object(), object()
    q.append(a)
    q.appendleft(b)
    q.extend([c])
    assert list(q) == [b, a, c] and len(q) == 3 and q
    assert q.popleft() is b
    q.clear()
    assert not q
    with pytest.raises(IndexError):
        q.popleft()


def _enqueue_front_python(queue: list, items, limit: int, in_flight: set) -> int:
    refills = 0
    for item in reversed(items):
        step = item.recurrent_step
        if not 0 <= step < limit:
            raise ValueError(f"recurrent_step must be in [0, {limit}), got {step}")
        in_flight.add(item.state.request_id)
        if step == 0 and queue:
            refills += 1
        queue.insert(0, item)
    return refills


def _pop_batch_python(queue: list, size: int, slot_of_step):
    first = queue.pop(0)
    batch = [first]
    if slot_of_step is None:
        while queue and len(batch) < size:
            batch.append(queue.pop(0))
        return batch
    target = slot_of_step[first.recurrent_step]
    deferred = []
    while queue and len(batch) < size:
        item = queue.pop(0)
        (batch if slot_of_step[item.recurrent_step] == target else deferred).append(item)
    queue[:0] = deferred
    return batch


@pytest.mark.parametrize("seed", range(8))
def test_queue_operations_match_the_scheduler_python(seed: int) -> None:
    # continuous_depth_batching/scheduler.py:142-180 (head re-insertion, refill counting) and
    # :322-346 (slot-homogeneous bucket); random interleavings of pushes and pops.
    rng = random.Random(seed)
    max_steps = 4
    slot_of_step = rng.choice([None, (0, 1, 2, 3), (0, 1, 1, 1), (0, 0, 0, 0)])
    q, ref = _tick.ItemQueue(), []
    in_flight, ref_in_flight = set(), set()
    refills = ref_refills = 0
    for _ in range(60):
        op = rng.random()
        if op < 0.5:
            items = _items(rng, rng.randrange(0, 6), max_steps)
            refills += _tick.enqueue_front(q, items, max_steps, in_flight)
            ref_refills += _enqueue_front_python(ref, items, max_steps, ref_in_flight)
        elif op < 0.6:
            item = _items(rng, 1, max_steps)[0]
            q.append(item)
            ref.append(item)
        elif len(ref):
            size = rng.randrange(1, 8)
            got = _tick.pop_batch(q, size, slot_of_step)
            assert got == _pop_batch_python(ref, size, slot_of_step)
        assert list(q) == ref and refills == ref_refills and in_flight == ref_in_flight
    n = rng.randrange(0, len(ref) + 2)
    assert _tick.pop_front(q, n) == ref[:n] and list(q) == ref[n:]
    bad = _items(rng, 1, max_steps)[0]
    bad.recurrent_step = max_steps
    with pytest.raises(ValueError, match="recurrent_step must be in"):
        _tick.enqueue_front(q, [bad], max_steps, in_flight)


def test_split_live_keeps_order() -> None:
    from continuous_depth_batching_amd.requests import RequestStatus

    rng = random.Random(3)
    items = _items(rng, 12, 4)
    for i, item in enumerate(items):
        if i % 3 == 1:
            item.state._status = RequestStatus.FINISHED
    live, dead = _tick.split_live(items, RequestStatus.FINISHED)
    assert live == [x for x in items if x.state.status != RequestStatus.FINISHED]
    assert dead == [x for x in items if x.state.status == RequestStatus.FINISHED]


def _select_eager_python(coda_items, block, allocate, token):
    """The engine's per-row eager successor selection (cdb/continuous_api.py:1304-1327)."""

    flags = [False] * len(coda_items)
    items, rows = [], []
    for idx, item in enumerate(coda_items):
        state = item.state
        if state.will_finish_on_pending_token():
            continue
        state.position_offset += 1
        current = state.current_len()
        fits = state.allocated_blocks * block - current >= 1 and state.allocated_blocks > 0
        if not fits and not allocate(state):
            state.position_offset -= 1
            continue
        flags[idx] = True
        state.reset_depth_state_for_next_token()
        items.append(DepthWorkItem(state=state, token_id=token, token_position=state.position_offset,
                                   recurrent_step=0, synthetic_exit_depth=state.next_synthetic_exit_depth()))
        rows.append(idx)
    return items, rows, flags


def _coda_states(rng: random.Random, n: int):
    from continuous_depth_batching_amd.requests import RequestStatus

    out = []
    for i in range(n):
        limit = rng.randrange(2, 12)
        state = RequestState(request_id=f"c{i}", initial_tokens=[1, 2, 3], max_new_tokens=limit,
                             synthetic_exit_depths=[rng.randrange(4) for _ in range(limit)],
                             replay_eos_finishes=rng.random() < 0.2)
        state._status = RequestStatus.DECODING
        state.generated_tokens = [7] * rng.randrange(0, limit)
        state.tokens_in_flight = rng.randrange(0, 3)
        state.position_offset = 3 + len(state.generated_tokens) + rng.randrange(0, 3)
        state.allocated_blocks = rng.choice([0, -(-state.position_offset // 4), -(-(state.position_offset + 1) // 4)])
        state._synthetic_exit_cursor = rng.randrange(0, 2)
        state.current_token_exit_depth = rng.randrange(4)
        out.append(DepthWorkItem(state=state, token_id=5, token_position=state.position_offset, recurrent_step=2))
    return out


def _eager_snapshot(items):
    return [(i.state.position_offset, i.state.allocated_blocks, i.state.current_token_exit_depth,
             i.state._synthetic_exit_cursor) for i in items]


@pytest.mark.parametrize("seed", range(8))
def test_select_eager_matches_the_per_row_python(seed: int) -> None:
    block = 4
    built = []
    for impl in ("c", "python"):
        rng = random.Random(seed)
        coda = _coda_states(rng, 24)
        budget = {"blocks": rng.randrange(0, 6)}

        def allocate(state, budget=budget):
            # Exact-ceil allocation from a small budget, as the engine's allocator takes blocks.
            need = -(-(state.position_offset + 1) // block) - state.allocated_blocks
            if need > budget["blocks"]:
                return False
            budget["blocks"] -= need
            state.allocated_blocks += need
            return True

        if impl == "c":
            items, rows, flags = _tick.select_eager(coda, block, allocate, DepthWorkItem, -1)
        else:
            items, rows, flags = _select_eager_python(coda, block, allocate, -1)
        built.append(([(i.state.request_id, i.token_id, i.token_position, i.recurrent_step, i.synthetic_exit_depth)
                       for i in items], rows, flags, _eager_snapshot(coda), budget["blocks"]))
    assert built[0] == built[1]
    assert any(built[0][2]) and not all(built[0][2])


def _update_python(state: RequestState, token: int) -> bool:
    """RequestState.update_and_check_completion as plain Python (requests.py:208-237)."""

    if state.status != RequestStatus.DECODING:
        raise RuntimeError(f"Cannot update request {state.request_id} while status is {state.status.name}")
    state.tokens_in_flight = max(0, state.tokens_in_flight - 1)
    is_eos = token in state._eos_token_ids
    n = len(state.generated_tokens)
    if is_eos or n < state._new_tokens_limit:
        if state.first_token_time < 0:
            state.first_token_time = 1.0
        state.generated_tokens.append(token)
        state.tokens_to_process = [token]
        n += 1
    stop = any(seq and len(state.generated_tokens) >= len(seq) and state.generated_tokens[-len(seq):] == seq
               for seq in state.stop_sequences)
    if is_eos or n >= state._new_tokens_limit or stop:
        state.status = RequestStatus.FINISHED
        return True
    return False


def _decoding_states(rng: random.Random, n: int) -> list[RequestState]:
    states = []
    for i in range(n):
        state = RequestState(request_id=f"q{i}", initial_tokens=[1, 2], max_new_tokens=rng.choice([None, 2, 5]),
                             eos_token_id=rng.choice([None, 7, [7, 9], -1]),
                             stop_sequences=rng.choice([[], [[3, 4]], [[], [5]], [[1, 2, 3]]]))
        state.status = RequestStatus.DECODING
        state.generated_tokens = [rng.randrange(10) for _ in range(rng.randrange(4))]
        state.tokens_in_flight = rng.randrange(3)
        state.position_offset = rng.randrange(50)
        if rng.random() < 0.3:
            state.first_token_time = 0.5
        if rng.random() < 0.15:
            state.status = RequestStatus.FINISHED
        states.append(state)
    return states


def _request_view(state: RequestState):
    return (int(state.status), list(state.generated_tokens), list(state.tokens_to_process), state.tokens_in_flight,
            state.position_offset, state.first_token_time >= 0)


@pytest.mark.parametrize("seed", range(8))
def test_update_completion_matches_the_python(seed: int) -> None:
    rng = random.Random(seed)
    for case in range(60):
        a, b = (_decoding_states(random.Random(seed * 1000 + case), 1)[0] for _ in range(2))
        if a.status == RequestStatus.FINISHED:
            with pytest.raises(RuntimeError, match="while status is FINISHED"):
                _tick.update_completion(a, 1)
            continue
        for _step in range(6):
            token = rng.randrange(10)
            if a.status != RequestStatus.DECODING:
                break
            assert _tick.update_completion(a, token) == _update_python(b, token)
            assert _request_view(a) == _request_view(b)


@pytest.mark.parametrize("seed", range(8))
def test_consume_coda_matches_the_per_row_python(seed: int) -> None:
    rng = random.Random(seed)
    n = rng.randint(1, 24)
    tokens = [rng.randrange(10) for _ in range(n)]
    eager = None if seed % 4 == 0 else [rng.random() < 0.6 for _ in range(n)]
    twins = [_decoding_states(random.Random(seed), n) for _ in range(2)]
    items = [[DepthWorkItem(state=s, token_id=0, token_position=0, recurrent_step=0) for s in states]
             for states in twins]
    got = [(s.request_id, stage) for s, stage in _tick.consume_coda(items[0], tokens, eager)]
    want = []
    for item, token, was_eager in zip(items[1], tokens, eager or [False] * n):
        state = item.state
        if state.status == RequestStatus.FINISHED:
            continue
        if was_eager:
            if _update_python(state, token):
                want.append((state.request_id, False))
            continue
        state.position_offset += 1
        want.append((state.request_id, not _update_python(state, token)))
    assert got == want
    assert [_request_view(s) for s in twins[0]] == [_request_view(s) for s in twins[1]]
    with pytest.raises(ValueError):
        _tick.consume_coda(items[0], tokens[:-1], eager)


@pytest.mark.parametrize("seed", range(8))
def test_coda_upload_matches_the_python_staging(seed: int) -> None:
    """The coda upload and the successors' hidden slots, as the runner built them in Python
    (LIFO free slots first, then fresh ones; cdb/model_runner.py:1193-1203)."""

    rng = random.Random(seed)
    n = rng.randint(1, 20)
    k = rng.randint(0, n)
    rows = sorted(rng.sample(range(n), k))
    free = [rng.randrange(100) for _ in range(rng.randrange(6))]
    next_slot, capacity = 100, 100 + k
    items = [DepthWorkItem(state=RequestState(request_id=f"c{i}", initial_tokens=[1]), token_id=0,
                           token_position=0, recurrent_step=0, hidden_slot=rng.randrange(100)) for i in range(n)]
    succ = [DepthWorkItem(state=items[r].state, token_id=-1, token_position=1, recurrent_step=0) for r in rows]
    upload = np.full(3 * n + 4, 77, dtype=np.int64)
    free_c = list(free)
    got_next = _tick.coda_upload(items, succ, rows, upload.ctypes.data, upload.size, free_c, next_slot, capacity)

    want = np.full_like(upload, 77)
    want[:n] = [it.hidden_slot for it in items]
    free_p, nxt, slots = list(free), next_slot, []
    for _ in range(k):
        if free_p:
            slots.append(free_p.pop())
        else:
            slots.append(nxt)
            nxt += 1
    if k:
        want[n:2 * n] = -1
        want[n + np.array(rows, dtype=np.int64)] = slots
        want[2 * n:2 * n + k] = slots
    assert upload.tolist() == want.tolist()
    assert got_next == nxt and free_c == free_p
    assert [s.hidden_slot for s in succ] == slots
    if k:
        with pytest.raises(RuntimeError, match="bank exhausted"):
            _tick.coda_upload(items, succ, rows, upload.ctypes.data, upload.size, [], capacity, capacity)
        with pytest.raises(ValueError):
            _tick.coda_upload(items, succ, rows, upload.ctypes.data, 2 * n, [], 0, capacity)
        # A row outside the coda is rejected before any hidden slot is taken.
        spare = [5, 6, 7]
        bad_rows = rows[:-1] + [n]
        with pytest.raises(ValueError, match="outside"):
            _tick.coda_upload(items, succ, bad_rows, upload.ctypes.data, upload.size, spare, next_slot, capacity)
        assert spare == [5, 6, 7]


def _route_delayed_python(items, flags, max_steps, pending, hist, backlog):
    coda, refills, exits = [], [], []
    for idx, item in enumerate(items):
        step = item.recurrent_step
        previous = pending.pop(id(item), None)
        leave = step == max_steps - 1 or (item.apply_exit_gate and previous is not None
                                          and previous[0].get(previous[1]))
        if not leave:
            pending[id(item)] = (flags, idx)
        exits.append(leave)
        if leave:
            if item.apply_exit_gate:
                item.state.current_token_exit_depth = step
                item.state.exit_depths.append(step)
                hist[step] += 1
            if backlog is not None and step < max_steps - 1:
                backlog.append((item, step))
            coda.append(item)
        else:
            item.recurrent_step = step + 1
            refills.append(item)
    return coda, refills, exits


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("with_backlog", [False, True])
def test_route_delayed_matches_the_per_row_routing(seed: int, with_backlog: bool) -> None:
    """Three launches in a row on the offset-one horizon: each row's exit comes from the flag
    its previous launch wrote, and the pending map carries the survivors' flags forward."""

    import torch

    from continuous_depth_batching_amd.model_runner import PendingFlags

    rng = random.Random(seed)
    max_steps = 4
    twins = [_items(random.Random(seed), 24, max_steps) for _ in range(2)]
    pendings: list[dict] = [{}, {}]
    hists = [Counter(), Counter()]
    backlogs = [[], []] if with_backlog else [None, None]
    for launch in range(3):
        bits = [rng.random() < 0.4 for _ in range(24)]
        flags = [PendingFlags(host=torch.tensor(bits, dtype=torch.uint8), event=None) for _ in range(2)]
        live = [[it for it in items if it.recurrent_step < max_steps] for items in twins]
        got = _tick.route_delayed(live[0], flags[0], max_steps, pendings[0], hists[0], backlogs[0])
        want = _route_delayed_python(live[1], flags[1], max_steps, pendings[1], hists[1], backlogs[1])
        assert [[it.state.request_id for it in part] for part in got[:2]] == \
               [[it.state.request_id for it in part] for part in want[:2]]
        assert got[2] == want[2]
        assert _snapshot(twins[0]) == _snapshot(twins[1])
        assert hists[0] == hists[1]
        assert sorted((live[0].index(next(i for i in live[0] if id(i) == k)), v[1]) for k, v in pendings[0].items()) \
            == sorted((live[1].index(next(i for i in live[1] if id(i) == k)), v[1]) for k, v in pendings[1].items())
        if with_backlog:
            assert [(it.state.request_id, s) for it, s in backlogs[0]] == \
                   [(it.state.request_id, s) for it, s in backlogs[1]]
        for part in (got[0], want[0]):  # exited rows leave; the rest step on
            for it in part:
                it.recurrent_step = max_steps
