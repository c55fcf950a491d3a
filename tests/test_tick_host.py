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
from continuous_depth_batching_amd.requests import DepthWorkItem, RequestState

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
