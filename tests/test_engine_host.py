"""The engine's scheduling on the host: the reference's token-increment vectors.

Every expected token stream and counter below is the one the reference's own
tests assert for the same model, configuration and exit trace
(tests/continuous_depth_batching/test_continuous_depth_batching.py, cited per
test). The engine, scheduler, block manager and the runner's metadata assembly
are the product's code; tests/host_runner.py only supplies the stage arithmetic.
"""

from __future__ import annotations

import numpy as np
import pytest

from continuous_depth_batching_amd.exit_policy import ExitDecisionRule, ExitPolicySpec
from continuous_depth_batching_amd.model_runner import ModelRunner
from continuous_depth_batching_amd.requests import DepthWorkItem, RequestState, RequestStatus
from tests.host_runner import make_engine

META = ModelRunner


def generate(engine, prompts, max_new_tokens, **kw):
    kw.setdefault("eos_token_id", None)
    outs = engine.generate_batch([list(p) for p in prompts], max_new_tokens=max_new_tokens, **kw)
    return [o.generated_tokens for o in outs]


def test_synthetic_exit_at_depth_zero_skips_recurrent_work() -> None:
    # test_continuous_depth_batching.py:214-239
    engine = make_engine(synthetic_exit_replay=True)
    tokens = generate(engine, [[1, 2], [5]], 3, exit_depths=[[0, 0], [0, 0]])
    s = engine.last_stats
    assert tokens == [[5, 6, 7], [8, 9, 10]]
    assert s.recurrent_steps == 4
    assert s.prefill_recurrent_steps == 9
    assert s.prefill_coda_tokens == 2
    assert s.coda_tokens == 4
    assert s.fixed_depth_recurrent_steps == 12
    assert s.skipped_recurrent_steps == 8
    assert s.exit_depth_histogram == {0: 4}
    assert s.recurrent_batches == s.mixed_recurrent_batches
    assert engine.cache.get_num_free_blocks() == engine.cache.num_blocks


def test_synthetic_exit_sequence_mixed_depths() -> None:
    # test_continuous_depth_batching.py:242-272
    engine = make_engine(synthetic_exit_replay=True)
    tokens = generate(engine, [[1, 2], [5]], 3, exit_depths=[[0, 2], [1, 0]])
    s = engine.last_stats
    assert [len(t) for t in tokens] == [3, 3]
    # Each token is the previous one plus its replayed depth + 1.
    assert tokens == [[5, 6, 9], [8, 10, 11]]
    assert s.recurrent_steps == 7
    assert s.prefill_recurrent_steps == 9
    assert s.fixed_depth_recurrent_steps == 12
    assert s.skipped_recurrent_steps == 5
    assert s.exit_depth_histogram == {0: 2, 1: 1, 2: 1}
    assert s.mixed_recurrent_batches == s.recurrent_batches
    assert s.max_mixed_depths_per_batch >= 1
    assert engine.runner.next_hidden_slot <= engine.cache.max_num_batched_tokens


@pytest.mark.parametrize("refill", [True, False])
def test_refill_and_no_refill_agree_token_for_token(refill: bool) -> None:
    # test_continuous_depth_batching.py:401-424: refill changes scheduling, never tokens.
    prompts = [[1, 2], [5], [3, 4, 5]]
    depths = [[0, 2], [1, 0], [2, 1]]
    base = make_engine(synthetic_exit_replay=True, refill=True)
    want = generate(base, prompts, 3, exit_depths=depths)
    engine = make_engine(synthetic_exit_replay=True, refill=refill)
    got = generate(engine, prompts, 3, exit_depths=depths)
    assert got == want
    assert engine.last_stats.exit_depth_histogram == base.last_stats.exit_depth_histogram
    assert engine.last_stats.recurrent_steps == base.last_stats.recurrent_steps
    assert engine.last_stats.coda_tokens == base.last_stats.coda_tokens
    if refill:
        assert engine.last_stats.scheduler_refills > 0
    else:
        assert engine.last_stats.scheduler_refills == 0
        assert engine.last_stats.mixed_recurrent_batches == 0
        for launch in engine.runner.launches:
            live = launch["slots"] >= 0
            assert len(set(launch["meta"][META.META_STEPS][live].tolist())) == 1


def test_full_depth_live_gate_sync_and_async_streams() -> None:
    # test_continuous_depth_batching.py:883-926: no threshold, so every token runs all 3 steps
    # (token + 3); eos 13 stops requests 0, 2 and 3; request 1 is length-capped.
    prompts = [[1], [2, 5], [7, 7, 1], [10]]
    mnt = [6, 2, 4, 3]
    expected = [[4, 7, 10, 13], [8, 11], [4, 7, 10, 13], [13]]
    sync = make_engine(num_blocks=64, max_num_batched_tokens=8, max_model_len=32, use_async_batching=False)
    assert generate(sync, prompts, mnt, eos_token_id=13) == expected
    asyn = make_engine(num_blocks=64, max_num_batched_tokens=8, max_model_len=32, use_async_batching=True)
    assert generate(asyn, prompts, mnt, eos_token_id=13) == expected
    assert asyn.last_stats.prelude_tokens["after_coda_eager"] > 0
    assert asyn.last_stats.prelude_tokens["after_prefill_eager"] > 0
    assert asyn.last_stats.cancelled_depth_items >= 2
    assert asyn.last_stats.recurrent_steps == sync.last_stats.recurrent_steps
    assert asyn.cache.get_num_free_blocks() == asyn.cache.num_blocks


def test_hazard_gate_exits_at_the_first_step() -> None:
    # The token-increment gate emits +10 at step 0: sigmoid(10) crosses a 0.5 CDF threshold at once,
    # so every decode token runs exactly one step and advances by 1.
    engine = make_engine(exit_threshold=0.5)
    tokens = generate(engine, [[1, 2], [5]], 4)
    assert tokens == [[5, 6, 7, 8], [8, 9, 10, 11]]
    assert engine.last_stats.exit_depth_histogram == {0: 6}


def test_direct_threshold_gate_exits_once_the_signal_drops() -> None:
    # Direct threshold 0: +10 at step 0 keeps the token, -10 at step 1 exits it (depth 1: token + 2).
    engine = make_engine(exit_threshold=0.0, spec=ExitPolicySpec(ExitDecisionRule.DIRECT_THRESHOLD))
    tokens = generate(engine, [[1, 2], [5]], 3)
    assert tokens == [[5, 7, 9], [8, 10, 12]]
    assert engine.last_stats.exit_depth_histogram == {1: 4}


def test_delayed_replay_exits_one_step_later() -> None:
    # test_continuous_depth_batching.py:731-760 and cdb/continuous_api.py:1711-1724: on the delayed
    # horizon a replayed depth d exits at step d + 1 (capped at the last step).
    engine = make_engine(synthetic_exit_replay=True, use_async_batching=True, delay_gate_consumption=True)
    prompts = [[1, 2], [5], [3, 4, 5]]
    depths = [[0, 1], [1, 0], [0, 1]]
    tokens = generate(engine, prompts, 3, exit_depths=depths)
    want = []
    for p, ds in zip(prompts, depths):
        t = [(p[-1] + 3) % 16]
        for d in ds:
            t.append((t[-1] + min(d + 1, 2) + 1) % 16)
        want.append(t)
    assert tokens == want
    assert engine.last_stats.exit_depth_histogram == {1: 3, 2: 3}


def test_recurrent_metadata_rows_and_padding() -> None:
    # cdb/model_runner.py:704-771 / test_continuous_depth_batching.py:1045-1081: per-row slots,
    # positions, block-table rows and depth-indexed cache layers; padding rows are inert.
    engine = make_engine(max_num_seqs=4, kv_policy="depth_indexed")
    items = []
    for idx in range(3):
        state = RequestState(request_id=f"r{idx}", initial_tokens=[idx + 1])
        state.status = RequestStatus.DECODING
        state.tokens_to_process = [idx + 1]
        engine.scheduler.active_requests[state.request_id] = state
        item = engine.staging.stage(state)
        assert item is not None
        items.append(item)
    items[2].recurrent_step = 2
    engine.runner.compute_prelude_batch(items)
    engine.runner.compute_recurrent_batch(items)
    launch = engine.runner.launches[-1]
    meta = launch["meta"]
    assert launch["slots"].tolist() == [0, 1, 2, -1]
    assert meta[META.META_POSITIONS].tolist() == [0, 0, 0, -1]
    rows = [engine.cache.table_row_of[f"r{i}"] for i in range(3)]
    assert meta[META.META_TABLE_ROWS].tolist() == rows + [0]
    assert meta[META.META_STEPS].tolist() == [0, 0, 2, 0]
    assert meta[META.META_LAYER_OFFSET].tolist() == [0, 0, 2, 0]  # depth_indexed: slot = step, 1 layer
    for r, i in zip(rows, range(3)):
        blocks = engine.cache.block_table[f"r{i}"]
        assert launch["table"][i].tolist() == blocks + [-1] * (engine.cache.table_width - len(blocks))


def test_hidden_slots_are_reused_lifo_after_coda() -> None:
    # test_continuous_depth_batching.py:974-1004
    engine = make_engine(max_num_seqs=2)
    s0 = RequestState(request_id="r0", initial_tokens=[1])
    s1 = RequestState(request_id="r1", initial_tokens=[2])
    items = [DepthWorkItem(state=s0, token_id=1, token_position=0, recurrent_step=0),
             DepthWorkItem(state=s1, token_id=2, token_position=0, recurrent_step=0)]
    runner = engine.runner
    runner.compute_prelude_batch(items)
    assert [i.hidden_slot for i in items] == [0, 1]
    runner.consume_coda_result(runner.stage_coda_batch(items))
    assert [i.hidden_slot for i in items] == [None, None]
    assert sorted(runner.free_hidden_slots) == [0, 1]
    nxt = [DepthWorkItem(state=s0, token_id=3, token_position=1, recurrent_step=0),
           DepthWorkItem(state=s1, token_id=4, token_position=1, recurrent_step=0)]
    runner.compute_prelude_batch(nxt)
    assert sorted(i.hidden_slot for i in nxt) == [0, 1]
    assert runner.next_hidden_slot == 2


def test_last_exited_copies_exit_kv_into_deeper_slots() -> None:
    # cdb/continuous_api.py:1225-1245: an exit at step e < R-1 copies its token's KV row from slot e
    # into every deeper slot before any launch reads them; counted once per exiting token.
    engine = make_engine(synthetic_exit_replay=True, kv_policy="last_exited", kv_pressure_mode="none")
    depths = [[0, 2, 1], [1, 1, 0]]
    generate(engine, [[1, 2], [5]], 4, exit_depths=depths)
    copies = engine.runner.exit_copies
    flat_slots = [s for _, slots in copies for s in slots]
    assert sorted(flat_slots) == sorted(d for ds in depths for d in ds if d < 2)
    assert engine.last_stats.exit_kv_copies == len(flat_slots)


def test_fused_prelude_from_device_tokens_matches_host_ids() -> None:
    # test_continuous_depth_batching.py:533-575: leading rows gathered from a staged result's
    # device tokens (rows 1 and 3) embed exactly what host ids would.
    from continuous_depth_batching_amd.model_runner import PendingCodaResult
    from continuous_depth_batching_amd.requests import TMP_TOKEN_ID
    import torch

    engine = make_engine(synthetic_exit_replay=True)
    runner = engine.runner
    ids = [5, 9, 3, 7]

    def items_for(tokens):
        return [DepthWorkItem(state=RequestState(request_id=f"r{i}", initial_tokens=[1]), token_id=t,
                              token_position=i, recurrent_step=0) for i, t in enumerate(tokens)]

    host = items_for(ids)
    runner.compute_prelude_batch(host)
    want = [runner.hidden[i.hidden_slot] for i in host]
    staged = PendingCodaResult(items=[], host_tokens=torch.tensor([0, 5, 0, 9]),
                               device_tokens=torch.tensor([0, 5, 0, 9]))
    mixed = items_for([TMP_TOKEN_ID, TMP_TOKEN_ID, 3, 7])
    runner.compute_prelude_batch(mixed, device_groups=[(staged, [1, 3])])
    assert [runner.hidden[i.hidden_slot] for i in mixed] == want


def test_block_allocation_is_fifo_and_blocks_return_after_generation() -> None:
    # cb/cache_manager.py:72-90: FIFO free list; every block comes back when requests finish.
    engine = make_engine(synthetic_exit_replay=True, num_blocks=16)
    generate(engine, [[1, 2, 3], [4, 5, 6, 7, 8]], 4, exit_depths=[[0, 1, 2], [2, 2, 2]])
    assert engine.cache.get_num_free_blocks() == 16
    bm = engine.cache._block_manager
    assert sorted(bm.free_list()) == list(range(16))
    assert np.all(engine.cache.host_table == -1)


def test_min_coda_batch_size_pools_codas_without_changing_tokens() -> None:
    # test_continuous_depth_batching.py:1006-1029: larger coda floors change launch counts only,
    # and a floor no workload can reach still completes through the idle flush.
    prompts = [[1, 2], [3, 4], [5, 6], [7, 8]]
    depths = [[0, 2, 1], [1, 0, 2], [2, 1, 0], [0, 1, 2]]
    out, stats = {}, {}
    for floor in (1, 3, 64):
        engine = make_engine(synthetic_exit_replay=True, refill=True, min_coda_batch_size=floor,
                             **({"max_num_seqs": 64} if floor == 64 else {}))
        out[floor] = generate(engine, prompts, 4, exit_depths=depths)
        stats[floor] = engine.last_stats
    assert out[3] == out[1]
    assert out[64] == out[1]
    assert stats[3].coda_tokens == stats[1].coda_tokens
    assert stats[3].coda_batches < stats[1].coda_batches


def test_min_coda_batch_size_must_be_positive() -> None:
    with pytest.raises(ValueError, match="min_coda_batch_size"):
        make_engine(min_coda_batch_size=0)


@pytest.mark.parametrize("refill", [True, False])
@pytest.mark.parametrize("horizon,use_async,delay,expected_depth", [
    ("same", False, False, 0),
    ("offset", True, True, 1),
])
def test_decision_horizon_sets_the_exact_exit_depth(refill, horizon, use_async, delay, expected_depth) -> None:
    # test_continuous_depth_batching.py:1114-1151: the +10 step-0 signal exits at step 0 on the
    # same-step horizon and one launch later on the offset-one horizon.
    from continuous_depth_batching_amd.exit_policy import DecisionHorizon

    h = DecisionHorizon.SAME_STEP if horizon == "same" else DecisionHorizon.OFFSET_ONE
    engine = make_engine(exit_threshold=0.5, refill=refill, use_async_batching=use_async,
                         delay_gate_consumption=delay, spec=ExitPolicySpec(ExitDecisionRule.CUMULATIVE_HAZARD, h))
    generate(engine, [[1]], 2)
    assert engine.last_stats.exit_depth_histogram == {expected_depth: 1}
    launched = [launch["meta"][META.META_STEPS][launch["slots"] >= 0].tolist() for launch in engine.runner.launches]
    assert launched == [[s] for s in range(expected_depth + 1)]


def _scheduler(max_num_seqs: int = 4, **kw):
    from continuous_depth_batching_amd.scheduler import CDBScheduler

    engine = make_engine(max_num_seqs=max_num_seqs, **kw.pop("engine", {}))
    return CDBScheduler(engine.cache, 3, max_num_seqs=max_num_seqs, **kw), engine.cache


def _decoding_item(scheduler, request_id: str, step: int = 0, token: int = 1, position: int = 2) -> DepthWorkItem:
    state = RequestState(request_id=request_id, initial_tokens=[1, 2], max_new_tokens=4)
    scheduler.active_requests[request_id] = state
    state.status = RequestStatus.DECODING
    return DepthWorkItem(state=state, token_id=token, token_position=position, recurrent_step=step)


def test_head_insertion_re_serves_stepped_items_tail_insertion_rotates() -> None:
    # test_resident_set_and_refill_discipline.py:357-380
    scheduler, _ = _scheduler()
    stepped = [_decoding_item(scheduler, f"w{i}") for i in range(2)]
    parked = [_decoding_item(scheduler, f"p{i}") for i in range(2)]
    for item in parked:
        scheduler.enqueue_depth(item)
    scheduler.enqueue_depth_front(stepped)
    assert [i.state.request_id for i in scheduler.ready_queue] == ["w0", "w1", "p0", "p1"]
    scheduler.ready_queue.clear()
    for item in parked + stepped:
        scheduler.enqueue_depth(item)
    assert [i.state.request_id for i in scheduler.ready_queue] == ["p0", "p1", "w0", "w1"]


def test_head_insertion_keeps_batch_order() -> None:
    # test_resident_set_and_refill_discipline.py:383-391
    scheduler, _ = _scheduler()
    items = [_decoding_item(scheduler, f"r{i}") for i in range(4)]
    scheduler.enqueue_depth_front(items)
    assert [i.state.request_id for i in scheduler.ready_queue] == ["r0", "r1", "r2", "r3"]


def test_scheduler_batches_mixed_recurrent_steps_fifo() -> None:
    # test_continuous_depth_batching.py:763-778
    scheduler, cache = _scheduler(max_num_seqs=2)
    state = RequestState(request_id="r0", initial_tokens=[1])
    for tok, pos, step in ((1, 0, 1), (2, 1, 2), (3, 2, 2)):
        scheduler.enqueue_depth(DepthWorkItem(state=state, token_id=tok, token_position=pos, recurrent_step=step))
    batch = scheduler.schedule_next(token_budget=cache.max_num_batched_tokens, cache_budget=cache.num_pages)
    assert batch is not None and batch.kind == "recurrent"
    assert [i.token_id for i in batch.depth_items] == [1, 2]
    assert [i.recurrent_step for i in batch.depth_items] == [1, 2]
    assert scheduler.mixed_batches_scheduled == 1


def test_scheduler_prefills_waiting_prompt_before_underfilled_recurrent_batch() -> None:
    # test_continuous_depth_batching.py:781-799
    scheduler, cache = _scheduler(max_num_seqs=2, safety_margin=0.0)
    depth_state = RequestState(request_id="decode", initial_tokens=[1])
    prefill_state = RequestState(request_id="prefill", initial_tokens=[4, 5])
    scheduler.enqueue_depth(DepthWorkItem(state=depth_state, token_id=1, token_position=0, recurrent_step=0))
    scheduler.add_waiting_request(prefill_state)
    batch = scheduler.schedule_next(token_budget=cache.max_num_batched_tokens, cache_budget=cache.num_pages)
    assert batch is not None and batch.kind == "prefill"
    assert [f.state.request_id for f in batch.requests] == ["prefill"]
    assert prefill_state.status is RequestStatus.DECODING
    assert prefill_state.tokens_to_process == [4, 5]
    assert prefill_state.remaining_prefill_tokens == []
    assert len(scheduler.ready_queue) == 1


def test_scheduler_holds_prefill_of_a_request_with_a_token_in_flight() -> None:
    # test_continuous_depth_batching.py:802-828
    scheduler, cache = _scheduler(max_num_seqs=4, safety_margin=0.0)
    state = RequestState(request_id="prefill", initial_tokens=[4, 5])
    state.status = RequestStatus.PREFILLING
    state.remaining_prefill_tokens = [5]
    state.tokens_to_process = [4]
    state.allocated_blocks = cache.allocate_blocks(1, state.request_id, state.allocated_blocks) or 0
    scheduler.active_requests[state.request_id] = state
    scheduler.enqueue_depth(DepthWorkItem(state=state, token_id=4, token_position=0, recurrent_step=0))
    batch = scheduler.schedule_next(token_budget=cache.max_num_batched_tokens, cache_budget=cache.num_pages)
    assert batch is not None and batch.kind == "recurrent"
    assert [i.state.request_id for i in batch.depth_items] == ["prefill"]
    assert state.remaining_prefill_tokens == [5]
    scheduler.release_in_flight_request(state.request_id)
    nxt = scheduler.schedule_next(token_budget=cache.max_num_batched_tokens, cache_budget=cache.num_pages)
    assert nxt is not None and nxt.kind == "prefill"
    assert [f.state.request_id for f in nxt.requests] == ["prefill"]


def test_scheduler_serves_coda_before_recurrent_and_prefill() -> None:
    # test_continuous_depth_batching.py:831-844
    scheduler, cache = _scheduler(max_num_seqs=2, safety_margin=0.0)
    state = RequestState(request_id="r0", initial_tokens=[1])
    scheduler.add_waiting_request(RequestState(request_id="prefill", initial_tokens=[2]))
    scheduler.enqueue_depth(DepthWorkItem(state=state, token_id=1, token_position=0, recurrent_step=0))
    scheduler.enqueue_coda(DepthWorkItem(state=state, token_id=1, token_position=0, recurrent_step=1))
    batch = scheduler.schedule_next(token_budget=cache.max_num_batched_tokens, cache_budget=cache.num_pages)
    assert batch is not None and batch.kind == "coda"
    assert [i.recurrent_step for i in batch.depth_items] == [1]


def test_no_refill_matches_refill_on_the_delayed_horizon() -> None:
    # test_continuous_depth_batching.py:427-440: both loops apply replayed exits one step late.
    prompts = [[1, 2], [5], [3, 4, 5]]
    depths = [[0, 1], [1, 0], [0, 1]]
    kw = dict(synthetic_exit_replay=True, use_async_batching=True, delay_gate_consumption=True)
    refill = make_engine(refill=True, **kw)
    wave = make_engine(refill=False, **kw)
    want = generate(refill, prompts, 3, exit_depths=depths)
    assert generate(wave, prompts, 3, exit_depths=depths) == want
    assert refill.last_stats.scheduler_refills > 0
    assert wave.last_stats.scheduler_refills == 0
    assert wave.last_stats.exit_depth_histogram == refill.last_stats.exit_depth_histogram
    assert wave.last_stats.recurrent_steps == refill.last_stats.recurrent_steps


def test_steady_window_opens_after_warmup_and_closes_after_the_last_admission() -> None:
    # scheduler_base.py:315-398: the window opens on the tick the warm-up count of requests has
    # completed while prompts still wait, and closes on the first tick after the last admission.
    prompts = [[1 + i, 2] for i in range(8)]
    depths = [[1, 0, 2] for _ in range(8)]
    engine = make_engine(synthetic_exit_replay=True, max_num_seqs=2, num_blocks=64, max_model_len=32)
    engine.scheduler.steady_warmup_requests = 2
    generate(engine, prompts, 4, exit_depths=depths)
    summary = engine.scheduler.steady_state_summary()
    assert summary is not None
    assert 0 < summary["completed_requests"] < 8 and summary["generated_tokens"] > 0
    assert 0 < summary["mean_resident_requests"] <= 2 and summary["ticks"] > 0
    assert not engine.scheduler.steady_window_open
    # No warm-up count, or every prompt admitted at once: no window.
    generate(make_engine(synthetic_exit_replay=True), prompts, 4, exit_depths=depths)
    wide = make_engine(synthetic_exit_replay=True, num_blocks=64, max_model_len=32, max_num_batched_tokens=16,
                       max_num_seqs=8)
    wide.scheduler.steady_warmup_requests = 2
    generate(wide, prompts, 4, exit_depths=depths)
    assert wide.scheduler.steady_state_summary() is None
