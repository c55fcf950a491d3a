"""Pins of the schedule oracle (oracle/scheduler.py) without a GPU.

Every expected value restates one of the reference's own tests for the token-increment model
(tests/continuous_depth_batching/test_continuous_depth_batching.py and test_schedule_trace.py,
cited per test), or follows from the semantics in closed form: tokens from the replayed depths,
FIFO block ids, LIFO hidden slots, and the trace/counter bookkeeping identities.
"""

from __future__ import annotations

from collections import Counter

import numpy as np
import pytest

from oracle.scheduler import DIRECT, HAZARD, ScheduleOracle, ScheduleOracleError

# The reference tests' engine config (test_continuous_depth_batching.py:149-161).
BASE = dict(num_blocks=16, block_size=4, max_num_batched_tokens=4, max_model_len=16, use_async_batching=False,
            max_recurrent_steps=3, vocab_size=16)


def oracle(**over) -> ScheduleOracle:
    kw = dict(BASE)
    kw.update(over)
    return ScheduleOracle(**kw)


def recurrent_steps_seen(result) -> list[list[int]]:
    return [[row[2] for row in ev[1]] for ev in result["events"] if ev[0] == "recurrent"]


def test_replay_depth_zero_skips_recurrent_work() -> None:
    # test_continuous_depth_batching.py:214-239
    r = oracle(synthetic_exit_replay=True).run([[1, 2], [5]], 3, exit_depths=[[0, 0], [0, 0]])
    s = r["stats"]
    assert r["tokens"] == [[5, 6, 7], [8, 9, 10]]
    assert s["recurrent_steps"] == 4
    assert s["prefill_recurrent_steps"] == 9
    assert s["prefill_coda_tokens"] == 2
    assert s["coda_tokens"] == 4
    assert s["fixed_depth_recurrent_steps"] == 12
    assert s["fixed_depth_recurrent_steps"] - s["recurrent_steps"] == 8
    assert s["exit_depth_histogram"] == {0: 4}
    assert s["recurrent_batches"] == s["mixed_recurrent_batches"]
    assert r["free_blocks_at_end"] == 16


def test_replay_mixed_depths() -> None:
    # test_continuous_depth_batching.py:242-272
    r = oracle(synthetic_exit_replay=True).run([[1, 2], [5]], 3, exit_depths=[[0, 2], [1, 0]])
    s = r["stats"]
    assert [len(t) for t in r["tokens"]] == [3, 3]
    assert s["recurrent_steps"] == 7
    assert s["prefill_recurrent_steps"] == 9
    assert s["fixed_depth_recurrent_steps"] - s["recurrent_steps"] == 5
    assert s["exit_depth_histogram"] == {0: 2, 1: 1, 2: 1}
    assert s["mixed_recurrent_batches"] == s["recurrent_batches"]
    assert s["max_mixed_depths_per_batch"] >= 1
    assert 2 <= r["next_hidden_slot"] <= 4


def closed_form_tokens(prompts, depths, steps, vocab, delayed=False):
    """First token: last prompt token + steps; each next token: previous + exit step + 1."""

    out = []
    for p, ds in zip(prompts, depths):
        t = [(p[-1] + steps) % vocab]
        for d in ds:
            e = min(d + 1, steps - 1) if delayed else d
            t.append((t[-1] + e + 1) % vocab)
        out.append(t)
    return out


@pytest.mark.parametrize("refill", [True, False])
def test_refill_and_no_refill_agree_and_differ_only_in_scheduling(refill: bool) -> None:
    # test_continuous_depth_batching.py:401-424 and :713-728
    prompts = [[1, 2], [5], [3, 4, 5]]
    depths = [[0, 2], [1, 0], [2, 1]]
    base = oracle(synthetic_exit_replay=True, refill=True).run(prompts, 3, exit_depths=depths)
    r = oracle(synthetic_exit_replay=True, refill=refill).run(prompts, 3, exit_depths=depths)
    assert r["tokens"] == base["tokens"] == closed_form_tokens(prompts, depths, 3, 16)
    for key in ("exit_depth_histogram", "recurrent_steps", "coda_tokens", "prefill_recurrent_steps"):
        assert r["stats"][key] == base["stats"][key]
    if refill:
        assert r["stats"]["scheduler_refills"] > 0
    else:
        assert r["stats"]["scheduler_refills"] == 0
        assert r["stats"]["mixed_recurrent_batches"] == 0
        assert all(len(set(steps)) == 1 for steps in recurrent_steps_seen(r))


def test_no_refill_launches_one_depth_per_launch() -> None:
    # test_continuous_depth_batching.py:713-728
    r = oracle(synthetic_exit_replay=True, refill=False).run([[1, 2], [5], [3, 4]], 3,
                                                             exit_depths=[[0, 2], [1, 0], [2, 1]])
    assert r["stats"]["scheduler_refills"] == 0
    assert r["stats"]["mixed_recurrent_batches"] == 0
    seen = recurrent_steps_seen(r)
    assert seen and all(len(set(steps)) == 1 for steps in seen)


def test_delayed_replay_exits_one_step_later_with_the_same_tokens_as_refill() -> None:
    # test_continuous_depth_batching.py:431-447 (force_delayed) and :731-760
    prompts = [[1, 2], [5], [3, 4, 5]]
    depths = [[0, 1], [1, 0], [0, 1]]
    r = oracle(synthetic_exit_replay=True, replay_offset_one=True).run(prompts, 3, exit_depths=depths)
    assert r["tokens"] == closed_form_tokens(prompts, depths, 3, 16, delayed=True)
    assert r["exit_depths"] == [[min(d + 1, 2) for d in ds] for ds in depths]
    assert r["stats"]["scheduler_refills"] > 0
    one = oracle(synthetic_exit_replay=True, replay_offset_one=True).run([[1]], 2, exit_depths=[[0]])
    assert one["stats"]["exit_depth_histogram"] == {1: 1}
    assert recurrent_steps_seen(one) == [[0], [1]]


def test_async_eager_reentry_matches_the_synchronous_streams() -> None:
    # test_continuous_depth_batching.py:883-926: full depth (token + 3), eos 13.
    prompts = [[1], [2, 5], [7, 7, 1], [10]]
    mnt = [6, 2, 4, 3]
    cfg = dict(num_blocks=64, max_num_batched_tokens=8, max_model_len=32)
    sync = oracle(**cfg, use_async_batching=False).run(prompts, mnt, eos_token_id=13)
    asyn = oracle(**cfg, use_async_batching=True).run(prompts, mnt, eos_token_id=13)
    assert sync["tokens"] == [[4, 7, 10, 13], [8, 11], [4, 7, 10, 13], [13]]
    assert asyn["tokens"] == sync["tokens"]
    assert asyn["stats"]["prelude_tokens"].get("after_coda_eager", 0) > 0
    assert asyn["stats"]["prelude_tokens"].get("after_prefill_eager", 0) > 0
    assert asyn["stats"]["cancelled_depth_items"] >= 2
    assert asyn["stats"]["recurrent_steps"] == sync["stats"]["recurrent_steps"]
    assert asyn["free_blocks_at_end"] == 64


@pytest.mark.parametrize("refill", [True, False])
@pytest.mark.parametrize("offset_one,use_async,delay,expected", [(False, False, False, 0), (True, True, True, 1)])
def test_decision_horizon_sets_the_exit_depth(refill, offset_one, use_async, delay, expected) -> None:
    # test_continuous_depth_batching.py:1117-1153
    r = oracle(exit_threshold=0.5, refill=refill, use_async_batching=use_async, delay_gate_consumption=delay,
               offset_one_signal=offset_one).run([[1]], 2)
    assert r["stats"]["exit_depth_histogram"] == {expected: 1}
    assert recurrent_steps_seen(r) == [[step] for step in range(expected + 1)]


def test_hazard_and_direct_threshold_gates() -> None:
    # +10 at step 0: sigmoid(10) crosses a 0.5 CDF at once (token + 1 per decode token);
    # direct threshold 0 keeps +10 and exits on -10 at step 1 (token + 2).
    h = oracle(exit_threshold=0.5, rule=HAZARD).run([[1, 2], [5]], 4)
    assert h["tokens"] == [[5, 6, 7, 8], [8, 9, 10, 11]]
    assert h["stats"]["exit_depth_histogram"] == {0: 6}
    d = oracle(exit_threshold=0.0, rule=DIRECT).run([[1, 2], [5]], 3)
    assert d["tokens"] == [[5, 7, 9], [8, 10, 12]]
    assert d["stats"]["exit_depth_histogram"] == {1: 4}


def test_min_coda_batch_size_changes_launches_not_tokens() -> None:
    # test_continuous_depth_batching.py:1006-1027
    prompts = [[1, 2], [3, 4], [5, 6], [7, 8]]
    depths = [[0, 2, 1], [1, 0, 2], [2, 1, 0], [0, 1, 2]]
    runs = {m: oracle(synthetic_exit_replay=True, min_coda_batch_size=m).run(prompts, 4, exit_depths=depths)
            for m in (1, 3, 64)}
    assert runs[3]["tokens"] == runs[1]["tokens"] == runs[64]["tokens"]
    assert runs[3]["stats"]["coda_tokens"] == runs[1]["stats"]["coda_tokens"]
    assert runs[3]["stats"]["coda_batches"] < runs[1]["stats"]["coda_batches"]


# -- schedule trace (test_schedule_trace.py:13-114) ----------------------------------------------------------------
TRACE_PROMPTS = [[1, 2], [5], [3, 4, 5], [6]]
TRACE_DEPTHS = [[0, 2, 1], [2, 0, 2], [1, 1, 0], [2, 2, 1]]


def traced(refill: bool):
    r = oracle(synthetic_exit_replay=True, refill=refill, max_num_seqs=3).run(TRACE_PROMPTS, 4,
                                                                               exit_depths=TRACE_DEPTHS)
    return r, r["trace"]


def check_trace_against_stats(r, events) -> None:
    s = r["stats"]
    assert [e["launch"] for e in events] == list(range(1, len(events) + 1))
    assert all(a["tick"] <= b["tick"] for a, b in zip(events, events[1:]))
    assert {e["stage"] for e in events} == {"prefill", "prelude", "recurrent", "coda"}
    assert events[0]["stage"] == "prefill"
    by = {st: [e for e in events if e["stage"] == st] for st in ("prefill", "prelude", "recurrent", "coda")}
    assert sum(e["size"] for e in by["prefill"]) == s["prefill_requests"]
    assert sum(e["size"] for e in by["prelude"]) == sum(s["prelude_tokens"].values())
    assert sum(e["size"] for e in by["coda"]) == s["coda_tokens"]
    assert sum(e["exited"] for e in by["recurrent"]) == s["coda_tokens"]
    assert sum(e["size"] for e in by["recurrent"]) == s["recurrent_steps"]
    for e in by["recurrent"]:
        assert sum(e["depths"].values()) == e["size"] <= 3
        assert 0 <= e["exited"] <= e["size"]
    for e in by["prefill"]:
        assert e["tokens"] >= e["size"]
    final = events[-1]
    assert (final["waiting"], final["recurrent_queue"], final["coda_queue"]) == (0, 0, 0)
    assert all(0 <= e["decode"] <= e["active"] for e in events)


def test_refill_trace_agrees_with_the_counters_and_mixes_depths() -> None:
    # test_schedule_trace.py:66-77
    r, events = traced(refill=True)
    check_trace_against_stats(r, events)
    recurrent = [e for e in events if e["stage"] == "recurrent"]
    assert any(len(e["depths"]) > 1 for e in recurrent)
    assert any(e["exited"] for e in recurrent)
    sites = {e["site"] for e in events if e["stage"] == "prelude"}
    assert sites <= {"after_prefill", "after_prefill_eager", "after_coda_staged", "after_coda_eager"}
    assert "after_coda_staged" in sites or "after_coda_eager" in sites


def test_no_refill_trace_is_a_sequence_of_shrinking_waves() -> None:
    # test_schedule_trace.py:90-113
    r, events = traced(refill=False)
    check_trace_against_stats(r, events)
    assert all(e["recurrent_queue"] == 0 and e["coda_queue"] == 0 for e in events)
    waves: dict[int, list] = {}
    for e in events:
        waves.setdefault(e["tick"], []).append(e)
    decode_waves = [w for w in waves.values() if any(e["stage"] == "recurrent" for e in w)]
    assert decode_waves
    for wave in decode_waves:
        rec = [e for e in wave if e["stage"] == "recurrent"]
        sizes = [e["size"] for e in rec]
        assert sizes == sorted(sizes, reverse=True)
        assert [list(e["depths"]) for e in rec] == [[step] for step in range(len(rec))]
        codas = [e for e in wave if e["stage"] == "coda"]
        assert len(codas) == 1 and codas[0]["size"] == sum(e["exited"] for e in rec)
        preludes = [e for e in wave if e["stage"] == "prelude"]
        assert len(preludes) == 1 and preludes[0]["site"] == "wave_cohort"
        assert preludes[0]["size"] == rec[0]["size"]
        assert wave.index(preludes[0]) < wave.index(rec[0])
        assert all(e["decode"] == preludes[0]["decode"] for e in rec)
        assert codas[0]["decode"] == preludes[0]["decode"] + preludes[0]["size"]


# -- closed-form state checks on seeded workloads ------------------------------------------------------------------
def random_workload(seed: int, n: int, steps: int, vocab: int = 16):
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, vocab, int(rng.integers(1, 12))).tolist() for _ in range(n)]
    mnt = [int(m) for m in rng.integers(1, 9, size=n)]
    depths = [rng.integers(0, steps, size=m - 1).tolist() for m in mnt]
    return prompts, mnt, depths


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("use_async", [False, True])
@pytest.mark.parametrize("policy", ["single", "last_exited", "first_then_shared"])
def test_state_invariants_on_seeded_workloads(seed: int, use_async: bool, policy: str) -> None:
    steps = 4
    prompts, mnt, depths = random_workload(seed, 9, steps)
    o = ScheduleOracle(max_recurrent_steps=steps, num_blocks=96, block_size=4, max_num_batched_tokens=24,
                       max_model_len=64, max_num_seqs=5, use_async_batching=use_async, delay_gate_consumption=False,
                       synthetic_exit_replay=True, kv_policy=policy, vocab_size=16)
    r = o.run(prompts, mnt, exit_depths=depths)
    assert r["tokens"] == closed_form_tokens(prompts, depths, steps, 16)
    assert r["exit_depths"] == depths
    assert r["free_blocks_at_end"] == 96
    s = r["stats"]
    assert s["recurrent_steps"] == sum(d + 1 for ds in depths for d in ds)
    assert s["exit_kv_copies"] == (sum(d < steps - 1 for ds in depths for d in ds) if policy == "last_exited" else 0)
    slot_of = {"single": lambda t: 0, "last_exited": lambda t: t, "first_then_shared": lambda t: min(t, 1)}[policy]
    live_slots: dict[int, str] = {}
    for ev in r["events"]:
        if ev[0] == "recurrent":
            rows = ev[1]
            assert len(rows) <= 5
            assert len({row[3] for row in rows}) == len(rows)
            if policy != "single":
                assert len({slot_of(row[2]) for row in rows}) == 1  # slot-homogeneous launches
            for rid, pos, step, slot, blocks in rows:
                assert len(blocks) == -(-(pos + 1) // 4)  # exact-ceil ownership at the launch
        if ev[0] == "prelude":
            for rid, _, slot in ev[2]:
                assert slot not in live_slots
                live_slots[slot] = rid
        if ev[0] == "coda":
            for rid, _, slot in ev[1]:
                assert live_slots.pop(slot) == rid


def test_first_request_gets_the_first_blocks_fifo() -> None:
    # cache_manager.py:72-90: ids leave the free deque from its head and return to its tail.
    r = oracle(synthetic_exit_replay=True, num_blocks=8, max_num_batched_tokens=8).run(
        [[1, 2, 3], [4, 5]], 3, exit_depths=[[0, 0], [0, 0]])
    first = [ev for ev in r["events"] if ev[0] == "recurrent"][0]
    owned = {row[0]: row[4] for row in first[1]}
    assert owned["request-0"] == (0,) and owned["request-1"] == (1,)


def test_hidden_slots_come_back_lifo_after_a_coda() -> None:
    # model_runner.py:1193-1203 (test_continuous_depth_batching.py:989-1012): slots 0 and 1 are
    # freed by the coda in row order and re-used from the back.
    r = oracle(synthetic_exit_replay=True, max_num_batched_tokens=4).run([[1], [2]], 3,
                                                                          exit_depths=[[0, 0], [0, 0]])
    preludes = [ev for ev in r["events"] if ev[0] == "prelude"]
    assert [row[2] for row in preludes[0][2]] == [0, 1]
    assert [row[2] for row in preludes[1][2]] == [1, 0]
    assert r["next_hidden_slot"] == 2


def test_kv_pressure_is_out_of_scope() -> None:
    with pytest.raises(ScheduleOracleError):
        # Each 4-token prompt fills a block and its first decode token needs a second one.
        oracle(synthetic_exit_replay=True, num_blocks=3).run([[1, 2, 3, 4], [5, 6, 7, 8]], 6,
                                                             exit_depths=[[0] * 5, [0] * 5])


def test_counter_identities() -> None:
    prompts, mnt, depths = random_workload(11, 12, 3)
    r = oracle(synthetic_exit_replay=True, num_blocks=128, max_num_batched_tokens=32, max_model_len=64,
               use_async_batching=True, delay_gate_consumption=False).run(prompts, mnt, exit_depths=depths)
    s = r["stats"]
    assert s["coda_tokens"] == sum(m - 1 for m in mnt)
    assert s["prefill_coda_tokens"] == len(prompts)
    assert Counter(d for ds in depths for d in ds) == Counter(s["exit_depth_histogram"])


# -- KV pressure (test_continuous_depth_batching.py:1581-1738, test_prefill_admission.py:330-431) ----------------
PRESSURE_PROMPTS = [[1, 2], [3, 4], [5, 6], [7, 8]]


def _pressured(mode: str, depths, swap_blocks: int = 0, **over):
    kw = dict(max_recurrent_steps=3, num_blocks=6, block_size=2, max_model_len=12, safety_margin=0.0,
              synthetic_exit_replay=True, delay_gate_consumption=False, kv_pressure_mode=mode,
              swap_blocks=swap_blocks, vocab_size=16)
    kw.update(over)
    return ScheduleOracle(**kw).run(PRESSURE_PROMPTS, 8, exit_depths=depths)


@pytest.mark.parametrize("refill", [True, False])
def test_soft_reset_at_full_depth_reproduces_the_uncontended_tokens(refill: bool) -> None:
    """Four requests that each grow to 5 blocks on a 6-block cache: at full depth a soft-reset
    resume (re-prefill of prompt + generated tokens) gives the tokens of an uncontended cache."""

    full = [[2] * 7 for _ in range(4)]
    calm = _pressured("none", full, num_blocks=64, refill=refill)
    hot = _pressured("recompute", full, refill=refill)
    assert hot["stats"]["recompute_preemptions"] > 0 and hot["stats"]["offload_preemptions"] == 0
    assert hot["tokens"] == calm["tokens"]
    assert hot["free_blocks_at_end"] == 6
    assert all(len(t) == 8 for t in hot["tokens"])


@pytest.mark.parametrize("refill", [True, False])
def test_swap_reproduces_the_uncontended_tokens_at_any_exit_schedule(refill: bool) -> None:
    varied = [[0, 1, 2, 1, 0, 2, 1] for _ in range(4)]
    calm = _pressured("none", varied, num_blocks=64, refill=refill)
    hot = _pressured("offload", varied, swap_blocks=64, refill=refill)
    s = hot["stats"]
    assert s["offload_preemptions"] > 0 and s["restores"] == s["offload_preemptions"]
    assert s["recompute_preemptions"] == 0
    assert hot["tokens"] == calm["tokens"] and hot["exit_depths"] == calm["exit_depths"]


def test_a_full_host_pool_falls_back_to_soft_reset_unless_exits_rewrite_kv() -> None:
    varied = [[0, 1, 2, 1, 0, 2, 1] for _ in range(4)]
    hot = _pressured("offload", varied, swap_blocks=1)
    assert hot["stats"]["recompute_preemptions"] > 0
    with pytest.raises(ScheduleOracleError):
        _pressured("offload", varied, swap_blocks=1, kv_policy="last_exited")


def test_a_single_request_that_cannot_fit_is_an_error() -> None:
    with pytest.raises(ScheduleOracleError, match="single request"):
        ScheduleOracle(max_recurrent_steps=3, num_blocks=2, block_size=2, max_model_len=12, safety_margin=0.0,
                       kv_pressure_mode="recompute").run([[1, 2]], 8)


def test_no_refill_delayed_wave_cancels_the_successor_of_a_late_eos() -> None:
    # test_continuous_depth_batching.py:596-624: on the delayed horizon an EOS is read only with
    # the boundary coda, one wave after its successor entered; request 2's first token is the EOS,
    # read after its carried successor was built, which is then dropped at the next wave's entry.
    prompts = [[1], [4], [5]]
    depths = [[0] * 5, [1] * 5, [0] * 5]
    kw = dict(synthetic_exit_replay=True, replay_offset_one=True)
    refill = oracle(**kw).run(prompts, 6, eos_token_id=8, exit_depths=depths)
    wave = oracle(**kw, refill=False).run(prompts, 6, eos_token_id=8, exit_depths=depths)
    assert wave["tokens"] == refill["tokens"]
    assert wave["tokens"][2] == [8]
    assert any(t and t[-1] == 8 for t in wave["tokens"])
    assert wave["stats"]["cancelled_depth_items"] > 0
    # One recurrent step for the cancelled successor (cancelled at step 0, after the launch) and
    # two for request 2's first decode token (depth 0 applied one step late) before its EOS is read.
    assert wave["stats"]["recurrent_steps"] == refill["stats"]["recurrent_steps"] + 3
    assert wave["stats"]["scheduler_refills"] == 0
    assert set(wave["stats"]["prelude_tokens"]) == {"wave_cohort"}
    assert wave["free_blocks_at_end"] == 16
