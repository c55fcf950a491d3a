"""The product engine's launch schedule against the schedule oracle, without a GPU.

The engine (scheduler, block manager, hidden slots, tick core, routing) runs on the host
runner of tests/host_runner.py with the token-increment model; the oracle
(oracle/scheduler.py, pinned by tests/test_oracle_scheduler.py) restates the reference's
scheduling independently. Every launch must match bit for bit: its kind, rows in launch order,
positions, loop steps, hidden-state slots, block ids, exit decisions, prelude sites and the
running refill count.
"""

from __future__ import annotations

import numpy as np
import pytest

from continuous_depth_batching_amd.exit_policy import DecisionHorizon, ExitDecisionRule, ExitPolicySpec
from oracle.scheduler import DIRECT, HAZARD, ScheduleOracle
from tests.host_runner import make_engine

VOCAB = 16


def workload(seed: int, n: int, steps: int, *, min_depth: int = 0, long_prompts: bool = False):
    rng = np.random.default_rng(seed)
    top = 40 if long_prompts else 14
    prompts = [rng.integers(0, VOCAB, int(rng.integers(1, top))).tolist() for _ in range(n)]
    mnt = [int(m) for m in rng.integers(1, 10, size=n)]
    depths = [rng.integers(min_depth, steps, size=m - 1).tolist() for m in mnt]
    return prompts, mnt, depths


def run_both(cfg: dict, prompts, mnt, *, depths=None, eos=None, rule=HAZARD, offset_one=False):
    spec = ExitPolicySpec(ExitDecisionRule.DIRECT_THRESHOLD if rule == DIRECT else ExitDecisionRule.CUMULATIVE_HAZARD,
                          DecisionHorizon.OFFSET_ONE if offset_one else DecisionHorizon.SAME_STEP)
    engine = make_engine(spec=spec, **cfg)
    engine.record_launches = True
    engine.consume_all_results = True
    outs = engine.generate_batch([list(p) for p in prompts], max_new_tokens=mnt, eos_token_id=eos,
                                 exit_depths=depths)
    okw = {k: v for k, v in cfg.items() if k not in ("use_cuda_graph", "kv_pressure_mode")}
    okw.setdefault("num_blocks", 16)
    okw.setdefault("block_size", 4)
    okw.setdefault("max_num_batched_tokens", 4)
    okw.setdefault("max_model_len", 16)
    okw.setdefault("use_async_batching", False)
    okw.setdefault("max_recurrent_steps", 3)
    want = ScheduleOracle(**okw, rule=rule, offset_one_signal=offset_one, vocab_size=VOCAB).run(
        prompts, mnt, eos_token_id=eos, exit_depths=depths)
    return engine, outs, want


def assert_same_schedule(engine, outs, want) -> None:
    got = engine.launch_log
    for k, (g, w) in enumerate(zip(got, want["events"])):
        assert g == w, f"launch {k} differs:\n engine {g}\n oracle {w}"
    assert len(got) == len(want["events"])
    assert [o.generated_tokens for o in outs] == want["tokens"]
    assert [o.exit_depths for o in outs] == want["exit_depths"]
    s, ws = engine.last_stats, want["stats"]
    assert s.recurrent_steps == ws["recurrent_steps"]
    assert s.recurrent_batches == ws["recurrent_batches"]
    assert s.coda_tokens == ws["coda_tokens"] and s.coda_batches == ws["coda_batches"]
    assert s.scheduler_refills == ws["scheduler_refills"]
    assert s.cancelled_depth_items == ws["cancelled_depth_items"]
    assert s.exit_kv_copies == ws["exit_kv_copies"]
    assert dict(s.prelude_tokens) == ws["prelude_tokens"]
    assert engine.cache.get_num_free_blocks() == want["free_blocks_at_end"]


BIG = dict(num_blocks=160, block_size=4, max_num_batched_tokens=24, max_model_len=64, max_recurrent_steps=4,
           kv_pressure_mode="none")


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("use_async", [False, True])
@pytest.mark.parametrize("refill", [True, False])
@pytest.mark.parametrize("policy", ["single", "last_exited", "first_then_shared"])
def test_replay_schedule_matches_on_the_synchronous_horizon(seed, use_async, refill, policy) -> None:
    min_depth = 1 if policy == "first_then_shared" else 0  # every depth must write both shared slots
    prompts, mnt, depths = workload(seed, 10, 4, min_depth=min_depth)
    cfg = dict(BIG, max_num_seqs=6, kv_policy=policy, refill=refill, use_async_batching=use_async,
               delay_gate_consumption=False, synthetic_exit_replay=True)
    assert_same_schedule(*run_both(cfg, prompts, mnt, depths=depths))


@pytest.mark.parametrize("seed", range(4))
def test_replay_schedule_matches_on_the_delayed_horizon(seed) -> None:
    prompts, mnt, depths = workload(seed + 10, 10, 4)
    cfg = dict(BIG, max_num_seqs=6, kv_policy="last_exited", use_async_batching=True,
               delay_gate_consumption=True, synthetic_exit_replay=True)
    assert_same_schedule(*run_both(cfg, prompts, mnt, depths=depths))


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("use_async", [False, True])
def test_chunked_prefill_eos_and_min_coda_batches(seed, use_async) -> None:
    prompts, mnt, depths = workload(seed + 20, 9, 4, long_prompts=True)
    cfg = dict(BIG, max_num_batched_tokens=16, max_num_seqs=5, min_coda_batch_size=3, use_async_batching=use_async,
               delay_gate_consumption=False, synthetic_exit_replay=True)
    assert_same_schedule(*run_both(cfg, prompts, mnt, depths=depths, eos=5))


@pytest.mark.parametrize("rule,threshold", [(HAZARD, 0.5), (DIRECT, 0.0)])
@pytest.mark.parametrize("use_async,delay", [(False, False), (True, False), (True, True)])
@pytest.mark.parametrize("refill", [True, False])
def test_live_gate_schedule_matches(rule, threshold, use_async, delay, refill) -> None:
    if not refill and delay:
        pytest.skip("the oracle restates the no-refill loop on the synchronous horizon")
    prompts, mnt, _ = workload(31, 8, 3)
    cfg = dict(BIG, max_recurrent_steps=3, max_num_seqs=4, refill=refill, use_async_batching=use_async,
               delay_gate_consumption=delay, exit_threshold=threshold)
    assert_same_schedule(*run_both(cfg, prompts, mnt, rule=rule, eos=7))


def test_reference_small_config_schedule_matches() -> None:
    # The reference tests' own config (test_continuous_depth_batching.py:150-161) and trace fixture
    # (test_schedule_trace.py:13-15).
    prompts = [[1, 2], [5], [3, 4, 5], [6]]
    depths = [[0, 2, 1], [2, 0, 2], [1, 1, 0], [2, 2, 1]]
    for refill in (True, False):
        cfg = dict(synthetic_exit_replay=True, refill=refill, max_num_seqs=3)
        assert_same_schedule(*run_both(cfg, prompts, 4, depths=depths))


@pytest.mark.parametrize("mistake", ["fifo_hidden_slots", "tail_reinsertion", "lifo_blocks"])
def test_the_comparison_catches_a_planted_scheduling_mistake(monkeypatch, mistake) -> None:
    """A plausible scheduling mistake, planted in the oracle, must make the comparison fail."""

    import oracle.scheduler as sched

    if mistake == "fifo_hidden_slots":
        def take(self, items):
            for it in items:
                if self.free_slots:
                    it.slot = self.free_slots.pop(0)
                else:
                    it.slot = self.next_slot
                    self.next_slot += 1
        monkeypatch.setattr(sched.ScheduleOracle, "_take_slots", take)
    elif mistake == "tail_reinsertion":
        monkeypatch.setattr(sched.ScheduleOracle, "_push_front",
                            lambda self, items: [self._push(it, False) for it in items])
    else:
        def grow_one(self, r):
            if r.blocks and len(r.blocks) * self.bs - r.pos >= 1:
                return True
            want = -(-(r.pos + 1) // self.bs) - len(r.blocks)
            if want > len(self.free_blocks):
                return False
            r.blocks.extend(self.free_blocks.pop() for _ in range(want))
            return True
        monkeypatch.setattr(sched.ScheduleOracle, "_grow_one", grow_one)
    prompts, mnt, depths = workload(3, 10, 4)
    cfg = dict(BIG, max_num_seqs=4, use_async_batching=True, delay_gate_consumption=False,
               synthetic_exit_replay=True)
    with pytest.raises(AssertionError):
        assert_same_schedule(*run_both(cfg, prompts, mnt, depths=depths))


@pytest.mark.parametrize("seed", range(3))
@pytest.mark.parametrize("policy", ["last_exited", "first_then_shared"])
def test_mixed_slot_launches_match_the_oracle_and_keep_results(seed, policy) -> None:
    """With mixed-slot launches the schedule still matches the oracle run with the same option,
    launches do mix KV slots, and tokens and exit depths equal the slot-homogeneous run's."""

    min_depth = 1 if policy == "first_then_shared" else 0
    prompts, mnt, depths = workload(seed + 40, 10, 4, min_depth=min_depth)
    base = dict(BIG, max_num_seqs=6, kv_policy=policy, use_async_batching=True, delay_gate_consumption=False,
                synthetic_exit_replay=True)
    engine, outs, want = run_both(dict(base, mixed_slot_recurrent_batches=True), prompts, mnt, depths=depths)
    assert_same_schedule(engine, outs, want)
    slot = (lambda t: t) if policy == "last_exited" else (lambda t: min(t, 1))
    mixed = [ev for ev in engine.launch_log if ev[0] == "recurrent" and len({slot(r[2]) for r in ev[1]}) > 1]
    assert mixed
    _, homogeneous, _ = run_both(base, prompts, mnt, depths=depths)
    assert [o.generated_tokens for o in outs] == [o.generated_tokens for o in homogeneous]
    assert [o.exit_depths for o in outs] == [o.exit_depths for o in homogeneous]
