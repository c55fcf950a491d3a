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
@pytest.mark.parametrize("refill", [True, False])
def test_replay_schedule_matches_on_the_delayed_horizon(seed, refill) -> None:
    """On the delayed horizon without refill, each wave carries its coda, the prompts' first
    tokens and the successors built ahead of them into the next wave (continuous_api.py:808-944)."""

    prompts, mnt, depths = workload(seed + 10, 10, 4)
    cfg = dict(BIG, max_num_seqs=6, kv_policy="last_exited", use_async_batching=True,
               delay_gate_consumption=True, synthetic_exit_replay=True, refill=refill)
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


# -- KV pressure: parking, preemption (swap or soft reset) and restores -------------------------------------------
PRESSURED = dict(num_blocks=8, block_size=4, max_num_batched_tokens=16, max_model_len=48, max_recurrent_steps=4,
                 safety_margin=0.0, max_num_seqs=6, synthetic_exit_replay=True, delay_gate_consumption=False)


def _host_pool_gib(blocks: int, **cfg) -> float:
    """cpu_offload_space that holds exactly ``blocks`` KV blocks of this engine's cache."""

    probe = make_engine(kv_pressure_mode="offload", cpu_offload_space=1.0, **cfg)
    return (blocks * probe.offloading_manager.bytes_per_block() + 1) / 1024 ** 3


def run_pressured(cfg: dict, prompts, mnt, depths):
    engine = make_engine(**cfg)
    engine.record_launches = True
    engine.consume_all_results = True
    outs = engine.generate_batch([list(p) for p in prompts], max_new_tokens=mnt, eos_token_id=None,
                                 exit_depths=depths)
    okw = {k: v for k, v in cfg.items() if k not in ("use_cuda_graph", "cpu_offload_space")}
    want = ScheduleOracle(**okw, vocab_size=VOCAB, swap_blocks=engine.offloading_manager.num_cpu_blocks).run(
        prompts, mnt, exit_depths=depths)
    return engine, outs, want


PRESSURE_CASES = {"recompute": ("recompute", 0), "offload": ("offload", 64), "offload-small-pool": ("offload", 2)}


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("use_async", [False, True])
@pytest.mark.parametrize("refill", [True, False])
@pytest.mark.parametrize("case", sorted(PRESSURE_CASES))
def test_replay_schedule_matches_under_kv_pressure(seed, use_async, refill, case) -> None:
    """An over-subscribed cache (8 blocks of 4 tokens for 10 requests of up to 22 tokens): every
    launch, every preemption's effect on the queues and blocks, and the tokens equal the oracle's,
    with decoders parked and retried, the least-computed one preempted, swapped to a host pool
    when it holds its blocks (restored first on later ticks) and soft-reset otherwise."""

    mode, pool = PRESSURE_CASES[case]
    prompts, mnt, depths = workload(seed + 40, 10, 4)
    cfg = dict(PRESSURED, refill=refill, use_async_batching=use_async, kv_pressure_mode=mode)
    if pool:
        cfg["cpu_offload_space"] = _host_pool_gib(pool, **PRESSURED)
    engine, outs, want = run_pressured(cfg, prompts, mnt, depths)
    assert_same_schedule(engine, outs, want)
    om, ws = engine.offloading_manager, want["stats"]
    assert om.num_offload_preemptions == ws["offload_preemptions"]
    assert om.num_recompute_preemptions == ws["recompute_preemptions"]
    assert om.num_restores == ws["restores"]


def test_pressure_replays_exercise_every_preemption_path() -> None:
    """Across the seeds above, each case preempts, the small pool both swaps and soft-resets, and
    swapped requests come back."""

    seen = {case: [0, 0, 0] for case in PRESSURE_CASES}
    for case, (mode, pool) in PRESSURE_CASES.items():
        for seed in range(4):
            prompts, mnt, depths = workload(seed + 40, 10, 4)
            cfg = dict(PRESSURED, refill=True, use_async_batching=True, kv_pressure_mode=mode)
            if pool:
                cfg["cpu_offload_space"] = _host_pool_gib(pool, **PRESSURED)
            _, _, want = run_pressured(cfg, prompts, mnt, depths)
            s = want["stats"]
            seen[case] = [a + b for a, b in zip(seen[case], (s["offload_preemptions"], s["recompute_preemptions"],
                                                              s["restores"]))]
    assert seen["recompute"][1] > 0 and seen["recompute"][0] == 0
    assert seen["offload"][0] > 0 and seen["offload"][1] == 0 and seen["offload"][2] == seen["offload"][0]
    assert seen["offload-small-pool"][0] > 0 and seen["offload-small-pool"][1] > 0


DELAYED_WAVE = dict(BIG, max_num_seqs=6, kv_policy="last_exited", use_async_batching=True,
                    delay_gate_consumption=True, synthetic_exit_replay=True, refill=False)


def test_delayed_waves_exercise_every_carry_path() -> None:
    """The delayed no-refill replays must reach successors gathered from a carried coda or
    prompt, and successors cancelled by a finish read one wave late."""

    gathered = cancelled = 0
    for seed in range(4):
        prompts, mnt, depths = workload(seed + 10, 10, 4)
        engine, outs, want = run_both(DELAYED_WAVE, prompts, mnt, depths=depths, eos=5)
        assert_same_schedule(engine, outs, want)
        gathered += engine.last_stats.prelude_gathered_tokens["wave_cohort"]
        cancelled += engine.last_stats.cancelled_depth_items
    assert gathered > 0 and cancelled > 0


@pytest.mark.parametrize("mistake", ["coda_read_before_the_wave", "successors_reversed", "no_coda_successors"])
def test_the_delayed_wave_comparison_catches_a_planted_mistake(monkeypatch, mistake) -> None:
    """A plausible mistake in the wave-boundary carry, planted in the oracle, must make the
    comparison fail: the last wave's coda read before the next wave's prelude (as on the
    synchronous horizon), the carried successors entering in reverse order, or no successors
    built for a wave's coda rows."""

    import oracle.scheduler as sched

    if mistake == "no_coda_successors":
        monkeypatch.setattr(sched.ScheduleOracle, "_successors", lambda self, staged: [])
    else:
        original = sched.ScheduleOracle._wave

        def planted(self, delayed):
            if mistake == "successors_reversed":
                self.ahead = self.ahead[::-1]
            elif self.unread_coda is not None:
                coda, self.unread_coda = self.unread_coda, None
                self._consume_coda(coda, restage=False)
            return original(self, delayed)
        monkeypatch.setattr(sched.ScheduleOracle, "_wave", planted)
    failures = 0
    for seed in range(4):
        prompts, mnt, depths = workload(seed + 10, 10, 4)
        try:
            assert_same_schedule(*run_both(DELAYED_WAVE, prompts, mnt, depths=depths, eos=5))
        except (AssertionError, sched.ScheduleOracleError):
            failures += 1
    assert failures > 0


@pytest.mark.parametrize("mistake", ["first_parked_victim", "soft_reset_keeps_cursor", "restore_after_prompts"])
def test_the_pressure_comparison_catches_a_planted_mistake(monkeypatch, mistake) -> None:
    """A plausible preemption mistake, planted in the oracle, must make the comparison fail: the
    first parked request as the victim instead of the least-computed one, a soft reset that
    replays the pending token's depth again, restores that wait behind fresh prompts."""

    import oracle.scheduler as sched

    case = "offload" if mistake == "restore_after_prompts" else "recompute"
    if mistake == "first_parked_victim":
        original = sched.ScheduleOracle._yield_parked

        def first(self):
            rid = next(iter(self.parked))
            keep = {k: v for k, v in self.parked.items()}
            self.parked = {rid: keep[rid]}  # the restated rule then has one candidate
            original(self)
            self.parked = {k: v for k, v in keep.items() if k != rid}
        monkeypatch.setattr(sched.ScheduleOracle, "_yield_parked", first)
    elif mistake == "soft_reset_keeps_cursor":
        original = sched.ScheduleOracle._yield_parked

        def keep_cursor(self):
            before = {rid: (r.depths, r.cursor) for rid, r in self.parked.items()}
            original(self)
            for rid, (depths, cursor) in before.items():
                r = self.waiting.get(rid)
                if r is not None and r.status == "pending" and not r.offloaded:
                    r.depths = depths[cursor:]
        monkeypatch.setattr(sched.ScheduleOracle, "_yield_parked", keep_cursor)
    else:
        original = sched.ScheduleOracle._restore

        def late(self):
            if any(not r.offloaded for r in self.waiting.values()):
                return []  # fresh prompts first
            return original(self)
        monkeypatch.setattr(sched.ScheduleOracle, "_restore", late)
    mode, pool = PRESSURE_CASES[case]
    failures = 0
    for seed in range(4):
        prompts, mnt, depths = workload(seed + 40, 10, 4)
        cfg = dict(PRESSURED, refill=True, use_async_batching=True, kv_pressure_mode=mode)
        if pool:
            cfg["cpu_offload_space"] = _host_pool_gib(pool, **PRESSURED)
        try:
            assert_same_schedule(*run_pressured(cfg, prompts, mnt, depths))
        except (AssertionError, sched.ScheduleOracleError):
            failures += 1
    assert failures > 0
