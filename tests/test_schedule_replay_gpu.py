"""Bit-exact schedule replay of the GPU engine against the schedule oracle.

The engine runs the real kernels (Ouro models on the MI355X); the oracle (oracle/scheduler.py,
pinned by tests/test_oracle_scheduler.py) restates the reference's scheduling on the host. With
staged results consumed at the next consume point (``consume_all_results``), the schedule is a
function of the inputs alone, so every launch must match: kind, rows in launch order, token
positions, loop steps, hidden-state slots, block ids, exit decisions, prelude sites and the
running refill count. Exit depths must equal the replayed trace.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.scheduler import ScheduleOracle

pytestmark = pytest.mark.gpu


def engine_for(model, **cfg):
    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine

    engine = ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(**cfg))
    engine.record_launches = True
    engine.consume_all_results = True
    return engine


ORACLE_KEYS = ("max_recurrent_steps", "num_blocks", "block_size", "max_num_batched_tokens", "max_model_len",
               "max_num_seqs", "min_free_slots", "min_coda_batch_size", "safety_margin", "kv_policy",
               "kv_slots_per_layer", "refill", "use_async_batching", "delay_gate_consumption",
               "synthetic_exit_replay", "exit_threshold")


def replay_and_compare(model, prompts, mnt, depths, **cfg):
    engine = engine_for(model, **cfg)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    torch.cuda.synchronize()
    o = ScheduleOracle(**{k: v for k, v in cfg.items() if k in ORACLE_KEYS}).run(prompts, mnt, exit_depths=depths)
    got, want = engine.launch_log, o["events"]
    for k, (g, w) in enumerate(zip(got, want)):
        assert g == w, f"launch {k} of {len(want)} differs:\n engine {g}\n oracle {w}"
    assert len(got) == len(want)
    # Replayed depths exit at their step, or one launch later on the delayed horizon.
    delayed = cfg.get("delay_gate_consumption", True) and cfg.get("use_async_batching", True)
    steps = cfg["max_recurrent_steps"]
    want_depths = [[min(d + 1, steps - 1) for d in ds] for ds in depths] if delayed else depths
    assert [out.exit_depths for out in outs] == o["exit_depths"] == want_depths
    s = engine.last_stats
    assert s.recurrent_steps == o["stats"]["recurrent_steps"] == sum(d + 1 for ds in want_depths for d in ds)
    assert s.scheduler_refills == o["stats"]["scheduler_refills"]
    assert s.exit_kv_copies == o["stats"]["exit_kv_copies"]
    assert engine.cache.get_num_free_blocks() == engine.cache.num_blocks
    return engine, outs, o


@pytest.mark.parametrize("policy,use_async,delay,refill", [
    ("single", True, False, True), ("single", False, False, True), ("single", True, True, True),
    ("last_exited", True, False, True), ("last_exited", True, True, True), ("single", False, False, False),
    ("last_exited", False, False, False), ("single", True, True, False), ("last_exited", True, True, False)])
def test_tiny_ouro_schedule_replay(policy, use_async, delay, refill) -> None:
    from tests.test_engine_gpu import build_model

    model, _ = build_model(seed=2)
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 49152, int(n)).tolist() for n in rng.integers(4, 90, size=20)]
    mnt = [int(m) for m in rng.integers(2, 24, size=20)]
    depths = [rng.integers(0, 4, size=m - 1).tolist() for m in mnt]
    replay_and_compare(model, prompts, mnt, depths, max_recurrent_steps=4, num_blocks=400, block_size=16,
                       max_model_len=512, max_num_seqs=8, max_num_batched_tokens=256, kv_policy=policy,
                       refill=refill, use_async_batching=use_async, delay_gate_consumption=delay,
                       synthetic_exit_replay=True, kv_pressure_mode="none")


def test_headline_workload_schedule_replay() -> None:
    """The 256-sequence Ouro-1.4B-shape decode workload, bf16, refill, shared KV."""

    from continuous_depth_batching_amd.ouro import build_ouro, ouro_1p4b_config
    from continuous_depth_batching_amd.workloads import ouro_decode_workload

    cfg = ouro_1p4b_config()
    model = build_ouro(cfg, seed=1, dtype=torch.bfloat16, device="cuda")
    prompts, mnt, depths = ouro_decode_workload(256, cfg.vocab_size)
    blocks = int(sum(-(-(len(p) + o + 1) // 16) for p, o in zip(prompts, mnt)) * 1.05) + 64
    engine, outs, o = replay_and_compare(
        model, prompts, mnt, depths, max_recurrent_steps=4, num_blocks=blocks, block_size=16, max_model_len=4096,
        max_num_seqs=256, kv_policy="single", refill=True, synthetic_exit_replay=True,
        delay_gate_consumption=False, kv_pressure_mode="none")
    recurrent = [ev for ev in engine.launch_log if ev[0] == "recurrent"]
    wide = [ev for ev in recurrent if len(ev[1]) > 128]
    assert wide, "the workload must reach the 256-row bucket"
    assert max(len({row[2] for row in ev[1]}) for ev in wide) >= 3  # mixed loop steps in wide launches
    assert sum(len(out.generated_tokens) for out in outs) == sum(mnt)
    print(f"\n[headline replay] {len(engine.launch_log)} launches, {len(recurrent)} recurrent, "
          f"{len(wide)} above 128 rows, refills {engine.last_stats.scheduler_refills}", flush=True)
    del engine
    torch.cuda.empty_cache()


def test_ouro_2p6b_shape_last_exited_schedule_replay_and_exit_copies() -> None:
    """48 layers, per-step KV with exit copies: the launch schedule and the copy count against the
    oracle, and refill against no-refill token streams.

    Sixteen sequences whose prompts fit one prefill batch, at launch widths up to 16 rows: every
    kernel then computes a row the same way whatever else shares its launch, so the two loops must
    produce identical tokens (the reference's own GPU refill tests run at such widths)."""

    from continuous_depth_batching_amd.ouro import build_ouro, ouro_1p4b_config
    from continuous_depth_batching_amd.workloads import ouro_decode_workload

    cfg = ouro_1p4b_config(num_hidden_layers=48)
    model = build_ouro(cfg, seed=1, dtype=torch.bfloat16, device="cuda")
    prompts, mnt, depths = ouro_decode_workload(16, cfg.vocab_size)
    prompts = [p[:400] for p in prompts]
    mnt = [min(m, 48) for m in mnt]
    depths = [d[: m - 1] for d, m in zip(depths, mnt)]
    assert sum(map(len, prompts)) <= 8192
    blocks = int(sum(-(-(len(p) + o + 1) // 16) for p, o in zip(prompts, mnt)) * 1.1) + 64
    common = dict(max_recurrent_steps=4, num_blocks=blocks, block_size=16, max_model_len=4096, max_num_seqs=16,
                  kv_policy="last_exited", synthetic_exit_replay=True, delay_gate_consumption=False,
                  kv_pressure_mode="none")
    engine, outs, o = replay_and_compare(model, prompts, mnt, depths, refill=True, **common)
    copies = sum(d < 3 for ds in depths for d in ds)
    assert engine.last_stats.exit_kv_copies == copies > 0
    refill_tokens = [out.generated_tokens for out in outs]
    del engine
    wave, wave_outs, _ = replay_and_compare(model, prompts, mnt, depths, refill=False, **common)
    assert wave.last_stats.scheduler_refills == 0
    assert wave.last_stats.exit_kv_copies == copies
    assert [out.generated_tokens for out in wave_outs] == refill_tokens


def test_huginn_0125_workload_schedule_replay() -> None:
    """The Huginn-0125 decode workload at its own size: 128 sequences x 256 new tokens, exit steps
    replayed from Poisson(12) truncated to [1, 32], shared KV, refill, bf16 (huginn/modeling_huginn.py
    through cdb/adapters/huginn.py:121-176). Every launch, exit depth, the refill count and the free
    blocks at the end equal the schedule oracle's."""

    from continuous_depth_batching_amd.huginn import HuginnConfig, build_huginn
    from continuous_depth_batching_amd.workloads import huginn_decode_workload

    cfg = HuginnConfig(block_size=2048, state_init="random", state_seed=1)
    model = build_huginn(cfg, seed=1, dtype=torch.bfloat16, device="cuda", qk_bias_std=0.02)
    prompts, mnt, depths = huginn_decode_workload(128, 256, cfg.vocab_size)
    blocks = int(sum(-(-(len(p) + o + 1) // 16) for p, o in zip(prompts, mnt)) * 1.05) + 64
    engine, outs, o = replay_and_compare(
        model, prompts, mnt, depths, max_recurrent_steps=32, num_blocks=blocks, block_size=16, max_model_len=2048,
        max_num_seqs=128, kv_policy="single", refill=True, synthetic_exit_replay=True,
        delay_gate_consumption=False, kv_pressure_mode="none")
    recurrent = [ev for ev in engine.launch_log if ev[0] == "recurrent"]
    assert max(len(ev[1]) for ev in recurrent) == 128
    assert max(len({row[2] for row in ev[1]}) for ev in recurrent) >= 8  # many loop steps share launches
    assert sum(len(out.generated_tokens) for out in outs) == sum(mnt)
    print(f"\n[huginn-0125 replay] {len(engine.launch_log)} launches, {len(recurrent)} recurrent, "
          f"refills {engine.last_stats.scheduler_refills}", flush=True)
    del engine, model
    torch.cuda.empty_cache()


def test_ouro_2p6b_512_sequence_single_kv_schedule_replay() -> None:
    """The 512-sequence Ouro-2.6B-shape workload (48 layers looped 4 steps) with shared KV and a
    pool sized for the batch, at its own size: every launch, exit depth, the refill count and the
    free blocks at the end equal the schedule oracle's."""

    from continuous_depth_batching_amd.ouro import build_ouro, ouro_1p4b_config
    from continuous_depth_batching_amd.workloads import ouro_decode_workload

    cfg = ouro_1p4b_config(num_hidden_layers=48)
    model = build_ouro(cfg, seed=1, dtype=torch.bfloat16, device="cuda")
    prompts, mnt, depths = ouro_decode_workload(512, cfg.vocab_size)
    blocks = int(sum(-(-(len(p) + o + 1) // 16) for p, o in zip(prompts, mnt)) * 1.05) + 64
    engine, outs, o = replay_and_compare(
        model, prompts, mnt, depths, max_recurrent_steps=4, num_blocks=blocks, block_size=16, max_model_len=4096,
        max_num_seqs=512, kv_policy="single", refill=True, synthetic_exit_replay=True,
        delay_gate_consumption=False, kv_pressure_mode="none")
    recurrent = [ev for ev in engine.launch_log if ev[0] == "recurrent"]
    assert max(len(ev[1]) for ev in recurrent) > 256  # the 512-row buckets are reached
    assert sum(len(out.generated_tokens) for out in outs) == sum(mnt)
    print(f"\n[ouro-2.6b 512 replay] {len(engine.launch_log)} launches, {len(recurrent)} recurrent, "
          f"refills {engine.last_stats.scheduler_refills}", flush=True)
    del engine, model
    torch.cuda.empty_cache()


def test_ouro_2p6b_shape_per_step_kv_under_pressure_schedule_replay() -> None:
    """The per-step workload under KV pressure: Ouro-2.6B shape (48 layers), last_exited KV with
    exit copies, 64 sequences of the headline distributions on a pool of a third of the blocks
    they need with no admission margin, offload to a pinned host pool (a soft reset would replace exit-step KV). Every launch,
    every swap-out and restore, the exit-copy count and the free blocks at the end equal the
    schedule oracle's run with the same host pool."""

    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine
    from continuous_depth_batching_amd.ouro import build_ouro, ouro_1p4b_config
    from continuous_depth_batching_amd.workloads import ouro_decode_workload

    cfg = ouro_1p4b_config(num_hidden_layers=48)
    model = build_ouro(cfg, seed=1, dtype=torch.bfloat16, device="cuda")
    prompts, mnt, depths = ouro_decode_workload(64, cfg.vocab_size)
    prompts = [p[:600] for p in prompts]
    mnt = [min(m, 96) for m in mnt]
    depths = [d[: m - 1] for d, m in zip(depths, mnt)]
    need = sum(-(-(len(p) + o + 1) // 16) for p, o in zip(prompts, mnt))
    common = dict(max_recurrent_steps=4, num_blocks=need // 3, block_size=16, max_model_len=4096, max_num_seqs=64,
                  kv_policy="last_exited", refill=True, synthetic_exit_replay=True, delay_gate_consumption=False,
                  kv_pressure_mode="offload", safety_margin=0.0)
    engine = ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(
        cpu_offload_space=64.0, **common))
    engine.record_launches = True
    engine.consume_all_results = True
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    torch.cuda.synchronize()
    om = engine.offloading_manager
    want = ScheduleOracle(swap_blocks=om.num_cpu_blocks, **{k: v for k, v in common.items() if k != "kv_pressure_mode"},
                          kv_pressure_mode="offload").run(prompts, mnt, exit_depths=depths)
    for k, (g, w) in enumerate(zip(engine.launch_log, want["events"])):
        assert g == w, f"launch {k} of {len(want['events'])} differs:\n engine {g}\n oracle {w}"
    assert len(engine.launch_log) == len(want["events"])
    assert [o.exit_depths for o in outs] == want["exit_depths"] == depths
    s, ws = engine.last_stats, want["stats"]
    assert s.exit_kv_copies == ws["exit_kv_copies"] > 0
    assert om.num_offload_preemptions == ws["offload_preemptions"] > 0
    assert om.num_restores == ws["restores"] == om.num_offload_preemptions
    assert om.num_recompute_preemptions == ws["recompute_preemptions"] == 0
    assert engine.cache.get_num_free_blocks() == engine.cache.num_blocks == want["free_blocks_at_end"]
    print(f"\n[per-step pressure replay] {len(engine.launch_log)} launches, {om.num_offload_preemptions} swaps, "
          f"{s.exit_kv_copies} exit copies", flush=True)
    del engine, model
    torch.cuda.empty_cache()
