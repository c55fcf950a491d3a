"""KV-pressure preemption on the host: soft reset (recompute) and swap to the host pool (offload).

Cases and expected outcomes follow the reference's own tests
(tests/continuous_depth_batching/test_continuous_depth_batching.py:1581-1738 and
test_prefill_admission.py:330-431) on the same token-increment model: at full
depth a soft-reset resume reproduces the uncontended tokens, a swap reproduces
them at any exit schedule, and every request completes on an over-subscribed
cache. The engine, scheduler and preemption bookkeeping are the product's code;
tests/host_runner.py supplies the stage arithmetic and moves swapped blocks with
tensor indexing in the product's host-pool layout.
"""

from __future__ import annotations

import pytest
import torch

from continuous_depth_batching_amd.cache import CacheFullError
from continuous_depth_batching_amd.offloading import host_block_runs
from continuous_depth_batching_amd.requests import RequestState, RequestStatus
from tests.host_runner import make_engine

# Four requests that each grow to 5 blocks (prompt 2 + 8 generated = 10 tokens, block_size 2) on a
# 6-block cache: any two decoding at once over-subscribe it, while one alone fits.
OVERSUBSCRIBED = dict(num_blocks=6, block_size=2, max_model_len=12, safety_margin=0.0)
PROMPTS = [[1, 2], [3, 4], [5, 6], [7, 8]]
FULL_DEPTH = [[2] * 7 for _ in range(4)]
VARIED = [[0, 1, 2, 1, 0, 2, 1] for _ in range(4)]


def replay(prompts, depths, max_new_tokens, **cfg):
    engine = make_engine(synthetic_exit_replay=True, **cfg)
    outs = engine.generate_batch([list(p) for p in prompts], max_new_tokens=max_new_tokens, eos_token_id=None,
                                 exit_depths=depths)
    return engine, outs


def tokens_of(outs):
    return [o.generated_tokens for o in outs]


# -- request transitions (test_continuous_depth_batching.py:1680-1738) -------------------------------------------
def _decoding_state() -> RequestState:
    state = RequestState(request_id="r", initial_tokens=[1, 2], max_new_tokens=5,
                         synthetic_exit_depths=[10, 11, 12, 13, 14])
    state._status = RequestStatus.DECODING
    for token in (101, 102):
        state.next_synthetic_exit_depth()
        state.generated_tokens.append(token)
    state.generated_tokens.append(103)  # pending token; its depth (cursor 2) is not consumed yet
    state.tokens_to_process = [103]
    return state


def test_recompute_resume_drops_the_pending_tokens_replayed_exit_depth() -> None:
    fresh = _decoding_state().create_equivalent_initial_request()
    assert fresh.initial_tokens == [1, 2, 101, 102, 103]
    assert fresh.remaining_prefill_tokens == [1, 2, 101, 102, 103]
    assert fresh.max_new_tokens == 2
    assert fresh.synthetic_exit_depths == [13, 14]
    assert fresh.prompt_len() == 2
    assert fresh.status == RequestStatus.PENDING
    out = fresh.to_generation_output()
    assert out.prompt_ids == [1, 2] and out.generated_tokens == [101, 102, 103]


def test_recompute_resume_keeps_the_requests_timing_identity() -> None:
    state = RequestState(request_id="r", initial_tokens=[1, 2], max_new_tokens=5)
    state.status = RequestStatus.PREFILLING
    first_scheduled = state.lifespan[0]
    state.status = RequestStatus.DECODING
    state.generated_tokens.append(101)
    fresh = state.create_equivalent_initial_request()
    assert fresh.created_time == state.created_time
    assert fresh.lifespan[0] == first_scheduled
    fresh.status = RequestStatus.PREFILLING
    assert fresh.lifespan[0] == first_scheduled


def test_offload_requeue_keeps_the_pending_tokens_replayed_exit_depth() -> None:
    state = _decoding_state()
    state.allocated_blocks = 3
    state.prepare_for_offload_requeue()
    assert state.allocated_blocks == 0 and state.remaining_prefill_tokens == []
    assert state.next_synthetic_exit_depth() == 12
    assert state.next_synthetic_exit_depth() == 13


def test_host_block_runs_split_at_gaps() -> None:
    assert host_block_runs([]) == []
    assert host_block_runs([4, 5, 6, 9, 2, 3]) == [(4, 0, 3), (9, 3, 1), (2, 4, 2)]
    assert host_block_runs([7]) == [(7, 0, 1)]


# -- engine under pressure --------------------------------------------------------------------------------------
def test_none_mode_raises_when_the_cache_is_oversubscribed() -> None:
    with pytest.raises(CacheFullError, match="does no preemption"):
        replay(PROMPTS, FULL_DEPTH, 8, kv_pressure_mode="none", **OVERSUBSCRIBED)


@pytest.mark.parametrize("refill", [True, False])
@pytest.mark.parametrize("use_async", [False, True])
def test_recompute_preemption_preserves_output_at_full_depth(refill: bool, use_async: bool) -> None:
    _, reference = replay(PROMPTS, FULL_DEPTH, 8, refill=refill, num_blocks=64, block_size=2, max_model_len=12)
    engine, outs = replay(PROMPTS, FULL_DEPTH, 8, refill=refill, use_async_batching=use_async,
                          kv_pressure_mode="recompute", **OVERSUBSCRIBED)
    assert tokens_of(outs) == tokens_of(reference)
    assert [o.prompt_ids for o in outs] == PROMPTS
    assert engine.cache.get_num_free_blocks() == engine.cache.num_blocks
    om = engine.offloading_manager
    assert om.num_recompute_preemptions > 0 and om.num_offload_preemptions == 0
    assert not om.offloading_enabled
    assert [e[2] for e in om.preemption_events] == ["recompute"] * om.num_recompute_preemptions
    # A soft reset re-prefills prompt + generated tokens (the pending one included).
    assert all(length > 2 for _, _, length in om.recompute_events)


@pytest.mark.parametrize("kv_policy", ["single", "last_exited"])
@pytest.mark.parametrize("refill", [True, False])
def test_offload_preemption_preserves_output(kv_policy: str, refill: bool) -> None:
    _, reference = replay(PROMPTS, VARIED, 8, refill=refill, num_blocks=64, block_size=2, max_model_len=12)
    engine, outs = replay(PROMPTS, VARIED, 8, refill=refill, kv_policy=kv_policy, kv_pressure_mode="offload",
                          cpu_offload_space=0.001, **OVERSUBSCRIBED)
    assert tokens_of(outs) == tokens_of(reference)
    assert [o.exit_depths for o in outs] == [o.exit_depths for o in reference]
    assert engine.cache.get_num_free_blocks() == engine.cache.num_blocks
    om = engine.offloading_manager
    assert om.num_offload_preemptions > 0 and om.num_restores == om.num_offload_preemptions
    assert om.num_recompute_preemptions == 0
    # Every restore batch reads back whole swap-outs: each one's host blocks, in their order.
    outstanding: list[tuple[int, ...]] = []
    for kind, _device, host in om.swap.moves:
        if kind == "out":
            outstanding.append(tuple(host))
            continue
        rest = tuple(host)
        while rest:
            match = next(key for key in outstanding if rest[:len(key)] == key)
            outstanding.remove(match)
            rest = rest[len(match):]
    assert not outstanding


def test_last_exited_full_offload_pool_raises_instead_of_recompute_fallback() -> None:
    with pytest.raises(RuntimeError, match="soft-reset fallback is disabled"):
        replay(PROMPTS, VARIED, 8, kv_policy="last_exited", kv_pressure_mode="offload", cpu_offload_space=1e-9,
               **OVERSUBSCRIBED)


def test_single_request_that_cannot_fit_raises() -> None:
    engine = make_engine(num_blocks=2, block_size=2, max_model_len=12, safety_margin=0.0)
    with pytest.raises(CacheFullError, match="single request"):
        engine.generate_batch([[1, 2]], max_new_tokens=8, eos_token_id=None)


# -- test_prefill_admission.py:330-431 ----------------------------------------------------------------------------
PRESSURE_MODES = [("recompute", None), ("offload", 0.05)]


def _admission_engine(num_blocks: int, refill: bool, **kw):
    return make_engine(num_blocks=num_blocks, block_size=4, max_num_batched_tokens=64, max_model_len=32,
                       safety_margin=0.0, refill=refill, **kw)


@pytest.mark.parametrize("refill", [True, False])
@pytest.mark.parametrize("mode,space", PRESSURE_MODES)
def test_oversubscribed_cache_completes_every_request(refill: bool, mode: str, space) -> None:
    engine = _admission_engine(6, refill, kv_pressure_mode=mode, cpu_offload_space=space)
    outs = engine.generate_batch([[1, 2, 3, 4]] * 6, max_new_tokens=6, eos_token_id=None)
    assert [len(o.generated_tokens) for o in outs] == [6] * 6
    assert engine.offloading_manager.num_preemptions > 0
    assert engine.cache.get_num_free_blocks() == engine.cache.num_blocks


@pytest.mark.parametrize("refill", [True, False])
@pytest.mark.parametrize("mode,space", PRESSURE_MODES)
def test_preemption_does_not_change_generated_tokens(refill: bool, mode: str, space) -> None:
    def run(num_blocks: int, use_async: bool = False, **pressure):
        engine = _admission_engine(num_blocks, refill, use_async_batching=use_async, **pressure)
        return tokens_of(engine.generate_batch([[1, 2, 3, 4]] * 6, max_new_tokens=6, eos_token_id=None))

    uncontended = run(64, kv_pressure_mode="none")
    assert run(6, kv_pressure_mode=mode, cpu_offload_space=space) == uncontended
    assert run(6, use_async=True, kv_pressure_mode=mode, cpu_offload_space=space) == uncontended


def test_swap_round_trip_moves_every_layer_of_the_victims_blocks() -> None:
    """Swap a decoder out, scribble over the pool, restore it into other blocks: its KV, every
    cache layer K and V, comes back in block order."""

    engine = make_engine(num_blocks=16, block_size=2, max_model_len=12, kv_policy="depth_indexed",
                         kv_pressure_mode="offload", cpu_offload_space=0.001)
    cache, sched, om = engine.cache, engine.scheduler, engine.offloading_manager
    victim = RequestState(request_id="v", initial_tokens=[1, 2, 3, 4, 5], max_new_tokens=4)
    victim._status = RequestStatus.DECODING
    victim.position_offset = 5
    victim.tokens_to_process = [6]
    sched.active_requests["v"] = victim
    other = RequestState(request_id="o", initial_tokens=[9], max_new_tokens=4)
    sched.active_requests["o"] = other
    assert sched._allocate_blocks_if_needed(other, 2)  # takes the first blocks, so the restore moves
    assert sched._allocate_blocks_if_needed(victim, 1)
    blocks = list(cache.block_table["v"])
    assert len(blocks) == 3 and cache.num_layers > 1
    gen = torch.Generator().manual_seed(0)
    cache.pool.copy_(torch.randn(cache.pool.shape, generator=gen))
    pages = cache.pool.view(cache.num_layers, 2, -1, cache.block_size, *cache.pool.shape[3:])
    saved = pages[:, :, blocks].clone()

    om.preempt_request("v", victim)
    assert victim.is_cpu_offloaded and "v" not in cache.block_table and sched.block_new_requests
    cache.pool.zero_()
    sched.block_new_requests = False
    sched.finish_request("o")  # the victim's restore now lands on the other request's old blocks
    restored = engine._restore_offloaded_requests()
    assert restored == [victim] and not victim.is_cpu_offloaded
    new_blocks = cache.block_table["v"]
    assert new_blocks[:3] != blocks
    assert torch.equal(pages[:, :, new_blocks[:3]], saved)
    assert om.num_restores == 1 and om.num_offload_preemptions == 1


# -- the soft-reset oracle composition the HIP-path test relies on -------------------------------------------------
@pytest.mark.parametrize("use_async", [False, True])
def test_recompute_matches_the_composed_token_increment_oracle(use_async: bool) -> None:
    """The over-subscribed workload of the HIP-path test on the token-increment model, whose
    per-request oracle is closed-form: prefill gives last + steps, a decode token tok + depth + 1."""

    from types import SimpleNamespace

    from tests.pressure_helpers import PRESSURE, composed_oracle, preemption_cuts, pressure_workload

    steps, vocab = 4, 16
    prompts, mnt, depths = pressure_workload(vocab=vocab)
    engine = make_engine(kv_policy="single", kv_pressure_mode="recompute", use_async_batching=use_async,
                         max_recurrent_steps=steps, **PRESSURE)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)

    def oracle_run(prompt, new_tokens, seg_depths):
        tokens = [(prompt[-1] + steps) % vocab]
        while len(tokens) < new_tokens:
            d = seg_depths[len(tokens) - 1]
            tokens.append((tokens[-1] + d + 1) % vocab)
        return SimpleNamespace(tokens=tokens, exit_depths=seg_depths[: new_tokens - 1])

    cuts = preemption_cuts(engine.offloading_manager.recompute_events, prompts)
    assert sum(len(c) for c in cuts.values()) > 2 and max(len(c) for c in cuts.values()) > 1
    for i, out in enumerate(outs):
        tokens, exits = composed_oracle(oracle_run, prompts[i], mnt[i], depths[i], cuts.get(i, []))
        assert out.generated_tokens == tokens
        assert out.exit_depths == exits
        assert len(tokens) == mnt[i]
    # Without preemption the composition is the plain oracle.
    plain = oracle_run(prompts[0], mnt[0], depths[0])
    assert composed_oracle(oracle_run, prompts[0], mnt[0], depths[0], []) == (plain.tokens, plain.exit_depths)
