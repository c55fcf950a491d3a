"""End-to-end CDB engine on the HIP kernels vs the per-request oracle (tiny fp32 Ouro).

The engine batches requests at mixed loop steps; the oracle decodes each
request alone. With fp32 weights the greedy token streams must agree on at
least 99% of tokens before the first divergence (in practice all of them), and
the per-token exit depths must agree exactly wherever the streams agree.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.ouro_model import OuroOracle
from tests.ouro_helpers import TINY, tiny_config, tiny_weights

pytestmark = pytest.mark.gpu


def build_model(seed: int, dtype=torch.float32):
    from continuous_depth_batching_amd.ouro import OuroForCausalLM

    weights = tiny_weights(seed)
    with torch.device("cuda"):
        model = OuroForCausalLM(tiny_config())
    model.load_state_dict({k: torch.from_numpy(v) for k, v in weights.items()})
    return model.to(dtype).eval(), weights


def workload(seed: int, n: int = 8, new_tokens: int = 32):
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, TINY["vocab"], int(rng.integers(16, 65))).tolist() for _ in range(n)]
    return prompts, [new_tokens] * n


def matched_prefix_fraction(got: list[list[int]], want: list[list[int]]) -> float:
    total = sum(len(w) for w in want)
    matched = 0
    for g, w in zip(got, want):
        k = 0
        while k < min(len(g), len(w)) and g[k] == w[k]:
            k += 1
        matched += k
    return matched / total


def run_oracle(weights, prompts, mnt, exit_depths=None, **kw):
    oracle = OuroOracle(weights, num_layers=TINY["num_layers"], num_heads=TINY["num_heads"],
                        num_kv_heads=TINY["num_heads"], head_dim=TINY["head_dim"], rope_theta=TINY["rope_theta"],
                        eps=TINY["eps"], dtype="f32", max_positions=512)
    depths = exit_depths if exit_depths is not None else [None] * len(prompts)
    return [oracle.generate(p, m, max_steps=TINY["steps"], exit_depths=d, **kw)
            for p, m, d in zip(prompts, mnt, depths)]


def make_engine(model, **cfg_kw):
    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine

    base = dict(max_recurrent_steps=TINY["steps"], num_blocks=512, max_model_len=512, max_num_seqs=16,
                kv_pressure_mode="none")
    base.update(cfg_kw)
    return ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(**base))


@pytest.mark.parametrize("refill", [False, True])
def test_config1_live_gate_last_exited(refill: bool) -> None:
    """Config-1 plumbing case: live exit gate (threshold 0.5), per-step KV with exit copies."""

    model, weights = build_model(seed=0)
    prompts, mnt = workload(seed=0)
    engine = make_engine(model, exit_threshold=0.5, kv_policy="last_exited", refill=refill,
                         use_async_batching=False)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None)
    want = run_oracle(weights, prompts, mnt, kv_policy="last_exited", threshold=0.5)
    got_tokens = [o.generated_tokens for o in outs]
    assert matched_prefix_fraction(got_tokens, [w.tokens for w in want]) >= 0.99
    for o, w in zip(outs, want):
        if o.generated_tokens == w.tokens:
            assert o.exit_depths == w.exit_depths
    hist = engine.last_stats.exit_depth_histogram
    assert sum(hist.values()) == sum(len(w.exit_depths) for w in want)
    assert engine.last_stats.exit_kv_copies == sum(w.exit_copies for w in want)


@pytest.mark.parametrize("async_batching,graphs", [(False, True), (True, True), (True, False)])
def test_synthetic_replay_single_policy_refill(async_batching: bool, graphs: bool) -> None:
    """Refill at mixed loop steps; ``graphs=False`` runs every stage eagerly (no recorded graph),
    including the block-table updates that the recorded recurrent graph otherwise applies."""

    model, weights = build_model(seed=1)
    prompts, mnt = workload(seed=1, n=12, new_tokens=24)
    rng = np.random.default_rng(2)
    depths = [rng.choice(4, size=m - 1, p=[0.15, 0.25, 0.3, 0.3]).tolist() for m in mnt]
    engine = make_engine(model, synthetic_exit_replay=True, kv_policy="single", delay_gate_consumption=False,
                         use_async_batching=async_batching, max_num_seqs=8, use_cuda_graph=graphs,
                         use_cuda_graph_prefill=graphs)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    want = run_oracle(weights, prompts, mnt, kv_policy="single", exit_depths=depths)
    assert [o.generated_tokens for o in outs] == [w.tokens for w in want]
    assert [o.exit_depths for o in outs] == depths
    stats = engine.last_stats
    assert stats.recurrent_steps == sum(sum(d + 1 for d in ds) for ds in depths)
    assert stats.max_mixed_depths_per_batch > 1  # rows at different loop steps shared launches


def test_delayed_synthetic_replay_exits_one_step_later() -> None:
    model, weights = build_model(seed=3)
    prompts, mnt = workload(seed=3, n=6, new_tokens=12)
    rng = np.random.default_rng(4)
    depths = [rng.integers(0, 3, size=m - 1).tolist() for m in mnt]
    engine = make_engine(model, synthetic_exit_replay=True, kv_policy="single", delay_gate_consumption=True,
                         use_async_batching=True)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    want = run_oracle(weights, prompts, mnt, kv_policy="single", exit_depths=depths, delayed=True)
    assert [o.generated_tokens for o in outs] == [w.tokens for w in want]
    assert [o.exit_depths for o in outs] == [[min(d + 1, 3) for d in ds] for ds in depths]


def test_bf16_model_tokens_track_oracle() -> None:
    """bf16 weights: the oracle emulates bf16 rounding per op; accumulation order differs, so
    only the first tokens are required to agree and the engine must run without NaNs."""

    model, weights = build_model(seed=5, dtype=torch.bfloat16)
    prompts, mnt = workload(seed=5, n=4, new_tokens=6)
    engine = make_engine(model, synthetic_exit_replay=True, kv_policy="single", delay_gate_consumption=False)
    depths = [[1] * (m - 1) for m in mnt]
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    bf = {k: torch.from_numpy(v).bfloat16().float().numpy() for k, v in weights.items()}
    oracle = OuroOracle(bf, num_layers=TINY["num_layers"], num_heads=TINY["num_heads"],
                        num_kv_heads=TINY["num_heads"], head_dim=TINY["head_dim"], rope_theta=TINY["rope_theta"],
                        eps=TINY["eps"], dtype="bf16", max_positions=512)
    want = [oracle.generate(p, m, max_steps=4, kv_policy="single", exit_depths=d)
            for p, m, d in zip(prompts, mnt, depths)]
    first_agree = np.mean([o.generated_tokens[0] == w.tokens[0] for o, w in zip(outs, want)])
    assert first_agree >= 0.75
    assert all(len(o.generated_tokens) == m for o, m in zip(outs, mnt))


@pytest.mark.parametrize("refill", [True])
def test_mixed_slot_launches_last_exited_follow_the_oracle(refill: bool) -> None:
    """Per-step KV with exit copies, one launch mixing rows that write different KV slots: the
    per-row cache layers and the exit-copy flush before each launch keep every token's math the
    per-request oracle's."""

    model, weights = build_model(seed=7)
    prompts, mnt = workload(seed=7, n=10, new_tokens=20)
    rng = np.random.default_rng(8)
    depths = [rng.choice(4, size=m - 1, p=[0.15, 0.25, 0.3, 0.3]).tolist() for m in mnt]
    engine = make_engine(model, synthetic_exit_replay=True, kv_policy="last_exited", delay_gate_consumption=False,
                         refill=refill, max_num_seqs=8, mixed_slot_recurrent_batches=True)
    engine.record_launches = True
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    want = run_oracle(weights, prompts, mnt, kv_policy="last_exited", exit_depths=depths)
    assert [o.generated_tokens for o in outs] == [w.tokens for w in want]
    assert [o.exit_depths for o in outs] == depths
    assert engine.last_stats.exit_kv_copies == sum(w.exit_copies for w in want)
    mixed = [ev for ev in engine.launch_log if ev[0] == "recurrent" and len({row[2] for row in ev[1]}) > 1]
    assert mixed, "launches must mix loop steps (and so KV slots)"


@pytest.mark.parametrize("async_batching", [False, True])
def test_eos_finishes_follow_the_oracle(async_batching: bool) -> None:
    """Requests that stop on EOS mid-stream: with async batching an EOS token arrives after the
    request's successor was already staged (eager re-entry), so the finish must cancel that
    queued successor. The EOS ids are decoded tokens of four of the oracle's streams; greedy
    decode is prefix-consistent, so each expected stream is the oracle's stream cut after its
    first EOS token (with one exit depth per decoded token)."""

    model, weights = build_model(seed=7)
    prompts, mnt = workload(seed=7, n=10, new_tokens=24)
    rng = np.random.default_rng(8)
    depths = [rng.choice(4, size=m - 1, p=[0.15, 0.25, 0.3, 0.3]).tolist() for m in mnt]
    free_run = run_oracle(weights, prompts, mnt, kv_policy="single", exit_depths=depths)
    eos = sorted({free_run[r].tokens[3 + 2 * r] for r in (0, 2, 4, 6)})
    want_tokens, want_depths = [], []
    for out in free_run:
        cut = next((k for k, t in enumerate(out.tokens) if t in eos), len(out.tokens) - 1)
        want_tokens.append(out.tokens[:cut + 1])
        want_depths.append(out.exit_depths[:cut])
    assert sum(len(t) < m for t, m in zip(want_tokens, mnt)) >= 4
    engine = make_engine(model, synthetic_exit_replay=True, kv_policy="single", delay_gate_consumption=False,
                         use_async_batching=async_batching, max_num_seqs=6)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=eos, exit_depths=depths)
    assert [o.generated_tokens for o in outs] == want_tokens
    for o, w in zip(outs, want_depths):
        if async_batching:
            # A successor staged ahead of its EOS token may already have left the recurrent path
            # (its exit recorded) before the finish cancels it, as in the reference's eager path.
            assert o.exit_depths[:len(w)] == w
            assert len(o.exit_depths) <= len(w) + 1
        else:
            assert o.exit_depths == w
    if async_batching:
        assert engine.last_stats.cancelled_depth_items > 0
