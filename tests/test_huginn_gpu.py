"""End-to-end CDB engine on the HIP kernels vs the per-request Huginn oracle (tiny fp32 Huginn).

Exercises the prelude and coda with their own paged attention (interleaved RoPE,
qk_bias), the adapter GEMM over [state | injection], the core blocks at per-row
loop slots, and the latent-difference direct-threshold exit gate on both horizons.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.huginn_helpers import TINY_HUGINN, make_huginn_oracle, tiny_huginn_config, tiny_huginn_weights

pytestmark = pytest.mark.gpu
T = TINY_HUGINN


def build_model(seed: int, dtype=torch.float32):
    from continuous_depth_batching_amd.huginn import HuginnForCausalLM

    weights = tiny_huginn_weights(seed)
    with torch.device("cuda"):
        model = HuginnForCausalLM(tiny_huginn_config())
    model.load_state_dict({k: torch.from_numpy(v) for k, v in weights.items()})
    return model.to(dtype).eval(), weights


def make_engine(model, **cfg_kw):
    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine

    base = dict(max_recurrent_steps=T["steps"], num_blocks=512, max_model_len=512, max_num_seqs=16,
                kv_pressure_mode="none")
    base.update(cfg_kw)
    return ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(**base))


def workload(seed: int, n: int, new_tokens: int):
    rng = np.random.default_rng(seed)
    prompts = [rng.integers(0, T["vocab"], int(rng.integers(8, 40))).tolist() for _ in range(n)]
    return prompts, [new_tokens] * n


def matched_prefix_fraction(got, want) -> float:
    total = sum(len(w) for w in want)
    matched = 0
    for g, w in zip(got, want):
        k = 0
        while k < min(len(g), len(w)) and g[k] == w[k]:
            k += 1
        matched += k
    return matched / total


@pytest.mark.parametrize("kv_policy", ["single", "last_exited"])
def test_huginn_synthetic_replay_matches_oracle(kv_policy: str) -> None:
    model, weights = build_model(seed=1)
    prompts, mnt = workload(seed=1, n=6, new_tokens=10)
    rng = np.random.default_rng(2)
    depths = [rng.integers(0, T["steps"], size=m - 1).tolist() for m in mnt]
    engine = make_engine(model, synthetic_exit_replay=True, kv_policy=kv_policy, delay_gate_consumption=False,
                         use_async_batching=True, max_num_seqs=4)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    oracle = make_huginn_oracle(weights)
    want = [oracle.generate(p, m, max_steps=T["steps"], kv_policy=kv_policy, exit_depths=d)
            for p, m, d in zip(prompts, mnt, depths)]
    assert [o.generated_tokens for o in outs] == [w.tokens for w in want]
    assert [o.exit_depths for o in outs] == depths
    if kv_policy == "last_exited":
        assert engine.last_stats.exit_kv_copies == sum(d < T["steps"] - 1 for ds in depths for d in ds)


def test_huginn_latent_gate_on_the_delayed_horizon() -> None:
    model, weights = build_model(seed=3)
    prompts, mnt = workload(seed=3, n=6, new_tokens=8)
    oracle = make_huginn_oracle(weights)
    # A threshold in the widest gap among the oracle's signals keeps decisions away from ties.
    probe = [oracle.generate(p, m, max_steps=T["steps"], threshold=-1.0, delayed=True) for p, m in zip(prompts, mnt)]
    sig = np.sort(np.unique([s for o in probe for ss in o.signals for s in ss]))
    mid = sig[(sig > np.quantile(sig, 0.2)) & (sig < np.quantile(sig, 0.8))]
    gaps = np.diff(mid)
    threshold = float((mid[np.argmax(gaps)] + mid[np.argmax(gaps) + 1]) / 2)
    engine = make_engine(model, exit_threshold=threshold, kv_policy="single", use_async_batching=True,
                         delay_gate_consumption=True)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None)
    want = [oracle.generate(p, m, max_steps=T["steps"], threshold=threshold, delayed=True)
            for p, m in zip(prompts, mnt)]
    got = [o.generated_tokens for o in outs]
    assert matched_prefix_fraction(got, [w.tokens for w in want]) >= 0.99
    for o, w in zip(outs, want):
        if o.generated_tokens == w.tokens:
            assert o.exit_depths == w.exit_depths
    assert len(engine.last_stats.exit_depth_histogram) > 1  # the gate really splits depths


def test_huginn_bf16_runs_and_tracks_oracle() -> None:
    model, weights = build_model(seed=5, dtype=torch.bfloat16)
    prompts, mnt = workload(seed=5, n=4, new_tokens=5)
    depths = [[1] * (m - 1) for m in mnt]
    engine = make_engine(model, synthetic_exit_replay=True, kv_policy="single", delay_gate_consumption=False)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    bf = {k: torch.from_numpy(v).bfloat16().float().numpy() for k, v in weights.items()}
    oracle = make_huginn_oracle(bf, dtype="bf16")
    want = [oracle.generate(p, m, max_steps=T["steps"], kv_policy="single", exit_depths=d)
            for p, m, d in zip(prompts, mnt, depths)]
    assert np.mean([o.generated_tokens[0] == w.tokens[0] for o, w in zip(outs, want)]) >= 0.75
    assert all(len(o.generated_tokens) == m for o, m in zip(outs, mnt))


def test_random_state_init_is_the_references_truncated_normal() -> None:
    """state_init="random" (huginn/modeling_huginn.py:418-427): N(0, s) with s = sqrt(2 / (5E)),
    clamped at 3 s, times sqrt(E). Clamping (not truncating) puts 2 (1 - Phi(3)) = 0.26998% of
    the draws exactly on the bounds and leaves a standard deviation of 0.99750 s
    (variance 1 - 6 phi(3) - (1 - 9) 2 (1 - Phi(3)) = 0.995007), so the rows must show
    sqrt(E) * s * 0.99750, that mass at +-3 s sqrt(E), and nothing beyond."""

    import math

    from continuous_depth_batching_amd.huginn import HuginnCDBAdapter, HuginnForCausalLM

    cfg = tiny_huginn_config(state_init="random", state_seed=3)
    with torch.device("cuda"):
        model = HuginnForCausalLM(cfg).float().eval()
    adapter = HuginnCDBAdapter(model)
    e = cfg.n_embd
    s = math.sqrt(2 / (5 * e))
    x = adapter._initial_state(torch.zeros((8192, e), device="cuda")).double()
    bound = 3 * s * math.sqrt(e)
    assert x.abs().max().item() <= bound * (1 + 1e-6)
    assert abs(x.mean().item()) < 0.01 * s * math.sqrt(e)
    assert abs(x.std().item() / (s * math.sqrt(e)) - 0.99750) < 0.002
    at_bound = (x.abs() >= bound * (1 - 1e-6)).double().mean().item()
    assert abs(at_bound / 0.0026998 - 1) < 0.1
    # Seeded: a second adapter over the same config draws the same rows.
    again = HuginnCDBAdapter(model)._initial_state(torch.zeros((8192, e), device="cuda")).double()
    assert torch.equal(x, again)


def test_random_state_init_engine_is_reproducible_under_a_seed() -> None:
    from continuous_depth_batching_amd.huginn import HuginnForCausalLM

    weights = tiny_huginn_weights(4)
    prompts, mnt = workload(seed=4, n=4, new_tokens=6)
    runs = []
    for seed in (9, 9, 10):
        with torch.device("cuda"):
            model = HuginnForCausalLM(tiny_huginn_config(state_init="random", state_seed=seed))
        model.load_state_dict({k: torch.from_numpy(v) for k, v in weights.items()})
        engine = make_engine(model.float().eval(), synthetic_exit_replay=True, kv_policy="single",
                             delay_gate_consumption=False)
        depths = [[1] * (m - 1) for m in mnt]
        outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
        runs.append([o.generated_tokens for o in outs])
    assert runs[0] == runs[1]
    assert all(0 <= t < T["vocab"] for ts in runs[0] for t in ts)
    assert runs[2] != runs[0]  # another seed starts every token from another state
