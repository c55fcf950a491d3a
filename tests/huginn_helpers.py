"""Tiny random-init Huginn used by the oracle and engine tests (head_dim 96, as Huginn-0125)."""

from __future__ import annotations

import numpy as np

TINY_HUGINN = dict(n_embd=192, n_heads=2, n_prelude=1, n_core=2, n_coda=1, steps=4, intermediate=256, vocab=512,
                   rope_base=50000.0, eps=1e-6)


def tiny_huginn_config(**overrides):
    from continuous_depth_batching_amd.huginn import HuginnConfig

    t = TINY_HUGINN
    kw = dict(n_embd=t["n_embd"], n_heads=t["n_heads"], n_layers=t["n_prelude"] + t["n_core"] + t["n_coda"],
              n_layers_in_prelude=t["n_prelude"], n_layers_in_recurrent_block=t["n_core"],
              n_layers_in_coda=t["n_coda"], mean_recurrence=t["steps"], block_size=1024, vocab_size=t["vocab"],
              intermediate_size=t["intermediate"], norm_eps=t["eps"], rope_base=t["rope_base"])
    kw.update(overrides)
    return HuginnConfig(**kw)


def tiny_huginn_weights(seed: int, std: float = 0.05, qk_bias_std: float = 0.05) -> dict[str, np.ndarray]:
    """fp32 weights with the reference's parameter names (CPU numpy); the tied LM head is included."""

    from continuous_depth_batching_amd.huginn import HuginnForCausalLM, init_huginn_weights

    model = HuginnForCausalLM(tiny_huginn_config())
    init_huginn_weights(model, seed=seed, std=std, qk_bias_std=qk_bias_std)
    return {k: v.detach().float().numpy().copy() for k, v in model.state_dict().items()}


def make_huginn_oracle(weights, dtype: str = "f32"):
    from oracle.huginn_model import HuginnOracle

    t = TINY_HUGINN
    return HuginnOracle(weights, n_embd=t["n_embd"], n_heads=t["n_heads"], n_prelude=t["n_prelude"],
                        n_core=t["n_core"], n_coda=t["n_coda"], rope_base=t["rope_base"], eps=t["eps"], dtype=dtype,
                        max_positions=1024)
