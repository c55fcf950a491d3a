"""Tiny random-init Ouro used across oracle, engine and smoke tests (config-1 shape)."""

from __future__ import annotations

import numpy as np

TINY = dict(hidden=256, num_layers=4, steps=4, num_heads=4, head_dim=64, intermediate=1024, vocab=49152,
            rope_theta=10000.0, eps=1e-6)


def tiny_config(**overrides):
    from continuous_depth_batching_amd.ouro import OuroConfig

    kw = dict(vocab_size=TINY["vocab"], hidden_size=TINY["hidden"], intermediate_size=TINY["intermediate"],
              num_hidden_layers=TINY["num_layers"], num_attention_heads=TINY["num_heads"],
              num_key_value_heads=TINY["num_heads"], head_dim=TINY["head_dim"], rms_norm_eps=TINY["eps"],
              rope_theta=TINY["rope_theta"], total_ut_steps=TINY["steps"], max_position_embeddings=4096)
    kw.update(overrides)
    return OuroConfig(**kw)


def tiny_weights(seed: int, std: float = 0.02) -> dict[str, np.ndarray]:
    """fp32 weights of the tiny Ouro with the reference's parameter names (CPU, numpy)."""

    import torch

    from continuous_depth_batching_amd.ouro import OuroForCausalLM, init_ouro_weights

    model = OuroForCausalLM(tiny_config())
    init_ouro_weights(model, seed=seed, std=std)
    return {k: v.detach().float().numpy().copy() for k, v in model.state_dict().items()}
