"""Oracle: row-wise stage ops of the CDB decode step (numpy).

Restates:
  * RMSNorm: w * R(x * rsqrt(mean(x^2) + eps)) with fp32 statistics and the
    weight product rounded to the storage dtype (ouro/modeling_ouro.py:445-450,
    huginn/modeling_huginn.py:141-146); the Ouro and Huginn sandwich residual
    orders (ouro/modeling_ouro.py:481-502, huginn/modeling_huginn.py:335-338);
  * SiLU gating silu(g) * u (ouro/modeling_ouro.py:167-169);
  * greedy argmax, first index of the maximum (cdb/model_runner.py:1062,1105);
  * the exit gate Linear(E, 1) and the cumulative-hazard / direct-threshold
    decision with forced final-step exit and synthetic replay
    (cdb/adapters/ouro.py:286-291, cdb/exit_policy.py:150-169,
    cdb/continuous_api.py:1671-1724); Huginn's latent difference
    (huginn/exit_gates.py:33-40);
  * copy-on-exit KV propagation (cdb/continuous_api.py:1225-1245,
    kv_cache_policy.py:235-258).

Pinned by (tests/test_oracle_stage.py): torch's own ops on the same inputs
(rms_norm, silu, argmax, sigmoid), the reference's exit-policy vectors
(tests/continuous_depth_batching/test_exit_policy.py:37-120: CDF 0.75 /
survival 0.25, the bf16 boundary 0.279296875 < 0.28) and the exit-copy layer
groups (tests/test_looped_kv_layout.py:94-107).
"""

from __future__ import annotations

import math

import numpy as np

from .bf16 import rounder


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, dtype: str) -> np.ndarray:
    rnd = rounder(dtype)
    xf = np.asarray(x, dtype=np.float32)
    var = (xf.astype(np.float64) ** 2).mean(axis=-1, keepdims=True)
    inv = (1.0 / np.sqrt(var + eps)).astype(np.float32)
    return rnd(np.asarray(w, np.float32) * rnd(xf * inv))


def ouro_sandwich(x: np.ndarray, residual: np.ndarray, w_a: np.ndarray, w_b: np.ndarray, eps: float,
                  dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """h = residual + norm_a(x); y = norm_b(h)."""

    rnd = rounder(dtype)
    h = rnd(np.asarray(residual, np.float32) + rmsnorm(x, w_a, eps, dtype))
    return h, rmsnorm(h, w_b, eps, dtype)


def huginn_sandwich(x: np.ndarray, residual: np.ndarray, w_a: np.ndarray, w_b: np.ndarray, eps: float,
                    dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """h = norm_a(residual + x); y = norm_b(h)."""

    rnd = rounder(dtype)
    h = rmsnorm(rnd(np.asarray(x, np.float32) + np.asarray(residual, np.float32)), w_a, eps, dtype)
    return h, rmsnorm(h, w_b, eps, dtype)


def silu_mul(gate_up: np.ndarray, dtype: str) -> np.ndarray:
    rnd = rounder(dtype)
    g, u = np.split(np.asarray(gate_up, np.float32), 2, axis=-1)
    s = rnd((g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32))
    return rnd(s * u)


def argmax(logits: np.ndarray) -> np.ndarray:
    return np.argmax(np.asarray(logits, np.float32), axis=-1).astype(np.int64)


def gate_logits(hidden: np.ndarray, weight: np.ndarray, bias: float, dtype: str) -> np.ndarray:
    rnd = rounder(dtype)
    acc = np.asarray(hidden, np.float64) @ np.asarray(weight, np.float64)
    return rnd((acc + bias).astype(np.float32))


def latent_diff(hidden: np.ndarray, prev: np.ndarray, dtype: str) -> np.ndarray:
    rnd = rounder(dtype)
    d = rnd(np.asarray(hidden, np.float32) - np.asarray(prev, np.float32))
    num = rnd(np.sqrt((d.astype(np.float64) ** 2).sum(-1)).astype(np.float32))
    # clamp_min(1e-9) on a model-dtype norm clamps to the model-dtype value of 1e-9.
    floor = rnd(np.array([1e-9], np.float32))[0]
    den = np.maximum(rnd(np.sqrt((np.asarray(hidden, np.float64) ** 2).sum(-1)).astype(np.float32)), floor)
    return rnd((num / den).astype(np.float32))


def sigmoid_f32(x: float) -> float:
    return float(np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-x), dtype=np.float32)))


class TokenPolicy:
    """Per-token exit state (cdb/exit_policy.py:43-48) and one decision step (:150-169)."""

    def __init__(self) -> None:
        self.exit_cdf = 0.0
        self.survival = 1.0

    def consume(self, *, rule: str, signal: float, source_step: int, threshold: float, min_steps: int,
                round_hazard: str | None = None) -> bool:
        can_exit = source_step + 1 >= min_steps
        if rule == "hazard":
            hazard = sigmoid_f32(signal)
            if round_hazard is not None:
                hazard = float(rounder(round_hazard)(np.array([hazard], np.float32))[0])
            self.exit_cdf += hazard * self.survival
            self.survival *= 1.0 - hazard
            return can_exit and self.exit_cdf >= threshold
        return can_exit and signal < threshold


def decide_exit(*, step: int, max_steps: int, synthetic_depth: int | None, policy: TokenPolicy | None,
                signal: float | None, rule: str, threshold: float | None, min_steps: int,
                round_hazard: str | None = None) -> bool:
    """SAME_STEP routing decision of one stepped token (cdb/continuous_api.py:1671-1697)."""

    if step == max_steps - 1:
        return True
    if synthetic_depth is not None:
        return step >= synthetic_depth
    if threshold is None or signal is None:
        return False
    return policy.consume(rule=rule, signal=signal, source_step=step, threshold=threshold, min_steps=min_steps,
                          round_hazard=round_hazard)


def exit_copy_groups(exit_slot: int, num_slots: int, core_layers: int, layer_base: int = 0) -> list[tuple[int, list[int]]]:
    """(source, targets) cache layers propagating an exit at ``exit_slot`` (kv_cache_policy.py:235-258)."""

    if exit_slot + 1 >= num_slots:
        return []
    return [(layer_base + exit_slot * core_layers + l,
             [layer_base + s * core_layers + l for s in range(exit_slot + 1, num_slots)])
            for l in range(core_layers)]


def exit_kv_copy(kv_pool: np.ndarray, rows: np.ndarray, exit_slot: np.ndarray, *, layer_base: int, core_layers: int,
                 num_slots: int) -> None:
    for row, slot in zip(rows, exit_slot):
        for src, targets in exit_copy_groups(int(slot), num_slots, core_layers, layer_base):
            for dst in targets:
                kv_pool[dst, :, row] = kv_pool[src, :, row]
