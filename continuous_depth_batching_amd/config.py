"""ContinuousDepthBatchingConfig: the engine's configuration surface.

Field names, defaults and validation rules follow the reference
(continuous_depth_batching/config.py:52-246) so existing configs carry over.
The attention-implementation check accepts the reference's
``paged|flash_attention*`` strings, which this package serves with its HIP
kernels, plus ``paged|cdb_hip``.
"""

from __future__ import annotations

import math
from copy import deepcopy
from dataclasses import dataclass
from typing import Any, Literal

from .kv_cache_policy import KV_CACHE_POLICIES, copies_exit_kv, resolve_kv_slots_per_layer

KVPressureMode = Literal["none", "reserve", "recompute", "offload"]
KV_PRESSURE_MODES = ("none", "reserve", "recompute", "offload")
DEFAULT_MAX_NUM_SEQS = 256
MIN_FREE_SLOTS_DIVISOR = 8


def is_supported_attention_implementation(config: Any) -> bool:
    """``paged|flash_attention``, ``paged|flash_attention_<N>`` or ``paged|cdb_hip`` (config.py:35-48)."""

    impl = getattr(config, "_attn_implementation", None)
    if not isinstance(impl, str) or not impl.startswith("paged|"):
        return False
    backend = impl[len("paged|"):]
    if backend in ("flash_attention", "cdb_hip"):
        return True
    return backend.startswith("flash_attention_") and backend[len("flash_attention_"):].isdigit()


def validate_cache_size_request(num_blocks: int | None, mem_fraction_static: float | None) -> None:
    """Explicit block count or a static memory fraction, not both (kv_cache_sizing.py:25-31)."""

    if num_blocks is not None and num_blocks <= 0:
        raise ValueError(f"num_blocks must be positive, but got {num_blocks}")
    if mem_fraction_static is not None and (not math.isfinite(mem_fraction_static)
                                            or not 0 < mem_fraction_static < 1):
        raise ValueError(f"mem_fraction_static must be finite and in (0, 1), but got {mem_fraction_static}")
    if num_blocks is not None and mem_fraction_static is not None:
        raise ValueError("Set either num_blocks or mem_fraction_static, not both")


def validate_kv_pressure_config(mode: str, cpu_offload_space: float | None) -> None:
    """utils.py:35-54."""

    if mode not in KV_PRESSURE_MODES:
        raise ValueError(f"kv_pressure_mode must be one of {KV_PRESSURE_MODES}, but got {mode!r}")
    if cpu_offload_space is not None and cpu_offload_space < 0:
        raise ValueError(f"cpu_offload_space must be non-negative when set, but got {cpu_offload_space}")
    if mode == "offload":
        if not cpu_offload_space:
            raise ValueError("kv_pressure_mode='offload' requires cpu_offload_space > 0 (the pinned CPU pool size)")
    elif cpu_offload_space:
        raise ValueError(f"cpu_offload_space is only used by kv_pressure_mode='offload', not {mode!r}")


def resolve_min_free_slots(min_free_slots: int | None, max_num_seqs: int) -> int:
    """utils.py:23-32."""

    if min_free_slots is None:
        return max(1, max_num_seqs // MIN_FREE_SLOTS_DIVISOR)
    return min(min_free_slots, max_num_seqs)


@dataclass
class ContinuousDepthBatchingConfig:
    """Configuration for continuous depth batching (same fields and defaults as the reference)."""

    block_size: int = 16
    num_blocks: int | None = None
    mem_fraction_static: float | None = None
    max_num_batched_tokens: int = 8192
    safety_margin: float = 0.2
    replay_eos_finishes: bool = False
    max_model_len: int = 16384
    use_async_batching: bool = True
    use_cuda_graph: bool = True
    use_cuda_graph_prefill: bool = True  # accepted; prefill chunks always run eagerly
    max_recurrent_steps: int | None = None
    exit_threshold: float | None = None
    synthetic_exit_replay: bool = False
    min_recurrent_steps: int = 1
    delay_gate_consumption: bool = True
    min_coda_batch_size: int = 1
    max_num_seqs: int = DEFAULT_MAX_NUM_SEQS
    min_free_slots: int | None = None
    refill: bool = True
    kv_policy: str = "single"
    kv_slots_per_layer: int | None = None
    kv_pressure_mode: KVPressureMode = "recompute"
    cpu_offload_space: float | None = None
    # Not a reference field. With a multi-slot KV policy, let one recurrent launch carry rows that
    # write different KV slots: the decode kernel reads a cache layer per row, so the reference's
    # slot-homogeneous launches are a constraint of its attention backend, not of the math. Off
    # (the default) keeps the reference's schedule; on changes which rows share a launch, never a
    # row's result.
    mixed_slot_recurrent_batches: bool = False

    def decode_block_table_width(self) -> int:
        return -(-self.max_model_len // self.block_size)

    def get_resolved(self, config: Any) -> "ContinuousDepthBatchingConfig":
        """Deep copy, validate, derive slot counts, validate again (config.py:125-135)."""

        resolved = deepcopy(self)
        resolved.validate(config)
        resolved.normalize_derived_values()
        resolved.validate_resolved()
        return resolved

    def validate(self, config: Any) -> None:
        if not is_supported_attention_implementation(config):
            raise NotImplementedError(
                "Continuous depth batching serves paged attention only ('paged|flash_attention*' or "
                f"'paged|cdb_hip'), got attn_implementation={getattr(config, '_attn_implementation', None)!r}")
        if self.block_size <= 0:
            raise ValueError(f"block_size must be positive, but got {self.block_size}")
        if self.block_size & (self.block_size - 1):
            raise ValueError(f"block_size must be a power of two for the paged kernels, got {self.block_size}")
        validate_cache_size_request(self.num_blocks, self.mem_fraction_static)
        if self.max_num_batched_tokens <= 0:
            raise ValueError(f"max_num_batched_tokens must be positive, but got {self.max_num_batched_tokens}")
        if self.max_model_len <= 0:
            raise ValueError(f"max_model_len must be positive, but got {self.max_model_len}")
        if self.max_recurrent_steps is None:
            raise ValueError("max_recurrent_steps must be explicitly set for CDB")
        if self.max_recurrent_steps <= 1:
            raise ValueError(f"max_recurrent_steps must be greater than 1, but got {self.max_recurrent_steps}")
        if self.max_num_seqs <= 0:
            raise ValueError(f"max_num_seqs must be positive, but got {self.max_num_seqs}")
        if self.min_free_slots is not None and self.min_free_slots <= 0:
            raise ValueError(f"min_free_slots must be positive, but got {self.min_free_slots}")
        if self.min_coda_batch_size <= 0:
            raise ValueError(f"min_coda_batch_size must be positive, but got {self.min_coda_batch_size}")
        if self.min_coda_batch_size > self.max_num_seqs:
            raise ValueError(f"min_coda_batch_size must not exceed max_num_seqs, but got "
                             f"{self.min_coda_batch_size} > {self.max_num_seqs}")
        if self.replay_eos_finishes and not self.use_async_batching:
            raise ValueError("replay_eos_finishes requires use_async_batching")
        if not 0 <= self.safety_margin < 1:
            raise ValueError(f"safety_margin must be in [0, 1), but got {self.safety_margin}")
        if self.kv_policy not in KV_CACHE_POLICIES:
            raise ValueError(f"Unsupported kv_policy={self.kv_policy!r}; expected one of {KV_CACHE_POLICIES}")
        if copies_exit_kv(self.kv_policy) and self.kv_pressure_mode == "recompute":
            raise ValueError("kv_policy='last_exited' cannot run with kv_pressure_mode='recompute': a full-depth "
                             "re-prefill would replace exited tokens' exit-step KV. Use 'reserve', 'offload' or 'none'.")
        if self.min_recurrent_steps <= 0:
            raise ValueError(f"min_recurrent_steps must be positive, but got {self.min_recurrent_steps}")
        validate_kv_pressure_config(self.kv_pressure_mode, self.cpu_offload_space)
        if self.exit_threshold is not None and self.synthetic_exit_replay:
            raise ValueError("Only one CDB exit policy can be active")
        layer_types = getattr(config, "layer_types", None)
        sliding = layer_types is not None and any(t != "full_attention" for t in layer_types)
        if getattr(config, "sliding_window", None) is not None or sliding:
            raise NotImplementedError("Continuous depth batching supports full-attention models only")

    def normalize_derived_values(self) -> None:
        assert self.max_recurrent_steps is not None
        self.kv_slots_per_layer = resolve_kv_slots_per_layer(
            self.kv_policy, total_recurrent_steps=self.max_recurrent_steps, requested_slots=self.kv_slots_per_layer)

    def validate_resolved(self) -> None:
        if self.max_recurrent_steps is None:
            raise ValueError("max_recurrent_steps must be resolved")
        if self.max_recurrent_steps <= 1:
            raise ValueError("max_recurrent_steps must be greater than 1")
        if self.min_recurrent_steps > self.max_recurrent_steps:
            raise ValueError(f"min_recurrent_steps={self.min_recurrent_steps} exceeds "
                             f"max_recurrent_steps={self.max_recurrent_steps}")
        if copies_exit_kv(self.kv_policy):
            return
        slots = resolve_kv_slots_per_layer(self.kv_policy, total_recurrent_steps=self.max_recurrent_steps,
                                           requested_slots=self.kv_slots_per_layer)
        if self.exit_threshold is not None and self.min_recurrent_steps < slots:
            raise ValueError("kv_slots_per_layer must be <= min_recurrent_steps for gated early exit, "
                             f"got kv_slots_per_layer={slots}, min_recurrent_steps={self.min_recurrent_steps}")
