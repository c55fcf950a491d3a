"""Looped KV layouts: which KV slot (cache layer) each recurrent step writes.

A looped model runs its core layers once per recurrent step. The policy maps a
0-based step to a KV slot, and a (physical layer, slot) pair to a cache layer
index of the paged pool, laid out as
``[prelude 0..P-1 | slot 0 core 0..C-1 | ... | slot S-1 core 0..C-1 | coda 0..D-1]``.

Same names and arithmetic as the reference (kv_cache_policy.py:25-263), since
the cache-layer numbering is part of the paged-cache contract.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

KvCachePolicy = Literal["depth_indexed", "last_exited", "single", "first_then_shared"]

DEPTH_INDEXED = "depth_indexed"
LAST_EXITED = "last_exited"
SINGLE = "single"
FIRST_THEN_SHARED = "first_then_shared"
KV_CACHE_POLICIES: tuple[str, ...] = (DEPTH_INDEXED, LAST_EXITED, SINGLE, FIRST_THEN_SHARED)


def validate_kv_cache_policy(policy: str) -> str:
    if policy not in KV_CACHE_POLICIES:
        raise ValueError(f"Unsupported KV cache policy {policy!r}; expected one of {KV_CACHE_POLICIES}")
    return policy


def copies_exit_kv(policy: str) -> bool:
    """Whether an early exit copies the exit-step KV into deeper slots (kv_cache_policy.py:47-50)."""

    return validate_kv_cache_policy(policy) == LAST_EXITED


def resolve_kv_slots_per_layer(policy: str, *, total_recurrent_steps: int, requested_slots: int | None = None) -> int:
    """KV slots per physical layer (kv_cache_policy.py:53-81)."""

    if total_recurrent_steps <= 0:
        raise ValueError(f"total_recurrent_steps must be positive, got {total_recurrent_steps}")
    policy = validate_kv_cache_policy(policy)
    fixed = {DEPTH_INDEXED: total_recurrent_steps, LAST_EXITED: total_recurrent_steps, SINGLE: 1}
    if policy in fixed:
        slots = fixed[policy]
        if requested_slots is not None and requested_slots != slots:
            raise ValueError(f"Policy {policy!r} uses exactly {slots} KV slot(s) per layer, got {requested_slots}")
        return slots
    slots = 2 if requested_slots is None else requested_slots
    if slots <= 0:
        raise ValueError(f"kv_slots_per_layer must be positive, got {slots}")
    if slots > total_recurrent_steps:
        raise ValueError(f"kv_slots_per_layer={slots} exceeds total_recurrent_steps={total_recurrent_steps}")
    return slots


def kv_slot_for_step(recurrent_step: int, *, policy: str, slots_per_layer: int) -> int:
    """0-based recurrent step -> KV slot (kv_cache_policy.py:84-103)."""

    if recurrent_step < 0:
        raise ValueError(f"recurrent_step must be non-negative, got {recurrent_step}")
    if slots_per_layer <= 0:
        raise ValueError(f"slots_per_layer must be positive, got {slots_per_layer}")
    policy = validate_kv_cache_policy(policy)
    if policy in (DEPTH_INDEXED, LAST_EXITED):
        return recurrent_step
    if policy == SINGLE:
        return 0
    return min(recurrent_step, slots_per_layer - 1)


def kv_layer_index(*, physical_layer_idx: int, num_hidden_layers: int, recurrent_step: int, policy: str,
                   slots_per_layer: int, explicit_slot: int | None = None) -> int:
    """Cache layer of a fully looped model's layer at a step (kv_cache_policy.py:106-128)."""

    if physical_layer_idx < 0:
        raise ValueError(f"physical_layer_idx must be non-negative, got {physical_layer_idx}")
    if num_hidden_layers <= 0:
        raise ValueError(f"num_hidden_layers must be positive, got {num_hidden_layers}")
    slot = kv_slot_for_step(recurrent_step, policy=policy, slots_per_layer=slots_per_layer) \
        if explicit_slot is None else explicit_slot
    if not 0 <= slot < slots_per_layer:
        raise ValueError(f"explicit_slot must be in [0, {slots_per_layer}), got {slot}")
    return slot * num_hidden_layers + physical_layer_idx


@dataclass(frozen=True)
class LoopedKvLayout:
    """Prelude / core-slots / coda placement of a looped decoder in the paged pool."""

    num_prelude_layers: int
    num_core_layers: int
    num_coda_layers: int
    total_recurrent_steps: int
    policy: str
    slots_per_layer: int

    def __post_init__(self) -> None:
        validate_kv_cache_policy(self.policy)
        if self.num_prelude_layers < 0 or self.num_coda_layers < 0:
            raise ValueError("prelude and coda layer counts must be non-negative")
        if self.num_core_layers <= 0:
            raise ValueError(f"num_core_layers must be positive, got {self.num_core_layers}")
        if self.total_recurrent_steps <= 0:
            raise ValueError(f"total_recurrent_steps must be positive, got {self.total_recurrent_steps}")
        if not 0 < self.slots_per_layer <= self.total_recurrent_steps:
            raise ValueError(f"slots_per_layer must be in [1, {self.total_recurrent_steps}], got {self.slots_per_layer}")

    @classmethod
    def build(cls, *, num_prelude_layers: int, num_core_layers: int, num_coda_layers: int,
              total_recurrent_steps: int, policy: str = DEPTH_INDEXED,
              requested_slots: int | None = None) -> "LoopedKvLayout":
        return cls(num_prelude_layers, num_core_layers, num_coda_layers, total_recurrent_steps, policy,
                   resolve_kv_slots_per_layer(policy, total_recurrent_steps=total_recurrent_steps,
                                              requested_slots=requested_slots))

    @property
    def num_cache_layers(self) -> int:
        return self.num_prelude_layers + self.slots_per_layer * self.num_core_layers + self.num_coda_layers

    @property
    def core_base(self) -> int:
        return self.num_prelude_layers

    def slot_for_step(self, recurrent_step: int) -> int:
        if not 0 <= recurrent_step < self.total_recurrent_steps:
            raise ValueError(f"recurrent_step must be in [0, {self.total_recurrent_steps}), got {recurrent_step}")
        return kv_slot_for_step(recurrent_step, policy=self.policy, slots_per_layer=self.slots_per_layer)

    def prelude_layer_index(self, physical_layer_idx: int) -> int:
        self._check_layer(physical_layer_idx, self.num_prelude_layers, "prelude")
        return physical_layer_idx

    def core_layer_index(self, physical_layer_idx: int, recurrent_step: int, *, explicit_slot: int | None = None) -> int:
        self._check_layer(physical_layer_idx, self.num_core_layers, "core")
        slot = self.slot_for_step(recurrent_step) if explicit_slot is None else explicit_slot
        if not 0 <= slot < self.slots_per_layer:
            raise ValueError(f"slot must be in [0, {self.slots_per_layer}), got {slot}")
        return self.num_prelude_layers + slot * self.num_core_layers + physical_layer_idx

    def coda_layer_index(self, physical_layer_idx: int) -> int:
        self._check_layer(physical_layer_idx, self.num_coda_layers, "coda")
        return self.num_prelude_layers + self.slots_per_layer * self.num_core_layers + physical_layer_idx

    def exit_copy_layer_groups(self, exit_step: int) -> list[tuple[int, list[int]]]:
        """(source, deeper targets) per core layer for an exit at ``exit_step`` (kv_cache_policy.py:235-258)."""

        source_slot = self.slot_for_step(exit_step)
        if source_slot + 1 == self.slots_per_layer:
            return []
        return [
            (self.core_layer_index(layer, exit_step),
             [self.core_layer_index(layer, exit_step, explicit_slot=s)
              for s in range(source_slot + 1, self.slots_per_layer)])
            for layer in range(self.num_core_layers)
        ]

    @staticmethod
    def _check_layer(physical_layer_idx: int, count: int, stage: str) -> None:
        if not 0 <= physical_layer_idx < count:
            raise ValueError(f"{stage} layer index must be in [0, {count}), got {physical_layer_idx}")
