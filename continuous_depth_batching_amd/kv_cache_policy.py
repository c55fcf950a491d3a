"""Looped KV layouts as lookup tables.

A looped decoder runs its core layers once per recurrent step; a KV policy decides which KV
slot each step writes. Everything downstream -- the tick core filling launch metadata, the
decode kernel's per-row cache layer, the exit-KV copy kernel -- only needs per-step facts, so
a layout is resolved once into tables:

  * ``step_slots[s]``   the slot recurrent step ``s`` writes;
  * ``step_bases[s]``   the cache layer of core layer 0 at step ``s`` (a row's layer offset);
  * ``copy_slots[s]``   the deeper slots an exit at step ``s`` copies its KV into.

The paged pool numbers its cache layers ``[prelude | slot 0 core | ... | slot S-1 core | coda]``
(reference kv_cache_policy.py:141-233); that numbering is the cache contract, so indices agree
with the reference's for every policy. The policy table below states each policy's slot count
and step -> slot rule (reference kv_cache_policy.py:53-103).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Literal

KvCachePolicy = Literal["depth_indexed", "last_exited", "single", "first_then_shared"]

DEPTH_INDEXED = "depth_indexed"
LAST_EXITED = "last_exited"
SINGLE = "single"
FIRST_THEN_SHARED = "first_then_shared"


@dataclass(frozen=True)
class _Rule:
    fixed_slots: Callable[[int], int] | None  # steps -> slot count, or None when the caller chooses
    slot: Callable[[int, int], int]  # (step, slots) -> slot
    copies_on_exit: bool = False


_RULES: dict[str, _Rule] = {
    DEPTH_INDEXED: _Rule(lambda steps: steps, lambda step, slots: step),
    LAST_EXITED: _Rule(lambda steps: steps, lambda step, slots: step, copies_on_exit=True),
    SINGLE: _Rule(lambda steps: 1, lambda step, slots: 0),
    FIRST_THEN_SHARED: _Rule(None, lambda step, slots: step if step < slots else slots - 1),
}
KV_CACHE_POLICIES: tuple[str, ...] = tuple(_RULES)
_DEFAULT_SHARED_SLOTS = 2


def _rule(policy: str) -> _Rule:
    rule = _RULES.get(policy)
    if rule is None:
        raise ValueError(f"Unsupported KV cache policy {policy!r}; expected one of {KV_CACHE_POLICIES}")
    return rule


def validate_kv_cache_policy(policy: str) -> str:
    _rule(policy)
    return policy


def copies_exit_kv(policy: str) -> bool:
    """Whether an early exit under ``policy`` propagates its exit-step KV to the deeper slots."""

    return _rule(policy).copies_on_exit


def resolve_kv_slots_per_layer(policy: str, *, total_recurrent_steps: int, requested_slots: int | None = None) -> int:
    """Slots per core layer: derived from the step count, except for the shared-tail policy, whose
    count is requested (two by default) and bounded by the step count."""

    if total_recurrent_steps < 1:
        raise ValueError(f"total_recurrent_steps must be at least 1, got {total_recurrent_steps}")
    rule = _rule(policy)
    if rule.fixed_slots is not None:
        slots = rule.fixed_slots(total_recurrent_steps)
        if requested_slots not in (None, slots):
            raise ValueError(f"{policy!r} keeps {slots} slot(s) per layer; kv_slots_per_layer={requested_slots} "
                             "does not apply")
        return slots
    slots = _DEFAULT_SHARED_SLOTS if requested_slots is None else requested_slots
    if not 1 <= slots <= total_recurrent_steps:
        raise ValueError(f"kv_slots_per_layer must be in [1, {total_recurrent_steps}] (the recurrent step "
                         f"count), got {slots}")
    return slots


def kv_slot_for_step(recurrent_step: int, *, policy: str, slots_per_layer: int) -> int:
    if recurrent_step < 0 or slots_per_layer < 1:
        raise ValueError(f"need recurrent_step >= 0 and slots_per_layer >= 1, got {recurrent_step}, "
                         f"{slots_per_layer}")
    return _rule(policy).slot(recurrent_step, slots_per_layer)


def kv_layer_index(*, physical_layer_idx: int, num_hidden_layers: int, recurrent_step: int, policy: str,
                   slots_per_layer: int, explicit_slot: int | None = None) -> int:
    """Cache layer of a fully looped model's layer at a step: ``slot * layers + layer``."""

    if not 0 <= physical_layer_idx < max(num_hidden_layers, 0) or num_hidden_layers < 1:
        raise ValueError(f"physical_layer_idx must be in [0, {num_hidden_layers}), got {physical_layer_idx}")
    slot = kv_slot_for_step(recurrent_step, policy=policy, slots_per_layer=slots_per_layer) \
        if explicit_slot is None else explicit_slot
    if not 0 <= slot < slots_per_layer:
        raise ValueError(f"explicit_slot must be in [0, {slots_per_layer}), got {slot}")
    return slot * num_hidden_layers + physical_layer_idx


@dataclass(frozen=True)
class LoopedKvLayout:
    """A looped decoder's cache layers, resolved into per-step tables."""

    num_prelude_layers: int
    num_core_layers: int
    num_coda_layers: int
    total_recurrent_steps: int
    policy: str
    slots_per_layer: int
    step_slots: tuple[int, ...] = field(init=False)
    step_bases: tuple[int, ...] = field(init=False)
    copy_slots: tuple[tuple[int, ...], ...] = field(init=False)

    def __post_init__(self) -> None:
        rule = _rule(self.policy)
        if min(self.num_prelude_layers, self.num_coda_layers) < 0 or self.num_core_layers < 1:
            raise ValueError("need at least one core layer and non-negative prelude/coda layer counts")
        if self.total_recurrent_steps < 1:
            raise ValueError(f"total_recurrent_steps must be at least 1, got {self.total_recurrent_steps}")
        if not 1 <= self.slots_per_layer <= self.total_recurrent_steps:
            raise ValueError(f"slots_per_layer must be in [1, {self.total_recurrent_steps}], got "
                             f"{self.slots_per_layer}")
        slots = tuple(rule.slot(s, self.slots_per_layer) for s in range(self.total_recurrent_steps))
        object.__setattr__(self, "step_slots", slots)
        object.__setattr__(self, "step_bases",
                           tuple(self.num_prelude_layers + slot * self.num_core_layers for slot in slots))
        copies = tuple(tuple(range(slot + 1, self.slots_per_layer)) if rule.copies_on_exit else ()
                       for slot in slots)
        object.__setattr__(self, "copy_slots", copies)

    @classmethod
    def build(cls, *, num_prelude_layers: int, num_core_layers: int, num_coda_layers: int,
              total_recurrent_steps: int, policy: str = DEPTH_INDEXED,
              requested_slots: int | None = None) -> "LoopedKvLayout":
        slots = resolve_kv_slots_per_layer(policy, total_recurrent_steps=total_recurrent_steps,
                                           requested_slots=requested_slots)
        return cls(num_prelude_layers, num_core_layers, num_coda_layers, total_recurrent_steps, policy, slots)

    @property
    def num_cache_layers(self) -> int:
        return self.num_prelude_layers + self.slots_per_layer * self.num_core_layers + self.num_coda_layers

    @property
    def core_base(self) -> int:
        return self.num_prelude_layers

    def slot_for_step(self, recurrent_step: int) -> int:
        return self.step_slots[self._step(recurrent_step)]

    def prelude_layer_index(self, physical_layer_idx: int) -> int:
        return self._layer(physical_layer_idx, self.num_prelude_layers, "prelude")

    def core_layer_index(self, physical_layer_idx: int, recurrent_step: int, *, explicit_slot: int | None = None) -> int:
        layer = self._layer(physical_layer_idx, self.num_core_layers, "core")
        if explicit_slot is None:
            return self.step_bases[self._step(recurrent_step)] + layer
        if not 0 <= explicit_slot < self.slots_per_layer:
            raise ValueError(f"slot must be in [0, {self.slots_per_layer}), got {explicit_slot}")
        return self.num_prelude_layers + explicit_slot * self.num_core_layers + layer

    def coda_layer_index(self, physical_layer_idx: int) -> int:
        return (self.num_prelude_layers + self.slots_per_layer * self.num_core_layers
                + self._layer(physical_layer_idx, self.num_coda_layers, "coda"))

    def exit_copy_layer_groups(self, exit_step: int) -> list[tuple[int, list[int]]]:
        """(source cache layer, deeper target cache layers) per core layer for an exit at ``exit_step``."""

        targets = self.copy_slots[self._step(exit_step)]
        if not targets:
            return []
        base, stride = self.step_bases[exit_step], self.num_core_layers
        first = self.num_prelude_layers
        return [(base + layer, [first + slot * stride + layer for slot in targets])
                for layer in range(self.num_core_layers)]

    def _step(self, recurrent_step: int) -> int:
        if not 0 <= recurrent_step < self.total_recurrent_steps:
            raise ValueError(f"recurrent_step must be in [0, {self.total_recurrent_steps}), got {recurrent_step}")
        return recurrent_step

    @staticmethod
    def _layer(index: int, count: int, stage: str) -> int:
        if not 0 <= index < count:
            raise ValueError(f"{stage} layer index must be in [0, {count}), got {index}")
        return index
