"""The looped KV layout (slot -> cache layer) against the reference's own vectors.

Expected values are those asserted by the reference's tests/test_looped_kv_layout.py
(cited per test) for the Huginn stage split (2 prelude + 4 core + 2 coda layers,
8 recurrent steps) and for a fully looped Ouro model.
"""

from __future__ import annotations

import pytest

from continuous_depth_batching_amd.kv_cache_policy import (
    LoopedKvLayout,
    copies_exit_kv,
    kv_layer_index,
    kv_slot_for_step,
    resolve_kv_slots_per_layer,
)


def _huginn(policy: str, steps: int = 8) -> LoopedKvLayout:
    return LoopedKvLayout.build(num_prelude_layers=2, num_core_layers=4, num_coda_layers=2,
                                total_recurrent_steps=steps, policy=policy)


@pytest.mark.parametrize("policy,slots,cache_layers", [
    ("depth_indexed", 8, 2 + 8 * 4 + 2),
    ("last_exited", 8, 2 + 8 * 4 + 2),
    ("single", 1, 2 + 1 * 4 + 2),
    ("first_then_shared", 2, 2 + 2 * 4 + 2),
])
def test_cache_layer_count(policy: str, slots: int, cache_layers: int) -> None:
    # test_looped_kv_layout.py:20-34
    layout = _huginn(policy)
    assert layout.slots_per_layer == slots
    assert layout.num_cache_layers == cache_layers


def test_prelude_and_coda_indices() -> None:
    # test_looped_kv_layout.py:37-42
    layout = _huginn("first_then_shared")
    assert [layout.prelude_layer_index(i) for i in range(2)] == [0, 1]
    assert [layout.coda_layer_index(i) for i in range(2)] == [10, 11]


def test_stage_indices_are_disjoint_and_dense() -> None:
    # test_looped_kv_layout.py:45-54
    layout = _huginn("first_then_shared")
    idx = {layout.prelude_layer_index(i) for i in range(2)} | {layout.coda_layer_index(i) for i in range(2)}
    for step in range(layout.total_recurrent_steps):
        idx |= {layout.core_layer_index(i, step) for i in range(4)}
    assert idx == set(range(layout.num_cache_layers))


@pytest.mark.parametrize("policy,expected", [
    ("single", [2, 2, 2, 2, 2, 2, 2, 2]),
    ("first_then_shared", [2, 6, 6, 6, 6, 6, 6, 6]),
    ("depth_indexed", [2, 6, 10, 14, 18, 22, 26, 30]),
    ("last_exited", [2, 6, 10, 14, 18, 22, 26, 30]),
])
def test_core_slot_assignment_per_step(policy: str, expected: list[int]) -> None:
    # test_looped_kv_layout.py:55-67
    layout = _huginn(policy)
    assert [layout.core_layer_index(0, step) for step in range(8)] == expected


@pytest.mark.parametrize("policy", ["single", "first_then_shared", "depth_indexed", "last_exited"])
def test_fully_looped_model_matches_flat_indexing(policy: str) -> None:
    # test_looped_kv_layout.py:70-90: no prelude/coda reproduces slot * L + layer.
    layout = LoopedKvLayout.build(num_prelude_layers=0, num_core_layers=24, num_coda_layers=0,
                                  total_recurrent_steps=4, policy=policy)
    for step in range(4):
        for layer in range(24):
            assert layout.core_layer_index(layer, step) == kv_layer_index(
                physical_layer_idx=layer, num_hidden_layers=24, recurrent_step=step, policy=policy,
                slots_per_layer=layout.slots_per_layer)


def test_exit_copy_groups_target_every_deeper_slot() -> None:
    # test_looped_kv_layout.py:93-107
    layout = _huginn("last_exited", steps=4)
    assert layout.exit_copy_layer_groups(1) == [
        (layout.core_layer_index(l, 1), [layout.core_layer_index(l, 1, explicit_slot=s) for s in (2, 3)])
        for l in range(4)]
    assert layout.exit_copy_layer_groups(3) == []
    assert layout.exit_copy_layer_groups(1)[0] == (2 + 1 * 4 + 0, [2 + 2 * 4, 2 + 3 * 4])


def test_slot_sharing_layouts_copy_nothing() -> None:
    # test_looped_kv_layout.py:110-114
    assert _huginn("single").exit_copy_layer_groups(0) == []
    assert _huginn("first_then_shared").exit_copy_layer_groups(1) == []
    assert copies_exit_kv("last_exited") and not copies_exit_kv("first_then_shared")
    assert not copies_exit_kv("single") and not copies_exit_kv("depth_indexed")


def test_out_of_range_layers_steps_and_slots_are_rejected() -> None:
    # test_looped_kv_layout.py:117-146
    layout = _huginn("single", steps=4)
    with pytest.raises(ValueError, match="prelude layer index"):
        layout.prelude_layer_index(2)
    with pytest.raises(ValueError, match="coda layer index"):
        layout.coda_layer_index(2)
    with pytest.raises(ValueError, match="core layer index"):
        layout.core_layer_index(4, 0)
    with pytest.raises(ValueError, match="recurrent_step"):
        layout.core_layer_index(0, 4)
    with pytest.raises(ValueError, match="slots_per_layer"):
        LoopedKvLayout(num_prelude_layers=2, num_core_layers=4, num_coda_layers=2, total_recurrent_steps=2,
                       policy="first_then_shared", slots_per_layer=4)


def test_slot_resolution_rules() -> None:
    # kv_cache_policy.py:53-103: fixed slot counts, the shared policy's default of 2, step -> slot.
    assert resolve_kv_slots_per_layer("depth_indexed", total_recurrent_steps=4) == 4
    assert resolve_kv_slots_per_layer("single", total_recurrent_steps=4) == 1
    assert resolve_kv_slots_per_layer("first_then_shared", total_recurrent_steps=4) == 2
    assert resolve_kv_slots_per_layer("first_then_shared", total_recurrent_steps=4, requested_slots=3) == 3
    with pytest.raises(ValueError):
        resolve_kv_slots_per_layer("single", total_recurrent_steps=4, requested_slots=2)
    with pytest.raises(ValueError):
        resolve_kv_slots_per_layer("first_then_shared", total_recurrent_steps=4, requested_slots=5)
    assert [kv_slot_for_step(s, policy="first_then_shared", slots_per_layer=3) for s in range(5)] == [0, 1, 2, 2, 2]


def test_prefill_tiles_cover_every_query_tile_once_longest_prefix_first() -> None:
    import numpy as np

    from continuous_depth_batching_amd import ops

    lens = np.array([130, 1, 64, 65, 0, 300])
    past = np.array([0, 500, 10, 0, 7, 64])
    seq, q0 = ops.prefill_tiles(lens, past)
    tiles = sorted(zip(seq.tolist(), q0.tolist()))
    want = sorted((s, t) for s, n in enumerate(lens.tolist()) for t in range(0, n, ops.PREFILL_TILE))
    assert tiles == want
    key_end = past[seq] + np.minimum(q0 + ops.PREFILL_TILE, lens[seq])
    assert (np.diff(key_end) <= 0).all()
    # Without past lengths the prefixes are the query positions alone.
    seq0, q00 = ops.prefill_tiles(lens)
    assert sorted(zip(seq0.tolist(), q00.tolist())) == want


@pytest.mark.parametrize("max_blocks", [8, 16, 37])
def test_prefill_split_work_partitions_each_tile_and_keeps_the_diagonal_in_the_last_part(max_blocks: int) -> None:
    """Every tile's key blocks [0, blocks) are covered once by consecutive parts of at most about
    max_blocks blocks; a split tile's last part starts at or before the block of the tile's first
    query (so each query sees a key of every part); slots are consecutive per merge and unique;
    items are listed longest first."""

    import numpy as np

    from continuous_depth_batching_amd import ops

    lens = np.array([130, 1, 64, 65, 300, 900])
    past = np.array([0, 5000, 10, 1000, 64, 0])
    work = ops.prefill_split_work(lens, past, num_heads=4, max_blocks=max_blocks)
    parts: dict[tuple[int, int], list[tuple[int, int, int]]] = {}
    for s, q0, kv, slot in work.items.tolist():
        parts.setdefault((s, q0), []).append((kv & 0xFFFF, kv >> 16, slot))
    want_tiles = sorted((s, t) for s, n in enumerate(lens.tolist()) for t in range(0, n, ops.PREFILL_TILE))
    assert sorted(parts) == want_tiles
    merges = {(s, q0): (first, n) for s, q0, first, n in work.merges.tolist()}
    slots = []
    for (s, q0), ps in parts.items():
        ps.sort()
        key_end = past[s] + min(q0 + ops.PREFILL_TILE, lens[s])
        blocks = -(-key_end // ops.PREFILL_KEY_BLOCK)
        assert ps[0][0] == 0 and ps[-1][1] == blocks
        assert all(a[1] == b[0] for a, b in zip(ps, ps[1:]))
        if len(ps) == 1:
            assert ps[0][2] == -1 and (s, q0) not in merges
            assert blocks <= max_blocks
            continue
        assert ps[-1][0] <= (past[s] + q0) // ops.PREFILL_KEY_BLOCK
        assert all(b - a <= max_blocks + 5 for a, b, _ in ps)
        first, n = merges[(s, q0)]
        assert [slot for _, _, slot in ps] == list(range(first, first + n))
        slots.extend(range(first, first + n))
    assert sorted(slots) == list(range(work.num_slots))
    length = (work.items[:, 2] >> 16) - (work.items[:, 2] & 0xFFFF)
    assert (np.diff(length) <= 0).all()


def test_prefill_split_plan_splits_only_a_tile_that_outlasts_the_launch() -> None:
    import numpy as np

    from continuous_depth_batching_amd import ops

    # Fresh prompts: many tiles, none longer than four even shares -> whole tiles.
    assert ops.prefill_split_plan(np.full(27, 300), None, num_heads=16, num_cus=256) is None
    # A short chunk after a long history: a handful of tiles with thousands of keys each.
    plan = ops.prefill_split_plan([128] * 4, [16000] * 4, num_heads=16, num_cus=256)
    assert plan is not None and plan.num_slots > 0 and len(plan.merges) == 4
    assert ops.prefill_partial_bytes(plan.num_slots, 16, 128) == plan.num_slots * 16 * 128 * 130 * 4
