"""Pin the attention/RoPE/slot-map oracle before trusting it as the checker.

Each check is chosen so that a plausible mistake (wrong page index, missing
scale, transposed operand, off-by-one in the causal length, wrong rotation
half) fails it.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.bf16 import round_bf16
from oracle.paged_attention import (
    apply_rope,
    inv_freq,
    paged_decode_attention,
    read_rows,
    rope_tables,
    write_rows,
)
from tests.decode_cases import make_case

GOLDEN = Path(__file__).parent / "golden"


def test_bf16_rounding_matches_torch() -> None:
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 100,
        np.array([0.0, -0.0, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 3.4e38, -3.4e38, 1e-40, np.inf, -np.inf], np.float32),
    ])
    expected = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(round_bf16(x), expected)


def test_slot_mapping_golden_vectors() -> None:
    data = json.loads((GOLDEN / "slot_mapping.json").read_text())
    for case in data["cases"]:
        blocks = np.array(case["blocks"])
        bs = case["block_size"]
        past, qlen = case["past_length"], case["query_length"]
        if case["kind"] == "read":
            got = read_rows(blocks, past + qlen, bs).tolist()
        elif case["kind"] == "write":
            got = write_rows(blocks, np.arange(past, past + qlen), bs).tolist()
        else:
            needed = -(-(past + qlen) // bs)
            got = [int(b) for b in blocks[:needed]] + [-1] * (case["width"] - needed)
        assert got == case["expected"], case


def _dense_reference(case, out_rows):
    """torch SDPA on K/V gathered densely per row (after the oracle's append)."""

    outs = []
    for b in out_rows:
        p = int(case.seqlens[b])
        rows = read_rows(case.block_table[b], p + 1, case.block_size)
        k = torch.from_numpy(case.kv_pool[case.cache_layer[b], 0, rows]).double().transpose(0, 1)  # [Hkv, T, D]
        v = torch.from_numpy(case.kv_pool[case.cache_layer[b], 1, rows]).double().transpose(0, 1)
        qb = torch.from_numpy(case.q[b]).double()
        if case.rope_style:
            cos, sin = case.rope
            qb = torch.from_numpy(apply_rope(case.q[b:b + 1], cos[[p]], sin[[p]], case.rope_style, case.dtype)[0]).double()
        group = qb.shape[0] // k.shape[0]
        k = k.repeat_interleave(group, 0)
        v = v.repeat_interleave(group, 0)
        o = torch.nn.functional.scaled_dot_product_attention(qb[:, None, :], k, v, scale=case.scale)
        outs.append(o[:, 0, :].numpy())
    return np.stack(outs)


@pytest.mark.parametrize("rope_style,num_kv_heads", [(0, 4), (1, 4), (2, 2)])
def test_oracle_matches_sdpa_on_gathered_kv(rope_style: int, num_kv_heads: int) -> None:
    case = make_case(seed=1, num_rows=6, num_heads=4, num_kv_heads=num_kv_heads, head_dim=64, max_context=70,
                     rope_style=rope_style, dtype="f32", padding_rows=1)
    out = paged_decode_attention(case.q, case.k_new, case.v_new, case.kv_pool, case.cache_layer, case.block_table,
                                 case.seqlens, case.block_size, case.scale, rope=case.rope,
                                 rope_style=case.rope_style, dtype="f32")
    live = [b for b in range(6) if case.seqlens[b] >= 0]
    np.testing.assert_allclose(out[live], _dense_reference(case, live), atol=2e-6, rtol=1e-5)
    assert np.all(out[5] == 0.0)


def test_single_token_attends_only_to_itself() -> None:
    case = make_case(seed=2, num_rows=3, num_heads=2, num_kv_heads=2, head_dim=64, max_context=1, rope_style=1,
                     dtype="f32")
    assert np.all(case.seqlens == 0)
    out = paged_decode_attention(case.q, case.k_new, case.v_new, case.kv_pool, case.cache_layer, case.block_table,
                                 case.seqlens, case.block_size, case.scale, rope=case.rope, rope_style=1, dtype="f32")
    np.testing.assert_allclose(out, case.v_new, atol=1e-6)


def test_identical_keys_give_mean_of_values() -> None:
    case = make_case(seed=3, num_rows=2, num_heads=2, num_kv_heads=2, head_dim=64, max_context=40, rope_style=0,
                     dtype="f32", min_context=30)
    case.kv_pool[:, 0] = 0.5
    case.k_new[:] = 0.5
    out = paged_decode_attention(case.q, case.k_new, case.v_new, case.kv_pool, case.cache_layer, case.block_table,
                                 case.seqlens, case.block_size, case.scale, dtype="f32")
    for b in range(2):
        rows = read_rows(case.block_table[b], int(case.seqlens[b]) + 1, case.block_size)
        mean_v = case.kv_pool[case.cache_layer[b], 1, rows].mean(axis=0)
        np.testing.assert_allclose(out[b], mean_v, atol=1e-5)


def test_page_permutation_invariance() -> None:
    case = make_case(seed=4, num_rows=4, num_heads=2, num_kv_heads=2, head_dim=64, max_context=90, rope_style=1,
                     dtype="f32")
    pool_before = case.kv_pool.copy()
    out = paged_decode_attention(case.q, case.k_new, case.v_new, case.kv_pool, case.cache_layer, case.block_table,
                                 case.seqlens, case.block_size, case.scale, rope=case.rope, rope_style=1, dtype="f32")
    # Move every page to a new physical block and remap the tables accordingly.
    num_pages = pool_before.shape[2] // case.block_size
    perm = np.random.default_rng(5).permutation(num_pages)
    paged = pool_before.reshape(pool_before.shape[0], 2, num_pages, case.block_size, *pool_before.shape[3:])
    moved = np.empty_like(paged)
    moved[:, :, perm] = paged
    moved = moved.reshape(pool_before.shape)
    table = np.where(case.block_table >= 0, perm[np.maximum(case.block_table, 0)], -1).astype(np.int32)
    out2 = paged_decode_attention(case.q, case.k_new, case.v_new, moved, case.cache_layer, table, case.seqlens,
                                  case.block_size, case.scale, rope=case.rope, rope_style=1, dtype="f32")
    np.testing.assert_array_equal(out, out2)


@pytest.mark.parametrize("style", [1, 2])
def test_rope_position_zero_is_identity_and_preserves_norm(style: int) -> None:
    cos, sin = rope_tables(64, 10000.0, 50, style, "f32")
    x = np.random.default_rng(6).standard_normal((50, 3, 64)).astype(np.float32)
    y = apply_rope(x, cos, sin, style, "f32")
    np.testing.assert_allclose(y[0], x[0], atol=1e-7)
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


def test_split_half_rope_matches_complex_rotation_of_halves() -> None:
    """Split-half RoPE rotates the pair (x[i], x[i + D/2]) by angle pos * inv_freq[i]."""

    cos, sin = rope_tables(64, 10000.0, 20, 1, "f32")
    x = np.random.default_rng(7).standard_normal((20, 1, 64)).astype(np.float32)
    y = apply_rope(x, cos, sin, 1, "f32")
    z = (x[..., :32] + 1j * x[..., 32:]) * np.exp(1j * (np.arange(20)[:, None, None] * inv_freq(64, 10000.0)))
    np.testing.assert_allclose(y[..., :32], z.real, atol=2e-5)
    np.testing.assert_allclose(y[..., 32:], z.imag, atol=2e-5)


def test_interleaved_rope_matches_complex_rotation_of_pairs() -> None:
    cos, sin = rope_tables(64, 50000.0, 20, 2, "f32")
    x = np.random.default_rng(8).standard_normal((20, 1, 64)).astype(np.float32)
    y = apply_rope(x, cos, sin, 2, "f32")
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * np.exp(1j * (np.arange(20)[:, None, None] * inv_freq(64, 50000.0)))
    np.testing.assert_allclose(y[..., 0::2], z.real, atol=2e-5)
    np.testing.assert_allclose(y[..., 1::2], z.imag, atol=2e-5)
