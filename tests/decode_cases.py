"""Seeded paged-decode-attention cases shared by the oracle and GPU tests."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle.bf16 import rounder
from oracle.paged_attention import rope_tables


@dataclass
class DecodeCase:
    q: np.ndarray          # [B, H, D] float32 (values representable in dtype)
    k_new: np.ndarray      # [B, Hkv, D]
    v_new: np.ndarray
    kv_pool: np.ndarray    # [layers, 2, rows, Hkv, D]
    cache_layer: np.ndarray  # [B] int32
    block_table: np.ndarray  # [B, W] int32, -1 padded
    seqlens: np.ndarray      # [B] int32 (new-token position; -1 = padding)
    block_size: int
    rope: tuple[np.ndarray, np.ndarray] | None
    rope_style: int
    q_bias: np.ndarray | None
    k_bias: np.ndarray | None
    dtype: str
    scale: float


def make_case(
    *,
    seed: int,
    num_rows: int,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    max_context: int,
    num_layers: int = 4,
    block_size: int = 16,
    rope_style: int = 1,
    dtype: str = "bf16",
    padding_rows: int = 0,
    qk_bias: bool = False,
    min_context: int = 1,
    value_scale: float = 1.0,
) -> DecodeCase:
    """Rows with random positions in [min_context-1, max_context-1], random cache
    layer per row (mixed depth), and block tables drawn from a random permutation
    of the page pool."""

    rng = np.random.default_rng(seed)
    rnd = rounder(dtype)
    positions = rng.integers(min_context - 1, max_context, size=num_rows).astype(np.int64)
    if padding_rows:
        positions[-padding_rows:] = -1
    pages_per_row = np.where(positions >= 0, (positions + 1 + block_size - 1) // block_size, 0)
    total_pages = int(pages_per_row.sum()) + 3  # a few never-referenced pages
    perm = rng.permutation(total_pages).astype(np.int32)
    width = max(1, int(pages_per_row.max()) + 2)
    table = np.full((num_rows, width), -1, dtype=np.int32)
    cursor = 0
    for b, n in enumerate(pages_per_row):
        table[b, :n] = perm[cursor:cursor + n]
        cursor += n
    rows = total_pages * block_size
    kv_pool = rnd(rng.standard_normal((num_layers, 2, rows, num_kv_heads, head_dim), dtype=np.float32) * value_scale)
    q = rnd(rng.standard_normal((num_rows, num_heads, head_dim), dtype=np.float32))
    k_new = rnd(rng.standard_normal((num_rows, num_kv_heads, head_dim), dtype=np.float32))
    v_new = rnd(rng.standard_normal((num_rows, num_kv_heads, head_dim), dtype=np.float32))
    cache_layer = rng.integers(0, num_layers, size=num_rows).astype(np.int32)
    rope = None
    if rope_style:
        theta = 10000.0 if rope_style == 1 else 50000.0
        rope = rope_tables(head_dim, theta, max(int(positions.max()) + 1, 1), rope_style, dtype)
    q_bias = k_bias = None
    if qk_bias:
        q_bias = rnd(rng.standard_normal((num_heads, head_dim), dtype=np.float32) * 0.1)
        k_bias = rnd(rng.standard_normal((num_kv_heads, head_dim), dtype=np.float32) * 0.1)
    return DecodeCase(
        q=q, k_new=k_new, v_new=v_new, kv_pool=kv_pool, cache_layer=cache_layer, block_table=table,
        seqlens=positions.astype(np.int32), block_size=block_size, rope=rope, rope_style=rope_style,
        q_bias=q_bias, k_bias=k_bias, dtype=dtype, scale=float(head_dim) ** -0.5,
    )
