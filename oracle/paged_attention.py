"""Oracle: paged KV slot mapping, RoPE, and paged decode attention (numpy).

Restates:
  * slot mapping: row = block_table[pos // block_size] * block_size + pos % block_size
    (continuous_batching/cache_manager.py:190-213, get_write_indices; read
    indices :167-188);
  * Ouro split-half RoPE with cos/sin cast to the model dtype
    (ouro/modeling_ouro.py:544-573 tables, :172-204 application);
  * Huginn interleaved RoPE in fp32, rounded once (huginn/modeling_huginn.py:150-196),
    with the pre-rotation qk_bias add (:260-263);
  * flash_attn_with_kvcache as the paged decode branch uses it
    (transformers integrations/flash_paged.py:100-147): append the new K/V at
    cache_seqlens = position, then causal softmax(q K^T * scale) V over
    positions 0..position. Padding rows (position < 0) write nothing.

Pinned by (tests/test_oracle_*.py): the reference's slot-map vectors
(tests/continuous_batching/test_continuous_batching_cache_manager.py), closed
forms (single token -> output = v; identical keys -> mean of values;
position 0 RoPE = identity), invariants (RoPE preserves norms in fp32;
permuting pages together with the block table leaves outputs unchanged) and
torch's scaled_dot_product_attention on the gathered dense K/V.
"""

from __future__ import annotations

import numpy as np

from .bf16 import rounder


def write_rows(block_row: np.ndarray, positions: np.ndarray, block_size: int) -> np.ndarray:
    """Physical cache rows of ``positions`` for one sequence (cache_manager.py:190-213)."""

    positions = np.asarray(positions, dtype=np.int64)
    return np.asarray(block_row, dtype=np.int64)[positions // block_size] * block_size + positions % block_size


def read_rows(block_row: np.ndarray, total_length: int, block_size: int) -> np.ndarray:
    """Rows of positions 0..total_length-1 (cache_manager.py:167-188)."""

    return write_rows(block_row, np.arange(total_length), block_size)


def inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """1 / theta ** (arange(0, D, 2) / D) in float32 (modeling_ouro.py:555-557)."""

    exponent = (np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / np.float32(head_dim)).astype(np.float32)
    return (np.float32(1.0) / np.power(np.float32(theta), exponent, dtype=np.float32)).astype(np.float32)


def rope_tables(head_dim: int, theta: float, max_positions: int, style: int, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """[max_positions, D/2] cos/sin tables as float32.

    style 1 (Ouro): fp32 angles pos * inv_freq, cos/sin rounded to the model
    dtype (modeling_ouro.py:568-573). style 2 (Huginn): fp32 values
    (modeling_huginn.py:172-175).
    """

    freqs = (np.arange(max_positions, dtype=np.float32)[:, None] * inv_freq(head_dim, theta)[None, :]).astype(np.float32)
    cos = np.cos(freqs.astype(np.float64)).astype(np.float32)
    sin = np.sin(freqs.astype(np.float64)).astype(np.float32)
    if style == 1:
        rnd = rounder(dtype)
        cos, sin = rnd(cos), rnd(sin)
    return cos, sin


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, style: int, dtype: str) -> np.ndarray:
    """Rotate ``x [..., D]`` whose leading row axis matches ``cos/sin [rows, D/2]``.

    ``x`` has shape [rows, heads, D]; every op rounds to ``dtype`` the way the
    reference's tensors do.
    """

    rnd = rounder(dtype)
    x = np.asarray(x, dtype=np.float32)
    if style == 0:
        return x.copy()
    c = cos[:, None, :]
    s = sin[:, None, :]
    if style == 1:
        half = x.shape[-1] // 2
        c_full = np.concatenate([c, c], axis=-1)
        s_full = np.concatenate([s, s], axis=-1)
        rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)  # rotate_half, :172-176
        return rnd(rnd(x * c_full) + rnd(rot * s_full))
    if style == 2:
        even, odd = x[..., 0::2], x[..., 1::2]
        out = np.empty_like(x)
        out[..., 0::2] = (even * c).astype(np.float32) - (odd * s).astype(np.float32)
        out[..., 1::2] = (odd * c).astype(np.float32) + (even * s).astype(np.float32)
        return rnd(out)
    raise ValueError(f"unknown rope style {style}")


def paged_decode_attention(
    q: np.ndarray,
    k_new: np.ndarray,
    v_new: np.ndarray,
    kv_pool: np.ndarray,
    cache_layer: np.ndarray,
    block_table: np.ndarray,
    seqlens: np.ndarray,
    block_size: int,
    scale: float,
    *,
    rope: tuple[np.ndarray, np.ndarray] | None = None,
    rope_style: int = 0,
    q_bias: np.ndarray | None = None,
    k_bias: np.ndarray | None = None,
    table_row: np.ndarray | None = None,
    dtype: str = "bf16",
) -> np.ndarray:
    """Append each row's rotated key/value into ``kv_pool`` (in place) and attend.

    kv_pool: [layers, 2, rows, Hkv, D] float32 holding values representable in
    ``dtype``. Returns out [B, H, D] float32 (rounded to ``dtype``); padding
    rows (seqlens < 0) give zeros.
    """

    rnd = rounder(dtype)
    num_rows, num_heads, head_dim = q.shape
    num_kv_heads = k_new.shape[1]
    group = num_heads // num_kv_heads
    seqlens = np.asarray(seqlens, dtype=np.int64)
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k_new, dtype=np.float32)
    if q_bias is not None:
        q = rnd(q + q_bias[None])
    if k_bias is not None:
        k = rnd(k + k_bias[None])
    pos = np.maximum(seqlens, 0)
    if rope_style:
        cos, sin = rope
        q = apply_rope(q, cos[pos], sin[pos], rope_style, dtype)
        k = apply_rope(k, cos[pos], sin[pos], rope_style, dtype)
    out = np.zeros((num_rows, num_heads, head_dim), dtype=np.float32)
    for b in range(num_rows):
        p = int(seqlens[b])
        if p < 0:
            continue
        layer = int(cache_layer[b])
        table = block_table[b if table_row is None else int(table_row[b])]
        row_p = write_rows(table, np.array([p]), block_size)[0]
        kv_pool[layer, 0, row_p] = k[b]
        kv_pool[layer, 1, row_p] = np.asarray(v_new[b], dtype=np.float32)
        rows = read_rows(table, p + 1, block_size)
        keys = kv_pool[layer, 0, rows].astype(np.float64)  # [T, Hkv, D]
        values = kv_pool[layer, 1, rows].astype(np.float64)
        for h in range(num_heads):
            kvh = h // group
            scores = keys[:, kvh, :] @ q[b, h].astype(np.float64) * scale
            scores -= scores.max()
            weights = np.exp(scores)
            weights /= weights.sum()
            out[b, h] = (weights @ values[:, kvh, :]).astype(np.float32)
    return rnd(out)


def prefill_attention(q: np.ndarray, kv_pool: np.ndarray, layer: int, block_table: np.ndarray,
                      table_row: np.ndarray, cu_q: np.ndarray, past: np.ndarray, block_size: int, scale: float,
                      dtype: str = "bf16") -> np.ndarray:
    """Causal varlen attention over K/V already in the pool
    (flash_attn_varlen_func after PagedAttentionCache.update, continuous_batching/cache.py:284-318
    and prefill_graph.py:265-309). q: [T, H, D] rotated; returns [T, H, D]."""

    rnd = rounder(dtype)
    tokens, num_heads, head_dim = q.shape
    num_kv_heads = kv_pool.shape[3]
    group = num_heads // num_kv_heads
    out = np.zeros_like(q, dtype=np.float32)
    for s in range(len(past)):
        begin, end = int(cu_q[s]), int(cu_q[s + 1])
        n = end - begin
        if n == 0:
            continue
        total = int(past[s]) + n
        rows = read_rows(block_table[int(table_row[s])], total, block_size)
        keys = kv_pool[layer, 0, rows].astype(np.float64)
        values = kv_pool[layer, 1, rows].astype(np.float64)
        qpos = int(past[s]) + np.arange(n)
        mask = np.arange(total)[None, :] <= qpos[:, None]
        for h in range(num_heads):
            kvh = h // group
            scores = q[begin:end, h].astype(np.float64) @ keys[:, kvh, :].T * scale
            scores = np.where(mask, scores, -np.inf)
            scores -= scores.max(axis=1, keepdims=True)
            w = np.exp(scores)
            w /= w.sum(axis=1, keepdims=True)
            out[begin:end, h] = (w @ values[:, kvh, :]).astype(np.float32)
    return rnd(out)
