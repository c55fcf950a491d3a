"""The cdb:: prefill operators against the raw C-ABI launches they wrap: same outputs and the same
pool contents, to the bit (the engine's prefill calls the operators)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_prefill_operators_equal_the_raw_launches() -> None:
    from continuous_depth_batching_amd import ops
    from continuous_depth_batching_amd.workloads import rope_tables_torch

    rng = np.random.default_rng(7)
    T, H, Hkv, D, bs, layers = 300, 8, 4, 128, 16, 3
    lens, pasts = np.array([100, 200]), np.array([0, 40])
    pages = (lens + pasts + bs - 1) // bs
    perm = rng.permutation(int(pages.sum()) + 4).astype(np.int32)
    table = np.full((2, int(pages.max())), -1, np.int32)
    table[0, :pages[0]], table[1, :pages[1]] = perm[:pages[0]], perm[pages[0]:pages.sum()]
    dev = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).cuda() if dt is None else \
        torch.from_numpy(np.ascontiguousarray(a)).cuda().to(dt)
    pool = dev(rng.standard_normal((layers, 2, (int(pages.sum()) + 4) * bs, Hkv, D)).astype(np.float32), torch.bfloat16)
    qkv = dev(rng.standard_normal((T, (H + 2 * Hkv) * D)).astype(np.float32), torch.bfloat16)
    q = qkv[:, :H * D].view(T, H, D)
    k = qkv[:, H * D:(H + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (H + Hkv) * D:].view(T, Hkv, D)
    pos = np.concatenate([pasts[s] + np.arange(lens[s]) for s in range(2)])
    rows = np.array([table[s, p // bs] * bs + p % bs for s in range(2) for p in pasts[s] + np.arange(lens[s])])
    cos, sin = rope_tables_torch(D, 10000.0, 1024, torch.bfloat16, torch.device("cuda"))
    rows_d, pos_d = dev(rows.astype(np.int64)), dev(pos.astype(np.int32))

    raw_pool = pool.clone()
    q_raw = torch.empty(T, H, D, dtype=torch.bfloat16, device="cuda")
    ops.rope_kv_write_raw(q, k, v, q_raw, ops.KVPoolView(raw_pool, bs), 2, rows_d, pos_d, cos, sin, 1, None, None)
    q_op = torch.ops.cdb.rope_kv_write(q, k, v, pool, 2, bs, rows_d, pos_d, cos, sin, 1, None, None)
    torch.cuda.synchronize()
    assert torch.equal(q_op, q_raw) and torch.equal(pool, raw_pool)

    tile_seq, tile_q0 = (dev(t) for t in ops.prefill_tiles(lens, pasts))
    tbl, trow = dev(table), dev(np.arange(2, dtype=np.int32))
    cu, past = dev(np.array([0, lens[0], T], np.int32)), dev(pasts.astype(np.int32))
    out_raw = torch.empty_like(q_raw)
    view = ops.KVPoolView(pool, bs)
    ops.prefill_attention_raw(q_op, view, 2, tbl, trow, cu, past, tile_seq, tile_q0, out_raw, D ** -0.5)
    out_op = torch.ops.cdb.prefill_attention(q_op, pool, 2, bs, tbl, trow, cu, past, tile_seq, tile_q0, D ** -0.5)
    work = ops.prefill_split_work(lens, pasts, num_heads=H, max_blocks=8)
    partials = torch.empty(ops.prefill_partial_bytes(work.num_slots, H, D) // 4, dtype=torch.float32, device="cuda")
    split_raw = torch.empty_like(q_raw)
    items, merges = dev(work.items), dev(work.merges)
    ops.prefill_attention_split_raw(q_op, view, 2, tbl, trow, cu, past, items, merges, work.num_slots, partials,
                                    split_raw, D ** -0.5)
    split_op = torch.ops.cdb.prefill_attention_split(q_op, pool, 2, bs, tbl, trow, cu, past, items, merges,
                                                     work.num_slots, partials, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(out_op, out_raw) and torch.equal(split_op, split_raw)
