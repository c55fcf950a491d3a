"""The reference-side binding of decode attention, run on the GPU.

A maintainer registering this library under the reference's attention registry
(continuous_batching/prefill_graph.py:333-346) replaces flash_attn_with_kvcache
(transformers integrations/flash_paged.py:100-147) with the ctypes stub below. It sees the
reference's own data structures: one K and one V tensor per cache layer, each allocated by
its own torch.empty (continuous_batching/cache.py:125-144, [(blocks + 2) * block, Hkv, D]),
a grouped block table [1, tokens, width] (input_outputs.py:181-186), cu_seq_lens_k that
count the new token, and q/k/v as [1, heads, tokens, D] already rotated by the model's
rotary module. The stub passes the module's layer tensors as a one-layer pool, so nothing
depends on where the allocator placed the other layers.

Checked against the float64 oracle: the attention output within the bf16 bar of the decode
kernel's own tests, and the appended K/V rows bit-exact in the layer's tensors (and no other
layer touched).
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def cdb_paged_decode(module, q, k, v, *, cache, block_table, cu_seq_lens_k, scaling, **kw):
    from continuous_depth_batching_amd import _lib   # loads libcdb_amd.so, sets argtypes

    # q: [1, H, B, D]; k, v: [1, Hkv, B, D], rotated by the caller's rotary module
    H, B, D = q.shape[1], q.shape[2], q.shape[3]
    Hkv = k.shape[1]
    k_layer = cache.key_cache[module.layer_idx]          # [(NB + 2) * block, Hkv, D]
    v_layer = cache.value_cache[module.layer_idx]
    block = cache.block_size
    table = block_table[0]                               # [B, W] int32
    seqlens = (cu_seq_lens_k[1:] - cu_seq_lens_k[:-1] - 1).to(torch.int32)   # the new token's position
    out = torch.empty(B, H, D, dtype=q.dtype, device=q.device)
    ws = torch.empty(_lib.lib().cdb_paged_decode_workspace_bytes(B, H, D, table.shape[-1] * block, block, 8) // 4,
                     dtype=torch.float32, device=q.device)
    qb, kb, vb = (t[0].transpose(0, 1).contiguous() for t in (q, k, v))     # [B, heads, D]
    rc = _lib.lib().cdb_paged_decode_attention(
        qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), k_layer.data_ptr(), v_layer.data_ptr(),
        0, 1, k_layer.shape[0] // block,                 # this layer's tensors as a one-layer pool
        None, 0,                                         # no per-row cache layer
        table.data_ptr(), None, table.shape[-1], seqlens.data_ptr(),
        None, None, 0, 0,                                # no fused RoPE
        None, None, out.data_ptr(), ws.data_ptr(), ws.numel() * 4,
        B, H, Hkv, D, block, 0, 8, scaling, 0, 0,
        _lib.CDB_DTYPE_BF16, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "cdb_paged_decode_attention")
    return out, None


@pytest.mark.parametrize("kv_heads", [16, 4])
def test_reference_binding_call_shape(kv_heads: int) -> None:
    from oracle.paged_attention import paged_decode_attention

    rng = np.random.default_rng(21 + kv_heads)
    heads, dim, block, layers, num_blocks = 16, 128, 16, 3, 96
    positions = np.array([0, 15, 16, 300, 511, 77], np.int64)   # the new token's position per row
    B = len(positions)
    width = int((positions.max() + 1 + block - 1) // block) + 2
    pages = [int((p + 1 + block - 1) // block) for p in positions]
    perm = rng.permutation(num_blocks)
    table = np.full((B, width), -1, np.int32)
    k0 = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[k0:k0 + n]
        k0 += n
    rows = (num_blocks + 2) * block
    r16 = lambda a: torch.from_numpy(a).to(torch.bfloat16)
    key_host = [r16(rng.standard_normal((rows, kv_heads, dim)).astype(np.float32)) for _ in range(layers)]
    val_host = [r16(rng.standard_normal((rows, kv_heads, dim)).astype(np.float32)) for _ in range(layers)]
    cache = SimpleNamespace(block_size=block, key_cache=[], value_cache=[])
    for li in range(layers):   # one allocation per layer tensor, as the reference's cache does
        cache.key_cache.append(key_host[li].cuda())
        cache.value_cache.append(val_host[li].cuda())
    q = r16(rng.standard_normal((1, heads, B, dim)).astype(np.float32))
    k = r16(rng.standard_normal((1, kv_heads, B, dim)).astype(np.float32))
    v = r16(rng.standard_normal((1, kv_heads, B, dim)).astype(np.float32))
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(positions + 1)]).astype(np.int32)).cuda()
    block_table = torch.from_numpy(table[None]).cuda()
    module = SimpleNamespace(layer_idx=1)
    scale = dim ** -0.5
    print(f"[binding] kv_heads {kv_heads} rows {B} positions {positions.tolist()}", flush=True)
    out, _ = cdb_paged_decode(module, q.cuda(), k.cuda(), v.cuda(), cache=cache, block_table=block_table,
                              cu_seq_lens_k=cu, scaling=scale)
    torch.cuda.synchronize()

    pool = np.stack([np.stack([key_host[li].float().numpy(), val_host[li].float().numpy()]) for li in range(layers)])
    want = paged_decode_attention(q[0].transpose(0, 1).float().numpy(), k[0].transpose(0, 1).float().numpy(),
                                  v[0].transpose(0, 1).float().numpy(), pool, np.full(B, 1), table, positions, block,
                                  scale, dtype="bf16")
    got = out.float().cpu().numpy()
    err = np.abs(got - want)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
    for li in range(layers):
        assert np.array_equal(cache.key_cache[li].float().cpu().numpy(), pool[li, 0]), f"layer {li} keys"
        assert np.array_equal(cache.value_cache[li].float().cpu().numpy(), pool[li, 1]), f"layer {li} values"


# ---------------------------------------------------------------------------------------------
# Prefill: the varlen branch (continuous_batching/prefill_graph.py:265-309). The reference writes
# the chunk's K/V at write_index rows of the layer's tensors, reads every sequence's [past | new]
# rows back through read_index (empty when no sequence has a past), and calls
# flash_attn_varlen_func with cu_seq_lens_q / cu_seq_lens_k. The stub below replaces both halves:
# cdb_rope_kv_write (no rotation: the model's rotary module already ran) at write_index, then
# cdb_prefill_attention through a block table whose pages are read off each sequence's run of
# read_index (write_index when the batch reads no cache). The 128-query tile list is host
# metadata; the stub reads cu_seq_lens_q back for it, where an integration would build it next
# to the reference's host-side cu_seq_lens_q (input_outputs.py:303-376).

def cdb_paged_prefill(module, q, k, v, *, cache, cu_seq_lens_q, cu_seq_lens_k, max_seqlen_k, read_index,
                      write_index, scaling, **kw):
    from continuous_depth_batching_amd import _lib, ops   # loads libcdb_amd.so, sets argtypes

    # q: [1, H, T, D]; k, v: [1, Hkv, T, D], rotated by the caller's rotary module
    H, T, D = q.shape[1], q.shape[2], q.shape[3]
    Hkv = k.shape[1]
    k_layer = cache.key_cache[module.layer_idx]          # [(NB + 2) * block, Hkv, D]
    v_layer = cache.value_cache[module.layer_idx]
    block = cache.block_size
    stream = torch.cuda.current_stream().cuda_stream
    qt, kt, vt = (t[0].transpose(0, 1).contiguous() for t in (q, k, v))     # [T, heads, D]
    q_same = torch.empty_like(qt)                        # rope_style 0 copies q
    unused_positions = torch.zeros(T, dtype=torch.int32, device=q.device)
    rc = _lib.lib().cdb_rope_kv_write(
        qt.data_ptr(), kt.data_ptr(), vt.data_ptr(), q_same.data_ptr(), k_layer.data_ptr(), v_layer.data_ptr(),
        0, 0, write_index.data_ptr(), k_layer.shape[0],    # this layer's tensors as a one-layer pool
        unused_positions.data_ptr(), None, None, 0, 0, None, None,
        T, H, Hkv, D, 0, 0, _lib.CDB_DTYPE_BF16, stream)
    _lib.check(rc, "cdb_rope_kv_write")
    cu_q, cu_k = cu_seq_lens_q.to(torch.int32), cu_seq_lens_k.to(torch.int32)
    lens_k = cu_k[1:] - cu_k[:-1]
    past = (lens_k - (cu_q[1:] - cu_q[:-1])).contiguous()
    src = read_index if read_index.numel() else write_index   # no reads: cu_seq_lens_k equals cu_seq_lens_q
    width = -(-int(max_seqlen_k) // block)
    offs = torch.arange(width, dtype=torch.int64, device=q.device) * block
    at = (cu_k[:-1, None].long() + offs[None, :]).clamp(max=src.numel() - 1)
    table = torch.where(offs[None, :] < lens_k[:, None], src[at] // block, -1).to(torch.int32).contiguous()
    seqs = past.numel()
    seq_rows = torch.arange(seqs, dtype=torch.int32, device=q.device)
    host_q = cu_seq_lens_q.cpu().numpy()
    tile_seq, tile_q0 = ops.prefill_tiles(np.diff(host_q), past.cpu().numpy())
    tile_seq, tile_q0 = (torch.from_numpy(t).to(q.device) for t in (tile_seq, tile_q0))
    out = torch.empty_like(qt)
    rc = _lib.lib().cdb_prefill_attention(
        qt.data_ptr(), k_layer.data_ptr(), v_layer.data_ptr(), 0, 0, 1, k_layer.shape[0] // block,
        table.data_ptr(), seq_rows.data_ptr(), width, cu_q.data_ptr(), past.data_ptr(), seqs,
        tile_seq.data_ptr(), tile_q0.data_ptr(), tile_seq.numel(), out.data_ptr(), H, Hkv, D, block, scaling,
        _lib.CDB_DTYPE_BF16, stream)
    _lib.check(rc, "cdb_prefill_attention")
    return out, None


def _reference_indices(blocks: list[int], past: int, query: int, block: int, reads: bool):
    """The write and read rows of one request, as FullAttentionCacheAllocator.get_write_indices /
    get_read_indices build them (continuous_batching/cache_manager.py:167-213)."""

    rows = [blocks[p // block] * block + p % block for p in range(past + query)]
    return rows[past:], rows if reads else []


@pytest.mark.parametrize("chunked", [False, True])
def test_reference_prefill_binding_call_shape(chunked: bool) -> None:
    from oracle.paged_attention import prefill_attention

    rng = np.random.default_rng(40 + chunked)
    heads, kv_heads, dim, block, layers, num_blocks = 8, 4, 128, 16, 3, 160
    pasts = np.array([0, 300, 0, 17] if chunked else [0, 0, 0, 0], np.int64)
    lens = np.array([37, 64, 150, 1], np.int64)
    pages = [int(-(-(p + n) // block)) for p, n in zip(pasts, lens)]
    perm = rng.permutation(num_blocks).tolist()
    blocks, k0 = [], 0
    for n in pages:
        blocks.append(perm[k0:k0 + n])
        k0 += n
    rows_total = (num_blocks + 2) * block
    r16 = lambda a: torch.from_numpy(a).to(torch.bfloat16)
    key_host = [r16(rng.standard_normal((rows_total, kv_heads, dim)).astype(np.float32)) for _ in range(layers)]
    val_host = [r16(rng.standard_normal((rows_total, kv_heads, dim)).astype(np.float32)) for _ in range(layers)]
    cache = SimpleNamespace(block_size=block, key_cache=[], value_cache=[])
    for li in range(layers):   # one allocation per layer tensor, as the reference's cache does
        cache.key_cache.append(key_host[li].cuda())
        cache.value_cache.append(val_host[li].cuda())
    write, read = [], []
    for b, p, n in zip(blocks, pasts, lens):
        w, r = _reference_indices(b, int(p), int(n), block, reads=bool(pasts.any()))
        write += w
        read += r
    T = int(lens.sum())
    q = r16(rng.standard_normal((1, heads, T, dim)).astype(np.float32))
    k = r16(rng.standard_normal((1, kv_heads, T, dim)).astype(np.float32))
    v = r16(rng.standard_normal((1, kv_heads, T, dim)).astype(np.float32))
    cu_q = np.concatenate([[0], np.cumsum(lens)])
    cu_k = np.concatenate([[0], np.cumsum(pasts + lens)]) if pasts.any() else cu_q
    i64 = lambda a: torch.tensor(a, dtype=torch.int64, device="cuda")
    module = SimpleNamespace(layer_idx=1)
    scale = dim ** -0.5
    print(f"[prefill binding] chunked {chunked} past {pasts.tolist()} lens {lens.tolist()}", flush=True)
    out, _ = cdb_paged_prefill(module, q.cuda(), k.cuda(), v.cuda(), cache=cache,
                               cu_seq_lens_q=i64(cu_q).to(torch.int32), cu_seq_lens_k=i64(cu_k).to(torch.int32),
                               max_seqlen_k=int((pasts + lens).max()), read_index=i64(read),
                               write_index=i64(write), scaling=scale)
    torch.cuda.synchronize()

    # The write half: exactly the chunk's rows of layer 1 change, to the chunk's K/V.
    pool = np.stack([np.stack([key_host[li].float().numpy(), val_host[li].float().numpy()]) for li in range(layers)])
    pool[1, 0, write] = k[0].transpose(0, 1).float().numpy()
    pool[1, 1, write] = v[0].transpose(0, 1).float().numpy()
    for li in range(layers):
        assert np.array_equal(cache.key_cache[li].float().cpu().numpy(), pool[li, 0]), f"layer {li} keys"
        assert np.array_equal(cache.value_cache[li].float().cpu().numpy(), pool[li, 1]), f"layer {li} values"
    # The attention half against the float64 oracle over the same pool and pages.
    table = np.full((len(lens), max(pages)), -1, np.int32)
    for s, b in enumerate(blocks):
        table[s, :len(b)] = b
    want = prefill_attention(q[0].transpose(0, 1).float().numpy(), pool, 1, table, np.arange(len(lens)),
                             cu_q, pasts, block, scale, "bf16")
    err = np.abs(out.float().cpu().numpy() - want)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())
