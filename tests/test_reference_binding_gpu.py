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
        B, H, Hkv, D, block, 0, 8, 32, scaling, 0, 0,
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
