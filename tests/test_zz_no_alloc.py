"""cdb_paged_decode_attention_noalloc against cdb_paged_decode_attention, through the C ABI.

The allocation-free variant keeps its split partials in a fixed per-GPU device array instead of
a caller workspace. Given a caller workspace of the same size, both entry points choose the same
splits, so outputs and appended KV rows must be bit-identical; both must also meet the decode
attention bar against the float64 oracle. Two calls in a row, the second with a smaller batch,
check that the array's previous contents never leak into a later call.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle.paged_attention import paged_decode_attention as oracle_decode
from tests.decode_cases import make_case

pytestmark = pytest.mark.gpu


def _args(case, tensors, out, *, workspace=None):
    from continuous_depth_batching_amd import ops

    q, k, v, pool, layer, table, seqlens, cos, sin = tensors
    rows, heads, dim = q.shape
    pool_rows = pool.shape[2]
    layer_stride = 2 * pool_rows * pool.shape[3] * dim
    common_head = [q.data_ptr(), k.data_ptr(), v.data_ptr(), pool[0, 0].data_ptr(), pool[0, 1].data_ptr(),
                   layer_stride, pool.shape[0], pool_rows // case.block_size, layer.data_ptr(), 0,
                   table.data_ptr(), None, table.shape[1], seqlens.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                   case.rope_style, cos.shape[0], None, None, out.data_ptr()]
    ws = [] if workspace is None else [workspace.data_ptr(), workspace.numel() * 4]
    tail = [rows, heads, k.shape[1], dim, case.block_size, 0, ops.MIN_SPLIT_PAGES,
            ctypes.c_float(case.scale), 0, 0, 1, torch.cuda.current_stream().cuda_stream]
    return common_head + ws + tail


def _device(case):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return [t(case.q).bfloat16(), t(case.k_new).bfloat16(), t(case.v_new).bfloat16(),
            t(case.kv_pool).bfloat16().contiguous(), t(case.cache_layer), t(case.block_table), t(case.seqlens),
            t(case.rope[0]), t(case.rope[1])]


@pytest.mark.parametrize("rows", [(48, 7), (256, 16)])
def test_noalloc_entry_point_matches_the_workspace_entry_point_on_two_calls(rows) -> None:
    from continuous_depth_batching_amd import _lib

    lib = _lib.lib()
    for call, num_rows in enumerate(rows):
        case = make_case(seed=40 + call, num_rows=num_rows, num_heads=16, num_kv_heads=16, head_dim=128,
                         max_context=700, rope_style=1, dtype="bf16", padding_rows=1)
        print(f"[no-alloc] call {call}: {num_rows} rows", flush=True)
        with_ws, without = _device(case), _device(case)
        out_ws = torch.empty_like(with_ws[0])
        out_na = torch.full_like(without[0], float("nan"))
        workspace = torch.empty(_lib.CDB_DECODE_SCRATCH_BYTES // 4, dtype=torch.float32, device="cuda")
        rc = lib.cdb_paged_decode_attention(*_args(case, with_ws, out_ws, workspace=workspace))
        assert rc == _lib.CDB_OK
        rc = lib.cdb_paged_decode_attention_noalloc(*_args(case, without, out_na))
        assert rc == _lib.CDB_OK
        torch.cuda.synchronize()
        assert torch.equal(out_ws, out_na)
        assert torch.equal(with_ws[3], without[3])  # the appended K/V rows
        want = oracle_decode(case.q, case.k_new, case.v_new, case.kv_pool.copy(), case.cache_layer,
                             case.block_table, case.seqlens, case.block_size, case.scale, rope=case.rope,
                             rope_style=1, dtype="bf16")
        err = np.abs(out_na.float().cpu().numpy() - want)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3


def test_noalloc_rejects_batches_beyond_its_scratch() -> None:
    from continuous_depth_batching_amd import _lib

    lib = _lib.lib()
    case = make_case(seed=50, num_rows=4, num_heads=16, num_kv_heads=16, head_dim=128, max_context=64,
                     rope_style=1, dtype="bf16")
    tensors = _device(case)
    out = torch.empty_like(tensors[0])
    args = _args(case, tensors, out)
    heads, dim = 16, 128
    too_many = _lib.CDB_DECODE_SCRATCH_BYTES // (heads * (dim + 2) * 4) + 1
    args[21] = too_many  # num_rows: the check runs before any pointer is read
    assert lib.cdb_paged_decode_attention_noalloc(*args) == _lib.CDB_ERR_CAPACITY
