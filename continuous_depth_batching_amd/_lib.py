"""ctypes binding of ``libcdb_amd.so``, the C ABI declared in ``include/cdb_amd.h``.

Loading fails loudly: there is no CPU or PyTorch fallback for any kernel. The
library must have been built (``continuous_depth_batching_amd._build``) before
the first call.
"""

from __future__ import annotations

import ctypes
from ctypes import c_double, c_float, c_int32, c_int64, c_void_p
from functools import lru_cache

from ._build import LIBRARY_PATH

CDB_OK = 0
CDB_ERR_NULL, CDB_ERR_SHAPE, CDB_ERR_UNSUPPORTED, CDB_ERR_HIP, CDB_ERR_CAPACITY = -1, -2, -3, -4, -5
CDB_ERRORS = {
    -1: "a required pointer is null",
    -2: "an extent or stride is out of range",
    -3: "unsupported dtype/head_dim combination",
    -4: "a HIP kernel launch failed",
    -5: "a caller buffer is too small",
}
CDB_DTYPE_F32 = 0
CDB_DTYPE_BF16 = 1
CDB_DECODE_SCRATCH_BYTES = 16 << 20  # include/cdb_amd.h
CDB_DECODE_STAGE_PLAN = 1
CDB_DECODE_STAGE_ATTEND = 2

_P = c_void_p
_I32P = c_void_p

# name -> (restype, argtypes); mirrors include/cdb_amd.h one to one.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "cdb_paged_decode_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "cdb_paged_decode_attention": (
        c_int32,
        [
            _P, _P, _P, _P, _P,  # q, k_new, v_new, k_pool, v_pool
            c_int64, c_int32, c_int64,  # layer_stride, num_cache_layers, pool_blocks
            _I32P, c_int32,  # cache_layer, cache_layer0
            _I32P, _I32P, c_int32,  # block_table, table_row, table_width
            _I32P,  # seqlens
            _P, _P, c_int32, c_int32,  # rope_cos, rope_sin, rope_style, max_positions
            _P, _P,  # q_bias, k_bias
            _P, _P, c_int64,  # out, workspace, workspace_bytes
            c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,  # rows, H, Hkv, D, block_size, split_pages
            c_int32,  # min_split_pages (split_pages <= 0)
            c_float, c_int64, c_int64, c_int32, _P,  # scale, q_stride, kv_stride, dtype, stream
        ],
    ),
    "cdb_paged_decode_attention_staged": (
        c_int32,
        [
            _P, _P, _P, _P, _P,  # q, k_new, v_new, k_pool, v_pool
            c_int64, c_int32, c_int64,  # layer_stride, num_cache_layers, pool_blocks
            _I32P, c_int32,  # cache_layer, cache_layer0
            _I32P, _I32P, c_int32,  # block_table, table_row, table_width
            _I32P,  # seqlens
            _P, _P, c_int32, c_int32,  # rope_cos, rope_sin, rope_style, max_positions
            _P, _P,  # q_bias, k_bias
            _P, _P, c_int64,  # out, workspace, workspace_bytes
            c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,  # rows, H, Hkv, D, block_size, split_pages
            c_int32,  # min_split_pages (split_pages <= 0)
            c_float, c_int64, c_int64, c_int32, c_int32, _P,  # scale, q_stride, kv_stride, dtype, stages, stream
        ],
    ),
    "cdb_paged_decode_attention_noalloc": (
        c_int32,
        [
            _P, _P, _P, _P, _P,  # q, k_new, v_new, k_pool, v_pool
            c_int64, c_int32, c_int64,  # layer_stride, num_cache_layers, pool_blocks
            _I32P, c_int32,  # cache_layer, cache_layer0
            _I32P, _I32P, c_int32,  # block_table, table_row, table_width
            _I32P,  # seqlens
            _P, _P, c_int32, c_int32,  # rope_cos, rope_sin, rope_style, max_positions
            _P, _P,  # q_bias, k_bias
            _P,  # out
            c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,  # rows, H, Hkv, D, block_size, split_pages
            c_int32,  # min_split_pages (split_pages <= 0)
            c_float, c_int64, c_int64, c_int32, _P,  # scale, q_stride, kv_stride, dtype, stream
        ],
    ),
    "cdb_rmsnorm_fused": (
        c_int32, [_P, _P, _P, _P, _P, _P, c_int64, c_int32, c_int32, c_float, c_float, c_int32, _P]),
    "cdb_rmsnorm_fused_parts": (
        c_int32,
        [
            _P, c_int32, _P, _P, _P, _P, _P,  # x_parts, splits, residual, w_a, w_b, out_h, out_y
            c_int64, c_int32, c_int32, c_float, c_float, c_int32, _P,  # rows, width, mode, eps_a, eps_b, dtype, stream
        ],
    ),
    "cdb_silu_mul": (c_int32, [_P, _P, c_int64, c_int32, c_int32, _P]),
    "cdb_copy_rows": (c_int32, [_P, _P, c_int64, _P, _P, c_int64, c_int64, c_int64, _P]),
    "cdb_argmax": (c_int32, [_P, _P, c_int64, c_int32, c_int32, _P]),
    "cdb_route_compact": (c_int32, [_P, _P, c_int32, _P, _P]),
    "cdb_table_updates": (c_int32, [_P, c_int64, _P, _P, _P, c_int32, _P]),
    "cdb_exit_gate": (
        c_int32,
        [
            _P, _P, _P, _P, _P,  # hidden, prev, weight, bias, signal
            _P, _P, _P, c_int64, _P,  # cdf, survival, pending, state_capacity, state_index
            _P, _P, _P, c_int64,  # steps, synthetic_depth, exit_flags, rows
            c_int32, c_int32, c_int32, c_int32, c_int32,  # width, kind, rule, delayed, round_hazard
            c_int32, c_int32, c_double, c_int32, c_int32, _P,  # min/max steps, threshold, has_threshold, dtype, stream
        ],
    ),
    "cdb_exit_gate_reset": (c_int32, [_P, _P, _P, c_int64, _P, c_int64, _P]),
    "cdb_exit_kv_copy": (
        c_int32, [_P, _P, c_int64, c_int64, c_int32, c_int32, _P, _P, c_int64, c_int32, c_int32, c_int32, c_int32, _P]),
    "cdb_rope_kv_write": (
        c_int32,
        [
            _P, _P, _P, _P, _P, _P,  # q, k, v, q_out, k_pool, v_pool
            c_int64, c_int32, _P, c_int64,  # layer_stride, layer, rows, pool_rows
            _P, _P, _P, c_int32, c_int32,  # positions, rope_cos, rope_sin, rope_style, max_positions
            _P, _P, c_int64,  # q_bias, k_bias, tokens
            c_int32, c_int32, c_int32, c_int64, c_int64,  # H, Hkv, D, q_stride, kv_stride
            c_int32, _P,  # dtype, stream
        ],
    ),
    "cdb_prefill_attention": (
        c_int32,
        [
            _P, _P, _P, c_int64, c_int32, c_int32, c_int64,  # q, k_pool, v_pool, layer_stride, layer, layers, blocks
            _P, _P, c_int32, _P, _P, c_int32,  # block_table, table_row, width, cu_q, past, num_seqs
            _P, _P, c_int32, _P,  # tile_seq, tile_q0, num_tiles, out
            c_int32, c_int32, c_int32, c_int32, c_float, c_int32, _P,  # H, Hkv, D, block_size, scale, dtype, stream
        ],
    ),
    "cdb_prefill_partial_bytes": (c_int64, [c_int32, c_int32, c_int32]),
    "cdb_prefill_attention_split": (
        c_int32,
        [
            _P, _P, _P, c_int64, c_int32, c_int32, c_int64,  # q, k_pool, v_pool, layer_stride, layer, layers, blocks
            _P, _P, c_int32, _P, _P, c_int32,  # block_table, table_row, width, cu_q, past, num_seqs
            _P, c_int32, _P, c_int32, c_int32,  # items, num_items, merges, num_merges, num_slots
            _P, c_int64, _P,  # partials, partials_bytes, out
            c_int32, c_int32, c_int32, c_int32, c_float, c_int32, _P,  # H, Hkv, D, block_size, scale, dtype, stream
        ],
    ),
    "cdb_linear_pack_weight": (c_int32, [_P, c_int64, _P, c_int64, c_int32, c_int32, _P]),
    "cdb_linear": (
        c_int32,
        [
            _P, c_int64, _P, _P, c_int64,  # x, ldx, w_packed, y, ldy
            c_int32, c_int32, c_int32, c_int32, c_int32, _P,  # rows, out_features, in_features, gated, dtype, stream
        ],
    ),
    "cdb_linear_parts_splits": (c_int32, [c_int64, c_int32, c_int32, c_int32]),
    "cdb_linear_argmax_workspace_bytes": (c_int64, [c_int32, c_int32]),
    "cdb_linear_argmax": (
        c_int32,
        [
            _P, c_int64, _P, _P, _P, c_int64,  # x, ldx, w_packed, out, workspace, workspace_bytes
            c_int32, c_int32, c_int32,  # rows, out_features, in_features
            _P, _P, c_int64, _P, c_int32,  # embed, bank, bank_rows, bank_slots, width
            c_int32, _P,  # dtype, stream
        ],
    ),
    "cdb_linear_parts": (
        c_int32,
        [
            _P, c_int64, _P, _P, c_int64,  # x, ldx, w_packed, parts, parts_elems
            c_int32, c_int32, c_int32, c_int32, _P,  # rows, out_features, in_features, dtype, stream
        ],
    ),
    "cdb_coda_greedy": (
        c_int32,
        [
            _P, _P, c_int32, c_int32,  # host_upload, dev_upload, rows, num_successors
            _P, c_int64, c_int32, _P, _P, c_int32,  # bank, bank_rows, width, hidden, w_packed, vocab
            _P, _P, c_int64, _P, _P,  # tokens, workspace, workspace_bytes, embed, host_tokens
            _P, _P, _P, c_int64, c_int32, _P,  # cdf, survival, pending, state_capacity, dtype, stream
        ],
    ),
}


class CdbKernelError(RuntimeError):
    """A C-ABI entry point returned an error code."""


@lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    """Load the kernel library once; raise ImportError when it has not been built."""

    if not LIBRARY_PATH.exists():
        raise ImportError(
            f"{LIBRARY_PATH} is missing: build the HIP kernels first "
            "(python -m continuous_depth_batching_amd._build)"
        )
    handle = ctypes.CDLL(str(LIBRARY_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def check(code: int, what: str) -> None:
    if code != CDB_OK:
        raise CdbKernelError(f"{what} failed with code {code}: {CDB_ERRORS.get(code, 'unknown error')}")
