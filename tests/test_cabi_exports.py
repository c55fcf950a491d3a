"""The C-ABI library loads and exports every function include/*.h declares."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from continuous_depth_batching_amd import _lib

INCLUDE = Path(__file__).resolve().parent.parent / "include"
DECL = re.compile(r"^\s*(?:int|int64_t|int32_t|void|const char\s*\*)\s+(cdb_\w+)\s*\(", re.M)


def declared_functions() -> set[str]:
    names: set[str] = set()
    for header in INCLUDE.glob("*.h"):
        names.update(DECL.findall(header.read_text()))
    return names


def test_header_declares_entry_points() -> None:
    assert "cdb_paged_decode_attention" in declared_functions()


def test_library_exports_every_declared_symbol() -> None:
    handle = ctypes.CDLL(str(_lib.LIBRARY_PATH))
    missing = [name for name in sorted(declared_functions()) if not hasattr(handle, name)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_every_declared_symbol() -> None:
    assert declared_functions() == set(_lib.SIGNATURES)
    lib = _lib.lib()
    for name in _lib.SIGNATURES:
        assert getattr(lib, name).argtypes is not None


def test_workspace_size_query_without_gpu() -> None:
    lib = _lib.lib()
    # A header (chunk size + chunk prefix of the rows, padded to 256 bytes, then 1 KiB of item-queue
    # counters, then one arrival counter per row and head, padded to 256 bytes), then
    # ceil(100 / 32) + 1 chunks per row, each a 64-byte descriptor and (D + 2) floats per head.
    per_chunk = 64 + 16 * 130 * 4
    assert lib.cdb_paged_decode_workspace_bytes(4, 16, 128, 100, 16, 2) == 256 + 1024 + 256 + 4 * 5 * per_chunk
    assert lib.cdb_paged_decode_workspace_bytes(100, 16, 128, 100, 16, 2) == \
        512 + 1024 + 6400 + 100 * 5 * per_chunk
    assert lib.cdb_paged_decode_workspace_bytes(-1, 16, 128, 100, 16, 2) == -1


def _decode_args(**over):
    # Non-null stand-in addresses: every case below is rejected on the host before any
    # device work, so the kernel never sees them.
    fake = ctypes.c_void_p(0x1000)
    args = dict(q=fake, k_new=fake, v_new=fake, k_pool=fake, v_pool=fake, layer_stride=1 << 20,
                num_cache_layers=4, pool_blocks=64, cache_layer=None, cache_layer0=0, block_table=fake,
                table_row=None, table_width=8, seqlens=fake, rope_cos=fake, rope_sin=fake, rope_style=1,
                max_positions=128, q_bias=None, k_bias=None, out=fake, workspace=fake, workspace_bytes=1 << 20,
                num_rows=4, num_heads=16, num_kv_heads=16, head_dim=128, block_size=16, split_pages=0,
                min_split_pages=2, scale=0.088, q_stride=0, kv_stride=0, dtype=1, stream=None)
    args.update(over)
    return list(args.values())


def test_decode_argument_errors_without_gpu() -> None:
    import torch

    if torch.cuda.is_available():
        pytest.skip("runs only where no device exists: the stand-in addresses must never reach a kernel")
    lib = _lib.lib()
    call = lambda **kw: lib.cdb_paged_decode_attention(*_decode_args(**kw))
    assert call(num_rows=0) == _lib.CDB_OK
    assert call(q=None) == _lib.CDB_ERR_NULL
    assert call(workspace=None) == _lib.CDB_ERR_NULL
    assert call(workspace_bytes=255) == _lib.CDB_ERR_CAPACITY  # smaller than the chunk header
    per_chunk = 64 + 16 * 130 * 4
    assert call(workspace_bytes=1536 + 3 * per_chunk) == _lib.CDB_ERR_CAPACITY  # 3 chunks for 4 rows
    assert call(block_size=24) == _lib.CDB_ERR_SHAPE
    assert call(num_kv_heads=5) == _lib.CDB_ERR_SHAPE
    assert call(min_split_pages=0) == _lib.CDB_ERR_SHAPE
    assert call(head_dim=80) == _lib.CDB_ERR_UNSUPPORTED
    assert call(dtype=7) == _lib.CDB_ERR_UNSUPPORTED
    assert call(rope_cos=None) == _lib.CDB_ERR_NULL
    assert call(q_stride=100) == _lib.CDB_ERR_SHAPE


def test_staged_decode_argument_errors_without_gpu() -> None:
    import torch

    if torch.cuda.is_available():
        pytest.skip("runs only where no device exists: the stand-in addresses must never reach a kernel")
    lib = _lib.lib()

    def call(stages, **kw):
        args = _decode_args(**kw)
        return lib.cdb_paged_decode_attention_staged(*args[:-1], stages, args[-1])

    assert call(_lib.CDB_DECODE_STAGE_PLAN, num_rows=0) == _lib.CDB_OK
    for bad in (0, 4, -1, 7):
        assert call(bad) == _lib.CDB_ERR_SHAPE
    assert call(_lib.CDB_DECODE_STAGE_ATTEND, q=None) == _lib.CDB_ERR_NULL
    assert call(_lib.CDB_DECODE_STAGE_PLAN, workspace_bytes=255) == _lib.CDB_ERR_CAPACITY


def test_table_update_argument_errors_without_gpu() -> None:
    import torch

    if torch.cuda.is_available():
        pytest.skip("runs only where no device exists: the stand-in addresses must never reach a kernel")
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x1000)
    assert lib.cdb_table_updates(fake, 64, fake, fake, fake, 0, None) == _lib.CDB_OK   # no slots: nothing to do
    assert lib.cdb_table_updates(None, 64, fake, fake, fake, 8, None) == _lib.CDB_ERR_NULL
    assert lib.cdb_table_updates(fake, 64, fake, fake, None, 8, None) == _lib.CDB_ERR_NULL
    assert lib.cdb_table_updates(fake, 0, fake, fake, fake, 8, None) == _lib.CDB_ERR_SHAPE
    assert lib.cdb_table_updates(fake, 64, fake, fake, fake, -1, None) == _lib.CDB_ERR_SHAPE


def test_linear_argument_errors_without_gpu() -> None:
    import torch

    if torch.cuda.is_available():
        pytest.skip("runs only where no device exists: the stand-in addresses must never reach a kernel")
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x1000)

    def call(**over):
        args = dict(x=fake, ldx=2048, w=fake, y=fake, ldy=2048, rows=8, out_features=2048, in_features=2048, gated=0,
                    dtype=_lib.CDB_DTYPE_BF16, stream=None)
        args.update(over)
        return lib.cdb_linear(*args.values())

    assert call(x=None) == _lib.CDB_ERR_NULL
    assert call(dtype=_lib.CDB_DTYPE_F32) == _lib.CDB_ERR_UNSUPPORTED
    assert call(rows=0) == _lib.CDB_ERR_SHAPE
    assert call(rows=65) == _lib.CDB_ERR_SHAPE                      # 2048 -> 2048 has no wide-tile path
    assert call(rows=257, out_features=6144, ldy=6144) == _lib.CDB_ERR_SHAPE
    assert call(rows=100, in_features=4096, ldx=4096) == _lib.CDB_ERR_SHAPE
    assert call(out_features=2040) == _lib.CDB_ERR_SHAPE
    assert call(in_features=2000, ldx=2000) == _lib.CDB_ERR_SHAPE
    assert call(ldx=2044) == _lib.CDB_ERR_SHAPE
    assert call(ldy=2046) == _lib.CDB_ERR_SHAPE
    assert call(w=ctypes.c_void_p(0x1008)) == _lib.CDB_ERR_SHAPE

    def pack(**over):
        args = dict(w=fake, ldw=2048, out=fake, rows=2048, in_features=2048, dtype=_lib.CDB_DTYPE_BF16, stream=None)
        args.update(over)
        return lib.cdb_linear_pack_weight(*args.values())

    assert pack(out=None) == _lib.CDB_ERR_NULL
    assert pack(rows=2040) == _lib.CDB_ERR_SHAPE
    assert pack(ldw=2000) == _lib.CDB_ERR_SHAPE
    assert pack(dtype=_lib.CDB_DTYPE_F32) == _lib.CDB_ERR_UNSUPPORTED

    bf16 = _lib.CDB_DTYPE_BF16
    assert lib.cdb_linear_parts_splits(16, 2048, 2048, bf16) == 4
    assert lib.cdb_linear_parts_splits(65, 2048, 2048, bf16) == 2
    assert lib.cdb_linear_parts_splits(129, 2048, 2048, bf16) == 0
    assert lib.cdb_linear_parts_splits(256, 2048, 5632, bf16) == 4
    assert lib.cdb_linear_parts_splits(257, 2048, 5632, bf16) == 0
    assert lib.cdb_linear_parts_splits(16, 2048, 4096, bf16) == 0
    assert lib.cdb_linear_parts_splits(16, 2000, 2048, bf16) == 0
    assert lib.cdb_linear_parts_splits(16, 2048, 2048, _lib.CDB_DTYPE_F32) == 0

    def parts(**over):
        args = dict(x=fake, ldx=2048, w=fake, parts=fake, parts_elems=4 * 16 * 2048, rows=16, out_features=2048,
                    in_features=2048, dtype=bf16, stream=None)
        args.update(over)
        return lib.cdb_linear_parts(*args.values())

    assert parts(parts=None) == _lib.CDB_ERR_NULL
    assert parts(dtype=_lib.CDB_DTYPE_F32) == _lib.CDB_ERR_UNSUPPORTED
    assert parts(rows=0) == _lib.CDB_ERR_SHAPE
    assert parts(rows=129, parts_elems=1 << 30) == _lib.CDB_ERR_SHAPE
    assert parts(in_features=4096, ldx=4096) == _lib.CDB_ERR_SHAPE
    assert parts(parts_elems=4 * 16 * 2048 - 1) == _lib.CDB_ERR_SHAPE
    assert parts(ldx=2044) == _lib.CDB_ERR_SHAPE
    assert parts(parts=ctypes.c_void_p(0x1004)) == _lib.CDB_ERR_SHAPE

    def norm(**over):
        args = dict(parts=fake, splits=4, residual=fake, w_a=fake, w_b=fake, h=fake, y=fake, rows=16, width=2048,
                    mode=1, eps_a=1e-6, eps_b=1e-6, dtype=bf16, stream=None)
        args.update(over)
        return lib.cdb_rmsnorm_fused_parts(*args.values())

    assert norm(parts=None) == _lib.CDB_ERR_NULL
    assert norm(residual=None) == _lib.CDB_ERR_NULL
    assert norm(y=None) == _lib.CDB_ERR_NULL
    assert norm(splits=0) == _lib.CDB_ERR_SHAPE
    assert norm(splits=65) == _lib.CDB_ERR_SHAPE
    assert norm(width=2044) == _lib.CDB_ERR_SHAPE
    assert norm(parts=ctypes.c_void_p(0x1008)) == _lib.CDB_ERR_SHAPE
    assert norm(dtype=_lib.CDB_DTYPE_F32) == _lib.CDB_ERR_UNSUPPORTED
    assert norm(rows=0) == _lib.CDB_OK

    assert lib.cdb_linear_argmax_workspace_bytes(16, 49152) == 16 * 3072 * 8
    assert lib.cdb_linear_argmax_workspace_bytes(16, 49150) == -1

    def am(**over):
        args = dict(x=fake, ldx=2048, w=fake, out=fake, ws=fake, ws_bytes=16 * 3072 * 8, rows=16, out_features=49152,
                    in_features=2048, embed=None, bank=None, bank_rows=0, bank_slots=None, width=0, dtype=bf16,
                    stream=None)
        args.update(over)
        return lib.cdb_linear_argmax(*args.values())

    assert am(out=None) == _lib.CDB_ERR_NULL
    assert am(ws=None) == _lib.CDB_ERR_NULL
    assert am(dtype=_lib.CDB_DTYPE_F32) == _lib.CDB_ERR_UNSUPPORTED
    assert am(rows=0) == _lib.CDB_ERR_SHAPE
    assert am(rows=65) == _lib.CDB_ERR_SHAPE
    assert am(out_features=49150) == _lib.CDB_ERR_SHAPE
    assert am(ldx=2044) == _lib.CDB_ERR_SHAPE
    assert am(ws=ctypes.c_void_p(0x1008)) == _lib.CDB_ERR_SHAPE
    assert am(ws_bytes=16 * 3072 * 8 - 1) == _lib.CDB_ERR_CAPACITY
    assert am(embed=fake) == _lib.CDB_ERR_NULL                       # the fused prelude needs bank and slots
    assert am(embed=fake, bank=fake, bank_slots=fake, bank_rows=512, width=2044) == _lib.CDB_ERR_SHAPE
    assert am(embed=fake, bank=fake, bank_slots=fake, bank_rows=0, width=2048) == _lib.CDB_ERR_SHAPE


def test_split_k_table_without_gpu() -> None:
    """cdb_linear_parts_splits is host arithmetic: the split forms of the Ouro O/down
    (2048 and 5632 inputs) and Huginn O/down (5280 and 17920 inputs) projections."""

    lib = _lib.lib()
    bf16 = _lib.CDB_DTYPE_BF16
    cases = {
        (16, 2048, 2048): 4, (64, 2048, 2048): 4, (128, 2048, 2048): 2, (129, 2048, 2048): 0,
        (1, 2048, 5632): 8, (16, 2048, 5632): 8, (17, 2048, 5632): 4, (256, 2048, 5632): 4, (257, 2048, 5632): 0,
        (16, 5280, 5280): 3, (128, 5280, 5280): 3, (256, 5280, 5280): 3,
        (16, 5280, 17920): 8, (64, 5280, 17920): 8, (65, 5280, 17920): 4, (128, 5280, 17920): 4,
        (64, 2040, 2048): 0,   # out_features not a multiple of 16
        (64, 5280, 4096): 0,   # no split form for this input width
        (0, 2048, 2048): 0,
    }
    got = {key: lib.cdb_linear_parts_splits(*key, bf16) for key in cases}
    assert got == cases
    assert lib.cdb_linear_parts_splits(16, 2048, 2048, _lib.CDB_DTYPE_F32) == 0
