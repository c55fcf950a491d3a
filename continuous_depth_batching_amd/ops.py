"""PyTorch custom ops (``torch.ops.cdb.*``) over the C ABI in ``include/cdb_amd.h``.

Each op validates shapes and dtypes on the host, then calls one ``extern "C"``
entry point of ``libcdb_amd.so`` on torch's current HIP stream. The ops are
registered for the CUDA (HIP) device only: a CPU tensor raises, and a missing
library raises on first use. Nothing here allocates inside the kernels, so the
ops can be captured into HIP graphs.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib

_DTYPE_CODES = {torch.float32: _lib.CDB_DTYPE_F32, torch.bfloat16: _lib.CDB_DTYPE_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise TypeError(f"CDB kernels support float32 and bfloat16, got {dtype}") from exc


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _require_cuda(*tensors: torch.Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("CDB kernels run on the GPU only; got a tensor on " + str(t.device))


def _require_contiguous(**tensors: torch.Tensor | None) -> None:
    for name, t in tensors.items():
        if t is not None and not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")


def _require_int32(**tensors: torch.Tensor | None) -> None:
    for name, t in tensors.items():
        if t is not None and t.dtype != torch.int32:
            raise TypeError(f"{name} must be int32, got {t.dtype}")


@dataclass(frozen=True)
class KVPoolView:
    """Pointer view of a paged KV pool ``[num_cache_layers, 2, pool_blocks * block_size, Hkv, D]``."""

    pool: torch.Tensor
    block_size: int

    @property
    def num_cache_layers(self) -> int:
        return self.pool.shape[0]

    @property
    def pool_rows(self) -> int:
        return self.pool.shape[2]

    @property
    def pool_blocks(self) -> int:
        return self.pool_rows // self.block_size

    @property
    def layer_stride(self) -> int:
        return self.pool.stride(0)

    @property
    def k_ptr(self) -> int:
        return self.pool.data_ptr()

    @property
    def v_ptr(self) -> int:
        return self.pool.data_ptr() + self.pool.stride(1) * self.pool.element_size()


def decode_workspace_bytes(num_rows: int, num_heads: int, head_dim: int, max_seqlen: int, block_size: int,
                           split_pages: int) -> int:
    n = _lib.lib().cdb_paged_decode_workspace_bytes(num_rows, num_heads, head_dim, max_seqlen, block_size, split_pages)
    if n < 0:
        raise ValueError("invalid arguments for the decode workspace size")
    return int(n)


def paged_decode_attention_raw(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_pool_ptr: int,
    v_pool_ptr: int,
    layer_stride: int,
    num_cache_layers: int,
    pool_blocks: int,
    cache_layer: torch.Tensor | None,
    cache_layer0: int,
    block_table: torch.Tensor,
    table_row: torch.Tensor | None,
    seqlens: torch.Tensor,
    rope_cos: torch.Tensor | None,
    rope_sin: torch.Tensor | None,
    rope_style: int,
    q_bias: torch.Tensor | None,
    k_bias: torch.Tensor | None,
    out: torch.Tensor,
    workspace: torch.Tensor,
    block_size: int,
    split_pages: int,
    scale: float,
) -> torch.Tensor:
    """Launch ``cdb_paged_decode_attention`` on explicit pool pointers (no allocation)."""

    num_rows, num_heads, head_dim = q.shape
    num_kv_heads = k_new.shape[1]
    if k_new.shape != (num_rows, num_kv_heads, head_dim) or v_new.shape != k_new.shape:
        raise ValueError(f"k_new/v_new must be [{num_rows}, Hkv, {head_dim}]")
    if out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError("out must match q")
    if seqlens.shape != (num_rows,):
        raise ValueError("seqlens must have one entry per row")
    if block_table.dim() != 2:
        raise ValueError("block_table must be [rows, width]")
    if table_row is None and block_table.shape[0] < num_rows:
        raise ValueError("block_table needs a row per batch row when table_row is not given")
    if cache_layer is not None and cache_layer.shape != (num_rows,):
        raise ValueError("cache_layer must have one entry per row")
    for t in (k_new, v_new, q_bias, k_bias):
        if t is not None and t.dtype != q.dtype:
            raise TypeError("q, k_new, v_new and the biases must share a dtype")
    if rope_style:
        if rope_cos is None or rope_sin is None or rope_cos.dtype != torch.float32 or rope_cos.shape != rope_sin.shape:
            raise ValueError("rope tables must be float32 [max_positions, D/2]")
        if rope_cos.shape[1] != head_dim // 2:
            raise ValueError("rope tables must have D/2 columns")
    if workspace.dtype != torch.float32:
        raise TypeError("workspace must be float32")
    _require_cuda(q, k_new, v_new, cache_layer, block_table, table_row, seqlens, rope_cos, rope_sin, out, workspace)
    _require_contiguous(q=q, k_new=k_new, v_new=v_new, block_table=block_table, seqlens=seqlens, out=out,
                        rope_cos=rope_cos, rope_sin=rope_sin, q_bias=q_bias, k_bias=k_bias)
    _require_int32(cache_layer=cache_layer, block_table=block_table, table_row=table_row, seqlens=seqlens)
    code = _lib.lib().cdb_paged_decode_attention(
        q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_pool_ptr, v_pool_ptr,
        layer_stride, num_cache_layers, pool_blocks,
        _ptr(cache_layer), cache_layer0,
        block_table.data_ptr(), _ptr(table_row), block_table.shape[1],
        seqlens.data_ptr(),
        _ptr(rope_cos), _ptr(rope_sin), rope_style, 0 if rope_cos is None else rope_cos.shape[0],
        _ptr(q_bias), _ptr(k_bias),
        out.data_ptr(), workspace.data_ptr(), workspace.numel() * 4,
        num_rows, num_heads, num_kv_heads, head_dim, block_size, split_pages,
        scale, dtype_code(q.dtype), _stream(),
    )
    _lib.check(code, "cdb_paged_decode_attention")
    return out


@torch.library.custom_op("cdb::paged_decode_attention", mutates_args=("kv_pool", "workspace"), device_types="cuda")
def paged_decode_attention(
    q: torch.Tensor,
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    kv_pool: torch.Tensor,
    cache_layer: torch.Tensor | None,
    cache_layer0: int,
    block_table: torch.Tensor,
    table_row: torch.Tensor | None,
    seqlens: torch.Tensor,
    rope_cos: torch.Tensor | None,
    rope_sin: torch.Tensor | None,
    rope_style: int,
    q_bias: torch.Tensor | None,
    k_bias: torch.Tensor | None,
    workspace: torch.Tensor,
    block_size: int,
    split_pages: int,
    scale: float,
) -> torch.Tensor:
    """Mixed-depth paged decode attention with fused RoPE + KV append over ``kv_pool``.

    ``kv_pool`` is ``[num_cache_layers, 2, pool_blocks * block_size, Hkv, D]`` (keys at
    index 0 of dim 1, values at 1) and is updated in place at each row's position.
    """

    if kv_pool.dim() != 5 or kv_pool.shape[1] != 2 or not kv_pool.is_contiguous():
        raise ValueError("kv_pool must be a contiguous [layers, 2, rows, Hkv, D] tensor")
    if kv_pool.dtype != q.dtype:
        raise TypeError("kv_pool dtype must match q")
    view = KVPoolView(kv_pool, block_size)
    out = torch.empty_like(q)
    return paged_decode_attention_raw(
        q, k_new, v_new, view.k_ptr, view.v_ptr, view.layer_stride, view.num_cache_layers, view.pool_blocks,
        cache_layer, cache_layer0, block_table, table_row, seqlens, rope_cos, rope_sin, rope_style,
        q_bias, k_bias, out, workspace, block_size, split_pages, scale,
    )


@paged_decode_attention.register_fake
def _(q, k_new, v_new, kv_pool, cache_layer, cache_layer0, block_table, table_row, seqlens, rope_cos, rope_sin,
      rope_style, q_bias, k_bias, workspace, block_size, split_pages, scale):
    return torch.empty_like(q)


def default_split_pages(num_rows: int, block_size: int) -> int:
    """Pages per split: smaller splits for narrow batches so the grid stays full."""

    tokens = 256 if num_rows >= 512 else 128 if num_rows >= 64 else 64
    return max(1, tokens // block_size)


def softmax_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
