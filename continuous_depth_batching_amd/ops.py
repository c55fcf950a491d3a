"""PyTorch custom ops (``torch.ops.cdb.*``) over the C ABI in ``include/cdb_amd.h``.

Each op validates shapes and dtypes on the host, then calls one ``extern "C"``
entry point of ``libcdb_amd.so`` on torch's current HIP stream. The ops are
registered for the CUDA (HIP) device only: a CPU tensor raises, and a missing
library raises on first use. Nothing here allocates inside the kernels, so the
ops can be captured into HIP graphs.
"""

from __future__ import annotations

import functools
import math
from dataclasses import dataclass

import torch

from . import _lib

_DTYPE_CODES = {torch.float32: _lib.CDB_DTYPE_F32, torch.bfloat16: _lib.CDB_DTYPE_BF16}

# Decode-attention KV chunk length in pages: ADAPTIVE_SPLIT uses MIN_SPLIT_PAGES (a
# negative value -m uses m). Chunks are lengthened only when the workspace cannot
# hold a launch's chunks.
ADAPTIVE_SPLIT = 0
MIN_SPLIT_PAGES = 8

# Stages of cdb_paged_decode_attention_staged (include/cdb_amd.h).
DECODE_PLAN = _lib.CDB_DECODE_STAGE_PLAN
DECODE_ATTEND = _lib.CDB_DECODE_STAGE_ATTEND
DECODE_PLAN_AND_ATTEND = DECODE_PLAN | DECODE_ATTEND


def decode_split_pages(rows: int) -> int:
    """The split_pages argument a decode launch of `rows` rows passes.

    Always the default chunk length: a row's chunks, and so its rounding, then do
    not depend on the size of the launch it lands in, and rows compute
    identically in any batch composition."""

    return ADAPTIVE_SPLIT


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise TypeError(f"CDB kernels support float32 and bfloat16, got {dtype}") from exc


if hasattr(torch._C, "_cuda_getCurrentRawStream") and hasattr(torch._C, "_cuda_getDevice"):
    def _stream() -> int:
        # The raw handle of torch's current stream without building a Stream object
        # (that costs ~10 us per call on the per-tick host path).
        return torch._C._cuda_getCurrentRawStream(torch._C._cuda_getDevice())
else:  # pragma: no cover - older torch builds
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
    min_split_pages: int = MIN_SPLIT_PAGES,
    stages: int = DECODE_PLAN_AND_ATTEND,
) -> torch.Tensor:
    """Launch ``cdb_paged_decode_attention`` on explicit pool pointers (no allocation).

    ``split_pages <= 0`` uses chunks of ``min_split_pages`` pages. ``stages`` other
    than plan-and-attend goes through ``cdb_paged_decode_attention_staged``: a
    caller that runs the same rows (positions, table rows, cache-layer offsets)
    through several layers plans at the first and attends at every layer.
    """

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
    for name, t in (("q", q), ("k_new", k_new), ("v_new", v_new)):
        if t.stride(2) != 1 or t.stride(1) != head_dim:
            raise ValueError(f"{name} must have contiguous heads and head dimension (row stride may differ)")
    if k_new.stride(0) != v_new.stride(0):
        raise ValueError("k_new and v_new must share a row stride")
    _require_contiguous(block_table=block_table, seqlens=seqlens, out=out, rope_cos=rope_cos, rope_sin=rope_sin,
                        q_bias=q_bias, k_bias=k_bias)
    _require_int32(cache_layer=cache_layer, block_table=block_table, table_row=table_row, seqlens=seqlens)
    head = (q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_pool_ptr, v_pool_ptr,
            layer_stride, num_cache_layers, pool_blocks,
            _ptr(cache_layer), cache_layer0,
            block_table.data_ptr(), _ptr(table_row), block_table.shape[1],
            seqlens.data_ptr(),
            _ptr(rope_cos), _ptr(rope_sin), rope_style, 0 if rope_cos is None else rope_cos.shape[0],
            _ptr(q_bias), _ptr(k_bias),
            out.data_ptr(), workspace.data_ptr(), workspace.numel() * 4,
            num_rows, num_heads, num_kv_heads, head_dim, block_size, split_pages, min_split_pages)
    tail = (scale, q.stride(0), k_new.stride(0), dtype_code(q.dtype))
    if stages == DECODE_PLAN_AND_ATTEND:
        code = _lib.lib().cdb_paged_decode_attention(*head, *tail, _stream())
        _lib.check(code, "cdb_paged_decode_attention")
    else:
        code = _lib.lib().cdb_paged_decode_attention_staged(*head, *tail, stages, _stream())
        _lib.check(code, "cdb_paged_decode_attention_staged")
    return out


@torch.library.custom_op("cdb::paged_decode_attention", mutates_args=("kv_pool", "workspace"),
                        device_types="cuda")
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
    stages: int = DECODE_PLAN_AND_ATTEND,
) -> torch.Tensor:
    """Mixed-depth paged decode attention with fused RoPE + KV append over ``kv_pool``.

    ``kv_pool`` is ``[num_cache_layers, 2, pool_blocks * block_size, Hkv, D]`` (keys at
    index 0 of dim 1, values at 1) and is updated in place at each row's position.
    ``stages`` as in ``paged_decode_attention_raw``.
    """

    if kv_pool.dim() != 5 or kv_pool.shape[1] != 2 or not kv_pool.is_contiguous():
        raise ValueError("kv_pool must be a contiguous [layers, 2, rows, Hkv, D] tensor")
    if kv_pool.dtype != q.dtype:
        raise TypeError("kv_pool dtype must match q")
    view = KVPoolView(kv_pool, block_size)
    out = torch.empty_like(q)
    min_split = -split_pages if split_pages < 0 else MIN_SPLIT_PAGES
    return paged_decode_attention_raw(
        q, k_new, v_new, view.k_ptr, view.v_ptr, view.layer_stride, view.num_cache_layers, view.pool_blocks,
        cache_layer, cache_layer0, block_table, table_row, seqlens, rope_cos, rope_sin, rope_style,
        q_bias, k_bias, out, workspace, block_size, max(split_pages, 0), scale, min_split_pages=min_split,
        stages=stages,
    )


@paged_decode_attention.register_fake
def _(q, k_new, v_new, kv_pool, cache_layer, cache_layer0, block_table, table_row, seqlens, rope_cos, rope_sin,
      rope_style, q_bias, k_bias, workspace, block_size, split_pages, scale, stages=DECODE_PLAN_AND_ATTEND):
    return torch.empty_like(q)


def softmax_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


# ---------------------------------------------------------------------------
# Row-wise stage kernels.
# ---------------------------------------------------------------------------

NORM_PLAIN, NORM_OURO_SANDWICH, NORM_HUGINN_SANDWICH = 0, 1, 2


def rmsnorm_fused_raw(x: torch.Tensor, residual: torch.Tensor | None, w_a: torch.Tensor, w_b: torch.Tensor | None,
                      out_h: torch.Tensor, out_y: torch.Tensor | None, mode: int, eps_a: float, eps_b: float) -> None:
    """Launch ``cdb_rmsnorm_fused`` on 2-D contiguous row tensors (no allocation)."""

    rows, width = x.shape[0], x.shape[-1]
    for name, t in (("residual", residual), ("out_h", out_h), ("out_y", out_y)):
        if t is not None and (t.shape != x.shape or t.dtype != x.dtype):
            raise ValueError(f"{name} must match x")
    for name, w in (("w_a", w_a), ("w_b", w_b)):
        if w is not None and (w.shape != (width,) or w.dtype != x.dtype):
            raise ValueError(f"{name} must be a [{width}] vector of x's dtype")
    _require_cuda(x, residual, w_a, w_b, out_h, out_y)
    _require_contiguous(x=x, residual=residual, w_a=w_a, w_b=w_b, out_h=out_h, out_y=out_y)
    code = _lib.lib().cdb_rmsnorm_fused(
        x.data_ptr(), _ptr(residual), w_a.data_ptr(), _ptr(w_b), out_h.data_ptr(), _ptr(out_y),
        rows, width, mode, eps_a, eps_b, dtype_code(x.dtype), _stream())
    _lib.check(code, "cdb_rmsnorm_fused")


@torch.library.custom_op("cdb::rmsnorm", mutates_args=(), device_types="cuda")
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm as OuroRMSNorm / HuginnRMSNorm computes it, over the last dimension."""

    x2 = x.reshape(-1, x.shape[-1])
    out = torch.empty_like(x2)
    rmsnorm_fused_raw(x2, None, weight, None, out, None, NORM_PLAIN, eps, eps)
    return out.view_as(x)


@rmsnorm.register_fake
def _(x, weight, eps):
    return torch.empty_like(x)


@torch.library.custom_op("cdb::residual_rmsnorm", mutates_args=(), device_types="cuda")
def residual_rmsnorm(x: torch.Tensor, residual: torch.Tensor, w_a: torch.Tensor, w_b: torch.Tensor, eps_a: float,
                     eps_b: float, mode: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Sandwich-norm residual step: returns (h, norm_b(h)); see ``cdb_rmsnorm_fused`` for ``mode``."""

    x2 = x.reshape(-1, x.shape[-1])
    r2 = residual.reshape(-1, x.shape[-1])
    h = torch.empty_like(x2)
    y = torch.empty_like(x2)
    rmsnorm_fused_raw(x2, r2, w_a, w_b, h, y, mode, eps_a, eps_b)
    return h.view_as(x), y.view_as(x)


@residual_rmsnorm.register_fake
def _(x, residual, w_a, w_b, eps_a, eps_b, mode):
    return torch.empty_like(x), torch.empty_like(x)


def silu_mul_raw(gate_up: torch.Tensor, out: torch.Tensor) -> None:
    rows, width = out.shape[0], out.shape[-1]
    if gate_up.shape != (rows, 2 * width) or gate_up.dtype != out.dtype:
        raise ValueError("gate_up must be [rows, 2 * width] of out's dtype")
    _require_cuda(gate_up, out)
    _require_contiguous(gate_up=gate_up, out=out)
    _lib.check(_lib.lib().cdb_silu_mul(gate_up.data_ptr(), out.data_ptr(), rows, width, dtype_code(out.dtype),
                                       _stream()), "cdb_silu_mul")


@torch.library.custom_op("cdb::silu_mul", mutates_args=(), device_types="cuda")
def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for gate_up = [gate | up] along the last dimension."""

    g2 = gate_up.reshape(-1, gate_up.shape[-1])
    out = torch.empty((g2.shape[0], g2.shape[1] // 2), dtype=gate_up.dtype, device=gate_up.device)
    silu_mul_raw(g2, out)
    return out.view(*gate_up.shape[:-1], gate_up.shape[-1] // 2)


@silu_mul.register_fake
def _(gate_up):
    return gate_up.new_empty((*gate_up.shape[:-1], gate_up.shape[-1] // 2))


# Rows up to which a projection runs on cdb_linear; larger batches use torch.mm (hipBLASLt).
LINEAR_MAX_ROWS = 64


def linear_packable(weight: torch.Tensor) -> bool:
    return (weight.dtype == torch.bfloat16 and weight.dim() == 2 and weight.shape[0] % 16 == 0
            and weight.shape[1] % 32 == 0)


def pack_linear_weight(weight: torch.Tensor) -> torch.Tensor:
    """The operand-ordered copy of a [rows, in_features] bf16 weight that cdb_linear reads."""

    _require_cuda(weight)
    if not linear_packable(weight):
        raise ValueError(f"cannot pack a {weight.dtype} weight of shape {tuple(weight.shape)} "
                         "(bfloat16, rows a multiple of 16, in_features a multiple of 32)")
    if weight.stride(1) != 1:
        weight = weight.contiguous()
    packed = torch.empty(weight.numel(), dtype=weight.dtype, device=weight.device)
    _lib.check(_lib.lib().cdb_linear_pack_weight(weight.data_ptr(), weight.stride(0), packed.data_ptr(),
                                                 weight.shape[0], weight.shape[1], _lib.CDB_DTYPE_BF16, _stream()),
               "cdb_linear_pack_weight")
    return packed


def maybe_pack_linear_weight(weight: torch.Tensor) -> torch.Tensor | None:
    """pack_linear_weight for a bf16 device weight cdb_linear can take, else None (torch.mm serves it)."""

    if weight.device.type != "cuda" or not linear_packable(weight):
        return None
    return pack_linear_weight(weight)


def linear_raw(x: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, *, gated: bool = False) -> None:
    """out = x @ W.T on the decode-batch projection kernel, W given packed (gated: silu(gate) * up)."""

    _require_cuda(x, packed, out)
    rows, in_features = x.shape
    out_features = out.shape[1]
    if x.dtype != torch.bfloat16 or packed.dtype != x.dtype or out.dtype != x.dtype:
        raise TypeError("cdb_linear takes bfloat16 x, weight and out")
    if packed.numel() != (2 if gated else 1) * out_features * in_features or out.shape[0] != rows:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, packed weight of {packed.numel()} elements, "
                         f"out {tuple(out.shape)}")
    if x.stride(1) != 1 or out.stride(1) != 1 or not packed.is_contiguous():
        raise ValueError("x and out must have unit stride along their last dimension; the packed weight is dense")
    _lib.check(_lib.lib().cdb_linear(x.data_ptr(), x.stride(0), packed.data_ptr(), out.data_ptr(), out.stride(0),
                                     rows, out_features, in_features, int(gated), _lib.CDB_DTYPE_BF16, _stream()),
               "cdb_linear")


# Batches up to this many rows run the wide-tile kernel when the shape qualifies.
LINEAR_WIDE_MAX_ROWS = 256


def linear_prefers_kernel(rows: int, out_features: int, gated: bool, in_features: int = 0) -> bool:
    """Whether cdb_linear beats torch.mm for this batch (measured on cold weights): always
    up to 32 rows; up to 64 for the gated MLP projection (its fused SiLU saves a pass) and
    for outputs of 4096 to 16384 columns; and up to 256 rows on the wide-tile kernel for
    2048-wide inputs with such outputs (a multiple of 128 columns), and up to 128 rows for
    5280-wide inputs with such outputs or a gated one. The LM heads (49152 and 65536
    columns) above 32 rows are faster on hipBLASLt, as are O and down projections."""

    if 1 <= rows <= 32:
        return True
    mid = 4096 <= out_features <= 16384
    if rows <= LINEAR_MAX_ROWS and (gated or mid):
        return True
    if in_features == 5280:  # Huginn QKV and gate/up on the wide-tile kernel up to 128 rows
        return rows <= 128 and (gated or mid)
    return rows <= LINEAR_WIDE_MAX_ROWS and mid and out_features % 128 == 0 and in_features == 2048


def _linear_fits(x: torch.Tensor, out_features: int, gated: bool) -> bool:
    return (x.dtype == torch.bfloat16 and linear_prefers_kernel(x.shape[0], out_features, gated, x.shape[1])
            and x.shape[1] % 32 == 0 and out_features % 16 == 0 and x.stride(1) == 1 and x.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0)


def linear_auto(x: torch.Tensor, weight: torch.Tensor, packed: torch.Tensor | None, gated: bool) -> torch.Tensor:
    """The body of cdb::linear, callable without op dispatch (eager per-tick paths)."""

    out_features = weight.shape[0] // 2 if gated else weight.shape[0]
    if packed is not None and _linear_fits(x, out_features, gated):
        out = x.new_empty((x.shape[0], out_features))
        linear_raw(x, packed, out, gated=gated)
        return out
    y = torch.mm(x, weight.t())
    if not gated:
        return y
    out = x.new_empty((x.shape[0], out_features))
    silu_mul_raw(y, out)
    return out


@torch.library.custom_op("cdb::linear", mutates_args=(), device_types="cuda")
def linear(x: torch.Tensor, weight: torch.Tensor, packed: torch.Tensor | None, gated: bool) -> torch.Tensor:
    """x @ weight.T for a decode batch; gated: silu(x @ gate.T) * (x @ up.T) with weight = [gate; up].

    bf16 batches that linear_prefers_kernel picks run on cdb_linear over `packed`
    (pack_linear_weight(weight)); others, or a missing packed copy, on torch.mm
    (followed by cdb_silu_mul when gated)."""

    return linear_auto(x, weight, packed, gated)


@linear.register_fake
def _(x, weight, packed, gated):
    return x.new_empty((x.shape[0], weight.shape[0] // 2 if gated else weight.shape[0]))


@functools.lru_cache(maxsize=4096)
def linear_parts_splits(rows: int, out_features: int, in_features: int) -> int:
    """K ranges of cdb_linear_parts for a bf16 projection of this shape; 0 when it has no split form."""

    return int(_lib.lib().cdb_linear_parts_splits(rows, out_features, in_features, _lib.CDB_DTYPE_BF16))


def linear_parts_raw(x: torch.Tensor, packed: torch.Tensor, parts: torch.Tensor) -> None:
    """parts[s] = fp32 partial x @ W.T over the s-th K range (split-K projection, no allocation)."""

    _require_cuda(x, packed, parts)
    rows, in_features = x.shape
    splits, p_rows, out_features = parts.shape
    if x.dtype != torch.bfloat16 or packed.dtype != x.dtype or parts.dtype != torch.float32:
        raise TypeError("cdb_linear_parts takes bfloat16 x and weight and float32 parts")
    if packed.numel() != out_features * in_features or p_rows != rows:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, packed weight of {packed.numel()} elements, "
                         f"parts {tuple(parts.shape)}")
    if splits != linear_parts_splits(rows, out_features, in_features):
        raise ValueError(f"parts must hold linear_parts_splits(...) = "
                         f"{linear_parts_splits(rows, out_features, in_features)} ranges, not {splits}")
    if x.stride(1) != 1 or not parts.is_contiguous() or not packed.is_contiguous():
        raise ValueError("x must have unit stride along its last dimension; parts and the packed weight are dense")
    _lib.check(_lib.lib().cdb_linear_parts(x.data_ptr(), x.stride(0), packed.data_ptr(), parts.data_ptr(),
                                           parts.numel(), rows, out_features, in_features, _lib.CDB_DTYPE_BF16,
                                           _stream()), "cdb_linear_parts")


def rmsnorm_fused_parts_raw(parts: torch.Tensor, residual: torch.Tensor | None, w_a: torch.Tensor,
                            w_b: torch.Tensor | None, out_h: torch.Tensor, out_y: torch.Tensor | None, mode: int,
                            eps_a: float, eps_b: float) -> None:
    """cdb_rmsnorm_fused on x = R(sum of the split-K partials `parts` [splits, rows, width]) (no allocation)."""

    splits, rows, width = parts.shape
    if parts.dtype != torch.float32:
        raise TypeError("parts must be float32")
    for name, t in (("residual", residual), ("out_h", out_h), ("out_y", out_y)):
        if t is not None and (t.shape != (rows, width) or t.dtype != out_h.dtype):
            raise ValueError(f"{name} must be [{rows}, {width}] of out_h's dtype")
    for name, w in (("w_a", w_a), ("w_b", w_b)):
        if w is not None and (w.shape != (width,) or w.dtype != out_h.dtype):
            raise ValueError(f"{name} must be a [{width}] vector of out_h's dtype")
    _require_cuda(parts, residual, w_a, w_b, out_h, out_y)
    _require_contiguous(parts=parts, residual=residual, w_a=w_a, w_b=w_b, out_h=out_h, out_y=out_y)
    code = _lib.lib().cdb_rmsnorm_fused_parts(
        parts.data_ptr(), splits, _ptr(residual), w_a.data_ptr(), _ptr(w_b), out_h.data_ptr(), _ptr(out_y),
        rows, width, mode, eps_a, eps_b, dtype_code(out_h.dtype), _stream())
    _lib.check(code, "cdb_rmsnorm_fused_parts")


def linear_residual_rmsnorm_auto(x: torch.Tensor, weight: torch.Tensor, packed: torch.Tensor | None,
                                 residual: torch.Tensor, w_a: torch.Tensor, w_b: torch.Tensor | None, eps_a: float,
                                 eps_b: float, mode: int) -> tuple[torch.Tensor, torch.Tensor | None]:
    """The body of cdb::linear_residual_rmsnorm, callable without op dispatch; without ``w_b``
    the second norm is skipped and y is None."""

    rows, in_features = x.shape
    out_features = weight.shape[0]
    splits = 0
    if (packed is not None and x.dtype == torch.bfloat16 and x.stride(1) == 1 and x.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0 and residual.is_contiguous()):
        splits = linear_parts_splits(rows, out_features, in_features)
    h = x.new_empty((rows, out_features))
    y = x.new_empty((rows, out_features)) if w_b is not None else None
    if splits:
        parts = torch.empty((splits, rows, out_features), dtype=torch.float32, device=x.device)
        linear_parts_raw(x, packed, parts)
        rmsnorm_fused_parts_raw(parts, residual, w_a, w_b, h, y, mode, eps_a, eps_b)
    else:
        o = linear_auto(x, weight, packed, False)
        rmsnorm_fused_raw(o, residual.contiguous(), w_a, w_b, h, y, mode, eps_a, eps_b)
    return h, y


@torch.library.custom_op("cdb::linear_residual_rmsnorm", mutates_args=(), device_types="cuda")
def linear_residual_rmsnorm(x: torch.Tensor, weight: torch.Tensor, packed: torch.Tensor | None,
                            residual: torch.Tensor, w_a: torch.Tensor, w_b: torch.Tensor, eps_a: float, eps_b: float,
                            mode: int) -> tuple[torch.Tensor, torch.Tensor]:
    """residual_rmsnorm(x @ weight.T, residual, ...): a projection into a residual norm.

    Shapes with a split-K form (linear_parts_splits > 0, given the packed weight)
    write fp32 partials that the norm adds in order and rounds once -- the
    projection's own bf16 output, never stored; others run cdb::linear then the
    fused norm."""

    return linear_residual_rmsnorm_auto(x, weight, packed, residual, w_a, w_b, eps_a, eps_b, mode)


@linear_residual_rmsnorm.register_fake
def _(x, weight, packed, residual, w_a, w_b, eps_a, eps_b, mode):
    shape = (x.shape[0], weight.shape[0])
    return x.new_empty(shape), x.new_empty(shape)


def copy_rows_raw(src: torch.Tensor, src_index: torch.Tensor | None, dst: torch.Tensor,
                  dst_index: torch.Tensor | None, rows: int) -> None:
    """dst[dst_index[i]] = src[src_index[i]] over whole rows of the first dimension (no allocation).

    Called several times per scheduler tick, so the checks touch each tensor
    property once (dtypes are singletons, compared by identity)."""

    shape = src.shape
    n_src, n_dst = shape[0], dst.shape[0]
    if src.dtype is not dst.dtype or shape[1:] != dst.shape[1:]:
        raise ValueError("src and dst rows must have the same shape and dtype")
    for name, idx, n in (("src_index", src_index, n_src), ("dst_index", dst_index, n_dst)):
        if idx is None:
            if n < rows:
                raise ValueError("identity index needs at least `rows` rows")
        elif idx.dtype is not torch.int64 or idx.numel() < rows or not idx.is_contiguous() or not idx.is_cuda:
            raise ValueError(f"{name} must be a contiguous CUDA int64 tensor with at least {rows} entries")
    if not (src.is_cuda and dst.is_cuda):
        raise RuntimeError("CDB kernels run on the GPU only; got a tensor on the CPU")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("src and dst must be contiguous")
    row_bytes = src.numel() // n_src * src.element_size() if n_src else 0
    code = _lib.lib().cdb_copy_rows(src.data_ptr(), None if src_index is None else src_index.data_ptr(), n_src,
                                    dst.data_ptr(), None if dst_index is None else dst_index.data_ptr(), n_dst, rows,
                                    row_bytes, _stream())
    if code:
        _lib.check(code, "cdb_copy_rows")


def gather_rows_raw(src: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """src[index] along dim 0 (negative indices give zero rows), without op dispatch."""

    out = src.new_empty((index.numel(), *src.shape[1:]))
    copy_rows_raw(src, index.contiguous(), out, None, index.numel())
    return out


@torch.library.custom_op("cdb::gather_rows", mutates_args=(), device_types="cuda")
def gather_rows(src: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """src[index] along dim 0; negative indices give zero rows."""

    return gather_rows_raw(src, index)


@gather_rows.register_fake
def _(src, index):
    return src.new_empty((index.numel(), *src.shape[1:]))


@torch.library.custom_op("cdb::scatter_rows_", mutates_args=("dst",), device_types="cuda")
def scatter_rows_(dst: torch.Tensor, index: torch.Tensor, src: torch.Tensor) -> None:
    """dst[index[i]] = src[i] along dim 0; negative indices skip the row."""

    copy_rows_raw(src, None, dst, index.contiguous(), index.numel())


def argmax_raw(logits: torch.Tensor, out: torch.Tensor) -> None:
    rows, vocab = logits.shape
    if out.dtype != torch.int64 or out.numel() < rows:
        raise ValueError("out must be int64 with a slot per row")
    _require_cuda(logits, out)
    _require_contiguous(logits=logits, out=out)
    _lib.check(_lib.lib().cdb_argmax(logits.data_ptr(), out.data_ptr(), rows, vocab, dtype_code(logits.dtype),
                                     _stream()), "cdb_argmax")


def _successor_embed_args(embed: torch.Tensor | None, bank: torch.Tensor | None, bank_slots: torch.Tensor | None,
                          rows: int) -> tuple:
    """(embed, bank, bank_rows, bank_slots, width) arguments of cdb_linear_argmax's fused prelude."""

    if embed is None:
        return None, None, 0, None, 0
    if bank is None or bank_slots is None:
        raise ValueError("the fused prelude needs the bank and the successors' bank slots")
    width = embed.shape[1]
    if (embed.dtype is not torch.bfloat16 or bank.dtype is not torch.bfloat16 or bank.dim() != 2
            or bank.shape[1] != width or not embed.is_contiguous() or not bank.is_contiguous()):
        raise ValueError("embed and bank must be contiguous bf16 [rows, width] tables of one width")
    if bank_slots.dtype is not torch.int64 or bank_slots.numel() < rows or not bank_slots.is_contiguous():
        raise ValueError(f"bank_slots must be a contiguous int64 tensor with at least {rows} entries")
    _require_cuda(embed, bank, bank_slots)
    return embed.data_ptr(), bank.data_ptr(), bank.shape[0], bank_slots.data_ptr(), width


def linear_argmax_raw(x: torch.Tensor, packed: torch.Tensor, out: torch.Tensor, workspace: torch.Tensor,
                      embed: torch.Tensor | None = None, bank: torch.Tensor | None = None,
                      bank_slots: torch.Tensor | None = None) -> None:
    """out[r] = argmax_n of the bf16 logits x @ W.T (torch.argmax order), the logits never stored.

    With ``embed``: bank[bank_slots[r]] = embed[out[r]] for rows whose slot is >= 0
    (the successor's prelude fused into the coda)."""

    _require_cuda(x, packed, out, workspace)
    rows, in_features = x.shape
    out_features = packed.numel() // in_features if in_features else 0
    if x.dtype != torch.bfloat16 or packed.dtype != x.dtype:
        raise TypeError("cdb_linear_argmax takes bfloat16 x and weight")
    if out.dtype != torch.int64 or out.numel() < rows or packed.numel() != out_features * in_features:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, packed weight of {packed.numel()} elements, "
                         f"out of {out.numel()} int64")
    if x.stride(1) != 1 or not packed.is_contiguous() or not out.is_contiguous() or not workspace.is_contiguous():
        raise ValueError("x must have unit stride along its last dimension; weight, out and workspace are dense")
    emb = _successor_embed_args(embed, bank, bank_slots, rows)
    _lib.check(_lib.lib().cdb_linear_argmax(x.data_ptr(), x.stride(0), packed.data_ptr(), out.data_ptr(),
                                            workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                                            rows, out_features, in_features, *emb, _lib.CDB_DTYPE_BF16, _stream()),
               "cdb_linear_argmax")


def lm_head_argmax(x: torch.Tensor, weight: torch.Tensor, packed: torch.Tensor | None,
                   embed: torch.Tensor | None = None, bank: torch.Tensor | None = None,
                   bank_slots: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy tokens of a coda batch: argmax over the vocabulary of x @ weight.T.

    Batches the projection kernel serves (linear_prefers_kernel) run the fused
    cdb_linear_argmax; others compute the logits (torch.mm) and cdb_argmax them.
    With ``embed``, rows whose ``bank_slots`` entry is >= 0 also get the embedding
    of their token written to that bank row (the next token's prelude): inside the
    fused call, or as one row copy after the unfused one."""

    rows, in_features = x.shape
    vocab = weight.shape[0]
    if (packed is not None and x.dtype is torch.bfloat16 and 1 <= rows <= LINEAR_MAX_ROWS
            and linear_prefers_kernel(rows, vocab, False, in_features) and vocab % 16 == 0
            and in_features % 32 == 0 and packed.numel() == vocab * in_features and packed.dtype is torch.bfloat16
            and x.is_cuda and packed.is_cuda and packed.is_contiguous()):
        stride = x.stride()
        ptr = x.data_ptr()
        if stride[1] == 1 and stride[0] % 8 == 0 and ptr % 16 == 0:
            out = torch.empty((rows,), dtype=torch.int64, device=x.device)
            workspace = torch.empty((rows * (vocab // 16) * 2,), dtype=torch.float32, device=x.device)
            emb = _successor_embed_args(embed, bank, bank_slots, rows)
            code = _lib.lib().cdb_linear_argmax(ptr, stride[0], packed.data_ptr(), out.data_ptr(),
                                                workspace.data_ptr(), workspace.numel() * 4, rows, vocab,
                                                in_features, *emb, _lib.CDB_DTYPE_BF16, _stream())
            if code:
                _lib.check(code, "cdb_linear_argmax")
            return out
    tokens = argmax_rows(linear_auto(x, weight, packed, False))
    if embed is not None:
        copy_rows_raw(embed, tokens, bank, bank_slots, rows)
    return tokens


CODA_DIRECT_MAX_ROWS = 64  # the fused LM head + argmax serves coda batches up to this size


@dataclass
class CodaWeights:
    """What cdb_coda_greedy reads besides the bank: the packed LM head and, when the coda
    fuses the successors' prelude, the token embedding."""

    packed: torch.Tensor  # bf16 LM head in cdb_linear_pack_weight order
    vocab: int
    width: int
    embed: torch.Tensor | None


class CodaScratch:
    """Device scratch of one coda turn plus the fixed arguments of cdb_coda_greedy.

    The pointers are resolved once, so a coda tick is one foreign call whose
    per-call arguments are the row and successor counts and the stream."""

    def __init__(self, weights: CodaWeights, bank: torch.Tensor, state: "GateState", host_upload: torch.Tensor,
                 dev_upload: torch.Tensor, host_tokens: torch.Tensor) -> None:
        rows = CODA_DIRECT_MAX_ROWS
        _require_cuda(bank, weights.packed, dev_upload)
        if bank.dtype is not torch.bfloat16 or bank.dim() != 2 or bank.shape[1] != weights.width \
                or not bank.is_contiguous():
            raise ValueError("the coda reads a contiguous bf16 bank of the LM head's input width")
        if weights.packed.dtype is not torch.bfloat16 or weights.packed.numel() != weights.vocab * weights.width:
            raise ValueError("the LM head must be packed bf16 [vocab, width]")
        if weights.embed is not None and (weights.embed.dtype is not torch.bfloat16
                                          or weights.embed.shape[1] != weights.width
                                          or not weights.embed.is_contiguous()):
            raise ValueError("the embedding must be a contiguous bf16 [vocab, width] table")
        if host_upload.numel() < 3 * rows or dev_upload.numel() < 3 * rows or host_tokens.numel() < rows:
            raise ValueError("coda upload buffers are smaller than a full direct coda")
        self.hidden = torch.empty((rows, weights.width), dtype=torch.bfloat16, device=bank.device)
        self.tokens = torch.empty((rows,), dtype=torch.int64, device=bank.device)
        ws_bytes = int(_lib.lib().cdb_linear_argmax_workspace_bytes(rows, weights.vocab))
        if ws_bytes < 0:
            raise ValueError(f"no fused argmax for a {weights.vocab}-column LM head")
        self.workspace = torch.empty((max(ws_bytes // 4, 4),), dtype=torch.float32, device=bank.device)
        embed = weights.embed.data_ptr() if weights.embed is not None else None
        self.head = (host_upload.data_ptr(), dev_upload.data_ptr())
        self.tail_plain = (bank.data_ptr(), bank.shape[0], weights.width, self.hidden.data_ptr(),
                           weights.packed.data_ptr(), weights.vocab, self.tokens.data_ptr(),
                           self.workspace.data_ptr(), self.workspace.numel() * 4, None, host_tokens.data_ptr(),
                           state.cdf.data_ptr(), state.survival.data_ptr(), state.pending.data_ptr(),
                           state.capacity, _lib.CDB_DTYPE_BF16)
        self.tail_fused = self.tail_plain[:9] + (embed,) + self.tail_plain[10:] if embed is not None else None

    def launch(self, rows: int, num_successors: int, fused: bool, stream: int) -> None:
        """Greedy tokens of `rows` coda rows whose slots (and successors) are in the host upload."""

        if not 1 <= rows <= CODA_DIRECT_MAX_ROWS:
            raise ValueError(f"a direct coda takes 1..{CODA_DIRECT_MAX_ROWS} rows, got {rows}")
        tail = self.tail_fused if fused else self.tail_plain
        if tail is None:
            raise ValueError("the fused successor prelude needs the token embedding")
        code = _lib.lib().cdb_coda_greedy(*self.head, rows, num_successors if fused else 0, *tail, stream)
        if code:
            _lib.check(code, "cdb_coda_greedy")


def table_updates_raw(table: torch.Tensor, idx: torch.Tensor, val: torch.Tensor, count: torch.Tensor,
                      capacity: int) -> None:
    """table.view(-1)[idx[i]] = val[i] for i < min(count[0], capacity), the count read on the device
    (a captured graph applies whatever the launch uploaded)."""

    if (table.dtype is not torch.int32 or idx.dtype is not torch.int64 or val.dtype is not torch.int32
            or count.dtype is not torch.int32):
        raise TypeError("table, val and count must be int32 and idx int64")
    if idx.numel() < capacity or val.numel() < capacity or count.numel() < 1 or not table.is_contiguous():
        raise ValueError(f"update buffers must hold {capacity} entries and the table be contiguous")
    code = _lib.lib().cdb_table_updates(table.data_ptr(), table.numel(), idx.data_ptr(), val.data_ptr(),
                                        count.data_ptr(), capacity, _stream())
    if code:
        _lib.check(code, "cdb_table_updates")


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    """Greedy token per row (first index of the max), without op dispatch."""

    l2 = logits.reshape(-1, logits.shape[-1])
    out = torch.empty((l2.shape[0],), dtype=torch.int64, device=logits.device)
    argmax_raw(l2, out)
    return out.view(logits.shape[:-1])


@torch.library.custom_op("cdb::argmax", mutates_args=(), device_types="cuda")
def argmax(logits: torch.Tensor) -> torch.Tensor:
    """Greedy token per row of a [rows, vocab] logits matrix (first index of the max)."""

    return argmax_rows(logits)


@argmax.register_fake
def _(logits):
    return logits.new_empty(logits.shape[:-1], dtype=torch.int64)


@dataclass
class GateState:
    """Device-resident exit-policy state, one entry per hidden-bank slot."""

    cdf: torch.Tensor        # float64 [capacity]
    survival: torch.Tensor   # float64 [capacity]
    pending: torch.Tensor    # float32 [capacity], NaN = no pending signal

    @classmethod
    def allocate(cls, capacity: int, device: torch.device) -> "GateState":
        return cls(
            cdf=torch.zeros(capacity, dtype=torch.float64, device=device),
            survival=torch.ones(capacity, dtype=torch.float64, device=device),
            pending=torch.full((capacity,), float("nan"), dtype=torch.float32, device=device),
        )

    @property
    def capacity(self) -> int:
        return self.cdf.numel()

    def reset(self, index: torch.Tensor, n: int | None = None) -> None:
        n = index.numel() if n is None else n
        _lib.check(_lib.lib().cdb_exit_gate_reset(self.cdf.data_ptr(), self.survival.data_ptr(),
                                                  self.pending.data_ptr(), self.capacity, index.data_ptr(), n,
                                                  _stream()), "cdb_exit_gate_reset")


GATE_HAZARD, GATE_LATENT_DIFF = 0, 1
RULE_CUMULATIVE_HAZARD, RULE_DIRECT_THRESHOLD = 0, 1


def exit_gate_raw(hidden: torch.Tensor, prev: torch.Tensor | None, weight: torch.Tensor | None,
                  bias: torch.Tensor | None, signal: torch.Tensor, state: GateState, state_index: torch.Tensor,
                  steps: torch.Tensor, synthetic_depth: torch.Tensor | None, exit_flags: torch.Tensor, rows: int,
                  *, kind: int, rule: int, delayed: bool, round_hazard: bool, min_steps: int, max_steps: int,
                  threshold: float | None) -> None:
    """Launch ``cdb_exit_gate`` for the first ``rows`` rows (no allocation)."""

    width = hidden.shape[-1]
    if hidden.dim() != 2 or hidden.shape[0] < rows:
        raise ValueError("hidden must be [>= rows, width]")
    if kind == GATE_HAZARD and (weight is None or weight.numel() != width):
        raise ValueError("the hazard gate needs a [width] weight")
    if kind == GATE_LATENT_DIFF and (prev is None or prev.shape != hidden.shape):
        raise ValueError("the latent-difference gate needs prev shaped like hidden")
    if state_index.dtype != torch.int64 or steps.dtype != torch.int32 or exit_flags.dtype != torch.uint8:
        raise TypeError("state_index int64, steps int32, exit_flags uint8 expected")
    if synthetic_depth is not None and synthetic_depth.dtype != torch.int32:
        raise TypeError("synthetic_depth must be int32")
    for t in (signal, state_index, steps, exit_flags, synthetic_depth):
        if t is not None and t.numel() < rows:
            raise ValueError("per-row buffers need at least `rows` entries")
    _require_cuda(hidden, prev, weight, bias, signal, state_index, steps, synthetic_depth, exit_flags)
    code = _lib.lib().cdb_exit_gate(
        hidden.data_ptr(), _ptr(prev), _ptr(weight), _ptr(bias), signal.data_ptr(),
        state.cdf.data_ptr(), state.survival.data_ptr(), state.pending.data_ptr(), state.capacity,
        state_index.data_ptr(), steps.data_ptr(), _ptr(synthetic_depth), exit_flags.data_ptr(), rows,
        width, kind, rule, int(delayed), int(round_hazard), min_steps, max_steps,
        0.0 if threshold is None else float(threshold), int(threshold is not None), dtype_code(hidden.dtype),
        _stream())
    _lib.check(code, "cdb_exit_gate")


@torch.library.custom_op("cdb::exit_gate", mutates_args=("signal", "cdf", "survival", "pending", "exit_flags"),
                        device_types="cuda")
def exit_gate(hidden: torch.Tensor, prev: torch.Tensor | None, weight: torch.Tensor | None, bias: torch.Tensor | None,
              signal: torch.Tensor, cdf: torch.Tensor, survival: torch.Tensor, pending: torch.Tensor,
              state_index: torch.Tensor, steps: torch.Tensor, synthetic_depth: torch.Tensor | None,
              exit_flags: torch.Tensor, rows: int, kind: int, rule: int, delayed: bool, round_hazard: bool,
              min_steps: int, max_steps: int, threshold: float | None) -> None:
    """The exit gate of one recurrent launch's first ``rows`` rows (cdb/adapters/ouro.py:286-291,
    cdb/exit_policy.py:150-169, huginn/exit_gates.py:33-40): the gate signal per row (``kind``
    GATE_HAZARD: the bf16 Linear(E, 1) logit; GATE_LATENT_DIFF: the relative L2 change against
    ``prev``), the per-token policy state (``cdf``, ``survival``, ``pending``, indexed by
    ``state_index``) and one exit byte per row in ``exit_flags``, all updated in place."""

    exit_gate_raw(hidden, prev, weight, bias, signal, GateState(cdf=cdf, survival=survival, pending=pending),
                  state_index, steps, synthetic_depth, exit_flags, rows, kind=kind, rule=rule, delayed=delayed,
                  round_hazard=round_hazard, min_steps=min_steps, max_steps=max_steps, threshold=threshold)


@exit_gate.register_fake
def _(hidden, prev, weight, bias, signal, cdf, survival, pending, state_index, steps, synthetic_depth, exit_flags,
      rows, kind, rule, delayed, round_hazard, min_steps, max_steps, threshold):
    return None


def route_compact_raw(exit_flags: torch.Tensor, bank_slots: torch.Tensor, lists: torch.Tensor) -> None:
    """Launch ``cdb_route_compact`` over ``bank_slots.numel()`` rows (no allocation): ``lists``
    int32 [2 + rows] gets [n_exit, n_stay, exiting rows, staying rows] in launch order."""

    rows = bank_slots.numel()
    if exit_flags.dtype != torch.uint8 or bank_slots.dtype != torch.int64 or lists.dtype != torch.int32:
        raise TypeError("exit_flags uint8, bank_slots int64 and lists int32 expected")
    if exit_flags.numel() < rows or lists.numel() < 2 + rows:
        raise ValueError("exit_flags needs a byte per row and lists 2 + rows entries")
    _require_cuda(exit_flags, bank_slots, lists)
    _require_contiguous(exit_flags=exit_flags, bank_slots=bank_slots, lists=lists)
    _lib.check(_lib.lib().cdb_route_compact(exit_flags.data_ptr(), bank_slots.data_ptr(), rows, lists.data_ptr(),
                                            _stream()), "cdb_route_compact")


@torch.library.custom_op("cdb::route_compact", mutates_args=("lists",), device_types="cuda")
def route_compact(exit_flags: torch.Tensor, bank_slots: torch.Tensor, lists: torch.Tensor) -> None:
    """Exit routing of one recurrent launch in launch order (cdb/continuous_api.py:1171-1183):
    ``lists`` = [n_exit, n_stay, the exiting rows, the staying rows]; padding rows (negative
    bank slot) are in neither list."""

    route_compact_raw(exit_flags, bank_slots, lists)


@route_compact.register_fake
def _(exit_flags, bank_slots, lists):
    return None


def exit_kv_copy_raw(view: KVPoolView, rows: torch.Tensor, exit_slot: torch.Tensor, n: int, *, layer_base: int,
                     core_layers: int, num_slots: int) -> None:
    """Copy each exiting token's exit-slot KV into its deeper slots (copy-on-exit layout)."""

    pool = view.pool
    if rows.dtype != torch.int64 or exit_slot.dtype != torch.int32:
        raise TypeError("rows int64 and exit_slot int32 expected")
    if layer_base + num_slots * core_layers > view.num_cache_layers:
        raise ValueError("slot layout exceeds the pool's cache layers")
    _require_cuda(pool, rows, exit_slot)
    code = _lib.lib().cdb_exit_kv_copy(view.k_ptr, view.v_ptr, view.layer_stride, view.pool_rows, pool.shape[3],
                                       pool.shape[4], rows.data_ptr(), exit_slot.data_ptr(), n, layer_base,
                                       core_layers, num_slots, dtype_code(pool.dtype), _stream())
    _lib.check(code, "cdb_exit_kv_copy")


@torch.library.custom_op("cdb::exit_kv_copy", mutates_args=("kv_pool",), device_types="cuda")
def exit_kv_copy(kv_pool: torch.Tensor, block_size: int, rows: torch.Tensor, exit_slot: torch.Tensor, n: int,
                 layer_base: int, core_layers: int, num_slots: int) -> None:
    """Exit-KV propagation under a copy-on-exit KV layout (cdb/continuous_api.py:1225-1245,
    cdb/cache.py:99-113): token i's K/V row ``rows[i]`` of cache layer
    ``layer_base + exit_slot[i] * core_layers + l`` is copied to every deeper slot's layer, for all
    core layers l, in ``kv_pool`` [num_cache_layers, 2, pool_rows, Hkv, D]."""

    exit_kv_copy_raw(KVPoolView(kv_pool, block_size), rows, exit_slot, n, layer_base=layer_base,
                     core_layers=core_layers, num_slots=num_slots)


@exit_kv_copy.register_fake
def _(kv_pool, block_size, rows, exit_slot, n, layer_base, core_layers, num_slots):
    return None


def rope_kv_write_raw(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_out: torch.Tensor, view: KVPoolView,
                      layer: int, rows: torch.Tensor, positions: torch.Tensor, rope_cos: torch.Tensor | None,
                      rope_sin: torch.Tensor | None, rope_style: int, q_bias: torch.Tensor | None,
                      k_bias: torch.Tensor | None) -> None:
    """Rotate q/k of T tokens, write k/v to pool rows of cache layer ``layer`` (no allocation).

    q, k and v may be token-strided views (e.g. column slices of a fused QKV output)
    whose [heads, head_dim] part is dense; k and v must share one token stride."""

    tokens, num_heads, head_dim = q.shape
    num_kv_heads = k.shape[1]
    if k.shape != (tokens, num_kv_heads, head_dim) or v.shape != k.shape or q_out.shape != q.shape:
        raise ValueError("q/k/v/q_out shapes disagree")
    if rows.dtype != torch.int64 or positions.dtype != torch.int32 or rows.numel() < tokens:
        raise TypeError("rows int64 and positions int32 with a slot per token expected")
    if not 0 <= layer < view.num_cache_layers:
        raise ValueError("layer out of range")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.stride(2) != 1 or t.stride(1) != head_dim:
            raise ValueError(f"{name} must be dense within a token ([heads, head_dim] contiguous)")
    if k.stride(0) != v.stride(0):
        raise ValueError("k and v must share one token stride")
    _require_cuda(q, k, v, q_out, rows, positions, rope_cos, rope_sin)
    _require_contiguous(q_out=q_out, rows=rows, positions=positions)
    code = _lib.lib().cdb_rope_kv_write(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), q_out.data_ptr(), view.k_ptr, view.v_ptr, view.layer_stride,
        layer, rows.data_ptr(), view.pool_rows, positions.data_ptr(), _ptr(rope_cos), _ptr(rope_sin), rope_style,
        0 if rope_cos is None else rope_cos.shape[0], _ptr(q_bias), _ptr(k_bias), tokens, num_heads,
        num_kv_heads, head_dim, q.stride(0), k.stride(0), dtype_code(q.dtype), _stream())
    _lib.check(code, "cdb_rope_kv_write")


@torch.library.custom_op("cdb::rope_kv_write", mutates_args=("kv_pool",), device_types="cuda")
def rope_kv_write(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_pool: torch.Tensor, layer: int,
                  block_size: int, rows: torch.Tensor, positions: torch.Tensor, rope_cos: torch.Tensor | None,
                  rope_sin: torch.Tensor | None, rope_style: int, q_bias: torch.Tensor | None,
                  k_bias: torch.Tensor | None) -> torch.Tensor:
    """RoPE + KV append of a prefill chunk's T tokens (cb/cache.py:284-318 with the write indices
    of cb/cache_manager.py:190-213; ouro/modeling_ouro.py:179-204, huginn/modeling_huginn.py:178-196
    and its qk_bias): token t's rotated key and its value go to pool row ``rows[t]`` of cache layer
    ``layer`` in ``kv_pool`` [num_cache_layers, 2, pool_rows, Hkv, D]; returns the rotated queries
    [T, H, D]. q, k and v may be column slices of one fused QKV output."""

    q_rot = q.new_empty(q.shape)
    rope_kv_write_raw(q, k, v, q_rot, KVPoolView(kv_pool, block_size), layer, rows, positions, rope_cos, rope_sin,
                      rope_style, q_bias, k_bias)
    return q_rot


@rope_kv_write.register_fake
def _(q, k, v, kv_pool, layer, block_size, rows, positions, rope_cos, rope_sin, rope_style, q_bias, k_bias):
    return q.new_empty(q.shape)


PREFILL_TILE = 128


def prefill_tiles(query_lens: "list[int] | np.ndarray",
                  past: "list[int] | np.ndarray | None" = None) -> tuple["np.ndarray", "np.ndarray"]:
    """Tile -> (sequence, first query) arrays for cdb_prefill_attention (128 queries per tile),
    longest causal prefix (past + last query of the tile) first, so the heaviest workgroups
    start first and the launch ends on short ones. Any order computes the same outputs."""

    import numpy as np

    lens = np.asarray(query_lens, dtype=np.int64)
    counts = (lens + PREFILL_TILE - 1) // PREFILL_TILE
    seq = np.repeat(np.arange(lens.size, dtype=np.int32), counts)
    starts = np.concatenate([[0], np.cumsum(counts)[:-1]]) if lens.size else np.zeros(0, np.int64)
    q0 = (np.arange(int(counts.sum())) - np.repeat(starts, counts)) * PREFILL_TILE
    base = np.zeros(lens.size, np.int64) if past is None else np.asarray(past, dtype=np.int64)
    key_end = base[seq] + np.minimum(q0 + PREFILL_TILE, lens[seq])
    order = np.argsort(-key_end, kind="stable")
    return seq[order].astype(np.int32), q0[order].astype(np.int32)


PREFILL_KEY_BLOCK = 32  # keys per block of the bf16 prefill kernel's key loop


@dataclass(frozen=True)
class PrefillSplitWork:
    """Host work list of cdb_prefill_attention_split.

    items  [n, 4] int32: (sequence, first query, first key block | end key block << 16, slot or -1)
    merges [m, 4] int32: (sequence, first query, first slot, parts)
    """

    items: "np.ndarray"
    merges: "np.ndarray"
    num_slots: int
    max_blocks: int


PREFILL_WGS_PER_CU = 3  # resident bf16 prefill workgroups per CU (LDS and registers)


def prefill_split_blocks(total_blocks: int, num_heads: int, num_cus: int) -> int:
    """Longest key range, in 32-key blocks, that one workgroup takes when tiles are split: an
    even share of all key blocks over the resident workgroup slots, at least 16 blocks (a part
    re-reads its tile's queries and writes a 66 KiB partial per head, which the merge reads)."""

    slots = PREFILL_WGS_PER_CU * int(num_cus)
    return max(16, -(-int(total_blocks) * int(num_heads) // slots))


def prefill_split_plan(query_lens: "list[int] | np.ndarray", past: "list[int] | np.ndarray | None" = None, *,
                       num_heads: int, num_cus: int = 256) -> "PrefillSplitWork | None":
    """The split work list when one tile's key range is long enough to outlast the whole rest of
    the launch (more than four times an even share of the key blocks over the workgroup slots,
    e.g. a chunk appended to a long history); None when whole tiles are the faster launch, as
    for a batch of fresh prompts, where the throughput of the full GPU sets the time."""

    import numpy as np

    seq, q0 = prefill_tiles(query_lens, past)
    if seq.size == 0:
        return None
    lens = np.asarray(query_lens, dtype=np.int64)
    base = np.zeros(lens.size, np.int64) if past is None else np.asarray(past, dtype=np.int64)
    key_end = base[seq] + np.minimum(q0 + PREFILL_TILE, lens[seq])
    blocks = (key_end + PREFILL_KEY_BLOCK - 1) // PREFILL_KEY_BLOCK
    share = int(blocks.sum()) * int(num_heads) / (PREFILL_WGS_PER_CU * int(num_cus))
    max_blocks = prefill_split_blocks(int(blocks.sum()), num_heads, num_cus)
    if int(blocks.max()) <= max(4 * share, max_blocks):
        return None
    return prefill_split_work(query_lens, past, num_heads=num_heads, num_cus=num_cus, max_blocks=max_blocks)


def prefill_split_work(query_lens: "list[int] | np.ndarray", past: "list[int] | np.ndarray | None" = None, *,
                       num_heads: int, num_cus: int = 256, max_blocks: int | None = None) -> PrefillSplitWork:
    """Split the 128-query tiles whose key range exceeds `max_blocks` blocks into parts of at
    most about that many blocks. A tile's last part holds its diagonal (it starts at or before
    the block of the tile's first query position), so every query sees a key in every part.
    Items are listed longest key range first."""

    import numpy as np

    seq, q0 = prefill_tiles(query_lens, past)
    lens = np.asarray(query_lens, dtype=np.int64)
    base = np.zeros(lens.size, np.int64) if past is None else np.asarray(past, dtype=np.int64)
    first_pos = base[seq] + q0
    key_end = first_pos + np.minimum(PREFILL_TILE, lens[seq] - q0)
    blocks = (key_end + PREFILL_KEY_BLOCK - 1) // PREFILL_KEY_BLOCK
    if max_blocks is None:
        max_blocks = prefill_split_blocks(int(blocks.sum()), num_heads, num_cus)
    if max_blocks < 8 or int(blocks.max(initial=0)) >= 1 << 15:
        raise ValueError("need max_blocks >= 8 and fewer than 32768 key blocks per tile")
    items, merges, slot = [], [], 0
    for s_, t0, nb, pos in zip(seq.tolist(), q0.tolist(), blocks.tolist(), first_pos.tolist()):
        if nb <= max_blocks:
            items.append((s_, t0, nb << 16, -1))
            continue
        parts = -(-nb // max_blocks)
        step = -(-nb // parts)
        starts = [k * step for k in range(parts)]
        starts[-1] = min(starts[-1], pos // PREFILL_KEY_BLOCK)
        ends = starts[1:] + [nb]
        assert all(a < b for a, b in zip(starts, ends))
        items.extend((s_, t0, a | (b << 16), slot + k) for k, (a, b) in enumerate(zip(starts, ends)))
        merges.append((s_, t0, slot, parts))
        slot += parts
    items_arr = np.asarray(items, dtype=np.int32).reshape(-1, 4)
    length = (items_arr[:, 2] >> 16) - (items_arr[:, 2] & 0xFFFF)
    items_arr = items_arr[np.argsort(-length, kind="stable")]
    return PrefillSplitWork(items=items_arr, merges=np.asarray(merges, dtype=np.int32).reshape(-1, 4),
                            num_slots=slot, max_blocks=int(max_blocks))


def prefill_partial_bytes(num_slots: int, num_heads: int, head_dim: int) -> int:
    n = int(_lib.lib().cdb_prefill_partial_bytes(num_slots, num_heads, head_dim))
    if n < 0:
        raise ValueError("invalid prefill partial-buffer shape")
    return n


def prefill_attention_split_raw(q: torch.Tensor, view: KVPoolView, layer: int, block_table: torch.Tensor,
                                table_row: torch.Tensor, cu_q: torch.Tensor, past: torch.Tensor,
                                items: torch.Tensor, merges: torch.Tensor, num_slots: int, partials: torch.Tensor,
                                out: torch.Tensor, scale: float) -> None:
    """Launch ``cdb_prefill_attention_split`` (bf16; no allocation): items [n, 4] and merges [m, 4]
    int32 on the GPU, partials a caller buffer of at least prefill_partial_bytes(num_slots) bytes."""

    tokens, num_heads, head_dim = q.shape
    pool = view.pool
    if out.shape != q.shape or out.dtype != q.dtype or pool.dtype != q.dtype:
        raise ValueError("out/pool must match q")
    num_seqs = past.numel()
    if cu_q.numel() != num_seqs + 1 or table_row.numel() < num_seqs:
        raise ValueError("inconsistent prefill metadata")
    if items.dim() != 2 or items.shape[1] != 4 or merges.dim() != 2 or merges.shape[1] != 4:
        raise ValueError("items and merges must be [n, 4]")
    _require_int32(block_table=block_table, table_row=table_row, cu_q=cu_q, past=past, items=items, merges=merges)
    _require_cuda(q, pool, block_table, table_row, cu_q, past, items, merges, partials, out)
    _require_contiguous(q=q, out=out, block_table=block_table, items=items, merges=merges, partials=partials)
    nbytes = partials.numel() * partials.element_size()
    code = _lib.lib().cdb_prefill_attention_split(
        q.data_ptr(), view.k_ptr, view.v_ptr, view.layer_stride, layer, view.num_cache_layers, view.pool_blocks,
        block_table.data_ptr(), table_row.data_ptr(), block_table.shape[1], cu_q.data_ptr(), past.data_ptr(),
        num_seqs, items.data_ptr(), items.shape[0], merges.data_ptr() if merges.numel() else None, merges.shape[0],
        num_slots, partials.data_ptr() if num_slots else None, nbytes, out.data_ptr(), num_heads, pool.shape[3],
        head_dim, view.block_size, scale, dtype_code(q.dtype), _stream())
    _lib.check(code, "cdb_prefill_attention_split")


@torch.library.custom_op("cdb::prefill_attention", mutates_args=(), device_types="cuda")
def prefill_attention(q: torch.Tensor, kv_pool: torch.Tensor, layer: int, block_size: int,
                      block_table: torch.Tensor, table_row: torch.Tensor, cu_q: torch.Tensor, past: torch.Tensor,
                      tile_seq: torch.Tensor, tile_q0: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal varlen prefill attention over [past | new] through the block table
    (cb/prefill_graph.py:265-309, flash_attn_varlen_func): sequence s's queries
    q[cu_q[s]:cu_q[s + 1]] sit at positions past[s]... and attend over the K/V of cache layer
    ``layer`` in ``kv_pool``, read through block-table row table_row[s]. Tiles of 128 queries are
    listed by (tile_seq, tile_q0) (prefill_tiles). Returns [T, H, D]."""

    out = q.new_empty(q.shape)
    prefill_attention_raw(q, KVPoolView(kv_pool, block_size), layer, block_table, table_row, cu_q, past, tile_seq,
                          tile_q0, out, scale)
    return out


@prefill_attention.register_fake
def _(q, kv_pool, layer, block_size, block_table, table_row, cu_q, past, tile_seq, tile_q0, scale):
    return q.new_empty(q.shape)


@torch.library.custom_op("cdb::prefill_attention_split", mutates_args=("partials",), device_types="cuda")
def prefill_attention_split(q: torch.Tensor, kv_pool: torch.Tensor, layer: int, block_size: int,
                            block_table: torch.Tensor, table_row: torch.Tensor, cu_q: torch.Tensor,
                            past: torch.Tensor, items: torch.Tensor, merges: torch.Tensor, num_slots: int,
                            partials: torch.Tensor, scale: float) -> torch.Tensor:
    """cdb::prefill_attention with long tiles' key ranges split over workgroups and merged
    (prefill_split_work): ``partials`` is scratch of at least prefill_partial_bytes(num_slots)."""

    out = q.new_empty(q.shape)
    prefill_attention_split_raw(q, KVPoolView(kv_pool, block_size), layer, block_table, table_row, cu_q, past,
                                items, merges, num_slots, partials, out, scale)
    return out


@prefill_attention_split.register_fake
def _(q, kv_pool, layer, block_size, block_table, table_row, cu_q, past, items, merges, num_slots, partials, scale):
    return q.new_empty(q.shape)


def prefill_attention_launch(q: torch.Tensor, kv_pool: torch.Tensor, layer: int, block_size: int,
                             block_table: torch.Tensor, launch, scale: float) -> torch.Tensor:
    """Prefill attention of one layer for a prefill launch (model_adapter.PrefillLaunch): the
    split work list when the launch carries one, else its whole tiles."""

    if launch.split_items is not None:
        return torch.ops.cdb.prefill_attention_split(q, kv_pool, layer, block_size, block_table, launch.table_rows,
                                                     launch.cu_q, launch.past, launch.split_items,
                                                     launch.split_merges, launch.split_slots, launch.partials, scale)
    return torch.ops.cdb.prefill_attention(q, kv_pool, layer, block_size, block_table, launch.table_rows, launch.cu_q,
                                           launch.past, launch.tile_seq, launch.tile_q0, scale)


def prefill_attention_raw(q: torch.Tensor, view: KVPoolView, layer: int, block_table: torch.Tensor,
                          table_row: torch.Tensor, cu_q: torch.Tensor, past: torch.Tensor, tile_seq: torch.Tensor,
                          tile_q0: torch.Tensor, out: torch.Tensor, scale: float) -> None:
    """Launch ``cdb_prefill_attention`` (no allocation); all index tensors int32 on the GPU."""

    tokens, num_heads, head_dim = q.shape
    pool = view.pool
    if out.shape != q.shape or out.dtype != q.dtype or pool.dtype != q.dtype:
        raise ValueError("out/pool must match q")
    num_seqs = past.numel()
    if cu_q.numel() != num_seqs + 1 or table_row.numel() < num_seqs or tile_seq.numel() != tile_q0.numel():
        raise ValueError("inconsistent prefill metadata")
    _require_int32(block_table=block_table, table_row=table_row, cu_q=cu_q, past=past, tile_seq=tile_seq,
                   tile_q0=tile_q0)
    _require_cuda(q, pool, block_table, table_row, cu_q, past, tile_seq, tile_q0, out)
    _require_contiguous(q=q, out=out, block_table=block_table)
    code = _lib.lib().cdb_prefill_attention(
        q.data_ptr(), view.k_ptr, view.v_ptr, view.layer_stride, layer, view.num_cache_layers, view.pool_blocks,
        block_table.data_ptr(), table_row.data_ptr(), block_table.shape[1], cu_q.data_ptr(), past.data_ptr(),
        num_seqs, tile_seq.data_ptr(), tile_q0.data_ptr(), tile_seq.numel(), out.data_ptr(), num_heads,
        pool.shape[3], head_dim, view.block_size, scale, dtype_code(q.dtype), _stream())
    _lib.check(code, "cdb_prefill_attention")
