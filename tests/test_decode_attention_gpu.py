"""HIP mixed-depth paged decode attention vs the oracle (through the C ABI).

Tolerances (bf16 storage, fp32 accumulate): max |err| <= 2e-2 and mean |err|
<= 2e-3 against the float64 oracle; fp32 storage: 2e-5 / 2e-6. The appended
KV rows must be bit-identical to the oracle's (same rounding of the rotated
key), and every other pool row must be untouched.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.paged_attention import paged_decode_attention as oracle_decode
from tests.decode_cases import make_case

pytestmark = pytest.mark.gpu

TOL = {"bf16": (2e-2, 2e-3), "f32": (2e-5, 2e-6)}
TORCH_DTYPE = {"bf16": torch.bfloat16, "f32": torch.float32}


def run_hip(case, split_pages: int, use_table_row: bool = False, workspace_split: int | None = None,
            repeats: int = 1):
    from continuous_depth_batching_amd import ops

    dev = torch.device("cuda")
    dt = TORCH_DTYPE[case.dtype]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    q, k, v = t(case.q).to(dt), t(case.k_new).to(dt), t(case.v_new).to(dt)
    pool = t(case.kv_pool).to(dt).contiguous()
    num_rows, num_heads, head_dim = case.q.shape
    table = t(case.block_table)
    table_row = None
    if use_table_row:
        # Reverse the table rows and index them through table_row.
        table = torch.flip(table, dims=[0]).contiguous()
        table_row = torch.arange(num_rows - 1, -1, -1, dtype=torch.int32, device=dev)
    max_pos = int(case.seqlens.max()) + 1
    ws_split = workspace_split or (split_pages if split_pages > 0 else ops.MIN_SPLIT_PAGES)
    ws = torch.empty(ops.decode_workspace_bytes(num_rows, num_heads, head_dim, max(max_pos, 1), case.block_size,
                                                ws_split) // 4, dtype=torch.float32, device=dev)
    cos = sin = None
    if case.rope_style:
        cos, sin = t(case.rope[0]), t(case.rope[1])
    qb = t(case.q_bias).to(dt) if case.q_bias is not None else None
    kb = t(case.k_bias).to(dt) if case.k_bias is not None else None
    pool0 = pool.clone()
    for _ in range(repeats):
        # Repeats re-run the same append onto a fresh copy of the pool: the workspace header
        # and partials left by the previous launch must not leak into the next one.
        pool.copy_(pool0)
        out = torch.ops.cdb.paged_decode_attention(
            q, k, v, pool, t(case.cache_layer), 0, table, table_row, t(case.seqlens), cos, sin, case.rope_style,
            qb, kb, ws, case.block_size, split_pages, case.scale)
    torch.cuda.synchronize()
    return out.float().cpu().numpy(), pool.float().cpu().numpy()


def run_oracle(case):
    pool = case.kv_pool.copy()
    out = oracle_decode(case.q, case.k_new, case.v_new, pool, case.cache_layer, case.block_table, case.seqlens,
                        case.block_size, case.scale, rope=case.rope, rope_style=case.rope_style,
                        q_bias=case.q_bias, k_bias=case.k_bias, dtype=case.dtype)
    return out, pool


def check(case, split_pages: int, use_table_row: bool = False, **kw) -> None:
    got, got_pool = run_hip(case, split_pages, use_table_row, **kw)
    want, want_pool = run_oracle(case)
    live = case.seqlens >= 0
    err = np.abs(got[live] - want[live])
    max_tol, mean_tol = TOL[case.dtype]
    assert np.isfinite(got[live]).all()
    assert err.max() <= max_tol, f"max err {err.max()}"
    assert err.mean() <= mean_tol, f"mean err {err.mean()}"
    assert np.all(got[~live] == 0.0)
    np.testing.assert_array_equal(got_pool, want_pool)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("split_pages", [0, 1, 4, 64, -4, -1])  # -m: adaptive with at least m pages
def test_ouro_shape_mixed_depth(dtype: str, split_pages: int) -> None:
    case = make_case(seed=10, num_rows=24, num_heads=16, num_kv_heads=16, head_dim=128, max_context=700,
                     rope_style=1, dtype=dtype, padding_rows=3)
    check(case, split_pages)


def test_adaptive_split_repeated_launches() -> None:
    case = make_case(seed=16, num_rows=33, num_heads=16, num_kv_heads=16, head_dim=128, max_context=1500,
                     rope_style=1, dtype="bf16", padding_rows=2)
    check(case, 0, repeats=3)


def test_adaptive_split_grows_to_fit_small_workspace() -> None:
    # A workspace sized for 64-page splits: the kernel must coarsen its splits to fit it.
    case = make_case(seed=17, num_rows=12, num_heads=16, num_kv_heads=16, head_dim=128, max_context=3000,
                     rope_style=1, dtype="bf16")
    check(case, 0, workspace_split=64)


def test_table_row_indirection() -> None:
    case = make_case(seed=11, num_rows=9, num_heads=16, num_kv_heads=16, head_dim=128, max_context=300,
                     rope_style=1, dtype="bf16")
    check(case, 2, use_table_row=True)


@pytest.mark.parametrize("head_dim,rope_style,num_kv_heads", [(64, 1, 4), (96, 2, 5), (128, 0, 16)])
def test_other_head_dims_and_rope_styles(head_dim: int, rope_style: int, num_kv_heads: int) -> None:
    case = make_case(seed=12, num_rows=10, num_heads=num_kv_heads * (2 if head_dim == 64 else 1),
                     num_kv_heads=num_kv_heads, head_dim=head_dim, max_context=400, rope_style=rope_style,
                     dtype="bf16", qk_bias=rope_style == 2)
    check(case, 4)


def test_huginn_shape_55_heads() -> None:
    case = make_case(seed=13, num_rows=5, num_heads=55, num_kv_heads=55, head_dim=96, max_context=200,
                     rope_style=2, dtype="bf16", qk_bias=True)
    check(case, 4)


def test_single_token_rows_and_block_size_32() -> None:
    case = make_case(seed=14, num_rows=7, num_heads=4, num_kv_heads=4, head_dim=64, max_context=1, rope_style=1,
                     dtype="f32", block_size=32)
    check(case, 1)


def test_long_context_rows() -> None:
    case = make_case(seed=15, num_rows=4, num_heads=16, num_kv_heads=16, head_dim=128, max_context=8192,
                     min_context=6000, rope_style=1, dtype="bf16")
    check(case, 16)


def test_more_than_64_splits_per_row() -> None:
    # One-page splits over ~6000 tokens: the merge walks its partials in chunks of 64.
    case = make_case(seed=18, num_rows=3, num_heads=4, num_kv_heads=4, head_dim=128, max_context=6000,
                     min_context=4500, rope_style=1, dtype="bf16")
    check(case, 1)


@pytest.mark.parametrize("block_size,split_pages", [(4, 64), (8, 0), (2, 5)])
def test_small_pages_cross_window_steps(block_size: int, split_pages: int) -> None:
    # Pages shorter than a 16-token step: block ids come per lane from the page window,
    # and steps that would leave the window reload it.
    case = make_case(seed=19, num_rows=6, num_heads=8, num_kv_heads=4, head_dim=64, max_context=900,
                     rope_style=1, dtype="bf16", block_size=block_size, padding_rows=1)
    check(case, split_pages)


def test_split_longer_than_page_window() -> None:
    # 128-page splits: one item walks past its first 64-page window.
    case = make_case(seed=20, num_rows=3, num_heads=16, num_kv_heads=16, head_dim=128, max_context=5000,
                     min_context=3000, rope_style=1, dtype="bf16")
    check(case, 128)


def test_out_of_range_row_is_flagged_nan_and_writes_nothing() -> None:
    case = make_case(seed=16, num_rows=3, num_heads=4, num_kv_heads=4, head_dim=64, max_context=40, rope_style=0,
                     dtype="f32")
    width = case.block_table.shape[1]
    case.seqlens[1] = width * case.block_size  # one past the table
    got, got_pool = run_hip(case, 1)
    assert np.isnan(got[1]).all()
    ok = np.array([True, False, True])
    case.seqlens[1] = -1
    want, want_pool = run_oracle(case)
    np.testing.assert_allclose(got[ok], want[ok], atol=2e-5)
    np.testing.assert_array_equal(got_pool, want_pool)


def _device_case(case):
    from continuous_depth_batching_amd import ops

    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    dt = TORCH_DTYPE[case.dtype]
    pool = t(case.kv_pool).to(dt).contiguous()
    tensors = dict(q=t(case.q).to(dt), k=t(case.k_new).to(dt), v=t(case.v_new).to(dt), pool=pool,
                   layer=t(case.cache_layer), table=t(case.block_table), seqlens=t(case.seqlens),
                   cos=t(case.rope[0]), sin=t(case.rope[1]),
                   q_bias=None if case.q_bias is None else t(case.q_bias).to(dt),
                   k_bias=None if case.k_bias is None else t(case.k_bias).to(dt))
    rows, heads, dim = case.q.shape
    ws = torch.empty(ops.decode_workspace_bytes(rows, heads, dim, int(case.seqlens.max()) + 1, case.block_size,
                                                ops.MIN_SPLIT_PAGES) // 4, dtype=torch.float32, device=dev)
    return tensors, ws


def _attend(case, d, ws, rows, cache_layer0=0, stages=None):
    """Decode attention over the batch rows `rows` (indices into the case) through table_row."""
    from continuous_depth_batching_amd import ops

    idx = torch.as_tensor(rows, dtype=torch.long, device="cuda")
    view = ops.KVPoolView(d["pool"], case.block_size)
    q, k, v = d["q"][idx].contiguous(), d["k"][idx].contiguous(), d["v"][idx].contiguous()
    out = torch.empty_like(q)
    ops.paged_decode_attention_raw(
        q, k, v, view.k_ptr, view.v_ptr, view.layer_stride, view.num_cache_layers, view.pool_blocks,
        d["layer"][idx].contiguous(), cache_layer0, d["table"], idx.to(torch.int32), d["seqlens"][idx].contiguous(),
        d["cos"], d["sin"], case.rope_style, d["q_bias"], d["k_bias"], out, ws, case.block_size, ops.ADAPTIVE_SPLIT,
        case.scale,
        **({} if stages is None else {"stages": stages}))
    return out


def test_row_output_is_bit_identical_in_any_batch_composition() -> None:
    # A row's chunks and their merge order depend only on the row: alone, inside the
    # full batch, or inside a shuffled half of it, its output is the same to the bit.
    # 272 rows run the persistent fast form and the merge launch (more than the deep form's
    # 256 rows at 128-wide heads); 136 rows, 30 rows and single rows the deep form, which
    # merges in the decode kernel.
    case = make_case(seed=31, num_rows=272, num_heads=16, num_kv_heads=16, head_dim=128, max_context=1500,
                     rope_style=1, dtype="bf16", padding_rows=3)
    d, ws = _device_case(case)
    full = _attend(case, d, ws, list(range(272)))
    rng = np.random.default_rng(3)
    half = rng.permutation(272)[:136].tolist()
    sub = _attend(case, d, ws, half)
    few = _attend(case, d, ws, half[:30])
    torch.cuda.synchronize()
    assert torch.equal(sub, full[half])
    assert torch.equal(few, full[half[:30]])
    for r in (0, int(np.argmax(case.seqlens)), 50):
        alone = _attend(case, d, ws, [r])
        assert torch.equal(alone[0], full[r])


def test_huginn_shape_row_output_is_bit_identical_in_any_batch_composition() -> None:
    # The same at Huginn-0125's attention shape (55 heads x 96, interleaved RoPE with q/k
    # bias): 150 rows run the persistent fast form, 75 rows and single rows the deep form.
    case = make_case(seed=34, num_rows=150, num_heads=55, num_kv_heads=55, head_dim=96, max_context=700,
                     rope_style=2, dtype="bf16", padding_rows=2, qk_bias=True)
    d, ws = _device_case(case)
    full = _attend(case, d, ws, list(range(150)))
    half = np.random.default_rng(4).permutation(150)[:75].tolist()
    sub = _attend(case, d, ws, half)
    few = _attend(case, d, ws, half[:30])
    torch.cuda.synchronize()
    assert torch.equal(sub, full[half])
    assert torch.equal(few, full[half[:30]])
    for r in (1, int(np.argmax(case.seqlens)), 70):
        assert torch.equal(_attend(case, d, ws, [r])[0], full[r])


FAST_FORM_SHAPES = {
    # name: (dtype, heads, kv_heads, head_dim, rope_style, qk_bias)
    "f32-mha-16x128": ("f32", 16, 16, 128, 1, False),
    "bf16-gqa-8x4x64": ("bf16", 8, 4, 64, 1, False),
    "bf16-huginn-55x96": ("bf16", 55, 55, 96, 2, True),
}


@pytest.mark.parametrize("rows", [96, 272])
@pytest.mark.parametrize("shape", sorted(FAST_FORM_SHAPES))
def test_wide_launches_against_the_oracle(shape: str, rows: int) -> None:
    """Against the float64 oracle: 272 rows (more than the deep form's limit, 256 rows at 128-wide
    heads and 120 at the others, so the persistent fast form with its XCD tail queues, cross-item
    prefetch, LDS stash and merge launch runs) and 96 rows (the deep form, whose last-arriving waves
    merge each row's chunks in the decode kernel). Both
    with padding rows, multi-chunk rows, one row past its block table and one row at a cache layer
    outside the pool: those two get NaN and write nothing, every other row is within the bar and
    its appended K/V row is bit-identical to the oracle's. Two calls run on one workspace, so the
    arrival counters and tail queues the first call leaves must serve the second."""

    dtype, heads, kv_heads, dim, rope_style, bias = FAST_FORM_SHAPES[shape]
    case = make_case(seed=35 + dim + rows, num_rows=rows, num_heads=heads, num_kv_heads=kv_heads, head_dim=dim,
                     max_context=420, rope_style=rope_style, dtype=dtype, padding_rows=5, qk_bias=bias)
    width = case.block_table.shape[1]
    case.seqlens[7] = width * case.block_size  # one past its table
    case.cache_layer[11] = case.kv_pool.shape[0]  # one past the pool's cache layers
    got, got_pool = run_hip(case, 0, repeats=2)
    assert np.isnan(got[7]).all() and np.isnan(got[11]).all()
    case.seqlens[7] = case.seqlens[11] = -1  # as padding for the oracle: no write, no output
    want, want_pool = run_oracle(case)
    live = case.seqlens >= 0
    err = np.abs(got[live] - want[live])
    max_tol, mean_tol = TOL[dtype]
    assert np.isfinite(got[live]).all()
    assert err.max() <= max_tol, f"max err {err.max()}"
    assert err.mean() <= mean_tol, f"mean err {err.mean()}"
    assert np.all(got[-5:] == 0.0)
    np.testing.assert_array_equal(got_pool, want_pool)


def test_plan_once_then_attend_per_layer_matches_planning_every_layer() -> None:
    from continuous_depth_batching_amd import ops

    case = make_case(seed=32, num_rows=40, num_heads=16, num_kv_heads=16, head_dim=128, max_context=900,
                     rope_style=1, dtype="bf16", num_layers=6)
    d, ws = _device_case(case)
    d["layer"] = d["layer"] % 4  # offsets 0..3 over 6 cache layers: bases 0, 1 and 2 are all in range
    rows = list(range(40))
    staged = [_attend(case, d, ws, rows, layer, ops.DECODE_PLAN_AND_ATTEND if layer == 0 else ops.DECODE_ATTEND)
              for layer in (0, 1, 2)]
    fresh = [_attend(case, d, ws, rows, layer) for layer in (0, 1, 2)]
    torch.cuda.synchronize()
    for a, b in zip(staged, fresh):
        assert torch.equal(a, b)
    assert not torch.equal(staged[0], staged[1])  # the layers really differ


def _expected_plan(case, chunk_tokens: int):
    """The chunk plan restated on the host: per row its chunks of chunk_tokens tokens (the last
    one ends at the new token), a descriptor per chunk (row | last flag, token range, position,
    partial slot, chunks in the row, table row, cache-layer offset, the chunk's 8 block ids), full
    chunks first in row order, then last chunks by decreasing ceil(tokens / 32)."""

    bs = case.block_size
    width = case.block_table.shape[1]
    full, last = [], []
    prefix = [0]
    for b, p in enumerate(case.seqlens.tolist()):
        n = (p + chunk_tokens) // chunk_tokens if 0 <= p < width * bs else 0
        for c in range(n):
            t0 = c * chunk_tokens
            is_last = c == n - 1
            page0 = t0 // bs
            ids = [int(case.block_table[b, page0 + j]) if page0 + j < width else -1 for j in range(8)]
            desc = [b | (1 << 30 if is_last else 0), t0, p if is_last else t0 + chunk_tokens, p,
                    prefix[-1] + c, n, b, int(case.cache_layer[b])] + ids
            (last if is_last else full).append(desc)
        prefix.append(prefix[-1] + n)
    key = lambda d: min((d[3] + 1 - d[1] + 31) // 32, 63)
    return prefix, full, last, key


def test_plan_descriptors_match_a_host_restatement() -> None:
    from continuous_depth_batching_amd import ops

    case = make_case(seed=33, num_rows=40, num_heads=16, num_kv_heads=16, head_dim=128, max_context=1300,
                     rope_style=1, dtype="bf16", padding_rows=2)
    width = case.block_table.shape[1]
    case.seqlens[5] = width * case.block_size  # one row past its table: no chunks
    d, ws = _device_case(case)
    d["seqlens"] = torch.from_numpy(case.seqlens).cuda()
    ws.fill_(float("nan"))
    rows = list(range(40))
    _attend(case, d, ws, rows, stages=ops.DECODE_PLAN)
    torch.cuda.synchronize()
    words = ws.view(torch.int32).cpu().numpy()
    chunk_tokens = ops.MIN_SPLIT_PAGES * case.block_size
    prefix, full, last, key = _expected_plan(case, chunk_tokens)
    assert words[0] == chunk_tokens
    np.testing.assert_array_equal(words[1:42], prefix)
    header_ints = (((40 + 2) * 4 + 255) // 256 * 256 + 1024 + 40 * 16 * 4) // 4  # prefix, queues, arrivals
    got = words[header_ints:header_ints + 16 * (len(full) + len(last))].reshape(-1, 16).tolist()
    assert got[:len(full)] == full  # full chunks in row order
    tail = got[len(full):]
    # Last chunks by decreasing length key; within a key the order is free.
    assert [key(x) for x in tail] == sorted((key(x) for x in last), reverse=True)
    assert sorted(map(tuple, tail)) == sorted(map(tuple, last))
