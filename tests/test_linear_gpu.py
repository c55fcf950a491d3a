"""Decode-batch projection kernel (cdb_linear) against float32 matmul.

The kernel sums in fp32 over all of K and rounds once, so each output must be
the bf16 rounding of the exact product up to the last bit (a different fp32
summation order may flip a rounding that sits within fp32 noise of a tie).
The gated form follows torch's bf16 chain: g and u rounded, silu rounded,
product rounded.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [  # (in_features, out_features): Ouro-1.4B QKV, O, down; Huginn-0125 QKV, adapter; one- and two-wave K
    (2048, 6144), (2048, 2048), (5632, 2048), (5280, 15840), (10560, 5280), (64, 32), (32, 16)]
ROWS = [1, 5, 16, 17, 32, 33, 48, 64]


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 values at |x| (8 significant bits)."""

    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126)))
    return torch.exp2(e - 7)


def _inputs(rows: int, k: int, n: int, seed: int):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((rows, k), generator=g, device="cuda").bfloat16()
    w = (torch.randn((n, k), generator=g, device="cuda") * 0.02).bfloat16()
    return x, w


def _sum_error(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Bound on fp32 summation-order differences: 2^-22 * sum_k |x_k w_k| (it only matters
    for results that nearly cancel)."""

    return (x.float().abs() @ w.float().abs().t()) * 2.0 ** -22


def _check_rounded(y: torch.Tensor, ref: torch.Tensor, *, max_mismatch: float, extra: torch.Tensor) -> None:
    """y within one bf16 step of ref plus `extra`; at most max_mismatch of y differs from bf16(ref)."""

    exact = ref.bfloat16()
    diff = (y.float() - exact.float()).abs()
    tol = _bf16_ulp(ref) * 1.0001 + extra
    assert (diff <= tol).all(), f"max excess {(diff - tol).max().item()}"
    assert (y != exact).float().mean().item() <= max_mismatch


@pytest.mark.parametrize("k,n", SHAPES)
@pytest.mark.parametrize("rows", ROWS)
def test_linear_matches_rounded_fp32_product(rows: int, k: int, n: int) -> None:
    from continuous_depth_batching_amd import ops

    x, w = _inputs(rows, k, n, seed=rows * 7 + k)
    y = torch.empty((rows, n), dtype=torch.bfloat16, device="cuda")
    ops.linear_raw(x, ops.pack_linear_weight(w), y)
    torch.cuda.synchronize()
    ref = x.float() @ w.float().t()
    _check_rounded(y, ref, max_mismatch=0.01, extra=_sum_error(x, w))


@pytest.mark.parametrize("rows,k,n", [(r, 2048, n) for r in (33, 65, 96, 128, 129, 200, 256) for n in (6144, 4096)]
                         + [(r, 5280, 15840) for r in (65, 100, 128)])
def test_wide_tile_path_matches_rounded_fp32_product(rows: int, k: int, n: int) -> None:
    """Batches above 32 rows with 2048-wide inputs and 4096+ outputs take the wide-tile kernel."""

    from continuous_depth_batching_amd import ops

    x, w = _inputs(rows, k, n, seed=rows + n)
    y = torch.empty((rows, n), dtype=torch.bfloat16, device="cuda")
    ops.linear_raw(x, ops.pack_linear_weight(w), y)
    torch.cuda.synchronize()
    _check_rounded(y, x.float() @ w.float().t(), max_mismatch=0.01, extra=_sum_error(x, w))


@pytest.mark.parametrize("rows", [1, 16, 20, 48, 64, 65, 100, 128, 129, 200, 256])
@pytest.mark.parametrize("k,f", [(2048, 5632), (5280, 17920), (64, 16)])
def test_gated_linear_follows_bf16_silu_chain(rows: int, k: int, f: int) -> None:
    from continuous_depth_batching_amd import ops

    if rows > ops.LINEAR_MAX_ROWS and not ops.linear_prefers_kernel(rows, f, True, k):
        pytest.skip("above 64 rows only the wide-tile shapes run on cdb_linear")

    x, w = _inputs(rows, k, 2 * f, seed=rows + f)
    y = torch.empty((rows, f), dtype=torch.bfloat16, device="cuda")
    ops.linear_raw(x, ops.pack_linear_weight(w), y, gated=True)
    torch.cuda.synchronize()
    gu = (x.float() @ w.float().t()).bfloat16().float()
    g, u = gu[:, :f], gu[:, f:]
    act = (g * torch.sigmoid(g)).bfloat16().float()
    ref = act * u
    # A g or u rounding that flips (see above) moves g or u by one bf16 step, which
    # propagates through silu(g) * u (|silu'| < 1.1); all else matches the chain exactly.
    err = _sum_error(x, w)
    dg = _bf16_ulp(g) + err[:, :f]
    du = _bf16_ulp(u) + err[:, f:]
    _check_rounded(y, ref, max_mismatch=0.02, extra=1.1 * u.abs() * dg + (act.abs() + dg) * du)
    # And the unfused path (torch.mm + cdb_silu_mul) agrees to the same bar.
    unfused = torch.empty_like(y)
    ops.silu_mul_raw(torch.mm(x, w.t()), unfused)
    torch.cuda.synchronize()
    assert ((y.float() - unfused.float()).abs() <= 2 * _bf16_ulp(ref) + 1e-6).float().mean().item() >= 0.98


@pytest.mark.parametrize("rows", [16, 100, 256])
def test_fused_silu_gives_torch_bits_for_every_normal_bf16_gate(rows: int) -> None:
    """One-hot x rows pick single weights, so every gate accumulator is exactly one bf16
    weight and every up value exactly 1, and each output is the SiLU of that bf16 value
    alone. Across the batch every finite normal bf16 value (and +0) is a gate once; each
    output must equal torch's bf16 SiLU bit for bit (the row kernel at 16 rows, the
    pipelined wide-tile forms at 100 and 256)."""

    from continuous_depth_batching_amd import ops

    f, k = 5632, 2048
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    exponent = (bits >> 7) & 0xFF
    values = bits[(exponent != 0) & (exponent != 0xFF)]   # finite normal values of both signs
    values = np.concatenate([[np.uint16(0)], values])      # and +0
    assert len(values) <= rows * f
    gates = np.zeros(rows * f, dtype=np.uint16)
    gates[:len(values)] = values
    gate = torch.from_numpy(gates.view(np.int16)).view(torch.bfloat16).reshape(rows, f).cuda()
    w = torch.zeros((2 * f, k), dtype=torch.bfloat16, device="cuda")
    w[:f, :rows] = gate.t()                                # w_gate[n, r] = gate[r, n]
    w[f:, :rows] = 1.0                                     # w_up[n, r] = 1
    x = torch.zeros((rows, k), dtype=torch.bfloat16, device="cuda")
    x[torch.arange(rows), torch.arange(rows)] = 1.0        # x[r] = e_r
    y = torch.empty((rows, f), dtype=torch.bfloat16, device="cuda")
    ops.linear_raw(x, ops.pack_linear_weight(w), y, gated=True)
    want = torch.nn.functional.silu(gate)
    torch.cuda.synchronize()
    differ = y.view(torch.int16) != want.view(torch.int16)
    assert not bool(differ.any()), f"{int(differ.sum())} gates differ, e.g. {gate[differ][:4].tolist()}"


def test_linear_strided_operands_and_determinism() -> None:
    from continuous_depth_batching_amd import ops

    rows, k, n = 24, 2048, 2048
    x_big, w = _inputs(rows, 3 * k, n, seed=5)
    x = x_big[:, k:2 * k]                   # row stride 3K
    w_big = torch.zeros((n, k + 64), dtype=torch.bfloat16, device="cuda")
    w_big[:, :k] = w[:, :k]
    w_view = w_big[:, :k]                   # row stride K + 64
    y_big = torch.full((rows, n + 16), 7.0, dtype=torch.bfloat16, device="cuda")
    y = y_big[:, :n]
    packed = ops.pack_linear_weight(w_view)
    assert torch.equal(packed, ops.pack_linear_weight(w[:, :k].contiguous()))  # the pack honours the row stride
    ops.linear_raw(x, packed, y)
    again = torch.empty((rows, n), dtype=torch.bfloat16, device="cuda")
    ops.linear_raw(x.contiguous(), packed, again)
    torch.cuda.synchronize()
    assert torch.equal(y, again)            # strides change no arithmetic; repeat runs are bit-identical
    assert (y_big[:, n:] == 7.0).all()      # columns past out_features untouched
    wk = w[:, :k]
    _check_rounded(y, x.float() @ wk.float().t(), max_mismatch=0.01, extra=_sum_error(x, wk))


def test_linear_op_dispatch_matches_torch_above_the_row_limit() -> None:
    from continuous_depth_batching_amd import ops

    x, w = _inputs(ops.LINEAR_MAX_ROWS + 8, 2048, 2048, seed=9)
    packed = ops.pack_linear_weight(w)
    y = torch.ops.cdb.linear(x, w, packed, False)
    torch.cuda.synchronize()
    assert torch.equal(y, torch.mm(x, w.t()))
    assert torch.equal(torch.ops.cdb.linear(x[:8], w, None, False), torch.mm(x[:8], w.t()))
    small = torch.ops.cdb.linear(x[:8], w, packed, False)
    torch.cuda.synchronize()
    _check_rounded(small, x[:8].float() @ w.float().t(), max_mismatch=0.01, extra=_sum_error(x[:8], w))


@pytest.mark.parametrize("n,k", [(32, 64), (2048, 2048), (48, 5632)])
def test_pack_layout_is_the_mfma_operand_order(n: int, k: int) -> None:
    """Unit l of the 1 KiB block (tile t, step s) holds w[16 t + l % 16][32 s + 8 (l // 16) .. +8]."""

    from continuous_depth_batching_amd import ops

    w = torch.randn((n, k), device="cuda").bfloat16()
    packed = ops.pack_linear_weight(w)
    torch.cuda.synchronize()
    expected = w.view(n // 16, 16, k // 32, 4, 8).permute(0, 2, 3, 1, 4).reshape(-1)
    assert torch.equal(packed, expected)


PARTS_CASES = [(r, k, n) for r in (1, 5, 16, 32, 33, 64, 65, 128) for k, n in ((2048, 2048), (5632, 2048))] + [
    (r, 5632, n) for r in (129, 200, 256) for n in (2048, 64)] + [(40, 2048, 1024), (3, 5632, 192)] + [
    # Huginn O and down: 5280 output columns end in a half-full 64-column range; 80 columns
    # leave the last range one 16-column tile wide.
    (r, 5280, 5280) for r in (1, 16, 40, 64, 100, 128, 256)] + [
    (r, 17920, 5280) for r in (1, 33, 128, 256)] + [(20, 5280, 80), (70, 17920, 112)]


@pytest.mark.parametrize("rows,k,n", PARTS_CASES)
def test_split_k_partials_sum_to_the_fp32_product(rows: int, k: int, n: int) -> None:
    from continuous_depth_batching_amd import ops

    splits = ops.linear_parts_splits(rows, n, k)
    assert splits in (2, 3, 4, 8)
    x, w = _inputs(rows, k, n, seed=rows * 11 + k + n)
    parts = torch.full((splits, rows, n), float("nan"), device="cuda")
    ops.linear_parts_raw(x, ops.pack_linear_weight(w), parts)
    torch.cuda.synchronize()
    # Each partial is its K range's fp32 product, up to summation order: both sides
    # chain a few dozen fp32 additions, so allow 2^-16 * sum |x_k w_k| -- about 1/60 of
    # one average product term over a 1024-wide range, so a dropped or repeated
    # K step still fails.
    width = k // splits
    for s in range(splits):
        xs, ws = x[:, s * width:(s + 1) * width], w[:, s * width:(s + 1) * width]
        ref = xs.float() @ ws.float().t()
        tol = (xs.float().abs() @ ws.float().abs().t()) * 2.0 ** -16
        assert ((parts[s] - ref).abs() <= tol).all(), f"split {s}: max excess {((parts[s] - ref).abs() - tol).max()}"
    total = parts[0].clone()
    for s in range(1, splits):
        total += parts[s]
    _check_rounded(total.bfloat16(), x.float() @ w.float().t(), max_mismatch=0.01, extra=_sum_error(x, w))


def test_wide_tile_forms_give_a_row_the_same_bits_in_any_batch() -> None:
    """Every wide-tile form adds an output's K steps in order in one accumulator, so a
    row's result does not depend on its batch: 48 rows (two-tile row ranges), 100 rows
    (four-tile; the gated one reads x ahead of its MFMAs) and 256 rows (eight-tile gated
    and down forms, both reading x ahead) agree bit for bit, for the gated projection and
    for the split-K partials. A dropped, repeated or reordered K step in one form fails."""

    from continuous_depth_batching_amd import ops

    x, w = _inputs(256, 2048, 2 * 5632, seed=31)
    packed = ops.pack_linear_weight(w)
    xd, wd = _inputs(256, 5632, 2048, seed=37)
    packed_d = ops.pack_linear_weight(wd)
    gated, parts = {}, {}
    for rows in (48, 100, 256):
        gated[rows] = torch.empty((rows, 5632), dtype=torch.bfloat16, device="cuda")
        ops.linear_raw(x[:rows], packed, gated[rows], gated=True)
        parts[rows] = torch.full((ops.linear_parts_splits(rows, 2048, 5632), rows, 2048), float("nan"), device="cuda")
        ops.linear_parts_raw(xd[:rows], packed_d, parts[rows])
    torch.cuda.synchronize()
    assert torch.equal(gated[256][:100], gated[100]) and torch.equal(gated[100][:48], gated[48])
    assert parts[48].shape[0] == parts[256].shape[0] == 4
    assert torch.equal(parts[256][:, :100], parts[100]) and torch.equal(parts[100][:, :48], parts[48])
    gu = (x[:256].float() @ w.float().t()).bfloat16().float()
    g, u = gu[:, :5632], gu[:, 5632:]
    ref = (g * torch.sigmoid(g)).bfloat16().float() * u
    assert ((gated[256].float() - ref).abs() <= 2 * _bf16_ulp(ref) + 1e-3).float().mean().item() >= 0.99


@pytest.mark.parametrize("rows,k,n", [(1, 2048, 2048), (16, 5632, 2048), (33, 2048, 2048), (96, 5632, 2048),
                                      (128, 2048, 2048), (256, 5632, 2048), (7, 5280, 5280), (128, 17920, 5280)])
def test_norm_from_partials_is_the_two_step_result(rows: int, k: int, n: int) -> None:
    """Partials added in order and rounded once, then the sandwich norm: bit-identical to
    running the fused norm on that rounded projection output."""

    from continuous_depth_batching_amd import ops

    x, w = _inputs(rows, k, n, seed=rows + 3 * k)
    g = torch.Generator(device="cuda")
    g.manual_seed(rows)
    residual = torch.randn((rows, n), generator=g, device="cuda").bfloat16()
    w_a = (1 + 0.1 * torch.randn(n, generator=g, device="cuda")).bfloat16()
    w_b = (1 + 0.1 * torch.randn(n, generator=g, device="cuda")).bfloat16()
    packed = ops.pack_linear_weight(w)
    for mode in (ops.NORM_OURO_SANDWICH, ops.NORM_HUGINN_SANDWICH):
        h, y = ops.linear_residual_rmsnorm_auto(x, w, packed, residual, w_a, w_b, 1e-6, 1e-5, mode)
        splits = ops.linear_parts_splits(rows, n, k)
        parts = torch.empty((splits, rows, n), device="cuda")
        ops.linear_parts_raw(x, packed, parts)
        o = parts[0].clone()
        for s in range(1, splits):
            o += parts[s]
        h_ref, y_ref = torch.ops.cdb.residual_rmsnorm(o.bfloat16(), residual, w_a, w_b, 1e-6, 1e-5, mode)
        torch.cuda.synchronize()
        assert torch.equal(h, h_ref) and torch.equal(y, y_ref)
        h2, y2 = ops.linear_residual_rmsnorm_auto(x, w, packed, residual, w_a, w_b, 1e-6, 1e-5, mode)
        assert torch.equal(h, h2) and torch.equal(y, y2)
        h3, y3 = ops.linear_residual_rmsnorm_auto(x, w, packed, residual, w_a, None, 1e-6, 1e-5, mode)
        torch.cuda.synchronize()
        assert y3 is None and torch.equal(h3, h_ref)


def test_linear_residual_rmsnorm_falls_back_without_a_split_form() -> None:
    from continuous_depth_batching_amd import ops

    rows, k, n = 160, 2048, 2048  # a 2048-wide input above 128 rows has no split form
    assert ops.linear_parts_splits(rows, n, k) == 0
    x, w = _inputs(rows, k, n, seed=5)
    residual = torch.randn((rows, n), device="cuda").bfloat16()
    w_a = torch.ones(n, device="cuda").bfloat16()
    h, y = torch.ops.cdb.linear_residual_rmsnorm(x, w, ops.pack_linear_weight(w), residual, w_a, w_a, 1e-6, 1e-6,
                                                 ops.NORM_OURO_SANDWICH)
    h_ref, y_ref = torch.ops.cdb.residual_rmsnorm(torch.mm(x, w.t()), residual, w_a, w_a, 1e-6, 1e-6,
                                                  ops.NORM_OURO_SANDWICH)
    torch.cuda.synchronize()
    assert torch.equal(h, h_ref) and torch.equal(y, y_ref)


@pytest.mark.parametrize("rows", [1, 5, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("k,n", [(2048, 49152), (2048, 1024), (64, 32)])
def test_fused_lm_head_argmax_equals_argmax_of_the_logits(rows: int, k: int, n: int) -> None:
    """cdb_linear_argmax picks exactly what torch.argmax picks on the projection kernel's bf16 logits."""

    from continuous_depth_batching_amd import ops

    x, w = _inputs(rows, k, n, seed=rows * 3 + n)
    packed = ops.pack_linear_weight(w)
    logits = torch.empty((rows, n), dtype=torch.bfloat16, device="cuda")
    ops.linear_raw(x, packed, logits)
    out = torch.full((rows,), -7, dtype=torch.int64, device="cuda")
    ws = torch.empty((rows * (n // 16) * 2,), dtype=torch.float32, device="cuda")
    ops.linear_argmax_raw(x, packed, out, ws)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.argmax(logits, dim=-1))
    assert torch.equal(out, ops.argmax_rows(logits))


def test_fused_lm_head_argmax_ties_and_nans_follow_torch() -> None:
    from continuous_depth_batching_amd import ops

    rows, k, n = 8, 2048, 49152
    x, w = _inputs(rows, k, n, seed=11)
    # Columns 100 and 5000 get the same weight row, aligned with every x row: a tie at
    # the maximum, which the first column wins.
    w[100] = (x.float().sum(0) * 0.01).bfloat16()
    w[5000] = w[100]
    packed = ops.pack_linear_weight(w)
    out = torch.empty((rows,), dtype=torch.int64, device="cuda")
    ws = torch.empty((rows * (n // 16) * 2,), dtype=torch.float32, device="cuda")
    ops.linear_argmax_raw(x, packed, out, ws)
    logits = torch.empty((rows, n), dtype=torch.bfloat16, device="cuda")
    ops.linear_raw(x, packed, logits)
    torch.cuda.synchronize()
    assert torch.equal(logits[:, 100], logits[:, 5000])
    assert torch.equal(out, torch.argmax(logits, dim=-1)) and (out == 100).all()
    # NaN logits count as the maximum; the first NaN column wins.
    w[30000] = float("nan")
    w[7001] = float("nan")
    packed = ops.pack_linear_weight(w)
    ops.linear_argmax_raw(x, packed, out, ws)
    torch.cuda.synchronize()
    assert (out == 7001).all()


def test_lm_head_argmax_routes_large_batches_through_the_logits() -> None:
    from continuous_depth_batching_amd import ops

    x, w = _inputs(48, 2048, 49152, seed=2)
    packed = ops.pack_linear_weight(w)
    tokens = ops.lm_head_argmax(x, w, packed)
    torch.cuda.synchronize()
    assert torch.equal(tokens, ops.argmax_rows(ops.linear_auto(x, w, packed, False)))
    small = ops.lm_head_argmax(x[:16], w, packed)
    logits = torch.empty((16, 49152), dtype=torch.bfloat16, device="cuda")
    ops.linear_raw(x[:16], packed, logits)
    torch.cuda.synchronize()
    assert torch.equal(small, torch.argmax(logits, dim=-1))


@pytest.mark.parametrize("rows", [1, 7, 16, 32, 48])
def test_coda_writes_the_successors_prelude(rows: int) -> None:
    """With an embedding table, rows with a successor slot get embed[token] in that bank row
    (fused into the argmax pass up to 32 rows, a row copy above); other bank rows keep their bits."""

    from continuous_depth_batching_amd import ops

    vocab, width = 49152, 2048
    x, w = _inputs(rows, width, vocab, seed=rows + 17)
    packed = ops.pack_linear_weight(w)
    g = torch.Generator(device="cuda")
    g.manual_seed(rows)
    embed = torch.randn((vocab, width), generator=g, device="cuda").bfloat16()
    bank = torch.randn((4 * rows + 8, width), generator=g, device="cuda").bfloat16()
    before = bank.clone()
    slots = torch.full((rows,), -1, dtype=torch.int64, device="cuda")
    with_successor = torch.arange(0, rows, 2, device="cuda")
    targets = 2 * rows + 3 + with_successor   # distinct rows away from anything else
    slots[with_successor] = targets
    tokens = ops.lm_head_argmax(x, w, packed, embed=embed, bank=bank, bank_slots=slots)
    plain = ops.lm_head_argmax(x, w, packed)
    torch.cuda.synchronize()
    assert torch.equal(tokens, plain)
    want = before.clone()
    want[targets] = embed[tokens[with_successor]]
    assert torch.equal(bank, want)
