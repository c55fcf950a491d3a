"""Pins of the oracle's prefill attention, gate logits and float32 sigmoid.

* ``prefill_attention`` (the checker of the MFMA prefill kernel): torch's
  scaled_dot_product_attention over K/V gathered through the block table, with a past prefix
  (bottom-right causal alignment) and grouped KV heads; closed forms (a fresh one-token
  sequence returns its value; identical keys give the mean of the visible values); invariance
  under a permutation of physical pages with the table remapped.
* ``gate_logits`` (the exit gate's Linear(E, 1) in the model dtype): F.linear in float64,
  rounded to bf16; and torch's own bf16 F.linear within one bf16 step.
* ``sigmoid_f32`` (the hazard of the exit policy): torch.sigmoid in float32 within four ulp over
  +-30 (the bound of a three-op float32 formula); exact values at 0 and the saturated tails;
  symmetry; monotonicity; and the bf16 path
  (torch.sigmoid of a bf16 tensor, as the reference's synchronous exit path computes it) equal
  to rounding the float32 result to bf16 on every bf16 value in [-30, 30].
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.bf16 import round_bf16
from oracle.paged_attention import prefill_attention, read_rows
from oracle.stage import gate_logits, sigmoid_f32


def prefill_case(seed: int, *, lens, past, heads=4, kv_heads=2, dim=32, block=16):
    rng = np.random.default_rng(seed)
    lens, past = np.asarray(lens), np.asarray(past)
    totals = lens + past
    pages = [-(-int(t) // block) for t in totals]
    width = max(pages)
    num_pages = sum(pages) + 3
    perm = rng.permutation(num_pages)
    table = np.full((len(lens), width), -1, np.int32)
    k = 0
    for s, n in enumerate(pages):
        table[s, :n] = perm[k:k + n]
        k += n
    pool = rng.standard_normal((2, 2, num_pages * block, kv_heads, dim)).astype(np.float32)
    q = rng.standard_normal((int(lens.sum()), heads, dim)).astype(np.float32)
    cu_q = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    return q, pool, table, np.arange(len(lens)), cu_q, past, block, dim ** -0.5


def sdpa_reference(q, pool, layer, table, cu_q, past, block, scale):
    out = np.zeros_like(q, dtype=np.float64)
    heads, kv_heads = q.shape[1], pool.shape[3]
    for s in range(len(past)):
        b, e = int(cu_q[s]), int(cu_q[s + 1])
        total = int(past[s]) + e - b
        rows = read_rows(table[s], total, block)
        k = torch.from_numpy(pool[layer, 0, rows]).double().transpose(0, 1)  # [Hkv, T, D]
        v = torch.from_numpy(pool[layer, 1, rows]).double().transpose(0, 1)
        k = k.repeat_interleave(heads // kv_heads, 0)
        v = v.repeat_interleave(heads // kv_heads, 0)
        qs = torch.from_numpy(q[b:e]).double().transpose(0, 1)  # [H, n, D]
        # Query i sits at position past + i and sees keys 0 .. past + i (bottom-right alignment).
        mask = torch.arange(total)[None, :] <= (int(past[s]) + torch.arange(e - b))[:, None]
        o = F.scaled_dot_product_attention(qs, k, v, attn_mask=mask, scale=scale)
        out[b:e] = o.transpose(0, 1).numpy()
    return out


@pytest.mark.parametrize("seed,lens,past", [(0, [5, 17, 33], [0, 0, 0]), (1, [3, 20, 1], [40, 7, 63]),
                                            (2, [64], [100]), (3, [1, 1, 2], [0, 15, 16])])
def test_prefill_attention_matches_sdpa_with_past_and_grouped_heads(seed, lens, past) -> None:
    q, pool, table, rows, cu_q, past, block, scale = prefill_case(seed, lens=lens, past=past)
    got = prefill_attention(q, pool, 1, table, rows, cu_q, past, block, scale, dtype="f32")
    want = sdpa_reference(q, pool, 1, table, cu_q, past, block, scale)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6)


def test_prefill_attention_fresh_single_token_returns_its_value() -> None:
    q, pool, table, rows, cu_q, past, block, scale = prefill_case(4, lens=[1, 1, 1], past=[0, 0, 0])
    got = prefill_attention(q, pool, 0, table, rows, cu_q, past, block, scale, dtype="f32")
    for s in range(3):
        v = pool[0, 1, read_rows(table[s], 1, block)[0]]  # [Hkv, D]
        np.testing.assert_allclose(got[s], np.repeat(v, 2, axis=0), atol=1e-6)


def test_prefill_attention_identical_keys_average_the_visible_values() -> None:
    q, pool, table, rows, cu_q, past, block, scale = prefill_case(5, lens=[6, 9], past=[11, 0])
    pool[:, 0] = 0.25
    got = prefill_attention(q, pool, 0, table, rows, cu_q, past, block, scale, dtype="f32")
    for s in range(2):
        vals = pool[0, 1, read_rows(table[s], int(past[s] + cu_q[s + 1] - cu_q[s]), block)]
        for i in range(int(cu_q[s + 1] - cu_q[s])):
            mean = vals[: int(past[s]) + i + 1].mean(axis=0)  # the query itself is visible, later keys are not
            np.testing.assert_allclose(got[cu_q[s] + i], np.repeat(mean, 2, axis=0), atol=1e-5)


def test_prefill_attention_is_invariant_to_page_placement() -> None:
    q, pool, table, rows, cu_q, past, block, scale = prefill_case(6, lens=[7, 30], past=[25, 3])
    got = prefill_attention(q, pool, 0, table, rows, cu_q, past, block, scale, dtype="f32")
    num_pages = pool.shape[2] // block
    perm = np.random.default_rng(7).permutation(num_pages)
    paged = pool.reshape(2, 2, num_pages, block, *pool.shape[3:])
    moved = np.empty_like(paged)
    moved[:, :, perm] = paged
    table2 = np.where(table >= 0, perm[np.maximum(table, 0)], -1).astype(np.int32)
    again = prefill_attention(q, moved.reshape(pool.shape), 0, table2, rows, cu_q, past, block, scale, dtype="f32")
    np.testing.assert_array_equal(got, again)


def test_gate_logits_is_the_bf16_rounded_linear() -> None:
    rng = np.random.default_rng(8)
    hidden = round_bf16(rng.standard_normal((64, 2048)).astype(np.float32))
    weight = round_bf16((rng.standard_normal(2048) * 0.02).astype(np.float32))
    bias = float(round_bf16(np.array([0.013], np.float32))[0])
    got = gate_logits(hidden, weight, bias, "bf16")
    exact = F.linear(torch.from_numpy(hidden).double(), torch.from_numpy(weight).double()[None],
                     torch.tensor([bias], dtype=torch.float64))[:, 0]
    np.testing.assert_array_equal(got, exact.float().bfloat16().float().numpy())
    # torch's own bf16 linear differs by its accumulation order only: at most one bf16 step.
    lib = F.linear(torch.from_numpy(hidden).bfloat16(), torch.from_numpy(weight).bfloat16()[None],
                   torch.tensor([bias]).bfloat16())[:, 0].float().numpy()
    step = np.abs(got) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(lib - got) <= step)
    # A transposed or dropped bias would move most outputs by far more than a step.
    assert np.mean(got != gate_logits(hidden, weight, 0.0, "bf16")) > 0.5


def test_sigmoid_f32_matches_torch_over_the_gate_range() -> None:
    x = np.linspace(-30.0, 30.0, 200001, dtype=np.float32)
    got = np.array([sigmoid_f32(float(v)) for v in x[::7]], np.float32)
    want = torch.sigmoid(torch.from_numpy(x[::7])).numpy()
    # 1 / (1 + exp(-x)) in float32 (the exit kernel's formula) carries exp's error plus two
    # roundings: within 4 ulp of torch's sigmoid everywhere, and bit-equal at most inputs.
    ulp = np.spacing(np.maximum(np.abs(want), np.float32(1e-38)))
    assert np.all(np.abs(got - want) <= 4 * ulp)
    assert np.mean(got == want) > 0.8
    assert sigmoid_f32(0.0) == 0.5
    assert sigmoid_f32(30.0) == 1.0 and 0.0 < sigmoid_f32(-30.0) < 1e-12
    pos = np.array([sigmoid_f32(float(v)) for v in x[100001::97]])
    neg = np.array([sigmoid_f32(-float(v)) for v in x[100001::97]])
    assert np.all(np.abs(pos + neg - 1.0) <= 2 * np.spacing(np.float32(1.0)))
    assert np.all(np.diff(got) >= 0)


def test_sigmoid_f32_rounded_to_bf16_is_torchs_bf16_sigmoid() -> None:
    # Every bf16 value in [-30, 30]: the synchronous exit path takes sigmoid of the bf16 gate logit.
    bits = np.arange(0, 1 << 16, dtype=np.uint32) << 16
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) <= 30.0)]
    got = round_bf16(np.array([sigmoid_f32(float(v)) for v in vals], np.float32))
    want = torch.sigmoid(torch.from_numpy(vals).bfloat16()).float().numpy()
    mismatch = np.flatnonzero(got != want)
    assert mismatch.size == 0, f"{mismatch.size} bf16 inputs differ, e.g. {vals[mismatch[:5]]}"
