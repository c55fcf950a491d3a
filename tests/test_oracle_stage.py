"""Pin the row-wise stage oracle (norms, gating, argmax, exit policy, exit-KV copy)."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import stage
from oracle.bf16 import round_bf16

GOLDEN = Path(__file__).parent / "golden"


def test_rmsnorm_matches_torch_rms_norm() -> None:
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    w = rng.standard_normal(256).astype(np.float32)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (256,), torch.from_numpy(w).double(), 1e-6)
    np.testing.assert_allclose(stage.rmsnorm(x, w, 1e-6, "f32"), want.numpy(), rtol=2e-6, atol=2e-6)


def test_rmsnorm_bf16_rounds_before_the_weight_product() -> None:
    """bf16 RMSNorm = R(w * R(x * inv)), as OuroRMSNorm computes it in bf16."""

    rng = np.random.default_rng(1)
    x = round_bf16(rng.standard_normal((4, 64)).astype(np.float32))
    w = round_bf16(rng.standard_normal(64).astype(np.float32))
    xt = torch.from_numpy(x).bfloat16()
    wt = torch.from_numpy(w).bfloat16()
    xf = xt.float()
    normed = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)
    want = (wt * normed.to(torch.bfloat16)).float().numpy()
    got = stage.rmsnorm(x, w, 1e-6, "bf16")
    assert np.mean(got == want) > 0.99
    np.testing.assert_allclose(got, want, rtol=1e-2)


def test_sandwiches_order_residual_and_norm_as_the_layers_do() -> None:
    rng = np.random.default_rng(2)
    x, r = rng.standard_normal((2, 3, 128)).astype(np.float32)
    wa, wb = rng.standard_normal((2, 128)).astype(np.float32)
    h, y = stage.ouro_sandwich(x, r, wa, wb, 1e-6, "f32")
    np.testing.assert_allclose(h, r + stage.rmsnorm(x, wa, 1e-6, "f32"), rtol=1e-6)
    np.testing.assert_allclose(y, stage.rmsnorm(h, wb, 1e-6, "f32"), rtol=1e-6)
    h2, _ = stage.huginn_sandwich(x, r, wa, wb, 1e-6, "f32")
    np.testing.assert_allclose(h2, stage.rmsnorm(x + r, wa, 1e-6, "f32"), rtol=1e-6)


def test_silu_mul_matches_torch() -> None:
    gu = np.random.default_rng(3).standard_normal((4, 64)).astype(np.float32) * 4
    g, u = torch.from_numpy(gu).chunk(2, dim=-1)
    np.testing.assert_allclose(stage.silu_mul(gu, "f32"), (torch.nn.functional.silu(g) * u).numpy(), rtol=1e-5,
                               atol=1e-6)


def test_argmax_takes_the_first_maximum() -> None:
    logits = np.array([[1.0, 3.0, 3.0, 0.0], [5.0, 5.0, 5.0, 5.0]], np.float32)
    assert stage.argmax(logits).tolist() == [1, 0]
    np.testing.assert_array_equal(stage.argmax(logits), torch.from_numpy(logits).argmax(-1).numpy())


def test_exit_policy_golden_vectors() -> None:
    data = json.loads((GOLDEN / "exit_policy.json").read_text())
    for seq in data["sequences"]:
        policy = stage.TokenPolicy()
        for step, (signal, want) in enumerate(zip(seq["signals"], seq["expected"])):
            if seq.get("signal_dtype") == "bf16":
                signal = float(round_bf16(np.array([signal], np.float32))[0])
            got = policy.consume(rule=seq["rule"], signal=signal, source_step=step, threshold=seq["threshold"],
                                 min_steps=seq["min_steps"])
            assert got == want, (seq, step)
        if "final_cdf" in seq:
            assert policy.exit_cdf == pytest.approx(seq["final_cdf"])
            assert policy.survival == pytest.approx(seq["final_survival"])


def test_forced_final_step_and_synthetic_replay() -> None:
    kw = dict(max_steps=4, policy=None, signal=None, rule="hazard", threshold=None, min_steps=1)
    assert stage.decide_exit(step=3, synthetic_depth=None, **kw)
    assert not stage.decide_exit(step=1, synthetic_depth=2, **kw)
    assert stage.decide_exit(step=2, synthetic_depth=2, **kw)
    assert stage.decide_exit(step=2, synthetic_depth=0, **kw)


def test_exit_copy_groups_match_reference_layout_vectors() -> None:
    """Reference tests/test_looped_kv_layout.py:94-107 on its Huginn layout (2 prelude
    layers, 4 core layers, 4 last_exited slots): core layer l at step s is cache
    layer 2 + 4*s + l, and an exit at step 1 feeds slots 2 and 3; step 3 feeds none."""

    assert stage.exit_copy_groups(1, 4, 4, layer_base=2) == [
        (2 + 4 + l, [2 + 8 + l, 2 + 12 + l]) for l in range(4)
    ]
    assert stage.exit_copy_groups(3, 4, 4, layer_base=2) == []


def test_latent_difference_is_relative_l2() -> None:
    h = np.array([[3.0, 4.0]], np.float32)
    prev = np.array([[0.0, 4.0]], np.float32)
    assert stage.latent_diff(h, prev, "f32")[0] == pytest.approx(3.0 / 5.0)
    assert stage.latent_diff(h, h, "f32")[0] == 0.0


def _torch_latent_diff(h: np.ndarray, p: np.ndarray) -> np.ndarray:
    """huginn/exit_gates.py:33-40 run by torch on bf16 tensors."""

    th, tp = torch.from_numpy(h).bfloat16(), torch.from_numpy(p).bfloat16()
    return ((th - tp).norm(dim=-1) / th.norm(dim=-1).clamp_min(1e-9)).float().numpy()


@pytest.mark.parametrize("scale", [1e-3, 1.0, 30.0])
def test_latent_difference_bf16_equals_torch_bf16(scale: float) -> None:
    """The bf16 rounding points R(R(||R(h - p)||) / max(R(||h||), R(1e-9))) are torch's own.
    On 3000 rows 5280 wide (Huginn-0125's state), the oracle equals the reference's
    expression evaluated by torch on bf16 tensors on all but at most 0.1% of rows. There
    torch's fp32 sum of squares and the oracle's fp64 one fall on either side of a bf16
    rounding boundary of a norm: one bf16 step in a norm, at most two in the signal. A dropped
    rounding point (e.g. no R() after the subtraction) differs on most rows."""

    from oracle.huginn_model import HuginnOracle

    rng = np.random.default_rng(int(scale * 1000))
    h = round_bf16((rng.standard_normal((3000, 5280)) * scale).astype(np.float32))
    rel = rng.uniform(0.0, 0.5, (3000, 1)).astype(np.float32)
    p = round_bf16(h + (rng.standard_normal(h.shape) * scale).astype(np.float32) * rel)
    p[:40] = h[:40]  # converged rows: signal 0
    want = _torch_latent_diff(h, p)
    got = stage.latent_diff(h, p, "bf16")
    differ = got != want
    assert differ.sum() <= 3, differ.sum()
    assert np.all(np.abs(got - want)[differ] <= np.abs(want[differ]) * 2.0 ** -6 * 1.0001)
    assert np.all(got[:40] == 0.0)
    # The same expression with the subtraction left unrounded: most rows differ.
    loose = np.sqrt(((h.astype(np.float64) - p) ** 2).sum(-1)) / np.sqrt((h.astype(np.float64) ** 2).sum(-1))
    assert np.mean(round_bf16(loose.astype(np.float32))[40:] != want[40:]) > 0.05
    # The model oracle's per-row restatement equals the batched one.
    rows = HuginnOracle.latent_diff.__get__(type("O", (), {"rnd": staticmethod(round_bf16)})())
    for i in range(0, 3000, 97):
        assert rows(h[i], p[i]) == got[i]


def test_latent_difference_bf16_zero_state_clamps_in_bf16() -> None:
    """An all-zero state: torch clamps the bf16 norm to bf16(1e-9), not to fp32 1e-9."""

    h = np.zeros((3, 64), np.float32)
    p = round_bf16(np.random.default_rng(5).standard_normal((3, 64)).astype(np.float32))
    want = _torch_latent_diff(h, p)
    np.testing.assert_array_equal(stage.latent_diff(h, p, "bf16"), want)
    assert want[0] != np.float32(round_bf16(np.array([np.linalg.norm(p[0]) / 1e-9], np.float32))[0])


@pytest.mark.parametrize("scale", [1.0, 4.0, 20.0])
def test_silu_mul_bf16_against_torch_bf16(scale: float) -> None:
    """R(R(silu(g)) * u) on bf16 inputs against F.silu(g) * u on bf16 tensors
    (ouro/modeling_ouro.py:167-169). The oracle takes silu in float64 and rounds
    once to fp32, then to bf16; torch computes silu in fp32. The two agree on all but
    a few in a million values (a double rounding at a bf16 midpoint), and those differ
    by one bf16 step."""

    rng = np.random.default_rng(int(scale))
    gu = round_bf16((rng.standard_normal((2000, 1024)) * scale).astype(np.float32))
    g, u = torch.from_numpy(gu).bfloat16().chunk(2, dim=-1)
    want = (torch.nn.functional.silu(g) * u).float().numpy()
    got = stage.silu_mul(gu, "bf16")
    differ = got != want
    assert differ.sum() <= 5, differ.sum()
    step = np.abs(want) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(got - want)[differ] <= step[differ] * 1.0001)
