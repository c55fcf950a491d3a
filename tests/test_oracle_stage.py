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
