"""Post-load KV budgeting (kv_cache_sizing.py:25-80), with the reference's own cases
(tests/test_kv_cache_sizing.py:83-146): device memory is read through a stand-in."""

from __future__ import annotations

import pytest
import torch

from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig, validate_cache_size_request
from continuous_depth_batching_amd.engine import resolve_num_blocks
from tests.host_runner import TokenIncrementConfig

# 2 layers x block 4 x 2 heads x dim 8 x fp16, K and V: one block is 512 bytes.
BYTES_PER_BLOCK = 2 * 2 * 4 * 2 * 8 * 2


def test_budget_excludes_runtime_reserve_and_unallocatable_blocks(monkeypatch) -> None:
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device: (8000, 10000))
    # budget 8000 - 10000 * 0.2 = 6000 bytes: 11 blocks, less the 2 spare blocks of the pool.
    blocks = resolve_num_blocks(None, 0.8, BYTES_PER_BLOCK, "cuda:0")
    assert blocks == 9
    assert resolve_num_blocks(None, None, BYTES_PER_BLOCK, "cuda:0") == blocks
    assert (blocks + 2) * BYTES_PER_BLOCK <= 6000 < (blocks + 3) * BYTES_PER_BLOCK


def test_manual_block_count_does_not_read_device_memory(monkeypatch) -> None:
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device: pytest.fail("device memory should not be read"))
    assert resolve_num_blocks(7, None, BYTES_PER_BLOCK, "cpu") == 7


@pytest.mark.parametrize("fraction", [-0.1, 0, 1, float("nan"), float("inf")])
def test_invalid_fraction(fraction: float) -> None:
    with pytest.raises(ValueError, match="mem_fraction_static"):
        validate_cache_size_request(None, fraction)
    with pytest.raises(ValueError, match="mem_fraction_static"):
        ContinuousDepthBatchingConfig(mem_fraction_static=fraction, max_recurrent_steps=3).get_resolved(
            TokenIncrementConfig())


def test_conflicting_settings_and_cpu_auto_sizing() -> None:
    with pytest.raises(ValueError, match="either num_blocks or mem_fraction_static"):
        resolve_num_blocks(7, 0.8, BYTES_PER_BLOCK, "cuda")
    with pytest.raises(ValueError, match="requires CUDA"):
        resolve_num_blocks(None, None, BYTES_PER_BLOCK, "cpu")
    with pytest.raises(ValueError, match="either num_blocks or mem_fraction_static"):
        ContinuousDepthBatchingConfig(num_blocks=7, mem_fraction_static=0.8, max_recurrent_steps=3).get_resolved(
            TokenIncrementConfig())
    assert ContinuousDepthBatchingConfig(max_recurrent_steps=3).get_resolved(TokenIncrementConfig()).num_blocks is None


def test_insufficient_budget(monkeypatch) -> None:
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device: (2000, 10000))
    with pytest.raises(ValueError, match="No usable KV blocks fit"):
        resolve_num_blocks(None, None, BYTES_PER_BLOCK, "cuda")
