"""The cdb:: operators the engine calls: each is registered with torch.library, marks the tensors
it writes as mutable in its schema, and has a fake implementation giving the output's shape and
dtype (run here under FakeTensorMode, with no device)."""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import continuous_depth_batching_amd.ops  # noqa: F401  (registers the operators)

OPERATORS = {
    # name: the arguments its schema must mark as written
    "paged_decode_attention": {"kv_pool", "workspace"},
    "rope_kv_write": {"kv_pool"},
    "prefill_attention": set(),
    "prefill_attention_split": {"partials"},
    "rmsnorm": set(),
    "residual_rmsnorm": set(),
    "exit_gate": {"signal", "cdf", "survival", "pending", "exit_flags"},
    "exit_kv_copy": {"kv_pool"},
    "route_compact": {"lists"},
    "gather_rows": set(),
    "scatter_rows_": {"dst"},
    "linear": set(),
    "linear_residual_rmsnorm": set(),
    "silu_mul": set(),
    "argmax": set(),
}


@pytest.mark.parametrize("name", sorted(OPERATORS))
def test_operator_is_registered_with_its_mutations(name: str) -> None:
    op = getattr(torch.ops.cdb, name).default
    written = {a.name for a in op._schema.arguments if a.alias_info is not None and a.alias_info.is_write}
    assert written == OPERATORS[name]


def test_fake_implementations_give_output_shapes() -> None:
    cuda = dict(device="cuda")
    bf = dict(dtype=torch.bfloat16, **cuda)
    i32 = dict(dtype=torch.int32, **cuda)
    with FakeTensorMode():
        T, H, Hkv, D = 40, 4, 2, 64
        qkv = torch.empty(T, (H + 2 * Hkv) * D, **bf)
        q = qkv[:, : H * D].view(T, H, D)
        k = qkv[:, H * D:(H + Hkv) * D].view(T, Hkv, D)
        v = qkv[:, (H + Hkv) * D:].view(T, Hkv, D)
        pool = torch.empty(3, 2, 64 * 16, Hkv, D, **bf)
        rows = torch.empty(T, dtype=torch.int64, device="cuda")
        pos = torch.empty(T, **i32)
        cos = torch.empty(128, D // 2, dtype=torch.float32, device="cuda")
        q_rot = torch.ops.cdb.rope_kv_write(q, k, v, pool, 1, 16, rows, pos, cos, cos, 1, None, None)
        assert q_rot.shape == (T, H, D) and q_rot.dtype == torch.bfloat16 and q_rot.is_contiguous()
        table, seq = torch.empty(2, 8, **i32), torch.empty(2, **i32)
        cu, tiles = torch.empty(3, **i32), torch.empty(1, **i32)
        out = torch.ops.cdb.prefill_attention(q_rot, pool, 1, 16, table, seq, cu, seq, tiles, tiles, 0.125)
        assert out.shape == (T, H, D) and out.dtype == torch.bfloat16
        items, merges = torch.empty(3, 4, **i32), torch.empty(1, 4, **i32)
        partials = torch.empty(1024, dtype=torch.float32, device="cuda")
        out = torch.ops.cdb.prefill_attention_split(q_rot, pool, 1, 16, table, seq, cu, seq, items, merges, 2,
                                                     partials, 0.125)
        assert out.shape == (T, H, D)
        hidden = torch.empty(8, 256, **bf)
        f64 = torch.empty(16, dtype=torch.float64, device="cuda")
        res = torch.ops.cdb.exit_gate(hidden, None, torch.empty(256, **bf), torch.empty(1, **bf),
                                      torch.empty(8, **bf), f64, f64.clone(),
                                      torch.empty(16, dtype=torch.float32, device="cuda"),
                                      torch.empty(8, dtype=torch.int64, device="cuda"), torch.empty(8, **i32), None,
                                      torch.empty(8, dtype=torch.uint8, device="cuda"), 8, 0, 0, False, True, 1, 4,
                                      0.5)
        assert res is None
        assert torch.ops.cdb.exit_kv_copy(pool, 16, rows[:4], pos[:4], 4, 0, 1, 3) is None
