"""Full-size workload shapes, checked through size-independent properties.

* Decode attention at the 1024-row microbench size (contexts up to 8192, 4 loop
  slots, 16 heads x 128): sampled rows against a float32 torch attention over the
  pages the kernel read (query rotated with the reference's bf16 RoPE ops), and
  invariance of the whole batch's output under a permutation of physical pages
  (swapping page contents together with their block-table entries changes no
  arithmetic, so the outputs are bit-identical).
* The engine at the Ouro-2.6B shape (48 layers) and the Huginn-0125 shape
  (55 heads x 96, 4 core layers looped 32 steps): the refill and no-refill
  schedulers must produce identical tokens, and replayed exit depths are
  recorded exactly.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _rope_split_half_bf16(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """q*cos + rotate_half(q)*sin with every op rounded to bf16 (ouro/modeling_ouro.py:172-204)."""

    r = lambda t: t.bfloat16().float()
    xf = x.float()
    half = x.shape[-1] // 2
    rot = torch.cat([-xf[..., half:], xf[..., :half]], dim=-1)
    c = torch.cat([cos, cos], dim=-1)
    s = torch.cat([sin, sin], dim=-1)
    return r(r(xf * c) + r(rot * s))


def test_microbench_size_decode_attention_sampled_rows_and_page_permutation() -> None:
    from continuous_depth_batching_amd import ops, workloads

    case = workloads.decode_attention_microbench(num_rows=1024, ctx_min=128, ctx_max=8192, num_slots=4, seed=3)
    rows, heads, dim = case.q.shape
    bs = case.block_size
    view = ops.KVPoolView(case.kv_pool, bs)
    maxp = int(case.contexts.max())
    ws = torch.empty(ops.decode_workspace_bytes(rows, heads, dim, maxp + 1, bs, ops.MIN_SPLIT_PAGES) // 4,
                     dtype=torch.float32, device="cuda")
    scale = dim ** -0.5

    def run(table: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(case.q)
        ops.paged_decode_attention_raw(case.q, case.k_new, case.v_new, view.k_ptr, view.v_ptr, view.layer_stride,
                                       view.num_cache_layers, view.pool_blocks, case.slot_offset, 0, table, None,
                                       case.seqlens, case.rope_cos, case.rope_sin, 1, None, None, out, ws, bs,
                                       ops.ADAPTIVE_SPLIT, scale)
        torch.cuda.synchronize()
        return out

    out = run(case.block_table)
    assert torch.isfinite(out.float()).all()

    # Sampled rows against float32 attention over the pool after the append.
    rng = np.random.default_rng(0)
    sample = rng.choice(rows, size=24, replace=False)
    table = case.block_table.cpu().numpy()
    slot = case.slot_offset.cpu().numpy()
    errs = []
    for b in sample:
        p = int(case.seqlens[b])
        pos = torch.arange(p + 1, device="cuda")
        blocks = torch.from_numpy(table[b]).cuda().long()[pos // bs]
        kv_rows = blocks * bs + pos % bs
        k = case.kv_pool[int(slot[b]), 0, kv_rows].float()  # [p+1, H, D]
        v = case.kv_pool[int(slot[b]), 1, kv_rows].float()
        q = _rope_split_half_bf16(case.q[b], case.rope_cos[p], case.rope_sin[p])  # [H, D]
        s = torch.einsum("hd,thd->ht", q, k) * scale
        ref = torch.einsum("ht,thd->hd", torch.softmax(s, dim=-1), v)
        errs.append((out[b].float() - ref).abs())
    err = torch.stack(errs)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3

    # Swap 20000 random pairs of physical pages (contents in every slot, and table entries).
    n_pages = case.kv_pool.shape[2] // bs
    pairs = torch.from_numpy(rng.choice(n_pages, size=(20000, 2), replace=False)).cuda().long()
    a, c = pairs[:, 0], pairs[:, 1]
    ra = (a[:, None] * bs + torch.arange(bs, device="cuda")).reshape(-1)
    rc = (c[:, None] * bs + torch.arange(bs, device="cuda")).reshape(-1)
    tmp = case.kv_pool[:, :, ra].clone()
    case.kv_pool[:, :, ra] = case.kv_pool[:, :, rc]
    case.kv_pool[:, :, rc] = tmp
    perm = torch.arange(n_pages, device="cuda", dtype=torch.int32)
    perm[a] = c.int()
    perm[c] = a.int()
    t2 = case.block_table.clone()
    live = t2 >= 0
    t2[live] = perm[t2[live].long()]
    out2 = run(t2)
    assert torch.equal(out, out2)


def _generate(engine, prompts, mnt, depths):
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    return [o.generated_tokens for o in outs], [o.exit_depths for o in outs]


def test_ouro_2p6b_shape_refill_and_wave_loops_agree() -> None:
    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine
    from continuous_depth_batching_amd.ouro import OuroConfig, build_ouro
    from continuous_depth_batching_amd.workloads import categorical_exit_trace

    cfg = OuroConfig(vocab_size=49152, hidden_size=2048, intermediate_size=5632, num_hidden_layers=48,
                     num_attention_heads=16, num_key_value_heads=16, head_dim=128, total_ut_steps=4,
                     max_position_embeddings=4096)
    model = build_ouro(cfg, seed=1, dtype=torch.bfloat16, device="cuda")
    rng = np.random.default_rng(7)
    prompts = [rng.integers(0, 49152, int(n)).tolist() for n in rng.integers(8, 200, size=6)]
    mnt = [12] * 6
    depths = categorical_exit_trace(mnt, (0.15, 0.25, 0.30, 0.30), seed=7)
    results = []
    for refill in (True, False):
        engine = ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(
            max_recurrent_steps=4, synthetic_exit_replay=True, delay_gate_consumption=False, kv_policy="single",
            refill=refill, num_blocks=512, max_model_len=1024, max_num_seqs=8, kv_pressure_mode="none"))
        results.append(_generate(engine, prompts, mnt, depths))
        del engine
        torch.cuda.empty_cache()
    (t_refill, d_refill), (t_wave, d_wave) = results
    assert d_refill == depths and d_wave == depths
    assert t_refill == t_wave


def test_huginn_0125_shape_replay_refill_and_wave_agree() -> None:
    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine
    from continuous_depth_batching_amd.huginn import HuginnConfig, build_huginn
    from continuous_depth_batching_amd.workloads import poisson_exit_trace

    cfg = HuginnConfig(block_size=1024)  # n_embd 5280, 55 heads x 96, 2 + 4 + 2 layers, vocab 65536
    model = build_huginn(cfg, seed=1, dtype=torch.bfloat16, device="cuda", qk_bias_std=0.02)
    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, 65536, int(n)).tolist() for n in rng.integers(8, 64, size=4)]
    mnt = [5] * 4
    depths = poisson_exit_trace(mnt, mean=12.0, max_steps=32, seed=11)
    results = []
    for refill in (True, False):
        engine = ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(
            max_recurrent_steps=32, synthetic_exit_replay=True, delay_gate_consumption=False, kv_policy="single",
            refill=refill, num_blocks=256, max_model_len=512, max_num_seqs=4, kv_pressure_mode="none"))
        results.append(_generate(engine, prompts, mnt, depths))
        del engine
        torch.cuda.empty_cache()
    (t_refill, d_refill), (t_wave, d_wave) = results
    assert d_refill == depths and d_wave == depths
    assert t_refill == t_wave
    assert all(0 <= t < 65536 for ts in t_refill for t in ts)
