"""KV-pressure preemption on the HIP path: the swap pool's block moves and both pressure modes.

* ``KvSwapPool`` round trip: random bf16 KV, a victim's blocks gathered to the
  pinned host pool (runs split by gaps, staging split into several chunks) and
  scattered back into other device blocks, bit-exact, and no other block touched.
* offload: a cache too small for the batch swaps decoders out and back; the
  token streams and exit depths equal the per-request oracle's, as if nothing
  had been preempted (tiny fp32 Ouro, replayed exit depths).
* recompute: each soft reset re-prefills prompt + generated tokens at full
  depth and drops the pending token's replayed depth (cdb/requests.py:111-126);
  the oracle is composed the same way from the engine's preemption points.
"""

from __future__ import annotations

import pytest
import torch

from continuous_depth_batching_amd.offloading import KvSwapPool
from tests.pressure_helpers import PRESSURE, composed_oracle, preemption_cuts, pressure_workload
from tests.test_engine_gpu import build_model, make_engine, run_oracle

pytestmark = pytest.mark.gpu


def _cache(num_blocks: int, block_size: int, policy: str = "depth_indexed"):
    from continuous_depth_batching_amd.cache import PagedKVCache
    from continuous_depth_batching_amd.kv_cache_policy import LoopedKvLayout

    layout = LoopedKvLayout.build(num_prelude_layers=0, num_core_layers=3, num_coda_layers=0,
                                  total_recurrent_steps=4, policy=policy)
    return PagedKVCache(layout=layout, num_blocks=num_blocks, block_size=block_size, num_kv_heads=2, head_dim=64,
                        max_model_len=64 * block_size, max_num_batched_tokens=256, max_requests=8,
                        dtype=torch.bfloat16, device=torch.device("cuda"))


def test_swap_pool_round_trip_is_bit_exact(monkeypatch) -> None:
    cache = _cache(num_blocks=40, block_size=16)
    block_bytes = 2 * cache.num_layers * 16 * 2 * 64 * 2
    monkeypatch.setattr(KvSwapPool, "STAGING_BYTES", 3 * block_bytes)  # 3 blocks per chunk
    pool = KvSwapPool(cache, num_host_blocks=24)
    assert pool.chunk_blocks == 3
    gen = torch.Generator(device="cuda").manual_seed(7)
    cache.pool.copy_(torch.randn(cache.pool.shape, generator=gen, device="cuda").to(torch.bfloat16))
    before = cache.pool.clone()
    pages = cache.pool.view(cache.num_layers, 2, -1, 16, 2, 64)
    victim = [5, 17, 2, 30, 31, 8, 11]
    host = [3, 4, 5, 9, 0, 1, 20]                # runs (3,4,5), (9), (0,1), (20) across chunk edges
    pool.swap_out(victim, host)
    torch.cuda.synchronize()
    want_host = pages[:, :, victim].permute(2, 0, 1, 3, 4, 5).reshape(len(victim), 2 * cache.num_layers, -1)
    # Host block j holds slab (layer, K/V) of device block victim[j] at row 2 * layer + kv.
    assert torch.equal(pool.host[host].to("cuda"), want_host)

    target = [36, 0, 22, 23, 24, 13, 39]
    cache.pool.zero_()
    pool.swap_in(host, target)
    torch.cuda.synchronize()
    back = cache.pool.view(cache.num_layers, 2, -1, 16, 2, 64)
    old = before.view(cache.num_layers, 2, -1, 16, 2, 64)
    assert torch.equal(back[:, :, target], old[:, :, victim])
    untouched = [b for b in range(cache.pool.shape[2] // 16) if b not in target]
    assert not back[:, :, untouched].any()


def test_swap_pool_moves_more_blocks_than_one_request_holds() -> None:
    """A restore batches every request restored in a tick: 100 blocks through a pool whose
    requests hold at most 64."""

    cache = _cache(num_blocks=240, block_size=16, policy="single")
    assert cache.max_blocks_per_request == 64
    pool = KvSwapPool(cache, num_host_blocks=120)
    gen = torch.Generator(device="cuda").manual_seed(11)
    cache.pool.copy_(torch.randn(cache.pool.shape, generator=gen, device="cuda").to(torch.bfloat16))
    before = cache.pool.clone()
    src = list(range(0, 200, 2))                 # 100 scattered device blocks
    host = list(range(10, 110))
    pool.swap_out(src[:50], host[:50])           # two requests' swap-outs
    pool.swap_out(src[50:], host[50:])
    dst = list(range(1, 201, 2))
    pool.swap_in(host, dst)                      # one batched restore of both
    torch.cuda.synchronize()
    pages = lambda t: t.view(cache.num_layers, 2, -1, 16, 2, 64)
    assert torch.equal(pages(cache.pool)[:, :, dst], pages(before)[:, :, src])
    assert torch.equal(pages(cache.pool)[:, :, src], pages(before)[:, :, src])  # sources untouched


def test_swap_pool_rejects_out_of_range_blocks() -> None:
    cache = _cache(num_blocks=8, block_size=16, policy="single")
    pool = KvSwapPool(cache, num_host_blocks=4)
    with pytest.raises(ValueError):
        pool.swap_out([1, 8], [0, 1])            # device block past the pool
    with pytest.raises(ValueError):
        pool.swap_out([1, 2], [0, 4])            # host block past the host pool
    with pytest.raises(ValueError):
        pool.swap_in([0], [1, 2])                # mismatched lengths


@pytest.mark.parametrize("kv_policy", ["single", "last_exited"])
@pytest.mark.parametrize("use_async", [False, True])
def test_offload_preemption_matches_the_oracle(kv_policy: str, use_async: bool) -> None:
    model, weights = build_model(seed=1)
    prompts, mnt, depths = pressure_workload()
    engine = make_engine(model, kv_policy=kv_policy, kv_pressure_mode="offload", cpu_offload_space=0.05,
                         use_async_batching=use_async, **PRESSURE)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    om = engine.offloading_manager
    assert om.num_offload_preemptions > 0 and om.num_restores == om.num_offload_preemptions
    assert om.num_recompute_preemptions == 0
    want = run_oracle(weights, prompts, mnt, kv_policy=kv_policy, exit_depths=depths)
    assert [o.generated_tokens for o in outs] == [w.tokens for w in want]
    assert [o.exit_depths for o in outs] == depths
    assert engine.cache.get_num_free_blocks() == engine.cache.num_blocks


@pytest.mark.parametrize("use_async", [False, True])
def test_recompute_preemption_matches_the_composed_oracle(use_async: bool) -> None:
    from oracle.ouro_model import OuroOracle
    from tests.ouro_helpers import TINY

    model, weights = build_model(seed=2)
    prompts, mnt, depths = pressure_workload()
    engine = make_engine(model, kv_policy="single", kv_pressure_mode="recompute", use_async_batching=use_async,
                         **PRESSURE)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None, exit_depths=depths)
    om = engine.offloading_manager
    assert om.num_recompute_preemptions > 0 and om.num_offload_preemptions == 0
    cuts = preemption_cuts(om.recompute_events, prompts)
    oracle = OuroOracle(weights, num_layers=TINY["num_layers"], num_heads=TINY["num_heads"],
                        num_kv_heads=TINY["num_heads"], head_dim=TINY["head_dim"], rope_theta=TINY["rope_theta"],
                        eps=TINY["eps"], dtype="f32", max_positions=512)

    def oracle_run(prompt, new_tokens, seg_depths):
        return oracle.generate(prompt, new_tokens, max_steps=TINY["steps"], kv_policy="single",
                               exit_depths=seg_depths)

    for i, out in enumerate(outs):
        tokens, exits = composed_oracle(oracle_run, prompts[i], mnt[i], depths[i], cuts.get(i, []))
        assert out.prompt_ids == prompts[i]
        assert out.generated_tokens == tokens, f"request {i}, cuts {cuts.get(i)}"
        assert out.exit_depths == exits
    assert engine.cache.get_num_free_blocks() == engine.cache.num_blocks


def test_auto_sized_cache_serves_a_batch() -> None:
    """num_blocks=None sizes the pool from free device memory after the model is loaded
    (kv_cache_sizing.py:34-80); the fraction leaves about 512 MiB for the KV pool."""

    import gc

    from tests.test_engine_gpu import workload

    model, weights = build_model(seed=0)
    gc.collect()
    torch.cuda.empty_cache()
    free, total = torch.cuda.mem_get_info()
    fraction = (total - free + 512 * 1024**2) / total
    engine = make_engine(model, num_blocks=None, mem_fraction_static=fraction, max_num_seqs=4)
    cache = engine.cache
    assert cache.num_blocks > 0 and engine.cdb_config.num_blocks == cache.num_blocks
    pool_bytes = cache.pool.numel() * cache.pool.element_size()
    assert 256 * 1024**2 < pool_bytes <= 576 * 1024**2  # 512 MiB, plus whatever a late free returned
    prompts, mnt = workload(seed=4, n=4, new_tokens=8)
    outs = engine.generate_batch(prompts, max_new_tokens=mnt, eos_token_id=None)
    want = run_oracle(weights, prompts, mnt)
    assert [o.generated_tokens for o in outs] == [w.tokens for w in want]
