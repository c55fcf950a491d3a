"""MI355X-native continuous-depth-batching (CDB) decode step.

The hot path of a looped LM's decode step -- mixed-depth paged decode
attention with fused RoPE and KV append, RMSNorm, the early-exit gates, and
on-device row compaction/refill -- runs as hand-written HIP kernels for gfx950
behind the C ABI in ``include/cdb_amd.h``, exposed to PyTorch as
``torch.ops.cdb.*`` custom ops (``continuous_depth_batching_amd.ops``). The
host side keeps the reference's Python API:
``ContinuousDepthBatchingEngine.from_model(...).generate_batch(...)`` and
``ContinuousDepthBatchingConfig``.
"""
