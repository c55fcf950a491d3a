"""Benchmark: Ouro-1.4B-shape CDB decode on one MI355X.

Workload (one "step" = one ``generate_batch`` over the whole batch): a random-init
bf16 Ouro with the 1.4B shape (hidden 2048, 24 layers looped 4 steps, 16 MHA heads
x 128, SwiGLU 5632, vocab 49152, weights N(0, 0.02) seed 1); 256 concurrent
sequences with prompt lengths lognormal(5.5, 1.0) clipped to [8, 2048] and output
lengths lognormal(5.0, 0.8) clipped to [16, 1024], uniform token ids; per-token
exit depths replayed from a seeded categorical over {1, 2, 3, 4} with
probabilities (0.15, 0.25, 0.30, 0.30); CDB with refill, paged KV block 16,
``kv_policy="single"``, synchronous exit horizon. Inputs are synthetic.

The JSON line carries:
  * ``value``: generated tokens / wall time of the timed generate_batch calls;
  * ``roofline``: the mixed-depth decode-attention kernel (the hot kernel of a
    recurrent step) timed with HIP events on its stream, at the recurrent
    shape of this workload (256 rows, every sequence at its mid-generation
    context), against MI355X's 8 TB/s HBM peak;
  * ``decode_attention_microbench``: the same kernel on the 1024-row,
    contexts-in-[128, 8192], 4-loop-slot microbench;
  * ``cpu_baseline``: the numpy oracle's decode of a bounded sample of the same
    workload on the host cores (a port of the reference algorithm, not the
    GPU path).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import threading
import time
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK = 2.5e15  # dense bf16 MFMA flop/s
FORCED_TOKENS = 64  # tokens of the teacher-forced parity pass


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--num-seqs", type=int, default=256)
    p.add_argument("--workload", choices=("ouro-cdb", "decode-attention", "kv-pressure", "ouro-2p6b", "huginn"),
                   default="ouro-cdb",
                   help="ouro-cdb: the end-to-end engine; decode-attention: only the kernel timings; "
                        "kv-pressure: KV swap timings and the engine on a cache too small for the batch; "
                        "ouro-2p6b: the 48-layer shape at 512 sequences, single vs per-step KV; "
                        "huginn: the Huginn-0125 shape at 128 sequences, 32 loop steps")
    p.add_argument("--pressure-fraction", type=float, default=0.6,
                   help="kv-pressure: cache size as a fraction of what the batch needs without preemption")
    p.add_argument("--pressure-safety-margin", type=float, default=0.0,
                   help="kv-pressure: prefill admission margin of the pressured runs (0 admits greedily, so "
                        "decode growth reaches the preemption path instead of being throttled at admission)")
    p.add_argument("--swap-only", action="store_true", help="kv-pressure: only the swap timings")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-microbench", action="store_true")
    p.add_argument("--cpu-sample-tokens", type=int, default=160)
    p.add_argument("--attention-iters", type=int, default=20)
    p.add_argument("--attention-rows", type=int, default=256,
                   help="decode-attention: time the first N rows of the 256-row shape (up to 256 rows of "
                        "128-wide heads run the deep form, which merges in the decode kernel); the bench "
                        "line keeps 256")
    return p.parse_args()


def c2_workload(num_seqs: int, vocab: int):
    from continuous_depth_batching_amd.workloads import ouro_decode_workload

    return ouro_decode_workload(num_seqs, vocab)


def ouro_1p4b_config():
    from continuous_depth_batching_amd.ouro import ouro_1p4b_config as config

    return config()


class GpuActivity:
    """GPU activity (amdsmi gfx_activity, percent) sampled every `interval` seconds while
    active, on a side thread; None when amdsmi is not importable or has no device."""

    def __init__(self, interval: float = 0.02) -> None:
        self.interval = interval
        self.samples: list[float] = []
        self._stop = threading.Event()
        self._thread: threading.Thread | None = None
        self.error: str | None = None

    def _run(self) -> None:
        try:
            import amdsmi

            amdsmi.amdsmi_init()
            try:
                handle = amdsmi.amdsmi_get_processor_handles()[0]
                while not self._stop.is_set():
                    self.samples.append(float(amdsmi.amdsmi_get_gpu_activity(handle)["gfx_activity"]))
                    self._stop.wait(self.interval)
            finally:
                amdsmi.amdsmi_shut_down()
        except Exception as exc:  # noqa: BLE001 - reported, never fatal to the benchmark
            self.error = f"{type(exc).__name__}: {exc}"

    def __enter__(self) -> "GpuActivity":
        self._thread = threading.Thread(target=self._run, daemon=True)
        self._thread.start()
        return self

    def __exit__(self, *exc) -> None:
        self._stop.set()
        if self._thread is not None:
            self._thread.join(timeout=5)

    def summary(self) -> dict | None:
        if not self.samples:
            return {"mean_pct": None, "samples": 0, "error": self.error}
        return {"mean_pct": round(float(np.mean(self.samples)), 1), "samples": len(self.samples),
                "interval_s": self.interval, "source": "amdsmi gfx_activity during the timed generate_batch calls"}


def time_decode_attention(case, split_pages: int, iters: int) -> dict:
    """One decode-attention call at the case's shape, as each layer of a recurrent launch makes it:
    the rows' chunk plan is written once (``plan_ms``, timed on its own), then ``iters`` attend calls
    (decode kernel + split merge) run from it on their own stream (``ms``)."""

    import torch

    from continuous_depth_batching_amd import ops

    view = ops.KVPoolView(case.kv_pool, case.block_size)
    rows, heads, dim = case.q.shape
    ws = torch.empty(ops.decode_workspace_bytes(rows, heads, dim, int(case.contexts.max()) + 1, case.block_size,
                                                split_pages or ops.MIN_SPLIT_PAGES) // 4,
                     dtype=torch.float32, device="cuda")
    out = torch.empty_like(case.q)
    stream = torch.cuda.Stream()

    def launch(stages):
        ops.paged_decode_attention_raw(case.q, case.k_new, case.v_new, view.k_ptr, view.v_ptr, view.layer_stride,
                                       view.num_cache_layers, view.pool_blocks, case.slot_offset, 0,
                                       case.block_table, None, case.seqlens, case.rope_cos, case.rope_sin, 1,
                                       None, None, out, ws, case.block_size, split_pages, dim ** -0.5,
                                       stages=stages)

    def timed(stages, n):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(n):
            launch(stages)
        end.record(stream)
        end.synchronize()
        return start.elapsed_time(end) / n

    with torch.cuda.stream(stream):
        for _ in range(3):
            launch(ops.DECODE_PLAN_AND_ATTEND)
        plan_ms = timed(ops.DECODE_PLAN, iters)
        ms = timed(ops.DECODE_ATTEND, iters)
    nbytes = case.algorithmic_bytes()
    gbps = nbytes / (ms * 1e-3) / 1e9
    return {"ms": ms, "plan_ms": plan_ms, "bytes": nbytes, "gbps": gbps, "rows": rows, "split_pages": split_pages,
            "mean_context": float(case.contexts.mean())}


def decode_attention_c2_case(prompts, outputs, device, rows: int | None = None):
    """The 256-row recurrent shape of the workload: each sequence mid-way through its output
    (its first ``rows`` rows when given)."""

    import torch

    from continuous_depth_batching_amd.workloads import DecodeAttentionCase, rope_tables_torch

    rng = np.random.default_rng(5)
    contexts = np.asarray([len(p) + max(1, o // 2) for p, o in zip(prompts, outputs)], dtype=np.int64)[:rows]
    rows = len(contexts)
    bs = 16
    pages = (contexts + bs - 1) // bs
    perm = rng.permutation(int(pages.sum())).astype(np.int32)
    table = np.full((rows, int(pages.max())), -1, np.int32)
    off = np.concatenate([[0], np.cumsum(pages)])
    for b in range(rows):
        table[b, :pages[b]] = perm[off[b]:off[b + 1]]
    gen = torch.Generator(device=device)
    gen.manual_seed(7)
    pool = torch.empty((1, 2, int(pages.sum()) * bs, 16, 128), dtype=torch.bfloat16, device=device)
    pool.normal_(generator=gen)
    mk = lambda: torch.randn((rows, 16, 128), generator=gen, device=device).bfloat16()
    cos, sin = rope_tables_torch(128, 10000.0, int(contexts.max()), torch.bfloat16, device)
    return DecodeAttentionCase(q=mk(), k_new=mk(), v_new=mk(), kv_pool=pool,
                               slot_offset=torch.zeros(rows, dtype=torch.int32, device=device),
                               block_table=torch.from_numpy(table).to(device),
                               seqlens=torch.from_numpy((contexts - 1).astype(np.int32)).to(device),
                               rope_cos=cos, rope_sin=sin, block_size=bs, contexts=contexts)


def graph_time_ms(fn, calls: int, reps: int = 3, warm: bool = True) -> float:
    """Average milliseconds of one ``fn()`` call, from a captured graph of ``calls`` calls replayed
    on a side stream and timed with events on that stream (launch gaps are the GPU's own).
    ``warm=False`` times the first replay, before the graph's inputs were ever read by it."""

    import torch

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        fn()  # first call outside the capture: lazy setup
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(calls):
                fn()
        if warm:
            graph.replay()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            graph.replay()
        end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / (reps * calls)


def decode_bytes(positions: np.ndarray, heads: int = 16, kv_heads: int = 16, dim: int = 128, bs: int = 16) -> int:
    """Algorithmic bytes of one decode-attention call over rows at ``positions`` (bf16): K and V of
    every attended position, q, out and the new K/V row, block ids and positions."""

    p = positions.astype(np.int64)
    return int((p + 1).sum() * kv_heads * dim * 4 + p.size * (heads * dim * 4 + kv_heads * dim * 4 + 4)
               + ((p + bs) // bs).sum() * 4)


DECODE_LAYERS = 24  # layers of the Ouro-1.4B stack: each recurrent launch plans once and attends 24 times


class LayeredDecode:
    """Decode attention over launches the way the engine's recurrent step runs it: one chunk plan
    per launch, then one attend per layer, each layer on its own cache layer of a pool of
    ``DECODE_LAYERS`` layers (so every layer's pages are cold), replayed from captured graphs.
    Each launch gets a fresh random block table over the pool's pages."""

    def __init__(self, max_rows: int, max_pos: int, pool_pages: int, seed: int) -> None:
        import torch

        from continuous_depth_batching_amd import ops
        from continuous_depth_batching_amd.workloads import rope_tables_torch

        dev = torch.device("cuda")
        self.bs, self.heads, self.dim, self.pool_pages = 16, 16, 128, pool_pages
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        self.pool = torch.empty((DECODE_LAYERS, 2, pool_pages * self.bs, self.heads, self.dim),
                                dtype=torch.bfloat16, device=dev)
        self.pool.normal_(generator=gen)
        self.view = ops.KVPoolView(self.pool, self.bs)
        self.q = torch.randn((max_rows, self.heads, self.dim), generator=gen, device=dev).bfloat16()
        self.kn, self.vn = self.q.clone(), self.q.clone()
        self.out = torch.empty_like(self.q)
        self.cos, self.sin = rope_tables_torch(self.dim, 10000.0, max_pos + 1, torch.bfloat16, dev)
        self.zeros = torch.zeros(max_rows, dtype=torch.int32, device=dev)
        self.rng = np.random.default_rng(seed + 1)
        self.dev = dev

    def tensors(self, pos: np.ndarray):
        import torch

        pages = (pos.astype(np.int64) + self.bs) // self.bs
        ids = self.rng.choice(self.pool_pages, size=int(pages.sum()), replace=False).astype(np.int32)
        table = np.full((len(pos), int(pages.max())), -1, np.int32)
        off = np.concatenate([[0], np.cumsum(pages)])
        for b in range(len(pos)):
            table[b, :pages[b]] = ids[off[b]:off[b + 1]]
        from continuous_depth_batching_amd import ops

        ws = torch.empty(ops.decode_workspace_bytes(len(pos), self.heads, self.dim, int(pos.max()) + 1, self.bs,
                                                    ops.MIN_SPLIT_PAGES) // 4, dtype=torch.float32, device=self.dev)
        return (torch.from_numpy(table).to(self.dev), torch.from_numpy(pos.astype(np.int32)).to(self.dev), ws)

    def launch(self, table, seqlens, ws) -> None:
        from continuous_depth_batching_amd import ops

        n = seqlens.numel()
        for layer in range(DECODE_LAYERS):
            ops.paged_decode_attention_raw(
                self.q[:n], self.kn[:n], self.vn[:n], self.view.k_ptr, self.view.v_ptr, self.view.layer_stride,
                self.view.num_cache_layers, self.view.pool_blocks, self.zeros[:n], layer, table, None, seqlens,
                self.cos, self.sin, 1, None, None, self.out[:n], ws, self.bs, ops.ADAPTIVE_SPLIT, self.dim ** -0.5,
                stages=ops.DECODE_PLAN_AND_ATTEND if layer == 0 else ops.DECODE_ATTEND)

    def time_ms(self, launches: list[np.ndarray]) -> float:
        """Summed per-layer milliseconds (plan included, 1/24 of it per layer) of ``launches``."""

        tensors = [self.tensors(pos) for pos in launches]
        state = {"i": 0}

        def call():
            self.launch(*tensors[state["i"] % len(tensors)])
            state["i"] += 1

        state["i"] = len(tensors) - 1  # the untimed first call takes the last launch; the capture starts at 0
        return graph_time_ms(call, len(tensors), reps=1, warm=False) * len(tensors) / DECODE_LAYERS


def run_weighted_decode(launches: list[np.ndarray], group: int = 16) -> dict:
    """Decode attention over every recurrent launch of the workload, at each launch's own rows and
    positions, as the engine runs it (one plan, then 24 layers on cold cache layers): summed
    algorithmic bytes of one layer pass over summed per-layer time."""

    import torch

    bs = 16
    need = max(int(((p.astype(np.int64) + bs) // bs).sum()) for p in launches)
    bench = LayeredDecode(max(len(p) for p in launches), max(int(p.max()) for p in launches), need + 64, seed=11)
    total_ms, total_bytes = 0.0, 0
    classes: dict[str, int] = {}
    for g0 in range(0, len(launches), group):
        chunk = launches[g0:g0 + group]
        total_ms += bench.time_ms(chunk)
        for pos in chunk:
            n = len(pos)
            key = "1-16" if n <= 16 else "17-64" if n <= 64 else "65-128" if n <= 128 else "129-256"
            classes[key] = classes.get(key, 0) + 1
            total_bytes += decode_bytes(pos)
    del bench
    torch.cuda.empty_cache()
    gbps = total_bytes / (total_ms * 1e-3) / 1e9
    return {"launches": len(launches), "ms": round(total_ms, 2), "bytes": total_bytes, "GBps": round(gbps, 1),
            "frac": round(gbps / HBM_PEAK_GBPS, 4),
            "launches_by_rows": dict(sorted(classes.items())),
            "note": "every recurrent launch of one generate_batch of the workload, as the recurrent step runs it: "
                    "one chunk plan, then decode attention on each of 24 cache layers (cold pages, a random block "
                    "table per launch); per-layer time includes 1/24 of the plan; captured graphs"}


def time_by_rows(positions_by_rows: dict[int, np.ndarray], launches_per_width: int = 4) -> dict:
    """Decode attention at fixed launch widths, as the recurrent step runs it (one plan, 24 cold
    cache layers), per layer, for ``launches_per_width`` launches with fresh block tables."""

    import torch

    bs = 16
    need = max(int(((p.astype(np.int64) + bs) // bs).sum()) for p in positions_by_rows.values())
    bench = LayeredDecode(max(positions_by_rows), max(int(p.max()) for p in positions_by_rows.values()),
                          need + 64, seed=13)
    results = {}
    for rows, pos in positions_by_rows.items():
        pos = pos.astype(np.int32)
        ms = bench.time_ms([pos] * launches_per_width) / launches_per_width
        nbytes = decode_bytes(pos)
        results[str(rows)] = {"us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                              "frac": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                              "mean_context": round(float(pos.mean()) + 1, 1)}
    del bench
    torch.cuda.empty_cache()
    return results


def time_rope_kv_write(tokens: int, heads: int = 16, dim: int = 128) -> tuple[float, int]:
    """(ms, algorithmic bytes) of one prefill RoPE + KV write of ``tokens`` tokens, reading q, k and
    v as column slices of one fused QKV output as the engine does, timed from a captured graph."""

    import torch

    from continuous_depth_batching_amd import ops
    from continuous_depth_batching_amd.workloads import rope_tables_torch

    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(15)
    bs = 16
    pages = 4 * tokens // bs + 64
    pool = torch.zeros((1, 2, pages * bs, heads, dim), dtype=torch.bfloat16, device=dev)
    view = ops.KVPoolView(pool, bs)
    qkv = torch.randn((tokens, 3, heads, dim), generator=gen, device=dev).bfloat16()
    q_out = torch.empty((tokens, heads, dim), dtype=torch.bfloat16, device=dev)
    write_rows = torch.from_numpy(np.random.default_rng(16).choice(pages * bs, tokens, replace=False)).to(dev)
    positions = torch.randint(0, 4096, (tokens,), generator=gen, device=dev, dtype=torch.int32)
    cos, sin = rope_tables_torch(dim, 10000.0, 4096, torch.bfloat16, dev)

    def rope_write():
        ops.rope_kv_write_raw(qkv[:, 0], qkv[:, 1], qkv[:, 2], q_out, view, 0, write_rows, positions, cos, sin, 1,
                              None, None)

    ms = graph_time_ms(rope_write, 20)
    del pool, qkv, q_out
    # q, k, v read; rotated q, k and v written (16-byte rows per head); positions and pool rows.
    return ms, 6 * tokens * heads * dim * 2 + tokens * 12


def time_companion_kernels(rows: int = 1024, hidden: int = 2048, prefill_tokens: int | None = None) -> dict:
    """The per-row kernels around decode attention at the microbench's batch size: the RoPE + KV
    write of ``rows`` tokens (the prefill append; also at ``prefill_tokens``, the workload's first
    prefill batch), and the exit gate plus the hidden-bank gather and scatter that compact and
    refill a launch's rows, each timed from a captured graph."""

    import torch

    from continuous_depth_batching_amd import ops

    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(17)
    rope_ms, rope_bytes = time_rope_kv_write(rows)
    rope_batch = time_rope_kv_write(prefill_tokens) if prefill_tokens else None

    bank = torch.randn((4 * rows + 64, hidden), generator=gen, device=dev).bfloat16()
    slots = torch.randperm(bank.shape[0], generator=gen, device=dev)[:rows].contiguous()
    staged = torch.empty((rows, hidden), dtype=torch.bfloat16, device=dev)
    weight = (torch.randn(hidden, generator=gen, device=dev) * 0.02).bfloat16()
    bias = torch.zeros(1, dtype=torch.bfloat16, device=dev)
    state = ops.GateState.allocate(bank.shape[0], dev)
    signal = torch.empty(rows, dtype=torch.bfloat16, device=dev)
    steps = torch.ones(rows, dtype=torch.int32, device=dev)
    flags = torch.empty(rows, dtype=torch.uint8, device=dev)

    def gate():
        ops.exit_gate_raw(staged, None, weight, bias, signal, state, slots, steps, None, flags, rows,
                          kind=ops.GATE_HAZARD, rule=ops.RULE_CUMULATIVE_HAZARD, delayed=False, round_hazard=True,
                          min_steps=1, max_steps=4, threshold=0.5)

    def compact():
        ops.copy_rows_raw(bank, slots, staged, None, rows)   # gather the launch's rows by bank slot
        ops.copy_rows_raw(staged, None, bank, slots, rows)   # scatter them back

    gate_ms = graph_time_ms(gate, 20)
    compact_ms = graph_time_ms(compact, 20)
    gate_bytes = rows * hidden * 2 + hidden * 2 + rows * (8 + 8 + 4 + 4 + 1 + 2)
    compact_bytes = 4 * rows * hidden * 2 + 2 * rows * 8
    del bank
    torch.cuda.empty_cache()
    row = lambda ms, b: {"us": round(ms * 1e3, 2), "bytes": b, "GBps": round(b / (ms * 1e-3) / 1e9, 1),
                         "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    out = {"rows": rows, "rope_kv_write": row(rope_ms, rope_bytes), "exit_gate": row(gate_ms, gate_bytes),
           "bank_gather_scatter": row(compact_ms, compact_bytes),
           "note": f"{rows} tokens/rows, 16 heads x 128 (KV write) and hidden {hidden} (gate, bank rows), bf16; "
                   "algorithmic bytes: q/k/v read + rotated q and k/v written; hidden read + gate state; "
                   "bank rows read and written twice"}
    if rope_batch is not None:
        out["rope_kv_write_first_prefill_batch"] = dict(row(*rope_batch), tokens=prefill_tokens)
    return out


def decode_kernels(rows: int) -> str:
    """The kernels one attend call runs at ``rows`` rows of 16-token pages (the decode library's
    form choice at 128-wide heads: the deep form, which merges in the decode kernel, up to 256 rows)."""

    if rows <= 256:
        return "cdb::paged_decode_deep_kernel<bf16,128> (merge in the kernel)"
    return "cdb::paged_decode_fast_kernel<bf16,128> + decode_merge_kernel"


TRAFFIC_RECORD = "profiles/decode_attention_c2_256rows_traffic.json"


DECODE_SOURCE = "continuous_depth_batching_amd/csrc/paged_decode_attention.hip"


def decode_source_sha256() -> str:
    """SHA-256 of the decode source's code: comments, blank lines and trailing spaces removed, so
    that a record counted on the kernels stays valid across comment edits and no longer."""

    import hashlib
    import re

    text = (REPO / DECODE_SOURCE).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    lines = (re.sub(r"//.*$", "", line).rstrip() for line in text.splitlines())
    return hashlib.sha256("\n".join(line for line in lines if line).encode()).hexdigest()


def measured_traffic(algorithmic_bytes: int) -> int | None:
    """HBM bytes per decode-attention call at this shape, from the FETCH_SIZE / WRITE_SIZE
    counter runs (scaled by a plain copy of known size) recorded with the profiles. A counter
    run cannot happen inside this process, so the record is used only when it was taken on
    this very shape (its algorithmic bytes equal this run's) with this very decode source (its
    SHA-256 equals the source's now); otherwise the figure is null."""

    path = REPO / TRAFFIC_RECORD
    if not path.exists():
        return None
    record = json.loads(path.read_text())
    if int(record.get("algorithmic_bytes_per_call", -1)) != int(algorithmic_bytes):
        return None
    if record.get("decode_source_sha256") != decode_source_sha256():
        return None  # counted on another version of the kernels
    return int(record["traffic_bytes_per_call"])


def time_prefill_attention(prompt_lens, iters: int, past=None) -> dict:
    """Average duration of one prefill-attention call over a batch (fresh prompts, or new tokens
    after `past` cached positions), on its stream, through the path the engine takes for it:
    whole tiles, or the split work list with its merge when one tile would outlast the rest."""

    import torch

    from continuous_depth_batching_amd import ops, workloads

    case = workloads.prefill_attention_batch(lens=prompt_lens, past=past)
    view = ops.KVPoolView(case.kv_pool, case.block_size)
    out = torch.empty_like(case.q)
    stream = torch.cuda.Stream()
    scale = case.q.shape[-1] ** -0.5
    plan = ops.prefill_split_plan(case.lens, case.past_lens, num_heads=case.q.shape[1],
                                  num_cus=torch.cuda.get_device_properties(0).multi_processor_count)
    with torch.cuda.stream(stream):
        if plan is None:
            def launch():
                ops.prefill_attention_raw(case.q, view, 0, case.block_table, case.table_row, case.cu_q, case.past,
                                          case.tile_seq, case.tile_q0, out, scale)
        else:
            items = torch.from_numpy(plan.items).cuda()
            merges = torch.from_numpy(plan.merges).cuda()
            partials = torch.empty(ops.prefill_partial_bytes(plan.num_slots, case.q.shape[1], case.q.shape[2]) // 4,
                                   dtype=torch.float32, device="cuda")

            def launch():
                ops.prefill_attention_split_raw(case.q, view, 0, case.block_table, case.table_row, case.cu_q,
                                                case.past, items, merges, plan.num_slots, partials, out, scale)
        for _ in range(2):
            launch()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(iters):
            launch()
        end.record(stream)
    end.synchronize()
    ms = start.elapsed_time(end) / iters
    flops = case.flops()
    result = {"ms": round(ms, 4), "flops": flops, "TFLOPs": round(flops / (ms * 1e-3) / 1e12, 1),
              "mfma_frac": round(flops / (ms * 1e-3) / MFMA_BF16_PEAK, 4), "tokens": int(case.lens.sum()),
              "sequences": int(case.lens.size), "max_len": int(case.lens.max()),
              "path": "tiles" if plan is None else "split"}
    if plan is not None:
        result.update(items=int(len(plan.items)), merges=int(len(plan.merges)), max_blocks=plan.max_blocks)
    return result


def time_decode_projections(rows: int = 16, layers: int = 24, reps: int = 4) -> dict:
    """The Ouro-1.4B layer's four projections at `rows` rows as a recurrent step runs them
    (QKV and gate/up + SiLU on cdb_linear; O and down as split-K fp32 partials on
    cdb_linear_parts, which the residual norm after them adds), each over `layers`
    distinct weights (one per layer, so every launch streams cold weights as in a layer
    stack), timed from a captured graph so launch gaps are the GPU's own."""

    import torch

    from continuous_depth_batching_amd import ops

    shapes = {"qkv": (2048, 6144, False), "o_split_k": (2048, 2048, False), "gate_up_silu": (2048, 5632, True),
              "down_split_k": (5632, 2048, False)}
    result = {}
    for name, (k, n, gated) in shapes.items():
        split = name.endswith("split_k")
        gen = torch.Generator(device="cuda")
        gen.manual_seed(3)
        weights = [ops.pack_linear_weight((torch.randn(((2 if gated else 1) * n, k), generator=gen, device="cuda")
                                           * 0.02).bfloat16()) for _ in range(layers)]
        x = torch.randn((rows, k), generator=gen, device="cuda").bfloat16()
        splits = ops.linear_parts_splits(rows, n, k) if split else 0
        y = (torch.empty((splits, rows, n), dtype=torch.float32, device="cuda") if split
             else torch.empty((rows, n), dtype=torch.bfloat16, device="cuda"))

        def run(w):
            if split:
                ops.linear_parts_raw(x, w, y)
            else:
                ops.linear_raw(x, w, y, gated=gated)

        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            for w in weights[:2]:
                run(w)
            stream.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for w in weights:
                    run(w)
            graph.replay()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(reps):
                graph.replay()
            end.record(stream)
        end.synchronize()
        us = start.elapsed_time(end) / (reps * layers) * 1e3
        nbytes = weights[0].numel() * 2 + rows * k * 2 + y.numel() * y.element_size()
        result[name] = {"us": round(us, 2), "bytes": nbytes, "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
        del weights
    torch.cuda.empty_cache()
    return {"rows": rows, "shapes": result}


def first_prefill_batch(prompts, token_budget: int = 8192) -> list[int]:
    """Prompt lengths of the workload's first full prefill batch (prompts admitted in order while
    they fit the engine's token budget)."""

    lens, total = [], 0
    for p in prompts:
        if total + len(p) > token_budget:
            break
        lens.append(len(p))
        total += len(p)
    return lens


def copy_calibration(nbytes: int = 1 << 30, iters: int = 5) -> dict:
    """A plain device-to-device copy of known size: the yardstick that scales the
    FETCH_SIZE / WRITE_SIZE counters into HBM bytes, and the copy bandwidth
    this part reaches in practice."""

    import torch

    src = torch.ones(nbytes // 2, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        dst.copy_(src)
    end.record()
    end.synchronize()
    ms = start.elapsed_time(end) / iters
    return {"bytes_read": nbytes, "bytes_written": nbytes, "ms": round(ms, 4),
            "GBps": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def time_kv_swap(blocks: int = 256, iters: int = 5) -> dict:
    """Swap one 4096-token Ouro-1.4B request (kv single: 24 cache layers, 16 heads x 128, bf16,
    256 blocks of 16 tokens, 3 MiB each) out to the pinned host pool and back, its device
    blocks scattered as after allocator churn. The yardstick is a plain pinned copy of the
    same bytes in one DMA; the gather kernel's HBM rate is timed on its own."""

    import torch

    from continuous_depth_batching_amd import ops
    from continuous_depth_batching_amd.cache import PagedKVCache
    from continuous_depth_batching_amd.kv_cache_policy import LoopedKvLayout
    from continuous_depth_batching_amd.offloading import KvSwapPool

    layout = LoopedKvLayout.build(num_prelude_layers=0, num_core_layers=24, num_coda_layers=0,
                                  total_recurrent_steps=4, policy="single")
    cache = PagedKVCache(layout=layout, num_blocks=2 * blocks + 8, block_size=16, num_kv_heads=16, head_dim=128,
                         max_model_len=16 * blocks, max_num_batched_tokens=8192, max_requests=4,
                         dtype=torch.bfloat16, device=torch.device("cuda"))
    stream = torch.cuda.Stream()
    pool = KvSwapPool(cache, num_host_blocks=blocks, stream=stream)
    device_blocks = np.random.default_rng(0).permutation(cache.num_blocks)[:blocks].tolist()
    host_blocks = list(range(blocks))
    nbytes = blocks * pool.slabs * pool.block_elems * 2

    def timed(fn, n: int) -> float:
        fn()
        stream.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            start.record()
            for _ in range(n):
                fn()
            end.record()
        end.synchronize()
        return start.elapsed_time(end) / n

    out_ms = timed(lambda: pool.swap_out(device_blocks, host_blocks), iters)
    in_ms = timed(lambda: pool.swap_in(host_blocks, device_blocks), iters)
    flat_dev = torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda")
    flat_host = pool.host.view(-1)
    with torch.cuda.stream(stream):
        d2h_ms = timed(lambda: flat_host.copy_(flat_dev, non_blocking=True), iters)
        h2d_ms = timed(lambda: flat_dev.copy_(flat_host, non_blocking=True), iters)
    rows = pool.chunk_blocks * pool.slabs
    with torch.cuda.stream(stream):
        index = pool._upload_index(device_blocks[: pool.chunk_blocks])
        gather_ms = timed(lambda: ops.copy_rows_raw(pool.device_rows, index, pool.staging, None, rows), 20)
    gather_bytes = 2 * rows * pool.block_elems * 2

    def gbps(b: int, ms: float) -> float:
        return round(b / (ms * 1e-3) / 1e9, 1)

    return {"request": f"{16 * blocks} tokens, {blocks} blocks, {nbytes} bytes", "chunk_blocks": pool.chunk_blocks,
            "swap_out_ms": round(out_ms, 3), "swap_out_GBps": gbps(nbytes, out_ms),
            "swap_in_ms": round(in_ms, 3), "swap_in_GBps": gbps(nbytes, in_ms),
            "plain_d2h_GBps": gbps(nbytes, d2h_ms), "plain_h2d_GBps": gbps(nbytes, h2d_ms),
            "swap_out_frac_of_plain": round(d2h_ms / out_ms, 3), "swap_in_frac_of_plain": round(h2d_ms / in_ms, 3),
            "gather_kernel_us": round(gather_ms * 1e3, 2), "gather_kernel_GBps": gbps(gather_bytes, gather_ms)}


def run_pressure_modes(model, prompts, outputs, depths, num_blocks: int, unpressured_blocks: int,
                       safety_margin: float) -> dict:
    """The end-to-end workload on a cache of ``num_blocks`` under each preempting pressure mode,
    beside the same run (no warmup either) on a cache that needs no preemption."""

    import torch

    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine

    results = {}
    for mode, blocks, space in (("none", unpressured_blocks, None), ("recompute", num_blocks, None),
                                ("offload", num_blocks, 16.0)):
        margin = 0.2 if mode == "none" else safety_margin
        cfg = ContinuousDepthBatchingConfig(
            max_recurrent_steps=4, synthetic_exit_replay=True, delay_gate_consumption=False, kv_policy="single",
            refill=True, block_size=16, max_num_seqs=256, num_blocks=blocks, max_model_len=4096,
            kv_pressure_mode=mode, cpu_offload_space=space, safety_margin=margin)
        engine = ContinuousDepthBatchingEngine.from_model(model, cfg)
        engine.runner.capture_all_buckets()
        swap = engine.offloading_manager.swap
        if swap is not None:
            swap.record_timings = True
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        outs = engine.generate_batch(prompts, max_new_tokens=outputs, eos_token_id=None, exit_depths=depths)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        generated = sum(len(o.generated_tokens) for o in outs)
        stats = engine.last_stats
        results[mode] = {"tok_per_s": round(generated / elapsed, 1), "seconds": round(elapsed, 2),
                         "generated_tokens": generated, **engine.offloading_manager.preemption_stats(),
                         "prefill_batches": stats.prefill_batches, "prefill_tokens_recomputed":
                             sum(length for _, _, length in engine.offloading_manager.recompute_events),
                         "recurrent_batches": stats.recurrent_batches,
                         "mean_recurrent_batch": round(stats.mean_recurrent_batch_size, 1),
                         "coda_batches": stats.coda_batches, "scheduler_ticks": stats.scheduler_ticks,
                         "swap": swap.transfer_summary() if swap is not None else None}
        print(json.dumps({"pressure_mode_done": mode, **results[mode]}), flush=True)
        del engine
        torch.cuda.empty_cache()
    return results


def run_ouro_2p6b(num_seqs: int = 512) -> dict:
    """Ouro-2.6B shape (48 layers looped 4 steps), 512 sequences with the headline prompt, output
    and exit-depth distributions, timed with shared (``single``) and per-step KV, the latter both
    with the reference's slot-homogeneous launches and with mixed-slot launches.

    Single KV gets a pool sized for the whole batch. Per-step KV (``last_exited``: 192 cache
    layers, 1.5 MiB per token) needs about 2.5x this GPU's HBM for the batch, so its pool is
    sized from free device memory after the model is loaded (``mem_fraction_static`` 0.8) and
    KV pressure swaps decoders to a 64 GiB pinned host pool (``offload``; a soft reset would
    replace exit-step KV). Each engine captures its graphs and runs a short warmup first."""

    import torch

    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine
    from continuous_depth_batching_amd.ouro import OuroConfig, build_ouro

    cfg = OuroConfig(vocab_size=49152, hidden_size=2048, intermediate_size=5632, num_hidden_layers=48,
                     num_attention_heads=16, num_key_value_heads=16, head_dim=128, total_ut_steps=4,
                     max_position_embeddings=4096)
    model = build_ouro(cfg, seed=1, dtype=torch.bfloat16, device="cuda")
    prompts, outputs, depths = c2_workload(num_seqs, cfg.vocab_size)
    need = sum(-(-(len(p) + o + 1) // 16) for p, o in zip(prompts, outputs))
    runs = {}
    for name in ("single", "last_exited", "last_exited_mixed_slots"):
        policy = "single" if name == "single" else "last_exited"
        common = dict(max_recurrent_steps=4, synthetic_exit_replay=True, delay_gate_consumption=False,
                      kv_policy=policy, refill=True, block_size=16, max_num_seqs=num_seqs, max_model_len=4096,
                      mixed_slot_recurrent_batches=name.endswith("mixed_slots"))
        if policy == "single":
            extra = dict(num_blocks=int(need * 1.05) + 64, kv_pressure_mode="none")
        else:
            extra = dict(num_blocks=None, kv_pressure_mode="offload", cpu_offload_space=64.0)
        engine = ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(**common, **extra))
        engine.runner.capture_all_buckets()
        k = 32
        engine.generate_batch(prompts[:k], max_new_tokens=[min(o, 24) for o in outputs[:k]], eos_token_id=None,
                              exit_depths=[d[: min(o, 24) - 1] for d, o in zip(depths[:k], outputs[:k])])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        outs = engine.generate_batch(prompts, max_new_tokens=outputs, eos_token_id=None, exit_depths=depths)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        generated = sum(len(o.generated_tokens) for o in outs)
        stats = engine.last_stats
        om = engine.offloading_manager
        runs[name] = {
            "tok_per_s": round(generated / elapsed, 1), "seconds": round(elapsed, 2), "generated_tokens": generated,
            "num_blocks": engine.cache.num_blocks, "blocks_for_whole_batch": need,
            "kv_bytes_per_block": om.bytes_per_block(), "cache_layers": engine.cache.num_layers,
            "recurrent_batches": stats.recurrent_batches,
            "mean_recurrent_batch": round(stats.mean_recurrent_batch_size, 1), "coda_batches": stats.coda_batches,
            "prefill_batches": stats.prefill_batches, "exit_kv_copies": stats.exit_kv_copies,
            **om.preemption_stats()}
        print(json.dumps({"ouro_2p6b_done": name, **runs[name]}), flush=True)
        del engine, om
        torch.cuda.empty_cache()
    return runs


def run_huginn_0125(num_seqs: int = 128, new_tokens: int = 256) -> dict:
    """Huginn-0125 shape (hidden 5280, 55 heads x 96, prelude 2 + core 4 + coda 2 layers, MLP 17920,
    vocab 65536), random-init bf16, seed 1. 128 sequences: prompts lognormal(5.0, 0.9) in [8, 1024]
    with uniform ids, 256 new tokens each; per-token exit steps replayed from Poisson(12)
    truncated to [1, 32]; kv single; refill. The latent state starts from the reference's
    state_init="random" (truncated normal, seeded)."""

    import torch

    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine
    from continuous_depth_batching_amd.huginn import HuginnConfig, build_huginn
    from continuous_depth_batching_amd.workloads import huginn_decode_workload

    cfg = HuginnConfig(block_size=2048, state_init="random", state_seed=1)
    model = build_huginn(cfg, seed=1, dtype=torch.bfloat16, device="cuda", qk_bias_std=0.02)
    prompts, outputs, depths = huginn_decode_workload(num_seqs, new_tokens, cfg.vocab_size)
    need = sum(-(-(len(p) + o + 1) // 16) for p, o in zip(prompts, outputs))
    engine = ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(
        max_recurrent_steps=32, synthetic_exit_replay=True, delay_gate_consumption=False, kv_policy="single",
        refill=True, block_size=16, max_num_seqs=num_seqs, num_blocks=int(need * 1.05) + 64, max_model_len=2048,
        kv_pressure_mode="none"))
    engine.runner.capture_all_buckets()
    k = 16
    engine.generate_batch(prompts[:k], max_new_tokens=[16] * k, eos_token_id=None,
                          exit_depths=[d[:15] for d in depths[:k]])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    outs = engine.generate_batch(prompts, max_new_tokens=outputs, eos_token_id=None, exit_depths=depths)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    generated = sum(len(o.generated_tokens) for o in outs)
    stats = engine.last_stats
    return {"tok_per_s": round(generated / elapsed, 1), "seconds": round(elapsed, 2), "generated_tokens": generated,
            "recurrent_batches": stats.recurrent_batches, "mean_recurrent_batch": round(stats.mean_recurrent_batch_size, 1),
            "recurrent_steps": stats.recurrent_steps, "coda_batches": stats.coda_batches,
            "prefill_batches": stats.prefill_batches, "mean_exit_depth":
                round(sum(d + 1 for ds in depths for d in ds) / sum(len(ds) for ds in depths), 2)}


def cpu_baseline(model, prompts, outputs, depths, sample_tokens: int, engine_tokens: list[list[int]]) -> dict:
    """Numpy oracle decoding a bounded sample of the workload on the host cores; also compares its
    tokens with the engine's tokens for the same request (matched prefix before the first divergence)."""

    import torch

    from oracle.ouro_model import OuroOracle

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    weights = {k: v.detach().float().cpu().numpy() for k, v in model.state_dict().items()}
    cfg = model.config
    oracle = OuroOracle(weights, num_layers=cfg.num_hidden_layers, num_heads=cfg.num_attention_heads,
                        num_kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, rope_theta=cfg.rope_theta,
                        eps=cfg.rms_norm_eps, dtype="bf16", max_positions=4096)
    # The shortest prompt among requests generating at least sample_tokens keeps the full-depth
    # prefill small, so most of the sample is decode.
    eligible = [i for i, o in enumerate(outputs) if o >= sample_tokens] or [int(np.argmax(outputs))]
    idx = min(eligible, key=lambda i: len(prompts[i]))
    n = min(sample_tokens, outputs[idx])
    t0 = time.perf_counter()
    out = oracle.generate(prompts[idx], n, max_steps=cfg.total_ut_steps, kv_policy="single",
                          exit_depths=depths[idx][: n - 1])
    dt = time.perf_counter() - t0
    got = engine_tokens[idx][: len(out.tokens)]
    matched = 0
    while matched < len(got) and got[matched] == out.tokens[matched]:
        matched += 1
    # Teacher-forced with the engine's tokens (untimed), against the oracle with fp64 projection
    # accumulation: at every step, whether the engine's token is that oracle's argmax and how far
    # below its best logit it sits. On this untrained model the top logits crowd together, so bf16
    # rounding noise flips greedy choices between any two correct implementations. The same
    # statistics for the fp32-accumulating oracle (forced with the same tokens) measure that noise:
    # an engine close to them differs from the fp64 oracle by rounding, not by a defect.
    # The forced passes cover the first FORCED_TOKENS tokens only: they are a check, not the
    # timed sample, and the GPU idles while they run.
    from oracle.ouro_model import forced_choice_stats

    nf = min(len(got), FORCED_TOKENS)
    steps = cfg.total_ut_steps
    wide = OuroOracle(weights, num_layers=cfg.num_hidden_layers, num_heads=cfg.num_attention_heads,
                      num_kv_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim, rope_theta=cfg.rope_theta,
                      eps=cfg.rms_norm_eps, dtype="bf16", max_positions=4096, accumulate="f64")
    ref = wide.forced_logits(prompts[idx], got[:nf], max_steps=steps, exit_depths=depths[idx])
    del wide
    narrow = oracle.forced_logits(prompts[idx], got[:nf], max_steps=steps, exit_depths=depths[idx])
    engine_vs_f64 = forced_choice_stats(ref, got[:nf])
    oracle_vs_f64 = forced_choice_stats(ref, narrow.argmax(axis=1).tolist())
    engine_vs_f32 = forced_choice_stats(narrow, got[:nf])
    rnd4 = lambda d: {k: round(v, 4) for k, v in d.items()}
    return {"value": len(out.tokens) / dt, "unit": "output tok/s", "cores": threads, "kind": "port",
            "sample": f"request {idx} of the workload (prompt {len(prompts[idx])} tokens): full-depth prefill "
                      f"+ {len(out.tokens)} generated tokens with its replayed exit depths, one request at a time "
                      f"in numpy (bf16-rounded fp32), {dt:.1f} s",
            "parity": {"request": idx, "tokens_compared": len(out.tokens), "matched_prefix": matched,
                       "matched_prefix_frac": round(matched / len(out.tokens), 4),
                       "first_token_equal": bool(got and got[0] == out.tokens[0]),
                       "teacher_forced_tokens": nf,
                       "engine_vs_f64_oracle": rnd4(engine_vs_f64),
                       "oracle_f32_vs_f64_oracle": rnd4(oracle_vs_f64),
                       "engine_vs_f32_oracle": rnd4(engine_vs_f32),
                       "oracle_self_agreement": round(oracle_vs_f64["argmax_agreement"], 4),
                       "oracle_self_max_margin": round(oracle_vs_f64["max_logit_margin"], 4),
                       "logit_std": round(float(ref.std(axis=1).mean()), 4),
                       "note": "bf16 greedy streams of an untrained model diverge on rounding noise; teacher-"
                               "forced with the engine's tokens, the engine's argmax agreement with the fp64-"
                               "accumulating oracle and its logit margins (oracle max logit minus the oracle "
                               "logit of the chosen token, against logits whose spread is logit_std) stand next "
                               "to the same figures for the fp32-accumulating oracle, which is the size of that "
                               "noise"}}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the CDB decode step is built "
                                   "for one GPU's share and has no multi-GPU path"}))
        return 2
    import torch

    from continuous_depth_batching_amd import workloads
    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine
    from continuous_depth_batching_amd.ouro import build_ouro

    device = torch.device("cuda")
    cfg = ouro_1p4b_config()
    prompts, outputs, depths = c2_workload(args.num_seqs, cfg.vocab_size)
    result: dict = {}
    blocks = int(sum(-(-(len(p) + o + 1) // 16) for p, o in zip(prompts, outputs)) * 1.05) + 64

    if args.workload == "huginn":
        run = run_huginn_0125()
        print(json.dumps({"metric": "output tok/s, Huginn-0125-shape CDB decode bs=128, 32 loop steps",
                          "value": run["tok_per_s"], "unit": "output tok/s", "n_gpus": 1, "dtype": "bf16",
                          "data": "synthetic", "run": run}))
        return 0

    if args.workload == "ouro-2p6b":
        runs = run_ouro_2p6b()
        print(json.dumps({"metric": "output tok/s, Ouro-2.6B-shape CDB decode bs=512, single vs per-step KV",
                          "value": runs["single"]["tok_per_s"], "unit": "output tok/s", "n_gpus": 1,
                          "dtype": "bf16", "data": "synthetic", "runs": runs}))
        return 0

    if args.workload == "kv-pressure":
        swap = time_kv_swap()
        line = {"metric": "KV swap-out host-link GB/s (4096-token Ouro-1.4B request)",
                "value": swap["swap_out_GBps"], "unit": "GB/s", "n_gpus": 1, "kv_swap": swap}
        if not args.swap_only:
            print(json.dumps({"kv_swap": swap}), flush=True)
            model = build_ouro(cfg, seed=1, dtype=torch.bfloat16, device=device)
            pressured = int(blocks * args.pressure_fraction)
            modes = run_pressure_modes(model, prompts, outputs, depths, pressured, blocks,
                                       args.pressure_safety_margin)
            line["pressure"] = {"num_blocks": pressured, "unpressured_num_blocks": blocks,
                                "fraction": args.pressure_fraction, "safety_margin": args.pressure_safety_margin,
                                "modes": modes}
        print(json.dumps(line))
        return 0

    rows = args.attention_rows if args.workload == "decode-attention" else None
    if rows is not None and not 1 <= rows <= len(prompts):
        raise SystemExit(f"--attention-rows must be in [1, {len(prompts)}]")
    attention = time_decode_attention(decode_attention_c2_case(prompts, outputs, device, rows),
                                      split_pages=0, iters=args.attention_iters)
    torch.cuda.empty_cache()
    roofline = {"bound": "hbm", "achieved": round(attention["gbps"], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(attention["gbps"] / HBM_PEAK_GBPS, 4), "traffic": measured_traffic(attention["bytes"]),
                "traffic_source": f"{TRAFFIC_RECORD}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on this shape, "
                                  "scaled by a 1 GiB copy",
                "kernel": decode_kernels(attention["rows"]) + " (one layer's attend)",
                "launch_ms": round(attention["ms"], 4), "algorithmic_bytes": attention["bytes"],
                "plan_ms": round(attention["plan_ms"], 4),
                "plan_note": "cdb::decode_plan_kernel runs once per recurrent launch for all 24 layers",
                "shape": f"{attention['rows']} rows x 16 heads x 128, mean context {attention['mean_context']:.0f}"}
    micro = None
    if not args.no_microbench:
        case = workloads.decode_attention_microbench(num_rows=1024, ctx_min=128, ctx_max=8192, num_slots=4)
        m = time_decode_attention(case, split_pages=0, iters=max(5, args.attention_iters // 2))
        micro = {"ms": round(m["ms"], 4), "GBps": round(m["gbps"], 1), "frac": round(m["gbps"] / HBM_PEAK_GBPS, 4),
                 "bytes": m["bytes"], "shape": "1024 rows x 16 heads x 128, ctx U[128,8192], 4 loop slots"}
        del case
        torch.cuda.empty_cache()

    companions = None
    if not args.no_microbench:
        companions = time_companion_kernels(prefill_tokens=int(sum(first_prefill_batch(prompts))))
    projections = time_decode_projections()
    prefill = time_prefill_attention(first_prefill_batch(prompts), iters=max(3, args.attention_iters // 4))
    prefill["shape"] = (f"{prefill['sequences']} fresh prompts, {prefill['tokens']} tokens (max {prefill['max_len']}), "
                        "16 heads x 128, causal")
    prefill_history = time_prefill_attention([128] * 4, iters=max(3, args.attention_iters // 4), past=[16000] * 4)
    prefill_history["shape"] = "4 sequences x 128 new tokens after 16000 cached positions, 16 heads x 128"
    torch.cuda.empty_cache()

    if args.workload == "decode-attention":
        print(json.dumps({"metric": "decode-attention HBM GB/s", "value": roofline["achieved"], "unit": "GB/s",
                          "n_gpus": 1, "roofline": roofline, "decode_attention_microbench": micro,
                          "companion_kernels_1024": companions, "prefill_attention": prefill,
                          "prefill_attention_after_history": prefill_history,
                          "decode_projections": projections, "copy_calibration": copy_calibration()}))
        return 0

    model = build_ouro(cfg, seed=1, dtype=torch.bfloat16, device=device)
    engine_cfg = ContinuousDepthBatchingConfig(
        max_recurrent_steps=4, synthetic_exit_replay=True, delay_gate_consumption=False, kv_policy="single",
        refill=True, block_size=16, max_num_seqs=256, num_blocks=blocks, max_model_len=4096,
        kv_pressure_mode="none")
    engine = ContinuousDepthBatchingEngine.from_model(model, engine_cfg)
    engine.runner.capture_all_buckets()
    # The reference's steady-state window (benchmarks/runner.py:592-596): opens once twice the
    # resident cap of requests have completed while prompts still wait.
    engine.scheduler.steady_warmup_requests = 2 * engine_cfg.max_num_seqs
    for _ in range(args.warmup):
        k = min(32, len(prompts))
        engine.generate_batch(prompts[:k], max_new_tokens=[min(o, 24) for o in outputs[:k]], eos_token_id=None,
                              exit_depths=[d[: min(o, 24) - 1] for d, o in zip(depths[:k], outputs[:k])])
    torch.cuda.synchronize()
    generated = 0
    with GpuActivity() as activity:
        t0 = time.perf_counter()
        for _ in range(args.steps):
            outs = engine.generate_batch(prompts, max_new_tokens=outputs, eos_token_id=None, exit_depths=depths)
            generated += sum(len(o.generated_tokens) for o in outs)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
    stats = engine.last_stats
    steady = engine.scheduler.steady_state_summary()
    value = generated / elapsed
    run_weighted = by_rows = None
    if not args.no_microbench:
        # One more (untimed) run records every recurrent launch's row positions; decode attention
        # is then timed over exactly those launches, and at fixed widths of the same contexts.
        launches: list[np.ndarray] = []
        launch = engine.runner.compute_recurrent_batch

        def recorded(items):
            launches.append(np.fromiter((it.token_position for it in items), np.int32, len(items)))
            return launch(items)

        engine.runner.compute_recurrent_batch = recorded
        engine.generate_batch(prompts, max_new_tokens=outputs, eos_token_id=None, exit_depths=depths)
        engine.runner.compute_recurrent_batch = launch
        torch.cuda.synchronize()
        run_weighted = run_weighted_decode(launches)
        mid = np.asarray([len(p) + max(1, o // 2) - 1 for p, o in zip(prompts, outputs)], dtype=np.int32)
        by_rows = time_by_rows({n: mid[:n] for n in (1, 4, 16, 32, 64, 128, 256)})
    result.update({
        "metric": "output tok/s, Ouro-1.4B-shape CDB decode bs=256; decode-attn HBM GB/s % of peak",
        "value": round(value, 1),
        "unit": "output tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, uniform token ids, seeded lognormal lengths and exit trace)",
        "config": {"workload": "Ouro-1.4B-shape CDB decode: 256 seqs, prompts lognormal(5.5,1.0)[8,2048], "
                               "outputs lognormal(5.0,0.8)[16,1024], exit depths {1:.15,2:.25,3:.30,4:.30}, "
                               "refill, block 16, kv single",
                   "global_batch": args.num_seqs, "parallelism": "none"},
        "roofline": roofline,
        "decode_attention_run_weighted": run_weighted,
        "decode_attention_by_rows": by_rows,
        "decode_attention_microbench": micro,
        "companion_kernels_1024": companions,
        "prefill_attention": prefill,
        "prefill_attention_after_history": prefill_history,
        "decode_projections": projections,
        "engine": {"generated_tokens": generated, "recurrent_batches": stats.recurrent_batches,
                   "mean_recurrent_batch": round(stats.mean_recurrent_batch_size, 1),
                   "coda_batches": stats.coda_batches, "prefill_batches": stats.prefill_batches,
                   "recurrent_steps": stats.recurrent_steps, "skipped_recurrent_steps": stats.skipped_recurrent_steps,
                   "graph_captures_in_timed_run": stats.recurrent_graph_captures},
        "steady_window": steady,
        "gpu_activity_timed": activity.summary(),
    })
    if steady is None:
        result["steady_window_note"] = ("the reference's steady-state window (after 2 x max_num_seqs completions, "
                                        "while prompts wait) never opened: no prompt was still waiting by then")
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(model, prompts, outputs, depths, args.cpu_sample_tokens,
                                              [o.generated_tokens for o in outs])
        result["matched_prefix_frac"] = result["cpu_baseline"]["parity"]["matched_prefix_frac"]
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
