"""CDB stage runner: device buffers, hidden-state bank, HIP graphs, readbacks.

Counterpart of continuous_depth_batching/model_runner.py. Differences that
follow from the MI355X design:
  * the hidden-state bank and the exit-gate state are fixed-capacity device
    arrays indexed by hidden slot; slots are handed out LIFO from a free list,
    then by monotonic growth, exactly like the reference (:1193-1203), so slot
    assignment is reproducible;
  * a recurrent launch uploads one packed int32 and one int64 metadata buffer
    (bank slots, positions, block-table rows, cache-layer offsets, steps,
    replayed depths); block tables stay resident on the device;
  * the whole recurrent stage -- bank gather, every layer, bank scatter and
    the exit decision -- is one HIP graph per batch bucket (captured on first
    use of the bucket); padding rows carry slot -1 / position -1 and are no-ops
    in every kernel;
  * exit decisions come back as one byte per row.
"""

from __future__ import annotations

import gc
from contextlib import contextmanager, nullcontext
from dataclasses import dataclass, field
from typing import Any, Callable, Iterator, Sequence

import numpy as np
import torch

from . import ops
from .cache import PagedKVCache
from .config import ContinuousDepthBatchingConfig
from .exit_policy import ExitDecisionRule, ExitPolicy
from .model_adapter import CDBModelAdapter, GateLaunch, PrefillLaunch, RecurrentLaunch, StageLaunch
from .offloading import KvSwapPool
from . import _tick
from .requests import TMP_TOKEN_ID, DepthWorkItem, FutureRequestState

CODA_PIPELINE_DEPTH = 2


def decode_graph_buckets(max_num_seqs: int) -> list[int]:
    """Batch buckets of the decode graphs (continuous_batching/utils.py:65-76)."""

    buckets = {1, 2, 4, 8, 12}
    buckets.update(range(16, min(256, max_num_seqs) + 1, 8))
    if max_num_seqs > 256:
        buckets.update(range(272, min(512, max_num_seqs) + 1, 16))
    if max_num_seqs > 512:
        buckets.update(range(544, max_num_seqs + 1, 32))
    buckets.add(max_num_seqs)
    return sorted(b for b in buckets if b <= max_num_seqs)


def pad_to_bucket(n: int, buckets: Sequence[int]) -> int:
    for b in buckets:
        if b >= n:
            return b
    raise ValueError(f"batch of {n} exceeds the largest bucket {buckets[-1]}")


@contextmanager
def gc_paused() -> Iterator[None]:
    enabled = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if enabled:
            gc.enable()


@dataclass
class PendingCodaResult:
    items: list[DepthWorkItem]
    host_tokens: torch.Tensor
    device_tokens: torch.Tensor | None = None
    ready_event: Any | None = None
    eager_reentries: list[bool] | None = None

    def is_ready(self) -> bool:
        return self.ready_event is None or self.ready_event.query()


@dataclass
class PendingPrefillResult:
    futures: list[FutureRequestState]
    host_tokens: torch.Tensor
    device_tokens: torch.Tensor | None = None
    ready_event: Any | None = None
    eager_entries: list[bool] | None = None

    def is_ready(self) -> bool:
        return self.ready_event is None or self.ready_event.query()


@dataclass
class PendingFlags:
    """Exit decisions of one launch, on their way to the host: one byte per row, or, when the
    device routed the launch (cdb_route_compact), the lists [n_exit, n_stay, exiting rows,
    staying rows] in launch order."""

    host: torch.Tensor | None
    event: Any | None
    lists: torch.Tensor | None = None
    _values: list[int] | None = None

    def _landed(self) -> None:
        if self.event is not None:
            self.event.synchronize()
            self.event = None

    def wait(self) -> np.ndarray:
        """The decision bytes, once the launch has written them (one per row, then padding)."""

        self._landed()
        if self.host is None:
            lists = self.lists.numpy()
            flags = np.zeros(int(lists[0]) + int(lists[1]), np.uint8)
            flags[lists[2:2 + int(lists[0])]] = 1
            return flags
        return self.host.numpy()

    def routing_lists(self) -> np.ndarray:
        """The device's routing lists, once the launch has written them."""

        self._landed()
        return self.lists.numpy()

    def get(self, index: int) -> bool:
        values = self._values
        if values is None:
            # Wait once, then read the bytes as a Python list: per-row tensor indexing costs
            # microseconds each on the routing path.
            values = self._values = self.wait().tolist()
        return bool(values[index])


@dataclass
class PrefillMetadata:
    tokens: np.ndarray       # [T] int64 chunk tokens
    positions: np.ndarray    # [T] int32
    write_rows: np.ndarray   # [T] int64 pool rows
    cu_q: np.ndarray         # [S+1] int32
    past: np.ndarray         # [S] int32
    table_rows: np.ndarray   # [S] int32
    lens: list[int]
    last_index: np.ndarray   # [N] int64 sampling rows


@dataclass
class _RecurrentBucket:
    rows: int
    # pinned int32: the int64 bank slots (2 * rows), the int32 rows (5 * rows), then the
    # block-table updates the launch carries: [count, pad | int64 cells (U) | int32 values (U)]
    host_meta: torch.Tensor
    dev_meta: torch.Tensor
    host_i64: torch.Tensor   # views of host_meta / dev_meta
    host_i32: torch.Tensor
    dev_i64: torch.Tensor
    dev_i32: torch.Tensor
    launch: RecurrentLaunch
    host_upd_count: Any = None  # numpy views of the update region
    host_upd_idx: Any = None
    host_upd_val: Any = None
    dev_upd_count: torch.Tensor | None = None
    dev_upd_idx: torch.Tensor | None = None
    dev_upd_val: torch.Tensor | None = None
    staged: Any | None = None
    graph: torch.cuda.CUDAGraph | None = None
    turn: int = 0
    host_flags: list[torch.Tensor] = field(default_factory=list)
    flag_events: list[Any] = field(default_factory=list)
    dev_lists: torch.Tensor | None = None  # cdb_route_compact output of the launch
    host_lists: list[torch.Tensor] = field(default_factory=list)


@dataclass
class _CodaTurn:
    host_upload: torch.Tensor  # pinned int64: coda slots | successor slots | successors' own slots
    dev_upload: torch.Tensor
    host_tokens: torch.Tensor  # pinned int64 greedy tokens
    event: Any
    direct: ops.CodaScratch | None = None  # one-call coda of up to CODA_DIRECT_MAX_ROWS rows
    upload_addr: int = 0  # host_upload.data_ptr()


class ModelRunner:
    META_POSITIONS, META_TABLE_ROWS, META_LAYER_OFFSET, META_STEPS, META_SYNTHETIC = range(5)
    FLAG_TURNS = 4
    CODA_TURNS = 4
    # Block-table cell updates a recurrent launch carries in its metadata upload and applies
    # inside its graph; more queued updates than this take the separate flush first.
    TABLE_UPDATE_SLOTS = 256

    def __init__(self, *, engine_config: ContinuousDepthBatchingConfig, cache: PagedKVCache,
                 model_adapter: CDBModelAdapter, exit_policy: ExitPolicy) -> None:
        self.engine_config = engine_config
        self.cache = cache
        self.adapter = model_adapter
        self.exit_policy = exit_policy
        # On the synchronous horizon the device routes each launch's rows (exit and stay lists in
        # launch order); on the delayed one the host reads each row's decision a launch later.
        self.device_routing = not exit_policy.delayed()
        self.device = cache.device
        self.dtype = model_adapter.dtype
        self.max_num_seqs = engine_config.max_num_seqs
        self.decode_graph_buckets = decode_graph_buckets(self.max_num_seqs)
        self.use_graphs = bool(engine_config.use_cuda_graph)
        self.layout = cache.layout
        self.stream = torch.cuda.Stream(device=self.device)
        self._stream_handle = self.stream.cuda_stream
        self._device_index = self.stream.device_index
        self.bank_capacity = 4 * self.max_num_seqs + 64
        self.bank = torch.zeros((self.bank_capacity, model_adapter.hidden_width), dtype=self.dtype,
                                device=self.device)
        self.gate_state = ops.GateState.allocate(self.bank_capacity, self.device)
        self.free_hidden_slots: list[int] = []
        self.next_hidden_slot = 0
        max_bucket = self.decode_graph_buckets[-1]
        num_kv_heads, head_dim = model_adapter.kv_geometry()
        # Decode attention sizes its KV splits on the device (the count of pages in the launch is
        # only known there); the workspace holds the partials of the finest split of the largest bucket.
        num_heads = max(model_adapter_num_heads(model_adapter), 1)
        ws_bytes = ops.decode_workspace_bytes(max_bucket, num_heads, head_dim, engine_config.max_model_len,
                                              cache.block_size, ops.MIN_SPLIT_PAGES)
        del num_kv_heads
        self.workspace = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=self.device)
        # bf16 prefill attention splits long tiles over several workgroups (ops.prefill_split_work);
        # the parts' partial results live in a buffer grown on demand on the runner's stream.
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_cus = torch.cuda.get_device_properties(self.device).multi_processor_count
        self.partials = torch.empty(0, dtype=torch.float32, device=self.device)
        self._buckets: dict[int, _RecurrentBucket] = {}
        self.graph_pool = torch.cuda.graph_pool_handle() if self.use_graphs else None
        spec = model_adapter.exit_policy_spec()
        self.gate_rule = ops.RULE_DIRECT_THRESHOLD if spec.rule is ExitDecisionRule.DIRECT_THRESHOLD \
            else ops.RULE_CUMULATIVE_HAZARD
        self.recurrent_graph_hits = 0
        self.recurrent_graph_captures = 0
        self.stage_graph_hits = 0
        self.stage_graph_captures = 0
        self._coda_turns: list[_CodaTurn | None] = [None] * self.CODA_TURNS
        self._coda_turn_index = 0
        self._coda_weights = model_adapter.coda_weights() if self.dtype is torch.bfloat16 else None
        # The cache, bank and workspace above were filled on the caller's stream; the compute
        # stream must not run ahead of those fills (a block table still being set to -1 while
        # the first prefill reads it).
        self.stream.wait_stream(torch.cuda.current_stream(self.device))

    # -- hidden slots (cdb/model_runner.py:1193-1203, 1359-1363) ------------------------------------------------
    def reset_cdb_runtime_counters(self) -> None:
        self.recurrent_graph_hits = self.recurrent_graph_captures = 0
        self.stage_graph_hits = self.stage_graph_captures = 0
        self.free_hidden_slots = []
        self.next_hidden_slot = 0

    def allocate_hidden_slots(self, count: int) -> list[int]:
        slots = []
        while self.free_hidden_slots and len(slots) < count:
            slots.append(self.free_hidden_slots.pop())
        while len(slots) < count:
            if self.next_hidden_slot >= self.bank_capacity:
                raise RuntimeError(f"hidden-state bank exhausted ({self.bank_capacity} slots)")
            slots.append(self.next_hidden_slot)
            self.next_hidden_slot += 1
        return slots

    def release_hidden_slots(self, items: list[DepthWorkItem]) -> None:
        for item in items:
            if item.hidden_slot is not None:
                self.free_hidden_slots.append(item.hidden_slot)
                item.hidden_slot = None

    # -- helpers --------------------------------------------------------------------------------------------------
    def stream_scope(self):
        """Make the compute stream current for a whole generate_batch, so the per-call
        scopes below find it already set. Work the caller queued before (on its own stream)
        is ordered before everything the call runs."""

        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        return torch.cuda.stream(self.stream)

    def _on_stream(self):
        """Scope of one runner call on the compute stream: free when it is already current."""

        if torch._C._cuda_getCurrentRawStream(self._device_index) == self._stream_handle:
            return nullcontext()
        self.stream.wait_stream(torch.cuda.current_stream(self.device))
        return torch.cuda.stream(self.stream)

    def _pinned(self, shape: tuple[int, ...] | int, dtype: torch.dtype) -> torch.Tensor:
        return torch.empty(shape, dtype=dtype, pin_memory=True)

    def _prefill_partials(self, num_slots: int) -> torch.Tensor:
        """The split prefill's partial-result buffer for `num_slots` slots (call on the runner's stream)."""

        need = -(-ops.prefill_partial_bytes(num_slots, self.num_heads, self.head_dim) // 4)
        if self.partials.numel() < need:
            self.partials = torch.empty(need, dtype=torch.float32, device=self.device)
        return self.partials

    def _to_device(self, array: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
        host = self._pinned(array.shape, dtype)
        host.numpy()[...] = array
        return host.to(self.device, non_blocking=True)

    # -- prelude ---------------------------------------------------------------------------------------------------
    def compute_prelude_batch(self, items: list[DepthWorkItem],
                              device_groups: Sequence[tuple[Any, list[int]]] = ()) -> None:
        """Embed the items' tokens into fresh bank slots; the first ``sum(len(rows))`` items take their
        token from the staged results' device tokens (cdb/model_runner.py:395-463)."""

        if not items:
            return
        n = len(items)
        num_device = sum(len(rows) for _, rows in device_groups)
        if any(item.token_id != TMP_TOKEN_ID for item in items[:num_device]):
            raise AssertionError("device_groups must cover a prefix of items")
        slots = self.allocate_hidden_slots(n)
        # One upload: [bank slots (n) | tokens (n) | each device group's row indices]. The first
        # num_device token entries are placeholders, overwritten on the device by gathers from the
        # staged results' device tokens; the rest are the host token ids.
        upload = np.empty(2 * n + num_device, dtype=np.int64)
        upload[:n] = slots
        upload[n:n + num_device] = 0
        upload[n + num_device:2 * n] = [item.token_id for item in items[num_device:]]
        offset = 2 * n
        for _, rows in device_groups:
            upload[offset:offset + len(rows)] = rows
            offset += len(rows)
        with self._on_stream():
            dev = self._to_device(upload, torch.int64)
            slot_dev, tokens = dev[:n], dev[n:2 * n]
            offset, index = 0, 2 * n
            for result, rows in device_groups:
                if result.device_tokens is None:
                    raise RuntimeError("Cannot gather prelude tokens from a staged result that carries none")
                k = len(rows)
                ops.copy_rows_raw(result.device_tokens.view(-1, 1), dev[index:index + k],
                                  tokens[offset:offset + k].view(-1, 1), None, k)
                offset += k
                index += k
            self.adapter.prelude(self._stage_launch(items, slot_dev, tokens=tokens))
            self.gate_state.reset(slot_dev, n)
        for item, slot in zip(items, slots):
            item.hidden_slot = slot

    def _stage_launch(self, items: list[DepthWorkItem], slots: torch.Tensor,
                      tokens: torch.Tensor | None = None) -> StageLaunch:
        """Prelude/coda inputs; stages with attention also get positions, table rows and the
        cache, with pending block-table updates applied first."""

        launch = StageLaunch(n=len(items), bank=self.bank, slots=slots, tokens=tokens)
        if self.adapter.stages_use_attention:
            self.cache.flush_table_updates()
            row_of = self.cache.table_row_of
            launch.positions = self._to_device(np.fromiter((it.token_position for it in items), dtype=np.int32,
                                                           count=len(items)), torch.int32)
            launch.table_rows = self._to_device(np.fromiter((row_of[it.state.request_id] for it in items),
                                                            dtype=np.int32, count=len(items)), torch.int32)
            launch.cache = self.cache
            launch.workspace = self.workspace
            launch.split_pages = ops.decode_split_pages(len(items))
        return launch

    # -- recurrent stage -------------------------------------------------------------------------------------
    def _bucket(self, rows: int) -> _RecurrentBucket:
        b = self._buckets.get(rows)
        if b is not None:
            return b
        # One pinned buffer and one device buffer per bucket, so a launch uploads its
        # metadata with a single copy.
        u = self.TABLE_UPDATE_SLOTS
        base = 7 * rows + (7 * rows) % 2  # the int64 cells start 8-byte aligned
        total = base + 2 + 3 * u
        host_meta = self._pinned((total,), torch.int32)
        host_meta.zero_()
        dev_meta = torch.zeros((total,), dtype=torch.int32, device=self.device)
        host_i64, host_i32 = host_meta[:2 * rows].view(torch.int64), host_meta[2 * rows:7 * rows].view(5, rows)
        dev_i64, dev_i32 = dev_meta[:2 * rows].view(torch.int64), dev_meta[2 * rows:7 * rows].view(5, rows)
        dev_i64.fill_(-1)
        dev_i32[self.META_POSITIONS].fill_(-1)
        dev_i32[self.META_SYNTHETIC].fill_(-1)
        policy = self.exit_policy
        gate = GateLaunch(
            state=self.gate_state,
            steps=dev_i32[self.META_STEPS],
            synthetic=dev_i32[self.META_SYNTHETIC],
            flags=torch.zeros(rows, dtype=torch.uint8, device=self.device),
            signal=torch.zeros(rows, dtype=self.dtype, device=self.device),
            rule=self.gate_rule,
            # The synchronous path reads the model-dtype hazard; the delayed path the fp32 one
            # (cdb/model_runner.py:807-813 vs continuous_api.py:1693-1697).
            round_hazard=policy.round_hazard,
            min_steps=policy.min_recurrent_steps,
            max_steps=policy.max_recurrent_steps,
            threshold=policy.threshold,
        )
        launch = RecurrentLaunch(
            rows=rows, bank=self.bank, bank_slots=dev_i64, positions=dev_i32[self.META_POSITIONS],
            table_rows=dev_i32[self.META_TABLE_ROWS], slot_offset=dev_i32[self.META_LAYER_OFFSET],
            cache=self.cache, workspace=self.workspace,
            split_pages=ops.decode_split_pages(rows), gate=gate)
        b = _RecurrentBucket(rows=rows, host_meta=host_meta, dev_meta=dev_meta, host_i64=host_i64,
                             host_i32=host_i32, dev_i64=dev_i64, dev_i32=dev_i32, launch=launch)
        hn = host_meta.numpy()
        b.host_upd_count = hn[base:base + 1]
        b.host_upd_idx = hn[base + 2:base + 2 + 2 * u].view(np.int64)
        b.host_upd_val = hn[base + 2 + 2 * u:total]
        b.dev_upd_count = dev_meta[base:base + 1]
        b.dev_upd_idx = dev_meta[base + 2:base + 2 + 2 * u].view(torch.int64)
        b.dev_upd_val = dev_meta[base + 2 + 2 * u:total]
        b.host_flags = [self._pinned((rows,), torch.uint8) for _ in range(self.FLAG_TURNS)]
        b.flag_events = [None] * self.FLAG_TURNS
        if self.device_routing:
            b.dev_lists = torch.zeros(2 + rows, dtype=torch.int32, device=self.device)
            b.host_lists = [self._pinned((2 + rows,), torch.int32) for _ in range(self.FLAG_TURNS)]
        self._buckets[rows] = b
        return b

    def compute_recurrent_batch(self, items: list[DepthWorkItem]) -> PendingFlags:
        """One recurrent step over ``items``; returns their exit decisions (host-visible later)."""

        if not items:
            raise ValueError("items must not be empty")
        n = len(items)
        rows = pad_to_bucket(n, self.decode_graph_buckets)
        b = self._bucket(rows)
        if b.staged is not None:
            b.staged.synchronize()  # the previous upload from these pinned buffers has completed
        self.fill_recurrent_metadata(items, b.host_i64.numpy(), b.host_i32.numpy())
        turn = b.turn
        b.turn = (turn + 1) % self.FLAG_TURNS
        if b.flag_events[turn] is not None:
            b.flag_events[turn].synchronize()
        with self._on_stream():
            # The block-table cells changed since the last launch ride in this launch's metadata
            # upload and are applied by the graph's first kernel; a larger backlog is flushed first.
            count = self.cache.take_table_updates(b.host_upd_idx, b.host_upd_val)
            if count is None:
                self.cache.flush_table_updates()
                count = 0
            b.host_upd_count[0] = count
            b.dev_meta.copy_(b.host_meta, non_blocking=True)
            if b.staged is None:
                b.staged = torch.cuda.Event()
            b.staged.record()
            self._run_recurrent(b)
            if self.device_routing:
                # The graph's last kernel routed the rows: one copy of the lists.
                host_lists = b.host_lists[turn][:2 + n]
                host_lists.copy_(b.dev_lists[:2 + n], non_blocking=True)
                host_flags = None
            else:
                host_lists = None
                host_flags = b.host_flags[turn]
                host_flags[:n].copy_(b.launch.gate.flags[:n], non_blocking=True)
            event = b.flag_events[turn]
            if event is None:
                event = b.flag_events[turn] = torch.cuda.Event()
            event.record()
        return PendingFlags(host=host_flags, event=event, lists=host_lists)

    def fill_recurrent_metadata(self, items: list[DepthWorkItem], i64: np.ndarray, i32: np.ndarray) -> None:
        """Host metadata of one recurrent launch over a bucket of ``len(i64)`` rows.

        i64[r]: bank slot of row r; i32[META_*, r]: position, block-table row, cache layer of
        core layer 0 at the row's step (prelude + slot * core layers), loop step, replayed
        exit depth (-1: none or gate not applied). Rows past ``len(items)`` are padding:
        slot -1 and position -1 make every kernel skip them
        (cdb/model_runner.py:704-754 assembles the same per-row facts)."""

        _tick.fill_recurrent(items, i64, i32, self.cache.table_row_of, self.layout.core_base,
                             self.layout.num_core_layers, self.layout.step_slots)

    def capture_all_buckets(self, buckets: Sequence[int] | None = None) -> int:
        """Capture the recurrent-stage graph of every bucket ahead of time.

        Each capture's eager pass runs an all-padding launch (bank slot -1, position
        -1, no gate state), which every kernel treats as a no-op, so warming up
        changes neither the KV pool, the bank nor the gate state."""

        if not self.use_graphs:
            return 0
        captured = 0
        for rows in buckets or self.decode_graph_buckets:
            b = self._bucket(rows)
            if b.graph is not None:
                continue
            if b.staged is not None:
                b.staged.synchronize()
            i32 = b.host_i32.numpy()
            b.host_i64.numpy()[:] = -1
            i32[self.META_POSITIONS] = -1
            i32[self.META_TABLE_ROWS] = 0
            i32[self.META_LAYER_OFFSET] = self.layout.core_base
            i32[self.META_STEPS] = 0
            i32[self.META_SYNTHETIC] = -1
            b.host_upd_count[0] = 0
            with self._on_stream():
                b.dev_meta.copy_(b.host_meta, non_blocking=True)
                if b.staged is None:
                    b.staged = torch.cuda.Event()
                b.staged.record()
                self._run_recurrent(b)
            captured += 1
        self.stream.synchronize()
        self.recurrent_graph_captures = 0
        return captured

    def _apply_table_updates(self, b: _RecurrentBucket) -> None:
        ops.table_updates_raw(self.cache.device_table, b.dev_upd_idx, b.dev_upd_val, b.dev_upd_count,
                              self.TABLE_UPDATE_SLOTS)

    def _recurrent_body(self, b: _RecurrentBucket) -> None:
        """One recurrent launch on the device: the block-table cells it carries, the loop step with
        its exit gate, and on the synchronous horizon the routing lists of its rows."""

        self._apply_table_updates(b)
        self.adapter.recurrent_step(b.launch)
        if self.device_routing:
            torch.ops.cdb.route_compact(b.launch.gate.flags, b.launch.bank_slots, b.dev_lists)

    def _run_recurrent(self, b: _RecurrentBucket) -> None:
        if not self.use_graphs:
            self._recurrent_body(b)
            return
        if b.graph is not None:
            self.recurrent_graph_hits += 1
            b.graph.replay()
            return
        # First use of this bucket: run it eagerly (this launch's real work), then capture.
        with gc_paused():
            self._recurrent_body(b)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=self.stream, pool=self.graph_pool, capture_error_mode="thread_local"):
                self._recurrent_body(b)
        b.graph = graph
        self.recurrent_graph_captures += 1

    # -- coda --------------------------------------------------------------------------------------------------
    def stage_coda_batch(self, items: list[DepthWorkItem], *, allow_async: bool = True,
                         successors: Callable[[list[DepthWorkItem]], tuple[list[DepthWorkItem], list[int]]] | None = None
                         ) -> PendingCodaResult:
        """Greedy next tokens of ``items`` (cdb/model_runner.py:1036-1125).

        ``successors``, once the items' tokens count as in flight, names the eager
        re-entries: (successor items with placeholder tokens, the coda rows they follow).
        Their prelude runs on the device tokens -- inside the coda launch when the
        adapter can fuse it, else as a prelude gathering from this result."""

        if not items:
            return PendingCodaResult(items=[], host_tokens=torch.empty(0, dtype=torch.int64))
        _tick.add_tokens_in_flight(items)
        n = len(items)
        eager_items, eager_rows = successors(items) if successors is not None else ([], [])
        fused = bool(eager_items) and self.adapter.coda_writes_successor_prelude
        m = n + n + len(eager_items) if fused else n
        turn = self._coda_turn(m, n)
        # One upload: [coda rows' slots | each row's successor slot or -1 | the successors' slots],
        # the successors taking hidden slots (LIFO free list first) in the same call.
        self.next_hidden_slot = _tick.coda_upload(
            items, eager_items if fused else [], eager_rows if fused else [], turn.upload_addr,
            turn.host_upload.numel(), self.free_hidden_slots, self.next_hidden_slot, self.bank_capacity)
        direct = turn.direct if n <= ops.CODA_DIRECT_MAX_ROWS and (fused or not eager_items) else None
        with self._on_stream():
            event = turn.event
            host = turn.host_tokens[:n]
            if direct is not None:
                # Upload, gather, LM head + argmax (+ successors' prelude), token download
                # and the successors' gate reset in one call.
                direct.launch(n, len(eager_items), fused, self._stream_handle)
                tokens = direct.tokens[:n]
                event.record(self.stream)
            else:
                dev = turn.dev_upload[:m]
                dev.copy_(turn.host_upload[:m], non_blocking=True)
                launch = self._stage_launch(items, dev[:n])
                if fused:
                    launch.successor_slots = dev[n:2 * n]
                tokens = self.adapter.coda(launch)
                host.copy_(tokens, non_blocking=True)
                event.record()
                if fused:
                    self.gate_state.reset(dev[2 * n:], len(eager_items))
        pending = PendingCodaResult(items=items, host_tokens=host, device_tokens=tokens, ready_event=event)
        if eager_items and not fused:
            self.compute_prelude_batch(eager_items, device_groups=[(pending, eager_rows)])
        if not allow_async:
            event.synchronize()
        return pending

    def _coda_turn(self, upload: int, rows: int) -> _CodaTurn:
        """The next of CODA_TURNS rotating coda buffers. At most CODA_PIPELINE_DEPTH codas are
        unconsumed at once, so a turn comes round again only after its result was read; its
        event is still waited on first."""

        k = self._coda_turn_index
        self._coda_turn_index = (k + 1) % self.CODA_TURNS
        turn = self._coda_turns[k]
        if turn is not None:
            turn.event.synchronize()
        if turn is None or turn.host_upload.numel() < upload or turn.host_tokens.numel() < rows:
            seqs = max(self.max_num_seqs, ops.CODA_DIRECT_MAX_ROWS)
            cap = max(upload, 3 * seqs)
            turn = self._coda_turns[k] = _CodaTurn(
                host_upload=self._pinned((cap,), torch.int64),
                dev_upload=torch.empty(cap, dtype=torch.int64, device=self.device),
                host_tokens=self._pinned((max(rows, seqs),), torch.int64),
                event=torch.cuda.Event())
            turn.upload_addr = turn.host_upload.data_ptr()
            if self._coda_weights is not None:
                turn.direct = ops.CodaScratch(self._coda_weights, self.bank, self.gate_state, turn.host_upload,
                                              turn.dev_upload, turn.host_tokens)
        return turn

    def consume_coda_result(self, pending: PendingCodaResult) -> list[int]:
        if pending.ready_event is not None:
            pending.ready_event.synchronize()
        tokens = pending.host_tokens.tolist()
        self.release_hidden_slots(pending.items)
        return tokens

    # -- prefill -----------------------------------------------------------------------------------------------
    def stage_prefill_batch(self, requests: list[FutureRequestState], *, allow_async: bool = True) -> PendingPrefillResult:
        """Full-depth prefill of the scheduled prompt chunks (cb/input_outputs.py:269-379 bookkeeping)."""

        cache = self.cache
        meta = self.prefill_metadata(requests)
        last_index = meta.last_index
        tile_seq, tile_q0 = ops.prefill_tiles(meta.lens, meta.past)
        split = None
        if self.dtype == torch.bfloat16 and len(meta.lens):
            split = ops.prefill_split_plan(meta.lens, meta.past, num_heads=self.num_heads, num_cus=self.num_cus)
        with self._on_stream():
            cache.flush_table_updates()
            launch = PrefillLaunch(
                tokens=self._to_device(meta.tokens, torch.int64),
                positions=self._to_device(meta.positions, torch.int32),
                write_rows=self._to_device(meta.write_rows, torch.int64),
                cu_q=self._to_device(meta.cu_q, torch.int32),
                past=self._to_device(meta.past, torch.int32),
                table_rows=self._to_device(meta.table_rows, torch.int32),
                tile_seq=self._to_device(tile_seq, torch.int32),
                tile_q0=self._to_device(tile_q0, torch.int32),
                last_index=self._to_device(last_index, torch.int64),
                cache=cache,
            )
            if split is not None:
                launch.split_items = self._to_device(split.items, torch.int32)
                launch.split_merges = self._to_device(split.merges, torch.int32)
                launch.split_slots = split.num_slots
                launch.partials = self._prefill_partials(split.num_slots)
            if len(last_index):
                device_tokens = self.adapter.prefill(launch)
            else:
                self.adapter.prefill(launch)
                device_tokens = torch.empty(0, dtype=torch.int64, device=self.device)
            host = self._pinned((len(last_index),), torch.int64)
            host.copy_(device_tokens, non_blocking=True)
            event = torch.cuda.Event()
            event.record()
        if not allow_async:
            event.synchronize()
        return PendingPrefillResult(futures=list(requests), host_tokens=host, device_tokens=device_tokens,
                                    ready_event=event)

    def prefill_metadata(self, requests: list[FutureRequestState]) -> "PrefillMetadata":
        """Host bookkeeping of one prefill launch (cb/input_outputs.py:269-379): the chunk tokens,
        their positions and pool write rows, cu_q, past lengths, block-table rows, and the index of
        each sampling row; advances every request's position and marks its sampled token in flight."""

        cache = self.cache
        tokens: list[int] = []
        positions: list[np.ndarray] = []
        rows: list[np.ndarray] = []
        cu_q = [0]
        past: list[int] = []
        table_rows: list[int] = []
        lens: list[int] = []
        last_index: list[int] = []
        for future in requests:
            state = future.state
            qlen = future.query_length
            p0 = state.position_offset
            tokens.extend(state.tokens_to_process)
            positions.append(np.arange(p0, p0 + qlen, dtype=np.int32))
            rows.append(cache.write_rows(state.request_id, p0, qlen))
            state.position_offset += qlen
            cu_q.append(cu_q[-1] + qlen)
            past.append(p0)
            table_rows.append(cache.table_row_of[state.request_id])
            lens.append(qlen)
            if future.has_new_token:
                last_index.append(cu_q[-1] - 1)
                state.tokens_to_process = [TMP_TOKEN_ID]
                state.tokens_in_flight += 1
        return PrefillMetadata(tokens=np.asarray(tokens, dtype=np.int64), positions=np.concatenate(positions),
                               write_rows=np.concatenate(rows), cu_q=np.asarray(cu_q, dtype=np.int32),
                               past=np.asarray(past, dtype=np.int32),
                               table_rows=np.asarray(table_rows, dtype=np.int32), lens=lens,
                               last_index=np.asarray(last_index, dtype=np.int64))

    def consume_prefill_result(self, pending: PendingPrefillResult) -> list[int]:
        if pending.ready_event is not None:
            pending.ready_event.synchronize()
        return pending.host_tokens.tolist()

    # -- exit-KV propagation ------------------------------------------------------------------------------------
    def copy_exit_kv(self, rows: list[int], exit_steps: list[int]) -> None:
        if not rows:
            return
        slots = [self.layout.slot_for_step(s) for s in exit_steps]
        with self._on_stream():
            torch.ops.cdb.exit_kv_copy(self.cache.pool, self.cache.block_size,
                                       self._to_device(np.asarray(rows, dtype=np.int64), torch.int64),
                                       self._to_device(np.asarray(slots, dtype=np.int32), torch.int32), len(rows),
                                       self.layout.core_base, self.layout.num_core_layers,
                                       self.layout.slots_per_layer)

    # -- KV swap (offload pressure mode) -------------------------------------------------------------------------
    def make_kv_swap_pool(self, num_host_blocks: int) -> KvSwapPool:
        """The pinned host pool that swapped-out KV blocks move to, on the compute stream."""

        return KvSwapPool(self.cache, num_host_blocks, stream=self.stream)

    def synchronize(self) -> None:
        self.stream.synchronize()


def model_adapter_num_heads(adapter: CDBModelAdapter) -> int:
    return int(getattr(adapter, "num_heads", 1))
