"""A host-only stand-in for the device runner, for CPU tests of the engine's scheduling.

The engine, scheduler, block manager, cache bookkeeping and the runner's host
metadata assembly are the product's own code; only the stage arithmetic runs on
the host here. The model is the reference tests' token-increment loop model
(tests/continuous_depth_batching/test_continuous_depth_batching.py:52-146):
  * prelude: the hidden state is the token id;
  * each recurrent step adds 1 and emits the exit signal +10 at step 0, -10 after;
  * coda: the next token is round(hidden) mod vocab;
  * prefill (full depth): the next token is (last prompt token + steps) mod vocab.
Exit decisions follow the exit-gate kernel's rule as the model adapters launch
it (cdb_exit_gate with delayed = 0: forced final step, replayed depth, hazard CDF
or direct threshold on this step's signal), restated here on the host. On the
delayed horizon the engine itself applies a launch's decisions one launch late.
"""

from __future__ import annotations

from contextlib import nullcontext

import numpy as np
import torch

from continuous_depth_batching_amd.exit_policy import ExitDecisionRule, ExitPolicySpec
from continuous_depth_batching_amd.kv_cache_policy import DEPTH_INDEXED, LoopedKvLayout
from continuous_depth_batching_amd.model_adapter import CDBModelAdapter
from continuous_depth_batching_amd.model_runner import (
    ModelRunner,
    PendingCodaResult,
    PendingFlags,
    PendingPrefillResult,
    decode_graph_buckets,
    pad_to_bucket,
)
from continuous_depth_batching_amd.requests import TMP_TOKEN_ID
from oracle.stage import sigmoid_f32


class TokenIncrementConfig:
    def __init__(self, **over) -> None:
        self.num_hidden_layers = 1
        self.num_attention_heads = 2
        self.num_key_value_heads = 1
        self.head_dim = 2
        self.hidden_size = 4
        self.vocab_size = 16
        self.total_ut_steps = 3
        self.model_type = "token_increment"
        self._attn_implementation = "paged|flash_attention_3"
        for k, v in over.items():
            setattr(self, k, v)


class TokenIncrementModel:
    def __init__(self, **over) -> None:
        self.config = TokenIncrementConfig(**over)


class TokenIncrementAdapter(CDBModelAdapter):
    def __init__(self, model: TokenIncrementModel, *, spec: ExitPolicySpec | None = None) -> None:
        self.model = model
        self.kv_policy = DEPTH_INDEXED
        self.kv_slots: int | None = None
        self._spec = spec or ExitPolicySpec(ExitDecisionRule.CUMULATIVE_HAZARD)

    @property
    def hidden_width(self) -> int:
        return self.model.config.hidden_size

    @property
    def dtype(self) -> torch.dtype:
        return torch.float32

    @property
    def device(self) -> torch.device:
        return torch.device("cpu")

    def configure_recurrent_steps(self, max_recurrent_steps: int) -> None:
        self.model.config.total_ut_steps = max_recurrent_steps

    def configure_kv_policy(self, kv_policy: str, kv_slots_per_layer: int | None) -> None:
        self.kv_policy = kv_policy
        self.kv_slots = kv_slots_per_layer

    def kv_cache_layout(self) -> LoopedKvLayout:
        c = self.model.config
        return LoopedKvLayout.build(num_prelude_layers=0, num_core_layers=c.num_hidden_layers, num_coda_layers=0,
                                    total_recurrent_steps=c.total_ut_steps, policy=self.kv_policy,
                                    requested_slots=self.kv_slots)

    def kv_geometry(self) -> tuple[int, int]:
        return self.model.config.num_key_value_heads, self.model.config.head_dim

    def exit_policy_spec(self) -> ExitPolicySpec:
        return self._spec

    # Device stages are never called by the host runner.
    def prelude(self, tokens, bank, slots, n):  # pragma: no cover
        raise NotImplementedError

    def recurrent_step(self, launch):  # pragma: no cover
        raise NotImplementedError

    def prefill(self, launch):  # pragma: no cover
        raise NotImplementedError

    def coda(self, bank, slots, n):  # pragma: no cover
        raise NotImplementedError


class HostLoopRunner(ModelRunner):
    """ModelRunner's interface and hidden-slot bookkeeping, with host stage arithmetic."""

    def __init__(self, *, engine_config, cache, model_adapter, exit_policy) -> None:  # no device setup
        self.engine_config = engine_config
        self.cache = cache
        self.adapter = model_adapter
        self.exit_policy = exit_policy
        self.layout = cache.layout
        self.max_num_seqs = engine_config.max_num_seqs
        self.decode_graph_buckets = decode_graph_buckets(self.max_num_seqs)
        self.bank_capacity = 4 * self.max_num_seqs + 64
        self.free_hidden_slots: list[int] = []
        self.next_hidden_slot = 0
        self.recurrent_graph_hits = self.recurrent_graph_captures = 0
        self.stage_graph_hits = self.stage_graph_captures = 0
        self.hidden: dict[int, float] = {}
        self.gate: dict[int, list[float]] = {}
        # Per recurrent launch: the padded bucket's metadata exactly as uploaded to the device.
        self.launches: list[dict[str, np.ndarray]] = []
        self.exit_copies: list[tuple[list[int], list[int]]] = []

    @property
    def vocab(self) -> int:
        return self.adapter.model.config.vocab_size

    # -- stages ------------------------------------------------------------------------------------------------
    def compute_prelude_batch(self, items, device_groups=()) -> None:
        if not items:
            return
        num_device = sum(len(rows) for _, rows in device_groups)
        if any(item.token_id != TMP_TOKEN_ID for item in items[:num_device]):
            raise AssertionError("device_groups must cover a prefix of items")
        tokens: list[int] = []
        for result, rows in device_groups:
            tokens.extend(int(result.device_tokens[r]) for r in rows)
        tokens.extend(item.token_id for item in items[num_device:])
        slots = self.allocate_hidden_slots(len(items))
        for item, slot, token in zip(items, slots, tokens):
            self.hidden[slot] = float(token)
            self.gate[slot] = [0.0, 1.0]
            item.hidden_slot = slot

    def compute_recurrent_batch(self, items) -> PendingFlags:
        if not items:
            raise ValueError("items must not be empty")
        rows = pad_to_bucket(len(items), self.decode_graph_buckets)
        i64 = np.empty(rows, np.int64)
        i32 = np.empty((5, rows), np.int32)
        self.fill_recurrent_metadata(items, i64, i32)
        self.launches.append({"slots": i64.copy(), "meta": i32.copy(),
                              "table": self.cache.host_table[i32[self.META_TABLE_ROWS]].copy()})
        flags = np.zeros(rows, np.uint8)
        for r in range(len(items)):
            slot, step, synth = int(i64[r]), int(i32[self.META_STEPS, r]), int(i32[self.META_SYNTHETIC, r])
            self.hidden[slot] += 1.0
            signal = 10.0 if step == 0 else -10.0
            flags[r] = self._decide(slot, step, synth, signal)
        if self.exit_policy.delayed():
            return PendingFlags(host=torch.from_numpy(flags), event=None)
        # The synchronous horizon routes from the lists cdb_route_compact writes: exiting rows,
        # then staying rows, each in launch order (padding rows have a negative bank slot).
        live = np.nonzero(i64 >= 0)[0]
        exits = [int(r) for r in live if flags[r]]
        stays = [int(r) for r in live if not flags[r]]
        lists = np.array([len(exits), len(stays)] + exits + stays, np.int32)
        return PendingFlags(host=None, event=None, lists=torch.from_numpy(lists))

    def _decide(self, slot: int, step: int, synth: int, signal: float) -> bool:
        p = self.exit_policy
        state = self.gate[slot]
        if step >= p.max_recurrent_steps - 1:
            return True
        if synth >= 0:
            return step >= synth
        if p.threshold is None:
            return False
        can_exit = step + 1 >= p.min_recurrent_steps
        if p.spec.rule is ExitDecisionRule.CUMULATIVE_HAZARD:
            hazard = float(sigmoid_f32(signal))  # fp32 model: rounding to the model dtype is exact
            state[0] += hazard * state[1]
            state[1] *= 1.0 - hazard
            return can_exit and state[0] >= p.threshold
        return can_exit and signal < p.threshold

    def stage_coda_batch(self, items, *, allow_async: bool = True, successors=None) -> PendingCodaResult:
        if not items:
            return PendingCodaResult(items=[], host_tokens=torch.empty(0, dtype=torch.int64))
        for item in items:
            item.state.tokens_in_flight += 1
        eager_items, eager_rows = successors(items) if successors is not None else ([], [])
        tokens = torch.tensor([round(self.hidden[item.hidden_slot]) % self.vocab for item in items],
                              dtype=torch.int64)
        pending = PendingCodaResult(items=items, host_tokens=tokens, device_tokens=tokens.clone())
        if eager_items:
            self.compute_prelude_batch(eager_items, device_groups=[(pending, eager_rows)])
        return pending

    def stage_prefill_batch(self, requests, *, allow_async: bool = True) -> PendingPrefillResult:
        meta = self.prefill_metadata(requests)
        steps = self.adapter.model.config.total_ut_steps
        tokens = torch.tensor([(int(meta.tokens[i]) + steps) % self.vocab for i in meta.last_index],
                              dtype=torch.int64)
        return PendingPrefillResult(futures=list(requests), host_tokens=tokens, device_tokens=tokens.clone())

    def copy_exit_kv(self, rows: list[int], exit_steps: list[int]) -> None:
        if rows:
            self.exit_copies.append((list(rows), [self.layout.slot_for_step(s) for s in exit_steps]))

    def capture_all_buckets(self, buckets=None) -> int:
        return 0

    def make_kv_swap_pool(self, num_host_blocks: int) -> "HostKvSwap":
        return HostKvSwap(self.cache, num_host_blocks)

    def synchronize(self) -> None:
        pass

    def stream_scope(self):
        return nullcontext()


class HostKvSwap:
    """KvSwapPool's block moves on a host cache: the same host-pool layout (one pool block holds
    a device block's slabs over every cache layer, K and V), moved with tensor indexing."""

    def __init__(self, cache, num_host_blocks: int) -> None:
        self.cache = cache
        self.slabs = 2 * cache.num_layers
        self.plane_blocks = cache.pool.shape[2] // cache.block_size
        self.block_elems = cache.block_size * cache.num_key_value_heads * cache.head_dim
        self.device_rows = cache.pool.view(self.slabs * self.plane_blocks, self.block_elems)
        self.host = torch.zeros((num_host_blocks, self.slabs, self.block_elems), dtype=cache.dtype)
        self.moves: list[tuple[str, list[int], list[int]]] = []

    def _rows(self, device_blocks: list[int]) -> torch.Tensor:
        blocks = torch.tensor(device_blocks, dtype=torch.int64)
        return (torch.arange(self.slabs)[None, :] * self.plane_blocks + blocks[:, None]).reshape(-1)

    def swap_out(self, device_blocks: list[int], host_blocks: list[int]) -> None:
        assert len(device_blocks) == len(host_blocks)
        self.moves.append(("out", list(device_blocks), list(host_blocks)))
        if device_blocks:
            slabs = self.device_rows[self._rows(device_blocks)].view(len(device_blocks), self.slabs, -1)
            self.host[torch.tensor(host_blocks)] = slabs

    def swap_in(self, host_blocks: list[int], device_blocks: list[int]) -> None:
        assert len(device_blocks) == len(host_blocks)
        self.moves.append(("in", list(device_blocks), list(host_blocks)))
        if device_blocks:
            self.device_rows[self._rows(device_blocks)] = self.host[torch.tensor(host_blocks)].reshape(
                -1, self.block_elems)


def make_engine(**cfg_over):
    """Engine over the token-increment model on the host runner, with the reference tests'
    small-cache configuration (test_continuous_depth_batching.py:150-161) unless overridden."""

    from continuous_depth_batching_amd.config import ContinuousDepthBatchingConfig
    from continuous_depth_batching_amd.engine import ContinuousDepthBatchingEngine

    spec = cfg_over.pop("spec", None)
    values = dict(num_blocks=16, block_size=4, max_num_batched_tokens=4, max_model_len=16,
                  use_async_batching=False, use_cuda_graph=False, max_recurrent_steps=3)
    values.update(cfg_over)
    model = TokenIncrementModel()
    adapter = TokenIncrementAdapter(model, spec=spec)
    return ContinuousDepthBatchingEngine.from_model(model, ContinuousDepthBatchingConfig(**values),
                                                    model_adapter=adapter, runner_factory=HostLoopRunner)
