"""Model adapter boundary between the CDB engine and a looped model.

Counterpart of the reference's CDBModelAdapter (continuous_depth_batching/model_adapter.py:14-122):
a model exposes a prelude (token embedding, plus prelude layers where the
model has them), one recurrent block application, and a coda (LM head).
Here each stage is a sequence of HIP kernel launches over static device
buffers owned by the runner, so a whole recurrent stage can be captured into
one HIP graph per batch bucket.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Any

import torch

from . import ops
from .cache import PagedKVCache
from .exit_policy import DecisionHorizon, ExitDecisionRule, ExitPolicySpec
from .kv_cache_policy import LoopedKvLayout


@dataclass
class GateLaunch:
    """Static per-bucket buffers of the exit gate (see ``cdb_exit_gate``)."""

    state: ops.GateState
    steps: torch.Tensor          # [Bp] int32
    synthetic: torch.Tensor      # [Bp] int32 (-1 = no replayed depth)
    flags: torch.Tensor          # [Bp] uint8
    signal: torch.Tensor         # [Bp] model dtype
    rule: int
    round_hazard: bool
    min_steps: int
    max_steps: int
    threshold: float | None
    enabled: bool = True


@dataclass
class RecurrentLaunch:
    """Static device inputs of one recurrent-stage bucket (rows = bucket size)."""

    rows: int
    bank: torch.Tensor           # [capacity, width] hidden-state bank
    bank_slots: torch.Tensor     # [rows] int64, -1 = padding
    positions: torch.Tensor      # [rows] int32 position of the token, -1 = padding
    table_rows: torch.Tensor     # [rows] int32 block-table row of the token's request
    slot_offset: torch.Tensor    # [rows] int32 cache layer of core layer 0 at the row's step (prelude + slot * C)
    cache: PagedKVCache
    workspace: torch.Tensor      # decode-attention workspace (split header + fp32 partials)
    split_pages: int             # pages per KV split; 0 = chosen by the kernel, -m = chosen with at least m
    gate: GateLaunch


@dataclass
class StageLaunch:
    """Device inputs of a prelude or coda launch over ``n`` work items.

    ``positions``, ``table_rows``, ``cache`` and ``workspace`` are set when the adapter's
    stages attend over their own KV (``stages_use_attention``; the reference's engine then
    passes the same paged-cache arguments to the prelude and coda, cdb/model_runner.py:1285-1357)."""

    n: int
    bank: torch.Tensor                 # [capacity, hidden_width] hidden-state bank
    slots: torch.Tensor                # [n] int64 bank slots of the items
    tokens: torch.Tensor | None = None         # [n] int64 token ids (prelude)
    positions: torch.Tensor | None = None      # [n] int32 token positions
    table_rows: torch.Tensor | None = None     # [n] int32 block-table rows
    cache: PagedKVCache | None = None
    workspace: torch.Tensor | None = None      # decode-attention workspace
    split_pages: int = 0
    # Coda only, with coda_writes_successor_prelude: [n] int64 bank slots of the rows'
    # eager successors (-1: none), whose prelude the coda runs on its greedy token.
    successor_slots: torch.Tensor | None = None


@dataclass
class PrefillLaunch:
    """Device inputs of one full-depth prefill forward over T prompt tokens."""

    tokens: torch.Tensor         # [T] int64
    positions: torch.Tensor      # [T] int32
    write_rows: torch.Tensor     # [T] int64 pool rows of each token
    cu_q: torch.Tensor           # [S+1] int32
    past: torch.Tensor           # [S] int32
    table_rows: torch.Tensor     # [S] int32
    tile_seq: torch.Tensor       # [tiles] int32
    tile_q0: torch.Tensor        # [tiles] int32
    last_index: torch.Tensor     # [N] int64 token index whose logits sample the next token
    cache: PagedKVCache
    # bf16 only: the tiles as a split work list (cdb_prefill_attention_split), with its
    # partial-result buffer; None runs the whole tiles above.
    split_items: torch.Tensor | None = None   # [n, 4] int32
    split_merges: torch.Tensor | None = None  # [m, 4] int32
    split_slots: int = 0
    partials: torch.Tensor | None = None


class CDBModelAdapter(ABC):
    """Model-specific stage kernels used by the CDB runner."""

    stages_use_attention: bool = False
    # The coda can also run the prelude of the rows' next tokens (an embedding lookup of
    # the greedy token into launch.successor_slots), so eager re-entries need no prelude
    # launch of their own (cdb/model_runner.py:439-457 gathers those tokens on device).
    coda_writes_successor_prelude: bool = False

    @property
    @abstractmethod
    def hidden_width(self) -> int:
        """Width of one hidden-bank row (the recurrent state carried between steps)."""

    @property
    @abstractmethod
    def dtype(self) -> torch.dtype: ...

    @property
    @abstractmethod
    def device(self) -> torch.device: ...

    @abstractmethod
    def configure_recurrent_steps(self, max_recurrent_steps: int) -> None: ...

    @abstractmethod
    def configure_kv_policy(self, kv_policy: str, kv_slots_per_layer: int | None) -> None: ...

    @abstractmethod
    def kv_cache_layout(self) -> LoopedKvLayout: ...

    @abstractmethod
    def kv_geometry(self) -> tuple[int, int]:
        """(num_key_value_heads, head_dim) of the paged cache."""

    def exit_policy_spec(self) -> ExitPolicySpec:
        return ExitPolicySpec(ExitDecisionRule.CUMULATIVE_HAZARD, DecisionHorizon.SAME_STEP)

    def configure_exit_signal(self, enabled: bool) -> None:
        del enabled

    def decides_exit_before_loop(self) -> bool:
        return self.exit_policy_spec().rule is ExitDecisionRule.PRELOOP_DISTRIBUTION

    @abstractmethod
    def prelude(self, launch: StageLaunch) -> None:
        """Write the prelude state of launch.tokens into bank rows launch.slots."""

    @abstractmethod
    def recurrent_step(self, launch: RecurrentLaunch) -> None:
        """One block application over the bucket: bank rows in, bank rows + gate decisions out."""

    @abstractmethod
    def prefill(self, launch: PrefillLaunch) -> torch.Tensor:
        """Full-depth prefill forward; returns the sampled next tokens [N] int64 of launch.last_index."""

    @abstractmethod
    def coda(self, launch: StageLaunch) -> torch.Tensor:
        """Greedy next tokens [n] int64 for the hidden states in bank rows launch.slots."""

    def coda_weights(self) -> Any | None:
        """The LM head (and embedding, for the fused successor prelude) of a coda that is
        exactly an LM head + argmax over the bank rows, as ``ops.CodaWeights``; the runner
        then runs small codas as one C-ABI call. None keeps every coda on ``coda``."""

        return None


def resolve_cdb_model_adapter(model: Any, adapter: CDBModelAdapter | None = None) -> CDBModelAdapter:
    """Explicit adapter, or one inferred from the model type (model_adapter.py:105-122)."""

    if adapter is not None:
        if not isinstance(adapter, CDBModelAdapter):
            raise TypeError(f"model_adapter must inherit CDBModelAdapter, got {type(adapter)!r}")
        return adapter
    model_type = getattr(getattr(model, "config", None), "model_type", None)
    if model_type == "ouro":
        from .ouro import OuroCDBAdapter

        if OuroCDBAdapter.supports(model):
            return OuroCDBAdapter(model)
    if model_type == "huginn":
        from .huginn import HuginnCDBAdapter

        if HuginnCDBAdapter.supports(model):
            return HuginnCDBAdapter(model)
    raise TypeError(f"Continuous depth batching requires an explicit model adapter or a supported looped model; "
                    f"got {type(model)!r}")
