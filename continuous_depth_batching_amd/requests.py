"""Request lifecycle and depth work items (host-side state of the CDB engine).

``RequestState`` tracks a request's prompt, generated tokens, KV length
(``position_offset``), allocated blocks and the tokens still in flight on the
device; ``DepthWorkItem`` is one decode token's trip through the recurrent
steps. Semantics follow continuous_batching/requests.py:75-346 and
continuous_depth_batching/requests.py:41-173 (length-finish prediction,
EOS/stop handling, the synthetic exit-depth replay cursor).
"""

from __future__ import annotations

import logging
import time
from dataclasses import dataclass, field
from enum import IntEnum

from . import _tick

logger = logging.getLogger("ContinuousBatchingLogger")

#: Placeholder id of a token that the device has sampled but the host has not seen.
TMP_TOKEN_ID = -1


class RequestStatus(IntEnum):
    PENDING = 0
    PREFILLING = 1
    DECODING = 2
    FINISHED = 3


@dataclass
class GenerationOutput:
    request_id: str
    prompt_ids: list[int] = field(default_factory=list)
    generated_tokens: list[int] = field(default_factory=list)
    exit_depths: list[int] = field(default_factory=list)
    status: RequestStatus = RequestStatus.PENDING
    created_time: float = field(default_factory=time.perf_counter)
    lifespan: tuple[float, float] = (-1.0, -1.0)
    first_token_time: float = -1.0

    def is_finished(self) -> bool:
        return self.status == RequestStatus.FINISHED


@dataclass(eq=False)
class RequestState:
    request_id: str
    initial_tokens: list[int]
    max_new_tokens: int | None = 20
    eos_token_id: int | list[int] | None = None
    stop_sequences: list[list[int]] = field(default_factory=list)
    synthetic_exit_depths: list[int] = field(default_factory=list)
    replay_eos_finishes: bool = False

    tokens_to_process: list[int] = field(default_factory=list)
    generated_tokens: list[int] = field(default_factory=list)
    remaining_prefill_tokens: list[int] = field(default_factory=list)
    position_offset: int = 0
    allocated_blocks: int = 0
    tokens_in_flight: int = 0
    is_cpu_offloaded: bool = False
    exit_depths: list[int] = field(default_factory=list)
    current_token_exit_depth: int | None = None
    created_time: float = field(default_factory=time.perf_counter)
    lifespan: tuple[float, float] = (-1.0, -1.0)
    first_token_time: float = -1.0
    _status: RequestStatus = RequestStatus.PENDING
    _synthetic_exit_cursor: int = 0
    _true_initial_tokens: int = 0

    def __post_init__(self) -> None:
        self._new_tokens_limit = 2**31 - 1 if self.max_new_tokens is None else self.max_new_tokens
        self.remaining_prefill_tokens = list(self.initial_tokens)
        if self.eos_token_id is None:
            self._eos_token_ids: set[int] = set()
        elif isinstance(self.eos_token_id, int):
            self._eos_token_ids = {self.eos_token_id} if self.eos_token_id >= 0 else set()
        else:
            self._eos_token_ids = {t for t in self.eos_token_id if t >= 0}

    @property
    def status(self) -> RequestStatus:
        return self._status

    @status.setter
    def status(self, value: RequestStatus) -> None:
        if self._status == RequestStatus.PENDING and self.lifespan[0] < 0:
            self.lifespan = (time.perf_counter(), -1.0)
        elif value == RequestStatus.FINISHED:
            self.lifespan = (self.lifespan[0], time.perf_counter())
        self._status = value

    def current_len(self) -> int:
        return self.position_offset

    def generated_len(self) -> int:
        return len(self.generated_tokens)

    def prompt_len(self) -> int:
        return self._true_initial_tokens or len(self.initial_tokens)

    def total_generated_len(self) -> int:
        return len(self.initial_tokens) - self.prompt_len() + len(self.generated_tokens)

    def has_grown_past_prompt(self) -> bool:
        return self.current_len() > self.prompt_len()

    def will_finish_on_pending_token(self) -> bool:
        """Length limit already met by in-flight tokens (continuous_batching/requests.py:196-206)."""

        if self.replay_eos_finishes:
            return False
        return self.tokens_in_flight > 0 and self.generated_len() + self.tokens_in_flight >= self._new_tokens_limit

    def update_and_check_completion(self, token_id: int) -> bool:
        """Record a sampled token; return whether the request finished (requests.py:208-237).

        One fewer token is in flight; the token is kept (and becomes the next token to
        process) when it is EOS or within the length limit; the request finishes on EOS, at
        the limit or when the generated tokens end with a stop sequence. Runs in the tick
        core, which also applies it row by row to coda results."""

        return _tick.update_completion(self, token_id)

    def reset_depth_state_for_next_token(self) -> None:
        self.current_token_exit_depth = None

    def next_synthetic_exit_depth(self) -> int | None:
        """Pop the replayed 0-based exit step of the next decode token (cdb/requests.py:57-80)."""

        if not self.synthetic_exit_depths:
            return None
        if self._synthetic_exit_cursor >= len(self.synthetic_exit_depths):
            if self.replay_eos_finishes and self._synthetic_exit_cursor == len(self.synthetic_exit_depths):
                self._synthetic_exit_cursor += 1
                return self.synthetic_exit_depths[-1]
            raise RuntimeError(f"Request {self.request_id}: synthetic exit-depth schedule exhausted; "
                               "expected one exit depth per decode token")
        depth = self.synthetic_exit_depths[self._synthetic_exit_cursor]
        self._synthetic_exit_cursor += 1
        return depth

    def prepare_for_offload_requeue(self) -> None:
        """Reset a request whose KV was just swapped out, so it resumes from the restored KV
        (continuous_batching/requests.py:275-288, cdb/requests.py:82-94).

        The block allocation is dropped (the blocks come back on restore); a decoder keeps its
        pending token and re-runs it through the recurrent path from step 0. The synthetic
        exit-depth cursor is untouched, so the pending token replays its own recorded depth."""

        self.allocated_blocks = 0
        if self._status == RequestStatus.DECODING:
            self.remaining_prefill_tokens = []
        self.reset_depth_state_for_next_token()

    def create_equivalent_initial_request(self) -> "RequestState":
        """Rebuild this request as a fresh prefill for soft-reset preemption
        (continuous_batching/requests.py:290-315, cdb/requests.py:111-126).

        The generated tokens, the pending one included, are folded onto the prompt and the
        length budget shrinks by as many. The re-prefill computes the pending token at full
        depth, so its recorded exit depth is spent: the replay resumes at ``cursor + 1``.
        Timing and the exit depths of the tokens already decoded carry over."""

        new_state = RequestState(
            request_id=self.request_id,
            initial_tokens=self.initial_tokens + self.generated_tokens,
            max_new_tokens=None if self.max_new_tokens is None else self.max_new_tokens - len(self.generated_tokens),
            eos_token_id=self.eos_token_id,
            stop_sequences=[list(s) for s in self.stop_sequences],
            synthetic_exit_depths=self.synthetic_exit_depths[self._synthetic_exit_cursor + 1:],
            replay_eos_finishes=self.replay_eos_finishes,
        )
        new_state._true_initial_tokens = self._true_initial_tokens or len(self.initial_tokens)
        new_state.exit_depths = list(self.exit_depths)
        new_state.created_time = self.created_time
        new_state.lifespan = self.lifespan
        new_state.first_token_time = self.first_token_time
        return new_state

    def to_generation_output(self) -> GenerationOutput:
        return GenerationOutput(
            request_id=self.request_id,
            prompt_ids=list(self.initial_tokens[: self.prompt_len()]),
            generated_tokens=list(self.initial_tokens[self.prompt_len():]) + list(self.generated_tokens),
            exit_depths=list(self.exit_depths),
            status=self.status,
            created_time=self.created_time,
            lifespan=self.lifespan,
            first_token_time=self.first_token_time,
        )


class FutureRequestState:
    """A request's place in a prefill batch (continuous_batching/requests.py:337-346)."""

    __slots__ = ("has_new_token", "query_length", "state")

    def __init__(self, state: RequestState, has_new_token: bool, query_length: int) -> None:
        self.state = state
        self.has_new_token = has_new_token
        self.query_length = query_length


@dataclass(eq=False)
class DepthWorkItem:
    """One decode token's recurrent work (cdb/requests.py:153-173); steps and positions are 0-based."""

    state: RequestState
    token_id: int
    token_position: int
    recurrent_step: int
    synthetic_exit_depth: int | None = None
    apply_exit_gate: bool = True
    hidden_slot: int | None = None


_tick.bind_request_types(RequestStatus, FutureRequestState)
