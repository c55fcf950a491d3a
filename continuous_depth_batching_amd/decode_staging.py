"""Decode staging under KV pressure: whether a decode token may start its loop now.

A decode token needs its K/V row before its first recurrent step. It either fits in the request's
last block or gets exactly the blocks that one more token needs (the exact-ceil rule of the
scheduler's prefill allocation; cdb/continuous_api.py:1654-1669). When neither works, the pressure
mode decides (cdb/config.py kv_pressure_mode; cdb/continuous_api.py:1584-1652):

  * ``none`` and ``reserve`` treat it as an error (``reserve`` admission guarantees it never
    happens, so there it reports inconsistent accounting);
  * ``recompute`` and ``offload`` park the request at this token boundary, the only point where
    no loop state is in flight. Parked requests are retried in the order they parked, ahead of
    each tick's scheduling; the first one that still finds no block ends the retry, since every
    parked request needs one new block. When no other work can run, one parked request gives up
    its KV: the one with the fewest computed tokens, the latest to park among equals.

The staged work item restarts the token's depth state: loop step 0, the replayed exit depth of the
token when a trace is replayed.
"""

from __future__ import annotations

from .cache import CacheFullError, PagedKVCache
from .requests import DepthWorkItem, RequestState

PARKING_MODES = ("recompute", "offload")


class DecodeStaging:
    def __init__(self, cache: PagedKVCache, pressure_mode: str, yield_kv) -> None:
        """``yield_kv(request_id, state)`` takes a parked request's KV away (swap or soft reset)."""

        self.cache = cache
        self.pressure_mode = pressure_mode
        self.yield_kv = yield_kv
        self.parked: dict[str, RequestState] = {}  # insertion order is park order

    # -- KV row of the next token ------------------------------------------------------------------
    def reserve_row(self, state: RequestState) -> bool:
        """Make room for one more token of ``state``: True when its last block already has a free
        row or the missing blocks were allocated; False, with nothing allocated, when the cache
        cannot provide them."""

        block = self.cache.block_size
        held = state.allocated_blocks
        length = state.current_len()
        if held > 0 and held * block > length:
            return True
        missing = (length + block) // block - held
        got = self.cache.allocate_blocks(missing, state.request_id, held)
        if got is None:
            return False
        state.allocated_blocks = held + got
        return True

    @staticmethod
    def work_item(state: RequestState, token_id: int | None = None) -> DepthWorkItem:
        """Step-0 work item of the request's pending token (``token_id`` overrides the token for an
        entry whose token the device fills in)."""

        state.reset_depth_state_for_next_token()
        token = state.tokens_to_process[0] if token_id is None else token_id
        return DepthWorkItem(state=state, token_id=token, token_position=state.position_offset, recurrent_step=0,
                             synthetic_exit_depth=state.next_synthetic_exit_depth())

    # -- staging -----------------------------------------------------------------------------------
    def stage(self, state: RequestState) -> DepthWorkItem | None:
        """The request's next decode token as a work item, or None when it parked."""

        pending = state.tokens_to_process
        if not pending or pending[0] < 0:
            raise RuntimeError(f"decode staging: request {state.request_id} has no sampled token to decode")
        if not self.reserve_row(state):
            self._on_full(state)
            return None
        self.parked.pop(state.request_id, None)
        return self.work_item(state)

    def _on_full(self, state: RequestState) -> None:
        mode = self.pressure_mode
        if mode in PARKING_MODES:
            self.parked[state.request_id] = state
            return
        rid = state.request_id
        if mode == "reserve":
            raise CacheFullError(f"request {rid} found no block for its next decode token although reserve "
                                 "admission had set its blocks aside: reservation accounting is inconsistent")
        raise CacheFullError(f"no KV block left for the next decode token of request {rid}, and "
                             f"kv_pressure_mode={mode!r} does no preemption (raise num_blocks, lower the load, "
                             "or choose 'reserve', 'recompute' or 'offload')")

    def retry_parked(self) -> list[DepthWorkItem]:
        """Stage parked requests in park order until the first that still cannot get its block."""

        staged: list[DepthWorkItem] = []
        for state in list(self.parked.values()):
            item = self.stage(state)
            if item is None:
                return staged
            staged.append(item)
        return staged

    def yield_one(self, active_requests: int) -> None:
        """Take one parked request's KV away so the others can drain. With a single active request
        there is nobody to drain: its KV cannot fit, which is an error."""

        if active_requests <= 1:
            rid = next(iter(self.parked))
            raise CacheFullError(f"request {rid} is a single request whose KV does not fit: it cannot grow by "
                                 "one block and no other request can be preempted (raise num_blocks or lower "
                                 "max_model_len)")
        order = list(self.parked)
        # Fewest computed tokens first; among equals the latest to park.
        victim = min(range(len(order)), key=lambda i: (self.parked[order[i]].current_len(), -i))
        rid = order[victim]
        self.yield_kv(rid, self.parked.pop(rid))

    def forget(self, request_id: str) -> None:
        self.parked.pop(request_id, None)

    def clear(self) -> None:
        self.parked.clear()
