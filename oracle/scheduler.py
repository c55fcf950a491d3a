"""CPU restatement of the reference's continuous-depth-batching schedule (test infrastructure only).

This module is a checker. Only tests/, the smoke entry and the bench's CPU-baseline leg may
import it; the product never does.

It replays one ``generate_batch`` call of the reference engine as a discrete simulation and
records every launch the engine would issue, with the state each launch reads:

  ("prefill",   ((request_id, start_position, query_length, has_new_token), ...))
  ("prelude",   site, ((request_id, token_position, hidden_slot), ...))
  ("recurrent", ((request_id, token_position, recurrent_step, hidden_slot, block_ids), ...),
                exits, refill_events_after_routing)
  ("coda",      ((request_id, token_position, hidden_slot), ...))

Scheduling follows, in the reference:
  * the refill loop and its tick order -- continuous_depth_batching/continuous_api.py:503-606;
  * ``schedule_next`` priority coda > prefill > recurrent > coda flush, recurrent batches popped
    FIFO and kept slot-homogeneous under multi-slot KV layouts -- scheduler.py:101-140, 322-346;
  * head re-insertion of stepped items and refill counting -- scheduler.py:142-180;
  * prefill admission, packing and chunking -- scheduler_base.py:154-206, 416-432, 473-545 and
    scheduler.py:221-320;
  * FIFO block ids with exact-ceil allocation -- continuous_batching/cache_manager.py:72-90,
    scheduler_base.py:416-432, continuous_api.py:1654-1669;
  * LIFO hidden-state slots, then monotonic growth; coda slots are freed when the coda is
    consumed -- model_runner.py:1154-1162, 1193-1203, 1359-1363;
  * prefill, coda and eager re-entry bookkeeping -- continuous_api.py:995-1088, 1282-1406,
    continuous_batching/requests.py:183-237, input_outputs.py:316-350;
  * exit routing on the synchronous and delayed horizons -- continuous_api.py:1090-1245,
    1671-1724, exit_policy.py:87-169;
  * the no-refill wave loop -- continuous_api.py:608-944, with its wave-boundary carry on the
    delayed horizon (the coda read after the next wave's first launch, first tokens at the next
    iteration's top, successors entering the next wave's one prelude) -- :636-642, 708-785,
    864-932, 1350-1368.

``mixed_slot_recurrent_batches`` drops the slot-homogeneous launch rule (an option of this build's
engine, not of the reference). ``replay_offset_one`` forces the replay horizon (the reference's tests force the delayed replay
path on CPU the same way); by default it follows the configuration.

Timing is taken out of the schedule: every staged prefill or coda result is treated as ready at
the next consume point (the order a host slower than its device sees, and the order the
reference's own CPU tests run in). The model is the reference tests' token-increment loop model
(tests/continuous_depth_batching/test_continuous_depth_batching.py:52-146): the prelude's hidden
value is the token id, each recurrent step adds one and emits the exit signal +10 at step 0 and
-10 after, the coda's token is round(hidden) mod vocab, and a full-depth prefill predicts
(token + steps) mod vocab.

KV pressure (``kv_pressure_mode`` "recompute" or "offload"; continuous_api.py:1584-1669,
offloading_manager.py:172-314, scheduler_base.py:400-460, requests.py:82-126 of both packages): a
decode token that cannot get its block parks its request at the token boundary; parked requests
are retried in park order ahead of each tick's scheduling, stopping at the first that still fails;
when no bucket can run, the parked request with the fewest tokens (the latest to park among
equals) gives up its KV -- swapped to a host pool of ``swap_blocks`` blocks when it holds them all
(offload), else soft-reset (prompt + generated tokens re-prefilled, the replay resumed at
``cursor + 1``). The victim rejoins the waiting queue, and new admissions wait until a request
finishes; swapped requests are restored first on later ticks (offload mode only), with blocks for
their pending token.

Not modelled (the restatement raises): reserve admission, open-loop arrivals and pre-loop exit
distributions.
"""

from __future__ import annotations

from collections import Counter, deque
from dataclasses import dataclass, field

import numpy as np

HAZARD = "cumulative_hazard"
DIRECT = "direct_threshold"
_PLACEHOLDER = -1  # the token id of a staged-but-unsampled token (continuous_batching/requests.py TMP_TOKEN_ID)


class ScheduleOracleError(RuntimeError):
    pass


@dataclass
class _Req:
    rid: str
    prompt: list[int]
    limit: int
    eos: frozenset
    depths: list[int]
    stop: list[list[int]]
    status: str = "pending"  # pending < prefilling < decoding < finished
    remaining: list[int] = field(default_factory=list)
    to_process: list[int] = field(default_factory=list)
    generated: list[int] = field(default_factory=list)
    exit_log: list[int] = field(default_factory=list)
    pos: int = 0
    blocks: list[int] = field(default_factory=list)
    in_flight_tokens: int = 0
    cursor: int = 0
    offloaded: bool = False
    earlier: list[int] = field(default_factory=list)  # tokens generated before soft resets


@dataclass
class _Item:
    req: _Req
    pos: int
    step: int
    depth: int | None
    value: float | None = None  # token-increment hidden value; None until the prelude ran
    slot: int | None = None
    cdf: float = 0.0
    survival: float = 1.0
    pending_step: int | None = None  # delayed replay: the step whose decision is still to apply
    pending_signal: tuple | None = None  # delayed live gate: (source step, signal)


@dataclass
class _Staged:
    kind: str
    tokens: list[int]
    items: list = field(default_factory=list)  # coda: the items; prefill: the (req, qlen, new) rows
    eager: list[bool] = field(default_factory=list)


_ORDER = {"pending": 0, "prefilling": 1, "decoding": 2, "finished": 3}


def _sigmoid_f32(x: float) -> float:
    v = np.float32(x)
    with np.errstate(over="ignore"):
        return float(np.float32(1.0) / (np.float32(1.0) + np.exp(-v, dtype=np.float32)))


class ScheduleOracle:
    """One engine configuration; ``run`` simulates one ``generate_batch`` call."""

    def __init__(self, *, max_recurrent_steps: int, num_blocks: int, block_size: int = 16,
                 max_num_batched_tokens: int = 8192, max_model_len: int = 16384, max_num_seqs: int = 256,
                 min_free_slots: int | None = None, min_coda_batch_size: int = 1, safety_margin: float = 0.2,
                 kv_policy: str = "single", kv_slots_per_layer: int | None = None, refill: bool = True,
                 use_async_batching: bool = True, delay_gate_consumption: bool = True,
                 synthetic_exit_replay: bool = False, exit_threshold: float | None = None,
                 rule: str = HAZARD, offset_one_signal: bool = False, min_recurrent_steps: int = 1,
                 vocab_size: int = 16, replay_eos_finishes: bool = False,
                 replay_offset_one: bool | None = None, mixed_slot_recurrent_batches: bool = False,
                 kv_pressure_mode: str = "none", swap_blocks: int = 0) -> None:
        self.R = max_recurrent_steps
        self.num_blocks = num_blocks
        self.bs = block_size
        self.token_budget = max_num_batched_tokens
        self.max_model_len = max_model_len
        self.cap = min(max_num_seqs, max_num_batched_tokens)
        self.min_free = max(1, self.cap // 8) if min_free_slots is None else min(min_free_slots, self.cap)
        self.min_coda = min(min_coda_batch_size, self.cap)
        self.margin_blocks = safety_margin * num_blocks
        self.fast_path_len = -(-max_model_len // block_size) * block_size
        self.policy = kv_policy
        if kv_policy in ("depth_indexed", "last_exited"):
            self.slots = max_recurrent_steps
        elif kv_policy == "single":
            self.slots = 1
        else:
            self.slots = 2 if kv_slots_per_layer is None else kv_slots_per_layer
        self.copy_on_exit = kv_policy == "last_exited"
        self.slot_homogeneous = self.slots > 1 and not mixed_slot_recurrent_batches
        self.refill = refill
        self.use_async = use_async_batching
        overlap = delay_gate_consumption and use_async_batching
        self.replay = synthetic_exit_replay
        self.threshold = exit_threshold
        self.rule = rule
        self.min_steps = min_recurrent_steps
        self.V = vocab_size
        self.replay_eos = replay_eos_finishes
        if offset_one_signal and not overlap:
            raise ScheduleOracleError("an offset-one signal needs async batching with delayed consumption")
        # Horizons (exit_policy.py:87-137): a live signal is consumed one launch late when the
        # adapter declares offset one or the overlap transport is on; replay follows the transport.
        self.delayed_live = exit_threshold is not None and (offset_one_signal or overlap)
        self.delayed_replay = synthetic_exit_replay and (overlap if replay_offset_one is None else replay_offset_one)
        if kv_pressure_mode not in ("none", "recompute", "offload"):
            raise ScheduleOracleError(f"kv_pressure_mode {kv_pressure_mode!r} is not restated")
        self.pressure = kv_pressure_mode
        # Only the offload mode has a host pool; a pool without room falls back to a soft reset,
        # which copy-on-exit layouts do not allow (offloading_manager.py:183-217).
        self.swap_blocks = swap_blocks if kv_pressure_mode == "offload" else 0

    # -- slot arithmetic (kv_cache_policy.py:84-103) -----------------------------------------------------------
    def _kv_slot(self, step: int) -> int:
        if self.policy in ("depth_indexed", "last_exited"):
            return step
        if self.policy == "single":
            return 0
        return min(step, self.slots - 1)

    # -- run ---------------------------------------------------------------------------------------------------
    def run(self, prompts: list[list[int]], max_new_tokens: int | list[int], *, eos_token_id=None,
            exit_depths: list[list[int]] | None = None, stop_sequences: list[list[int]] | None = None) -> dict:
        n = len(prompts)
        mnt = list(max_new_tokens) if isinstance(max_new_tokens, list) else [max_new_tokens] * n
        mnt = [min(m, self.max_model_len - len(p)) for m, p in zip(mnt, prompts)]
        eos = frozenset() if eos_token_id is None else frozenset(
            [eos_token_id] if isinstance(eos_token_id, int) else list(eos_token_id))
        eos = frozenset(e for e in eos if e >= 0)
        self.reqs = [_Req(f"request-{i}", list(p), mnt[i], eos, list(exit_depths[i]) if exit_depths else [],
                          [list(s) for s in (stop_sequences or [])], remaining=list(p))
                     for i, p in enumerate(prompts)]
        self.free_blocks: deque[int] = deque(range(self.num_blocks))
        self.host_free: deque[int] = deque(range(self.swap_blocks))
        self.host_of: dict[str, list[int]] = {}
        self.parked: dict[str, _Req] = {}  # insertion order is park order
        self.free_slots: list[int] = []
        self.next_slot = 0
        self.waiting: dict[str, _Req] = {}
        self.waiting_order: deque[str] = deque()
        self.active: dict[str, _Req] = {}
        self.in_flight: set[str] = set()
        self.ready: deque[_Item] = deque()
        self.coda_q: deque[_Item] = deque()
        self.staged_prefills: deque[_Staged] = deque()
        self.staged_codas: deque[_Staged] = deque()
        self.backlog: list[tuple[_Item, int]] = []
        self.events: list[tuple] = []
        self.trace: list[dict] = []
        self.tick = 0
        self.block_new = False
        self.stats = Counter()
        self.exit_hist: Counter = Counter()
        self.prelude_tokens: Counter = Counter()
        self.max_mixed = 0
        for r in self.reqs:
            self.waiting[r.rid] = r
            self.waiting_order.append(r.rid)
        if self.refill:
            self._refill_loop()
        else:
            self._wave_loop()
        s = self.stats
        return {
            "tokens": [r.earlier + r.generated for r in self.reqs],
            "exit_depths": [r.exit_log for r in self.reqs],
            "events": self.events,
            "trace": self.trace,
            "free_blocks_at_end": len(self.free_blocks),
            "next_hidden_slot": self.next_slot,
            "stats": {
                "prefill_batches": s["prefill_batches"], "prefill_requests": s["prefill_requests"],
                "prefill_recurrent_steps": s["prefill_recurrent_steps"], "prefill_coda_tokens": s["prefill_coda_tokens"],
                "recurrent_batches": s["recurrent_batches"], "mixed_recurrent_batches": s["mixed_recurrent_batches"],
                "recurrent_steps": s["recurrent_steps"], "coda_batches": s["coda_batches"],
                "coda_tokens": s["coda_tokens"], "scheduler_refills": s["refills"],
                "cancelled_depth_items": s["cancelled"], "exit_kv_copies": s["exit_kv_copies"],
                "scheduler_ticks": s["ticks"], "fixed_depth_recurrent_steps": s["coda_tokens"] * self.R,
                "exit_depth_histogram": dict(self.exit_hist), "prelude_tokens": dict(self.prelude_tokens),
                "max_mixed_depths_per_batch": self.max_mixed,
                "offload_preemptions": s["offload_preemptions"], "recompute_preemptions": s["recompute_preemptions"],
                "restores": s["restores"],
            },
        }

    # -- request bookkeeping (continuous_batching/requests.py:183-237) -------------------------------------------
    def _will_finish_on_pending(self, r: _Req) -> bool:
        if self.replay_eos:
            return False
        return r.in_flight_tokens > 0 and len(r.generated) + r.in_flight_tokens >= r.limit

    def _take_token(self, r: _Req, token: int) -> bool:
        if r.status != "decoding":
            raise ScheduleOracleError(f"{r.rid}: token for a request in state {r.status}")
        r.in_flight_tokens = max(0, r.in_flight_tokens - 1)
        is_eos = token in r.eos
        count = len(r.generated)
        if is_eos or count < r.limit:
            r.generated.append(token)
            r.to_process = [token]
            count += 1
        stop = any(len(s) and len(r.generated) >= len(s) and r.generated[-len(s):] == s for s in r.stop)
        if is_eos or count >= r.limit or stop:
            r.status = "finished"
            return True
        return False

    def _retire(self, r: _Req) -> None:
        self.free_blocks.extend(r.blocks)
        r.blocks = []
        self.parked.pop(r.rid, None)
        self.active.pop(r.rid, None)
        self.in_flight.discard(r.rid)
        if self.waiting.pop(r.rid, None) is not None:
            self.waiting_order.remove(r.rid)
        self.block_new = False

    # -- KV blocks ------------------------------------------------------------------------------------------------
    def _grow_one(self, r: _Req) -> bool:
        """Room for one more decode token: exact-ceil, FIFO block ids (continuous_api.py:1654-1669)."""

        if r.blocks and len(r.blocks) * self.bs - r.pos >= 1:
            return True
        want = -(-(r.pos + 1) // self.bs) - len(r.blocks)
        if want > len(self.free_blocks):
            return False
        r.blocks.extend(self.free_blocks.popleft() for _ in range(want))
        return True

    def _grow_prefill(self, r: _Req, qlen: int) -> bool:
        have = len(r.blocks) * self.bs - r.pos
        if have >= qlen:
            return True
        want = -(-(r.pos + qlen) // self.bs) - len(r.blocks)
        if want > len(self.free_blocks):
            return False
        r.blocks.extend(self.free_blocks.popleft() for _ in range(want))
        return True

    # -- hidden slots -----------------------------------------------------------------------------------------------
    def _take_slots(self, items: list[_Item]) -> None:
        for it in items:
            if self.free_slots:
                it.slot = self.free_slots.pop()
            else:
                it.slot = self.next_slot
                self.next_slot += 1

    def _free_slots(self, items: list[_Item]) -> None:
        for it in items:
            if it.slot is not None:
                self.free_slots.append(it.slot)
                it.slot = None

    # -- queues (scheduler.py:142-189) -------------------------------------------------------------------------------
    def _push(self, it: _Item, front: bool) -> None:
        if not 0 <= it.step < self.R:
            raise ScheduleOracleError(f"step {it.step} out of range")
        self.in_flight.add(it.req.rid)
        if it.step == 0 and self.ready:
            self.stats["refills"] += 1
        if front:
            self.ready.appendleft(it)
        else:
            self.ready.append(it)

    def _push_front(self, items: list[_Item]) -> None:
        for it in reversed(items):
            self._push(it, True)

    def _record(self, stage: str, size: int, **detail) -> None:
        decoding = sum(1 for r in self.active.values() if r.status == "decoding")
        self.trace.append({"launch": len(self.trace) + 1, "tick": self.tick, "stage": stage, "size": size,
                           "waiting": len(self.waiting), "recurrent_queue": len(self.ready),
                           "coda_queue": len(self.coda_q), "decode": decoding - detail.pop("cohort", 0),
                           "active": len(self.active), **detail})

    # -- decode items ----------------------------------------------------------------------------------------------------
    def _new_item(self, r: _Req, value: float | None) -> _Item:
        depth = None
        if r.depths:
            if r.cursor >= len(r.depths):
                if self.replay_eos and r.cursor == len(r.depths):
                    r.cursor += 1
                    depth = r.depths[-1]
                else:
                    raise ScheduleOracleError(f"{r.rid}: replay schedule exhausted")
            else:
                depth = r.depths[r.cursor]
                r.cursor += 1
        return _Item(req=r, pos=r.pos, step=0, depth=depth, value=value)

    def _stage_decode(self, r: _Req) -> _Item | None:
        """The request's next decode item, or None when it parks for lack of a block."""

        if not r.to_process or r.to_process[0] < 0:
            raise ScheduleOracleError(f"{r.rid}: no sampled token to decode")
        if not self._grow_one(r):
            if self.pressure == "none":
                raise ScheduleOracleError(f"{r.rid}: KV cache full and no pressure mode")
            self.parked[r.rid] = r
            return None
        self.parked.pop(r.rid, None)
        return self._new_item(r, float(r.to_process[0]))

    def _retry_parked(self) -> list[_Item]:
        items = []
        for r in list(self.parked.values()):
            it = self._stage_decode(r)
            if it is None:
                break
            items.append(it)
        return items

    # -- preemption and restore (continuous_api.py:1625-1652, offloading_manager.py:172-314) -----------------
    def _yield_parked(self) -> None:
        if len(self.active) <= 1:
            raise ScheduleOracleError("a single request's KV does not fit the cache")
        order = list(self.parked)
        k = min(range(len(order)), key=lambda i: (self.parked[order[i]].pos, -i))
        r = self.parked.pop(order[k])
        if r.blocks and len(self.host_free) >= len(r.blocks):
            self.host_of[r.rid] = [self.host_free.popleft() for _ in r.blocks]
            r.offloaded = True
            self.stats["offload_preemptions"] += 1
        else:
            if self.copy_on_exit:
                raise ScheduleOracleError(f"{r.rid}: no host room and no soft reset under copy-on-exit KV")
            # Soft reset: prompt + generated (the pending token included) re-prefilled as a new
            # prompt, the budget reduced by as many, the replay resumed past the pending token.
            r.earlier = r.earlier + r.generated
            r.prompt = r.prompt + r.generated
            r.limit -= len(r.generated)
            r.depths = r.depths[r.cursor + 1:]
            r.cursor = 0
            r.generated = []
            r.remaining = list(r.prompt)
            r.to_process = []
            r.pos = 0
            r.status = "pending"
            r.in_flight_tokens = 0
            self.stats["recompute_preemptions"] += 1
        self.free_blocks.extend(r.blocks)
        r.blocks = []
        self.active.pop(r.rid, None)
        self.in_flight.discard(r.rid)
        self.waiting[r.rid] = r
        self.waiting_order.append(r.rid)
        self.block_new = True

    def _restore(self) -> list[_Req]:
        """Swapped-out requests back into the active set, in waiting order, each with blocks for
        its pending token; stops at the first that does not fit (scheduler_base.py:434-460)."""

        if self.block_new or self.pressure != "offload":
            return []
        restored = []
        for rid in list(self.waiting_order):
            r = self.waiting[rid]
            if not r.offloaded:
                continue
            if self._open_slots() == 0 or not self._grow_one(r):
                break
            self.active[rid] = r
            del self.waiting[rid]
            self.waiting_order.remove(rid)
            self.host_free.extend(self.host_of.pop(rid))
            r.offloaded = False
            self.stats["restores"] += 1
            restored.append(r)
        return restored

    def _prelude(self, items: list[_Item], site: str) -> None:
        if not items:
            return
        self.prelude_tokens[site] += len(items)
        self._take_slots(items)
        self.events.append(("prelude", site, tuple((it.req.rid, it.pos, it.slot) for it in items)))

    def _drop_finished(self, items: list[_Item]) -> list[_Item]:
        live = [it for it in items if it.req.status != "finished"]
        dead = [it for it in items if it.req.status == "finished"]
        if dead:
            self._free_slots(dead)
            self.stats["cancelled"] += len(dead)
        return live

    # -- exit decisions (continuous_api.py:1671-1724, exit_policy.py:150-169) -----------------------------------------
    def _policy(self, it: _Item, source_step: int, signal: float) -> bool:
        if self.threshold is None:
            return False
        can_exit = source_step + 1 >= self.min_steps
        if self.rule == HAZARD:
            hazard = _sigmoid_f32(signal)
            it.cdf += hazard * it.survival
            it.survival *= 1.0 - hazard
            return can_exit and it.cdf >= self.threshold
        return can_exit and signal < self.threshold

    def _decide_now(self, it: _Item, signal: float) -> bool:
        if it.step == self.R - 1:
            return True
        if it.depth is not None:
            return it.step >= it.depth
        if self.threshold is None:
            return False
        return self._policy(it, it.step, signal)

    def _mark_exit(self, it: _Item, step: int) -> None:
        it.req.exit_log.append(step)
        self.exit_hist[step] += 1
        it.pending_step = None
        it.pending_signal = None
        if self.copy_on_exit and step < self.R - 1:
            self.backlog.append((it, step))

    def _flush_copies(self) -> None:
        self.stats["exit_kv_copies"] += len(self.backlog)
        self.backlog = []

    # -- stages ------------------------------------------------------------------------------------------------------
    def _step_rows(self, items: list[_Item]) -> list[float]:
        signals = []
        for it in items:
            if it.value is None:
                raise ScheduleOracleError("recurrent step on an item without a prelude")
            it.value += 1.0
            signals.append(10.0 if it.step == 0 else -10.0)
        return signals

    def _recurrent_event(self, items: list[_Item]) -> list:
        return [(it.req.rid, it.pos, it.step, it.slot, tuple(it.req.blocks)) for it in items]

    def _run_recurrent(self, items: list[_Item]) -> None:
        items = self._drop_finished(items)
        if not items:
            return
        self.stats["mixed_recurrent_batches"] += 1
        steps = Counter(it.step for it in items)
        self.max_mixed = max(self.max_mixed, len(steps))
        rows = self._recurrent_event(items)
        signals = self._step_rows(items)
        self.stats["recurrent_batches"] += 1
        self.stats["recurrent_steps"] += len(items)
        exits = []
        back: list[_Item] = []
        for it, sig in zip(items, signals):
            step = it.step
            if self.delayed_live:
                prev, it.pending_signal = it.pending_signal, None
                gate = prev is not None and self._policy(it, prev[0], prev[1])
                leave = step == self.R - 1 or gate
                if not leave:
                    it.pending_signal = (step, sig)
            elif self.delayed_replay:
                prev, it.pending_step = it.pending_step, None
                gate = prev is not None and it.depth is not None and prev >= it.depth
                leave = step == self.R - 1 or gate
                if not leave:
                    it.pending_step = step
            else:
                leave = self._decide_now(it, sig)
            exits.append(leave)
            if leave:
                self._mark_exit(it, step)
                self.in_flight.add(it.req.rid)
                self.coda_q.append(it)
            else:
                it.step = step + 1
                back.append(it)
        if back:
            self._push_front(back)
        self._flush_copies()
        self.events.append(("recurrent", tuple(rows), tuple(exits), self.stats["refills"]))
        self._record("recurrent", len(items), depths=dict(steps), exited=sum(exits))

    def _stage_coda(self, items: list[_Item], *, eager_ok: bool) -> _Staged:
        for it in items:
            it.req.in_flight_tokens += 1
        tokens = [int(round(it.value)) % self.V for it in items]
        self.events.append(("coda", tuple((it.req.rid, it.pos, it.slot) for it in items)))
        self._record("coda", len(items))
        staged = _Staged("coda", tokens, items=items, eager=[False] * len(items))
        if eager_ok:
            succ = self._successors(staged)
            if succ:
                self._prelude(succ, "after_coda_eager")
                self._push_front(succ)
                self._record("prelude", len(succ), site="after_coda_eager")
        return staged

    def _successors(self, staged: _Staged) -> list[_Item]:
        """Next items built before the coda's tokens are read (continuous_api.py:1304-1327): every
        row whose request does not finish on its pending token and gets room for one more token."""

        succ = []
        for idx, it in enumerate(staged.items):
            r = it.req
            if self._will_finish_on_pending(r):
                continue
            r.pos += 1
            if not self._grow_one(r):
                r.pos -= 1
                continue
            staged.eager[idx] = True
            succ.append(self._new_item(r, float(staged.tokens[idx])))
        return succ

    def _consume_coda(self, staged: _Staged, *, restage: bool) -> None:
        self.stats["coda_batches"] += 1
        self.stats["coda_tokens"] += len(staged.items)
        self._free_slots(staged.items)
        fresh = []
        for it, tok, eager in zip(staged.items, staged.tokens, staged.eager):
            r = it.req
            if r.status == "finished":
                continue
            if eager:
                if self._take_token(r, tok):
                    self._retire(r)
                continue
            r.pos += 1
            if self._take_token(r, tok):
                self._retire(r)
                continue
            if restage and (it := self._stage_decode(r)) is not None:
                fresh.append(it)
        if fresh:
            self._prelude(fresh, "after_coda_staged")
            self._push_front(fresh)
            self._record("prelude", len(fresh), site="after_coda_staged")

    def _stage_prefill(self, batch: list[tuple[_Req, int, bool]], num_q: int) -> _Staged:
        self.stats["prefill_batches"] += 1
        self.stats["prefill_requests"] += len(batch)
        self.stats["prefill_recurrent_steps"] += num_q * self.R
        rows = []
        tokens = []
        for r, qlen, new in batch:
            rows.append((r.rid, r.pos, qlen, new))
            chunk = r.to_process
            r.pos += qlen
            if new:
                tokens.append((chunk[-1] + self.R) % self.V)
                r.to_process = [_PLACEHOLDER]
                r.in_flight_tokens += 1
        self.events.append(("prefill", tuple(rows)))
        self._record("prefill", len(batch), tokens=num_q)
        return _Staged("prefill", tokens, items=batch)

    # -- admission and prefill packing (scheduler_base.py:154-206, 473-545; scheduler.py:221-320) -------------------
    def _has_decode_work(self) -> bool:
        return any(r.status == "decoding" for r in self.active.values())

    def _admit_prefill(self) -> bool:
        return not self._has_decode_work() or len(self.free_blocks) > self.margin_blocks

    def _open_slots(self) -> int:
        return max(0, self.cap - len(self.active))

    def _prefill_candidates(self) -> list[_Req]:
        bucket = [r for r in self.active.values() if r.status == "prefilling" and r.rid not in self.in_flight]
        if not self.block_new:
            limit = self._open_slots()
            fresh = [self.waiting[rid] for rid in self.waiting_order if not self.waiting[rid].offloaded]
            bucket += fresh[:limit]
        if not bucket:
            return []
        if any(r.status == "prefilling" for r in bucket):
            return bucket
        return bucket if self._open_slots() >= self.min_free else []

    def _pack_prefill(self) -> tuple[list[tuple[_Req, int, bool]], int] | None:
        cands = self._prefill_candidates()
        if not cands:
            return None
        budget = self.token_budget
        cache_budget = self.num_blocks * self.bs
        fast = True
        out: list[tuple[_Req, int, bool]] = []
        taken: set[str] = set()
        for r in cands:
            free = len(self.free_blocks)
            if free < self.margin_blocks and out:
                break
            qlen = min(len(r.remaining), budget)
            if qlen == 0:
                continue
            eligible = qlen == 1 and r.pos < self.fast_path_len
            read = r.pos
            if not (fast and eligible) and cache_budget < read:
                continue
            if not self._grow_prefill(r, qlen):
                if free == 0 and r.rid in self.waiting:
                    break
                continue
            if len(r.remaining) <= qlen:
                if r.status == "pending":
                    self.active[r.rid] = r
                    taken.add(r.rid)
                if _ORDER[r.status] <= _ORDER["prefilling"]:
                    r.to_process = r.remaining
                    r.remaining = []
                    r.status = "decoding"
            else:
                if r.status == "pending":
                    self.active[r.rid] = r
                    r.status = "prefilling"
                    taken.add(r.rid)
                r.to_process = r.remaining[:qlen]
                r.remaining = r.remaining[qlen:]
            self.in_flight.add(r.rid)
            qlen = len(r.to_process)
            fast = fast and qlen == 1 and r.pos < self.fast_path_len
            budget -= qlen
            cache_budget -= read
            out.append((r, qlen, not r.remaining))
            if self.waiting.pop(r.rid, None) is not None:
                taken.add(r.rid)
            if budget == 0 or (cache_budget <= 0 and not fast):
                break
        self.waiting_order = deque(rid for rid in self.waiting_order if rid not in taken)
        if not out:
            return None
        return out, self.token_budget - budget

    # -- refill loop (continuous_api.py:503-606) ---------------------------------------------------------------------
    def _pending_work(self) -> bool:
        return bool(self.coda_q or self.ready or self.active or self.waiting)

    def _consume_all(self) -> None:
        while self.staged_prefills:
            self._consume_prefill(self.staged_prefills.popleft())
        while self.staged_codas:
            self._consume_coda(self.staged_codas.popleft(), restage=True)

    def _consume_prefill(self, staged: _Staged) -> None:
        fresh = []
        k = 0
        for r, _, new in staged.items:
            if not new:
                continue
            tok, eager = staged.tokens[k], staged.eager[k]
            k += 1
            if r.status == "finished":
                continue
            if eager:
                if self._take_token(r, tok):
                    self._retire(r)
                continue
            if self._take_token(r, tok):
                self._retire(r)
                continue
            if (it := self._stage_decode(r)) is not None:
                fresh.append(it)
        if fresh:
            self._prelude(fresh, "after_prefill")
            for it in fresh:
                self._push(it, False)
            self._record("prelude", len(fresh), site="after_prefill")

    def _refill_loop(self) -> None:
        while self._pending_work() or self.staged_codas or self.staged_prefills:
            self._consume_all()
            if not self._pending_work():
                continue
            # Restored requests, then parked ones, share one prelude at the queue head.
            resumed = [it for r in self._restore() if (it := self._stage_decode(r)) is not None]
            resumed += self._retry_parked()
            if resumed:
                self._prelude(resumed, "resumed")
                self._push_front(resumed)
                self._record("prelude", len(resumed), site="resumed")
            self.stats["ticks"] += 1
            self.tick = self.stats["ticks"]
            kind, payload = self._schedule_next()
            if kind is None:
                if self.parked:
                    self._yield_parked()
                    continue
                raise ScheduleOracleError("no work could be scheduled")
            if kind == "coda":
                items = self._drop_finished(payload)
                if items:
                    self.staged_codas.append(self._stage_coda(items, eager_ok=self.use_async))
            elif kind == "prefill":
                batch, num_q = payload
                staged = self._stage_prefill(batch, num_q)
                succ = []
                for r, _, new in batch:
                    if not new:
                        self.in_flight.discard(r.rid)
                        continue
                    self.stats["prefill_coda_tokens"] += 1
                    eager = self.use_async and not self._will_finish_on_pending(r) and self._grow_one(r)
                    if eager:
                        succ.append(self._new_item(r, float(staged.tokens[len(staged.eager)])))
                    staged.eager.append(eager)
                if succ:
                    self._prelude(succ, "after_prefill_eager")
                    for it in succ:
                        self._push(it, False)
                    self._record("prelude", len(succ), site="after_prefill_eager")
                self.staged_prefills.append(staged)
            else:
                self._run_recurrent(payload)
        self._consume_all()

    def _schedule_next(self):
        if len(self.coda_q) >= self.min_coda:
            batch = [self.coda_q.popleft() for _ in range(min(self.cap, len(self.coda_q)))]
            if batch:
                return "coda", batch
        if self._admit_prefill():
            packed = self._pack_prefill()
            if packed is not None:
                return "prefill", packed
        if self.ready:
            return "recurrent", self._pop_recurrent()
        if self.coda_q:
            return "coda", [self.coda_q.popleft() for _ in range(min(self.cap, len(self.coda_q)))]
        return None, None

    def _pop_recurrent(self) -> list[_Item]:
        size = min(self.cap, len(self.ready))
        head = self.ready.popleft()
        batch = [head]
        if self.slot_homogeneous:
            target = self._kv_slot(head.step)
            rest: deque[_Item] = deque()
            while self.ready and len(batch) < size:
                it = self.ready.popleft()
                (batch if self._kv_slot(it.step) == target else rest).append(it)
            rest.extend(self.ready)
            self.ready = rest
        else:
            while self.ready and len(batch) < size:
                batch.append(self.ready.popleft())
        return batch

    # -- no-refill waves (continuous_api.py:608-944) ----------------------------------------------------------------
    def _wave_loop(self) -> None:
        """Prefill while admission allows, then one lockstep wave over the sampled decoders.

        On the delayed horizon (continuous_api.py:636-642, 708-785, 864-932) a wave's coda is read
        only after the next wave's first launch and a prefill's first tokens at the next iteration's
        top; the successors built ahead of those tokens (``self.ahead``, coda successors first, then
        prompt successors) open the next wave, whose prelude takes their hidden slots."""

        delayed = self.delayed_live or self.delayed_replay
        self.ahead: list[_Item] = []
        self.unread_coda: _Staged | None = None
        unread_prefills: list[_Staged] = []
        while self._pending_work():
            self.tick += 1
            for staged in unread_prefills:
                self._first_tokens(staged)
            unread_prefills = []
            self._restore()  # restored decoders join this wave's cohort scan
            ran_prefill = False
            while self._admit_prefill():
                packed = self._pack_prefill()
                if packed is None:
                    break
                batch, num_q = packed
                staged = self._stage_prefill(batch, num_q)
                room = max(0, self.cap - len(self.ahead))
                entered = []
                for r, _, new in batch:
                    if new:
                        self.stats["prefill_coda_tokens"] += 1
                        enter = (delayed and len(entered) < room and not self._will_finish_on_pending(r)
                                 and self._grow_one(r))
                        if enter:
                            entered.append(self._new_item(r, float(staged.tokens[len(staged.eager)])))
                        staged.eager.append(enter)
                    self.in_flight.discard(r.rid)
                if delayed:
                    self.ahead += entered
                    unread_prefills.append(staged)
                else:
                    self._first_tokens(staged)
                ran_prefill = True
            ran_wave = self._wave(delayed)
            if not ran_prefill and not ran_wave:
                if self.parked:
                    self._yield_parked()
                    continue
                if not self._pending_work():
                    continue
                raise ScheduleOracleError("no-refill loop stalled")
        if unread_prefills or self.ahead or self.unread_coda is not None:
            raise ScheduleOracleError("no-refill loop ended with unread results")

    def _first_tokens(self, staged: _Staged) -> None:
        k = 0
        for r, _, new in staged.items:
            if not new:
                continue
            tok = staged.tokens[k]
            k += 1
            if r.status != "finished" and self._take_token(r, tok):
                self._retire(r)

    def _wave(self, delayed: bool) -> bool:
        ahead = [it for it in self.ahead if it.req.status != "finished"]
        self.stats["cancelled"] += len(self.ahead) - len(ahead)
        self.ahead = []
        coda, self.unread_coda = self.unread_coda, None
        behind = {it.req.rid for it in coda.items} if coda is not None else set()
        cohort = [r for r in self.active.values()
                  if r.status == "decoding" and r.to_process and r.to_process[0] >= 0 and r.rid not in behind]
        cohort = cohort[: max(0, self.cap - len(ahead))]
        items = ahead + [it for r in cohort if (it := self._stage_decode(r)) is not None]
        if not items:
            if coda is None:
                return False
            self._consume_coda(coda, restage=False)
            return True
        self._prelude(items, "wave_cohort")
        self._record("prelude", len(items), site="wave_cohort", cohort=len(items))
        live = items
        done: list[_Item] = []
        for step in range(self.R):
            for it in live:
                it.step = step
            rows = self._recurrent_event(live)
            signals = self._step_rows(live)
            self.stats["recurrent_batches"] += 1
            self.stats["recurrent_steps"] += len(live)
            if coda is not None:
                self._consume_coda(coda, restage=False)
                coda = None
            keep, out, exits, dead = [], [], [], []
            for it, sig in zip(live, signals):
                if it.req.status == "finished":
                    dead.append(it)
                    exits.append(False)
                    continue
                if self.delayed_live:
                    prev, it.pending_signal = it.pending_signal, None
                    leave = step == self.R - 1 or (prev is not None and self._policy(it, prev[0], prev[1]))
                    if not leave:
                        it.pending_signal = (step, sig)
                elif self.delayed_replay:
                    prev, it.pending_step = it.pending_step, None
                    leave = step == self.R - 1 or (prev is not None and it.depth is not None and prev >= it.depth)
                    if not leave:
                        it.pending_step = step
                else:
                    leave = self._decide_now(it, sig)
                exits.append(leave)
                if leave:
                    self._mark_exit(it, step)
                    out.append(it)
                else:
                    keep.append(it)
            if dead:
                self._free_slots(dead)
                self.stats["cancelled"] += len(dead)
            self._flush_copies()
            self.events.append(("recurrent", tuple(rows), tuple(exits), self.stats["refills"]))
            self._record("recurrent", len(live), depths={step: len(live)}, exited=len(out), cohort=len(items))
            done.extend(out)
            live = keep
            if not live:
                break
        if not done:
            return True
        staged = self._stage_coda(done, eager_ok=False)
        if delayed:
            self.ahead = self._successors(staged)
            self.unread_coda = staged
        else:
            self._consume_coda(staged, restage=False)
        return True


__all__ = ["ScheduleOracle", "ScheduleOracleError", "HAZARD", "DIRECT"]
