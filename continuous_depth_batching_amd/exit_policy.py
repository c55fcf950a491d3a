"""The exit gate's launch record.

Every per-token exit decision runs on the device in ``cdb_exit_gate``. The host only needs the
gate's launch parameters, and one routing fact: whether a launch's decisions route the item
right away or one launch later. ``ExitPolicy`` takes the adapter's signal spec and the engine
configuration (the reference's ExitPolicy fields, continuous_depth_batching/exit_policy.py:
50-58) and resolves them once into that record:

  * ``lag``           launches between a decision and the routing that applies it (0 or 1);
  * ``round_hazard``  whether the hazard is rounded to the model dtype before it is accumulated
                      (a synchronous decision reads the model-dtype sigmoid, a delayed one the
                      float32 signal; cdb/model_runner.py:807-813);
  * the rule, threshold and step bounds, checked against the rule's signal scale.

Resolution (reference exit_policy.py:87-146): a live signal waits one launch when the adapter
declares an offset-one signal or when delayed consumption runs on the async path; a replayed
trace waits one launch only in the latter case; a pre-loop distribution never waits.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from enum import Enum, IntEnum


class ExitDecisionRule(str, Enum):
    CUMULATIVE_HAZARD = "cumulative_hazard"
    DIRECT_THRESHOLD = "direct_threshold"
    PRELOOP_DISTRIBUTION = "preloop_distribution"


class DecisionHorizon(IntEnum):
    SAME_STEP = 0
    OFFSET_ONE = 1


@dataclass(frozen=True)
class ExitPolicySpec:
    """What an adapter's gate signal means, and when the adapter can first deliver it."""

    rule: ExitDecisionRule
    decision_horizon: DecisionHorizon = DecisionHorizon.SAME_STEP


# The threshold each rule accepts: a probability for the CDF rules, a nonnegative score for the
# direct comparison (the latent difference is a norm ratio).
_THRESHOLD_SCALE = {
    ExitDecisionRule.CUMULATIVE_HAZARD: ("in (0, 1] for probability policies", lambda t: 0.0 < t <= 1.0),
    ExitDecisionRule.PRELOOP_DISTRIBUTION: ("in (0, 1] for probability policies", lambda t: 0.0 < t <= 1.0),
    ExitDecisionRule.DIRECT_THRESHOLD: ("nonnegative for direct-threshold policies", lambda t: t >= 0.0),
}


@dataclass(frozen=True)
class ExitPolicy:
    spec: ExitPolicySpec
    threshold: float | None
    min_recurrent_steps: int
    max_recurrent_steps: int
    delay_gate_consumption: bool
    use_async_batching: bool
    synthetic_exit_replay: bool
    lag: int = field(init=False)
    round_hazard: bool = field(init=False)

    def __post_init__(self) -> None:
        if self.threshold is not None:
            scale, accepts = _THRESHOLD_SCALE[self.spec.rule]
            if not math.isfinite(self.threshold):
                raise ValueError("exit_threshold must be finite")
            if not accepts(self.threshold):
                raise ValueError(f"exit_threshold must be {scale}, got {self.threshold}")
        overlap = self.delay_gate_consumption and self.use_async_batching
        preloop = self.spec.rule is ExitDecisionRule.PRELOOP_DISTRIBUTION
        live_late = (self.threshold is not None and not preloop
                     and (overlap or self.spec.decision_horizon is DecisionHorizon.OFFSET_ONE))
        replay_late = self.synthetic_exit_replay and overlap
        lag = 1 if (live_late or replay_late) else 0
        object.__setattr__(self, "lag", lag)
        object.__setattr__(self, "round_hazard", lag == 0)

    def delayed(self) -> bool:
        """Whether a launch's decisions route the item only after its next launch."""

        return self.lag == 1

    def validate_serving_timing(self) -> None:
        """An offset-one signal exists only where a launch's decisions are applied one launch later."""

        overlap = self.delay_gate_consumption and self.use_async_batching
        if self.spec.decision_horizon is DecisionHorizon.OFFSET_ONE and not overlap:
            raise ValueError("An offset-1 exit signal needs delayed gate consumption on the async path "
                             "(use_async_batching=True and delay_gate_consumption=True).")
