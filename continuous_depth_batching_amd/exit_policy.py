"""Exit-decision policy: which rule interprets a gate signal and when it is consumed.

Mirrors the reference's ExitPolicy surface (continuous_depth_batching/exit_policy.py:12-183):
the rule (cumulative hazard for Ouro's sigmoid gate, direct threshold for
Huginn's latent difference), the decision horizon (same step, or one launch
later on the delayed/lookahead path) and the serving-time validation. The
per-token arithmetic itself runs on the GPU in ``cdb_exit_gate``; this class
only resolves the parameters the kernel is launched with. ``should_exit`` is
kept as the host-side restatement of one decision for callers that hold a
signal on the host.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
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
    rule: ExitDecisionRule
    decision_horizon: DecisionHorizon = DecisionHorizon.SAME_STEP


@dataclass
class TokenExitPolicyState:
    exit_cdf: float = 0.0
    survival: float = 1.0


@dataclass(frozen=True)
class ExitPolicy:
    spec: ExitPolicySpec
    threshold: float | None
    min_recurrent_steps: int
    max_recurrent_steps: int
    delay_gate_consumption: bool
    use_async_batching: bool
    synthetic_exit_replay: bool

    def __post_init__(self) -> None:
        if self.threshold is None:
            return
        if not math.isfinite(self.threshold):
            raise ValueError("exit_threshold must be finite")
        if self.spec.rule is ExitDecisionRule.DIRECT_THRESHOLD:
            if self.threshold < 0:
                raise ValueError("exit_threshold must be nonnegative for direct-threshold policies")
        elif not 0 < self.threshold <= 1:
            raise ValueError("exit_threshold must be in (0, 1] for probability policies")

    @property
    def delayed_transport_enabled(self) -> bool:
        return self.delay_gate_consumption and self.use_async_batching

    @property
    def decision_horizon(self) -> DecisionHorizon:
        if self.spec.rule is ExitDecisionRule.PRELOOP_DISTRIBUTION:
            return DecisionHorizon.SAME_STEP
        if self.spec.decision_horizon is DecisionHorizon.OFFSET_ONE or self.delayed_transport_enabled:
            return DecisionHorizon.OFFSET_ONE
        return DecisionHorizon.SAME_STEP

    @property
    def synthetic_decision_horizon(self) -> DecisionHorizon:
        return DecisionHorizon.OFFSET_ONE if self.delayed_transport_enabled else DecisionHorizon.SAME_STEP

    def validate_serving_timing(self) -> None:
        if self.spec.decision_horizon is DecisionHorizon.OFFSET_ONE and not self.delayed_transport_enabled:
            raise ValueError("An adapter-declared offset-1 exit signal requires the delayed-gate-consumption path "
                             "(use_async_batching=True and delay_gate_consumption=True).")

    def decides_before_loop(self) -> bool:
        return self.spec.rule is ExitDecisionRule.PRELOOP_DISTRIBUTION

    def uses_delayed_online_signal(self, *, signal_enabled: bool) -> bool:
        return (signal_enabled and self.threshold is not None and not self.decides_before_loop()
                and self.decision_horizon is DecisionHorizon.OFFSET_ONE)

    def uses_delayed_synthetic_exit(self) -> bool:
        return self.synthetic_exit_replay and self.synthetic_decision_horizon is DecisionHorizon.OFFSET_ONE

    def delayed(self, *, signal_enabled: bool = True) -> bool:
        """Whether routing after a launch uses the previous launch's decision input."""

        return self.uses_delayed_online_signal(signal_enabled=signal_enabled) or self.uses_delayed_synthetic_exit()

    def should_exit(self, state: TokenExitPolicyState, *, source_step: int, signal: float) -> bool:
        """One host-side decision (exit_policy.py:150-169); the engine uses the device kernel instead."""

        if self.threshold is None:
            return False
        can_exit = source_step + 1 >= self.min_recurrent_steps
        if self.spec.rule is ExitDecisionRule.CUMULATIVE_HAZARD:
            hazard = 1.0 / (1.0 + math.exp(-float(signal)))
            state.exit_cdf += hazard * state.survival
            state.survival *= 1.0 - hazard
            return can_exit and state.exit_cdf >= self.threshold
        if self.spec.rule is ExitDecisionRule.DIRECT_THRESHOLD:
            return can_exit and float(signal) < self.threshold
        raise RuntimeError("Preloop exit distributions do not consume per-step signals")
