"""Per-sample step scheduling from two online error measurements (recap/controller.py).

* the prediction mismatch ``m`` observed at a computed step, over the ``h`` steps since
  the previous computed step (``m / h`` is its rate);
* the refinement error ``e_detail`` measured at a dense refresh (the validation
  statistics the operator drains).

The controller grows the reuse interval while the mismatch rate stays under ``tau``,
leases the cached refinement for a number of steps while ``e_detail`` stays under
``tau * detail_tau_mult``, and paces computations against an optional budget.  It holds
no tensors: the session asks it questions and reports measurements.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from .config import ScheduleConfig

# A checked interval that passes grows by this many steps; the first reuse interval and
# the first refinement lease span are this long (recap/controller.py:17).
EARN = 2


@dataclass
class Controller:
    """Scheduling state of one sample (recap/controller.py:20-131)."""

    config: ScheduleConfig

    streak: int = 0                 # consecutive one-step mismatches under tau
    licensed: bool = False          # reuse has started
    next_gap: int | None = None     # next reuse interval
    detail_lease: int | None = None  # oldest refinement age a sparse step may use
    lease_span: int = EARN
    rate_last: float | None = None
    rate_sum: float = 0.0
    rate_obs: int = 0
    computed: int = 0               # transformer evaluations so far
    validations: list[dict] = field(default_factory=list)

    # -- measurements ----------------------------------------------------------------------

    @property
    def lease_tolerance(self) -> float:
        """tau_detail = tau * detail_tau_mult."""
        return self.config.tau * self.config.detail_tau_mult

    def observe_residual(self, h: int, m: float, t: int | None = None) -> None:
        """Fold in the mismatch ``m`` of an extrapolation over ``h`` steps."""
        tau = self.config.tau
        if h <= 0 or not math.isfinite(m) or m <= 0.0:
            return
        if not self.licensed:
            # Before reuse: two consecutive one-step mismatches under tau (at or after
            # prefix_floor) start it.
            if h != 1:
                return
            self.streak = self.streak + 1 if m < tau else 0
            if self.streak >= 2 and (t is None or t >= self.config.prefix_floor):
                self.license()
            return
        rate = m / float(h)
        self.rate_last = rate
        self.rate_sum += rate
        self.rate_obs += 1
        if h >= EARN:
            # An interval that passed grows by EARN; one that failed is kept.
            self.next_gap = h + EARN if rate < tau else h

    def observe_validation(self, age: int, error: float) -> bool:
        """Renew (error under tau_detail) or revoke the refinement lease."""
        passed = math.isfinite(error) and error < self.lease_tolerance
        if passed:
            self.detail_lease = age + self.lease_span
            self.lease_span += EARN
        else:
            self.detail_lease = None
            self.lease_span = EARN
        return passed

    def lease_ok(self, age: int) -> bool:
        """May a sparse step use a refinement refreshed ``age`` steps ago?"""
        return self.detail_lease is not None and age <= self.detail_lease

    # -- placement -------------------------------------------------------------------------

    def license(self) -> None:
        """Start reuse at the shortest interval."""
        self.licensed = True
        self.next_gap = EARN

    def in_exact_tail(self, t: int) -> bool:
        tail = self.config.tail_exact
        return tail > 0 and t >= self.config.num_steps - tail

    def pacing_gap(self, t: int) -> int | None:
        """The interval that spends the remaining budget evenly over the remaining steps,
        shortened (never lengthened) while the latest mismatch rate is above its mean."""
        budget = self.config.budget
        if budget is None:
            return None
        remaining = budget - self.computed - self.config.tail_exact
        if remaining <= 0:
            return None
        steps_left = self.config.num_steps - self.config.tail_exact - t
        gap = max(1, math.ceil(steps_left / remaining))
        if self.rate_obs and self.rate_last:
            mean_rate = self.rate_sum / self.rate_obs
            gap = min(gap, max(1, round(gap * mean_rate / max(self.rate_last, 1e-12))))
        return gap

    def allowed_gap(self, t: int) -> int:
        if self.next_gap is None:
            raise RuntimeError("allowed_gap queried before reuse was licensed")
        pace = self.pacing_gap(t)
        return self.next_gap if pace is None else min(self.next_gap, pace)

    def budget_exhausted(self) -> bool:
        budget = self.config.budget
        return budget is not None and self.computed >= budget

    def mid_budget_exhausted(self) -> bool:
        """No computations left outside the exact tail."""
        budget = self.config.budget
        return budget is not None and self.computed >= budget - self.config.tail_exact

    def prefix_overspent(self) -> bool:
        """The dense prefix has used half of the budget."""
        budget = self.config.budget
        return budget is not None and 2 * self.computed >= budget

    def state(self) -> dict:
        return {
            "computed_endpoints": self.computed,
            "budget": self.config.budget,
            "validation_history": list(self.validations),
        }
