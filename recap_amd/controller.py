"""Scheduling policy of the step loop: when a denoising step is computed and when the
attention refinement may be used (the decisions of recap/controller.py:20-131).

The policy is three independent pieces of state, each fed by one measurement:

``ReuseInterval``  the prediction mismatch ``m`` over an interval of ``h`` steps.  Before
                   reuse is licensed, two consecutive one-step mismatches under ``tau`` (at
                   or after the prefix floor) license it at the shortest interval; once
                   licensed, an interval whose rate ``m / h`` stays under ``tau`` grows by
                   ``STEP`` and one that does not is kept.
``DetailLease``    the refinement error ``e_detail`` measured at a refresh.  A pass
                   (``e_detail < tau_detail``) lets sparse steps use refinements up to
                   ``age + span`` steps old and widens the span by ``STEP``; a failure (or a
                   non-finite error) revokes the lease and resets the span.
``Budget``         computed steps against the budget ``B``: the pace that spends what is left
                   evenly over the steps left (shortened, never lengthened, when the latest
                   mismatch rate runs above its running mean), the exact tail, and the
                   half-spent mark that licenses reuse early.

``Controller`` composes them and answers the step loop's questions.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from .config import ScheduleConfig

STEP = 2   # growth of a reuse interval or of the refinement lease after a passed check


@dataclass
class ReuseInterval:
    """When extrapolated (reused) steps are allowed, and how far apart computed steps are."""

    tau: float
    prefix_floor: int
    passes: int = 0               # consecutive one-step mismatches under tau, before licensing
    licensed: bool = False
    gap: int | None = None        # steps from one computed step to the next

    def grant(self) -> None:
        self.licensed, self.gap = True, STEP

    def observe(self, h: int, m: float, t: int | None) -> float | None:
        """Take one mismatch; returns the licensed rate m / h (None before licensing)."""
        if not self.licensed:
            if h == 1:
                self.passes = self.passes + 1 if m < self.tau else 0
                if self.passes >= 2 and (t is None or t >= self.prefix_floor):
                    self.grant()
            return None
        rate = m / float(h)
        if h >= STEP:
            self.gap = h + STEP if rate < self.tau else h
        return rate


@dataclass
class DetailLease:
    """How old a refinement the sparse steps may use."""

    tolerance: float
    horizon: int | None = None    # the oldest usable age, None: no valid lease
    span: int = STEP

    def judge(self, age: int, error: float) -> bool:
        passed = math.isfinite(error) and error < self.tolerance
        if passed:
            self.horizon, self.span = age + self.span, self.span + STEP
        else:
            self.horizon, self.span = None, STEP
        return passed

    def covers(self, age: int) -> bool:
        return self.horizon is not None and age <= self.horizon


@dataclass
class Budget:
    """Computed steps against the budget B, and the mismatch rates that pace them."""

    limit: int | None
    num_steps: int
    tail: int
    computed: int = 0
    rate_latest: float | None = None
    rate_total: float = 0.0
    rate_count: int = 0

    def note_rate(self, rate: float) -> None:
        self.rate_latest = rate
        self.rate_total += rate
        self.rate_count += 1

    def spent(self, reserve: int = 0) -> bool:
        """At least B - reserve computed steps (never, without a budget)."""
        return self.limit is not None and self.computed >= self.limit - reserve

    def half_spent(self) -> bool:
        return self.limit is not None and 2 * self.computed >= self.limit

    def in_tail(self, t: int) -> bool:
        return self.tail > 0 and t >= self.num_steps - self.tail

    def pace(self, t: int) -> int | None:
        """Steps between computed steps that spend the rest of the budget (the exact tail
        held back) evenly over the steps left; None without a budget or with nothing left."""
        if self.limit is None:
            return None
        left = self.limit - self.computed - self.tail
        if left <= 0:
            return None
        pace = max(1, math.ceil((self.num_steps - self.tail - t) / left))
        if self.rate_count and self.rate_latest:
            mean = self.rate_total / self.rate_count
            pace = min(pace, max(1, round(pace * mean / max(self.rate_latest, 1e-12))))
        return pace


@dataclass
class Controller:
    """The scheduling state of one sample."""

    config: ScheduleConfig
    interval: ReuseInterval = field(init=False)
    lease: DetailLease = field(init=False)
    budget: Budget = field(init=False)
    validations: list[dict] = field(default_factory=list)

    def __post_init__(self) -> None:
        c = self.config
        self.interval = ReuseInterval(c.tau, c.prefix_floor)
        self.lease = DetailLease(c.tau * c.detail_tau_mult)
        self.budget = Budget(c.budget, c.num_steps, c.tail_exact)

    # -- measurements --------------------------------------------------------------------

    def record_mismatch(self, h: int, m: float, t: int | None = None) -> None:
        """The relative mismatch ``m`` of a computed step ``h`` steps after the previous
        one; ignored unless h > 0 and m is finite and positive."""
        if h <= 0 or not math.isfinite(m) or m <= 0.0:
            return
        rate = self.interval.observe(h, m, t)
        if rate is not None:
            self.budget.note_rate(rate)

    def record_refinement_error(self, age: int, error: float) -> bool:
        """``e_detail`` of a refinement ``age`` steps old; True when it passed."""
        return self.lease.judge(age, error)

    def count_computed(self) -> None:
        self.budget.computed += 1

    # -- questions -----------------------------------------------------------------------

    @property
    def licensed(self) -> bool:
        return self.interval.licensed

    @property
    def computed(self) -> int:
        return self.budget.computed

    def start_reuse(self) -> None:
        self.interval.grant()

    def refinement_usable(self, age: int) -> bool:
        return self.lease.covers(age)

    def reuse_span(self, t: int) -> int:
        """Steps until the next computed step: the reuse interval, or the budget's pace when
        that is shorter."""
        if self.interval.gap is None:
            raise RuntimeError("reuse_span asked before reuse was licensed")
        pace = self.budget.pace(t)
        return self.interval.gap if pace is None else min(self.interval.gap, pace)

    def in_exact_tail(self, t: int) -> bool:
        return self.budget.in_tail(t)

    def budget_spent(self) -> bool:
        return self.budget.spent()

    def budget_spent_before_tail(self) -> bool:
        return self.budget.spent(reserve=self.config.tail_exact)

    def half_budget_spent(self) -> bool:
        return self.budget.half_spent()

    def state(self) -> dict:
        """The record keys of recap/controller.py:126-131."""
        return {"computed_endpoints": self.budget.computed, "budget": self.config.budget,
                "validation_history": list(self.validations)}
