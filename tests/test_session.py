"""The step loop (session) and its controller on the CPU, with a stand-in operator and toy
transformers whose outputs follow known trajectories (recap/session.py,
recap/controller.py)."""

from __future__ import annotations

import dataclasses
from dataclasses import dataclass

import pytest
import torch

import recap_amd
from recap_amd import EXACT, REFRESH, REUSE, SPARSE, Controller, RecapSession
from recap_amd.config import GeometryConfig, RecapConfig, ScheduleConfig


class StubOperator:
    """The Operator surface the session drives; records the calls."""

    def __init__(self, n_streams=1, validations=None):
        self.n_streams = n_streams
        self.banks_valid = False
        self.calls = []
        self.validations = list(validations or [])
        self.stream = 0

    def reset(self):
        self.banks_valid = False
        self.calls.append(("reset",))

    def begin_step(self, step, kind):
        self.calls.append(("begin", step, kind))
        if kind == REFRESH:
            self.banks_valid = True

    def set_stream(self, stream):
        self.stream = stream

    def drain_validation(self):
        return self.validations.pop(0) if self.validations else None


@dataclass
class Out:
    sample: torch.Tensor


class LinearTransformer:
    """Output x0 + t * x1 at step t (the step counter advances once per call group)."""

    def __init__(self, calls_per_step=1, slope=0.01, wrap_output=False, seed=0):
        g = torch.Generator().manual_seed(seed)
        self.x0 = torch.randn(4, 64, generator=g)
        self.x1 = slope * torch.randn(4, 64, generator=g)
        self.calls = 0
        self.calls_per_step = calls_per_step
        self.wrap_output = wrap_output

    def truth(self, t):
        return self.x0 + t * self.x1

    def forward(self, t):
        self.calls += 1
        out = self.truth(t)
        return Out(out) if self.wrap_output else (out,)


class Pipe:
    def __init__(self, transformer):
        self.transformer = transformer


def run(session, transformer, steps):
    outs = []
    for t in range(steps):
        for _ in range(session.calls_per_step):
            outs.append(transformer.forward(t))
    return outs


def config(**schedule):
    return dataclasses.replace(RecapConfig(), sync_step_timing=False,
                               geometry=GeometryConfig(grid=(4, 32, 32), text_tokens=0),
                               schedule=ScheduleConfig(**schedule))


def test_controller_license_interval_growth_and_lease():
    ctl = Controller(ScheduleConfig(num_steps=20, tau=0.1))
    ctl.record_mismatch(1, 0.05, t=1)
    assert not ctl.licensed
    ctl.record_mismatch(1, 0.2, t=2)         # a miss resets the run of passes
    ctl.record_mismatch(1, 0.05, t=3)
    assert not ctl.licensed
    ctl.record_mismatch(2, 0.05, t=5)        # intervals other than 1 do not count yet
    assert not ctl.licensed
    ctl.record_mismatch(1, 0.05, t=4)
    assert ctl.licensed and ctl.interval.gap == 2
    ctl.record_mismatch(2, 0.1, t=6)         # rate 0.05 < tau: the interval grows by 2
    assert ctl.interval.gap == 4
    ctl.record_mismatch(4, 0.8, t=10)        # rate 0.2: the interval is kept
    assert ctl.interval.gap == 4
    ctl.record_mismatch(4, float("nan"), t=14)   # ignored
    ctl.record_mismatch(0, 0.01, t=14)
    assert ctl.interval.gap == 4 and ctl.budget.rate_count == 2
    assert ctl.record_refinement_error(age=3, error=0.05)
    assert ctl.refinement_usable(5) and not ctl.refinement_usable(6)
    assert ctl.record_refinement_error(age=2, error=0.05)   # the lease span grows by 2
    assert ctl.refinement_usable(6) and not ctl.refinement_usable(7)
    assert not ctl.record_refinement_error(age=1, error=float("nan"))
    assert not ctl.refinement_usable(0)
    assert ctl.record_refinement_error(age=1, error=0.01)   # the span restarts at 2
    assert ctl.refinement_usable(3) and not ctl.refinement_usable(4)


def test_controller_licensing_waits_for_the_prefix_floor():
    ctl = Controller(ScheduleConfig(num_steps=20, tau=0.1, prefix_floor=5))
    for t in (1, 2, 3):
        ctl.record_mismatch(1, 0.01, t=t)
    assert not ctl.licensed                  # passes before the floor do not license
    ctl.record_mismatch(1, 0.01, t=5)
    assert ctl.licensed


def test_controller_budget_pacing():
    ctl = Controller(ScheduleConfig(num_steps=50, tau=0.1, budget=10, tail_exact=2))
    ctl.start_reuse()
    ctl.budget.computed = 4
    # 10 - 4 - 2 = 4 computations left for steps 20..47: every 7 steps
    assert ctl.budget.pace(20) == 7
    assert ctl.reuse_span(20) == 2
    ctl.interval.gap = 12
    assert ctl.reuse_span(20) == 7
    # a mismatch rate above its running mean shortens the pace: mean 0.05, latest 0.1
    ctl.budget.note_rate(0.0)
    ctl.budget.note_rate(0.1)
    assert ctl.budget.pace(20) == 4          # round(7 * 0.05 / 0.1) = round(3.5) = 4
    assert ctl.in_exact_tail(48) and not ctl.in_exact_tail(47)
    ctl.budget.computed = 8
    assert ctl.budget_spent_before_tail() and not ctl.budget_spent()
    assert ctl.half_budget_spent()
    assert ctl.budget.pace(20) is None       # nothing left before the tail
    with pytest.raises(RuntimeError):
        Controller(ScheduleConfig()).reuse_span(0)


def test_reuse_extrapolation_is_exact_on_a_linear_trajectory():
    steps = 12
    tr = LinearTransformer(slope=0.01)
    op = StubOperator()
    session = RecapSession(config(num_steps=steps, tau=0.05), op)
    session.install(tr)
    outs = run(session, tr, steps)
    actions = [row["a"] for row in session.actions]
    assert REUSE in actions and actions[0] == EXACT
    # The fitted gain is 1 and every reused output equals the true one.
    assert session.gain == pytest.approx(1.0, rel=1e-5)
    for t, (row, out) in enumerate(zip(session.actions, outs)):
        assert row["t"] == t
        torch.testing.assert_close(out[0], tr.truth(t), rtol=1e-5, atol=1e-5)
    # The transformer ran only on computed steps.
    assert tr.calls == sum(a != REUSE for a in actions)
    # The first computation after reuse started is a refresh; later computed steps
    # inside a valid lease may be sparse.
    computed = [a for a in actions if a != REUSE]
    first_after = computed[computed.index(EXACT) + 1:]
    assert first_after and REFRESH in first_after


def test_no_reuse_when_the_mismatch_stays_above_tau():
    steps = 8
    tr = LinearTransformer(slope=1.0)   # one-step mismatch ~ 1/|x0 + t x1| >> tau
    session = RecapSession(config(num_steps=steps, tau=0.01), StubOperator())
    session.install(tr)
    run(session, tr, steps)
    assert [row["a"] for row in session.actions] == [EXACT] * steps
    assert not session.controller.licensed


def test_sparse_steps_only_inside_the_validated_lease():
    steps = 20
    tr = LinearTransformer(slope=0.001)
    op = StubOperator(validations=[(2, 0.01), (2, 0.01), (2, 0.01), (2, 0.01)])
    session = RecapSession(config(num_steps=steps, tau=0.05), op)
    session.install(tr)
    run(session, tr, steps)
    last_refresh = None
    lease = None
    for row in session.actions:
        if row["a"] == REFRESH:
            last_refresh = row["t"]
            if "validation" in row:
                lease = row["validation"]["age"] + 2 if lease is None else lease
        if row["a"] == SPARSE:
            assert last_refresh is not None and row["t"] > last_refresh
    begins = [c for c in op.calls if c[0] == "begin"]
    assert [c[2] for c in begins] == [r["a"] for r in session.actions if r["a"] != REUSE]


def test_calls_per_step_share_one_decision_and_the_horizon_is_enforced():
    steps = 6
    tr = LinearTransformer(calls_per_step=2, slope=0.01, wrap_output=True)
    op = StubOperator(n_streams=2)
    session = RecapSession(config(num_steps=steps, tau=0.05), op, calls_per_step=2)
    session.install(tr)
    outs = run(session, tr, steps)
    assert len(session.actions) == steps
    assert isinstance(outs[0], Out)
    with pytest.raises(RuntimeError, match="past the configured horizon"):
        tr.forward(steps)
    with pytest.raises(ValueError, match="streams"):
        RecapSession(config(), StubOperator(n_streams=1), calls_per_step=2)


def test_install_reset_and_registry():
    tr = LinearTransformer()
    session = RecapSession(config(num_steps=4, tau=0.05), StubOperator())
    session.install(tr)
    with pytest.raises(RuntimeError, match="already has"):
        session.install(tr)
    run(session, tr, 4)
    # A pipeline that restored the original forward (CPU offload) is re-wrapped on reset.
    tr.forward = LinearTransformer.forward.__get__(tr)
    session.reset()
    assert session.call_index == 0 and session.actions == []
    run(session, tr, 4)
    assert len(session.actions) == 4

    cfg = config(num_steps=4, tau=0.05)
    with pytest.raises(RuntimeError, match="register"):
        recap_amd.install(Pipe(LinearTransformer()), cfg, model="hunyuan")
    with pytest.raises(ValueError, match="no integration"):
        recap_amd.install(Pipe(LinearTransformer()), cfg, model="nonexistent")

    def build(pipe, cfg):
        return StubOperator(), {"calls_per_step": 1, "model": "toy"}

    recap_amd.register_builder("toy", build)
    try:
        pipe = Pipe(LinearTransformer())
        session = recap_amd.install(pipe, cfg, model="toy")
        run(session, pipe.transformer, 4)
        assert session.summary()["model"]["model"] == "toy"
        assert sum(session.summary()["counts"].values()) == 4
    finally:
        recap_amd._BUILDERS.pop("toy", None)
