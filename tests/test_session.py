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
    ctl.observe_residual(1, 0.05, t=1)
    assert not ctl.licensed
    ctl.observe_residual(1, 0.2, t=2)        # a miss resets the streak
    ctl.observe_residual(1, 0.05, t=3)
    assert not ctl.licensed
    ctl.observe_residual(1, 0.05, t=4)
    assert ctl.licensed and ctl.next_gap == 2
    ctl.observe_residual(2, 0.1, t=6)        # rate 0.05 < tau: interval grows by 2
    assert ctl.next_gap == 4
    ctl.observe_residual(4, 0.8, t=10)       # rate 0.2: the interval is kept
    assert ctl.next_gap == 4
    assert ctl.observe_validation(age=3, error=0.05)
    assert ctl.lease_ok(5) and not ctl.lease_ok(6)
    assert ctl.observe_validation(age=2, error=0.05)   # the lease span grows by 2
    assert ctl.lease_ok(6) and not ctl.lease_ok(7)
    assert not ctl.observe_validation(age=1, error=float("nan"))
    assert not ctl.lease_ok(0)


def test_controller_budget_pacing():
    ctl = Controller(ScheduleConfig(num_steps=50, tau=0.1, budget=10, tail_exact=2))
    ctl.license()
    ctl.computed = 4
    # 10 - 4 - 2 = 4 computations left for steps 20..47: every 7 steps
    assert ctl.pacing_gap(20) == 7
    assert ctl.allowed_gap(20) == 2
    ctl.next_gap = 12
    assert ctl.allowed_gap(20) == 7
    assert ctl.in_exact_tail(48) and not ctl.in_exact_tail(47)
    ctl.computed = 8
    assert ctl.mid_budget_exhausted() and not ctl.budget_exhausted()


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
