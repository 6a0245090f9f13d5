"""Step-loop scenarios shared by the session golden generator (which drives the
reference's RecapSession, recap/session.py) and the CPU test that replays them through
recap_amd.RecapSession: schedule settings, a stand-in operator with scripted refinement
errors, and toy transformers whose outputs follow known trajectories.  Plain test data and
drivers; nothing here is reference code."""

from __future__ import annotations

import dataclasses
import math
import random
from dataclasses import dataclass

import torch

REFRESH = "refresh"


def _schedule(rng: random.Random) -> dict:
    """Random valid schedule settings (the rules of recap/config.py:95-111)."""
    n = rng.choice([6, 8, 10, 12, 16, 20, 25, 30, 40, 50])
    tail = rng.choice([0, 0, 1, 2, 3]) if n > 4 else 0
    tail = min(tail, n - 1)
    budget = rng.choice([None, None, max(3, tail + 1), n // 2, n // 3 + 2, n - 2, n + 5])
    if budget is not None:
        budget = max(int(budget), 3, tail + 1)
    floor = rng.choice([0, 0, 1, 2, 4, n // 3])
    cap = rng.choice([0, 0, floor, floor + 3, n // 2])
    if cap and cap < floor:
        cap = floor
    return {"num_steps": n, "tau": rng.choice([0.01, 0.03, 0.05, 0.1, 0.2, 0.5]),
            "detail_tau_mult": rng.choice([0.5, 1.0, 2.0]), "budget": budget,
            "prefix_floor": floor, "prefix_cap": cap, "tail_exact": tail}


def make_cases(count: int = 40, seed: int = 2024) -> list[dict]:
    """`count` scenarios: schedule settings, streams, trajectory and refinement errors."""
    rng = random.Random(seed)
    cases = []
    for i in range(count):
        errors = [rng.choice([0.001, 0.01, 0.02, 0.05, 0.08, 0.15, 0.4, 1.5,
                              float("nan"), float("inf")]) for _ in range(16)]
        cases.append({
            "name": f"case{i:02d}",
            "schedule": _schedule(rng),
            "calls_per_step": rng.choice([1, 1, 2]),
            "samples": rng.choice([1, 2]),
            "trajectory": {"slope": rng.choice([0.002, 0.01, 0.05, 0.2]),
                           "curve": rng.choice([0.0, 0.01, 0.1, 0.5]),
                           "wiggle": rng.choice([0.0, 0.005, 0.05]),
                           "freq": rng.choice([0.3, 1.0, 2.5]),
                           "noise": rng.choice([0.0, 0.0, 1e-3, 2e-2]),
                           "dtype": rng.choice(["float32", "float32", "bfloat16"]),
                           "wrap": rng.choice(["tuple", "sample", "tensor"])},
            "errors": errors,
            "seed": rng.randrange(1 << 30),
        })
    return cases


class StubOperator:
    """The Operator surface the session drives (recap/operator.py:175-258, 531-547): banks
    become valid at a REFRESH; a REFRESH of valid banks leaves a scripted refinement error
    whose age is the steps since the previous refresh, read once by drain_validation."""

    def __init__(self, n_streams: int, errors: list[float]):
        self.n_streams = n_streams
        self.errors = list(errors)
        self.reset()

    def reset(self) -> None:
        self.banks_valid = False
        self.last_refresh: int | None = None
        self.pending = None
        self.used = 0
        self.stream = 0
        self.kinds: list[tuple[int, str]] = []

    def begin_step(self, step: int, kind: str) -> None:
        self.kinds.append((int(step), kind))
        if kind == REFRESH:
            if self.banks_valid and self.last_refresh is not None:
                error = self.errors[self.used % len(self.errors)]
                self.used += 1
                self.pending = (int(step) - self.last_refresh, error)
            self.banks_valid = True
            self.last_refresh = int(step)

    def set_stream(self, stream: int) -> None:
        if stream not in range(self.n_streams):
            raise ValueError("bad stream")
        self.stream = stream

    def drain_validation(self):
        out, self.pending = self.pending, None
        return out


@dataclass
class Prediction:
    sample: torch.Tensor


class ToyTransformer:
    """Stream s at step t outputs x0 + slope u x1 + curve u^2 x2 + wiggle sin(freq t) x3
    (+ noise), u = t / num_steps, in the case's dtype and output wrapping."""

    def __init__(self, trajectory: dict, calls_per_step: int, num_steps: int, seed: int):
        self.p = trajectory
        self.cps = calls_per_step
        self.n = num_steps
        g = torch.Generator().manual_seed(seed)
        self.basis = torch.randn(calls_per_step, 4, 2, 8, 16, generator=g, dtype=torch.float64)
        self.seed = seed
        self.calls = 0
        self.dtype = getattr(torch, trajectory["dtype"])

    def forward(self, *args, **kwargs):
        t, s = divmod(self.calls, self.cps)
        t %= self.n                      # a second sample restarts the trajectory
        self.calls += 1
        p, b = self.p, self.basis[s]
        u = t / self.n
        x = b[0] + p["slope"] * u * b[1] + p["curve"] * u * u * b[2] \
            + p["wiggle"] * math.sin(p["freq"] * t) * b[3]
        if p["noise"]:
            g = torch.Generator().manual_seed(self.seed * 7919 + t * 31 + s)
            x = x + p["noise"] * torch.randn(x.shape, generator=g, dtype=torch.float64)
        x = x.to(self.dtype)
        if p["wrap"] == "tuple":
            return (x,)
        if p["wrap"] == "sample":
            return Prediction(x)
        return x


def _tensor(out):
    if isinstance(out, tuple):
        return out[0]
    return getattr(out, "sample", out)


def run_case(case: dict, session_cls, config_module) -> dict:
    """Drive `case` through `session_cls` (the reference's or recap_amd's RecapSession) with
    configs from `config_module`; returns the per-step records (without wall-clock seconds),
    the validation history and a checksum of every output the pipeline received."""
    sched = config_module.ScheduleConfig(**case["schedule"])
    config = dataclasses.replace(
        config_module.RecapConfig(),
        geometry=config_module.GeometryConfig(grid=(4, 32, 32), text_tokens=0),
        schedule=sched, sync_step_timing=False)
    cps = case["calls_per_step"]
    op = StubOperator(cps, case["errors"])
    transformer = ToyTransformer(case["trajectory"], cps, sched.num_steps, case["seed"])
    session = session_cls(config, op, calls_per_step=cps)
    session.install(transformer)
    samples = []
    for _ in range(case["samples"]):
        session.reset()
        sums = []
        for _t in range(sched.num_steps):
            for _s in range(cps):
                out = _tensor(transformer.forward())
                sums.append([float(out.double().sum()), float(out.double().abs().sum()),
                             str(out.dtype).replace("torch.", "")])
        rows = []
        for row in session.actions:
            rows.append({k: v for k, v in row.items() if k != "sec"})
        summary = session.summary()
        samples.append({"actions": rows, "kinds": [list(k) for k in op.kinds],
                        "output_sums": sums,
                        "counts": summary["counts"],
                        "gain": summary["reuse_gain_final"],
                        "validation_history": summary["validation_history"]})
    return {"name": case["name"], "samples": samples}
