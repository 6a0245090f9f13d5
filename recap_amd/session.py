"""The per-sample step loop around a transformer's ``forward`` (recap/session.py).

Every denoising step gets one decision, shared by the ``calls_per_step`` transformer calls a
pipeline makes per step (one per guidance branch):

``EXACT``    dense evaluation;
``REFRESH``  dense evaluation that also renews every layer's attention refinement and
             scores the old one;
``SPARSE``   corrected sparse evaluation (the operator's hot path);
``REUSE``    no evaluation: each stream's output is extrapolated as ``o + g h v`` from its
             latest computed output ``o`` and velocity ``v`` (per step), ``h`` steps ahead,
             with one gain ``g`` fitted by least squares over the computed steps.

The pieces: ``_Planner`` decides a step from the controller (recap_amd/controller.py) and
the sample's progress; ``_StreamCache`` holds one stream's prediction state on the device of
its outputs; ``_GainFit`` is the running least-squares gain; ``RecapSession`` wraps the
forward, runs the operator and keeps the per-step records (keys ``t, a, h, m, g, sec,
validation``, the reference's record format).
"""

from __future__ import annotations

import dataclasses
import math
import time
from dataclasses import dataclass, field
from typing import Any

import torch

from .config import RecapConfig
from .controller import Controller
from .operator import EXACT, REFRESH, SPARSE, Operator

REUSE = "reuse"


# -- transformer outputs ------------------------------------------------------------------


def _prediction(out: Any) -> torch.Tensor:
    """The prediction tensor of a transformer output: a tensor, a tuple's first item or a
    ``.sample`` field."""
    if isinstance(out, tuple):
        return out[0]
    return getattr(out, "sample", out)


def _replace_prediction(template: Any, tensor: torch.Tensor) -> Any:
    """``template`` with its prediction tensor replaced."""
    if isinstance(template, tuple):
        return (tensor, *template[1:])
    if hasattr(template, "sample"):
        return dataclasses.replace(template, sample=tensor)
    return tensor


# -- prediction state ---------------------------------------------------------------------


@dataclass
class _GainFit:
    """g = sum <delta, h v> / sum |h v|^2 over computed steps; a step's terms are staged
    while its streams run and enter the fit when the step completes."""

    value: float = 0.0
    num: float = 0.0
    den: float = 0.0
    staged_num: float = 0.0
    staged_den: float = 0.0

    def stage(self, num: float, den: float) -> None:
        self.staged_num += num
        self.staged_den += den

    def commit(self) -> None:
        if self.staged_den > 0.0:
            self.num += self.staged_num
            self.den += self.staged_den
            self.value = self.num / max(self.den, 1e-30)
        self.staged_num = self.staged_den = 0.0


@dataclass
class _StreamCache:
    """One stream's latest computed output (fp32, on its device), its velocity per step,
    and the output object and dtype an extrapolated step is returned in."""

    output: torch.Tensor
    template: Any
    dtype: torch.dtype
    velocity: torch.Tensor | None = None

    @torch.no_grad()
    def absorb(self, output: torch.Tensor, template: Any, dtype: torch.dtype, h: int,
               gain: float, fit: _GainFit) -> tuple[torch.Tensor, torch.Tensor]:
        """Take the output computed ``h`` steps after the cached one.  Returns the squared
        norms of the extrapolation's miss (``o + g h v`` against the new output, or the step
        itself before a velocity exists) and of the new output, and stages the gain's
        terms."""
        change = output - self.output
        miss = change
        if self.velocity is not None:
            predicted = self.velocity * float(h)
            if gain:
                miss = change - predicted * gain
            norm_sq = float(torch.linalg.vector_norm(predicted) ** 2)
            if norm_sq > 0.0:
                fit.stage(float((change * predicted).sum()), norm_sq)
        self.output, self.velocity = output, change / float(h)
        self.template, self.dtype = template, dtype
        return torch.linalg.vector_norm(miss) ** 2, torch.linalg.vector_norm(output) ** 2

    @torch.no_grad()
    def extrapolate(self, h: int, gain: float) -> Any:
        if not gain or self.velocity is None:
            return self.template
        guess = (self.output + self.velocity * (gain * float(h))).to(self.dtype)
        return _replace_prediction(self.template, guess)


# -- decisions ----------------------------------------------------------------------------


@dataclass
class _Progress:
    """Where the sample stands: the last computed and refreshed steps, whether the
    refinement phase has begun, and the midpoint check after the last refresh (the first
    step half-way to the end, which is validated when it runs sparse)."""

    last_computed: int | None = None
    last_refresh: int | None = None
    refining: bool = False
    midpoint: int | None = None
    midpoint_checked: bool = False


class _Planner:
    """The decision of one step (recap/session.py:109-172).

    First whether the step is covered by extrapolation (``REUSE``) or computed, and whether
    a computed step may run sparse; then the kind: ``EXACT`` before the refinement phase and
    in the exact tail, ``SPARSE`` inside a valid refinement lease, ``REFRESH`` otherwise.
    """

    DENSE, SPARSE_OK = "dense", "sparse-ok"

    def __init__(self, config: RecapConfig, controller: Controller, operator: Operator,
                 progress: _Progress):
        self.schedule = config.schedule
        self.ctl, self.op, self.prog = controller, operator, progress

    def _cover(self, t: int) -> str:
        ctl, prog, schedule = self.ctl, self.prog, self.schedule
        if prog.last_computed is None:
            return self.DENSE                       # nothing to extrapolate from yet
        if ctl.in_exact_tail(t):
            return REUSE if ctl.budget_spent() else self.DENSE
        if ctl.budget_spent_before_tail():
            return REUSE                            # what is left is the tail's
        if not ctl.licensed:
            early = t < schedule.prefix_floor
            due = ctl.half_budget_spent() or (schedule.prefix_cap and t >= schedule.prefix_cap)
            if early or not due:
                return self.DENSE
            ctl.start_reuse()                       # the prefix ran out: reuse from now on
        if t - prog.last_computed < ctl.reuse_span(t):
            return REUSE
        fresh = (self.op.banks_valid and prog.refining and prog.last_refresh is not None
                 and ctl.refinement_usable(t - prog.last_refresh))
        return self.SPARSE_OK if fresh else self.DENSE

    def _final_step_sparse(self, t: int) -> bool:
        """The last step runs sparse when the span from the midpoint check to it is longer
        than what that check validated (or there was no check), the refinement is usable
        and budget remains."""
        prog = self.prog
        if t != self.schedule.num_steps - 1 or not self.op.banks_valid:
            return False
        if prog.last_refresh is not None and prog.midpoint is not None and prog.midpoint_checked:
            validated = prog.midpoint - (prog.last_refresh + 1)
            if t - prog.midpoint <= validated:
                return False
        if prog.last_refresh is not None and not self.ctl.refinement_usable(t - prog.last_refresh):
            return False
        return not self.ctl.budget_spent()

    def decide(self, t: int) -> str:
        cover = self._cover(t)
        if cover != REUSE and self.ctl.in_exact_tail(t):
            return EXACT
        if self._final_step_sparse(t):
            cover = self.SPARSE_OK
        if cover == REUSE:
            return REUSE
        if cover == self.DENSE and self.ctl.licensed:
            self.prog.refining = True               # the first computation once reuse began
        if not self.prog.refining:
            return EXACT
        return SPARSE if cover == self.SPARSE_OK and self.op.banks_valid else REFRESH


# -- the session --------------------------------------------------------------------------


@dataclass
class _StepLog:
    """The running step's decision and measurements across its streams."""

    action: str | None = None
    gain: float = 0.0
    seconds: float = 0.0
    miss_sq: list = field(default_factory=list)
    output_sq: list = field(default_factory=list)


class RecapSession:
    """Per-sample scheduling state wrapped around a transformer (recap/session.py:46-359).
    Call :meth:`reset` before every sample."""

    def __init__(self, config: RecapConfig, operator: Operator, *, calls_per_step: int = 1,
                 model_info: dict[str, Any] | None = None):
        self.config = config
        self.operator = operator
        self.calls_per_step = int(calls_per_step)
        if self.calls_per_step < 1:
            raise ValueError("calls_per_step must be positive")
        if operator.n_streams != self.calls_per_step:
            raise ValueError(f"operator has {operator.n_streams} streams but the pipeline makes "
                             f"{self.calls_per_step} transformer calls per step")
        self.model_info = dict(model_info or {})
        self._transformer = None
        self._wrapped_forward = None
        self.reset()

    def reset(self) -> None:
        """Start a new sample."""
        tr = self._transformer
        if tr is not None and tr.forward is not self._wrapped_forward:
            self._wrap(tr)      # offload hooks restored the unwrapped forward
        self.controller = Controller(self.config.schedule)
        self.operator.reset()
        self.progress = _Progress()
        self.planner = _Planner(self.config, self.controller, self.operator, self.progress)
        self.caches: list[_StreamCache | None] = [None] * self.calls_per_step
        self.fit = _GainFit()
        self.log = _StepLog()
        self.actions: list[dict] = []
        self.step = 0
        self.call_index = 0

    @property
    def gain(self) -> float:
        return self.fit.value

    # -- one step ------------------------------------------------------------------------

    def begin(self, t: int) -> str:
        """Decide step t; a computed step counts against the budget and sets the operator's
        kind (recap/session.py:231-238)."""
        action = self.planner.decide(t)
        if action != REUSE:
            self.controller.count_computed()
            self.operator.begin_step(t, action)
            if action == SPARSE and t == self.progress.midpoint:
                self.progress.midpoint_checked = True
        return action

    def _after_refresh(self, t: int) -> dict[str, Any]:
        """Score the refinement just replaced and set the next midpoint check."""
        out: dict[str, Any] = {}
        scored = self.operator.drain_validation()
        if scored is not None:
            age, error = scored
            passed = self.controller.record_refinement_error(age, error)
            out["validation"] = {"t": t, "age": age, "error": round(error, 6), "passed": passed}
            self.controller.validations.append(out["validation"])
        last = self.config.schedule.num_steps - 1
        self.progress.last_refresh = t
        self.progress.midpoint = int(math.ceil((t + last) / 2.0))
        self.progress.midpoint_checked = False
        return out

    def _close_step(self, t: int) -> dict[str, Any]:
        """The computed step's record: the relative miss ``m`` of the extrapolation over all
        streams and the gain after this step."""
        log = self.log
        row: dict[str, Any] = {"t": t, "a": log.action}
        if log.action == REFRESH:
            row.update(self._after_refresh(t))
        self.fit.commit()
        if log.miss_sq:
            miss = torch.sqrt(torch.stack(log.miss_sq).sum())
            size = torch.sqrt(torch.stack(log.output_sq).sum())
            h = t - int(self.progress.last_computed)
            row.update(h=h, m=round(float(miss / size.clamp_min(1e-30)), 6),
                       g=round(self.fit.value, 4))
            self.controller.record_mismatch(h, row["m"], t)
        self.progress.last_computed = t
        return row

    # -- the wrapped forward -------------------------------------------------------------

    def install(self, transformer) -> None:
        """Wrap ``transformer.forward`` with the step loop (recap/session.py:252-316)."""
        if getattr(transformer, "_recap_installed", False):
            raise RuntimeError("this transformer already has a RECAP step loop")
        self._transformer = transformer
        self._wrap(transformer)
        transformer._recap_installed = True

    def _wrap(self, transformer) -> None:
        inner = transformer.forward

        def forward(*args, **kwargs):
            return self._call(inner, args, kwargs)

        transformer.forward = forward
        self._wrapped_forward = forward

    def _call(self, inner, args, kwargs):
        streams, num_steps = self.calls_per_step, self.config.schedule.num_steps
        t, stream = divmod(self.call_index, streams)
        if t >= num_steps:
            raise RuntimeError(
                f"transformer call {self.call_index} is past the configured horizon of "
                f"{num_steps} steps x {streams} calls; check schedule.num_steps and the "
                "pipeline's guidance settings")
        started = time.perf_counter()
        if stream == 0:
            self.log = _StepLog(action=self.begin(t), gain=self.fit.value)
        log = self.log
        if log.action == REUSE:
            cache = self.caches[stream]
            if cache is None or self.progress.last_computed is None:
                raise RuntimeError("reuse requested before any computed step")
            out = cache.extrapolate(t - self.progress.last_computed, self.fit.value)
        else:
            self.operator.set_stream(stream)
            out = inner(*args, **kwargs)
            if self.config.sync_step_timing and torch.cuda.is_available():
                torch.cuda.synchronize()
            self._observe(t, stream, out)
        log.seconds += time.perf_counter() - started
        self.call_index += 1
        if stream == streams - 1:
            if log.action == REUSE:
                row = {"t": t, "a": REUSE, "h": t - int(self.progress.last_computed),
                       "g": round(self.fit.value, 4), "sec": round(log.seconds, 4)}
            else:
                row = self._close_step(t)
                row["sec"] = round(log.seconds, 3)
            self.actions.append(row)
            self.step = t + 1
        return out

    def _observe(self, t: int, stream: int, out: Any) -> None:
        """Fold a computed output into its stream's cache; measure the extrapolation's miss
        from the second computed step on."""
        prediction = _prediction(out)
        output = prediction.detach().float()
        cache = self.caches[stream]
        if cache is None:
            self.caches[stream] = _StreamCache(output, out, prediction.dtype)
            return
        if self.progress.last_computed is None:
            raise RuntimeError("prediction cache exists without a previous computed step")
        h = t - int(self.progress.last_computed)
        if h <= 0:
            raise RuntimeError(f"non-positive computed-state gap {h} at step {t}")
        miss_sq, output_sq = cache.absorb(output, out, prediction.dtype, h, self.log.gain,
                                          self.fit)
        self.log.miss_sq.append(miss_sq)
        self.log.output_sq.append(output_sq)

    # -- records -------------------------------------------------------------------------

    def summary(self) -> dict[str, Any]:
        counts: dict[str, int] = {}
        for row in self.actions:
            counts[row["a"]] = counts.get(row["a"], 0) + 1
        return {"model": dict(self.model_info), "counts": counts,
                "schedule": [row["a"] for row in self.actions],
                "per_step_sec": [row.get("sec") for row in self.actions],
                "reuse_gain_final": round(self.fit.value, 4), **self.controller.state()}
