"""The per-sample step loop around a transformer's ``forward`` (recap/session.py).

Each denoising step takes one decision, shared by the ``calls_per_step`` transformer calls
a pipeline makes per step (one per guidance branch):

``EXACT``    dense evaluation;
``REFRESH``  dense evaluation that also renews every layer's attention refinement and
             scores the old one;
``SPARSE``   corrected sparse evaluation (the operator's hot path);
``REUSE``    no evaluation: the output is extrapolated from the prediction cache as
             ``o + g h v`` (latest computed output ``o``, its velocity ``v`` per step,
             ``h`` steps ahead), with the gain ``g`` fitted online by least squares over
             every computed step.

The prediction cache and all the arithmetic on it stay on the device of the outputs; the
only host values are the scalar norms the controller needs.
"""

from __future__ import annotations

import dataclasses
import math
import time
from typing import Any

import torch

from .config import RecapConfig
from .controller import Controller
from .operator import EXACT, REFRESH, SPARSE, Operator

REUSE = "reuse"
_COMPUTE = "compute"   # cover decision: evaluate (dense or refresh)
_SPARSE_COVER = "sparse"


def _sample_of(out: Any) -> torch.Tensor:
    """The prediction tensor of a transformer output (tensor, tuple or ``.sample``)."""
    if isinstance(out, tuple):
        return out[0]
    return out.sample if hasattr(out, "sample") else out


def _with_sample(template: Any, tensor: torch.Tensor) -> Any:
    """``template`` with its prediction replaced by ``tensor``."""
    if isinstance(template, tuple):
        return (tensor,) + tuple(template[1:])
    if hasattr(template, "sample"):
        return dataclasses.replace(template, sample=tensor)
    return tensor


class RecapSession:
    """Per-sample scheduling state wrapped around a transformer (recap/session.py:44-359)."""

    def __init__(self, config: RecapConfig, operator: Operator, *, calls_per_step: int = 1,
                 model_info: dict[str, Any] | None = None):
        self.config = config
        self.operator = operator
        self.calls_per_step = int(calls_per_step)
        if self.calls_per_step < 1:
            raise ValueError("calls_per_step must be positive")
        if operator.n_streams != self.calls_per_step:
            raise ValueError(
                f"operator has {operator.n_streams} streams but the pipeline makes "
                f"{self.calls_per_step} transformer calls per step")
        self.model_info = dict(model_info or {})
        self._transformer = None
        self._wrapped_forward = None
        self.reset()

    # -- per-sample state ------------------------------------------------------------------

    def reset(self) -> None:
        """Start a new sample (call before every pipeline call)."""
        transformer = self._transformer
        if transformer is not None and transformer.forward is not self._wrapped_forward:
            # Offload hooks may have restored the unwrapped forward.
            self._wrap(transformer)
        self.controller = Controller(self.config.schedule)
        self.operator.reset()
        self.step = 0
        self.call_index = 0
        self.last_computed: int | None = None
        self.last_refresh: int | None = None
        self.phase_active = False
        self.actions: list[dict] = []
        n = self.calls_per_step
        self.caches: list[dict | None] = [None] * n   # per stream: {"o": ..., "v": ...}
        self.output_objects: list[Any] = [None] * n
        self.output_dtypes: list[torch.dtype | None] = [None] * n
        self.gain = 0.0
        self._gain_num = 0.0
        self._gain_den = 0.0
        self.midpoint_step: int | None = None
        self.midpoint_done = False
        self._begin_step_state(None)

    def _begin_step_state(self, action: str | None) -> None:
        self._step_action = action
        self._step_gain = self.gain
        self._step_seconds = 0.0
        self._step_residual_sq: list[torch.Tensor] = []
        self._step_output_sq: list[torch.Tensor] = []
        self._step_gain_num = 0.0
        self._step_gain_den = 0.0

    # -- decisions -------------------------------------------------------------------------

    def _cover(self, t: int) -> str:
        """Whether step t is computed, reused or (if allowed) sparse."""
        ctl = self.controller
        if self.last_computed is None:
            return _COMPUTE
        if ctl.in_exact_tail(t):
            return REUSE if ctl.budget_exhausted() else _COMPUTE
        if ctl.mid_budget_exhausted():
            return REUSE
        if not ctl.licensed:
            schedule = self.config.schedule
            if t < schedule.prefix_floor:
                return _COMPUTE
            if ctl.prefix_overspent() or (schedule.prefix_cap and t >= schedule.prefix_cap):
                ctl.license()
            else:
                return _COMPUTE
        if t - self.last_computed < ctl.allowed_gap(t):
            return REUSE
        if not self.phase_active or not self.operator.banks_valid:
            return _COMPUTE
        if self.last_refresh is None or not ctl.lease_ok(t - self.last_refresh):
            return _COMPUTE  # the refinement is too old: refresh it
        return _SPARSE_COVER

    def _terminal_unvalidated(self, t: int) -> bool:
        """Is step t farther from the midpoint check than the span that check validated?"""
        if self.last_refresh is None or self.midpoint_step is None or not self.midpoint_done:
            return True
        validated = self.midpoint_step - (self.last_refresh + 1)
        return t - self.midpoint_step > validated

    def _terminal_sparse(self, t: int) -> bool:
        """Compute the final step sparsely when its interval is not validated."""
        schedule = self.config.schedule
        if not (t == schedule.num_steps - 1 and self.operator.banks_valid
                and self._terminal_unvalidated(t)):
            return False
        if self.last_refresh is not None and not self.controller.lease_ok(t - self.last_refresh):
            return False
        return not self.controller.budget_exhausted()

    def _action(self, t: int) -> str:
        cover = self._cover(t)
        if cover != REUSE and self.controller.in_exact_tail(t):
            return EXACT
        if self._terminal_sparse(t):
            cover = _SPARSE_COVER
        if cover == REUSE:
            return REUSE
        if cover == _COMPUTE and self.controller.licensed and not self.phase_active:
            self.phase_active = True  # the first computation once reuse has started
        if not self.phase_active:
            return EXACT
        if cover == _SPARSE_COVER and self.operator.banks_valid:
            return SPARSE
        return REFRESH

    def begin(self, t: int) -> str:
        """Decide step t and prepare the operator for it."""
        action = self._action(t)
        if action != REUSE:
            self.controller.computed += 1
            self.operator.begin_step(t, action)
            if t == self.midpoint_step and action == SPARSE:
                self.midpoint_done = True
        return action

    def complete(self, t: int, action: str, diagnostics: dict[str, Any]) -> dict[str, Any]:
        """Record a computed step and feed its measurements to the controller."""
        row: dict[str, Any] = {"t": t, "a": action}
        if action == REFRESH:
            row.update(self._after_refresh(t))
        row.update(diagnostics)
        if "m" in row and "h" in row:
            self.controller.observe_residual(int(row["h"]), float(row["m"]), t)
        self.last_computed = t
        return row

    def _after_refresh(self, t: int) -> dict[str, Any]:
        out: dict[str, Any] = {}
        measured = self.operator.drain_validation()
        if measured is not None:
            age, error = measured
            passed = self.controller.observe_validation(age, error)
            record = {"t": t, "age": age, "error": round(error, 6), "passed": passed}
            self.controller.validations.append(record)
            out["validation"] = record
        self.last_refresh = t
        last = self.config.schedule.num_steps - 1
        self.midpoint_step = int(math.ceil((t + last) / 2.0))
        self.midpoint_done = False
        return out

    # -- prediction cache ------------------------------------------------------------------

    @torch.no_grad()
    def _observe_stream(self, t: int, stream: int, output: torch.Tensor) -> None:
        """Renew stream's prediction cache with a computed output; accumulate the
        mismatch of what the extrapolation would have given and the gain's normal
        equation (sums of <delta, h v> and |h v|^2)."""
        cache = self.caches[stream]
        if cache is None:
            self.caches[stream] = {"o": output, "v": None}
            return
        if self.last_computed is None:
            raise RuntimeError("prediction cache exists without a previous computed step")
        h = t - int(self.last_computed)
        if h <= 0:
            raise RuntimeError(f"non-positive computed-state gap {h} at step {t}")
        delta = output - cache["o"]
        velocity = cache["v"]
        residual = delta
        if velocity is not None:
            predicted = velocity * float(h)
            if self._step_gain:
                residual = delta - predicted * self._step_gain
            pred_sq = float(torch.linalg.vector_norm(predicted) ** 2)
            if pred_sq > 0.0:
                self._step_gain_num += float((delta * predicted).sum())
                self._step_gain_den += pred_sq
        self._step_residual_sq.append(torch.linalg.vector_norm(residual) ** 2)
        self._step_output_sq.append(torch.linalg.vector_norm(output) ** 2)
        self.caches[stream] = {"o": output, "v": delta / float(h)}

    def _finish_observation(self, t: int) -> dict[str, Any]:
        """The step's relative mismatch over all streams and the updated gain."""
        if not self._step_residual_sq:
            return {}
        if self._step_gain_den > 0.0:
            self._gain_num += self._step_gain_num
            self._gain_den += self._step_gain_den
            self.gain = self._gain_num / max(self._gain_den, 1e-30)
        residual = torch.sqrt(torch.stack(self._step_residual_sq).sum())
        output = torch.sqrt(torch.stack(self._step_output_sq).sum())
        misfit = float(residual / output.clamp_min(1e-30))
        h = t - int(self.last_computed)
        return {"h": h, "m": round(misfit, 6), "g": round(self.gain, 4)}

    def _reuse(self, t: int, stream: int) -> Any:
        cache = self.caches[stream]
        if cache is None or self.last_computed is None:
            raise RuntimeError("reuse requested before any computed step")
        velocity = cache["v"]
        if self.gain and velocity is not None:
            h = t - int(self.last_computed)
            extrapolated = (cache["o"] + velocity * (self.gain * float(h))).to(
                self.output_dtypes[stream])
            return _with_sample(self.output_objects[stream], extrapolated)
        return self.output_objects[stream]

    # -- the wrapped forward ---------------------------------------------------------------

    def install(self, transformer) -> None:
        """Wrap ``transformer.forward`` with the step loop."""
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
        streams = self.calls_per_step
        stream, t = self.call_index % streams, self.call_index // streams
        if t >= self.config.schedule.num_steps:
            raise RuntimeError(
                f"transformer call {self.call_index} is past the configured horizon of "
                f"{self.config.schedule.num_steps} steps x {streams} calls; check "
                "schedule.num_steps and the pipeline's guidance settings")
        started = time.perf_counter()
        if stream == 0:
            self._begin_step_state(self.begin(t))
        action = self._step_action
        last_stream = stream == streams - 1

        if action == REUSE:
            out = self._reuse(t, stream)
            self._step_seconds += time.perf_counter() - started
            self.call_index += 1
            if last_stream:
                self.actions.append({"t": t, "a": REUSE, "h": t - int(self.last_computed),
                                     "g": round(self.gain, 4),
                                     "sec": round(self._step_seconds, 4)})
                self.step = t + 1
            return out

        self.operator.set_stream(stream)
        out = inner(*args, **kwargs)
        if self.config.sync_step_timing and torch.cuda.is_available():
            torch.cuda.synchronize()
        self._step_seconds += time.perf_counter() - started
        sample = _sample_of(out)
        self._observe_stream(t, stream, sample.detach().float())
        self.output_objects[stream] = out
        self.output_dtypes[stream] = sample.dtype
        self.call_index += 1
        if last_stream:
            row = self.complete(t, action, self._finish_observation(t))
            row["sec"] = round(self._step_seconds, 3)
            self.actions.append(row)
            self.step = t + 1
        return out

    # -- records ---------------------------------------------------------------------------

    def summary(self) -> dict[str, Any]:
        counts: dict[str, int] = {}
        for row in self.actions:
            counts[row["a"]] = counts.get(row["a"], 0) + 1
        return {
            "model": dict(self.model_info),
            "counts": counts,
            "schedule": [row["a"] for row in self.actions],
            "per_step_sec": [row.get("sec") for row in self.actions],
            "reuse_gain_final": round(self.gain, 4),
            **self.controller.state(),
        }
