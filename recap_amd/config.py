"""Settings of the corrected sparse-attention operator and of the step loop around it.

The schema is the reference's interface: the section and field names, their defaults, the
config-file format ``{model, preset, operating_point, example}`` and the nine preset
profiles under ``recap_amd/profiles/`` (recap/config.py:20-216, recap/profiles/*.json).
The ``OperatorConfig`` fields parameterise the attention path.

How it is organised here: every constraint is data.  A field's own rule sits in its
``metadata`` (``_rule``), rules between fields in the class's ``RELATIONS`` table, and one
checker (``_check``) applies both; one reader (``_read_section``) turns a JSON object into a
section, rejecting unknown keys and passing each value through its field's reader.
``validate()`` keeps the reference's calling convention (install() calls it; it returns the
config) and raises ``ValueError`` for a bad value, ``TypeError`` for a section that is not an
object.
"""

from __future__ import annotations

import json
import math
from dataclasses import MISSING, asdict, dataclass, field, fields
from pathlib import Path
from typing import Any, Callable

PRESETS = ("normal_slow", "normal_fast", "fast")
MODELS = ("cogvideox1.5", "wan2.1-1.3b", "hunyuan")
PROFILE_DIR = Path(__file__).resolve().parent / "profiles"
CONFIG_KEYS = frozenset({"model", "preset", "operating_point", "example"})
PROFILE_KEYS = frozenset({"model", "geometry", "operator", "schedule", "sync_step_timing"})
BLOCK_SIZE = 128   # the block-sparse kernels tile 128 x 128


# -- rules --------------------------------------------------------------------------------


def _number(x) -> bool:
    return isinstance(x, (int, float)) and not isinstance(x, bool)


def _finite_positive(x) -> bool:
    return _number(x) and math.isfinite(x) and x > 0


def _rule(test: Callable[[Any], bool] | None, requirement: str = "", default=MISSING,
          read: Callable[[Any], Any] | None = None):
    """A dataclass field whose value must pass ``test`` (``requirement`` completes the
    sentence 'field must ...' of the error) and which a config file's value becomes through
    ``read`` (None: taken as it is)."""
    return field(default=default,
                 metadata={"test": test, "requirement": requirement, "read": read})


def _check(section: str, obj) -> None:
    """Apply the field rules and then the class's relations; the first failure raises."""
    for f in fields(obj):
        test = f.metadata.get("test")
        if test is not None and not test(getattr(obj, f.name)):
            raise ValueError(f"{section}.{f.name} must {f.metadata['requirement']}"
                             f" (got {getattr(obj, f.name)!r})")
    for holds, message in getattr(type(obj), "RELATIONS", ()):
        if not holds(obj):
            raise ValueError(f"{section}: {message}")


# -- sections -----------------------------------------------------------------------------


@dataclass(frozen=True)
class OperatingPoint:
    """The operating point of a config file: compute budget ``B`` (transformer evaluations
    per sample) and the prediction and refinement error tolerances (recap/config.py:20-35)."""

    B: int = _rule(lambda x: type(x) is int and x >= 3, "be an integer of at least 3")
    tau_pred: float = _rule(_finite_positive, "be finite and positive")
    tau_detail: float = _rule(_finite_positive, "be finite and positive")

    def validate(self) -> None:
        _check("operating_point", self)


@dataclass(frozen=True)
class GeometryConfig:
    """Token layout: the latent video grid (T, H, W), the text tokens beside it and the
    attention block size (recap/config.py:38-53)."""

    grid: tuple = _rule(lambda g: len(g) == 3 and all(int(x) > 0 for x in g),
                        "be three positive integers (T, H, W)",
                        read=lambda v: tuple(int(x) for x in v))
    text_tokens: int = _rule(lambda x: x >= 0, "be non-negative", default=226, read=int)
    block_size: int = _rule(lambda x: x == BLOCK_SIZE,
                            f"be {BLOCK_SIZE} (the block-sparse kernels' tile)",
                            default=BLOCK_SIZE, read=int)

    def validate(self) -> None:
        _check("geometry", self)


@dataclass(frozen=True)
class OperatorConfig:
    """The corrected sparse-attention operator (recap/config.py:56-80): the share of key
    blocks attended exactly, the coarse tail's variance gate and closure rank, the overlap
    below which a refresh re-selects, and the refinement banks' placement and chunking."""

    head_density: float = _rule(lambda x: 0.0 < x < 1.0, "lie in (0, 1)", default=0.10)
    closure_gate_theta: float = _rule(lambda x: x > 0, "be positive", default=2.0)
    closure_rank: int = _rule(lambda x: x >= 0, "be non-negative", default=4)
    rerank_min_overlap: float = _rule(lambda x: 0.0 <= x <= 1.0, "lie in [0, 1]", default=0.95)
    host_banks: bool = False
    prefetch_banks: bool = True
    bank_chunks: int = _rule(lambda x: x >= 1, "be at least 1", default=1)
    block_size: int = BLOCK_SIZE

    def validate(self) -> None:
        _check("operator", self)


@dataclass(frozen=True)
class ScheduleConfig:
    """The step loop (recap/config.py:83-111): steps per sample, the prediction tolerance
    ``tau`` and the refinement tolerance as its multiple, the compute budget, the prefix
    window that may license reuse early, and the exact steps at the end."""

    num_steps: int = _rule(lambda x: x >= 1, "be positive", default=50)
    tau: float = _rule(lambda x: x > 0.0, "be positive", default=0.10)
    detail_tau_mult: float = _rule(lambda x: x > 0.0, "be positive", default=1.0)
    budget: int | None = _rule(lambda x: x is None or x >= 3,
                               "allow at least 3 computed steps (or be null)", default=None,
                               read=lambda v: None if v is None else int(v))
    prefix_floor: int = _rule(lambda x: x >= 0, "be non-negative", default=0)
    prefix_cap: int = 0
    tail_exact: int = _rule(lambda x: x >= 0, "be non-negative", default=0)

    RELATIONS = (
        (lambda s: not s.prefix_cap or s.prefix_cap >= s.prefix_floor,
         "prefix_cap must not be below prefix_floor"),
        (lambda s: s.budget is None or s.tail_exact < s.budget,
         "tail_exact must leave room in the budget"),
        (lambda s: s.tail_exact < s.num_steps, "tail_exact must be smaller than num_steps"),
    )

    def validate(self) -> None:
        _check("schedule", self)


@dataclass(frozen=True)
class RecapConfig:
    """A whole configuration (recap/config.py:114-138)."""

    model: str = "cogvideox1.5"
    geometry: GeometryConfig = None  # type: ignore[assignment]
    operator: OperatorConfig = field(default_factory=OperatorConfig)
    schedule: ScheduleConfig = field(default_factory=ScheduleConfig)
    sync_step_timing: bool = True

    @property
    def operating_point(self) -> OperatingPoint:
        s = self.schedule
        if s.budget is None:
            raise ValueError("an operating point requires a finite budget")
        return OperatingPoint(s.budget, s.tau, s.tau * s.detail_tau_mult)

    def validate(self) -> "RecapConfig":
        for part in (self.geometry, self.operator, self.schedule):
            part.validate()
        return self

    def to_dict(self) -> dict[str, Any]:
        out = asdict(self)
        out["geometry"]["grid"] = list(self.geometry.grid)
        return out


# -- reading files ------------------------------------------------------------------------

def _read_section(raw: dict[str, Any], name: str, cls: type, **fixed) -> Any:
    """``cls`` from ``raw[name]`` (missing or null: all defaults), each value through its
    field's ``read``; keys that are not fields raise; ``fixed`` overrides (the operator's
    block size follows the geometry's)."""
    value = raw.get(name) or {}
    if not isinstance(value, dict):
        raise TypeError(f"config section {name!r} must be an object")
    known = {f.name: f for f in fields(cls)}
    unknown = sorted(set(value) - set(known))
    if unknown:
        raise ValueError(f"unknown key(s) in config section {name!r}: {unknown}; "
                         f"known keys are {sorted(known)}")
    kwargs = {}
    for key, v in value.items():
        if key not in fixed:
            read = known[key].metadata.get("read")
            kwargs[key] = v if read is None else read(v)
    return cls(**kwargs, **fixed)


def config_from_profile(model: str, raw: dict[str, Any]) -> RecapConfig:
    """A validated config from a profile object (recap/config.py:182-211)."""
    unknown = sorted(set(raw) - PROFILE_KEYS)
    if unknown:
        raise ValueError(f"unknown profile keys: {unknown}")
    if "grid" not in (raw.get("geometry") or {}):
        raise ValueError("geometry.grid is required")
    geometry = _read_section(raw, "geometry", GeometryConfig)
    return RecapConfig(
        model=str(model), geometry=geometry,
        operator=_read_section(raw, "operator", OperatorConfig, block_size=geometry.block_size),
        schedule=_read_section(raw, "schedule", ScheduleConfig),
        sync_step_timing=bool(raw.get("sync_step_timing", True)),
    ).validate()


def config_from_dict(raw: dict[str, Any]) -> RecapConfig:
    """A validated config from a config file's object: the preset's profile with the
    operating point applied (budget = B, tau = tau_pred, detail_tau_mult =
    tau_detail / tau_pred; recap/config.py:158-179)."""
    unknown = sorted(set(raw) - CONFIG_KEYS)
    if unknown:
        raise ValueError(f"unknown config keys: {unknown}; a config gives model, preset, "
                         "operating_point and optionally example")
    model, preset = raw.get("model"), raw.get("preset")
    if model not in MODELS or preset not in PRESETS:
        raise ValueError(f"unsupported model/preset: {model!r}/{preset!r}")
    point = raw.get("operating_point")
    if not isinstance(point, dict) or set(point) != {"B", "tau_pred", "tau_detail"}:
        raise ValueError("operating_point must contain exactly B, tau_pred, tau_detail")
    op = OperatingPoint(**point)
    op.validate()
    profile = json.loads((PROFILE_DIR / f"{model}_{preset}.json").read_text())
    schedule = dict(profile.get("schedule") or {})
    if op.B > schedule.get("num_steps", ScheduleConfig.num_steps):
        raise ValueError("operating_point.B cannot exceed num_steps")
    schedule.update(budget=op.B, tau=op.tau_pred, detail_tau_mult=op.tau_detail / op.tau_pred)
    return config_from_profile(model, {**profile, "schedule": schedule})


def load_config(path: str | Path) -> RecapConfig:
    """Read a config JSON file (recap/config.py:214-216)."""
    return config_from_dict(json.loads(Path(path).read_text()))
