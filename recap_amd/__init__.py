"""MI355X-native RECAP corrected sparse attention.

The operator surface of lyraxtg/RECAP (``Operator``, ``HostBankOperator``, the config
loader and the EXACT / REFRESH / SPARSE / REUSE step kinds, the step-loop session and its
controller, ``install``) over hand-written gfx950 HIP kernels behind the C ABI of
``librecap_hip.so`` (include/recap_hip.h).

Usage (recap/__init__.py:11-18)::

    config = load_config("configs/hunyuan.json")
    session = install(pipe, config)
    for prompt in prompts:
        session.reset()
        video = pipe(prompt, num_inference_steps=config.schedule.num_steps)
"""

from __future__ import annotations

from typing import Any, Callable

from .config import (OperatingPoint, OperatorConfig, RecapConfig, config_from_dict,
                     load_config)
from .controller import Controller
from .host_banks import HostBankOperator
from .layout import Layout, SparseGeometry, hilbert_permutation
from .operator import EXACT, REFRESH, SPARSE, DetailBank, Operator, SparseAttention
from .session import REUSE, RecapSession
from .types import AttentionBranch, BlockSummary, ClosureBank

__all__ = [
    "EXACT", "REFRESH", "REUSE", "SPARSE", "AttentionBranch", "BlockSummary", "ClosureBank",
    "Controller", "DetailBank", "HostBankOperator",
    "Layout", "OperatingPoint", "Operator", "OperatorConfig", "RecapConfig", "RecapSession",
    "SparseAttention", "SparseGeometry", "config_from_dict", "hilbert_permutation", "install",
    "load_config", "register_builder",
]

# model name -> build_operator(pipe, config) -> (operator, info), the contract of the
# reference's recap/models/{cogvideox,wan,hunyuan}.py:build_operator.  The diffusers
# attention processors those install are not part of this build (diffusers is absent);
# a model integration registers its builder here.
_BUILDERS: dict[str, Callable[[Any, RecapConfig], tuple[Operator, dict]]] = {}
_REFERENCE_MODELS = ("cogvideox1.5", "hunyuan", "wan2.1-1.3b")


def register_builder(model: str,
                     build_operator: Callable[[Any, RecapConfig], tuple[Operator, dict]]) -> None:
    """Register the integration of ``model``: ``build_operator(pipe, config)`` builds the
    operator, installs the attention processors that call ``Operator.attend`` and returns
    ``(operator, info)`` with ``info["calls_per_step"]``."""
    _BUILDERS[str(model)] = build_operator


def install(pipe, config: RecapConfig, *, model: str | None = None) -> RecapSession:
    """Install RECAP into ``pipe`` and return the session (recap/__init__.py:51-69).  Call
    :meth:`RecapSession.reset` before every sample."""
    model = str(model or config.model)
    builder = _BUILDERS.get(model)
    if builder is None:
        if model in _REFERENCE_MODELS:
            raise RuntimeError(
                f"no integration registered for model {model!r}: this build ships the "
                "operator and the step loop, not the diffusers attention processors; "
                "register one with recap_amd.register_builder")
        raise ValueError(f"no integration for model {model!r}; have "
                         f"{sorted(set(_BUILDERS) | set(_REFERENCE_MODELS))}")
    operator, info = builder(pipe, config.validate())
    session = RecapSession(config, operator, calls_per_step=int(info.get("calls_per_step", 1)),
                           model_info=info)
    session.install(pipe.transformer)
    return session
