"""Token layout: native model order <-> [Hilbert-ordered video | text].

Mirrors recap/sparse/geometry.py and recap/sparse/layout.py.  The permutation is computed
by the native library (host code); the kernels consume it as an int32 row map
(``rowmap(device)``) and gather through it, so the reorder and restore never materialise
on the attention path.  ``reorder``/``restore`` remain as tensor utilities.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np
import torch

from . import kernels


def validate_permutation(permutation: np.ndarray, grid: Sequence[int]) -> np.ndarray:
    """Check a reordered-position -> native-index permutation (recap/sparse/geometry.py:13-24)."""
    grid = tuple(int(x) for x in grid)
    n = int(np.prod(grid))
    permutation = np.asarray(permutation, dtype=np.int64)
    if permutation.shape != (n,):
        raise ValueError(f"permutation shape {permutation.shape} != ({n},)")
    if permutation.min(initial=0) != 0 or permutation.max(initial=-1) != n - 1:
        raise ValueError("permutation is outside [0, prod(grid))")
    if np.unique(permutation).size != n:
        raise ValueError("permutation is not one-to-one")
    return permutation


def hilbert_permutation(grid: Sequence[int]) -> np.ndarray:
    """Video tokens along a 3-D Hilbert curve over ``grid = (T, H, W)``; returns the
    reordered-position -> native-index permutation (recap/sparse/geometry.py:27-67)."""
    perm = kernels.hilbert_permutation_native(grid).numpy()
    return validate_permutation(perm, grid)


@dataclass
class Layout:
    """Reorder/restore of a native sequence (recap/sparse/layout.py:11-92)."""

    permutation: torch.Tensor  # reordered video position -> native video position
    inverse: torch.Tensor
    video_tokens: int
    text_tokens: int
    text_first: bool
    _gather_cache: dict = field(default_factory=dict, repr=False, compare=False)

    @classmethod
    def from_permutation(cls, permutation, *, text_tokens: int, text_first: bool) -> "Layout":
        p = torch.as_tensor(permutation, dtype=torch.long, device="cpu")
        if p.ndim != 1 or torch.unique(p).numel() != p.numel():
            raise ValueError("invalid layout permutation")
        return cls(permutation=p, inverse=torch.argsort(p), video_tokens=p.numel(),
                   text_tokens=int(text_tokens), text_first=bool(text_first))

    @property
    def video_offset(self) -> int:
        return self.text_tokens if self.text_first else 0

    @property
    def tokens(self) -> int:
        return self.video_tokens + self.text_tokens

    def _gather_indices(self, device) -> tuple[torch.Tensor, torch.Tensor]:
        key = f"gather:{device}"
        cached = self._gather_cache.get(key)
        if cached is not None:
            return cached
        nv, tt = self.video_tokens, self.text_tokens
        text = torch.arange(tt, dtype=torch.long)
        if self.text_first:
            fwd = torch.cat((self.permutation + tt, text))
            inv = torch.cat((text + nv, self.inverse))
        else:
            fwd = torch.cat((self.permutation, text + nv))
            inv = torch.cat((self.inverse, text + nv))
        pair = (fwd.to(device), inv.to(device))
        self._gather_cache[key] = pair
        return pair

    def rowmap(self, device) -> torch.Tensor:
        """int32 [tokens]: native token of each reordered row, on ``device`` (cached)."""
        key = f"rowmap:{device}"
        cached = self._gather_cache.get(key)
        if cached is None:
            fwd, _ = self._gather_indices("cpu")
            cached = fwd.to(torch.int32).to(device)
            self._gather_cache[key] = cached
        return cached

    def video_permutation(self, device) -> torch.Tensor:
        key = f"video:{device}"
        cached = self._gather_cache.get(key)
        if cached is None:
            cached = self.permutation.to(device)
            self._gather_cache[key] = cached
        return cached

    def _check(self, x: torch.Tensor) -> None:
        if x.shape[-2] != self.video_tokens + self.text_tokens:
            raise ValueError(f"sequence {x.shape[-2]} != video+text "
                             f"{self.video_tokens + self.text_tokens}")

    def reorder(self, x: torch.Tensor) -> torch.Tensor:
        """Native model order -> [reordered video | text]."""
        self._check(x)
        return x.index_select(-2, self._gather_indices(x.device)[0])

    def restore(self, x: torch.Tensor) -> torch.Tensor:
        """[reordered video | text] -> native model order."""
        self._check(x)
        return x.index_select(-2, self._gather_indices(x.device)[1])


@dataclass
class SparseGeometry:
    """Model-level block data shared by all layers (recap/sparse/attention.py:33-57)."""

    layout: Layout
    block_size: int
    n_blocks: int
    block_counts: torch.Tensor  # [n_blocks] fp32

    @classmethod
    def build(cls, layout: Layout, block_size: int) -> "SparseGeometry":
        n_blocks = math.ceil(layout.video_tokens / block_size)
        counts = torch.full((n_blocks,), float(block_size), dtype=torch.float32)
        counts[-1] = layout.video_tokens - block_size * (n_blocks - 1)
        return cls(layout=layout, block_size=int(block_size), n_blocks=int(n_blocks),
                   block_counts=counts)

    def to(self, device) -> None:
        if self.block_counts.device != torch.device(device):
            self.block_counts = self.block_counts.to(device)
