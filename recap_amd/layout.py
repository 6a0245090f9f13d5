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
    """The permutation (reordered position -> native index) as int64, after checking that it
    maps the prod(grid) positions one-to-one onto [0, prod(grid)); ValueError otherwise
    (the contract of recap/sparse/geometry.py:13-24)."""
    n = math.prod(int(x) for x in grid)
    perm = np.asarray(permutation, dtype=np.int64)
    if perm.ndim != 1 or perm.size != n:
        raise ValueError(f"permutation has shape {perm.shape}, expected ({n},)")
    if n and (perm.min() < 0 or perm.max() >= n):
        raise ValueError(f"permutation values leave [0, {n})")
    # Every index in range appears exactly once iff no index is hit twice.
    if n and np.bincount(perm, minlength=n).max() > 1:
        raise ValueError("permutation repeats an index")
    return perm


def hilbert_permutation(grid: Sequence[int]) -> np.ndarray:
    """Video tokens along a 3-D Hilbert curve over ``grid = (T, H, W)``; returns the
    reordered-position -> native-index permutation (recap/sparse/geometry.py:27-67)."""
    perm = kernels.hilbert_permutation_native(grid).numpy()
    return validate_permutation(perm, grid)


@dataclass
class Layout:
    """A native token sequence seen as [Hilbert-ordered video | text] (the contract of
    recap/sparse/layout.py:11-92).  The attribute names are the reference's: the model
    integrations set ``text_tokens`` per prompt and then clear ``_gather_cache``
    (recap/models/hunyuan.py:30-39).

    Everything derives from one forward map, forward[r] = native token of reordered row r
    (video rows first, then text), which is also the kernels' int32 row map; the backward
    map is its inverse.
    """

    permutation: torch.Tensor  # reordered video position -> native video position
    inverse: torch.Tensor      # native video position -> reordered video position
    video_tokens: int
    text_tokens: int
    text_first: bool
    _gather_cache: dict = field(default_factory=dict, repr=False, compare=False)

    @classmethod
    def from_permutation(cls, permutation, *, text_tokens: int, text_first: bool) -> "Layout":
        p = torch.as_tensor(permutation, dtype=torch.long, device="cpu")
        n = p.numel()
        ok = p.ndim == 1 and (n == 0 or (int(p.min()) >= 0 and int(p.max()) < n
                                         and int(torch.bincount(p, minlength=n).max()) == 1))
        if not ok:
            raise ValueError("invalid layout permutation")
        inverse = torch.empty_like(p)
        inverse[p] = torch.arange(n)
        return cls(permutation=p, inverse=inverse, video_tokens=n,
                   text_tokens=int(text_tokens), text_first=bool(text_first))

    @property
    def video_offset(self) -> int:
        """Native position of the first video token."""
        return self.text_tokens if self.text_first else 0

    @property
    def tokens(self) -> int:
        return self.video_tokens + self.text_tokens

    def _cached(self, what: str, device, make):
        key = (what, str(device))
        if key not in self._gather_cache:
            self._gather_cache[key] = make()
        return self._gather_cache[key]

    def _maps(self, device) -> tuple[torch.Tensor, torch.Tensor]:
        """(forward, backward) on ``device``: forward[r] is the native token of reordered
        row r, backward[t] the reordered row of native token t."""
        def make():
            text_start = 0 if self.text_first else self.video_tokens
            forward = torch.cat((self.permutation + self.video_offset,
                                 torch.arange(self.text_tokens) + text_start))
            backward = torch.empty_like(forward)
            backward[forward] = torch.arange(forward.numel())
            return forward.to(device), backward.to(device)
        return self._cached("maps", device, make)

    def rowmap(self, device) -> torch.Tensor:
        """int32 [tokens]: the forward map on ``device``, as the kernels read it."""
        return self._cached("rowmap", device,
                            lambda: self._maps("cpu")[0].to(torch.int32).to(device))

    def video_permutation(self, device) -> torch.Tensor:
        return self._cached("video", device, lambda: self.permutation.to(device))

    def _check(self, x: torch.Tensor) -> None:
        if x.shape[-2] != self.tokens:
            raise ValueError(f"sequence {x.shape[-2]} != video+text {self.tokens}")

    def reorder(self, x: torch.Tensor) -> torch.Tensor:
        """Native model order -> [reordered video | text]."""
        self._check(x)
        return x.index_select(-2, self._maps(x.device)[0])

    def restore(self, x: torch.Tensor) -> torch.Tensor:
        """[reordered video | text] -> native model order."""
        self._check(x)
        return x.index_select(-2, self._maps(x.device)[1])


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
