"""Synthetic attention inputs for the four reference workloads.

Q and K are N(0, 1) noise plus a smooth 3-D sinusoidal positional field shared by Q and
K, so that block-mean scores are spatially local, as in a video transformer; V is N(0, 1)
(plus the field where the workload says so); text tokens are N(0, 1).  Every
(tensor, batch, head) slice is drawn from its own seeded generator, so any subset of
heads is reproducible on its own and a CPU slice equals the same slice of a full CPU
tensor.  Noise drawn on a GPU uses the device generator and differs from the CPU draw.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Workload:
    """Shape of one attention call: ``[batch, heads, video + text, dim]``."""

    name: str
    heads: int
    dim: int
    grid: tuple[int, int, int]
    text_tokens: int
    text_first: bool
    density: float
    dtype: torch.dtype
    value_field: bool = False

    @property
    def video_tokens(self) -> int:
        return self.grid[0] * self.grid[1] * self.grid[2]

    @property
    def tokens(self) -> int:
        return self.video_tokens + self.text_tokens

    def dense_flops(self, batch: int = 1) -> float:
        """4 N^2 d H: QK^T and PV of dense attention."""
        return 4.0 * self.tokens ** 2 * self.dim * self.heads * batch


WORKLOADS = {
    "cpu-plumbing": Workload("cpu-plumbing", 2, 64, (4, 32, 32), 0, False, 0.25,
                             torch.float32),
    "wan2.1-480p": Workload("wan2.1-480p", 12, 128, (21, 30, 52), 0, False, 0.2,
                            torch.bfloat16, value_field=True),
    "cogvideox1.5": Workload("cogvideox1.5", 48, 64, (11, 48, 85), 226, True, 0.25,
                             torch.bfloat16),
    "hunyuan-720p": Workload("hunyuan-720p", 24, 128, (33, 45, 80), 256, False, 0.2,
                             torch.bfloat16),
}

_TENSOR_IDS = {"q": 1, "k": 2, "v": 3, "field": 4, "drift": 5}


def _generator(device, seed: int, tensor: str, batch: int, head: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed((int(seed) * 1_000_003 + _TENSOR_IDS[tensor] * 10_007
                   + batch * 4_099 + head) % (2 ** 62))
    return g


def positional_field(workload: Workload, head: int, *, seed: int = 0, device="cpu",
                     amplitude: float = 2.0) -> torch.Tensor:
    """``[Nv, dim]`` fp32 field on native video order ``t*H*W + y*W + x``.

    Channel c: ``A sin(2 pi (t/lt_c + y/ly_c + x/lx_c) + phi_c)`` with wavelengths drawn
    from U[8, 64] tokens per axis and phases from U[0, 2 pi).
    """
    g = _generator("cpu", seed, "field", 0, head)
    lam = 8.0 + 56.0 * torch.rand(3, workload.dim, generator=g, dtype=torch.float64)
    phase = 2.0 * math.pi * torch.rand(workload.dim, generator=g, dtype=torch.float64)
    frames, height, width = workload.grid
    t = torch.arange(frames, dtype=torch.float64, device=device)
    y = torch.arange(height, dtype=torch.float64, device=device)
    x = torch.arange(width, dtype=torch.float64, device=device)
    lam, phase = lam.to(device), phase.to(device)
    arg = (t.view(-1, 1, 1, 1) / lam[0] + y.view(1, -1, 1, 1) / lam[1]
           + x.view(1, 1, -1, 1) / lam[2])
    field = amplitude * torch.sin(2.0 * math.pi * arg + phase)
    return field.reshape(-1, workload.dim).to(torch.float32)


def make_qkv(workload: Workload, *, batch: int = 1, heads=None, seed: int = 0,
             dtype: torch.dtype | None = None, device="cpu"):
    """Native-order ``q, k, v`` of shape ``[batch, len(heads), N, dim]``."""
    heads = list(range(workload.heads)) if heads is None else list(heads)
    dtype = workload.dtype if dtype is None else dtype
    n, nv, d = workload.tokens, workload.video_tokens, workload.dim
    v0 = workload.text_tokens if workload.text_first else 0
    out = {name: torch.empty(batch, len(heads), n, d, dtype=dtype, device=device)
           for name in ("q", "k", "v")}
    for hi, h in enumerate(heads):
        field = positional_field(workload, h, seed=seed, device=device)
        for b in range(batch):
            for name in ("q", "k", "v"):
                g = _generator(device, seed, name, b, h)
                x = torch.randn(n, d, generator=g, dtype=torch.float32, device=device)
                if name != "v" or workload.value_field:
                    x[v0:v0 + nv] += field
                out[name][b, hi] = x.to(dtype)
    return out["q"], out["k"], out["v"]


def perturb(x: torch.Tensor, eps: float, *, seed: int, step: int) -> torch.Tensor:
    """``x + eps * xi`` with fresh N(0, 1) noise per step (per-step input drift)."""
    out = torch.empty_like(x)
    for b in range(x.shape[0]):
        for h in range(x.shape[1]):
            g = _generator(x.device, seed * 131 + step, "drift", b, h)
            xi = torch.randn(x.shape[2], x.shape[3], generator=g, dtype=torch.float32,
                             device=x.device)
            out[b, h] = (x[b, h].to(torch.float32) + eps * xi).to(x.dtype)
    return out
