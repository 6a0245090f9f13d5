"""Helpers shared by the GPU parity tests."""

from __future__ import annotations

import math

import numpy as np
import torch

import oracle as O
from recap_amd.kernels import BLOCK
from recap_amd.synthetic import Workload

# Small shapes that still exercise every layout case the reference configurations have.
SMALL = {
    # the CPU-plumbing configuration's shape, bf16
    "tiny": Workload("tiny", 2, 64, (4, 32, 32), 0, False, 0.25, torch.bfloat16),
    # CogVideoX-like: text first, ragged last video block shared with text
    "text-first-ragged": Workload("text-first-ragged", 2, 64, (3, 15, 25), 226, True, 0.25,
                                  torch.bfloat16),
    # HunyuanVideo-like: d=128, text last, ragged shared block
    "text-last-d128": Workload("text-last-d128", 3, 128, (3, 15, 20), 256, False, 0.2,
                               torch.bfloat16),
    # Wan-like: d=128, video only, ragged last block
    "video-ragged-d128": Workload("video-ragged-d128", 2, 128, (5, 10, 13), 0, False, 0.2,
                                  torch.bfloat16, value_field=True),
}


def banks_view(x: torch.Tensor, fwd: torch.Tensor) -> torch.Tensor:
    """Native [B, H, N, d] -> reordered [B*H, N, d] on the CPU."""
    b, h, n, d = x.shape
    return O.reorder(x.cpu(), fwd).reshape(b * h, n, d)


def metrics(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    g, r = got.double().flatten().cpu(), ref.double().flatten().cpu()
    max_abs = float((g - r).abs().max())
    cos = float(torch.dot(g, r) / (g.norm() * r.norm()).clamp_min(1e-300))
    return max_abs, cos


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (8 significant bits)."""
    mag = x.abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(mag)) - 7)


def bf16_tolerance(got: torch.Tensor, ref: torch.Tensor, max_abs: float = 2e-2) -> torch.Tensor:
    """Per-element bound of a bf16 output against the oracle's fp32 output:
    max(max_abs, 2 ulp_bf16(max(|got|, |ref|))).  The ulp term only matters for values >= 2,
    where three roundings the two sides do not share add up: the output's own (0.5 ulp), the
    reference's bf16 rounding of its head branch (recap/kernels/block_sparse.py stores a bf16
    head, which the oracle follows; this build keeps it in fp32, 0.5 ulp), and the bf16
    probabilities of the head's PV product (as in the reference's external attention kernel;
    the oracle's head is exact): 2^-9 relative per term, up to ~1 ulp when one key dominates a
    row of large values.  Measured worst case: 0.027 at 3.89 (Wan's value field, full
    length).  The ulp is taken at the larger magnitude because the two can straddle a binade
    boundary (reference 3.999 with a head rounded to 4.0, output 4.031 from a head of 4.016),
    where the reference's own ulp is half the output's."""
    mag = torch.maximum(got.abs(), ref.abs())
    return torch.clamp_min(2.0 * bf16_ulp(mag), max_abs)


def assert_close_bf16(got, ref, what, max_abs=2e-2, cos=0.999):
    """bf16 output vs an fp32 reference: |err| <= bf16_tolerance(got, ref) and cosine >=
    cos."""
    g, r = got.double().cpu(), ref.double().cpu()
    m, c = metrics(g, r)
    tol = bf16_tolerance(g, r, max_abs)
    excess = float(((g - r).abs() - tol).max())
    big = float((r.abs() >= 2).double().mean())
    print(f"[{what}] max_abs={m:.3e} cos={c:.6f} worst-vs-tolerance={excess:+.3e} "
          f"(|ref|>=2: {big:.1%})", flush=True)
    assert excess <= 0 and c >= cos, f"{what}: max_abs={m} cos={c} excess={excess}"


def swz(row: int, chunks: int) -> int:
    """XOR pattern of the packed tile images (csrc/common.hpp TileGeom::swz)."""
    return (row & 15) if chunks == 16 else ((row & 7) ^ ((row >> 3) & 1))


def k_tile_to_rows(tile: torch.Tensor, d: int) -> torch.Tensor:
    """Undo the K tile image (chunk c of key row k stored at chunk c ^ swz(k))."""
    nch = d // 8
    img = tile.reshape(BLOCK, nch, 8)
    out = torch.empty_like(img)
    for key in range(BLOCK):
        for c in range(nch):
            out[key, c] = img[key, c ^ swz(key, nch)]
    return out.reshape(BLOCK, d)


def vt_tile_to_rows(tile: torch.Tensor, d: int) -> torch.Tensor:
    """Undo the V^T tile image: half h (positions 64h..64h+63) is [d][64] with 128-byte rows,
    chunk c of row r stored at chunk c ^ swz(r, 8); position p holds key swap23(p).
    Returns V rows [128, d]."""
    halves = tile.reshape(2, d, 8, 8)
    vt = torch.empty(d, BLOCK, dtype=tile.dtype)
    for h in range(2):
        for row in range(d):
            for c in range(8):
                vt[row, 64 * h + 8 * c:64 * h + 8 * c + 8] = halves[h, row, c ^ swz(row, 8)]
    keys = [(p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1) for p in range(BLOCK)]
    out = torch.empty(BLOCK, d, dtype=tile.dtype)
    out[keys] = vt.T
    return out


def video_query_blocks(n_video: int, count: int, seed: int = 0) -> list[int]:
    """A spread-out subset of query blocks (always including the first and last)."""
    rows = n_video // BLOCK
    if rows <= count:
        return list(range(rows))
    rng = np.random.default_rng(seed)
    pick = set(rng.choice(rows, size=count - 2, replace=False).tolist()) | {0, rows - 1}
    return sorted(pick)


def scale_for(d: int) -> float:
    return 1.0 / math.sqrt(d)
