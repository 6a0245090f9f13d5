"""Value types of the sparse path (recap/sparse/types.py:14-40, recap/sparse/closure.py:34-39).

An ``AttentionBranch`` is an attention output normalised over a subset of the keys plus the
log-sum-exp of those keys' logits; branches over disjoint key subsets merge exactly into
the softmax over their union.  The fused kernels of this build keep branches in registers
(the merge epilogue of ``recap_sparse_merge_attn``); these containers are what the host
side hands around and what a caller of the kernel-level API receives.

The reference's ``CoarseTailPlan`` (padded omitted-block ids for its coarse-tail kernel)
has no counterpart: the coarse kernel builds its plan from the partition row on chip.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class BlockSummary:
    """Block means and token counts (recap/sparse/types.py:14-19)."""

    mean: torch.Tensor    # [..., blocks, dim] fp32
    counts: torch.Tensor  # [blocks] fp32


@dataclass
class AttentionBranch:
    """Output normalised over this branch's keys and their log-sum-exp
    (recap/sparse/types.py:22-26)."""

    output: torch.Tensor  # [..., rows, dim]
    lse: torch.Tensor     # [..., rows] natural log

    def merge(self, other: "AttentionBranch") -> "AttentionBranch":
        """The branch over the union of two disjoint key subsets (fp32 arithmetic; a
        branch with no keys has lse -inf and drops out)."""
        a, b = self.lse.float(), other.lse.float()
        top = torch.maximum(a, b)
        top = torch.where(torch.isfinite(top), top, torch.zeros_like(top))
        wa, wb = torch.exp(a - top), torch.exp(b - top)
        total = wa + wb
        lse = top + torch.log(total)
        denom = total.clamp_min(1e-30).unsqueeze(-1)
        out = (self.output.float() * wa.unsqueeze(-1) + other.output.float() * wb.unsqueeze(-1)) / denom
        return AttentionBranch(out.to(self.output.dtype), lse)


@dataclass
class ClosureBank:
    """Moment statistics of one call (recap/sparse/closure.py:34-39)."""

    basis: torch.Tensor           # [banks, d, d] orthonormal columns
    key_variance: torch.Tensor    # [banks, blocks, d] diag(U^T C_b U) per block
    value_operator: torch.Tensor  # [banks, dv, dk] pooled value-key covariance
