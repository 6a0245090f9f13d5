"""CPU oracle: a restatement of RECAP's corrected sparse-attention path (test infrastructure).

This module is the checker for the HIP product path in ``recap_amd``.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it; the product
never routes through it.  Every function cites the reference file:line it follows
(paths relative to the lyraxtg/RECAP tree).

Numerics follow the reference's dtype casts exactly (bf16 tables, bf16 query squares,
fp16 refinement, bf16 outputs) so that the oracle reproduces the reference operator,
not an idealised one.  Two functions additionally fix a reduction order, because the
block masks must be bit-exact between the oracle and the GPU kernels:

* ``pool_blocks``: per block and channel, the 128 tokens are summed in ``rp`` interleaved
  lanes (lane ``l`` adds tokens ``l, l+rp, l+2rp, ...`` in order), then the ``rp`` lane
  partials are combined by a halving tree; ``rp = 2048 / d`` (16 for d=128, 32 for d=64).
* ``block_scores``: each score is a sequential fp32 sum over the channels of separately
  rounded products, then multiplied by ``fp32(scale)``.

Top-k ties are broken by the lower key-block index (the reference's ``torch.topk`` leaves
the tie order unspecified; the tests log the top-k margin to show ties do not occur).

Pinning status (how each function is checked, see tests/test_oracle.py):
  hilbert_permutation   golden vector from the reference + bijection/locality invariants
  gather_indices        closed form + restore(reorder(x)) == x
  pool_blocks           closed form (plain mean) within 1 ulp + exact order contract
  block_scores/topk     brute-force argsort; golden masks from the reference
  block_sparse_attention  textbook dense softmax with -inf outside the mask; LSE
  closure statistics    closed forms (covariance, eigh), rotation invariance, sign flips
  coarse_tail           brute-force per-row softmax; constant-block exactness case
  gate_margin (helper)  brute-force scalar loop over (row, block) pairs
  sparse_merge/capture  refresh-then-sparse reproduces the dense output; alpha=0 case
  refresh_detail stats  closed forms of the old sparse output for an offset refinement, an
                        offset log-mass and a per-row drift weight below one
  OracleOperator rerank the new partition is the fresh head_partition; the recaptured
                        refinement reproduces the dense output on the refresh inputs
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

BLOCK = 128

__all__ = [
    "BLOCK", "hilbert_permutation", "gather_indices", "reorder", "restore",
    "block_geometry", "pool_blocks", "block_scores", "topk_mask", "head_partition",
    "kernel_block_mask", "block_sparse_attention", "dense_attention",
    "within_block_scatter", "closure_basis", "split_hi_lo", "rotated_moments",
    "value_key_covariance", "order_basis", "fold_rank", "rotated_query_square",
    "value_drift", "coarse_tail", "drift_center", "sparse_merge", "refresh_detail",
    "OracleLayer", "OracleOperator", "cast", "topk_margin", "gate_margin",
]


def cast(x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Round ``x`` through ``dtype`` and return fp32 (the reference's ``.to(dtype)``)."""
    return x.to(dtype).to(torch.float32)


def _f32(x: float) -> torch.Tensor:
    return torch.tensor(np.float32(x), dtype=torch.float32)


# -- layout: recap/sparse/geometry.py, recap/sparse/layout.py ----------------------------


def hilbert_permutation(grid) -> np.ndarray:
    """Reordered position -> native video index along a 3-D Hilbert curve.

    Follows recap/sparse/geometry.py:27-67: J. Skilling's "axes to transpose" transform
    (Programming the Hilbert curve, AIP Conf. Proc. 707, 2004) with ``x`` as the leading
    axis, then the transposed bits interleaved most significant first, and a stable sort
    of the native indices ``t*H*W + y*W + x`` by that key.
    """
    frames, height, width = (int(v) for v in grid)
    order_bits = max(1, math.ceil(math.log2(max(frames, height, width))))
    t, y, x = np.meshgrid(np.arange(frames), np.arange(height), np.arange(width),
                          indexing="ij")
    native = (t * height * width + y * width + x).reshape(-1).astype(np.int64)
    axes = [x.reshape(-1).astype(np.int64), y.reshape(-1).astype(np.int64),
            t.reshape(-1).astype(np.int64)]
    top = 1 << (order_bits - 1)
    bit = top
    while bit > 1:
        low = bit - 1
        for i in range(3):
            hit = (axes[i] & bit) != 0
            swap = np.where(hit, 0, (axes[0] ^ axes[i]) & low)
            axes[0] = np.where(hit, axes[0] ^ low, axes[0]) ^ swap
            if i:
                axes[i] = axes[i] ^ swap
        bit >>= 1
    axes[1] ^= axes[0]
    axes[2] ^= axes[1]
    flip = np.zeros_like(axes[0])
    bit = top
    while bit > 1:
        flip = np.where((axes[2] & bit) != 0, flip ^ (bit - 1), flip)
        bit >>= 1
    axes = [a ^ flip for a in axes]
    key = np.zeros_like(axes[0])
    for b in range(order_bits - 1, -1, -1):
        for i in range(3):
            key = (key << 1) | ((axes[i] >> b) & 1)
    return native[np.argsort(key, kind="stable")]


def gather_indices(permutation, text_tokens: int, text_first: bool):
    """(fwd, inv) gather indices of recap/sparse/layout.py:44-61.

    ``fwd[r]`` is the native token of reordered row ``r`` ([Hilbert video | text]);
    ``inv[n]`` is the reordered row of native token ``n``.
    """
    p = torch.as_tensor(np.asarray(permutation), dtype=torch.long)
    nv, tt = p.numel(), int(text_tokens)
    text = torch.arange(tt, dtype=torch.long)
    inverse = torch.argsort(p)
    if text_first:
        return torch.cat((p + tt, text)), torch.cat((text + nv, inverse))
    return torch.cat((p, text + nv)), torch.cat((inverse, text + nv))


def reorder(x: torch.Tensor, fwd: torch.Tensor) -> torch.Tensor:
    """Native -> reordered along the token axis (recap/sparse/layout.py:82-86)."""
    return x.index_select(-2, fwd)


def restore(x: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    """Reordered -> native along the token axis (recap/sparse/layout.py:88-92)."""
    return x.index_select(-2, inv)


def block_geometry(n_video: int, n_tokens: int, block: int = BLOCK) -> dict:
    """Block counts of recap/sparse/attention.py:42-52 and recap/kernels/block_sparse.py:60-74."""
    nb = (n_video + block - 1) // block
    tb = (n_tokens + block - 1) // block
    shared = n_video % block != 0 and n_tokens > n_video
    counts = torch.full((nb,), float(block), dtype=torch.float32)
    counts[-1] = n_video - block * (nb - 1)
    return {"nb": nb, "tb": tb, "ds": nb - 1 if shared else nb,
            "rows": (n_video // block) * block, "counts": counts}


# -- stage 1: pooling and selection --------------------------------------------------------


def pool_blocks(x: torch.Tensor, n_video: int, block: int = BLOCK):
    """fp32 block means over the video tokens (recap/sparse/pooling.py:10-34).

    ``x`` is ``[..., N, d]`` in reordered order.  The reduction order is the fixed
    interleaved-lane + halving-tree order described in the module docstring.
    """
    d = x.shape[-1]
    lanes = 2048 // d
    passes = block // lanes
    nb = (n_video + block - 1) // block
    xv = x[..., :n_video, :].to(torch.float32)
    pad = nb * block - n_video
    if pad:
        xv = torch.nn.functional.pad(xv, (0, 0, 0, pad))
    xb = xv.reshape(*xv.shape[:-2], nb, passes, lanes, d)
    acc = xb[..., 0, :, :].clone()
    for p in range(1, passes):
        acc = acc + xb[..., p, :, :]
    half = lanes // 2
    while half >= 1:
        acc = acc[..., :half, :] + acc[..., half:2 * half, :]
        half //= 2
    sums = acc[..., 0, :]
    counts = torch.full((nb,), float(block), dtype=torch.float32)
    counts[-1] = float(n_video - block * (nb - 1))
    return sums / counts.reshape(nb, 1), counts


def block_scores(qm: torch.Tensor, km: torch.Tensor, scale: float) -> torch.Tensor:
    """fp32 ``scale * qbar . kbar`` with a fixed order (recap/sparse/router.py:18-19)."""
    acc = qm[..., :, None, 0] * km[..., None, :, 0]
    for c in range(1, qm.shape[-1]):
        acc = acc + qm[..., :, None, c] * km[..., None, :, c]
    return acc * _f32(scale)


def _order_keys(scores: torch.Tensor) -> np.ndarray:
    """Monotone uint32 keys of fp32 scores (larger score -> larger key)."""
    bits = scores.contiguous().numpy().view(np.uint32)
    return np.where(bits >> 31, ~bits, bits | np.uint32(0x80000000)).astype(np.uint32)


def topk_mask(scores: torch.Tensor, keep: int) -> torch.Tensor:
    """Top-``keep`` per row (recap/sparse/router.py:20-22), ties to the lower index."""
    keep = max(1, min(int(keep), scores.shape[-1]))
    keys = _order_keys(scores)
    order = np.argsort(~keys, axis=-1, kind="stable")[..., :keep]
    mask = np.zeros(scores.shape, dtype=bool)
    np.put_along_axis(mask, order, True, axis=-1)
    return torch.from_numpy(mask)


def topk_margin(scores: torch.Tensor, keep: int) -> float:
    """Smallest gap between the keep-th and (keep+1)-th score over all rows."""
    keep = max(1, min(int(keep), scores.shape[-1]))
    if keep >= scores.shape[-1]:
        return float("inf")
    top = torch.topk(scores.to(torch.float64), keep + 1, dim=-1).values
    return float((top[..., keep - 1] - top[..., keep]).min())


def head_partition(ql: torch.Tensor, kl: torch.Tensor, scale: float, density: float,
                   n_video: int, block: int = BLOCK) -> torch.Tensor:
    """Selected key blocks per query block (recap/sparse/attention.py:74-94)."""
    qm, _ = pool_blocks(ql, n_video, block)
    km, _ = pool_blocks(kl, n_video, block)
    nb = qm.shape[-2]
    keep = max(1, round(float(density) * nb))
    mask = topk_mask(block_scores(qm, km, scale), keep)
    if n_video % block:
        mask[..., -1, :] = True
        mask[..., :, -1] = True
    return mask


def kernel_block_mask(partition: torch.Tensor, n_tokens: int, n_video: int,
                      block: int = BLOCK) -> torch.Tensor:
    """Video partition on the kernel's block grid, text dense (recap/kernels/block_sparse.py:52-75)."""
    g = block_geometry(n_video, n_tokens, block)
    nb, tb, ds = g["nb"], g["tb"], g["ds"]
    if partition.shape[-2:] != (nb, nb):
        raise ValueError("video mask shape does not match video token count")
    out = torch.zeros((*partition.shape[:-2], tb, tb), dtype=torch.bool)
    out[..., :nb, :nb] = partition
    out[..., ds:, :] = True
    out[..., :, ds:] = True
    return out


# -- stage 2: exact attention over the selected blocks ------------------------------------


def block_sparse_attention(q, k, v, kmask, scale, block=BLOCK, query_blocks=None,
                           acc=torch.float64):
    """Softmax attention over the masked 128x128 blocks, with natural-log LSE.

    Semantics of the external ``block_sparse_attn_func`` as called at
    recap/kernels/block_sparse.py:111-138 (non-causal, ``softmax_scale=None`` i.e.
    1/sqrt(d)): each query row attends to every key in the key blocks its query block
    selects; ragged last blocks hold fewer tokens.  ``q, k, v`` are ``[banks, N, d]``
    (reordered order), ``kmask`` is ``[banks, tb, tb]``.  Returns fp32 ``(out, lse)``;
    rows of query blocks not in ``query_blocks`` are left zero / -inf.  ``acc`` is the
    accumulation type (float64 for checking, float32 for a CPU timing baseline).
    """
    banks, n, d = q.shape
    tb = kmask.shape[-1]
    out = torch.zeros(banks, n, d, dtype=torch.float32)
    lse = torch.full((banks, n), -math.inf, dtype=torch.float32)
    qf, kf, vf = (t.to(torch.float32) for t in (q, k, v))
    blocks = range(tb) if query_blocks is None else query_blocks
    for b in range(banks):
        for i in blocks:
            r0, r1 = i * block, min((i + 1) * block, n)
            cols = torch.nonzero(kmask[b, i]).flatten().tolist()
            idx = torch.cat([torch.arange(j * block, min((j + 1) * block, n)) for j in cols])
            s = (qf[b, r0:r1].to(acc) @ kf[b, idx].to(acc).T) * scale
            m = s.max(dim=-1, keepdim=True).values
            p = torch.exp(s - m)
            l = p.sum(dim=-1, keepdim=True)
            out[b, r0:r1] = ((p @ vf[b, idx].to(acc)) / l).float()
            lse[b, r0:r1] = (m + torch.log(l)).squeeze(-1).float()
    return out, lse


def dense_attention(q, k, v, scale, block=BLOCK, query_blocks=None):
    """Dense attention with LSE (recap/operator.py:254-256), as the all-true mask case."""
    tb = (q.shape[1] + block - 1) // block
    full = torch.ones(q.shape[0], tb, tb, dtype=torch.bool)
    return block_sparse_attention(q, k, v, full, scale, block, query_blocks)


# -- stage 3: closure statistics and the coarse tail ----------------------------------------


def _video_blocks(x: torch.Tensor, n_video: int, block: int = BLOCK):
    """``[banks, nb, block, d]`` fp32 video tokens (zero padded) and the valid mask."""
    nb = (n_video + block - 1) // block
    xv = x[..., :n_video, :].to(torch.float32)
    pad = nb * block - n_video
    if pad:
        xv = torch.nn.functional.pad(xv, (0, 0, 0, pad))
    valid = torch.arange(nb * block) < n_video
    return xv.reshape(*xv.shape[:-2], nb, block, x.shape[-1]), valid.reshape(nb, block)


def within_block_scatter(kl, km, counts, n_video, block=BLOCK):
    """Pooled within-block key covariance (recap/sparse/closure.py:42-72), fp64 accumulate."""
    kb, valid = _video_blocks(kl, n_video, block)
    centred = (kb - km.unsqueeze(-2)) * valid.unsqueeze(-1)
    flat = centred.reshape(centred.shape[0], -1, centred.shape[-1]).double()
    return (flat.transpose(-1, -2) @ flat).float() / counts.sum()


def closure_basis(scatter: torch.Tensor) -> torch.Tensor:
    """Orthonormal eigenbasis of the symmetrised scatter (recap/sparse/closure.py:75-81)."""
    sym = 0.5 * (scatter + scatter.transpose(-1, -2))
    return torch.linalg.eigh(sym.float())[1]


def split_hi_lo(x: torch.Tensor):
    """fp32 value as a sum of two bf16 terms (recap/kernels/closure_stats.py:83-86, 133-135)."""
    hi = x.to(torch.bfloat16).to(torch.float32)
    lo = (x - hi).to(torch.bfloat16).to(torch.float32)
    return hi, lo


def rotated_moments(kl, basis, counts, n_video, block=BLOCK):
    """Per-block mean and clamped variance of ``U^T k`` (recap/kernels/closure_stats.py:96-242).

    ``basis`` is used as the bf16 hi+lo pair the reference kernel multiplies with; keys
    are taken at their stored precision.
    """
    kb, valid = _video_blocks(kl, n_video, block)
    hi, lo = split_hi_lo(basis.to(torch.float32))
    spun = (kb.double() @ hi.double().unsqueeze(-3) + kb.double() @ lo.double().unsqueeze(-3))
    spun = spun.float()
    vm = valid.unsqueeze(-1)
    cnt = counts.reshape(-1, 1)
    mean = (spun * vm).sum(-2) / cnt
    var = (((spun - mean.unsqueeze(-2)) * vm) ** 2).sum(-2) / cnt
    return mean, var.clamp_min(0.0)


def value_key_covariance(kl, vl, km, counts, n_video, block=BLOCK):
    """Pooled value-key covariance ``C_vk`` (recap/kernels/closure_stats.py:27-94, 245-290)."""
    kb, valid = _video_blocks(kl, n_video, block)
    vb, _ = _video_blocks(vl, n_video, block)
    centred = (kb - km.unsqueeze(-2)) * valid.unsqueeze(-1)
    hi, lo = split_hi_lo(centred)
    banks, d = kb.shape[0], kb.shape[-1]
    v2 = vb.reshape(banks, -1, d).double()
    c = v2.transpose(-1, -2) @ hi.reshape(banks, -1, d).double()
    c = c + v2.transpose(-1, -2) @ lo.reshape(banks, -1, d).double()
    return c.float() / counts.sum()


def order_basis(basis, variance, counts):
    """Sort basis columns by pooled within-block variance, descending (recap/sparse/attention.py:136-152)."""
    weights = counts.reshape(1, -1, 1)
    pooled = (variance * weights).sum(1) / weights.sum().clamp_min(1.0)
    order = torch.argsort(pooled, dim=-1, descending=True)
    b = torch.gather(basis, 2, order.unsqueeze(1).expand(-1, basis.shape[1], -1))
    v = torch.gather(variance, 2, order.unsqueeze(1).expand(-1, variance.shape[1], -1))
    return b.contiguous(), v.contiguous()


def fold_rank(variance: torch.Tensor, rank: int) -> torch.Tensor:
    """Leading ``rank`` variances kept, the rest averaged (recap/sparse/closure.py:96-104)."""
    d = variance.shape[-1]
    if rank <= 0 or rank >= d:
        return variance
    residual = variance[..., rank:].sum(-1, keepdim=True) / float(d - rank)
    return torch.cat([variance[..., :rank], residual.expand(*variance.shape[:-1], d - rank)], -1)


def rotated_query_square(q, basis, dtype):
    """``(U^T q)^2`` in the query dtype (recap/sparse/closure.py:84-86)."""
    rot = cast(q.to(torch.float64) @ cast(basis, dtype).to(torch.float64), dtype)
    return cast(rot * rot, dtype)


def value_drift(q, operator, scale, dtype):
    """``s C_vk q`` in the query dtype (recap/sparse/closure.py:89-93)."""
    prod = cast(q.to(torch.float64) @ cast(operator, dtype).transpose(-1, -2).to(torch.float64),
                dtype)
    return cast(prod * _f32(scale), dtype)


def coarse_tail(ql, qsq, drift, km, vm, w, counts, partition, scale, theta, n_video, dtype,
                block=BLOCK, query_blocks=None):
    """Corrected coarse attention over the omitted key blocks.

    Follows recap/kernels/coarse_tail.py:79-186 (kernel math) and :206-312 plus
    recap/sparse/attention.py:204-231 (wrapper casts, ``+ g * drift`` in the query dtype):
    for video row r in query block i and omitted block j (``~partition[i, j]``),
    ``l_j = s q.kbar_j + ln n_j + [s^2 qsq.w_j <= theta^2] (s^2/2) qsq.w_j``.
    Returns fp32 ``(out [banks, Nv, d], lse [banks, Nv])``; empty tails give (0, -inf).
    """
    banks, _, d = ql.shape
    nb = km.shape[-2]
    kb16, vb16, w16 = cast(km, dtype), cast(vm, dtype), cast(w, dtype)
    s32, ssq, half, thsq = (_f32(x) for x in (scale, scale * scale, 0.5 * scale * scale,
                                              theta * theta))
    logn = torch.log(counts.to(torch.float32))
    out = torch.zeros(banks, n_video, d, dtype=torch.float32)
    lse = torch.full((banks, n_video), -math.inf, dtype=torch.float32)
    qf = ql[:, :n_video].to(torch.float32)
    blocks = range(nb) if query_blocks is None else query_blocks
    for b in range(banks):
        for i in blocks:
            r0, r1 = i * block, min((i + 1) * block, n_video)
            omitted = torch.nonzero(~partition[b, i]).flatten()
            if omitted.numel() == 0:
                continue
            dots = (qf[b, r0:r1].double() @ kb16[b, omitted].double().T).float()
            scores = dots * s32 + logn[omitted]
            quad = (qsq[b, r0:r1].double() @ w16[b, omitted].double().T).float()
            gate = quad * ssq <= thsq
            scores = scores + torch.where(gate, quad * half, torch.zeros(()))
            m = scores.max(dim=-1, keepdim=True).values
            p = torch.exp(scores - m)
            l = p.sum(-1)
            g = torch.where(gate, p, torch.zeros(())).sum(-1) / l
            acc = (cast(p, dtype).double() @ vb16[b, omitted].double()).float()
            o = cast(acc / l.unsqueeze(-1), dtype)
            gd = cast(cast(g, dtype).unsqueeze(-1) * drift[b, r0:r1], dtype)
            out[b, r0:r1] = cast(o + gd, dtype)
            lse[b, r0:r1] = m.squeeze(-1) + torch.log(l)
    return out, lse


# -- stage 4: drift weight, merge and refresh capture ---------------------------------------


def gate_margin(qsq, w, partition, scale, theta, n_video, dtype, block=BLOCK):
    """Test helper for the coarse tail's gate ``fl(s^2 qsq.w) <= theta^2``
    (recap/kernels/coarse_tail.py:139-140): per reordered video row, the smallest relative
    distance ``|fl(s^2 quad) - theta^2| / theta^2`` over the row's omitted blocks, with quad
    computed as :func:`coarse_tail` does (fp64 dot of the type-rounded operands, rounded to
    fp32).  Two fp32 summation orders of quad agree to ~1e-7 relative, so only rows with a
    margin of that order can take a different gate decision.  Rows with no omitted block
    get +inf.  Returns ``[banks, n_video]`` fp64."""
    banks = qsq.shape[0]
    nb = partition.shape[-1]
    w16 = cast(w, dtype)
    ssq, thsq = _f32(scale * scale), _f32(theta * theta)
    out = torch.full((banks, n_video), math.inf, dtype=torch.float64)
    for b in range(banks):
        for i in range(nb):
            r0, r1 = i * block, min((i + 1) * block, n_video)
            omitted = torch.nonzero(~partition[b, i]).flatten()
            if omitted.numel() == 0:
                continue
            quad = (qsq[b, r0:r1].double() @ w16[b, omitted].double().T).float()
            rel = ((quad * ssq - thsq).abs() / thsq).double()
            out[b, r0:r1] = rel.min(dim=-1).values
    return out


def drift_center(gl: torch.Tensor, glref: torch.Tensor) -> torch.Tensor:
    """Per-bank mean shift of the coarse log-mass (recap/operator.py:148-150)."""
    return (gl - glref).mean(dim=1)


def _tail_with_refinement(go, gl, det, dl, admit):
    """Drift-weighted tail (recap/kernels/detail_cache.py:267-284)."""
    corrected = gl + dl
    common = torch.maximum(gl, corrected)
    sparse_mass = (1.0 - admit) * torch.exp(gl - common)
    cache_mass = admit * torch.exp(corrected - common)
    den = torch.clamp_min(sparse_mass + cache_mass, 1.0e-30)
    tail_o = (go * sparse_mass.unsqueeze(-1) + (go + det) * cache_mass.unsqueeze(-1)) \
        / den.unsqueeze(-1)
    return tail_o, common + torch.log(den)


def _merge_head(oh, lh, tail_o, tail_l):
    """Head (+) tail in log-mass space (recap/kernels/detail_cache.py:288-292)."""
    common = torch.maximum(lh, tail_l)
    wh = torch.exp(lh - common)
    wt = torch.exp(tail_l - common)
    den = torch.clamp_min(wh + wt, 1.0e-30)
    return (oh * wh.unsqueeze(-1) + tail_o * wt.unsqueeze(-1)) / den.unsqueeze(-1)


def sparse_merge(oh, lh, go, gl, det, dl, rows, glref, center, alpha_override=None):
    """Head merged with coarse tail and drift-weighted refinement.

    recap/kernels/detail_cache.py:188-301, 402-456.  ``oh`` holds the head output at
    its stored precision (bf16 values), ``det`` the fp16 refinement.  Rows ``>= rows``
    keep the head.  ``alpha_override`` replaces the per-row drift weight (test knob).
    Returns fp32 values; the caller rounds to the head dtype.
    """
    ohv, lhv = oh[:, :rows], lh[:, :rows]
    if alpha_override is None:
        admit = torch.exp(-torch.abs(gl - glref - center.unsqueeze(-1)))
    else:
        admit = torch.full_like(gl, float(alpha_override))
    tail_o, tail_l = _tail_with_refinement(go, gl, det, dl, admit)
    out = oh.clone().to(torch.float32)
    out[:, :rows] = _merge_head(ohv, lhv, tail_o, tail_l)
    return out


def refresh_detail(of_native, lf_native, oh, lh, go, gl, permutation, video_offset,
                   old=None):
    """Refinement capture at a refresh (recap/kernels/detail_cache.py:25-186, 304-379).

    ``of_native``/``lf_native`` are the dense output and LSE in native order
    (``[banks, N(, d)]``); ``oh, lh, go, gl`` are in reordered order.  ``old`` is
    ``(det, dl, glref, center)`` of the previous refinement for validation, or None.
    Returns ``(det fp16-valued fp32, dl fp32, stats or None)``.
    """
    rows = go.shape[1]
    native = video_offset + torch.as_tensor(np.asarray(permutation[:rows]), dtype=torch.long)
    lf = lf_native[:, native].to(torch.float32)
    of = of_native[:, native].to(torch.float32)
    lhv, ohv = lh[:, :rows].to(torch.float32), oh[:, :rows].to(torch.float32)
    ratio = torch.exp(torch.clamp_max(lhv - lf, 0.0))
    ratio = torch.clamp_max(ratio, 1.0 - 1.0e-6)
    den = 1.0 - ratio
    stats = None
    if old is not None:
        det0, dl0, glref, center = old
        admit = torch.exp(-torch.abs(gl - glref - center.unsqueeze(-1)))
        tail_o, tail_l = _tail_with_refinement(go, gl, det0, dl0, admit)
        old_sparse = _merge_head(ohv, lhv, tail_o, tail_l)
        stats = torch.stack([((old_sparse - of) ** 2).double().sum(),
                             (of ** 2).double().sum()]).float()
    tail = (of - ratio.unsqueeze(-1) * ohv) / den.unsqueeze(-1)
    cached = torch.clamp(tail - go, -6.0e4, 6.0e4)
    cached = torch.where((ratio > 1.0 - 1.0e-3).unsqueeze(-1), torch.zeros(()), cached)
    det = cast(cached, torch.float16)
    dl = torch.clamp(lf + torch.log(den) - gl, -30.0, 30.0)
    return det, dl, stats


# -- operator-level orchestration: recap/operator.py ---------------------------------------


@dataclass
class OracleLayer:
    """Per-layer state of recap/operator.py:33-59 plus the frozen basis of
    recap/sparse/attention.py:60-70."""

    basis: torch.Tensor | None = None
    partition: torch.Tensor | None = None
    kmask: torch.Tensor | None = None
    det: torch.Tensor | None = None
    dl: torch.Tensor | None = None
    glref: torch.Tensor | None = None
    valid: bool = False
    pending_stats: torch.Tensor | None = None


class OracleOperator:
    """REFRESH and SPARSE calls of recap/operator.py:330-527 on the CPU.

    Inputs are native-order ``[B, H, N, d]``; outputs native-order tensors of the input
    dtype.  ``dtype`` is the compute dtype of the reference's casts (bf16 for the GPU
    shapes, fp32 for the CPU plumbing configuration).
    """

    def __init__(self, grid, text_tokens, text_first, density, theta=2.0, rank=4,
                 rerank_min_overlap=0.95, block=BLOCK, permutation=None):
        self.permutation = (hilbert_permutation(grid) if permutation is None
                            else np.asarray(permutation))
        self.n_video = int(self.permutation.size)
        self.text_tokens = int(text_tokens)
        self.text_first = bool(text_first)
        self.video_offset = self.text_tokens if self.text_first else 0
        self.fwd, self.inv = gather_indices(self.permutation, text_tokens, text_first)
        self.density, self.theta, self.rank = float(density), float(theta), int(rank)
        self.rerank_min_overlap = float(rerank_min_overlap)
        self.block = block
        self.layers: dict[int, OracleLayer] = {}
        self.last: dict = {}

    def layer(self, index: int) -> OracleLayer:
        return self.layers.setdefault(index, OracleLayer())

    def load_state(self, index: int, *, basis, partition, det, dl, glref, n_tokens: int):
        """Adopt a refinement state captured elsewhere (e.g. by the GPU operator), so a
        sparse call can be compared on identical state.  Arrays are CPU tensors in the
        layouts of recap/operator.py:33-59 (partition flattened to [banks, nb, nb])."""
        state = self.layer(index)
        state.basis = basis.float()
        state.partition = partition.bool()
        state.kmask = kernel_block_mask(state.partition, n_tokens, self.n_video, self.block)
        state.det, state.dl, state.glref = det.float(), dl.float(), glref.float()
        state.valid = True

    def _banks(self, x):
        b, h, n, d = x.shape
        return reorder(x, self.fwd).reshape(b * h, n, d)

    def _context(self, state, ql, kl, vl, dtype):
        """recap/sparse/attention.py:156-202."""
        g = block_geometry(self.n_video, ql.shape[1], self.block)
        counts = g["counts"]
        km, _ = pool_blocks(kl, self.n_video, self.block)
        vm, _ = pool_blocks(vl, self.n_video, self.block)
        first = state.basis is None
        basis = state.basis
        if first:
            basis = closure_basis(within_block_scatter(kl, km, counts, self.n_video, self.block))
        _, var = rotated_moments(kl, basis, counts, self.n_video, self.block)
        cvk = value_key_covariance(kl, vl, km, counts, self.n_video, self.block)
        if first:
            basis, var = order_basis(basis, var, counts)
            state.basis = basis
        w = fold_rank(var, self.rank)
        scale = 1.0 / math.sqrt(ql.shape[-1])
        qv = ql[:, :self.n_video].to(torch.float32)
        qsq = rotated_query_square(qv, basis, dtype)
        drift = value_drift(qv, cvk, scale, dtype)
        return {"km": km, "vm": vm, "w": w, "qsq": qsq, "drift": drift, "counts": counts,
                "cvk": cvk, "var": var}

    def _coarse(self, ql, ctx, partition, dtype, rows):
        scale = 1.0 / math.sqrt(ql.shape[-1])
        go, gl = coarse_tail(ql, ctx["qsq"], ctx["drift"], ctx["km"], ctx["vm"], ctx["w"],
                             ctx["counts"], partition, scale, self.theta, self.n_video, dtype,
                             self.block)
        return go[:, :rows], gl[:, :rows]

    def _select(self, ql, kl, banks):
        scale = 1.0 / math.sqrt(ql.shape[-1])
        part = head_partition(ql, kl, scale, self.density, self.n_video, self.block)
        kmask = kernel_block_mask(part, ql.shape[1], self.n_video, self.block)
        return part, kmask

    def refresh(self, index, q, k, v, dtype=torch.bfloat16):
        """Dense call that (re)captures the refinement (recap/operator.py:254-258, 330-473)."""
        state = self.layer(index)
        b, h, n, d = q.shape
        banks = b * h
        scale = 1.0 / math.sqrt(d)
        rows = (self.n_video // self.block) * self.block
        ql, kl, vl = self._banks(q), self._banks(k), self._banks(v)
        full_o32, full_l = dense_attention(ql, kl, vl, scale, self.block)
        full_o = cast(full_o32, dtype)
        of_native = restore(full_o, self.inv)
        lf_native = full_l.index_select(-1, self.inv)
        revalidating = state.valid
        if not revalidating:
            state.partition, state.kmask = self._select(ql, kl, banks)
        ctx = self._context(state, ql, kl, vl, dtype)
        oh, lh = block_sparse_attention(ql, kl, vl, state.kmask, scale, self.block)
        oh = cast(oh, dtype)
        go, gl = self._coarse(ql, ctx, state.partition, dtype, rows)
        old = None
        if revalidating:
            center = drift_center(gl, state.glref)
            old = (state.det, state.dl, state.glref, center)
        det, dl, stats = refresh_detail(of_native, lf_native, oh, lh, go, gl, self.permutation,
                                        self.video_offset, old)
        state.pending_stats = stats
        rerank = None
        if revalidating:
            part, kmask = self._select(ql, kl, banks)
            kept = (part & state.partition).sum()
            total = part.sum().clamp_min(1)
            keep_split = float(kept) / float(total) >= self.rerank_min_overlap
            rerank = not keep_split
            if rerank:
                state.partition, state.kmask = part, kmask
                oh, lh = block_sparse_attention(ql, kl, vl, state.kmask, scale, self.block)
                oh = cast(oh, dtype)
                go, gl = self._coarse(ql, ctx, state.partition, dtype, rows)
                det, dl, _ = refresh_detail(of_native, lf_native, oh, lh, go, gl,
                                            self.permutation, self.video_offset, None)
        state.det, state.dl, state.glref = det, dl, gl.clone()
        state.valid = True
        self.last = {"ctx": ctx, "oh": oh, "lh": lh, "go": go, "gl": gl, "rerank": rerank,
                     "full_o": full_o, "full_l": full_l,
                     "out_f32": restore(full_o32, self.inv).reshape(b, h, n, d)}
        return of_native.reshape(b, h, n, d)

    def sparse(self, index, q, k, v, dtype=torch.bfloat16, alpha_override=None):
        """Corrected sparse call (recap/operator.py:477-527)."""
        state = self.layer(index)
        if not state.valid:
            raise RuntimeError("a sparse call was requested before an exact refresh")
        b, h, n, d = q.shape
        scale = 1.0 / math.sqrt(d)
        rows = (self.n_video // self.block) * self.block
        ql, kl, vl = self._banks(q), self._banks(k), self._banks(v)
        oh32, lh = block_sparse_attention(ql, kl, vl, state.kmask, scale, self.block)
        oh = cast(oh32, dtype)
        ctx = self._context(state, ql, kl, vl, dtype)
        go, gl = self._coarse(ql, ctx, state.partition, dtype, rows)
        center = drift_center(gl, state.glref)
        merged32 = sparse_merge(oh, lh, go, gl, state.det, state.dl, rows, state.glref, center,
                                alpha_override)
        self.last = {"ctx": ctx, "oh": oh, "oh_f32": oh32, "lh": lh, "go": go, "gl": gl,
                     "center": center, "out_f32": restore(merged32, self.inv).reshape(b, h, n, d)}
        return restore(cast(merged32, dtype), self.inv).reshape(b, h, n, d)
