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


def ulp(x: torch.Tensor, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Spacing of ``dtype`` numbers at |x| (bf16: 8 significant bits, fp16: 11)."""
    bits = {torch.bfloat16: 8, torch.float16: 11}.get(dtype, 24)
    tiny = {torch.float16: 2.0 ** -14}.get(dtype, 2.0 ** -126)
    mag = x.abs().clamp_min(tiny)
    return torch.exp2(torch.floor(torch.log2(mag)) - (bits - 1))


def parity_tolerance(ref: torch.Tensor, dtype: torch.dtype = torch.bfloat16,
                     max_abs: float = 2e-2) -> torch.Tensor:
    """Per-element bound against the oracle's output ``ref`` rounded to the output dtype (the
    reference stores its outputs in that dtype): max-abs ``max_abs``, or one ulp of the
    rounded value where one ulp is larger (bf16 at |x| >= 4)."""
    r = ref.to(dtype).double() if dtype in (torch.bfloat16, torch.float16) else ref.double()
    return torch.clamp_min(ulp(r, dtype), max_abs) if dtype != torch.float32 else \
        torch.full_like(r, max_abs)


def assert_parity(got, ref, what, dtype=torch.bfloat16, max_abs=2e-2, cos=0.999, mask=None):
    """Output ``got`` (values of ``dtype``) against the oracle's ``ref``: every element within
    ``parity_tolerance`` of ``ref`` rounded to ``dtype`` and cosine >= ``cos``.  ``mask``
    (broadcastable bool) limits the element check to where it is True.  Prints the worst
    case, and how many elements lie where one ulp exceeds ``max_abs``."""
    g = got.double().cpu()
    r = ref.cpu().to(dtype).double() if dtype != torch.float32 else ref.double().cpu()
    m, c = metrics(g, r)
    tol = parity_tolerance(r, dtype, max_abs)
    err = (g - r).abs()
    excess = err - tol
    if mask is not None:
        excess = excess.masked_fill(~mask.expand_as(excess), -math.inf)
    worst = float(excess.max())
    wide = tol > max_abs
    n_wide = int(wide.sum())
    wide_ulps = float((err[wide] / ulp(r[wide], dtype)).max()) if n_wide else 0.0
    print(f"[{what}] max_abs={m:.3e} cos={c:.7f} worst-vs-bound={worst:+.3e} "
          f"elements with ulp>{max_abs:g}: {n_wide} (max {wide_ulps:.2f} ulp)", flush=True)
    assert worst <= 0 and c >= cos, f"{what}: max_abs={m} cos={c} excess={worst}"


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


def gate_alternates(ref, q, wl, rel: float = 1e-5, dtype=torch.bfloat16, alpha_override=None,
                    layer: int = 0):
    """The oracle's last sparse output with the coarse tail's gate threshold theta^2 moved
    up and down by ``rel`` (relative), for the rows whose gate decision lies within ``rel``
    of the threshold (``O.gate_margin``).  Two fp32 summation orders of qsq.w (the
    reference's own ``tl.dot`` leaves the order open, recap/kernels/coarse_tail.py:139-140)
    may decide such a (row, block) pair either way; moving the threshold across it gives
    the other decision.  Returns ``(borderline [B, H, N, 1] bool, [out_up, out_down])``,
    outputs fp32 in native order.  Needs ``ref.sparse(layer, q, ...)`` to have just run."""
    last, state = ref.last, ref.layers[layer]
    ctx = last["ctx"]
    b, h, n, d = q.shape
    scale = 1.0 / math.sqrt(d)
    theta = ref.theta
    margin = O.gate_margin(ctx["qsq"], ctx["w"], state.partition, scale, theta, ref.n_video,
                           dtype)
    rows = (ref.n_video // BLOCK) * BLOCK
    border_rows = margin < rel                                   # [banks, n_video]
    blocks = sorted({int(r) // BLOCK for r in torch.nonzero(border_rows.any(0)).flatten()})
    ql = ref._banks(q)
    outs = []
    for sign in (1.0, -1.0):
        th = theta * math.sqrt(1.0 + sign * rel)
        go_alt, gl_alt = last["go"].clone(), last["gl"].clone()
        if blocks:
            go2, gl2 = O.coarse_tail(ql, ctx["qsq"], ctx["drift"], ctx["km"], ctx["vm"],
                                     ctx["w"], ctx["counts"], state.partition, scale, th,
                                     ref.n_video, dtype, query_blocks=blocks)
            for i in blocks:
                r0, r1 = i * BLOCK, min((i + 1) * BLOCK, rows)
                if r0 < r1:
                    go_alt[:, r0:r1], gl_alt[:, r0:r1] = go2[:, r0:r1], gl2[:, r0:r1]
        merged = O.sparse_merge(last["oh"], last["lh"], go_alt, gl_alt, state.det, state.dl,
                                rows, state.glref, last["center"], alpha_override)
        outs.append(O.restore(merged, ref.inv).reshape(b, h, n, d))
    full = torch.cat([border_rows, torch.zeros(border_rows.shape[0], n - ref.n_video,
                                               dtype=torch.bool)], dim=1)
    native = O.restore(full.unsqueeze(-1), ref.inv).reshape(b, h, n, 1)
    return native, outs


def rows_within(got, ref, dtype=torch.bfloat16, max_abs=2e-2) -> torch.Tensor:
    """[..., N, 1] bool: every element of the row is within ``parity_tolerance``."""
    g, r = got.double().cpu(), ref.cpu().to(dtype).double()
    ok = (g - r).abs() <= parity_tolerance(r, dtype, max_abs)
    return ok.all(dim=-1, keepdim=True)


def neighbour16(x: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """The adjacent value of ``x``'s 16-bit float type above (``up``) or below each element
    (from +-0: the smallest subnormal of that sign)."""
    bits = x.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    neg = bits >= 0x8000
    mag = bits & 0x7FFF
    zero = mag == 0
    away = up ^ neg  # up from a positive value, down from a negative one: larger magnitude
    mag = torch.where(away | zero, mag + 1, mag - 1)
    sign = torch.where(zero, ~up, neg)
    out = mag | (sign.to(torch.int32) << 15)
    return torch.where(out >= 0x8000, out - 0x10000, out).to(torch.int16).view(x.dtype)


def head_alternate(ref, op, q, k, v, device, dtype=torch.bfloat16, alpha_override=None,
                   need=None, layer: int = 0):
    """The oracle's last sparse output with its head branch rounded the other way at the
    elements where a kernel that rounds P may legitimately do so.

    The reference's head is the bf16 output of an attention kernel that rounds P to bf16
    (block_sparse_attn_func, recap/kernels/block_sparse.py:117-134); the oracle's head is the
    exact softmax rounded once.  With each probability rounded to the type (relative error
    at most u = 2^-8 in bf16, 2^-11 in fp16) and the row sum taken before rounding, such a
    kernel's unrounded output lies within E = u sum_j p_j |v_j| / l of the exact one (plus
    fp32 accumulation, a few 2^-24 relative), so it lands on the other side of the
    head's rounding exactly where the exact value lies within E of the rounding midpoint;
    the merge can carry that one-ulp step into an output next to a binade boundary.  The
    alternate head is the oracle's own: its exact value rounded to the other neighbour at
    the elements where the GPU's head (``K.block_sparse_attn`` over the operator's mask, the
    head the fused merge uses bit for bit) took that neighbour and the exact value lies
    within E (computed by the oracle, as the attention of |v|) of the midpoint; ``need``
    (native bool, optional) limits that search to the elements that need an alternate.
    Checks the head itself (every element within max(2e-2, 1 ulp) of the exact head, LSE
    within 2e-3) and returns ``(flip [B, H, N, d] bool native, out_alt [B, H, N, d] fp32
    native)``."""
    from recap_amd import kernels as K

    last, state = ref.last, ref.layers[layer]
    bank = op.banks[0][layer]
    b, h, n, d = q.shape
    qg, kg, vg = (x.to(device) for x in (q, k, v))
    geo = op._geometry(qg)
    rowmap = op.layout.rowmap(device)
    kv = K.kv_pack(kg, vg, rowmap, geo)
    oh_g, lh_g = K.block_sparse_attn(qg, kv, rowmap, bank.head_kernel_mask, geo,
                                     1.0 / math.sqrt(d))
    oh_g, lh_g = oh_g.cpu().float(), lh_g.cpu()
    oh_o, exact = last["oh"], last["oh_f32"].double()
    assert float((lh_g - last["lh"]).abs().max()) < 2e-3
    hd = (oh_g.double() - oh_o.double()).abs()
    hu = ulp(torch.maximum(oh_g.abs(), oh_o.abs()).double(), dtype)
    assert bool((hd <= torch.clamp_min(hu, 2e-2)).all()), float((hd - hu).max())
    other = neighbour16(oh_o.to(dtype), exact > oh_o.double()).float()
    flip = (exact != oh_o.double()) & (oh_g == other)
    if need is not None:
        flip &= banks_view(need, ref.fwd)
    rows = (ref.n_video // BLOCK) * BLOCK
    blocks = sorted({int(r) // BLOCK for r in torch.nonzero(flip.any(-1).any(0)).flatten()})
    if blocks:
        ql, kl, vl = ref._banks(q), ref._banks(k), ref._banks(v)
        spread, _ = O.block_sparse_attention(ql, kl, vl.abs(), state.kmask, 1.0 / math.sqrt(d),
                                             query_blocks=blocks)
        spread = spread.double()
        mid = (oh_o.double() + other.double()) / 2
        unit = 2.0 ** -{torch.bfloat16: 8, torch.float16: 11}[dtype]
        bound = unit * 1.02 * spread + 2.0 ** -22 * (spread + exact.abs())
        near = (exact - mid).abs() <= bound
        ratio = ((exact - mid).abs() / (unit * spread)).masked_fill(~flip, 0.0)
        print(f"  head elements on the other rounding {int(flip.sum())}, of them within the "
              f"P-rounding bound of the midpoint {int((flip & near).sum())}; largest distance "
              f"to the midpoint {float(ratio.max()):.3f} x u sum p|v|/l", flush=True)
        for i in torch.nonzero(flip & ~near)[:8].tolist():
            print(f"    bank {i[0]} row {i[1]} dim {i[2]}: exact {float(exact[tuple(i)]):.9g} "
                  f"oracle {float(oh_o[tuple(i)]):.9g} gpu {float(oh_g[tuple(i)]):.9g} "
                  f"sum p|v|/l {float(spread[tuple(i)]):.6g} lse gpu {float(lh_g[i[0], i[1]]):.7f} "
                  f"oracle {float(last['lh'][i[0], i[1]]):.7f}", flush=True)
        flip &= near
    head_alt = torch.where(flip, other, oh_o)
    merged = O.sparse_merge(head_alt, last["lh"], last["go"], last["gl"], state.det, state.dl,
                            rows, state.glref, last["center"], alpha_override)
    out_alt = O.restore(merged, ref.inv).reshape(b, h, n, d)
    flip_native = O.restore(flip, ref.inv).reshape(b, h, n, d)
    return flip_native, out_alt


def inject(ref, op, layer_index, wl):
    """Give the oracle the GPU operator's refinement state (basis, partition, D, DL, gl_ref)
    of one layer (stream 0)."""
    bank, layer = op.banks[0][layer_index], op.layers[0][layer_index]
    nb = bank.partition.shape[-1]
    ref.load_state(layer_index, basis=layer.basis.cpu(),
                   partition=bank.partition.reshape(-1, nb, nb).cpu(),
                   det=bank.value.cpu(), dl=bank.log_mass.cpu(), glref=bank.coarse_lse.cpu(),
                   n_tokens=wl.tokens)


def elements_within(got, ref, dtype=torch.bfloat16, max_abs=2e-2) -> torch.Tensor:
    """Elementwise: within ``parity_tolerance`` of ``ref`` rounded to ``dtype``."""
    g, r = got.double().cpu(), ref.cpu().to(dtype).double()
    return (g - r).abs() <= parity_tolerance(r, dtype, max_abs)


def assert_sparse_parity(got, ref, op, q, k, v, wl, device, what, dtype=torch.bfloat16,
                         alpha_override=None, cos=0.999, layer: int = 0):
    """A corrected sparse output (``layer`` of ``op``, stream 0; ``ref.sparse`` on the same
    inputs and state has just run) against the oracle: every element within ``parity_tolerance`` of the
    oracle's output, or of the oracle with one legitimately ambiguous rounding decided the
    other way -- the coarse tail's gate for a (row, block) pair within 1e-5 of theta^2
    (``gate_alternates``) or the head branch's bf16 rounding (``head_alternate``) -- and
    cosine >= ``cos``.  No element is left unchecked; the counts are printed."""
    got = got.double().cpu()
    want = ref.last["out_f32"]
    borderline, gate_alt = gate_alternates(ref, q, wl, dtype=dtype, alpha_override=alpha_override,
                                           layer=layer)
    ok = elements_within(got, want, dtype)
    flip, head_alt = head_alternate(ref, op, q, k, v, device, dtype, alpha_override, need=~ok,
                                    layer=layer)
    by_gate = borderline & (elements_within(got, gate_alt[0], dtype)
                            | elements_within(got, gate_alt[1], dtype))
    by_head = flip & elements_within(got, head_alt, dtype)
    passed = ok | by_gate | by_head
    print(f"  [{what}] elements {ok.numel()}: within the bar {int(ok.sum())}; otherwise with "
          f"the gate decided the other way {int((by_gate & ~ok).sum())} (rows with a pair "
          f"within 1e-5: {int(borderline.sum())}), with the head rounded the other way "
          f"{int((by_head & ~ok & ~by_gate).sum())} (of them needing it, head elements on "
          f"the other rounding within the P-rounding bound of its midpoint: "
          f"{int(flip.sum())}); neither {int((~passed).sum())}", flush=True)
    assert bool(passed.all()), f"{what}: {int((~passed).sum())} elements outside the bar"
    assert_parity(got, want, what, dtype=dtype, mask=ok, cos=cos)


def capture_inputs(d, dtype, text_first, seed, banks=3, blocks=5):
    """Synthetic capture inputs covering the capture's cases: ratios spread over (0, 1),
    ratios above 1 - 1e-3 (zeroed rows), lh >= lf (ratio clamped at 1 - 1e-6), log-mass
    refinements past +-30 (clamped), on 3 banks of a ragged video (5 blocks + 37 tokens)
    with 100 text tokens before or after it (``banks`` and ``blocks`` change the size)."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    n_video, text = blocks * 128 + 37, 100
    n = n_video + text
    rows = (n_video // 128) * 128
    perm = rng.permutation(n_video)
    offset = text if text_first else 0
    text_idx = np.arange(text) if text_first else np.arange(n_video, n)
    rowmap = np.concatenate([offset + perm, text_idx]).astype(np.int32)
    of = (1.5 * torch.randn(1, banks, n, d, generator=g)).to(dtype)
    lf = 2.0 * torch.randn(banks, n, generator=g) + 5.0
    lf_row = lf[:, torch.as_tensor(rowmap, dtype=torch.long)]           # reordered rows
    u = torch.rand(banks, n, generator=g) * 0.98 + 0.01
    kind = torch.randint(0, 10, (banks, n), generator=g)
    u = torch.where(kind == 0, 1.0 - 1e-4 * torch.rand(banks, n, generator=g), u)  # zeroed
    u = torch.where(kind == 1, torch.ones(()), u)                       # ratio 1 -> clamp
    u = torch.where(kind == 2, 1.0 + torch.rand(banks, n, generator=g), u)  # lh > lf
    lh = (lf_row + torch.log(u)).float()
    oh = (of[0][:, torch.as_tensor(rowmap, dtype=torch.long)]
          + 0.3 * torch.randn(banks, n, d, generator=g)).to(dtype)
    go = torch.randn(banks, rows, d, generator=g).to(dtype)
    gl = (lf_row[:, :rows] + torch.log1p(-u[:, :rows].clamp_max(0.999))
          + 0.2 * torch.randn(banks, rows, generator=g)).float()
    gl[:, ::97] += 45.0     # DL below -30
    gl[:, 5::89] -= 45.0    # DL above +30
    old_det = (0.5 * torch.randn(banks, rows, d, generator=g)).to(torch.float16)
    old_dl = 0.3 * torch.randn(banks, rows, generator=g)
    glref = gl + 0.1 * torch.randn(banks, rows, generator=g)
    center = 0.05 * torch.randn(banks, generator=g)
    return dict(of=of, lf=lf.reshape(1, banks, n), oh=oh, lh=lh, go=go, gl=gl, perm=perm,
                offset=offset, rowmap=rowmap, n=n, n_video=n_video, rows=rows,
                old=(old_det, old_dl, glref, center))
