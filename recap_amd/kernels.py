"""torch-facing wrappers of the HIP kernels: argument checks, output allocation, streams.

Every function runs on ``torch.cuda.current_stream()`` and allocates its outputs with the
caching allocator; the kernels themselves never allocate.  Tensors are passed to the C ABI
as raw device pointers with explicit strides.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import call

BLOCK = 128


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return _lib.RECAP_BF16
    if dtype == torch.float16:
        return _lib.RECAP_F16
    raise ValueError(f"unsupported attention dtype {dtype}; use bfloat16 or float16")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


@dataclass(frozen=True)
class Geometry:
    """Block geometry of one sequence (recap/sparse/attention.py:42-52,
    recap/kernels/block_sparse.py:60-74)."""

    n_tokens: int
    n_video: int
    # Video blocks per closure-statistics workgroup, fixed for a whole layer (the partial
    # sums, and so the rounding, depend on it); None: chosen from the call's banks.
    closure_group: int | None = None

    @property
    def nb(self) -> int:
        return (self.n_video + BLOCK - 1) // BLOCK

    @property
    def tb(self) -> int:
        return (self.n_tokens + BLOCK - 1) // BLOCK

    @property
    def ds(self) -> int:
        shared = self.n_video % BLOCK != 0 and self.n_tokens > self.n_video
        return self.nb - 1 if shared else self.nb

    @property
    def rows(self) -> int:
        return (self.n_video // BLOCK) * BLOCK

    @property
    def partial(self) -> bool:
        return self.n_video % BLOCK != 0

    def counts(self, device) -> torch.Tensor:
        c = torch.full((self.nb,), float(BLOCK), dtype=torch.float32, device=device)
        c[-1] = float(self.n_video - BLOCK * (self.nb - 1))
        return c


def prepare(x: torch.Tensor, name: str) -> torch.Tensor:
    """A ``[B, H, N, D]`` view the kernels can read: unit dim stride, strides and base
    pointer 16-byte aligned; otherwise a contiguous copy."""
    if x.ndim != 4:
        raise ValueError(f"{name} must be [batch, heads, tokens, dim], got {tuple(x.shape)}")
    if not x.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    dtype_code(x.dtype)
    if x.shape[-1] not in (64, 128):
        raise ValueError(f"{name}: head dim {x.shape[-1]} unsupported (64 or 128)")
    ok = (x.stride(-1) == 1 and all(s % 8 == 0 for s in x.stride()[:3])
          and x.data_ptr() % 16 == 0)
    if not ok:
        x = x.contiguous()
        if x.data_ptr() % 16:
            x = x.clone()
    return x


def _same_type(q: torch.Tensor, kv: "PackedKV") -> None:
    """The kernels read Q and the packed K/V tiles in one element type."""
    if q.dtype != kv.dtype:
        raise ValueError(f"Q is {q.dtype} but the packed K/V tiles are {kv.dtype}")


def _qkv_args(x: torch.Tensor):
    b, h, _, d = x.shape
    return [x.data_ptr(), dtype_code(x.dtype), b, h, d, x.stride(0), x.stride(1), x.stride(2)]


# -- stage 1 -------------------------------------------------------------------------------


@dataclass
class PackedKV:
    """Packed K / V^T tiles and fp32 block means of one call."""

    k_tiles: torch.Tensor   # [banks, tb, 128*d] (K tile images)
    vt_tiles: torch.Tensor  # [banks, tb, 128*d] (V^T tile images)
    k_means: torch.Tensor   # [banks, nb, d] fp32
    v_means: torch.Tensor   # [banks, nb, d] fp32
    dtype: torch.dtype
    dim: int


def kv_pack(k: torch.Tensor, v: torch.Tensor, rowmap: torch.Tensor, geo: Geometry) -> PackedKV:
    if k.shape != v.shape or k.dtype != v.dtype:
        raise ValueError("K and V must have the same shape and dtype")
    b, h, n, d = k.shape
    banks = b * h
    kt = torch.empty(banks, geo.tb, BLOCK * d, dtype=k.dtype, device=k.device)
    vt = torch.empty_like(kt)
    km = torch.empty(banks, geo.nb, d, dtype=torch.float32, device=k.device)
    vm = torch.empty_like(km)
    call("recap_kv_pack", k.data_ptr(), v.data_ptr(), dtype_code(k.dtype), b, h, d,
         k.stride(0), k.stride(1), k.stride(2), v.stride(0), v.stride(1), v.stride(2),
         rowmap.data_ptr(), n, geo.n_video, kt.data_ptr(), vt.data_ptr(), km.data_ptr(),
         vm.data_ptr(), _stream())
    return PackedKV(kt, vt, km, vm, k.dtype, d)


def pool_blocks(x: torch.Tensor, rowmap: torch.Tensor, geo: Geometry) -> torch.Tensor:
    b, h, n, d = x.shape
    out = torch.empty(b * h, geo.nb, d, dtype=torch.float32, device=x.device)
    call("recap_pool_blocks", *_qkv_args(x), rowmap.data_ptr(), n, geo.n_video, out.data_ptr(),
         _stream())
    return out


def block_scores(q_means: torch.Tensor, k_means: torch.Tensor, scale: float) -> torch.Tensor:
    q_means, k_means = q_means.contiguous(), k_means.contiguous()
    banks, nb, d = q_means.shape
    out = torch.empty(banks, nb, nb, dtype=torch.float32, device=q_means.device)
    call("recap_block_scores", q_means.data_ptr(), k_means.data_ptr(), banks, nb, d,
         float(scale), out.data_ptr(), _stream())
    return out


def topk_blocks(scores: torch.Tensor, keep: int, force_last: bool) -> torch.Tensor:
    banks, nb, _ = scores.shape
    out = torch.empty(banks, nb, nb, dtype=torch.bool, device=scores.device)
    call("recap_topk_blocks", scores.data_ptr(), banks, nb, int(keep), int(bool(force_last)),
         out.data_ptr(), _stream())
    return out


def kernel_block_mask(partition: torch.Tensor, geo: Geometry) -> torch.Tensor:
    banks = partition.numel() // (geo.nb * geo.nb)
    partition = partition.contiguous()
    out = torch.empty(banks, geo.tb, geo.tb, dtype=torch.bool, device=partition.device)
    call("recap_kernel_block_mask", partition.data_ptr(), banks, geo.n_tokens, geo.n_video,
         out.data_ptr(), _stream())
    return out


def mask_overlap(new: torch.Tensor, old: torch.Tensor) -> tuple[int, int]:
    """(|new & old|, |new|); synchronises the stream to read the counts, as the reference's
    ``float(kept)`` does (recap/operator.py:427)."""
    new, old = new.contiguous(), old.contiguous()
    work = torch.empty(514, dtype=torch.int64, device=new.device)
    call("recap_mask_overlap", new.data_ptr(), old.data_ptr(), new.numel(), work.data_ptr(),
         _stream())
    kept, total = work[:2].tolist()
    return int(kept), int(total)


def pool_select(q: torch.Tensor, k_means: torch.Tensor, rowmap: torch.Tensor, geo: Geometry,
                density: float, scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Stage 1 in one library call: (partition [banks, nb, nb], kernel mask [banks, tb, tb])."""
    b, h, n, d = q.shape
    banks = b * h
    k_means = k_means.contiguous()
    size = int(_lib.load().recap_pool_select_workspace_size(banks, geo.nb, d))
    work = torch.empty(size, dtype=torch.uint8, device=q.device)
    part = torch.empty(banks, geo.nb, geo.nb, dtype=torch.bool, device=q.device)
    kmask = torch.empty(banks, geo.tb, geo.tb, dtype=torch.bool, device=q.device)
    call("recap_pool_select", *_qkv_args(q), rowmap.data_ptr(), n, geo.n_video,
         k_means.data_ptr(), float(scale), float(density), work.data_ptr(), size,
         part.data_ptr(), kmask.data_ptr(), _stream())
    return part, kmask


def select_blocks(q: torch.Tensor, k_means: torch.Tensor, rowmap: torch.Tensor, geo: Geometry,
                  density: float, scale: float) -> torch.Tensor:
    """Partition ``[banks, nb, nb]`` bool (recap/sparse/attention.py:74-94)."""
    q_means = pool_blocks(q, rowmap, geo)
    keep = max(1, round(float(density) * geo.nb))
    keep = min(keep, geo.nb)
    return topk_blocks(block_scores(q_means, k_means, scale), keep, geo.partial)


# -- stage 3 -------------------------------------------------------------------------------


CLOSURE_GROUP = 8


def closure_group(banks: int, nb: int) -> int:
    """Video blocks per closure workgroup: up to CLOSURE_GROUP, fewer when the call has too
    few blocks to give every CU several workgroups (about 1024 in all)."""
    return max(1, min(CLOSURE_GROUP, (banks * nb) // 1024))


def closure_stats(kv: PackedKV, geo: Geometry, flags: int, u_hi_t=None, u_lo_t=None,
                  group: int | None = None):
    """(variance, C_vk, scatter) for the requested statistics; absent ones are None."""
    banks, d = kv.k_means.shape[0], kv.dim
    if group is None:
        group = geo.closure_group or closure_group(banks, geo.nb)
    dev = kv.k_means.device
    groups = int(_lib.load().recap_closure_groups(geo.n_video, group))
    var = cvk_part = scat_part = None
    if flags & _lib.CLOSURE_ROT:
        var = torch.empty(banks, geo.nb, d, dtype=torch.float32, device=dev)
    if flags & _lib.CLOSURE_CVK:
        cvk_part = torch.empty(banks, groups, d, d, dtype=torch.float32, device=dev)
    if flags & _lib.CLOSURE_SCATTER:
        scat_part = torch.empty(banks, groups, d, d, dtype=torch.float32, device=dev)
    call("recap_closure_stats", kv.k_tiles.data_ptr(), kv.vt_tiles.data_ptr(),
         kv.k_means.data_ptr(), dtype_code(kv.dtype), _p(u_hi_t), _p(u_lo_t), banks, d,
         geo.n_tokens, geo.n_video, group, flags, _p(var), _p(cvk_part), _p(scat_part), _stream())
    cvk = scatter = None
    if cvk_part is not None:
        cvk = partial_reduce(cvk_part, float(geo.n_video))
    if scat_part is not None:
        scatter = partial_reduce(scat_part, float(geo.n_video))
    return var, cvk, scatter


def partial_reduce(part: torch.Tensor, divisor: float) -> torch.Tensor:
    banks, groups = part.shape[:2]
    elems = part[0, 0].numel()
    out = torch.empty(banks, *part.shape[2:], dtype=torch.float32, device=part.device)
    call("recap_partial_reduce", part.data_ptr(), banks, groups, elems, float(divisor),
         out.data_ptr(), _stream())
    return out


def symmetric_eigen(a: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(eigenvalues ascending ``[..., n]``, eigenvectors as columns ``[..., n, n]``) of the
    symmetrised fp32 ``0.5 (a + a^T)``, n <= 128: the contract of ``torch.linalg.eigh``
    that closure_basis relies on (recap/sparse/closure.py:75-81)."""
    if a.dim() < 2 or a.shape[-1] != a.shape[-2]:
        raise ValueError(f"symmetric_eigen needs square matrices, got {tuple(a.shape)}")
    n = a.shape[-1]
    flat = a.reshape(-1, n, n).to(torch.float32).contiguous()
    values = torch.empty(flat.shape[0], n, dtype=torch.float32, device=a.device)
    vectors = torch.empty_like(flat)
    call("recap_symmetric_eigen", flat.data_ptr(), flat.shape[0], n, values.data_ptr(),
         vectors.data_ptr(), _stream())
    return values.reshape(a.shape[:-1]), vectors.reshape(a.shape)


@dataclass
class BasisTables:
    u_hi_t: torch.Tensor | None = None
    u_lo_t: torch.Tensor | None = None
    u_t: torch.Tensor | None = None
    cvk_t: torch.Tensor | None = None


def basis_tables(basis: torch.Tensor | None, cvk: torch.Tensor | None, dtype: torch.dtype, *,
                 split: bool = False, query: bool = False, cvk_table: bool = False) -> BasisTables:
    basis = None if basis is None else basis.to(torch.float32).contiguous()
    cvk = None if cvk is None else cvk.to(torch.float32).contiguous()
    src = basis if basis is not None else cvk
    banks, d = src.shape[0], src.shape[-1]
    mk = lambda: torch.empty(banks, d, d, dtype=dtype, device=src.device)  # noqa: E731
    out = BasisTables(u_hi_t=mk() if split else None, u_lo_t=mk() if split else None,
                      u_t=mk() if query else None, cvk_t=mk() if cvk_table else None)
    dummy = basis if basis is not None else cvk
    call("recap_basis_tables", dummy.data_ptr(), _p(cvk), dtype_code(dtype), banks, d,
         _p(out.u_hi_t), _p(out.u_lo_t), _p(out.u_t), _p(out.cvk_t), _stream())
    return out


COARSE_SLOTS = 32  # key blocks per coarse-tail table tile


def coarse_tables(var: torch.Tensor, kv: PackedKV, rank: int):
    """w, kbar, vbar tables [banks, ceil(nb/32)*32, width], one row per key block (see
    recap_coarse_tables; w is [.., 16] in the folded form)."""
    var = var.to(torch.float32).contiguous()
    banks, nb, d = var.shape
    padded = -(-nb // COARSE_SLOTS) * COARSE_SLOTS
    width = int(_lib.load().recap_coarse_w_width(dtype_code(kv.dtype), d, int(rank)))
    if width < 0:
        raise ValueError(f"coarse_tables: invalid dtype/dim/rank ({kv.dtype}, {d}, {rank})")
    mk = lambda c: torch.empty(banks, padded, c, dtype=kv.dtype, device=var.device)  # noqa: E731
    w, kbar, vbar = mk(width), mk(d), mk(d)
    call("recap_coarse_tables", var.data_ptr(), kv.k_means.data_ptr(), kv.v_means.data_ptr(),
         dtype_code(kv.dtype), banks, nb, d, int(rank), w.data_ptr(), kbar.data_ptr(),
         vbar.data_ptr(), _stream())
    return w, kbar, vbar


def coarse_tail(q: torch.Tensor, rowmap: torch.Tensor, partition: torch.Tensor, geo: Geometry,
                tables: dict, scale: float, theta: float, glref: torch.Tensor | None = None):
    """(go [banks, R, d], gl [banks, R], drift partial [banks, R/128] or None).  `tables`
    holds the coarse tables and the closure rank they were built with (key "rank")."""
    for key in ("kbar", "vbar", "w", "u_t", "cvk_t"):
        if tables[key].dtype != q.dtype:
            raise ValueError(f"coarse_tail: table {key} is {tables[key].dtype}, Q is {q.dtype}")
    b, h, n, d = q.shape
    banks = b * h
    partition = partition.contiguous()
    glref = None if glref is None else glref.contiguous()
    go = torch.empty(banks, geo.rows, d, dtype=q.dtype, device=q.device)
    gl = torch.empty(banks, geo.rows, dtype=torch.float32, device=q.device)
    part = None
    if glref is not None:
        part = torch.empty(banks, max(1, geo.rows // BLOCK), dtype=torch.float32, device=q.device)
    call("recap_coarse_tail", *_qkv_args(q), rowmap.data_ptr(), partition.data_ptr(),
         tables["kbar"].data_ptr(), tables["vbar"].data_ptr(), tables["w"].data_ptr(),
         tables["u_t"].data_ptr(), tables["cvk_t"].data_ptr(), n, geo.n_video, float(scale),
         float(theta), int(tables["rank"]), _p(glref), go.data_ptr(), gl.data_ptr(), _p(part),
         _stream())
    return go, gl, part


def drift_center(part: torch.Tensor, geo: Geometry) -> torch.Tensor:
    banks = part.shape[0]
    out = torch.empty(banks, dtype=torch.float32, device=part.device)
    call("recap_drift_center", part.data_ptr(), banks, geo.n_video, out.data_ptr(), _stream())
    return out


# -- stage 2 -------------------------------------------------------------------------------


def block_sparse_attn(q: torch.Tensor, kv: PackedKV, rowmap: torch.Tensor,
                      kernel_mask: torch.Tensor, geo: Geometry, scale: float):
    """Head branch (reordered order): (out [banks, N, d] in the query dtype, lse [banks, N])."""
    _same_type(q, kv)
    b, h, n, d = q.shape
    kernel_mask = kernel_mask.contiguous()
    out = torch.empty(b * h, n, d, dtype=q.dtype, device=q.device)
    lse = torch.empty(b * h, n, dtype=torch.float32, device=q.device)
    call("recap_block_sparse_attn", *_qkv_args(q), kv.k_tiles.data_ptr(), kv.vt_tiles.data_ptr(),
         rowmap.data_ptr(), kernel_mask.data_ptr(), n, float(scale), out.data_ptr(),
         lse.data_ptr(), _stream())
    return out, lse


def dense_attn(q: torch.Tensor, kv: PackedKV, rowmap: torch.Tensor, scale: float,
               out: torch.Tensor | None = None):
    """Dense attention, native order: (out [B, H, N, d], lse [B, H, N])."""
    _same_type(q, kv)
    b, h, n, d = q.shape
    if out is None:
        out = torch.empty(b, h, n, d, dtype=q.dtype, device=q.device)
    lse = torch.empty(b, h, n, dtype=torch.float32, device=q.device)
    call("recap_dense_attn", *_qkv_args(q), kv.k_tiles.data_ptr(), kv.vt_tiles.data_ptr(),
         rowmap.data_ptr(), n, float(scale), out.data_ptr(), out.stride(0), out.stride(1),
         out.stride(2), lse.data_ptr(), _stream())
    return out, lse


def _work_queue(device, balance: bool):
    """Claim counters for a load-balanced attention launch (zeroed by the call), or None."""
    if not balance:
        return None
    return torch.empty(int(_lib.load().recap_attn_queue_words()), dtype=torch.int32,
                       device=device)


def dense_head_attn(q: torch.Tensor, kv: PackedKV, rowmap: torch.Tensor,
                    kernel_mask: torch.Tensor, scale: float, out: torch.Tensor | None = None,
                    balance: bool = True):
    """A refresh's dense attention and head branch in one pass:
    (out [B, H, N, d] native, lse [B, H, N], head_out [banks, N, d] reordered in the query
    dtype, head_lse [banks, N]).  `balance` lets XCDs that finish early take the others' last query
    blocks (same outputs)."""
    _same_type(q, kv)
    b, h, n, d = q.shape
    kernel_mask = kernel_mask.contiguous()
    if out is None:
        out = torch.empty(b, h, n, d, dtype=q.dtype, device=q.device)
    lse = torch.empty(b, h, n, dtype=torch.float32, device=q.device)
    head_out = torch.empty(b * h, n, d, dtype=q.dtype, device=q.device)
    head_lse = torch.empty(b * h, n, dtype=torch.float32, device=q.device)
    call("recap_dense_head_attn", *_qkv_args(q), kv.k_tiles.data_ptr(), kv.vt_tiles.data_ptr(),
         rowmap.data_ptr(), kernel_mask.data_ptr(), n, float(scale), out.data_ptr(),
         out.stride(0), out.stride(1), out.stride(2), lse.data_ptr(), head_out.data_ptr(),
         head_lse.data_ptr(), _p(_work_queue(q.device, balance)), _stream())
    return out, lse, head_out, head_lse


def sparse_merge_attn(q: torch.Tensor, kv: PackedKV, rowmap: torch.Tensor,
                      kernel_mask: torch.Tensor, geo: Geometry, scale: float, go, gl, det, dl,
                      glref, center, alpha_override: float | None = None,
                      out: torch.Tensor | None = None, balance: bool = True) -> torch.Tensor:
    """Corrected sparse output [B, H, N, d] in native order (one fused kernel); `balance` as
    for dense_head_attn."""
    _same_type(q, kv)
    b, h, n, d = q.shape
    kernel_mask = kernel_mask.contiguous()
    if any(t is not None and not t.is_contiguous() for t in (go, gl, det, dl, glref, center)):
        raise ValueError("merge inputs must be contiguous")
    if out is None:
        out = torch.empty(b, h, n, d, dtype=q.dtype, device=q.device)
    alpha = -1.0 if alpha_override is None else float(alpha_override)
    call("recap_sparse_merge_attn", *_qkv_args(q), kv.k_tiles.data_ptr(),
         kv.vt_tiles.data_ptr(), rowmap.data_ptr(), kernel_mask.data_ptr(), n, geo.n_video,
         float(scale), _p(go), _p(gl), _p(det), _p(dl), _p(glref), _p(center), alpha,
         out.data_ptr(), out.stride(0), out.stride(1), out.stride(2),
         _p(_work_queue(q.device, balance)), _stream())
    return out


# -- stage 4 -------------------------------------------------------------------------------


def _check_capture(dense_out, dense_lse, head_out, head_lse, go, gl, det, dl, glref, center):
    """Argument checks shared by both capture entry points: the kernels read the head and
    coarse outputs as 16-bit values of the dense output's type and the refinement as fp16."""
    if not all(t.is_contiguous() for t in (dense_lse, head_out, head_lse, go, gl, det, dl)):
        raise ValueError("capture inputs must be contiguous")
    if head_out.dtype != dense_out.dtype or go.dtype != dense_out.dtype:
        raise ValueError("capture: head and coarse outputs must have the dense output's dtype")
    if det.dtype != torch.float16 or dl.dtype != torch.float32:
        raise ValueError("capture: the refinement is fp16 values and fp32 log-masses")
    if (glref is None) != (center is None):
        raise ValueError("capture: validation needs both glref and center")


def refresh_capture(dense_out: torch.Tensor, dense_lse: torch.Tensor, head_out: torch.Tensor,
                    head_lse: torch.Tensor, go: torch.Tensor, gl: torch.Tensor,
                    rowmap: torch.Tensor, geo: Geometry, det: torch.Tensor, dl: torch.Tensor,
                    glref: torch.Tensor | None = None, center: torch.Tensor | None = None):
    """Write the refinement in place; with (glref, center) return the validation pair."""
    b, h, n, d = dense_out.shape
    _check_capture(dense_out, dense_lse, head_out, head_lse, go, gl, det, dl, glref, center)
    stats = part = None
    if glref is not None:
        npart = int(_lib.load().recap_capture_partials(b * h, d, geo.n_video))
        part = torch.empty(max(1, npart), 2, dtype=torch.float32, device=dense_out.device)
        stats = torch.empty(2, dtype=torch.float32, device=dense_out.device)
    call("recap_refresh_capture", dense_out.data_ptr(), dtype_code(dense_out.dtype), b, h, d,
         dense_out.stride(0), dense_out.stride(1), dense_out.stride(2), dense_lse.data_ptr(),
         head_out.data_ptr(), head_lse.data_ptr(), go.data_ptr(), gl.data_ptr(),
         rowmap.data_ptr(), n, geo.n_video, det.data_ptr(), dl.data_ptr(), _p(glref),
         _p(center), _p(part), _p(stats), _stream())
    return stats


def refresh_capture_noalloc(dense_out: torch.Tensor, dense_lse: torch.Tensor,
                            head_out: torch.Tensor, head_lse: torch.Tensor, go: torch.Tensor,
                            gl: torch.Tensor, rowmap: torch.Tensor, geo: Geometry,
                            det: torch.Tensor, dl: torch.Tensor, stats: torch.Tensor | None,
                            glref: torch.Tensor | None = None,
                            center: torch.Tensor | None = None) -> None:
    """refresh_capture through recap_refresh_capture_noalloc: the library allocates nothing
    (its validation partials live in a static 4 MiB device array); the caller passes the
    validation pair's output ``stats`` ([2] fp32) when validating."""
    b, h, n, d = dense_out.shape
    _check_capture(dense_out, dense_lse, head_out, head_lse, go, gl, det, dl, glref, center)
    if glref is not None and stats is None:
        raise ValueError("capture: a validating call (glref given) needs the stats output")
    call("recap_refresh_capture_noalloc", dense_out.data_ptr(), dtype_code(dense_out.dtype), b,
         h, d, dense_out.stride(0), dense_out.stride(1), dense_out.stride(2),
         dense_lse.data_ptr(), head_out.data_ptr(), head_lse.data_ptr(), go.data_ptr(),
         gl.data_ptr(), rowmap.data_ptr(), n, geo.n_video, det.data_ptr(), dl.data_ptr(),
         _p(glref), _p(center), _p(stats), _stream())


def bank_copy_async(dst: torch.Tensor, src: torch.Tensor, stream=None) -> None:
    """Asynchronous device <-> pinned-host copy of a whole bank tensor on ``stream``."""
    if dst.numel() * dst.element_size() != src.numel() * src.element_size():
        raise ValueError("bank copy size mismatch")
    if not (dst.is_contiguous() and src.is_contiguous()):
        raise ValueError("bank copies need contiguous tensors")
    handle = (stream or torch.cuda.current_stream()).cuda_stream
    call("recap_bank_copy_async", dst.data_ptr(), src.data_ptr(),
         dst.numel() * dst.element_size(), handle)


def hilbert_permutation_native(grid) -> "torch.Tensor":
    frames, height, width = (int(x) for x in grid)
    out = torch.empty(frames * height * width, dtype=torch.int64)
    call("recap_hilbert_permutation", frames, height, width, out.data_ptr())
    return out


def scale_for(dim: int) -> float:
    return 1.0 / math.sqrt(dim)
