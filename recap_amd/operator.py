"""Attention for the EXACT, REFRESH and SPARSE steps on MI355X (recap/operator.py).

``EXACT``    dense attention (torch SDPA, as the reference).
``REFRESH``  dense attention with LSE on the HIP kernel; stores the refinement (exact tail
             minus coarse tail) and measures the error of the previous one.
``SPARSE``   the corrected sparse call: selected blocks exactly, the coarse tail over the
             omitted blocks, and the cached refinement weighted by the drift weight,
             merged in log-mass space -- four HIP stages:

    kv_pack          K/V gathered through the Hilbert row map into packed tiles + block means
    closure_stats    rotated block variances and C_vk (the frozen basis from the first call)
    coarse_tail      corrected coarse attention over the omitted blocks + drift partials
    sparse_merge_attn  block-sparse flash attention with the merge fused in its epilogue,
                     stored straight to native order

The public surface (``build``, ``reset``, ``begin_step``, ``set_stream``, ``attend``,
``banks_valid``, ``n_streams``, ``drain_validation``, ``peak_bank_bytes``, ``layout``) is
the reference's, so the diffusers processors call it unchanged.
"""

from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from . import _lib
from . import kernels as K
from .config import OperatorConfig
from .layout import Layout, SparseGeometry

EXACT = "exact"
REFRESH = "refresh"
SPARSE = "sparse"
_KINDS = (EXACT, REFRESH, SPARSE)


class SparseAttention:
    """Per-layer state: the covariance basis frozen at the first call of a sample
    (recap/sparse/attention.py:60-231), with its query-type tables cached."""

    def __init__(self, geometry: SparseGeometry, config: OperatorConfig):
        self.geometry = geometry
        self.config = config
        self.reset()

    def reset(self) -> None:
        self._basis: torch.Tensor | None = None
        self._tables: K.BasisTables | None = None

    @property
    def basis(self) -> torch.Tensor | None:
        return self._basis

    def head_partition(self, q: torch.Tensor, kv: K.PackedKV, rowmap: torch.Tensor,
                       geo: K.Geometry, scale: float) -> torch.Tensor:
        """Selected key blocks ``[banks, nb, nb]`` (recap/sparse/attention.py:74-94)."""
        return K.select_blocks(q, kv.k_means, rowmap, geo, self.config.head_density, scale)

    def coarse_tail_context(self, kv: K.PackedKV, geo: K.Geometry) -> dict:
        """Partition-independent statistics (recap/sparse/attention.py:98-202)."""
        dtype = kv.dtype
        if self._basis is None:
            _, cvk, scatter = K.closure_stats(kv, geo, _lib.CLOSURE_CVK | _lib.CLOSURE_SCATTER)
            basis = K.symmetric_eigen(scatter)[1]   # symmetrises 0.5 (S + S^T) itself
            split = K.basis_tables(basis, None, dtype, split=True)
            var, _, _ = K.closure_stats(kv, geo, _lib.CLOSURE_ROT, split.u_hi_t, split.u_lo_t)
            # Order the basis by pooled within-block variance (recap/sparse/attention.py:137-152).
            weights = geo.counts(var.device).reshape(1, -1, 1)
            pooled = (var * weights).sum(1) / weights.sum().clamp_min(1.0)
            order = torch.argsort(pooled, dim=-1, descending=True)
            idx = order.unsqueeze(1)
            basis = torch.gather(basis, 2, idx.expand(-1, basis.shape[1], -1)).contiguous()
            var = torch.gather(var, 2, idx.expand(-1, var.shape[1], -1)).contiguous()
            self._basis = basis
            self._tables = K.basis_tables(basis, None, dtype, split=True, query=True)
        else:
            var, cvk, _ = K.closure_stats(kv, geo, _lib.CLOSURE_ROT | _lib.CLOSURE_CVK,
                                          self._tables.u_hi_t, self._tables.u_lo_t)
        cvk_t = K.basis_tables(None, cvk, dtype, cvk_table=True).cvk_t
        rank = int(self.config.closure_rank)
        w, kbar, vbar = K.coarse_tables(var, kv, rank)
        return {"w": w, "kbar": kbar, "vbar": vbar, "u_t": self._tables.u_t, "cvk_t": cvk_t,
                "rank": rank, "variance": var, "cvk": cvk}

    def coarse_tail_apply(self, q, rowmap, context, partition, geo, scale, glref=None):
        """Coarse tail over the omitted blocks (recap/sparse/attention.py:204-231)."""
        return K.coarse_tail(q, rowmap, partition, geo, context, scale,
                             self.config.closure_gate_theta, glref)


@dataclass
class DetailBank:
    """One layer's cached refinement and its partition.  The field names and layouts are
    the reference's (recap/operator.py:33-59): host paging and the model integrations
    read them."""

    head_kernel_mask: torch.Tensor | None = None  # [banks, tb, tb] bool
    partition: torch.Tensor | None = None         # [B, H, nb, nb] bool
    value: torch.Tensor | None = None             # [banks, rows, dim] fp16
    log_mass: torch.Tensor | None = None          # [banks, rows] fp32
    coarse_lse: torch.Tensor | None = None        # [banks, rows] fp32
    valid: bool = False
    refreshed_at: int = 0
    pending_stats: torch.Tensor | None = None     # [2] fp32: sum sq error, sum sq output
    pending_age: int | None = None

    def release(self) -> None:
        """Forget the refinement: every field back to its declared default."""
        for f in dataclasses.fields(self):
            setattr(self, f.name, f.default)

    def take_pending(self) -> tuple[torch.Tensor, int] | None:
        """The error statistics a refresh left for the controller, cleared as they are read."""
        stats, age = self.pending_stats, self.pending_age
        self.pending_stats = self.pending_age = None
        return None if stats is None or age is None else (stats, int(age))

    def refinement_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.value, self.log_mass)
                   if t is not None)


_BANK_TENSORS = ("head_kernel_mask", "partition", "value", "log_mass", "coarse_lse")


@dataclass(frozen=True)
class _HeadGroup:
    """Where one group of heads (``bank_chunks``, recap/operator.py:62-145, 260-326) sits in
    a layer's bank tensors: banks lo..hi of total, heads head0..head1 of batch ``batch``."""

    lo: int
    hi: int
    total: int
    batch: int
    head0: int
    head1: int
    heads: int

    def rows(self, name: str, whole: torch.Tensor | None) -> torch.Tensor | None:
        if whole is None:
            return None
        if name == "partition":  # [B, H, nb, nb]
            return whole[self.batch:self.batch + 1, self.head0:self.head1]
        return whole[self.lo:self.hi]

    def layer_shape(self, name: str, part: torch.Tensor) -> tuple:
        if name == "partition":
            return (max(1, self.total // self.heads), self.heads, *part.shape[2:])
        return (self.total, *part.shape[1:])

    def open(self, bank: DetailBank) -> DetailBank:
        """The group's own DetailBank: the layer's tensors as views of the group's rows and a
        copy of the layer-level flags."""
        own = DetailBank(valid=bank.valid, refreshed_at=bank.refreshed_at,
                         pending_stats=bank.pending_stats, pending_age=bank.pending_age)
        for name in _BANK_TENSORS:
            setattr(own, name, self.rows(name, getattr(bank, name)))
        return own

    def close(self, bank: DetailBank, own: DetailBank) -> None:
        """Bring back the tensors the group's computation replaced (a view it wrote in place
        needs nothing); a field it dropped is dropped for the layer."""
        for name in _BANK_TENSORS:
            part, whole = getattr(own, name), getattr(bank, name)
            view = self.rows(name, whole)
            if part is None:
                if whole is not None:
                    setattr(bank, name, None)
                continue
            if view is not None and part.data_ptr() == view.data_ptr() and part.shape == view.shape:
                continue
            shape = self.layer_shape(name, part)
            if whole is None or tuple(whole.shape) != shape:
                whole = torch.empty(shape, dtype=part.dtype, device=part.device)
                setattr(bank, name, whole)
            self.rows(name, whole).copy_(part)


def _publish_groups(bank: DetailBank, groups: list[DetailBank]) -> None:
    """Layer-level flags after all head groups ran: the last group's, with the validation
    sums added over the groups."""
    last = groups[-1]
    bank.valid, bank.refreshed_at, bank.pending_age = last.valid, last.refreshed_at, last.pending_age
    stats = [g.pending_stats for g in groups if g.pending_stats is not None]
    bank.pending_stats = torch.stack(stats).sum(dim=0) if len(stats) > 1 else (
        stats[0] if stats else None)


@dataclass
class Operator:
    """Dispatches one attention call per layer and owns the detail banks."""

    config: OperatorConfig
    layout: Layout
    layers: list[list[SparseAttention]]
    banks: list[list[DetailBank]] = field(default_factory=list)
    kind: str = EXACT
    step: int = 0
    stream: int = 0
    refreshed_layers: int = 0
    alpha_override: float | None = None
    #: when a dict, SPARSE calls record timing events after each stage (name -> events)
    stage_events: dict | None = None
    _chunk_states: dict = field(default_factory=dict)
    _forced_partition: torch.Tensor | None = None
    _forced_rerank: bool | None = None

    # The per-(stream, layer) state is a grid of cells: the sparse state in ``layers`` and
    # the refinement in ``banks``, both indexed [stream][layer] (the reference's indexing,
    # which host paging and the integrations use).  The current call is the cursor
    # (kind, step, stream, refreshed_layers), set by begin_step / set_stream.

    def __post_init__(self) -> None:
        rows = self.layers
        if not rows or not all(isinstance(row, (list, tuple)) and row for row in rows):
            raise TypeError("Operator.layers must be indexed [stream][layer]")
        self.banks = [[DetailBank() for _ in row] for row in rows]

    @classmethod
    def build(cls, config: OperatorConfig, geometry: SparseGeometry, *, n_layers: int,
              n_streams: int = 1) -> "Operator":
        """A fresh sparse state in every cell (recap/operator.py:176-191)."""
        if min(n_layers, n_streams) < 1:
            raise ValueError("n_layers and n_streams must be positive")
        grid = [[SparseAttention(geometry, config) for _ in range(n_layers)]
                for _ in range(n_streams)]
        return cls(config, geometry.layout, grid)

    @property
    def n_streams(self) -> int:
        return len(self.layers)

    def _cells(self):
        """Every (sparse state, bank) pair, stream by stream."""
        for states, banks in zip(self.layers, self.banks):
            yield from zip(states, banks)

    def _start_call(self, kind: str, step: int) -> None:
        self.kind, self.step, self.stream, self.refreshed_layers = kind, int(step), 0, 0

    def reset(self) -> None:
        """Back to the state right after build (recap/operator.py:197-210)."""
        for state, bank in self._cells():
            state.reset()
            bank.release()
        for state in self._chunk_states.values():
            state.reset()
        self._start_call(EXACT, 0)

    @property
    def banks_valid(self) -> bool:
        """Every layer of every stream holds a refinement."""
        flags = [bank.valid for _, bank in self._cells()]
        return bool(flags) and all(flags)

    def begin_step(self, step: int, kind: str) -> None:
        """Start the calls of one computed step (stream 0 first)."""
        if kind not in _KINDS:
            raise ValueError(f"unknown computed call kind {kind!r}")
        self._start_call(kind, step)

    def set_stream(self, stream: int) -> None:
        """Select the stream (CFG branch) the next calls belong to."""
        if stream not in range(self.n_streams):
            raise ValueError(f"stream {stream} outside 0..{self.n_streams - 1}")
        self.stream = int(stream)

    # -- dispatch ------------------------------------------------------------------------

    def _geometry(self, query: torch.Tensor) -> K.Geometry:
        self.layout._check(query)
        banks = query.shape[0] * query.shape[1]
        nb = -(-self.layout.video_tokens // K.BLOCK)
        return K.Geometry(n_tokens=query.shape[-2], n_video=self.layout.video_tokens,
                          closure_group=K.closure_group(banks, nb))

    @torch.no_grad()
    def attend(self, layer_index: int, query: torch.Tensor, key: torch.Tensor,
               value: torch.Tensor) -> torch.Tensor:
        """One attention call (recap/operator.py:233-258)."""
        if self.kind == EXACT:
            return F.scaled_dot_product_attention(query, key, value, dropout_p=0.0,
                                                  is_causal=False)
        if query.shape != key.shape or key.shape != value.shape:
            raise ValueError("Q/K/V shapes differ")
        if not query.dtype == key.dtype == value.dtype:
            raise ValueError(f"Q/K/V dtypes differ ({query.dtype}, {key.dtype}, {value.dtype})")
        chunks = int(self.config.bank_chunks)
        if chunks > 1:
            return self._attend_in_chunks(layer_index, query, key, value, chunks)
        layer = self.layers[self.stream][layer_index]
        bank = self.banks[self.stream][layer_index]
        q, k, v = (K.prepare(x, n) for x, n in ((query, "query"), (key, "key"), (value, "value")))
        geo = self._geometry(q)
        rowmap = self.layout.rowmap(q.device)
        if self.kind == SPARSE:
            return self._sparse(layer, bank, q, k, v, geo, rowmap)
        kv = K.kv_pack(k, v, rowmap, geo)
        # The head branch comes out of the dense pass: its mask is the stored one, or on a
        # bank's first refresh the selection made now.
        selection = None if bank.valid else self._select(layer, q, kv, geo, rowmap)
        kmask = bank.head_kernel_mask if selection is None else selection[1]
        out, lse, head_out, head_lse = K.dense_head_attn(q, kv, rowmap, kmask,
                                                         K.scale_for(q.shape[-1]))
        self._refresh(layer, bank, q, kv, geo, rowmap, out, lse, head=(head_out, head_lse),
                      selection=selection)
        return out

    @torch.no_grad()
    def _attend_in_chunks(self, layer_index, query, key, value, chunks):
        """One layer in groups of heads (recap/operator.py:260-326); result-identical."""
        b, h, n, d = query.shape
        q, k, v = (K.prepare(x, n) for x, n in ((query, "query"), (key, "key"), (value, "value")))
        geo = self._geometry(q)
        rowmap = self.layout.rowmap(q.device)
        bank = self.banks[self.stream][layer_index]
        out = torch.empty(b, h, n, d, dtype=q.dtype, device=q.device)
        lse = head_all = selection_all = None
        if self.kind == REFRESH:
            kv_all = K.kv_pack(k, v, rowmap, geo)
            if not bank.valid:
                selection_all = self._select(self.layers[self.stream][layer_index], q, kv_all,
                                             geo, rowmap)
            kmask = bank.head_kernel_mask if selection_all is None else selection_all[1]
            _, lse, head_out, head_lse = K.dense_head_attn(q, kv_all, rowmap, kmask,
                                                           K.scale_for(d), out=out)
            head_all = (head_out, head_lse)
            del kv_all
        forced = None
        if self.kind == REFRESH and bank.valid and bank.partition is not None:
            layer0 = self.layers[self.stream][layer_index]
            kv_all = K.kv_pack(k, v, rowmap, geo)
            forced = layer0.head_partition(q, kv_all, rowmap, geo, K.scale_for(d))
            del kv_all
            kept, total = K.mask_overlap(forced, bank.partition)
            self._forced_rerank = kept / max(total, 1) < self.config.rerank_min_overlap
            forced = forced.reshape(b, h, geo.nb, geo.nb)
        per = max(1, math.ceil(h / chunks))
        opened: list[DetailBank] = []
        group = 0
        refreshed_before = self.refreshed_layers
        for bi in range(b):
            for h0 in range(0, h, per):
                h1 = min(h0 + per, h)
                state = self._chunk_states.get((self.stream, layer_index, group))
                if state is None:
                    state = SparseAttention(self.layers[self.stream][layer_index].geometry,
                                            self.config)
                    self._chunk_states[(self.stream, layer_index, group)] = state
                span = _HeadGroup(lo=bi * h + h0, hi=bi * h + h1, total=b * h, batch=bi,
                                  head0=h0, head1=h1, heads=h)
                view = span.open(bank)
                opened.append(view)
                qs, ks, vs = (x[bi:bi + 1, h0:h1] for x in (q, k, v))
                self._forced_partition = (None if forced is None
                                          else forced[bi:bi + 1, h0:h1].reshape(-1, geo.nb, geo.nb))
                if self.kind == SPARSE:
                    self._sparse(state, view, qs, ks, vs, geo, rowmap, out=out[bi:bi + 1, h0:h1])
                else:
                    kv = K.kv_pack(ks, vs, rowmap, geo)
                    lo, hi = bi * h + h0, bi * h + h1
                    sel = None if selection_all is None else (
                        selection_all[0][bi:bi + 1, h0:h1], selection_all[1][lo:hi])
                    self._refresh(state, view, qs, kv, geo, rowmap, out[bi:bi + 1, h0:h1],
                                  lse[bi:bi + 1, h0:h1],
                                  head=(head_all[0][lo:hi], head_all[1][lo:hi]), selection=sel)
                span.close(bank, view)
                group += 1
        self._forced_partition = None
        self._forced_rerank = None
        if opened:
            _publish_groups(bank, opened)
        if self.refreshed_layers > refreshed_before:
            self.refreshed_layers = refreshed_before + 1
        return out

    # -- refresh -------------------------------------------------------------------------

    def _select(self, layer, q, kv, geo, rowmap):
        """Partition and kernel mask in one library call (recap/operator.py:353-361)."""
        b, h = q.shape[:2]
        part, kmask = K.pool_select(q, kv.k_means, rowmap, geo, layer.config.head_density,
                                    K.scale_for(q.shape[-1]))
        return part.reshape(b, h, geo.nb, geo.nb), kmask

    @torch.no_grad()
    def _refresh(self, layer, bank, q, kv, geo, rowmap, full_output, full_lse, head=None,
                 selection=None) -> None:
        """Store the refinement and measure the previous one (recap/operator.py:330-473).

        ``head`` is the head branch of the bank's current (or, on a first refresh, newly
        selected ``selection``) mask when the dense pass already produced it."""
        b, h, n, d = q.shape
        banks = b * h
        scale = K.scale_for(d)
        revalidating = bank.valid
        if not revalidating:
            bank.partition, bank.head_kernel_mask = (
                selection if selection is not None else self._select(layer, q, kv, geo, rowmap))
        if head is not None:
            head_out, head_lse = head
        else:
            head_out, head_lse = K.block_sparse_attn(q, kv, rowmap, bank.head_kernel_mask, geo,
                                                     scale)
        context = layer.coarse_tail_context(kv, geo)
        flat_part = bank.partition.reshape(banks, geo.nb, geo.nb)
        old_lse = bank.coarse_lse if revalidating else None
        go, gl, drift_part = layer.coarse_tail_apply(q, rowmap, context, flat_part, geo, scale,
                                                     glref=old_lse)
        if bank.value is None:
            bank.value = torch.empty(banks, geo.rows, d, dtype=torch.float16, device=q.device)
            bank.log_mass = torch.empty(banks, geo.rows, dtype=torch.float32, device=q.device)
        center = K.drift_center(drift_part, geo) if old_lse is not None else None
        stats = K.refresh_capture(full_output, full_lse, head_out, head_lse, go, gl, rowmap, geo,
                                  bank.value, bank.log_mass, glref=old_lse, center=center)
        if stats is not None:
            bank.pending_stats = stats
            bank.pending_age = self.step - bank.refreshed_at

        if revalidating:
            if self._forced_partition is not None:
                partition = self._forced_partition.reshape(b, h, geo.nb, geo.nb)
                kmask = K.kernel_block_mask(partition, geo)
            else:
                partition, kmask = self._select(layer, q, kv, geo, rowmap)
            if bank.partition is not None:
                if self._forced_rerank is None:
                    kept, total = K.mask_overlap(partition, bank.partition)
                    keep_split = kept / max(total, 1) >= self.config.rerank_min_overlap
                else:
                    keep_split = not self._forced_rerank
                if keep_split:
                    bank.coarse_lse = gl.clone()
                    bank.refreshed_at = self.step
                    bank.valid = True
                    self.refreshed_layers += 1
                    return
            bank.partition, bank.head_kernel_mask = partition, kmask
            head_out, head_lse = K.block_sparse_attn(q, kv, rowmap, bank.head_kernel_mask, geo,
                                                     scale)
            go, gl, _ = layer.coarse_tail_apply(
                q, rowmap, context, bank.partition.reshape(banks, geo.nb, geo.nb), geo, scale)
            K.refresh_capture(full_output, full_lse, head_out, head_lse, go, gl, rowmap, geo,
                              bank.value, bank.log_mass)
        bank.coarse_lse = gl.clone()
        bank.refreshed_at = self.step
        bank.valid = True
        self.refreshed_layers += 1

    # -- sparse --------------------------------------------------------------------------

    def _mark(self, name: str) -> None:
        if self.stage_events is not None:
            event = torch.cuda.Event(enable_timing=True)
            event.record()
            self.stage_events.setdefault(name, []).append(event)

    @torch.no_grad()
    def _sparse(self, layer, bank, q, k, v, geo, rowmap, out=None) -> torch.Tensor:
        """Head exactly, plus coarse tail and weighted cached refinement
        (recap/operator.py:477-527), as four launches with the merge fused."""
        if not bank.valid or bank.head_kernel_mask is None:
            raise RuntimeError("a sparse call was requested before an exact refresh")
        b, h, n, d = q.shape
        banks = b * h
        scale = K.scale_for(d)
        self._mark("start")
        kv = K.kv_pack(k, v, rowmap, geo)
        self._mark("pack")
        context = layer.coarse_tail_context(kv, geo)
        self._mark("closure")
        old_lse = bank.coarse_lse
        go, gl, drift_part = layer.coarse_tail_apply(
            q, rowmap, context, bank.partition.reshape(banks, geo.nb, geo.nb), geo, scale,
            glref=old_lse)
        center = K.drift_center(drift_part, geo) if geo.rows else None
        self._mark("coarse")
        out = K.sparse_merge_attn(q, kv, rowmap, bank.head_kernel_mask, geo, scale, go, gl,
                                  bank.value, bank.log_mass, old_lse, center,
                                  alpha_override=self.alpha_override, out=out)
        self._mark("attention")
        return out

    # -- the refinement error ------------------------------------------------------------

    def drain_validation(self) -> tuple[int, float] | None:
        """(smallest refinement age, relative RMS error over all layers) of the refreshes
        since the last drain, or None (recap/operator.py:531-547).  The error pools every
        layer's sums: sqrt(sum sq error / sum sq output)."""
        pending = [p for p in (bank.take_pending() for _, bank in self._cells()) if p]
        if not pending:
            return None
        err_sq, out_sq = torch.stack([stats for stats, _ in pending]).sum(dim=0).tolist()
        error = math.sqrt(err_sq / out_sq) if out_sq > 0.0 else float("inf")
        return min(age for _, age in pending), error

    def peak_bank_bytes(self) -> int:
        """Bytes of the refinement values and log-masses held on the device."""
        return sum(bank.refinement_bytes() for _, bank in self._cells())
