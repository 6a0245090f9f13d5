"""Refinement banks in pinned host memory, paged to the GPU layer by layer
(recap/host_banks.py).

Each (stream, layer) keeps its fp16 refinement and fp32 log-mass in pinned host memory;
two GPU slots stage them.  While layer ``l`` computes, layer ``l+1``'s bank is copied in
on a prefetch stream; a refresh writes its new bank back on a write-back stream.  Events
fence every reuse of a slot.  Copies go through ``recap_bank_copy_async``
(hipMemcpyAsync on the given stream).  Outputs are identical to keeping the banks on the
GPU.  All streams keep the default priority.
"""

from __future__ import annotations

import torch

from . import kernels as K
from .operator import REFRESH, SPARSE, Operator

_FIELDS = ("value", "log_mass")
_SPLIT_FIELDS = ("partition", "head_kernel_mask", "coarse_lse")


class HostBankOperator(Operator):
    """An :class:`Operator` with the refinement in pinned host memory and two GPU slots."""

    def __post_init__(self) -> None:
        super().__post_init__()
        self._host: dict = {}
        self._slots: list[dict] = []
        self._slot_ready: list = [None, None]  # write-back to host finished
        self._slot_free: list = [None, None]   # compute finished reading the slot
        self._want_prefetch = True
        self._prefetch_stream = None
        self._out_stream = None
        self._host_split: dict = {}
        self._split_slots: dict = {}
        self._device = None
        self._prefetched = None
        self._split_prefetched = None
        self.copy_events: list[tuple[str, torch.cuda.Event, torch.cuda.Event]] = []
        self.record_copies = False

    def set_prefetch(self, enabled: bool) -> None:
        self._want_prefetch = bool(enabled)

    # -- slots ---------------------------------------------------------------------------

    def _rows(self) -> int:
        block = self.config.block_size
        return (self.layout.video_tokens // block) * block

    def _alloc_slots(self, n_banks: int, rows: int, dim: int, device) -> None:
        self._slots = [{
            "value": torch.empty((n_banks, rows, dim), dtype=torch.float16, device=device),
            "log_mass": torch.empty((n_banks, rows), dtype=torch.float32, device=device),
        } for _ in range(2 if self._want_prefetch else 1)]
        if self._want_prefetch and self._prefetch_stream is None:
            self._prefetch_stream = torch.cuda.Stream(device=device)
        if self._out_stream is None:
            self._out_stream = torch.cuda.Stream(device=device)

    def _ensure_slots(self, query: torch.Tensor) -> None:
        b, h, _, dim = query.shape
        n_banks, rows = b * h, self._rows()
        if self._slots and tuple(self._slots[0]["value"].shape) == (n_banks, rows, dim):
            return
        self._alloc_slots(n_banks, rows, dim, query.device)

    @staticmethod
    def _new_host_bank(n_banks: int, rows: int, dim: int) -> dict:
        return {
            "value": torch.empty((n_banks, rows, dim), dtype=torch.float16, pin_memory=True),
            "log_mass": torch.empty((n_banks, rows), dtype=torch.float32, pin_memory=True),
        }

    def _host_bank(self, key_id) -> dict:
        existing = self._host.get(key_id)
        if existing is not None:
            return existing
        n_banks, rows, dim = self._slots[0]["value"].shape
        made = self._new_host_bank(n_banks, rows, dim)
        self._host[key_id] = made
        return made

    def preallocate_host(self, n_layers: int, n_banks: int, dim: int) -> int:
        """Allocate all host banks and the GPU slots; returns the host bytes."""
        rows = self._rows()
        for stream in range(self.n_streams):
            for layer in range(min(n_layers, len(self.layers[stream]))):
                if (stream, layer) not in self._host:
                    self._host[(stream, layer)] = self._new_host_bank(n_banks, rows, dim)
        if torch.cuda.is_available() and not self._slots:
            self._alloc_slots(n_banks, rows, dim, torch.device("cuda"))
        return self.peak_bank_bytes()

    def _copy(self, dst: dict, src: dict, kind: str, fields=_FIELDS) -> None:
        stream = torch.cuda.current_stream()
        start = end = None
        if self.record_copies:
            start = torch.cuda.Event(enable_timing=True)
            start.record(stream)
        for name in fields:
            if dst.get(name) is not None and src.get(name) is not None:
                K.bank_copy_async(dst[name], src[name], stream)
        if self.record_copies:
            end = torch.cuda.Event(enable_timing=True)
            end.record(stream)
            self.copy_events.append((kind, start, end))

    @staticmethod
    def _attach(bank, slot: dict) -> None:
        bank.value, bank.log_mass = slot["value"], slot["log_mass"]

    @staticmethod
    def _detach(bank) -> None:
        bank.value = bank.log_mass = None

    # -- per-layer partition state -------------------------------------------------------

    def _split_slot(self, key_id) -> dict:
        return self._split_slots.setdefault(key_id[1] % max(1, len(self._slots)), {})

    def _copy_split(self, key_id, stream=None) -> dict:
        """Copy the layer's partition, kernel mask and drift reference into its split slot
        (recap/host_banks.py:116-130) on `stream` (default: the current stream)."""
        slot = self._split_slot(key_id)
        for name, tensor in self._host_split.get(key_id, {}).items():
            dev = slot.get(name)
            if dev is None or dev.shape != tensor.shape or dev.dtype != tensor.dtype:
                dev = torch.empty(tensor.shape, dtype=tensor.dtype, device=self._device)
                slot[name] = dev
            K.bank_copy_async(dev, tensor, stream)
        return slot

    def _split_in(self, bank, key_id, prefetched: bool) -> None:
        """Point the bank at its split state in the split slot: already copied there with
        the bank on the prefetch stream when `prefetched`, else copied now on the current
        stream (recap/host_banks.py:116-130)."""
        if not self._host_split.get(key_id):
            return
        slot = self._split_slot(key_id) if prefetched else self._copy_split(key_id)
        for name in self._host_split[key_id]:
            setattr(bank, name, slot[name])

    def _split_out(self, bank, key_id) -> None:
        """Queue the layer's split state (partition, kernel mask, drift reference) for its
        pinned host buffers on the current stream, which is the write-back stream when
        called from _stage_out.  The reference copies it synchronously
        (recap/host_banks.py:132-146); here the slot event that fences the bank write-back
        also fences these copies, and record_stream keeps the device tensors alive until
        they are done."""
        host = self._host_split.setdefault(key_id, {})
        stream = torch.cuda.current_stream()
        for name in _SPLIT_FIELDS:
            tensor = getattr(bank, name, None)
            if tensor is None:
                host.pop(name, None)
                continue
            tensor = tensor.contiguous()
            buf = host.get(name)
            if buf is None or buf.shape != tensor.shape or buf.dtype != tensor.dtype:
                buf = torch.empty(tensor.shape, dtype=tensor.dtype, pin_memory=True)
                host[name] = buf
            K.bank_copy_async(buf, tensor, stream)
            tensor.record_stream(stream)

    @staticmethod
    def _split_detach(bank) -> None:
        for name in _SPLIT_FIELDS:
            setattr(bank, name, None)

    # -- dispatch ------------------------------------------------------------------------

    @torch.no_grad()
    def attend(self, layer_index: int, query, key, value):
        if self.kind not in (REFRESH, SPARSE):
            return super().attend(layer_index, query, key, value)
        bank = self.banks[self.stream][layer_index]
        self._ensure_slots(query)
        index = layer_index % len(self._slots)
        slot = self._slots[index]
        key_id = (self.stream, layer_index)
        host = self._host.get(key_id)
        if host is not None and tuple(host["value"].shape) != tuple(slot["value"].shape):
            self._host.pop(key_id)
            host = None
        pending = self._slot_ready[index]
        if pending is not None:
            torch.cuda.current_stream().wait_event(pending)
            self._slot_ready[index] = None
        self._device = query.device
        # What the prefetch stream queued during the previous layer (normally this layer's
        # bank and split state) is waited for here, before this layer touches a slot or
        # queues the next layer's prefetch on that stream.  Which parts were for this layer
        # is read now: _stage_in below starts the next prefetch and moves both markers on.
        bank_ready = self._prefetched == key_id
        split_ready = self._split_prefetched == key_id
        if (self._prefetched is not None or self._split_prefetched is not None) \
                and self._prefetch_stream is not None:
            torch.cuda.current_stream().wait_stream(self._prefetch_stream)
        self._prefetched = self._split_prefetched = None
        if self.kind == SPARSE:
            if host is None:
                raise RuntimeError("a sparse call was requested before an exact refresh")
            self._stage_in(key_id, slot, bank_ready)
        elif bank.valid and host is not None:
            self._stage_in(key_id, slot, bank_ready)  # the refresh scores the old refinement
        self._attach(bank, slot)
        self._split_in(bank, key_id, split_ready)
        try:
            out = super().attend(layer_index, query, key, value)
        finally:
            if self.kind == REFRESH:
                self._stage_out(key_id, slot, index, bank)
            self._split_detach(bank)
            released = torch.cuda.Event()
            released.record()
            self._slot_free[index] = released
            self._detach(bank)
        return out

    def _stage_in(self, key_id, slot: dict, prefetched: bool) -> None:
        """Bring the layer's bank into its slot: already there when `prefetched` (the
        caller has waited for the prefetch stream), else a copy on the current stream.
        Then start the next layer's prefetch."""
        if not prefetched:
            self._copy(slot, self._host[key_id], "h2d-sync")
        self._maybe_prefetch(key_id)

    def _maybe_prefetch(self, key_id) -> None:
        """Start copying the next layer's bank and split state into the other slot while
        this layer computes (recap/host_banks.py:209-225).  After the stream's last layer
        the next one is layer 0 of the following step, when it uses the other slot.  The
        split state rides along here; the reference copies it on the compute stream.  The
        slot's write-back event stays set, so a fallback synchronous copy still waits."""
        if self._prefetch_stream is None:
            return
        stream, layer = key_id
        nxt = (stream, layer + 1)
        if nxt not in self._host:
            nxt = (stream, 0)
            if layer == 0 or nxt not in self._host:
                return
        index = nxt[1] % len(self._slots)
        if index == layer % len(self._slots):
            return
        with torch.cuda.stream(self._prefetch_stream):
            released = self._slot_free[index]
            if released is not None:
                self._prefetch_stream.wait_event(released)
            # A refresh's write-back of the slot must finish reading it first (the
            # reference skips the prefetch instead, so refresh steps never overlap).
            written = self._slot_ready[index]
            if written is not None:
                self._prefetch_stream.wait_event(written)
            self._copy(self._slots[index], self._host[nxt], "h2d-prefetch")
            if self._host_split.get(nxt):
                self._copy_split(nxt, self._prefetch_stream)
                self._split_prefetched = nxt
        self._prefetched = nxt

    def _stage_out(self, key_id, slot: dict, index: int, bank) -> None:
        """Copy the new refinement and split state to host memory on the write-back stream
        after the compute that produced them (recap/host_banks.py:227-242); the slot event
        fences every later reuse of the slot and of the host buffers."""
        host = self._host_bank(key_id)
        written = torch.cuda.Event()
        written.record()
        with torch.cuda.stream(self._out_stream):
            self._out_stream.wait_event(written)
            self._copy(host, slot, "d2h")
            self._split_out(bank, key_id)
            event = torch.cuda.Event()
            event.record()
        self._slot_ready[index] = event

    # -- bookkeeping ---------------------------------------------------------------------

    def finish(self) -> None:
        """Wait for all transfers in flight."""
        for events in (self._slot_ready, self._slot_free):
            for event in events:
                if event is not None:
                    event.synchronize()
        if self._prefetch_stream is not None:
            self._prefetch_stream.synchronize()
        if self._out_stream is not None:
            self._out_stream.synchronize()
        self._slot_ready = [None, None]
        self._slot_free = [None, None]
        self._prefetched = None
        self._split_prefetched = None

    def reset(self) -> None:
        self.finish()
        super().reset()

    def __del__(self):  # pragma: no cover - teardown path
        try:
            self.finish()
        except Exception:
            pass

    def peak_bank_bytes(self) -> int:
        """Host bytes held by the refinement."""
        return sum(t.numel() * t.element_size() for bank in self._host.values()
                   for t in bank.values() if t is not None)
