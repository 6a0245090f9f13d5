"""Refinement banks in pinned host memory, paged to the GPU layer by layer
(recap/host_banks.py), over the native pager of librecap_hip.so (``recap_pager_*``).

Every (stream, layer) key's bank -- the fp16 refinement, its log-mass, the partition, the
kernel mask and the drift reference, i.e. everything a sparse call of that layer reads --
lives in pinned host memory the pager allocates.  Device slots (two with prefetch, one
without) hold the bank of the layer that runs: the pager stages it in on the compute
stream or takes it from a prefetch issued during the previous layer, and writes a refresh's
new bank back on its own stream.  This class only binds the slots' device tensors to the
bank each layer sees.  Outputs are identical to keeping the banks on the GPU.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .operator import REFRESH, SPARSE, Operator

# The paged fields, in the pager's field order; the last three are the layer's split state.
FIELDS = ("value", "log_mass", "partition", "head_kernel_mask", "coarse_lse")
SPLIT = FIELDS[2:]


class _Pager:
    """Owner of one native pager handle."""

    def __init__(self, n_keys: int, n_slots: int, field_bytes: list[int], timing: bool):
        self.lib = _lib.load()
        handle = ctypes.c_void_p()
        sizes = (ctypes.c_int64 * len(field_bytes))(*field_bytes)
        _lib.call("recap_pager_create", n_keys, n_slots, ctypes.cast(sizes, ctypes.c_void_p),
                  len(field_bytes), _lib.PAGER_TIMING if timing else 0, ctypes.byref(handle))
        self.handle = handle.value

    def __call__(self, name: str, *args):
        return _lib.call(f"recap_pager_{name}", self.handle, *args)

    def stored(self, key: int) -> bool:
        return self.lib.recap_pager_stored(self.handle, key) == 1

    def host_bytes(self) -> int:
        return int(self.lib.recap_pager_host_bytes(self.handle))

    def counts(self) -> dict[str, int]:
        out = (ctypes.c_int64 * 4)()
        self("counts", ctypes.cast(out, ctypes.c_void_p))
        return dict(zip(("from_prefetch", "copied", "prefetches", "written_back"), out))

    def copy_time(self) -> tuple[float, int]:
        ms, n = ctypes.c_double(), ctypes.c_int64()
        self("copy_time", ctypes.byref(ms), ctypes.byref(n))
        return ms.value, n.value

    def close(self) -> None:
        if self.handle:
            self.lib.recap_pager_destroy(self.handle)   # waits for its transfers
            self.handle = None


class HostBankOperator(Operator):
    """An :class:`Operator` whose refinement banks are paged from pinned host memory."""

    def __post_init__(self) -> None:
        super().__post_init__()
        self._pager: _Pager | None = None
        self._slots: list[dict[str, torch.Tensor]] = []
        self._specs: dict | None = None
        self._turn = 0            # the slot the next call uses (slots alternate call by call)
        self._want_prefetch = True
        #: time every bank copy (set before the first call or preallocate_host)
        self.record_copies = False

    def set_prefetch(self, enabled: bool) -> None:
        """Overlap the next layer's transfer with this layer's compute."""
        self._want_prefetch = bool(enabled)

    # -- geometry of a bank --------------------------------------------------------------

    def _field_specs(self, banks: int, dim: int) -> dict[str, tuple]:
        """Shape and dtype of each paged field (the partition is kept per bank here and
        viewed [B, H, nb, nb] when a layer runs)."""
        block = self.config.block_size
        n_video = self.layout.video_tokens
        rows, nb = (n_video // block) * block, -(-n_video // block)
        tb = -(-self.layout.tokens // block)
        return {"value": ((banks, rows, dim), torch.float16),
                "log_mass": ((banks, rows), torch.float32),
                "partition": ((banks, nb, nb), torch.bool),
                "head_kernel_mask": ((banks, tb, tb), torch.bool),
                "coarse_lse": ((banks, rows), torch.float32)}

    def _setup(self, banks: int, dim: int, device) -> None:
        """A pager and device slots for banks of this geometry.  The geometry is every
        field's shape: the kernel mask [banks, tb, tb] follows the text length, which the
        model integrations retarget per prompt (recap/models/hunyuan.py:30-39, 96-97).  A
        new geometry drops the banks held so far; the pinned host memory is kept where it
        is large enough (recap_pager_resize) and the slots' changed fields are reallocated."""
        specs = self._field_specs(banks, dim)
        if self._pager is not None and self._specs == specs:
            return
        n_slots = 2 if self._want_prefetch else 1
        sizes = [torch.Size(s).numel() * torch.empty((), dtype=t).element_size()
                 for s, t in specs.values()]
        if self._pager is not None and len(self._slots) == n_slots:
            arr = (ctypes.c_int64 * len(sizes))(*sizes)
            self._pager("resize", ctypes.cast(arr, ctypes.c_void_p), len(sizes))
        else:
            self._close()
            self._pager = _Pager(self._key(self.n_streams, 0), n_slots, sizes,
                                 self.record_copies)
            self._slots = [{} for _ in range(n_slots)]
        for slot, tensors in enumerate(self._slots):
            for name, (shape, dtype) in specs.items():
                old = tensors.get(name)
                if old is None or tuple(old.shape) != tuple(shape) or old.dtype != dtype:
                    tensors[name] = torch.empty(shape, dtype=dtype, device=device)
            ptrs = (ctypes.c_void_p * len(FIELDS))(*(tensors[n].data_ptr() for n in FIELDS))
            self._pager("bind", slot, ctypes.cast(ptrs, ctypes.c_void_p))
        self._specs = specs
        self._turn = 0

    def preallocate_host(self, n_layers: int, n_banks: int, dim: int) -> int:
        """Allocate the pinned banks of the first ``n_layers`` layers (of every stream) and
        the device slots now; returns the pinned host bytes (recap/host_banks.py:85-97)."""
        if torch.cuda.is_available():
            self._setup(n_banks, dim, torch.device("cuda"))
            layers = min(n_layers, self._layers_per_stream())
            if layers > 0:
                self._pager("reserve", self._key(self.n_streams - 1, layers - 1) + 1)
        return self.peak_bank_bytes()

    # -- one layer -----------------------------------------------------------------------

    def _layers_per_stream(self) -> int:
        return max(len(row) for row in self.layers)

    def _key(self, stream: int, layer: int) -> int:
        return stream * self._layers_per_stream() + layer

    @torch.no_grad()
    def attend(self, layer_index: int, query, key, value):
        if self.kind not in (REFRESH, SPARSE):
            return super().attend(layer_index, query, key, value)
        b, h, _, dim = query.shape
        self._setup(b * h, dim, query.device)
        bank = self.banks[self.stream][layer_index]
        bank_key = self._key(self.stream, layer_index)
        slot = self._turn
        self._turn = (slot + 1) % len(self._slots)
        stored = self._pager.stored(bank_key)
        if self.kind == SPARSE and not stored:
            raise RuntimeError("a sparse call was requested before an exact refresh")
        if bank.valid and not stored:
            bank.valid = False   # its bank was dropped (new shape): refresh from scratch
        compute = torch.cuda.current_stream().cuda_stream
        # A sparse call reads the bank; a refresh of a valid bank scores it first.
        load = stored and (self.kind == SPARSE or bank.valid)
        if load:
            self._pager("stage_in", bank_key, slot, compute)
            self._prefetch_next(layer_index)
        else:
            self._pager("acquire", slot, compute)
        slot_tensors = self._slots[slot]
        nb = slot_tensors["partition"].shape[-1]
        views = dict(slot_tensors, partition=slot_tensors["partition"].view(b, h, nb, nb))
        bank.value, bank.log_mass = views["value"], views["log_mass"]
        if load:
            for name in SPLIT:
                setattr(bank, name, views[name])
        try:
            out = super().attend(layer_index, query, key, value)
            if self.kind == REFRESH:
                # The refresh may have put its split state in new tensors: gather it into
                # the slot, whose whole contents then go back to host memory.
                for name in SPLIT:
                    tensor = getattr(bank, name)
                    if tensor is not None and tensor.data_ptr() != views[name].data_ptr():
                        views[name].copy_(tensor.reshape(views[name].shape))
                self._pager("stage_out", bank_key, slot, compute)
                if not load:
                    # A refresh that loaded nothing prefetched nothing; with its bank on its
                    # way out, the next call's bank, if host memory holds one, can come in
                    # while this call ends.
                    self._prefetch_next(layer_index, stored_only=True)
        finally:
            self._pager("release", slot, compute)
            for name in FIELDS:
                setattr(bank, name, None)
        return out

    def _next_call(self, layer: int) -> tuple[int, int]:
        """(stream, layer) of the call expected after this one: the next layer of this
        stream; after its last layer, layer 0 of the next stream (the session runs the
        streams of a step in turn, recap/session.py:264-308), which with one stream is the
        next step's layer 0."""
        if layer + 1 < len(self.layers[self.stream]):
            return self.stream, layer + 1
        return (self.stream + 1) % self.n_streams, 0

    def _prefetch_next(self, layer: int, stored_only: bool = False) -> None:
        """Bring the next call's bank into the slot that call will use while this layer
        computes.  With `stored_only`, only a bank that host memory already holds."""
        if len(self._slots) < 2:
            return
        key = self._key(*self._next_call(layer))
        if stored_only and not self._pager.stored(key):
            return
        self._pager("prefetch", key, self._turn)

    # -- bookkeeping ---------------------------------------------------------------------

    def finish(self) -> None:
        """Wait for all transfers in flight (recap/host_banks.py:246-258)."""
        if self._pager is not None:
            self._pager("finish")

    def reset(self) -> None:
        self.finish()
        super().reset()

    def _close(self) -> None:
        if self._pager is not None:
            self._pager.close()
        self._pager, self._slots, self._specs, self._turn = None, [], None, 0

    def __del__(self):  # pragma: no cover - teardown path
        try:
            self._close()
        except Exception:
            pass

    def peak_bank_bytes(self) -> int:
        """Pinned host bytes held by the banks."""
        return 0 if self._pager is None else self._pager.host_bytes()

    def pager_counts(self) -> dict[str, int]:
        """Stage-ins served by a prefetch / copied on the compute stream, prefetches issued,
        write-backs."""
        return {} if self._pager is None else self._pager.counts()

    def copy_time(self) -> tuple[float, int]:
        """(milliseconds, batches) of the timed bank copies (with record_copies)."""
        return (0.0, 0) if self._pager is None else self._pager.copy_time()
