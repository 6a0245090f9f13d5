"""Write golden vectors from the reference's own pure-torch/numpy functions.

Run in the development container only (it reads the reference tree at
/root/reference, which is absent on GPU machines):

    python tests/golden/make_golden.py

Only the two functions that nothing else pins exactly are imported:
``hilbert_permutation`` (recap/sparse/geometry.py:27-67) and the block selection
``SparseAttention.head_partition`` + ``build_kernel_block_mask``
(recap/sparse/attention.py:74-94, recap/kernels/block_sparse.py:52-75).  Inputs come from
``recap_amd.synthetic`` (seed 0, CPU).  Outputs: ``golden.npz`` (data only, no pickle)
and ``golden.json`` (SHA-256 digests and top-k margins).
"""

from __future__ import annotations

import hashlib
import json
import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, "/root/reference")

from recap.config import OperatorConfig  # noqa: E402
from recap.kernels.block_sparse import build_kernel_block_mask  # noqa: E402
from recap.sparse.attention import SparseAttention, SparseGeometry  # noqa: E402
from recap.sparse.geometry import hilbert_permutation  # noqa: E402
from recap.sparse.layout import Layout  # noqa: E402
from recap.sparse.pooling import pool_blocks  # noqa: E402

from recap_amd.synthetic import WORKLOADS, make_qkv  # noqa: E402

# (workload, heads used for the mask golden)
MASK_CASES = [("cpu-plumbing", None), ("wan2.1-480p", None), ("cogvideox1.5", [0, 1, 2, 3]),
              ("hunyuan-720p", [0, 1])]


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main() -> None:
    arrays: dict[str, np.ndarray] = {}
    meta: dict = {"seed": 0, "hilbert": {}, "masks": {}}
    for name, wl in WORKLOADS.items():
        perm = hilbert_permutation(wl.grid).astype(np.int64)
        meta["hilbert"][name] = {"grid": list(wl.grid), "sha256_int64": sha(perm)}
        if wl.video_tokens <= 4096:
            arrays[f"hilbert_{name}"] = perm.astype(np.int32)
    for name, heads in MASK_CASES:
        wl = WORKLOADS[name]
        perm = hilbert_permutation(wl.grid)
        layout = Layout.from_permutation(perm, text_tokens=wl.text_tokens,
                                         text_first=wl.text_first)
        geometry = SparseGeometry.build(layout, 128)
        layer = SparseAttention(geometry, OperatorConfig(head_density=wl.density))
        q, k, _ = make_qkv(wl, heads=heads, seed=0)
        ql, kl = layout.reorder(q), layout.reorder(k)
        scale = 1.0 / math.sqrt(wl.dim)
        part = layer.head_partition(ql, kl, scale)
        banks = part.shape[0] * part.shape[1]
        flat = part.reshape(banks, part.shape[-2], part.shape[-1])
        kmask = build_kernel_block_mask(flat, sequence_tokens=wl.tokens,
                                        video_tokens=wl.video_tokens, block_size=128)
        qb = pool_blocks(ql, 128, wl.video_tokens).mean
        kb = pool_blocks(kl, 128, wl.video_tokens).mean
        scores = torch.matmul(qb.float(), kb.float().transpose(-1, -2)) * scale
        nb = qb.shape[-2]
        keep = max(1, round(wl.density * nb))
        top = torch.topk(scores.double(), keep + 1, dim=-1).values
        margin = float((top[..., keep - 1] - top[..., keep]).min())
        pnp = part.numpy().astype(bool)
        knp = kmask.numpy().astype(bool)
        meta["masks"][name] = {
            "heads": heads if heads is not None else list(range(wl.heads)),
            "partition_shape": list(pnp.shape), "kernel_mask_shape": list(knp.shape),
            "partition_sha256_u8": sha(pnp.astype(np.uint8)),
            "kernel_mask_sha256_u8": sha(knp.astype(np.uint8)),
            "keep": keep, "min_topk_margin": margin,
        }
        if pnp.size <= 1_000_000:
            arrays[f"partition_{name}"] = np.packbits(pnp.reshape(-1))
        print(name, "keep", keep, "margin", margin, flush=True)
    np.savez_compressed(HERE / "golden.npz", **arrays)
    (HERE / "golden.json").write_text(json.dumps(meta, indent=1) + "\n")


if __name__ == "__main__":
    main()
