"""INTEGRATION.md's kernel-level example, run verbatim on the GPU against the oracle's
block-sparse attention (recap/kernels/block_sparse.py:78-139 semantics): the head output in
the query type within the output bar, the LSE within 2e-3."""

import pytest
import torch

import oracle as O
from gpu_util import SMALL, assert_parity, banks_view, metrics, scale_for
from integration_example import load_example
from recap_amd.layout import Layout, hilbert_permutation
from recap_amd.synthetic import make_qkv

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,dtype", [("tiny", torch.bfloat16),
                                        ("text-first-ragged", torch.bfloat16),
                                        ("text-last-d128", torch.float16)])
def test_integration_example_block_sparse_exact(cuda, name, dtype):
    wl = SMALL[name]
    print(f"case {name} {dtype}", flush=True)
    ns = load_example()
    perm = hilbert_permutation(wl.grid)
    layout = Layout.from_permutation(perm, text_tokens=wl.text_tokens, text_first=wl.text_first)
    fwd, _ = O.gather_indices(perm, wl.text_tokens, wl.text_first)
    q, k, v = make_qkv(wl, seed=3, dtype=dtype)
    ql, kl, vl = (banks_view(x, fwd) for x in (q, k, v))
    scale = scale_for(wl.dim)
    part = O.head_partition(ql, kl, scale, wl.density, wl.video_tokens)
    kmask = O.kernel_block_mask(part, wl.tokens, wl.video_tokens)
    out, lse = ns["block_sparse_exact"](q.to(cuda), k.to(cuda), v.to(cuda), kmask.to(cuda),
                                        layout.rowmap(cuda), wl.video_tokens)
    torch.cuda.synchronize()
    assert out.dtype == dtype and lse.dtype == torch.float32
    ref, ref_lse = O.block_sparse_attention(ql, kl, vl, kmask, scale)
    assert_parity(out.cpu().float(), ref, f"example {name}", dtype=dtype)
    m, _ = metrics(lse.cpu(), ref_lse)
    assert m < 2e-3, m
