"""Property-based checks (hypothesis) of the oracle and of the host-side pieces of the
library over random small shapes: each property is a closed form or an invariant that a
plausible slip (an off-by-one block edge, a transposed index, a wrong tie rule) breaks."""

from __future__ import annotations

import math

import numpy as np
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle as O
from recap_amd import AttentionBranch
from recap_amd.kernels import hilbert_permutation_native

SETTINGS = dict(max_examples=30, deadline=None,
                suppress_health_check=[HealthCheck.too_slow])

grids = st.tuples(st.integers(1, 9), st.integers(1, 12), st.integers(1, 12))


@settings(**SETTINGS)
@given(grids)
def test_native_hilbert_equals_oracle_and_is_a_permutation(grid):
    ref = O.hilbert_permutation(grid)
    got = hilbert_permutation_native(grid).numpy()
    assert np.array_equal(got, ref)
    assert np.array_equal(np.sort(ref), np.arange(int(np.prod(grid))))


@settings(**SETTINGS)
@given(grids, st.integers(0, 300), st.booleans())
def test_gather_indices_are_inverse_permutations(grid, text_tokens, text_first):
    perm = O.hilbert_permutation(grid)
    fwd, inv = O.gather_indices(perm, text_tokens, text_first)
    n = perm.size + text_tokens
    assert torch.equal(fwd[inv], torch.arange(n))
    assert torch.equal(inv[fwd], torch.arange(n))
    # Reordered order is [Hilbert video | text] whatever the native placement of the text.
    video_native = fwd[:perm.size]
    offset = text_tokens if text_first else 0
    assert torch.equal(video_native - offset, torch.as_tensor(perm, dtype=torch.long))


@settings(**SETTINGS)
@given(st.integers(1, 3), st.integers(1, 400), st.sampled_from([16, 32]), st.integers(0, 2**31 - 1))
def test_block_sparse_attention_equals_masked_softmax(banks, n, d, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(banks, n, d, generator=g) for _ in range(3))
    tb = -(-n // 128)
    kmask = torch.rand(banks, tb, tb, generator=g) > 0.5
    kmask[:, :, -1] = True  # every row keeps at least one block
    out, lse = O.block_sparse_attention(q, k, v, kmask, 0.25)
    tok = torch.arange(n) // 128
    for b in range(banks):
        s = (q[b].double() @ k[b].double().T) * 0.25
        s = s.masked_fill(~kmask[b][tok][:, tok], -math.inf)
        torch.testing.assert_close(out[b].double(), torch.softmax(s, -1) @ v[b].double(),
                                   atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(lse[b].double(), torch.logsumexp(s, -1), atol=1e-5, rtol=1e-5)


@settings(**SETTINGS)
@given(st.integers(1, 4), st.integers(2, 40), st.integers(1, 40), st.integers(0, 2**31 - 1),
       st.integers(1, 4))
def test_topk_keeps_the_largest_with_ties_to_the_lower_index(rows, cols, keep, seed, levels):
    g = torch.Generator().manual_seed(seed)
    # few distinct levels force ties
    scores = torch.randint(0, levels, (rows, cols), generator=g).float()
    mask = O.topk_mask(scores, keep)
    k = max(1, min(keep, cols))
    for i in range(rows):
        order = sorted(range(cols), key=lambda j: (-scores[i, j].item(), j))
        assert set(torch.nonzero(mask[i]).flatten().tolist()) == set(order[:k])


@settings(**SETTINGS)
@given(st.integers(2, 30), st.integers(0, 2**31 - 1))
def test_attention_branch_merge_is_order_independent(n_keys, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(5, 8, generator=g, dtype=torch.float64)
    k = torch.randn(n_keys, 8, generator=g, dtype=torch.float64)
    v = torch.randn(n_keys, 8, generator=g, dtype=torch.float64)
    perm = torch.randperm(n_keys, generator=g)
    cuts = sorted(torch.randint(1, n_keys, (2,), generator=g).tolist())
    parts = [perm[:cuts[0]], perm[cuts[0]:cuts[1]], perm[cuts[1]:]]

    def branch(idx):
        s = q @ k[idx].T
        if idx.numel() == 0:
            return AttentionBranch(torch.zeros(5, 8, dtype=torch.float64),
                                   torch.full((5,), -math.inf, dtype=torch.float64))
        return AttentionBranch(torch.softmax(s, -1) @ v[idx], torch.logsumexp(s, -1))

    a, b, c = (branch(p) for p in parts)
    full = branch(torch.arange(n_keys))
    for merged in (a.merge(b).merge(c), c.merge(a.merge(b)), b.merge(c).merge(a)):
        torch.testing.assert_close(merged.output, full.output, atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(merged.lse.double(), full.lse, atol=1e-5, rtol=1e-5)
