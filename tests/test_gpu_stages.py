"""GPU parity of each HIP stage against the CPU oracle, on the same seeded inputs.

Masks, pooled means and block scores must be bit-exact; bf16 outputs within max-abs 2e-2
of the oracle's output rounded to bf16 (one bf16 ulp where that is larger, |x| >= 4) and
cosine >= 0.999; fp32 statistics within the tolerance stated per test."""

import math

import pytest
import torch

import oracle as O
from gpu_util import (SMALL, assert_parity, banks_view, k_tile_to_rows, metrics,
                      scale_for, vt_tile_to_rows)
from recap_amd import _lib
from recap_amd import kernels as K
from recap_amd.layout import Layout, hilbert_permutation
from recap_amd.synthetic import WORKLOADS, Workload, make_qkv

pytestmark = pytest.mark.gpu

STAGE1_CASES = [("tiny", None), ("text-first-ragged", None), ("text-last-d128", None),
                ("video-ragged-d128", None), ("wan2.1-480p", [0, 5]), ("cogvideox1.5", [0, 7]),
                ("hunyuan-720p", [0, 1])]


# A video-only shape whose rows hold 1,101 blocks: the coarse kernel scans partition rows of
# more than 1,024 blocks with its 16-chunk code.
LONG = {"long-row-d64": Workload("long-row-d64", 1, 64, (4, 35, 1006), 0, False, 0.25,
                                 torch.bfloat16),
        # 71 video blocks, the last one ragged (40 tokens)
        "mid-row-d128": Workload("mid-row-d128", 2, 128, (3, 25, 120), 0, False, 0.2,
                                 torch.bfloat16),
        # The largest shape the kernels take: 2,048 kernel blocks (the attention kernel's
        # kept list holds at most 2,048): 36 x 75 x 97 = 261,900 video tokens (2,047 blocks,
        # the last one 12 tokens, shared with the text) + 200 text tokens = 262,100.
        "max-blocks-d128": Workload("max-blocks-d128", 1, 128, (36, 75, 97), 200, False, 0.2,
                                    torch.bfloat16)}


def _setup(name, heads, cuda, seed=0, dtype=None, k_factors=None):
    """Inputs of workload ``name``; with ``k_factors``, the keys of reordered block i are
    scaled by ``k_factors[i % len(k_factors)]`` (in fp32, before the cast)."""
    wl = SMALL.get(name) or LONG.get(name) or WORKLOADS[name]
    dtype = dtype or (torch.bfloat16 if wl.dtype == torch.float32 else wl.dtype)
    print(f"case {name} heads={heads} N={wl.tokens} d={wl.dim} k_factors={k_factors}",
          flush=True)
    perm = hilbert_permutation(wl.grid)
    layout = Layout.from_permutation(perm, text_tokens=wl.text_tokens, text_first=wl.text_first)
    fwd, _ = O.gather_indices(perm, wl.text_tokens, wl.text_first)
    if k_factors is None:
        q, k, v = make_qkv(wl, heads=heads, seed=seed, dtype=dtype)
    else:
        q, k, v = make_qkv(wl, heads=heads, seed=seed, dtype=torch.float32)
        f = torch.tensor(k_factors)[(torch.arange(wl.tokens) // 128) % len(k_factors)]
        native = torch.empty(wl.tokens)
        native[fwd] = f
        k = k * native.view(1, 1, -1, 1)
        q, k, v = (x.to(dtype) for x in (q, k, v))
    geo = K.Geometry(wl.tokens, wl.video_tokens)
    return wl, (q, k, v), tuple(x.to(cuda) for x in (q, k, v)), layout.rowmap(cuda), fwd, geo


@pytest.mark.parametrize("name,heads", STAGE1_CASES)
def test_stage1_pool_scores_masks_bit_exact(cuda, name, heads):
    wl, (q, k, v), (qg, kg, vg), rowmap, fwd, geo = _setup(name, heads, cuda)
    ql, kl = banks_view(q, fwd), banks_view(k, fwd)
    kv = K.kv_pack(kg, vg, rowmap, geo)
    qm = K.pool_blocks(qg, rowmap, geo)
    qm_ref, _ = O.pool_blocks(ql, wl.video_tokens)
    km_ref, _ = O.pool_blocks(kl, wl.video_tokens)
    assert torch.equal(qm.cpu().view(torch.int32), qm_ref.view(torch.int32))
    assert torch.equal(kv.k_means.cpu().view(torch.int32), km_ref.view(torch.int32))
    vm_ref, _ = O.pool_blocks(banks_view(v, fwd), wl.video_tokens)
    assert torch.equal(kv.v_means.cpu().view(torch.int32), vm_ref.view(torch.int32))
    scale = scale_for(wl.dim)
    scores = K.block_scores(qm, kv.k_means, scale)
    scores_ref = O.block_scores(qm_ref, km_ref, scale)
    assert torch.equal(scores.cpu().view(torch.int32), scores_ref.view(torch.int32))
    part = K.select_blocks(qg, kv.k_means, rowmap, geo, wl.density, scale)
    part_ref = O.head_partition(ql, kl, scale, wl.density, wl.video_tokens)
    keep = max(1, round(wl.density * geo.nb))
    print(f"  top-k margin {O.topk_margin(scores_ref, keep):.3e}", flush=True)
    assert torch.equal(part.cpu(), part_ref)
    kmask = K.kernel_block_mask(part, geo)
    assert torch.equal(kmask.cpu(), O.kernel_block_mask(part_ref, wl.tokens, wl.video_tokens))
    # the one-call stage 1 gives the same partition and kernel mask
    part1, kmask1 = K.pool_select(qg, kv.k_means, rowmap, geo, wl.density, scale)
    assert torch.equal(part1, part) and torch.equal(kmask1, kmask)


@pytest.mark.parametrize("nb", [1, 63, 64, 65, 256, 257, 929, 1024, 1025, 4096])
def test_topk_radix_select_with_ties_vs_oracle(cuda, nb):
    """The radix-select top-k against the oracle's stable sort on rows built to tie: plain
    normal scores, a handful of integer values, fully tied rows, signed zeros among tiny
    values; random keep, the forced partial block on and off; every size class of the
    kernel (up to 256, 1024 and 4096 blocks per row)."""
    g = torch.Generator().manual_seed(nb)
    banks = 3
    scores = torch.randn(banks, nb, nb, generator=g)
    scores[0, ::3] = torch.randint(-3, 3, (len(range(0, nb, 3)), nb), generator=g).float()
    scores[1, ::4] = 1.5
    tiny = torch.randn(nb, generator=g) * 1e-30
    tiny[::5] = 0.0
    tiny[1::7] = -0.0
    scores[2, ::2] = tiny
    for keep in sorted({1, max(1, nb // 5), max(1, nb // 2), nb}):
        for force_last in (False, True):
            got = K.topk_blocks(scores.to(cuda), keep, force_last).cpu()
            want = O.topk_mask(scores, keep)
            if force_last:
                want[:, :, -1] = True
                want[:, -1, :] = True
            assert torch.equal(got, want), (nb, keep, force_last)


@pytest.mark.parametrize("name", list(SMALL))
def test_kv_pack_tile_images(cuda, name):
    wl, (q, k, v), (qg, kg, vg), rowmap, fwd, geo = _setup(name, None, cuda)
    kv = K.kv_pack(kg, vg, rowmap, geo)
    kl, vl = banks_view(k, fwd), banks_view(v, fwd)
    kt, vt = kv.k_tiles.cpu(), kv.vt_tiles.cpu()
    n = wl.tokens
    for bank in range(kl.shape[0]):
        for tile in sorted({0, geo.tb // 2, geo.tb - 1}):
            rows = min(128, n - 128 * tile)
            krows = k_tile_to_rows(kt[bank, tile], wl.dim)
            vrows = vt_tile_to_rows(vt[bank, tile], wl.dim)
            assert torch.equal(krows[:rows], kl[bank, 128 * tile:128 * tile + rows])
            assert torch.equal(vrows[:rows], vl[bank, 128 * tile:128 * tile + rows])
            assert not krows[rows:].any() and not vrows[rows:].any()


@pytest.mark.parametrize("name", list(SMALL))
def test_head_and_dense_attention(cuda, name):
    wl, (q, k, v), (qg, kg, vg), rowmap, fwd, geo = _setup(name, None, cuda)
    scale = scale_for(wl.dim)
    kv = K.kv_pack(kg, vg, rowmap, geo)
    ql, kl, vl = (banks_view(x, fwd) for x in (q, k, v))
    part_ref = O.head_partition(ql, kl, scale, wl.density, wl.video_tokens)
    kmask_ref = O.kernel_block_mask(part_ref, wl.tokens, wl.video_tokens)
    out, lse = K.block_sparse_attn(qg, kv, rowmap, kmask_ref.to(cuda), geo, scale)
    ref, ref_lse = O.block_sparse_attention(ql, kl, vl, kmask_ref, scale)
    assert_parity(out.cpu().float(), ref, f"head {name}")
    m, _ = metrics(lse.cpu(), ref_lse)
    assert m < 2e-3, m
    dense, dlse = K.dense_attn(qg, kv, rowmap, scale)
    dref, dref_lse = O.dense_attention(ql, kl, vl, scale)
    _, inv = O.gather_indices(hilbert_permutation(wl.grid), wl.text_tokens, wl.text_first)
    b, h = q.shape[:2]
    assert_parity(dense.cpu().float(), O.restore(dref.reshape(b, h, -1, wl.dim), inv),
                      f"dense {name}")
    m, _ = metrics(dlse.cpu(), dref_lse.reshape(b, h, -1).index_select(-1, inv))
    assert m < 2e-3, m


@pytest.mark.parametrize("name", list(SMALL))
def test_dense_head_attention_one_pass(cuda, name):
    """The refresh's fused pass: its dense part against the oracle's dense attention and the
    dense kernel, its head part (stored mid-walk) against the oracle's block-sparse attention
    and the head kernel, for masks whose kept ragged block goes first."""
    wl, (q, k, v), (qg, kg, vg), rowmap, fwd, geo = _setup(name, None, cuda)
    scale = scale_for(wl.dim)
    kv = K.kv_pack(kg, vg, rowmap, geo)
    ql, kl, vl = (banks_view(x, fwd) for x in (q, k, v))
    part_ref = O.head_partition(ql, kl, scale, wl.density, wl.video_tokens)
    kmask_ref = O.kernel_block_mask(part_ref, wl.tokens, wl.video_tokens)
    dense, dlse, hout, hlse = K.dense_head_attn(qg, kv, rowmap, kmask_ref.to(cuda), scale)
    ref, ref_lse = O.block_sparse_attention(ql, kl, vl, kmask_ref, scale)
    assert_parity(hout.cpu().float(), ref, f"fused head {name}")
    m, _ = metrics(hlse.cpu(), ref_lse)
    assert m < 2e-3, m
    # Same kept blocks in the same order (a kept ragged block first in both), and the head
    # branch is stored before the first block after the kept ones can move the running max:
    # the head branch equals the head kernel's bit for bit.
    alone, alone_lse = K.block_sparse_attn(qg, kv, rowmap, kmask_ref.to(cuda), geo, scale)
    assert torch.equal(hout, alone)
    assert torch.equal(hlse, alone_lse)
    dref, dref_lse = O.dense_attention(ql, kl, vl, scale)
    _, inv = O.gather_indices(hilbert_permutation(wl.grid), wl.text_tokens, wl.text_first)
    b, h = q.shape[:2]
    assert_parity(dense.cpu().float(), O.restore(dref.reshape(b, h, -1, wl.dim), inv),
                      f"fused dense {name}")
    m, _ = metrics(dlse.cpu(), dref_lse.reshape(b, h, -1).index_select(-1, inv))
    assert m < 2e-3, m
    dense2, dlse2 = K.dense_attn(qg, kv, rowmap, scale)
    assert float((dense.float() - dense2.float()).abs().max()) <= 2e-2
    assert float((dlse - dlse2).abs().max()) < 1e-4


@pytest.mark.parametrize("n,d,keep_last", [(100, 64, True), (200, 128, True), (200, 128, False),
                                          (300, 64, False), (384, 128, True), (700, 128, False)])
def test_attention_modes_short_and_ragged(cuda, n, d, keep_last):
    """Head, dense, dense-head and merge modes on one to six blocks, with the ragged last
    block kept (walked first) or not kept (walked last in dense-head mode), against the
    oracle."""
    print(f"case n={n} d={d} keep_last={keep_last}", flush=True)
    g = torch.Generator().manual_seed(n + d)
    banks, tb = 2, -(-n // 128)
    q, k, v = (torch.randn(1, banks, n, d, generator=g).to(torch.bfloat16) for _ in range(3))
    kmask = torch.rand(banks, tb, tb, generator=g) > 0.5
    kmask[:, torch.arange(tb), torch.arange(tb)] = True
    kmask[:, :, -1] = keep_last
    if not keep_last:
        kmask[:, -1, -1] = True   # the last row keeps at least its own block
    geo = K.Geometry(n, n)
    rowmap = torch.arange(n, dtype=torch.int32, device=cuda)
    kv = K.kv_pack(k.to(cuda), v.to(cuda), rowmap, geo)
    scale = scale_for(d)
    ql, kl, vl = (x[0].float() for x in (q, k, v))
    ref, ref_lse = O.block_sparse_attention(ql, kl, vl, kmask, scale)
    dref, dref_lse = O.dense_attention(ql, kl, vl, scale)
    head, head_lse = K.block_sparse_attn(q.to(cuda), kv, rowmap, kmask.to(cuda), geo, scale)
    assert_parity(head.cpu().float(), ref, "head")
    dense, dlse = K.dense_attn(q.to(cuda), kv, rowmap, scale)
    assert_parity(dense.cpu().float()[0], dref, "dense")
    fd, flse, fh, fhlse = K.dense_head_attn(q.to(cuda), kv, rowmap, kmask.to(cuda), scale)
    assert_parity(fh.cpu().float(), ref, "dense-head: head")
    assert_parity(fd.cpu().float()[0], dref, "dense-head: dense")
    # One walk order for every masked mode: the head branch of the dense-head pass and the
    # head the merge epilogue uses are the head kernel's, bit for bit.  With fewer than 128
    # video tokens no row is refined (R = 0), so the merge output is the head itself.
    assert torch.equal(fh, head) and torch.equal(fhlse, head_lse)
    merged = K.sparse_merge_attn(q.to(cuda), kv, rowmap, kmask.to(cuda),
                                 K.Geometry(n, min(n, 100)), scale, None, None, None, None,
                                 None, None)
    assert torch.equal(merged[0], head)
    for got, want in ((head_lse, ref_lse), (fhlse, ref_lse), (dlse[0], dref_lse),
                      (flse[0], dref_lse)):
        m, _ = metrics(got.cpu(), want)
        assert m < 2e-3, m


@pytest.mark.parametrize("d", [64, 128])
def test_attention_running_max_jumps(cuda, d):
    """Keys of each 64-key sub-tile scaled by factors from 0.1 to 80, so that a row's scores
    rise by tens of log2 units between sub-tiles (and fall): the lazy running max (d = 128),
    the probability-sum check with its redo (d = 64), and the dense-head pass's head snapshot
    in the middle of such a walk, in head, dense and dense-head modes against the oracle."""
    n, banks = 1000, 2
    print(f"case n={n} d={d}", flush=True)
    g = torch.Generator().manual_seed(17 + d)
    tb = -(-n // 128)
    q, k, v = (torch.randn(1, banks, n, d, generator=g) for _ in range(3))
    factors = torch.tensor([1.0, 8.0, 0.25, 24.0, 2.0, 40.0, 0.5, 12.0, 3.0, 60.0, 1.0, 0.1,
                            16.0, 5.0, 80.0, 1.0])
    k = k * factors[torch.arange(n) // 64].view(1, 1, n, 1)
    q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    kmask = torch.rand(banks, tb, tb, generator=g) > 0.4
    kmask[:, torch.arange(tb), torch.arange(tb)] = True
    geo = K.Geometry(n, n)
    rowmap = torch.arange(n, dtype=torch.int32, device=cuda)
    kv = K.kv_pack(k.to(cuda), v.to(cuda), rowmap, geo)
    scale = scale_for(d)
    ql, kl, vl = (x[0].float() for x in (q, k, v))
    ref, ref_lse = O.block_sparse_attention(ql, kl, vl, kmask, scale)
    dref, dref_lse = O.dense_attention(ql, kl, vl, scale)
    head, head_lse = K.block_sparse_attn(q.to(cuda), kv, rowmap, kmask.to(cuda), geo, scale)
    assert_parity(head.cpu().float(), ref, "head")
    dense, dlse = K.dense_attn(q.to(cuda), kv, rowmap, scale)
    assert_parity(dense.cpu().float()[0], dref, "dense")
    fd, flse, fh, fhlse = K.dense_head_attn(q.to(cuda), kv, rowmap, kmask.to(cuda), scale)
    assert torch.equal(fh, head) and torch.equal(fhlse, head_lse)
    assert_parity(fd.cpu().float()[0], dref, "dense-head: dense")
    for got, want in ((head_lse, ref_lse), (dlse[0], dref_lse), (flse[0], dref_lse)):
        # the scores reach a few hundred: fp32 accumulation of their products
        err = (got.cpu().double() - want.double()).abs()
        bound = 2e-3 + 1e-5 * want.double().abs()
        print(f"  lse max-abs {float(err.max()):.3e} (|lse| up to "
              f"{float(want.abs().max()):.1f})", flush=True)
        assert bool((err <= bound).all()), float((err - bound).max())


def test_dense_attention_matches_torch_sdpa(cuda):
    wl = SMALL["text-last-d128"]
    q, k, v = (x.to(cuda) for x in make_qkv(wl, seed=1))
    layout = Layout.from_permutation(hilbert_permutation(wl.grid), text_tokens=wl.text_tokens,
                                     text_first=False)
    rowmap = layout.rowmap(cuda)
    geo = K.Geometry(wl.tokens, wl.video_tokens)
    kv = K.kv_pack(k, v, rowmap, geo)
    out, _ = K.dense_attn(q, kv, rowmap, scale_for(wl.dim))
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    assert_parity(out.float(), ref, "dense vs sdpa fp32")


@pytest.mark.parametrize("name", ["tiny", "text-last-d128", "video-ragged-d128"])
@pytest.mark.parametrize("group", [None, 3, 8])
def test_closure_statistics(cuda, name, group):
    """The three flag sets of the closure kernel against the oracle and each other, with
    the default blocks per workgroup (one at these sizes) and with groups of 3 and 8 (a
    partial last group, several blocks streamed through the kernel's four LDS slots)."""
    wl, (q, k, v), (qg, kg, vg), rowmap, fwd, geo = _setup(name, None, cuda)
    print(f"  group {group}", flush=True)
    kv = K.kv_pack(kg, vg, rowmap, geo)
    kl, vl = banks_view(k, fwd), banks_view(v, fwd)
    km_ref, counts = O.pool_blocks(kl, wl.video_tokens)
    _, cvk, scatter = K.closure_stats(kv, geo, _lib.CLOSURE_CVK | _lib.CLOSURE_SCATTER,
                                      group=group)
    scatter_ref = O.within_block_scatter(kl, km_ref, counts, wl.video_tokens)
    cvk_ref = O.value_key_covariance(kl, vl, km_ref, counts, wl.video_tokens)
    rel = float((scatter.cpu() - scatter_ref).abs().max() / scatter_ref.abs().max())
    print(f"  scatter rel {rel:.2e}", flush=True)
    assert rel < 1e-4
    m, c = metrics(cvk.cpu(), cvk_ref)
    print(f"  cvk max_abs {m:.2e} cos {c:.6f}", flush=True)
    assert m < 1e-4 * max(1.0, float(cvk_ref.abs().max()))
    basis = O.closure_basis(scatter_ref)
    split = K.basis_tables(basis.to(cuda), None, kv.dtype, split=True)
    var, cvk2, _ = K.closure_stats(kv, geo, _lib.CLOSURE_ROT | _lib.CLOSURE_CVK, split.u_hi_t,
                                   split.u_lo_t, group=group)
    assert torch.equal(cvk2, cvk)
    var_only, _, _ = K.closure_stats(kv, geo, _lib.CLOSURE_ROT, split.u_hi_t, split.u_lo_t,
                                     group=group)
    assert torch.equal(var_only, var)
    if group is not None:  # the variances do not depend on the grouping at all
        var1, _, _ = K.closure_stats(kv, geo, _lib.CLOSURE_ROT, split.u_hi_t, split.u_lo_t,
                                     group=1)
        assert torch.equal(var1, var)
    _, var_ref = O.rotated_moments(kl, basis, counts, wl.video_tokens)
    rel = float(((var.cpu() - var_ref).abs() / (var_ref.abs() + 1e-3)).max())
    print(f"  rotated variance rel {rel:.2e}", flush=True)
    assert rel < 1e-3


@pytest.mark.parametrize("name,rank", [("tiny", 4), ("text-first-ragged", 4),
                                       ("text-last-d128", 4), ("video-ragged-d128", 4),
                                       ("text-last-d128", 0), ("text-last-d128", 13),
                                       ("video-ragged-d128", 20), ("long-row-d64", 4)])
def test_coarse_tail(cuda, name, rank):
    """The coarse kernel against the oracle fed with the same closure statistics.  Ranks
    1-13 take the folded w table (16 features) in bf16, the others the full one."""
    _check_coarse_tail(cuda, name, rank)


@pytest.mark.parametrize("name", ["mid-row-d128", "long-row-d64"])
def test_coarse_tail_score_jumps(cuda, name):
    """Keys of each block scaled by factors from 0.5 to 10, so that the coarse scores jump by
    tens of log2 units between tiles of omitted blocks, up and down: the probability-sum
    check and its redo under a raised running max, against the oracle."""
    _check_coarse_tail(cuda, name, 4, k_factors=(1.0, 3.0, 0.5, 6.0, 1.5, 10.0, 0.75, 4.0))


def _rows_of(blocks, n):
    return torch.cat([torch.arange(128 * i, min(128 * (i + 1), n)) for i in blocks])


def test_max_blocks_stage1_and_attention(cuda):
    """The largest shape the kernels take: 2,048 kernel blocks, one head of d = 128, the text
    sharing the ragged last video block.  Stage 1 bit-exact in full (2,047 x 2,047 block
    scores); the head and dense attention against the oracle on sampled query blocks: the
    first, a middle one, the last full video block, the ragged shared block and the text
    block (both dense rows: the text block walks all 2,048 key tiles, the kept list's
    capacity)."""
    wl, (q, k, v), (qg, kg, vg), rowmap, fwd, geo = _setup("max-blocks-d128", None, cuda)
    assert geo.tb == 2048 and geo.nb == 2047
    scale = scale_for(wl.dim)
    kv = K.kv_pack(kg, vg, rowmap, geo)
    ql, kl, vl = (banks_view(x, fwd) for x in (q, k, v))
    part, kmask = K.pool_select(qg, kv.k_means, rowmap, geo, wl.density, scale)
    part_ref = O.head_partition(ql, kl, scale, wl.density, wl.video_tokens)
    kmask_ref = O.kernel_block_mask(part_ref, wl.tokens, wl.video_tokens)
    assert torch.equal(part.cpu(), part_ref) and torch.equal(kmask.cpu(), kmask_ref)
    print(f"  partition and kernel mask bit-exact; kept per video row "
          f"{int(part_ref[0, 0].sum())}, text row {int(kmask_ref[0, -1].sum())}", flush=True)
    blocks = [0, geo.nb // 2, geo.ds - 1, geo.nb - 1, geo.tb - 1]
    rows = _rows_of(blocks, wl.tokens)
    out, lse = K.block_sparse_attn(qg, kv, rowmap, kmask, geo, scale)
    ref, ref_lse = O.block_sparse_attention(ql, kl, vl, kmask_ref, scale, query_blocks=blocks)
    assert_parity(out.cpu().float()[:, rows], ref[:, rows], "head, 2,048 blocks")
    m, _ = metrics(lse.cpu()[:, rows], ref_lse[:, rows])
    assert m < 2e-3, m
    dense, dlse = K.dense_attn(qg, kv, rowmap, scale)
    dblocks = [0, geo.tb - 1]
    drows = _rows_of(dblocks, wl.tokens)
    dref, dref_lse = O.dense_attention(ql, kl, vl, scale, query_blocks=dblocks)
    native = torch.as_tensor(fwd, dtype=torch.long)[drows]
    got = dense.cpu().float().reshape(1, wl.tokens, wl.dim)[:, native]
    assert_parity(got, dref[:, drows], "dense, 2,048 blocks")
    m, _ = metrics(dlse.cpu().reshape(1, wl.tokens)[:, native], dref_lse[:, drows])
    assert m < 2e-3, m


def test_max_blocks_coarse_tail_sampled(cuda):
    """The coarse kernel at 2,048 kernel blocks (rows of ~1,640 omitted blocks, 52 tiles)
    against the oracle on the first, a middle and the last full video block."""
    _check_coarse_tail(cuda, "max-blocks-d128", 4, blocks=[0, 1023, 2045])


def test_max_blocks_refresh_then_sparse_reproduces_dense(cuda):
    """The whole operator at 2,048 kernel blocks: the refresh's dense output against torch
    SDPA, and a sparse call on the refresh's own inputs reproduces it (the refinement holds
    exactly what the head and coarse tail miss)."""
    from recap_amd import REFRESH, SPARSE, Operator, OperatorConfig
    from recap_amd.layout import SparseGeometry

    wl = LONG["max-blocks-d128"]
    perm = hilbert_permutation(wl.grid)
    layout = Layout.from_permutation(perm, text_tokens=wl.text_tokens, text_first=wl.text_first)
    op = Operator.build(OperatorConfig(head_density=wl.density),
                        SparseGeometry.build(layout, 128), n_layers=1)
    q, k, v = make_qkv(wl, seed=0, device=cuda)
    op.begin_step(0, REFRESH)
    dense = op.attend(0, q, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    assert_parity(dense.float(), ref, "dense vs sdpa, 2,048 blocks")
    op.begin_step(1, SPARSE)
    sparse = op.attend(0, q, k, v)
    assert_parity(sparse.float(), dense.float(), "refresh -> sparse == dense, 2,048 blocks")


def _check_coarse_tail(cuda, name, rank, k_factors=None, blocks=None):
    """The coarse kernel against the oracle on the same closure statistics, on every row or
    (``blocks``) on the rows of those query blocks."""
    wl, (q, k, v), (qg, kg, vg), rowmap, fwd, geo = _setup(name, None, cuda,
                                                          k_factors=k_factors)
    scale = scale_for(wl.dim)
    kv = K.kv_pack(kg, vg, rowmap, geo)
    ql, kl, vl = (banks_view(x, fwd) for x in (q, k, v))
    km_ref, counts = O.pool_blocks(kl, wl.video_tokens)
    vm_ref, _ = O.pool_blocks(vl, wl.video_tokens)
    scatter = O.within_block_scatter(kl, km_ref, counts, wl.video_tokens)
    basis = O.closure_basis(scatter)
    _, var = O.rotated_moments(kl, basis, counts, wl.video_tokens)
    basis, var = O.order_basis(basis, var, counts)
    cvk = O.value_key_covariance(kl, vl, km_ref, counts, wl.video_tokens)
    w = O.fold_rank(var, rank)
    part = O.head_partition(ql, kl, scale, wl.density, wl.video_tokens)
    qv = ql[:, :wl.video_tokens].float()
    qsq = O.rotated_query_square(qv, basis, torch.bfloat16)
    drift = O.value_drift(qv, cvk, scale, torch.bfloat16)
    go_ref, gl_ref = O.coarse_tail(ql, qsq, drift, km_ref, vm_ref, w, counts, part, scale, 2.0,
                                   wl.video_tokens, torch.bfloat16, query_blocks=blocks)
    rows = geo.rows
    sel = (torch.arange(rows) if blocks is None else
           torch.cat([torch.arange(128 * i, min(128 * (i + 1), rows)) for i in blocks]))
    qt = K.basis_tables(basis.to(cuda), cvk.to(cuda), kv.dtype, query=True, cvk_table=True)
    wt, kbar, vbar = K.coarse_tables(var.to(cuda), kv, rank)
    assert wt.shape[-1] == (16 if 1 <= rank <= 13 and kv.dtype == torch.bfloat16 else wl.dim)
    nb = kv.k_means.shape[1]  # one table row per key block, zero rows after the last
    for table, means in ((kbar, kv.k_means), (vbar, kv.v_means)):
        assert torch.equal(table[:, :nb], means.to(kv.dtype)), f"table rows {name}"
        assert not table[:, nb:].any()
    assert not wt[:, nb:].any()
    tables = {"w": wt, "kbar": kbar, "vbar": vbar, "u_t": qt.u_t, "cvk_t": qt.cvk_t,
              "rank": rank}
    glref = torch.randn(kl.shape[0], rows, generator=torch.Generator().manual_seed(3)).to(cuda)
    go, gl, dpart = K.coarse_tail(qg, rowmap, part.to(cuda), geo, tables, scale, 2.0, glref)
    assert_parity(go.cpu().float()[:, sel], go_ref[:, sel], f"coarse {name}")
    gl_s = gl.cpu()[:, sel]
    fin = torch.isfinite(gl_ref[:, sel])
    assert torch.equal(torch.isfinite(gl_s), fin)
    err = torch.where(fin, (gl_s - gl_ref[:, sel]).abs(), torch.zeros(()))
    bad = err > 2e-3
    if bad.any():
        # The gate fl(s^2 qsq.w) <= theta^2 is discontinuous: the other decision moves a
        # block's logit by up to theta^2 / 2.  Two causes can flip it, and a row that differs
        # must match the oracle under one of them, for its query blocks:
        # (a) two fp32 summation orders of qsq.w (~1e-7 relative) on a pair at the threshold:
        #     theta^2 moved by 1e-5 one way or the other;
        # (b) qsq itself: the reference's U^T q is a bf16 GEMM whose fp32 accumulation order
        #     is open (recap/sparse/closure.py:84-86), and one element of it can round to the
        #     neighbouring bf16 value; qsq from an MFMA-accumulated GEMM on the GPU.
        bad_blocks = sorted({int(sel[r]) // 128 for r in torch.nonzero(bad.any(0)).flatten()})
        ub = O.cast(basis, torch.bfloat16).to(torch.bfloat16).to(cuda)
        rot = torch.stack([qv[i].to(torch.bfloat16).to(cuda) @ ub[i].contiguous()
                           for i in range(qv.shape[0])]).float().cpu()
        qsq_gemm = O.cast(rot * rot, torch.bfloat16)
        rel = 1e-5
        alternates = [(qsq, 2.0 * math.sqrt(1.0 + rel)), (qsq, 2.0 * math.sqrt(1.0 - rel)),
                      (qsq_gemm, 2.0)]
        best = torch.full_like(err, math.inf)
        for qsq_alt, th in alternates:
            _, gl_alt = O.coarse_tail(ql, qsq_alt, drift, km_ref, vm_ref, w, counts, part, scale,
                                      th, wl.video_tokens, torch.bfloat16,
                                      query_blocks=bad_blocks)
            best = torch.minimum(best, (gl_s - gl_alt[:, sel]).abs())
        print(f"  gl: {int(bad.sum())} rows over 2e-3 (max {float(err.max()):.3e}); against "
              f"the gate and qsq alternates max {float(best[bad].max()):.3e}", flush=True)
        assert float(best[bad].max()) < 2e-3, float(best[bad].max())
    center = K.drift_center(dpart, geo)
    cref = O.drift_center(gl.cpu(), glref.cpu())
    assert torch.allclose(center.cpu(), cref, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("name", ["tiny", "text-last-d128", "mid-row-d128"])
def test_coarse_tail_extreme_partitions(cuda, name):
    """The coarse kernel on partitions the selection never makes but the kernel must take:
    query blocks that keep every block (no tail: output 0, LSE -inf), that keep only
    themselves (every other block omitted, the last one ragged), that omit 1 to 40 blocks
    (a partial tile, a full one, one more), against the oracle on the same partition."""
    wl, (q, k, v), (qg, kg, vg), rowmap, fwd, geo = _setup(name, None, cuda)
    scale, rank = scale_for(wl.dim), 4
    kv = K.kv_pack(kg, vg, rowmap, geo)
    ql, kl, vl = (banks_view(x, fwd) for x in (q, k, v))
    km_ref, counts = O.pool_blocks(kl, wl.video_tokens)
    vm_ref, _ = O.pool_blocks(vl, wl.video_tokens)
    basis = O.closure_basis(O.within_block_scatter(kl, km_ref, counts, wl.video_tokens))
    _, var = O.rotated_moments(kl, basis, counts, wl.video_tokens)
    basis, var = O.order_basis(basis, var, counts)
    cvk = O.value_key_covariance(kl, vl, km_ref, counts, wl.video_tokens)
    w = O.fold_rank(var, rank)
    nb = km_ref.shape[1]
    part = O.head_partition(ql, kl, scale, wl.density, wl.video_tokens).clone()
    g = torch.Generator().manual_seed(11)
    for i in range(nb):
        kind = i % 4
        if kind == 0:
            part[:, i] = True                               # nothing omitted
        elif kind == 1:
            part[:, i] = False
            part[:, i, i] = True                            # all but the block itself
        elif kind == 2:
            part[:, i] = True
            n_om = min((1, 2, 31, 32, 33, 40)[(i // 4) % 6], nb - 1)
            omit = torch.randperm(nb, generator=g)[:n_om]
            part[:, i, omit] = False                        # 1 .. 40 omitted
    qv = ql[:, :wl.video_tokens].float()
    qsq = O.rotated_query_square(qv, basis, torch.bfloat16)
    drift = O.value_drift(qv, cvk, scale, torch.bfloat16)
    go_ref, gl_ref = O.coarse_tail(ql, qsq, drift, km_ref, vm_ref, w, counts, part, scale, 2.0,
                                   wl.video_tokens, torch.bfloat16)
    rows = geo.rows
    qt = K.basis_tables(basis.to(cuda), cvk.to(cuda), kv.dtype, query=True, cvk_table=True)
    wt, kbar, vbar = K.coarse_tables(var.to(cuda), kv, rank)
    tables = {"w": wt, "kbar": kbar, "vbar": vbar, "u_t": qt.u_t, "cvk_t": qt.cvk_t,
              "rank": rank}
    glref = torch.zeros(kl.shape[0], rows, device=cuda)
    go, gl, _ = K.coarse_tail(qg, rowmap, part.to(cuda), geo, tables, scale, 2.0, glref)
    assert_parity(go.cpu().float(), go_ref[:, :rows], f"coarse extreme {name}")
    fin = torch.isfinite(gl_ref[:, :rows])
    assert torch.equal(torch.isfinite(gl.cpu()), fin)
    empty = ~(~part).any(-1)                                # [banks, nb] query blocks, no tail
    erows = empty.repeat_interleave(128, dim=1)[:, :rows]
    assert erows.any() and not fin[erows].any()
    assert not go.cpu()[erows].any()
    m, _ = metrics(gl.cpu()[fin], gl_ref[:, :rows][fin])
    assert m < 2e-3, m
