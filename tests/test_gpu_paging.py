"""Host-bank paging in the combinations the reference's own profiles ship (every
recap/profiles/*.json sets host_banks): a per-prompt text length retargeted after the banks
were preallocated (HunyuanVideo, recap/models/hunyuan.py:30-39, 96-97, 296-302), host banks
with bank_chunks = 4 (the HunyuanVideo profiles), and two streams (Wan's two CFG calls per
step, recap/models/wan.py:22).  In each, paged outputs equal resident ones bit for bit."""

import dataclasses
import math

import pytest
import torch

from gpu_util import SMALL
from recap_amd import HostBankOperator, Operator, OperatorConfig, REFRESH, SPARSE
from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
from recap_amd.synthetic import make_qkv, perturb

pytestmark = pytest.mark.gpu


def _geometry(wl):
    perm = hilbert_permutation(wl.grid)
    layout = Layout.from_permutation(perm, text_tokens=wl.text_tokens, text_first=wl.text_first)
    return SparseGeometry.build(layout, 128)


def _pair(wl, geometry, *, layers, streams=1, chunks=1):
    """A resident and a paged operator over the same geometry (one shared layout, as the
    model integrations share it with their processors)."""
    cfg = OperatorConfig(head_density=wl.density, bank_chunks=chunks)
    resident = Operator.build(cfg, geometry, n_layers=layers, n_streams=streams)
    paged = HostBankOperator.build(dataclasses.replace(cfg, host_banks=True), geometry,
                                   n_layers=layers, n_streams=streams)
    return resident, paged


def _run_step(ops, step, kind, calls):
    """One computed step on every operator: calls = [(stream, layer, (q, k, v)), ...]; the
    outputs must agree bit for bit call by call."""
    for op in ops:
        op.begin_step(step, kind)
    for stream, layer, qkv in calls:
        outs = []
        for op in ops:
            op.set_stream(stream)
            outs.append(op.attend(layer, *qkv))
        for other in outs[1:]:
            assert torch.equal(outs[0], other), (step, kind, stream, layer)
    if kind == REFRESH:
        return [op.drain_validation() for op in ops]
    return None


def _tb(layout) -> int:
    return -(-layout.tokens // 128)


def test_text_retarget_after_preallocation(cuda):
    """The HunyuanVideo integration preallocates the host banks at install with the
    profile's text length (16) and retargets it per prompt after session.reset().  The
    kernel mask [banks, tb, tb] changes with tb = ceil((Nv + T) / 128): the pager takes the
    new field sizes, keeps host memory that is still large enough, and paged == resident
    over REFRESH/SPARSE before the retarget, after growing T across two block boundaries,
    and after shrinking it again."""
    base = SMALL["text-last-d128"]               # 3 heads x 128, 900 video tokens, text last
    layers = 2
    wl16 = dataclasses.replace(base, text_tokens=16)
    geometry = _geometry(wl16)
    layout = geometry.layout
    resident, paged = _pair(wl16, geometry, layers=layers)
    paged.set_prefetch(True)
    host0 = paged.preallocate_host(n_layers=layers, n_banks=wl16.heads, dim=wl16.dim)
    assert host0 > 0
    print(f"preallocated {host0} B at T=16 (tb={_tb(layout)})", flush=True)
    step = 0
    for text in (16, 256, 140):
        if text != layout.text_tokens:
            for op in (resident, paged):
                op.reset()
            layout.text_tokens = text                # recap/models/hunyuan.py:30-39
            layout._gather_cache.clear()
        wl = dataclasses.replace(base, text_tokens=text)
        q, k, v = make_qkv(wl, seed=text, device=cuda)
        schedule = [REFRESH, SPARSE, REFRESH, SPARSE]
        for i, kind in enumerate(schedule):
            inputs = tuple(perturb(x, 0.02, seed=j, step=i) for j, x in enumerate((q, k, v)))
            stats = _run_step((resident, paged), step, kind,
                              [(0, layer, inputs) for layer in range(layers)])
            if stats is not None:
                assert stats[0] == stats[1], (step, stats)
            if i == 2:
                assert stats[0] is not None and stats[0][0] == 2
            step += 1
        paged.finish()
        mask = paged.banks[0][0].head_kernel_mask
        assert mask is None  # the slots are unbound from the bank between calls
        print(f"  T={text} tb={_tb(layout)}: paged == resident, host bytes "
              f"{paged.peak_bank_bytes()}, counts {paged.pager_counts()}", flush=True)
        if text == 140:
            # shrinking the mask reuses the host memory allocated for T=256
            assert paged.peak_bank_bytes() == grown
        grown = paged.peak_bank_bytes()
    assert _tb(layout) == 9


def test_host_banks_with_bank_chunks(cuda):
    """host_banks together with bank_chunks = 4 (the HunyuanVideo profiles' combination)
    over REFRESH / SPARSE / REFRESH (validating) / SPARSE on two layers: paged head groups
    equal resident head groups, and both equal the whole-layer run, bit for bit (the
    whole layer's validation error within 1e-6 relative: its pairs add in another order)."""
    wl = dataclasses.replace(SMALL["text-last-d128"], heads=8)
    layers = 2
    geometry = _geometry(wl)
    resident, paged = _pair(wl, geometry, layers=layers, chunks=4)
    whole = Operator.build(OperatorConfig(head_density=wl.density), geometry, n_layers=layers)
    q, k, v = make_qkv(wl, seed=4, device=cuda)
    schedule = [REFRESH, SPARSE, REFRESH, SPARSE]
    for step, kind in enumerate(schedule):
        inputs = tuple(perturb(x, 0.03, seed=j, step=step) for j, x in enumerate((q, k, v)))
        stats = _run_step((whole, resident, paged), step, kind,
                          [(0, layer, inputs) for layer in range(layers)])
        if stats is not None:
            # paged and resident head groups validate identically; the whole layer adds the
            # same per-workgroup pairs in another order (the groups' sums are added last)
            assert stats[1] == stats[2], (step, stats)
            if stats[0] is not None:
                assert stats[0][0] == stats[1][0]
                assert abs(stats[0][1] - stats[1][1]) <= 1e-6 * stats[0][1], (step, stats)
        print(f"  step {step} {kind}: whole == chunks4 == chunks4+host", flush=True)
    paged.finish()
    counts = paged.pager_counts()
    print(f"  pager counts {counts}", flush=True)
    assert counts["written_back"] == layers * schedule.count(REFRESH)
    assert counts["copied"] == 0 and counts["from_prefetch"] == layers * (len(schedule) - 1)


@pytest.mark.parametrize("layers", [2, 3])
def test_host_banks_with_two_streams(cuda, layers):
    """Two streams (two CFG calls per step, run in turn: stream 0's layers, then stream 1's)
    with host banks, over REFRESH / SPARSE / SPARSE / REFRESH / SPARSE: paged == resident
    call by call with equal validations, and every stage-in is served by a prefetch, the
    layer 0 of each stream included (it is fetched during the other stream's last layer)."""
    wl = SMALL["video-ragged-d128"]
    geometry = _geometry(wl)
    resident, paged = _pair(wl, geometry, layers=layers, streams=2)
    per_stream = [make_qkv(wl, seed=20 + s, device=cuda) for s in range(2)]
    schedule = [REFRESH, SPARSE, SPARSE, REFRESH, SPARSE]
    for step, kind in enumerate(schedule):
        calls = []
        for s in range(2):
            inputs = tuple(perturb(x, 0.03, seed=10 * s + j, step=step)
                           for j, x in enumerate(per_stream[s]))
            calls += [(s, layer, inputs) for layer in range(layers)]
        stats = _run_step((resident, paged), step, kind, calls)
        if stats is not None:
            assert stats[0] == stats[1], (step, stats)
        print(f"  step {step} {kind}: paged == resident over 2 streams x {layers} layers",
              flush=True)
    paged.finish()
    counts = paged.pager_counts()
    print(f"  pager counts {counts}", flush=True)
    loads = 2 * layers * (len(schedule) - 1)
    assert counts["written_back"] == 2 * layers * schedule.count(REFRESH)
    assert counts["copied"] == 0 and counts["from_prefetch"] == loads


def test_timed_copies_fold_over_a_long_run(cuda):
    """With every bank copy timed (record_copies), a run of more than 64 copy batches keeps
    a bounded number of timing events (finished batches are folded into a running total as
    new ones start) and copy_time() reports every batch: stage-ins copied on the compute
    stream, prefetches and write-backs, with a positive total."""
    wl = SMALL["tiny"]
    geometry = _geometry(wl)
    layers = 2
    resident, paged = _pair(wl, geometry, layers=layers)
    paged.record_copies = True
    q, k, v = make_qkv(wl, seed=9, device=cuda)
    steps = 40
    for step in range(steps):
        kind = REFRESH if step % 10 == 0 else SPARSE
        inputs = tuple(perturb(x, 0.02, seed=j, step=step) for j, x in enumerate((q, k, v)))
        _run_step((resident, paged), step, kind, [(0, layer, inputs) for layer in range(layers)])
    paged.finish()
    counts = paged.pager_counts()
    ms, batches = paged.copy_time()
    print(f"  counts {counts}, timed batches {batches}, {ms:.3f} ms", flush=True)
    assert batches == counts["copied"] + counts["prefetches"] + counts["written_back"]
    assert batches > 64 and ms > 0
    assert paged.copy_time() == (ms, batches)   # folded batches are counted once


def test_host_banks_with_no_refined_rows(cuda):
    """A video of fewer than 128 tokens (100 video + 60 text): the paged bank's refinement
    fields are empty (zero bytes) and the kernel mask is the only field with data; paged ==
    resident over REFRESH / SPARSE / REFRESH / SPARSE on two layers, validations included."""
    from recap_amd.synthetic import Workload

    wl = Workload("short", 2, 64, (1, 5, 20), 60, False, 0.25, torch.bfloat16)
    geometry = _geometry(wl)
    layers = 2
    resident, paged = _pair(wl, geometry, layers=layers)
    q, k, v = make_qkv(wl, seed=3, device=cuda)
    schedule = [REFRESH, SPARSE, REFRESH, SPARSE]
    for step, kind in enumerate(schedule):
        inputs = tuple(perturb(x, 0.02, seed=j, step=step) for j, x in enumerate((q, k, v)))
        stats = _run_step((resident, paged), step, kind,
                          [(0, layer, inputs) for layer in range(layers)])
        if stats is not None and stats[0] is not None:
            assert stats[0] == stats[1], (step, stats)
            assert math.isinf(stats[0][1])
        print(f"  step {step} {kind}: paged == resident", flush=True)
    paged.finish()
    print(f"  pager counts {paged.pager_counts()}", flush=True)


@pytest.mark.parametrize("chunks", [1, 2])
def test_host_banks_with_batched_calls(cuda, chunks):
    """CFG-batched calls (batch 2, so banks = 2 x heads, as CogVideoX runs its two guidance
    branches in one call, recap/models/cogvideox.py:109) with host banks, with and without
    bank_chunks: paged == resident over REFRESH / SPARSE / REFRESH / SPARSE, validations
    included."""
    wl = SMALL["text-first-ragged"]
    geometry = _geometry(wl)
    layers = 2
    resident, paged = _pair(wl, geometry, layers=layers, chunks=chunks)
    q, k, v = make_qkv(wl, seed=7, batch=2, device=cuda)
    schedule = [REFRESH, SPARSE, REFRESH, SPARSE]
    for step, kind in enumerate(schedule):
        inputs = tuple(perturb(x, 0.03, seed=j, step=step) for j, x in enumerate((q, k, v)))
        stats = _run_step((resident, paged), step, kind,
                          [(0, layer, inputs) for layer in range(layers)])
        if stats is not None:
            assert stats[0] == stats[1], (step, stats)
        print(f"  step {step} {kind}: paged == resident (batch 2, chunks {chunks})", flush=True)
    paged.finish()
    counts = paged.pager_counts()
    print(f"  pager counts {counts}", flush=True)
    assert counts["copied"] == 0
