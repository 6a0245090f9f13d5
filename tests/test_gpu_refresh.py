"""The REFRESH side of the operator on the GPU: the refinement capture fed identical inputs
as the oracle's capture, the re-selection (rerank) branch of a revalidating refresh, and
the ten-step paged schedule at the HunyuanVideo-720p shape."""

import math

import pytest
import torch

import oracle as O
from gpu_util import SMALL, assert_parity, assert_sparse_parity, capture_inputs, ulp
from recap_amd import HostBankOperator, Operator, OperatorConfig, REFRESH, SPARSE
from recap_amd import kernels as K
from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
from recap_amd.synthetic import WORKLOADS, make_qkv, perturb

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,dtype,text_first,validate", [
    (128, torch.bfloat16, False, False), (128, torch.bfloat16, False, True),
    (64, torch.bfloat16, True, True), (64, torch.float16, True, False),
    (128, torch.float16, False, True)])
def test_refresh_capture_vs_oracle_identical_inputs(cuda, d, dtype, text_first, validate):
    """K.refresh_capture against O.refresh_detail on identical inputs (dense output and LSE,
    head branch, coarse tail, and for validation the old refinement with its drift inputs):
    D within its fp16 rounding plus the conditioning of (of - ratio oh) / (1 - ratio), DL
    within fp32 rounding, identical zeroed rows, validation sums within 1e-4 relative."""
    x = capture_inputs(d, dtype, text_first, seed=d + 7 * int(validate))
    print(f"case d={d} {dtype} text_first={text_first} validate={validate}", flush=True)
    banks, rows = x["oh"].shape[0], x["rows"]
    det = x["old"][0].clone() if validate else torch.zeros(banks, rows, d, dtype=torch.float16)
    dl = x["old"][1].clone() if validate else torch.zeros(banks, rows)
    det_g, dl_g = det.to(cuda), dl.to(cuda)
    geo = K.Geometry(x["n"], x["n_video"])
    glref, center = x["old"][2], x["old"][3]
    stats = K.refresh_capture(
        x["of"].to(cuda), x["lf"].reshape(banks, -1).contiguous().to(cuda), x["oh"].to(cuda),
        x["lh"].to(cuda), x["go"].to(cuda), x["gl"].to(cuda),
        torch.as_tensor(x["rowmap"]).to(cuda), geo, det_g, dl_g,
        glref=glref.to(cuda) if validate else None, center=center.to(cuda) if validate else None)
    old = (det.float(), dl, glref, center) if validate else None
    det_ref, dl_ref, stats_ref = O.refresh_detail(
        x["of"][0], x["lf"][0], x["oh"], x["lh"], x["go"].float(), x["gl"], x["perm"],
        x["offset"], old)
    det_got, dl_got = det_g.cpu().float(), dl_g.cpu()

    # ratio and its pieces, as the capture forms them (recap/kernels/detail_cache.py:76-86)
    native = x["offset"] + torch.as_tensor(x["perm"][:rows], dtype=torch.long)
    lf = x["lf"][0][:, native]
    ratio = torch.clamp_max(torch.exp(torch.clamp_max(x["lh"][:, :rows] - lf, 0.0)), 1 - 1e-6)
    of = x["of"][0][:, native].float()
    oh = x["oh"][:, :rows].float()
    zero_ref = ratio > 1.0 - 1.0e-3
    near = (ratio - (1.0 - 1.0e-3)).abs() < 4 * 2.0 ** -24
    zeroed_got = (det_got == 0).all(-1)
    print(f"  zeroed rows {int(zero_ref.sum())} of {zero_ref.numel()}, within 4 ulp of the "
          f"threshold {int(near.sum())}", flush=True)
    assert torch.equal(zeroed_got[~near], zero_ref[~near])
    assert torch.equal((det_ref == 0).all(-1)[~near], zero_ref[~near])
    # D: fp16 rounding of either side, plus the fp32 conditioning: d tail / d ratio =
    # (of - oh) / (1 - ratio)^2 times a few ulp of ratio, and a few ulp of |tail| + |go|.
    r = ratio.unsqueeze(-1)
    tail = (of - r * oh) / (1 - r)
    cond = 4e-7 * (of - oh).abs() * r / (1 - r) ** 2 + 1e-6 * (tail.abs() + x["go"].float().abs())
    bound = ulp(torch.maximum(det_got.abs(), det_ref.abs()), torch.float16) + cond
    live = ~(zero_ref | near).unsqueeze(-1)
    err = (det_got - det_ref).abs()
    worst = float(((err - bound) * live).max())
    print(f"  D max_abs {float(err[live.expand_as(err)].max()):.3e} worst-vs-bound {worst:+.3e}",
          flush=True)
    assert worst <= 0
    # DL: log(1 - ratio) carries ratio's relative error divided by 1 - ratio.
    dl_bound = 1e-5 + 4e-7 * ratio / (1 - ratio) + 2e-7 * (lf.abs() + x["gl"].abs())
    dl_err = (dl_got - dl_ref).abs()
    print(f"  DL max_abs {float(dl_err.max()):.3e} worst-vs-bound "
          f"{float((dl_err - dl_bound).max()):+.3e} clamped {int((dl_ref.abs() == 30).sum())}",
          flush=True)
    assert bool((dl_err <= dl_bound).all())
    assert int((dl_ref.abs() == 30).sum()) > 0
    if validate:
        got, want = stats.cpu().double(), stats_ref.double()
        rel = ((got - want).abs() / want.abs()).max()
        print(f"  validation sums gpu {got.tolist()} oracle {want.tolist()} rel {float(rel):.2e}",
              flush=True)
        assert float(rel) < 1e-4
    else:
        assert stats is None and stats_ref is None


def _build(wl, *, chunks=1, host_banks=False, layers=1, rerank=0.95):
    perm = hilbert_permutation(wl.grid)
    layout = Layout.from_permutation(perm, text_tokens=wl.text_tokens, text_first=wl.text_first)
    geo = SparseGeometry.build(layout, 128)
    cfg = OperatorConfig(head_density=wl.density, bank_chunks=chunks, host_banks=host_banks,
                         rerank_min_overlap=rerank)
    cls = HostBankOperator if host_banks else Operator
    return cls.build(cfg, geo, n_layers=layers), perm


def _inject(ref, op, wl):
    """Hand the GPU operator's layer-0 state to the oracle; with bank_chunks the basis is
    held by one state per head group, in bank order."""
    bank = op.banks[0][0]
    if op.config.bank_chunks > 1:
        groups = sorted(key for key in op._chunk_states if key[:2] == (0, 0))
        basis = torch.cat([op._chunk_states[key].basis for key in groups])
    else:
        basis = op.layers[0][0].basis
    nb = bank.partition.shape[-1]
    ref.load_state(0, basis=basis.cpu(), partition=bank.partition.reshape(-1, nb, nb).cpu(),
                   det=bank.value.cpu(), dl=bank.log_mass.cpu(), glref=bank.coarse_lse.cpu(),
                   n_tokens=wl.tokens)


@pytest.mark.parametrize("name,chunks", [("text-last-d128", 1), ("text-last-d128", 4),
                                         ("video-ragged-d128", 1), ("video-ragged-d128", 4),
                                         ("text-first-ragged", 1)])
def test_rerank_at_refresh_vs_oracle(cuda, name, chunks):
    """A revalidating refresh whose new selection overlaps the old one by less than
    rerank_min_overlap (1.0 here: any changed block) re-selects, recomputes the head and the
    coarse tail with the new partition and recaptures the refinement without validation
    (recap/operator.py:414-469; with bank_chunks the decision is made once for the layer,
    :283-292).  Checked against the oracle operator: the rerank decision, the new partition
    bit for bit, the dense output, the validation error (scored on the old split before the
    rerank), a sparse call on the same inputs reproducing the dense output, and the next
    sparse call on the GPU's state.  With bank_chunks = 4 everything equals the whole-layer
    run bit for bit."""
    wl = SMALL[name]
    print(f"case {name} bank_chunks={chunks}", flush=True)
    q, k, v = make_qkv(wl, seed=11)
    g = lambda t: t.to(cuda)  # noqa: E731
    runs = {}
    for c in sorted({1, chunks}):
        op, perm = _build(wl, chunks=c, rerank=1.0)
        ref = O.OracleOperator(wl.grid, wl.text_tokens, wl.text_first, wl.density,
                               rerank_min_overlap=1.0, permutation=perm)
        op.begin_step(0, REFRESH)
        op.attend(0, g(q), g(k), g(v))
        ref.refresh(0, q, k, v)
        old_part = op.banks[0][0].partition.clone()
        # K and V from another positional field than Q: the block scores lose their
        # diagonal, so the selection changes (i.i.d. noise would average out over a block's
        # 128 tokens, and a common field keeps every block's own neighbourhood on top).
        _, k2, v2 = make_qkv(wl, seed=12)
        q2 = q
        op.begin_step(2, REFRESH)
        dense = op.attend(0, g(q2), g(k2), g(v2))
        ref.refresh(0, q2, k2, v2)
        assert ref.last["rerank"] is True
        new_part = op.banks[0][0].partition
        assert not torch.equal(new_part, old_part)
        assert torch.equal(new_part.cpu().reshape(ref.layers[0].partition.shape),
                           ref.layers[0].partition)
        assert_parity(dense.cpu().float(), ref.last["out_f32"], f"rerank refresh {name} c{c}")
        age, error = op.drain_validation()
        num, den = (float(t) for t in ref.layers[0].pending_stats)
        print(f"  validation error gpu={error:.5f} oracle={math.sqrt(num / den):.5f}", flush=True)
        assert age == 2 and abs(error - math.sqrt(num / den)) < 2e-3
        # The recaptured refinement belongs to the new split: a sparse call on the refresh's
        # own inputs reproduces its dense output (drift weight 1, D exact up to fp16).
        op.begin_step(3, SPARSE)
        again = op.attend(0, g(q2), g(k2), g(v2))
        assert_parity(again.cpu().float(), dense.cpu().float(), f"rerank sparse==dense {name} c{c}")
        _inject(ref, op, wl)
        q4, k4, v4 = (perturb(x, 0.02, seed=5, step=4) for x in (q2, k2, v2))
        op.begin_step(4, SPARSE)
        out = op.attend(0, g(q4), g(k4), g(v4))
        ref.sparse(0, q4, k4, v4)
        assert_sparse_parity(out, ref, op, q4, k4, v4, wl, cuda, f"rerank next sparse {name} c{c}")
        bank = op.banks[0][0]
        runs[c] = (dense.cpu(), again.cpu(), out.cpu(), bank.value.cpu(), bank.log_mass.cpu(),
                   bank.partition.cpu(), error)
    if chunks > 1:
        for a, b in zip(runs[1][:-1], runs[chunks][:-1]):
            assert torch.equal(a, b)
        # the validation sums add the head groups' pairs in another order
        assert abs(runs[1][-1] - runs[chunks][-1]) <= 1e-6 * runs[1][-1]


def test_hunyuan_ten_step_paged_schedule(cuda):
    """The step sequence at the HunyuanVideo-720p shape: three layers (so the next step's
    layer-0 prefetch wraps around), REFRESH at steps 0 and 5 and SPARSE otherwise, 3% fresh
    input drift per step.  Refinement banks paged through pinned host memory give the same
    output as banks resident on the GPU, call by call, and the same step-5 validation."""
    wl = WORKLOADS["hunyuan-720p"]
    layers = 3
    schedule = [REFRESH] + [SPARSE] * 4 + [REFRESH] + [SPARSE] * 4
    base = make_qkv(wl, seed=0, device=cuda)
    resident, _ = _build(wl, layers=layers)
    paged, _ = _build(wl, layers=layers, host_banks=True)
    stats = {}
    for step, kind in enumerate(schedule):
        inputs = tuple(perturb(x, 0.03, seed=i, step=step) for i, x in enumerate(base))
        for op in (resident, paged):
            op.begin_step(step, kind)
        for layer in range(layers):
            a = resident.attend(layer, *inputs)
            b = paged.attend(layer, *inputs)
            assert torch.equal(a, b), (step, kind, layer)
        if kind == REFRESH:
            stats[step] = (resident.drain_validation(), paged.drain_validation())
        del inputs
        print(f"  step {step} {kind}: paged == resident over {layers} layers", flush=True)
    paged.finish()
    torch.cuda.synchronize()
    assert stats[0] == (None, None)
    (age_r, err_r), (age_p, err_p) = stats[5]
    print(f"  step-5 validation resident (age {age_r}, {err_r:.6f}) paged (age {age_p}, "
          f"{err_p:.6f})", flush=True)
    assert age_r == age_p == 5 and err_r == err_p and math.isfinite(err_r)
