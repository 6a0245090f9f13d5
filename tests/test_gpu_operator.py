"""The whole operator on the GPU: REFRESH and SPARSE calls against the oracle operator at
small shapes, and size-independent properties at the full HunyuanVideo-720p shape."""

import math

import pytest
import torch

import oracle as O
from gpu_util import SMALL, assert_close_bf16, metrics
from recap_amd import HostBankOperator, Operator, OperatorConfig, REFRESH, SPARSE
from recap_amd.layout import Layout, SparseGeometry, hilbert_permutation
from recap_amd.synthetic import WORKLOADS, make_qkv, perturb

pytestmark = pytest.mark.gpu


def build(wl, *, chunks=1, host_banks=False, prefetch=True, layers=2):
    perm = hilbert_permutation(wl.grid)
    layout = Layout.from_permutation(perm, text_tokens=wl.text_tokens, text_first=wl.text_first)
    geo = SparseGeometry.build(layout, 128)
    cfg = OperatorConfig(head_density=wl.density, bank_chunks=chunks, host_banks=host_banks)
    cls = HostBankOperator if host_banks else Operator
    op = cls.build(cfg, geo, n_layers=layers)
    if host_banks:
        op.set_prefetch(prefetch)
    return op, perm


@pytest.mark.parametrize("name", list(SMALL))
def test_refresh_sparse_sequence_vs_oracle(cuda, name):
    wl = SMALL[name]
    print(f"case {name}", flush=True)
    q, k, v = make_qkv(wl, seed=0)
    op, perm = build(wl)
    ref = O.OracleOperator(wl.grid, wl.text_tokens, wl.text_first, wl.density, permutation=perm)
    g = lambda x: x.to(cuda)  # noqa: E731
    # step 0: first refresh (selection, basis, capture)
    op.begin_step(0, REFRESH)
    out = op.attend(0, g(q), g(k), g(v))
    dense_ref = ref.refresh(0, q, k, v)
    assert_close_bf16(out.cpu().float(), dense_ref, f"refresh-0 {name}")
    bank = op.banks[0][0]
    assert torch.equal(bank.partition.cpu().reshape(ref.layers[0].partition.shape),
                       ref.layers[0].partition)
    # step 1: sparse call on drifted inputs
    q1, k1, v1 = (perturb(x, 0.02, seed=1, step=1) for x in (q, k, v))
    op.begin_step(1, SPARSE)
    out = op.attend(0, g(q1), g(k1), g(v1))
    assert_close_bf16(out.cpu().float(), ref.sparse(0, q1, k1, v1), f"sparse-1 {name}")
    # step 2: refresh with revalidation of the old refinement
    q2, k2, v2 = (perturb(x, 0.03, seed=1, step=2) for x in (q, k, v))
    op.begin_step(2, REFRESH)
    out = op.attend(0, g(q2), g(k2), g(v2))
    assert_close_bf16(out.cpu().float(), ref.refresh(0, q2, k2, v2), f"refresh-2 {name}")
    age, error = op.drain_validation()
    num, den = (float(x) for x in ref.layers[0].pending_stats)
    print(f"  validation error gpu={error:.5f} oracle={math.sqrt(num / den):.5f}", flush=True)
    assert age == 2 and abs(error - math.sqrt(num / den)) < 2e-3
    # step 3: sparse again
    q3, k3, v3 = (perturb(x, 0.02, seed=1, step=3) for x in (q, k, v))
    op.begin_step(3, SPARSE)
    out = op.attend(0, g(q3), g(k3), g(v3))
    assert_close_bf16(out.cpu().float(), ref.sparse(0, q3, k3, v3), f"sparse-3 {name}")


def test_alpha_override_knob_vs_oracle(cuda):
    wl = SMALL["tiny"]
    q, k, v = make_qkv(wl, seed=2)
    op, perm = build(wl)
    ref = O.OracleOperator(wl.grid, wl.text_tokens, wl.text_first, wl.density, permutation=perm)
    op.begin_step(0, REFRESH)
    op.attend(0, q.to(cuda), k.to(cuda), v.to(cuda))
    ref.refresh(0, q, k, v)
    q1, k1, v1 = (perturb(x, 0.05, seed=2, step=1) for x in (q, k, v))
    op.alpha_override = 0.8
    op.begin_step(1, SPARSE)
    out = op.attend(0, q1.to(cuda), k1.to(cuda), v1.to(cuda))
    assert_close_bf16(out.cpu().float(), ref.sparse(0, q1, k1, v1, alpha_override=0.8),
                      "alpha=0.8")


def test_sparse_before_refresh_raises(cuda):
    wl = SMALL["tiny"]
    op, _ = build(wl)
    q, k, v = (x.to(cuda) for x in make_qkv(wl, seed=0))
    op.begin_step(0, SPARSE)
    with pytest.raises(RuntimeError, match="before an exact refresh"):
        op.attend(0, q, k, v)
    hop, _ = build(wl, host_banks=True)
    hop.begin_step(0, SPARSE)
    with pytest.raises(RuntimeError, match="before an exact refresh"):
        hop.attend(0, q, k, v)


def test_non_contiguous_inputs_and_exact_kind(cuda):
    wl = SMALL["text-last-d128"]
    q, k, v = (x.to(cuda) for x in make_qkv(wl, seed=4))
    op, _ = build(wl)
    # diffusers hands [B, N, H, D] projections transposed to [B, H, N, D]
    qt, kt, vt = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k, v))
    op.begin_step(0, REFRESH)
    a = op.attend(0, q, k, v)
    op2, _ = build(wl)
    op2.begin_step(0, REFRESH)
    b = op2.attend(0, qt, kt, vt)
    assert torch.equal(a, b)
    op.begin_step(1, SPARSE)
    op2.begin_step(1, SPARSE)
    assert torch.equal(op.attend(0, q, k, v), op2.attend(0, qt, kt, vt))
    op.begin_step(2, "exact")
    exact = op.attend(0, q, k, v)
    assert_close_bf16(exact.float(), a.float(), "exact vs refresh dense")


# -- full HunyuanVideo-720p shape: size-independent properties ----------------------------


@pytest.fixture(scope="module")
def hunyuan_inputs(cuda):
    wl = WORKLOADS["hunyuan-720p"]
    q, k, v = make_qkv(wl, seed=0, device=cuda)
    return wl, q, k, v


def test_hunyuan_refresh_then_sparse_reproduces_dense(hunyuan_inputs):
    wl, q, k, v = hunyuan_inputs
    op, _ = build(wl)
    op.begin_step(0, REFRESH)
    dense = op.attend(0, q, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(q[:, :2], k[:, :2], v[:, :2])
    assert_close_bf16(dense[:, :2].float(), ref.float(), "hunyuan dense vs sdpa (2 heads)")
    op.begin_step(1, SPARSE)
    sparse = op.attend(0, q, k, v)
    assert_close_bf16(sparse.float(), dense.float(), "hunyuan refresh->sparse == dense")


def test_hunyuan_bank_chunks_and_host_banks_are_identical(hunyuan_inputs):
    wl, q, k, v = hunyuan_inputs
    q1, k1, v1 = (perturb(x, 0.03, seed=5, step=1) for x in (q, k, v))
    outs = {}
    for label, kw in [("plain", {}), ("chunks4", {"chunks": 4}),
                      ("host", {"host_banks": True}),
                      ("host-noprefetch", {"host_banks": True, "prefetch": False})]:
        op, _ = build(wl, layers=2, **kw)
        res = []
        op.begin_step(0, REFRESH)
        for layer in range(2):
            res.append(op.attend(layer, q, k, v))
        op.begin_step(1, SPARSE)
        for layer in range(2):
            res.append(op.attend(layer, q1, k1, v1))
        if hasattr(op, "finish"):
            op.finish()
        torch.cuda.synchronize()
        outs[label] = res
        print(f"  {label}: done", flush=True)
    for label in ("chunks4", "host", "host-noprefetch"):
        for a, b in zip(outs["plain"], outs[label]):
            assert torch.equal(a, b), label
