"""GPU checks of the symmetric eigen-solver that gives the closure basis, against what the
mathematics fixes: eigenvalues of a matrix built from a known orthogonal basis, the LAPACK
eigenvalues (fp64, CPU) of random symmetric matrices, orthonormality, the eigen-residual,
eigenvectors up to sign where the eigenvalues are separated, and the trivial cases
(diagonal, zero, identity, order 1 and odd orders).

Tolerances (fp32 solver, n <= 128): eigenvalues within 8e-6 of max |lambda| and
||S U - U diag(lambda)||_F within 8e-6 of ||S||_F (the backward-error scale n * eps_fp32 of
any fp32 solver; LAPACK's fp32 figure on the same input is printed beside ours), U^T U
within 2e-6 of I, |u . u_ref| >= 1 - 1e-4 for eigenvalues whose relative gap to their
neighbours exceeds 1e-2."""

import pytest
import torch

import oracle as O
from gpu_util import SMALL
from recap_amd import _lib
from recap_amd import kernels as K
from recap_amd.layout import Layout, hilbert_permutation
from recap_amd.synthetic import make_qkv

pytestmark = pytest.mark.gpu


def _check(a_cpu, lam, u, *, vec_gap=1e-2):
    s = (0.5 * (a_cpu + a_cpu.transpose(-1, -2))).double()
    lam, u = lam.cpu().double(), u.cpu().double()
    ref_lam, ref_u = torch.linalg.eigh(s)
    n = s.shape[-1]
    scale = ref_lam.abs().amax(-1, keepdim=True).clamp_min(1e-30)
    err_lam = float(((lam - ref_lam).abs() / scale).max())
    orth = float((u.transpose(-1, -2) @ u - torch.eye(n, dtype=torch.float64)).abs().max())
    res = torch.linalg.matrix_norm(s @ u - u * lam.unsqueeze(-2)) / \
        torch.linalg.matrix_norm(s).clamp_min(1e-30)
    lapack32 = torch.linalg.eigh(s.float())[0].double()
    err32 = float(((lapack32 - ref_lam).abs() / scale).max())
    print(f"  n={n} eig {err_lam:.2e} (LAPACK fp32 {err32:.2e}) orth {orth:.2e} "
          f"residual {float(res.max()):.2e}", flush=True)
    assert torch.all(lam[..., 1:] >= lam[..., :-1])
    assert err_lam < 8e-6
    assert orth < 2e-6
    assert float(res.max()) < 8e-6
    # Eigenvectors of well separated eigenvalues agree up to sign.
    for b in range(s.shape[0]):
        lv = ref_lam[b]
        gap = torch.full((n,), float("inf"), dtype=torch.float64)
        if n > 1:
            d = (lv[1:] - lv[:-1]).abs()
            gap[1:] = torch.minimum(gap[1:], d)
            gap[:-1] = torch.minimum(gap[:-1], d)
        sep = gap / lv.abs().max().clamp_min(1e-30) > vec_gap
        dots = (u[b] * ref_u[b]).sum(0).abs()
        assert torch.all(dots[sep] > 1 - 1e-4), dots[sep].min()


@pytest.mark.parametrize("n", [1, 2, 5, 64, 127, 128])
def test_random_scatter_matrices(cuda, n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(3, 4 * n + 8, n, generator=g)
    a = x.transpose(-1, -2) @ x / x.shape[1]
    a = a + 1e-3 * torch.randn(3, n, n, generator=g)   # the antisymmetric part must not matter
    lam, u = K.symmetric_eigen(a.to(cuda))
    _check(a, lam, u)


def test_indefinite_and_known_basis(cuda):
    g = torch.Generator().manual_seed(7)
    n = 128
    q = torch.linalg.qr(torch.randn(2, n, n, generator=g, dtype=torch.float64))[0]
    lv = torch.linspace(-3.0, 5.0, n, dtype=torch.float64).expand(2, n)
    a = (q * lv.unsqueeze(-2)) @ q.transpose(-1, -2)
    lam, u = K.symmetric_eigen(a.float().to(cuda))
    _check(a.float(), lam, u)
    # Ascending order: column i is +-q[:, i] for the known basis.
    dots = (u.cpu().double() * q).sum(-2).abs()
    assert float(dots.min()) > 1 - 1e-5
    sym = torch.randn(2, 96, 96, generator=g)
    lam, u = K.symmetric_eigen(sym.to(cuda))
    _check(sym, lam, u)


def test_diagonal_zero_and_identity(cuda):
    n = 64
    diag = torch.diag_embed(torch.tensor([[float((7 * i) % n) for i in range(n)]]))
    lam, u = K.symmetric_eigen(diag.to(cuda))
    assert torch.equal(lam.cpu()[0], torch.arange(n, dtype=torch.float32))
    perm = torch.argsort(torch.diagonal(diag[0]))
    assert torch.equal(u.cpu()[0], torch.eye(n)[:, perm])   # no rotation on a diagonal input
    zero = torch.zeros(2, 33, 33)
    lam, u = K.symmetric_eigen(zero.to(cuda))
    assert torch.equal(lam.cpu(), torch.zeros(2, 33)) and torch.equal(u.cpu()[1], torch.eye(33))
    eye = torch.eye(128).expand(1, 128, 128).contiguous()
    lam, u = K.symmetric_eigen(eye.to(cuda))
    assert torch.equal(lam.cpu(), torch.ones(1, 128)) and torch.equal(u.cpu()[0], torch.eye(128))


@pytest.mark.parametrize("name", ["tiny", "text-last-d128"])
def test_closure_scatter_basis(cuda, name):
    """The solver on the real closure scatter; the basis it gives leaves the rotated
    variances (sign-invariant) equal to those of the oracle's LAPACK basis."""
    wl = SMALL[name]
    print(f"case {name} d={wl.dim}", flush=True)
    q, k, v = make_qkv(wl, seed=3, dtype=torch.bfloat16)
    perm = hilbert_permutation(wl.grid)
    layout = Layout.from_permutation(perm, text_tokens=wl.text_tokens, text_first=wl.text_first)
    geo = K.Geometry(wl.tokens, wl.video_tokens)
    kv = K.kv_pack(k.to(cuda), v.to(cuda), layout.rowmap(cuda), geo)
    _, _, scatter = K.closure_stats(kv, geo, _lib.CLOSURE_CVK | _lib.CLOSURE_SCATTER)
    lam, u = K.symmetric_eigen(scatter)
    _check(scatter.cpu(), lam, u)
    ref = O.closure_basis(scatter.cpu())
    split = K.basis_tables(u, None, kv.dtype, split=True)
    var, _, _ = K.closure_stats(kv, geo, _lib.CLOSURE_ROT, split.u_hi_t, split.u_lo_t)
    split_ref = K.basis_tables(ref.to(cuda), None, kv.dtype, split=True)
    var_ref, _, _ = K.closure_stats(kv, geo, _lib.CLOSURE_ROT, split_ref.u_hi_t, split_ref.u_lo_t)
    # The per-block trace is the same in every orthonormal basis, and the columns of
    # separated eigenvalues (same ascending order in both) carry the same variances.
    var, var_ref = var.cpu().double(), var_ref.cpu().double()
    tot, tot_ref = var.sum(-1), var_ref.sum(-1)
    rel = float(((tot - tot_ref).abs() / tot_ref.abs().clamp_min(1e-6)).max())
    lv = torch.linalg.eigh(0.5 * (scatter + scatter.transpose(-1, -2)).cpu().double())[0]
    gap = torch.full_like(lv, float("inf"))
    d = lv[:, 1:] - lv[:, :-1]
    gap[:, 1:] = torch.minimum(gap[:, 1:], d)
    gap[:, :-1] = torch.minimum(gap[:, :-1], d)
    sep = (gap / lv.abs().amax(-1, keepdim=True)) > 1e-2          # [banks, d]
    col = ((var - var_ref).abs() / var_ref.abs().clamp_min(1e-3))   # [banks, nb, d]
    col_rel = float(col.amax(1)[sep].max())
    print(f"  block-variance trace rel {rel:.2e}; separated columns rel {col_rel:.2e} "
          f"({int(sep.sum())} of {sep.numel()})", flush=True)
    assert rel < 1e-4
    assert int(sep.sum()) > 0 and col_rel < 1e-2
