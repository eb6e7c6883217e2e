"""Pins the CPU oracle before it is trusted as the checker of the HIP path.

Every check compares the oracle with something independent of its own formulas:
LAPACK geqrf through the closed-form post-map, textbook unblocked routines in
Python floats, scipy's LU, and invariants (orthogonality, triangularity, the exact
size of the Cholesky jitter).  No GPU is needed.
"""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import checker, closed_form, rnr, textbook

EPS32 = float(torch.finfo(torch.float32).eps)


def _randn(b, n, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(b, n, n, generator=g, dtype=torch.float64).to(dtype)


def _wellcond(b, n, seed, workloads, lo=-2.0, dtype=torch.float64):
    return workloads.well_conditioned(b, n, seed=seed, lo=lo, dtype=dtype)


# --------------------------------------------------------------------------- whole path


@pytest.mark.parametrize("n", [5, 33, 64, 100])
def test_whole_path_equals_postmapped_geqrf_fp64(n, workloads):
    """jitter 0, float64: the oracle must equal geqrf + post-map to rounding."""
    A = _wellcond(3, n, seed=n, workloads=workloads)
    H, tau = rnr.custom_kernel(A, jitter=0.0, compute_dtype=torch.float64)
    Hc, tc = closed_form.geqrf_postmapped(A)
    assert (H - Hc).abs().max().item() < 1e-10
    assert (tau - tc).abs().max().item() < 1e-10


def test_jitter_is_present_and_small(workloads):
    """With the 1e-7 jitter the fp64 result moves by O(1e-7) -- not 0, not O(1)."""
    A = _wellcond(2, 48, seed=7, workloads=workloads)
    H1, _ = rnr.custom_kernel(A, compute_dtype=torch.float64)
    H0, _ = rnr.custom_kernel(A, jitter=0.0, compute_dtype=torch.float64)
    d = (H1 - H0).abs().max().item() / A.abs().max().item()
    assert 1e-9 < d < 1e-5


@pytest.mark.parametrize("n", [16, 64, 128])
def test_whole_path_fp32_close_to_closed_form(n, workloads):
    A = _wellcond(4, n, seed=100 + n, workloads=workloads, dtype=torch.float32)
    H, tau = rnr.custom_kernel(A)
    assert H.dtype == torch.float32 and tau.dtype == torch.float32
    Hc, tc = closed_form.geqrf_postmapped(A)
    scale = A.abs().amax(dim=(-2, -1), keepdim=True).double()
    # upper part is R (scale of A); lower part and tau are O(1)
    errR = ((torch.triu(H.double()) - torch.triu(Hc)) / scale).abs().max().item()
    errY = (torch.tril(H.double(), -1) - torch.tril(Hc, -1)).abs().max().item()
    errt = (tau.double() - tc).abs().max().item()
    assert errR < 2e-4 and errY < 2e-4 and errt < 2e-4


def test_tiny_whole_path_against_textbook():
    """Python-float unblocked pipeline == oracle (fp64) on 6x6 and 8x8 cases."""
    for n, seed in ((6, 1), (8, 2), (3, 3)):
        A = _randn(1, n, seed)
        H, tau = rnr.custom_kernel(A, compute_dtype=torch.float64)
        Ht, tt = textbook.qr_pipeline(A[0].tolist())
        assert np.max(np.abs(H[0].numpy() - np.array(Ht))) < 1e-12
        assert np.max(np.abs(tau[0].numpy() - np.array(tt))) < 1e-12


# --------------------------------------------------------------------------- stages


def test_lu_matches_textbook_and_scipy():
    for n, seed in ((4, 0), (7, 1), (8, 5), (12, 9)):
        A = _randn(1, n, seed)
        perm, L = rnr.lu_factor(A)
        pt, Lt, Ut = textbook.getrf(A[0].tolist())
        assert perm[0].tolist() == pt
        assert np.max(np.abs(L[0].numpy() - np.array(Lt))) < 1e-12
        _P, Ls, _U = scipy.linalg.lu(A[0].numpy())
        assert np.max(np.abs(L[0].numpy() - Ls)) < 1e-12
    # invariants at a larger size
    A = _randn(3, 70, 11)
    perm, L = rnr.lu_factor(A)
    assert L.abs().max().item() <= 1.0 + 1e-15
    assert torch.equal(torch.diagonal(L, dim1=-2, dim2=-1), torch.ones(3, 70, dtype=L.dtype))
    assert (torch.triu(L, 1) == 0).all()
    # A[perm] = L U: U = L^{-1} A[perm] must be upper triangular
    Ap = torch.gather(A, 1, perm[..., None].expand(-1, -1, 70))
    U = torch.linalg.solve_triangular(L, Ap, upper=False, unitriangular=True)
    assert torch.tril(U, -1).abs().max().item() < 1e-10 * A.abs().max().item()


def test_lu_first_max_tie_rule():
    """Equal |a| in a column: LAPACK takes the first; the oracle must too."""
    A = torch.tensor([[[1.0, 2.0, 0.5], [-3.0, 1.0, 1.0], [3.0, 0.0, 2.0]]], dtype=torch.float64)
    perm, _ = rnr.lu_factor(A)
    pt, _, _ = textbook.getrf(A[0].tolist())
    assert perm[0].tolist() == pt and pt[0] == 1


def test_cholqr_jitter_is_exactly_mean_diag():
    """R^T R - M^T M = mu I with mu = 1e-7 ||M||_F^2 / n, and Q R = M (fp64)."""
    M = _randn(3, 24, 4)
    Q, R = rnr.cholqr(M)
    n = 24
    mu = 1e-7 * (M * M).sum(dim=(-2, -1)) / n
    D = R.mT @ R - M.mT @ M
    eye = torch.eye(n, dtype=torch.float64)
    # mu ~ 2.5e-6 here; rounding of M^T M leaves ~1e-14, a wrong mu (sum, max, 1e-6 ...) is >= 1e-7 off
    assert (D - mu[:, None, None] * eye).abs().max().item() < 1e-11
    assert (torch.tril(R, -1) == 0).all()
    assert (Q @ R - M).abs().max().item() < 1e-12
    # textbook potrf/trsm agree
    Qt, Rt = textbook.cholqr(M[0].tolist(), 1e-7)
    assert np.max(np.abs(R[0].numpy() - np.array(Rt))) < 1e-12
    assert np.max(np.abs(Q[0].numpy() - np.array(Qt))) < 1e-12


def test_frame_is_orthonormal_and_triangularizes_A(workloads):
    A = _randn(2, 96, 21)
    Q = rnr.frame(A, jitter=0.0)
    eye = torch.eye(96, dtype=torch.float64)
    assert (Q.mT @ Q - eye).abs().max().item() < 1e-12
    T = Q.mT @ A
    assert torch.tril(T, -1).abs().max().item() < 1e-11 * A.abs().max().item()


def test_chart_equals_postmapped_geqrf_of_Q(workloads):
    Q = workloads.haar(3, 80, torch.Generator().manual_seed(5), "cpu")
    Y, s = rnr.chart(Q)
    Hc, tc = closed_form.geqrf_postmapped(Q)
    assert (torch.tril(Y, -1) - torch.tril(Hc, -1)).abs().max().item() < 1e-11
    tau = rnr.tau_from_reflectors(Y)
    assert (tau - tc).abs().max().item() < 1e-11
    # R of an orthogonal Q is a sign diagonal; the chart's signs fold it to -1 on Z ... here
    # triu(s * Q^T Q) must equal triu(Hc), i.e. s_k = Hc[k,k] (|.| = 1)
    assert (s - torch.diagonal(Hc, dim1=-2, dim2=-1)).abs().max().item() < 1e-11


@pytest.mark.parametrize("bs", [1, 7, 32, 200])
def test_chart_blocking_does_not_change_result(bs, workloads):
    Q = workloads.haar(2, 70, torch.Generator().manual_seed(9), "cpu")
    Y1, s1, d1 = rnr.chart(Q, bs=1, return_diag=True)
    Yb, sb, db = rnr.chart(Q, bs=bs, return_diag=True)
    assert torch.equal(s1, sb)
    assert (Y1 - Yb).abs().max().item() < 1e-12
    assert (d1 - db).abs().max().item() < 1e-12
    Yt, st, dt = textbook.chart_unblocked(Q[0].tolist())
    assert np.max(np.abs(Yb[0].numpy() - np.array(Yt))) < 1e-12
    assert sb[0].tolist() == st


def test_tau_closed_form_makes_each_reflector_orthogonal(workloads):
    A = _wellcond(2, 40, seed=3, workloads=workloads)
    H, tau = rnr.custom_kernel(A, compute_dtype=torch.float64)
    assert tau.min().item() >= 1.0 - 1e-15 and tau.max().item() <= 2.0 + 1e-15
    assert torch.all(tau[:, -1] == 2.0)
    Q = torch.linalg.householder_product(H, tau)
    eye = torch.eye(40, dtype=torch.float64)
    assert (Q.mT @ Q - eye).abs().max().item() < 1e-13


# --------------------------------------------------------------------------- special cases


def test_upper_triangular_input_gives_minus_A_and_tau_2():
    A = torch.triu(_randn(3, 20, 13))
    H, tau = rnr.custom_kernel(A, compute_dtype=torch.float64)
    assert (H + A).abs().max().item() < 1e-6 * A.abs().max().item()
    assert (tau - 2.0).abs().max().item() == 0.0


def test_n1_and_zero_matrix():
    A = torch.tensor([[[3.0]], [[-2.0]]])
    H, tau = rnr.custom_kernel(A)
    assert torch.allclose(H, -A, rtol=1e-6, atol=0) and torch.all(tau == 2.0)
    Z = torch.zeros(2, 9, 9)
    H, tau = rnr.custom_kernel(Z)
    assert torch.all(H == 0) and torch.all(tau == 2.0)


def test_dtype_and_batch_dims_follow_the_input():
    A = _randn(6, 12, 2).reshape(2, 3, 12, 12)
    H, tau = rnr.custom_kernel(A.to(torch.bfloat16))
    assert H.dtype == torch.bfloat16 and H.shape == (2, 3, 12, 12) and tau.shape == (2, 3, 12)
    H2, tau2 = rnr.custom_kernel(A[0, 0].float())
    assert H2.shape == (12, 12) and tau2.shape == (12,)


# --------------------------------------------------------------------------- checker and classes


def test_checker_accepts_exact_and_rejects_planted_error():
    A = _randn(2, 32, 8).float()
    Hg, tg = torch.geqrf(A.double())
    fr, og, ft, ot, ok = checker.check(A, Hg, tg)
    assert fr < 1e-13 and og < 1e-13 and bool(ok.all())
    Hbad = Hg.clone()
    Hbad[:, 0, :] *= 1.01            # 1 % error in the first row of R
    fr, og, ft, ot, ok = checker.check(A, Hbad, tg)
    assert fr > ft and not bool(ok.any())
    tbad = tg.clone()
    tbad[:, 3] *= 1.001              # reflector no longer orthogonal
    _, og, _, ot, ok = checker.check(A, Hg, tbad)
    assert og > ot and not bool(ok.any())


@pytest.mark.parametrize("cls", ["dense", "logspace12", "rankdef", "rowscaled", "nearrank", "uppertri"])
def test_gates_pass_on_every_headline_class(cls, workloads):
    g = torch.Generator().manual_seed(hash(cls) % 1000)
    A = workloads.headline_class_batch(cls, 2, 96, g, "cpu").float()
    H, tau = rnr.custom_kernel(A)
    fr, og, ft, ot, ok = checker.check(A, H, tau)
    assert bool(ok.all()), (cls, fr, og)
    assert tau.min().item() >= 1.0 - 2 * EPS32 and tau.max().item() <= 2.0


def test_config1_batch_layout_and_gates(workloads):
    A = workloads.make_batch(1)
    assert A.shape == (16, 64, 64) and A.dtype == torch.float32
    H, tau = rnr.custom_kernel(A)
    assert H.shape == A.shape and tau.shape == (16, 64)
    fr, og, ft, ot, ok = checker.check(A, H, tau)
    assert bool(ok.all())
    # margins well inside the gates, in line with the reference's README:93-105 table
    assert fr < ft / 100 and og < ot / 100


def test_checker_fails_nan_like_the_reference():
    """A NaN anywhere in H or tau fails the gates: the reference compares with `<`, which is
    False for NaN (common/oracle.py:166-168).  The GPU checker must do the same."""
    A = _randn(3, 24, 9).float()
    Hg, tg = torch.geqrf(A.double())
    H, tau = Hg.float(), tg.float()
    H[0, 2, 5] = float("nan")       # in R
    H[1, 9, 3] = float("nan")       # in a reflector tail
    tau[2, 4] = float("nan")
    fr, og, ft, ot, ok = checker.check(A, H, tau)
    assert not bool(ok.any())
    ratio, og2, okc = checker.check_percol(A, H, tau)
    assert not bool(okc.any())


def test_stress_cases_have_their_structure(workloads):
    """The nine cases of the reference's stress battery (common/oracle.py:43-146)."""
    n = 40
    for case in workloads.STRESS_CASES:
        A = workloads.stress_batch(case, 8, n, seed=3)
        assert A.shape == (8, n, n) and A.dtype == torch.float32 and bool(torch.isfinite(A).all()), case
        s = torch.linalg.svdvals(A.double())
        if case == "rankdef":
            assert s[:, n // 2:].max().item() < 1e-5 and s[:, : n // 2].min().item() > 0.09
        elif case == "nearrank":
            assert (s[:, n // 2:] - 1e-8).abs().max().item() < 1e-6
        elif case == "clustered":
            assert (s[:, : n // 2] - 1).abs().max().item() < 1e-5 and s[:, n // 2:].max().item() < 1e-5
        elif case == "banded":
            i = torch.arange(n)
            assert A[:, (i.view(n, 1) - i.view(1, n)).abs() > n // 8].abs().max().item() == 0.0
        elif case == "nearcollinear":
            assert (A[:, :, 1] - A[:, :, 0]).abs().max().item() < 1e-5
        elif case == "uppertri":
            assert torch.equal(A, torch.triu(A))
        elif case == "mixed":  # matrices 3 and 7 are stress cases: rankdef, then nearrank
            assert torch.linalg.svdvals(A[3].double())[n // 2:].max().item() < 1e-5
            assert torch.linalg.svdvals(A[7].double())[n // 2:].max().item() < 1e-6
    # seeded: the same call twice gives the same batch, another seed another one
    assert torch.equal(workloads.stress_batch("dense", 2, 16, seed=5), workloads.stress_batch("dense", 2, 16, seed=5))
    assert not torch.equal(workloads.stress_batch("dense", 2, 16, seed=5), workloads.stress_batch("dense", 2, 16, seed=6))


@pytest.mark.parametrize("case", ["dense", "mixed", "rankdef", "nearrank", "clustered", "banded", "rowscaled",
                                  "nearcollinear", "uppertri"])
def test_oracle_passes_the_stress_battery(case, workloads):
    """The reference algorithm (oracle) passes the per-column gate on every stress case."""
    A = workloads.stress_batch(case, 8, 64, seed=0)
    H, tau = rnr.custom_kernel(A)
    ratio, og, ok = checker.check_percol(A, H, tau)
    assert bool(ok.all()), (case, ratio, og)
    assert tau.min().item() >= 1.0 - 16 * EPS32 and tau.max().item() <= 2.0
