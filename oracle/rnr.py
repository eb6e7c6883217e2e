"""torch-CPU restatement of the reference's reflector-free QR (test infrastructure only).

Follows ``/root/reference/reflection_no_reflectors.py`` stage by stage.  The dense
primitives the reference takes from ``torch.linalg`` (the third-party boundary:
PyTorch 2.10.0 in this image, LAPACK ``sgetrf``/``spotrf``/``strsm`` underneath on
CPU; the reference pins no version) are called the same way here, so in fp32 this
module reproduces the reference's own CPU arithmetic.  Every function also runs in
float64, which the pinning tests use to separate algebra mistakes from rounding.

Two knobs exist only for those tests: ``jitter`` (the reference's always-on 1e-7,
``:74``) and ``bs`` (the chart's panel width 32, ``:86``).
"""
from __future__ import annotations

import torch

JITTER = 1e-7       # reflection_no_reflectors.py:74
CHART_BS = 32       # reflection_no_reflectors.py:86


def lu_factor(A: torch.Tensor):
    """Partial-pivot LU, ``A = P L U`` (reference ``:66``, ``torch.linalg.lu``).

    Returns ``(perm, L)``: ``perm[..., i]`` is the original row that lands in
    position i (so ``A[perm] = L U``) and L is unit lower-triangular.  U is not
    returned because the reference discards it.
    """
    P, L, _ = torch.linalg.lu(A)
    # P[r, i] = 1  <=>  row r of A is row i of L U
    perm = P.argmax(dim=-2)
    return perm, L


def cholqr(M: torch.Tensor, jitter: float = JITTER):
    """One CholeskyQR pass with the diagonal jitter (reference ``:68-77``).

    ``G = M^T M``; ``mu = jitter * mean(diag G)`` per matrix; ``R = chol(G + mu I)``
    (upper); returns ``(M R^{-1}, R)``.
    """
    n = M.shape[-1]
    G = M.mT @ M
    mu = jitter * torch.diagonal(G, dim1=-2, dim2=-1).mean(dim=-1)
    G = G + mu[..., None, None] * torch.eye(n, dtype=M.dtype)
    R = torch.linalg.cholesky(G, upper=True)
    Qm = torch.linalg.solve_triangular(R, M, upper=True, left=False)
    return Qm, R


def frame(A: torch.Tensor, jitter: float = JITTER) -> torch.Tensor:
    """The orthogonal frame Q (reference ``_frame``, ``:55-81``).

    LU with partial pivoting, CholeskyQR twice on the unit-lower L, then the row
    permutation back to A's row order, done as the reference does it: a product
    with the dense permutation matrix P (exact, since P holds only 0 and 1).
    """
    P, L, _ = torch.linalg.lu(A)
    Q1, _ = cholqr(L, jitter)
    Q2, _ = cholqr(Q1, jitter)
    return P @ Q2


def closure(Q: torch.Tensor, A: torch.Tensor) -> torch.Tensor:
    """R = triu(Q^T A) (reference ``:186``)."""
    return torch.triu(Q.mT @ A)


def chart(Q: torch.Tensor, bs: int = CHART_BS, return_diag: bool = False):
    """Sign-ruled unpivoted LU of ``I - Q S`` run on a copy of Q (reference ``_chart``, ``:86-176``).

    Returns ``(Y, s)``: Y holds the multipliers (the reflector tails) strictly below
    the diagonal, s the +-1 signs.  With ``return_diag`` also the live diagonal
    d_k of every column, which the parity tests use to find sign-rule near-ties.

    Panel by panel (width ``bs``): each column k picks ``s_k = +1`` when
    ``|1 - d| >= |1 + d|`` (pivot ``1 - d``), else ``s_k = -1`` (pivot ``1 + d``)
    (``:149-155``); its multipliers ``-s_k M[k+1:, k] / pivot`` go to Y (``:157-159``)
    and update the remaining panel columns only (``:160-162``).  After the panel,
    the panel rows are forwarded through the panel's own unit-lower factor
    (``:167-171``) and the trailing block takes one rank-``bs`` product (``:172-174``).
    """
    n = Q.shape[-1]
    batch = Q.shape[:-2]
    M = Q.clone()
    Y = torch.zeros_like(Q)
    s = torch.ones(*batch, n, dtype=Q.dtype)
    dvals = torch.zeros(*batch, n, dtype=Q.dtype)
    one = torch.ones((), dtype=Q.dtype)
    for p0 in range(0, n, bs):
        p1 = min(p0 + bs, n)
        for k in range(p0, p1):
            d = M[..., k, k]
            dvals[..., k] = d
            plus = (1.0 - d).abs() >= (1.0 + d).abs()
            sk = torch.where(plus, one, -one)
            pivot = torch.where(plus, 1.0 - d, 1.0 + d)
            s[..., k] = sk
            if k + 1 == n:
                continue
            mult = (-sk[..., None] * M[..., k + 1:, k]) / pivot[..., None]
            Y[..., k + 1:, k] = mult
            if k + 1 < p1:
                M[..., k + 1:, k + 1:p1] -= mult[..., :, None] * M[..., k, None, k + 1:p1]
        if p1 < n:
            for k in range(p0, p1 - 1):
                M[..., k + 1:p1, p1:] -= Y[..., k + 1:p1, k, None] * M[..., k, None, p1:]
            M[..., p1:, p1:] -= Y[..., p1:, p0:p1] @ M[..., p0:p1, p1:]
    if return_diag:
        return Y, s, dvals
    return Y, s


def tau_from_reflectors(Y: torch.Tensor) -> torch.Tensor:
    """tau_k = 2 / (1 + sum_{i>k} Y[i,k]^2) (reference ``:192``); the last column gives 2."""
    return 2.0 / (torch.tril(Y, -1).square().sum(dim=-2) + 1.0)


def pack(R: torch.Tensor, Y: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """H = triu(s_i * R_ij) + tril(Y, -1) (reference ``:195``)."""
    return torch.triu(s[..., :, None] * R) + torch.tril(Y, -1)


def custom_kernel(data: torch.Tensor, jitter: float = JITTER, bs: int = CHART_BS,
                  compute_dtype=torch.float32, return_diag: bool = False):
    """(H, tau) in geqrf layout (reference ``custom_kernel``, ``:181-196``).

    ``compute_dtype`` is float32 in the reference (``:183``); the tests also run
    it in float64.  Outputs are cast back to ``data.dtype`` (``:196``).
    """
    dtype = data.dtype
    A = data.to(compute_dtype)
    Q = frame(A, jitter)
    R = closure(Q, A)
    if return_diag:
        Y, s, dvals = chart(Q, bs, return_diag=True)
    else:
        Y, s = chart(Q, bs)
    tau = tau_from_reflectors(Y)
    H = pack(R, Y, s)
    if return_diag:
        return H.to(dtype), tau.to(dtype), dvals
    return H.to(dtype), tau.to(dtype)
