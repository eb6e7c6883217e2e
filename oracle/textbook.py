"""Textbook unblocked routines in pure Python floats (float64) -- test infrastructure only.

Small-case brute force for pinning ``oracle.rnr``: each routine is the plain
column-by-column algorithm from the literature, with no blocking and no library
call, so a mistake in the blocked/library-backed oracle shows up as a mismatch.

* ``getrf``      -- LAPACK ``xGETF2`` semantics: partial pivoting with the FIRST
                    maximum of |a_ij| (``IxAMAX``), row swaps, unit-lower L; a zero
                    pivot skips the scaling.  (``torch.linalg.lu`` at
                    ``/root/reference/reflection_no_reflectors.py:66``.)
* ``potrf_upper`` -- Cholesky ``G = R^T R`` row by row.  (``:76``)
* ``trsm_right_upper`` -- ``X R = B`` by forward substitution over columns.  (``:77``)
* ``chart_unblocked`` -- the sign-ruled elimination of ``I - Q S`` one column at a
                    time on the Q copy (``:86-176`` with panel width 1).
"""
from __future__ import annotations

import math


def _copy(A):
    return [list(map(float, row)) for row in A]


def getrf(A):
    """Returns (perm, L, U) with A[perm[i]] = (L U)[i]."""
    a = _copy(A)
    n = len(a)
    perm = list(range(n))
    for j in range(n):
        p = j
        best = abs(a[j][j])
        for i in range(j + 1, n):
            if abs(a[i][j]) > best:
                best = abs(a[i][j])
                p = i
        if a[p][j] != 0.0:
            if p != j:
                a[p], a[j] = a[j], a[p]
                perm[p], perm[j] = perm[j], perm[p]
            inv = 1.0 / a[j][j]
            for i in range(j + 1, n):
                a[i][j] *= inv
        for i in range(j + 1, n):
            lij = a[i][j]
            for c in range(j + 1, n):
                a[i][c] -= lij * a[j][c]
    L = [[(a[i][j] if j < i else (1.0 if i == j else 0.0)) for j in range(n)] for i in range(n)]
    U = [[(a[i][j] if j >= i else 0.0) for j in range(n)] for i in range(n)]
    return perm, L, U


def potrf_upper(G):
    n = len(G)
    R = [[0.0] * n for _ in range(n)]
    for i in range(n):
        s = G[i][i] - sum(R[k][i] * R[k][i] for k in range(i))
        if not s > 0.0:
            raise ValueError("not positive definite")
        R[i][i] = math.sqrt(s)
        for j in range(i + 1, n):
            R[i][j] = (G[i][j] - sum(R[k][i] * R[k][j] for k in range(i))) / R[i][i]
    return R


def trsm_right_upper(B, R):
    """X with X R = B."""
    m, n = len(B), len(R)
    X = [[0.0] * n for _ in range(m)]
    for r in range(m):
        for j in range(n):
            X[r][j] = (B[r][j] - sum(X[r][k] * R[k][j] for k in range(j))) / R[j][j]
    return X


def gram(M):
    n = len(M[0])
    return [[sum(M[r][i] * M[r][j] for r in range(len(M))) for j in range(n)] for i in range(n)]


def cholqr(M, jitter):
    n = len(M[0])
    G = gram(M)
    mu = jitter * sum(G[i][i] for i in range(n)) / n
    for i in range(n):
        G[i][i] += mu
    R = potrf_upper(G)
    return trsm_right_upper(M, R), R


def chart_unblocked(Q):
    """Returns (Y, s, d): multipliers, signs and live diagonals."""
    m = _copy(Q)
    n = len(m)
    Y = [[0.0] * n for _ in range(n)]
    s = [1.0] * n
    d = [0.0] * n
    for k in range(n):
        dk = m[k][k]
        d[k] = dk
        if abs(1.0 - dk) >= abs(1.0 + dk):
            s[k], piv = 1.0, 1.0 - dk
        else:
            s[k], piv = -1.0, 1.0 + dk
        for i in range(k + 1, n):
            Y[i][k] = (-s[k] * m[i][k]) / piv
            for c in range(k + 1, n):
                m[i][c] -= Y[i][k] * m[k][c]
    return Y, s, d


def qr_pipeline(A, jitter=1e-7):
    """The whole reflector-free pipeline, unblocked, in Python floats: (H, tau)."""
    n = len(A)
    perm, L, _ = getrf(A)
    Q1, _ = cholqr(L, jitter)
    Q2, _ = cholqr(Q1, jitter)
    Q = [[0.0] * n for _ in range(n)]
    for i in range(n):
        Q[perm[i]] = list(Q2[i])
    R = [[sum(Q[r][i] * A[r][j] for r in range(n)) if j >= i else 0.0 for j in range(n)]
         for i in range(n)]
    Y, s, _ = chart_unblocked(Q)
    tau = [2.0 / (1.0 + sum(Y[i][k] ** 2 for i in range(k + 1, n))) for k in range(n)]
    H = [[(s[i] * R[i][j] if j >= i else Y[i][j]) for j in range(n)] for i in range(n)]
    return H, tau
