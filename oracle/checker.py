"""The contest gates for (H, tau) in geqrf layout -- test infrastructure only.

Restates ``/root/reference/common/oracle.py:152-195``: Q is rebuilt from the
reflectors in float64 (``torch.linalg.householder_product``), then

* factor residual  ``||triu(H) - Q^T A||_1 / ||A||_1 < 20 n eps32``  (``:163,166``)
* orthogonality    ``||Q^T Q - I||_1 < 100 n eps32``                  (``:165-166``)

with the matrix 1-norm (max absolute column sum) per matrix.  ``check_percol``
is the stricter per-column variant (``:171-195``).
"""
from __future__ import annotations

import torch

EPS32 = float(torch.finfo(torch.float32).eps)


def _norm1(X: torch.Tensor) -> torch.Tensor:
    return X.abs().sum(dim=-2).amax(dim=-1)


def factor_and_ortho(A: torch.Tensor, H: torch.Tensor, tau: torch.Tensor):
    """Per-matrix (factor residual, orthogonality defect), both float64 tensors."""
    n = A.shape[-1]
    Ad, Hd, td = A.double(), H.double(), tau.double()
    Q = torch.linalg.householder_product(Hd, td)
    R = torch.triu(Hd)
    QtA = Q.mT @ Ad
    fac = _norm1(R - QtA) / _norm1(Ad)
    eye = torch.eye(n, dtype=torch.float64, device=Q.device)
    orth = _norm1(Q.mT @ Q - eye)
    return fac, orth


def gates(n: int):
    return 20.0 * n * EPS32, 100.0 * n * EPS32


def check(A, H, tau):
    """(max factor residual, max orthogonality, factor gate, ortho gate, per-matrix pass mask)."""
    n = A.shape[-1]
    fac, orth = factor_and_ortho(A, H, tau)
    ft, ot = gates(n)
    passed = (fac < ft) & (orth < ot)
    return fac.max().item(), orth.max().item(), ft, ot, passed


def check_percol(A, H, tau):
    """Per-column-relative factor gate: (max budget fraction, max ortho, pass mask)."""
    n = A.shape[-1]
    Ad, Hd, td = A.double(), H.double(), tau.double()
    Q = torch.linalg.householder_product(Hd, td)
    res = (torch.triu(Hd) - Q.mT @ Ad).abs().sum(dim=-2)
    acol = Ad.abs().sum(dim=-2).clamp_min(1e-300)
    ft, ot = gates(n)
    ratio = (res / (ft * acol)).amax(dim=-1)
    eye = torch.eye(n, dtype=torch.float64, device=Q.device)
    orth = _norm1(Q.mT @ Q - eye)
    passed = (ratio < 1.0) & (orth < ot)
    return ratio.max().item(), orth.max().item(), passed
