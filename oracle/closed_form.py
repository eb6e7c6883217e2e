"""Closed-form oracle: LAPACK geqrf plus a sign/tau post-map -- test infrastructure only.

For full-rank A, in exact arithmetic, the reflector-free pipeline
(``/root/reference/reflection_no_reflectors.py:181-196``) returns LAPACK's
``geqrf(A)`` except on the index set Z = {n-1} U {k : geqrf tau_k = 0}:

* ``tril(H, -1)`` equals geqrf's reflector tails;
* ``triu(H)`` equals geqrf's R with the rows k in Z negated;
* ``tau[k]`` equals geqrf's tau_k for k not in Z and 2 for k in Z.

Reason: the chart's sign rule ``s_k = -sign(d_k)`` (``:149-155``) picks the same
reflector as LAPACK's ``beta = -sign(alpha) ||x||`` whenever LAPACK applies a
reflector; where LAPACK applies none (tau = 0, an exactly zero column tail, and
always the last column) the chart still applies ``I - 2 e_k e_k^T``, which only
flips row k of R.  The LU of ``I - Q S`` is unique because its pivots are >= 1,
so the frame's pivot order and CholeskyQR details drop out.
"""
from __future__ import annotations

import torch


def geqrf_postmapped(A: torch.Tensor, zero_tol: float = 0.0):
    """(H, tau) that the reference returns in exact arithmetic, from float64 geqrf."""
    Hg, tg = torch.geqrf(A.double())
    Z = tg.abs() <= zero_tol
    Z[..., -1] = True
    sign = torch.where(Z, -1.0, 1.0).to(torch.float64)
    H = torch.triu(sign[..., :, None] * Hg) + torch.tril(Hg, -1)
    tau = torch.where(Z, torch.full_like(tg, 2.0), tg)
    return H, tau
