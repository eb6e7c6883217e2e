"""The contest gates of (H, tau) evaluated on the GPU in float64 (``rnr_check_f64``).

A restatement of the reference checker, ``common/oracle.py:152-195`` (``check`` and
``check_percol``), for the path's output at full batch size: Q is rebuilt from the
reflectors in float64 and

* factor residual  ``||triu(H) - Q^T A||_1 / ||A||_1 < 20 n eps32``
* orthogonality    ``||Q^T Q - I||_1 < 100 n eps32``
* per column       ``max_j ||(triu(H) - Q^T A)[:, j]||_1 / (20 n eps32 ||A[:, j]||_1) < 1``

with the matrix 1-norm.  Runs on the tensors' GPU, on the current stream.
"""
from __future__ import annotations

import torch

from . import _native

EPS32 = float(torch.finfo(torch.float32).eps)

__all__ = ["gate_values", "check", "check_percol", "gates"]


def gates(n: int):
    """(factor gate, orthogonality gate) for size n."""
    return 20.0 * n * EPS32, 100.0 * n * EPS32


def gate_values(A: torch.Tensor, H: torch.Tensor, tau: torch.Tensor):
    """Per-matrix float64 (factor, ortho, colratio) tensors on A's device."""
    if A.dim() < 2 or A.shape[-1] != A.shape[-2] or H.shape != A.shape or tau.shape != A.shape[:-1]:
        raise ValueError("gate_values: expected A, H of shape (..., n, n) and tau of shape (..., n)")
    if not (A.is_cuda and H.is_cuda and tau.is_cuda):
        raise RuntimeError("gate_values: the checker runs on the GPU only")
    n = int(A.shape[-1])
    A = A.to(torch.float32).reshape(-1, n, n).contiguous()
    H = H.to(torch.float32).reshape(-1, n, n).contiguous()
    tau = tau.to(torch.float32).reshape(-1, n).contiguous()
    batch = A.shape[0]
    out = torch.empty(3, max(batch, 1), dtype=torch.float64, device=A.device)
    if batch:
        nbytes = _native.workspace_bytes("check", batch, n)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=A.device)
        with torch.cuda.device(A.device):
            st = _native.lib().rnr_check_f64(
                A.data_ptr(), n * n, H.data_ptr(), tau.data_ptr(), batch, n, out[0].data_ptr(),
                out[1].data_ptr(), out[2].data_ptr(), ws.data_ptr(), ws.numel(),
                torch.cuda.current_stream(A.device).cuda_stream)
        _native.check("rnr_check_f64", st)
    return out[0, :batch], out[1, :batch], out[2, :batch]


def check(A, H, tau):
    """(max factor residual, max orthogonality, factor gate, ortho gate, per-matrix pass mask)
    -- the return of the reference ``check`` (common/oracle.py:156-168)."""
    fac, orth, _ = gate_values(A, H, tau)
    ft, ot = gates(int(A.shape[-1]))
    passed = (fac < ft) & (orth < ot)
    return fac.max().item(), orth.max().item(), ft, ot, passed


def check_percol(A, H, tau):
    """(max per-column budget fraction, max orthogonality, pass mask) -- the reference
    ``check_percol`` (common/oracle.py:171-195)."""
    _, orth, ratio = gate_values(A, H, tau)
    _, ot = gates(int(A.shape[-1]))
    passed = (ratio < 1.0) & (orth < ot)
    return ratio.max().item(), orth.max().item(), passed
