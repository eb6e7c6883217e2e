"""Consumers of the compact ``(H, tau)`` output on the GPU (``README.md:122-128`` of the
reference: ``Q = torch.linalg.householder_product(H, tau)``, ``R = triu(H)``).

* ``householder_product(H, tau)`` -- Q (``rnr_orgqr_f32``);
* ``ormqr(H, tau, C, transpose=False)`` -- Q C or Q^T C (``rnr_ormqr_f32``, torch.ormqr with
  ``left=True``).

Both take ``(..., n, n)`` H, ``(..., n)`` tau and work in float32 on the tensors' GPU, on the
current stream, with blocked-WY updates on MFMA (32-reflector panels); the result comes back in
H's dtype.
"""
from __future__ import annotations

import torch

from . import _native

__all__ = ["householder_product", "ormqr"]


def _prep(H: torch.Tensor, tau: torch.Tensor, who: str):
    if H.dim() < 2 or H.shape[-1] != H.shape[-2] or tau.shape != H.shape[:-1]:
        raise ValueError(f"{who}: expected H of shape (..., n, n) and tau of shape (..., n)")
    if not (H.is_cuda and tau.is_cuda):
        raise RuntimeError(f"{who}: runs on the GPU only (no CPU fallback)")
    n = int(H.shape[-1])
    Hf = H.to(torch.float32).reshape(-1, n, n).contiguous()
    tf = tau.to(torch.float32).reshape(-1, n).contiguous()
    return Hf, tf, n


def householder_product(H: torch.Tensor, tau: torch.Tensor) -> torch.Tensor:
    """Q = H_0 H_1 ... H_{n-1} from the compact factorization (torch.linalg.householder_product)."""
    Hf, tf, n = _prep(H, tau, "householder_product")
    batch = Hf.shape[0]
    Q = torch.empty_like(Hf)
    if batch:
        need = _native.workspace_bytes("orgqr", batch, n)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=Hf.device)
        with torch.cuda.device(Hf.device):
            st = _native.lib().rnr_orgqr_f32(Hf.data_ptr(), tf.data_ptr(), batch, n, Q.data_ptr(), ws.data_ptr(),
                                             need, torch.cuda.current_stream(Hf.device).cuda_stream)
        _native.check("rnr_orgqr_f32", st)
    return Q.reshape(H.shape).to(H.dtype)


def ormqr(H: torch.Tensor, tau: torch.Tensor, C: torch.Tensor, transpose: bool = False) -> torch.Tensor:
    """Q C (or Q^T C with ``transpose``) for C of shape (..., n, k) (torch.ormqr, left side)."""
    Hf, tf, n = _prep(H, tau, "ormqr")
    if C.dim() < 2 or C.shape[-2] != n or C.shape[:-2] != H.shape[:-2]:
        raise ValueError("ormqr: C must have shape (..., n, k) with H's batch dimensions")
    if not C.is_cuda:
        raise RuntimeError("ormqr: runs on the GPU only (no CPU fallback)")
    k = int(C.shape[-1])
    Y = C.to(torch.float32).reshape(-1, n, k).clone(memory_format=torch.contiguous_format)
    batch = Y.shape[0]
    if batch and k:
        need = _native.workspace_bytes("ormqr", batch, n)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=Y.device)
        with torch.cuda.device(Y.device):
            st = _native.lib().rnr_ormqr_f32(Hf.data_ptr(), tf.data_ptr(), batch, n, Y.data_ptr(), k, k, n * k,
                                             1 if transpose else 0, ws.data_ptr(), need,
                                             torch.cuda.current_stream(Y.device).cuda_stream)
        _native.check("rnr_ormqr_f32", st)
    return Y.reshape(C.shape).to(C.dtype)
