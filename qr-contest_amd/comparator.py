"""Benchmark comparator: Householder blocked-WY QR in ``torch.geqrf`` layout on the GPU
(``rnr_hh_geqrf_f32``).  The reflector-free path (``custom_kernel``) never calls it; ``bench.py``
times it on the same batch as the classical speed reference, as the reference does for its own
route (``householder/submission_routed_v3.py:225-281``).
"""
from __future__ import annotations

import torch

from . import _native

__all__ = ["hh_geqrf"]


def hh_geqrf(A: torch.Tensor):
    """``(H, tau)`` of ``A`` (``(..., n, n)``, float32 on the GPU) in ``torch.geqrf`` layout."""
    if A.dim() < 2 or A.shape[-1] != A.shape[-2]:
        raise ValueError("hh_geqrf: expected (..., n, n)")
    if not A.is_cuda:
        raise RuntimeError("hh_geqrf: runs on the GPU only (no CPU fallback)")
    n = int(A.shape[-1])
    H = A.to(torch.float32).reshape(-1, n, n).clone(memory_format=torch.contiguous_format)
    batch = H.shape[0]
    tau = torch.empty(batch, n, dtype=torch.float32, device=H.device)
    if batch:
        need = _native.workspace_bytes("hh_geqrf", batch, n)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=H.device)
        with torch.cuda.device(H.device):
            st = _native.lib().rnr_hh_geqrf_f32(H.data_ptr(), batch, n, tau.data_ptr(), ws.data_ptr(), need,
                                               torch.cuda.current_stream(H.device).cuda_stream)
        _native.check("rnr_hh_geqrf_f32", st)
    return H.reshape(A.shape), tau.reshape(A.shape[:-1])
