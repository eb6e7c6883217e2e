"""``custom_kernel(A) -> (H, tau)`` on MI355X through the gfx950 HIP library.

Mirrors ``/root/reference/reflection_no_reflectors.py``: same entry name and contract
(``(..., n, n)`` input of any float dtype, work in fp32, outputs in the input dtype, compact
``torch.geqrf`` layout, batch dimensions kept), same stage names (``_frame``, ``_chart``),
same failure behaviour (a non-positive-definite Gram -- only non-finite input produces
one -- raises ``torch.linalg.LinAlgError`` as ``torch.linalg.cholesky`` does at ``:76``;
a non-square input raises).  Every FLOP runs in ``librnrqr.so`` on the tensor's GPU, on
the current stream; there is no CPU path: CPU tensors are rejected.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native

__all__ = ["custom_kernel", "qr", "QRPlan", "_frame", "_chart", "lu", "cholqr"]


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _as_batch(data: torch.Tensor, who: str):
    if data.dim() < 2 or data.shape[-1] != data.shape[-2]:
        raise ValueError(f"{who}: expected a (..., n, n) square input, got {tuple(data.shape)}")
    if not data.is_cuda:
        raise RuntimeError(f"{who}: input is on {data.device}; librnrqr runs on the GPU only "
                           "(no CPU fallback)")
    n = int(data.shape[-1])
    if n > _native.RNR_MAX_N:
        raise ValueError(f"{who}: n = {n} exceeds the supported maximum {_native.RNR_MAX_N}")
    A = data.to(torch.float32).reshape(-1, n, n)
    if not A.is_contiguous():
        A = A.contiguous()
    return A, n, data.shape[:-2]


def _workspace(kind: str, batch: int, n: int, device) -> torch.Tensor:
    nbytes = _native.workspace_bytes(kind, batch, n)
    # torch's caching allocator returns 512-byte aligned blocks, above the 256 the ABI needs
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def _check_f32_rows(A: torch.Tensor, who: str) -> int:
    """n of a float32 (batch, n, n) CUDA tensor whose rows are contiguous; raises otherwise."""
    if A.dim() != 3 or A.shape[-1] != A.shape[-2]:
        raise ValueError(f"{who}: expected a (batch, n, n) tensor, got {tuple(A.shape)}")
    if A.dtype != torch.float32:
        raise ValueError(f"{who}: expected float32, got {A.dtype}")
    if not A.is_cuda:
        raise RuntimeError(f"{who}: input is on {A.device}; librnrqr runs on the GPU only")
    n = int(A.shape[-1])
    if n > _native.RNR_MAX_N:
        raise ValueError(f"{who}: n = {n} exceeds the supported maximum {_native.RNR_MAX_N}")
    if n > 0 and (A.stride(-1) != 1 or (n > 1 and A.stride(-2) != n)):
        raise ValueError(f"{who}: rows must be contiguous with row stride n")
    return n


def _raise_on_info(info: torch.Tensor) -> None:
    bad = torch.nonzero(info).flatten()
    if bad.numel():
        i = int(bad[0])
        k = int(info[i])
        raise torch.linalg.LinAlgError(
            f"custom_kernel: the Cholesky of matrix {i} could not be completed because the Gram "
            f"matrix is not positive-definite (leading minor of order {k}); the input holds "
            "non-finite values")


class QRPlan:
    """Preallocated buffers for repeated factorizations of one (batch, n) on one device.

    ``run(A)`` launches the whole path on the current stream and returns (H, tau) views
    into the plan's own output buffers; it neither allocates nor synchronizes.
    """

    def __init__(self, batch: int, n: int, device="cuda"):
        self.batch, self.n = int(batch), int(n)
        self.device = torch.device(device)
        self.ws = _workspace("qr", self.batch, self.n, self.device)
        self.H = torch.empty(self.batch, self.n, self.n, dtype=torch.float32, device=self.device)
        self.tau = torch.empty(self.batch, self.n, dtype=torch.float32, device=self.device)
        self.info = torch.zeros(self.batch, dtype=torch.int32, device=self.device)

    def run(self, A: torch.Tensor, stream: int | None = None):
        _check_f32_rows(A, "QRPlan.run")
        if tuple(A.shape) != (self.batch, self.n, self.n):
            raise ValueError(f"QRPlan.run: expected shape {(self.batch, self.n, self.n)}, got {tuple(A.shape)}")
        if A.device != self.H.device:
            raise ValueError(f"QRPlan.run: input is on {A.device}, the plan on {self.H.device}")
        bs = A.stride(0) if self.batch > 1 else self.n * self.n
        with torch.cuda.device(self.H.device):
            st = _native.lib().rnr_qr_f32(
                A.data_ptr(), self.batch, self.n, bs, self.H.data_ptr(), self.tau.data_ptr(),
                self.info.data_ptr(), self.ws.data_ptr(), self.ws.numel(),
                _stream(self.H.device) if stream is None else stream)
        _native.check("rnr_qr_f32", st)
        return self.H, self.tau


def qr(A: torch.Tensor, check_errors: bool = True):
    """(H, tau) of a float32 (batch, n, n) CUDA tensor with contiguous rows."""
    n = _check_f32_rows(A, "qr")
    batch = int(A.shape[0])
    H = torch.empty(batch, n, n, dtype=torch.float32, device=A.device)
    tau = torch.empty(batch, n, dtype=torch.float32, device=A.device)
    if batch == 0:
        return H, tau
    ws = _workspace("qr", batch, n, A.device)
    info = torch.zeros(batch, dtype=torch.int32, device=A.device)
    bs = A.stride(0) if batch > 1 else n * n
    with torch.cuda.device(A.device):
        st = _native.lib().rnr_qr_f32(A.data_ptr(), batch, n, bs, H.data_ptr(), tau.data_ptr(),
                                      info.data_ptr(), ws.data_ptr(), ws.numel(), _stream(A.device))
    _native.check("rnr_qr_f32", st)
    if check_errors:
        _raise_on_info(info)
    return H, tau


def custom_kernel(data: torch.Tensor):
    """(H, tau) in geqrf layout -- reference ``custom_kernel``, reflection_no_reflectors.py:181-196."""
    dtype = data.dtype
    A, n, lead = _as_batch(data, "custom_kernel")
    H, tau = qr(A)
    return H.reshape(*lead, n, n).to(dtype), tau.reshape(*lead, n).to(dtype)


# ----------------------------------------------------------------------------- stages


def lu(data: torch.Tensor):
    """(perm, L): partial-pivot LU, ``A[perm] = L U`` (torch.linalg.lu at reference :66)."""
    A, n, lead = _as_batch(data, "lu")
    batch = A.shape[0]
    L = torch.empty_like(A)
    perm = torch.empty(batch, n, dtype=torch.int32, device=A.device)
    if batch:
        ws = _workspace("lu", batch, n, A.device)
        with torch.cuda.device(A.device):
            st = _native.lib().rnr_lu_f32(A.data_ptr(), batch, n, n * n, L.data_ptr(), perm.data_ptr(),
                                          ws.data_ptr(), ws.numel(), _stream(A.device))
        _native.check("rnr_lu_f32", st)
    return perm.reshape(*lead, n).long(), L.reshape(*lead, n, n)


def cholqr(data: torch.Tensor, check_errors: bool = True):
    """(Q, R): one jittered CholeskyQR pass, Q = M R^-1 (``_cholqr`` at reference :68-77).

    R is returned upper-triangular (its strict lower part is zeroed here)."""
    M, n, lead = _as_batch(data, "cholqr")
    batch = M.shape[0]
    Q = torch.empty_like(M)
    R = torch.empty_like(M)
    info = torch.zeros(max(batch, 1), dtype=torch.int32, device=M.device)
    if batch:
        ws = _workspace("cholqr", batch, n, M.device)
        with torch.cuda.device(M.device):
            st = _native.lib().rnr_cholqr_f32(M.data_ptr(), batch, n, n * n, Q.data_ptr(), R.data_ptr(),
                                              info.data_ptr(), ws.data_ptr(), ws.numel(),
                                              _stream(M.device))
        _native.check("rnr_cholqr_f32", st)
        if check_errors:
            _raise_on_info(info)
    return Q.reshape(*lead, n, n), torch.triu(R).reshape(*lead, n, n)


def _frame(data: torch.Tensor, check_errors: bool = True) -> torch.Tensor:
    """The orthogonal frame Q = P CholQR2(L) (reference ``_frame``, :55-81)."""
    A, n, lead = _as_batch(data, "_frame")
    batch = A.shape[0]
    Q = torch.empty_like(A)
    info = torch.zeros(max(batch, 1), dtype=torch.int32, device=A.device)
    if batch:
        ws = _workspace("frame", batch, n, A.device)
        with torch.cuda.device(A.device):
            st = _native.lib().rnr_frame_f32(A.data_ptr(), batch, n, n * n, Q.data_ptr(), info.data_ptr(),
                                             ws.data_ptr(), ws.numel(), _stream(A.device))
        _native.check("rnr_frame_f32", st)
        if check_errors:
            _raise_on_info(info)
    return Q.reshape(*lead, n, n)


def _chart(Q: torch.Tensor):
    """(Y, s, tau) of an orthonormal Q (reference ``_chart``, :86-176, and tau at :192).

    Y holds the reflector tails strictly below the diagonal and zeros elsewhere."""
    M, n, lead = _as_batch(Q, "_chart")
    M = M.clone()
    batch = M.shape[0]
    s = torch.empty(batch, n, dtype=torch.float32, device=M.device)
    tau = torch.empty(batch, n, dtype=torch.float32, device=M.device)
    if batch:
        with torch.cuda.device(M.device):
            st = _native.lib().rnr_chart_f32(M.data_ptr(), batch, n, s.data_ptr(), tau.data_ptr(),
                                             _stream(M.device))
        _native.check("rnr_chart_f32", st)
    return torch.tril(M, -1).reshape(*lead, n, n), s.reshape(*lead, n), tau.reshape(*lead, n)
