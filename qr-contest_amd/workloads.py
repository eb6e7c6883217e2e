"""Seeded synthetic batches for the five benchmark configurations.

The reference ships no generators for this path: its dev scaffolding builds
test batches in ``common/oracle.py:43-146`` (``_with_singular_values`` at
:53-57, ``gen_rankdef`` at :60-64, ``gen_uppertri`` at :121-123) and the real
contest generators are not vendored (``common/oracle.py:4``).  These follow the
same construction style:

* "dense": i.i.d. N(0, 1) entries;
* "haar(sigma)": ``U diag(sigma) V^T`` with U, V Haar-distributed orthogonal
  matrices, drawn as the Q factor of an N(0, 1) matrix with the signs of
  ``diag(R)`` folded into Q (the standard Haar correction);
* "rowscaled": N(0, 1) with row i multiplied by ``10**u_i``, u_i ~ U(-6, 6);
* "uppertri": ``triu`` of an N(0, 1) matrix.

Everything is generated in float64 from a ``torch.Generator`` seeded with the
configuration's seed and cast to float32 at the end.  The same call on another
device (``device='cuda'``) yields a different (but equally distributed) batch,
because the random streams of the two devices differ.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

__all__ = ["CONFIGS", "Config", "make_batch", "haar", "with_singular_values",
           "HEADLINE_CLASSES", "headline_class_batch", "STRESS_CASES", "stress_batch"]


@dataclass(frozen=True)
class Config:
    idx: int
    name: str
    batch: int
    n: int
    seed: int
    # bytes and nominal flops per matrix, used for the roofline figures
    @property
    def bytes_per_matrix(self) -> int:
        return 4 * (2 * self.n * self.n + self.n)

    @property
    def nominal_flops_per_matrix(self) -> float:
        return 4.0 / 3.0 * self.n ** 3


CONFIGS = {
    1: Config(1, "cpu_plumbing_16x64", 16, 64, 0),
    2: Config(2, "small_n_4096x32", 4096, 32, 1),
    3: Config(3, "mid_1024x128_logspace6", 1024, 128, 2),
    4: Config(4, "headline_hetero_256x512", 256, 512, 3),
    5: Config(5, "large_n_16x2048", 16, 2048, 4),
}

# The six pathology classes of the headline batch, cycled as i % 6.
HEADLINE_CLASSES = ("dense", "logspace12", "rankdef", "rowscaled", "nearrank", "uppertri")


def haar(b: int, n: int, gen: torch.Generator, device) -> torch.Tensor:
    """Haar-distributed orthogonal (b, n, n) float64 matrices."""
    Z = torch.randn(b, n, n, dtype=torch.float64, generator=gen, device=device)
    Q, R = torch.linalg.qr(Z)
    d = torch.sign(torch.diagonal(R, dim1=-2, dim2=-1))
    d = torch.where(d == 0, torch.ones_like(d), d)
    return Q * d.unsqueeze(-2)


def with_singular_values(b: int, sigma: torch.Tensor, gen: torch.Generator, device) -> torch.Tensor:
    """(b, n, n) float64 ``U diag(sigma) V^T`` with independent Haar U and V."""
    n = sigma.numel()
    U = haar(b, n, gen, device)
    V = haar(b, n, gen, device)
    return (U * sigma.to(device=device, dtype=torch.float64).view(1, 1, n)) @ V.mT


def _head_tail_sigma(n: int, tail: float) -> torch.Tensor:
    r = n // 2
    s = torch.full((n,), float(tail), dtype=torch.float64)
    s[:r] = torch.logspace(0, -1, r, dtype=torch.float64)
    return s


def headline_class_batch(cls: str, b: int, n: int, gen: torch.Generator, device) -> torch.Tensor:
    """b float64 matrices of one headline class."""
    if cls == "dense":
        return torch.randn(b, n, n, dtype=torch.float64, generator=gen, device=device)
    if cls == "logspace12":
        return with_singular_values(b, torch.logspace(0, -12, n, dtype=torch.float64), gen, device)
    if cls == "rankdef":
        return with_singular_values(b, _head_tail_sigma(n, 0.0), gen, device)
    if cls == "rowscaled":
        A = torch.randn(b, n, n, dtype=torch.float64, generator=gen, device=device)
        u = torch.rand(b, n, 1, dtype=torch.float64, generator=gen, device=device) * 12.0 - 6.0
        return A * torch.pow(10.0, u)
    if cls == "nearrank":
        return with_singular_values(b, _head_tail_sigma(n, 1e-10), gen, device)
    if cls == "uppertri":
        return torch.triu(torch.randn(b, n, n, dtype=torch.float64, generator=gen, device=device))
    raise ValueError(f"unknown class {cls!r}")


def _fill_cycled(classes, b, n, gen, device) -> torch.Tensor:
    out = torch.empty(b, n, n, dtype=torch.float64, device=device)
    k = len(classes)
    for c, cls in enumerate(classes):
        idx = list(range(c, b, k))
        if idx:
            out[idx] = headline_class_batch(cls, len(idx), n, gen, device)
    return out


def make_batch(config: int, *, batch: int | None = None, n: int | None = None,
               device="cpu", dtype=torch.float32, seed: int | None = None) -> torch.Tensor:
    """The seeded batch of BASELINE configuration ``config`` (1..5).

    ``batch`` / ``n`` override the configuration's size (tests use smaller
    instances of the same distribution); ``seed`` overrides its seed.
    """
    cfg = CONFIGS[config]
    b = cfg.batch if batch is None else int(batch)
    nn = cfg.n if n is None else int(n)
    gen = torch.Generator(device=device)
    gen.manual_seed(cfg.seed if seed is None else int(seed))
    if config in (1, 2):
        A = torch.randn(b, nn, nn, dtype=torch.float64, generator=gen, device=device)
    elif config == 3:
        A = with_singular_values(b, torch.logspace(0, -6, nn, dtype=torch.float64), gen, device)
    elif config == 4:
        A = _fill_cycled(HEADLINE_CLASSES, b, nn, gen, device)
    elif config == 5:
        A = _config5(b, nn, gen, device)
    else:
        raise ValueError(config)
    return A.to(dtype).contiguous()


def _config5(b, n, gen, device):
    out = torch.empty(b, n, n, dtype=torch.float64, device=device)
    even = list(range(0, b, 2))
    odd = list(range(1, b, 2))
    if even:
        out[even] = torch.randn(len(even), n, n, dtype=torch.float64, generator=gen, device=device)
    if odd:
        out[odd] = with_singular_values(len(odd), torch.logspace(0, -8, n, dtype=torch.float64),
                                        gen, device)
    return out


def well_conditioned(b: int, n: int, seed: int = 0, device="cpu", lo: float = -2.0,
                     dtype=torch.float32) -> torch.Tensor:
    """Haar U, V with sigma = logspace(0, lo, n): the elementwise-parity input."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    A = with_singular_values(b, torch.logspace(0, lo, n, dtype=torch.float64), gen, device)
    return A.to(dtype).contiguous()


# ----------------------------------------------------------------------------- stress battery
# The reference's nine generator cases (common/oracle.py:43-146, dispatched by make_batch at
# :126-146), which its validation scripts run over n in {176, ..., 4096} and seeds 0..7
# (householder/_validate_v3.py:8-28, householder/tf32_seedvar_derisk.py:28-40).  Built the way
# the reference builds them -- float32 throughout, orthogonal factors as the plain Q of a
# Gaussian matrix -- on any device (the tests run them on the GPU, where the reference's
# generators run too).
STRESS_CASES = ("dense", "mixed", "rankdef", "nearrank", "clustered", "banded", "rowscaled",
                "nearcollinear", "uppertri")


def _stress_gauss(b, n, gen, device):
    return torch.randn(b, n, n, dtype=torch.float32, generator=gen, device=device)


def _stress_sv(b, n, sigma, gen, device):
    """U diag(sigma) V^T with U, V the Q factors of Gaussian matrices (oracle.py:53-57)."""
    U = torch.linalg.qr(_stress_gauss(b, n, gen, device))[0]
    V = torch.linalg.qr(_stress_gauss(b, n, gen, device))[0]
    return (U * sigma.view(1, 1, n)) @ V.mT.contiguous()


def _stress_head(n, device, tail):
    """n/2 singular values logspace(0, -1), the rest `tail` (oracle.py:60-73)."""
    r = n // 2
    s = torch.full((n,), float(tail), dtype=torch.float32, device=device)
    s[:r] = torch.logspace(0, -1, r, device=device)
    return s


def _stress_one(case, b, n, cond, gen, device):
    if case == "dense":  # columns scaled by logspace(0, -cond, n) (oracle.py:48-51)
        return _stress_gauss(b, n, gen, device) * torch.logspace(0, -float(cond), n, device=device).view(1, 1, n)
    if case == "rankdef":
        return _stress_sv(b, n, _stress_head(n, device, 0.0), gen, device)
    if case == "nearrank":
        return _stress_sv(b, n, _stress_head(n, device, 1e-8), gen, device)
    if case == "clustered":  # two clusters, 1 and 1e-6 (oracle.py:76-79)
        s = torch.ones(n, device=device)
        s[n // 2:] = 1e-6
        return _stress_sv(b, n, s, gen, device)
    if case == "mixed":  # dense, every fourth matrix a stress case in turn (oracle.py:82-90)
        A = _stress_one("dense", b, n, cond, gen, device)
        stress = ("rankdef", "nearrank", "clustered")
        for i in range(3, b, 4):
            A[i] = _stress_one(stress[(i // 4) % 3], 1, n, cond, gen, device)[0]
        return A
    if case == "banded":  # zero outside |i - j| <= n / 8 (oracle.py:98-106)
        bw = max(1, n // 8)
        i = torch.arange(n, device=device)
        band = (i.view(n, 1) - i.view(1, n)).abs() <= bw
        return _stress_gauss(b, n, gen, device) * band.view(1, n, n)
    if case == "rowscaled":  # rows scaled by logspace(0, -cond, n) (oracle.py:109-113)
        return _stress_gauss(b, n, gen, device) * torch.logspace(0, -float(cond), n, device=device).view(1, n, 1)
    if case == "nearcollinear":  # column 1 = column 0 + 1e-7 noise (oracle.py:116-121)
        A = _stress_gauss(b, n, gen, device)
        noise = torch.randn(b, n, dtype=torch.float32, generator=gen, device=device)
        A[:, :, 1] = A[:, :, 0] + 1e-7 * noise
        return A
    if case == "uppertri":
        return torch.triu(_stress_gauss(b, n, gen, device))
    raise ValueError(f"unknown stress case {case!r}")


def stress_batch(case: str, b: int, n: int, cond: float = 2.0, seed: int = 0, device="cpu") -> torch.Tensor:
    """b float32 matrices of one of the reference's nine stress cases (STRESS_CASES)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(int(seed))
    return _stress_one(case, int(b), int(n), cond, gen, device).contiguous()
