"""Device generators (rnr_generate_f32, qr-contest_amd/generate.py) against the numpy oracle
(oracle/gen.py, pinned in tests/test_oracle_gen.py) and at full size through properties.

Tolerance against the oracle: both compute in float64 and round once to float32; the float64
values differ in the last bits (libm, and blocked versus unblocked reflector products), so an
entry may round to the neighbouring float32: |gpu - oracle| <= 1 ulp32(|oracle|) + 1e-12 max|A|.
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import gen as ogen

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def g():
    return importlib.import_module("qr-contest_amd.generate")


def _close_to_oracle(A, ref):
    A = A.astype(np.float64)
    ref64 = ref.astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    tol = ulp + 1e-12 * np.abs(ref64).max()
    bad = np.abs(A - ref64) > tol
    return int(bad.sum()), float(np.abs(A - ref64).max())


@pytest.mark.parametrize("config,b,n", [(1, 6, 8), (2, 8, 32), (3, 4, 33), (4, 12, 24), (4, 6, 64),
                                        (5, 4, 40), (4, 7, 1), (4, 7, 2)])
def test_device_batch_matches_oracle(g, config, b, n):
    print(f"[case] gen config={config} b={b} n={n}", flush=True)
    A = g.device_batch(config, batch=b, n=n, seed=21, device=DEV).cpu().numpy()
    ref = ogen.make_batch(config, b, n, seed=21)
    nbad, err = _close_to_oracle(A, ref)
    assert nbad == 0, (nbad, err)


def test_deterministic_and_prefix_stable(g):
    a = g.device_batch(4, batch=18, n=48, seed=5, device=DEV)
    b = g.device_batch(4, batch=18, n=48, seed=5, device=DEV)
    c = g.device_batch(4, batch=7, n=48, seed=5, device=DEV)
    d = g.device_batch(4, batch=7, n=48, seed=6, device=DEV)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(a[:7], c)
    assert not torch.equal(c, d)


def test_full_headline_batch_classes(g):
    """256 x 512^2 on the device: spectra of the Haar classes, the direct classes' structure."""
    A = g.device_batch(4, device=DEV)
    torch.cuda.synchronize()
    assert A.shape == (256, 512, 512) and torch.isfinite(A).all()
    n = 512
    for i, spec in ((1, ("log", 12.0)), (2, ("headtail", 0.0)), (4, ("headtail", 1e-10)), (253, ("log", 12.0))):
        sv = torch.linalg.svdvals(A[i].cpu().double()).numpy()
        s = np.sort(ogen.sigma(spec, n))[::-1]
        assert np.abs(sv - s).max() < 1e-5, (i, np.abs(sv - s).max())
    dense = A[0::6].cpu().double()
    assert abs(dense.mean().item()) < 1e-3 and abs(dense.var().item() - 1.0) < 1e-2
    up = A[5::6].cpu()
    assert torch.equal(up, torch.triu(up))
    rs = A[3::6].cpu().double().abs()
    rowmax = rs.amax(dim=-1)
    assert rowmax.max().item() < 1e7 and rowmax.min().item() > 1e-7


def test_path_on_device_batch_passes_the_gates(g):
    rnr = importlib.import_module("qr-contest_amd.reflection_no_reflectors")
    chk = importlib.import_module("qr-contest_amd.check")
    A = g.device_batch(4, device=DEV)
    H, tau = rnr.custom_kernel(A)
    factor, ortho, _ = chk.gate_values(A, H, tau)
    gf, go = chk.gates(512)
    assert factor.max().item() <= gf and ortho.max().item() <= go
