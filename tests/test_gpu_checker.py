"""The GPU fp64 gate checker (rnr_check_f64, qr-contest_amd/check.py) against the CPU fp64
restatement of the reference checker (oracle/checker.py <- common/oracle.py:152-195).

Both evaluate the same float64 formulas on the same float32 (A, H, tau); they differ only in
the order of float64 rounding, so the gate values must agree to float64 accuracy relative to
the quantities being differenced: |gpu - cpu| <= 1e-9 * max(1, value scale) with the scale of
the residual's summands, i.e. an absolute 1e-11 on values that are themselves ~1e-7..1e-3."""
import importlib

import pytest
import torch

from oracle import checker

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def chk():
    return importlib.import_module("qr-contest_amd.check")


@pytest.fixture(scope="module")
def rnr():
    return importlib.import_module("qr-contest_amd.reflection_no_reflectors")


@pytest.fixture(scope="module")
def wl():
    return importlib.import_module("qr-contest_amd.workloads")


def _cpu_values(A, H, tau):
    fac, orth = checker.factor_and_ortho(A, H, tau)
    Ad, Hd, td = A.double(), H.double(), tau.double()
    Q = torch.linalg.householder_product(Hd, td)
    res = (torch.triu(Hd) - Q.mT @ Ad).abs().sum(dim=-2)
    acol = Ad.abs().sum(dim=-2).clamp_min(1e-300)
    ft, _ = checker.gates(A.shape[-1])
    ratio = (res / (ft * acol)).amax(dim=-1)
    return fac, orth, ratio


@pytest.mark.parametrize("b,n", [(6, 16), (4, 64), (3, 100), (2, 257), (2, 512)])
def test_gpu_checker_matches_cpu_checker(chk, rnr, wl, b, n):
    print(f"[case] checker b={b} n={n}", flush=True)
    A = wl.make_batch(4, batch=b, n=n, seed=7)
    H, tau = rnr.custom_kernel(A.to(DEV))
    # one matrix with a planted 1% error in R, one with a perturbed tau: both must fail
    H2, tau2 = H.clone(), tau.clone()
    H2[0] = H2[0] + 0.01 * torch.triu(H2[0])
    tau2[-1, 0] = tau2[-1, 0] * 1.01
    for Hx, tx in ((H, tau), (H2, tau2)):
        f, o, r = chk.gate_values(A.to(DEV), Hx, tx)
        torch.cuda.synchronize()
        fc, oc, rc = _cpu_values(A, Hx.cpu(), tx.cpu())
        assert torch.allclose(f.cpu(), fc, rtol=1e-9, atol=1e-11), (f, fc)
        assert torch.allclose(o.cpu(), oc, rtol=1e-9, atol=1e-11), (o, oc)
        assert torch.allclose(r.cpu(), rc, rtol=1e-9, atol=1e-9), (r, rc)
    _, _, _, _, ok = chk.check(A.to(DEV), H2, tau2)
    assert not bool(ok[0]) and not bool(ok[-1])


def test_gpu_checker_exact_factorization_passes_tightly(chk):
    """(H, tau) of torch.geqrf in float64 rounded to float32: factor and ortho at fp32 level."""
    g = torch.Generator().manual_seed(3)
    A = torch.randn(4, 96, 96, generator=g, dtype=torch.float64)
    Hg, tg = torch.geqrf(A)
    A32, H32, t32 = A.float(), Hg.float(), tg.float()
    f, o, r = chk.gate_values(A32.to(DEV), H32.to(DEV), t32.to(DEV))
    torch.cuda.synchronize()
    assert f.max().item() < 1e-5 and o.max().item() < 1e-5


def test_full_headline_batch_passes_the_gates_on_gpu(chk, rnr, wl):
    """Configuration 4 at full size (256 x 512, six classes): every matrix within both gates and
    the per-column gate -- checked in float64 on the GPU."""
    print("[case] config 4 full batch gates on GPU", flush=True)
    A = wl.make_batch(4).to(DEV)
    H, tau = rnr.custom_kernel(A)
    fac, orth, ft, ot, ok = chk.check(A, H, tau)
    ratio, _, okc = chk.check_percol(A, H, tau)
    torch.cuda.synchronize()
    print(f"factor {fac:.3e} (gate {ft:.3e}) ortho {orth:.3e} (gate {ot:.3e}) percol {ratio:.3e}")
    assert bool(ok.all()) and bool(okc.all())
    assert fac < ft / 100 and orth < ot / 100  # the reference's own margins are ~1e5


def test_full_large_n_batch_passes_the_gates_on_gpu(chk, rnr, wl):
    """Configuration 5 at full size (16 x 2048)."""
    print("[case] config 5 full batch gates on GPU", flush=True)
    A = wl.make_batch(5).to(DEV)
    H, tau = rnr.custom_kernel(A)
    fac, orth, ft, ot, ok = chk.check(A, H, tau)
    torch.cuda.synchronize()
    print(f"factor {fac:.3e} (gate {ft:.3e}) ortho {orth:.3e} (gate {ot:.3e})")
    assert bool(ok.all())
