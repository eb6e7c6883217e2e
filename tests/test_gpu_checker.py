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


def test_gpu_checker_fails_nan(chk, rnr, wl):
    """A NaN in R, in a reflector tail or in tau fails both gates, as in the reference checker
    (whose `<` comparisons are False for NaN, common/oracle.py:166-168) and its CPU
    restatement; the untouched matrices still pass."""
    print("[case] checker NaN planting", flush=True)
    A = wl.make_batch(4, batch=4, n=96, seed=9)
    H, tau = rnr.custom_kernel(A.to(DEV))
    H, tau = H.clone(), tau.clone()
    H[0, 2, 5] = float("nan")
    H[1, 9, 3] = float("nan")
    tau[2, 4] = float("nan")
    Ad = A.to(DEV)
    _, _, _, _, ok = chk.check(Ad, H, tau)
    _, _, okc = chk.check_percol(Ad, H, tau)
    f, o, r = chk.gate_values(Ad, H, tau)
    torch.cuda.synchronize()
    assert ok.cpu().tolist() == [False, False, False, True], (f, o)
    assert okc.cpu().tolist() == [False, False, False, True], (r, o)
    _, _, _, _, okcpu = checker.check(A, H.cpu(), tau.cpu())
    assert okcpu.tolist() == ok.cpu().tolist()


def _full_batch_gates(chk, A, H, tau, label, margin=100.0):
    assert bool(torch.isfinite(H).all()) and bool(torch.isfinite(tau).all()), label
    assert tau.min().item() >= 1.0 - 16 * checker.EPS32 and tau.max().item() <= 2.0, label
    fac, orth, ft, ot, ok = chk.check(A, H, tau)
    ratio, _, okc = chk.check_percol(A, H, tau)
    torch.cuda.synchronize()
    print(f"{label}: factor {fac:.3e} (gate {ft:.3e}) ortho {orth:.3e} (gate {ot:.3e}) percol {ratio:.3e}")
    assert bool(ok.all()) and bool(okc.all()), label
    assert fac < ft / margin and orth < ot / margin, label  # the reference's own margins are ~1e5


def test_full_headline_batch_passes_the_gates_on_gpu(chk, rnr, wl):
    """Configuration 4 at full size (256 x 512, six classes): every matrix within both gates and
    the per-column gate -- checked in float64 on the GPU."""
    print("[case] config 4 full batch gates on GPU", flush=True)
    A = wl.make_batch(4).to(DEV)
    H, tau = rnr.custom_kernel(A)
    _full_batch_gates(chk, A, H, tau, "config 4")


def test_full_large_n_batch_passes_the_gates_on_gpu(chk, rnr, wl):
    """Configuration 5 at full size (16 x 2048): the split form (one launch per panel)."""
    print("[case] config 5 full batch gates on GPU", flush=True)
    A = wl.make_batch(5).to(DEV)
    H, tau = rnr.custom_kernel(A)
    _full_batch_gates(chk, A, H, tau, "config 5")


def test_full_mid_batch_passes_the_gates_on_gpu(chk, rnr, wl):
    """Configuration 3 at full size (1024 x 128, sigma in [1e-6, 1]): the 128-row solve blocks
    that only a batch this large selects."""
    print("[case] config 3 full batch gates on GPU", flush=True)
    A = wl.make_batch(3).to(DEV)
    H, tau = rnr.custom_kernel(A)
    _full_batch_gates(chk, A, H, tau, "config 3")


def test_full_small_n_batch_passes_the_gates_on_gpu(chk, rnr, wl):
    """Configuration 2 at full size (4096 x 32): every matrix through the GPU checker."""
    print("[case] config 2 full batch gates on GPU", flush=True)
    A = wl.make_batch(2).to(DEV)
    H, tau = rnr.custom_kernel(A)
    _full_batch_gates(chk, A, H, tau, "config 2")
