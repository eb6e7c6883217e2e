"""Pinning of the generator oracle (oracle/gen.py) on the CPU.

Each check is fixed by something outside the restatement: published known-answer vectors, the
normal / uniform CDFs (scipy), numpy's QR of a Gaussian matrix (the textbook Haar sampler), and
numpy's SVD for the prescribed spectra."""
import numpy as np
import pytest
from scipy import stats

from oracle import gen


# Random123 kat_vectors, philox4x32 with 10 rounds: (counter, key) -> output
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,out", KAT)
def test_philox_known_answers(ctr, key, out):
    w = gen.philox4x32(*[np.array([c], dtype=np.uint64) for c in ctr], *key)
    assert tuple(int(x[0]) for x in w) == out


def test_uniform_and_normal_streams_match_their_distributions():
    e = np.arange(200_000)
    u = gen.uniforms(7, 3, gen.P_ROW, e)
    assert u.min() >= 0.0 and u.max() < 1.0
    assert stats.kstest(u, "uniform").pvalue > 1e-4
    z = gen.normals(7, 3, gen.P_DENSE, e)
    assert stats.kstest(z, "norm").pvalue > 1e-4
    assert abs(z.mean()) < 5 / np.sqrt(z.size)
    assert abs(z.var() - 1.0) < 5 * np.sqrt(2 / z.size)
    assert abs((z ** 4).mean() - 3.0) < 5 * np.sqrt(96 / z.size)
    # the two halves of a draw are independent (no correlation between z0 and z1)
    assert abs(np.corrcoef(z[0::2], z[1::2])[0, 1]) < 5 / np.sqrt(z.size / 2)


def test_streams_are_separated_by_seed_matrix_and_purpose():
    e = np.arange(64)
    base = gen.normals(1, 0, gen.P_DENSE, e)
    for other in (gen.normals(2, 0, gen.P_DENSE, e), gen.normals(1, 1, gen.P_DENSE, e),
                  gen.normals(1, 0, gen.P_U, e)):
        assert not np.any(base == other)


def _numpy_haar(rng, n):
    Z = rng.standard_normal((n, n))
    Q, R = np.linalg.qr(Z)
    return Q * np.sign(np.diag(R))[None, :]


def test_stewart_haar_is_orthogonal_and_haar_distributed():
    Q = gen.haar(5, 0, gen.P_U, 40)
    assert np.abs(Q.T @ Q - np.eye(40)).max() < 1e-13
    n, N = 4, 3000
    st = np.stack([gen.haar(11, i, gen.P_W, n) for i in range(N)])
    rng = np.random.default_rng(0)
    ref = np.stack([_numpy_haar(rng, n) for _ in range(N)])
    tr = np.trace(st, axis1=1, axis2=2)
    # Haar on O(n): E tr Q = 0, E (tr Q)^2 = 1; without the sign fix E tr Q is about -0.8 at n = 4
    assert abs(tr.mean()) < 5 / np.sqrt(N)
    assert abs((tr ** 2).mean() - 1.0) < 0.15
    for stat in (lambda Q: Q[:, 0, 0], lambda Q: Q[:, 1, 2], lambda Q: np.trace(Q, axis1=1, axis2=2),
                 lambda Q: np.linalg.det(Q)):
        assert stats.ks_2samp(stat(st), stat(ref)).pvalue > 1e-4


def test_stewart_matches_the_sign_fixed_qr_of_its_gaussian_columns():
    """Stewart's reflector k comes from an independent Gaussian vector: for k = 0 it IS column 0
    of a Gaussian matrix, so Q[:, 0] = sign-fixed normalized column (closed form)."""
    n = 9
    x = gen.normals(3, 2, gen.P_U, np.arange(n))
    Q = gen.haar(3, 2, gen.P_U, n)
    assert np.allclose(Q[:, 0], x / np.linalg.norm(x), atol=1e-14)


@pytest.mark.parametrize("config,i,spec", [(4, 1, ("log", 12.0)), (4, 2, ("headtail", 0.0)),
                                            (4, 4, ("headtail", 1e-10)), (3, 0, ("log", 6.0)),
                                            (5, 1, ("log", 8.0))])
def test_haar_classes_have_the_prescribed_singular_values(config, i, spec):
    n = 24
    A = gen.matrix64(config, i, n, seed=4)
    sv = np.linalg.svd(A, compute_uv=False)
    s = np.sort(gen.sigma(spec, n))[::-1]
    assert np.abs(sv - s).max() < 1e-13
    assert gen.recipe(config, i)[0] == gen.HAAR


def test_sigma_specs_follow_logspace():
    assert np.allclose(gen.sigma(("log", 12.0), 5), np.logspace(0, -12, 5), rtol=1e-14)
    s = gen.sigma(("headtail", 1e-10), 10)
    assert np.allclose(s[:5], np.logspace(0, -1, 5), rtol=1e-14) and np.all(s[5:] == 1e-10)
    assert np.all(gen.sigma(("headtail", 0.0), 1) == 0.0)
    assert np.all(gen.sigma(("log", 3.0), 1) == 1.0)


def test_direct_classes():
    n = 16
    Z = gen.normals(9, 0, gen.P_DENSE, np.arange(n * n)).reshape(n, n)
    assert np.array_equal(gen.matrix64(4, 0, n, 9), Z)
    R = gen.matrix64(4, 5, n, 9)
    assert np.array_equal(R, np.triu(gen.normals(9, 5, gen.P_DENSE, np.arange(n * n)).reshape(n, n)))
    S = gen.matrix64(4, 3, n, 9)
    Z3 = gen.normals(9, 3, gen.P_DENSE, np.arange(n * n)).reshape(n, n)
    expo = np.log10(S / Z3)
    assert np.allclose(expo, expo[:, :1], atol=1e-12)       # one scale per row
    assert expo.min() >= -6.0 and expo.max() <= 6.0


def test_config_layout_and_prefix_stability():
    assert [gen.recipe(4, i)[0] for i in range(12)] == [0, 1, 1, 2, 1, 3] * 2
    assert [gen.recipe(5, i)[0] for i in range(4)] == [0, 1, 0, 1]
    a = gen.make_batch(4, 7, 8, seed=1)
    b = gen.make_batch(4, 3, 8, seed=1)
    assert np.array_equal(a[:3], b)
