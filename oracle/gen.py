"""numpy restatement of the device-side seeded generators -- TEST INFRASTRUCTURE ONLY.

The reference builds its test batches in ``common/oracle.py:43-146`` with torch's generator:
Gaussian entries (``_randn`` :43-44), column/row log-scaling (:47-50, :112-116), prescribed
singular values through two Haar-distributed orthogonal factors (``_with_singular_values``
:53-57), rank-deficient / near-rank / clustered spectra (:60-82), and ``triu`` (:121-123).
The five benchmark configurations of this build draw from those constructions (the
class table is in ``qr-contest_amd/workloads.py``).  The device generator
(``rnr_generate_f32``) defines its own random streams, so it is compared with THIS module,
which follows the same stream layout step by step:

* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
  SC 2011), key = (seed low, seed high), counter = (t low, t high, purpose, matrix index);
* a 53-bit uniform from each 64-bit half of the output (u = (w0:w1 >> 11) 2^-53);
* Box-Muller: z0 = r cos(2 pi u_b), z1 = r sin(2 pi u_b), r = sqrt(-2 log(1 - u_a)); element e
  of a stream is z_{e mod 2} of draw t = e // 2;
* Haar factors by Stewart's construction (G. W. Stewart, "The efficient generation of random
  orthogonal matrices with an application to condition estimators", SIAM J. Numer. Anal. 17,
  1980): reflector k is the LAPACK ``dlarfg`` Householder vector of an independent
  N(0, I_{n-k}) vector (stream elements k n + j, j < n - k), and Q = H_0 ... H_{n-1} D with
  D = diag(sign(beta_k)) -- the Q factor of a Gaussian matrix with the signs of diag(R) folded
  in, the construction ``workloads.haar`` uses;
* A = U diag(sigma) W with U, W independent Haar (purposes 1 and 2), formed as
  Y = W_H; Y[r, c] *= sigma_r dU_r dW_c; Y = U_H Y; A = float32(Y).

Pinning (``tests/test_oracle_gen.py``): the published Philox4x32-10 known-answer vectors; the
normal and uniform streams against their CDFs (Kolmogorov-Smirnov) and moments; the Haar
factors against numpy's QR of a Gaussian matrix with the sign fix (two-sample KS on entries and
traces, E tr Q = 0, E tr(Q)^2 = 1, Q^T Q = I); the composed matrices against their prescribed
singular values (numpy SVD); class layout and prefix stability.
"""
from __future__ import annotations

import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK = np.uint64(0xFFFFFFFF)

# purposes (counter word 2)
P_DENSE, P_U, P_W, P_ROW = 0, 1, 2, 3

# classes
DENSE, HAAR, ROWSCALED, UPPERTRI = 0, 1, 2, 3
HEADLINE = (("dense", DENSE, None), ("logspace12", HAAR, ("log", 12.0)),
            ("rankdef", HAAR, ("headtail", 0.0)), ("rowscaled", ROWSCALED, None),
            ("nearrank", HAAR, ("headtail", 1e-10)), ("uppertri", UPPERTRI, None))


def philox4x32(c0, c1, c2, c3, k0, k1):
    """Philox4x32-10 on arrays of counters (uint32 values held in uint64 arrays)."""
    c = [np.asarray(x, dtype=np.uint64) & MASK for x in (c0, c1, c2, c3)]
    k0, k1 = int(k0) & 0xFFFFFFFF, int(k1) & 0xFFFFFFFF
    for _ in range(10):
        p0 = M0 * c[0]
        p1 = M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK
        c = [hi1 ^ c[1] ^ np.uint64(k0), lo1, hi0 ^ c[3] ^ np.uint64(k1), lo0]
        k0, k1 = (k0 + W0) & 0xFFFFFFFF, (k1 + W1) & 0xFFFFFFFF
    return c


def _draws(seed, matrix, purpose, t):
    t = np.asarray(t, dtype=np.uint64)
    w = philox4x32(t & MASK, t >> np.uint64(32), np.full_like(t, purpose), np.full_like(t, matrix),
                   seed & 0xFFFFFFFF, seed >> 32)
    ua = ((w[0] << np.uint64(32) | w[1]) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    ub = ((w[2] << np.uint64(32) | w[3]) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    return ua, ub


def uniforms(seed, matrix, purpose, e):
    """Uniform [0, 1) element(s) e of stream (seed, matrix, purpose)."""
    e = np.asarray(e, dtype=np.int64)
    ua, ub = _draws(seed, matrix, purpose, (e >> 1).astype(np.uint64))
    return np.where((e & 1) == 0, ua, ub)


def normals(seed, matrix, purpose, e):
    """N(0, 1) element(s) e of stream (seed, matrix, purpose) by Box-Muller."""
    e = np.asarray(e, dtype=np.int64)
    ua, ub = _draws(seed, matrix, purpose, (e >> 1).astype(np.uint64))
    r = np.sqrt(-2.0 * np.log1p(-ua))
    th = 2.0 * np.pi * ub
    return np.where((e & 1) == 0, r * np.cos(th), r * np.sin(th))


def reflectors(seed, matrix, purpose, n):
    """Stewart's Haar reflectors: (V [n, n] with v_k in column k below the diagonal, tau, d)."""
    V = np.zeros((n, n))
    tau = np.zeros(n)
    d = np.ones(n)
    for k in range(n):
        x = normals(seed, matrix, purpose, k * n + np.arange(n - k))
        alpha, xn = x[0], np.linalg.norm(x[1:])
        if xn == 0.0:
            d[k] = 1.0 if alpha >= 0 else -1.0
            continue
        beta = -np.copysign(np.hypot(alpha, xn), alpha)
        tau[k] = (beta - alpha) / beta
        V[k + 1:, k] = x[1:] / (alpha - beta)
        d[k] = 1.0 if beta > 0 else -1.0
    return V, tau, d


def apply_q(V, tau, Y):
    """Y <- H_0 ... H_{n-1} Y (unblocked; H_k = I - tau_k v_k v_k^T, v_k = e_k + V[k+1:, k])."""
    n = V.shape[0]
    Y = Y.copy()
    for k in range(n - 1, -1, -1):
        if tau[k] == 0.0:
            continue
        v = np.concatenate(([1.0], V[k + 1:, k]))
        Y[k:, :] -= tau[k] * np.outer(v, v @ Y[k:, :])
    return Y


def haar(seed, matrix, purpose, n):
    """The Haar factor H_0 ... H_{n-1} D of stream (seed, matrix, purpose)."""
    V, tau, d = reflectors(seed, matrix, purpose, n)
    return apply_q(V, tau, np.eye(n)) * d[None, :]


def sigma(spec, n):
    """Singular values: ("log", c) = logspace(0, -c, n); ("headtail", t) = logspace(0, -1, n // 2)
    followed by t (``common/oracle.py:60-73``)."""
    kind, p = spec
    if kind == "log":
        if n == 1:
            return np.ones(1)
        return 10.0 ** (-p * np.arange(n) / (n - 1))
    r = n // 2
    s = np.full(n, float(p))
    if r == 1:
        s[0] = 1.0
    elif r > 1:
        s[:r] = 10.0 ** (-1.0 * np.arange(r) / (r - 1))
    return s


def recipe(config, i):
    """(class, sigma spec) of matrix i of configuration ``config``."""
    if config in (1, 2):
        return DENSE, None
    if config == 3:
        return HAAR, ("log", 6.0)
    if config == 4:
        _, cls, spec = HEADLINE[i % 6]
        return cls, spec
    if config == 5:
        return (DENSE, None) if i % 2 == 0 else (HAAR, ("log", 8.0))
    raise ValueError(config)


def matrix64(config, i, n, seed):
    """Matrix i of the configuration's batch in float64 (before the float32 cast)."""
    cls, spec = recipe(config, i)
    e = np.arange(n * n)
    if cls == HAAR:
        Vw, tw, dw = reflectors(seed, i, P_W, n)
        Vu, tu, du = reflectors(seed, i, P_U, n)
        s = sigma(spec, n)
        Y = apply_q(Vw, tw, np.eye(n))
        Y *= (s * du)[:, None] * dw[None, :]
        return apply_q(Vu, tu, Y)
    Z = normals(seed, i, P_DENSE, e).reshape(n, n)
    if cls == ROWSCALED:
        u = uniforms(seed, i, P_ROW, np.arange(n)) * 12.0 - 6.0
        Z = Z * (10.0 ** u)[:, None]
    elif cls == UPPERTRI:
        Z = np.triu(Z)
    return Z


def make_batch(config, batch, n, seed):
    """The float32 batch the device generator produces for (config, batch, n, seed)."""
    return np.stack([matrix64(config, i, n, seed) for i in range(batch)]).astype(np.float32)
