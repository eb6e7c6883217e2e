"""Writes the golden fixtures of the reflector-free QR from the reference implementation.

Run once, in the build container (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py

It imports ``custom_kernel`` from ``/root/reference/reflection_no_reflectors.py`` on CPU
(torch fp32, this image's torch 2.10.0 / MKL), runs it on small seeded inputs and saves
inputs and outputs as ``.npy`` next to this script.  The fixtures pin the one thing the
closed form, the textbook routines and the invariants cannot: the reference's exact fp32
rounding sequence, which the CPU oracle (oracle/rnr.py) claims to reproduce op for op.
"""
from __future__ import annotations

import importlib.util
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference/reflection_no_reflectors.py"

# (name, batch, n, seed, kind)
CASES = [
    ("randn_4x16", 4, 16, 101, "randn"),
    ("randn_2x48", 2, 48, 102, "randn"),
    ("randn_1x96", 1, 96, 103, "randn"),
    ("wellcond_2x64", 2, 64, 104, "wellcond"),
    ("uppertri_2x24", 2, 24, 105, "uppertri"),
    # benchmark-size cases: the blocked path (64-wide panels, 64-column Cholesky blocks,
    # 128-row solve blocks at 512; the 64-wide tiles of the mid sizes at 128)
    ("wellcond_2x128", 2, 128, 106, "wellcond"),
    ("wellcond_2x512", 2, 512, 107, "wellcond"),
]


def make_input(batch, n, seed, kind):
    g = torch.Generator().manual_seed(seed)
    if kind == "randn":
        A = torch.randn(batch, n, n, generator=g, dtype=torch.float64)
    elif kind == "uppertri":
        A = torch.triu(torch.randn(batch, n, n, generator=g, dtype=torch.float64))
    else:  # Haar U, V with sigma = logspace(0, -2, n)
        def haar():
            Z = torch.randn(batch, n, n, generator=g, dtype=torch.float64)
            Q, R = torch.linalg.qr(Z)
            d = torch.sign(torch.diagonal(R, dim1=-2, dim2=-1))
            d = torch.where(d == 0, torch.ones_like(d), d)
            return Q * d.unsqueeze(-2)
        U, V = haar(), haar()
        s = torch.logspace(0, -2, n, dtype=torch.float64)
        A = (U * s.view(1, 1, n)) @ V.mT
    return A.float().contiguous()


def main():
    spec = importlib.util.spec_from_file_location("ref_rnr", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    meta = {"torch": torch.__version__, "threads": torch.get_num_threads(), "cases": []}
    for name, batch, n, seed, kind in CASES:
        A = make_input(batch, n, seed, kind)
        H, tau = mod.custom_kernel(A.clone())
        np.save(os.path.join(HERE, f"{name}_A.npy"), A.numpy())
        np.save(os.path.join(HERE, f"{name}_H.npy"), H.numpy())
        np.save(os.path.join(HERE, f"{name}_tau.npy"), tau.numpy())
        meta["cases"].append({"name": name, "batch": batch, "n": n, "seed": seed, "kind": kind})
    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print("wrote", len(CASES), "cases")


if __name__ == "__main__":
    main()
