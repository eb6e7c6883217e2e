"""Device-side seeded generators for the five benchmark configurations (the input step; the
reference builds its batches with torch's generator, ``common/oracle.py:43-146``).

``device_batch(config)`` returns the configuration's float32 batch generated on the GPU by
``rnr_generate_f32``: the same classes and spectra as ``workloads.make_batch`` (dense, the
Haar-based prescribed spectra, rowscaled, uppertri), but from the library's own Philox4x32-10
streams, so the matrices differ from the host generator's (they are equally distributed).
Matrix i depends only on (config, n, seed, i).
"""
from __future__ import annotations

import torch

from . import _native
from .workloads import CONFIGS

__all__ = ["device_batch"]


def device_batch(config: int, *, batch: int | None = None, n: int | None = None,
                 seed: int | None = None, device="cuda") -> torch.Tensor:
    """The seeded batch of configuration ``config`` (1..5), generated on ``device``."""
    cfg = CONFIGS[config]
    b = cfg.batch if batch is None else int(batch)
    nn = cfg.n if n is None else int(n)
    sd = cfg.seed if seed is None else int(seed)
    if not 0 <= sd < 2 ** 64:
        raise ValueError("seed must fit in 64 bits")
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("device_batch: runs on the GPU only (no CPU fallback)")
    A = torch.empty(b, nn, nn, dtype=torch.float32, device=dev)
    lib = _native.lib()
    import ctypes
    need = ctypes.c_size_t(0)
    _native.check("rnr_generate_workspace", lib.rnr_generate_workspace(config, b, nn, ctypes.byref(need)))
    ws = torch.empty(max(int(need.value), 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        st = lib.rnr_generate_f32(config, b, nn, sd, A.data_ptr(), ws.data_ptr(), int(need.value),
                                  torch.cuda.current_stream(dev).cuda_stream)
    _native.check("rnr_generate_f32", st)
    return A
