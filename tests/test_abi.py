"""The C ABI without a GPU: the library loads, exports every function the header declares,
and rejects bad arguments before it launches anything.  Also the host-side checks of the
Python layer (no CPU fallback, shape validation)."""
import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT, load_package

HEADER = os.path.join(ROOT, "include", "rnrqr.h")


@pytest.fixture(scope="module")
def native():
    import importlib
    load_package()
    return importlib.import_module("qr-contest_amd._native")


@pytest.fixture(scope="module")
def lib(native):
    return native.lib()


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(rnr_\w+)\s*\(", text, re.M)))


def test_header_declares_the_abi():
    names = _declared()
    for want in ("rnr_qr_f32", "rnr_qr_f32_workspace", "rnr_status_string", "rnr_lu_f32",
                 "rnr_cholqr_f32", "rnr_frame_f32", "rnr_chart_f32"):
        assert want in names


def test_library_exports_every_declared_symbol(lib, native):
    names = _declared()
    assert names, "no declarations parsed"
    for name in names:
        assert hasattr(lib, name), name
        assert name in native.SIGNATURES, f"{name} has no ctypes signature"


def test_status_strings(lib, native):
    for code in range(7):
        assert native.status_string(code)
    assert native.status_string(0) == "success"
    assert "unknown" in native.status_string(99)
    assert lib.rnr_version().decode().count(".") == 2


def test_workspace_queries(native, lib):
    assert native.workspace_bytes("qr", 0, 96) == 0
    a = native.workspace_bytes("qr", 4, 96)
    b = native.workspace_bytes("qr", 8, 96)
    assert 0 < a < b
    # four n*n float buffers per matrix at least
    assert a >= 4 * 4 * 96 * 96 * 4
    # n <= 64 runs the fused one-launch kernel, which needs no workspace
    for n in (1, 16, 33, 64):
        assert native.workspace_bytes("qr", 4, n) == 0
    assert native.workspace_bytes("qr", 4, 65) > 0
    for kind in ("lu", "cholqr", "frame"):
        assert native.workspace_bytes(kind, 3, 100) > 0
    out = ctypes.c_size_t(0)
    assert lib.rnr_qr_f32_workspace(4, 0, ctypes.byref(out)) == native.RNR_ERR_UNSUPPORTED_N
    assert lib.rnr_qr_f32_workspace(4, 2049, ctypes.byref(out)) == native.RNR_ERR_UNSUPPORTED_N
    assert lib.rnr_qr_f32_workspace(-1, 8, ctypes.byref(out)) == native.RNR_ERR_INVALID_ARG
    assert lib.rnr_qr_f32_workspace(4, 8, None) == native.RNR_ERR_INVALID_ARG


def test_argument_validation_before_any_launch(native, lib):
    """Every call here must return an error without touching the device."""
    fake = 1 << 20  # never dereferenced: validation fails first
    n, nn = 80, 80 * 80  # the blocked path (n > 64), which takes a workspace
    need = native.workspace_bytes("qr", 2, n)
    f = lib.rnr_qr_f32
    assert f(None, 2, n, nn, fake, fake, None, fake, need, None) == native.RNR_ERR_INVALID_ARG
    assert f(fake, 2, n, nn - 1, fake, fake, None, fake, need, None) == native.RNR_ERR_INVALID_ARG
    assert f(fake, 2, 0, nn, fake, fake, None, fake, need, None) == native.RNR_ERR_UNSUPPORTED_N
    assert f(fake, 2, 4096, 4096 ** 2, fake, fake, None, fake, need, None) == native.RNR_ERR_UNSUPPORTED_N
    assert f(fake, 2, n, nn, fake, fake, None, fake, need - 1, None) == native.RNR_ERR_WORKSPACE
    assert f(fake, 2, n, nn, fake, fake, None, None, need, None) == native.RNR_ERR_WORKSPACE
    assert f(fake, 2, n, nn, fake, fake, None, fake + 4, need, None) == native.RNR_ERR_MISALIGNED
    assert f(fake + 2, 2, n, nn, fake, fake, None, fake, need, None) == native.RNR_ERR_MISALIGNED
    # the fused small-n path validates the same arguments before it launches
    assert f(None, 2, 16, 256, fake, fake, None, None, 0, None) == native.RNR_ERR_INVALID_ARG
    assert f(fake, 2, 16, 255, fake, fake, None, None, 0, None) == native.RNR_ERR_INVALID_ARG
    assert f(fake, 2, 16, 256, fake + 2, fake, None, None, 0, None) == native.RNR_ERR_MISALIGNED
    # batch 0 is a no-op that succeeds with null pointers
    assert f(None, 0, 16, 256, None, None, None, None, 0, None) == native.RNR_OK
    assert lib.rnr_chart_f32(None, 2, 8, fake, fake, None) == native.RNR_ERR_INVALID_ARG
    assert lib.rnr_lu_f32(fake, 2, 8, 64, fake, None, fake, 1 << 30, None) == native.RNR_ERR_INVALID_ARG
    assert lib.rnr_cholqr_f32(fake, 2, 8, 64, None, None, None, fake, 1 << 30, None) == native.RNR_ERR_INVALID_ARG
    # the GPU gate checker
    c = lib.rnr_check_f64
    cneed = native.workspace_bytes("check", 2, 16)
    assert cneed > 0
    assert c(None, 256, fake, fake, 2, 16, fake, fake, None, fake, cneed, None) == native.RNR_ERR_INVALID_ARG
    assert c(fake, 255, fake, fake, 2, 16, fake, fake, None, fake, cneed, None) == native.RNR_ERR_INVALID_ARG
    assert c(fake, 256, fake, fake, 2, 0, fake, fake, None, fake, cneed, None) == native.RNR_ERR_UNSUPPORTED_N
    assert c(fake, 256, fake, fake, 2, 16, fake, fake, None, fake, cneed - 1, None) == native.RNR_ERR_WORKSPACE
    assert c(fake, 256, fake, fake, 2, 16, fake, fake, None, fake + 8, cneed, None) == native.RNR_ERR_MISALIGNED
    assert c(None, 256, None, None, 0, 16, None, None, None, None, 0, None) == native.RNR_OK
    # the device generators
    gw = ctypes.c_size_t(0)
    assert lib.rnr_generate_workspace(4, 256, 512, ctypes.byref(gw)) == native.RNR_OK
    assert gw.value >= 128 * 3 * 512 * 512 * 8          # 128 Haar matrices: U, W and Y in float64
    assert lib.rnr_generate_workspace(1, 16, 64, ctypes.byref(gw)) == native.RNR_OK and gw.value == 0
    assert lib.rnr_generate_workspace(4, 1, 64, ctypes.byref(gw)) == native.RNR_OK and gw.value == 0
    assert lib.rnr_generate_workspace(0, 1, 64, ctypes.byref(gw)) == native.RNR_ERR_INVALID_ARG
    gn = lib.rnr_generate_f32
    assert gn(6, 2, 16, 0, fake, None, 0, None) == native.RNR_ERR_INVALID_ARG
    assert gn(4, 2, 0, 0, fake, None, 0, None) == native.RNR_ERR_UNSUPPORTED_N
    assert gn(4, 2, 16, 0, None, None, 0, None) == native.RNR_ERR_INVALID_ARG
    assert gn(4, 2, 16, 0, fake, None, 0, None) == native.RNR_ERR_WORKSPACE   # matrix 1 is Haar
    assert gn(4, 2, 16, 0, fake, fake + 8, 1 << 30, None) == native.RNR_ERR_MISALIGNED
    assert gn(4, 0, 16, 0, None, None, 0, None) == native.RNR_OK
    # the Householder comparator
    hw = ctypes.c_size_t(0)
    assert lib.rnr_hh_geqrf_workspace(2, 100, ctypes.byref(hw)) == native.RNR_OK and hw.value == 2 * 32 * 32 * 4
    hq = lib.rnr_hh_geqrf_f32
    assert hq(None, 2, 16, fake, fake, hw.value, None) == native.RNR_ERR_INVALID_ARG
    assert hq(fake, 2, 0, fake, fake, hw.value, None) == native.RNR_ERR_UNSUPPORTED_N
    assert hq(fake, 2, 16, fake, fake, hw.value - 1, None) == native.RNR_ERR_WORKSPACE
    assert hq(fake, 2, 16, fake, fake + 8, hw.value, None) == native.RNR_ERR_MISALIGNED
    assert hq(None, 0, 16, None, None, 0, None) == native.RNR_OK
    # the Q consumers
    qw = native.workspace_bytes("orgqr", 2, 100)
    assert qw >= 2 * 4 * 32 * 32 * 4 and native.workspace_bytes("ormqr", 2, 100) == qw
    o = lib.rnr_orgqr_f32
    assert o(None, fake, 2, 16, fake, fake, qw, None) == native.RNR_ERR_INVALID_ARG
    assert o(fake, fake, 2, 0, fake, fake, qw, None) == native.RNR_ERR_UNSUPPORTED_N
    assert o(fake, fake, 2, 4096, fake, fake, qw, None) == native.RNR_ERR_UNSUPPORTED_N
    assert o(fake, fake, 2, 100, fake, None, qw, None) == native.RNR_ERR_WORKSPACE
    assert o(fake, fake, 2, 100, fake, fake, qw - 1, None) == native.RNR_ERR_WORKSPACE
    assert o(fake, fake, 2, 100, fake, fake + 8, qw, None) == native.RNR_ERR_MISALIGNED
    assert o(None, None, 0, 16, None, None, 0, None) == native.RNR_OK
    m = lib.rnr_ormqr_f32
    assert m(fake, fake, 2, 16, None, 5, 5, 80, 0, fake, qw, None) == native.RNR_ERR_INVALID_ARG
    assert m(fake, fake, 2, 16, fake, 5, 4, 80, 0, fake, qw, None) == native.RNR_ERR_INVALID_ARG   # ldc < ncol
    assert m(fake, fake, 2, 16, fake, 5, 5, 79, 1, fake, qw, None) == native.RNR_ERR_INVALID_ARG   # stride < n ldc
    assert m(fake, fake, 2, 16, fake, -1, 5, 80, 1, fake, qw, None) == native.RNR_ERR_INVALID_ARG
    assert m(fake, fake, 2, 100, fake, 5, 5, 500, 1, None, qw, None) == native.RNR_ERR_WORKSPACE
    assert m(None, None, 2, 16, None, 0, 0, 0, 1, None, 0, None) == native.RNR_OK


def test_python_layer_rejects_cpu_and_non_square(pkg):
    with pytest.raises(RuntimeError, match="GPU only"):
        pkg.custom_kernel(torch.randn(2, 8, 8))
    with pytest.raises(ValueError):
        pkg.custom_kernel(torch.randn(2, 8, 7))
    with pytest.raises(ValueError):
        pkg.custom_kernel(torch.randn(8))
    # the raw float32 entry point checks dtype and device before any pointer reaches the library
    import importlib
    rnr = importlib.import_module("qr-contest_amd.reflection_no_reflectors")
    with pytest.raises(ValueError, match="float32"):
        rnr.qr(torch.randn(2, 8, 8, dtype=torch.float64))
    with pytest.raises(RuntimeError, match="GPU only"):
        rnr.qr(torch.randn(2, 8, 8))


def test_build_command_targets_gfx950_without_packed_fp32(pkg):
    import importlib
    b = importlib.import_module("qr-contest_amd.build")
    cmd = b.command("/tmp/x.so")
    assert "--offload-arch=gfx950" in cmd
    i = cmd.index("-packed-fp32-ops")
    assert cmd[i - 1] == "-Xclang" and cmd[i - 2] == "-target-feature"


def test_noalloc_entry_rejects_before_touching_the_gpu(lib, native):
    """rnr_qr_f32_noalloc validates sizes on the host before it looks up its scratch or
    launches: a problem whose workspace exceeds RNR_NOALLOC_SCRATCH_BYTES is refused."""
    f = lib.rnr_qr_f32_noalloc
    fake = 1 << 20
    assert f(fake, 32, 512, 512 * 512, fake, fake, None, None) == native.RNR_ERR_SCRATCH_LIMIT
    assert f(fake, 2, 2048, 2048 * 2048, fake, fake, None, None) == native.RNR_ERR_SCRATCH_LIMIT
    assert f(fake, 4, 2049, 2049 * 2049, fake, fake, None, None) == native.RNR_ERR_UNSUPPORTED_N
    assert f(fake, -1, 8, 64, fake, fake, None, None) == native.RNR_ERR_INVALID_ARG
    assert f(None, 0, 100, 0, None, None, None, None) == native.RNR_OK  # empty batch: nothing to do
