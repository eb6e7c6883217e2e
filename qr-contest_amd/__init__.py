"""MI355X-native reflector-free batched QR, ``custom_kernel(A) -> (H, tau)``.

The directory name is not a Python identifier; load it with
``importlib.import_module("qr-contest_amd")`` (the repository's tests, bench and
entry script do).  Submodules:

* ``reflection_no_reflectors`` -- ``custom_kernel`` plus the stage functions,
  mirroring ``/root/reference/reflection_no_reflectors.py``;
* ``_native``   -- ctypes binding of ``librnrqr.so`` (the C-ABI in ``include/rnrqr.h``);
* ``workloads`` -- seeded batches of the five benchmark configurations.
"""


def custom_kernel(data):
    from .reflection_no_reflectors import custom_kernel as _ck
    return _ck(data)
