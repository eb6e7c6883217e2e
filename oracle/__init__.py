"""CPU oracle for the reflector-free batched QR -- TEST INFRASTRUCTURE ONLY.

Nothing in the product (the ``qr-contest_amd`` package and its HIP library)
imports, links or calls this package.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker
(or, for ``cpu_baseline``, as the timed CPU restatement of the reference).

Modules
-------
``rnr``          torch-CPU restatement of ``/root/reference/reflection_no_reflectors.py``
``checker``      the fp64 factor-residual / orthogonality gates of ``common/oracle.py:152-195``
``closed_form``  LAPACK ``geqrf`` plus the sign/tau post-map that the path equals in exact arithmetic
``textbook``     pure-Python unblocked getrf / potrf / trsm / chart for tiny matrices (brute force)
``gen``          numpy restatement of the device generators (Philox4x32-10, Box-Muller, Stewart's
                 Haar factors, the five configurations' classes)

Pinning status (what checks each function; see ``tests/test_oracle.py``)
-----------------------------------------------------------------------
* ``rnr.lu_factor``   -- textbook getrf (first-max pivot) on n <= 8, scipy.linalg.lu, P L U = A, |L| <= 1.
* ``rnr.cholqr``      -- textbook potrf; R^T R - M^T M = mu I with mu = 1e-7 ||M||_F^2 / n (fp64).
* ``rnr.frame``       -- Q^T Q = I and Q^T A upper-triangular in fp64 with jitter 0.
* ``rnr.chart``       -- geqrf(Q) post-map (fp64); blocked bs=32 equals unblocked bs=1 and the textbook chart.
* ``rnr.custom_kernel`` -- geqrf(A) post-map (fp64, jitter 0: 1e-10; fp32: tolerance), special cases
  (upper-triangular, n = 1, zero matrix), the contest gates on all six pathology classes.
* ``checker.check``   -- exact geqrf factors give ~1e-15; a planted 1 % error in R fails the gate.
* ``gen``             -- Random123 Philox4x32-10 known-answer vectors; KS / moment tests of the streams;
  Haar factors against numpy's sign-fixed QR of Gaussian matrices (two-sample KS, E tr Q = 0,
  E (tr Q)^2 = 1); prescribed singular values by numpy SVD (``tests/test_oracle_gen.py``).
The only part no check fixes to the last bit is the reference's exact fp32 rounding sequence inside
torch.linalg (LAPACK); parity is therefore stated to an fp32 tolerance, not bitwise.
"""
