"""CPU oracle for the ConvRot QuantLinear + LoRA path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import this
package, and only as the checker.  The product (the ``krea-2_amd`` package) never imports, calls or links it:
the HIP library is the only implementation of the path, and the module raises when it is missing.

Contents: :mod:`oracle.convrot` restates the path's arithmetic in numpy (float32 where the kernels must be
bit-exact, float64 where the kernels are held to a tolerance).  Every function cites the reference
``file:line`` it follows, or the ``BASELINE.json`` north_star clause it restates where the reference has no
code for it.  Each function's pin (golden vector, closed form, invariant or brute force) lives in
``tests/test_oracle.py``; there is no "parity unpinned" function in this oracle.
"""
