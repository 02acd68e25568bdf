"""CPU oracle for the Token-Union W4A16 MoE path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (float64 arithmetic with bf16 rounding at the
reference's own rounding points), every function of GemmaInfer's W4A16 MoE hot
path.  It is the checker the HIP kernels are compared against.

Rules of use:
  * Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
    ``bench.py`` may import anything from here, and only as the checker or the
    timed CPU baseline -- never as the product path.  ``gemmainfer_amd`` and
    ``gemmainfer_csrc`` never import this package.
  * ``oracle/_ref/`` (built by ``oracle/Makefile`` from the reference's own
    ``csrc/pybind.cpp``) is the reference's CPU C++ fallback, compiled from its
    source; it is used only to pin this restatement.

Pinning status of each function is listed in ``oracle/moe_oracle.py``'s header.
"""
