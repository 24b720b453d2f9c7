"""CPU oracle for the pair-stack hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this package, and only as the
checker (or, for the bench, as the timed stock CPU statement).  The product path (``fpf_hip``) never imports it: every face
raises when the HIP library is missing instead of falling back to anything here.

Modules:
    stock    the stock PyTorch statements of the path, restated in plain torch on the CPU (fp32 / fp64)
    vectors  the reference's golden-vector input generators, restated (inputs are pinned by the SHA-256 digests the reference
             recorded in its manifests)

Parity status of each function is stated in its docstring ("pinned by ..." or "parity unpinned").
"""
