"""CPU oracle: test infrastructure only.

This package restates, in plain PyTorch on the CPU, the algorithms of the
reference (Parity-LRX/FSCTEP) that the HIP kernels replace.  It is the checker:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path (``fsctep_amd``) never imports it
and has no CPU fallback.
"""
