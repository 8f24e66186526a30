"""CPU restatement of Edifice's fused sequence-mixing semantics — TEST INFRASTRUCTURE ONLY.

This package is the parity checker for the HIP kernels in ``edifice_amd``.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it, and only to check or to time a CPU baseline beside the GPU.  The
product path (``edifice_amd``) never imports, links or calls anything here and
raises when its HIP library is missing.

Contents
  * ``scans.py``      numpy (float64) restatement of every hot-path function,
                      forward and backward, each citing the reference file:line
                      it follows.
  * ``blocks.py``     numpy restatement of the block-level callers (layer norm,
                      dense, MinGRU / DeltaNet / Mamba / GQA models) used to pin
                      the scans against the reference's safetensors fixtures.
  * ``cref.c``        plain-C (OpenMP, float32) restatement of the same
                      recurrences, used as the timed CPU baseline.

Pinning status of every function is listed in the module docstrings; a function
with no independent check says "parity unpinned" there.
"""
