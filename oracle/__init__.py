"""CPU oracle for the AxiomLM quantized decode step -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference's CPU semantics of the path the
MI355X build implements (packed weight formats, KV quantizers, the quantized
decoder forward, decode and tree attention).  It exists to check the HIP
implementation: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or
as the timed CPU baseline.  Nothing in ``axiomlm_amd`` imports it; the product
path fails loudly when the HIP library is missing.

Every function cites the reference file:line it follows (paths relative to the
AxiomLM source tree).  Pinning of each function (golden vectors, known-answer
tests, closed forms, invariants) is listed in the module docstrings.
"""

from . import formats, model  # noqa: F401
