"""CPU oracle for the FP8 paged-attention decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in numpy (plus one plain-C file), the
algorithms the reference uses on this path:

* ``fp8``       -- OCP float8 e4m3fn and bfloat16 codecs (the arithmetic that
                   ``tensor.to(torch.float8_e4m3fn)`` / ``.to(torch.bfloat16)``
                   perform in the reference harness).
* ``quant``     -- per-token / per-tensor KV quantisers and the paged KV-cache
                   layouts (tests/kernels/test_pa.py:177-211, 334-429;
                   tests/utils.py:29-73).
* ``attention`` -- the torch reference ``torch_mha_extend`` /
                   ``reference_masked_attention`` (tests/kernels/test_pa.py:214-331),
                   the split-partition partial contract and the log-sum-exp
                   reduce (kernels/pa_decode_fp8.py:2291-2320,
                   kernels/pa_decode_swa.py:954-1130).
* ``planners``  -- the integer planners: split heuristic, partition ranges,
                   sliding-window tiles, page data and the ``get_pa_metadata_v1``
                   worklist scheduler (kernels/pa_decode_fp8.py:1729-1949,
                   kernels/pa_metadata.py:53-420).
* ``pa_metadata_ref.c`` -- the same scheduler in plain C (built by
                   ``oracle/Makefile`` into ``oracle/_build``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker.  The product
path (``flydsl_amd``) never imports it and has no CPU fallback.
"""

from . import fp8, quant, attention, planners  # noqa: F401
