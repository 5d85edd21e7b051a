"""CPU oracle for the Qwen3-0.6B Q4 decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the algorithm of the reference's CPU path:

* the FP32 "manual" decode of ``Qwen3-0.6B-Base/python_each_module/common.py``
  (lines 129-298) and ``10_validate_full_run_one_token.py`` (lines 17-56);
* the integer Q4 contract of ``Source/Q4_FORMAT.md`` (lines 75-190) and the
  exporters ``13_export_q4_gemv_vectors.py``, ``28_export_mlp_gate_up_vectors.py``,
  ``35_export_lm_head_full_vocab_vectors.py`` and
  ``56_export_persistent_multitoken_layer_golden.py``.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or as the timed CPU
baseline.  The product package (``llm_accelerator_amd``) never imports it and
has no CPU fallback.

How each function is pinned (so that a dropped term, a wrong sign or index,
or a transposed operand fails a test) is listed in ``PINS`` below and
exercised by ``tests/test_oracle_*.py``.
"""

from .q4_oracle import *  # noqa: F401,F403
from .q4_oracle import PINS  # noqa: F401
