"""MI355X (gfx950) Qwen3-0.6B Q4 decode hot path.

Python host layer over ``libq4dec.so`` (hand-written HIP kernels behind the C
ABI in ``include/q4dec.h``).  Torch tensors are used only as device buffers
and for stream handles.

* :mod:`.model`   -- Q4 weights, HF-shaped model object, KV cache, workspace
* :mod:`.common`  -- drop-in mirror of the reference's ``common.py`` /
  ``run_manual_one_token`` functions
* :mod:`.decode`  -- greedy decode driver with device-side token feedback
* :mod:`.build`   -- in-tree build of ``libq4dec.so`` for gfx950
"""

__version__ = "0.1.0"
