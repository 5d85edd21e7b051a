"""q4d_diag_launch_chain, the launch-floor probe bench.py times: n dependent launches
with the given grids, kernel i reading the 4 KB half of the buffer that kernel i - 1
wrote and (block 0) writing the other half as value + 1, so after n launches from a
zero buffer the last-written half holds n everywhere and the other n - 1."""

import ctypes

import pytest
import torch

from llm_accelerator_amd import _lib
from llm_accelerator_amd.model import current_stream

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 2, 141])
def test_launch_chain_values(dev, n):
    lib = _lib.load()
    shapes = [(512, 1, 256), (6, 8, 256), (128, 1, 512), (384, 1, 256), (256, 1, 384)] * 28 + [(238, 1, 1024)]
    shapes = shapes[:n]
    gx = (ctypes.c_int32 * n)(*[s[0] for s in shapes])
    gy = (ctypes.c_int32 * n)(*[s[1] for s in shapes])
    bl = (ctypes.c_int32 * n)(*[s[2] for s in shapes])
    buf = torch.zeros(2048, dtype=torch.float32, device=dev)
    print(f"[diag] chain of {n}", flush=True)
    rc = lib.q4d_diag_launch_chain(ctypes.cast(gx, ctypes.c_void_p), ctypes.cast(gy, ctypes.c_void_p),
                                   ctypes.cast(bl, ctypes.c_void_p), n, buf.data_ptr(), current_stream())
    assert rc == 0
    torch.cuda.synchronize()
    last = buf[(n & 1) * 1024:(n & 1) * 1024 + 1024]
    other = buf[((n + 1) & 1) * 1024:((n + 1) & 1) * 1024 + 1024]
    assert torch.all(last == float(n))
    assert torch.all(other == float(n - 1))
