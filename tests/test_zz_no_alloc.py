"""q4d_run_one_token_noalloc (the one-token step without a workspace argument, its
scratch a device array inside the library) against q4d_run_one_token with a
caller workspace: the same kernels on the same inputs, so next token, score, every
logit and the appended K/V rows must be equal bit for bit.  Two calls in a row on
the same GPU, the second with a smaller model view (context capacity 1024, then
256) at a smaller position, then a device-side bad position that must set the
caller's status word and write nothing.  Also the host-side rejection of models
whose workspace exceeds the 4 MiB scratch.
"""

import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import PLANS, decode_plan
from llm_accelerator_amd import _lib
from llm_accelerator_amd._lib import check
from llm_accelerator_amd.model import (KVCache, Qwen3Config, Workspace, build_model, current_stream,
                                       random_host_weights, with_context)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(dev):
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=2048)
    host = random_host_weights(cfg, seed=5, num_layers=2)
    return cfg, build_model(cfg, host, max_ctx=1024, device=dev)


def _step(lib, model, kv, token, position, noalloc, status=None):
    dev = model.device
    desc, kvd = model.descriptor(), kv.descriptor()
    tok = torch.tensor([token], dtype=torch.int32, device=dev)
    pos = torch.tensor([position], dtype=torch.int32, device=dev)
    nxt = torch.full((1,), -1, dtype=torch.int32, device=dev)
    score = torch.zeros(1, dtype=torch.float32, device=dev)
    logits = torch.zeros(model.config.vocab_size, dtype=torch.float32, device=dev)
    if noalloc:
        check(lib.q4d_run_one_token_noalloc(ctypes.byref(desc), tok.data_ptr(), pos.data_ptr(), ctypes.byref(kvd),
                                            nxt.data_ptr(), score.data_ptr(), logits.data_ptr(), status.data_ptr(),
                                            current_stream()), "q4d_run_one_token_noalloc")
    else:
        ws = Workspace(model, 1)
        check(lib.q4d_run_one_token(ctypes.byref(desc), tok.data_ptr(), pos.data_ptr(), ctypes.byref(kvd),
                                    nxt.data_ptr(), score.data_ptr(), logits.data_ptr(), ws.ptr, ws.nbytes,
                                    current_stream()), "q4d_run_one_token")
    torch.cuda.synchronize()
    return nxt, score, logits


def _filled_cache(cfg, model, upto, seed, dev):
    kv = KVCache(cfg, 2, 1, model.max_ctx, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    kv.data[..., :upto, :].normal_(generator=g)
    return kv


@pytest.mark.parametrize("plan_id,plan,precision", PLANS, ids=[p[0] for p in PLANS])
def test_noalloc_equals_workspace_path_twice(dev, small, plan_id, plan, precision):
    cfg, model = small
    lib = _lib.load()
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    for m, position, token, seed in ((model, 700, 1234, 1), (with_context(model, 256), 100, 77, 2)):
        print(f"[noalloc] plan {plan_id} max_ctx={m.max_ctx} position={position}", flush=True)
        kv_ref = _filled_cache(cfg, m, position, seed, dev)
        kv_got = KVCache(cfg, 2, 1, m.max_ctx, dev)
        kv_got.data.copy_(kv_ref.data)
        with decode_plan(plan, precision):
            ref = _step(lib, m, kv_ref, token, position, noalloc=False)
            got = _step(lib, m, kv_got, token, position, noalloc=True, status=status)
        for r, g in zip(ref, got):
            assert torch.equal(r, g)
        assert torch.equal(kv_ref.data, kv_got.data)
        assert int(status.item()) == 0
        assert kv_got.data[:, :, 0, :, position].abs().sum().item() > 0  # the step appended its row


def test_noalloc_reports_bad_position_in_callers_status(dev, small):
    cfg, model = small
    lib = _lib.load()
    m = with_context(model, 256)
    kv = _filled_cache(cfg, m, 10, 3, dev)
    before = kv.data.clone()
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    _step(lib, m, kv, 5, m.max_ctx, noalloc=True, status=status)   # one past the last slot
    assert int(status.item()) & _lib.STATUS_BAD_POSITION
    assert torch.equal(kv.data, before)
    # the scratch keeps nothing that breaks the next good call
    status.zero_()
    kv_ref = _filled_cache(cfg, m, 10, 3, dev)
    ref = _step(lib, m, kv_ref, 5, 10, noalloc=False)
    got = _step(lib, m, kv, 5, 10, noalloc=True, status=status)
    for r, g in zip(ref, got):
        assert torch.equal(r, g)
    assert int(status.item()) == 0
