"""The persistent batch-1 decode kernel (q4d_set_persistent_decode(1), for
models with max_ctx <= 1024) against the five-kernel default path on the
same inputs; the five-kernel path is checked against the oracle by the other
GPU tests.

Tolerances (stated): both paths run the same dequant dot products and
reduction orders per output row; the RMSNorm sums over the hidden vector are
split over a different number of waves, so the normalised activations (and
everything after) may differ in the last bits.  Bars:
- layer output: max-abs <= 2e-5 * max|out| (fp32 rounding only);
- appended K/V rows: within one fp16 ulp of the row's largest element;
- logits of a multi-launch model (10 layers = launches of 8 + 2 layers):
  max-abs <= 1e-4 * max|logits|, same argmax;
- the persistent path repeated on the same input: bit-identical;
- the status word stays 0 (no wait gave up, no bad position).
"""

import ctypes

import numpy as np
import pytest
import torch

from llm_accelerator_amd import _lib
from llm_accelerator_amd._lib import check
from llm_accelerator_amd.model import (KVCache, Qwen3Config, Workspace, build_model, current_stream,
                                       random_host_weights)

pytestmark = pytest.mark.gpu

CTX = 1024


@pytest.fixture(scope="module")
def lib():
    lib = _lib.load()
    yield lib
    check(lib.q4d_set_persistent_decode(0), "q4d_set_persistent_decode")  # back to the default


@pytest.fixture(scope="module")
def one_layer(dev):
    cfg = Qwen3Config(num_hidden_layers=1, vocab_size=2048)
    host = random_host_weights(cfg, seed=11, num_layers=1)
    model = build_model(cfg, host, max_ctx=CTX, device=dev)
    return cfg, model


def status(lib, model, ws):
    out = ctypes.c_int32(0)
    check(lib.q4d_read_status(ws.ptr, ws.nbytes, ctypes.byref(model.descriptor()), 1, ctypes.byref(out),
                              current_stream()), "q4d_read_status")
    return out.value


def run_layer(lib, model, kv, ws, h, pos, persistent):
    check(lib.q4d_set_persistent_decode(persistent), "q4d_set_persistent_decode")
    out = torch.empty_like(h)
    p = torch.tensor([pos], dtype=torch.int32, device=h.device)
    desc, kvd = model.descriptor(), kv.descriptor()
    check(lib.q4d_decoder_layer(ctypes.byref(desc), 0, h.data_ptr(), out.data_ptr(), ctypes.byref(kvd),
                                p.data_ptr(), ws.ptr, ws.nbytes, current_stream()), "q4d_decoder_layer")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("pos", [0, 1, 127, 128, 129, 511, 640, 1023])
def test_layer_matches_multikernel(lib, one_layer, dev, pos):
    cfg, model = one_layer
    print(f"[persist] layer pos={pos}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(pos)
    kv0 = KVCache(cfg, 1, 1, CTX, dev)
    kv0.data[..., :pos, :].normal_(generator=gen)
    h = torch.randn(1, 1024, generator=gen, device=dev)
    ws = Workspace(model, 1)
    kv_a, kv_b = KVCache(cfg, 1, 1, CTX, dev), KVCache(cfg, 1, 1, CTX, dev)
    kv_a.data.copy_(kv0.data)
    kv_b.data.copy_(kv0.data)
    ref = run_layer(lib, model, kv_a, ws, h, pos, 0)
    got = run_layer(lib, model, kv_b, ws, h, pos, 1)
    assert status(lib, model, ws) == 0
    err = (got - ref).abs().max().item()
    scale = ref.abs().max().item()
    print(f"[persist] pos={pos} max-abs {err:.3e} (max|out| {scale:.3f})", flush=True)
    assert err <= 2e-5 * scale
    # everything but the appended row is untouched and equal
    a, b = kv_a.data.float(), kv_b.data.float()
    rows_a, rows_b = a[..., pos, :], b[..., pos, :]
    ulp = rows_a.abs().amax(dim=-1, keepdim=True) * 2.0 ** -10
    assert torch.all((rows_a - rows_b).abs() <= ulp)
    mask = torch.ones(CTX, dtype=torch.bool, device=dev)
    mask[pos] = False
    assert torch.equal(kv_a.data[..., mask, :], kv_b.data[..., mask, :])
    assert torch.equal(kv_b.data[..., mask, :], kv0.data[..., mask, :])


def test_layer_repeat_is_bit_identical(lib, one_layer, dev):
    cfg, model = one_layer
    gen = torch.Generator(device=dev).manual_seed(5)
    kv = KVCache(cfg, 1, 1, CTX, dev)
    kv.data[..., :300, :].normal_(generator=gen)
    h = torch.randn(1, 1024, generator=gen, device=dev)
    ws = Workspace(model, 1)
    outs = [run_layer(lib, model, kv, ws, h, 300, 1) for _ in range(3)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[1], outs[2])
    assert status(lib, model, ws) == 0


def test_multi_launch_model_matches_multikernel(lib, dev):
    """10 layers: one launch of 8 layers and one of 2, through q4d_run_one_token."""
    layers = 10
    cfg = Qwen3Config(num_hidden_layers=layers, vocab_size=4096)
    host = random_host_weights(cfg, seed=3, num_layers=layers)
    model = build_model(cfg, host, max_ctx=256, device=dev)
    tokens = np.random.default_rng(2).integers(0, cfg.vocab_size, 40).tolist()
    results = {}
    for mode in (0, 1):
        print(f"[persist] 10-layer run, persistent={mode}", flush=True)
        check(lib.q4d_set_persistent_decode(mode), "q4d_set_persistent_decode")
        kv = KVCache(cfg, layers, 1, 256, dev)
        ws = Workspace(model, 1)
        desc, kvd = model.descriptor(), kv.descriptor()
        tok = torch.zeros(1, dtype=torch.int32, device=dev)
        pos = torch.zeros(1, dtype=torch.int32, device=dev)
        nxt = torch.zeros(1, dtype=torch.int32, device=dev)
        score = torch.zeros(1, dtype=torch.float32, device=dev)
        logits = torch.empty(cfg.vocab_size, dtype=torch.float32, device=dev)
        all_logits, argmax = [], []
        for i, t in enumerate(tokens):
            tok.fill_(t)
            pos.fill_(i)
            check(lib.q4d_run_one_token(ctypes.byref(desc), tok.data_ptr(), pos.data_ptr(), ctypes.byref(kvd),
                                        nxt.data_ptr(), score.data_ptr(), logits.data_ptr(), ws.ptr, ws.nbytes,
                                        current_stream()), "q4d_run_one_token")
            all_logits.append(logits.clone())
            argmax.append(nxt.clone())
        torch.cuda.synchronize()
        assert status(lib, model, ws) == 0
        results[mode] = (torch.stack(all_logits).cpu(), torch.cat(argmax).cpu(), kv.data.float().cpu())
    (l0, a0, k0), (l1, a1, k1) = results[0], results[1]
    err = (l0 - l1).abs().max().item()
    print(f"[persist] 10-layer logits max-abs {err:.3e} (max {l0.abs().max().item():.3f})", flush=True)
    assert err <= 1e-4 * l0.abs().max().item()
    assert torch.equal(a0, a1)
    ulp = k0.abs().amax(dim=-1, keepdim=True) * 2.0 ** -9
    assert torch.all((k0 - k1).abs() <= ulp)
