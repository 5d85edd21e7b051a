"""The XCD-split decode plan's guards.

* Device check: an MI355X passes it (the plan runs); with the check forced to fail
  (q4d_diag_set_xcd_check(1)) the same calls run the staged plan, bit for bit what
  an explicit staged plan gives.
* Status path: the host presets one workgroup's exchange flag ahead of the others
  (a count no workgroup will reach), so that workgroup's bounded waits give up after
  their 20 ms and every kernel exits normally; the status word then carries
  Q4D_STATUS_SYNC_TIMEOUT, the drop-in and the greedy decoder raise
  Q4DecError(Q4D_ERR_STATUS), and a workspace reset restores correct steps.
"""

import ctypes

import numpy as np
import pytest
import torch

from llm_accelerator_amd import _lib, common
from llm_accelerator_amd._lib import check
from llm_accelerator_amd.decode import GreedyDecoder
from llm_accelerator_amd.model import KVCache, Qwen3Config, Workspace, build_model, current_stream, random_host_weights

pytestmark = pytest.mark.gpu

# workspace byte offset of the [8][32] exchange flags for batch 1: status (256 B), then
# the attention counters (8 int32, padded to 256 B), the LM-head argmax hand-off
# (8 group keys and counters and the top counter on 128-byte lines: 2176 B, padded
# to 2304 B)
XFLAGS_OFFSET = 2816


@pytest.fixture(scope="module")
def small(dev):
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=2048)
    host = random_host_weights(cfg, seed=9, num_layers=2)
    return cfg, build_model(cfg, host, max_ctx=256, device=dev)


def _one_token(lib, model, kv, ws, token, position):
    dev = model.device
    tok = torch.tensor([token], dtype=torch.int32, device=dev)
    pos = torch.tensor([position], dtype=torch.int32, device=dev)
    nxt = torch.full((1,), -1, dtype=torch.int32, device=dev)
    score = torch.zeros(1, dtype=torch.float32, device=dev)
    logits = torch.zeros(model.config.vocab_size, dtype=torch.float32, device=dev)
    check(lib.q4d_run_one_token(ctypes.byref(model.descriptor()), tok.data_ptr(), pos.data_ptr(),
                                ctypes.byref(kv.descriptor()), nxt.data_ptr(), score.data_ptr(), logits.data_ptr(),
                                ws.ptr, ws.nbytes, current_stream()), "q4d_run_one_token")
    torch.cuda.synchronize()
    return nxt.clone(), score.clone(), logits.clone()


def _cache(cfg, model, upto, seed, dev):
    kv = KVCache(cfg, 2, 1, model.max_ctx, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    kv.data[..., :upto, :].normal_(generator=g)
    return kv


def test_device_check_passes_and_forced_fallback_runs_staged(dev, small):
    cfg, model = small
    lib = _lib.load()
    desc = model.descriptor()
    assert lib.q4d_decode_plan_active(ctypes.byref(desc), current_stream()) == _lib.DECODE_XCD
    kv_staged, kv_forced = _cache(cfg, model, 50, 1, dev), _cache(cfg, model, 50, 1, dev)
    prev = lib.q4d_set_decode_plan(_lib.DECODE_STAGED)
    try:
        ref = _one_token(lib, model, kv_staged, Workspace(model, 1), 101, 50)
    finally:
        lib.q4d_set_decode_plan(prev)
    assert lib.q4d_diag_set_xcd_check(1) == 0
    try:
        assert lib.q4d_decode_plan_active(ctypes.byref(desc), current_stream()) == _lib.DECODE_STAGED
        assert GreedyDecoder(model, use_graph=False).plan() == _lib.DECODE_STAGED
        ws = Workspace(model, 1)
        got = _one_token(lib, model, kv_forced, ws, 101, 50)
        assert ws.status() == 0
    finally:
        assert lib.q4d_diag_set_xcd_check(0) == 1
    assert lib.q4d_decode_plan_active(ctypes.byref(desc), current_stream()) == _lib.DECODE_XCD
    for r, g in zip(ref, got):
        assert torch.equal(r, g)
    assert torch.equal(kv_staged.data, kv_forced.data)
    assert lib.q4d_diag_set_xcd_check(2) == -11  # only modes 0 and 1 exist


def _preset_flag(ws: Workspace, value: int):
    flags = ws.buf[XFLAGS_OFFSET:XFLAGS_OFFSET + 8 * 32 * 4].view(torch.int32)
    flags[0] = value  # XCD group 0, workgroup 0


def test_exchange_timeout_sets_status_and_raises(dev, small):
    cfg, model = small
    lib = _lib.load()
    assert lib.q4d_decode_plan_active(ctypes.byref(model.descriptor()), current_stream()) == _lib.DECODE_XCD
    kv = _cache(cfg, model, 30, 2, dev)
    kcs, vcs = common.layer_views(kv, 30)
    rt = common.runtime(model)
    rt.ws.reset()
    h = torch.from_numpy(np.random.default_rng(3).normal(size=(1, 1, 1024)).astype(np.float32)).to(dev)
    args = (model.model.layers[0], model.model.rotary_emb, torch.tensor([[30]]), kcs[0], vcs[0], 1, 16, 8, 128, 2, cfg)
    ref, _, _ = common.manual_decoder_layer_cached(h, *args)
    print("[xcd guard] presetting exchange flag 0 ahead: its waits give up after 20 ms each", flush=True)
    _preset_flag(rt.ws, 1000 << 4)
    with pytest.raises(_lib.Q4DecError) as e:
        common.manual_decoder_layer_cached(h, *args)
    assert e.value.code == -6 and e.value.status & _lib.STATUS_SYNC_TIMEOUT
    assert "SYNC_TIMEOUT" in str(e.value)
    # the drop-in reset the workspace: the same call is correct again (the append at
    # position 30 rewrites the same row)
    assert rt.ws.status() == 0
    again, _, _ = common.manual_decoder_layer_cached(h, *args)
    assert torch.equal(again, ref)


def test_greedy_decoder_history_raises_on_status(dev, small):
    cfg, model = small
    dec = GreedyDecoder(model, use_graph=False)
    dec.prefill([5, 6, 7])
    dec.generate(2)
    good, _ = dec.history()
    assert len(good) == 3
    print("[xcd guard] greedy decoder: preset exchange flag, one step", flush=True)
    _preset_flag(dec.ws, 1000 << 4)
    dec.step()
    torch.cuda.synchronize()
    with pytest.raises(_lib.Q4DecError) as e:
        dec.history()
    assert e.value.status & _lib.STATUS_SYNC_TIMEOUT
    dec.prefill([5, 6, 7])   # reset() clears the workspace: the same run is valid again
    dec.generate(2)
    assert dec.history()[0] == good
