"""q4d_run_one_token_feedback (one decode step whose LM head also stores the greedy
feedback, with the embedding built inside layer 0's q|k|v launch) against the
separate launches it replaces: q4d_embedding, q4d_decoder_layer per layer,
q4d_lm_head_argmax and q4d_advance (the feedback loop of
10_validate_full_run_one_token.py:135-172).  Same kernels on the same inputs
apart from where the embedding row and the feedback are computed, so the next
token, score, every logit, the fed-back token and position, the history and its
count, and the K/V cache must be equal bit for bit, step after step.  A history
of capacity 3 over 5 recorded steps checks the capacity rule; a first step with
no history checks the unrecorded form.  A token id outside the vocabulary must
set Q4D_STATUS_BAD_TOKEN and give the zero embedding, as q4d_embedding does.
q4d_run_one_token (also folded) is checked against the same launches.
"""

import ctypes

import pytest
import torch

from gpu_helpers import PLANS, decode_plan
from llm_accelerator_amd import _lib
from llm_accelerator_amd._lib import check
from llm_accelerator_amd.model import (KVCache, Qwen3Config, Workspace, build_model, current_stream,
                                       random_host_weights)

pytestmark = pytest.mark.gpu

LAYERS, VOCAB, CTX = 2, 2048, 256


@pytest.fixture(params=PLANS, ids=[p[0] for p in PLANS])
def plan(request):
    """Each test runs under the XCD-split plan, the staged plan and the staged plan with
    fp16 activations (the separate launches and the folded step use the same plan)."""
    _, pl, prec = request.param
    with decode_plan(pl, prec):
        yield pl


@pytest.fixture(scope="module")
def small(dev):
    cfg = Qwen3Config(num_hidden_layers=LAYERS, vocab_size=VOCAB)
    host = random_host_weights(cfg, seed=7, num_layers=LAYERS)
    return cfg, build_model(cfg, host, max_ctx=CTX, device=dev)


class Loop:
    """Device state of one greedy loop: token, position, outputs and history."""

    def __init__(self, cfg, model, kv_init, token, position, cap):
        dev = model.device
        self.lib = _lib.load()
        self.model = model
        self.desc = model.descriptor()
        self.table = model.lm_head.weight.descriptor()
        self.kv = KVCache(cfg, LAYERS, 1, model.max_ctx, dev)
        self.kv.data.copy_(kv_init)
        self.kvd = self.kv.descriptor()
        self.ws = Workspace(model, 1)
        self.tok = torch.tensor([token], dtype=torch.int32, device=dev)
        self.pos = torch.tensor([position], dtype=torch.int32, device=dev)
        self.nxt = torch.full((1,), -1, dtype=torch.int32, device=dev)
        self.score = torch.zeros(1, dtype=torch.float32, device=dev)
        self.logits = torch.zeros(cfg.vocab_size, dtype=torch.float32, device=dev)
        self.hist_tok = torch.full((cap + 2,), -5, dtype=torch.int32, device=dev)
        self.hist_score = torch.full((cap + 2,), -5.0, dtype=torch.float32, device=dev)
        self.hist_count = torch.zeros(1, dtype=torch.int32, device=dev)
        self.cap = cap
        self.hidden = torch.zeros(1024, dtype=torch.float32, device=dev)
        self.emb_status = torch.zeros(1, dtype=torch.int32, device=dev)

    def _hist(self, record):
        return (self.hist_tok.data_ptr(), self.hist_score.data_ptr()) if record else (None, None)

    def separate(self, record):
        """q4d_embedding, the layers, q4d_lm_head_argmax, q4d_advance."""
        lib, st, ws = self.lib, current_stream(), self.ws
        check(lib.q4d_embedding(ctypes.byref(self.table), self.tok.data_ptr(), 1, self.hidden.data_ptr(),
                                self.emb_status.data_ptr(), st), "q4d_embedding")
        for li in range(LAYERS):
            check(lib.q4d_decoder_layer(ctypes.byref(self.desc), li, self.hidden.data_ptr(), self.hidden.data_ptr(),
                                        ctypes.byref(self.kvd), self.pos.data_ptr(), ws.ptr, ws.nbytes, st),
                  "q4d_decoder_layer")
        check(lib.q4d_lm_head_argmax(ctypes.byref(self.desc), self.hidden.data_ptr(), self.nxt.data_ptr(),
                                     self.score.data_ptr(), self.logits.data_ptr(), ws.ptr, ws.nbytes, st),
              "q4d_lm_head_argmax")
        ht, hs = self._hist(record)
        check(lib.q4d_advance(self.tok.data_ptr(), self.pos.data_ptr(), self.nxt.data_ptr(), self.score.data_ptr(),
                              ht, hs, self.hist_count.data_ptr(), self.cap, st), "q4d_advance")

    def plain(self, record):
        """q4d_run_one_token, then q4d_advance."""
        lib, st, ws = self.lib, current_stream(), self.ws
        check(lib.q4d_run_one_token(ctypes.byref(self.desc), self.tok.data_ptr(), self.pos.data_ptr(),
                                    ctypes.byref(self.kvd), self.nxt.data_ptr(), self.score.data_ptr(),
                                    self.logits.data_ptr(), ws.ptr, ws.nbytes, st), "q4d_run_one_token")
        ht, hs = self._hist(record)
        check(lib.q4d_advance(self.tok.data_ptr(), self.pos.data_ptr(), self.nxt.data_ptr(), self.score.data_ptr(),
                              ht, hs, self.hist_count.data_ptr(), self.cap, st), "q4d_advance")

    def feedback(self, record):
        ht, hs = self._hist(record)
        check(self.lib.q4d_run_one_token_feedback(
            ctypes.byref(self.desc), self.tok.data_ptr(), self.pos.data_ptr(), ctypes.byref(self.kvd),
            self.nxt.data_ptr(), self.score.data_ptr(), self.logits.data_ptr(), ht, hs, self.hist_count.data_ptr(),
            self.cap, self.ws.ptr, self.ws.nbytes, current_stream()), "q4d_run_one_token_feedback")

    def status(self):
        out = ctypes.c_int32(0)
        check(self.lib.q4d_read_status(self.ws.ptr, self.ws.nbytes, ctypes.byref(self.desc), 1, ctypes.byref(out),
                                       current_stream()), "q4d_read_status")
        return out.value | int(self.emb_status.item())

    def state(self):
        torch.cuda.synchronize()
        return [t.clone() for t in (self.tok, self.pos, self.nxt, self.score, self.logits, self.hist_tok,
                                    self.hist_score, self.hist_count, self.kv.data)]


NAMES = ("token", "position", "next", "score", "logits", "hist_tokens", "hist_scores", "hist_count", "kv")


def _cache(cfg, model, upto, seed, dev):
    kv = KVCache(cfg, LAYERS, 1, model.max_ctx, dev)
    g = torch.Generator(device=dev).manual_seed(seed)
    kv.data[..., :upto, :].normal_(generator=g)
    return kv.data


def test_feedback_step_equals_separate_launches(dev, small, plan):
    cfg, model = small
    p0, steps = 40, 6
    kv0 = _cache(cfg, model, p0, 11, dev)
    loops = {k: Loop(cfg, model, kv0, 321, p0, cap=3) for k in ("separate", "plain", "feedback")}
    for i in range(steps):
        record = i > 0          # the first step records nothing, then 5 recorded steps into capacity 3
        print(f"[feedback] plan {plan} step {i} position {p0 + i} record={record}", flush=True)
        for k, lp in loops.items():
            getattr(lp, k)(record)
        ref = loops["separate"].state()
        for k in ("plain", "feedback"):
            for name, r, g in zip(NAMES, ref, loops[k].state()):
                assert torch.equal(r, g), (k, i, name)
    ref = loops["separate"].state()
    assert int(ref[1].item()) == p0 + steps
    assert int(ref[7].item()) == 3                          # capacity reached, later tokens not recorded
    assert ref[5][:3].tolist() != [-5, -5, -5] and ref[5][3:].tolist() == [-5, -5]
    for lp in loops.values():
        assert lp.status() == 0


def test_feedback_bad_token_sets_status_and_zero_embedding(dev, small, plan):
    cfg, model = small
    p0 = 17
    kv0 = _cache(cfg, model, p0, 12, dev)
    for bad in (cfg.vocab_size, cfg.vocab_size + 1000, -1):
        print(f"[feedback] bad token {bad}", flush=True)
        ref = Loop(cfg, model, kv0, bad, p0, cap=4)
        got = Loop(cfg, model, kv0, bad, p0, cap=4)
        ref.separate(True)
        got.feedback(True)
        for name, r, g in zip(NAMES, ref.state(), got.state()):
            assert torch.equal(r, g), (bad, name)
        assert ref.status() & _lib.STATUS_BAD_TOKEN
        assert got.status() & _lib.STATUS_BAD_TOKEN
        # the step after a bad token runs on the fed-back (valid) token; the status word keeps its bit
        ref.separate(True)
        got.feedback(True)
        for name, r, g in zip(NAMES, ref.state(), got.state()):
            assert torch.equal(r, g), (bad, "second", name)
        assert got.status() & _lib.STATUS_BAD_TOKEN
