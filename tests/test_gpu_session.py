"""The decode session with its GPU runners.

- Float runner (q4d_session_gpu_runner = one q4d_run_one_token per step): the
  generated tokens and scores equal the eager greedy decoder's on the same model
  (same kernels per step; the decoder itself is checked against the oracle in
  test_gpu_decode.py); the event stream has one PREFILL per prompt token but the
  last, then TOKEN events, then DONE with the stop reason: MAX_NEW, EOS (the end
  token set to the token the decoder produces at step 3) and CONTEXT (a model whose
  capacity ends two tokens after the prompt).
- Fixed-point runner (q4d_session_fixed_runner): tokens and Q26 scores equal the
  oracle's fixed_run_one_token loop exactly.
- Stop rules on the device (q4d_advance_session via GreedyDecoder.run_session, eager
  and HIP-graph replays): the same tokens and stop reason as the host session for the
  budget, end-of-text, end-of-turn and context-cap cases.
"""

import numpy as np
import pytest
import torch

from oracle import q4_fixed as F
import oracle as o
from llm_accelerator_amd import fixed as X
from llm_accelerator_amd.decode import GreedyDecoder
from llm_accelerator_amd.model import Qwen3Config, build_model, random_host_weights
from llm_accelerator_amd.session import DecodeSession

pytestmark = pytest.mark.gpu

PROMPT = [11, 257, 1999, 4, 3000]


@pytest.fixture(scope="module")
def small(dev):
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=4096)
    host = random_host_weights(cfg, seed=12, num_layers=2)
    return cfg, host


def greedy(model, prompt, n):
    dec = GreedyDecoder(model, use_graph=False)
    dec.prefill(prompt)
    dec.generate(n - 1)
    torch.cuda.synchronize()
    return dec.history()


def test_float_runner_matches_greedy_decoder(dev, small):
    cfg, host = small
    model = build_model(cfg, host, max_ctx=64, device=dev)
    ref_tokens, ref_scores = greedy(model, PROMPT, 8)
    print(f"[session] greedy tokens {ref_tokens}", flush=True)
    sess = DecodeSession.on_gpu(build_model(cfg, host, max_ctx=64, device=dev))
    events, toks, why = sess.run(PROMPT, max_new_tokens=8, eos_token_id=4095, im_end_token_id=4094)
    assert toks == list(ref_tokens) and why == "MAX_NEW"
    np.testing.assert_array_equal(np.array([e["score"] for e in events if e["kind"] == "TOKEN"], np.float32),
                                  np.array(ref_scores, np.float32))
    kinds = [e["kind"] for e in events]
    assert kinds == ["PREFILL"] * 4 + ["TOKEN"] * 8 + ["DONE"]
    assert [e["input_position"] for e in events[:-1]] == list(range(12))
    assert [e["input_token_id"] for e in events[:5]] == PROMPT
    assert [e["input_token_id"] for e in events[5:12]] == list(ref_tokens[:7])


def test_float_runner_stop_reasons(dev, small):
    cfg, host = small
    model = build_model(cfg, host, max_ctx=64, device=dev)
    ref_tokens, _ = greedy(model, PROMPT, 8)
    eos = int(ref_tokens[3])
    first = next(i for i, t in enumerate(ref_tokens) if t == eos)
    sess = DecodeSession.on_gpu(build_model(cfg, host, max_ctx=64, device=dev))
    _, toks, why = sess.run(PROMPT, max_new_tokens=20, eos_token_id=eos, im_end_token_id=4094)
    assert why == "EOS" and toks == list(ref_tokens[:first + 1])
    small_ctx = build_model(cfg, host, max_ctx=len(PROMPT) + 2, device=dev)
    sess = DecodeSession.on_gpu(small_ctx)
    events, toks, why = sess.run(PROMPT, max_new_tokens=20, eos_token_id=4095, im_end_token_id=4094)
    assert why == "CONTEXT" and toks == list(ref_tokens[:3])
    assert events[-2]["stop_reason"] == "CONTEXT" and events[-1]["kind"] == "DONE"


def test_fixed_runner_matches_oracle(dev, small):
    cfg, host = small
    model = build_model(cfg, host, max_ctx=32, device=dev)
    fx = X.FixedQ4Model(model, host)
    sess = DecodeSession.on_gpu_fixed(fx)
    events, toks, why = sess.run(PROMPT, max_new_tokens=6, eos_token_id=4095, im_end_token_id=4094)
    q = lambda v: F.quantize_signed(v, 16, 7)[0]  # noqa: E731
    mats = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
    layers = [F.FixedLayer(*[L[m] for m in mats], q(L["input_layernorm"]), q(L["post_attention_layernorm"]),
                           q(L["q_norm"]), q(L["k_norm"])) for L in host["layers"]]
    cos, sin = F.rope_table_q1_15(o.rope_inv_freq(cfg.rope_theta, cfg.head_dim), np.arange(32))
    om = F.FixedModel(layers, host["embed_tokens"], q(host["norm"]), cos, sin, F.score_scale_q0_31(128 ** -0.5))
    kcs = [np.zeros((32, 8, 128), dtype=np.int64) for _ in range(2)]
    vcs = [np.zeros((32, 8, 128), dtype=np.int64) for _ in range(2)]
    ref_toks, ref_scores, tok = [], [], PROMPT[0]
    for pos in range(len(PROMPT) + 5):
        t, s, _, _ = F.fixed_run_one_token(tok, pos, om, kcs, vcs)
        if pos >= len(PROMPT) - 1:
            ref_toks.append(t)
            ref_scores.append(s)
            tok = t
        else:
            tok = PROMPT[pos + 1]
    print(f"[session] fixed-point tokens {toks} oracle {ref_toks}", flush=True)
    assert toks == ref_toks and why == "MAX_NEW"
    assert [e["score_q26"] for e in events if e["kind"] == "TOKEN"] == ref_scores


@pytest.mark.parametrize("graph", [False, True])
def test_device_stops_match_host_session(dev, small, graph):
    """GreedyDecoder.run_session (stop rules on the device, graph replays) = the host session."""
    cfg, host = small
    model = build_model(cfg, host, max_ctx=24, device=dev)
    ref_tokens, _ = greedy(model, PROMPT, 8)
    dec = GreedyDecoder(model, steps_per_graph=4, use_graph=graph)
    cases = [dict(max_new_tokens=7, eos_token_id=4095, im_end_token_id=4094),          # budget
             dict(max_new_tokens=20, eos_token_id=int(ref_tokens[2]), im_end_token_id=4094),  # end-of-text
             dict(max_new_tokens=20, eos_token_id=4095, im_end_token_id=int(ref_tokens[4])),  # end-of-turn
             dict(max_new_tokens=40, eos_token_id=None, im_end_token_id=None)]            # context cap
    for kw in cases:
        toks, scores, why = dec.run_session(PROMPT, **kw)
        hk = {k: (v if v is not None else 0) for k, v in kw.items()}
        hk.update(stop_on_eos=int(kw["eos_token_id"] is not None), stop_on_im_end=int(kw["im_end_token_id"] is not None))
        sess = DecodeSession.on_gpu(build_model(cfg, host, max_ctx=24, device=dev))
        _, htoks, hwhy = sess.run(PROMPT, **hk)
        print(f"[session] device stop {why} {toks} host {hwhy} {htoks}", flush=True)
        assert (toks, why) == (htoks, hwhy)
    assert dec.status() == 0
