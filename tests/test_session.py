"""The decode session state machine (q4d_session_*) against the reference's own
session loop, compiled from its C sources into oracle/_ref/libqot_session.so
(FPGA_Project/software/qmap_prompt_demo/qot_session.c; oracle/build_ref.sh).

Both are driven by the same scripted runner (outputs, return codes) and must
produce the same return codes, the same event stream (kind, stop reason, input
token and position, prompts consumed, generated index, error code, result) and
the same session state after every step, and call the runner with the same
(token, position) sequence.  Scenarios: the cases of the reference's
test_session_host.c (prefill + feedback, EOS, <|im_end|>, context cap, runner
errors, out-of-vocabulary outputs, begin validation) and 400 seeded random ones
(prompt lengths, start positions up to the cap, budgets, stop tokens and flags,
errors).  No GPU.  Bar: equality.
"""

import ctypes
import subprocess
from ctypes import POINTER, c_int, c_int64, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np
import pytest

from llm_accelerator_amd import _lib
from llm_accelerator_amd._lib import Q4dSession, Q4dSessionEvent, Q4dSessionOptions, Q4dTokenResult

ROOT = Path(__file__).resolve().parents[1]
REF_SO = ROOT / "oracle" / "_ref" / "libqot_session.so"
MAX_CONTEXT, VOCAB = 256, 151936   # QOT_MAX_CONTEXT, QOT_VOCAB_SIZE (qmap_one_token_regs.h:14-16)
EOS, IM_END = 151643, 151645


# ------------------------------------------------------------ the reference's structs (qot_session.h)
class QotRunConfig(ctypes.Structure):
    _fields_ = [("layer_start", c_uint32), ("layer_count", c_uint32), ("position", c_uint32),
                ("runtime_context_enable", c_uint32), ("input_token_id", c_uint32), ("embedding_enable", c_uint32),
                ("embedding_weight_base", c_uint64), ("embedding_scale_base", c_uint64),
                ("input_hidden_base", c_uint64), ("output_hidden_base", c_uint64), ("kv_cache_base", c_uint64),
                ("final_tail_qmap_base", c_uint64), ("final_hidden_override_valid", c_uint32),
                ("final_hidden_override_base", c_uint64), ("layer_qmap_bases", c_void_p),
                ("layer_qmap_base_count", c_uint32)]


class QotResult(ctypes.Structure):
    _fields_ = [("status", c_uint32), ("token_id", c_uint32), ("score_q26", c_int64), ("layers_started", c_uint32),
                ("layers_completed", c_uint32), ("layer_done_mask", c_uint32), ("layer_error_mask", c_uint32),
                ("last_output_base", c_uint64), ("tail_hidden_base", c_uint64), ("tail_tiles_started", c_uint32),
                ("tail_tiles_completed", c_uint32), ("mem_read_reqs", c_uint32), ("mem_read_words", c_uint32),
                ("mem_write_reqs", c_uint32), ("mem_write_words", c_uint32)]


class QotOptions(ctypes.Structure):
    _fields_ = [("max_new_tokens", c_uint32), ("max_polls_per_token", c_uint32), ("eos_token_id", c_uint32),
                ("im_end_token_id", c_uint32), ("stop_on_eos", c_uint32), ("stop_on_im_end", c_uint32)]


class QotEvent(ctypes.Structure):
    _fields_ = [("kind", c_int), ("stop_reason", c_int), ("input_token_id", c_uint32), ("input_position", c_uint32),
                ("prompt_tokens_consumed", c_uint32), ("generated_index", c_uint32), ("error_code", c_int),
                ("result", QotResult)]


class QotSession(ctypes.Structure):
    _fields_ = [("base", ctypes.c_size_t), ("config", QotRunConfig), ("runner", c_void_p),
                ("runner_context", c_void_p), ("prompt_token_ids", c_void_p), ("prompt_token_count", c_uint32),
                ("prompt_index", c_uint32), ("next_position", c_uint32), ("pending_token_id", c_uint32),
                ("generated_count", c_uint32), ("options", QotOptions), ("last_result", QotResult),
                ("last_error", c_int), ("state", c_int), ("stop_reason", c_int)]


QOT_RUNNER = ctypes.CFUNCTYPE(c_int, c_void_p, ctypes.c_size_t, POINTER(QotRunConfig), c_uint32, c_uint32, c_uint32,
                              POINTER(QotResult))


@pytest.fixture(scope="module")
def ref():
    if not REF_SO.exists():
        subprocess.run(["bash", str(ROOT / "oracle" / "build_ref.sh")], check=True, capture_output=True)
    if not REF_SO.exists():
        pytest.skip("oracle/_ref/libqot_session.so is not built (the reference sources are not present)")
    lib = ctypes.CDLL(str(REF_SO))
    lib.qot_session_init.argtypes = [POINTER(QotSession), ctypes.c_size_t, POINTER(QotRunConfig), c_void_p, c_void_p]
    lib.qot_session_begin.argtypes = [POINTER(QotSession), c_void_p, c_uint32, POINTER(QotOptions)]
    lib.qot_session_step.argtypes = [POINTER(QotSession), POINTER(QotEvent)]
    lib.qot_session_reset.argtypes = [POINTER(QotSession)]
    lib.qot_session_default_options.argtypes = [POINTER(QotOptions)]
    lib.qot_session_is_terminal.argtypes = [POINTER(QotSession)]
    lib.qot_session_state_name.restype = ctypes.c_char_p
    lib.qot_session_stop_reason_name.restype = ctypes.c_char_p
    return lib


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


class Script:
    """The scripted runner: call i returns (outputs[i], codes[i]); records its inputs."""

    def __init__(self, outputs, codes=None):
        self.outputs, self.codes = list(outputs), list(codes or [0] * len(outputs))
        self.calls = []

    def next(self, token, position):
        i = len(self.calls)
        self.calls.append((int(token), int(position)))
        if i >= len(self.outputs):
            return -9, 0, 0   # QOT_ERR_CAPACITY, as the reference mock does past its script
        return self.codes[i], self.outputs[i], 1000 + i


def run_ref(ref, script, start, prompt, opts, steps=80, reset_and_rebegin=False):
    def cb(_ctx, _base, _cfg, token, position, _polls, result):
        rc, tok, score = script.next(token, position)
        ctypes.memset(result, 0, ctypes.sizeof(QotResult))
        result.contents.token_id, result.contents.score_q26 = tok, score
        return rc
    fn = QOT_RUNNER(cb)
    cfg = QotRunConfig(position=start, runtime_context_enable=1, embedding_enable=1)
    s = QotSession()
    log = [("init", ref.qot_session_init(ctypes.byref(s), 0xA0040000, ctypes.byref(cfg), ctypes.cast(fn, c_void_p), None))]
    return _drive(ref.qot_session_begin, ref.qot_session_step, ref.qot_session_reset, s, QotEvent, prompt,
                  None if opts is None else QotOptions(opts["max_new_tokens"], 0, opts["eos_token_id"],
                                                       opts["im_end_token_id"], opts["stop_on_eos"],
                                                       opts["stop_on_im_end"]), steps, log, reset_and_rebegin, fn)


def run_ours(lib, script, start, prompt, opts, steps=80, reset_and_rebegin=False):
    def cb(_ctx, token, position, result):
        rc, tok, score = script.next(token, position)
        ctypes.memset(result, 0, ctypes.sizeof(Q4dTokenResult))
        result.contents.token_id, result.contents.score_q26 = tok, score
        return rc
    fn = _lib.SESSION_RUNNER(cb)
    s = Q4dSession()
    log = [("init", lib.q4d_session_init(ctypes.byref(s), start, MAX_CONTEXT, VOCAB, ctypes.cast(fn, c_void_p), None))]
    return _drive(lib.q4d_session_begin, lib.q4d_session_step, lib.q4d_session_reset, s, Q4dSessionEvent, prompt,
                  None if opts is None else Q4dSessionOptions(opts["max_new_tokens"], opts["eos_token_id"],
                                                              opts["im_end_token_id"], opts["stop_on_eos"],
                                                              opts["stop_on_im_end"]), steps, log, reset_and_rebegin,
                  fn)


def _drive(begin, step, reset, s, Event, prompt, opts, steps, log, reset_and_rebegin, _keep):
    ids = (c_uint32 * max(1, len(prompt)))(*prompt)
    rounds = 2 if reset_and_rebegin else 1
    for _ in range(rounds):
        rc = begin(ctypes.byref(s), ids if prompt is not None else None, len(prompt),
                   ctypes.byref(opts) if opts is not None else None)
        log.append(("begin", rc, s.state))
        for _ in range(steps):
            ev = Event()
            rc = step(ctypes.byref(s), ctypes.byref(ev))
            log.append(("step", rc, ev.kind, ev.stop_reason, ev.input_token_id, ev.input_position,
                        ev.prompt_tokens_consumed, ev.generated_index, ev.error_code, ev.result.token_id,
                        ev.result.score_q26, s.state, s.stop_reason, s.next_position, s.generated_count))
            if rc != 0 and ev.kind == 0:
                break  # a state error: nothing more happens
        reset(ctypes.byref(s))
        log.append(("reset", s.state, s.next_position))
    return log


def both(ref, lib, outputs, codes=None, start=0, prompt=(1, 2), opts=None, steps=80, rebegin=False):
    a, b = Script(outputs, codes), Script(outputs, codes)
    la = run_ref(ref, a, start, list(prompt), opts, steps, rebegin)
    lb = run_ours(lib, b, start, list(prompt), opts, steps, rebegin)
    assert la == lb
    assert a.calls == b.calls
    return la, a.calls


def opts(max_new=1, eos=EOS, im_end=IM_END, stop_eos=1, stop_im=1):
    return {"max_new_tokens": max_new, "eos_token_id": eos, "im_end_token_id": im_end, "stop_on_eos": stop_eos,
            "stop_on_im_end": stop_im}


def test_reference_builds_and_passes_its_own_test(ref):
    out = (ROOT / "oracle" / "_ref" / "test_session_host.out")
    assert out.exists() and "PASS" in out.read_text()


def test_names_and_defaults(ref, lib):
    for i in range(-1, 9):
        assert ref.qot_session_state_name(i) == lib.q4d_session_state_name(i)
        assert ref.qot_session_stop_reason_name(i) == lib.q4d_session_stop_reason_name(i)
    a, b = QotOptions(), Q4dSessionOptions()
    ref.qot_session_default_options(ctypes.byref(a))
    lib.q4d_session_default_options(ctypes.byref(b))
    assert (a.max_new_tokens, a.eos_token_id, a.im_end_token_id, a.stop_on_eos, a.stop_on_im_end) == \
        (b.max_new_tokens, b.eos_token_id, b.im_end_token_id, b.stop_on_eos, b.stop_on_im_end) == (1, EOS, IM_END, 1, 1)


def test_reference_cases(ref, lib):
    """The scenarios of test_session_host.c, run on both."""
    log, calls = both(ref, lib, [99, 20, 21, 22], prompt=(10, 11), opts=opts(3))   # prefill + feedback, MAX_NEW
    assert calls == [(10, 0), (11, 1), (20, 2), (21, 3)]
    both(ref, lib, [7, EOS], prompt=(5,), opts=opts(5))                            # EOS
    both(ref, lib, [8, IM_END], prompt=(5,), opts=opts(5))                         # <|im_end|>
    both(ref, lib, [8, IM_END, 9], prompt=(5,), opts=opts(3, stop_im=0))           # flag off: continues
    both(ref, lib, [1, 2, 3, 4], start=MAX_CONTEXT - 2, prompt=(3, 4), opts=opts(8))  # prompt fills the context
    both(ref, lib, [6, 7], codes=[0, -5], prompt=(5,), opts=opts(3))                # runner timeout
    both(ref, lib, [VOCAB], prompt=(5,), opts=opts(3))                             # out-of-vocabulary output
    both(ref, lib, [1], start=MAX_CONTEXT - 1, prompt=(1, VOCAB), opts=opts(3))    # bad prompt token
    both(ref, lib, [1], start=MAX_CONTEXT - 1, prompt=(1, 2), opts=opts(3))        # prompt past the context
    both(ref, lib, [1], start=MAX_CONTEXT - 1, prompt=(1,), opts=opts(0))          # no budget
    both(ref, lib, [1], prompt=(1,), opts=opts(2, eos=VOCAB))                      # stop token outside vocab
    both(ref, lib, [1], prompt=(1,), opts=opts(2, eos=VOCAB, stop_eos=0))          # ... unused: fine
    both(ref, lib, [1, 2, 3], prompt=(1,), opts=None)                              # default options
    both(ref, lib, [4, 5, 6, 7, 8, 9], prompt=(2, 3), opts=opts(2), rebegin=True)  # reset, then a new sequence
    both(ref, lib, [], prompt=(), opts=opts(2))                                    # empty prompt


def test_state_errors(ref, lib):
    """Stepping an IDLE (never begun) or finished session is a state error on both."""
    for api in ("ref", "ours"):
        if api == "ref":
            s, ev = QotSession(), QotEvent()
            cfg = QotRunConfig(position=0, runtime_context_enable=1, embedding_enable=1)
            fn = QOT_RUNNER(lambda *a: 0)
            assert ref.qot_session_init(ctypes.byref(s), 0, ctypes.byref(cfg), ctypes.cast(fn, c_void_p), None) == 0
            assert ref.qot_session_step(ctypes.byref(s), ctypes.byref(ev)) == -100
        else:
            s, ev = Q4dSession(), Q4dSessionEvent()
            fn = _lib.SESSION_RUNNER(lambda *a: 0)
            assert lib.q4d_session_init(ctypes.byref(s), 0, MAX_CONTEXT, VOCAB, ctypes.cast(fn, c_void_p), None) == 0
            assert lib.q4d_session_step(ctypes.byref(s), ctypes.byref(ev)) == -100
            assert lib.q4d_session_init(ctypes.byref(s), MAX_CONTEXT, MAX_CONTEXT, VOCAB, ctypes.cast(fn, c_void_p),
                                        None) == -10
            assert lib.q4d_session_is_terminal(None) == 1


@pytest.mark.parametrize("seed", range(8))
def test_random_scenarios(ref, lib, seed):
    rng = np.random.default_rng(seed)
    for _ in range(50):
        n_prompt = int(rng.integers(0, 9))
        start = int(rng.choice([0, int(rng.integers(0, MAX_CONTEXT)), MAX_CONTEXT - int(rng.integers(1, 12))]))
        prompt = [int(t) for t in rng.integers(0, VOCAB, n_prompt)]
        if n_prompt and rng.random() < 0.05:
            prompt[int(rng.integers(0, n_prompt))] = VOCAB + int(rng.integers(0, 3))
        n = int(rng.integers(1, 40))
        outputs = [int(t) for t in rng.integers(0, 200, n)]
        for i in range(n):
            r = rng.random()
            if r < 0.06:
                outputs[i] = EOS
            elif r < 0.12:
                outputs[i] = IM_END
            elif r < 0.14:
                outputs[i] = VOCAB + int(rng.integers(0, 5))
        codes = [0 if rng.random() > 0.03 else int(rng.choice([-5, -6, -12])) for _ in range(n)]
        o = opts(int(rng.choice([0, 1, 2, 5, 17, 300])), int(rng.choice([EOS, 7, VOCAB])),
                 int(rng.choice([IM_END, 9, VOCAB + 1])), int(rng.integers(0, 2)), int(rng.integers(0, 2)))
        both(ref, lib, outputs, codes, start, prompt, None if rng.random() < 0.1 else o, steps=int(rng.integers(1, 60)),
             rebegin=bool(rng.random() < 0.2))
