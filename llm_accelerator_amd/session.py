"""Decode session: the board session loop's state machine driving GPU decode steps.

Mirrors ``qot_session`` (FPGA_Project/software/qmap_prompt_demo/qot_session.{h,c}):
``begin(prompt, options)`` then one ``step()`` per model invocation, each returning
one event: PREFILL while prompt tokens are consumed (their predictions dropped),
TOKEN for every generated token (fed back as the next input), DONE once a stop
reason holds (end-of-text 151643, end-of-turn 151645, the new-token budget, the
context cap), ERROR if a step fails.  The state machine runs in libq4dec
(``q4d_session_*``); the runner is one GPU decode step (``q4d_session_gpu_runner``,
float path, or ``q4d_session_fixed_runner``, the RTL-exact integer path), or any
callable for host tests.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import (Q4dGpuRunner, Q4dSession, Q4dSessionEvent, Q4dSessionOptions, Q4dTokenResult, SESSION_RUNNER,
                   check)
from .model import KVCache, Q4ForCausalLM, Workspace, current_stream

EVENT_KINDS = ["NONE", "PREFILL", "TOKEN", "DONE", "ERROR"]
STATES = ["UNINITIALIZED", "IDLE", "PREFILL", "DECODE", "STOPPING", "DONE", "ERROR"]
STOP_REASONS = ["NONE", "EOS", "IM_END", "MAX_NEW", "CONTEXT", "HW_ERROR"]
EOS_TOKEN_ID, IM_END_TOKEN_ID = 151643, 151645


def default_options(**kw) -> Q4dSessionOptions:
    """``qot_session_default_options`` with keyword overrides."""
    o = Q4dSessionOptions()
    _lib.load().q4d_session_default_options(ctypes.byref(o))
    for k, v in kw.items():
        setattr(o, k, int(v))
    return o


def event_dict(ev: Q4dSessionEvent) -> dict:
    return {"kind": EVENT_KINDS[ev.kind], "stop_reason": STOP_REASONS[ev.stop_reason],
            "input_token_id": ev.input_token_id, "input_position": ev.input_position,
            "prompt_tokens_consumed": ev.prompt_tokens_consumed, "generated_index": ev.generated_index,
            "error_code": ev.error_code, "token_id": ev.result.token_id, "score": ev.result.score,
            "score_q26": ev.result.score_q26, "status": ev.result.status}


class DecodeSession:
    """One sequence's decode session over a runner (see module docstring)."""

    def __init__(self, runner_fn, runner_context, max_context: int, vocab_size: int, start_position: int = 0,
                 keepalive=()):
        self._lib = _lib.load()
        self._keep = list(keepalive)
        self.s = Q4dSession()
        check(self._lib.q4d_session_init(ctypes.byref(self.s), start_position, max_context, vocab_size, runner_fn,
                                         runner_context), "q4d_session_init")
        self._prompt = None

    @classmethod
    def on_gpu(cls, model: Q4ForCausalLM, kv: KVCache | None = None, ws: Workspace | None = None,
               start_position: int = 0) -> "DecodeSession":
        """Runner = ``q4d_run_one_token`` on ``model`` (a fresh cache / workspace if not given)."""
        kv = kv or KVCache(model.config, model.config.num_hidden_layers, 1, model.max_ctx, model.device)
        ws = ws or Workspace(model, 1)
        io = torch.zeros(8, dtype=torch.int32, device=model.device)
        desc, kvd = model.descriptor(), kv.descriptor()
        ctx = Q4dGpuRunner(ctypes.addressof(desc), ctypes.addressof(kvd), ws.ptr, ws.nbytes, current_stream(),
                           io.data_ptr())
        lib = _lib.load()
        fn = ctypes.cast(lib.q4d_session_gpu_runner, ctypes.c_void_p).value
        sess = cls(fn, ctypes.addressof(ctx), model.max_ctx, model.config.vocab_size, start_position,
                   keepalive=(kv, ws, io, desc, kvd, ctx))
        sess.kv, sess.ws = kv, ws
        return sess

    @classmethod
    def on_gpu_fixed(cls, fixed_model, kv=None, start_position: int = 0) -> "DecodeSession":
        """Runner = ``q4d_fixed_run_one_token`` (RTL-exact integer decode) on a FixedQ4Model."""
        kv = kv or fixed_model.new_cache()
        io = torch.zeros(8, dtype=torch.int32, device=fixed_model.model.device)
        desc, kvd = fixed_model.descriptor(), kv.descriptor()
        ctx = Q4dGpuRunner(ctypes.addressof(desc), ctypes.addressof(kvd), fixed_model.ws.data_ptr(),
                           fixed_model.ws_bytes, current_stream(), io.data_ptr())
        lib = _lib.load()
        fn = ctypes.cast(lib.q4d_session_fixed_runner, ctypes.c_void_p).value
        sess = cls(fn, ctypes.addressof(ctx), fixed_model.model.max_ctx, fixed_model.config.vocab_size,
                   start_position, keepalive=(kv, io, desc, kvd, ctx, fixed_model))
        sess.kv = kv
        return sess

    @classmethod
    def with_callable(cls, fn, max_context: int, vocab_size: int, start_position: int = 0) -> "DecodeSession":
        """Runner = ``fn(token, position) -> (rc, token_id, score)`` (host tests)."""
        def tramp(_ctx, token, position, result):
            rc, tok, score = fn(int(token), int(position))
            result.contents.token_id = tok
            result.contents.score_q26 = int(score)
            return rc
        cb = SESSION_RUNNER(tramp)
        return cls(ctypes.cast(cb, ctypes.c_void_p).value, None, max_context, vocab_size, start_position,
                   keepalive=(cb,))

    # -------------------------------------------------------------- qot_session API
    def begin(self, prompt, options: Q4dSessionOptions | None = None, **kw) -> None:
        ids = (ctypes.c_uint32 * max(1, len(prompt)))(*[int(t) for t in prompt])
        self._prompt = ids  # the library keeps the pointer until DONE / ERROR
        opts = options if options is not None else (default_options(**kw) if kw else None)
        check(self._lib.q4d_session_begin(ctypes.byref(self.s), ids, len(prompt),
                                          ctypes.byref(opts) if opts is not None else None), "q4d_session_begin")

    def step(self) -> dict:
        ev = Q4dSessionEvent()
        rc = self._lib.q4d_session_step(ctypes.byref(self.s), ctypes.byref(ev))
        if rc not in (0,) and ev.kind != 4:
            check(rc, "q4d_session_step")
        return event_dict(ev)

    def run(self, prompt, **kw) -> tuple[list, list, str]:
        """begin + step until terminal: (events, generated token ids, stop reason)."""
        self.begin(prompt, **kw)
        events = []
        while not self.is_terminal:
            events.append(self.step())
        toks = [e["token_id"] for e in events if e["kind"] == "TOKEN"]
        return events, toks, STOP_REASONS[self.s.stop_reason]

    def reset(self) -> None:
        self._lib.q4d_session_reset(ctypes.byref(self.s))

    @property
    def is_terminal(self) -> bool:
        return bool(self._lib.q4d_session_is_terminal(ctypes.byref(self.s)))

    @property
    def state(self) -> str:
        return STATES[self.s.state]

    @property
    def stop_reason(self) -> str:
        return STOP_REASONS[self.s.stop_reason]


__all__ = ["DecodeSession", "default_options", "event_dict", "EOS_TOKEN_ID", "IM_END_TOKEN_ID", "Q4dTokenResult"]
