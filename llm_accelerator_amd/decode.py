"""Greedy decode driver: serial prefill, then device-resident token feedback.

The loop is the reference's (``10_validate_full_run_one_token.py:81-172``,
``Qwen3-0.6B-Base/pc_testing/02_serial_decode.py:33-59``, and the board's
``qot_decode_token_ids``, ``qmap_one_token_runtime.h:399+``): every prompt
token runs one full step at its position, the argmax after the last prompt
token is the first generated id, and each generated id is fed back at the
next position.  Here the token and position live in device memory and the
step moves them forward itself (``q4d_run_one_token_feedback``: the LM head's
last block stores the feedback; the session mode uses ``q4d_advance_session``
for its stop rules), so a HIP graph of ``steps_per_graph`` captured steps
replays the loop with no host round trip per token.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import check
from .model import KVCache, Q4ForCausalLM, Workspace, current_stream


class GreedyDecoder:
    def __init__(self, model: Q4ForCausalLM, steps_per_graph: int = 16, use_graph: bool = True):
        self.model = model
        cfg = model.config
        dev = model.device
        self.kv = KVCache(cfg, len(model.model.layers), 1, model.max_ctx, dev)
        self.ws = Workspace(model, 1)
        self.tok = torch.zeros(1, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.next_tok = torch.zeros(1, dtype=torch.int32, device=dev)
        self.score = torch.zeros(1, dtype=torch.float32, device=dev)
        self.hist_cap = model.max_ctx
        self.hist_tok = torch.zeros(self.hist_cap, dtype=torch.int32, device=dev)
        self.hist_score = torch.zeros(self.hist_cap, dtype=torch.float32, device=dev)
        self.hist_count = torch.zeros(1, dtype=torch.int32, device=dev)
        self.steps_per_graph = steps_per_graph
        self.use_graph = use_graph
        self._graph = None
        self._desc = model.descriptor()
        self._kvd = self.kv.descriptor()
        self._lib = _lib.load()
        self._prefill = None
        self.position = 0
        # device stop state of the session mode (q4d_advance_session): done, reason, generated,
        # max new, end-of-text id, end-of-turn id, max context, unused; None = plain feedback
        self._stop = None
        self._stop_buf = torch.zeros(8, dtype=torch.int32, device=dev)  # captured graphs keep its address
        self._graph_session = None

    # -- one step, launched on the current stream ---------------------------------
    def _launch_step(self, logits: torch.Tensor | None = None, record: bool = True) -> None:
        st = current_stream()
        if self._stop is None:
            check(self._lib.q4d_run_one_token_feedback(
                ctypes.byref(self._desc), self.tok.data_ptr(), self.pos.data_ptr(), ctypes.byref(self._kvd),
                self.next_tok.data_ptr(), self.score.data_ptr(), logits.data_ptr() if logits is not None else None,
                self.hist_tok.data_ptr() if record else None, self.hist_score.data_ptr() if record else None,
                self.hist_count.data_ptr(), self.hist_cap, self.ws.ptr, self.ws.nbytes, st),
                "q4d_run_one_token_feedback")
            return
        check(self._lib.q4d_run_one_token(ctypes.byref(self._desc), self.tok.data_ptr(), self.pos.data_ptr(),
                                          ctypes.byref(self._kvd), self.next_tok.data_ptr(),
                                          self.score.data_ptr(), logits.data_ptr() if logits is not None else None,
                                          self.ws.ptr, self.ws.nbytes, st), "q4d_run_one_token")
        if record:
            check(self._lib.q4d_advance_session(self.tok.data_ptr(), self.pos.data_ptr(), self.next_tok.data_ptr(),
                                                self.score.data_ptr(), self.hist_tok.data_ptr(),
                                                self.hist_score.data_ptr(), self.hist_count.data_ptr(), self.hist_cap,
                                                self._stop.data_ptr(), st), "q4d_advance_session")
            return
        check(self._lib.q4d_advance(self.tok.data_ptr(), self.pos.data_ptr(), self.next_tok.data_ptr(),
                                    self.score.data_ptr(), None, None, self.hist_count.data_ptr(),
                                    self.hist_cap, st), "q4d_advance")

    def reset(self) -> None:
        self.kv.data.zero_()
        self.hist_count.zero_()
        self.pos.zero_()
        self.position = 0
        self.ws.reset()

    def plan(self) -> int:
        """The decode plan the steps run (q4d_decode_plan_active: DECODE_XCD or DECODE_STAGED)."""
        return int(self._lib.q4d_decode_plan_active(ctypes.byref(self._desc), current_stream()))

    def step(self, token: int | None = None, logits: torch.Tensor | None = None, record: bool = True) -> None:
        """One eager step; ``token`` overrides the fed-back id (teacher forcing)."""
        if self.position >= self.model.max_ctx:
            raise _lib.Q4DecError(-10, "GreedyDecoder.step")
        if token is not None:
            if not 0 <= int(token) < self.model.config.vocab_size:
                raise _lib.Q4DecError(-8, "GreedyDecoder.step")
            self.tok.fill_(int(token))
        self._launch_step(logits, record)
        self.position += 1

    def prefill(self, prompt: list[int], parallel: bool = False) -> None:
        """Serial prefill (default): one full step per prompt token, as the
        reference does; only the step after the last prompt token records its
        argmax as generated token 0.  ``parallel=True`` runs all prompt tokens
        through each layer at once (q4d_prefill: MFMA GEMMs and causal
        attention), then records the same generated token 0."""
        self.reset()
        if not parallel:
            for i, t in enumerate(prompt):
                self.step(int(t), record=(i == len(prompt) - 1))
            return
        if not prompt or len(prompt) > self.model.max_ctx:
            raise _lib.Q4DecError(-10, "GreedyDecoder.prefill")
        if self._prefill is None or self._prefill.max_tokens < len(prompt):
            self._prefill = Prefill(self.model, self.kv, max(len(prompt), 64))
        self._prefill.run(prompt, start_pos=0, seq=0, next_token=self.next_tok, score=self.score)
        # q4d_advance feeds the argmax back at position len(prompt) and records it
        self.pos.fill_(len(prompt) - 1)
        check(self._lib.q4d_advance(self.tok.data_ptr(), self.pos.data_ptr(), self.next_tok.data_ptr(),
                                    self.score.data_ptr(), self.hist_tok.data_ptr(), self.hist_score.data_ptr(),
                                    self.hist_count.data_ptr(), self.hist_cap, current_stream()), "q4d_advance")
        self.position = len(prompt)

    def _capture(self) -> None:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                for _ in range(self.steps_per_graph):
                    self._launch_step()
        torch.cuda.current_stream().wait_stream(s)
        self._graph = g

    def generate(self, n: int) -> None:
        """Run ``n`` more feedback steps (graph replays when enabled)."""
        if self.position + n > self.model.max_ctx:
            raise _lib.Q4DecError(-10, "GreedyDecoder.generate")
        if not self.use_graph:
            for _ in range(n):
                self.step()
            return
        k = self.steps_per_graph
        full, rest = divmod(n, k)
        if full:
            if self._graph is None:
                # capturing records launches only; the captured steps run on replay
                self._capture()
            for _ in range(full):
                self._graph.replay()
            self.position += full * k
        for _ in range(rest):
            self.step()

    def run_session(self, prompt: list[int], max_new_tokens: int, eos_token_id: int | None = 151643,
                    im_end_token_id: int | None = 151645) -> tuple[list[int], list[float], str]:
        """The decode session (qot_session semantics: serial prefill, stop on end-of-text /
        end-of-turn / the new-token budget / the context cap) with the stop rules applied on
        the device: graphs of ``steps_per_graph`` steps replay until the device says done, one
        host read per replay.  ``None`` disables a stop token.  Returns (generated ids, their
        logits, stop reason)."""
        if max_new_tokens <= 0:
            raise _lib.Q4DecError(-9, "GreedyDecoder.run_session")
        vocab = self.model.config.vocab_size
        for t in (eos_token_id, im_end_token_id):
            if t is not None and not 0 <= t < vocab:
                raise _lib.Q4DecError(-8, "GreedyDecoder.run_session")
        if not prompt or len(prompt) > self.model.max_ctx:
            raise _lib.Q4DecError(-10, "GreedyDecoder.run_session")
        self._stop_buf.copy_(torch.tensor([0, 0, 0, max_new_tokens, -1 if eos_token_id is None else eos_token_id,
                                           -1 if im_end_token_id is None else im_end_token_id, self.model.max_ctx,
                                           0], dtype=torch.int32))
        self._stop = self._stop_buf
        try:
            self.prefill(prompt)
            while not int(self._stop[0].item()):
                if self.use_graph:
                    if self._graph_session is None:
                        self._graph_session = self._capture_steps()
                    self._graph_session.replay()
                else:
                    self._launch_step()
            self.position = int(self.pos.item()) + 1
            toks, scores = self.history()
            reasons = ["NONE", "EOS", "IM_END", "MAX_NEW", "CONTEXT", "HW_ERROR"]
            return toks, scores, reasons[int(self._stop[1].item())]
        finally:
            self._stop = None

    def _capture_steps(self):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                for _ in range(self.steps_per_graph):
                    self._launch_step()
        torch.cuda.current_stream().wait_stream(s)
        return g

    def history(self) -> tuple[list[int], list[float]]:
        """Generated ids and their logits so far.  Raises Q4DecError(Q4D_ERR_STATUS) when
        the device status word reports a failed step (the history is then not valid)."""
        st = self.status()
        if st:
            _lib.check_status(st, "GreedyDecoder")
        c = int(self.hist_count.item())
        return self.hist_tok[:c].tolist(), self.hist_score[:c].tolist()

    def status(self) -> int:
        return self.ws.status()


class Prefill:
    """Many tokens of one sequence through every layer at once (q4d_prefill).

    Per token the result is ``run_manual_one_token`` at that token's position
    (``10_validate_full_run_one_token.py:17-56``; the reference feeds a prompt
    through it one token at a time, ``:81-135``): every position's K/V row is
    appended to the cache and the argmax after the last token is returned.
    The projections run as MFMA GEMMs over the tokens (activations rounded to
    fp16) and attention is causal flash attention on MFMA.
    """

    def __init__(self, model: Q4ForCausalLM, kv: KVCache, max_tokens: int):
        self.model, self.kv, self.max_tokens = model, kv, int(max_tokens)
        self._desc = model.descriptor()
        self._kvd = kv.descriptor()
        lib = _lib.load()
        self.nbytes = int(lib.q4d_prefill_workspace_bytes(ctypes.byref(self._desc), self.max_tokens))
        if self.nbytes == 0:
            raise _lib.Q4DecError(-11, "q4d_prefill_workspace_bytes")
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=model.device)
        check(lib.q4d_workspace_init(self.buf.data_ptr(), self.nbytes, ctypes.byref(self._desc), 1,
                                     current_stream()), "q4d_workspace_init")
        self.tokens = torch.zeros(self.max_tokens, dtype=torch.int32, device=model.device)

    def run(self, tokens, start_pos: int = 0, seq: int = 0, next_token: torch.Tensor | None = None,
            score: torch.Tensor | None = None, logits: torch.Tensor | None = None):
        """tokens: list of ids or a device int32 tensor.  Returns (next_token, score) device tensors."""
        n = len(tokens)
        if n > self.max_tokens:
            raise _lib.Q4DecError(-9, "Prefill.run")
        if isinstance(tokens, torch.Tensor) and tokens.is_cuda and tokens.dtype == torch.int32:
            self.tokens[:n].copy_(tokens)
        else:
            self.tokens[:n].copy_(torch.as_tensor([int(t) for t in tokens], dtype=torch.int32))
        dev = self.model.device
        next_token = next_token if next_token is not None else torch.zeros(1, dtype=torch.int32, device=dev)
        score = score if score is not None else torch.zeros(1, dtype=torch.float32, device=dev)
        check(_lib.load().q4d_prefill(ctypes.byref(self._desc), self.tokens.data_ptr(), n, int(start_pos), int(seq),
                                      ctypes.byref(self._kvd), next_token.data_ptr(), score.data_ptr(),
                                      logits.data_ptr() if logits is not None else None, self.buf.data_ptr(),
                                      self.nbytes, current_stream()), "q4d_prefill")
        return next_token, score


def greedy_generate(model: Q4ForCausalLM, prompt: list[int], max_new_tokens: int, use_graph: bool = True,
                    steps_per_graph: int = 16) -> tuple[list[int], list[float]]:
    """Prompt ids -> ``max_new_tokens`` greedy ids and their winning logits."""
    dec = GreedyDecoder(model, steps_per_graph=steps_per_graph, use_graph=use_graph)
    dec.prefill(prompt)
    dec.generate(max_new_tokens - 1)
    torch.cuda.synchronize()
    return dec.history()


class BatchedDecoder:
    """One decode step for many independent sequences at once (q4d_decode_batch).

    Every sequence has its own cache slot and position; per sequence the step
    is ``run_manual_one_token`` (``10_validate_full_run_one_token.py:17-56``).
    The projections and the LM head run as MFMA GEMMs over the batch, so the
    weights are read once per step for all sequences.
    """

    def __init__(self, model: Q4ForCausalLM, batch: int, cache: KVCache | None = None):
        dev = model.device
        self.model, self.batch = model, batch
        self.kv = cache if cache is not None else KVCache(model.config, len(model.model.layers), batch,
                                                          model.max_ctx, dev)
        if self.kv.batch < batch:
            raise ValueError(f"cache holds {self.kv.batch} sequences, need {batch}")
        self.ws = Workspace(model, batch)
        self.next_tok = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.score = torch.zeros(batch, dtype=torch.float32, device=dev)
        self._desc = model.descriptor()
        self._kvd = self.kv.descriptor()

    def step(self, tokens: torch.Tensor, positions: torch.Tensor,
             logits: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """tokens, positions: device int32 [batch].  Appends K/V at each
        sequence's position and returns (next tokens, winning logits)."""
        for t, name in ((tokens, "tokens"), (positions, "positions")):
            if t.dtype != torch.int32 or t.numel() != self.batch or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous device int32 tensor of {self.batch} elements")
        if logits is not None and (logits.dtype != torch.float32 or
                                   logits.numel() != self.batch * self.model.config.vocab_size):
            raise ValueError("logits must be fp32 [batch, vocab]")
        check(_lib.load().q4d_decode_batch(ctypes.byref(self._desc), tokens.data_ptr(), positions.data_ptr(),
                                           self.batch, ctypes.byref(self._kvd), self.next_tok.data_ptr(),
                                           self.score.data_ptr(), logits.data_ptr() if logits is not None else None,
                                           self.ws.ptr, self.ws.nbytes, current_stream()), "q4d_decode_batch")
        return self.next_tok, self.score

    def status(self) -> int:
        return self.ws.status()
