"""Helpers shared by the GPU tests: thin calls through the C ABI."""

import ctypes

import numpy as np
import torch

from llm_accelerator_amd import _lib
from llm_accelerator_amd._lib import Q4D_F16, Q4D_F32, Q4dModel, check
from llm_accelerator_amd.model import Q4Tensor, current_stream


def q4(packed, scale, dev="cuda"):
    return Q4Tensor.from_numpy(packed, scale, device=dev)


def linear(w: Q4Tensor, x: torch.Tensor, y_dtype=Q4D_F32) -> torch.Tensor:
    """q4d_linear over x [batch, K] (fp16 or fp32)."""
    rows, cols = w.shape
    x = x.contiguous()
    xd = Q4D_F16 if x.dtype == torch.float16 else Q4D_F32
    batch = x.numel() // cols
    y = torch.empty((batch, rows), dtype=torch.float16 if y_dtype == Q4D_F16 else torch.float32, device=x.device)
    desc = w.descriptor()
    check(_lib.load().q4d_linear(ctypes.byref(desc), x.data_ptr(), xd, y.data_ptr(), y_dtype, batch,
                                 current_stream()), "q4d_linear")
    return y


def head_model(table: Q4Tensor, final_norm: torch.Tensor, max_ctx=64) -> Q4dModel:
    """Model descriptor carrying just what q4d_lm_head_argmax reads."""
    rows, cols = table.shape
    m = Q4dModel(hidden_size=cols, intermediate_size=3072, num_layers=1, num_q_heads=16, num_kv_heads=8,
                 head_dim=128, vocab_size=rows, max_ctx=max_ctx, rms_norm_eps=1e-6, attn_scaling=128 ** -0.5)
    m.embed_tokens = table.descriptor()
    m.final_norm = final_norm.data_ptr()
    return m


def lm_head_argmax(table: Q4Tensor, hidden: torch.Tensor, final_norm: torch.Tensor, want_logits=True):
    lib = _lib.load()
    m = head_model(table, final_norm)
    nbytes = int(lib.q4d_workspace_bytes(ctypes.byref(m), 1))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=hidden.device)
    tok = torch.full((1,), -1, dtype=torch.int32, device=hidden.device)
    score = torch.zeros(1, dtype=torch.float32, device=hidden.device)
    logits = torch.empty(table.shape[0], dtype=torch.float32, device=hidden.device) if want_logits else None
    check(lib.q4d_lm_head_argmax(ctypes.byref(m), hidden.contiguous().data_ptr(), tok.data_ptr(), score.data_ptr(),
                                 logits.data_ptr() if logits is not None else None, ws.data_ptr(), nbytes,
                                 current_stream()), "q4d_lm_head_argmax")
    torch.cuda.synchronize()
    return int(tok.item()), float(score.item()), logits, ws


def abs_dot_bound(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """sum_j |W_ij x_j| per row: the scale of fp32 accumulation error."""
    return np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64))


def report(name, got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    mx = float(err.max()) if err.size else 0.0
    rel = mx / max(float(np.abs(ref).max()), 1e-30)
    print(f"[{name}] max_abs_err={mx:.3e} rel_err={rel:.3e} max|ref|={float(np.abs(ref).max()):.3e}", flush=True)
    return mx, rel


PLANS = [("xcd", 0, 2), ("staged", 1, 2), ("staged-fp16", 1, 1)]   # (id, decode plan, activation precision)


class decode_plan:
    """Run a block under one batch-1 decode plan and activation precision, restoring
    the previous plan and precision 2 afterwards."""

    def __init__(self, plan: int, precision: int = 2):
        self.plan, self.precision = plan, precision

    def __enter__(self):
        lib = _lib.load()
        self.prev = lib.q4d_set_decode_plan(self.plan)
        check(lib.q4d_set_activation_precision(self.precision), "q4d_set_activation_precision")
        return self

    def __exit__(self, *exc):
        lib = _lib.load()
        lib.q4d_set_decode_plan(self.prev)
        check(lib.q4d_set_activation_precision(2), "q4d_set_activation_precision")
        return False
