"""Device drop-in for the reference's integer (fixed-point) Q4 GEMV helpers.

Same names and argument meaning as the exporters' numpy functions, with the
weight given as a packed :class:`~llm_accelerator_amd.model.Q4Tensor`
(codes + Q2.14 scales, Source/Q4_FORMAT.md) instead of unpacked int8 codes
and a separate scale array, and tensors on the GPU:

* ``compute_q4_gemv_q26`` / ``q26_to_q12_12``
  (Qwen3-0.6B-Base/python_each_module/28_export_mlp_gate_up_vectors.py:124-138);
* ``q4_gemv_from_ints`` (13_export_q4_gemv_vectors.py:138-154);
* ``streamed_argmax_q26``: the LM-head scan's result
  (56_export_persistent_multitoken_layer_golden.py:766-798,860).

Every result is exact (int64 accumulation of the Q26 row sums).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import check
from .model import Q4Tensor, current_stream

ACT_FRAC = 12
SCALE_FRAC = 14


def _act(x: torch.Tensor, k: int) -> torch.Tensor:
    if x.numel() != k:
        raise ValueError(f"activation of {x.numel()} values for a matrix of {k} columns")
    x = x.reshape(-1)
    if x.dtype != torch.int32:
        if x.dtype.is_floating_point:
            raise TypeError("integer activations expected (Q12.12 / Q4.12 codes)")
        x = x.to(torch.int32)
    return x.to(device="cuda").contiguous() if not x.is_cuda else x.contiguous()


def compute_q4_gemv_q26(activation_q12_12: torch.Tensor, weight: Q4Tensor) -> torch.Tensor:
    """int64 [rows]: sum over 64-column groups of scale * sum(x * q)."""
    rows, cols = weight.shape
    x = _act(activation_q12_12, cols)
    y = torch.empty(rows, dtype=torch.int64, device=x.device)
    desc = weight.descriptor()
    check(_lib.load().q4d_linear_q26(ctypes.byref(desc), x.data_ptr(), y.data_ptr(), None, None, current_stream()),
          "q4d_linear_q26")
    return y


def compute_q4_gemv_q12_12(activation_q12_12: torch.Tensor, weight: Q4Tensor) -> tuple[torch.Tensor, torch.Tensor, int]:
    """(Q12.12 int32 [rows], Q26 int64 [rows], saturated row count) in one pass:
    ``q26_to_q12_12(compute_q4_gemv_q26(...))`` fused."""
    rows, cols = weight.shape
    x = _act(activation_q12_12, cols)
    y26 = torch.empty(rows, dtype=torch.int64, device=x.device)
    y12 = torch.empty(rows, dtype=torch.int32, device=x.device)
    sat = torch.zeros(1, dtype=torch.int32, device=x.device)
    desc = weight.descriptor()
    check(_lib.load().q4d_linear_q26(ctypes.byref(desc), x.data_ptr(), y26.data_ptr(), y12.data_ptr(),
                                     sat.data_ptr(), current_stream()), "q4d_linear_q26")
    return y12, y26, int(sat.item())


def q26_to_q12_12(row_sum_q26: torch.Tensor) -> tuple[torch.Tensor, int]:
    """Arithmetic shift right by 14, signed 24-bit saturation: (values, saturated count).

    On a device tensor of Q26 sums this is plain tensor arithmetic (the fused
    form is :func:`compute_q4_gemv_q12_12`)."""
    shifted = row_sum_q26.to(torch.int64) >> SCALE_FRAC
    lo, hi = -(1 << 23), (1 << 23) - 1
    sat = int(((shifted < lo) | (shifted > hi)).sum().item())
    return shifted.clamp(lo, hi), sat


def q4_gemv_from_ints(x_q4_12: torch.Tensor, weight: Q4Tensor) -> torch.Tensor:
    """float32 [rows] = Q26 sum / 2^(12 + 14) (the reference's float view of the
    integer GEMV; its partial / scaled sums stay on the device inside the kernel)."""
    y = compute_q4_gemv_q26(x_q4_12, weight)
    return (y.to(torch.float64) / float(1 << (ACT_FRAC + SCALE_FRAC))).to(torch.float32)


def streamed_argmax_q26(scores_q26: torch.Tensor) -> tuple[int, int]:
    """(row, score) of the highest int64 score, lowest row on ties."""
    s = scores_q26.reshape(-1).contiguous()
    if s.dtype != torch.int64 or not s.is_cuda:
        raise TypeError("device int64 scores expected")
    tok = torch.empty(1, dtype=torch.int32, device=s.device)
    score = torch.empty(1, dtype=torch.int64, device=s.device)
    check(_lib.load().q4d_argmax_q26(s.data_ptr(), s.numel(), tok.data_ptr(), score.data_ptr(), current_stream()),
          "q4d_argmax_q26")
    return int(tok.item()), int(score.item())
