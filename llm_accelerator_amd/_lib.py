"""ctypes binding of libq4dec.so (declared in include/q4dec.h).

The library is built in-tree by ``llm_accelerator_amd.build``.  There is no
fallback: if the shared object is missing or a symbol is absent, loading
raises immediately.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_float, c_int32, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libq4dec.so")

Q4D_F16 = 0
Q4D_F32 = 1
Q4D_BF16 = 2
STATUS_BAD_TOKEN = 1
STATUS_BAD_POSITION = 2
STATUS_XCD_MAP = 4
STATUS_SYNC_TIMEOUT = 8
STATUS_NAMES = {STATUS_BAD_TOKEN: "BAD_TOKEN", STATUS_BAD_POSITION: "BAD_POSITION", STATUS_XCD_MAP: "XCD_MAP",
                STATUS_SYNC_TIMEOUT: "SYNC_TIMEOUT"}
DECODE_XCD = 0
DECODE_STAGED = 1

# Status codes (include/q4dec.h); 0..-10 mirror QOT_ERR_* of
# FPGA_Project/software/qmap_one_token_runtime/qmap_one_token_runtime.h:17-29.
ERRORS = {
    -1: "BUSY", -2: "BAD_LAYER", -3: "BAD_TABLE", -4: "BAD_ADDR", -5: "TIMEOUT", -6: "STATUS",
    -7: "NULL", -8: "BAD_TOKEN", -9: "CAPACITY", -10: "CONTEXT", -11: "SHAPE", -12: "LAUNCH",
    -13: "DTYPE",
}


class Q4DecError(RuntimeError):
    """A libq4dec entry point returned a negative status code."""

    def __init__(self, code: int, what: str):
        self.code = code
        name = ERRORS.get(code, "UNKNOWN")
        super().__init__(f"{what} failed: Q4D_ERR_{name} ({code})")


class Q4dMatrix(ctypes.Structure):
    _fields_ = [("w", c_void_p), ("s", c_void_p), ("rows", c_int32), ("cols", c_int32)]


class Q4dLayer(ctypes.Structure):
    _fields_ = [(n, Q4dMatrix) for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                                         "down_proj")] + [
        ("input_layernorm", c_void_p), ("post_attention_layernorm", c_void_p),
        ("q_norm", c_void_p), ("k_norm", c_void_p)]


class Q4dModel(ctypes.Structure):
    _fields_ = [
        ("hidden_size", c_int32), ("intermediate_size", c_int32), ("num_layers", c_int32),
        ("num_q_heads", c_int32), ("num_kv_heads", c_int32), ("head_dim", c_int32),
        ("vocab_size", c_int32), ("max_ctx", c_int32), ("rms_norm_eps", c_float), ("attn_scaling", c_float),
        ("layers", POINTER(Q4dLayer)), ("embed_tokens", Q4dMatrix), ("final_norm", c_void_p),
        ("rope_cos", c_void_p), ("rope_sin", c_void_p),
    ]


class Q4dKVCache(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("num_layers", c_int32), ("batch", c_int32), ("num_kv_heads", c_int32),
                ("max_ctx", c_int32), ("head_dim", c_int32)]


class Q4dFixedLayer(ctypes.Structure):
    _fields_ = [("input_gamma", c_void_p), ("post_gamma", c_void_p), ("q_gamma", c_void_p), ("k_gamma", c_void_p)]


class Q4dFixedModel(ctypes.Structure):
    _fields_ = [("base", POINTER(Q4dModel)), ("layers", POINTER(Q4dFixedLayer)), ("final_gamma", c_void_p),
                ("rope_cos", c_void_p), ("rope_sin", c_void_p), ("score_scale_q0_31", c_int32)]


class Q4dFixedKV(ctypes.Structure):
    _fields_ = [("data", c_void_p), ("num_layers", c_int32), ("num_kv_heads", c_int32), ("max_ctx", c_int32),
                ("head_dim", c_int32)]


class Q4dTokenResult(ctypes.Structure):
    _fields_ = [("status", ctypes.c_uint32), ("token_id", ctypes.c_uint32), ("score", c_float),
                ("reserved", c_int32), ("score_q26", ctypes.c_int64)]


SESSION_RUNNER = ctypes.CFUNCTYPE(c_int32, c_void_p, ctypes.c_uint32, ctypes.c_uint32, POINTER(Q4dTokenResult))


class Q4dSessionOptions(ctypes.Structure):
    _fields_ = [("max_new_tokens", ctypes.c_uint32), ("eos_token_id", ctypes.c_uint32),
                ("im_end_token_id", ctypes.c_uint32), ("stop_on_eos", ctypes.c_uint32),
                ("stop_on_im_end", ctypes.c_uint32)]


class Q4dSessionEvent(ctypes.Structure):
    _fields_ = [("kind", c_int32), ("stop_reason", c_int32), ("input_token_id", ctypes.c_uint32),
                ("input_position", ctypes.c_uint32), ("prompt_tokens_consumed", ctypes.c_uint32),
                ("generated_index", ctypes.c_uint32), ("error_code", c_int32), ("result", Q4dTokenResult)]


class Q4dSession(ctypes.Structure):
    _fields_ = [("start_position", ctypes.c_uint32), ("max_context", ctypes.c_uint32),
                ("vocab_size", ctypes.c_uint32), ("runner", c_void_p), ("runner_context", c_void_p),
                ("prompt", c_void_p), ("prompt_count", ctypes.c_uint32), ("prompt_index", ctypes.c_uint32),
                ("next_position", ctypes.c_uint32), ("pending_token", ctypes.c_uint32),
                ("generated_count", ctypes.c_uint32), ("options", Q4dSessionOptions),
                ("last_result", Q4dTokenResult), ("last_error", c_int32), ("state", c_int32),
                ("stop_reason", c_int32)]


class Q4dGpuRunner(ctypes.Structure):
    _fields_ = [("model", c_void_p), ("kv", c_void_p), ("ws", c_void_p), ("ws_bytes", c_size_t),
                ("stream", c_void_p), ("io", c_void_p)]


# Fixed-point workspace counters (Q4D_FX_* in include/q4dec.h).
FX_COUNT_NAMES = ["status", "input_norm", "qkv", "qk_norm", "rope", "attention", "o_proj", "post_residual",
                  "post_norm", "gate", "up", "silu", "mlp_hidden", "down", "layer_residual", "final_norm"]

_P = c_void_p
_FM = POINTER(Q4dFixedModel)
_FKV = POINTER(Q4dFixedKV)
SIGNATURES = {
    "q4d_version": ([], c_int32),
    "q4d_status_string": ([c_int32], ctypes.c_char_p),
    "q4d_workspace_bytes": ([POINTER(Q4dModel), c_int32], c_size_t),
    "q4d_workspace_init": ([_P, c_size_t, POINTER(Q4dModel), c_int32, _P], c_int32),
    "q4d_set_activation_precision": ([c_int32], c_int32),
    "q4d_set_decode_plan": ([c_int32], c_int32),
    "q4d_decode_plan_active": ([POINTER(Q4dModel), _P], c_int32),
    "q4d_diag_set_xcd_check": ([c_int32], c_int32),
    "q4d_read_status": ([_P, c_size_t, POINTER(Q4dModel), c_int32, POINTER(c_int32), _P], c_int32),
    "q4d_linear": ([POINTER(Q4dMatrix), _P, c_int32, _P, c_int32, c_int32, _P], c_int32),
    "q4d_linear_group": ([POINTER(Q4dMatrix), _P, c_int32, _P, c_int32, c_int32, c_int32, _P], c_int32),
    "q4d_rms_norm": ([_P, _P, c_float, c_int32, c_int32, _P, c_int32, _P], c_int32),
    "q4d_qk_norm_rope": ([_P, _P, _P, c_float, c_int32, c_int32, c_int32, _P, _P, c_int32, _P, _P, _P], c_int32),
    "q4d_kv_append": ([POINTER(Q4dKVCache), c_int32, _P, _P, _P, _P, _P], c_int32),
    "q4d_cached_attention": ([POINTER(Q4dModel), POINTER(Q4dKVCache), c_int32, _P, _P, _P, c_int32, _P,
                              c_size_t, _P], c_int32),
    "q4d_embedding": ([POINTER(Q4dMatrix), _P, c_int32, _P, _P, _P], c_int32),
    "q4d_lm_head_argmax": ([POINTER(Q4dModel), _P, _P, _P, _P, _P, c_size_t, _P], c_int32),
    "q4d_decoder_layer": ([POINTER(Q4dModel), c_int32, _P, _P, POINTER(Q4dKVCache), _P, _P, c_size_t, _P],
                          c_int32),
    "q4d_layer_stage": ([POINTER(Q4dModel), c_int32, c_int32, _P, _P, POINTER(Q4dKVCache), _P, _P, c_size_t, _P],
                        c_int32),
    "q4d_lm_head_argmax_batch": ([POINTER(Q4dModel), _P, c_int32, _P, _P, _P, _P, c_size_t, _P], c_int32),
    "q4d_gemm": ([POINTER(Q4dMatrix), _P, c_int32, _P, c_int32, _P, _P], c_int32),
    "q4d_gemm_splitk": ([POINTER(Q4dMatrix), _P, c_int32, _P, c_int32, _P, _P, c_size_t, c_int32, _P], c_int32),
    "q4d_linear_q26": ([POINTER(Q4dMatrix), _P, _P, _P, _P, _P], c_int32),
    "q4d_argmax_q26": ([_P, c_int32, _P, _P, _P], c_int32),
    "q4d_decode_batch": ([POINTER(Q4dModel), _P, _P, c_int32, POINTER(Q4dKVCache), _P, _P, _P, _P, c_size_t, _P],
                         c_int32),
    "q4d_run_one_token": ([POINTER(Q4dModel), _P, _P, POINTER(Q4dKVCache), _P, _P, _P, _P, c_size_t, _P],
                          c_int32),
    "q4d_run_one_token_feedback": ([POINTER(Q4dModel), _P, _P, POINTER(Q4dKVCache), _P, _P, _P, _P, _P, _P,
                                    c_int32, _P, c_size_t, _P], c_int32),
    "q4d_run_one_token_noalloc": ([POINTER(Q4dModel), _P, _P, POINTER(Q4dKVCache), _P, _P, _P, _P, _P], c_int32),
    "q4d_apply_rope": ([_P, _P, _P, _P, c_int32, c_int32, c_int32, _P], c_int32),
    "q4d_apply_rope_seq": ([_P, _P, _P, _P, c_int32, c_int32, c_int32, c_int32, _P], c_int32),
    "q4d_rotate_half": ([_P, _P, ctypes.c_int64, c_int32, _P], c_int32),
    "q4d_causal_attention_workspace_bytes": ([c_int32, c_int32, c_int32, c_int32], c_size_t),
    "q4d_causal_attention": ([_P, _P, _P, _P, c_int32, c_int32, c_int32, c_int32, c_int32, c_float, _P, c_size_t,
                              _P], c_int32),
    "q4d_diag_launch_chain": ([_P, _P, _P, c_int32, _P, _P], c_int32),
    "q4d_advance": ([_P, _P, _P, _P, _P, _P, _P, c_int32, _P], c_int32),
    "q4d_advance_session": ([_P, _P, _P, _P, _P, _P, _P, c_int32, _P, _P], c_int32),
    "q4d_prefill_workspace_bytes": ([POINTER(Q4dModel), c_int32], c_size_t),
    "q4d_prefill": ([POINTER(Q4dModel), _P, c_int32, c_int32, c_int32, POINTER(Q4dKVCache), _P, _P, _P, _P,
                     c_size_t, _P], c_int32),
    "q4d_fixed_tables": ([_P, c_int32, _P, c_int32], c_int32),
    "q4d_fixed_workspace_bytes": ([_FM], c_size_t),
    "q4d_fixed_workspace_init": ([_P, c_size_t, _FM, _P], c_int32),
    "q4d_fixed_read_counts": ([_P, c_size_t, _P, c_int32, _P], c_int32),
    "q4d_fixed_rms_norm": ([_P, _P, c_int32, c_int32, c_int32, _P, _P, _P], c_int32),
    "q4d_fixed_qk_norm_rope": ([_P, _P, c_int32, c_int32, _P, _P, _P, _P, _P, _P, _P, _P, _P], c_int32),
    "q4d_fixed_attention_workspace_bytes": ([c_int32, c_int32], c_size_t),
    "q4d_fixed_attention": ([_FKV, c_int32, c_int32, c_int32, _P, c_int32, _P, _P, _P, _P, _P, _P, _P, c_size_t, _P],
                            c_int32),
    "q4d_fixed_kv_append": ([_FKV, c_int32, _P, _P, _P, _P], c_int32),
    "q4d_fixed_silu_mul": ([_P, _P, c_int32, _P, _P, _P, _P, _P, _P], c_int32),
    "q4d_fixed_residual_add": ([_P, _P, c_int32, _P, _P], c_int32),
    "q4d_fixed_embedding": ([POINTER(Q4dMatrix), _P, c_int32, _P, _P], c_int32),
    "q4d_fixed_q4_gemv": ([POINTER(Q4dMatrix), _P, _P, _P, _P], c_int32),
    "q4d_quantize_q4": ([_P, c_int32, ctypes.c_int64, c_int32, c_int32, _P, _P, _P, _P], c_int32),
    "q4d_quantize_q4_batch": ([_P, c_int32, ctypes.c_int64, c_int32, c_int32, c_int32, _P, _P, _P, _P], c_int32),
    "q4d_fixed_decoder_layer": ([_FM, c_int32, _P, _P, _FKV, _P, _P, c_size_t, _P], c_int32),
    "q4d_fixed_run_one_token": ([_FM, _P, _P, _FKV, _P, _P, _P, _P, _P, c_size_t, _P], c_int32),
    "q4d_session_default_options": ([POINTER(Q4dSessionOptions)], None),
    "q4d_session_init": ([POINTER(Q4dSession), ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, _P, _P], c_int32),
    "q4d_session_begin": ([POINTER(Q4dSession), _P, ctypes.c_uint32, POINTER(Q4dSessionOptions)], c_int32),
    "q4d_session_step": ([POINTER(Q4dSession), POINTER(Q4dSessionEvent)], c_int32),
    "q4d_session_reset": ([POINTER(Q4dSession)], None),
    "q4d_session_is_terminal": ([POINTER(Q4dSession)], c_int32),
    "q4d_session_state_name": ([c_int32], ctypes.c_char_p),
    "q4d_session_stop_reason_name": ([c_int32], ctypes.c_char_p),
    "q4d_session_gpu_runner": ([_P, ctypes.c_uint32, ctypes.c_uint32, POINTER(Q4dTokenResult)], c_int32),
    "q4d_session_fixed_runner": ([_P, ctypes.c_uint32, ctypes.c_uint32, POINTER(Q4dTokenResult)], c_int32),
}

_lib = None


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load libq4dec.so once; raise if it (or any declared symbol) is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise ImportError(f"{p} is not built; run `python -m llm_accelerator_amd.build` (no CPU fallback exists)")
    lib = ctypes.CDLL(str(p))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is absent
        fn.argtypes = args
        fn.restype = res
    if path is None:
        _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise Q4DecError(rc, what)


def status_names(status: int) -> list[str]:
    """Names of the Q4D_STATUS_* bits set in a device status word."""
    return [n for bit, n in STATUS_NAMES.items() if status & bit] + (["UNKNOWN"] if status & ~0xF else [])


def check_status(status: int, what: str) -> None:
    """Raise Q4DecError(Q4D_ERR_STATUS) if the device status word has any bit set:
    the results of the calls that set it are not valid (q4d_read_status)."""
    if status:
        err = Q4DecError(-6, what)
        err.status = status
        err.args = (f"{what}: device status {status:#x} ({', '.join(status_names(status))}); "
                    "the results are not valid",)
        raise err
