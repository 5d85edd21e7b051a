"""Fixed-point (RTL-exact) decode on the GPU: host mirror of the reference's integer path.

The reference defines the FPGA datapath's arithmetic in Python
(``Qwen3-0.6B-Base/python_each_module/56_export_persistent_multitoken_layer_golden.py``
and the stage exporters it loads).  This module keeps those functions' names,
argument meaning and results, with every computation running in libq4dec's
HIP kernels (``q4d_fixed_*`` in include/q4dec.h) on int32 / int64 GPU tensors:

* ``fixed_rmsnorm_reference`` (17_export_rmsnorm_fixed_vectors.py:108-150) and
  ``fixed_rmsnorm_heads`` / ``fixed_rope_reference`` (22_...:169-212);
* ``attention_score_value`` (56_...:347-381) with ``fixed_softmax_probs`` /
  ``fixed_value_accum`` (46_...:105-137);
* ``silu_mul`` (56_...:547-556, 29_...:86-93), ``residual_add`` (56_...:530-533);
* ``build_exp_lut`` / ``build_sigmoid_lut`` (46_...:88-93, 29_...:77-83);
* :class:`FixedQ4Model` with ``run_fixed_layer`` / ``run_one_token``
  (56_...:468-561, 684-798).

Setup-time conversions (gamma and RoPE-table quantisation, 22_...:72-80 and
54_export_rope_runtime_table.py:48-55) run on the host once per model.
"""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import FX_COUNT_NAMES, Q4dFixedKV, Q4dFixedLayer, Q4dFixedModel, check
from .model import Q4ForCausalLM, Qwen3Config, current_stream

GAMMA_WIDTH, GAMMA_FRAC = 16, 7
TRIG_WIDTH, TRIG_FRAC = 16, 15
SCALE_FRAC = 31
EXP_LUT_SIZE, SIGMOID_LUT_SIZE = 257, 1025


def _i32(x, device="cuda") -> torch.Tensor:
    t = torch.as_tensor(np.asarray(x) if not isinstance(x, torch.Tensor) else x)
    return t.to(device=device, dtype=torch.int32).contiguous()


def _i16(x, device="cuda") -> torch.Tensor:
    return torch.as_tensor(np.asarray(x)).to(device=device, dtype=torch.int16).contiguous()


# ---------------------------------------------------------------- host-side setup
def quantize_signed(values, width_bits: int, frac_bits: int) -> tuple[np.ndarray, int]:
    """``clip(rint(x * 2**frac))`` with the saturation count (22_...:72-80)."""
    scaled = np.rint(np.asarray(values, dtype=np.float64) * float(1 << frac_bits))
    lo, hi = -(1 << (width_bits - 1)), (1 << (width_bits - 1)) - 1
    return np.clip(scaled, lo, hi).astype(np.int64), int(np.count_nonzero((scaled < lo) | (scaled > hi)))


def rope_table_q1_15(cfg: Qwen3Config, max_ctx: int) -> tuple[np.ndarray, np.ndarray]:
    """Q1.15 cos/sin [max_ctx, head_dim]: the fp32 HF rotary values (inv_freq from the
    default init, ``cat(f, f)``, cos/sin in fp32) quantised to 16 bits
    (56_...:943-955, 54_export_rope_runtime_table.py:86-91)."""
    d = cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    pos = torch.arange(max_ctx, dtype=torch.float32)[:, None]
    freqs = pos @ inv[None, :].float()
    emb = torch.cat([freqs, freqs], dim=-1)
    cos = quantize_signed(emb.cos().numpy(), TRIG_WIDTH, TRIG_FRAC)[0]
    sin = quantize_signed(emb.sin().numpy(), TRIG_WIDTH, TRIG_FRAC)[0]
    return cos, sin


def score_scale_q0_31(scaling: float) -> int:
    """``round(scaling * 2**31)`` (56_...:449-451)."""
    return int(round(float(scaling) * float(1 << SCALE_FRAC)))


def _tables() -> tuple[np.ndarray, np.ndarray]:
    lib = _lib.load()
    e = np.zeros(EXP_LUT_SIZE, dtype=np.int32)
    s = np.zeros(SIGMOID_LUT_SIZE, dtype=np.int32)
    check(lib.q4d_fixed_tables(e.ctypes.data, EXP_LUT_SIZE, s.ctypes.data, SIGMOID_LUT_SIZE), "q4d_fixed_tables")
    return e, s


def build_exp_lut() -> np.ndarray:
    """``round(exp(-i/16) * 2**20)``, i = 0..256 (46_...:88-93), as the library builds it."""
    return _tables()[0].astype(np.int64)


def build_sigmoid_lut() -> np.ndarray:
    """``clip(round(sigmoid(-8 + i/64) * 2**16), 0, 65535)``, i = 0..1024 (29_...:77-83)."""
    return _tables()[1].astype(np.int64)


# ---------------------------------------------------------------- stage functions (GPU)
def fixed_rmsnorm_reference(input_q14_10, gamma_q8_7, kind: int = 0) -> dict:
    """Integer RMSNorm of one vector (kind 0: hidden, 17_...:108-150; kind 1: one head,
    22_...:127-166).  Returns the reference's dict: sum_squares, mean_square,
    sqrt_radicand, rms, inv_rms, output_q12_12 (int32 GPU tensor), saturation."""
    lib = _lib.load()
    x = _i32(input_q14_10)
    g = _i16(gamma_q8_7)
    y = torch.empty_like(x)
    st = torch.zeros(6, dtype=torch.int64, device=x.device)
    check(lib.q4d_fixed_rms_norm(x.data_ptr(), g.data_ptr(), 1, x.numel(), kind, y.data_ptr(), st.data_ptr(),
                                 current_stream()), "q4d_fixed_rms_norm")
    s = st.cpu().tolist()
    return {"sum_squares": s[0], "mean_square": s[1], "sqrt_radicand": s[2], "rms": s[3], "inv_rms": s[4],
            "output_q12_12": y, "saturation": s[5] > 0, "saturation_count": s[5]}


def fixed_qk_norm_rope(q_heads, k_heads, q_gamma, k_gamma, cos_q1_15, sin_q1_15):
    """Per-head q/k RMSNorm then RoPE of one position (22_...:169-212); with both gammas
    None the RoPE alone (fixed_rope_reference).  Returns (q_rope, k_rope, q_norm, k_norm)."""
    lib = _lib.load()
    q, k = _i32(q_heads), _i32(k_heads)
    qh, kvh = q.numel() // 128, k.numel() // 128
    qg = _i16(q_gamma) if q_gamma is not None else None
    kg = _i16(k_gamma) if k_gamma is not None else None
    c, s = _i16(cos_q1_15), _i16(sin_q1_15)
    qr, kr, qn, kn = (torch.empty_like(q), torch.empty_like(k), torch.empty_like(q), torch.empty_like(k))
    check(lib.q4d_fixed_qk_norm_rope(q.data_ptr(), k.data_ptr(), qh, kvh, qg.data_ptr() if qg is not None else None,
                                     kg.data_ptr() if kg is not None else None, c.data_ptr(), s.data_ptr(),
                                     qr.data_ptr(), kr.data_ptr(), qn.data_ptr(), kn.data_ptr(), current_stream()),
          "q4d_fixed_qk_norm_rope")
    return qr.view(qh, 128), kr.view(kvh, 128), qn.view(qh, 128), kn.view(kvh, 128)


def fixed_rope_reference(x_q12_12, cos_q1_15, sin_q1_15) -> torch.Tensor:
    """RoPE alone of [heads, 128] Q12.12 (22_...:185-212)."""
    x = _i32(x_q12_12).reshape(-1)
    qr, _, _, _ = fixed_qk_norm_rope(x, x[:128], None, None, cos_q1_15, sin_q1_15)
    return qr


def attention_score_value(q_current, k_cache, v_cache, score_scale: int, exp_lut=None) -> dict:
    """Scores, LUT softmax and value sums of one token (56_...:347-381).
    q_current [16, 128]; k_cache / v_cache [T, 8, 128] (position-major, as the reference
    holds them).  The exp LUT is the library's (``exp_lut`` given for checking only)."""
    lib = _lib.load()
    q = _i32(q_current)
    kc, vc = _i32(k_cache), _i32(v_cache)
    t, kvh, d = kc.shape
    qh = q.numel() // d
    kv = FixedKVCache(1, kvh, t, q.device)
    kv.data[0, 0] = kc.permute(1, 0, 2)
    kv.data[0, 1] = vc.permute(1, 0, 2)
    lut = _i32(build_exp_lut() if exp_lut is None else exp_lut)
    out = torch.empty(qh * d, dtype=torch.int32, device=q.device)
    raw = torch.empty(qh, t, dtype=torch.int64, device=q.device)
    scaled = torch.empty_like(raw)
    idx = torch.empty(qh, t, dtype=torch.int32, device=q.device)
    prob = torch.empty_like(idx)
    desc = kv.descriptor()
    nbytes = int(lib.q4d_fixed_attention_workspace_bytes(qh, t))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=q.device)
    check(lib.q4d_fixed_attention(ctypes.byref(desc), 0, qh, t, q.data_ptr(), int(score_scale), lut.data_ptr(),
                                  out.data_ptr(), raw.data_ptr(), scaled.data_ptr(), idx.data_ptr(), prob.data_ptr(),
                                  ws.data_ptr(), nbytes, current_stream()), "q4d_fixed_attention")
    return {"raw": raw, "scaled": scaled, "probs": prob, "lut_indices": idx, "output": out.view(qh, d)}


def silu_mul(gate_q12_12, up_q12_12) -> dict:
    """Sigmoid-LUT SiLU(gate) * up (56_...:547-556): lut_index, sigmoid, silu_gate, hidden."""
    lib = _lib.load()
    g, u = _i32(gate_q12_12), _i32(up_q12_12)
    lut = _i32(build_sigmoid_lut())
    hidden, idx, sig, silu = (torch.empty_like(g) for _ in range(4))
    check(lib.q4d_fixed_silu_mul(g.data_ptr(), u.data_ptr(), g.numel(), lut.data_ptr(), hidden.data_ptr(),
                                 idx.data_ptr(), sig.data_ptr(), silu.data_ptr(), current_stream()),
          "q4d_fixed_silu_mul")
    return {"lut_index": idx, "sigmoid": sig, "silu_gate": silu, "hidden": hidden}


def projection(activation, weight, input_gamma=None) -> torch.Tensor:
    """Integer Q4 projection of one vector (``projection``, 56_...:300-317, over
    ``compute_matrix_outputs``, 21_export_qmap_qkv_projection_image.py:163-191): Q12.12
    activations (or, with ``input_gamma``, the Q14.10 hidden state through the hidden
    RMSNorm) times the Q4 matrix ``weight`` (a Q4Tensor or its (packed, scale) pair) ->
    Q12.12 rows, int32 on the GPU."""
    from .model import Q4Tensor
    w = weight if isinstance(weight, Q4Tensor) else Q4Tensor.from_numpy(*weight, device="cuda")
    x = _i32(activation, w.device).reshape(-1)
    g = _i16(input_gamma, w.device) if input_gamma is not None else None
    y = torch.empty(w.shape[0], dtype=torch.int32, device=w.device)
    d = w.descriptor()
    check(_lib.load().q4d_fixed_q4_gemv(ctypes.byref(d), x.data_ptr(), g.data_ptr() if g is not None else None,
                                        y.data_ptr(), current_stream()), "q4d_fixed_q4_gemv")
    return y


def residual_add(hidden_q14_10, x_q12_12) -> torch.Tensor:
    """sat24(hidden + (x >> 2)) (56_...:530-533, 558-561)."""
    lib = _lib.load()
    h, x = _i32(hidden_q14_10), _i32(x_q12_12)
    out = torch.empty_like(h)
    check(lib.q4d_fixed_residual_add(h.data_ptr(), x.data_ptr(), h.numel(), out.data_ptr(), current_stream()),
          "q4d_fixed_residual_add")
    return out


# ---------------------------------------------------------------- model, cache, workspace
class FixedKVCache:
    """int32 Q12.12 cache [layers][2 (K,V)][kv_heads][max_ctx][128], the reference's
    physical order (23_export_kv_cache_append_vectors.py:64-84)."""

    def __init__(self, num_layers: int, num_kv_heads: int, max_ctx: int, device="cuda"):
        self.data = torch.zeros((num_layers, 2, num_kv_heads, max_ctx, 128), dtype=torch.int32, device=device)
        self.num_layers, self.num_kv_heads, self.max_ctx = num_layers, num_kv_heads, max_ctx

    def descriptor(self) -> Q4dFixedKV:
        return Q4dFixedKV(self.data.data_ptr(), self.num_layers, self.num_kv_heads, self.max_ctx, 128)


class FixedQ4Model:
    """The integer parameters next to a :class:`Q4ForCausalLM`: the same Q4 matrices,
    Q8.7 gammas quantised from the float ones (``quantize_layer_parameters``,
    56_...:238-291), the Q1.15 RoPE table and the Q0.31 score scale."""

    def __init__(self, model: Q4ForCausalLM, host: dict):
        q = lambda v: quantize_signed(v, GAMMA_WIDTH, GAMMA_FRAC)[0]  # noqa: E731
        gammas = [{"input": q(L["input_layernorm"]), "post": q(L["post_attention_layernorm"]),
                   "q": q(L["q_norm"]), "k": q(L["k_norm"])} for L in host["layers"]]
        cos, sin = rope_table_q1_15(model.config, model.max_ctx)
        self._setup(model, gammas, q(host["norm"]), cos, sin, score_scale_q0_31(model.config.head_dim ** -0.5))

    @classmethod
    def from_parts(cls, model: Q4ForCausalLM, gammas: list, final_gamma, rope_cos, rope_sin,
                   score_scale: int) -> "FixedQ4Model":
        """A model from integer parameters already in device format (a board runtime's):
        per layer ``{"input", "post", "q", "k"}`` Q8.7 gammas, the final Q8.7 gamma,
        Q1.15 cos/sin rows for positions ``0 .. model.max_ctx - 1`` and the Q0.31 score scale."""
        cfg = model.config
        if len(gammas) != cfg.num_hidden_layers:
            raise ValueError(f"{len(gammas)} layers of gammas for a {cfg.num_hidden_layers}-layer model")
        for L in gammas:
            for k, n in (("input", cfg.hidden_size), ("post", cfg.hidden_size), ("q", cfg.head_dim),
                         ("k", cfg.head_dim)):
                if np.asarray(L[k]).shape != (n,):
                    raise ValueError(f"gamma {k} has shape {np.asarray(L[k]).shape}, expected ({n},)")
        if np.asarray(final_gamma).shape != (cfg.hidden_size,):
            raise ValueError("final gamma shape")
        for t in (rope_cos, rope_sin):
            if np.asarray(t).shape != (model.max_ctx, cfg.head_dim):
                raise ValueError(f"RoPE table shape {np.asarray(t).shape}, expected ({model.max_ctx}, {cfg.head_dim})")
        if not 0 < int(score_scale) < 2 ** 31:
            raise ValueError("score scale must be a positive Q0.31 value")
        self = cls.__new__(cls)
        self._setup(model, gammas, final_gamma, rope_cos, rope_sin, int(score_scale))
        return self

    def _setup(self, model, gammas, final_gamma, cos, sin, score_scale):
        cfg, dev = model.config, model.device
        self.model, self.config = model, cfg
        self.gammas = [{k: _i16(L[k], dev) for k in ("input", "post", "q", "k")} for L in gammas]
        self.final_gamma = _i16(final_gamma, dev)
        self.rope_cos, self.rope_sin = _i16(cos, dev), _i16(sin, dev)
        self.score_scale = score_scale
        self._base = model.descriptor()
        self._layers = (Q4dFixedLayer * len(self.gammas))(*[
            Q4dFixedLayer(g["input"].data_ptr(), g["post"].data_ptr(), g["q"].data_ptr(), g["k"].data_ptr())
            for g in self.gammas])
        self._desc = Q4dFixedModel(ctypes.pointer(self._base), self._layers, self.final_gamma.data_ptr(),
                                   self.rope_cos.data_ptr(), self.rope_sin.data_ptr(), self.score_scale)
        lib = _lib.load()
        self.ws_bytes = int(lib.q4d_fixed_workspace_bytes(ctypes.byref(self._desc)))
        if self.ws_bytes == 0:
            raise _lib.Q4DecError(-11, "q4d_fixed_workspace_bytes")
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=dev)
        check(lib.q4d_fixed_workspace_init(self.ws.data_ptr(), self.ws_bytes, ctypes.byref(self._desc),
                                           current_stream()), "q4d_fixed_workspace_init")

    def descriptor(self) -> Q4dFixedModel:
        return self._desc

    def new_cache(self) -> FixedKVCache:
        return FixedKVCache(self._base.num_layers, self.config.num_key_value_heads, self.model.max_ctx,
                            self.model.device)

    def counts(self) -> dict:
        """Saturation counters accumulated since the workspace was initialised."""
        out = np.zeros(len(FX_COUNT_NAMES), dtype=np.int32)
        check(_lib.load().q4d_fixed_read_counts(self.ws.data_ptr(), self.ws_bytes, out.ctypes.data, len(out),
                                                current_stream()), "q4d_fixed_read_counts")
        return dict(zip(FX_COUNT_NAMES, out.tolist()))

    def embed(self, tokens) -> torch.Tensor:
        """Q14.10 embedding rows of the tied Q4 table (56_...:214-221)."""
        t = _i32(tokens, self.model.device).reshape(-1)
        out = torch.empty(t.numel(), self.config.hidden_size, dtype=torch.int32, device=t.device)
        emb = self._base.embed_tokens
        check(_lib.load().q4d_fixed_embedding(ctypes.byref(emb), t.data_ptr(), t.numel(), out.data_ptr(),
                                              current_stream()), "q4d_fixed_embedding")
        return out

    def run_fixed_layer(self, layer: int, hidden_q14_10: torch.Tensor, kv: FixedKVCache, position) -> torch.Tensor:
        """One integer decoder layer at ``position`` (56_...:468-561)."""
        h = _i32(hidden_q14_10, self.model.device).reshape(-1)
        out = torch.empty_like(h)
        pos = position if isinstance(position, torch.Tensor) else torch.tensor([int(position)], dtype=torch.int32,
                                                                                device=h.device)
        kvd = kv.descriptor()
        check(_lib.load().q4d_fixed_decoder_layer(ctypes.byref(self._desc), layer, h.data_ptr(), out.data_ptr(),
                                                  ctypes.byref(kvd), pos.data_ptr(), self.ws.data_ptr(),
                                                  self.ws_bytes, current_stream()), "q4d_fixed_decoder_layer")
        return out

    def run_one_token(self, token, position, kv: FixedKVCache, want_logits: bool = False):
        """Embedding, every layer, final norm and the full-vocabulary scan (56_...:684-798).
        Returns (token, score_q26, logits or None, final hidden Q14.10)."""
        dev = self.model.device
        tok = token if isinstance(token, torch.Tensor) else torch.tensor([int(token)], dtype=torch.int32, device=dev)
        pos = position if isinstance(position, torch.Tensor) else torch.tensor([int(position)], dtype=torch.int32,
                                                                                device=dev)
        nxt = torch.zeros(1, dtype=torch.int32, device=dev)
        score = torch.zeros(1, dtype=torch.int64, device=dev)
        logits = torch.empty(self.config.vocab_size, dtype=torch.int64, device=dev) if want_logits else None
        hidden = torch.empty(self.config.hidden_size, dtype=torch.int32, device=dev)
        kvd = kv.descriptor()
        check(_lib.load().q4d_fixed_run_one_token(ctypes.byref(self._desc), tok.data_ptr(), pos.data_ptr(),
                                                  ctypes.byref(kvd), nxt.data_ptr(), score.data_ptr(),
                                                  logits.data_ptr() if logits is not None else None,
                                                  hidden.data_ptr(), self.ws.data_ptr(), self.ws_bytes,
                                                  current_stream()), "q4d_fixed_run_one_token")
        return nxt, score, logits, hidden
