"""numpy restatement of the reference's Qwen3-0.6B Q4 decode path (oracle only).

Test infrastructure: imported by ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg only.  Every function cites the reference
file:line it follows (paths relative to the reference repository root;
``pem/`` abbreviates ``Qwen3-0.6B-Base/python_each_module/``).

Two arithmetic families live here:

* integer (bit-exact): int4 pack/unpack, Q2.14 scale rule, the Q26 Q4 GEMV,
  the Q26 -> Q12.12 conversion and the lowest-index-wins argmax;
* floating point: the FP32 "manual" decode of ``pem/common.py`` with every
  Q4 weight dequantised as ``W = q * scale_q2_14 / 2**14`` (exact in fp32).
  ``dtype`` selects float32 (the reference's own precision) or float64.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

__all__ = [
    "HIDDEN_SIZE", "GROUP_SIZE", "Q4_MIN", "Q4_MAX", "SCALE_FRAC",
    "pack_signed_int4", "unpack_signed_int4", "scale_q2_14_from_float",
    "quantize_weight_q4", "dequantize_q4", "words32_to_packed_bytes",
    "words32_to_scales", "q4_gemv_q26", "q26_to_q12_12", "argmax_first",
    "lm_head_streamed_argmax_q26",
    "manual_rms_norm", "manual_linear_from_weight", "rope_inv_freq",
    "manual_rope_cos_sin", "manual_rotate_half", "manual_apply_rope",
    "manual_repeat_kv", "softmax", "silu", "manual_cached_attention", "manual_causal_attention",
    "OracleConfig", "OracleLayer", "OracleModel", "manual_decoder_layer_cached",
    "embed_tokens", "final_logits", "run_manual_one_token", "greedy_decode",
    "serial_prompt_all_at_once",
    "top2_gap",
]

HIDDEN_SIZE = 1024
GROUP_SIZE = 64
Q4_MIN = -8
Q4_MAX = 7
SCALE_FRAC = 14


# --------------------------------------------------------------------------
# Q4 format (Source/Q4_FORMAT.md:75-140)
# --------------------------------------------------------------------------

def pack_signed_int4(q: np.ndarray) -> np.ndarray:
    """Two signed int4 per byte, even column in the low nibble.

    Follows ``pem/13_export_q4_gemv_vectors.py:67-80`` and
    ``Source/Q4_FORMAT.md:111-128``.
    """
    q = np.asarray(q)
    if q.ndim != 2 or q.shape[1] % 2:
        raise ValueError(f"expected [N, even K] int4 matrix, got {q.shape}")
    q16 = q.astype(np.int16)
    if np.any(q16 < Q4_MIN) or np.any(q16 > Q4_MAX):
        raise ValueError("int4 values must lie in [-8, 7]")
    nib = (q16 & 0xF).astype(np.uint8)
    return (nib[:, 0::2] | (nib[:, 1::2] << 4)).astype(np.uint8)


def _nibble_pair_table() -> np.ndarray:
    """[256, 2] int8: byte b -> (low nibble, high nibble), each n -> n - 16 if n >= 8."""
    b = np.arange(256, dtype=np.int16)
    pair = np.stack([b & 0x0F, (b >> 4) & 0x0F], axis=1)
    pair[pair >= 8] -= 16
    return pair.astype(np.int8)


_NIBBLE_PAIRS = _nibble_pair_table()


def unpack_signed_int4(packed: np.ndarray, k: int) -> np.ndarray:
    """Inverse of :func:`pack_signed_int4`: nibble n -> n - 16 if n >= 8, even
    column from the low nibble.

    Follows ``pem/13_export_q4_gemv_vectors.py:83-98`` (evaluated through a
    256-entry byte table, which holds the same rule for every byte value).
    """
    packed = np.asarray(packed, dtype=np.uint8)
    if k % 2 or packed.shape[-1] != k // 2:
        raise ValueError(f"packed width {packed.shape[-1]} does not hold {k} int4 values")
    return _NIBBLE_PAIRS[packed].reshape(packed.shape[:-1] + (k,))


def scale_q2_14_from_float(raw_scale: np.ndarray, nonzero: np.ndarray | None = None) -> np.ndarray:
    """Q2.14 scale code with round-half-even and the nonzero rule.

    ``scale_q2_14 = rint(raw * 2**14)``; a group whose absmax is nonzero but
    whose code rounds to 0 stores 1 (``pem/13_export_q4_gemv_vectors.py:115-121``).
    ``nonzero`` defaults to ``raw_scale > 0``.
    """
    raw = np.asarray(raw_scale, dtype=np.float32)
    code = np.rint(raw * np.float32(1 << SCALE_FRAC)).astype(np.int64)
    nz = raw > 0 if nonzero is None else np.asarray(nonzero)
    code = np.where(nz & (code == 0), 1, code)
    if np.any(code < 0) or np.any(code > 0xFFFF):
        raise ValueError("Q4 scale does not fit unsigned 16-bit Q2.14")
    return code.astype(np.uint16)


def quantize_weight_q4(weight: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Float -> (packed uint8 [N,K/2], scale uint16 [N,K/64], q int8 [N,K]).

    Follows ``pem/13_export_q4_gemv_vectors.py:101-135`` (absmax/7 scale,
    Q2.14, nonzero rule, ``rint(w / scale)`` clipped to [-8, 7]).
    """
    w = np.ascontiguousarray(np.asarray(weight, dtype=np.float32))
    n, k = w.shape
    if k % GROUP_SIZE:
        raise ValueError("K must be a multiple of 64")
    grouped = w.reshape(n, k // GROUP_SIZE, GROUP_SIZE)
    absmax = np.max(np.abs(grouped), axis=2)
    scale = scale_q2_14_from_float(absmax / np.float32(Q4_MAX), absmax > 0.0)
    used = scale.astype(np.float32) / np.float32(1 << SCALE_FRAC)
    safe = np.where(used > 0.0, used, np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(grouped / safe[:, :, None]), Q4_MIN, Q4_MAX).astype(np.int8)
    q = q.reshape(n, k)
    packed = pack_signed_int4(q)
    return packed, scale, q


def dequantize_q4(packed: np.ndarray, scale: np.ndarray, dtype=np.float32) -> np.ndarray:
    """W[n,k] = q[n,k] * scale_q2_14[n, k//64] / 2**14 (exact in fp32).

    This is the float weight the reference's ``manual_linear_from_weight``
    (``pem/common.py:137-145``) multiplies by once Q4 replaces the FP32
    checkpoint (``Source/Q4_FORMAT.md:83-104``).
    """
    packed = np.asarray(packed, dtype=np.uint8)
    k = packed.shape[-1] * 2
    q = unpack_signed_int4(packed, k)
    s = np.asarray(scale).astype(dtype) / dtype(1 << SCALE_FRAC)
    out = np.empty(q.shape, dtype=dtype)
    np.multiply(q.reshape(q.shape[:-1] + (k // GROUP_SIZE, GROUP_SIZE)), s[..., None],
                out=out.reshape(q.shape[:-1] + (k // GROUP_SIZE, GROUP_SIZE)), dtype=dtype)
    return out


def words32_to_packed_bytes(words: np.ndarray, k: int) -> np.ndarray:
    """Reference ``*_weight_words32.hex`` layout -> packed bytes [N, K/2].

    A words32 value holds eight Q4 values, lowest index in the lowest nibble
    (``pem/35_export_lm_head_full_vocab_vectors.py:80-88``), so its
    little-endian bytes are exactly the packed row bytes of Q4_FORMAT.
    """
    w = np.asarray(words, dtype=np.uint32)
    return w.astype("<u4").view(np.uint8).reshape(-1, k // 2)


def words32_to_scales(words: np.ndarray, groups: int) -> np.ndarray:
    """``*_scale_words32.hex`` (two Q2.14 per word, low half first) -> [N, G].

    Follows ``pem/35_export_lm_head_full_vocab_vectors.py:91-96``.
    """
    w = np.asarray(words, dtype=np.uint32)
    return w.astype("<u4").view(np.uint16).reshape(-1, groups)


# --------------------------------------------------------------------------
# Integer Q4 GEMV (Source/Q4_FORMAT.md:155-190)
# --------------------------------------------------------------------------

def q4_gemv_q26(x_int: np.ndarray, q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """Exact integer Q4 GEMV with a Q26 row accumulator.

    partial[n,g] = sum_j x[64g+j] * q[n,64g+j]; scaled = partial * scale;
    row = sum_g scaled.  Follows ``pem/28_export_mlp_gate_up_vectors.py:124-133``
    (also ``pem/13_export_q4_gemv_vectors.py:138-154``,
    ``pem/35_export_lm_head_full_vocab_vectors.py:120-130``).
    ``x_int`` is Q4.12 or Q12.12 (the result is Q26 either way).
    """
    x = np.asarray(x_int, dtype=np.int64)
    q = np.asarray(q, dtype=np.int64)
    n, k = q.shape
    g = k // GROUP_SIZE
    partial = np.einsum("ngj,gj->ng", q.reshape(n, g, GROUP_SIZE), x.reshape(g, GROUP_SIZE))
    return np.sum(partial * np.asarray(scale, dtype=np.int64), axis=1, dtype=np.int64)


def q26_to_q12_12(row_q26: np.ndarray, width_bits: int = 24) -> tuple[np.ndarray, int]:
    """Arithmetic shift right by 14 then signed saturation to 24 bits.

    Follows ``pem/28_export_mlp_gate_up_vectors.py:136-138`` with
    ``saturate_signed_array`` (``:93-96``).
    """
    shifted = np.asarray(row_q26, dtype=np.int64) >> SCALE_FRAC
    lo, hi = -(1 << (width_bits - 1)), (1 << (width_bits - 1)) - 1
    sat = int(np.count_nonzero((shifted < lo) | (shifted > hi)))
    return np.clip(shifted, lo, hi).astype(np.int64), sat


def argmax_first(scores: np.ndarray) -> tuple[int, float | int]:
    """Running argmax, strict greater-than in ascending index order.

    The lowest index wins ties: ``pem/56_export_persistent_multitoken_layer_golden.py:775-779,860``
    and ``rtl/model/lm_head/lm_head_argmax_row_bram_scheduler.sv:371-375``.
    A strict-greater scan in ascending order keeps the first index that
    attains the maximum, which is what this vectorised form returns;
    ``tests/test_oracle_pins.py`` checks it against a literal scan.
    """
    s = np.asarray(scores).reshape(-1)
    if s.size == 0:
        raise ValueError("empty score vector")
    best_i = int(np.flatnonzero(s == s.max())[0])
    best = s[best_i]
    return best_i, best.item()


def lm_head_streamed_argmax_q26(x_int: np.ndarray, q: np.ndarray, scale: np.ndarray,
                                chunk_rows: int = 1024, row_base: int = 0) -> tuple[int, int, np.ndarray]:
    """Chunked LM-head scan keeping a strict-greater running best.

    Follows ``pem/56_export_persistent_multitoken_layer_golden.py:766-798``:
    per chunk a local first-max, then ``if local > best`` across chunks.
    Returns (token, score_q26, all logits).
    """
    n = q.shape[0]
    logits = np.empty(n, dtype=np.int64)
    best_tok, best = -1, -(1 << 62)
    for start in range(0, n, chunk_rows):
        end = min(start + chunk_rows, n)
        lg = q4_gemv_q26(x_int, q[start:end], scale[start:end])
        logits[start:end] = lg
        li, ls = argmax_first(lg)
        if ls > best:
            best, best_tok = int(ls), row_base + start + li
    return best_tok, best, logits


# --------------------------------------------------------------------------
# Float path: pem/common.py:129-298
# --------------------------------------------------------------------------

def manual_rms_norm(x: np.ndarray, weight: np.ndarray, eps: float, dtype=np.float32) -> np.ndarray:
    """``x * rsqrt(mean(x**2, -1) + eps) * weight`` (``pem/common.py:129-134``)."""
    xf = np.asarray(x, dtype=dtype)
    wf = np.asarray(weight, dtype=dtype)
    ms = np.mean(xf * xf, axis=-1, keepdims=True, dtype=dtype)
    inv = (dtype(1.0) / np.sqrt(ms + dtype(eps))).astype(dtype)
    return (xf * inv * wf).astype(dtype)


def manual_linear_from_weight(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None = None,
                              dtype=np.float32) -> np.ndarray:
    """``y = x @ W.T (+ b)`` (``pem/common.py:137-145``)."""
    y = np.asarray(x, dtype=dtype) @ np.asarray(weight, dtype=dtype).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=dtype)
    return y.astype(dtype)


def rope_inv_freq(theta: float, head_dim: int) -> np.ndarray:
    """Default RoPE inverse frequencies ``1 / theta**(arange(0,d,2)/d)`` in fp32.

    The reference takes ``rotary_emb.inv_freq`` from the HF model
    (``pem/common.py:160``); its default init is this formula with
    ``attention_scaling = 1`` (config.json: rope_scaling null, theta 1e6),
    evaluated by torch on the CPU.  torch's fp32 ``pow`` differs from numpy's
    by an ulp on some entries, so the same torch expression is used here.
    """
    import torch
    base = int(theta) if float(theta).is_integer() else float(theta)
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    return inv.numpy().astype(np.float32)


def manual_rope_cos_sin(inv_freq: np.ndarray, position_ids: np.ndarray,
                        attention_scaling: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin of ``cat(f, f)`` with ``f = pos * inv_freq`` (``pem/common.py:155-170``).

    ``position_ids``: int [B, S]; returns float32 [B, S, head_dim].
    """
    pos = np.asarray(position_ids).astype(np.float32)
    freqs = pos[..., None] * np.asarray(inv_freq, dtype=np.float32)[None, None, :]
    emb = np.concatenate([freqs, freqs], axis=-1).astype(np.float32)
    s = np.float32(attention_scaling)
    return (np.cos(emb) * s).astype(np.float32), (np.sin(emb) * s).astype(np.float32)


def manual_rotate_half(x: np.ndarray) -> np.ndarray:
    """``cat(-x2, x1)`` over the last dim (``pem/common.py:148-152``)."""
    half = x.shape[-1] // 2
    return np.concatenate([-x[..., half:], x[..., :half]], axis=-1)


def manual_apply_rope(q: np.ndarray, k: np.ndarray, cos: np.ndarray, sin: np.ndarray):
    """``x*cos + rotate_half(x)*sin`` with cos/sin broadcast over heads
    (``pem/common.py:173-183``).  q/k: [B, H, S, D]; cos/sin: [B, S, D]."""
    c = cos[:, None, :, :]
    s = sin[:, None, :, :]
    return (q * c + manual_rotate_half(q) * s), (k * c + manual_rotate_half(k) * s)


def manual_repeat_kv(x: np.ndarray, repeat: int) -> np.ndarray:
    """[B, KVH, T, D] -> [B, KVH*repeat, T, D], each kv head repeated in place
    (``pem/common.py:192-198``): q head h reads kv head ``h // repeat``."""
    if repeat == 1:
        return x
    b, h, t, d = x.shape
    return np.broadcast_to(x[:, :, None], (b, h, repeat, t, d)).reshape(b, h * repeat, t, d)


def softmax(x: np.ndarray, axis: int = -1) -> np.ndarray:
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def silu(x: np.ndarray) -> np.ndarray:
    """``x * sigmoid(x)`` (``F.silu`` as used at ``pem/common.py:295``)."""
    one = x.dtype.type(1.0)
    return x / (one + np.exp(-x))


def manual_cached_attention(q: np.ndarray, k_rep: np.ndarray, v_rep: np.ndarray, scaling: float):
    """``softmax(q @ k.T * scaling) @ v`` in the working dtype
    (``pem/common.py:219-228``).  q: [B,H,S,D]; k/v: [B,H,T,D]."""
    dt = q.dtype.type
    scores = (q @ np.swapaxes(k_rep, 2, 3)) * dt(scaling)
    w = softmax(scores.astype(dt), axis=-1).astype(dt)
    return (w @ v_rep).astype(dt), w


def manual_causal_attention(q: np.ndarray, k_rep: np.ndarray, v_rep: np.ndarray, scaling: float):
    """``softmax(q @ k.T * scaling)`` with keys after the query position filled with
    the dtype's most negative finite value, then ``@ v`` (``pem/common.py:201-216``).
    q, k/v: [B, H, S, D] (k/v already repeated); returns ``(output, weights)``."""
    dt = q.dtype.type
    scores = (q @ np.swapaxes(k_rep, 2, 3)) * dt(scaling)
    s = scores.shape[-1]
    future = np.triu(np.ones((s, s), dtype=bool), k=1)
    scores = np.where(future[None, None], np.finfo(dt).min, scores).astype(dt)
    w = softmax(scores, axis=-1).astype(dt)
    return (w @ v_rep).astype(dt), w


# --------------------------------------------------------------------------
# Model container and the cached decoder layer
# --------------------------------------------------------------------------

@dataclass
class OracleConfig:
    """Qwen3-0.6B shapes (``Qwen3-0.6B-Base/config.json:1-30``)."""
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    vocab_size: int = 151936

    @property
    def kv_repeat(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @property
    def scaling(self) -> float:
        return float(self.head_dim) ** -0.5


@dataclass
class OracleLayer:
    """Dequantised weights of one layer (attribute names follow the HF layer
    object that ``pem/common.py:245-296`` reads)."""
    q_proj: np.ndarray
    k_proj: np.ndarray
    v_proj: np.ndarray
    o_proj: np.ndarray
    gate_proj: np.ndarray
    up_proj: np.ndarray
    down_proj: np.ndarray
    input_layernorm: np.ndarray
    post_attention_layernorm: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray


@dataclass
class OracleModel:
    config: OracleConfig
    layers: list[OracleLayer]
    embed_tokens: np.ndarray          # [vocab, hidden] dequantised (tied with lm_head)
    norm: np.ndarray                  # final RMSNorm gamma
    inv_freq: np.ndarray = field(default=None)  # type: ignore[assignment]
    dtype: type = np.float32

    def __post_init__(self):
        if self.inv_freq is None:
            self.inv_freq = rope_inv_freq(self.config.rope_theta, self.config.head_dim)

    @classmethod
    def from_q4(cls, cfg: OracleConfig, layers_q4: Sequence[dict], embed_packed: np.ndarray,
                embed_scale: np.ndarray, final_norm: np.ndarray, dtype=np.float32) -> "OracleModel":
        """Build from Q4 arrays: each layer dict maps ``q_proj`` ... ``down_proj``
        to ``(packed, scale)`` and the four norm names to gamma vectors."""
        mats = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
        norms = ("input_layernorm", "post_attention_layernorm", "q_norm", "k_norm")
        layers = []
        for lq in layers_q4:
            kw = {m: dequantize_q4(*lq[m], dtype=dtype) for m in mats}
            kw.update({nm: np.asarray(lq[nm], dtype=dtype) for nm in norms})
            layers.append(OracleLayer(**kw))
        return cls(cfg, layers, dequantize_q4(embed_packed, embed_scale, dtype=dtype),
                   np.asarray(final_norm, dtype=dtype), dtype=dtype)


def manual_decoder_layer_cached(hidden: np.ndarray, layer: OracleLayer, cfg: OracleConfig,
                                inv_freq: np.ndarray, position_ids: np.ndarray,
                                k_cache: np.ndarray | None, v_cache: np.ndarray | None,
                                kv_store_dtype=None, trace: dict | None = None):
    """One cached decoder layer, ``pem/common.py:231-298``.

    hidden: [B, 1, hidden]; caches: [B, KVH, T, D] or None; returns
    ``(layer_output, k_cache, v_cache)`` with the caches grown by one
    position (``append_cache``, ``pem/common.py:186-189``).
    ``kv_store_dtype=np.float16`` rounds the appended K/V through fp16 to
    mirror an fp16 cache (the reference keeps them in fp32).
    """
    dt = hidden.dtype.type
    b = hidden.shape[0]
    nq, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps = cfg.rms_norm_eps

    residual = hidden
    input_norm = manual_rms_norm(hidden, layer.input_layernorm, eps, dt)
    q_flat = manual_linear_from_weight(input_norm, layer.q_proj, dtype=dt)
    k_flat = manual_linear_from_weight(input_norm, layer.k_proj, dtype=dt)
    v_flat = manual_linear_from_weight(input_norm, layer.v_proj, dtype=dt)

    q_view = q_flat.reshape(b, 1, nq, hd)
    k_view = k_flat.reshape(b, 1, nkv, hd)
    v_view = v_flat.reshape(b, 1, nkv, hd)
    q_norm = manual_rms_norm(q_view, layer.q_norm, eps, dt)
    k_norm = manual_rms_norm(k_view, layer.k_norm, eps, dt)

    q_states = np.swapaxes(q_norm, 1, 2)
    k_states = np.swapaxes(k_norm, 1, 2)
    v_states = np.swapaxes(v_view, 1, 2)

    cos, sin = manual_rope_cos_sin(inv_freq, position_ids)
    cos, sin = cos.astype(dt), sin.astype(dt)
    q_rope, k_rope = manual_apply_rope(q_states, k_states, cos, sin)

    k_new, v_new = k_rope, v_states
    if kv_store_dtype is not None:
        k_new = k_new.astype(kv_store_dtype).astype(dt)
        v_new = v_new.astype(kv_store_dtype).astype(dt)
    k_cache = k_new.copy() if k_cache is None else np.concatenate([k_cache, k_new], axis=2)
    v_cache = v_new.copy() if v_cache is None else np.concatenate([v_cache, v_new], axis=2)

    k_rep = manual_repeat_kv(k_cache, cfg.kv_repeat)
    v_rep = manual_repeat_kv(v_cache, cfg.kv_repeat)
    attn, _w = manual_cached_attention(q_rope.astype(dt), k_rep.astype(dt), v_rep.astype(dt), cfg.scaling)
    attn_concat = np.swapaxes(attn, 1, 2).reshape(b, 1, nq * hd)

    o = manual_linear_from_weight(attn_concat, layer.o_proj, dtype=dt)
    after_attention = (residual + o).astype(dt)
    post_norm = manual_rms_norm(after_attention, layer.post_attention_layernorm, eps, dt)
    gate = manual_linear_from_weight(post_norm, layer.gate_proj, dtype=dt)
    up = manual_linear_from_weight(post_norm, layer.up_proj, dtype=dt)
    mlp_hidden = (silu(gate) * up).astype(dt)
    down = manual_linear_from_weight(mlp_hidden, layer.down_proj, dtype=dt)
    out = (after_attention + down).astype(dt)
    if trace is not None:
        trace.update(input_norm=input_norm, q_flat=q_flat, k_flat=k_flat, v_flat=v_flat,
                     q_rope=q_rope, k_rope=k_rope, v_states=v_states, attn=attn_concat,
                     after_attention=after_attention, post_norm=post_norm, gate=gate, up=up,
                     mlp_hidden=mlp_hidden, out=out)
    return out, k_cache, v_cache


def embed_tokens(model: OracleModel, token_ids: np.ndarray) -> np.ndarray:
    """``embedding_table[token]`` (``pem/10_validate_full_run_one_token.py:31``)
    with the tied Q4 table dequantised; token_ids [B, 1] -> [B, 1, hidden]."""
    ids = np.asarray(token_ids, dtype=np.int64)
    if np.any(ids < 0) or np.any(ids >= model.config.vocab_size):
        raise ValueError("token id outside the vocabulary")
    return model.embed_tokens[ids].astype(model.dtype)


def final_logits(model: OracleModel, hidden: np.ndarray) -> np.ndarray:
    """Final RMSNorm then the tied LM head
    (``pem/10_validate_full_run_one_token.py:52-54``)."""
    dt = model.dtype
    fh = manual_rms_norm(hidden, model.norm, model.config.rms_norm_eps, dt)
    return manual_linear_from_weight(fh, model.embed_tokens, dtype=dt)


def run_manual_one_token(current_token_ids: np.ndarray, position: int | np.ndarray, model: OracleModel,
                         k_caches: list, v_caches: list, kv_store_dtype=None,
                         layer_trace: list | None = None):
    """One full decode step, ``pem/10_validate_full_run_one_token.py:17-56``.

    ``position`` is an int or an int array [B] (batched decode with a
    position per sequence is only meaningful with equal lengths here).
    Returns ``(logits [B,1,vocab], next_token [B,1])``; caches updated in place.
    """
    hidden = embed_tokens(model, current_token_ids)
    b = hidden.shape[0]
    pos = np.broadcast_to(np.asarray(position, dtype=np.int64).reshape(-1, 1), (b, 1))
    for li, layer in enumerate(model.layers):
        hidden, k_caches[li], v_caches[li] = manual_decoder_layer_cached(
            hidden, layer, model.config, model.inv_freq, pos, k_caches[li], v_caches[li],
            kv_store_dtype=kv_store_dtype)
        if layer_trace is not None:
            layer_trace.append(hidden.copy())
    logits = final_logits(model, hidden)
    next_token = np.array([[argmax_first(logits[i, -1])[0]] for i in range(b)], dtype=np.int64)
    return logits, next_token


def serial_prompt_all_at_once(model: OracleModel, token_ids: Sequence[int], kv_store_dtype=None,
                              last_only: bool = False, _future_offset: int = 1):
    """The serial prompt loop (``pem/10_validate_full_run_one_token.py:81-135``:
    ``run_manual_one_token`` at positions 0 .. n-1 on an empty cache) evaluated for
    all n positions at once, for prompts too long for the one-token loop.

    At step i every layer appends token i's K/V row and attends over rows 0..i, and
    those rows hold tokens 0..i's K/V, each computed by the same layer from its own
    hidden state; no row of a later token exists yet.  So per layer, computing every
    token's q/k/v first and masking keys j > i gives the serial loop's numbers up to
    the order of floating-point sums.  Each stage is the one of
    ``manual_decoder_layer_cached`` (``pem/common.py:231-298``) with the batch axis
    used for the n positions.

    Returns ``(logits [n, vocab] of every position (``last_only``: [1, vocab] of the
    last), k_caches, v_caches)``; caches are [1, kv_heads, n, head_dim] per layer, as
    the serial loop leaves them.
    ``_future_offset`` exists for the tests that plant a wrong mask (0: a query misses
    its own key; 2: it sees the next one); the default 1 masks exactly keys j > i.
    """
    cfg = model.config
    dt = model.dtype
    n = len(token_ids)
    nq, nkv, hd, eps = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.rms_norm_eps
    hidden = embed_tokens(model, np.asarray(token_ids, dtype=np.int64).reshape(n, 1))   # [n, 1, H]
    cos, sin = manual_rope_cos_sin(model.inv_freq, np.arange(n).reshape(n, 1))       # [n, 1, D]
    cos, sin = cos.astype(dt), sin.astype(dt)
    future = np.triu(np.ones((n, n), dtype=bool), k=_future_offset)                    # key j > query i
    k_caches, v_caches = [], []
    for layer in model.layers:
        residual = hidden
        xn = manual_rms_norm(hidden, layer.input_layernorm, eps, dt)
        q = manual_linear_from_weight(xn, layer.q_proj, dtype=dt).reshape(n, 1, nq, hd)
        k = manual_linear_from_weight(xn, layer.k_proj, dtype=dt).reshape(n, 1, nkv, hd)
        v = manual_linear_from_weight(xn, layer.v_proj, dtype=dt).reshape(n, 1, nkv, hd)
        qn = np.swapaxes(manual_rms_norm(q, layer.q_norm, eps, dt), 1, 2)              # [n, nq, 1, D]
        kn = np.swapaxes(manual_rms_norm(k, layer.k_norm, eps, dt), 1, 2)
        q_rope, k_rope = manual_apply_rope(qn, kn, cos, sin)
        v_rows = np.swapaxes(v, 1, 2)
        if kv_store_dtype is not None:
            k_rope = k_rope.astype(kv_store_dtype).astype(dt)
            v_rows = v_rows.astype(kv_store_dtype).astype(dt)
        kc = np.swapaxes(k_rope[:, :, 0, :], 0, 1)[None]                                # [1, nkv, n, D]
        vc = np.swapaxes(v_rows[:, :, 0, :], 0, 1)[None]
        k_caches.append(kc)
        v_caches.append(vc)
        k_rep = manual_repeat_kv(kc, cfg.kv_repeat)[0]                                  # [nq, n, D]
        v_rep = manual_repeat_kv(vc, cfg.kv_repeat)[0]
        qh = np.swapaxes(q_rope[:, :, 0, :], 0, 1).astype(dt)                           # [nq, n, D]
        scores = (qh @ np.swapaxes(k_rep, 1, 2)) * dt(cfg.scaling)                      # [nq, n(q), n(k)]
        scores[:, future] = -np.inf
        w = softmax(scores.astype(dt), axis=-1).astype(dt)
        attn = np.swapaxes(w @ v_rep, 0, 1).reshape(n, 1, nq * hd).astype(dt)           # [n, 1, nq*D]
        after_attention = (residual + manual_linear_from_weight(attn, layer.o_proj, dtype=dt)).astype(dt)
        post = manual_rms_norm(after_attention, layer.post_attention_layernorm, eps, dt)
        gate = manual_linear_from_weight(post, layer.gate_proj, dtype=dt)
        up = manual_linear_from_weight(post, layer.up_proj, dtype=dt)
        down = manual_linear_from_weight((silu(gate) * up).astype(dt), layer.down_proj, dtype=dt)
        hidden = (after_attention + down).astype(dt)
    return final_logits(model, hidden[-1:] if last_only else hidden)[:, 0], k_caches, v_caches


def top2_gap(logits_row: np.ndarray) -> float:
    """Gap between the largest and second-largest logit (near-tie measure)."""
    part = np.partition(np.asarray(logits_row, dtype=np.float64), -2)
    return float(part[-1] - part[-2])


def greedy_decode(model: OracleModel, prompt: Sequence[int], max_new_tokens: int,
                  kv_store_dtype=None, forced: Sequence[int] | None = None):
    """Serial prefill one token at a time, then greedy feedback.

    Follows ``pem/10_validate_full_run_one_token.py:81-172`` and
    ``Qwen3-0.6B-Base/pc_testing/02_serial_decode.py:33-59``.  ``forced``
    (teacher forcing) replaces the fed-back token at step i by ``forced[i]``
    so a trajectory can be compared step by step after a near-tie.
    Returns ``(generated ids, per-step top-2 gaps, per-step logits argmax score)``.
    """
    L = model.config.num_hidden_layers
    kc: list = [None] * L
    vc: list = [None] * L
    nxt = None
    pos = 0
    for tok in prompt:
        logits, nxt = run_manual_one_token(np.array([[tok]]), pos, model, kc, vc, kv_store_dtype)
        pos += 1
    gen, gaps, scores = [], [], []
    last_logits = logits
    for i in range(max_new_tokens):
        t = int(nxt[0, 0])
        gen.append(t)
        gaps.append(top2_gap(last_logits[0, -1]))
        scores.append(float(last_logits[0, -1, t]))
        if i == max_new_tokens - 1:
            break
        feed = t if forced is None else int(forced[i])
        last_logits, nxt = run_manual_one_token(np.array([[feed]]), pos, model, kc, vc, kv_store_dtype)
        pos += 1
    return gen, gaps, scores


PINS = {
    "pack_signed_int4/unpack_signed_int4": "Q4_FORMAT.md:120-128 examples; all 256 byte values; "
                                            "reference words32 fixtures round trip",
    "scale_q2_14_from_float": "Q4_FORMAT.md:93-97 rule incl. nonzero rule; hand cases",
    "q4_gemv_q26": "reference fixtures q4_gemv_projection_1024_real, q4_gemv_tile_1024, "
                   "mlp_gate_up_proj_stage_real (gate, up), o_proj_stage_real, "
                   "mlp_down_proj_stage_real, lm_head_argmax_stage_real; dot64 KAT 24751/3019622; "
                   "row KAT -3482169",
    "q26_to_q12_12": "reference *_expected_q12_12 fixtures",
    "argmax_first / lm_head_streamed_argmax_q26": "lm_head_argmax_stage_real best token 264 / score 1365150750; "
                                                  "constructed ties; numpy first-max",
    "dequantize_q4 + manual_linear_from_weight": "fixture expected_q26 / 2**26 is the exact real dot product",
    "manual_rms_norm": "torch.nn.functional.rms_norm; scale invariance; unit RMS",
    "rope_inv_freq / manual_rope_cos_sin / manual_apply_rope": "transformers Qwen3RotaryEmbedding + "
                                                              "apply_rotary_pos_emb; norm preservation; "
                                                              "relative-position invariance",
    "manual_cached_attention": "torch scaled_dot_product_attention with enable_gqa; brute force",
    "manual_causal_attention": "torch scaled_dot_product_attention(is_causal=True, enable_gqa); every query row "
                               "equals manual_cached_attention over keys 0..i; planted off-by-one masks fail",
    "manual_decoder_layer_cached / run_manual_one_token": "transformers Qwen3ForCausalLM (eager, fp32) "
                                                          "loaded with the same dequantised weights",
    "serial_prompt_all_at_once": "the one-token serial loop (run_manual_one_token) on the same prompts, every "
                                 "position's logits and every cache row; planted non-causal / off-by-one masks fail",
}
