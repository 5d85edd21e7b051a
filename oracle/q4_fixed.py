"""numpy restatement of the reference's fixed-point (RTL-exact) decode layer (oracle only).

Test infrastructure: imported by ``tests/`` only.  ``pem/`` abbreviates
``Qwen3-0.6B-Base/python_each_module/``; every function cites the reference
file:line it follows.  The composition of a layer is
``pem/56_export_persistent_multitoken_layer_golden.py:468-561`` (``run_fixed_layer``);
each stage is one of the exporter helpers that script loads (``:862-875``).

Formats (``pem/56_...:1087-1095``): hidden states and layer outputs are signed
24-bit Q14.10, everything between the norms and the residuals signed 24-bit
Q12.12, RoPE tables signed Q1.15, attention scores signed 64-bit Q24.24,
softmax probabilities unsigned Q0.16, LM-head scores Q26.  Shifts are
arithmetic (floor), saturation is to the signed width.

Arithmetic width: products that can exceed 64 bits (the Q0.31 score scale) are
taken in Python integers; everything else stays inside int64 by the input
ranges stated beside each function.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from .q4_oracle import q4_gemv_q26, q26_to_q12_12, unpack_signed_int4

__all__ = [
    "saturate", "quantize_signed", "fixed_rmsnorm", "fixed_rmsnorm_hidden", "fixed_rmsnorm_head",
    "fixed_rmsnorm_heads", "fixed_rope", "rope_table_q1_15", "score_scale_q0_31",
    "attention_scores", "build_exp_lut", "score_diff_to_lut_index", "fixed_softmax_probs",
    "fixed_value_accum", "attention_score_value", "build_sigmoid_lut", "gate_to_lut_index",
    "silu_mul", "residual_add", "embed_q14_10", "kv_addr", "FixedLayer", "FixedModel",
    "fixed_decoder_layer", "fixed_final_tail", "fixed_run_one_token", "PINS_FIXED",
]

NUM_Q_HEADS = 16
NUM_KV_HEADS = 8
HEAD_DIM = 128
KV_REPEAT = NUM_Q_HEADS // NUM_KV_HEADS

EXP_FRAC = 20            # pem/46_...:31
EXP_LUT_STEP_FRAC = 4    # pem/46_...:32
EXP_LUT_SIZE = (16 << EXP_LUT_STEP_FRAC) + 1
SCORE_FRAC = 24
SCALE_FRAC = 31
PROB_FRAC = 16
SIGMOID_FRAC = 16        # pem/29_...:30-35
SIGMOID_INDEX_FRAC = 6
SIGMOID_MIN, SIGMOID_MAX = -8.0, 8.0
SIGMOID_LUT_SIZE = int((SIGMOID_MAX - SIGMOID_MIN) * (1 << SIGMOID_INDEX_FRAC)) + 1


def saturate(values, width_bits: int = 24) -> tuple[np.ndarray, int]:
    """Clip to the signed width; also the number of clipped elements
    (``saturate_signed_array``, ``pem/27_...:95-98``)."""
    v = np.asarray(values, dtype=np.int64)
    lo, hi = -(1 << (width_bits - 1)), (1 << (width_bits - 1)) - 1
    return np.clip(v, lo, hi), int(np.count_nonzero((v < lo) | (v > hi)))


def quantize_signed(values, width_bits: int, frac_bits: int) -> tuple[np.ndarray, int]:
    """``clip(rint(x * 2**frac))`` in float64, with the saturation count
    (``pem/22_...:72-80``; gammas Q8.7, RoPE Q1.15)."""
    scaled = np.rint(np.asarray(values, dtype=np.float64) * float(1 << frac_bits))
    lo, hi = -(1 << (width_bits - 1)), (1 << (width_bits - 1)) - 1
    return np.clip(scaled, lo, hi).astype(np.int64), int(np.count_nonzero((scaled < lo) | (scaled > hi)))


def fixed_rmsnorm(x, gamma, *, mean_shift: int, eps: int, num_shift: int, out_shift: int) -> dict:
    """Integer RMSNorm of one vector.

    sum_squares = sum x^2; mean = sum_squares >> mean_shift; rms = isqrt(mean + eps);
    inv = min(2**num_shift // rms, 2**24 - 1) (2**24 - 1 when rms is 0);
    y = sat24((x * inv * gamma) >> out_shift).
    Follows ``pem/17_...:108-150`` (hidden, Q14.10 in) and ``pem/22_...:127-166``
    (per head, Q12.12 in).  |x| <= 2**23, inv < 2**24, |gamma| <= 2**15 keep the
    product inside int64.
    """
    xv = np.asarray(x, dtype=np.int64)
    g = np.asarray(gamma, dtype=np.int64)
    sum_squares = int(np.sum(xv * xv, dtype=np.int64))
    mean_square = sum_squares >> mean_shift
    radicand = mean_square + eps
    rms = math.isqrt(radicand)
    inv = (1 << 24) - 1 if rms == 0 else min((1 << num_shift) // rms, (1 << 24) - 1)
    out, sat = saturate((xv * inv * g) >> out_shift, 24)
    return {"sum_squares": sum_squares, "mean_square": mean_square, "sqrt_radicand": radicand,
            "rms": rms, "inv_rms": inv, "output": out, "saturation": sat}


def fixed_rmsnorm_hidden(x_q14_10, gamma_q8_7) -> dict:
    """Input / post-attention / final RMSNorm over the 1024-wide hidden state:
    Q14.10 in, Q12.12 out, mean shift 10, eps 1 (Q20), numerator 2**26,
    output shift 21 (``pem/17_...:31-47``, ``pem/27_...:34-49``, ``pem/32_...:31-47``)."""
    return fixed_rmsnorm(x_q14_10, gamma_q8_7, mean_shift=10, eps=1, num_shift=26, out_shift=21)


def fixed_rmsnorm_head(x_q12_12, gamma_q8_7) -> dict:
    """q_norm / k_norm over one 128-wide head: Q12.12 in and out, mean shift
    log2(128) = 7, eps 17 (Q24), numerator 2**28, output shift 23
    (``pem/22_...:41-57,127-166``)."""
    return fixed_rmsnorm(x_q12_12, gamma_q8_7, mean_shift=7, eps=17, num_shift=28, out_shift=23)


def fixed_rmsnorm_heads(x_heads, gamma_q8_7) -> tuple[np.ndarray, int]:
    """``fixed_rmsnorm_heads`` (``pem/22_...:169-182``): each head on its own."""
    xh = np.asarray(x_heads, dtype=np.int64)
    out = np.empty_like(xh)
    sat = 0
    for h in range(xh.shape[0]):
        r = fixed_rmsnorm_head(xh[h], gamma_q8_7)
        out[h] = r["output"]
        sat += r["saturation"]
    return out, sat


def fixed_rope(x_heads, cos_q1_15, sin_q1_15) -> tuple[np.ndarray, int]:
    """y[d] = sat24((x[d] * cos[d] + rot[d] * sin[d]) >> 15) with
    rot = (-x[d + 64] for d < 64, x[d - 64] otherwise)
    (``fixed_rope_reference``, ``pem/22_...:185-212``)."""
    x = np.asarray(x_heads, dtype=np.int64)
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    acc = x * np.asarray(cos_q1_15, dtype=np.int64) + rot * np.asarray(sin_q1_15, dtype=np.int64)
    return saturate(acc >> 15, 24)


def rope_table_q1_15(inv_freq, positions) -> tuple[np.ndarray, np.ndarray]:
    """Q1.15 cos/sin rows for the given positions: the float32 HF rotary
    cos/sin quantised by ``quantize_signed(., 16, 15)``
    (``pem/56_...:943-955``, ``pem/54_export_rope_runtime_table.py:48-55,86-91``).
    cos = 1.0 saturates to 32767.  The reference evaluates cos/sin with torch on
    the CPU (``manual_rope_cos_sin``, ``pem/common.py:155-170``); numpy's float32
    cos/sin differ from torch's by an ulp on ~0.03 % of entries, which moves a
    few Q1.15 codes, so the same torch calls are made here."""
    import torch
    pos = torch.as_tensor(np.asarray(positions, dtype=np.int64)).float()[:, None]
    freqs = pos @ torch.as_tensor(np.asarray(inv_freq, dtype=np.float32))[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return quantize_signed(emb.cos().numpy(), 16, 15)[0], quantize_signed(emb.sin().numpy(), 16, 15)[0]


def score_scale_q0_31(scaling: float) -> int:
    """``round(scaling * 2**31)`` (``pem/56_...:449-451``)."""
    return int(round(float(scaling) * float(1 << SCALE_FRAC)))


def attention_scores(q_heads, k_cache, scale_q0_31: int) -> tuple[np.ndarray, np.ndarray]:
    """raw[h, p] = sum_d q[h, d] * k[p, h // 2, d] (Q24.24);
    scaled = (raw * scale) >> 31 in unbounded integers
    (``pem/56_...:347-368``).  q: [16, 128]; k_cache: [T, 8, 128]."""
    q = np.asarray(q_heads, dtype=np.int64)
    k = np.asarray(k_cache, dtype=np.int64)
    kv_of_q = np.arange(q.shape[0]) // KV_REPEAT
    raw = np.einsum("hd,phd->hp", q, k[:, kv_of_q, :])
    scaled = np.array([(int(r) * int(scale_q0_31)) >> SCALE_FRAC for r in raw.reshape(-1)],
                      dtype=np.int64).reshape(raw.shape)
    return raw, scaled


def build_exp_lut() -> np.ndarray:
    """``round(exp(-i / 16) * 2**20)``, i = 0..256 (``pem/46_...:88-93``)."""
    return np.array([int(round(math.exp(-float(i) / float(1 << EXP_LUT_STEP_FRAC)) * float(1 << EXP_FRAC)))
                     for i in range(EXP_LUT_SIZE)], dtype=np.int64)


def score_diff_to_lut_index(max_score: int, score: int) -> int:
    """min((max - s + 2**19) >> 20, 256), 0 when s >= max (``pem/46_...:96-102``)."""
    neg = int(max_score) - int(score)
    if neg <= 0:
        return 0
    shift = SCORE_FRAC - EXP_LUT_STEP_FRAC
    return int(min((neg + (1 << (shift - 1))) >> shift, EXP_LUT_SIZE - 1))


def fixed_softmax_probs(scores, exp_lut) -> tuple[np.ndarray, np.ndarray]:
    """Per row: LUT index from the distance to the row max, e = lut[index],
    p = (e << 16) // sum(e) (``pem/46_...:105-121``)."""
    s = np.asarray(scores, dtype=np.int64)
    lut = np.asarray(exp_lut, dtype=np.int64)
    probs = np.zeros_like(s)
    idx = np.zeros_like(s)
    for h in range(s.shape[0]):
        m = int(np.max(s[h]))
        idx[h] = [score_diff_to_lut_index(m, int(v)) for v in s[h]]
        e = lut[idx[h]]
        total = int(np.sum(e))
        if total <= 0:
            raise RuntimeError("softmax exp_sum underflowed to zero")
        probs[h] = (e << PROB_FRAC) // total
    return probs, idx


def fixed_value_accum(probs_q0_16, v_cache) -> tuple[np.ndarray, int]:
    """out[h, d] = sat24((sum_p p[h, p] * v[p, h // 2, d]) >> 16)
    (``pem/46_...:124-137``); sum_p p <= 2**16 bounds the sum by 2**39."""
    p = np.asarray(probs_q0_16, dtype=np.int64)
    v = np.asarray(v_cache, dtype=np.int64)
    kv_of_q = np.arange(p.shape[0]) // KV_REPEAT
    acc = np.einsum("hp,phd->hd", p, v[:, kv_of_q, :])
    return saturate(acc >> PROB_FRAC, 24)


def attention_score_value(q_heads, k_cache, v_cache, scale_q0_31: int, exp_lut) -> dict:
    """Scores, softmax and value accumulation of one token
    (``attention_score_value``, ``pem/56_...:347-381``)."""
    raw, scaled = attention_scores(q_heads, k_cache, scale_q0_31)
    probs, idx = fixed_softmax_probs(scaled, exp_lut)
    out, sat = fixed_value_accum(probs, v_cache)
    return {"raw": raw, "scaled": scaled, "probs": probs, "lut_indices": idx, "output": out, "saturation": sat}


def build_sigmoid_lut() -> np.ndarray:
    """``clip(round(sigmoid(-8 + i/64) * 2**16), 0, 65535)``, i = 0..1024
    (``pem/29_...:77-83``)."""
    vals = []
    for i in range(SIGMOID_LUT_SIZE):
        x = SIGMOID_MIN + float(i) / float(1 << SIGMOID_INDEX_FRAC)
        y = 1.0 / (1.0 + math.exp(-x))
        vals.append(int(np.clip(round(y * float(1 << SIGMOID_FRAC)), 0, (1 << 16) - 1)))
    return np.array(vals, dtype=np.int64)


def gate_to_lut_index(gate_q12_12) -> np.ndarray:
    """Round-to-nearest index of the gate on the 1/64 grid over [-8, 8]:
    (clip(g, -32768, 32768) + 32768 + 32) >> 6, clipped to 0..1024
    (``pem/29_...:86-93``)."""
    min_q, max_q = int(round(SIGMOID_MIN * 4096)), int(round(SIGMOID_MAX * 4096))
    shift = 12 - SIGMOID_INDEX_FRAC
    c = np.clip(np.asarray(gate_q12_12, dtype=np.int64), min_q, max_q)
    return np.clip((c - min_q + (1 << (shift - 1))) >> shift, 0, SIGMOID_LUT_SIZE - 1)


def silu_mul(gate_q12_12, up_q12_12, sigmoid_lut) -> dict:
    """silu = sat24((gate * lut[index]) >> 16); hidden = sat24((silu * up) >> 12)
    (``pem/56_...:547-556``)."""
    g = np.asarray(gate_q12_12, dtype=np.int64)
    idx = gate_to_lut_index(g)
    sig = np.asarray(sigmoid_lut, dtype=np.int64)[idx]
    silu, sat0 = saturate((g * sig) >> SIGMOID_FRAC, 24)
    hidden, sat1 = saturate((silu * np.asarray(up_q12_12, dtype=np.int64)) >> 12, 24)
    return {"lut_index": idx, "sigmoid": sig, "silu_gate": silu, "hidden": hidden,
            "silu_saturation": sat0, "hidden_saturation": sat1}


def residual_add(hidden_q14_10, x_q12_12) -> tuple[np.ndarray, int]:
    """sat24(hidden + (x >> 2)): Q12.12 branch output onto the Q14.10 stream
    (``pem/56_...:530-533`` after o_proj, ``:558-561`` after down_proj)."""
    return saturate(np.asarray(hidden_q14_10, dtype=np.int64) + (np.asarray(x_q12_12, dtype=np.int64) >> 2), 24)


def embed_q14_10(packed_row, scale_row) -> np.ndarray:
    """Tied Q4 embedding row as Q14.10: (q * scale) >> 4 (``pem/56_...:214-221``,
    ``pem/49_export_q4_embedding_vectors.py:20-22``)."""
    packed_row = np.asarray(packed_row).reshape(1, -1)
    k = packed_row.shape[1] * 2
    q = unpack_signed_int4(packed_row, k).astype(np.int64)[0]
    s = np.repeat(np.asarray(scale_row, dtype=np.int64).reshape(-1), 64)
    return (q * s) >> 4


def kv_addr(base: int, layer: int, kind: int, head: int, position: int, dim: int, max_context: int = 256) -> int:
    """Byte address of a word32 K/V element, layout [layer][K/V][kv_head][position][dim]
    (``pem/23_export_kv_cache_append_vectors.py:64-84``)."""
    pos_stride = HEAD_DIM * 4
    head_stride = max_context * pos_stride
    kind_stride = NUM_KV_HEADS * head_stride
    return base + layer * 2 * kind_stride + kind * kind_stride + head * head_stride + position * pos_stride + dim * 4


@dataclass
class FixedLayer:
    """One layer's integer parameters: the Q4 matrices (packed, Q2.14 scales) and
    the Q8.7 gammas (``quantize_layer_parameters``, ``pem/56_...:238-291``)."""
    q_proj: tuple
    k_proj: tuple
    v_proj: tuple
    o_proj: tuple
    gate_proj: tuple
    up_proj: tuple
    down_proj: tuple
    input_gamma: np.ndarray
    post_gamma: np.ndarray
    q_gamma: np.ndarray
    k_gamma: np.ndarray


@dataclass
class FixedModel:
    layers: list
    embed: tuple              # tied (packed [vocab, 512], scale [vocab, 16])
    final_gamma: np.ndarray   # Q8.7
    rope_cos: np.ndarray      # [max_ctx, 128] Q1.15
    rope_sin: np.ndarray
    score_scale: int          # Q0.31
    exp_lut: np.ndarray = None    # type: ignore[assignment]
    sigmoid_lut: np.ndarray = None  # type: ignore[assignment]

    def __post_init__(self):
        if self.exp_lut is None:
            self.exp_lut = build_exp_lut()
        if self.sigmoid_lut is None:
            self.sigmoid_lut = build_sigmoid_lut()


def _proj(x, mat) -> np.ndarray:
    packed, scale = mat
    q = unpack_signed_int4(packed, packed.shape[1] * 2)
    return q26_to_q12_12(q4_gemv_q26(x, q, scale))[0]


def fixed_decoder_layer(hidden_q14_10, layer: FixedLayer, model: FixedModel, k_cache, v_cache,
                        position: int) -> tuple[np.ndarray, dict]:
    """One integer decoder layer at ``position`` (``run_fixed_layer``,
    ``pem/56_...:468-561``).  ``k_cache`` / ``v_cache``: int64 [max_ctx, 8, 128],
    row ``position`` is written here; positions 0..position are attended."""
    h = np.asarray(hidden_q14_10, dtype=np.int64)
    t: dict = {}
    t["input_norm"] = fixed_rmsnorm_hidden(h, layer.input_gamma)["output"]
    t["q"] = _proj(t["input_norm"], layer.q_proj)
    t["k"] = _proj(t["input_norm"], layer.k_proj)
    t["v"] = _proj(t["input_norm"], layer.v_proj)
    qn, _ = fixed_rmsnorm_heads(t["q"].reshape(NUM_Q_HEADS, HEAD_DIM), layer.q_gamma)
    kn, _ = fixed_rmsnorm_heads(t["k"].reshape(NUM_KV_HEADS, HEAD_DIM), layer.k_gamma)
    t["q_rope"], _ = fixed_rope(qn, model.rope_cos[position], model.rope_sin[position])
    t["k_rope"], _ = fixed_rope(kn, model.rope_cos[position], model.rope_sin[position])
    k_cache[position] = t["k_rope"]
    v_cache[position] = t["v"].reshape(NUM_KV_HEADS, HEAD_DIM)
    att = attention_score_value(t["q_rope"], k_cache[:position + 1], v_cache[:position + 1],
                                model.score_scale, model.exp_lut)
    t["attention"] = att
    t["attn_out"] = att["output"].reshape(-1)
    t["o"] = _proj(t["attn_out"], layer.o_proj)
    t["post_hidden"], _ = residual_add(h, t["o"])
    t["post_norm"] = fixed_rmsnorm_hidden(t["post_hidden"], layer.post_gamma)["output"]
    t["gate"] = _proj(t["post_norm"], layer.gate_proj)
    t["up"] = _proj(t["post_norm"], layer.up_proj)
    t["mlp_hidden"] = silu_mul(t["gate"], t["up"], model.sigmoid_lut)["hidden"]
    t["down"] = _proj(t["mlp_hidden"], layer.down_proj)
    out, _ = residual_add(t["post_hidden"], t["down"])
    return out, t


def fixed_final_tail(hidden_q14_10, model: FixedModel) -> tuple[int, int, np.ndarray, np.ndarray]:
    """Final RMSNorm and the full-vocabulary tied-Q4 LM-head scan with the
    lowest-index-wins argmax (``run_final_tail``, ``pem/56_...:684-798``).
    Returns (token, score_q26, logits_q26, final_norm_q12_12)."""
    norm = fixed_rmsnorm_hidden(hidden_q14_10, model.final_gamma)["output"]
    packed, scale = model.embed
    q = unpack_signed_int4(packed, packed.shape[1] * 2)
    logits = q4_gemv_q26(norm, q, scale)
    tok = int(np.flatnonzero(logits == logits.max())[0])
    return tok, int(logits[tok]), logits, norm


def fixed_run_one_token(token: int, position: int, model: FixedModel, k_caches, v_caches):
    """Embedding, every layer, final tail for one token (``pem/56_...:1004-1044``).
    ``k_caches[l]`` / ``v_caches[l]``: int64 [max_ctx, 8, 128].  Returns
    (token, score, logits, final hidden)."""
    packed, scale = model.embed
    h = embed_q14_10(packed[token], scale[token])
    for li, layer in enumerate(model.layers):
        h, _ = fixed_decoder_layer(h, layer, model, k_caches[li], v_caches[li], position)
    tok, score, logits, _ = fixed_final_tail(h, model)
    return tok, score, logits, h


PINS_FIXED = {
    "fixed_rmsnorm_hidden": "rmsnorm_1024_real, layer1/2_chained_input_rmsnorm_stage_real, "
                            "final_rmsnorm_stage_real, final_rmsnorm_layer2_chained_stage_real "
                            "(sum_squares, mean, radicand, rms, inv_rms, outputs); math.isqrt brute force",
    "fixed_rmsnorm_head / fixed_rope": "qk_norm_rope_stage_128_real + layer1/2 chained (q/k norm and "
                                       "rope outputs); rope_qk_layer_128_real",
    "rope_table_q1_15": "cos/sin of position 4 in the qk_norm_rope fixtures (incl. the 66 saturated 1.0s)",
    "attention_scores / softmax / value": "attention_score_stage_real + softmax_value_stage_real for "
                                          "layer 0, layer 1, layer 1/2 chained (raw, scaled, LUT index, "
                                          "prob, out); exp LUT fixture; score scale 189812531",
    "silu_mul / build_sigmoid_lut / gate_to_lut_index": "mlp_silu_mul_stage_real + layer1/2 chained",
    "residual_add": "post_attention_residual_norm_stage_real (residual), mlp_residual_add_stage_real "
                    "+ chained",
    "kv_addr": "kv_cache_append_real expected addresses (2048 writes)",
    "embed_q14_10": "closed form: equals the Q4 GEMV of a one-hot Q12.12 activation >> 4",
    "fixed_decoder_layer": "stage fixtures chained: each stage's expected output is the next "
                           "fixture's input; composition restates pem/56_...:468-561",
}
