"""Float -> Q4 conversion, host side (CPU): the oracle's quantizer pinned on the
reference's own Q4 matrices, planted mistakes, C-ABI validation and checkpoint checks.

Pins for the quantizer rule (13_export_q4_gemv_vectors.py:101-135):
- fixed points: every 64-column group of the reference's real Q4 matrices (gate, up,
  o, down, q_proj rows, LM-head window) whose codes reach +-7 without -8 was produced
  by this rule from some float group, and its exact dequantisation must quantise back
  to the same codes and scale (absmax = 7 s exactly, s = code / 2^14, 7 s / 7 = s);
- constructed ties: groups whose w / s or absmax / 7 * 2^14 land exactly on k + 1/2
  (exactly representable), where half-even rounding, the fp32 quotient and the clip
  at -8 / 7 decide the codes; written out by hand below;
- planted mistakes (multiplying by 1/s, rounding half away from zero, no nonzero
  rule) each fail one of these checks.
"""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle as o
from llm_accelerator_amd import _lib
from llm_accelerator_amd.model import Qwen3Config
from llm_accelerator_amd.quantize import check_checkpoint, checkpoint_files, expected_tensors, quantize_weight_q4

FAKE = 0x7F0000000000  # aligned, never dereferenced: validation fails before launch
REAL = ["mlp_gate_proj_real", "mlp_up_proj_real", "o_proj_real", "mlp_down_proj_real",
        "q4_gemv_projection_1024_real", "lm_head_argmax_real"]


def fixed_point_groups(golden, name):
    d = golden(name)
    k = d["weight_packed"].shape[1] * 2
    q = o.unpack_signed_int4(d["weight_packed"], k).astype(np.int64).reshape(-1, k // 64, 64)
    s = d["scale_q2_14"].astype(np.int64)
    keep = (np.abs(q).max(-1) == 7) & (q.min(-1) > -8)
    return q[keep], s[keep]


@pytest.mark.parametrize("name", REAL)
def test_reference_q4_groups_are_fixed_points(golden, name):
    q, s = fixed_point_groups(golden, name)
    assert len(q) > 0.9 * golden(name)["scale_q2_14"].size   # nearly every group qualifies
    w = (q * s[:, None]).astype(np.float32) / np.float32(16384)   # exact dequantisation
    packed, scale, codes = o.quantize_weight_q4(w)
    np.testing.assert_array_equal(scale[:, 0], s)
    np.testing.assert_array_equal(codes, q)


def tie_cases():
    """(w [rows, 64] fp32, expected codes, expected scale) built from exact binary values."""
    rows, want_q, want_s = [], [], []
    # 1. w / s = k + 1/2 for every k in -7..6, code 1000 (absmax 7 s sets it exactly)
    s = 1000 / 16384
    ks = np.arange(-7, 7)
    vals = np.concatenate([[7 * s], (ks + 0.5) * s, np.zeros(64 - 1 - len(ks))]).astype(np.float32)
    rows.append(vals)
    half_even = np.rint(ks + 0.5)  # -6, -6, -4, -4, ... 6 (half-even)
    want_q.append(np.concatenate([[7], np.clip(half_even, -8, 7), np.zeros(64 - 1 - len(ks))]))
    want_s.append(1000)
    # 2. absmax / 7 * 2^14 = n + 1/2: n = 2 rounds to 2, n = 3 to 4; small codes clip at -8 / 7
    for n, code in ((2, 2), (3, 4)):
        a = 7 * (n + 0.5) / 16384
        vals = np.zeros(64, np.float32)
        vals[0], vals[1], vals[2] = a, -a, a / 2
        rows.append(vals)
        r = a / (code / 16384)
        want_q.append(np.concatenate([[min(np.rint(r), 7), max(-np.rint(r), -8), np.rint(r / 2)], np.zeros(61)]))
        want_s.append(code)
    # 3. a nonzero group whose code rounds to 0 stores 1 (nonzero rule); an all-zero group 0
    vals = np.zeros(64, np.float32)
    vals[5] = 1e-6
    rows.append(vals)
    want_q.append(np.zeros(64))
    want_s.append(1)
    rows.append(np.zeros(64, np.float32))
    want_q.append(np.zeros(64))
    want_s.append(0)
    return np.stack(rows), np.stack(want_q).astype(np.int8), np.array(want_s, np.uint16)


def test_ties_by_hand():
    w, want_q, want_s = tie_cases()
    assert want_q[0].tolist()[:15] == [7, -6, -6, -4, -4, -2, -2, 0, 0, 2, 2, 4, 4, 6, 6]
    assert want_q[1].tolist()[:3] == [7, -8, 4] and want_q[2].tolist()[:3] == [6, -6, 3]
    _, scale, q = o.quantize_weight_q4(w)
    np.testing.assert_array_equal(scale[:, 0], want_s)
    np.testing.assert_array_equal(q, want_q)


def _mistaken(w, mistake):
    g = w.reshape(w.shape[0], -1, 64).astype(np.float32)
    absmax = np.abs(g).max(-1)
    code = np.rint(absmax / np.float32(7) * np.float32(16384)).astype(np.int64)
    if mistake == "half_away":
        code = np.floor(absmax / np.float32(7) * np.float32(16384) + 0.5).astype(np.int64)
    if mistake != "no_nonzero_rule":
        code = np.where((absmax > 0) & (code == 0), 1, code)
    s = (code.astype(np.float32) / np.float32(16384))
    safe = np.where(s > 0, s, np.float32(1))
    if mistake == "reciprocal":
        r = g * (np.float32(1) / safe[..., None])
    else:
        r = g / safe[..., None]
    if mistake == "half_away":
        q = np.sign(r) * np.floor(np.abs(r) + 0.5)
    else:
        q = np.rint(r)
    return np.clip(q, -8, 7).astype(np.int8).reshape(w.shape), code.astype(np.uint16)


@pytest.mark.parametrize("mistake", ["reciprocal", "half_away", "no_nonzero_rule"])
def test_planted_mistakes_fail(golden, mistake):
    w, want_q, want_s = tie_cases()
    q, s = _mistaken(w, mistake)
    caught = not (np.array_equal(q, want_q) and np.array_equal(s[:, 0], want_s))
    if mistake == "reciprocal" and not caught:   # the fixed points of the real matrices catch it
        for name in REAL:
            qq, ss = fixed_point_groups(golden, name)
            wf = (qq * ss[:, None]).astype(np.float32) / np.float32(16384)
            caught |= not np.array_equal(_mistaken(wf, mistake)[0], qq)
    assert caught


def test_quantize_entry_validation():
    lib = _lib.load()
    st = FAKE + 256

    def call(w=FAKE, dtype=1, ld=1024, rows=4, cols=1024, packed=FAKE, scale=FAKE, status=st):
        return lib.q4d_quantize_q4(w, dtype, ld, rows, cols, packed, scale, status, None)
    assert call(cols=1000) == -11
    assert call(ld=512) == -11
    assert call(rows=0) == -11
    assert call(dtype=0) == -13                 # fp16 input is not a checkpoint format here
    assert call(status=None) == -7
    assert call(w=None) == -7
    assert call(w=FAKE + 4) == -4               # rows need 16-byte alignment
    assert call(w=FAKE + 8, dtype=2) == -4
    assert call(dtype=2, ld=1028) == -4         # bf16 row pitch of 2056 bytes
    assert call(packed=FAKE + 4, dtype=2) == -4  # 8-byte packed stores for bf16
    assert call(ld=1026) == -4                  # row pitch breaks the 16-byte alignment
    with pytest.raises(ValueError, match="2D"):
        quantize_weight_q4(np.zeros(64, np.float32))
    with pytest.raises(ValueError, match="divisible"):
        quantize_weight_q4(np.zeros((2, 100), np.float32))


def test_checkpoint_layout(tmp_path):
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=512)
    names = expected_tensors(cfg)
    assert len(names) == 2 + 2 * 11
    assert names["model.layers.1.self_attn.o_proj.weight"] == (1024, 2048)
    assert names["model.layers.0.mlp.down_proj.weight"] == (1024, 3072)
    check_checkpoint(dict(names), cfg)
    bad = dict(names)
    del bad["model.layers.1.self_attn.k_norm.weight"]
    with pytest.raises(ValueError, match="lacks model.layers.1.self_attn.k_norm"):
        check_checkpoint(bad, cfg)
    bad = dict(names, **{"model.layers.0.mlp.up_proj.weight": (3072, 1000)})
    with pytest.raises(ValueError, match="up_proj"):
        check_checkpoint(bad, cfg)
    with pytest.raises(ValueError, match="untied"):
        check_checkpoint(dict(names, **{"lm_head.weight": (512, 1024)}),
                         Qwen3Config(num_hidden_layers=2, vocab_size=512, tie_word_embeddings=False))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(
        {"weight_map": {"a": "model-00002-of-00002.safetensors", "b": "model-00001-of-00002.safetensors"}}))
    assert [p.name for p in checkpoint_files(tmp_path)] == ["model-00001-of-00002.safetensors",
                                                            "model-00002-of-00002.safetensors"]
    with pytest.raises(FileNotFoundError):
        checkpoint_files(tmp_path / "nowhere")


def test_reference_config_parses():
    cfg = Qwen3Config.from_json(Path(__file__).parent / "golden" / "qwen3_0p6b_config.json")
    assert (cfg.num_hidden_layers, cfg.vocab_size, cfg.tie_word_embeddings) == (28, 151936, True)
