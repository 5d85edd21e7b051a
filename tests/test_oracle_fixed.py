"""The fixed-point (RTL-exact) oracle against the reference's stage vectors.

Every stage of the integer decode layer is checked against the expected
outputs the reference exported for layer 0 (position 4 of the prompt
[785, 3853, 315, 89462, 374]) and for the layer-1/2 variants, including the
intermediate RMSNorm quantities (sum of squares, mean, radicand, rms, inverse
rms), the exp and sigmoid LUTs, the softmax LUT indices and probabilities, and
the K/V write addresses.  Beyond the fixtures: isqrt and the shifts against
brute force, and planted mistakes in the oracle (a dropped rounding term, an
unrotated RoPE half, a truncating instead of flooring shift) that these
fixtures catch.  Bar: equality.
"""

import math

import numpy as np
import pytest

import oracle as o
from oracle import q4_fixed as F

RMS = ["fixed_rmsnorm_input_l0", "fixed_rmsnorm_input_l1c", "fixed_rmsnorm_input_l2c", "fixed_rmsnorm_final",
       "fixed_rmsnorm_final_l2c"]
QK = ["fixed_qk_norm_rope_l0", "fixed_qk_norm_rope_l1c", "fixed_qk_norm_rope_l2c"]
ATT = ["fixed_attention_l0", "fixed_attention_l1", "fixed_attention_l1c", "fixed_attention_l2c"]
TAGS = ["l0", "l1c", "l2c"]


def check_norm_stats(r, d, prefix=""):
    for key in ("sum_squares", "mean_square", "sqrt_radicand", "rms", "inv_rms"):
        assert r[key] == int(d[prefix + key][0]), key


@pytest.mark.parametrize("name", RMS)
def test_rmsnorm_hidden(golden, name):
    d = golden(name)
    r = F.fixed_rmsnorm_hidden(d["input"], d["gamma"])
    check_norm_stats(r, d)
    np.testing.assert_array_equal(r["output"], d["expected"])
    assert (r["saturation"] > 0) == bool(d["saturation"][0])


@pytest.mark.parametrize("name", QK)
def test_qk_norm_rope(golden, name):
    d = golden(name)
    qn, qs = F.fixed_rmsnorm_heads(d["q_input"].reshape(16, 128), d["q_gamma"])
    kn, ks = F.fixed_rmsnorm_heads(d["k_input"].reshape(8, 128), d["k_gamma"])
    np.testing.assert_array_equal(qn.reshape(-1), d["q_norm_expected"])
    np.testing.assert_array_equal(kn.reshape(-1), d["k_norm_expected"])
    qr, qrs = F.fixed_rope(qn, d["cos"], d["sin"])
    kr, krs = F.fixed_rope(kn, d["cos"], d["sin"])
    np.testing.assert_array_equal(qr.reshape(-1), d["q_rope_expected"])
    np.testing.assert_array_equal(kr.reshape(-1), d["k_rope_expected"])
    assert (qs + ks > 0) == bool(d["norm_saturation"][0])
    assert (qrs + krs > 0) == bool(d["rope_saturation"][0])


def test_rope_alone(golden):
    d = golden("fixed_rope_qk_l0")
    np.testing.assert_array_equal(F.fixed_rope(d["q_input"].reshape(16, 128), d["cos"], d["sin"])[0].reshape(-1),
                                  d["q_expected"])
    np.testing.assert_array_equal(F.fixed_rope(d["k_input"].reshape(8, 128), d["cos"], d["sin"])[0].reshape(-1),
                                  d["k_expected"])


def test_rope_table_position_4(golden):
    """The Q1.15 table row of position 4 equals the fixtures' cos/sin, incl. 66 saturated cos = 1.0."""
    inv = o.rope_inv_freq(1_000_000.0, 128)
    cos, sin = F.rope_table_q1_15(inv, np.arange(8))
    for name in QK + ["fixed_rope_qk_l0"]:
        d = golden(name)
        np.testing.assert_array_equal(cos[4], d["cos"])
        np.testing.assert_array_equal(sin[4], d["sin"])
    cf, _ = o.manual_rope_cos_sin(inv, np.array([[4]]))
    assert F.quantize_signed(cf[0, 0], 16, 15)[1] == 66  # the reference meta's cos_quantize_count
    assert np.all(cos[0] == 32767) and np.all(sin[0] == 0)


@pytest.mark.parametrize("name", ATT)
def test_attention_stages(golden, name):
    d = golden(name)
    t = int(d["cache_length"][0])
    q = d["q_input"].reshape(16, 128)
    k = d["k_cache"].reshape(t, 8, 128)
    v = d["v_cache"].reshape(t, 8, 128)
    scale = int(d["score_scale_q0_31"][0])
    assert scale == F.score_scale_q0_31(128 ** -0.5) == 189812531
    raw, scaled = F.attention_scores(q, k, scale)
    np.testing.assert_array_equal(raw.reshape(-1), d["expected_raw"])
    np.testing.assert_array_equal(scaled.reshape(-1), d["expected_scaled"])
    np.testing.assert_array_equal(d["expected_q_head"], np.repeat(np.arange(16), t))
    np.testing.assert_array_equal(d["expected_position"], np.tile(np.arange(t), 16))
    np.testing.assert_array_equal(d["score_input"], d["expected_scaled"])
    lut = F.build_exp_lut()
    np.testing.assert_array_equal(lut, d["exp_lut"])
    probs, idx = F.fixed_softmax_probs(scaled, lut)
    np.testing.assert_array_equal(idx.reshape(-1), d["expected_lut_index"])
    np.testing.assert_array_equal(probs.reshape(-1), d["expected_prob"])
    out, _ = F.fixed_value_accum(probs, v)
    np.testing.assert_array_equal(out.reshape(-1), d["expected_out"])
    full = F.attention_score_value(q, k, v, scale, lut)
    np.testing.assert_array_equal(full["output"], out)


@pytest.mark.parametrize("tag", TAGS)
def test_post_attention_residual_norm(golden, tag):
    d = golden(f"fixed_post_residual_norm_{tag}")
    res, sat = F.residual_add(d["residual_input"], d["o_proj_input"])
    np.testing.assert_array_equal(res, d["expected_residual"])
    assert (sat > 0) == bool(d["residual_saturation"][0])
    r = F.fixed_rmsnorm_hidden(res, d["gamma"])
    check_norm_stats(r, d)
    np.testing.assert_array_equal(r["output"], d["expected_norm"])


@pytest.mark.parametrize("tag", TAGS)
def test_silu_mul(golden, tag):
    d = golden(f"fixed_silu_mul_{tag}")
    lut = F.build_sigmoid_lut()
    np.testing.assert_array_equal(lut, d["sigmoid_lut"])
    r = F.silu_mul(d["gate_input"], d["up_input"], lut)
    np.testing.assert_array_equal(r["lut_index"], d["expected_lut_index"])
    np.testing.assert_array_equal(r["sigmoid"], d["expected_sigmoid_q0_16"])
    np.testing.assert_array_equal(r["silu_gate"], d["expected_silu_gate_q12_12"])
    np.testing.assert_array_equal(r["hidden"], d["expected_hidden_q12_12"])


@pytest.mark.parametrize("tag", TAGS)
def test_mlp_residual_add(golden, tag):
    d = golden(f"fixed_residual_add_{tag}")
    out, sat = F.residual_add(d["post_attn_hidden"], d["down_out"])
    np.testing.assert_array_equal(out, d["expected_layer_out"])
    assert (sat > 0) == bool(d["residual_saturation"][0])


def test_stage_chain_consistency(golden):
    """Layer 0's stage fixtures are one chain: the post-attention residual feeds the MLP residual."""
    post = golden("fixed_post_residual_norm_l0")
    res = golden("fixed_residual_add_l0")
    np.testing.assert_array_equal(post["expected_residual"], res["post_attn_hidden"])
    np.testing.assert_array_equal(golden("fixed_rmsnorm_input_l0")["input"], post["residual_input"])
    att = golden("fixed_attention_l0")
    np.testing.assert_array_equal(golden("fixed_qk_norm_rope_l0")["q_rope_expected"], att["q_input"])


def test_kv_append_addresses(golden):
    d = golden("fixed_kv_append_l0")
    addr, data = [], []
    for kind, src in ((0, d["k_input"]), (1, d["v_input"])):
        for head in range(8):
            for dim in range(128):
                addr.append(F.kv_addr(0x4_1410_0000, 0, kind, head, 4, dim, 256))
                data.append(int(src[head * 128 + dim]))
    np.testing.assert_array_equal(np.array(addr, dtype=np.int64), d["expected_addr"])
    np.testing.assert_array_equal(np.array(data, dtype=np.int64), d["expected_data"])
    np.testing.assert_array_equal(d["expected_kind"], np.repeat([0, 1], 1024))
    np.testing.assert_array_equal(d["expected_head"], np.tile(np.repeat(np.arange(8), 128), 2))
    np.testing.assert_array_equal(d["expected_dim"], np.tile(np.arange(128), 16))


def test_isqrt_and_floor_shift_brute_force():
    rng = np.random.default_rng(0)
    for v in list(range(0, 300)) + [int(x) for x in rng.integers(0, 1 << 57, 300)]:
        r = math.isqrt(v)
        assert r * r <= v < (r + 1) * (r + 1)
    x = rng.integers(-(1 << 40), 1 << 40, 1000)
    for s in (2, 14, 16, 21, 23):
        np.testing.assert_array_equal(x >> s, np.floor(x / float(1 << s)).astype(np.int64))


def test_embedding_is_onehot_gemv():
    rng = np.random.default_rng(1)
    q = rng.integers(-8, 8, size=(5, 1024))
    s = rng.integers(1, 1 << 16, size=(5, 16)).astype(np.uint16)
    packed = o.pack_signed_int4(q)
    row = F.embed_q14_10(packed[3], s[3])
    for c in (0, 63, 64, 511, 1023):
        e = np.zeros(1024, dtype=np.int64)
        e[c] = 1
        assert row[c] == o.q4_gemv_q26(e, q, s)[3] >> 4


def test_planted_mistakes_fail(golden):
    """Plausible slips in the oracle are caught by the fixtures."""
    d = golden("fixed_attention_l0")
    t = int(d["cache_length"][0])
    _, scaled = F.attention_scores(d["q_input"].reshape(16, 128), d["k_cache"].reshape(t, 8, 128),
                                   int(d["score_scale_q0_31"][0]))
    lut = F.build_exp_lut()
    m = scaled.max(axis=1, keepdims=True)
    idx_no_round = np.minimum((m - scaled) >> 20, 256)  # rounding term dropped
    assert not np.array_equal(idx_no_round.reshape(-1), d["expected_lut_index"])
    q = golden("fixed_qk_norm_rope_l0")
    qn, _ = F.fixed_rmsnorm_heads(q["q_input"].reshape(16, 128), q["q_gamma"])
    wrong = (qn * q["cos"] + qn * q["sin"]) >> 15  # rotate_half forgotten
    assert not np.array_equal(np.clip(wrong, -(1 << 23), (1 << 23) - 1).reshape(-1), q["q_rope_expected"])
    s = golden("fixed_silu_mul_l0")
    g = s["gate_input"]
    trunc = np.trunc(g * F.build_sigmoid_lut()[F.gate_to_lut_index(g)] / 65536.0).astype(np.int64)
    assert not np.array_equal(trunc, s["expected_silu_gate_q12_12"])  # truncation instead of floor
    r = golden("fixed_rmsnorm_input_l0")
    bad = F.fixed_rmsnorm(r["input"], r["gamma"], mean_shift=10, eps=0, num_shift=26, out_shift=21)
    good = F.fixed_rmsnorm_hidden(r["input"], r["gamma"])
    assert bad["sqrt_radicand"] != int(r["sqrt_radicand"][0]) and good["sqrt_radicand"] == int(r["sqrt_radicand"][0])
