"""Pin the oracle's integer Q4 path on the reference's own golden vectors.

Fixtures come from FPGA_Project/sim/vectors of the reference (converted by
tests/golden/make_fixtures.py, provenance + sha256 in tests/golden/MANIFEST.json).
"""

import numpy as np
import pytest

import oracle as o

GEMV_FIXTURES = ["q4_gemv_projection_1024_real", "q4_gemv_tile_1024", "mlp_gate_proj_real", "mlp_up_proj_real",
                 "o_proj_real", "mlp_down_proj_real"]


@pytest.mark.parametrize("name", GEMV_FIXTURES)
def test_q26_gemv_matches_reference_vectors(golden, name):
    d = golden(name)
    k = d["weight_packed"].shape[1] * 2
    q = o.unpack_signed_int4(d["weight_packed"], k)
    got = o.q4_gemv_q26(d["activation"], q, d["scale_q2_14"])
    np.testing.assert_array_equal(got, d["expected_q26"])
    if "expected_q12_12" in d:
        q12, sat = o.q26_to_q12_12(got)
        np.testing.assert_array_equal(q12, d["expected_q12_12"])
        assert sat == 0


def test_gate_proj_fixture_has_the_c1_shape(golden):
    d = golden("mlp_gate_proj_real")
    assert d["weight_packed"].shape == (3072, 512) and d["scale_q2_14"].shape == (3072, 16)


@pytest.mark.parametrize("name", GEMV_FIXTURES)
def test_float_gemv_is_exact_real_dot(golden, name):
    """fixture activation/2^12 and W = q*s/2^14 are exact, so expected_q26/2^26 is
    the exact dot product; the fp64 float oracle must reproduce it."""
    d = golden(name)
    W = o.dequantize_q4(d["weight_packed"], d["scale_q2_14"], dtype=np.float64)
    x = d["activation"].astype(np.float64) / 4096.0
    np.testing.assert_allclose(W @ x, d["expected_q26"] / 2.0 ** 26, rtol=0, atol=1e-12)


def test_dot64_known_answer(golden):
    """tb_q4_dot_product_64.sv:33-44: partial 24751, scaled 3019622."""
    d = golden("q4_dot64_kat")
    q = o.unpack_signed_int4(d["weight_packed"], 64)[0].astype(np.int64)
    partial = int(np.sum(q * d["activation_q4_12"]))
    assert partial == int(d["expected_partial"]) == 24751
    assert partial * int(d["scale_q2_14"][0, 0]) == int(d["expected_scaled_q26"]) == 3019622
    # the same numbers through the full GEMV routine
    assert o.q4_gemv_q26(d["activation_q4_12"], q[None], d["scale_q2_14"])[0] == 3019622


def test_row1024_known_answer(golden):
    """Source/Q4_FORMAT.md:212-215: q_proj row 0 = -3482169 (board row1024 smoke)."""
    d = golden("q4_gemv_projection_1024_real")
    q = o.unpack_signed_int4(d["weight_packed"], 1024)
    assert o.q4_gemv_q26(d["activation"], q[:1], d["scale_q2_14"][:1])[0] == -3482169


def test_lm_head_window_argmax_known_answer(golden):
    """lm_head_argmax_stage_real_meta.json: token 264 (' a'), score 1365150750."""
    d = golden("lm_head_argmax_real")
    q = o.unpack_signed_int4(d["weight_packed"], 1024)
    tok, score, logits = o.lm_head_streamed_argmax_q26(d["activation"], q, d["scale_q2_14"], chunk_rows=64)
    np.testing.assert_array_equal(logits, d["expected_logits_q26"])
    assert tok == int(d["expected_best_token"][0]) == 264
    assert score == int(d["expected_best_score_q26"][0]) == 1365150750


def test_words32_fixture_layout_round_trips(golden):
    """words32 <-> packed bytes is the identity on Q4_FORMAT rows."""
    d = golden("mlp_up_proj_real")
    words = d["weight_packed"].view("<u4").reshape(-1)
    np.testing.assert_array_equal(o.words32_to_packed_bytes(words, 1024), d["weight_packed"])
    sw = d["scale_q2_14"].view("<u4").reshape(-1)
    np.testing.assert_array_equal(o.words32_to_scales(sw, 16), d["scale_q2_14"])
