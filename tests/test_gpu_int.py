"""Integer Q4 GEMV (the reference's fixed-point path) on the GPU, bit-exact.

Pins: the reference's own golden vectors (FPGA_Project/sim/vectors, converted
by tests/golden/make_fixtures.py): q_proj rows with Q4.12 activations, the
gate / up / o / down stage vectors with Q12.12 activations and their
expected Q26 sums and Q12.12 outputs, the dot64 and row1024 known answers,
and the 1024-row LM-head window with its best token 264.  Beyond the
fixtures: the oracle's q4_gemv_q26 / q26_to_q12_12 / argmax_first on
extreme inputs (activations at -2^23 and 2^23 - 1, codes at -8 and 7, the
widths the int32 partial sums are sized for), saturating rows, and planted
argmax ties across the scan's thread and wave boundaries.  Bar: equality.
"""

import numpy as np
import pytest
import torch

import oracle as o
from gpu_helpers import q4
from llm_accelerator_amd import integer as I

pytestmark = pytest.mark.gpu

GEMV_FIXTURES = ["q4_gemv_projection_1024_real", "q4_gemv_tile_1024", "mlp_gate_proj_real", "mlp_up_proj_real",
                 "o_proj_real", "mlp_down_proj_real"]


def act(x, dev):
    return torch.from_numpy(np.asarray(x, dtype=np.int64).astype(np.int32)).to(dev)


@pytest.mark.parametrize("name", GEMV_FIXTURES)
def test_q26_gemv_matches_reference_vectors(dev, golden, name):
    d = golden(name)
    print(f"[int gemv] {name} {d['weight_packed'].shape}", flush=True)
    w = q4(d["weight_packed"], d["scale_q2_14"])
    y26 = I.compute_q4_gemv_q26(act(d["activation"], dev), w).cpu().numpy()
    np.testing.assert_array_equal(y26, d["expected_q26"])
    if "expected_q12_12" in d:
        y12, y26b, sat = I.compute_q4_gemv_q12_12(act(d["activation"], dev), w)
        np.testing.assert_array_equal(y12.cpu().numpy(), d["expected_q12_12"])
        np.testing.assert_array_equal(y26b.cpu().numpy(), d["expected_q26"])
        assert sat == 0


def test_known_answers(dev, golden):
    d = golden("q4_dot64_kat")  # tb_q4_dot_product_64.sv:33-44
    y = I.compute_q4_gemv_q26(act(d["activation_q4_12"], dev), q4(d["weight_packed"], d["scale_q2_14"]))
    assert int(y[0]) == int(d["expected_scaled_q26"]) == 3019622
    d = golden("q4_gemv_projection_1024_real")  # Source/Q4_FORMAT.md:212-215
    y = I.compute_q4_gemv_q26(act(d["activation"], dev), q4(d["weight_packed"][:1], d["scale_q2_14"][:1]))
    assert int(y[0]) == -3482169


def test_lm_head_window_scan(dev, golden):
    d = golden("lm_head_argmax_real")  # lm_head_argmax_stage_real_meta.json: token 264, score 1365150750
    logits = I.compute_q4_gemv_q26(act(d["activation"], dev), q4(d["weight_packed"], d["scale_q2_14"]))
    np.testing.assert_array_equal(logits.cpu().numpy(), d["expected_logits_q26"])
    tok, score = I.streamed_argmax_q26(logits)
    assert tok + int(d["scan_base_token"][0]) == int(d["expected_best_token"][0]) == 264
    assert score == int(d["expected_best_score_q26"][0]) == 1365150750


@pytest.mark.parametrize("rows,cols", [(257, 3072), (64, 2048), (130, 1024), (3, 64)])
def test_extreme_inputs_match_oracle(dev, rows, cols):
    rng = np.random.default_rng(rows * cols)
    # activations at the ends of the 24-bit range and random, codes at -8 / 7 and random
    x = rng.integers(-(1 << 23), 1 << 23, size=cols)
    x[::3] = -(1 << 23)
    x[1::7] = (1 << 23) - 1
    q = rng.integers(-8, 8, size=(rows, cols))
    q[0] = -8  # row 0: every product at its extreme, positive with x = -2^23
    q[1] = 7
    scale = rng.integers(1, 1 << 16, size=(rows, cols // 64)).astype(np.uint16)
    packed = o.pack_signed_int4(q)
    print(f"[int gemv] extreme rows={rows} cols={cols}", flush=True)
    ref = o.q4_gemv_q26(x, q, scale)
    ref12, ref_sat = o.q26_to_q12_12(ref)
    assert ref_sat > 0  # these inputs do saturate Q12.12
    y12, y26, sat = I.compute_q4_gemv_q12_12(act(x, dev), q4(packed, scale))
    np.testing.assert_array_equal(y26.cpu().numpy(), ref)
    np.testing.assert_array_equal(y12.cpu().numpy(), ref12)
    assert sat == ref_sat


@pytest.mark.parametrize("n", [1, 5, 1023, 1024, 1025, 151936])
def test_argmax_ties_lowest_index(dev, n):
    rng = np.random.default_rng(n)
    s = rng.integers(-(1 << 50), 1 << 50, size=n)
    top = (1 << 51) + 17
    # planted ties: the same top score at several rows across thread / wave boundaries
    plant = sorted({n - 1, n // 2, (n * 3) // 4, min(n - 1, 1024 + 63), min(n - 1, 64)})
    for i in plant:
        s[i] = top
    ref_i, ref_s = o.argmax_first(s)
    tok, score = I.streamed_argmax_q26(torch.from_numpy(s).to(dev))
    assert (tok, score) == (ref_i, ref_s) == (plant[0], top)
