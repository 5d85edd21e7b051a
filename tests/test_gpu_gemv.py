"""Q4 dequant-GEMV and LM-head argmax on the GPU vs the oracle.

Bars: integer unpack and argmax indices bit-exact; fp32-activation GEMV within
fp32 accumulation error (|err| <= 4e-6 * sum_j |W_ij x_j|) of the exact
reference fixtures; fp16-output GEMV additionally within half an fp16 ulp.
"""

import numpy as np
import pytest
import torch

import oracle as o
from gpu_helpers import abs_dot_bound, linear, lm_head_argmax, q4, report
from llm_accelerator_amd._lib import Q4D_F16, Q4D_F32

pytestmark = pytest.mark.gpu

ACC = 4e-6  # fp32 accumulation error relative to sum |w x|


@pytest.mark.parametrize("k", [1024, 2048, 3072])
@pytest.mark.parametrize("xdtype", [torch.float16, torch.float32])
def test_unpack_bit_exact_via_one_hot(dev, k, xdtype):
    """scale code 16384 (= 1.0) and x = e_j give y[n] = q[n, j] exactly."""
    rng = np.random.default_rng(100 + k)
    n = 96
    packed = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    scale = np.full((n, k // 64), 16384, dtype=np.uint16)
    cols = np.unique(np.concatenate([[0, 1, 2, 3, 4, 5, 6, 7, 8, 15, 16, 31, 32, 63, 64, k - 1],
                                     rng.integers(0, k, 48)]))
    x = torch.zeros((len(cols), k), dtype=xdtype, device=dev)
    x[torch.arange(len(cols)), torch.from_numpy(cols)] = 1
    y = linear(q4(packed, scale, dev), x, Q4D_F16).float().cpu().numpy()
    expect = o.unpack_signed_int4(packed, k)[:, cols].T.astype(np.float32)
    np.testing.assert_array_equal(y, expect)


@pytest.mark.parametrize("name", ["mlp_gate_proj_real", "mlp_up_proj_real", "o_proj_real", "mlp_down_proj_real",
                                  "q4_gemv_projection_1024_real", "q4_gemv_tile_1024"])
def test_reference_fixture_fp32_activation(dev, golden, name):
    """Fixture activation (Q12.12 or Q4.12)/2^12 is exact in fp32 and in the
    hi+lo fp16 split, so y must equal expected_q26/2^26 to accumulation error."""
    d = golden(name)
    x = d["activation"].astype(np.float64) / 4096.0
    y = linear(q4(d["weight_packed"], d["scale_q2_14"], dev),
               torch.from_numpy(x.astype(np.float32)).to(dev)[None], Q4D_F32)[0].cpu().numpy()
    exact = d["expected_q26"] / 2.0 ** 26
    W = o.dequantize_q4(d["weight_packed"], d["scale_q2_14"], dtype=np.float64)
    bound = ACC * abs_dot_bound(W, x) + 1e-30
    report(name, y, exact)
    assert np.all(np.abs(y - exact) <= bound), float(np.max(np.abs(y - exact) / bound))


def test_gate_proj_fixture_fp16_activation(dev, golden):
    """3072x1024 benchmark shape, fp16 activation: matches the oracle on the fp16-rounded x."""
    d = golden("mlp_gate_proj_real")
    x16 = (d["activation"].astype(np.float64) / 4096.0).astype(np.float16)
    y = linear(q4(d["weight_packed"], d["scale_q2_14"], dev), torch.from_numpy(x16).to(dev)[None],
               Q4D_F32)[0].cpu().numpy()
    W = o.dequantize_q4(d["weight_packed"], d["scale_q2_14"], dtype=np.float64)
    ref = W @ x16.astype(np.float64)
    report("gate fp16-x", y, ref)
    assert np.all(np.abs(y - ref) <= ACC * abs_dot_bound(W, x16))


def test_c1_synthetic_fp16_in_fp16_out(dev):
    """The benchmark GEMV: W 3072x1024 Q4 random, x fp16 ~ N(0,1), y fp16."""
    from llm_accelerator_amd.model import random_q4
    rng = np.random.default_rng(0)
    packed, scale = random_q4(rng, 3072, 1024)
    x16 = np.random.default_rng(1).normal(size=1024).astype(np.float16)
    y = linear(q4(packed, scale, dev), torch.from_numpy(x16).to(dev)[None], Q4D_F16)[0].float().cpu().numpy()
    W = o.dequantize_q4(packed, scale, dtype=np.float64)
    ref = W @ x16.astype(np.float64)
    report("gemv 3072x1024 fp16", y, ref)
    ulp_half = np.abs(ref) * 2.0 ** -11 + 2.0 ** -25
    assert np.all(np.abs(y - ref) <= ulp_half + ACC * abs_dot_bound(W, x16))


def test_batched_rows_are_independent(dev):
    """batch > 1 reuses the kernel per activation row."""
    from llm_accelerator_amd.model import random_q4
    rng = np.random.default_rng(5)
    packed, scale = random_q4(rng, 1024, 2048)
    x = rng.normal(size=(3, 2048)).astype(np.float32)
    w = q4(packed, scale, dev)
    yb = linear(w, torch.from_numpy(x).to(dev), Q4D_F32).cpu().numpy()
    for i in range(3):
        yi = linear(w, torch.from_numpy(x[i:i + 1]).to(dev), Q4D_F32).cpu().numpy()[0]
        np.testing.assert_array_equal(yb[i], yi)


def test_lm_head_window_fixture_argmax(dev, golden):
    """Reference LM-head window (rows 0..1023): argmax 264 ('a'), lowest index on ties."""
    d = golden("lm_head_argmax_real")
    x = (d["activation"].astype(np.float64) / 4096.0).astype(np.float32)
    table = q4(d["weight_packed"], d["scale_q2_14"], dev)
    gamma = torch.ones(1024, dtype=torch.float32, device=dev)
    tok, score, logits, _ = lm_head_argmax(table, torch.from_numpy(x).to(dev), gamma)
    assert tok == 264
    xn = o.manual_rms_norm(x.astype(np.float64), np.ones(1024), 1e-6, dtype=np.float64)
    W = o.dequantize_q4(d["weight_packed"], d["scale_q2_14"], dtype=np.float64)
    ref = W @ xn
    lg = logits.cpu().numpy()
    report("lm window", lg, ref)
    assert np.all(np.abs(lg - ref) <= 1e-5 * abs_dot_bound(W, xn) + 1e-6)
    assert score == lg[264] == lg.max()
    assert int(np.argmax(ref)) == 264


def _planted_table(rng, vocab, winners, k=1024):
    from llm_accelerator_amd.model import random_q4
    packed, scale = random_q4(rng, vocab, k)
    x = rng.normal(size=k).astype(np.float32)
    q = np.where(x > 0, 7, -8).astype(np.int8)[None]
    row = o.pack_signed_int4(q)[0]
    for r in winners:
        packed[r] = row
        scale[r] = 4000
    return packed, scale, x


@pytest.mark.parametrize("winners", [[151935, 5, 70001, 70000], [2, 3], [1, 149999, 150000], [151934, 151935]])
def test_lm_head_full_vocab_tie_rule(dev, winners):
    """Identical winning rows in different lanes, waves and blocks: the
    lowest index wins through the block and grid reductions."""
    rng = np.random.default_rng(sum(winners))
    packed, scale, x = _planted_table(rng, 151936, winners)
    gamma = torch.ones(1024, dtype=torch.float32, device=dev)
    tok, score, logits, _ = lm_head_argmax(q4(packed, scale, dev), torch.from_numpy(x).to(dev), gamma)
    lg = logits.cpu().numpy()
    assert len(set(lg[winners].tolist())) == 1
    assert tok == min(winners)
    assert score == lg[min(winners)] == lg.max()


def test_lm_head_repeatable_and_counter_resets(dev):
    """Back-to-back launches reuse the workspace counter (self-resetting)."""
    rng = np.random.default_rng(9)
    from llm_accelerator_amd.model import random_q4
    packed, scale = random_q4(rng, 151936, 1024)
    table = q4(packed, scale, dev)
    gamma = torch.from_numpy((1 + 0.1 * rng.normal(size=1024)).astype(np.float32)).to(dev)
    h = torch.from_numpy(rng.normal(size=1024).astype(np.float32) * 30).to(dev)
    res = [lm_head_argmax(table, h, gamma)[:2] for _ in range(3)]
    assert res[0] == res[1] == res[2]
    # oracle argmax on the same fp32 activations (near-tie aware)
    W = o.dequantize_q4(packed, scale)
    xn = o.manual_rms_norm(h.cpu().numpy(), gamma.cpu().numpy(), 1e-6)
    ref = W.astype(np.float64) @ xn.astype(np.float64)
    top = np.argsort(ref)[-2:]
    if ref[top[1]] - ref[top[0]] > 1e-3:
        assert res[0][0] == int(top[1])


@pytest.mark.parametrize("k,xdtype,ydtype,batch,count,precision", [(1024, torch.float16, Q4D_F16, 1, 70, 2),
                                                                   (2048, torch.float32, Q4D_F32, 3, 5, 2),
                                                                   (3072, torch.float32, Q4D_F16, 2, 9, 2),
                                                                   (1024, torch.float32, Q4D_F32, 1, 64, 2),
                                                                   (2048, torch.float32, Q4D_F32, 2, 66, 1)])
def test_linear_group_equals_single_calls(dev, k, xdtype, ydtype, batch, count, precision):
    """q4d_linear_group over `count` matrices (70: launches of 64 + 6), each with its own
    x and y, equals one q4d_linear call per matrix bit for bit, at either activation
    precision (fp32 x as hi + lo fp16 pairs, or one fp16 value); one matrix also meets the
    oracle's accumulation bound."""
    import ctypes
    from llm_accelerator_amd import _lib
    from llm_accelerator_amd.model import current_stream
    rng = np.random.default_rng(k + count)
    n = 2 * (96 + count)  # rows: even, not a multiple of the block's rows
    mats = [q4(rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8),
               rng.integers(50, 3000, size=(n, k // 64)).astype(np.uint16), dev) for _ in range(count)]
    xs = [torch.randn(batch, k, device=dev, dtype=torch.float32).to(xdtype) for _ in range(count)]
    ydt = torch.float16 if ydtype == Q4D_F16 else torch.float32
    ys = [torch.full((batch, n), float('nan'), device=dev, dtype=ydt) for _ in range(count)]
    descs = (_lib.Q4dMatrix * count)(*[m.descriptor() for m in mats])
    xp = (ctypes.c_void_p * count)(*[x.data_ptr() for x in xs])
    yp = (ctypes.c_void_p * count)(*[y.data_ptr() for y in ys])
    print(f"[gemv] group {count} x {n}x{k} batch {batch}", flush=True)
    xcode = Q4D_F16 if xdtype == torch.float16 else Q4D_F32
    lib = _lib.load()
    _lib.check(lib.q4d_set_activation_precision(precision), "q4d_set_activation_precision")
    try:
        _lib.check(lib.q4d_linear_group(descs, xp, xcode, yp, ydtype, batch, count, current_stream()),
                   "q4d_linear_group")
        for i in range(count):
            want = linear(mats[i], xs[i], ydtype)
            assert torch.equal(ys[i], want), i
    finally:
        _lib.check(lib.q4d_set_activation_precision(2), "q4d_set_activation_precision")
    W = o.dequantize_q4(mats[0].packed.cpu().numpy(), mats[0].scale.cpu().numpy(), dtype=np.float64)
    x0 = xs[0][0].float().cpu().numpy()
    ref = W @ x0.astype(np.float64)
    y0 = ys[0][0].float().cpu().numpy()
    half_ulp = np.abs(ref) * 2.0 ** -11 + 2.0 ** -25 if ydtype == Q4D_F16 else 0.0
    # fp32 activations enter as fp16 hi + lo halves (~22 bits, 2^-21 relative each) at
    # precision 2, as one fp16 value (2^-11) at precision 1
    xerr = (2.0 ** -21 if precision == 2 else 2.0 ** -11) * abs_dot_bound(W, x0) if xdtype == torch.float32 else 0.0
    assert np.all(np.abs(y0 - ref) <= half_ulp + xerr + ACC * abs_dot_bound(W, x0))
