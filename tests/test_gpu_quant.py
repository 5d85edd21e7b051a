"""The float -> Q4 quantizer kernel (q4d_quantize_q4) against the oracle, bit for bit.

Cases: normal weights at several scales (including groups small enough for the
nonzero rule and fp32 subnormals), K = 64 .. 3072 with row counts that leave partial
waves, the hand-built ties of test_quant_host (w / s and absmax / 7 * 2^14 exactly on
k + 1/2, clipping at -8 / 7), the reference's real Q4 matrices dequantised (fixed
points), bf16 input (equal to its fp32 widening), strided rows, the overflow and
non-finite errors, a full-size tied table (151936 x 1024, bf16) checked on sampled
rows, and a Hugging Face-layout checkpoint converted and decoded.
"""

import json

import numpy as np
import pytest
import torch

import oracle as o
from llm_accelerator_amd.decode import greedy_generate
from llm_accelerator_amd.model import Qwen3Config, build_model
from llm_accelerator_amd.quantize import convert_checkpoint, expected_tensors, quantize_weight_q4
from test_quant_host import REAL, fixed_point_groups, tie_cases

pytestmark = pytest.mark.gpu


def check(w32: np.ndarray, dev, dtype=torch.float32):
    want_p, want_s, want_q = o.quantize_weight_q4(w32)
    t = torch.from_numpy(w32).to(dev).to(dtype)
    p, s, q = quantize_weight_q4(t)
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)
    np.testing.assert_array_equal(p.cpu().numpy(), want_p)
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)


@pytest.mark.parametrize("rows,cols,sigma", [(300, 1024, 0.02), (37, 3072, 1.0), (5, 2048, 3e-5),
                                             (3, 320, 1e-39), (1, 64, 4.0), (129, 1024, 1e-4)])
def test_random_matrices_match_oracle(dev, rows, cols, sigma):
    rng = np.random.default_rng(rows + cols)
    w = (rng.standard_normal((rows, cols)) * sigma).astype(np.float32)
    w[0, :64] = 0.0                      # an all-zero group
    if cols >= 192:
        w[-1, 128:192] *= 1e-3           # a group that leans on the nonzero rule
    print(f"[quant] random {rows}x{cols} sigma {sigma}", flush=True)
    check(w, dev)


def test_ties_match_oracle(dev):
    w, want_q, want_s = tie_cases()
    check(w, dev)
    _, s, q = quantize_weight_q4(torch.from_numpy(w).to(dev))
    np.testing.assert_array_equal(q.cpu().numpy(), want_q)
    np.testing.assert_array_equal(s.cpu().numpy()[:, 0], want_s)


@pytest.mark.parametrize("name", REAL)
def test_reference_fixed_points(dev, golden, name):
    qq, ss = fixed_point_groups(golden, name)
    w = ((qq * ss[:, None]).astype(np.float32) / np.float32(16384))
    _, s, q = quantize_weight_q4(torch.from_numpy(w).to(dev))
    np.testing.assert_array_equal(q.cpu().numpy(), qq)
    np.testing.assert_array_equal(s.cpu().numpy()[:, 0], ss)


@pytest.mark.parametrize("sigma", [0.03, 1.0, 5.0, 1e-3, 1e-30])
def test_bf16_matrices_match_oracle(dev, sigma):
    """bf16 weights (8 significant bits) land exactly on rounding ties often (about 1 in
    400 elements at sigma 0.03): every one must round half to even as numpy does."""
    g = torch.Generator().manual_seed(int(sigma * 1e3) + 5)
    wb = (torch.randn(2048, 1024, generator=g) * sigma).to(torch.bfloat16)
    print(f"[quant] bf16 2048x1024 sigma {sigma}", flush=True)
    check(wb.float().numpy(), dev, torch.bfloat16)


def test_bf16_and_strided_input(dev):
    rng = np.random.default_rng(3)
    wb = torch.from_numpy((rng.standard_normal((65, 1024)) * 0.05).astype(np.float32)).to(torch.bfloat16)
    w32 = wb.float().numpy()
    check(w32, dev, torch.bfloat16)
    wide = torch.from_numpy(rng.standard_normal((40, 2048 + 64)).astype(np.float32)).to(dev)
    view = wide[:, 64:]                   # row pitch 2112 elements, 16-byte aligned start
    p, s, _ = quantize_weight_q4(view)
    want_p, want_s, _ = o.quantize_weight_q4(view.cpu().numpy())
    np.testing.assert_array_equal(p.cpu().numpy(), want_p)
    np.testing.assert_array_equal(s.cpu().numpy(), want_s)


def test_errors_like_the_reference(dev):
    w = np.zeros((2, 128), np.float32)
    w[1, 70] = 30.0                       # absmax / 7 * 2^14 > 65535
    with pytest.raises(ValueError, match="Q2.14"):
        o.quantize_weight_q4(w)
    with pytest.raises(ValueError, match="1 groups with absmax too large, 0 groups with non-finite"):
        quantize_weight_q4(torch.from_numpy(w).to(dev))
    w[1, 70] = np.nan
    with pytest.raises(ValueError, match="0 groups with absmax too large, 1 groups with non-finite"):
        quantize_weight_q4(torch.from_numpy(w).to(dev))
    w[1, 70] = 28.0                       # 28 / 7 * 2^14 = 65536: one past the top
    with pytest.raises(ValueError):
        quantize_weight_q4(torch.from_numpy(w).to(dev))
    w[1, 70] = np.float32(65535 * 7 / 16384)   # largest absmax that still fits
    _, s, _ = quantize_weight_q4(torch.from_numpy(w).to(dev))
    assert int(s.cpu().numpy()[1, 1]) == int(o.quantize_weight_q4(w)[1][1, 1])


def test_full_size_table_sampled_rows(dev):
    g = torch.Generator(device=dev).manual_seed(7)
    w = (torch.randn(151936, 1024, device=dev, generator=g) * 0.03).to(torch.bfloat16)
    p, s, _ = quantize_weight_q4(w, return_codes=False)
    torch.cuda.synchronize()
    rows = np.r_[0:64, 75000:75064, 151872:151936]
    w32 = w[torch.from_numpy(rows).to(dev)].float().cpu().numpy()
    want_p, want_s, _ = o.quantize_weight_q4(w32)
    np.testing.assert_array_equal(p.cpu().numpy()[rows], want_p)
    np.testing.assert_array_equal(s.cpu().numpy()[rows], want_s)


def test_checkpoint_conversion(dev, tmp_path):
    from safetensors.torch import save_file
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=4096)
    rng = np.random.default_rng(11)
    tensors = {}
    for name, shape in expected_tensors(cfg).items():
        scale = 1.0 if len(shape) == 1 else 0.03
        base = 1.0 if len(shape) == 1 else 0.0
        tensors[name] = torch.from_numpy((base + rng.standard_normal(shape) * scale).astype(np.float32)).to(
            torch.bfloat16)
    save_file(tensors, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({"num_hidden_layers": 2, "vocab_size": 4096}))
    got_cfg, host = convert_checkpoint(tmp_path, device=dev)
    assert got_cfg == cfg
    hf = {"q_proj": "self_attn.q_proj", "k_proj": "self_attn.k_proj", "v_proj": "self_attn.v_proj",
          "o_proj": "self_attn.o_proj", "gate_proj": "mlp.gate_proj", "up_proj": "mlp.up_proj",
          "down_proj": "mlp.down_proj"}
    for li in range(2):
        for ours, theirs in hf.items():
            want_p, want_s, _ = o.quantize_weight_q4(tensors[f"model.layers.{li}.{theirs}.weight"].float().numpy())
            np.testing.assert_array_equal(host["layers"][li][ours][0], want_p)
            np.testing.assert_array_equal(host["layers"][li][ours][1], want_s)
        np.testing.assert_array_equal(host["layers"][li]["q_norm"],
                                      tensors[f"model.layers.{li}.self_attn.q_norm.weight"].float().numpy())
    emb = o.quantize_weight_q4(tensors["model.embed_tokens.weight"].float().numpy())
    np.testing.assert_array_equal(host["embed_tokens"][0], emb[0])
    np.testing.assert_array_equal(host["embed_tokens"][1], emb[1])
    np.testing.assert_array_equal(host["norm"], tensors["model.norm.weight"].float().numpy())
    tokens, _ = greedy_generate(build_model(cfg, host, max_ctx=16, device=dev), [5, 9], 4, use_graph=False)
    print(f"[quant] converted checkpoint decodes {tokens}", flush=True)
    assert len(tokens) == 4 and all(0 <= t < cfg.vocab_size for t in tokens)


def _batch_call(ws, dtype_code, status):
    """q4d_quantize_q4_batch over device matrices of one shape -> [(packed, scale)]."""
    import ctypes
    from llm_accelerator_amd import _lib
    from llm_accelerator_amd.model import current_stream
    rows, cols = ws[0].shape
    dev = ws[0].device
    packed = [torch.empty(rows, cols // 2, dtype=torch.uint8, device=dev) for _ in ws]
    scale = [torch.empty(rows, cols // 64, dtype=torch.uint16, device=dev) for _ in ws]
    n = len(ws)
    wp = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
    pp = (ctypes.c_void_p * n)(*[t.data_ptr() for t in packed])
    sp = (ctypes.c_void_p * n)(*[t.data_ptr() for t in scale])
    _lib.check(_lib.load().q4d_quantize_q4_batch(wp, dtype_code, ws[0].stride(0), rows, cols, n, pp, sp,
                                                 status.data_ptr(), current_stream()), "q4d_quantize_q4_batch")
    return list(zip(packed, scale))


@pytest.mark.parametrize("dtype,rows,cols,count", [(torch.bfloat16, 3072, 1024, 3), (torch.bfloat16, 37, 2048, 70),
                                                   (torch.float32, 129, 1024, 5), (torch.float32, 1, 64, 2)])
def test_batch_equals_single_calls(dev, dtype, rows, cols, count):
    """One launch over `count` matrices (70: two launches, 64 + 6) equals count single
    conversions bit for bit; sampled matrices also equal the oracle."""
    from llm_accelerator_amd._lib import Q4D_BF16, Q4D_F32
    g = torch.Generator(device=dev).manual_seed(rows + count)
    ws = [(torch.randn(rows, cols, device=dev, generator=g) * (0.02 * (i + 1))).to(dtype) for i in range(count)]
    ws[0][0, :64] = 0                      # an all-zero group
    status = torch.zeros(2, dtype=torch.int32, device=dev)
    print(f"[quant] batch {count} x {rows}x{cols} {dtype}", flush=True)
    got = _batch_call(ws, Q4D_BF16 if dtype == torch.bfloat16 else Q4D_F32, status)
    assert status.tolist() == [0, 0]
    for i, w in enumerate(ws):
        p, s, _ = quantize_weight_q4(w, return_codes=False)
        assert torch.equal(got[i][0], p) and torch.equal(got[i][1], s), i
    for i in (0, count - 1):
        w32 = ws[i][:64].float().cpu().numpy()
        want_p, want_s, _ = o.quantize_weight_q4(w32)
        np.testing.assert_array_equal(got[i][0][:64].cpu().numpy(), want_p)
        np.testing.assert_array_equal(got[i][1][:64].cpu().numpy(), want_s)


def test_batch_status_sums_and_python_errors(dev):
    """Bad groups of several matrices add up in the one status pair; the list wrapper
    returns the matrices in order (mixed shapes and dtypes) and names the first failing one."""
    from llm_accelerator_amd._lib import Q4D_F32
    from llm_accelerator_amd.quantize import quantize_weights_q4
    rng = np.random.default_rng(11)
    base = [(rng.standard_normal((4, 256)) * 0.1).astype(np.float32) for _ in range(4)]
    base[1][2, 70] = 30.0                  # overflow in matrix 1
    base[3][0, 5] = np.inf                 # non-finite in matrix 3
    base[3][3, 200] = 40.0                 # and an overflow
    ws = [torch.from_numpy(b).to(dev) for b in base]
    status = torch.zeros(2, dtype=torch.int32, device=dev)
    _batch_call(ws, Q4D_F32, status)
    assert status.tolist() == [2, 1]
    with pytest.raises(ValueError, match="matrix 1: Q4 scale does not fit"):
        quantize_weights_q4(ws)
    mixed = [torch.from_numpy((rng.standard_normal(s) * 0.05).astype(np.float32)).to(dev)
             for s in ((8, 128), (16, 64), (8, 128), (3, 192))]
    mixed[2] = mixed[2].to(torch.bfloat16)
    got = quantize_weights_q4(mixed)
    for w, (p, s) in zip(mixed, got):
        want_p, want_s, _ = quantize_weight_q4(w, return_codes=False)
        assert torch.equal(p, want_p) and torch.equal(s, want_s)


@pytest.mark.parametrize("dtype,count", [(torch.bfloat16, 70), (torch.float32, 3)])
def test_batch_strided_rows(dev, dtype, count):
    """Column slices of wider matrices (one row pitch for all, 16-byte aligned starts) through
    one batch call and through the list wrapper equal single conversions of contiguous copies."""
    from llm_accelerator_amd._lib import Q4D_BF16, Q4D_F32
    from llm_accelerator_amd.quantize import quantize_weights_q4
    g = torch.Generator(device=dev).manual_seed(count)
    rows, cols, pad = 24, 1024, 64 if dtype == torch.float32 else 128
    wides = [(torch.randn(rows, cols + pad, device=dev, generator=g) * 0.03).to(dtype) for _ in range(count)]
    views = [w[:, pad:] for w in wides]
    assert views[0].stride(0) == cols + pad and views[0].data_ptr() % 16 == 0
    status = torch.zeros(2, dtype=torch.int32, device=dev)
    print(f"[quant] strided batch {count} x {rows}x{cols} pitch {cols + pad} {dtype}", flush=True)
    got = _batch_call(views, Q4D_BF16 if dtype == torch.bfloat16 else Q4D_F32, status)
    assert status.tolist() == [0, 0]
    listed = quantize_weights_q4(views)
    for i, v in enumerate(views):
        p, s, _ = quantize_weight_q4(v.contiguous(), return_codes=False)
        assert torch.equal(got[i][0], p) and torch.equal(got[i][1], s), i
        assert torch.equal(listed[i][0], p) and torch.equal(listed[i][1], s), i
    want_p, want_s, _ = o.quantize_weight_q4(views[-1].float().cpu().numpy())
    np.testing.assert_array_equal(got[-1][0].cpu().numpy(), want_p)
    np.testing.assert_array_equal(got[-1][1].cpu().numpy(), want_s)
