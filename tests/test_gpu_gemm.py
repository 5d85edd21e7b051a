"""MFMA Q4 GEMM (prefill / batched decode path) on the GPU vs the oracle.

The GEMM multiplies fp16 activations by Q4 tiles dequantised to fp16
(W16 = fp16(q * fp16(code / 2^14))) with fp32 accumulation.

Tolerances (stated):
- integer-exact cases (|q * code| < 2^11, small-integer x) are exact in every
  step, so the output must equal the float64 product bit for bit; this pins
  the MFMA operand layout, the nibble order and the scale indexing;
- real Qwen3 weights (the reference's exported gate/down projections) against
  the float64 product with the same fp16 operands: |err| <= 2^-16 * sum|x w|
  (fp32 accumulation only); against the exact Q4 weights:
  |err| <= 2^-10 * sum|x w| (two fp16 roundings of each weight);
- argmax indices must be bit-exact, lowest index on ties;
- batched decode (all layers, fp16 activations into every projection) against
  the oracle run per sequence: logits max-abs <= 5e-3 * max|ref|, next tokens
  identical unless the oracle's top-2 gap is within the measured error.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as o
from gpu_helpers import abs_dot_bound, head_model, q4, report
from llm_accelerator_amd import _lib
from llm_accelerator_amd._lib import Q4D_F16, Q4D_F32, check
from llm_accelerator_amd.decode import BatchedDecoder
from llm_accelerator_amd.model import KVCache, Qwen3Config, build_model, current_stream, random_host_weights

pytestmark = pytest.mark.gpu


def gemm(w, x: torch.Tensor, y_dtype=Q4D_F32, resid: torch.Tensor | None = None) -> torch.Tensor:
    rows, cols = w.shape
    M = x.shape[0]
    assert x.dtype == torch.float16 and x.shape[1] == cols and x.is_contiguous()
    y = torch.empty((M, rows), dtype=torch.float16 if y_dtype == Q4D_F16 else torch.float32, device=x.device)
    desc = w.descriptor()
    check(_lib.load().q4d_gemm(ctypes.byref(desc), x.data_ptr(), M, y.data_ptr(), y_dtype,
                               resid.data_ptr() if resid is not None else None, current_stream()), "q4d_gemm")
    torch.cuda.synchronize()
    return y


def exact_case(rng, N, K, M):
    q = rng.integers(-8, 8, size=(N, K))
    packed = o.pack_signed_int4(q)
    scale = rng.integers(1, 128, size=(N, K // 64)).astype(np.uint16)
    x = rng.integers(-4, 5, size=(M, K)).astype(np.float16)
    W = o.dequantize_q4(packed, scale, np.float64)
    ref = x.astype(np.float64) @ W.T
    # every partial sum is a multiple of 2^-14 below 2^10: exact in fp32
    assert (np.abs(x.astype(np.float64)) @ np.abs(W).T).max() < 1024
    return packed, scale, x, ref


def w16_of(packed, scale, K):
    q = o.unpack_signed_int4(packed, K).astype(np.float16)
    s16 = (scale.astype(np.float64) / 16384.0).astype(np.float16)
    return (q * np.repeat(s16, 64, axis=1)).astype(np.float16)  # fp16 product, one rounding


@pytest.mark.parametrize("N,K", [(256, 1024), (128, 3072), (384, 2048)])
@pytest.mark.parametrize("M", [1, 7, 64, 65, 130, 256])
def test_gemm_integer_exact(dev, N, K, M):
    rng = np.random.default_rng(N * 7 + K + M)
    packed, scale, x, ref = exact_case(rng, N, K, M)
    print(f"[gemm exact] M={M} N={N} K={K}", flush=True)
    y = gemm(q4(packed, scale), torch.from_numpy(x).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(y, ref.astype(np.float32))


@pytest.mark.parametrize("N,K,M", [(4096, 1024, 2048), (4096, 1024, 900), (4096, 2048, 1100), (4096, 3072, 1000)])
def test_gemm_128_row_tiles_integer_exact(dev, N, K, M):
    """Shapes whose 128-row tiles fill the device (N / 128 * ceil(M / 128) >= 256), so
    q4d_gemm takes the 128-row-tile kernel the 2048-token prefill's q|k|v projection
    runs (N = 4096, M = 2048); M = 900 / 1100 / 1000 end on a partial row tile."""
    assert N // 128 * ((M + 127) // 128) >= 256
    rng = np.random.default_rng(N + 3 * K + M)
    packed, scale, x, ref = exact_case(rng, N, K, M)
    print(f"[gemm exact 128-row tiles] M={M} N={N} K={K}", flush=True)
    y = gemm(q4(packed, scale), torch.from_numpy(x).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(y, ref.astype(np.float32))


def test_gemm_epilogues_exact(dev):
    rng = np.random.default_rng(11)
    packed, scale, x, ref = exact_case(rng, 256, 1024, 70)
    w = q4(packed, scale)
    xd = torch.from_numpy(x).to(dev)
    y16 = gemm(w, xd, Q4D_F16).cpu().numpy()
    np.testing.assert_array_equal(y16, ref.astype(np.float32).astype(np.float16))
    resid = rng.normal(size=ref.shape).astype(np.float32)
    r = torch.from_numpy(resid).to(dev)
    y = gemm(w, xd, Q4D_F32, resid=r).cpu().numpy()
    np.testing.assert_array_equal(y, resid + ref.astype(np.float32))
    # in place: y aliases resid (the decoder's residual stream)
    desc = w.descriptor()
    check(_lib.load().q4d_gemm(ctypes.byref(desc), xd.data_ptr(), 70, r.data_ptr(), Q4D_F32, r.data_ptr(),
                               current_stream()), "q4d_gemm")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(r.cpu().numpy(), resid + ref.astype(np.float32))


def test_gemm_many_rows_epilogues_exact(dev):
    """Prefill-sized M (300 rows, a partial last row tile): fp16 output, residual add
    and the in-place residual (y aliasing resid)."""
    rng = np.random.default_rng(12)
    M = 300
    packed, scale, x, ref = exact_case(rng, 512, 1024, M)
    w = q4(packed, scale)
    xd = torch.from_numpy(x).to(dev)
    print(f"[gemm epilogues many rows] M={M} N=512 K=1024", flush=True)
    y16 = gemm(w, xd, Q4D_F16).cpu().numpy()
    np.testing.assert_array_equal(y16, ref.astype(np.float32).astype(np.float16))
    resid = rng.normal(size=ref.shape).astype(np.float32)
    r = torch.from_numpy(resid).to(dev)
    y = gemm(w, xd, Q4D_F32, resid=r).cpu().numpy()
    np.testing.assert_array_equal(y, resid + ref.astype(np.float32))
    desc = w.descriptor()
    check(_lib.load().q4d_gemm(ctypes.byref(desc), xd.data_ptr(), M, r.data_ptr(), Q4D_F32, r.data_ptr(),
                               current_stream()), "q4d_gemm")
    torch.cuda.synchronize()
    np.testing.assert_array_equal(r.cpu().numpy(), resid + ref.astype(np.float32))


def gemm_splitk(w, x: torch.Tensor, ksplit: int, y_dtype=Q4D_F32, resid: torch.Tensor | None = None,
                y: torch.Tensor | None = None) -> torch.Tensor:
    rows, cols = w.shape
    M = x.shape[0]
    if y is None:
        y = torch.empty((M, rows), dtype=torch.float16 if y_dtype == Q4D_F16 else torch.float32, device=x.device)
    part = torch.full((max(ksplit, 16) * M * rows,), float("nan"), dtype=torch.float32, device=x.device)
    desc = w.descriptor()
    check(_lib.load().q4d_gemm_splitk(ctypes.byref(desc), x.data_ptr(), M, y.data_ptr(), y_dtype,
                                      resid.data_ptr() if resid is not None else None, part.data_ptr(),
                                      part.numel() * 4, ksplit, current_stream()), "q4d_gemm_splitk")
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("ksplit", [0, 2, 5, 16])
@pytest.mark.parametrize("N,K,M", [(1024, 2048, 64), (1024, 3072, 37), (256, 1024, 1)])
def test_gemm_splitk_integer_exact(dev, N, K, M, ksplit):
    """Split-K on integer-exact inputs (every fp32 sum exact, whatever its
    grouping) equals the float64 product bit for bit; ksplit = 0 lets the
    library choose.  The partial buffer starts as NaN, so a split tile left
    unwritten or read twice shows up."""
    if ksplit > K // 64:
        pytest.skip("more splits than K steps")
    rng = np.random.default_rng(N + K + M + ksplit)
    packed, scale, x, ref = exact_case(rng, N, K, M)
    print(f"[gemm splitk] M={M} N={N} K={K} ksplit={ksplit}", flush=True)
    w = q4(packed, scale)
    xd = torch.from_numpy(x).to(dev)
    y = gemm_splitk(w, xd, ksplit).cpu().numpy()
    np.testing.assert_array_equal(y, ref.astype(np.float32))
    y16 = gemm_splitk(w, xd, ksplit, Q4D_F16).cpu().numpy()
    np.testing.assert_array_equal(y16, ref.astype(np.float32).astype(np.float16))
    resid = rng.normal(size=ref.shape).astype(np.float32)
    r = torch.from_numpy(resid).to(dev)
    gemm_splitk(w, xd, ksplit, Q4D_F32, resid=r, y=r)  # in place, as the residual stream
    np.testing.assert_array_equal(r.cpu().numpy(), resid + ref.astype(np.float32))


@pytest.mark.parametrize("ksplit", [0, 2, 4])
@pytest.mark.parametrize("N,K,M", [(1024, 2048, 300), (1024, 3072, 2048)])
def test_gemm_many_rows_splitk_integer_exact(dev, N, K, M, ksplit):
    """Split-K at prefill-sized M with the residual epilogue: the prefill down shape
    (N = 1024, K = 3072, M = 2048) with a 2-way split runs the pipelined kernel
    (128 tiles x 2 splits fill the device in one round), 4-way and automatic splits
    the 128-row-tile kernel; M = 300 ends on a partial row tile."""
    rng = np.random.default_rng(N + K + M + ksplit)
    packed, scale, x, ref = exact_case(rng, N, K, M)
    print(f"[gemm splitk many rows] M={M} N={N} K={K} ksplit={ksplit}", flush=True)
    resid = rng.normal(size=ref.shape).astype(np.float32)
    y = gemm_splitk(q4(packed, scale), torch.from_numpy(x).to(dev), ksplit,
                    resid=torch.from_numpy(resid).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(y, resid + ref.astype(np.float32))


def test_gemm_splitk_real_weights_match_unsplit(dev, golden):
    f = golden("mlp_down_proj_real")
    packed, scale = f["weight_packed"], f["scale_q2_14"]
    N, K = packed.shape[0], packed.shape[1] * 2
    x = np.random.default_rng(8).normal(size=(64, K)).astype(np.float16)
    w = q4(packed, scale)
    xd = torch.from_numpy(x).to(dev)
    y1 = gemm(w, xd).cpu().numpy().astype(np.float64)
    Wex = o.dequantize_q4(packed, scale, np.float64)
    bound = np.abs(x.astype(np.float64)) @ np.abs(Wex).T
    for ks in (3, 16):
        y = gemm_splitk(w, xd, ks).cpu().numpy().astype(np.float64)
        assert np.all(np.abs(y - y1) <= 2.0 ** -16 * bound + 1e-30), ks


@pytest.mark.parametrize("name,M", [("mlp_gate_proj_real", 64), ("mlp_down_proj_real", 33)])
def test_gemm_real_weights(dev, golden, name, M):
    f = golden(name)
    packed, scale = f["weight_packed"], f["scale_q2_14"]
    N, K = packed.shape[0], packed.shape[1] * 2
    rng = np.random.default_rng(5)
    x = np.empty((M, K), dtype=np.float16)
    x[0] = (f["activation"] / 4096.0).astype(np.float16)  # the exported Q12.12 activation
    x[1:] = rng.normal(size=(M - 1, K)).astype(np.float16)
    y = gemm(q4(packed, scale), torch.from_numpy(x).to(dev)).cpu().numpy().astype(np.float64)
    W16 = w16_of(packed, scale, K).astype(np.float64)
    ref16 = x.astype(np.float64) @ W16.T
    Wex = o.dequantize_q4(packed, scale, np.float64)
    ref = x.astype(np.float64) @ Wex.T
    bound = np.abs(x.astype(np.float64)) @ np.abs(Wex).T
    report(f"{name} vs fp16-operand product", y, ref16)
    report(f"{name} vs exact Q4 product", y, ref)
    assert np.all(np.abs(y - ref16) <= 2.0 ** -16 * bound + 1e-30)
    assert np.all(np.abs(y - ref) <= 2.0 ** -10 * bound)
    # row 0 against the reference's own GEMV vector (Q26 = 2^26 * value); the
    # bound adds what rounding the exported activation to fp16 can move
    exp0 = f["expected_q26"].astype(np.float64) / 2.0 ** 26
    dx = np.abs(f["activation"] / 4096.0 - x[0].astype(np.float64))
    assert np.all(np.abs(y[0] - exp0) <= 2.0 ** -10 * bound[0] + abs_dot_bound(Wex, dx) + 1e-9)


def lm_head_batch(table, hidden: torch.Tensor, final_norm: torch.Tensor):
    lib = _lib.load()
    m = head_model(table, final_norm)
    B = hidden.shape[0]
    nbytes = int(lib.q4d_workspace_bytes(ctypes.byref(m), B))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=hidden.device)
    tok = torch.full((B,), -1, dtype=torch.int32, device=hidden.device)
    score = torch.zeros(B, dtype=torch.float32, device=hidden.device)
    logits = torch.empty((B, table.shape[0]), dtype=torch.float32, device=hidden.device)
    check(lib.q4d_lm_head_argmax_batch(ctypes.byref(m), hidden.contiguous().data_ptr(), B, tok.data_ptr(),
                                       score.data_ptr(), logits.data_ptr(), ws.data_ptr(), nbytes,
                                       current_stream()), "q4d_lm_head_argmax_batch")
    torch.cuda.synchronize()
    return tok.cpu().numpy(), score.cpu().numpy(), logits.cpu().numpy()


def test_lm_head_batch_argmax_and_ties(dev):
    """Planted duplicate rows make exact ties; the lower index must win, also
    across 128-column blocks and across the two waves of one block."""
    rng = np.random.default_rng(21)
    V, H, B = 4096, 1024, 9
    q = rng.integers(-8, 8, size=(V, H))
    scale = rng.integers(100, 400, size=(V, H // 64)).astype(np.uint16)
    hidden = rng.normal(size=(B, H)).astype(np.float32)
    gamma = np.ones(H, dtype=np.float32)
    xn = o.manual_rms_norm(hidden.astype(np.float64), gamma, 1e-6, np.float64)
    # per row b: make row w_b the winner by aligning it with xn[b], duplicate it later
    # same lane group, next block, same wave, cross-wave (2100 | 2150), cross-tile (64 | 100)
    winners = [7, 127, 128, 1000, 2047, 2100, 3000, 4000, 64]
    dups = [4095, 255, 129, 1001, 3071, 2150, 3001, 4094, 100]
    for b, (wi, di) in enumerate(zip(winners, dups)):
        sgn = np.sign(xn[b]).astype(np.int64)
        q[wi] = np.where(sgn >= 0, 7, -8) * (sgn != 0)
        scale[wi] = 400
    for b, (wi, di) in enumerate(zip(winners, dups)):
        q[di] = q[wi]
        scale[di] = scale[wi]
    packed = o.pack_signed_int4(q)
    tok, score, logits = lm_head_batch(q4(packed, scale), torch.from_numpy(hidden).to(dev),
                                       torch.from_numpy(gamma).to(dev))
    for b in range(B):
        first = int(np.argmax(logits[b]))  # numpy argmax returns the first maximum
        assert tok[b] == first, (b, tok[b], first)
        assert score[b] == logits[b, first]
        wi, di = winners[b], dups[b]
        if wi < di:  # duplicate after the winner: exact tie, lower index wins
            assert logits[b, wi] == logits[b, di]
            assert tok[b] == wi, (b, tok[b], wi)
    # logits against the float64 product of fp16 operands; the device's fp32
    # RMSNorm may round an element of x to the neighbouring fp16 value
    x16 = xn.astype(np.float16).astype(np.float64)
    ref = x16 @ w16_of(packed, scale, H).astype(np.float64).T
    report("lm head batch logits", logits, ref)
    bound = np.abs(x16) @ np.abs(o.dequantize_q4(packed, scale, np.float64)).T
    assert np.all(np.abs(logits - ref) <= 2.0 ** -10 * bound)


@pytest.fixture(scope="module")
def batch_setup(dev):
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=2048)
    host = random_host_weights(cfg, seed=3, num_layers=2)
    model = build_model(cfg, host, max_ctx=512, device=dev)
    om = o.OracleModel.from_q4(o.OracleConfig(num_hidden_layers=2, vocab_size=2048), host["layers"],
                               *host["embed_tokens"], host["norm"], dtype=np.float64)
    return cfg, model, om


@pytest.mark.parametrize("positions", [[0, 1, 63, 64, 300], [511] * 3, list(range(0, 448, 7))])
def test_decode_batch_vs_oracle(dev, batch_setup, positions):
    cfg, model, om = batch_setup
    B = len(positions)
    rng = np.random.default_rng(B)
    tokens = rng.integers(0, cfg.vocab_size, B)
    kv = KVCache(cfg, 2, B, model.max_ctx, dev)
    pre = rng.normal(size=(2, 2, B, 8, model.max_ctx, 128)).astype(np.float16)
    for b, p in enumerate(positions):
        pre[:, :, b, :, p:] = 0
    kv.data.copy_(torch.from_numpy(pre).to(dev))
    print(f"[decode batch] B={B} positions={positions[:6]}...", flush=True)
    dec = BatchedDecoder(model, B, kv)
    logits = torch.empty((B, cfg.vocab_size), dtype=torch.float32, device=dev)
    nt, sc = dec.step(torch.tensor(tokens, dtype=torch.int32, device=dev),
                      torch.tensor(positions, dtype=torch.int32, device=dev), logits)
    torch.cuda.synchronize()
    assert dec.status() == 0
    nt, sc, lg = nt.cpu().numpy(), sc.cpu().numpy(), logits.cpu().numpy().astype(np.float64)
    kvd = kv.data.float().cpu().numpy()
    worst, near = 0.0, []
    for b, p in enumerate(positions):
        kc = [pre[li, 0, b][None, :, :p].astype(np.float64) for li in range(2)]
        vc = [pre[li, 1, b][None, :, :p].astype(np.float64) for li in range(2)]
        rl, rt = o.run_manual_one_token(np.array([[tokens[b]]]), p, om, kc, vc, kv_store_dtype=np.float16)
        r = rl[0, -1]
        err = np.abs(lg[b] - r)
        worst = max(worst, float(err.max() / np.abs(r).max()))
        first = int(np.argmax(lg[b]))
        assert nt[b] == first and sc[b] == np.float32(lg[b, first])
        if nt[b] != rt[0, 0]:
            gap = r[rt[0, 0]] - r[nt[b]]
            assert gap <= err[rt[0, 0]] + err[nt[b]], (b, gap)
            near.append((b, int(rt[0, 0]), int(nt[b]), float(gap)))
        for li in range(2):  # appended K/V rows
            for kind, ref_c in ((0, kc[li]), (1, vc[li])):
                want = ref_c[0, :, p]
                got = kvd[li, kind, b, :, p]
                assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want).max(axis=-1, keepdims=True)), (b, li, kind)
    print(f"[decode batch] B={B} max rel logit err={worst:.3e} near_ties={near}", flush=True)
    assert worst < 5e-3


LONG_CTX = 4097   # the batched-decode benchmark's cache: 4096 filled positions + the new one


@pytest.fixture(scope="module")
def batch_long_setup(dev):
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=2048)
    host = random_host_weights(cfg, seed=3, num_layers=2)
    model = build_model(cfg, host, max_ctx=LONG_CTX, device=dev)
    om = o.OracleModel.from_q4(o.OracleConfig(num_hidden_layers=2, vocab_size=2048), host["layers"],
                               *host["embed_tokens"], host["norm"], dtype=np.float64)
    return cfg, model, om


def test_decode_batch_64_sequences_4096_positions(dev, batch_long_setup):
    """The batched-decode benchmark's shape (64 sequences, caches of 4097 positions,
    attention over up to 4096 + 1 positions per sequence) on 2 layers: the span
    attention kernel with its double-buffered 64-position sub-chunks and its merge of
    up to 8 splits, against the oracle's full-softmax attention per sequence
    (common.py:219-228).  Positions cover an empty cache, sub-chunk and span edges
    and the last slot."""
    cfg, model, om = batch_long_setup
    edges = [0, 1, 63, 64, 65, 575, 576, 2047, 2048, 4000, 4095, 4096]
    rng = np.random.default_rng(64)
    positions = edges + rng.integers(0, LONG_CTX, 64 - len(edges)).tolist()
    B = len(positions)
    tokens = rng.integers(0, cfg.vocab_size, B)
    print(f"[decode batch long] B={B} max_ctx={LONG_CTX}: filling caches", flush=True)
    pre = np.empty((2, 2, B, 8, LONG_CTX, 128), dtype=np.float16)
    for li in range(2):
        for kind in range(2):
            pre[li, kind] = rng.standard_normal(size=(B, 8, LONG_CTX, 128), dtype=np.float32)
    for b, p in enumerate(positions):
        pre[:, :, b, :, p:] = 0
    kv = KVCache(cfg, 2, B, LONG_CTX, dev)
    kv.data.copy_(torch.from_numpy(pre).to(dev))
    dec = BatchedDecoder(model, B, kv)
    logits = torch.empty((B, cfg.vocab_size), dtype=torch.float32, device=dev)
    nt, sc = dec.step(torch.tensor(tokens, dtype=torch.int32, device=dev),
                      torch.tensor(positions, dtype=torch.int32, device=dev), logits)
    torch.cuda.synchronize()
    assert dec.status() == 0
    nt, sc, lg = nt.cpu().numpy(), sc.cpu().numpy(), logits.cpu().numpy().astype(np.float64)
    print("[decode batch long] comparing with the oracle per sequence", flush=True)
    worst, near = 0.0, []
    for b, p in enumerate(positions):
        kc = [pre[li, 0, b][None, :, :p].astype(np.float64) for li in range(2)]
        vc = [pre[li, 1, b][None, :, :p].astype(np.float64) for li in range(2)]
        rl, rt = o.run_manual_one_token(np.array([[tokens[b]]]), p, om, kc, vc, kv_store_dtype=np.float16)
        r = rl[0, -1]
        err = np.abs(lg[b] - r)
        worst = max(worst, float(err.max() / np.abs(r).max()))
        first = int(np.argmax(lg[b]))
        assert nt[b] == first and sc[b] == np.float32(lg[b, first])
        if nt[b] != rt[0, 0]:
            gap = r[rt[0, 0]] - r[nt[b]]
            assert gap <= err[rt[0, 0]] + err[nt[b]], (b, p, gap)
            near.append((b, int(rt[0, 0]), int(nt[b]), float(gap)))
        for li in range(2):
            for kind, ref_c in ((0, kc[li]), (1, vc[li])):
                want = ref_c[0, :, p]
                got = kv.data[li, kind, b, :, p].float().cpu().numpy()
                assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want).max(axis=-1, keepdims=True)), (b, li, kind)
    # nothing written past each sequence's position
    for b, p in enumerate(positions):
        assert not kv.data[:, :, b, :, p + 1:].any(), (b, p)
    print(f"[decode batch long] B={B} max rel logit err={worst:.3e} near_ties={near}", flush=True)
    assert worst < 5e-3


FULL_B, FULL_P = 64, 4096   # the batched-decode benchmark: 64 sequences, 4096 cached positions each


@pytest.mark.slow
def test_decode_batch_full_model_64x4096(dev, qwen3_full):
    """The batched-decode benchmark's workload at full size, under a check: 64
    sequences, each with a 4096-position fp16 cache of N(0,1) values (the same
    generator, seed and token draw as the benchmark), one step through all 28 layers
    and the 151936-row batched LM head with its per-row argmax over 1187 block
    partials.  Per sequence that is run_manual_one_token
    (10_validate_full_run_one_token.py:17-56) at position 4096; every sequence's token
    is the lowest-index argmax of its logits, and 8 sequences spread over the batch are
    compared with the oracle (logits, token up to a reported near-tie, the K/V rows
    appended at position 4096 in layers 0, 1, 13 and 27)."""
    cfg, host, om = qwen3_full
    L = cfg.num_hidden_layers
    model = build_model(cfg, host, max_ctx=FULL_P + 1, device=dev)
    print(f"[decode batch full] {FULL_B} x {FULL_P}: filling 28-layer caches", flush=True)
    gen = torch.Generator(device=dev).manual_seed(5)
    kv = KVCache(cfg, L, FULL_B, FULL_P + 1, dev)
    kv.data[..., :FULL_P, :].normal_(generator=gen)
    pre_slot = kv.data[..., FULL_P, :].clone()
    assert not pre_slot.any()
    tokens = np.random.default_rng(3).integers(0, cfg.vocab_size, FULL_B).astype(np.int32)
    dec = BatchedDecoder(model, FULL_B, kv)
    logits = torch.empty((FULL_B, cfg.vocab_size), dtype=torch.float32, device=dev)
    nt, sc = dec.step(torch.from_numpy(tokens).to(dev), torch.full((FULL_B,), FULL_P, dtype=torch.int32, device=dev),
                      logits)
    torch.cuda.synchronize()
    assert dec.status() == 0
    nt, sc, lg = nt.cpu().numpy(), sc.cpu().numpy(), logits.cpu().numpy()
    for b in range(FULL_B):
        first = int(np.argmax(lg[b]))
        assert nt[b] == first and sc[b] == lg[b, first], (b, int(nt[b]), first)
    print("[decode batch full] comparing 8 sequences with the oracle", flush=True)
    worst, near = 0.0, []
    for b in range(0, FULL_B, 9):
        kc = [kv.data[li, 0, b, :, :FULL_P].float().cpu().numpy()[None] for li in range(L)]
        vc = [kv.data[li, 1, b, :, :FULL_P].float().cpu().numpy()[None] for li in range(L)]
        rl, rt = o.run_manual_one_token(np.array([[int(tokens[b])]]), FULL_P, om, kc, vc, kv_store_dtype=np.float16)
        r = rl[0, -1].astype(np.float64)
        err = np.abs(lg[b].astype(np.float64) - r)
        rel = float(err.max() / np.abs(r).max())
        worst = max(worst, rel)
        if nt[b] != rt[0, 0]:
            gap = r[rt[0, 0]] - r[nt[b]]
            assert gap <= err[rt[0, 0]] + err[nt[b]], (b, gap)
            near.append((b, int(rt[0, 0]), int(nt[b]), float(gap)))
        for li in (0, 1, 13, 27):
            for kind, ref_c in ((0, kc[li]), (1, vc[li])):
                want = ref_c[0, :, FULL_P].astype(np.float64)
                got = kv.data[li, kind, b, :, FULL_P].float().cpu().numpy()
                assert np.all(np.abs(got - want) <= 2e-2 * np.abs(want).max(axis=-1, keepdims=True)), (b, li, kind)
        print(f"[decode batch full] seq {b}: token {int(nt[b])} (oracle {int(rt[0, 0])}), max rel logit err "
              f"{rel:.3e}", flush=True)
        del kc, vc
    print(f"[decode batch full] worst rel logit err={worst:.3e} near_ties={near}", flush=True)
    assert worst < 5e-3
    # the step wrote position 4096 of every sequence and layer, and nothing else changed
    assert kv.data[..., FULL_P, :].abs().amax(dim=-1).gt(0).all()


@pytest.mark.slow
def test_lm_head_batch_full_vocab_64_rows_ties(dev):
    """The batched LM head at the benchmark's size (151936 rows, 64 sequences): planted
    winners and exact duplicates of them across the last 128-row blocks, block pairs in
    the middle and the first/last row resolve to the lower index, and every row's token
    is the first maximum of its logits (logits against the float64 product of the fp16
    operands)."""
    rng = np.random.default_rng(151936)
    V, H, B = 151936, 1024, 64
    print(f"[lm head full] {V} x {H}, {B} rows: building the table", flush=True)
    packed = rng.integers(0, 256, size=(V, H // 2), dtype=np.uint8)
    scale = rng.integers(100, 400, size=(V, H // 64)).astype(np.uint16)
    hidden = rng.normal(size=(B, H)).astype(np.float32)
    gamma = np.ones(H, dtype=np.float32)
    xn = o.manual_rms_norm(hidden.astype(np.float64), gamma, 1e-6, np.float64)
    # (winner, duplicate) rows, 128 distinct rows: inside the last 128-row block (1186:
    # rows 151808..151935), from block 1185 into 1186, across 128-row block edges in the
    # middle, the first rows against the last ones, and across 64-row tile edges
    pairs = []
    for i in range(8):
        pairs.append((151808 + 4 * i, 151810 + 4 * i))
    for i in range(8):
        pairs.append((151680 + 4 * i, 151873 + 4 * i))
    for i in range(16):
        k = 500 + 2 * i
        pairs.append((128 * k + 127, 128 * (k + 1)))
    for i in range(16):
        pairs.append((i, 151935 - i))
    for i in range(16):
        w = 10000 + 1000 * i + 63
        pairs.append((w, w + 65))
    assert len({r for pr in pairs for r in pr}) == 2 * B
    for b, (wi, di) in enumerate(pairs):
        sgn = np.sign(xn[b]).astype(np.int64)
        qrow = np.where(sgn >= 0, 7, -8) * (sgn != 0)
        packed[wi] = o.pack_signed_int4(qrow[None])[0]
        scale[wi] = 400
        packed[di] = packed[wi]
        scale[di] = scale[wi]
    tok, score, logits = lm_head_batch(q4(packed, scale), torch.from_numpy(hidden).to(dev),
                                       torch.from_numpy(gamma).to(dev))
    for b, (wi, di) in enumerate(pairs):
        first = int(np.argmax(logits[b]))
        assert tok[b] == first and score[b] == logits[b, first], (b, tok[b], first)
        # the planted pair is an exact tie and the lower index wins
        assert logits[b, wi] == logits[b, di] and tok[b] == wi, (b, int(tok[b]), wi, di)
    print("[lm head full] float64 reference", flush=True)
    x16 = xn.astype(np.float16).astype(np.float64)
    for r0 in range(0, V, 16384):
        w16 = w16_of(packed[r0:r0 + 16384], scale[r0:r0 + 16384], H).astype(np.float64)
        ref = x16 @ w16.T
        bound = np.abs(x16) @ np.abs(o.dequantize_q4(packed[r0:r0 + 16384], scale[r0:r0 + 16384], np.float64)).T
        assert np.all(np.abs(logits[:, r0:r0 + 16384] - ref) <= 2.0 ** -10 * bound), r0
