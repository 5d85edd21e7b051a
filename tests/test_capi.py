"""CPU-side checks of the C ABI: the library loads, exports every function
include/q4dec.h declares, and host validation fails closed (negative codes,
no launch) on bad descriptors.  No kernel is launched here."""

import ctypes
import re
from pathlib import Path

import pytest

from llm_accelerator_amd import _lib
from llm_accelerator_amd._lib import Q4dKVCache, Q4dLayer, Q4dMatrix, Q4dModel

HEADER = Path(__file__).resolve().parents[1] / "include" / "q4dec.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(q4d_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libq4dec.so is not built: run `python -m llm_accelerator_amd.build`")
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared_functions()
    assert len(names) >= 17
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_version_and_status_strings(lib):
    assert lib.q4d_version() == 1
    assert lib.q4d_status_string(0) == b"ok"
    assert lib.q4d_status_string(-8) == b"token id outside the vocabulary"
    assert lib.q4d_status_string(-10) == b"position outside the context"


FAKE = 0x7F0000000000  # aligned, never dereferenced: validation fails before launch


def _model(layers_arr, **kw):
    d = dict(hidden_size=1024, intermediate_size=3072, num_layers=len(layers_arr), num_q_heads=16, num_kv_heads=8,
             head_dim=128, vocab_size=151936, max_ctx=512, rms_norm_eps=1e-6, attn_scaling=128 ** -0.5)
    d.update(kw)
    m = Q4dModel(**d)
    m.layers = ctypes.cast(layers_arr, ctypes.POINTER(Q4dLayer))
    m.embed_tokens = Q4dMatrix(FAKE, FAKE, 151936, 1024)
    m.final_norm = m.rope_cos = m.rope_sin = FAKE
    return m


def _layers(n=1):
    arr = (Q4dLayer * n)()
    for i in range(n):
        L = arr[i]
        for name, (r, c) in dict(q_proj=(2048, 1024), k_proj=(1024, 1024), v_proj=(1024, 1024), o_proj=(1024, 2048),
                                 gate_proj=(3072, 1024), up_proj=(3072, 1024), down_proj=(1024, 3072)).items():
            setattr(L, name, Q4dMatrix(FAKE, FAKE, r, c))
        L.input_layernorm = L.post_attention_layernorm = L.q_norm = L.k_norm = FAKE
    return arr


def test_workspace_bytes_grows_with_context(lib):
    arr = _layers()
    a = lib.q4d_workspace_bytes(ctypes.byref(_model(arr, max_ctx=512)), 1)
    b = lib.q4d_workspace_bytes(ctypes.byref(_model(arr, max_ctx=4096)), 1)
    assert 0 < a < b
    assert lib.q4d_workspace_bytes(None, 1) == 0


def test_linear_rejects_bad_shapes_before_launch(lib):
    m = Q4dMatrix(FAKE, FAKE, 3072, 1000)  # cols not supported
    assert lib.q4d_linear(ctypes.byref(m), FAKE, 0, FAKE, 0, 1, None) == -11
    m = Q4dMatrix(FAKE, FAKE, 3071, 1024)  # odd rows: a row pair would run off the matrix
    assert lib.q4d_linear(ctypes.byref(m), FAKE, 0, FAKE, 0, 1, None) == -11
    m = Q4dMatrix(FAKE + 8, FAKE, 3072, 1024)  # 128-bit loads need 16-byte rows
    assert lib.q4d_linear(ctypes.byref(m), FAKE, 0, FAKE, 0, 1, None) == -4
    m = Q4dMatrix(None, FAKE, 3072, 1024)
    assert lib.q4d_linear(ctypes.byref(m), FAKE, 0, FAKE, 0, 1, None) == -7
    m = Q4dMatrix(FAKE, FAKE, 3072, 1024)
    assert lib.q4d_linear(ctypes.byref(m), FAKE, 7, FAKE, 0, 1, None) == -13
    assert lib.q4d_linear(ctypes.byref(m), FAKE, 0, FAKE, 0, 0, None) == -11


def test_model_validation_codes(lib):
    arr = _layers(2)
    kv = Q4dKVCache(data=FAKE, num_layers=2, batch=1, num_kv_heads=8, max_ctx=512, head_dim=128)
    ws = FAKE
    # wrong layer shape -> BAD_LAYER
    arr[1].down_proj = Q4dMatrix(FAKE, FAKE, 1024, 2048)
    m = _model(arr)
    assert lib.q4d_decoder_layer(ctypes.byref(m), 0, FAKE, FAKE, ctypes.byref(kv), FAKE, ws, 1 << 30, None) == -2
    arr[1].down_proj = Q4dMatrix(FAKE, FAKE, 1024, 3072)
    # bad layer index
    assert lib.q4d_decoder_layer(ctypes.byref(m), 5, FAKE, FAKE, ctypes.byref(kv), FAKE, ws, 1 << 30, None) == -2
    # workspace too small
    assert lib.q4d_decoder_layer(ctypes.byref(m), 0, FAKE, FAKE, ctypes.byref(kv), FAKE, ws, 16, None) == -9
    # cache geometry mismatch
    kv2 = Q4dKVCache(data=FAKE, num_layers=2, batch=1, num_kv_heads=8, max_ctx=256, head_dim=128)
    assert lib.q4d_decoder_layer(ctypes.byref(m), 0, FAKE, FAKE, ctypes.byref(kv2), FAKE, ws, 1 << 30, None) == -11
    # unsupported head geometry
    m3 = _model(arr, num_q_heads=24)
    assert lib.q4d_run_one_token(ctypes.byref(m3), FAKE, FAKE, ctypes.byref(kv), FAKE, FAKE, None, ws, 1 << 30,
                                 None) == -11
    # null outputs
    assert lib.q4d_run_one_token(ctypes.byref(m), FAKE, FAKE, ctypes.byref(kv), None, FAKE, None, ws, 1 << 30,
                                 None) == -7


def test_batched_entry_validation_codes(lib):
    arr = _layers(2)
    m = _model(arr)
    kv = Q4dKVCache(data=FAKE, num_layers=2, batch=2, num_kv_heads=8, max_ctx=512, head_dim=128)
    # cache holds 2 sequences, 4 requested
    assert lib.q4d_decode_batch(ctypes.byref(m), FAKE, FAKE, 4, ctypes.byref(kv), FAKE, FAKE, None, FAKE, 1 << 30,
                                None) == -9
    # workspace too small for the batch
    assert lib.q4d_decode_batch(ctypes.byref(m), FAKE, FAKE, 2, ctypes.byref(kv), FAKE, FAKE, None, FAKE, 4096,
                                None) == -9
    assert lib.q4d_decode_batch(ctypes.byref(m), FAKE, FAKE, 0, ctypes.byref(kv), FAKE, FAKE, None, FAKE, 1 << 30,
                                None) == -11
    assert lib.q4d_decode_batch(ctypes.byref(m), None, FAKE, 2, ctypes.byref(kv), FAKE, FAKE, None, FAKE, 1 << 30,
                                None) == -7
    # vocabulary not a multiple of the 128-column GEMM tile
    m2 = _model(arr, vocab_size=1000)
    m2.embed_tokens = Q4dMatrix(FAKE, FAKE, 1000, 1024)
    assert lib.q4d_lm_head_argmax_batch(ctypes.byref(m2), FAKE, 2, FAKE, FAKE, None, FAKE, 1 << 30, None) == -11
    # GEMM shapes: rows % 128, cols % 64, dtype
    w = Q4dMatrix(FAKE, FAKE, 200, 1024)
    assert lib.q4d_gemm(ctypes.byref(w), FAKE, 4, FAKE, 1, None, None) == -11
    w = Q4dMatrix(FAKE, FAKE, 256, 1000)
    assert lib.q4d_gemm(ctypes.byref(w), FAKE, 4, FAKE, 1, None, None) != 0
    w = Q4dMatrix(FAKE, FAKE, 256, 1024)
    assert lib.q4d_gemm(ctypes.byref(w), FAKE, 4, FAKE, 7, None, None) == -13
    assert lib.q4d_gemm(ctypes.byref(w), FAKE, 4, FAKE, 0, FAKE, None) == -13  # resid needs fp32 y
    assert lib.q4d_gemm(ctypes.byref(w), FAKE, 0, FAKE, 1, None, None) == -11
    assert lib.q4d_gemm(ctypes.byref(w), FAKE + 2, 4, FAKE, 1, None, None) == -4


def test_gemm_splitk_validation_codes(lib):
    w = Q4dMatrix(FAKE, FAKE, 1024, 2048)
    args = dict(x=FAKE, M=64, y=FAKE, dt=1, resid=None, part=FAKE, nbytes=64 * 1024 * 16 * 4, ks=16)

    def call(**kw):
        a = dict(args, **kw)
        return lib.q4d_gemm_splitk(ctypes.byref(w), a["x"], a["M"], a["y"], a["dt"], a["resid"], a["part"],
                                   a["nbytes"], a["ks"], None)
    assert call(part=None) == -7
    assert call(ks=17) == -11            # more than 16 splits
    assert call(ks=-1) == -11
    assert call(nbytes=64 * 1024 * 15 * 4) == -9   # 16 split tiles do not fit
    assert call(part=FAKE + 4) == -4     # 16-byte aligned tiles
    assert call(dt=0, resid=FAKE) == -13


def test_integer_gemv_validation_codes(lib):
    w = Q4dMatrix(FAKE, FAKE, 3072, 1024)
    assert lib.q4d_linear_q26(ctypes.byref(w), FAKE, None, None, None, None) == -7   # no output
    assert lib.q4d_linear_q26(ctypes.byref(w), None, FAKE, None, None, None) == -7
    assert lib.q4d_linear_q26(ctypes.byref(Q4dMatrix(FAKE, FAKE, 8, 1000)), FAKE, FAKE, None, None, None) == -11
    assert lib.q4d_linear_q26(ctypes.byref(Q4dMatrix(FAKE, FAKE, 8, 4096)), FAKE, FAKE, None, None, None) == -11
    assert lib.q4d_linear_q26(ctypes.byref(w), FAKE + 4, FAKE, None, None, None) == -4  # 16-byte activations
    assert lib.q4d_linear_q26(ctypes.byref(w), FAKE, FAKE + 4, None, None, None) == -4  # 8-byte int64 outputs
    assert lib.q4d_argmax_q26(FAKE, 0, FAKE, FAKE, None) == -11
    assert lib.q4d_argmax_q26(None, 5, FAKE, FAKE, None) == -7
    assert lib.q4d_argmax_q26(FAKE + 4, 5, FAKE, FAKE, None) == -4


def test_prefill_validation_codes(lib):
    arr = _layers(2)
    m = _model(arr)
    kv = Q4dKVCache(data=FAKE, num_layers=2, batch=2, num_kv_heads=8, max_ctx=512, head_dim=128)
    need = lib.q4d_prefill_workspace_bytes(ctypes.byref(m), 64)
    assert need > lib.q4d_workspace_bytes(ctypes.byref(m), 1)
    assert lib.q4d_prefill_workspace_bytes(ctypes.byref(m), 128) > need
    assert lib.q4d_prefill_workspace_bytes(ctypes.byref(m), 0) == 0
    assert lib.q4d_prefill_workspace_bytes(None, 64) == 0

    def prefill(n=64, start=0, seq=0, ws=FAKE, nbytes=need, tokens=FAKE, model=m, cache=kv):
        return lib.q4d_prefill(ctypes.byref(model), tokens, n, start, seq, ctypes.byref(cache), FAKE, FAKE, None, ws,
                               nbytes, None)
    assert prefill(tokens=None) == -7
    assert prefill(ws=None) == -7
    assert prefill(n=0) == -11
    assert prefill(start=500, n=13) == -10   # 500 + 13 > max_ctx 512
    assert prefill(start=-1) == -10
    assert prefill(seq=2) == -9              # the cache holds sequences 0 and 1
    assert prefill(nbytes=need - 1) == -9
    assert prefill(n=65) == -9               # the workspace was sized for 64 tokens
    assert prefill(ws=FAKE + 64) == -4       # workspace must be 256-byte aligned
    kv_bad = Q4dKVCache(data=FAKE, num_layers=2, batch=2, num_kv_heads=8, max_ctx=256, head_dim=128)
    assert prefill(cache=kv_bad) == -11
    arr[0].q_proj = Q4dMatrix(FAKE, FAKE, 2048, 512)
    assert prefill(model=_model(arr)) == -2


def test_activation_precision_setter(lib):
    assert lib.q4d_set_activation_precision(3) == -13
    assert lib.q4d_set_activation_precision(2) == 0


def test_noalloc_step_rejects_models_beyond_its_scratch(lib):
    """q4d_run_one_token_noalloc validates on the host before it touches the device:
    a model whose batch-1 workspace exceeds the 4 MiB scratch (Qwen3-0.6B shapes past
    27328 positions) is refused with Q4D_ERR_CAPACITY; missing pointers with NULL."""
    arr = _layers()
    big = _model(arr, max_ctx=27329)
    assert lib.q4d_workspace_bytes(ctypes.byref(big), 1) > 4 << 20
    kv = Q4dKVCache(FAKE, 1, 1, 8, 27329, 128)
    assert lib.q4d_run_one_token_noalloc(ctypes.byref(big), FAKE, FAKE, ctypes.byref(kv), FAKE, FAKE, None, FAKE,
                                         None) == -9
    ok = _model(arr, max_ctx=27328)
    assert lib.q4d_workspace_bytes(ctypes.byref(ok), 1) <= 4 << 20
    kv2 = Q4dKVCache(FAKE, 1, 1, 8, 27328, 128)
    assert lib.q4d_run_one_token_noalloc(ctypes.byref(ok), FAKE, FAKE, ctypes.byref(kv2), FAKE, FAKE, None, None,
                                         None) == -7


def test_feedback_step_validates_on_host(lib):
    """q4d_run_one_token_feedback fails closed before any launch: missing token,
    position or output pointers, a history without its count, a negative history
    capacity, a cache of the wrong batch or a short workspace."""
    arr = _layers()
    m = _model(arr)
    kv = Q4dKVCache(FAKE, 1, 1, 8, 512, 128)
    ws_bytes = lib.q4d_workspace_bytes(ctypes.byref(m), 1)
    f = lib.q4d_run_one_token_feedback

    def call(tok=FAKE, pos=FAKE, nxt=FAKE, score=FAKE, ht=None, hc=None, cap=0, kvd=kv, wsb=ws_bytes):
        return f(ctypes.byref(m), tok, pos, ctypes.byref(kvd), nxt, score, None, ht, None, hc, cap, FAKE, wsb, None)

    assert call(tok=None) == -7 and call(pos=None) == -7 and call(nxt=None) == -7 and call(score=None) == -7
    assert call(ht=FAKE, hc=None, cap=4) == -7
    assert call(ht=FAKE, hc=FAKE, cap=-1) == -7
    assert call(kvd=Q4dKVCache(FAKE, 1, 2, 8, 512, 128)) == -9
    assert call(wsb=ws_bytes - 1) == -9


def test_launch_chain_validates_on_host(lib):
    """q4d_diag_launch_chain (the launch-floor probe) rejects a missing array or buffer,
    a chain length outside 1..4096, a grid outside 1..65535, a block that is not a
    multiple of 64 up to 1024, and an unaligned buffer, before any launch."""
    f = lib.q4d_diag_launch_chain

    def arr(*v):
        a = (ctypes.c_int32 * len(v))(*v)
        return ctypes.cast(a, ctypes.c_void_p), a

    gx, _kx = arr(4, 4)
    gy, _ky = arr(1, 1)
    bl, _kb = arr(256, 256)
    assert f(None, gy, bl, 2, FAKE, None) == -7
    assert f(gx, gy, bl, 2, None, None) == -7
    assert f(gx, gy, bl, 0, FAKE, None) == -11
    assert f(gx, gy, bl, 4097, FAKE, None) == -11
    assert f(gx, gy, bl, 2, FAKE + 4, None) == -4
    for bad_gx, bad_gy, bad_bl in (((0, 4), (1, 1), (256, 256)), ((4, 65536), (1, 1), (256, 256)),
                                   ((4, 4), (1, 0), (256, 256)), ((4, 4), (1, 1), (256, 96)),
                                   ((4, 4), (1, 1), (2048, 256))):
        x, _a = arr(*bad_gx)
        y, _b = arr(*bad_gy)
        b, _c = arr(*bad_bl)
        assert f(x, y, b, 2, FAKE, None) == -11, (bad_gx, bad_gy, bad_bl)


def test_quantize_batch_validates_on_host(lib):
    """q4d_quantize_q4_batch rejects bad arguments before any launch."""
    f = lib.q4d_quantize_q4_batch
    arr = lambda *v: (ctypes.c_void_p * len(v))(*v)  # noqa: E731
    good = arr(FAKE, FAKE + 4096)
    # count, shapes, dtype
    assert f(good, 2, 1024, 4, 1024, 0, good, good, FAKE, None) == -11
    assert f(good, 2, 1024, 4, 1000, 2, good, good, FAKE, None) == -11   # cols % 64
    assert f(good, 2, 512, 4, 1024, 2, good, good, FAKE, None) == -11    # ld < cols
    assert f(good, 5, 1024, 4, 1024, 2, good, good, FAKE, None) == -13
    # null arrays or entries, misaligned matrices or outputs
    assert f(None, 2, 1024, 4, 1024, 2, good, good, FAKE, None) == -7
    assert f(good, 2, 1024, 4, 1024, 2, good, good, None, None) == -7
    assert f(arr(FAKE, None), 2, 1024, 4, 1024, 2, good, good, FAKE, None) == -7
    assert f(arr(FAKE, FAKE + 8), 2, 1024, 4, 1024, 2, good, good, FAKE, None) == -4
    assert f(good, 2, 1024, 4, 1024, 2, arr(FAKE, FAKE + 4), good, FAKE, None) == -4
    assert f(good, 2, 1028, 4, 1024, 2, good, good, FAKE, None) == -4    # rows not 16-byte aligned


def test_linear_group_validates_on_host(lib):
    """q4d_linear_group rejects bad arguments before any launch."""
    f = lib.q4d_linear_group
    ptrs = (ctypes.c_void_p * 2)(FAKE, FAKE + 4096)
    mats = (Q4dMatrix * 2)(Q4dMatrix(FAKE, FAKE, 256, 1024), Q4dMatrix(FAKE, FAKE, 256, 1024))
    assert f(mats, ptrs, 1, ptrs, 1, 1, 0, None) == -11        # count
    assert f(mats, ptrs, 1, ptrs, 1, 0, 2, None) == -11        # batch
    assert f(mats, ptrs, 7, ptrs, 1, 1, 2, None) == -13        # x dtype
    assert f(None, ptrs, 1, ptrs, 1, 1, 2, None) == -7
    odd = (Q4dMatrix * 2)(Q4dMatrix(FAKE, FAKE, 256, 1024), Q4dMatrix(FAKE, FAKE, 258, 1024))
    assert f(odd, ptrs, 1, ptrs, 1, 1, 2, None) == -3          # shapes differ
    bad = (Q4dMatrix * 2)(Q4dMatrix(FAKE, FAKE, 256, 1000), Q4dMatrix(FAKE, FAKE, 256, 1000))
    assert f(bad, ptrs, 1, ptrs, 1, 1, 2, None) == -11         # K not 1024 / 2048 / 3072
    assert f(mats, (ctypes.c_void_p * 2)(FAKE, FAKE + 8), 1, ptrs, 1, 1, 2, None) == -4   # x alignment
    assert f(mats, (ctypes.c_void_p * 2)(FAKE, None), 1, ptrs, 1, 1, 2, None) == -7


def test_linear_group_checks_every_matrix_before_the_first_launch(lib):
    """A bad entry past the first launch's 64 matrices is reported before anything runs
    (without a GPU, a launch would fail with a HIP error instead)."""
    f = lib.q4d_linear_group
    n = 70
    good = Q4dMatrix(FAKE, FAKE, 256, 1024)
    ptrs = (ctypes.c_void_p * n)(*[FAKE + 4096 * i for i in range(n)])
    mats = (Q4dMatrix * n)(*([good] * (n - 1) + [Q4dMatrix(FAKE, FAKE, 258, 1024)]))
    assert f(mats, ptrs, 1, ptrs, 1, 1, n, None) == -3          # shape of matrix 69
    mats = (Q4dMatrix * n)(*([good] * n))
    ys = (ctypes.c_void_p * n)(*([FAKE] * (n - 1) + [None]))
    assert f(mats, ptrs, 1, ys, 1, 1, n, None) == -7            # y[69]
    xs = (ctypes.c_void_p * n)(*([FAKE] * (n - 1) + [FAKE + 8]))
    assert f(mats, xs, 1, ptrs, 1, 1, n, None) == -4            # x[69] alignment
