"""CPU-side checks of the fixed-point (RTL-exact) path: the library's host-built
LUTs and the host RoPE table against the reference's vectors, and host
validation of every q4d_fixed_* entry point (negative codes, no launch)."""

import ctypes

import numpy as np
import pytest

import oracle as o
from oracle import q4_fixed as F
from llm_accelerator_amd import _lib
from llm_accelerator_amd import fixed as X
from llm_accelerator_amd._lib import Q4dFixedKV, Q4dFixedLayer, Q4dFixedModel, Q4dLayer, Q4dMatrix, Q4dModel
from llm_accelerator_amd.model import Qwen3Config

FAKE = 0x7F0000000000  # aligned, never dereferenced: validation fails before launch


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("libq4dec.so is not built: run `python -m llm_accelerator_amd.build`")
    return _lib.load()


def test_library_luts_match_reference_vectors(golden):
    e, s = X.build_exp_lut(), X.build_sigmoid_lut()
    for name in ("fixed_attention_l0", "fixed_attention_l1", "fixed_attention_l2c"):
        np.testing.assert_array_equal(e, golden(name)["exp_lut"])
    for tag in ("l0", "l1c", "l2c"):
        np.testing.assert_array_equal(s, golden(f"fixed_silu_mul_{tag}")["sigmoid_lut"])
    assert e[0] == 1 << 20 and s[512] == 32768 and s[-1] == 65514


def test_rope_table_matches_reference_and_oracle(golden):
    cos, sin = X.rope_table_q1_15(Qwen3Config(), 1024)
    for name in ("fixed_qk_norm_rope_l0", "fixed_qk_norm_rope_l2c", "fixed_rope_qk_l0"):
        np.testing.assert_array_equal(cos[4], golden(name)["cos"])
        np.testing.assert_array_equal(sin[4], golden(name)["sin"])
    oc, os_ = F.rope_table_q1_15(o.rope_inv_freq(1_000_000.0, 128), np.arange(1024))
    np.testing.assert_array_equal(cos, oc)
    np.testing.assert_array_equal(sin, os_)
    assert X.score_scale_q0_31(128 ** -0.5) == 189812531


def test_tables_entry_validation(lib):
    e = np.zeros(257, np.int32)
    s = np.zeros(1025, np.int32)
    assert lib.q4d_fixed_tables(None, 257, s.ctypes.data, 1025) == -7
    assert lib.q4d_fixed_tables(e.ctypes.data, 256, s.ctypes.data, 1025) == -11
    assert lib.q4d_fixed_tables(e.ctypes.data, 257, s.ctypes.data, 1024) == -11


def _fixed_model(n_layers=2, max_ctx=256, **kw):
    layers = (Q4dLayer * n_layers)()
    for i in range(n_layers):
        L = layers[i]
        for name, (r, c) in dict(q_proj=(2048, 1024), k_proj=(1024, 1024), v_proj=(1024, 1024), o_proj=(1024, 2048),
                                 gate_proj=(3072, 1024), up_proj=(3072, 1024), down_proj=(1024, 3072)).items():
            setattr(L, name, Q4dMatrix(FAKE, FAKE, r, c))
    d = dict(hidden_size=1024, intermediate_size=3072, num_layers=n_layers, num_q_heads=16, num_kv_heads=8,
             head_dim=128, vocab_size=151936, max_ctx=max_ctx, rms_norm_eps=1e-6, attn_scaling=128 ** -0.5)
    d.update(kw)
    base = Q4dModel(**d)
    base.layers = ctypes.cast(layers, ctypes.POINTER(Q4dLayer))
    base.embed_tokens = Q4dMatrix(FAKE, FAKE, 151936, 1024)
    fl = (Q4dFixedLayer * n_layers)(*[Q4dFixedLayer(FAKE, FAKE, FAKE, FAKE) for _ in range(n_layers)])
    keep = (layers, base, fl)
    fm = Q4dFixedModel(ctypes.pointer(base), fl, FAKE, FAKE, FAKE, 189812531)
    return fm, keep


def test_fixed_model_validation(lib):
    fm, keep = _fixed_model()
    need = lib.q4d_fixed_workspace_bytes(ctypes.byref(fm))
    # counters, LUTs, hidden, q|k|v, attention, post, SwiGLU, per-block LM-head results
    assert need >= 16384 + 1280 + 4352 + 4096 + 16384 + 8192 + 4096 + 12288 + 4748 * 12
    kv = Q4dFixedKV(FAKE, 2, 8, 256, 128)

    def layer(model=fm, cache=kv, l=0, ws=FAKE, nbytes=need, hin=FAKE, pos=FAKE):
        return lib.q4d_fixed_decoder_layer(ctypes.byref(model), l, hin, FAKE, ctypes.byref(cache), pos, ws, nbytes,
                                           None)
    assert layer(hin=None) == -7
    assert layer(pos=None) == -7
    assert layer(l=2) == -2
    assert layer(l=-1) == -2
    assert layer(nbytes=need - 1) == -9
    assert layer(ws=FAKE + 64) == -4
    assert layer(hin=FAKE + 4) == -4
    assert layer(cache=Q4dFixedKV(FAKE, 2, 8, 512, 128)) == -11   # cache capacity differs from the model
    assert layer(cache=Q4dFixedKV(FAKE, 1, 8, 256, 128)) == -11
    assert layer(cache=Q4dFixedKV(None, 2, 8, 256, 128)) == -7
    big, keep2 = _fixed_model(max_ctx=8192)
    assert lib.q4d_fixed_workspace_bytes(ctypes.byref(big)) == 0   # more positions than one block holds
    assert layer(model=big) == -10
    bad = Q4dFixedModel(fm.base, fm.layers, None, FAKE, FAKE, 189812531)
    assert layer(model=bad) == -7
    bad = Q4dFixedModel(fm.base, fm.layers, FAKE, FAKE, FAKE, 0)
    assert layer(model=bad) == -11
    keep[0][1].o_proj = Q4dMatrix(FAKE, FAKE, 1024, 1024)            # o_proj must read 16 heads x 128
    assert layer(l=0) == -2
    keep[0][1].o_proj = Q4dMatrix(FAKE, FAKE, 1024, 2048)
    keep[2][1] = Q4dFixedLayer(FAKE, None, FAKE, FAKE)
    assert layer() == -7

    def token(model=fm, ws=FAKE, nbytes=need, score=FAKE, logits=None):
        return lib.q4d_fixed_run_one_token(ctypes.byref(model), FAKE, FAKE, ctypes.byref(kv), FAKE, score, logits,
                                           None, ws, nbytes, None)
    keep[2][1] = Q4dFixedLayer(FAKE, FAKE, FAKE, FAKE)
    assert token(score=None) == -7
    assert token(score=FAKE + 4) == -4
    assert token(logits=FAKE + 4) == -4
    assert token(nbytes=16) == -9
    assert lib.q4d_fixed_workspace_init(FAKE, 16, ctypes.byref(fm), None) == -9
    assert lib.q4d_fixed_read_counts(FAKE, 4096, FAKE, 17, None) == -11
    assert lib.q4d_fixed_read_counts(None, 4096, FAKE, 4, None) == -7


def test_stage_entry_validation(lib):
    kv = Q4dFixedKV(FAKE, 2, 8, 256, 128)
    assert lib.q4d_fixed_rms_norm(FAKE, FAKE, 1, 1024, 2, FAKE, None, None) == -11
    assert lib.q4d_fixed_rms_norm(FAKE, FAKE, 1, 128, 0, FAKE, None, None) == -11
    assert lib.q4d_fixed_rms_norm(FAKE, FAKE, 4, 1024, 1, FAKE, None, None) == -11
    assert lib.q4d_fixed_rms_norm(None, FAKE, 1, 1024, 0, FAKE, None, None) == -7
    assert lib.q4d_fixed_rms_norm(FAKE, FAKE, 1, 1024, 0, FAKE, FAKE + 4, None) == -4
    assert lib.q4d_fixed_qk_norm_rope(FAKE, FAKE, 16, 8, FAKE, None, FAKE, FAKE, FAKE, FAKE, None, None, None) == -7
    assert lib.q4d_fixed_qk_norm_rope(FAKE, FAKE, 0, 8, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, None, None) == -11

    need = lib.q4d_fixed_attention_workspace_bytes(16, 256)
    assert need >= 16 * 256 * 8 + 16 * 16 * 8 and lib.q4d_fixed_attention_workspace_bytes(16, 8192) == 0

    def att(cache=kv, layer=0, qh=16, t=5, scale=189812531, lut=FAKE, raw=None, ws=FAKE, nbytes=need):
        return lib.q4d_fixed_attention(ctypes.byref(cache), layer, qh, t, FAKE, scale, lut, FAKE, raw, None, None,
                                       None, ws, nbytes, None)
    assert att(ws=None) == -7
    assert att(ws=FAKE + 64) == -4
    assert att(nbytes=need - 1) == -9
    assert att(t=257) == -10
    assert att(t=0) == -10
    assert att(layer=2) == -2
    assert att(qh=12) == -11          # not a multiple of the 8 kv heads
    assert att(scale=0) == -11
    assert att(lut=None) == -7
    assert att(raw=FAKE + 4) == -4
    assert att(cache=Q4dFixedKV(FAKE, 2, 8, 8192, 128)) == -11
    assert lib.q4d_fixed_kv_append(ctypes.byref(kv), 2, FAKE, FAKE, FAKE, None) == -2
    assert lib.q4d_fixed_kv_append(ctypes.byref(kv), 0, None, FAKE, FAKE, None) == -7
    assert lib.q4d_fixed_silu_mul(FAKE, FAKE, 0, FAKE, FAKE, None, None, None, None) == -11
    assert lib.q4d_fixed_silu_mul(FAKE, FAKE, 8, None, FAKE, None, None, None, None) == -7
    assert lib.q4d_fixed_residual_add(FAKE, FAKE, 0, FAKE, None) == -11
    assert lib.q4d_fixed_embedding(ctypes.byref(Q4dMatrix(FAKE, FAKE, 10, 100)), FAKE, 1, FAKE, None) == -11
    m = lambda rows, cols, w=FAKE: ctypes.byref(Q4dMatrix(w, FAKE, rows, cols))  # noqa: E731
    assert lib.q4d_fixed_q4_gemv(m(16, 512), FAKE, None, FAKE, None) == -11       # K not 1024 / 2048 / 3072
    assert lib.q4d_fixed_q4_gemv(m(16, 2048), FAKE, FAKE, FAKE, None) == -11      # norm prologue needs K = 1024
    assert lib.q4d_fixed_q4_gemv(m(0, 1024), FAKE, None, FAKE, None) == -11
    assert lib.q4d_fixed_q4_gemv(m(16, 1024, None), FAKE, None, FAKE, None) == -7
    assert lib.q4d_fixed_q4_gemv(m(16, 1024), None, None, FAKE, None) == -7
    assert lib.q4d_fixed_q4_gemv(m(16, 1024, FAKE + 8), FAKE, None, FAKE, None) == -4
    assert lib.q4d_fixed_q4_gemv(m(16, 1024), FAKE + 4, None, FAKE, None) == -4
