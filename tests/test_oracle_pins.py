"""Pin the oracle's float path and Q4 helpers against closed forms, invariants
and independent implementations (torch / transformers), so a dropped term,
a wrong sign or index, or a transposed operand fails here."""

import numpy as np
import pytest
import torch

import oracle as o


# ---------------------------------------------------------------- int4 format
def test_unpack_all_byte_values_closed_form():
    b = np.arange(256, dtype=np.uint8).reshape(1, 256)
    q = o.unpack_signed_int4(b, 512)[0]
    lo, hi = q[0::2].astype(int), q[1::2].astype(int)
    for v in range(256):
        n0, n1 = v & 0xF, v >> 4
        assert lo[v] == (n0 - 16 if n0 >= 8 else n0)
        assert hi[v] == (n1 - 16 if n1 >= 8 else n1)


def test_q4_format_examples():
    """Source/Q4_FORMAT.md:120-128: 0->0x0, 7->0x7, -1->0xF, -8->0x8, even index low nibble."""
    q = np.array([[0, 7, -1, -8]], dtype=np.int8)
    p = o.pack_signed_int4(q)
    assert p.tolist() == [[0x70, 0x8F]]
    np.testing.assert_array_equal(o.unpack_signed_int4(p, 4), q)


def test_pack_unpack_round_trip_random():
    rng = np.random.default_rng(0)
    q = rng.integers(-8, 8, size=(37, 256)).astype(np.int8)
    np.testing.assert_array_equal(o.unpack_signed_int4(o.pack_signed_int4(q), 256), q)
    with pytest.raises(ValueError):
        o.pack_signed_int4(np.array([[8, 0]]))


def test_scale_rule_half_even_and_nonzero():
    raw = np.array([0.0, 0.25, 0.5, 1.5, 2.5, 1000.4], dtype=np.float32) / np.float32(16384)
    # rint: 0, 0 (->1 nonzero), 0 (half-even -> 0 -> 1 nonzero), 2, 2, 1000
    assert o.scale_q2_14_from_float(raw).tolist() == [0, 1, 1, 2, 2, 1000]
    with pytest.raises(ValueError):
        o.scale_q2_14_from_float(np.array([4.0], dtype=np.float32))


def test_quantize_dequantize_error_bound():
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.02, size=(64, 1024)).astype(np.float32)
    packed, scale, q = o.quantize_weight_q4(w)
    wd = o.dequantize_q4(packed, scale, dtype=np.float64)
    s = np.repeat(scale.astype(np.float64) / 16384, 64, axis=1)
    assert np.all(np.abs(wd - w) <= 0.5 * s + 1e-12)
    assert np.array_equal(o.unpack_signed_int4(packed, 1024), q)


def test_swapped_nibble_mistake_is_caught(golden):
    """A plausible mistake planted in the oracle (nibble order swapped) must
    fail the reference fixture, showing the fixture discriminates."""
    d = golden("q4_gemv_projection_1024_real")
    good = o.unpack_signed_int4(d["weight_packed"], 1024)
    bad = good.reshape(16, 512, 2)[:, :, ::-1].reshape(16, 1024)
    assert not np.array_equal(o.q4_gemv_q26(d["activation"], bad, d["scale_q2_14"]), d["expected_q26"])
    # and a sign mistake (unsigned nibbles)
    uns = np.where(good < 0, good + 16, good)
    assert not np.array_equal(o.q4_gemv_q26(d["activation"], uns, d["scale_q2_14"]), d["expected_q26"])


# ---------------------------------------------------------------- argmax rule
def test_argmax_first_equals_literal_strict_greater_scan():
    rng = np.random.default_rng(2)
    for _ in range(50):
        s = rng.integers(-3, 4, size=rng.integers(1, 300))
        best_i, best = 0, s[0]
        for i in range(1, len(s)):
            if s[i] > best:
                best_i, best = i, s[i]
        assert o.argmax_first(s) == (best_i, best)


def test_streamed_argmax_lowest_index_across_chunks():
    rng = np.random.default_rng(3)
    q = rng.integers(-8, 8, size=(300, 64)).astype(np.int8)
    q[250] = q[17]  # identical rows -> identical logits
    scale = rng.integers(1, 200, size=(300, 1)).astype(np.uint16)
    scale[250] = scale[17] = 60000
    x = rng.integers(-100, 100, size=64)
    x = x * np.sign(q[17]).astype(np.int64)  # make row 17 large
    tok, score, logits = o.lm_head_streamed_argmax_q26(x, q, scale, chunk_rows=64)
    assert logits[17] == logits[250] == logits.max()
    assert tok == 17


# ---------------------------------------------------------------- float path
def test_rms_norm_matches_torch_and_invariants():
    rng = np.random.default_rng(4)
    x = rng.normal(0, 3, size=(5, 1024)).astype(np.float32)
    g = (1 + rng.normal(0, 0.1, 1024)).astype(np.float32)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x), (1024,), torch.from_numpy(g), eps=1e-6).numpy()
    got = o.manual_rms_norm(x, g, 1e-6)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)
    # scale invariance and unit RMS with gamma = 1
    np.testing.assert_allclose(o.manual_rms_norm(7.0 * x, g, 0.0), o.manual_rms_norm(x, g, 0.0), rtol=1e-5)
    u = o.manual_rms_norm(x, np.ones(1024, np.float32), 0.0, dtype=np.float64)
    np.testing.assert_allclose(np.sqrt(np.mean(u * u, axis=-1)), 1.0, rtol=1e-12)


def _hf_config(layers=2, vocab=1024):
    from transformers import Qwen3Config
    return Qwen3Config(hidden_size=1024, intermediate_size=3072, num_hidden_layers=layers, num_attention_heads=16,
                       num_key_value_heads=8, head_dim=128, rms_norm_eps=1e-6, rope_theta=1_000_000.0,
                       vocab_size=vocab, tie_word_embeddings=True, max_position_embeddings=32768,
                       attention_bias=False, attn_implementation="eager", torch_dtype=torch.float32)


def test_rope_matches_transformers_qwen3():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RotaryEmbedding, apply_rotary_pos_emb
    cfg = _hf_config()
    rot = Qwen3RotaryEmbedding(cfg)
    inv = o.rope_inv_freq(1_000_000.0, 128)
    np.testing.assert_array_equal(inv, rot.inv_freq.numpy())
    pos = np.array([[0, 1, 7, 511, 512, 4095]])
    x = torch.zeros(1, 6, 1024)
    c_ref, s_ref = rot(x, torch.from_numpy(pos))
    c, s = o.manual_rope_cos_sin(inv, pos)
    np.testing.assert_allclose(c, c_ref.numpy(), rtol=0, atol=2e-6)
    np.testing.assert_allclose(s, s_ref.numpy(), rtol=0, atol=2e-6)
    rng = np.random.default_rng(5)
    q = rng.normal(size=(1, 16, 6, 128)).astype(np.float32)
    k = rng.normal(size=(1, 8, 6, 128)).astype(np.float32)
    qr, kr = o.manual_apply_rope(q, k, c, s)
    qh, kh = apply_rotary_pos_emb(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(c),
                                  torch.from_numpy(s))
    np.testing.assert_allclose(qr, qh.numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(kr, kh.numpy(), rtol=1e-6, atol=1e-6)


def test_rope_invariants():
    inv = o.rope_inv_freq(1_000_000.0, 128).astype(np.float64)
    rng = np.random.default_rng(6)
    q = rng.normal(size=(1, 1, 1, 128))
    k = rng.normal(size=(1, 1, 1, 128))

    def rope(x, p):
        f = p * inv
        c = np.cos(np.concatenate([f, f]))[None, None, :]
        s = np.sin(np.concatenate([f, f]))[None, None, :]
        return o.manual_apply_rope(x, x, c, s)[0]
    # rotation preserves the norm of every (d, d+64) pair
    r = rope(q, 37)
    np.testing.assert_allclose(r[..., :64] ** 2 + r[..., 64:] ** 2, q[..., :64] ** 2 + q[..., 64:] ** 2, rtol=1e-12)
    # scores depend only on the position difference
    a = np.sum(rope(q, 100) * rope(k, 40))
    b = np.sum(rope(q, 1060) * rope(k, 1000))
    np.testing.assert_allclose(a, b, rtol=1e-9)


def test_attention_matches_torch_sdpa_gqa():
    rng = np.random.default_rng(7)
    q = rng.normal(size=(2, 16, 1, 128))
    k = rng.normal(size=(2, 8, 33, 128))
    v = rng.normal(size=(2, 8, 33, 128))
    out, w = o.manual_cached_attention(q, o.manual_repeat_kv(k, 2), o.manual_repeat_kv(v, 2), 128 ** -0.5)
    ref = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                                           torch.from_numpy(v), scale=128 ** -0.5, enable_gqa=True)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-12)
    # q head h uses kv head h // 2: swapping kv heads 0 and 1 makes q heads 0, 1
    # attend to the old kv head 1 (and heads 2, 3 to the old kv head 0)
    perm = np.array([1, 0, 2, 3, 4, 5, 6, 7])
    out2, _ = o.manual_cached_attention(q, o.manual_repeat_kv(k[:, perm], 2), o.manual_repeat_kv(v[:, perm], 2),
                                        128 ** -0.5)
    for h, kvh in ((0, 1), (1, 1), (2, 0), (3, 0), (4, 2)):
        single = o.manual_cached_attention(q[:, h:h + 1], k[:, kvh:kvh + 1], v[:, kvh:kvh + 1], 128 ** -0.5)[0]
        np.testing.assert_allclose(out2[:, h], single[:, 0], rtol=1e-12, atol=1e-14)


def _causal_vs_sdpa(q, k, v, scale):
    out, w = o.manual_causal_attention(q, o.manual_repeat_kv(k, q.shape[1] // k.shape[1]),
                                       o.manual_repeat_kv(v, q.shape[1] // k.shape[1]), scale)
    ref = torch.nn.functional.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k),
                                                           torch.from_numpy(v), is_causal=True, scale=scale,
                                                           enable_gqa=True)
    return out, w, ref.numpy()


def test_causal_attention_matches_sdpa_and_the_cached_prefixes():
    """manual_causal_attention (common.py:201-216) against torch's causal SDPA with GQA,
    and row i against manual_cached_attention over keys 0..i (the serial prompt loop
    sees exactly those keys at step i)."""
    rng = np.random.default_rng(17)
    for b, qh, kvh, s in ((1, 16, 8, 37), (2, 4, 1, 5), (1, 2, 2, 1)):
        q = rng.normal(size=(b, qh, s, 128))
        k = rng.normal(size=(b, kvh, s, 128))
        v = rng.normal(size=(b, kvh, s, 128))
        out, w, ref = _causal_vs_sdpa(q, k, v, 128 ** -0.5)
        np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
        np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-12)
        assert np.all(np.triu(w[0, 0], k=1) == 0)
        rep = qh // kvh
        for i in range(s):
            cached, _ = o.manual_cached_attention(q[:, :, i:i + 1], o.manual_repeat_kv(k[:, :, :i + 1], rep),
                                                  o.manual_repeat_kv(v[:, :, :i + 1], rep), 128 ** -0.5)
            np.testing.assert_allclose(out[:, :, i:i + 1], cached, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("offset", [0, 2])
def test_causal_attention_planted_mask_errors_fail(monkeypatch, offset):
    """A mask that hides the query's own key (offset 0) or shows the next key
    (offset 2) in the oracle no longer matches the causal SDPA."""
    import oracle.q4_oracle as qo

    class _Np:
        def __getattr__(self, name):
            return getattr(np, name)

        @staticmethod
        def triu(m, k=0):
            return np.triu(m, k=offset)
    monkeypatch.setattr(qo, "np", _Np())
    rng = np.random.default_rng(18)
    q, k, v = (rng.normal(size=(1, 2, 9, 128)) for _ in range(3))
    out, _, ref = _causal_vs_sdpa(q, k, v, 128 ** -0.5)
    assert not np.allclose(out, ref, rtol=1e-6, atol=1e-8)


def _small_q4_model(layers=2, vocab=1024, seed=11):
    from llm_accelerator_amd.model import Qwen3Config, random_host_weights
    cfg = Qwen3Config(num_hidden_layers=layers, vocab_size=vocab)
    host = random_host_weights(cfg, seed=seed)
    ocfg = o.OracleConfig(num_hidden_layers=layers, vocab_size=vocab)
    om = o.OracleModel.from_q4(ocfg, host["layers"], *host["embed_tokens"], host["norm"])
    return host, om


def _hf_model_from(host, layers, vocab):
    from transformers import Qwen3ForCausalLM
    hf = Qwen3ForCausalLM(_hf_config(layers, vocab)).eval()
    mats = ("q_proj", "k_proj", "v_proj", "o_proj")
    with torch.no_grad():
        for L, hl in zip(host["layers"], hf.model.layers):
            for n in mats:
                getattr(hl.self_attn, n).weight.copy_(torch.from_numpy(o.dequantize_q4(*L[n])))
            for n in ("gate_proj", "up_proj", "down_proj"):
                getattr(hl.mlp, n).weight.copy_(torch.from_numpy(o.dequantize_q4(*L[n])))
            hl.input_layernorm.weight.copy_(torch.from_numpy(L["input_layernorm"]))
            hl.post_attention_layernorm.weight.copy_(torch.from_numpy(L["post_attention_layernorm"]))
            hl.self_attn.q_norm.weight.copy_(torch.from_numpy(L["q_norm"]))
            hl.self_attn.k_norm.weight.copy_(torch.from_numpy(L["k_norm"]))
        hf.model.embed_tokens.weight.copy_(torch.from_numpy(o.dequantize_q4(*host["embed_tokens"])))
        hf.model.norm.weight.copy_(torch.from_numpy(host["norm"]))
    return hf


def test_decode_composition_matches_transformers_qwen3():
    """The reference validates its manual decode against HF eager fp32 at
    atol=rtol=1e-5 (10_validate_full_run_one_token.py:81-172); do the same for
    the oracle, on seeded random Q4 weights, over serial positions + feedback."""
    layers, vocab = 2, 1024
    host, om = _small_q4_model(layers, vocab)
    hf = _hf_model_from(host, layers, vocab)
    assert hf.lm_head.weight.data_ptr() == hf.model.embed_tokens.weight.data_ptr()
    kc, vc = [None] * layers, [None] * layers
    past = None
    toks = [5, 900, 17, 3]
    with torch.no_grad():
        for pos, t in enumerate(toks):
            out = hf(input_ids=torch.tensor([[t]]), past_key_values=past, use_cache=True)
            past = out.past_key_values
            logits, nxt = o.run_manual_one_token(np.array([[t]]), pos, om, kc, vc)
            ref = out.logits.numpy()
            scale = np.max(np.abs(ref))
            assert np.max(np.abs(logits - ref)) <= 2e-5 * scale, (pos, np.max(np.abs(logits - ref)), scale)
            assert int(nxt[0, 0]) == int(np.argmax(ref[0, -1]))
        # caches of every layer agree (K after norm+RoPE, V raw)
        for li in range(layers):
            hk = past.layers[li].keys.numpy()
            hv = past.layers[li].values.numpy()
            np.testing.assert_allclose(kc[li], hk, rtol=1e-4, atol=1e-4 * np.abs(hk).max())
            np.testing.assert_allclose(vc[li], hv, rtol=1e-4, atol=1e-4 * np.abs(hv).max())


def test_greedy_decode_teacher_forcing_identity():
    """Forcing the oracle's own tokens reproduces its free-running trajectory."""
    host, om = _small_q4_model(1, 512, seed=12)
    gen, gaps, _ = o.greedy_decode(om, [1, 2, 3], 6)
    gen2, _, _ = o.greedy_decode(om, [1, 2, 3], 6, forced=gen[:-1])
    assert gen == gen2 and len(gaps) == 6 and min(gaps) >= 0


def test_all_positions_prompt_equals_serial_loop_and_transformers():
    """serial_prompt_all_at_once (the serial prompt loop of
    10_validate_full_run_one_token.py:81-135 evaluated for every position at once)
    against (a) the oracle's own one-token loop in fp64, every position's logits and
    every cache row, and (b) transformers' Qwen3ForCausalLM run over the whole prompt
    with its causal mask (fp32, the reference's 1e-5 class bar).  Planted mask
    mistakes (a query that misses its own key, or sees the next one) fail (a)."""
    layers, vocab = 2, 1024
    host, om32 = _small_q4_model(layers, vocab)
    om64 = o.OracleModel.from_q4(o.OracleConfig(num_hidden_layers=layers, vocab_size=vocab), host["layers"],
                                 *host["embed_tokens"], host["norm"], dtype=np.float64)
    for n in (1, 5, 37):
        toks = np.random.default_rng(n).integers(0, vocab, n).tolist()
        kc, vc = [None] * layers, [None] * layers
        serial = []
        for pos, t in enumerate(toks):
            lg, _ = o.run_manual_one_token(np.array([[t]]), pos, om64, kc, vc)
            serial.append(lg[0, 0])
        serial = np.stack(serial)
        allpos, ak, av = o.serial_prompt_all_at_once(om64, toks)
        assert allpos.shape == (n, vocab)
        np.testing.assert_allclose(allpos, serial, rtol=0, atol=1e-11 * np.abs(serial).max())
        for li in range(layers):
            np.testing.assert_allclose(ak[li], kc[li], rtol=0, atol=1e-12 * np.abs(kc[li]).max())
            np.testing.assert_allclose(av[li], vc[li], rtol=0, atol=1e-12 * np.abs(vc[li]).max())
        if n > 1:
            for bad in (0, 2):
                wrong, _, _ = o.serial_prompt_all_at_once(om64, toks, _future_offset=bad)
                assert not np.allclose(wrong, serial, rtol=0, atol=1e-3 * np.abs(serial).max()), bad  # NaN counts as wrong
    hf = _hf_model_from(host, layers, vocab)
    toks = np.random.default_rng(3).integers(0, vocab, 23).tolist()
    with torch.no_grad():
        out = hf(input_ids=torch.tensor([toks]), use_cache=True)
    ref = out.logits.numpy()[0]
    got, ak, av = o.serial_prompt_all_at_once(om32, toks)
    assert np.max(np.abs(got - ref)) <= 2e-5 * np.abs(ref).max()
    for li in range(layers):
        hk = out.past_key_values.layers[li].keys.numpy()
        np.testing.assert_allclose(ak[li], hk, rtol=1e-4, atol=1e-4 * np.abs(hk).max())
