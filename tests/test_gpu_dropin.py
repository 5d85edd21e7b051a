"""The prompt-shaped drop-in functions of llm_accelerator_amd.common against the
oracle: manual_rotate_half (common.py:148-152), manual_apply_rope over a whole
prompt (common.py:173-183, as 04_validate_qk_norm_rope.py:59-60 calls it) and
manual_causal_attention (common.py:201-216, as 06_validate_attention.py:71 calls
it), at one position, 37 positions and 2048 positions."""

import numpy as np
import pytest
import torch

import oracle as o
from llm_accelerator_amd import common
from llm_accelerator_amd.model import Qwen3Config, build_model, random_host_weights

from gpu_helpers import report

pytestmark = pytest.mark.gpu

LN2 = float(np.log(2.0))
LOG2E = 1.4426950408889634


@pytest.mark.parametrize("shape", [(1, 16, 1, 128), (1, 8, 37, 128), (2, 16, 2048, 128), (3, 5, 64)])
def test_rotate_half_exact(dev, shape):
    rng = np.random.default_rng(len(shape) + shape[-2])
    x = rng.normal(size=shape).astype(np.float32)
    got = common.manual_rotate_half(torch.from_numpy(x).to(dev)).cpu().numpy()
    assert np.array_equal(got, o.manual_rotate_half(x))


@pytest.mark.parametrize("seq", [1, 37, 2048])
def test_apply_rope_over_a_prompt(dev, seq):
    """q/k as the validator builds them: transposed views [B, H, S, D] of [B, S, H, D]
    projections, with cos/sin [1, S, D] from manual_rope_cos_sin over arange(S)."""
    rng = np.random.default_rng(seq)
    print(f"[rope] seq={seq}", flush=True)
    q = rng.normal(size=(1, seq, 16, 128)).astype(np.float32)
    k = rng.normal(size=(1, seq, 8, 128)).astype(np.float32)
    inv = o.rope_inv_freq(1_000_000.0, 128)
    cos, sin = o.manual_rope_cos_sin(inv, np.arange(seq)[None])
    qd = torch.from_numpy(q).to(dev).transpose(1, 2)
    kd = torch.from_numpy(k).to(dev).transpose(1, 2)
    gq, gk = common.manual_apply_rope(qd, kd, torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev))
    rq, rk = o.manual_apply_rope(np.swapaxes(q, 1, 2).astype(np.float64), np.swapaxes(k, 1, 2).astype(np.float64),
                                 cos.astype(np.float64), sin.astype(np.float64))
    for name, g, r in (("q", gq, rq), ("k", gk, rk)):
        g = g.cpu().numpy()
        assert g.shape == r.shape
        # two fp32 products and a sum, each within half an ulp of its value
        bound = 2.0 ** -23 * (np.abs(np.swapaxes(q if name == "q" else k, 1, 2)) * 2 + np.abs(r)) * 2
        report(f"rope {name} seq={seq}", g, r)
        assert np.all(np.abs(g - r) <= bound + 1e-30)


def test_apply_rope_tables_of_the_model(dev):
    """manual_rope_cos_sin of the device tables feeds manual_apply_rope at positions
    0..S-1 exactly like the oracle's RoPE (transformers' Qwen3 rotary pins the oracle)."""
    cfg = Qwen3Config(num_hidden_layers=1, vocab_size=2048)
    model = build_model(cfg, random_host_weights(cfg, seed=1, num_layers=1), max_ctx=2048, device=dev)
    seq = 300
    pos = torch.arange(seq, dtype=torch.long)[None]
    cos, sin = common.manual_rope_cos_sin(model.model.rotary_emb, None, pos)
    rc, rs = o.manual_rope_cos_sin(o.rope_inv_freq(1_000_000.0, 128), np.arange(seq)[None])
    assert cos.shape == (1, seq, 128)
    assert np.max(np.abs(cos.cpu().numpy() - rc)) < 2e-4  # fp32 angle rounding at positions < 300
    assert np.max(np.abs(sin.cpu().numpy() - rs)) < 2e-4


def _causal_inputs(rng, b, qh, kvh, s):
    q = rng.normal(size=(b, qh, s, 128)).astype(np.float32)
    k = rng.normal(size=(b, kvh, s, 128)).astype(np.float32)
    v = rng.normal(size=(b, kvh, s, 128)).astype(np.float32)
    return q, k, v


def _fp16_model_of_kernel(q, k, v, scale):
    """The arithmetic the kernel performs, in float64: q rounded to fp16 after the
    softmax scale and log2(e) are folded in, k and v rounded to fp16, probabilities
    2^(s - max).  Returns (output, weighted mean of |v|) per query."""
    rep = q.shape[1] // k.shape[1]
    mul = np.float32(np.float32(scale) * np.float32(LOG2E))  # the fp32 factor the host folds in
    q16 = (q.astype(np.float32) * mul).astype(np.float16).astype(np.float64)
    k16 = o.manual_repeat_kv(k.astype(np.float16).astype(np.float64), rep)
    v16 = o.manual_repeat_kv(v.astype(np.float16).astype(np.float64), rep)
    out, w = o.manual_causal_attention(q16, k16, v16, LN2)
    return out, w @ np.abs(v16)


@pytest.mark.parametrize("b,qh,kvh,s", [(1, 16, 8, 1), (1, 16, 8, 37), (1, 16, 8, 2048), (2, 4, 1, 100)])
def test_causal_attention_vs_oracle(dev, b, qh, kvh, s):
    rng = np.random.default_rng(s + qh)
    print(f"[causal] b={b} heads={qh}/{kvh} seq={s}", flush=True)
    q, k, v = _causal_inputs(rng, b, qh, kvh, s)
    scale = 128 ** -0.5
    kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    out, w = common.manual_causal_attention(torch.from_numpy(q).to(dev), common.manual_repeat_kv(kd, qh // kvh),
                                            common.manual_repeat_kv(vd, qh // kvh), scale)
    assert list(w.shape) == [b, qh, s, s]  # what 06_validate_attention.py prints
    got = out.cpu().numpy().astype(np.float64)
    # 1. the kernel's own arithmetic: fp16 probabilities (2^-11 relative each), fp32 sums
    #    and the fp16 output rounding bound the difference by 2^-9 of the weighted |v|
    ref16, wabs = _fp16_model_of_kernel(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), scale)
    report(f"causal vs fp16 operands s={s}", got, ref16)
    assert np.all(np.abs(got - ref16) <= 2.0 ** -9 * wabs + 1e-6)
    # 2. the reference function on the fp32 inputs (stated fp16 tolerance)
    rep = qh // kvh
    ref, _ = o.manual_causal_attention(q.astype(np.float64), o.manual_repeat_kv(k.astype(np.float64), rep),
                                       o.manual_repeat_kv(v.astype(np.float64), rep), scale)
    mx, rel = report(f"causal vs fp64 oracle s={s}", got, ref)
    assert np.all(np.abs(got - ref) <= 4e-3 * wabs + 1e-5)


def test_causal_attention_equal_kv_heads_and_errors(dev):
    """k/v given already repeated (a [B, H, S, D] tensor, repeat 1) equal the GQA call;
    shapes that do not fit raise."""
    rng = np.random.default_rng(5)
    q, k, v = _causal_inputs(rng, 1, 4, 2, 19)
    qd, kd, vd = (torch.from_numpy(a).to(dev) for a in (q, k, v))
    a, _ = common.manual_causal_attention(qd, common.manual_repeat_kv(kd, 2), common.manual_repeat_kv(vd, 2), 0.1)
    kr = torch.from_numpy(np.ascontiguousarray(o.manual_repeat_kv(k, 2))).to(dev)
    vr = torch.from_numpy(np.ascontiguousarray(o.manual_repeat_kv(v, 2))).to(dev)
    b, _ = common.manual_causal_attention(qd, kr, vr, 0.1)
    assert torch.equal(a, b)
    with pytest.raises(ValueError):
        common.manual_causal_attention(qd, kd, vd, 0.1)  # 2 kv heads without the repeat marker
    with pytest.raises(ValueError):
        common.manual_causal_attention(qd[:, :, :5], common.manual_repeat_kv(kd, 2), common.manual_repeat_kv(vd, 2), 0.1)


def test_validator_06_flow(dev):
    """06_validate_attention.py:48-73 with this package's functions on a random Q4
    layer over a 64-token prompt: q/k/v projections of the normed input, per-head
    RMSNorm, RoPE over the prompt, repeat_kv, causal attention, the concat that
    feeds o_proj; against the same chain of oracle functions in float64."""
    cfg = Qwen3Config(num_hidden_layers=1, vocab_size=2048)
    host = random_host_weights(cfg, seed=6, num_layers=1)
    model = build_model(cfg, host, max_ctx=128, device=dev)
    om = o.OracleModel.from_q4(o.OracleConfig(num_hidden_layers=1, vocab_size=2048), host["layers"],
                               *host["embed_tokens"], host["norm"], dtype=np.float64)
    L, OL = model.model.layers[0], om.layers[0]
    attn0 = L.self_attn
    rng = np.random.default_rng(60)
    S = 64
    input_norm_np = rng.normal(size=(1, S, 1024)).astype(np.float32)
    input_norm = torch.from_numpy(input_norm_np).to(dev)
    position_ids = torch.arange(S, dtype=torch.long).unsqueeze(0)
    eps = common.get_rms_norm_eps(L.input_layernorm, cfg)

    q_flat = common.manual_linear_from_weight(input_norm, attn0.q_proj.weight)
    k_flat = common.manual_linear_from_weight(input_norm, attn0.k_proj.weight)
    v_flat = common.manual_linear_from_weight(input_norm, attn0.v_proj.weight)
    q_view = q_flat.view(1, S, 16, 128)
    k_view = k_flat.view(1, S, 8, 128)
    v_view = v_flat.view(1, S, 8, 128)
    q_norm = common.manual_rms_norm(q_view, attn0.q_norm.weight, eps)
    k_norm = common.manual_rms_norm(k_view, attn0.k_norm.weight, eps)
    cos, sin = common.manual_rope_cos_sin(model.model.rotary_emb, input_norm, position_ids)
    q_rope, k_rope = common.manual_apply_rope(q_norm.transpose(1, 2), k_norm.transpose(1, 2), cos, sin)
    heads, weights = common.manual_causal_attention(q_rope, common.manual_repeat_kv(k_rope, 2),
                                                    common.manual_repeat_kv(v_view.transpose(1, 2), 2),
                                                    float(attn0.scaling))
    concat = heads.transpose(1, 2).contiguous().reshape(1, S, -1).cpu().numpy()
    assert list(weights.shape) == [1, 16, S, S]

    x = input_norm_np.astype(np.float64)
    qn = o.manual_rms_norm(o.manual_linear_from_weight(x, OL.q_proj, dtype=np.float64).reshape(1, S, 16, 128),
                           OL.q_norm, eps, np.float64)
    kn = o.manual_rms_norm(o.manual_linear_from_weight(x, OL.k_proj, dtype=np.float64).reshape(1, S, 8, 128),
                           OL.k_norm, eps, np.float64)
    vv = o.manual_linear_from_weight(x, OL.v_proj, dtype=np.float64).reshape(1, S, 8, 128)
    c, s_ = o.manual_rope_cos_sin(om.inv_freq, np.arange(S)[None])
    qr, kr = o.manual_apply_rope(np.swapaxes(qn, 1, 2), np.swapaxes(kn, 1, 2), c.astype(np.float64),
                                 s_.astype(np.float64))
    ref, _ = o.manual_causal_attention(qr, o.manual_repeat_kv(kr, 2), o.manual_repeat_kv(np.swapaxes(vv, 1, 2), 2),
                                       128 ** -0.5)
    ref = np.swapaxes(ref, 1, 2).reshape(1, S, -1)
    mx, rel = report("validator 06 flow concat", concat, ref)
    assert rel < 5e-3
