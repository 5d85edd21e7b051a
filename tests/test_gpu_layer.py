"""One decoder layer (one decode step at context 512) and the primitive ops on the GPU vs
the oracle restatement of common.py:129-298.

Config 2: hidden 1024, 16 q / 8 kv heads, head_dim 128, intermediate 3072,
eps 1e-6, theta 1e6, random Q4 weights, fp16 KV cache pre-filled with
N(0, 1) for 512 positions, one decode step at position 512.

Tolerances (stated): against the oracle that stores K/V through fp16 like the
device, the layer output must agree to max-abs <= 1e-4 * max|ref| with fp32
activations (precision mode 2) and <= 3e-3 * max|ref| with fp16 activations
(mode 1); the appended K/V row to within one fp16 ulp of the row's largest
element (mode 2) or 1.2e-2 of it (mode 1).  Against the pure fp32 reference
(fp32 K/V) the errors are reported.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as o
from gpu_helpers import report
from llm_accelerator_amd import _lib, common
from llm_accelerator_amd._lib import check
from llm_accelerator_amd.model import KVCache, Qwen3Config, build_model, current_stream, random_host_weights

pytestmark = pytest.mark.gpu

CTX = 512


@pytest.fixture(scope="module")
def layer_setup(dev):
    cfg = Qwen3Config(num_hidden_layers=1, vocab_size=2048)
    host = random_host_weights(cfg, seed=0, num_layers=1)
    model = build_model(cfg, host, max_ctx=1024, device=dev)
    ocfg = o.OracleConfig(num_hidden_layers=1, vocab_size=2048)
    om64 = o.OracleModel.from_q4(ocfg, host["layers"], *host["embed_tokens"], host["norm"], dtype=np.float64)
    om32 = o.OracleModel.from_q4(ocfg, host["layers"], *host["embed_tokens"], host["norm"], dtype=np.float32)
    rng = np.random.default_rng(2)
    kv_k = rng.normal(size=(1, 8, CTX, 128)).astype(np.float16)
    kv_v = rng.normal(size=(1, 8, CTX, 128)).astype(np.float16)
    hidden = np.random.default_rng(1).normal(size=(1, 1, 1024)).astype(np.float32)
    return cfg, model, om64, om32, kv_k, kv_v, hidden


def _run_gpu_layer(cfg, model, kv_k, kv_v, hidden, precision, dev):
    lib = _lib.load()
    check(lib.q4d_set_activation_precision(precision), "set precision")
    kv = KVCache(cfg, 1, 1, model.max_ctx, dev)
    kv.data[0, 0, 0, :, :CTX] = torch.from_numpy(kv_k[0]).to(dev)
    kv.data[0, 1, 0, :, :CTX] = torch.from_numpy(kv_v[0]).to(dev)
    kcs, vcs = common.layer_views(kv, CTX)
    h = torch.from_numpy(hidden).to(dev)
    out, k2, v2 = common.manual_decoder_layer_cached(
        hidden=h, layer=model.model.layers[0], rotary_emb=model.model.rotary_emb,
        position_ids=torch.tensor([[CTX]]), k_cache=kcs[0], v_cache=vcs[0], batch_size=1, num_q_heads=16,
        num_kv_heads=8, head_dim=128, kv_repeat=2, model_config=cfg)
    torch.cuda.synchronize()
    check(lib.q4d_set_activation_precision(2), "set precision")
    assert k2.length == v2.length == CTX + 1
    return out.cpu().numpy(), kv.data[0, 0, 0, :, CTX].float().cpu().numpy(), kv.data[0, 1, 0, :, CTX].float().cpu().numpy()


def _oracle_layer(om, kv_k, kv_v, hidden, kv_store):
    dt = om.dtype
    return o.manual_decoder_layer_cached(hidden.astype(dt), om.layers[0], om.config, om.inv_freq,
                                         np.array([[CTX]]), kv_k.astype(dt), kv_v.astype(dt),
                                         kv_store_dtype=kv_store)


@pytest.mark.parametrize("precision,tol,plan", [(2, 1e-4, 0), (2, 1e-4, 1), (1, 3e-3, 1)],
                         ids=["xcd", "staged", "staged-fp16"])
def test_decoder_layer_config2(dev, layer_setup, precision, tol, plan):
    """One decoder layer at context 512 (config 2) for both kernel plans (the XCD-split
    layer needs activation precision 2; precision 1 runs staged)."""
    cfg, model, om64, om32, kv_k, kv_v, hidden = layer_setup
    lib = _lib.load()
    prev = lib.q4d_set_decode_plan(plan)
    try:
        check(lib.q4d_set_activation_precision(precision), "set precision")
        active = lib.q4d_decode_plan_active(ctypes.byref(model.descriptor()), current_stream())
        check(lib.q4d_set_activation_precision(2), "set precision")
        out, knew, vnew = _run_gpu_layer(cfg, model, kv_k, kv_v, hidden, precision, dev)
    finally:
        lib.q4d_set_decode_plan(prev)
    # an MI355X passes the XCD-split plan's device check, so the xcd case runs that plan
    assert active == plan, (active, plan)
    # the drop-in raised on a status bit; read the word explicitly as well
    assert common.runtime(model).ws.status() == 0
    ref, kc, vc = _oracle_layer(om64, kv_k, kv_v, hidden, np.float16)
    mx, rel = report(f"layer mode{precision} vs fp16-KV oracle", out, ref)
    assert rel <= tol
    # appended row (fp16 in both): within one fp16 ulp of the row's largest
    # element (fp32 error ahead of the rounding can flip a rounding boundary)
    for name, got, want in (("k row", knew, kc[0, :, CTX]), ("v row", vnew, vc[0, :, CTX])):
        ulp_row = np.spacing(np.abs(want).max(axis=-1, keepdims=True).astype(np.float16)).astype(np.float64)
        bound = ulp_row if precision == 2 else 4 * tol * np.abs(want).max(axis=-1, keepdims=True)
        report(f"appended {name} mode{precision}", got, want)
        assert np.all(np.abs(got - want) <= bound), float(np.max(np.abs(got - want) / bound))
    ref32, _, _ = _oracle_layer(om32, kv_k, kv_v, hidden, None)
    report(f"layer mode{precision} vs fp32 reference", out, ref32)


def test_layer_repeat_is_deterministic(dev, layer_setup):
    cfg, model, _, _, kv_k, kv_v, hidden = layer_setup
    a = _run_gpu_layer(cfg, model, kv_k, kv_v, hidden, 2, dev)
    b = _run_gpu_layer(cfg, model, kv_k, kv_v, hidden, 2, dev)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_primitive_ops_match_oracle(dev, layer_setup):
    """manual_rms_norm, manual_linear_from_weight, qk-norm + RoPE via
    manual_rope_cos_sin / manual_apply_rope, append_cache and
    manual_cached_attention, composed exactly as common.py:245-284 does."""
    cfg, model, om64, _, kv_k, kv_v, hidden = layer_setup
    L = model.model.layers[0]
    OL = om64.layers[0]
    h = torch.from_numpy(hidden).to(dev)
    eps = cfg.rms_norm_eps
    xn = common.manual_rms_norm(h, L.input_layernorm.weight, eps)
    xn_ref = o.manual_rms_norm(hidden.astype(np.float64), OL.input_layernorm, eps, np.float64)
    assert report("rms_norm", xn.cpu().numpy(), xn_ref)[1] < 1e-6
    q = common.manual_linear_from_weight(xn, L.self_attn.q_proj.weight)
    k = common.manual_linear_from_weight(xn, L.self_attn.k_proj.weight)
    v = common.manual_linear_from_weight(xn, L.self_attn.v_proj.weight)
    q_ref = xn_ref @ OL.q_proj.T
    assert report("q_proj", q.cpu().numpy(), q_ref)[1] < 1e-5
    qn = common.manual_rms_norm(q.view(1, 1, 16, 128), L.self_attn.q_norm.weight, eps).transpose(1, 2)
    kn = common.manual_rms_norm(k.view(1, 1, 8, 128), L.self_attn.k_norm.weight, eps).transpose(1, 2)
    pos = torch.tensor([[CTX]])
    cos, sin = common.manual_rope_cos_sin(model.model.rotary_emb, h, pos)
    c_ref, s_ref = o.manual_rope_cos_sin(om64.inv_freq, np.array([[CTX]]))
    np.testing.assert_allclose(cos.cpu().numpy(), c_ref, atol=2e-6)
    qr, kr = common.manual_apply_rope(qn, kn, cos, sin)
    kv = KVCache(cfg, 1, 1, model.max_ctx, dev)
    kv.data[0, 0, 0, :, :CTX] = torch.from_numpy(kv_k[0]).to(dev)
    kv.data[0, 1, 0, :, :CTX] = torch.from_numpy(kv_v[0]).to(dev)
    kcs, vcs = common.layer_views(kv, CTX)
    kc = common.append_cache(kcs[0], kr)
    vc = common.append_cache(vcs[0], v.view(1, 1, 8, 128).transpose(1, 2))
    out, weights = common.manual_cached_attention(qr, common.manual_repeat_kv(kc, 2), common.manual_repeat_kv(vc, 2),
                                                  L.self_attn.scaling)
    assert weights is None and kc.length == CTX + 1
    trace = {}
    o.manual_decoder_layer_cached(hidden.astype(np.float64), OL, om64.config, om64.inv_freq, np.array([[CTX]]),
                                  kv_k.astype(np.float64), kv_v.astype(np.float64), kv_store_dtype=np.float16,
                                  trace=trace)
    attn_ref = trace["attn"].reshape(1, 16, 1, 128)
    assert report("attention", out.cpu().numpy(), attn_ref)[1] < 1e-4


def test_embedding_gather_exact(dev, layer_setup):
    cfg, model, om64, _, _, _, _ = layer_setup
    lib = _lib.load()
    toks = torch.tensor([0, 7, 2047], dtype=torch.int32, device=dev)
    out = torch.empty((3, 1024), dtype=torch.float32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    desc = model.lm_head.weight.descriptor()
    check(lib.q4d_embedding(ctypes.byref(desc), toks.data_ptr(), 3, out.data_ptr(), status.data_ptr(),
                            current_stream()), "q4d_embedding")
    np.testing.assert_array_equal(out.cpu().numpy(), om64.embed_tokens[[0, 7, 2047]].astype(np.float32))
    assert int(status.item()) == 0
    # a device-side token outside the vocabulary: zero row and a status bit, no fault
    bad = torch.tensor([2048], dtype=torch.int32, device=dev)
    check(lib.q4d_embedding(ctypes.byref(desc), bad.data_ptr(), 1, out.data_ptr(), status.data_ptr(),
                            current_stream()), "q4d_embedding")
    torch.cuda.synchronize()
    assert int(status.item()) == _lib.STATUS_BAD_TOKEN and float(out[0].abs().sum()) == 0.0


def test_bad_position_is_reported_not_executed(dev, layer_setup):
    cfg, model, _, _, _, _, hidden = layer_setup
    lib = _lib.load()
    ws = common.runtime(model).ws
    kv = KVCache(cfg, 1, 1, model.max_ctx, dev)
    before = kv.data.clone()
    pos = torch.tensor([model.max_ctx], dtype=torch.int32, device=dev)  # one past the end
    h = torch.from_numpy(hidden.reshape(1, 1024)).to(dev)
    out = torch.empty_like(h)
    desc, kvd = model.descriptor(), kv.descriptor()
    check(lib.q4d_decoder_layer(ctypes.byref(desc), 0, h.data_ptr(), out.data_ptr(), ctypes.byref(kvd),
                                pos.data_ptr(), ws.ptr, ws.nbytes, current_stream()), "q4d_decoder_layer")
    st = ctypes.c_int32(0)
    check(lib.q4d_read_status(ws.ptr, ws.nbytes, ctypes.byref(desc), 1, ctypes.byref(st), current_stream()),
          "q4d_read_status")
    assert st.value & _lib.STATUS_BAD_POSITION
    assert torch.equal(kv.data, before)
    # clear the sticky status for later tests
    ws.buf[:256].zero_()
    with pytest.raises(_lib.Q4DecError) as e:
        common.manual_decoder_layer_cached(h.view(1, 1, 1024), model.model.layers[0], model.model.rotary_emb,
                                           torch.tensor([[5]]), *[x[0] for x in common.layer_views(kv, 3)], 1, 16, 8,
                                           128, 2, cfg)
    assert e.value.code == -10


@pytest.mark.parametrize("lengths", [[1], [63], [64], [65], [256], [257], [1000], [5, 300, 64, 777]])
def test_attention_context_lengths_and_batch(dev, lengths):
    """q4d_cached_attention over a batch whose sequences have their own
    positions: chunk boundaries (64), group boundaries (4 x 64) and ragged
    batches, against the oracle (common.py:192-228) per sequence."""
    from llm_accelerator_amd._lib import Q4dModel
    lib = _lib.load()
    B, max_ctx = len(lengths), 1024
    cfg = Qwen3Config()
    kv = KVCache(cfg, 1, B, max_ctx, dev)
    rng = np.random.default_rng(sum(lengths))
    kv_host = rng.normal(size=(2, B, 8, max_ctx, 128)).astype(np.float16)
    kv.data[0] = torch.from_numpy(kv_host).to(dev)
    q = rng.normal(size=(B, 16, 128)).astype(np.float32)
    m = Q4dModel(hidden_size=1024, intermediate_size=3072, num_layers=1, num_q_heads=16, num_kv_heads=8,
                 head_dim=128, vocab_size=2, max_ctx=max_ctx, rms_norm_eps=1e-6, attn_scaling=128 ** -0.5)
    nbytes = int(lib.q4d_workspace_bytes(ctypes.byref(m), B))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    pos = torch.tensor([n - 1 for n in lengths], dtype=torch.int32, device=dev)
    out = torch.empty(B, 2048, dtype=torch.float32, device=dev)
    qd = torch.from_numpy(q).to(dev)
    kvd = kv.descriptor()
    check(lib.q4d_cached_attention(ctypes.byref(m), ctypes.byref(kvd), 0, qd.data_ptr(), pos.data_ptr(),
                                   out.data_ptr(), 1, ws.data_ptr(), nbytes, current_stream()), "attention")
    got = out.cpu().numpy().reshape(B, 16, 128)
    for bi, n in enumerate(lengths):
        k = kv_host[0, bi:bi + 1, :, :n].astype(np.float64)
        v = kv_host[1, bi:bi + 1, :, :n].astype(np.float64)
        ref, _ = o.manual_cached_attention(q[bi:bi + 1, :, None].astype(np.float64), o.manual_repeat_kv(k, 2),
                                           o.manual_repeat_kv(v, 2), 128 ** -0.5)
        mx, rel = report(f"attention T={n}", got[bi], ref[0, :, 0])
        assert mx <= 2e-6 * max(1.0, float(np.abs(ref).max())) + 1e-6, (n, mx)


LONG_CASES = [(plan, cap, pos) for plan, cap, name in ((0, 4096, "xcd-4096"), (0, 2048, "xcd-2048"),
                                                       (1, 4097, "staged-4097"))
              for pos in (1024, 1151, 2047, 4095) if pos < cap]
# the XCD-split layer past 4096 positions (16, 32 or 64 groups of 16 per workgroup, and the
# loop stopping at a short chunk's end)
LONG_CASES += [(0, 8193, 4100), (0, 8193, 8192), (0, 32768, 1000), (0, 32768, 32767)]
LONG_IDS = [f"{'xcd' if p == 0 else 'staged'}-{c}-{q}" for p, c, q in LONG_CASES]


@pytest.mark.parametrize("plan,max_ctx,position", LONG_CASES, ids=LONG_IDS)
def test_decoder_layer_long_context(dev, layer_setup, position, plan, max_ctx):
    """Batch-1 decode layer past 1024 cached positions against the fp16-KV oracle at
    the layer-test bar, for both kernel plans: the XCD-split layer at a capacity of
    2048 to 32768 positions (each of the 32 attention workgroups of an XCD takes up to
    4 .. 64 groups of 16 positions, fewer when the chunk is short), and the five staged
    launches past 4096 positions (the o_proj prologue merges more than eight 128-position
    chunks, its loop over further batches of eight)."""
    from llm_accelerator_amd.model import with_context
    cfg, model, om64, _, _, _, hidden = layer_setup
    m = with_context(model, max_ctx)
    rng = np.random.default_rng(position)
    kv_k = rng.normal(size=(1, 8, position, 128)).astype(np.float16)
    kv_v = rng.normal(size=(1, 8, position, 128)).astype(np.float16)
    kv = KVCache(cfg, 1, 1, m.max_ctx, dev)
    kv.data[0, 0, 0, :, :position] = torch.from_numpy(kv_k[0]).to(dev)
    kv.data[0, 1, 0, :, :position] = torch.from_numpy(kv_v[0]).to(dev)
    lib = _lib.load()
    desc, kvd = m.descriptor(), kv.descriptor()
    ws = torch.zeros(int(lib.q4d_workspace_bytes(ctypes.byref(desc), 1)), dtype=torch.uint8, device=dev)
    check(lib.q4d_workspace_init(ws.data_ptr(), ws.numel(), ctypes.byref(desc), 1, current_stream()), "ws init")
    h = torch.from_numpy(hidden.reshape(1, 1024)).to(dev)
    out = torch.empty_like(h)
    pos = torch.tensor([position], dtype=torch.int32, device=dev)
    print(f"[layer long ctx] plan={plan} max_ctx={max_ctx} position={position}", flush=True)
    prev = lib.q4d_set_decode_plan(plan)
    try:
        check(lib.q4d_decoder_layer(ctypes.byref(desc), 0, h.data_ptr(), out.data_ptr(), ctypes.byref(kvd),
                                    pos.data_ptr(), ws.data_ptr(), ws.numel(), current_stream()), "q4d_decoder_layer")
    finally:
        lib.q4d_set_decode_plan(prev)
    st = ctypes.c_int32(0)
    check(lib.q4d_read_status(ws.data_ptr(), ws.numel(), ctypes.byref(desc), 1, ctypes.byref(st), current_stream()),
          "q4d_read_status")
    assert st.value == 0
    ref, kc, vc = o.manual_decoder_layer_cached(hidden.astype(np.float64), om64.layers[0], om64.config, om64.inv_freq,
                                                np.array([[position]]), kv_k.astype(np.float64),
                                                kv_v.astype(np.float64), kv_store_dtype=np.float16)
    mx, rel = report(f"layer at position {position}", out.cpu().numpy(), ref)
    assert rel <= 1e-4
    for kind, want in ((0, kc[0, :, position]), (1, vc[0, :, position])):
        got = kv.data[0, kind, 0, :, position].float().cpu().numpy()
        ulp_row = np.spacing(np.abs(want).max(axis=-1, keepdims=True).astype(np.float16)).astype(np.float64)
        assert np.all(np.abs(got - want) <= ulp_row), kind


@pytest.mark.parametrize("plan", [0, 1], ids=["xcd", "staged"])
@pytest.mark.parametrize("position", [0, 1, 63, 64, 200, 511])
def test_decoder_layer_64_position_chunks(dev, layer_setup, position, plan):
    """A context capacity of 512 positions: the staged plan splits batch-1 attention
    into 64-position chunks (at most 8, merged by the o_proj prologue in one batch of
    loads), the XCD-split plan gives each of an XCD's 32 workgroups one group of 16
    positions; chunk edges and the last slot against the fp16-KV oracle at the
    layer-test bar.  The cache rows at and past the position hold NaN bit patterns
    (rows never written): they stand in for absent positions in the kernels' loads
    and must not reach the output."""
    from llm_accelerator_amd.model import with_context
    cfg, model, om64, _, _, _, hidden = layer_setup
    m = with_context(model, 512)
    rng = np.random.default_rng(1000 + position)
    kv_k = rng.normal(size=(1, 8, position, 128)).astype(np.float16)
    kv_v = rng.normal(size=(1, 8, position, 128)).astype(np.float16)
    kv = KVCache(cfg, 1, 1, m.max_ctx, dev)
    kv.data.fill_(float("nan"))
    kv.data[0, 0, 0, :, :position] = torch.from_numpy(kv_k[0]).to(dev)
    kv.data[0, 1, 0, :, :position] = torch.from_numpy(kv_v[0]).to(dev)
    lib = _lib.load()
    desc, kvd = m.descriptor(), kv.descriptor()
    ws = torch.zeros(int(lib.q4d_workspace_bytes(ctypes.byref(desc), 1)), dtype=torch.uint8, device=dev)
    check(lib.q4d_workspace_init(ws.data_ptr(), ws.numel(), ctypes.byref(desc), 1, current_stream()), "ws init")
    h = torch.from_numpy(hidden.reshape(1, 1024)).to(dev)
    out = torch.empty_like(h)
    pos = torch.tensor([position], dtype=torch.int32, device=dev)
    print(f"[layer 64-position chunks] plan={plan} position={position}", flush=True)
    prev = lib.q4d_set_decode_plan(plan)
    try:
        assert lib.q4d_decode_plan_active(ctypes.byref(desc), current_stream()) == plan
        check(lib.q4d_decoder_layer(ctypes.byref(desc), 0, h.data_ptr(), out.data_ptr(), ctypes.byref(kvd),
                                    pos.data_ptr(), ws.data_ptr(), ws.numel(), current_stream()), "q4d_decoder_layer")
    finally:
        lib.q4d_set_decode_plan(prev)
    st = ctypes.c_int32(0)
    check(lib.q4d_read_status(ws.data_ptr(), ws.numel(), ctypes.byref(desc), 1, ctypes.byref(st), current_stream()),
          "q4d_read_status")
    assert st.value == 0
    assert torch.isfinite(out).all()
    ref, kc, vc = o.manual_decoder_layer_cached(hidden.astype(np.float64), om64.layers[0], om64.config, om64.inv_freq,
                                                np.array([[position]]),
                                                kv_k.astype(np.float64) if position else None,
                                                kv_v.astype(np.float64) if position else None,
                                                kv_store_dtype=np.float16)
    mx, rel = report(f"layer at position {position} (64-position chunks)", out.cpu().numpy(), ref)
    assert rel <= 1e-4
