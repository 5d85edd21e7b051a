"""QMAP v1 images and the PL-DDR runtime manifest (CPU).

Pins, all from the reference's own files:
- every committed board image (FPGA_Project/sim/vectors/qmap_*_image_words32.hex)
  parses, with the descriptor tables QMAP_FORMAT.md documents;
- decoded tensors reproduce the reference's known answers: the dot64 image gives
  partial 24751 / scaled 3019622 (tb_q4_dot_product_64.sv:33-44), the row1024 image
  -3482169 (Q4_FORMAT.md:212-215), each through its own EXPECTED descriptor;
- the stage packets' parameters equal the stage fixtures (input gamma, q/k gammas,
  cos/sin row, exp and sigmoid LUTs, score scale) and the library's tables;
- the input-norm packet and the layer-0 q|k|v packet (real weights) are each their own
  known answer through the oracle: norm(activation, gamma) = its EXPECTED tensor, and
  projection(that, q/k/v weights) = the q|k|v packet's EXPECTED tensor;
- the 61-segment manifest validates (no overlaps, entries inside segments, sizes of
  Qwen3-0.6B shapes), tampered manifests and images are rejected;
- a runtime written in the manifest's layout (2 layers, 4096-row vocabulary) loads back
  to the same arrays, and missing / resized / altered segment files are rejected.
"""

import copy
import json
import struct
from pathlib import Path

import numpy as np
import pytest

from llm_accelerator_amd import qmap as Q
from llm_accelerator_amd.model import Qwen3Config, random_host_weights
from oracle import q4_fixed as F
from oracle import q4_oracle as O
import qmap_synth as S

GOLD = Path(__file__).parent / "golden"


@pytest.fixture(scope="module")
def images():
    z = np.load(GOLD / "qmap_stage_images.npz")
    return {k[len("qmap_"):-len("_image")]: Q.QmapImage.parse(z[k].tobytes()) for k in z.files}


@pytest.fixture(scope="module")
def qkv():
    z = np.load(GOLD / "qmap_qkv_layer0_image.npz")
    return Q.QmapImage.parse(z["image"].tobytes()), z["expected_q12_12"]


@pytest.fixture(scope="module")
def manifest_doc():
    return json.loads((GOLD / "pl_ddr_binary_segments.json").read_text())


def fx(name):
    return np.load(GOLD / f"{name}.npz")


def test_images_parse_with_documented_tables(images, qkv):
    assert set(images) == {"dot64", "row1024", "input_rmsnorm", "attention_frontend", "attention_score_value",
                           "o_proj", "post_attention_residual_norm", "mlp_silu_mul", "mlp_down",
                           "final_token_tail_compact"}
    d = images["dot64"]
    # QMAP_FORMAT.md:150-175, 287-300
    assert (d.image_base_addr, d.descriptor_table_addr, d.payload_base_addr, d.image_bytes) == \
        (0x4_1B10_0000, 0x4_1B10_0100, 0x4_1B10_0500, 0x600)
    assert [(t.tensor_id, t.role, t.dtype, t.shape, t.base_addr, t.nbytes) for t in d.descriptors] == [
        (1, Q.ROLE_ACTIVATION, 18, (64,), 0x4_1B10_0500, 128), (2, Q.ROLE_Q4_WEIGHT, 16, (1, 64), 0x4_1B10_0580, 32),
        (3, Q.ROLE_Q4_SCALE, 17, (1, 1), 0x4_1B10_05A0, 2), (4, Q.ROLE_EXPECTED, 8, (2,), 0x4_1B10_05C0, 16)]
    img, _ = qkv
    w = img.find(Q.ROLE_Q4_WEIGHT)
    assert [(t.aux[0], t.shape, t.strides_bytes[0]) for t in w] == [(1, (2048, 1024), 512), (2, (1024, 1024), 512),
                                                                     (3, (1024, 1024), 512)]
    assert img.descriptor_capacity >= 32
    for t in w:
        assert t.flags & Q.F_PACKED_Q4_LOW_EVEN and img.by_id(t.scale_tensor_id).shape == (t.shape[0], 16)


def _q26(image):
    x = Q.tensor(image.find(Q.ROLE_ACTIVATION)[0], image).astype(np.int64)
    wd = image.find(Q.ROLE_Q4_WEIGHT)[0]
    packed = Q.tensor(wd, image)
    scale = Q.tensor(image.by_id(wd.scale_tensor_id), image)
    q = O.unpack_signed_int4(packed, wd.shape[1]).astype(np.int64)
    partial = (q.reshape(q.shape[0], -1, 64) * x.reshape(-1, 64)).sum(-1)
    return partial, (partial * scale.astype(np.int64)).sum(-1), Q.tensor(image.find(Q.ROLE_EXPECTED)[0], image)


def test_dot64_and_row1024_known_answers(images):
    partial, scaled, expected = _q26(images["dot64"])
    assert (int(partial[0, 0]), int(scaled[0])) == (24751, 3019622)
    assert expected.tolist() == [24751, 3019622]
    _, scaled, expected = _q26(images["row1024"])
    assert int(scaled[0]) == -3482169 and expected.tolist() == [-3482169]


def test_stage_packet_parameters_match_fixtures(images):
    from llm_accelerator_amd import fixed as X
    rn = images["input_rmsnorm"]
    np.testing.assert_array_equal(Q.tensor(rn.by_id(88), rn), fx("fixed_rmsnorm_input_l0")["gamma"])
    np.testing.assert_array_equal(Q.tensor(rn.by_id(87), rn), fx("fixed_rmsnorm_input_l0")["input"])
    fe, qk = images["attention_frontend"], fx("fixed_qk_norm_rope_l0")
    for tid, key in ((34, "q_gamma"), (35, "k_gamma"), (36, "cos"), (37, "sin")):
        np.testing.assert_array_equal(Q.tensor(fe.by_id(tid), fe), qk[key])
    sv = images["attention_score_value"]
    lut = Q.tensor(sv.by_id(43), sv)
    np.testing.assert_array_equal(lut, fx("fixed_attention_l0")["exp_lut"])
    np.testing.assert_array_equal(lut, F.build_exp_lut())
    np.testing.assert_array_equal(lut, X.build_exp_lut())
    assert sv.find(Q.ROLE_METADATA)[0].aux[0] == int(fx("fixed_attention_l0")["score_scale_q0_31"][0]) == \
        F.score_scale_q0_31(128 ** -0.5) == 189812531
    si = images["mlp_silu_mul"]
    sig = Q.tensor(si.by_id(72), si)
    np.testing.assert_array_equal(sig, fx("fixed_silu_mul_l0")["sigmoid_lut"])
    np.testing.assert_array_equal(sig, X.build_sigmoid_lut())
    post = images["post_attention_residual_norm"]
    np.testing.assert_array_equal(Q.tensor(post.by_id(54), post), fx("fixed_post_residual_norm_l0")["gamma"])
    tail = images["final_token_tail_compact"]
    np.testing.assert_array_equal(Q.tensor(tail.by_id(27), tail), fx("fixed_rmsnorm_final")["gamma"])
    emb = tail.find(Q.ROLE_Q4_WEIGHT)[0]
    assert emb.shape == (151936, 1024) and not tail.contains(emb.base_addr) and emb.base_addr == 0x4_0010_0000
    with pytest.raises(Q.QmapError, match="outside the image"):
        Q.tensor(emb, tail)


def test_input_norm_and_qkv_packets_are_known_answers(images, qkv):
    rn = images["input_rmsnorm"]
    x, g, want = (Q.tensor(rn.by_id(t), rn) for t in (87, 88, 90))
    normed = F.fixed_rmsnorm_hidden(x, g)["output"]
    np.testing.assert_array_equal(normed, want)
    img, expected = qkv
    act = img.find(Q.ROLE_ACTIVATION)[0]
    assert act.base_addr == rn.by_id(89).base_addr  # the q|k|v input is the norm packet's output
    space = Q.AddressSpace()
    space.add_image(rn)
    outs = []
    for w in img.find(Q.ROLE_Q4_WEIGHT):
        q = O.unpack_signed_int4(Q.tensor(w, img), 1024)
        row_q26 = O.q4_gemv_q26(want, q, Q.tensor(img.by_id(w.scale_tensor_id), img))
        outs.append(O.q26_to_q12_12(row_q26)[0])
    np.testing.assert_array_equal(np.concatenate(outs), expected)
    np.testing.assert_array_equal(Q.tensor(img.find(Q.ROLE_EXPECTED)[0], img), expected)
    # the EXTERNAL activation resolves through an address space holding the norm packet
    np.testing.assert_array_equal(Q.tensor(act, img, space), Q.tensor(rn.by_id(89), rn))


def test_manifest_validates_board_layout(manifest_doc):
    man = Q.SegmentManifest(manifest_doc)
    assert len(man.segments) == 61 and man.num_layers == 28
    assert man.doc["total_segment_bytes"] == 394547200
    e = man.entries
    assert (e["tied_embedding_weight"].address, e["tied_embedding_weight"].nbytes) == (0x4_0010_0000, 151936 * 512)
    assert e["tied_embedding_scale"].nbytes == 151936 * 16 * 2
    for li in range(28):
        assert e[f"layer{li}.o_proj_weight"].nbytes == 1024 * 2048 // 2
        assert e[f"layer{li}.mlp_down_scale"].nbytes == 1024 * 48 * 2
        assert e[f"layer{li}.qkv_qmap"].nbytes == 2273280
    assert e["runtime_rope_table"].nbytes == 2 * 256 * 128 * 4
    assert e["kv_cache"].operation == "zero" and e["kv_cache"].nbytes == 28 * 2 * 8 * 256 * 128 * 4


@pytest.mark.parametrize("fault", ["overlap", "outside", "duplicate", "total", "count"])
def test_manifest_rejects_tampering(manifest_doc, fault):
    doc = copy.deepcopy(manifest_doc)
    s1, s2 = doc["segments"][1], doc["segments"][2]
    if fault == "overlap":
        s2["address"] = s1["address"] + 16
        for ent in s2["entries"]:
            ent["address"] = s2["address"]
        s2["entries"] = s2["entries"][:1]
    elif fault == "outside":
        s1["entries"][0]["nbytes"] = s1["nbytes"] + 1
    elif fault == "duplicate":
        s2["entries"][0]["name"] = s1["entries"][0]["name"]
    elif fault == "total":
        doc["total_segment_bytes"] += 1
    else:
        doc["segment_count"] = 60
    with pytest.raises(Q.QmapError):
        Q.SegmentManifest(doc)


@pytest.mark.parametrize("fault", ["magic", "version", "count", "overlap", "outside", "size", "dtype", "reserved"])
def test_image_rejects_corruption(images, fault):
    img = images["row1024"]
    b = bytearray(img.data)
    t0 = img.descriptor_table_addr - img.image_base_addr
    if fault == "magic":
        b[0] ^= 1
    elif fault == "version":
        struct.pack_into("<I", b, 4, 2)
    elif fault == "count":
        struct.pack_into("<I", b, 0x10, img.descriptor_capacity + 1)
    elif fault == "overlap":  # tensor 2's payload moved onto tensor 1's
        struct.pack_into("<Q", b, t0 + 128 + 0x20, img.by_id(1).base_addr + 64)
    elif fault == "outside":  # tensor 1's payload runs past the image end
        struct.pack_into("<Q", b, t0 + 0x28, img.image_bytes)
    elif fault == "size":  # fewer bytes than [1024] int16 needs
        struct.pack_into("<Q", b, t0 + 0x28, 2046)
    elif fault == "dtype":
        struct.pack_into("<I", b, t0 + 8, 9)
    else:
        struct.pack_into("<I", b, 0x80, 1)
    with pytest.raises(Q.QmapError):
        Q.QmapImage.parse(bytes(b))
    with pytest.raises(Q.QmapError):
        Q.QmapImage.parse(bytes(b[:255]))


def _runtime_parts(cfg, layers):
    host = random_host_weights(cfg, seed=5, num_layers=layers)
    qz = lambda v: F.quantize_signed(v, 16, 7)[0]  # noqa: E731
    gammas = [{"input": qz(L["input_layernorm"]), "post": qz(L["post_attention_layernorm"]), "q": qz(L["q_norm"]),
               "k": qz(L["k_norm"])} for L in host["layers"]]
    cos, sin = F.rope_table_q1_15(O.rope_inv_freq(cfg.rope_theta, cfg.head_dim), np.arange(256))
    return host, gammas, qz(host["norm"]), cos, sin


@pytest.fixture(scope="module")
def synth_runtime(tmp_path_factory, manifest_doc):
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=4096)
    host, gammas, fg, cos, sin = _runtime_parts(cfg, 2)
    d = tmp_path_factory.mktemp("runtime")
    path = S.write_runtime(d, manifest_doc, host, gammas, fg, cos, sin, F.score_scale_q0_31(128 ** -0.5),
                           F.build_exp_lut(), F.build_sigmoid_lut(), 2)
    return path, host, gammas, fg, cos, sin


def test_runtime_round_trip(synth_runtime):
    path, host, gammas, fg, cos, sin = synth_runtime
    rt = Q.load_runtime(path, path.parent)
    assert len(rt.layers) == 2
    for L, H, G in zip(rt.layers, host["layers"], gammas):
        for m in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            np.testing.assert_array_equal(L[m][0], H[m][0])
            np.testing.assert_array_equal(L[m][1], H[m][1])
        for k, n in (("input_gamma", "input"), ("post_gamma", "post"), ("q_gamma", "q"), ("k_gamma", "k")):
            np.testing.assert_array_equal(L[k], G[n])
    np.testing.assert_array_equal(rt.embed[0], host["embed_tokens"][0])
    np.testing.assert_array_equal(rt.embed[1], host["embed_tokens"][1])
    np.testing.assert_array_equal(rt.final_gamma, fg)
    np.testing.assert_array_equal(rt.rope_cos, cos)
    np.testing.assert_array_equal(rt.rope_sin, sin)
    assert rt.score_scale == 189812531
    hw = rt.host_weights()
    np.testing.assert_array_equal(F.quantize_signed(hw["layers"][1]["q_norm"], 16, 7)[0], gammas[1]["q"])
    assert hw["embed_tokens"][0].shape == (4096, 512)


@pytest.mark.parametrize("fault", ["missing", "resized", "altered"])
def test_runtime_rejects_bad_segment_files(synth_runtime, tmp_path, fault):
    path = synth_runtime[0]
    doc = json.loads(path.read_text())
    for s in doc["segments"]:
        (tmp_path / s["file"]).write_bytes((path.parent / s["file"]).read_bytes())
    victim = tmp_path / doc["segments"][1]["file"]
    if fault == "missing":
        victim.unlink()
        err = FileNotFoundError
    elif fault == "resized":
        victim.write_bytes(victim.read_bytes() + b"\0")
        err = Q.QmapError
    else:
        b = bytearray(victim.read_bytes())
        b[4096] ^= 0xFF
        victim.write_bytes(bytes(b))
        err = Q.QmapError
    (tmp_path / "m.json").write_text(json.dumps(doc))
    with pytest.raises(err):
        Q.load_runtime(tmp_path / "m.json", tmp_path)
