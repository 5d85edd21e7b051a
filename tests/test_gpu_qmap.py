"""The integer Q4 projection on the reference's real weights, and board runtimes on the GPU.

- ``fixed.projection`` (q4d_fixed_q4_gemv) equals the reference's real-weight vectors
  bit for bit: the o_proj (K = 2048), mlp_down (K = 3072), mlp_gate (3072 rows) and
  q_proj row-block vectors (expected Q26 >> 14, saturated, and the exported Q12.12), the
  row1024 QMAP image's known answer (-3482169 >> 14), and the layer-0 q|k|v QMAP packet
  (real q/k/v weights): from the input-norm packet's Q14.10 activation and gamma through
  the fused RMSNorm prologue, and from the norm packet's Q12.12 output, both equal the
  packet's EXPECTED tensor.
- A runtime in the board manifest's layout (2 layers, 4096-row vocabulary), loaded by
  ``qmap.load_runtime`` into the float and fixed-point models, decodes the same tokens
  and Q26 scores as the fixed-point model built straight from the same weights.
- With ``Q4D_BOARD_RUNTIME_DIR`` naming a directory that holds the 61 board segment files,
  the loaded board runtime reproduces the board's two-token run: token 374 at position
  0 -> 28458 (Q26 score 1227344433), then 28458 at position 1 -> 64 (1015661901).
"""

import json
import os
from pathlib import Path

import numpy as np
import pytest
import torch

from llm_accelerator_amd import fixed as X
from llm_accelerator_amd import qmap as Q
from llm_accelerator_amd.model import Qwen3Config, build_model, random_host_weights
from oracle import q4_fixed as F
from oracle import q4_oracle as O
import qmap_synth as S

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).parent / "golden"


def sat24_shift(q26):
    return np.clip(np.asarray(q26, np.int64) >> 14, -(1 << 23), (1 << 23) - 1)


@pytest.mark.parametrize("name", ["o_proj_real", "mlp_down_proj_real", "mlp_gate_proj_real",
                                  "q4_gemv_projection_1024_real", "q4_gemv_tile_1024"])
def test_projection_real_vectors(dev, name):
    z = np.load(GOLD / f"{name}.npz")
    print(f"[qmap] projection {name} {z['weight_packed'].shape}", flush=True)
    y = X.projection(z["activation"], (z["weight_packed"], z["scale_q2_14"])).cpu().numpy()
    np.testing.assert_array_equal(y, sat24_shift(z["expected_q26"]))
    if "expected_q12_12" in z.files:
        np.testing.assert_array_equal(y, z["expected_q12_12"])


def test_row1024_image_known_answer(dev):
    img = Q.QmapImage.parse(np.load(GOLD / "qmap_stage_images.npz")["qmap_row1024_image"].tobytes())
    w = img.find(Q.ROLE_Q4_WEIGHT)[0]
    y = X.projection(Q.tensor(img.by_id(1), img), (Q.tensor(w, img), Q.tensor(img.by_id(w.scale_tensor_id), img)))
    assert y.cpu().tolist() == [-3482169 >> 14]


def test_qkv_packet_real_weights(dev):
    rn = Q.QmapImage.parse(np.load(GOLD / "qmap_stage_images.npz")["qmap_input_rmsnorm_image"].tobytes())
    z = np.load(GOLD / "qmap_qkv_layer0_image.npz")
    img = Q.QmapImage.parse(z["image"].tobytes())
    x, g, normed = (Q.tensor(rn.by_id(t), rn) for t in (87, 88, 90))
    mats = [(Q.tensor(w, img), Q.tensor(img.by_id(w.scale_tensor_id), img)) for w in img.find(Q.ROLE_Q4_WEIGHT)]
    print("[qmap] q|k|v packet, fused norm and plain", flush=True)
    fused = torch.cat([X.projection(x, m, input_gamma=g) for m in mats]).cpu().numpy()
    plain = torch.cat([X.projection(normed, m) for m in mats]).cpu().numpy()
    np.testing.assert_array_equal(fused, z["expected_q12_12"])
    np.testing.assert_array_equal(plain, z["expected_q12_12"])


def test_synthetic_runtime_decodes_like_direct_model(dev, tmp_path):
    cfg = Qwen3Config(num_hidden_layers=2, vocab_size=4096)
    host = random_host_weights(cfg, seed=21, num_layers=2)
    qz = lambda v: F.quantize_signed(v, 16, 7)[0]  # noqa: E731
    gammas = [{"input": qz(L["input_layernorm"]), "post": qz(L["post_attention_layernorm"]), "q": qz(L["q_norm"]),
               "k": qz(L["k_norm"])} for L in host["layers"]]
    cos, sin = F.rope_table_q1_15(O.rope_inv_freq(cfg.rope_theta, cfg.head_dim), np.arange(256))
    doc = json.loads((GOLD / "pl_ddr_binary_segments.json").read_text())
    path = S.write_runtime(tmp_path, doc, host, gammas, qz(host["norm"]), cos, sin, F.score_scale_q0_31(128 ** -0.5),
                           F.build_exp_lut(), F.build_sigmoid_lut(), 2)
    rt = Q.load_runtime(path, tmp_path)
    model = build_model(cfg, rt.host_weights(), max_ctx=32, device=dev)
    fx_rt = rt.fixed_model(model)
    fx_direct = X.FixedQ4Model(build_model(cfg, host, max_ctx=32, device=dev), host)
    prompt = [17, 900, 3]
    got = []
    for m in (fx_rt, fx_direct):
        kv = m.new_cache()
        out, tok = [], prompt[0]
        for pos in range(len(prompt) + 4):
            t, s, _, _ = m.run_one_token(tok, pos, kv)
            if pos >= len(prompt) - 1:
                out.append((int(t), int(s)))
                tok = int(t)
            else:
                tok = prompt[pos + 1]
        got.append(out)
    print(f"[qmap] runtime tokens {got[0]}", flush=True)
    assert got[0] == got[1]


def test_board_runtime_two_token_known_answer(dev):
    d = os.environ.get("Q4D_BOARD_RUNTIME_DIR")
    if not d or not (Path(d) / "qwen3_runtime_00.bin").exists():
        pytest.skip("board segment files not present (set Q4D_BOARD_RUNTIME_DIR)")
    man = Path(d) / "pl_ddr_binary_segments.json"
    rt = Q.load_runtime(man if man.exists() else GOLD / "pl_ddr_binary_segments.json", d)
    cfg = Qwen3Config()
    model = build_model(cfg, rt.host_weights(), max_ctx=256, device=dev)
    fx = rt.fixed_model(model)
    kv = fx.new_cache()
    t0, s0, _, _ = fx.run_one_token(374, 0, kv)
    t1, s1, _, _ = fx.run_one_token(int(t0), 1, kv)
    assert (int(t0), int(s0), int(t1), int(s1)) == (28458, 1227344433, 64, 1015661901)
