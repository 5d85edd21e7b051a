"""Convert a few of the reference's golden hex vectors into small npz fixtures.

Run in the build container only (it reads the reference checkout):

    python tests/golden/make_fixtures.py [--ref /root/reference]

The fixtures are data (inputs and expected outputs) taken from
``FPGA_Project/sim/vectors/`` of Tyler913/LLM_Accelerator, produced there by
``Qwen3-0.6B-Base/python_each_module/{15,26,28,30,33,35}_export_*.py`` from the
real Qwen3-0.6B-Base weights (Apache-2.0, ``Qwen3-0.6B-Base/LICENSE``), plus
the dot64 known answer held in ``FPGA_Project/sim/tb_q4_dot_product_64.sv:33-44``.
Each output records the source files and their sha256 in ``MANIFEST.json``.
Nothing here runs reference code; it only parses hex text.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import re
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def sha256(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def read_hex(path: Path, width: int, signed: bool) -> np.ndarray:
    vals = []
    sign = 1 << (width - 1)
    full = 1 << width
    mask = full - 1
    for line in path.read_text().split():
        v = int(line, 16) & mask
        if signed and v & sign:
            v -= full
        vals.append(v)
    return np.array(vals, dtype=np.int64)


def pack_nibble_lines(nibbles: np.ndarray, k: int) -> np.ndarray:
    """One signed int4 per hex line (row-major) -> packed bytes [N, K/2]."""
    n = nibbles.reshape(-1, k).astype(np.int64) & 0xF
    return (n[:, 0::2] | (n[:, 1::2] << 4)).astype(np.uint8)


def words_to_bytes(words: np.ndarray, k: int) -> np.ndarray:
    return words.astype(np.uint32).astype("<u4").view(np.uint8).reshape(-1, k // 2)


def words_to_scales(words: np.ndarray, groups: int) -> np.ndarray:
    return words.astype(np.uint32).astype("<u4").view(np.uint16).reshape(-1, groups)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    args = ap.parse_args()
    ref = Path(args.ref)
    vec = ref / "FPGA_Project" / "sim" / "vectors"
    manifest: dict[str, dict] = {}

    def record(name: str, sources: list[Path], note: str, **arrays):
        out = HERE / f"{name}.npz"
        np.savez_compressed(out, **arrays)
        manifest[name] = {
            "file": out.name,
            "note": note,
            "sources": {str(p.relative_to(ref)): sha256(p) for p in sources},
            "arrays": {k: [list(np.asarray(v).shape), str(np.asarray(v).dtype)] for k, v in arrays.items()},
        }

    # 1. dot64 known answer (q_proj layer 0 row 0 group 0), from the SV testbench constants.
    tb = ref / "FPGA_Project" / "sim" / "tb_q4_dot_product_64.sv"
    text = tb.read_text()
    act_hex = re.search(r"TEST_ACTIVATION_FLAT\s*=\s*\d+'h([0-9a-fA-F]+)", text).group(1)
    w_hex = re.search(r"TEST_WEIGHT_PACKED\s*=\s*\d+'h([0-9a-fA-F]+)", text).group(1)
    scale = int(re.search(r"TEST_SCALE_Q2_14\s*=\s*\d+'d(\d+)", text).group(1))
    partial = int(re.search(r"EXPECTED_PARTIAL_SUM\s*=\s*\d+'sd(-?\d+)", text).group(1))
    scaled = int(re.search(r"EXPECTED_SCALED_SUM_Q26\s*=\s*\d+'sd(-?\d+)", text).group(1))
    act_int = int(act_hex, 16)
    act = np.array([(act_int >> (16 * i)) & 0xFFFF for i in range(64)], dtype=np.int64)
    act[act >= 0x8000] -= 0x10000
    w_int = int(w_hex, 16)
    w_bytes = np.array([(w_int >> (8 * i)) & 0xFF for i in range(32)], dtype=np.uint8)
    record("q4_dot64_kat", [tb], "flat vectors: element i at bits [16i +: 16] / byte i at bits [8i +: 8]",
           activation_q4_12=act, weight_packed=w_bytes.reshape(1, 32), scale_q2_14=np.array([[scale]], np.uint16),
           expected_partial=np.array(partial), expected_scaled_q26=np.array(scaled))

    # 2. q_proj layer 0 rows 0..15 and rows 0..3 (Q4.12 activation, Q26 48-bit).
    for prefix, rows in (("q4_gemv_projection_1024_real", 16), ("q4_gemv_tile_1024", 4)):
        srcs = [vec / f"{prefix}_{s}.hex" for s in ("activation", "weight", "scale", "expected")]
        a = read_hex(srcs[0], 16, True)
        w = read_hex(srcs[1], 4, True)
        s = read_hex(srcs[2], 16, False)
        e = read_hex(srcs[3], 48, True)
        record(prefix, srcs, "Q4.12 activation; expected = Q26 row sums",
               activation=a, weight_packed=pack_nibble_lines(w, 1024),
               scale_q2_14=s.reshape(rows, 16).astype(np.uint16), expected_q26=e)

    # 3. gate_proj full (the 3072x1024 shape) and up_proj rows 0..511, Q12.12 activation.
    p = "mlp_gate_up_proj_stage_real"
    a_src = vec / f"{p}_activation.hex"
    act = read_hex(a_src, 24, True)
    for mat, rows in (("gate", 3072), ("up", 512)):
        srcs = [a_src] + [vec / f"{p}_{mat}_{s}.hex" for s in
                          ("weight_words32", "scale_words32", "expected_q26", "expected_q12_12")]
        w = words_to_bytes(read_hex(srcs[1], 32, False), 1024)[:rows]
        s = words_to_scales(read_hex(srcs[2], 32, False), 16)[:rows]
        e26 = read_hex(srcs[3], 56, True)[:rows]
        e12 = read_hex(srcs[4], 24, True)[:rows]
        record(f"mlp_{mat}_proj_real", srcs, f"layer 0 {mat}_proj rows 0..{rows - 1}; Q12.12 activation",
               activation=act, weight_packed=w, scale_q2_14=s, expected_q26=e26, expected_q12_12=e12)

    # 4. o_proj (K=2048) and down_proj (K=3072), first 256 rows each.
    for p, k, w26, rows, name in (("o_proj_stage_real", 2048, 64, 256, "o_proj_real"),
                                  ("mlp_down_proj_stage_real", 3072, 58, 256, "mlp_down_proj_real")):
        srcs = [vec / f"{p}_{s}.hex" for s in
                ("activation", "weight_words32", "scale_words32", "expected_q26", "expected_q12_12")]
        a = read_hex(srcs[0], 24, True)
        w = words_to_bytes(read_hex(srcs[1], 32, False), k)[:rows]
        s = words_to_scales(read_hex(srcs[2], 32, False), k // 64)[:rows]
        e26 = read_hex(srcs[3], w26, True)[:rows]
        e12 = read_hex(srcs[4], 24, True)[:rows]
        record(name, srcs, f"layer 0 rows 0..{rows - 1}; K={k}; Q12.12 activation",
               activation=a, weight_packed=w, scale_q2_14=s, expected_q26=e26, expected_q12_12=e12)

    # 5. LM-head 1024-row window with the argmax known answer.
    p = "lm_head_argmax_stage_real"
    srcs = [vec / f"{p}_{s}.hex" for s in ("activation", "weight_words32", "scale_words32",
                                           "expected_scan_logits_q26", "expected_best_token",
                                           "expected_best_score_q26", "scan_base_token")]
    record("lm_head_argmax_real", srcs + [vec / f"{p}_meta.json"],
           "tied LM head rows 0..1023 (the window holds the full-vocab argmax, meta argmax.*)",
           activation=read_hex(srcs[0], 24, True),
           weight_packed=words_to_bytes(read_hex(srcs[1], 32, False), 1024),
           scale_q2_14=words_to_scales(read_hex(srcs[2], 32, False), 16),
           expected_logits_q26=read_hex(srcs[3], 56, True),
           expected_best_token=read_hex(srcs[4], 32, False)[:1],
           expected_best_score_q26=read_hex(srcs[5], 56, True)[:1],
           scan_base_token=read_hex(srcs[6], 32, False)[:1])

    # 6. Fixed-point stages of the integer decode layer (exporters 17, 18, 22-25, 27, 29, 31, 32,
    #    46): layer 0 at position 4 of the prompt [785, 3853, 315, 89462, 374] and the layer-1/2
    #    variants (``*_chained``: inputs chained from the previous layer's integer outputs).
    def stage(prefix: str, fields: dict[str, tuple[int, bool]]) -> tuple[list[Path], dict]:
        srcs, arrays = [], {}
        for key, (width, signed) in fields.items():
            src = vec / f"{prefix}_{key}.hex"
            srcs.append(src)
            arrays[key] = read_hex(src, width, signed)
        return srcs, arrays

    s24, u24, s64, u64, s16, u16 = (24, True), (24, False), (64, True), (64, False), (16, True), (16, False)
    rms_fields = {"input": s24, "gamma": s16, "expected": s24, "sum_squares": u64, "mean_square": u64,
                  "sqrt_radicand": u64, "rms": u24, "inv_rms": u24, "saturation": (4, False)}
    for prefix, name, note in (
            ("rmsnorm_1024_real", "fixed_rmsnorm_input_l0", "layer 0 input RMSNorm (17)"),
            ("layer1_chained_input_rmsnorm_stage_real", "fixed_rmsnorm_input_l1c", "layer 1 input RMSNorm"),
            ("layer2_chained_input_rmsnorm_stage_real", "fixed_rmsnorm_input_l2c", "layer 2 input RMSNorm"),
            ("final_rmsnorm_stage_real", "fixed_rmsnorm_final", "final RMSNorm (32)"),
            ("final_rmsnorm_layer2_chained_stage_real", "fixed_rmsnorm_final_l2c", "final RMSNorm after layer 2")):
        srcs, arr = stage(prefix, rms_fields)
        record(name, srcs, f"{note}: Q14.10 in, Q8.7 gamma, Q12.12 out", **arr)

    qk_fields = {"q_input": s24, "k_input": s24, "q_gamma": s16, "k_gamma": s16, "cos": s16, "sin": s16,
                 "q_norm_expected": s24, "k_norm_expected": s24, "q_rope_expected": s24,
                 "k_rope_expected": s24, "norm_saturation": (4, False), "rope_saturation": (4, False)}
    for prefix, name in (("qk_norm_rope_stage_128_real", "fixed_qk_norm_rope_l0"),
                         ("layer1_chained_qk_norm_rope_stage_128_real", "fixed_qk_norm_rope_l1c"),
                         ("layer2_chained_qk_norm_rope_stage_128_real", "fixed_qk_norm_rope_l2c")):
        srcs, arr = stage(prefix, qk_fields)
        record(name, srcs, "per-head q/k RMSNorm (Q12.12, eps 17, shift 23) then RoPE with Q1.15 "
                           "cos/sin of position 4", **arr)
    srcs, arr = stage("rope_qk_layer_128_real", {"q_input": s24, "k_input": s24, "cos": s16, "sin": s16,
                                                  "q_expected": s24, "k_expected": s24})
    record("fixed_rope_qk_l0", srcs, "RoPE alone (18), position 4", **arr)

    for sp, vp, name in (("attention_score_stage_real", "attention_softmax_value_stage_real", "fixed_attention_l0"),
                         ("layer1_attention_score_stage_real", "layer1_attention_softmax_value_stage_real",
                          "fixed_attention_l1"),
                         ("layer1_chained_attention_score_stage_real",
                          "layer1_chained_attention_softmax_value_stage_real", "fixed_attention_l1c"),
                         ("layer2_chained_attention_score_stage_real",
                          "layer2_chained_attention_softmax_value_stage_real", "fixed_attention_l2c")):
        s1, a1 = stage(sp, {"q_input": s24, "k_cache": s24, "score_scale_q0_31": (32, False),
                            "cache_length": u16, "expected_raw": s64, "expected_scaled": s64,
                            "expected_q_head": (8, False), "expected_position": (8, False)})
        s2, a2 = stage(vp, {"score_input": s64, "v_cache": s24, "exp_lut": u24, "expected_lut_index": u16,
                            "expected_prob": u24, "expected_out": s24})
        record(name, s1 + s2, "score stage (q [16,128], k_cache [T,8,128], Q0.31 scale; raw/scaled "
                              "[q_head][position]) and softmax/value stage (v_cache [T,8,128])", **a1, **a2)

    post_fields = {"residual_input": s24, "o_proj_input": s24, "gamma": s16, "expected_residual": s24,
                   "expected_norm": s24, "sum_squares": u64, "mean_square": u64, "sqrt_radicand": u64,
                   "rms": u24, "inv_rms": u24, "residual_saturation": (4, False), "norm_saturation": (4, False)}
    silu_fields = {"gate_input": s24, "up_input": s24, "sigmoid_lut": u16, "expected_lut_index": u16,
                   "expected_sigmoid_q0_16": u16, "expected_silu_gate_q12_12": s24,
                   "expected_hidden_q12_12": s24}
    res_fields = {"post_attn_hidden": s24, "down_out": s24, "expected_layer_out": s24,
                  "residual_saturation": (4, False)}
    for tag, pre in (("l0", ""), ("l1c", "layer1_chained_"), ("l2c", "layer2_chained_")):
        srcs, arr = stage(f"{pre}post_attention_residual_norm_stage_real", post_fields)
        record(f"fixed_post_residual_norm_{tag}", srcs, "hidden + (o_proj >> 2), saturated, then RMSNorm", **arr)
        srcs, arr = stage(f"{pre}mlp_silu_mul_stage_real", silu_fields)
        record(f"fixed_silu_mul_{tag}", srcs, "sigmoid LUT SiLU(gate) * up", **arr)
        srcs, arr = stage(f"{pre}mlp_residual_add_stage_real", res_fields)
        record(f"fixed_residual_add_{tag}", srcs, "post-attention hidden + (down >> 2), saturated", **arr)

    srcs, arr = stage("kv_cache_append_real", {"k_input": s24, "v_input": s24, "expected_addr": u64,
                                               "expected_data": (32, True), "expected_kind": (4, False),
                                               "expected_head": (8, False), "expected_dim": (8, False)})
    record("fixed_kv_append_l0", srcs + [vec / "kv_cache_append_real_meta.json"],
           "layer 0, position 4, base 0x414100000, max context 256, word32 elements", **arr)

    # 7. QMAP v1 images (Source/QMAP_FORMAT.md:134-296) as raw little-endian bytes, and the
    #    PL-DDR segment manifest of the board-validated runtime (a data file, copied as is).
    def image(name: str) -> tuple[Path, np.ndarray]:
        src = vec / f"{name}_words32.hex"
        return src, read_hex(src, 32, False).astype("<u4").view(np.uint8)

    small = {}
    srcs = []
    for name in ("qmap_dot64_image", "qmap_row1024_image", "qmap_input_rmsnorm_image", "qmap_attention_frontend_image",
                 "qmap_attention_score_value_image", "qmap_o_proj_image", "qmap_post_attention_residual_norm_image",
                 "qmap_mlp_silu_mul_image", "qmap_mlp_down_image", "qmap_final_token_tail_compact_image"):
        src, b = image(name)
        srcs.append(src)
        small[name] = b
    record("qmap_stage_images", srcs, "layer-0 QMAP packets / smoke images, raw bytes (little-endian words)", **small)
    src, b = image("qmap_qkv_projection_from_input_rmsnorm_image")
    e_src = vec / "qmap_qkv_projection_expected_from_input_rmsnorm_words32.hex"
    record("qmap_qkv_layer0_image", [src, e_src],
           "layer-0 q|k|v packet with the full Q4 q/k/v weights in the image; expected q|k|v Q12.12 for the "
           "input-RMSNorm output of qmap_input_rmsnorm_image", image=b,
           expected_q12_12=read_hex(e_src, 32, True))
    seg = ref / "lmdeploy" / "qwen3-0p6b-q4-qweb-demo" / "model" / "pl_ddr_binary_segments.json"
    (HERE / "pl_ddr_binary_segments.json").write_bytes(seg.read_bytes())
    manifest["pl_ddr_binary_segments"] = {"file": "pl_ddr_binary_segments.json",
                                          "note": "61-segment PL-DDR runtime manifest (data file, copied verbatim)",
                                          "sources": {str(seg.relative_to(ref)): sha256(seg)}}

    # 8. The model's config.json (hyperparameters the checkpoint converter reads; data file).
    cfg = ref / "Qwen3-0.6B-Base" / "config.json"
    (HERE / "qwen3_0p6b_config.json").write_bytes(cfg.read_bytes())
    manifest["qwen3_0p6b_config"] = {"file": "qwen3_0p6b_config.json",
                                     "note": "Qwen3-0.6B-Base config.json (data file, copied verbatim)",
                                     "sources": {str(cfg.relative_to(ref)): sha256(cfg)}}

    (HERE / "MANIFEST.json").write_text(json.dumps(manifest, indent=2) + "\n")
    for k, v in manifest.items():
        print(k, v.get("arrays", v["file"]))


if __name__ == "__main__":
    main()
