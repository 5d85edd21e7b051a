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

    (HERE / "MANIFEST.json").write_text(json.dumps(manifest, indent=2) + "\n")
    for k, v in manifest.items():
        print(k, v["arrays"])


if __name__ == "__main__":
    main()
