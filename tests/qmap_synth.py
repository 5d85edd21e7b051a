"""Test helper: QMAP v1 images and a PL-DDR runtime written from a host model.

``pack_image`` lays out a QMAP v1 image (256-byte header, 128-byte descriptors,
64-byte-aligned payloads; ``Source/QMAP_FORMAT.md:134-296``).  ``write_runtime`` writes
segment files and a manifest with the board runtime's layout
(``pl_ddr_binary_segments.json``: the tied embedding in segment 0, per layer the q|k|v
image and the raw o/gate/up/down arrays, the per-layer stage packets, the final-tail
packet, the RoPE table), truncated to the given layer count and vocabulary.  Used to
round-trip ``llm_accelerator_amd.qmap.load_runtime``.
"""

from __future__ import annotations

import copy
import hashlib
import json
import struct
from pathlib import Path

import numpy as np

from llm_accelerator_amd import qmap as Q

RO = Q.F_ROW_MAJOR | Q.F_READ_ONLY
PACKED = Q.F_ROW_MAJOR | Q.F_PACKED_Q4_LOW_EVEN | Q.F_READ_ONLY


def _align(x: int, a: int) -> int:
    return (x + a - 1) // a * a


def words32(values) -> bytes:
    """Values widened to little-endian 32-bit words (the stage images' storage)."""
    return np.asarray(values, dtype=np.int64).astype("<i4").tobytes()


def desc(tid, role, dtype, shape, strides, payload=None, ext=None, flags=RO, bits=32, scale_tid=0xFFFFFFFF,
         group=0, aux=(0, 0, 0, 0)) -> dict:
    """One descriptor: ``payload`` bytes placed in the image, or ``ext`` = (address, nbytes)."""
    return dict(tid=tid, role=role, dtype=dtype, shape=tuple(shape), strides=tuple(strides), payload=payload, ext=ext,
                flags=flags, bits=bits, scale_tid=scale_tid, group=group, aux=tuple(aux))


def pack_image(base: int, descs: list, capacity: int | None = None, min_bytes: int = 0) -> bytes:
    cap = capacity or max(8, _align(len(descs), 8))
    table = base + Q.HEADER_BYTES
    payload_base = _align(table + cap * Q.DESCRIPTOR_BYTES, 64)
    cursor = payload_base
    placed = []
    for d in descs:
        if d["payload"] is not None:
            placed.append((cursor, len(d["payload"])))
            cursor = _align(cursor + len(d["payload"]), 64)
        else:
            placed.append(d["ext"])
    nbytes = max(_align(cursor - base, 4096), min_bytes)
    img = bytearray(nbytes)
    struct.pack_into("<6I4Q2I", img, 0, Q.MAGIC, 1, Q.HEADER_BYTES, Q.DESCRIPTOR_BYTES, len(descs), cap, table,
                     payload_base, base, nbytes, 0, 0)
    for i, (d, (addr, n)) in enumerate(zip(descs, placed)):
        off = table - base + i * Q.DESCRIPTOR_BYTES
        rank = len(d["shape"])
        struct.pack_into("<8I2Q", img, off, d["tid"], d["role"], d["dtype"], rank, d["flags"], d["bits"], d["group"],
                         d["scale_tid"], addr, n)
        struct.pack_into("<4I", img, off + 0x30, *(list(d["shape"]) + [0] * (4 - rank)))
        struct.pack_into("<4Q", img, off + 0x40, *(list(d["strides"]) + [0] * (4 - rank)))
        struct.pack_into("<4I", img, off + 0x60, *d["aux"])
        if d["payload"] is not None:
            img[addr - base:addr - base + n] = d["payload"]
    return bytes(img)


def q4_descs(tid_w, tid_s, packed, scale, mid, ext=None) -> list:
    rows, half = packed.shape
    groups = scale.shape[1]
    aux = (mid, 0, 0, 0)
    if ext is None:
        wp, sp, we, se = packed.tobytes(), scale.astype("<u2").tobytes(), None, None
    else:
        wp = sp = None
        we, se = (ext[0], packed.nbytes), (ext[1], scale.nbytes)
    return [desc(tid_w, Q.ROLE_Q4_WEIGHT, Q.DT_PACKED_Q4, (rows, 2 * half), (half, 0), wp, we, PACKED, 4, tid_s, 64,
                 aux),
            desc(tid_s, Q.ROLE_Q4_SCALE, Q.DT_Q2_14, (rows, groups), (2 * groups, 2), sp, se, RO, 16, aux=aux)]


def write_runtime(out_dir, manifest_doc: dict, host: dict, gammas: list, final_gamma, rope_cos, rope_sin,
                  score_scale: int, exp_lut, sigmoid_lut, num_layers: int) -> Path:
    """Segment files + manifest for ``num_layers`` layers of ``host`` (random_host_weights
    layout) at the board runtime's addresses.  ``gammas``: per layer {"input", "post",
    "q", "k"} Q8.7; ``rope_cos`` / ``rope_sin``: Q1.15 [positions, 128]."""
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    doc = copy.deepcopy(manifest_doc)
    entries = {e["name"]: (s, e) for s in doc["segments"] for e in s["entries"]}
    keep = {0, 59, 60, 58}
    for li in range(num_layers):
        keep.add(entries[f"layer{li}.qkv_qmap"][0]["index"])
        keep.add(entries[f"layer{li}.attn_frontend_qmap"][0]["index"])
    doc["segments"] = [s for s in doc["segments"] if s["index"] in keep]
    seg_bytes = {s["index"]: bytearray(int(s["nbytes"])) for s in doc["segments"]}
    seg_of = {e["name"]: s for s in doc["segments"] for e in s["entries"]}

    def put(name: str, data: bytes) -> None:
        s = seg_of[name]
        e = next(e for e in s["entries"] if e["name"] == name)
        if len(data) > int(e["nbytes"]):
            raise ValueError(f"{name}: {len(data)} bytes exceed the entry's {e['nbytes']}")
        o = int(e["address"]) - int(s["address"])
        seg_bytes[s["index"]][o:o + len(data)] = data

    def addr(name: str) -> int:
        return int(next(e for s in doc["segments"] for e in s["entries"] if e["name"] == name)["address"])

    # segment 0: the tied table, shrunk to this vocabulary
    emb_w, emb_s = host["embed_tokens"]
    s0 = next(s for s in doc["segments"] if s["index"] == 0)
    w_addr = int(s0["address"])
    s_addr = w_addr + _align(emb_w.nbytes, 0x10000)
    s0["entries"] = [dict(name="tied_embedding_weight", operation="file", address=w_addr, nbytes=emb_w.nbytes),
                     dict(name="tied_embedding_scale", operation="file", address=s_addr, nbytes=emb_s.nbytes)]
    s0["nbytes"] = s_addr - w_addr + emb_s.nbytes
    seg_bytes[0] = bytearray(s0["nbytes"])
    seg_bytes[0][:emb_w.nbytes] = emb_w.tobytes()
    seg_bytes[0][s_addr - w_addr:] = emb_s.astype("<u2").tobytes()

    rope = words32(np.concatenate([np.asarray(rope_cos).reshape(-1), np.asarray(rope_sin).reshape(-1)]))
    put("runtime_rope_table", rope)
    rope_base = addr("runtime_rope_table")
    plane = np.asarray(rope_cos).size * 4
    positions = np.asarray(rope_cos).shape[0]
    kv_base = 0x4_1410_0000
    for li in range(num_layers):
        L, G = host["layers"][li], gammas[li]
        p = f"layer{li}"
        qkv = []
        for mid, (tw, m) in enumerate(((3, "q_proj"), (5, "k_proj"), (7, "v_proj")), start=1):
            qkv += q4_descs(tw, tw + 1, *L[m], mid)
        base = addr(f"{p}.qkv_qmap")
        put(f"{p}.qkv_qmap", pack_image(base, qkv, capacity=32))
        for m, ent in (("o_proj", "o_proj"), ("gate_proj", "mlp_gate"), ("up_proj", "mlp_up"),
                       ("down_proj", "mlp_down")):
            put(f"{p}.{ent}_weight", L[m][0].tobytes())
            put(f"{p}.{ent}_scale", L[m][1].astype("<u2").tobytes())
        kv = (kv_base + li * 0x20_0000, 2 * 8 * positions * 128 * 4)
        fe = [desc(34, Q.ROLE_PARAMETER, Q.DT_Q8_7, (128,), (4,), words32(G["q"]), bits=16),
              desc(35, Q.ROLE_PARAMETER, Q.DT_Q8_7, (128,), (4,), words32(G["k"]), bits=16),
              desc(36, Q.ROLE_ROPE_TABLE, Q.DT_Q1_15, (positions, 128), (512, 4), ext=(rope_base, plane), bits=16),
              desc(37, Q.ROLE_ROPE_TABLE, Q.DT_Q1_15, (positions, 128), (512, 4), ext=(rope_base + plane, plane),
                   bits=16),
              desc(38, Q.ROLE_KV_CACHE, 19, (2, 8, positions, 128), (8 * positions * 512, positions * 512, 512, 4),
                   ext=kv, flags=Q.F_ROW_MAJOR, bits=24)]
        put(f"{p}.attn_frontend_qmap", pack_image(addr(f"{p}.attn_frontend_qmap"), fe, capacity=16))
        put(f"{p}.input_rmsnorm_qmap", pack_image(addr(f"{p}.input_rmsnorm_qmap"), [
            desc(88, Q.ROLE_PARAMETER, Q.DT_Q8_7, (1024,), (4,), words32(G["input"]), bits=16)]))
        put(f"{p}.post_attn_norm_qmap", pack_image(addr(f"{p}.post_attn_norm_qmap"), [
            desc(54, Q.ROLE_PARAMETER, Q.DT_Q8_7, (1024,), (4,), words32(G["post"]), bits=16)]))
        put(f"{p}.attn_score_value_qmap", pack_image(addr(f"{p}.attn_score_value_qmap"), [
            desc(40, Q.ROLE_METADATA, 5, (16,), (4,), bytes(64), aux=(score_scale, 0, 5, 4)),
            desc(43, Q.ROLE_PARAMETER, Q.DT_Q0_20, (257,), (4,), words32(exp_lut), bits=24)]))
        put(f"{p}.mlp_silu_mul_qmap", pack_image(addr(f"{p}.mlp_silu_mul_qmap"), [
            desc(72, Q.ROLE_PARAMETER, Q.DT_Q0_16, (1025,), (4,), words32(sigmoid_lut), bits=16)]))
        for other in ("o_proj_qmap", "mlp_gate_up_qmap", "mlp_down_qmap", "mlp_residual_add_qmap"):
            put(f"{p}.{other}", pack_image(addr(f"{p}.{other}"), [
                desc(1, Q.ROLE_METADATA, 5, (4,), (4,), bytes(16))]))
    tail = q4_descs(22, 23, emb_w, emb_s, 8, ext=(w_addr, s_addr)) + [
        desc(27, Q.ROLE_PARAMETER, Q.DT_Q8_7, (1024,), (4,), words32(final_gamma), bits=16)]
    put("final_tail_qmap", pack_image(addr("final_tail_qmap"), tail))

    for s in doc["segments"]:
        data = bytes(seg_bytes[s["index"]])
        s["nbytes"] = len(data)
        s["sha256"] = hashlib.sha256(data).hexdigest()
        (out / s["file"]).write_bytes(data)
    doc["segment_count"] = len(doc["segments"])
    doc["total_segment_bytes"] = sum(int(s["nbytes"]) for s in doc["segments"])
    path = out / "pl_ddr_binary_segments.json"
    path.write_text(json.dumps(doc))
    return path
