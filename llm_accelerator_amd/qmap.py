"""QMAP v1 images and the PL-DDR runtime of the board deployment, read into device models.

The board keeps the model in PL DDR4 as 61 binary segments
(``lmdeploy/qwen3-0p6b-q4-qweb-demo/model/pl_ddr_binary_segments.json``): the tied
embedding / LM-head table (segment 0), per layer a q|k|v QMAP image that holds the
q/k/v Q4 weights, the o_proj / gate / up / down weights and scales as raw arrays,
and the per-stage QMAP work packets that carry the layer's parameters (RMSNorm
gammas, q/k norm gammas, RoPE rows, the exp and sigmoid LUTs, the score scale), then
the final-tail packet (final gamma) and the RoPE table.  QMAP itself is
``Source/QMAP_FORMAT.md:134-296``: a 256-byte header, 128-byte tensor descriptors,
payloads at absolute byte addresses.

This module parses and validates images and manifests (``QmapImage``,
``SegmentManifest``), resolves descriptor addresses in an ``AddressSpace`` assembled
from segment files (or any images), and builds the device models:
``load_runtime(manifest, segment_dir)`` -> ``BoardRuntime`` with ``host_weights()``
(the layout ``model.build_model`` takes) and ``fixed_model(model)`` (the
RTL-exact ``fixed.FixedQ4Model`` with the board's own Q8.7 gammas and Q1.15 table).
Q4 payloads need no conversion: QMAP ``PACKED_Q4_S4`` / ``U16_Q2_14`` is the on-device
format.
"""

from __future__ import annotations

import hashlib
import json
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

MAGIC = 0x50414D51  # "QMAP"
HEADER_BYTES = 256
DESCRIPTOR_BYTES = 128

# Role and dtype enums (QMAP_FORMAT.md:218-253), tensor flags (:255-263).
ROLE_UNUSED, ROLE_ACTIVATION, ROLE_Q4_WEIGHT, ROLE_Q4_SCALE, ROLE_OUTPUT, ROLE_EXPECTED, ROLE_METADATA, \
    ROLE_KV_CACHE, ROLE_ROPE_TABLE, ROLE_PARAMETER = range(10)
F_ROW_MAJOR, F_PACKED_Q4_LOW_EVEN, F_READ_ONLY, F_WRITE_ONLY, F_DEBUG_ONLY = (1, 2, 4, 8, 16)
# Signed dtypes (QMAP_FORMAT.md:230-253); the rest are unsigned.  Storage width comes
# from the descriptor's innermost byte stride: the fixed-point types of the decode
# stages sit widened in 32-bit words, Q2.14 scales and the dot-product inputs in 16.
SIGNED_DTYPES = {2, 4, 6, 8, 18, 19, 20, 22, 23}
KNOWN_DTYPES = {1, 2, 3, 4, 5, 6, 7, 8, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25}
DT_PACKED_Q4, DT_Q2_14, DT_Q8_7, DT_Q1_15, DT_Q0_20, DT_Q0_16 = 16, 17, 22, 23, 24, 25
MATRIX_IDS = {1: "q_proj", 2: "k_proj", 3: "v_proj", 4: "o_proj", 5: "gate_proj", 6: "up_proj", 7: "down_proj",
              8: "embed_lm_head"}


class QmapError(ValueError):
    """A malformed image, manifest or address."""


@dataclass
class Descriptor:
    tensor_id: int
    role: int
    dtype: int
    rank: int
    flags: int
    element_bits: int
    group_size: int
    scale_tensor_id: int
    base_addr: int
    nbytes: int
    dims: tuple
    strides_bytes: tuple
    aux: tuple
    checksum32: int

    @property
    def shape(self) -> tuple:
        return tuple(int(d) for d in self.dims[:self.rank])


@dataclass
class QmapImage:
    """One QMAP image: header fields, descriptors and its bytes (relocatable: payloads are
    read relative to ``image_base_addr``)."""
    version: int
    descriptor_count: int
    descriptor_capacity: int
    descriptor_table_addr: int
    payload_base_addr: int
    image_base_addr: int
    image_bytes: int
    flags: int
    descriptors: list
    data: bytes = field(repr=False)

    @classmethod
    def parse(cls, data: bytes) -> "QmapImage":
        data = bytes(data)
        if len(data) < HEADER_BYTES:
            raise QmapError(f"image of {len(data)} bytes is shorter than the {HEADER_BYTES}-byte header")
        magic, version, hb, db, count, cap, dta, pba, iba, ib, flags, _ck = struct.unpack_from("<6I4Q2I", data, 0)
        if magic != MAGIC:
            raise QmapError(f"bad magic 0x{magic:08X}")
        if version != 1 or hb != HEADER_BYTES or db != DESCRIPTOR_BYTES:
            raise QmapError(f"unsupported QMAP version/sizes {version}/{hb}/{db}")
        if count > cap:
            raise QmapError(f"{count} descriptors exceed the {cap} reserved slots")
        if ib != len(data):
            raise QmapError(f"header says {ib} image bytes, the image has {len(data)}")
        if any(struct.unpack_from("<48I", data, 0x40)):
            raise QmapError("reserved header words are not zero")
        t0 = dta - iba
        if t0 < HEADER_BYTES or t0 + cap * DESCRIPTOR_BYTES > pba - iba or pba - iba > len(data):
            raise QmapError("descriptor table overlaps the header or the payload region")
        descs = []
        for i in range(count):
            off = t0 + i * DESCRIPTOR_BYTES
            tid, role, dtype, rank, fl, eb, gs, stid, base, nb = struct.unpack_from("<8I2Q", data, off)
            dims = struct.unpack_from("<4I", data, off + 0x30)
            strides = struct.unpack_from("<4Q", data, off + 0x40)
            aux = struct.unpack_from("<4I", data, off + 0x60)
            ck = struct.unpack_from("<I", data, off + 0x70)[0]
            if role > ROLE_PARAMETER or dtype not in KNOWN_DTYPES or not 1 <= rank <= 4:
                raise QmapError(f"descriptor {tid}: role {role} / dtype {dtype} / rank {rank} not in QMAP v1")
            descs.append(Descriptor(tid, role, dtype, rank, fl, eb, gs, stid, base, nb, dims, strides, aux, ck))
        img = cls(version, count, cap, dta, pba, iba, ib, flags, descs, data)
        img._check_payloads()
        return img

    @classmethod
    def from_words32_hex(cls, path: str | Path) -> "QmapImage":
        """The repository's ``*_words32.hex`` form: one little-endian 32-bit word per line."""
        words = np.array([int(w, 16) for w in Path(path).read_text().split()], dtype="<u4")
        return cls.parse(words.view(np.uint8).tobytes())

    def _check_payloads(self) -> None:
        ids = set()
        spans = []
        for d in self.descriptors:
            if d.tensor_id in ids:
                raise QmapError(f"duplicate tensor id {d.tensor_id}")
            ids.add(d.tensor_id)
            if self.contains(d.base_addr):
                if d.base_addr < self.payload_base_addr or d.base_addr + d.nbytes > self.image_base_addr + self.image_bytes:
                    raise QmapError(f"tensor {d.tensor_id} payload leaves the image's payload region")
                spans.append((d.base_addr, d.base_addr + d.nbytes, d.tensor_id))
            if d.base_addr % 4:
                raise QmapError(f"tensor {d.tensor_id} payload is not 4-byte aligned")
            need = expected_nbytes(d)
            if need is not None and d.nbytes < need:
                raise QmapError(f"tensor {d.tensor_id}: {d.nbytes} bytes hold less than its shape {d.shape}")
        spans.sort()
        for (a0, a1, t0), (b0, b1, t1) in zip(spans, spans[1:]):
            if b0 < a1:
                raise QmapError(f"payloads of tensors {t0} and {t1} overlap")

    def contains(self, addr: int) -> bool:
        return self.image_base_addr <= addr < self.image_base_addr + self.image_bytes

    def by_id(self, tensor_id: int) -> Descriptor:
        for d in self.descriptors:
            if d.tensor_id == tensor_id:
                return d
        raise QmapError(f"no tensor id {tensor_id}")

    def find(self, role: int, dtype: int | None = None, **aux) -> list:
        out = [d for d in self.descriptors if d.role == role and (dtype is None or d.dtype == dtype)]
        for k, v in aux.items():
            i = {"aux0": 0, "aux1": 1, "aux2": 2, "aux3": 3}[k]
            out = [d for d in out if d.aux[i] == v]
        return out


def _storage_bytes(d: Descriptor) -> int:
    if d.dtype == DT_PACKED_Q4:
        return 1
    sb = int(d.strides_bytes[d.rank - 1])
    if sb not in (1, 2, 4, 8) or sb * 8 < d.element_bits:
        raise QmapError(f"tensor {d.tensor_id}: innermost stride {sb} cannot hold {d.element_bits}-bit elements")
    return sb


def expected_nbytes(d: Descriptor) -> int | None:
    """Bytes the descriptor's shape and strides span (packed Q4: rows of cols/2 bytes at
    the row stride, ``QMAP_FORMAT.md:320-335``)."""
    shape = d.shape
    if d.dtype == DT_PACKED_Q4:
        if shape[-1] % 2:
            raise QmapError(f"tensor {d.tensor_id}: packed Q4 with an odd column count")
        lead = sum((n - 1) * int(s) for n, s in zip(shape[:-1], d.strides_bytes))
        return lead + shape[-1] // 2
    if any(n == 0 for n in shape):
        return 0
    return sum((n - 1) * int(s) for n, s in zip(shape, d.strides_bytes)) + _storage_bytes(d)


class AddressSpace:
    """Byte regions at absolute addresses (segment files, images); reads must fall in one."""

    def __init__(self):
        self.regions = []  # (start, memoryview-like)

    def add(self, addr: int, data) -> None:
        buf = memoryview(data).cast("B") if not isinstance(data, np.ndarray) else memoryview(data.reshape(-1).view(np.uint8))
        for s, b in self.regions:
            if addr < s + len(b) and s < addr + len(buf):
                raise QmapError(f"region at 0x{addr:X} overlaps region at 0x{s:X}")
        self.regions.append((addr, buf))

    def add_image(self, img: QmapImage) -> None:
        self.add(img.image_base_addr, img.data)

    def read(self, addr: int, nbytes: int) -> memoryview:
        for s, b in self.regions:
            if s <= addr and addr + nbytes <= s + len(b):
                return b[addr - s:addr - s + nbytes]
        raise QmapError(f"0x{addr:X}+{nbytes} is not inside one loaded region")


def tensor(d: Descriptor, image: QmapImage | None = None, space: AddressSpace | None = None) -> np.ndarray:
    """The payload of ``d`` as a contiguous numpy array read through its strides: packed Q4
    as bytes [rows, cols/2], every other dtype as its storage integer (sign taken from
    the dtype) in the logical shape."""
    n = expected_nbytes(d)
    if image is not None and image.contains(d.base_addr):
        off = d.base_addr - image.image_base_addr
        if off + n > image.image_bytes:
            raise QmapError(f"tensor {d.tensor_id} runs past the image")
        raw = image.data[off:off + n]
    elif space is not None:
        raw = bytes(space.read(d.base_addr, n))
    else:
        raise QmapError(f"tensor {d.tensor_id} at 0x{d.base_addr:X} is outside the image and no address space given")
    shape = d.shape
    if d.dtype == DT_PACKED_Q4:
        out_shape = shape[:-1] + (shape[-1] // 2,)
        strides = tuple(int(s) for s in d.strides_bytes[:len(shape) - 1]) + (1,)
        dt = np.dtype(np.uint8)
    else:
        sb = _storage_bytes(d)
        dt = np.dtype(("<i" if d.dtype in SIGNED_DTYPES else "<u") + str(sb))
        out_shape, strides = shape, tuple(int(s) for s in d.strides_bytes[:len(shape)])
    if n == 0:
        return np.zeros(out_shape, dt)
    return np.ndarray(out_shape, dt, buffer=raw, strides=strides).copy()


# ---------------------------------------------------------------- the PL-DDR runtime manifest
@dataclass
class SegmentEntry:
    name: str
    operation: str  # "file" (bytes from the segment file) or "zero"
    address: int
    nbytes: int
    segment: int


class SegmentManifest:
    """``pl_ddr_binary_segments.json``: segments (file, address, bytes, sha256) and the
    named entries inside them."""

    def __init__(self, doc: dict):
        self.doc = doc
        self.segments = doc["segments"]
        if len(self.segments) != doc.get("segment_count", len(self.segments)):
            raise QmapError("segment_count disagrees with the segment list")
        self.entries = {}
        for s in self.segments:
            s0, s1 = int(s["address"]), int(s["address"]) + int(s["nbytes"])
            for e in s["entries"]:
                a, n = int(e["address"]), int(e["nbytes"])
                if not (s0 <= a and a + n <= s1):
                    raise QmapError(f"entry {e['name']} leaves segment {s['index']}")
                if e["name"] in self.entries:
                    raise QmapError(f"duplicate entry {e['name']}")
                self.entries[e["name"]] = SegmentEntry(e["name"], e["operation"], a, n, int(s["index"]))
        spans = sorted((int(s["address"]), int(s["address"]) + int(s["nbytes"]), s["index"]) for s in self.segments)
        for (a0, a1, i0), (b0, b1, i1) in zip(spans, spans[1:]):
            if b0 < a1:
                raise QmapError(f"segments {i0} and {i1} overlap")
        total = sum(int(s["nbytes"]) for s in self.segments)
        if total != doc.get("total_segment_bytes", total):
            raise QmapError("total_segment_bytes disagrees with the segments")

    @classmethod
    def load(cls, path: str | Path) -> "SegmentManifest":
        return cls(json.loads(Path(path).read_text()))

    @property
    def num_layers(self) -> int:
        return sum(1 for n in self.entries if n.endswith(".qkv_qmap"))

    def address_space(self, segment_dir: str | Path, verify_sha256: bool = True) -> AddressSpace:
        """Map every segment file (read in full; zero entries stay zero) into an AddressSpace."""
        space = AddressSpace()
        d = Path(segment_dir)
        for s in self.segments:
            f = d / s["file"]
            if not f.exists():
                raise FileNotFoundError(f"segment {s['index']} file {f} is missing")
            data = f.read_bytes()
            if len(data) != int(s["nbytes"]):
                raise QmapError(f"segment file {f} has {len(data)} bytes, the manifest says {s['nbytes']}")
            if verify_sha256 and s.get("sha256") and hashlib.sha256(data).hexdigest() != s["sha256"]:
                raise QmapError(f"segment file {f} does not match its sha256")
            space.add(int(s["address"]), data)
        return space


# ---------------------------------------------------------------- runtime -> device model
@dataclass
class BoardRuntime:
    """The model the board runtime holds, read out of its address space."""
    layers: list            # per layer: {"q_proj": (packed, scale), ..., gammas as int16 Q8.7}
    embed: tuple            # tied (packed [vocab, 512], scale [vocab, 16])
    final_gamma: np.ndarray  # int16 Q8.7
    rope_cos: np.ndarray    # int16 Q1.15 [positions, 128]
    rope_sin: np.ndarray
    score_scale: int
    exp_lut: np.ndarray
    sigmoid_lut: np.ndarray

    def host_weights(self) -> dict:
        """``model.random_host_weights``-shaped dict (Q4 arrays + float gammas = Q8.7 / 128)."""
        g = lambda v: (np.asarray(v, np.float32) / np.float32(128.0)).astype(np.float32)  # noqa: E731
        mats = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
        layers = []
        for L in self.layers:
            d = {m: L[m] for m in mats}
            d.update(input_layernorm=g(L["input_gamma"]), post_attention_layernorm=g(L["post_gamma"]),
                     q_norm=g(L["q_gamma"]), k_norm=g(L["k_gamma"]))
            layers.append(d)
        return {"layers": layers, "embed_tokens": self.embed, "norm": g(self.final_gamma)}

    def fixed_model(self, model):
        """The RTL-exact model over ``model`` (a Q4ForCausalLM built from ``host_weights()``)
        with the board's own gammas, RoPE table and score scale.  The library's exp and
        sigmoid tables must equal the board's (they are built once in the library)."""
        from .fixed import FixedQ4Model, build_exp_lut, build_sigmoid_lut
        if not (np.array_equal(self.exp_lut, build_exp_lut()) and np.array_equal(self.sigmoid_lut, build_sigmoid_lut())):
            raise QmapError("the runtime's exp / sigmoid LUTs differ from the library's")
        if model.max_ctx > self.rope_cos.shape[0]:
            raise QmapError(f"model context {model.max_ctx} exceeds the runtime's {self.rope_cos.shape[0]}-position "
                            "RoPE table")
        return FixedQ4Model.from_parts(model, [{"input": L["input_gamma"], "post": L["post_gamma"], "q": L["q_gamma"],
                                                "k": L["k_gamma"]} for L in self.layers], self.final_gamma,
                                       self.rope_cos[:model.max_ctx], self.rope_sin[:model.max_ctx], self.score_scale)


def _raw_matrix(space: AddressSpace, man: SegmentManifest, name: str, rows: int, cols: int) -> tuple:
    w = man.entries[f"{name}_weight"]
    s = man.entries[f"{name}_scale"]
    if w.nbytes != rows * cols // 2 or s.nbytes != rows * (cols // 64) * 2:
        raise QmapError(f"{name}: {w.nbytes} / {s.nbytes} bytes do not hold a {rows} x {cols} Q4 matrix")
    packed = np.frombuffer(space.read(w.address, w.nbytes), np.uint8).reshape(rows, cols // 2).copy()
    scale = np.frombuffer(space.read(s.address, s.nbytes), "<u2").reshape(rows, cols // 64).astype(np.uint16)
    return packed, scale


def _packet(space: AddressSpace, man: SegmentManifest, name: str) -> QmapImage:
    e = man.entries[name]
    if e.nbytes < HEADER_BYTES:
        raise QmapError(f"{name}: {e.nbytes} bytes cannot hold a QMAP header")
    ib = struct.unpack_from("<Q", space.read(e.address, HEADER_BYTES), 0x30)[0]
    if ib > e.nbytes:
        raise QmapError(f"{name}: image of {ib} bytes exceeds its {e.nbytes}-byte entry")
    img = QmapImage.parse(bytes(space.read(e.address, ib)))
    if img.image_base_addr != e.address:
        raise QmapError(f"{name}: image based at 0x{img.image_base_addr:X}, loaded at 0x{e.address:X}")
    return img


def _one(lst: list, what: str) -> Descriptor:
    if len(lst) != 1:
        raise QmapError(f"expected one {what}, found {len(lst)}")
    return lst[0]


def read_runtime(man: SegmentManifest, space: AddressSpace, hidden: int = 1024, intermediate: int = 3072,
                 q_heads: int = 16, kv_heads: int = 8, head_dim: int = 128) -> BoardRuntime:
    """The model held by a loaded runtime (names follow the board manifest)."""
    qd, kd = q_heads * head_dim, kv_heads * head_dim
    layers = []
    exp_lut = sigmoid_lut = rope = None
    score_scale = None
    for li in range(man.num_layers):
        p = f"layer{li}"
        qkv = _packet(space, man, f"{p}.qkv_qmap")
        L = {}
        for mid, name, rows in ((1, "q_proj", qd), (2, "k_proj", kd), (3, "v_proj", kd)):
            wd = _one(qkv.find(ROLE_Q4_WEIGHT, DT_PACKED_Q4, aux0=mid), f"{p} {name} weight")
            if wd.shape != (rows, hidden) or not wd.flags & F_PACKED_Q4_LOW_EVEN:
                raise QmapError(f"{p} {name}: shape {wd.shape} / flags {wd.flags}")
            sd = qkv.by_id(wd.scale_tensor_id)
            L[name] = (tensor(wd, qkv, space), tensor(sd, qkv, space))
        L["o_proj"] = _raw_matrix(space, man, f"{p}.o_proj", hidden, qd)
        L["gate_proj"] = _raw_matrix(space, man, f"{p}.mlp_gate", intermediate, hidden)
        L["up_proj"] = _raw_matrix(space, man, f"{p}.mlp_up", intermediate, hidden)
        L["down_proj"] = _raw_matrix(space, man, f"{p}.mlp_down", hidden, intermediate)
        fe = _packet(space, man, f"{p}.attn_frontend_qmap")
        # q gamma precedes k gamma, cos precedes sin, by tensor id (37_...:54-57)
        gam = sorted((d for d in fe.find(ROLE_PARAMETER, DT_Q8_7) if d.shape == (head_dim,)),
                     key=lambda d: d.tensor_id)
        if len(gam) != 2:
            raise QmapError(f"{p} attention front end: {len(gam)} q/k gammas")
        L["q_gamma"], L["k_gamma"] = (tensor(d, fe, space) for d in gam)
        trig = sorted(fe.find(ROLE_ROPE_TABLE, DT_Q1_15), key=lambda d: d.tensor_id)
        if len(trig) != 2 or trig[0].rank != 2 or trig[0].shape[1] != head_dim or trig[0].shape != trig[1].shape:
            raise QmapError(f"{p} attention front end: no [positions, {head_dim}] cos/sin table "
                            "(a single-position packet is not a runtime packet)")
        cos, sin = (tensor(d, fe, space) for d in trig)
        if rope is None:
            rope = (cos, sin)
        elif not (np.array_equal(cos, rope[0]) and np.array_equal(sin, rope[1])):
            raise QmapError(f"{p}: RoPE table differs from layer 0")
        for key, packet in (("input_gamma", "input_rmsnorm_qmap"), ("post_gamma", "post_attn_norm_qmap")):
            img = _packet(space, man, f"{p}.{packet}")
            d = _one([d for d in img.find(ROLE_PARAMETER, DT_Q8_7) if d.shape == (hidden,)], f"{p} {key}")
            L[key] = tensor(d, img, space)
        sv = _packet(space, man, f"{p}.attn_score_value_qmap")
        lut = tensor(_one(sv.find(ROLE_PARAMETER, DT_Q0_20), f"{p} exp LUT"), sv, space)
        sc = int(_one(sv.find(ROLE_METADATA), f"{p} score metadata").aux[0])
        si = _packet(space, man, f"{p}.mlp_silu_mul_qmap")
        sig = tensor(_one(si.find(ROLE_PARAMETER, DT_Q0_16), f"{p} sigmoid LUT"), si, space)
        if exp_lut is None:
            exp_lut, sigmoid_lut, score_scale = lut, sig, sc
        elif not (np.array_equal(lut, exp_lut) and np.array_equal(sig, sigmoid_lut) and sc == score_scale):
            raise QmapError(f"{p}: LUTs or score scale differ from layer 0")
        layers.append(L)
    tail = _packet(space, man, "final_tail_qmap")
    emb_w = _one(tail.find(ROLE_Q4_WEIGHT, DT_PACKED_Q4), "LM-head weight")
    embed = (tensor(emb_w, tail, space), tensor(tail.by_id(emb_w.scale_tensor_id), tail, space))
    final_gamma = tensor(_one(tail.find(ROLE_PARAMETER, DT_Q8_7), "final gamma"), tail, space)
    return BoardRuntime(layers, embed, final_gamma, rope[0].astype(np.int16), rope[1].astype(np.int16),
                        score_scale, exp_lut.astype(np.int64), sigmoid_lut.astype(np.int64))


def load_runtime(manifest: str | Path, segment_dir: str | Path, verify_sha256: bool = True) -> BoardRuntime:
    """Read the board's PL-DDR runtime (manifest + its segment files) into a BoardRuntime."""
    man = SegmentManifest.load(manifest)
    return read_runtime(man, man.address_space(segment_dir, verify_sha256))


__all__ = ["QmapImage", "Descriptor", "QmapError", "AddressSpace", "tensor", "SegmentManifest", "SegmentEntry",
           "BoardRuntime", "read_runtime", "load_runtime", "expected_nbytes", "MATRIX_IDS"]
