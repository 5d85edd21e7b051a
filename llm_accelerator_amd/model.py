"""Device-resident Qwen3-0.6B Q4 model, KV cache and workspace.

The object graph mirrors the attribute surface the reference's Python path
reads from the Hugging Face model (``Qwen3-0.6B-Base/python_each_module/
common.py:245-296`` and ``10_validate_full_run_one_token.py:31,53-54``):
``model.model.layers[i].self_attn.q_proj.weight``, ``.mlp.gate_proj.weight``,
``.input_layernorm.weight``, ``model.model.rotary_emb.inv_freq``,
``model.model.norm.weight``, ``model.lm_head.weight`` (tied to
``model.model.embed_tokens.weight``) and ``model.config``.  Every ``.weight``
of a projection is a :class:`Q4Tensor` in the reference Q4 layout
(``Source/Q4_FORMAT.md:75-140``).

Synthetic weights: packed bytes uniform over 0..255 (two independent uniform
int4 codes per byte, read as signed values in [-8, 7]); scale codes
``max(1, rint(|N(0, 0.02)| * 2**14))`` as uint16 Q2.14 (the nonzero rule of
``13_export_q4_gemv_vectors.py:115-121``); RMSNorm gammas ``1 + N(0, 0.1)``
rounded to fp16 values and stored as fp32.
"""

from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _lib
from ._lib import Q4dKVCache, Q4dLayer, Q4dMatrix, Q4dModel

GROUP_SIZE = 64


@dataclass
class Qwen3Config:
    """Hyperparameters of ``Qwen3-0.6B-Base/config.json:1-30``."""
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    vocab_size: int = 151936
    tie_word_embeddings: bool = True
    max_position_embeddings: int = 32768

    @classmethod
    def from_json(cls, path: str | Path) -> "Qwen3Config":
        d = json.loads(Path(path).read_text())
        keys = cls.__dataclass_fields__.keys()
        return cls(**{k: d[k] for k in keys if k in d})

    @property
    def kv_repeat(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @property
    def scaling(self) -> float:
        return float(self.head_dim) ** -0.5


class Q4Tensor:
    """Q4 weight: ``packed`` uint8 [rows, cols/2] and ``scale`` uint16 [rows, cols/64]."""

    def __init__(self, packed: torch.Tensor, scale: torch.Tensor):
        if packed.dtype != torch.uint8 or scale.dtype != torch.uint16:
            raise TypeError("Q4Tensor needs uint8 packed codes and uint16 Q2.14 scales")
        rows, half = packed.shape
        if scale.shape != (rows, 2 * half // GROUP_SIZE):
            raise ValueError(f"scale shape {tuple(scale.shape)} does not match packed {tuple(packed.shape)}")
        self.packed = packed.contiguous()
        self.scale = scale.contiguous()

    @property
    def shape(self) -> tuple[int, int]:
        return (self.packed.shape[0], self.packed.shape[1] * 2)

    @property
    def device(self) -> torch.device:
        return self.packed.device

    @property
    def nbytes(self) -> int:
        return self.packed.numel() + 2 * self.scale.numel()

    def to(self, device) -> "Q4Tensor":
        return Q4Tensor(self.packed.to(device), self.scale.to(device))

    def descriptor(self) -> Q4dMatrix:
        r, c = self.shape
        return Q4dMatrix(self.packed.data_ptr(), self.scale.data_ptr(), r, c)

    def numpy(self) -> tuple[np.ndarray, np.ndarray]:
        return self.packed.cpu().numpy(), self.scale.cpu().numpy()

    @classmethod
    def from_numpy(cls, packed: np.ndarray, scale: np.ndarray, device="cpu") -> "Q4Tensor":
        return cls(torch.from_numpy(np.ascontiguousarray(packed, dtype=np.uint8)).to(device),
                   torch.from_numpy(np.ascontiguousarray(scale, dtype=np.uint16)).to(device))


class _Linear:
    def __init__(self, weight: Q4Tensor):
        self.weight = weight
        self.bias = None


class _RMSNorm:
    def __init__(self, weight: torch.Tensor, eps: float):
        self.weight = weight
        self.variance_epsilon = eps


class _Attention:
    def __init__(self, q, k, v, o, q_norm, k_norm, cfg: Qwen3Config):
        self.q_proj, self.k_proj, self.v_proj, self.o_proj = q, k, v, o
        self.q_norm, self.k_norm = q_norm, k_norm
        self.scaling = cfg.scaling
        self.head_dim = cfg.head_dim


class _MLP:
    def __init__(self, gate, up, down):
        self.gate_proj, self.up_proj, self.down_proj = gate, up, down


class Q4DecoderLayer:
    def __init__(self, self_attn: _Attention, mlp: _MLP, input_layernorm: _RMSNorm,
                 post_attention_layernorm: _RMSNorm):
        self.self_attn = self_attn
        self.mlp = mlp
        self.input_layernorm = input_layernorm
        self.post_attention_layernorm = post_attention_layernorm


class RotaryEmbedding:
    """``inv_freq`` exactly as the HF default RoPE init computes it (fp32),
    ``attention_scaling`` = 1, plus device cos/sin tables [max_ctx, head_dim/2]
    holding ``cos(pos * inv_freq)`` / ``sin(pos * inv_freq)`` in fp32 (the
    values ``manual_rope_cos_sin`` forms, common.py:155-170)."""

    def __init__(self, cfg: Qwen3Config, max_ctx: int, device):
        d = cfg.head_dim
        self.inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
        self.attention_scaling = 1.0
        pos = torch.arange(max_ctx, dtype=torch.float32)[:, None]
        freqs = pos @ self.inv_freq[None, :].float()
        self.cos_table = (freqs.cos() * self.attention_scaling).contiguous().to(device)
        self.sin_table = (freqs.sin() * self.attention_scaling).contiguous().to(device)
        self.max_ctx = max_ctx


class Q4Backbone:
    def __init__(self, layers, embed_tokens: _Linear, norm: _RMSNorm, rotary_emb: RotaryEmbedding):
        self.layers = layers
        self.embed_tokens = embed_tokens
        self.norm = norm
        self.rotary_emb = rotary_emb


class Q4ForCausalLM:
    """HF-shaped container; ``descriptor()`` builds the C-ABI model struct."""

    def __init__(self, config: Qwen3Config, backbone: Q4Backbone, max_ctx: int):
        self.config = config
        self.model = backbone
        self.lm_head = backbone.embed_tokens  # tie_word_embeddings
        self.max_ctx = max_ctx
        self._desc = None
        for i, layer in enumerate(backbone.layers):
            layer._q4d_owner = self  # lets the fused layer call find its model descriptor
            layer._q4d_index = i

    @property
    def device(self) -> torch.device:
        return self.model.embed_tokens.weight.device

    def descriptor(self) -> Q4dModel:
        if self._desc is not None:
            return self._desc
        cfg, bb = self.config, self.model
        arr = (Q4dLayer * len(bb.layers))()
        for i, L in enumerate(bb.layers):
            a, m = L.self_attn, L.mlp
            arr[i] = Q4dLayer(a.q_proj.weight.descriptor(), a.k_proj.weight.descriptor(),
                              a.v_proj.weight.descriptor(), a.o_proj.weight.descriptor(),
                              m.gate_proj.weight.descriptor(), m.up_proj.weight.descriptor(),
                              m.down_proj.weight.descriptor(), L.input_layernorm.weight.data_ptr(),
                              L.post_attention_layernorm.weight.data_ptr(), a.q_norm.weight.data_ptr(),
                              a.k_norm.weight.data_ptr())
        d = Q4dModel(cfg.hidden_size, cfg.intermediate_size, len(bb.layers), cfg.num_attention_heads,
                     cfg.num_key_value_heads, cfg.head_dim, cfg.vocab_size, self.max_ctx, cfg.rms_norm_eps,
                     cfg.scaling, ctypes.cast(arr, ctypes.POINTER(Q4dLayer)),
                     bb.embed_tokens.weight.descriptor(), bb.norm.weight.data_ptr(),
                     bb.rotary_emb.cos_table.data_ptr(), bb.rotary_emb.sin_table.data_ptr())
        d._layers_keepalive = arr  # type: ignore[attr-defined]
        self._desc = d
        return d

    def weight_bytes(self) -> dict:
        per_layer = sum(getattr(getattr(L, blk), n).weight.nbytes
                        for L in self.model.layers[:1]
                        for blk, names in (("self_attn", ("q_proj", "k_proj", "v_proj", "o_proj")),
                                           ("mlp", ("gate_proj", "up_proj", "down_proj")))
                        for n in names)
        return {"per_layer": per_layer, "lm_head": self.lm_head.weight.nbytes,
                "total": per_layer * len(self.model.layers) + self.lm_head.weight.nbytes}


def with_context(model: Q4ForCausalLM, max_ctx: int) -> Q4ForCausalLM:
    """The same device weights under another context capacity (its own RoPE tables
    and descriptor); the layers keep pointing at ``model`` for the fused layer call."""
    bb = model.model
    view = Q4ForCausalLM.__new__(Q4ForCausalLM)
    view.config = model.config
    view.model = Q4Backbone(bb.layers, bb.embed_tokens, bb.norm, RotaryEmbedding(model.config, max_ctx, model.device))
    view.lm_head = view.model.embed_tokens
    view.max_ctx = max_ctx
    view._desc = None
    return view


# ---------------------------------------------------------------- synthetic init
def random_q4(rng: np.random.Generator, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray]:
    packed = rng.integers(0, 256, size=(rows, cols // 2), dtype=np.uint8)
    s = np.abs(rng.normal(0.0, 0.02, size=(rows, cols // GROUP_SIZE)).astype(np.float32))
    code = np.maximum(1, np.rint(s * np.float32(16384.0))).astype(np.uint16)
    return packed, code


def random_gamma(rng: np.random.Generator, n: int) -> np.ndarray:
    return (1.0 + rng.normal(0.0, 0.1, size=n)).astype(np.float16).astype(np.float32)


def random_host_weights(cfg: Qwen3Config, seed: int = 0, num_layers: int | None = None) -> dict:
    """Seeded synthetic Q4 weights as numpy arrays (shared by device and oracle)."""
    rng = np.random.default_rng(seed)
    h, i = cfg.hidden_size, cfg.intermediate_size
    qd, kd = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    shapes = {"q_proj": (qd, h), "k_proj": (kd, h), "v_proj": (kd, h), "o_proj": (h, qd),
              "gate_proj": (i, h), "up_proj": (i, h), "down_proj": (h, i)}
    layers = []
    for _ in range(cfg.num_hidden_layers if num_layers is None else num_layers):
        L = {n: random_q4(rng, *s) for n, s in shapes.items()}
        L["input_layernorm"] = random_gamma(rng, h)
        L["post_attention_layernorm"] = random_gamma(rng, h)
        L["q_norm"] = random_gamma(rng, cfg.head_dim)
        L["k_norm"] = random_gamma(rng, cfg.head_dim)
        layers.append(L)
    embed = random_q4(rng, cfg.vocab_size, h)
    return {"layers": layers, "embed_tokens": embed, "norm": random_gamma(rng, h)}


def build_model(cfg: Qwen3Config, host: dict, max_ctx: int, device="cuda") -> Q4ForCausalLM:
    """Upload host weights (from :func:`random_host_weights`) to `device`."""
    eps = cfg.rms_norm_eps

    def vec(a):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)

    layers = []
    for L in host["layers"]:
        lin = {n: _Linear(Q4Tensor.from_numpy(*L[n], device=device)) for n in
               ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")}
        attn = _Attention(lin["q_proj"], lin["k_proj"], lin["v_proj"], lin["o_proj"],
                          _RMSNorm(vec(L["q_norm"]), eps), _RMSNorm(vec(L["k_norm"]), eps), cfg)
        mlp = _MLP(lin["gate_proj"], lin["up_proj"], lin["down_proj"])
        layers.append(Q4DecoderLayer(attn, mlp, _RMSNorm(vec(L["input_layernorm"]), eps),
                                     _RMSNorm(vec(L["post_attention_layernorm"]), eps)))
    emb = _Linear(Q4Tensor.from_numpy(*host["embed_tokens"], device=device))
    bb = Q4Backbone(layers, emb, _RMSNorm(vec(host["norm"]), eps), RotaryEmbedding(cfg, max_ctx, device))
    return Q4ForCausalLM(cfg, bb, max_ctx)


# ---------------------------------------------------------------- KV cache
class KVCache:
    """fp16 cache [layers][2 (K,V)][batch][kv_heads][max_ctx][head_dim]
    (the reference's [layer][kind][head][pos][dim] order,
    ``23_export_kv_cache_append_vectors.py:64-84``, with a batch axis)."""

    def __init__(self, cfg: Qwen3Config, num_layers: int, batch: int, max_ctx: int, device="cuda"):
        self.data = torch.zeros((num_layers, 2, batch, cfg.num_key_value_heads, max_ctx, cfg.head_dim),
                                dtype=torch.float16, device=device)
        self.num_layers, self.batch, self.max_ctx = num_layers, batch, max_ctx
        self.num_kv_heads, self.head_dim = cfg.num_key_value_heads, cfg.head_dim
        self.length = [0] * batch

    def k(self, layer: int) -> torch.Tensor:
        return self.data[layer, 0]

    def v(self, layer: int) -> torch.Tensor:
        return self.data[layer, 1]

    def descriptor(self) -> Q4dKVCache:
        return Q4dKVCache(self.data.data_ptr(), self.num_layers, self.batch, self.num_kv_heads, self.max_ctx,
                          self.head_dim)


class Workspace:
    """Caller-owned scratch for the fused entry points (q4d_workspace_bytes)."""

    def __init__(self, model: Q4ForCausalLM, batch: int = 1):
        lib = _lib.load()
        desc = model.descriptor()
        self.nbytes = int(lib.q4d_workspace_bytes(ctypes.byref(desc), batch))
        if self.nbytes == 0:
            raise _lib.Q4DecError(-11, "q4d_workspace_bytes")
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=model.device)
        self.batch = batch
        self._desc = desc
        self.reset()

    @property
    def ptr(self) -> int:
        return self.buf.data_ptr()

    def reset(self) -> None:
        """Zero the status word, counters and exchange flags (q4d_workspace_init)."""
        _lib.check(_lib.load().q4d_workspace_init(self.buf.data_ptr(), self.nbytes, ctypes.byref(self._desc),
                                                  self.batch, current_stream()), "q4d_workspace_init")

    def status(self) -> int:
        """The device status word (Q4D_STATUS_* bits; synchronises the stream)."""
        out = ctypes.c_int32(0)
        _lib.check(_lib.load().q4d_read_status(self.buf.data_ptr(), self.nbytes, ctypes.byref(self._desc),
                                               self.batch, ctypes.byref(out), current_stream()), "q4d_read_status")
        return out.value

    def raise_for_status(self, what: str) -> None:
        """Raise Q4DecError(Q4D_ERR_STATUS) if the status word has a bit set; the
        workspace is reset first, so the next call starts from a clean state."""
        st = self.status()
        if st:
            self.reset()
            _lib.check_status(st, what)


def current_stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def algorithmic_bytes_layer(cfg: Qwen3Config, ctx: int) -> int:
    """HBM bytes one decode step of one layer must move at context ``ctx``
    (positions attended = ctx + 1 after the append): Q4 weights + scales, the
    fp16 K/V read of the existing positions, the new K/V row and the hidden
    vector in and out counted at 2 bytes per element (10,461,184 B at ctx 512)."""
    h, i = cfg.hidden_size, cfg.intermediate_size
    qd, kd = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    elems = qd * h + 2 * kd * h + h * qd + 2 * i * h + h * i
    weights = elems // 2 + 2 * (elems // GROUP_SIZE)
    kv_read = 2 * kd * ctx * 2
    kv_write = 2 * kd * 2
    return weights + kv_read + kv_write + 2 * h * 2


def fixed_layer_bytes(cfg: Qwen3Config, ctx: int) -> int:
    """HBM bytes of one fixed-point decode layer at context ``ctx``: the same Q4
    weights + scales, the int32 K/V of ``ctx`` positions read and one row of each
    written, the int32 hidden state in and out, int16 gammas."""
    h, i = cfg.hidden_size, cfg.intermediate_size
    qd, kd = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    elems = qd * h + 2 * kd * h + h * qd + 2 * i * h + h * i
    weights = elems // 2 + 2 * (elems // GROUP_SIZE)
    return weights + 2 * kd * ctx * 4 + 2 * kd * 4 + 2 * h * 4 + 2 * (2 * h + 2 * cfg.head_dim)


def stage_bytes_layer(cfg: Qwen3Config, ctx: int) -> dict:
    """Algorithmic bytes per launch of each decode-layer stage at context
    ``ctx``, in the dtypes the kernels read and write: Q4 codes + Q2.14
    scales, fp32 activations (and fp32 gammas for the RMSNorm prologues),
    fp16 K/V."""
    h, i, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    qh, kvh = cfg.num_attention_heads, cfg.num_key_value_heads

    def w(rows, cols):
        return rows * cols // 2 + 2 * rows * (cols // GROUP_SIZE)
    qkv_rows = (qh + 2 * kvh) * d
    return {
        "qkv": w(qkv_rows, h) + 4 * h + 4 * h + 4 * qkv_rows,
        "attention": 2 * kvh * ctx * d * 2 + 2 * kvh * d * 2 + 4 * qkv_rows + 4 * qh * d + 4 * 2 * d,
        "o_proj": w(h, qh * d) + 4 * qh * d + 4 * h + 4 * h,
        "gate_up": 2 * w(i, h) + 4 * h + 4 * h + 4 * i,
        "down": w(h, i) + 4 * i + 4 * h + 4 * h,
    }


def prefill_flops(cfg: Qwen3Config, n: int) -> int:
    """Flops of prefilling n tokens from position 0: the projections
    (2 per weight per token), causal attention (q.k and p.v over positions
    0..t for token t) and the LM head of the last token."""
    h, i, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    qh, kvh, L = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.num_hidden_layers
    per_layer = qh * d * h + 2 * kvh * d * h + h * qh * d + 2 * i * h + h * i
    linear = 2 * n * per_layer * L
    attention = 2 * 2 * d * qh * L * (n * (n + 1) // 2)
    return linear + attention + 2 * cfg.vocab_size * h


def batched_step_bytes(cfg: Qwen3Config, batch: int, ctx: int) -> int:
    """HBM bytes of one batched decode step: every sequence's fp16 K/V over
    ``ctx`` positions in every layer plus all Q4 weights once."""
    h, i, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    qh, kvh, L = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.num_hidden_layers
    elems = qh * d * h + 2 * kvh * d * h + h * qh * d + 2 * i * h + h * i
    weights = L * (elems // 2 + 2 * (elems // GROUP_SIZE)) + cfg.vocab_size * h // 2 + 2 * cfg.vocab_size * (h // GROUP_SIZE)
    return batch * L * 2 * kvh * ctx * d * 2 + weights


def gemv_bytes(rows: int, cols: int, x_bytes: int = 2, y_bytes: int = 2) -> int:
    return rows * cols // 2 + 2 * rows * (cols // GROUP_SIZE) + x_bytes * cols + y_bytes * rows


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


__all__ = ["Qwen3Config", "Q4Tensor", "Q4ForCausalLM", "Q4DecoderLayer", "Q4Backbone", "RotaryEmbedding",
           "KVCache", "Workspace", "random_q4", "random_gamma", "random_host_weights", "build_model",
           "algorithmic_bytes_layer", "fixed_layer_bytes", "with_context", "stage_bytes_layer", "prefill_flops", "batched_step_bytes", "gemv_bytes",
           "current_stream", "ceil_div"]
