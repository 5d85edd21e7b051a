"""Float -> Q4 conversion on the GPU: the reference's quantizer and a checkpoint converter.

``quantize_weight_q4`` keeps the reference's name, rule and errors
(``Qwen3-0.6B-Base/python_each_module/13_export_q4_gemv_vectors.py:101-135``: per
64-column group ``code = rint(fp32(absmax / 7) * 2**14)`` round-half-even, 1 for a
nonzero group that rounds to 0, ``q = clip(rint(w / (code / 2**14)), -8, 7)``), with the
work in libq4dec's ``q4d_quantize_q4`` kernel; its codes equal numpy's bit for bit.

``convert_checkpoint`` turns a Hugging Face Qwen3 checkpoint (``model.safetensors`` or
its shards, plus ``config.json``) into the host weight layout ``model.build_model``
takes: every projection and the tied embedding / LM-head table as Q4, the RMSNorm
weights as fp32 (bf16 widens exactly).  The reference obtains the same Q4 matrices
from the HF model in fp32 (``56_...:241-291``, ``as_float32``).
"""

from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np
import torch

from . import _lib
from ._lib import Q4D_BF16, Q4D_F32, check
from .model import Qwen3Config, current_stream

GROUP_SIZE = 64
Q4_MIN, Q4_MAX = -8, 7


def _unpack(packed: torch.Tensor, cols: int) -> torch.Tensor:
    lo = (packed & 0xF).to(torch.int8)
    hi = (packed >> 4).to(torch.int8)
    q = torch.stack([lo, hi], dim=-1).reshape(packed.shape[0], cols)
    return torch.where(q >= 8, q - 16, q)


def _prepare(weight) -> tuple:
    """(device matrix with 16-byte aligned rows, rows, cols, Q4D dtype), with the reference's
    ValueErrors for the shape."""
    if not isinstance(weight, torch.Tensor):
        weight = torch.from_numpy(np.ascontiguousarray(weight, dtype=np.float32))
    if weight.dim() != 2:
        raise ValueError(f"Expected 2D weight matrix, got shape {tuple(weight.shape)}")
    rows, cols = weight.shape
    if cols % GROUP_SIZE:
        raise ValueError("Input feature count must be divisible by Q4_GROUP_SIZE")
    if rows == 0:
        raise ValueError("Expected at least one row")
    if weight.dtype not in (torch.float32, torch.bfloat16):
        weight = weight.float()
    dev = weight.device if weight.is_cuda else torch.device("cuda")
    w = weight.to(dev)
    if w.stride(1) != 1 or w.stride(0) < cols or (w.stride(0) * w.element_size()) % 16 or w.data_ptr() % 16:
        w = w.contiguous()   # the kernel reads 16-byte aligned rows
    return w, rows, cols, (Q4D_F32 if w.dtype == torch.float32 else Q4D_BF16)


def _raise_on_status(status: torch.Tensor) -> None:
    overflow, nonfinite = status.tolist()
    if overflow or nonfinite:
        raise ValueError(f"Q4 scale does not fit unsigned 16-bit Q2.14 storage ({overflow} groups with absmax "
                         f"too large, {nonfinite} groups with non-finite values)")


def quantize_weight_q4(weight: torch.Tensor, return_codes: bool = True):
    """Q4 quantisation of a 2-D fp32 / bf16 matrix on the GPU -> (packed uint8 [N, K/2],
    scale uint16 [N, K/64], q int8 [N, K] or None), device tensors.  Raises ValueError as
    the reference does: not 2-D, K not a multiple of 64, or a scale that does not fit
    Q2.14 (absmax above ~28, or a non-finite weight)."""
    w, rows, cols, dtype = _prepare(weight)
    dev = w.device
    packed = torch.empty(rows, cols // 2, dtype=torch.uint8, device=dev)
    scale = torch.empty(rows, cols // GROUP_SIZE, dtype=torch.uint16, device=dev)
    status = torch.zeros(2, dtype=torch.int32, device=dev)
    check(_lib.load().q4d_quantize_q4(w.data_ptr(), dtype, w.stride(0), rows, cols, packed.data_ptr(),
                                      scale.data_ptr(), status.data_ptr(), current_stream()), "q4d_quantize_q4")
    _raise_on_status(status)
    return packed, scale, (_unpack(packed, cols) if return_codes else None)


def quantize_weights_q4(weights) -> list:
    """quantize_weight_q4 over a list of matrices -> [(packed, scale)] in the same order,
    the same codes bit for bit; matrices of one shape, dtype and row pitch are converted
    by one launch each (q4d_quantize_q4_batch).  Raises the same ValueErrors, naming the
    first failing matrix's index."""
    prepared = [_prepare(w) for w in weights]
    out = [None] * len(prepared)
    groups = {}
    for i, (w, rows, cols, dtype) in enumerate(prepared):
        groups.setdefault((rows, cols, dtype, w.stride(0), w.device), []).append(i)
    lib = _lib.load()
    for (rows, cols, dtype, ld, dev), idx in groups.items():
        packed = [torch.empty(rows, cols // 2, dtype=torch.uint8, device=dev) for _ in idx]
        scale = [torch.empty(rows, cols // GROUP_SIZE, dtype=torch.uint16, device=dev) for _ in idx]
        status = torch.zeros(2, dtype=torch.int32, device=dev)
        n = len(idx)
        wp = (ctypes.c_void_p * n)(*[prepared[i][0].data_ptr() for i in idx])
        pp = (ctypes.c_void_p * n)(*[t.data_ptr() for t in packed])
        sp = (ctypes.c_void_p * n)(*[t.data_ptr() for t in scale])
        check(lib.q4d_quantize_q4_batch(wp, dtype, ld, rows, cols, n, pp, sp, status.data_ptr(), current_stream()),
              "q4d_quantize_q4_batch")
        if status.any():  # find the first failing matrix of the group, as one call each would
            for i in idx:
                try:
                    quantize_weight_q4(prepared[i][0], return_codes=False)
                except ValueError as e:
                    raise ValueError(f"matrix {i}: {e}") from None
            _raise_on_status(status)  # no single call failed: report the group's own status
        for k, i in enumerate(idx):
            out[i] = (packed[k], scale[k])
    return out


# Hugging Face Qwen3 tensor names (transformers' Qwen3ForCausalLM state dict).
_LAYER_MATS = {"q_proj": "self_attn.q_proj", "k_proj": "self_attn.k_proj", "v_proj": "self_attn.v_proj",
               "o_proj": "self_attn.o_proj", "gate_proj": "mlp.gate_proj", "up_proj": "mlp.up_proj",
               "down_proj": "mlp.down_proj"}
_LAYER_VECS = {"input_layernorm": "input_layernorm", "post_attention_layernorm": "post_attention_layernorm",
               "q_norm": "self_attn.q_norm", "k_norm": "self_attn.k_norm"}


def expected_tensors(cfg: Qwen3Config) -> dict:
    """Checkpoint tensor name -> shape for ``cfg`` (the untied ``lm_head.weight`` is optional)."""
    h, i, d = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    qd, kd = cfg.num_attention_heads * d, cfg.num_key_value_heads * d
    mats = {"q_proj": (qd, h), "k_proj": (kd, h), "v_proj": (kd, h), "o_proj": (h, qd), "gate_proj": (i, h),
            "up_proj": (i, h), "down_proj": (h, i)}
    vecs = {"input_layernorm": (h,), "post_attention_layernorm": (h,), "q_norm": (d,), "k_norm": (d,)}
    out = {"model.embed_tokens.weight": (cfg.vocab_size, h), "model.norm.weight": (h,)}
    for li in range(cfg.num_hidden_layers):
        for k, v in _LAYER_MATS.items():
            out[f"model.layers.{li}.{v}.weight"] = mats[k]
        for k, v in _LAYER_VECS.items():
            out[f"model.layers.{li}.{v}.weight"] = vecs[k]
    return out


def checkpoint_files(path: str | Path) -> list:
    """The safetensors files of a checkpoint directory (single file or index-listed shards)."""
    p = Path(path)
    if p.is_file():
        return [p]
    index = p / "model.safetensors.index.json"
    if index.exists():
        shards = sorted(set(json.loads(index.read_text())["weight_map"].values()))
        return [p / s for s in shards]
    single = p / "model.safetensors"
    if single.exists():
        return [single]
    raise FileNotFoundError(f"no model.safetensors (or index) under {p}")


def check_checkpoint(names_shapes: dict, cfg: Qwen3Config) -> None:
    """Raise ValueError naming the first missing or mis-shaped tensor."""
    for name, shape in expected_tensors(cfg).items():
        if name not in names_shapes:
            raise ValueError(f"checkpoint lacks {name}")
        if tuple(names_shapes[name]) != shape:
            raise ValueError(f"{name} has shape {tuple(names_shapes[name])}, expected {shape}")
    if "lm_head.weight" in names_shapes and not cfg.tie_word_embeddings:
        raise ValueError("an untied LM head has no place in the tied Q4 layout")


def convert_checkpoint(path: str | Path, cfg: Qwen3Config | None = None, device="cuda") -> tuple:
    """(cfg, host weights) from a Hugging Face Qwen3 checkpoint, Q4 on ``device``'s kernel."""
    from contextlib import ExitStack

    from safetensors import safe_open
    p = Path(path)
    if cfg is None:
        cfg = Qwen3Config.from_json((p if p.is_dir() else p.parent) / "config.json")
    with ExitStack() as stack:
        handles = [stack.enter_context(safe_open(str(f), framework="pt", device="cpu")) for f in checkpoint_files(p)]
        where, shapes = {}, {}
        for h in handles:
            for name in h.keys():
                where[name] = h
                shapes[name] = tuple(h.get_slice(name).get_shape())
        check_checkpoint(shapes, cfg)

        def vec(name):
            return where[name].get_tensor(name).float().numpy().astype(np.float32)

        # every matrix on the device, then one grouped conversion (one launch per shape)
        names = [f"model.layers.{li}.{v}.weight" for li in range(cfg.num_hidden_layers) for v in _LAYER_MATS.values()]
        names.append("model.embed_tokens.weight")
        q = quantize_weights_q4([where[n].get_tensor(n).to(device) for n in names])
        q4 = {n: (p.cpu().numpy(), sc.cpu().numpy()) for n, (p, sc) in zip(names, q)}
        del q
        layers = []
        for li in range(cfg.num_hidden_layers):
            pre = f"model.layers.{li}."
            L = {k: q4[pre + v + ".weight"] for k, v in _LAYER_MATS.items()}
            L.update({k: vec(pre + v + ".weight") for k, v in _LAYER_VECS.items()})
            layers.append(L)
        host = {"layers": layers, "embed_tokens": q4["model.embed_tokens.weight"], "norm": vec("model.norm.weight")}
    return cfg, host


__all__ = ["quantize_weight_q4", "quantize_weights_q4", "convert_checkpoint", "expected_tensors", "check_checkpoint", "checkpoint_files"]
