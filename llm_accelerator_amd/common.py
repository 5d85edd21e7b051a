"""Device drop-in for the reference's hot-path functions.

Same names, argument order and return tuples as
``Qwen3-0.6B-Base/python_each_module/common.py`` (lines 129-298) and
``10_validate_full_run_one_token.py`` (lines 17-56), but every tensor lives on
the GPU and every op is a libq4dec kernel launched on torch's current stream.
What changes is only the types:

* a projection ``.weight`` is a :class:`~llm_accelerator_amd.model.Q4Tensor`;
* K/V caches are :class:`KVLayerView` handles into one preallocated fp16
  :class:`~llm_accelerator_amd.model.KVCache` (append writes in place, no
  reallocation); ``append_cache(None, v)`` allocates a standalone cache;
* ``manual_repeat_kv`` returns a :class:`RepeatedKV` marker instead of a
  copy: the attention kernel maps q head ``h`` to kv head ``h // repeat``;
* ``manual_cached_attention`` returns ``(output, None)`` and
  ``manual_causal_attention`` ``(output, AttentionWeights)`` (shape only): the
  softmax weights are never materialised.

Errors: a failing entry point raises :class:`~llm_accelerator_amd._lib.Q4DecError`
(a ``RuntimeError``, as the reference's ``require_*``/``finish`` raise).
"""

from __future__ import annotations

import ctypes
from typing import Any

import torch

from . import _lib
from ._lib import Q4D_F16, Q4D_F32, check
from .model import KVCache, Q4ForCausalLM, Q4Tensor, Qwen3Config, Workspace, current_stream

DEFAULT_STANDALONE_CTX = 4096


def _dev_f32(x: torch.Tensor, name: str) -> torch.Tensor:
    if not x.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (libq4dec has no CPU path)")
    return x.to(torch.float32).contiguous()


def get_rms_norm_eps(norm_module: Any, model_config: Any) -> float:
    """Same lookup order as the reference (common.py:51-56)."""
    if hasattr(norm_module, "variance_epsilon"):
        return float(norm_module.variance_epsilon)
    if hasattr(norm_module, "eps"):
        return float(norm_module.eps)
    return float(model_config.rms_norm_eps)


def manual_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps) * weight`` over the last dim (common.py:129-134)."""
    xf = _dev_f32(x, "x")
    w = _dev_f32(weight, "weight")
    dim = xf.shape[-1]
    if w.numel() != dim:
        raise ValueError(f"weight has {w.numel()} elements, last dim is {dim}")
    y = torch.empty_like(xf)
    check(_lib.load().q4d_rms_norm(xf.data_ptr(), w.data_ptr(), float(eps), xf.numel() // dim, dim,
                                   y.data_ptr(), Q4D_F32, current_stream()), "q4d_rms_norm")
    return y


def manual_linear_from_weight(x: torch.Tensor, weight: Q4Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """``y = x @ W.T`` with W in Q4 (common.py:137-145); fp32 in, fp32 out."""
    if not isinstance(weight, Q4Tensor):
        raise TypeError("weight must be a Q4Tensor")
    if bias is not None:
        raise ValueError("bias is not supported: Qwen3 projections have none (config.json attention_bias=false)")
    rows, cols = weight.shape
    xf = _dev_f32(x, "x")
    if xf.shape[-1] != cols:
        raise ValueError(f"x last dim {xf.shape[-1]} != weight cols {cols}")
    batch = xf.numel() // cols
    y = torch.empty(xf.shape[:-1] + (rows,), dtype=torch.float32, device=xf.device)
    desc = weight.descriptor()
    check(_lib.load().q4d_linear(ctypes.byref(desc), xf.data_ptr(), Q4D_F32, y.data_ptr(), Q4D_F32, batch,
                                 current_stream()), "q4d_linear")
    return y


def manual_rope_cos_sin(rotary_emb: Any, x: torch.Tensor, position_ids: torch.Tensor):
    """``cos/sin`` of ``cat(f, f)``, ``f = pos * inv_freq`` (common.py:155-170),
    gathered from the device tables; returns fp32 [batch, seq, head_dim]."""
    pos = position_ids.to(device=rotary_emb.cos_table.device, dtype=torch.long)
    c = rotary_emb.cos_table[pos]
    s = rotary_emb.sin_table[pos]
    return torch.cat((c, c), dim=-1), torch.cat((s, s), dim=-1)


def manual_rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``cat(-x[..., D/2:], x[..., :D/2])`` over the last dim (common.py:148-152); fp32."""
    xf = _dev_f32(x, "x")
    d = xf.shape[-1]
    y = torch.empty_like(xf)
    if xf.numel():
        check(_lib.load().q4d_rotate_half(xf.data_ptr(), y.data_ptr(), xf.numel() // d, d, current_stream()),
              "q4d_rotate_half")
    return y


def manual_apply_rope(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """``x*cos + rotate_half(x)*sin`` (common.py:173-183) for q [B,H,S,D] and
    k [B,KVH,S,D] with cos/sin [B,S,D] (a batch of 1 broadcasts over B), for one
    decode position or a whole prompt (04_validate_qk_norm_rope.py:59-60)."""
    lib = _lib.load()
    if q.dim() != 4 or k.dim() != 4 or q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:]:
        raise ValueError("q and k must be [B, heads, S, D] with the same B, S, D")
    b, _, seq, d = q.shape
    if cos.shape[-2:] != (seq, d) or sin.shape != cos.shape or cos.dim() != 3 or cos.shape[0] not in (1, b):
        raise ValueError(f"cos/sin must be [B, {seq}, {d}] (or [1, {seq}, {d}])")
    c = _dev_f32(cos.expand(b, seq, d), "cos")
    s = _dev_f32(sin.expand(b, seq, d), "sin")
    out = []
    for t in (q, k):
        tf = _dev_f32(t, "q/k")
        y = torch.empty_like(tf)
        if tf.numel():
            check(lib.q4d_apply_rope_seq(tf.data_ptr(), y.data_ptr(), c.data_ptr(), s.data_ptr(), b, tf.shape[1],
                                         seq, d, current_stream()), "q4d_apply_rope_seq")
        out.append(y)
    return out[0], out[1]


class KVLayerView:
    """One layer's K or V cache inside a :class:`KVCache` plus its valid length."""

    def __init__(self, cache: KVCache, layer: int, kind: int, length: int):
        self.cache, self.layer, self.kind, self.length = cache, layer, kind, length

    @property
    def shape(self):
        return (self.cache.batch, self.cache.num_kv_heads, self.length, self.cache.head_dim)

    def tensor(self) -> torch.Tensor:
        """[batch, kv_heads, length, head_dim] fp16 view of the valid positions."""
        return self.cache.data[self.layer, self.kind, :, :, : self.length]


class RepeatedKV:
    """``manual_repeat_kv`` result: the cache view (or the K/V tensor) plus the GQA
    repeat factor; ``shape`` is the shape the reference's repeated copy would have."""

    def __init__(self, view, repeat: int):
        self.view, self.repeat = view, repeat

    @property
    def shape(self):
        b, kvh, t, d = tuple(self.view.shape)
        return torch.Size((b, kvh * self.repeat, t, d))


class AttentionWeights:
    """Stand-in for the softmax weights ``manual_causal_attention`` returns
    (common.py:213-216): the flash-attention kernel never materialises them, so
    only their shape [B, H, S, S] and dtype are given."""

    def __init__(self, shape, dtype=torch.float32):
        self.shape, self.dtype = torch.Size(shape), dtype

    def __repr__(self) -> str:
        return f"AttentionWeights(shape={list(self.shape)}, not materialised)"


def layer_views(cache: KVCache, length: int = 0) -> tuple[list, list]:
    """Per-layer K and V views, the analogue of the reference's
    ``manual_k_caches`` / ``manual_v_caches`` lists."""
    return ([KVLayerView(cache, i, 0, length) for i in range(cache.num_layers)],
            [KVLayerView(cache, i, 1, length) for i in range(cache.num_layers)])


def append_cache(old_cache: KVLayerView | None, current_value: torch.Tensor) -> KVLayerView:
    """Append one position (common.py:186-189) in place; returns the grown view.
    ``current_value``: [B, KVH, 1, D]."""
    b, kvh, s, d = current_value.shape
    if s != 1:
        raise ValueError("append_cache appends one position per call")
    if old_cache is None:
        cfg = Qwen3Config(num_key_value_heads=kvh, head_dim=d)
        old_cache = KVLayerView(KVCache(cfg, 1, b, DEFAULT_STANDALONE_CTX, current_value.device), 0, 0, 0)
    view = old_cache
    if view.length >= view.cache.max_ctx:
        raise _lib.Q4DecError(-10, "append_cache")
    c = view.cache
    val = _dev_f32(current_value, "current_value")[:, :, 0].contiguous()
    k, v = (val.data_ptr(), None) if view.kind == 0 else (None, val.data_ptr())
    pos = torch.full((b,), view.length, dtype=torch.int32, device=val.device)
    status = torch.zeros(1, dtype=torch.int32, device=val.device)
    kvd = c.descriptor()
    check(_lib.load().q4d_kv_append(ctypes.byref(kvd), view.layer, k, v, pos.data_ptr(),
                                    status.data_ptr(), current_stream()), "q4d_kv_append")
    return KVLayerView(c, view.layer, view.kind, view.length + 1)


def manual_repeat_kv(x, repeat_count: int) -> RepeatedKV:
    """GQA repeat as a marker (common.py:192-198) over a cache view or a
    [B, KVH, S, D] tensor: q head h reads kv head h // repeat_count."""
    if isinstance(x, RepeatedKV):
        return RepeatedKV(x.view, x.repeat * repeat_count)
    return RepeatedKV(x, repeat_count)


def manual_causal_attention(q: torch.Tensor, k, v, scaling: float):
    """``softmax(q k^T * scaling, causal) v`` (common.py:201-216), the prompt
    attention 06_validate_attention.py:71 calls.  q [B,H,S,D]; k, v: the
    :func:`manual_repeat_kv` markers of [B,KVH,S,D] tensors or [B,H,S,D] tensors.
    Returns ``(output [B,H,S,D] fp32, AttentionWeights)``: MFMA flash attention
    over fp16-rounded operands (q4d_causal_attention), no weights materialised."""
    def unwrap(x, name):
        if isinstance(x, RepeatedKV):
            if not isinstance(x.view, torch.Tensor):
                raise TypeError(f"{name}: causal attention takes tensors (cache views go to manual_cached_attention)")
            return x.view, x.repeat
        return x, 1
    kt, kr = unwrap(k, "k")
    vt, vr = unwrap(v, "v")
    if q.dim() != 4 or kt.dim() != 4 or vt.shape != kt.shape or kr != vr:
        raise ValueError("q [B,H,S,D]; k and v of one shape [B,KVH,S,D] with one repeat factor")
    b, h, s, d = q.shape
    kvh = kt.shape[1]
    if kt.shape[0] != b or kt.shape[2:] != (s, d) or kvh * kr != h:
        raise ValueError(f"k/v {tuple(kt.shape)} x repeat {kr} do not match q {tuple(q.shape)}")
    lib = _lib.load()
    qf, kf, vf = _dev_f32(q, "q"), _dev_f32(kt, "k"), _dev_f32(vt, "v")
    out = torch.empty_like(qf)
    if qf.numel():
        nbytes = int(lib.q4d_causal_attention_workspace_bytes(b, h, kvh, s))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=qf.device)
        check(lib.q4d_causal_attention(qf.data_ptr(), kf.data_ptr(), vf.data_ptr(), out.data_ptr(), b, h, kvh, s, d,
                                       float(scaling), ws.data_ptr(), nbytes, current_stream()),
              "q4d_causal_attention")
    return out, AttentionWeights((b, h, s, s))


_model_registry: dict[int, tuple] = {}


def _model_for(cache: KVCache, num_q_heads: int, scaling: float):
    """Minimal model descriptor for standalone attention calls (no weights)."""
    key = (id(cache), num_q_heads, float(scaling))
    if key in _model_registry:
        return _model_registry[key]
    from ._lib import Q4dModel
    d = Q4dModel()
    d.hidden_size, d.head_dim = 1024, cache.head_dim
    d.num_q_heads, d.num_kv_heads = num_q_heads, cache.num_kv_heads
    d.num_layers, d.max_ctx = cache.num_layers, cache.max_ctx
    d.intermediate_size, d.vocab_size = 3072, 2
    d.attn_scaling = scaling
    nbytes = int(_lib.load().q4d_workspace_bytes(ctypes.byref(d), cache.batch))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=cache.data.device)
    _model_registry[key] = (d, ws)
    return d, ws


def manual_cached_attention(q_current: torch.Tensor, k_cache_repeated: RepeatedKV,
                            v_cache_repeated: RepeatedKV, scaling: float):
    """``softmax(q k^T * scaling) v`` over the cached positions
    (common.py:219-228); q [B,H,1,D] fp32 -> ([B,H,1,D], None)."""
    kv = k_cache_repeated.view
    if not isinstance(kv, KVLayerView) or not isinstance(v_cache_repeated.view, KVLayerView):
        raise TypeError("cached attention reads KVLayerView caches (prompt tensors go to manual_causal_attention)")
    if v_cache_repeated.view.cache is not kv.cache or v_cache_repeated.view.layer != kv.layer:
        raise ValueError("k and v views must come from the same cache layer")
    cache = kv.cache
    b, h, s, d = q_current.shape
    if s != 1 or h != k_cache_repeated.repeat * cache.num_kv_heads:
        raise ValueError("q heads must equal repeat * kv heads, one query position")
    if kv.length < 1:
        raise ValueError("empty cache")
    desc, ws = _model_for(cache, h, scaling)
    qf = _dev_f32(q_current, "q")
    out = torch.empty((b, h * d), dtype=torch.float32, device=qf.device)
    pos = torch.full((b,), kv.length - 1, dtype=torch.int32, device=qf.device)
    kvd = cache.descriptor()
    check(_lib.load().q4d_cached_attention(ctypes.byref(desc), ctypes.byref(kvd), kv.layer, qf.data_ptr(),
                                           pos.data_ptr(), out.data_ptr(), Q4D_F32, ws.data_ptr(), ws.numel(),
                                           current_stream()), "q4d_cached_attention")
    return out.view(b, h, 1, d), None


class _Runtime:
    """Per-model workspace and small device scalars for the fused calls."""

    def __init__(self, model: Q4ForCausalLM):
        dev = model.device
        self.ws = Workspace(model, 1)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.tok = torch.zeros(1, dtype=torch.int32, device=dev)
        self.next_tok = torch.zeros(1, dtype=torch.int32, device=dev)
        self.score = torch.zeros(1, dtype=torch.float32, device=dev)


def runtime(model: Q4ForCausalLM) -> _Runtime:
    rt = getattr(model, "_q4d_runtime", None)
    if rt is None:
        rt = _Runtime(model)
        model._q4d_runtime = rt
    return rt


def manual_decoder_layer_cached(hidden: torch.Tensor, layer: Any, rotary_emb: Any, position_ids: torch.Tensor,
                                k_cache: KVLayerView, v_cache: KVLayerView, batch_size: int, num_q_heads: int,
                                num_kv_heads: int, head_dim: int, kv_repeat: int, model_config: Any):
    """One fused cached decoder layer (common.py:231-298), batch 1.

    Returns ``(layer_output [1,1,hidden] fp32, k_cache, v_cache)`` with both
    views grown by one position.  ``layer`` must belong to a
    :class:`Q4ForCausalLM` (it carries ``_q4d_owner``/``_q4d_index``)."""
    model: Q4ForCausalLM = layer._q4d_owner
    li: int = layer._q4d_index
    if batch_size != 1:
        raise ValueError("the fused layer path runs batch 1")
    cfg = model.config
    if (num_q_heads, num_kv_heads, head_dim, kv_repeat) != (cfg.num_attention_heads, cfg.num_key_value_heads,
                                                            cfg.head_dim, cfg.kv_repeat):
        raise ValueError("head geometry does not match the model")
    if not isinstance(k_cache, KVLayerView) or k_cache.layer != li or v_cache.layer != li:
        raise ValueError("k_cache / v_cache must be KVLayerView handles of this layer")
    position = int(position_ids.reshape(-1)[0])
    if position != k_cache.length:
        raise _lib.Q4DecError(-10, f"position {position} != cache length {k_cache.length}")
    if position >= model.max_ctx:
        raise _lib.Q4DecError(-10, "manual_decoder_layer_cached")
    rt = runtime(model)
    h_in = _dev_f32(hidden, "hidden").reshape(1, cfg.hidden_size)
    h_out = torch.empty_like(h_in)
    rt.pos.fill_(position)
    desc, kvd = model.descriptor(), k_cache.cache.descriptor()
    check(_lib.load().q4d_decoder_layer(ctypes.byref(desc), li, h_in.data_ptr(), h_out.data_ptr(),
                                        ctypes.byref(kvd), rt.pos.data_ptr(), rt.ws.ptr, rt.ws.nbytes,
                                        current_stream()), "q4d_decoder_layer")
    # synchronous like the reference function: a device-side failure (an exchange of the
    # XCD-split layer that timed out or ran off its XCD) raises here
    rt.ws.raise_for_status("q4d_decoder_layer")
    return (h_out.view(1, 1, cfg.hidden_size), KVLayerView(k_cache.cache, li, 0, position + 1),
            KVLayerView(v_cache.cache, li, 1, position + 1))


def run_manual_one_token(current_token_ids: torch.Tensor, position: int, embedding_table: Q4Tensor, backbone: Any,
                         model: Q4ForCausalLM, manual_k_caches: list, manual_v_caches: list, batch_size: int,
                         num_q_heads: int, num_kv_heads: int, head_dim: int, kv_repeat: int,
                         return_logits: bool = True):
    """Embedding -> 28 fused layers -> final norm -> LM head -> argmax
    (10_validate_full_run_one_token.py:17-56).  Returns ``(logits, next_token)``:
    logits fp32 [1,1,vocab] (None when ``return_logits`` is False) and
    next_token int64 [1,1]; the cache views in the two lists advance by one."""
    if batch_size != 1:
        raise ValueError("the fused one-token path runs batch 1")
    cfg = model.config
    if embedding_table is not model.lm_head.weight:
        raise ValueError("embedding_table must be the model's tied Q4 table")
    tok = int(current_token_ids.reshape(-1)[0])
    if not 0 <= tok < cfg.vocab_size:
        raise _lib.Q4DecError(-8, "run_manual_one_token")
    k0 = manual_k_caches[0]
    if position != k0.length or position >= model.max_ctx:
        raise _lib.Q4DecError(-10, "run_manual_one_token")
    rt = runtime(model)
    rt.tok.fill_(tok)
    rt.pos.fill_(position)
    logits = torch.empty((1, 1, cfg.vocab_size), dtype=torch.float32, device=model.device) if return_logits else None
    desc, kvd = model.descriptor(), k0.cache.descriptor()
    check(_lib.load().q4d_run_one_token(ctypes.byref(desc), rt.tok.data_ptr(), rt.pos.data_ptr(), ctypes.byref(kvd),
                                        rt.next_tok.data_ptr(), rt.score.data_ptr(),
                                        logits.data_ptr() if logits is not None else None, rt.ws.ptr,
                                        rt.ws.nbytes, current_stream()), "q4d_run_one_token")
    rt.ws.raise_for_status("q4d_run_one_token")
    for i in range(len(manual_k_caches)):
        manual_k_caches[i] = KVLayerView(k0.cache, i, 0, position + 1)
        manual_v_caches[i] = KVLayerView(k0.cache, i, 1, position + 1)
    return logits, rt.next_tok.to(torch.int64).view(1, 1).clone()


__all__ = ["get_rms_norm_eps", "manual_rms_norm", "manual_linear_from_weight", "manual_rope_cos_sin",
           "manual_rotate_half", "manual_apply_rope", "append_cache", "manual_repeat_kv",
           "manual_causal_attention", "manual_cached_attention", "AttentionWeights",
           "manual_decoder_layer_cached", "run_manual_one_token", "KVLayerView", "RepeatedKV", "layer_views",
           "runtime", "Q4D_F16"]
