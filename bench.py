#!/usr/bin/env python3
"""Benchmark of the Qwen3-0.6B Q4 decode hot path on one MI355X.

Headline (``value``): one 3072 x 1024 Q4 dequant-GEMV, the Qwen3-0.6B MLP
gate_proj shape (4-bit codes uniform over 0..15, Q2.14 scales ~ |N(0, 0.02)|
per 64 columns, fp16 x ~ N(0, 1), batch 1, fp16 y).  A "step" is one GEMV
launch.  Consecutive steps read distinct copies of the matrix (``--copies`` x
1.68 MB, above the 256 MB Infinity Cache), so each step streams its weights
from HBM: the cache-flushed rate.  ``value`` = algorithmic bytes per step
(1,679,360 B: codes + scales + x + y) / average step time; the step time is
HIP events around exactly ``--steps`` launches replayed from HIP graphs, after
an untimed lead-in replay that keeps the GPU busy while the host enqueues the
timed graphs.  Beside it: the cache-resident rate (one copy, repeated) and a
measured single-launch floor (the same kernel on a 2 x 1024 matrix: launch,
one dependent memory round trip and the completion, with no bytes to speak of).

``roofline``: that GEMV kernel; ``traffic`` = its HBM bytes per launch from the
rocprofv3 FETCH_SIZE / WRITE_SIZE summary under profiles/ (copy-calibrated).

``decode``: full 28-layer greedy decode, batch 1 (64-token prompt of uniform
random ids, then 256 generated tokens, the LM-head argmax fed back on the
device; HIP graphs of 15 steps).  tok/s from HIP events over the 255 feedback
steps, and its HBM roofline fraction (Q4 weights + the tied table + fp16 K/V
of every attended position, averaged over the steps, over 8 TB/s).  The
model's 306 MB of weights exceed the 256 MB cache; ``resident`` repeats the
loop with every layer aliased to layer 0's weights (91 MB working set) for the
cache-resident figure.  The layer runs as two launches split over the eight XCDs
(one kv head per XCD); ``staged`` repeats the loop with the five-launch layer, and
``launch_floor`` times the step's launches with their grids and no work.

``lm_head``: final RMSNorm + 151936 x 1024 Q4 GEMV + argmax alone, flushed
(rotating over 4 copies of the table, 331 MB) and repeated.

``extras``: one decoder layer's decode step at context 512 (flushed over 40
distinct layers, resident, per-stage times and rates); prefill of one
2048-token sequence through 28 layers (tok/s, TFLOP/s against the dense fp16
MFMA peak); batched decode of 64 sequences over 4096 cached positions; the
fixed-point (RTL-exact) layer and token; bf16 -> Q4 conversion of every
matrix; torch's device copy of 512 MiB windows (a measured HBM rate, also
quoted in ``roofline``); and more CPU legs (``extras.cpu_legs``).

``cpu_baseline``: the oracle's fp32 matvec for the same GEMV (y = x @ W.T on
the pre-dequantised fp32 matrix, as manual_linear_from_weight computes it,
common.py:137-145) on the host cores, a ~10 s sample, in GB/s of the same
algorithmic bytes.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

METRIC = "Q4 GEMV HBM GB/s (% peak) + batch-1 decode tok/s, Qwen3-0.6B-Q4"
HBM_PEAK_GBPS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16
GEMV_ROWS, GEMV_COLS = 3072, 1024
GEMV_WARM_S = 0.3        # sustained GEMV launches before the timed regions (clock ramp)
GEMV_TIMED_S = 0.1       # target GPU time of the timed regions together
GEMV_MIN_REPLAYS = 11    # timed regions of --steps launches at least (median reported)
PROMPT = 64
PREFILL_TOKENS = 2048              # prefill of one 2048-token sequence
BATCH_SEQS, BATCH_CTX = 64, 4096  # batched decode: 64 sequences over 4096 cached positions
STAGE_KERNELS = {"qkv": "input RMSNorm + q|k|v Q4 GEMV", "attention": "q/k norm + RoPE + KV append + split-K GQA attention",
                 "o_proj": "o_proj Q4 GEMV + residual", "gate_up": "post-norm + gate/up Q4 GEMV + SwiGLU",
                 "down": "down Q4 GEMV + residual"}
GEMV_KERNEL = "gemv_kernel<1, 8, 0, 1, 0, false, 1>"
PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000, help="timed GEMV launches")
    ap.add_argument("--warmup", type=int, default=200, help="untimed GEMV launches before the timed ones")
    ap.add_argument("--copies", type=int, default=200, help="distinct copies of the GEMV matrix (flushed rate)")
    ap.add_argument("--ctx", type=int, default=512, help="context of the decoder-layer leg")
    ap.add_argument("--layer-copies", type=int, default=40)
    ap.add_argument("--precision", type=int, default=2, choices=(1, 2),
                    help="fp32 activations enter the decode GEMVs as fp16 hi+lo pairs (2) or fp16 (1)")
    ap.add_argument("--no-extras", action="store_true", help="run the GEMV headline only")
    ap.add_argument("--legs", default="decode,lm,layer,prefill,batch,fx,q4c,group",
                    help="comma list of the legs beside the GEMV headline: decode (28-layer decode), "
                         "lm (LM head alone), lmsweep (LM head over 4096..151936 rows, not by default), "
                         "layer (one decoder layer at --ctx), layerlong (one layer at 4096..32768 cached "
                         "positions under both decode plans, not by default), prefill, batch (batched decode), "
                         "fx fixed-point (RTL-exact) layer and token, q4c float -> Q4 conversion of the model, "
                         "group (the headline GEMV over 64 matrices per launch)")
    ap.add_argument("--extras", dest="legs", default=argparse.SUPPRESS, help="the same as --legs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--decode-gen", type=int, default=256)
    ap.add_argument("--gemv-replays", type=int, default=0,
                    help="timed regions of --steps GEMV launches (0: enough for ~0.1 s, 11..200)")
    ap.add_argument("--gemv-warm-s", type=float, default=GEMV_WARM_S,
                    help="seconds of sustained GEMV launches before the timed regions")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy (scales FETCH_SIZE/WRITE_SIZE counters)")
    return ap.parse_args()


def graph_of(fn, n, torch):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(n):
                fn(i)
    torch.cuda.current_stream().wait_stream(s)
    return g


def time_graph(g, replays, torch):
    """Average ms per replay over `replays`, HIP events on the current stream."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / replays


def load_json(name):
    path = os.path.join(PROFILES, name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


# ------------------------------------------------------------------ GEMV headline
def leg_gemv(args, lib, torch, np, dev, st):
    from llm_accelerator_amd._lib import check
    from llm_accelerator_amd.model import Q4Tensor, gemv_bytes, random_q4
    rng = np.random.default_rng(0)
    packed, scale = random_q4(rng, GEMV_ROWS, GEMV_COLS)
    ncop = max(1, args.copies)
    P = torch.from_numpy(packed).to(dev).unsqueeze(0).repeat(ncop, 1, 1).contiguous()
    S = torch.from_numpy(scale).to(dev).unsqueeze(0).repeat(ncop, 1, 1).contiguous()
    mats = [Q4Tensor(P[i], S[i]).descriptor() for i in range(ncop)]
    gen = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(1, GEMV_COLS, generator=gen, device=dev).half()
    y = torch.empty(1, GEMV_ROWS, device=dev, dtype=torch.float16)
    # the floor: the same kernel on a 2 x 1024 matrix
    tiny = Q4Tensor(P[0, :2].contiguous(), S[0, :2].contiguous())
    tiny_desc = tiny.descriptor()

    def launch(m):
        check(lib.q4d_linear(ctypes.byref(m), x.data_ptr(), 0, y.data_ptr(), 0, 1, st()), "q4d_linear")

    gb = gemv_bytes(GEMV_ROWS, GEMV_COLS)
    for i in range(args.warmup):
        launch(mats[i % ncop])
    torch.cuda.synchronize()
    # step i of the timed region reads copy i % ncop: full rotations, then the rest
    full, rest = divmod(args.steps, ncop)
    g_rot = graph_of(lambda i: launch(mats[i]), ncop, torch)
    g_rest = graph_of(lambda i: launch(mats[i]), rest, torch) if rest else None
    g_rot.replay()
    if g_rest is not None:
        g_rest.replay()
    timed = [g_rot] * full + ([g_rest] if g_rest is not None else [])
    # the GPU leaves its idle clocks only under sustained load: ~0.3 s of the same launches
    # first, whatever --warmup asks (a cold start read 18 % slower at --steps 20 --warmup 5)
    t_w = time.perf_counter()
    while time.perf_counter() - t_w < args.gemv_warm_s:
        g_rot.replay()
        torch.cuda.synchronize()
    # the K timed steps, as REPLAYS separate timed regions; before each, an untimed full
    # rotation (200 copies, 336 MB > the 256 MB cache) evicts the copies the region reads
    # and keeps the GPU busy, so the region starts right after it on a warm device
    reps = args.gemv_replays or max(GEMV_MIN_REPLAYS, min(200, int(GEMV_TIMED_S * 1e6 / (2.0 * args.steps))))
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1 in ev:
        g_rot.replay()                # lead-in, untimed
        e0.record()
        for g in timed:
            g.replay()
        e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = sorted(e0.elapsed_time(e1) * 1e3 / args.steps for e0, e1 in ev)
    us = per[len(per) // 2]
    spread = {"replays": reps, "min": round(per[0], 3), "p25": round(per[len(per) // 4], 3),
              "median": round(us, 3), "p75": round(per[(3 * len(per)) // 4], 3), "max": round(per[-1], 3)}
    ok = bool(torch.isfinite(y.float()).all().item())
    log(f"[bench] GEMV 3072x1024 flushed: {us:.3f} us/launch (median of {reps} timed regions of {args.steps} "
        f"launches; spread {spread}), {gb / us / 1e3:.1f} GB/s (wall incl. lead-ins {wall * 1e3:.2f} ms)")

    g_res = graph_of(lambda i: launch(mats[0]), ncop, torch)
    g_res.replay()
    us_res = time_graph(g_res, max(2, args.steps // ncop), torch) / ncop * 1e3
    g_tiny = graph_of(lambda i: launch(tiny_desc), ncop, torch)
    g_tiny.replay()
    us_floor = time_graph(g_tiny, max(2, args.steps // ncop), torch) / ncop * 1e3
    log(f"[bench] GEMV resident {us_res:.3f} us, single-launch floor (2x1024) {us_floor:.3f} us")
    out = {"us": us, "GBps": gb / us / 1e3, "bytes": gb, "wall_s": wall, "finite": ok, "spread": spread,
           "resident_us": us_res, "resident_GBps": gb / us_res / 1e3, "floor_us": us_floor}
    del P, S, g_rot, g_rest, g_res, g_tiny, tiny
    torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------ decoder layer
# (KV capacity, position) cases of the long-context layer leg: the first position past each
# power-of-two capacity, Qwen3's full 32768-position context, and short positions in long caches
LAYER_LONG_CASES = ((4097, 4096), (8193, 8192), (16385, 16384), (32768, 32767), (32768, 1000),
                    (4096, 200), (4096, 1000), (4096, 4000), (1024, 1000), (2048, 300), (2048, 2000))


def leg_layer_long(lib, torch, dev, st):
    """One decoder layer (resident weights, random cache) at long contexts, under the
    XCD-split plan (q4d_set_decode_plan(0)) and the staged plan (1)."""
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd._lib import check
    cfg = M.Qwen3Config(num_hidden_layers=1, vocab_size=2048)
    host = M.random_host_weights(cfg, seed=0, num_layers=1)
    rows = []
    for cap, pos_v in LAYER_LONG_CASES:
        model = M.build_model(cfg, host, max_ctx=cap, device=dev)
        kv = M.KVCache(cfg, 1, 1, cap, dev)
        gen = torch.Generator(device=dev).manual_seed(2)
        kv.data.normal_(generator=gen)
        ws = M.Workspace(model, 1)
        pos = torch.tensor([pos_v], dtype=torch.int32, device=dev)
        h_in = torch.randn(1, 1024, generator=gen, device=dev, dtype=torch.float32)
        h_out = torch.empty_like(h_in)
        desc, kvd = model.descriptor(), kv.descriptor()

        def step(i):
            check(lib.q4d_decoder_layer(ctypes.byref(desc), 0, h_in.data_ptr(), h_out.data_ptr(), ctypes.byref(kvd),
                                        pos.data_ptr(), ws.ptr, ws.nbytes, st()), "q4d_decoder_layer")

        row = {"max_ctx": cap, "position": pos_v}
        for name, plan in (("xcd", 0), ("staged", 1)):
            prev = lib.q4d_set_decode_plan(plan)
            try:
                active = int(lib.q4d_decode_plan_active(ctypes.byref(desc), st()))
                step(0)
                g = graph_of(step, 20, torch)
                g.replay()
                us = min(time_graph(g, 10, torch) for _ in range(3)) / 20 * 1e3
                del g
            finally:
                lib.q4d_set_decode_plan(prev)
            row[f"{name}_us"] = round(us, 2)
            row[f"{name}_plan_active"] = active
            row[f"{name}_status"] = ws.status()
        log(f"[bench] layer at max_ctx {cap}, position {pos_v}: xcd {row['xcd_us']} us, staged {row['staged_us']} us")
        rows.append(row)
        del model, kv, ws
        torch.cuda.empty_cache()
    return {"workload": "one Qwen3-0.6B decoder layer, one decode step, resident weights, fp16 cache of "
                        "max_ctx positions (random), graphs of 20 steps (best of 3 x 10 replays)",
            "plan_active": "q4d_decode_plan_active: 0 the XCD-split layer, 1 the staged launches",
            "cases": rows}


def leg_layer(args, lib, torch, dev, st):
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd._lib import check
    ctx, copies = args.ctx, args.layer_copies
    cfg = M.Qwen3Config(num_hidden_layers=copies, vocab_size=2048)
    t = time.time()
    host = M.random_host_weights(cfg, seed=0, num_layers=copies)
    model = M.build_model(cfg, host, max_ctx=ctx + 1, device=dev)
    del host
    kv = M.KVCache(cfg, copies, 1, ctx + 1, dev)
    gen = torch.Generator(device=dev).manual_seed(2)
    kv.data.normal_(generator=gen)
    ws = M.Workspace(model, 1)
    pos = torch.tensor([ctx], dtype=torch.int32, device=dev)
    h_in = torch.randn(1, 1024, generator=gen, device=dev, dtype=torch.float32)
    h_out = torch.empty_like(h_in)
    desc, kvd = model.descriptor(), kv.descriptor()
    log(f"[bench] layer setup {time.time() - t:.1f}s: {copies} layers, ctx {ctx}")

    def layer_step(i):
        check(lib.q4d_decoder_layer(ctypes.byref(desc), i % copies, h_in.data_ptr(), h_out.data_ptr(),
                                    ctypes.byref(kvd), pos.data_ptr(), ws.ptr, ws.nbytes, st()),
              "q4d_decoder_layer")

    layer_step(0)
    g_flush = graph_of(layer_step, copies, torch)
    g_flush.replay()
    reps = 10
    fl_us = time_graph(g_flush, reps, torch) / copies * 1e3
    g_res = graph_of(lambda i: layer_step(0), copies, torch)
    g_res.replay()
    res_us = time_graph(g_res, reps, torch) / copies * 1e3
    step_bytes = M.algorithmic_bytes_layer(M.Qwen3Config(), ctx)
    stage_names = ["qkv", "attention", "o_proj", "gate_up", "down"]
    stage_us = {}
    for sidx, sname in enumerate(stage_names):
        def stage(i, sidx=sidx):
            check(lib.q4d_layer_stage(ctypes.byref(desc), i % copies, sidx, h_in.data_ptr(), h_out.data_ptr(),
                                      ctypes.byref(kvd), pos.data_ptr(), ws.ptr, ws.nbytes, st()),
                  "q4d_layer_stage")
        g = graph_of(stage, copies, torch)
        g.replay()
        stage_us[sname] = time_graph(g, reps, torch) / copies * 1e3
    stage_bytes = M.stage_bytes_layer(M.Qwen3Config(), ctx)
    out = {"workload": f"one Qwen3-0.6B decoder layer, one decode step at ctx {ctx}, weights rotated over "
                       f"{copies} distinct layers (flushed) or one layer repeated (resident)",
           "plan": "q4d_decoder_layer: the XCD-split layer (launch A, launch B, output sum); "
                   "stage_us_flushed: the five staged launches of q4d_layer_stage",
           "bytes_per_step": step_bytes, "flushed_us": round(fl_us, 3),
           "flushed_GBps": round(step_bytes / fl_us / 1e3, 1), "resident_us": round(res_us, 3),
           "resident_GBps": round(step_bytes / res_us / 1e3, 1),
           "stage_us_flushed": {k: round(v, 3) for k, v in stage_us.items()},
           "stage_GBps": {k: round(stage_bytes[k] / stage_us[k] / 1e3, 1) for k in stage_names},
           "stage_kernels": STAGE_KERNELS}
    xj = load_json("decode_xcd_layer_hbm_traffic.json")
    if xj and ctx == 512 and args.precision == 2:
        # the plan flushed_us times: counter-measured HBM bytes of its two launches
        out["traffic_bytes"] = {k: v["total_bytes"] for k, v in xj["launches"].items()}
        out["traffic_algorithmic_bytes"] = {k: v["algorithmic_bytes"] for k, v in xj["launches"].items()}
        out["traffic_source"] = xj["source"]
    tj = load_json("decode_layer_ctx512_hbm_traffic.json")
    if tj and ctx == 512 and args.precision == 2:
        out["stage_traffic_bytes"] = {k: v["total_bytes"] for k, v in tj["stages"].items()}
        out["stage_traffic_source"] = tj["source"]
    log(f"[bench] decoder layer: {json.dumps(out)}")
    del model, kv, ws, g_flush, g_res
    torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------ 28-layer decode
def aliased_descriptor(model):
    """The model's descriptor with every layer pointing at layer 0's weights."""
    from llm_accelerator_amd._lib import Q4dLayer, Q4dModel
    d0 = model.descriptor()
    n = d0.num_layers
    arr = (Q4dLayer * n)(*([d0.layers[0]] * n))
    d = Q4dModel.from_buffer_copy(d0)
    d.layers = ctypes.cast(arr, ctypes.POINTER(Q4dLayer))
    d._layers_keepalive = arr  # type: ignore[attr-defined]
    return d


def run_decode(fmodel, prompt, gen_steps, per_graph, torch, desc=None):
    from llm_accelerator_amd.decode import GreedyDecoder
    dec = GreedyDecoder(fmodel, steps_per_graph=per_graph, use_graph=True)
    if desc is not None:
        dec._desc = desc   # noqa: SLF001  (the aliased-weights variant)
    dec.prefill(prompt)
    dec.generate(per_graph)        # captures and warms the graph
    dec.prefill(prompt)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    dec.generate(gen_steps)
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1)
    toks, _ = dec.history()
    out = {"us_per_token": ms * 1e3 / gen_steps, "wall_us_per_token": wall * 1e6 / gen_steps,
           "generated": len(toks), "status": dec.status()}
    del dec
    return out


def decode_launch_floor(torch, fmodel, tokens=15, replays=20, staged=False):
    """A decode step's launches with their grids, each kernel reduced to one dependent
    read of the previous launch's 4 KB output (q4d_diag_launch_chain), graph-replayed:
    what the launches of a token cost without their work.  Grids (blocks x threads) of
    the step's kernels, as the kernel trace of this leg shows them.  XCD-split plan:
    per layer launch A and launch B, 256 x 320 each, then the LM head 256 x 1024 (which
    forms the last layer's output in its prologue).  Staged plan: q|k|v 512 x 256, attention
    ceil(max_ctx / 64) x kv_heads blocks of 256, o_proj 128 x 512, gate/up 384 x 256,
    down 256 x 384, LM head 256 x 1024."""
    from llm_accelerator_amd import _lib
    lib = _lib.load()
    cfg = fmodel.config
    if staged:
        layer = [(512, 1, 256), ((fmodel.max_ctx + 63) // 64, cfg.num_key_value_heads, 256), (128, 1, 512),
                 (384, 1, 256), (256, 1, 384)]
        shapes = layer * cfg.num_hidden_layers + [(256, 1, 1024)]
    else:
        shapes = [(256, 1, 320), (256, 1, 320)] * cfg.num_hidden_layers + [(256, 1, 1024)]
    n = len(shapes)
    gx = (ctypes.c_int32 * n)(*[x for x, _, _ in shapes])
    gy = (ctypes.c_int32 * n)(*[y for _, y, _ in shapes])
    bl = (ctypes.c_int32 * n)(*[b for _, _, b in shapes])
    buf = torch.zeros(2048, dtype=torch.float32, device=fmodel.device)

    def chain(i):
        rc = lib.q4d_diag_launch_chain(ctypes.cast(gx, ctypes.c_void_p), ctypes.cast(gy, ctypes.c_void_p),
                                       ctypes.cast(bl, ctypes.c_void_p), n, buf.data_ptr(),
                                       torch.cuda.current_stream().cuda_stream)
        if rc:
            raise RuntimeError(f"q4d_diag_launch_chain: {rc}")
    g = graph_of(chain, tokens, torch)
    time_graph(g, 2, torch)
    us = time_graph(g, replays, torch) / tokens * 1e3
    return {"us_per_token": round(us, 2), "launches_per_token": n,
            "us_per_launch": round(us / n, 3)}


def leg_decode(args, torch, np, fmodel):
    from llm_accelerator_amd import model as M
    fcfg = fmodel.config
    prompt = np.random.default_rng(1).integers(0, fcfg.vocab_size, PROMPT).tolist()
    steps = args.decode_gen - 1                     # token 0 comes from the last prompt step
    per_graph = max(d for d in range(1, 17) if steps % d == 0)
    from llm_accelerator_amd import _lib
    lib = _lib.load()
    flushed = run_decode(fmodel, prompt, steps, per_graph, torch)
    resident = run_decode(fmodel, prompt, steps, per_graph, torch, desc=aliased_descriptor(fmodel))
    floor = decode_launch_floor(torch, fmodel, tokens=per_graph)
    # the staged five-launch layer (q4d_set_decode_plan), for comparison
    prev = lib.q4d_set_decode_plan(1)
    try:
        staged = run_decode(fmodel, prompt, steps, per_graph, torch)
    finally:
        lib.q4d_set_decode_plan(prev)
    staged_floor = decode_launch_floor(torch, fmodel, tokens=per_graph, staged=True)
    # step p feeds position p and attends p + 1 positions
    tok_bytes = sum(M.batched_step_bytes(fcfg, 1, p + 1) for p in range(PROMPT, PROMPT + steps)) / steps
    wb = fmodel.weight_bytes()
    res_bytes = tok_bytes - (wb["per_layer"] * (fcfg.num_hidden_layers - 1))
    tok_s = 1e6 / flushed["us_per_token"]
    out = {"workload": f"28-layer greedy decode, batch 1: {PROMPT}-token uniform random prompt, "
                       f"{args.decode_gen} generated (argmax fed back on the device, HIP graphs of {per_graph} steps)",
           "tok_s": round(tok_s, 1), "us_per_token": round(flushed["us_per_token"], 2),
           "wall_us_per_token": round(flushed["wall_us_per_token"], 2),
           "bytes_per_token": int(tok_bytes), "GBps": round(tok_bytes * tok_s / 1e9, 1),
           "roofline_frac": round(tok_bytes * tok_s / 1e9 / HBM_PEAK_GBPS, 4),
           "generated": flushed["generated"], "status": flushed["status"],
           "plan": "XCD-split layer: 2 launches per layer (one kv head per XCD), LM head (forms the last layer's output)",
           "launches_per_token": floor["launches_per_token"],
           "launch_floor": dict(floor, note=f"the same {floor['launches_per_token']} launches with their grids, "
                                            "each kernel only one dependent 4 KB read and write "
                                            "(q4d_diag_launch_chain)",
                                share=round(floor["us_per_token"] / flushed["us_per_token"], 3)),
           "staged": {"note": "the five-launch layer of q4d_layer_stage (q4d_set_decode_plan(1))",
                      "tok_s": round(1e6 / staged["us_per_token"], 1),
                      "us_per_token": round(staged["us_per_token"], 2), "status": staged["status"],
                      "launches_per_token": staged_floor["launches_per_token"],
                      "launch_floor_us_per_token": staged_floor["us_per_token"]},
           "resident": {"note": "every layer aliased to layer 0's weights: 91 MB per token, inside the 256 MB cache",
                        "tok_s": round(1e6 / resident["us_per_token"], 1),
                        "us_per_token": round(resident["us_per_token"], 2),
                        "bytes_per_token": int(res_bytes), "status": resident["status"]}}
    log(f"[bench] 28-layer decode: {json.dumps(out)}")
    return out


def leg_lm(lib, torch, dev, st, fmodel):
    """Final RMSNorm + 151936x1024 Q4 GEMV + argmax alone, rotating over 4 copies
    of the table (flushed) and on one copy (repeated)."""
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd._lib import Q4dMatrix, Q4dModel, check
    fcfg = fmodel.config
    lw = fmodel.lm_head.weight
    copies = [lw] + [type(lw)(lw.packed.clone(), lw.scale.clone()) for _ in range(3)]
    base = fmodel.descriptor()
    descs = []
    for c in copies:
        d = Q4dModel.from_buffer_copy(base)
        d.embed_tokens = Q4dMatrix(c.packed.data_ptr(), c.scale.data_ptr(), fcfg.vocab_size, fcfg.hidden_size)
        descs.append(d)
    gen = torch.Generator(device=dev).manual_seed(3)
    hid = torch.randn(1, fcfg.hidden_size, generator=gen, device=dev)
    lm_tok = torch.zeros(1, dtype=torch.int32, device=dev)
    lm_score = torch.zeros(1, dtype=torch.float32, device=dev)
    lws = M.Workspace(fmodel, 1)

    def lm_head(d):
        check(lib.q4d_lm_head_argmax(ctypes.byref(d), hid.data_ptr(), lm_tok.data_ptr(), lm_score.data_ptr(),
                                     None, lws.ptr, lws.nbytes, st()), "lm_head")
    g_fl = graph_of(lambda i: lm_head(descs[i % 4]), 8, torch)
    g_rp = graph_of(lambda i: lm_head(descs[0]), 8, torch)
    g_fl.replay()
    g_rp.replay()
    fl_us = time_graph(g_fl, 10, torch) / 8 * 1e3
    rp_us = time_graph(g_rp, 10, torch) / 8 * 1e3
    lm_bytes = lw.nbytes + 4 * fcfg.hidden_size * 2
    lm = {"workload": "final RMSNorm + 151936x1024 Q4 GEMV + argmax; flushed = rotating over 4 copies of the "
                      "table (331 MB), repeated = one copy", "bytes": lm_bytes,
          "flushed_us": round(fl_us, 2), "flushed_GBps": round(lm_bytes / fl_us / 1e3, 1),
          "flushed_frac": round(lm_bytes / fl_us / 1e3 / HBM_PEAK_GBPS, 4),
          "repeated_us": round(rp_us, 2), "repeated_GBps": round(lm_bytes / rp_us / 1e3, 1)}
    tj = load_json("lm_head_hbm_traffic.json")
    if tj:
        lm["traffic"] = tj.get("total_bytes")
        lm["traffic_source"] = tj.get("source")
    log(f"[bench] LM head: {json.dumps(lm)}")
    del copies, descs, lws, g_fl, g_rp
    torch.cuda.empty_cache()
    return lm


def leg_lmsweep(lib, torch, dev, st, fmodel, np):
    """The LM head (final RMSNorm + Q4 GEMV + argmax) over the first R rows of the
    table for several R, flushed (rotating over 4 copies), and a least-squares line
    time = fixed + bytes / rate over R >= 32768: the kernel's marginal streaming rate
    and its fixed cost (prologue, ramp, tail, argmax hand-off)."""
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd._lib import Q4dMatrix, Q4dModel, check
    fcfg = fmodel.config
    lw = fmodel.lm_head.weight
    copies = [lw] + [type(lw)(lw.packed.clone(), lw.scale.clone()) for _ in range(3)]
    base = fmodel.descriptor()
    gen = torch.Generator(device=dev).manual_seed(3)
    hid = torch.randn(1, fcfg.hidden_size, generator=gen, device=dev)
    tok = torch.zeros(1, dtype=torch.int32, device=dev)
    score = torch.zeros(1, dtype=torch.float32, device=dev)
    lws = M.Workspace(fmodel, 1)
    rows_list = [4096, 8192, 16384, 32768, 65536, 98304, 131072, fcfg.vocab_size]
    pts = []
    H = fcfg.hidden_size
    for R in rows_list:
        # every disjoint R-row window of the 4 tables (331 MB > the 256 MB cache for each R),
        # in turn: each launch reads rows no launch has read since they left the cache
        descs = []
        for j in range(fcfg.vocab_size // R):
            for c in copies:
                d = Q4dModel.from_buffer_copy(base)
                d.vocab_size = R
                d.embed_tokens = Q4dMatrix(c.packed.data_ptr() + j * R * (H // 2), c.scale.data_ptr() + j * R * (H // 32),
                                           R, H)
                descs.append(d)
        n = len(descs)

        def lm_head(i, descs=descs):
            check(lib.q4d_lm_head_argmax(ctypes.byref(descs[i]), hid.data_ptr(), tok.data_ptr(),
                                         score.data_ptr(), None, lws.ptr, lws.nbytes, st()), "lm_head")
        g = graph_of(lm_head, n, torch)
        g.replay()
        us = time_graph(g, max(2, 80 // n), torch) / n * 1e3
        nbytes = R * (fcfg.hidden_size // 2 + fcfg.hidden_size // 32) + 4 * fcfg.hidden_size * 2
        pts.append({"rows": R, "bytes": nbytes, "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1)})
        del g, descs
    big = [p for p in pts if p["rows"] >= 32768]
    xb = np.array([p["bytes"] for p in big], dtype=np.float64)
    yt = np.array([p["us"] for p in big], dtype=np.float64)
    slope, icpt = np.polyfit(xb, yt, 1)
    out = {"workload": "final RMSNorm + R x 1024 Q4 GEMV + argmax over R-row windows of the table; one graph "
                       "runs every disjoint R-row window of 4 table copies (331 MB, flushed) in turn",
           "points": pts,
           "fit_rows_min": 32768, "marginal_GBps": round(1e-3 / slope, 1), "fixed_us": round(icpt, 3)}
    log(f"[bench] LM head size sweep: {json.dumps(out)}")
    del copies, lws
    torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------ prefill, batched, fixed point, Q4 conversion
def leg_prefill(torch, np, dev, fmodel):
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd.decode import Prefill
    fcfg = fmodel.config
    T = PREFILL_TOKENS
    pkv = M.KVCache(fcfg, fcfg.num_hidden_layers, 1, fmodel.max_ctx, dev)
    pf = Prefill(fmodel, pkv, T)
    ptok = torch.from_numpy(np.random.default_rng(4).integers(0, fcfg.vocab_size, T).astype(np.int32)).to(dev)
    pf.run(ptok)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        pf.run(ptok)
    e1.record()
    torch.cuda.synchronize()
    pms = e0.elapsed_time(e1) / 5
    pflops = M.prefill_flops(fcfg, T)
    out = {"tokens": T, "ms": round(pms, 3), "tok_s": round(T / pms * 1e3, 1),
           "TFLOPs": round(pflops / pms / 1e9, 1), "flops": pflops,
           "mfma_frac": round(pflops / pms / 1e9 / MFMA_PEAK_TFLOPS, 4)}
    log(f"[bench] prefill 2048: {json.dumps(out)}")
    del pkv, pf
    torch.cuda.empty_cache()
    return out


def leg_batch(torch, np, dev, fmodel):
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd.decode import BatchedDecoder
    fcfg = fmodel.config
    B = BATCH_SEQS
    gen = torch.Generator(device=dev).manual_seed(5)
    bkv = M.KVCache(fcfg, fcfg.num_hidden_layers, B, BATCH_CTX + 1, dev)
    bkv.data[..., :BATCH_CTX, :].normal_(generator=gen)
    bd = BatchedDecoder(fmodel, B, bkv)
    btok = torch.from_numpy(np.random.default_rng(3).integers(0, fcfg.vocab_size, B).astype(np.int32)).to(dev)
    bpos = torch.full((B,), BATCH_CTX, dtype=torch.int32, device=dev)
    bd.step(btok, bpos)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(5):
        bd.step(btok, bpos)
    e1.record()
    torch.cuda.synchronize()
    bms = e0.elapsed_time(e1) / 5
    bbytes = M.batched_step_bytes(fcfg, B, BATCH_CTX)
    out = {"batch": B, "ctx": BATCH_CTX, "ms_per_step": round(bms, 3), "tok_s": round(B / bms * 1e3, 1),
           "bytes_per_step": bbytes, "GBps": round(bbytes / bms / 1e6, 1),
           "hbm_frac": round(bbytes / bms / 1e6 / HBM_PEAK_GBPS, 4), "status": bd.status()}
    log(f"[bench] batched decode 64x4096: {json.dumps(out)}")
    del bkv, bd
    torch.cuda.empty_cache()
    return out


def leg_fixed(args, lib, torch, dev, st, fmodel, fnorms):
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd._lib import check
    from llm_accelerator_amd.fixed import FixedQ4Model
    fcfg = fmodel.config
    ctx = args.ctx
    gen = torch.Generator(device=dev).manual_seed(6)
    fxm = FixedQ4Model(M.with_context(fmodel, ctx + 1), fnorms)
    fkv = fxm.new_cache()
    fkv.data.copy_(torch.randint(-8192, 8192, fkv.data.shape, generator=gen, device=dev, dtype=torch.int32))
    fdesc, fkvd = fxm.descriptor(), fkv.descriptor()
    fpos = torch.tensor([ctx], dtype=torch.int32, device=dev)
    fh = torch.randint(-4096, 4096, (1024,), generator=gen, device=dev, dtype=torch.int32)
    fo = torch.empty_like(fh)

    def fx_layer(i):
        check(lib.q4d_fixed_decoder_layer(ctypes.byref(fdesc), i, fh.data_ptr(), fo.data_ptr(),
                                          ctypes.byref(fkvd), fpos.data_ptr(), fxm.ws.data_ptr(), fxm.ws_bytes,
                                          st()), "q4d_fixed_decoder_layer")
    L = fcfg.num_hidden_layers
    g_fx = graph_of(fx_layer, L, torch)
    g_fx.replay()
    fx_us = time_graph(g_fx, 10, torch) / L * 1e3
    fx_bytes = M.fixed_layer_bytes(fcfg, ctx)
    # one-token steps: serial prompt of 64 tokens, then graphs of 16 steps feeding the argmax back
    ftok = torch.tensor([1], dtype=torch.int32, device=dev)
    fnxt = torch.zeros(1, dtype=torch.int32, device=dev)
    fscore = torch.zeros(1, dtype=torch.int64, device=dev)
    fpos.zero_()

    def fx_token(i):
        check(lib.q4d_fixed_run_one_token(ctypes.byref(fdesc), ftok.data_ptr(), fpos.data_ptr(),
                                          ctypes.byref(fkvd), fnxt.data_ptr(), fscore.data_ptr(), None, None,
                                          fxm.ws.data_ptr(), fxm.ws_bytes, st()), "q4d_fixed_run_one_token")
        ftok.copy_(fnxt)
        fpos.add_(1)
    for i in range(64):
        fx_token(i)
    g_tok = graph_of(fx_token, 16, torch)
    g_tok.replay()
    tok_ms = time_graph(g_tok, (args.decode_gen - 16) // 16, torch) / 16
    counts = fxm.counts()
    out = {"layer_us": round(fx_us, 3), "layer_bytes": fx_bytes, "layer_GBps": round(fx_bytes / fx_us / 1e3, 1),
           "token_ms": round(tok_ms, 4), "tok_s": round(1e3 / tok_ms, 1), "positions": [64, int(fpos.item())],
           "status": counts["status"]}
    log(f"[bench] fixed-point decode: {json.dumps(out)}")
    del fxm, fkv, g_fx, g_tok
    torch.cuda.empty_cache()
    return out


def leg_q4c(lib, torch, dev, st):
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd._lib import check
    qcfg = M.Qwen3Config()
    gen = torch.Generator(device=dev).manual_seed(7)
    h, I = qcfg.hidden_size, qcfg.intermediate_size
    shapes = [(2048, h), (1024, h), (1024, h), (h, 2048), (I, h), (I, h), (h, I)] * qcfg.num_hidden_layers
    shapes.append((qcfg.vocab_size, h))
    mats = [(torch.randn(r, c, generator=gen, device=dev) * 0.03).to(torch.bfloat16) for r, c in shapes]
    outs = [(torch.empty(r, c // 2, dtype=torch.uint8, device=dev),
             torch.empty(r, c // 64, dtype=torch.uint16, device=dev)) for r, c in shapes]
    qstatus = torch.zeros(2, dtype=torch.int32, device=dev)

    def quant(i):
        w, (pk, sc) = mats[i], outs[i]
        check(lib.q4d_quantize_q4(w.data_ptr(), 2, w.shape[1], w.shape[0], w.shape[1], pk.data_ptr(),
                                  sc.data_ptr(), qstatus.data_ptr(), st()), "q4d_quantize_q4")
    # the matrices of one shape in one launch each (q4d_quantize_q4_batch): 6 launches
    groups = {}
    for i, rc in enumerate(shapes):
        groups.setdefault(rc, []).append(i)
    garr = []
    for (r, c), idx in groups.items():
        n = len(idx)
        garr.append((r, c, n, (ctypes.c_void_p * n)(*[mats[i].data_ptr() for i in idx]),
                     (ctypes.c_void_p * n)(*[outs[i][0].data_ptr() for i in idx]),
                     (ctypes.c_void_p * n)(*[outs[i][1].data_ptr() for i in idx])))

    def quant_group(k):
        r, c, n, wp, pp, sp = garr[k]
        check(lib.q4d_quantize_q4_batch(wp, 2, c, r, c, n, pp, sp, qstatus.data_ptr(), st()),
              "q4d_quantize_q4_batch")
    for i in range(len(shapes)):
        quant(i)
    for k in range(len(garr)):
        quant_group(k)
    torch.cuda.synchronize()
    # HIP graphs: the grouped conversion of the model, the 197 single conversions, the table
    g_all = graph_of(quant_group, len(garr), torch)
    g_one = graph_of(quant, len(shapes), torch)
    g_tab = graph_of(lambda i: quant(len(shapes) - 1), 1, torch)
    g_all.replay()
    g_one.replay()
    g_tab.replay()
    all_ms = time_graph(g_all, 10, torch)
    one_ms = time_graph(g_one, 10, torch)
    emb_us = time_graph(g_tab, 20, torch) * 1e3
    params = sum(r * c for r, c in shapes)
    qbytes = params * 2 + params // 2 + params // 64 * 2   # bf16 in, codes + Q2.14 scales out
    er, ec = shapes[-1]
    ebytes = er * ec * 2 + er * ec // 2 + er * ec // 64 * 2
    out = {"workload": "bf16 -> Q4 of every Qwen3-0.6B projection and the tied table (197 matrices, "
                       f"{len(garr)} launches of same-shape matrices)",
           "params": params, "bytes": qbytes, "ms": round(all_ms, 4), "GBps": round(qbytes / all_ms / 1e6, 1),
           "hbm_frac": round(qbytes / all_ms / 1e6 / HBM_PEAK_GBPS, 4),
           "one_call_per_matrix_ms": round(one_ms, 4), "table_us": round(emb_us, 2),
           "table_GBps": round(ebytes / emb_us / 1e3, 1), "status": qstatus.tolist()}
    log(f"[bench] Q4 conversion: {json.dumps(out)}")
    del mats, outs, g_all, g_one, g_tab
    torch.cuda.empty_cache()
    return out


def leg_group(lib, torch, dev, st):
    """The headline GEMV's kernel over 64 independent 3072 x 1024 matrices per launch
    (q4d_linear_group; each matrix its own fp16 x and y).  Launches rotate over 256 copies
    (430 MB, past the 256 MB cache): launch i reads copies 64 (i % 4) .. + 63, so every launch
    reads weights that left the cache.  Time per launch = graph time / launches."""
    import numpy as np
    from llm_accelerator_amd._lib import Q4dMatrix, check
    from llm_accelerator_amd.model import Q4Tensor, gemv_bytes, random_q4
    G, NCOP = 64, 256
    rng = np.random.default_rng(0)
    packed, scale = random_q4(rng, GEMV_ROWS, GEMV_COLS)
    P = torch.from_numpy(packed).to(dev).unsqueeze(0).repeat(NCOP, 1, 1).contiguous()
    S = torch.from_numpy(scale).to(dev).unsqueeze(0).repeat(NCOP, 1, 1).contiguous()
    gen = torch.Generator(device=dev).manual_seed(1)
    X = torch.randn(NCOP, GEMV_COLS, generator=gen, device=dev).half()
    Y = torch.empty(NCOP, GEMV_ROWS, device=dev, dtype=torch.float16)
    sets = []
    for r in range(NCOP // G):
        idx = range(r * G, (r + 1) * G)
        sets.append(((Q4dMatrix * G)(*[Q4Tensor(P[i], S[i]).descriptor() for i in idx]),
                     (ctypes.c_void_p * G)(*[X[i].data_ptr() for i in idx]),
                     (ctypes.c_void_p * G)(*[Y[i].data_ptr() for i in idx])))

    def launch(i):
        d, xp, yp = sets[i % len(sets)]
        check(lib.q4d_linear_group(d, xp, 0, yp, 0, 1, G, st()), "q4d_linear_group")
    for i in range(len(sets)):
        launch(i)
    torch.cuda.synchronize()
    g = graph_of(launch, 4 * len(sets), torch)
    g.replay()
    us = time_graph(g, 25, torch) / (4 * len(sets)) * 1e3
    gb = G * gemv_bytes(GEMV_ROWS, GEMV_COLS)
    ok = bool(torch.isfinite(Y.float()).all().item())
    out = {"workload": f"{G} independent 3072x1024 Q4 GEMVs per launch (fp16 x / y, batch 1), flushed",
           "bytes_per_launch": gb, "us_per_launch": round(us, 3), "GBps": round(gb / us / 1e3, 1),
           "hbm_frac": round(gb / us / 1e3 / HBM_PEAK_GBPS, 4), "finite": ok,
           "kernel": "gemv_group_kernel<1, 8, 0, 1, 0> (the headline gemv_kernel's body per matrix)"}
    log(f"[bench] grouped GEMV: {json.dumps(out)}")
    del P, S, X, Y, g
    torch.cuda.empty_cache()
    return out


def leg_copy(torch, dev):
    """torch's device copy of 512 MiB windows rotating over 2 GiB (past the 256 MB
    cache): read + written bytes over the time."""
    buf = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    w = 512 << 20
    for _ in range(2):
        buf[w:2 * w].copy_(buf[:w])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(8):
        k = i % 2
        buf[(2 * k + 1) * w:(2 * k + 2) * w].copy_(buf[2 * k * w:(2 * k + 1) * w])
    e1.record()
    torch.cuda.synchronize()
    cms = e0.elapsed_time(e1) / 8
    out = {"bytes_moved": 2 * w, "us": round(cms * 1e3, 1), "GBps": round(2 * w / (cms * 1e-3) / 1e9, 1)}
    log(f"[bench] measured copy: {json.dumps(out)}")
    del buf
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        sys.exit(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path")
    if args.steps < 1 or args.warmup < 0:
        sys.exit("--steps must be >= 1 and --warmup >= 0")
    legs = set() if args.no_extras else {x.strip() for x in args.legs.split(",") if x.strip()}
    known = {"decode", "lm", "lmsweep", "layer", "layerlong", "prefill", "batch", "fx", "q4c", "group"}
    if legs - known:
        sys.exit(f"unknown legs {sorted(legs - known)}")
    import numpy as np
    import torch

    from llm_accelerator_amd import _lib
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd._lib import check

    lib = _lib.load()
    check(lib.q4d_set_activation_precision(args.precision), "precision")
    dev = torch.device("cuda:0")
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731


    gemv = leg_gemv(args, lib, torch, np, dev, st)
    extras = {"gemv_resident_us": round(gemv["resident_us"], 3),
              "gemv_resident_GBps": round(gemv["resident_GBps"], 1)}
    if "layer" in legs:
        extras["decoder_layer"] = leg_layer(args, lib, torch, dev, st)
    if "layerlong" in legs:
        extras["decoder_layer_long_context"] = leg_layer_long(lib, torch, dev, st)

    decode = lm = None
    if legs & {"decode", "lm", "lmsweep", "prefill", "batch", "fx"}:
        fcfg = M.Qwen3Config()
        t = time.time()
        fhost = M.random_host_weights(fcfg, seed=0)
        fmodel = M.build_model(fcfg, fhost, max_ctx=max(PROMPT + args.decode_gen + 16, BATCH_CTX + 1), device=dev)
        norm_keys = ("input_layernorm", "post_attention_layernorm", "q_norm", "k_norm")
        fnorms = {"layers": [{k: L[k] for k in norm_keys} for L in fhost["layers"]], "norm": fhost["norm"]}
        del fhost
        log(f"[bench] 28-layer model setup {time.time() - t:.1f}s")
        if "decode" in legs:
            # decode at its own context capacity (prompt + generated), as a caller would size it
            decode = leg_decode(args, torch, np, M.with_context(fmodel, PROMPT + args.decode_gen + 16))
        if "lm" in legs:
            lm = leg_lm(lib, torch, dev, st, fmodel)
        if "lmsweep" in legs:
            extras["lm_head_size_sweep"] = leg_lmsweep(lib, torch, dev, st, fmodel, np)
        if "prefill" in legs:
            extras["prefill_2048"] = leg_prefill(torch, np, dev, fmodel)
        if "batch" in legs:
            extras["batched_decode_64x4096"] = leg_batch(torch, np, dev, fmodel)
        if "fx" in legs:
            extras["fx_fixed_point"] = leg_fixed(args, lib, torch, dev, st, fmodel, fnorms)
        del fmodel
        torch.cuda.empty_cache()
    if "q4c" in legs:
        extras["q4c_quantize"] = leg_q4c(lib, torch, dev, st)
    if "group" in legs:
        extras["gemv_group_64x3072x1024"] = leg_group(lib, torch, dev, st)
    if legs:
        extras["hbm_copy"] = leg_copy(torch, dev)

    if args.copy_calibration:
        # a plain copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch
        # converts the counters of the other dispatches to bytes
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        extras["copy_calibration_bytes"] = 256 << 20
        del src, dst

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"[bench] CPU baseline: {json.dumps(cpu)}")
        if legs:
            extras["cpu_legs"] = cpu_extra_legs(args.ctx, M.algorithmic_bytes_layer(M.Qwen3Config(), args.ctx))
            log(f"[bench] CPU legs: {json.dumps(extras['cpu_legs'])}")

    gb = gemv["bytes"]
    value = gemv["GBps"]
    floor_us = gemv["floor_us"]
    roofline = {"bound": "hbm", "kernel": f"{GEMV_KERNEL} (3072x1024 Q4 GEMV, fp16 x / y)",
                "achieved": round(value, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(value / HBM_PEAK_GBPS, 4), "traffic": None,
                "bytes_per_launch": gb, "avg_launch_us": round(gemv["us"], 3),
                "timing": {"method": f"median over {gemv['spread']['replays']} timed regions of exactly "
                                     f"{args.steps} launches (HIP events), each after an untimed 200-copy rotation",
                           "us_per_launch": gemv["spread"]},
                "single_launch_floor_us": round(floor_us, 3),
                "single_launch_ceiling_GBps": round(gb / (floor_us * 1e3 + gb / HBM_PEAK_GBPS), 1)}
    tj = load_json("gemv_3072x1024_hbm_traffic.json")
    if tj:
        roofline["traffic"] = tj["total_bytes"]
        roofline["traffic_source"] = tj["source"]
        roofline["tcc_hit_rate"] = tj.get("tcc_hit_rate")
    if "hbm_copy" in extras:
        roofline["measured_copy_GBps"] = extras["hbm_copy"]["GBps"]
        roofline["frac_of_measured_copy"] = round(value / extras["hbm_copy"]["GBps"], 4)
    line = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(gemv["us"] * 1e-3, 6), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None,
            "dtype": "q4 weights x f16 activations, f32 accumulate",
            "data": "synthetic (seeded random-init Q4 weights, N(0,1) fp16 x; decode: random prompt ids)",
            "config": {"workload": f"one 3072x1024 Q4 dequant-GEMV (Qwen3-0.6B gate_proj shape), fp16 x ~ N(0,1), "
                                   f"batch 1, fp16 y; each step reads another of {max(1, args.copies)} copies of the "
                                   f"matrix ({max(1, args.copies) * gb / 1e6:.0f} MB > the 256 MB cache: flushed)",
                       "rows": GEMV_ROWS, "cols": GEMV_COLS, "batch": 1, "bytes_per_step": gb,
                       "copies": max(1, args.copies), "value_pct_of_peak": round(100 * value / HBM_PEAK_GBPS, 2),
                       "decode_activation_precision": "fp16 hi+lo pairs (~22 bits)" if args.precision == 2
                       else "fp16", "kv_cache": "fp16"},
            "roofline": roofline, "cpu_baseline": cpu, "decode": decode, "lm_head": lm, "extras": extras}
    print(json.dumps(line), flush=True)


def cpu_baseline(seconds):
    """The oracle's fp32 matvec for the 3072x1024 GEMV (manual_linear_from_weight,
    common.py:137-145, on the matrix dequantised once) on the host cores, a
    bounded sample, in GB/s of the GEMV's algorithmic bytes."""
    import numpy as np

    import oracle as o
    from llm_accelerator_amd import model as M
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:  # threadpoolctl missing: numpy default
        threads = os.cpu_count() or 1
    rng = np.random.default_rng(0)
    packed, scale = M.random_q4(rng, GEMV_ROWS, GEMV_COLS)
    W = o.dequantize_q4(packed, scale, np.float32)
    x = rng.normal(size=(1, GEMV_COLS)).astype(np.float32)
    o.manual_linear_from_weight(x, W)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(100):
            o.manual_linear_from_weight(x, W)
        n += 100
    dt = (time.perf_counter() - t0) / n
    gb = M.gemv_bytes(GEMV_ROWS, GEMV_COLS)
    return {"value": round(gb / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} fp32 matvecs y = x @ W.T, W 3072x1024 dequantised once (oracle restatement of "
                      f"manual_linear_from_weight, common.py:137-145), {dt * 1e6:.2f} us each = "
                      f"{GEMV_ROWS * GEMV_COLS * 4 / dt / 1e9:.1f} GB/s of fp32 weights; rate quoted over the Q4 "
                      f"GEMV's {gb} algorithmic bytes; os.cpu_count()={os.cpu_count()}, "
                      f"affinity={len(os.sched_getaffinity(0))}"}


def _median_time(fn, reps, budget_s):
    fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < reps or (time.perf_counter() < t_end and len(ts) < 10 * reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], len(ts)


def cpu_extra_legs(ctx, step_bytes):
    """The other CPU baselines: the int64 Q26 restatement of the GEMV
    (compute_q4_gemv_q26, 28_export_mlp_gate_up_vectors.py:124-133), the
    decoder-layer step at context ``ctx`` on all threads and on one
    (manual_decoder_layer_cached, common.py:231-298), the 28-layer decode
    (run_manual_one_token, 10_validate_full_run_one_token.py:17-56, 8 serial
    steps of the 28-layer model, per token) and the oracle's quantizer.
    Medians of >= 10 timed runs after a warm-up."""
    import numpy as np

    import oracle as o
    from llm_accelerator_amd import model as M
    try:
        from threadpoolctl import threadpool_limits
    except Exception:  # threadpoolctl missing: no one-thread leg
        threadpool_limits = None
    out = {"cores": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    rng = np.random.default_rng(0)
    packed, scale = M.random_q4(rng, GEMV_ROWS, GEMV_COLS)
    q = o.unpack_signed_int4(packed, GEMV_COLS)
    xi = rng.integers(-(1 << 20), 1 << 20, size=GEMV_COLS)
    gb = M.gemv_bytes(GEMV_ROWS, GEMV_COLS)
    t, n = _median_time(lambda: o.q4_gemv_q26(xi, q, scale), 10, 2.0)
    out["gemv_int64_q26"] = {"us": round(t * 1e6, 1), "GBps": round(gb / t / 1e9, 3), "runs": n}
    cfg = M.Qwen3Config(num_hidden_layers=1, vocab_size=2048)
    host = M.random_host_weights(cfg, seed=0, num_layers=1)
    om = o.OracleModel.from_q4(o.OracleConfig(num_hidden_layers=1, vocab_size=2048), host["layers"],
                               *host["embed_tokens"], host["norm"])
    k = rng.normal(size=(1, 8, ctx, 128)).astype(np.float32)
    v = rng.normal(size=(1, 8, ctx, 128)).astype(np.float32)
    h = rng.normal(size=(1, 1, 1024)).astype(np.float32)
    pos = np.array([[ctx]])

    def layer():
        o.manual_decoder_layer_cached(h, om.layers[0], om.config, om.inv_freq, pos, k, v)
    t, n = _median_time(layer, 10, 3.0)
    out["layer_all_threads"] = {"ms_per_step": round(t * 1e3, 3), "GBps": round(step_bytes / t / 1e9, 3), "runs": n}
    if threadpool_limits is not None:
        with threadpool_limits(limits=1):
            t, n = _median_time(layer, 10, 3.0)
        out["layer_one_thread"] = {"ms_per_step": round(t * 1e3, 3), "GBps": round(step_bytes / t / 1e9, 3),
                                   "runs": n}
    fcfg = M.Qwen3Config()
    fhost = M.random_host_weights(fcfg, seed=0)
    om = o.OracleModel.from_q4(o.OracleConfig(), fhost["layers"], *fhost["embed_tokens"], fhost["norm"])
    del fhost
    kc, vc = [None] * fcfg.num_hidden_layers, [None] * fcfg.num_hidden_layers
    toks = rng.integers(0, fcfg.vocab_size, 8)
    ts = []
    for p, tk in enumerate(toks):
        t0 = time.perf_counter()
        o.run_manual_one_token(np.array([[int(tk)]]), p, om, kc, vc)
        ts.append(time.perf_counter() - t0)
    tt = sorted(ts[1:])[len(ts[1:]) // 2]
    out["decode_per_token"] = {"ms": round(tt * 1e3, 1), "tok_s": round(1.0 / tt, 2), "steps": len(ts),
                               "note": "median of steps 1-7 at positions 1-7 (the first step is the warm-up)"}
    wq = (rng.standard_normal((GEMV_ROWS, GEMV_COLS)) * 0.03).astype(np.float32)
    t, n = _median_time(lambda: o.quantize_weight_q4(wq), 5, 2.0)
    qb = GEMV_ROWS * GEMV_COLS * 4 + GEMV_ROWS * 512 + GEMV_ROWS * 16 * 2
    out["q4c_oracle"] = {"shape": "3072x1024 fp32 -> Q4", "ms": round(t * 1e3, 2), "GBps": round(qb / t / 1e9, 3),
                         "runs": n}
    return out


if __name__ == "__main__":
    main()
