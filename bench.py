#!/usr/bin/env python3
"""Benchmark of the Qwen3-0.6B Q4 decode hot path on one MI355X.

Default workload (the headline line): one Qwen3-0.6B decoder layer, one
decode step at context 512 (hidden 1024, 16 q / 8 kv heads, head_dim 128,
intermediate 3072, Q4 random-init weights, fp16 KV cache pre-filled with
N(0,1) for 512 positions).  A "step" is one such layer step.  Weights are
rotated over ``--copies`` distinct layers (40 x 8.36 MB > the 256 MB
Infinity Cache), so the headline is the cache-flushed rate; the
cache-resident rate (one layer repeated) is reported beside it.

``value`` = algorithmic HBM bytes per step (10,461,184 B: Q4 weights +
scales, K/V read of 512 positions, new K/V row, hidden in/out) / step time.
Steps run as HIP-graph replays of ``--copies`` captured layer steps.

``roofline`` is that of the dominant kernel of the layer step (the stage
with the largest time, HIP events around graph replays of that stage alone):
its algorithmic bytes per launch (model.stage_bytes_layer) over its average
launch time; every stage's rate is listed beside it.

Also reported (same run, under "extras"): the 3072x1024 Q4 GEMV
GB/s flushed and resident; the LM head alone; full 28-layer greedy decode
tok/s (64-token prompt, 256 generated); prefill of one 2048-token
sequence (tok/s and TFLOP/s against the dense fp16 MFMA peak);
batched decode of 64 sequences over 4096 cached positions (tok/s
and GB/s of K/V + weights); the fixed-point (RTL-exact) layer and token;
bf16 -> Q4 conversion of every matrix of the model (GB/s of bf16 read plus
codes and scales written); a measured HBM rate (torch's device copy of
512 MiB windows, read + written bytes) that ``roofline`` also quotes its
rate against, beside the 8 TB/s vendor figure; and the oracle's CPU rates on
the host cores (``cpu_baseline``: the layer step on all cores;
``extras.cpu_legs``: the 3072x1024 GEMV as an fp32 matvec and as the int64 Q26
restatement, the layer step on one thread, the 28-layer decode per token, the oracle's
quantizer on a 3072x1024 fp32 matrix).
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

METRIC = "Q4 GEMV HBM GB/s (% peak) + batch-1 decode tok/s, Qwen3-0.6B-Q4"
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16
STAGE_KERNELS = {"qkv": "input RMSNorm + q|k|v Q4 GEMV", "attention": "q/k norm + RoPE + KV append + split-K GQA attention",
                 "o_proj": "o_proj Q4 GEMV + residual", "gate_up": "post-norm + gate/up Q4 GEMV + SwiGLU",
                 "down": "down Q4 GEMV + residual"}
HBM_PEAK_GBPS = 8000.0
PREFILL_TOKENS = 2048              # prefill of one 2048-token sequence
BATCH_SEQS, BATCH_CTX = 64, 4096  # batched decode: 64 sequences over 4096 cached positions


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--ctx", type=int, default=512)
    ap.add_argument("--copies", type=int, default=40)
    ap.add_argument("--precision", type=int, default=2, choices=(1, 2))
    ap.add_argument("--no-extras", action="store_true", help="skip every leg beside the layer step")
    ap.add_argument("--extras", default="gemv,decode,prefill,batch,fx,q4c",
                    help="comma list of the legs to run beside the layer step: gemv (3072x1024 GEMV), "
                         "decode (28-layer decode + LM head), prefill, batch (batched decode), "
                         "fx fixed-point (RTL-exact) layer and token, "
                         "q4c float -> Q4 conversion of the whole model")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--decode-gen", type=int, default=256)
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


def main():
    args = parse()
    if args.gpus != 1:
        sys.exit(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path")
    import numpy as np
    import torch

    from llm_accelerator_amd import _lib
    from llm_accelerator_amd import model as M
    from llm_accelerator_amd._lib import check

    lib = _lib.load()
    check(lib.q4d_set_activation_precision(args.precision), "precision")
    dev = torch.device("cuda:0")
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    # ------------------------------------------------------------ layer step
    ctx, copies = args.ctx, args.copies
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
    log(f"[bench] layer-step setup {time.time() - t:.1f}s: {copies} layers, ctx {ctx}")

    def layer_step(i):
        check(lib.q4d_decoder_layer(ctypes.byref(desc), i % copies, h_in.data_ptr(), h_out.data_ptr(),
                                    ctypes.byref(kvd), pos.data_ptr(), ws.ptr, ws.nbytes, st()),
              "q4d_decoder_layer")

    for i in range(args.warmup):
        layer_step(i)
    torch.cuda.synchronize()
    g_flush = graph_of(layer_step, copies, torch)
    g_flush.replay()
    torch.cuda.synchronize()
    full, rest = divmod(args.steps, copies)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(full):
        g_flush.replay()
    for i in range(rest):
        layer_step(i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    step_bytes = M.algorithmic_bytes_layer(M.Qwen3Config(), ctx)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"[bench] layer step flushed: {ms_per_step * 1e3:.2f} us/step, {value:.1f} GB/s")

    g_res = graph_of(lambda i: layer_step(0), copies, torch)
    res_ms = time_graph(g_res, max(1, args.steps // copies), torch) / copies
    resident = step_bytes / (res_ms * 1e-3) / 1e9
    log(f"[bench] layer step resident: {res_ms * 1e3:.2f} us/step, {resident:.1f} GB/s")

    # per-stage durations (graphs of `copies` launches of one stage, HIP events)
    stage_names = ["qkv", "attention", "o_proj", "gate_up", "down"]
    stage_us = {}
    for sidx, sname in enumerate(stage_names):
        def stage(i, sidx=sidx):
            check(lib.q4d_layer_stage(ctypes.byref(desc), i % copies, sidx, h_in.data_ptr(), h_out.data_ptr(),
                                      ctypes.byref(kvd), pos.data_ptr(), ws.ptr, ws.nbytes, st()),
                  "q4d_layer_stage")
        g = graph_of(stage, copies, torch)
        g.replay()
        stage_us[sname] = time_graph(g, max(1, args.steps // copies), torch) / copies * 1e3
    log(f"[bench] stage us (flushed): {json.dumps({k: round(v, 2) for k, v in stage_us.items()})}")
    # roofline of the dominant kernel (the slowest stage of the layer step):
    # algorithmic bytes per launch in the dtypes each kernel reads and writes
    stage_bytes = M.stage_bytes_layer(M.Qwen3Config(), ctx)
    stage_rate = {k: stage_bytes[k] / (stage_us[k] * 1e-6) / 1e9 for k in stage_names}
    dom = max(stage_names, key=lambda k: stage_us[k])
    # HBM bytes per launch of that kernel, measured with rocprofv3 FETCH_SIZE /
    # WRITE_SIZE (copy-calibrated) and committed under profiles/
    traffic, traffic_src = None, None
    tfile = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                         "decode_layer_ctx512_hbm_traffic.json")
    if os.path.exists(tfile) and args.precision == 2:
        with open(tfile) as f:
            tj = json.load(f)
        ent = tj["stages"].get(dom) if "stages" in tj else None
        if ent:
            traffic, traffic_src = ent["total_bytes"], tj["source"]
    roofline = {"bound": "hbm", "kernel": f"{dom} stage ({STAGE_KERNELS[dom]})",
                "achieved": round(stage_rate[dom], 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(stage_rate[dom] / HBM_PEAK_GBPS, 4), "traffic": traffic, "traffic_source": traffic_src,
                "bytes_per_launch": stage_bytes[dom], "avg_launch_us": round(stage_us[dom], 3),
                "per_stage_GBps": {k: round(v, 1) for k, v in stage_rate.items()}}

    extras = {"layer_resident_GBps": round(resident, 1), "layer_resident_us_per_step": round(res_ms * 1e3, 3),
              "layer_flushed_us_per_step": round(ms_per_step * 1e3, 3), "stage_us_flushed": stage_us}
    del model, kv, ws, g_flush, g_res
    torch.cuda.empty_cache()

    legs = set() if args.no_extras else {x.strip() for x in args.extras.split(",") if x.strip()}
    known = {"gemv", "decode", "prefill", "batch", "fx", "q4c"}
    if legs - known:
        sys.exit(f"unknown legs {sorted(legs - known)}")
    if "gemv" in legs:
        # -------------------------------------------------------- 3072x1024 GEMV
        from llm_accelerator_amd.model import Q4Tensor, gemv_bytes, random_q4
        rng = np.random.default_rng(0)
        packed, scale = random_q4(rng, 3072, 1024)
        ncop = 200
        P = torch.from_numpy(packed).to(dev).unsqueeze(0).repeat(ncop, 1, 1).contiguous()
        S = torch.from_numpy(scale).to(dev).unsqueeze(0).repeat(ncop, 1, 1).contiguous()
        mats = [Q4Tensor(P[i], S[i]).descriptor() for i in range(ncop)]
        x = torch.randn(1, 1024, generator=gen, device=dev).half()
        y = torch.empty(1, 3072, device=dev, dtype=torch.float16)

        def gemv(i, fixed=False):
            m = mats[0 if fixed else i]
            check(lib.q4d_linear(ctypes.byref(m), x.data_ptr(), 0, y.data_ptr(), 0, 1, st()), "q4d_linear")
        gb = gemv_bytes(3072, 1024)
        g1 = graph_of(gemv, ncop, torch)
        us_fl = time_graph(g1, 20, torch) / ncop * 1e3
        g2 = graph_of(lambda i: gemv(i, True), ncop, torch)
        us_res = time_graph(g2, 20, torch) / ncop * 1e3
        extras["gemv_3072x1024"] = {"shape": "3072x1024 q4, fp16 x/y", "bytes": gb,
                             "flushed_us": round(us_fl, 3), "flushed_GBps": round(gb / us_fl / 1e3, 1),
                             "resident_us": round(us_res, 3), "resident_GBps": round(gb / us_res / 1e3, 1)}
        log(f"[bench] GEMV 3072x1024: {json.dumps(extras['gemv_3072x1024'])}")
        del P, S, g1, g2
        torch.cuda.empty_cache()

    if legs & {"decode", "prefill", "batch", "fx"}:
        fcfg = M.Qwen3Config()
        t = time.time()
        fhost = M.random_host_weights(fcfg, seed=0)
        fmodel = M.build_model(fcfg, fhost, max_ctx=max(64 + args.decode_gen + 16, BATCH_CTX + 1), device=dev)
        norm_keys = ("input_layernorm", "post_attention_layernorm", "q_norm", "k_norm")
        fnorms = {"layers": [{k: L[k] for k in norm_keys} for L in fhost["layers"]], "norm": fhost["norm"]}
        del fhost
        log(f"[bench] 28-layer model setup {time.time() - t:.1f}s")
    if "decode" in legs:
        # -------------------------------------------------------- 28-layer decode tok/s
        from llm_accelerator_amd.decode import GreedyDecoder
        prompt = np.random.default_rng(1).integers(0, fcfg.vocab_size, 64).tolist()
        dec = GreedyDecoder(fmodel, steps_per_graph=16, use_graph=True)
        dec.prefill(prompt)
        dec.generate(16)  # captures and warms the graph
        torch.cuda.synchronize()
        dec.prefill(prompt)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        dec.prefill(prompt)
        torch.cuda.synchronize()
        t_pre = time.perf_counter() - t0
        t0 = time.perf_counter()
        dec.generate(args.decode_gen - 1)
        torch.cuda.synchronize()
        t_gen = time.perf_counter() - t0
        toks, _ = dec.history()
        # LM head alone: final RMSNorm + 151936x1024 Q4 GEMV + argmax
        lm_desc = fmodel.descriptor()
        hid = torch.randn(1, 1024, generator=gen, device=dev)
        lm_tok = torch.zeros(1, dtype=torch.int32, device=dev)
        lm_score = torch.zeros(1, dtype=torch.float32, device=dev)
        lws = M.Workspace(fmodel, 1)

        def lm_head(i):
            check(lib.q4d_lm_head_argmax(ctypes.byref(lm_desc), hid.data_ptr(), lm_tok.data_ptr(),
                                         lm_score.data_ptr(), None, lws.ptr, lws.nbytes, st()), "lm_head")
        g_lm = graph_of(lm_head, 10, torch)
        g_lm.replay()
        lm_us = time_graph(g_lm, 10, torch) / 10 * 1e3
        lm_bytes = wb_lm = fmodel.lm_head.weight.nbytes + 4 * 1024
        extras["lm_head"] = {"us": round(lm_us, 2), "bytes": wb_lm, "GBps": round(lm_bytes / lm_us / 1e3, 1)}
        log(f"[bench] LM head: {json.dumps(extras['lm_head'])}")
        wb = fmodel.weight_bytes()
        avg_ctx = 64 + args.decode_gen / 2
        tok_bytes = wb["total"] + 2 * 2 * 1024 * avg_ctx * 28
        tok_s = (args.decode_gen - 1) / t_gen
        extras["decode_28_layers"] = {"prompt": 64, "generated": len(toks), "tok_s": round(tok_s, 1),
                               "us_per_token": round(1e6 / tok_s, 2),
                               "serial_prefill_tok_s": round(64 / t_pre, 1),
                               "GBps_equiv": round(tok_bytes * tok_s / 1e9, 1),
                               "hbm_frac": round(tok_bytes * tok_s / 1e9 / HBM_PEAK_GBPS, 4),
                               "status": dec.status()}
        log(f"[bench] 28-layer decode: {json.dumps(extras['decode_28_layers'])}")
        del dec, lws
        torch.cuda.empty_cache()

    if "prefill" in legs:
        # -------------------------------------------------------- prefill of 2048 tokens
        from llm_accelerator_amd.decode import Prefill
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
        extras["prefill_2048"] = {"tokens": T, "ms": round(pms, 3), "tok_s": round(T / pms * 1e3, 1),
                                "TFLOPs": round(pflops / pms / 1e9, 1), "flops": pflops,
                                "mfma_frac": round(pflops / pms / 1e9 / MFMA_PEAK_TFLOPS, 4)}
        log(f"[bench] prefill 2048: {json.dumps(extras['prefill_2048'])}")
        del pkv, pf
        torch.cuda.empty_cache()

    if "batch" in legs:
        # -------------------------------------------------------- batched decode 64 x 4096
        from llm_accelerator_amd.decode import BatchedDecoder
        B = BATCH_SEQS
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
        extras["batched_decode_64x4096"] = {"batch": B, "ctx": BATCH_CTX, "ms_per_step": round(bms, 3),
                                       "tok_s": round(B / bms * 1e3, 1), "bytes_per_step": bbytes,
                                       "GBps": round(bbytes / bms / 1e6, 1),
                                       "hbm_frac": round(bbytes / bms / 1e6 / HBM_PEAK_GBPS, 4),
                                       "status": bd.status()}
        log(f"[bench] batched decode 64x4096: {json.dumps(extras['batched_decode_64x4096'])}")
        del bkv, bd
    if "fx" in legs:
        # -------------------------------------------------------- fixed-point (RTL-exact) decode
        from llm_accelerator_amd.fixed import FixedQ4Model
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
        extras["fx_fixed_point"] = {
            "layer_us": round(fx_us, 3), "layer_bytes": fx_bytes, "layer_GBps": round(fx_bytes / fx_us / 1e3, 1),
            "token_ms": round(tok_ms, 4), "tok_s": round(1e3 / tok_ms, 1), "positions": [64, int(fpos.item())],
            "status": counts["status"]}
        log(f"[bench] fixed-point decode: {json.dumps(extras['fx_fixed_point'])}")
        del fxm, fkv, g_fx, g_tok
    if legs & {"decode", "prefill", "batch", "fx"}:
        del fmodel
        torch.cuda.empty_cache()
    if "q4c" in legs:
        # -------------------------------------------------------- float -> Q4 conversion of the whole model
        qcfg = M.Qwen3Config()
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
        for i in range(len(shapes)):
            quant(i)
        torch.cuda.synchronize()
        # HIP graphs: one of the 197 conversions, one of the table alone
        g_all = graph_of(quant, len(shapes), torch)
        g_tab = graph_of(lambda i: quant(len(shapes) - 1), 1, torch)
        g_all.replay()
        g_tab.replay()
        all_ms = time_graph(g_all, 10, torch)
        emb_us = time_graph(g_tab, 20, torch) * 1e3
        params = sum(r * c for r, c in shapes)
        qbytes = params * 2 + params // 2 + params // 64 * 2   # bf16 in, codes + Q2.14 scales out
        er, ec = shapes[-1]
        ebytes = er * ec * 2 + er * ec // 2 + er * ec // 64 * 2
        extras["q4c_quantize"] = {
            "workload": "bf16 -> Q4 of every Qwen3-0.6B projection and the tied table (197 matrices)",
            "params": params, "bytes": qbytes, "ms": round(all_ms, 4), "GBps": round(qbytes / all_ms / 1e6, 1),
            "hbm_frac": round(qbytes / all_ms / 1e6 / HBM_PEAK_GBPS, 4), "table_us": round(emb_us, 2),
            "table_GBps": round(ebytes / emb_us / 1e3, 1), "status": qstatus.tolist()}
        log(f"[bench] Q4 conversion: {json.dumps(extras['q4c_quantize'])}")
        del mats, outs, g_all, g_tab
        torch.cuda.empty_cache()

    if legs:
        # measured HBM ceiling beside the 8 TB/s vendor figure: torch's device
        # copy of 512 MiB windows rotating over 2 GiB (past the 256 MB cache),
        # read + written bytes over the time
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
        extras["hbm_copy"] = {"bytes_moved": 2 * w, "us": round(cms * 1e3, 1),
                              "GBps": round(2 * w / (cms * 1e-3) / 1e9, 1)}
        log(f"[bench] measured copy: {json.dumps(extras['hbm_copy'])}")
        del buf
        torch.cuda.empty_cache()

    if args.copy_calibration:
        # a plain copy of known size: its FETCH_SIZE / WRITE_SIZE per dispatch
        # converts the counters of the GEMV dispatches to bytes
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        extras["copy_calibration_bytes"] = 256 << 20
        del src, dst

    cpu = None
    if not args.no_cpu and legs:
        cpu = cpu_baseline(args.cpu_seconds, ctx, step_bytes)
        log(f"[bench] CPU baseline: {json.dumps(cpu)}")
        extras["cpu_legs"] = cpu_extra_legs(ctx, step_bytes)
        log(f"[bench] CPU legs: {json.dumps(extras['cpu_legs'])}")

    if "hbm_copy" in extras:
        roofline["measured_copy_GBps"] = extras["hbm_copy"]["GBps"]
        roofline["frac_of_measured_copy"] = round(roofline["achieved"] / extras["hbm_copy"]["GBps"], 4)
    line = {"metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "q4xf32",
            "data": "synthetic (seeded random-init Q4 weights, N(0,1) fp16 KV, N(0,1) hidden)",
            "config": {"workload": "one Qwen3-0.6B decoder layer, one decode step at ctx 512, "
                                   f"weights rotated over {copies} distinct layers (cache-flushed)",
                       "hidden": 1024, "q_heads": 16, "kv_heads": 8, "head_dim": 128, "intermediate": 3072,
                       "ctx": ctx, "batch": 1, "bytes_per_step": step_bytes, "activation_precision": args.precision},
            "roofline": roofline, "cpu_baseline": cpu, "extras": extras}
    print(json.dumps(line), flush=True)


def cpu_baseline(seconds, ctx, step_bytes):
    """The oracle's fp32 layer step (the reference's CPU path, common.py:231-298)
    on a bounded sample of the same workload, timed on the host cores."""
    import numpy as np

    import oracle as o
    from llm_accelerator_amd import model as M
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:  # threadpoolctl missing: numpy default
        threads = os.cpu_count() or 1
    cfg = M.Qwen3Config(num_hidden_layers=1, vocab_size=2048)
    host = M.random_host_weights(cfg, seed=0, num_layers=1)
    om = o.OracleModel.from_q4(o.OracleConfig(num_hidden_layers=1, vocab_size=2048), host["layers"],
                               *host["embed_tokens"], host["norm"])
    rng = np.random.default_rng(2)
    k = rng.normal(size=(1, 8, ctx, 128)).astype(np.float32)
    v = rng.normal(size=(1, 8, ctx, 128)).astype(np.float32)
    h = rng.normal(size=(1, 1, 1024)).astype(np.float32)
    pos = np.array([[ctx]])
    o.manual_decoder_layer_cached(h, om.layers[0], om.config, om.inv_freq, pos, k, v)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        o.manual_decoder_layer_cached(h, om.layers[0], om.config, om.inv_freq, pos, k, v)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return {"value": round(step_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{n} fp32 numpy layer steps at ctx {ctx} (oracle restatement of common.py:231-298), "
                      f"{dt * 1e3:.2f} ms/step; os.cpu_count()={os.cpu_count()}, "
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
    """The other CPU baselines: the 3072x1024 GEMV (fp32 matvec on pre-dequantised
    weights as manual_linear_from_weight holds them, common.py:137-145, and the
    int64 Q26 restatement of compute_q4_gemv_q26, 28_export_mlp_gate_up_vectors.py:124-133),
    the layer step on one thread, and the 28-layer decode (run_manual_one_token,
    10_validate_full_run_one_token.py:17-56, 8 serial steps of the 28-layer
    model, per token).  Medians of >= 10 timed runs after a warm-up."""
    import numpy as np

    import oracle as o
    from llm_accelerator_amd import model as M
    try:
        from threadpoolctl import threadpool_limits
    except Exception:  # threadpoolctl missing: no one-thread leg
        threadpool_limits = None
    out = {"cores": os.cpu_count(), "affinity": len(os.sched_getaffinity(0))}
    rng = np.random.default_rng(0)
    packed, scale = M.random_q4(rng, 3072, 1024)
    W = o.dequantize_q4(packed, scale, np.float32)
    q = o.unpack_signed_int4(packed, 1024)
    x = rng.normal(size=1024).astype(np.float32)
    xi = rng.integers(-(1 << 20), 1 << 20, size=1024)
    gb = M.gemv_bytes(3072, 1024)
    t, n = _median_time(lambda: W @ x, 10, 2.0)
    out["gemv_fp32"] = {"us": round(t * 1e6, 1), "GBps": round(gb / t / 1e9, 2), "runs": n}
    t, n = _median_time(lambda: o.q4_gemv_q26(xi, q, scale), 10, 2.0)
    out["gemv_int64_q26"] = {"us": round(t * 1e6, 1), "GBps": round(gb / t / 1e9, 3), "runs": n}
    if threadpool_limits is not None:
        cfg = M.Qwen3Config(num_hidden_layers=1, vocab_size=2048)
        host = M.random_host_weights(cfg, seed=0, num_layers=1)
        om = o.OracleModel.from_q4(o.OracleConfig(num_hidden_layers=1, vocab_size=2048), host["layers"],
                                   *host["embed_tokens"], host["norm"])
        k = rng.normal(size=(1, 8, ctx, 128)).astype(np.float32)
        v = rng.normal(size=(1, 8, ctx, 128)).astype(np.float32)
        h = rng.normal(size=(1, 1, 1024)).astype(np.float32)
        pos = np.array([[ctx]])
        with threadpool_limits(limits=1):
            t, n = _median_time(lambda: o.manual_decoder_layer_cached(h, om.layers[0], om.config, om.inv_freq,
                                                                      pos, k, v), 10, 3.0)
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
    wq = (rng.standard_normal((3072, 1024)) * 0.03).astype(np.float32)
    t, n = _median_time(lambda: o.quantize_weight_q4(wq), 5, 2.0)
    qb = 3072 * 1024 * 4 + 3072 * 512 + 3072 * 16 * 2
    out["q4c_oracle"] = {"shape": "3072x1024 fp32 -> Q4", "ms": round(t * 1e3, 2), "GBps": round(qb / t / 1e9, 3),
                         "runs": n}
    return out


if __name__ == "__main__":
    main()
