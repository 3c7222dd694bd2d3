#!/usr/bin/env python3
"""Benchmark of the LFM3 continuous-batching step on one MI355X (gfx950).

Workload (the metric's decode half): one decode round of eight ragged
sessions through the full 24-layer Q8_0 model at the reference checkpoint's
dims (hidden 2048, FFN 7680, 16 query / 4 KV heads x 128, vocab 128000;
13 convolution, 5 sliding-256 and 6 global attention layers), session
contexts uniform in [128, 8192], random-init weights and synthesized session
state (conv history N(0, 1), F16 K/V rings N(0, 1)). Each round's greedy ids
are the next round's tokens, as in a temperature-0 serving loop
(Session::ForwardBatch, engine.cpp:1160-1216, then the sampler's pick).

Printed as one JSON line:
  value      decode tokens/s of the whole round (8 tokens per round);
  roofline   the Q8_0 skinny GEMV at its own shape (W 8192 x 2048 Q8_0, 8 FP32
             rows) against the 8 TB/s HBM peak: back-to-back launches replayed
             from a HIP graph, timed with HIP events on the stream they run on,
             rotating 32 weight copies so that no launch finds its matrix in
             the 256 MB MALL;
  round      the whole round's algorithmic HBM bytes and fraction of peak;
  cpu_baseline  the CPU oracle (a scalar FP32 restatement of reference.cpp)
             running the same round on the host: one thread per session.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import threading
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "lfm3-gufo-extension_amd", "python"))

import numpy as np  # noqa: E402

import lfm3amd as L  # noqa: E402

HBM_PEAK_GBS = 8000.0
SESSIONS = 8
CTX_LO, CTX_HI = 128, 8192


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q8_bytes(rows: int, cols: int) -> int:
    return rows * (cols // 32) * 34


def weight_bytes(d: L.Dims) -> int:
    """Q8_0 weight bytes one decode round streams (the tied vocabulary head
    included, the 8 embedding rows not)."""
    H, F, D = d.hidden, d.intermediate, d.head_dim
    total = q8_bytes(d.vocab, H)
    for i in range(d.n_layers):
        total += 2 * q8_bytes(F, H) + q8_bytes(H, F)
        if d.layer_type(i) == L.LAYER_CONV:
            total += q8_bytes(3 * H, H) + q8_bytes(H, H)
        else:
            total += q8_bytes(d.heads * D, H) + 2 * q8_bytes(d.kv_heads * D, H)
            total += q8_bytes(d.heads, H) + q8_bytes(H, d.heads * D)
    return total


def round_bytes(d: L.Dims, positions) -> int:
    """Algorithmic HBM bytes of one round at the given positions: weights,
    K/V rows read (keys [first, p]) and written, conv histories read and
    written."""
    kv_row = 2 * d.kv_heads * d.head_dim * 2  # K + V, F16
    total = weight_bytes(d)
    for p in positions:
        for i in range(d.n_layers):
            t = d.layer_type(i)
            if t == L.LAYER_CONV:
                total += 2 * d.hidden * (d.conv_width - 1) * 4
            else:
                keys = p + 1 if t == L.LAYER_FULL else min(p + 1, d.window)
                total += keys * kv_row + kv_row
    return total


def gemv_roofline(batch: int, copies: int, passes: int):
    """Q8_0 GEMV W 8192 x 2048 on `batch` FP32 rows over `copies` rotated
    weight buffers. One pass launches every copy once; the passes are
    captured in a HIP graph and replayed, bracketed by HIP events on the
    stream the kernels run on, so host launch overhead is not timed."""
    import ctypes as C
    M, K = 8192, 2048
    src = L.q8(L.SEED, "gemv.W", M, K)
    cb, sb = C.c_size_t(), C.c_size_t()
    L.lib().lfm3_q8_tiled_bytes(M, K, C.byref(cb), C.byref(sb))
    codes = np.zeros(cb.value, np.uint8)
    scales = np.zeros(sb.value, np.uint8)
    L.check(L.lib().lfm3_q8_pack_host(L.ptr(src), M, K, L.ptr(codes), L.ptr(scales), 0, 1))
    mats = [(L.DeviceBuffer.of(codes), L.DeviceBuffer.of(scales)) for _ in range(copies)]
    x = L.DeviceBuffer.of(L.normal(L.SEED, f"gemv.X{batch}", batch * K))
    y = L.DeviceBuffer(batch * M * 4)
    stream = L.Stream()
    fn = L.lib().lfm3_q8_gemv

    def one_pass():
        for c, s in mats:
            L.check(fn(c.addr, s.addr, M, K, x.addr, K, y.addr, M, batch, None, 0,
                       stream.handle))

    graph = L.Graph(stream, one_pass)
    graph.launch()  # warm-up
    stream.synchronize()
    a, b = L.Event(), L.Event()
    a.record(stream.handle)
    for _ in range(passes):
        graph.launch()
    b.record(stream.handle)
    b.synchronize()
    us = a.elapsed_ms(b) * 1000.0 / (passes * copies)
    graph.close()
    a.close()
    b.close()
    stream.close()
    nbytes = q8_bytes(M, K) + batch * K * 4 + batch * M * 4
    return {"batch": batch, "bytes": nbytes, "us": us}


def cpu_baseline(dims, weights, ctx, tokens, seed):
    """One decode round of the eight sessions on the CPU oracle, one thread
    per session, from the same synthesized state as the GPU sessions.
    Returns (result dict, per-session greedy ids, per-session top-2 margin)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    om = O.Model(dims, weights)
    sessions = []
    for sid, c in enumerate(ctx):
        position = int(c) - 1
        s = om.session(int(c) + 256, f16=True)
        for l in range(dims.n_layers):
            if dims.layer_type(l) == L.LAYER_CONV:
                s.conv(l)[:] = L.synth_conv_state(seed, sid, l, dims)
            else:
                rows = L.live_slots(position, s.capacity(l))
                n = rows * dims.kv_heads * dims.head_dim
                for view, tag in ((s.k, "k"), (s.v, "v")):
                    view(l)[:n] = O.half_to_float(L.synth_kv_state(seed, sid, l, tag, rows, dims))
        s.set_position(position)
        sessions.append(s)
    out = [None] * len(sessions)

    def work(i):
        out[i] = sessions[i].step(int(tokens[i]))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(sessions))]
    t0 = time.perf_counter()
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    wall = time.perf_counter() - t0
    ids = [O.argmax(o) for o in out]
    margins = [float(np.diff(np.sort(o)[-2:])[0]) for o in out]
    for s in sessions:
        s.close()
    om.close()
    res = {"value": round(len(sessions) / wall, 4), "unit": "tok/s", "cores": len(sessions),
           "kind": "port",
           "sample": (f"one decode round of {len(sessions)} sessions (one token each) through "
                      f"the full model at the same contexts and state, one thread per session; "
                      f"{wall:.1f} s wall")}
    return res, ids, margins


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--gemv-copies", type=int, default=32)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported (the decode "
              f"round is data-parallel over sessions and runs on one GPU here)", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 1:
        print("--steps and --warmup must be at least 1", file=sys.stderr)
        sys.exit(2)
    L.lib()
    if L.gpu_count() < 1:
        print("bench.py needs a GPU (hipGetDeviceCount reports none)", file=sys.stderr)
        sys.exit(1)

    seed = L.SEED
    dims = L.Dims(context=CTX_HI + 1024)
    t0 = time.perf_counter()
    weights = L.synth_weights(dims, seed=seed)
    log(f"synthesized weights in {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    model = L.Model(weights)
    log(f"loaded model in {time.perf_counter() - t0:.1f} s")
    ctx = L.uniform_u32(seed, "bench.ctx", SESSIONS, CTX_LO, CTX_HI)
    tokens0 = L.uniform_u32(seed, "bench.tokens", SESSIONS, 0, dims.vocab - 1)
    sessions = []
    for sid, c in enumerate(ctx):
        s = model.session(int(c) + args.warmup + args.steps + 8)
        L.inject_synth_state(s, dims, seed, sid, int(c) - 1)
        sessions.append(s)
    log(f"sessions at contexts {ctx.tolist()}")

    # Warm-up rounds; the first starts from the synthesized state.
    first_ids = None
    toks = tokens0
    for w in range(args.warmup):
        toks = model.forward_batch_greedy(sessions, toks)
        if w == 0:
            first_ids = toks.copy()
    L.synchronize()
    positions = [[s.position + k for s in sessions] for k in range(args.steps)]
    stream = model.stream()
    ev0, ev1 = L.Event(), L.Event()
    ev0.record(stream)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        toks = model.forward_batch_greedy(sessions, toks)
    L.synchronize()
    wall = time.perf_counter() - t0
    ev1.record(stream)
    ev1.synchronize()
    ms_per_step = wall * 1000.0 / args.steps
    value = SESSIONS / (ms_per_step / 1000.0)
    rbytes = statistics.mean(round_bytes(dims, p) for p in positions)
    round_gbs = rbytes / (ms_per_step / 1000.0) / 1e9
    log(f"round {ms_per_step:.3f} ms, {value:.1f} tok/s, {round_gbs:.0f} GB/s")

    # The GEMV kernel alone (the round's dominant kernel), B = 8 and a sweep.
    sweep = [gemv_roofline(b, args.gemv_copies, 8) for b in (1, 2, 4, 8)]
    g8 = sweep[-1]
    achieved = g8["bytes"] / (g8["us"] * 1e-6) / 1e9
    for g in sweep:
        log(f"gemv B={g['batch']}: {g['us']:.2f} us/launch, "
            f"{g['bytes'] / (g['us'] * 1e-6) / 1e9:.0f} GB/s")

    result = {
        "metric": "decode tok/s @8 sessions (HBM GB/s % peak)",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 x f32",
        "data": "synthetic (random-init Q8_0 weights, synthesized session state)",
        "config": {
            "workload": ("LFM3 decode round, 8 ragged sessions: 24 layers (13 conv7, 5 sliding-256, "
                         "6 global), hidden 2048, FFN 7680, 16q/4kv heads x 128, vocab 128000, "
                         "Q8_0 weights; contexts uniform in [128, 8192]; greedy ids fed back"),
            "sessions": SESSIONS,
            "contexts": [int(c) for c in ctx],
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "Q8_0 skinny GEMV, W 8192 x 2048, 8 FP32 rows",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "bytes_per_launch": g8["bytes"],
            "us_per_launch": round(g8["us"], 3),
        },
        "round": {
            "bytes": int(rbytes),
            "achieved_GBps": round(round_gbs, 1),
            "frac_of_peak": round(round_gbs / HBM_PEAK_GBS, 4),
            "gpu_ms_per_step": round(ev0.elapsed_ms(ev1) / args.steps, 4),
        },
        "gemv_sweep": [{"batch": g["batch"], "us": round(g["us"], 3),
                        "GBps": round(g["bytes"] / (g["us"] * 1e-6) / 1e9, 1)}
                       for g in sweep],
    }
    if not args.no_cpu:
        log("CPU oracle round (one thread per session) ...")
        cpu, ids, margins = cpu_baseline(dims, weights, ctx, tokens0, seed)
        result["cpu_baseline"] = cpu
        result["greedy_ids_match_oracle"] = [int(a) == int(b) for a, b in zip(first_ids, ids)]
        result["oracle_top2_margin_min"] = round(min(margins), 6)
        log(cpu["sample"])
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
