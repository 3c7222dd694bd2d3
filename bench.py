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
             running the same round on the host: one thread per session;
  prefill    the metric's prefill half: one 512-token prompt pass
             (Session::Forward) at depth 24576 of a synthesized session, its
             algorithmic FLOPs (projections 2 n W plus attention 4 D h keys,
             over what runs after the reference's trailing-row pruning) and
             fraction of the 2.5 PFLOP/s dense FP16 MFMA peak, with the MFMA
             roofline of its dominant kernel (the gate/up SwiGLU GEMM,
             15360 x 2048 Q8_0 on 512 FP16 rows);
  mixed_round  one scheduler round at depth: 7 decode sessions at contexts
             uniform in [16384, 32768] plus the 512-token pass.
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
MFMA_PEAK_TFLOPS = 2500.0  # dense FP16 MFMA, MI355X
SESSIONS = 8
CTX_LO, CTX_HI = 128, 8192
PASS_ROWS, PASS_DEPTH = 512, 24576
MIXED_DECODE, MIXED_LO, MIXED_HI = 7, 16384, 32768

# HBM bytes per launch of the two roofline kernels at the shapes timed here,
# counted by `rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` over
# `bench.py --roofline-only` and scaled by what each counter reads for a
# plain 256 MiB device-to-device copy in the same program (FETCH_SIZE x 2.0,
# WRITE_SIZE x 1.0). Re-measure after a change to either kernel.
GEMV_TRAFFIC = {"read": 18_477_766, "write": 262_144}
# The same for the round's dominant launch, the residual norm (2 K parts)
# fused with the SwiGLU operand-image GEMV (2 x 7680 x 2048, 8 rows):
# 1.024 x its algorithmic bytes.
SWIGLU_TRAFFIC = {"read": 34_396_183, "write": 444_621}
# The prompt pass's gate/up SwiGLU GEMM as the pass launches it, with the
# trailing blocks that write the FP16 hidden rows: 1.40 x its algorithmic
# bytes (the trailing blocks re-read the 15.7 MB of FP32 outputs; the GEMM
# alone moves 1.23 x, as each XCD fetches the activation block).
GEMM_TRAFFIC = {"read": 103_034_560, "write": 23_731_712}


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def q8_bytes(rows: int, cols: int) -> int:
    return rows * (cols // 32) * 34


def bf16_bytes(rows: int, cols: int) -> int:
    return rows * cols * 2


def weight_bytes(d: L.Dims, bf16: bool = False) -> int:
    """Weight bytes one decode round streams (Q8_0, or BF16 with bf16; the
    tied vocabulary head included, the 8 embedding rows not)."""
    H, F, D = d.hidden, d.intermediate, d.head_dim
    mb = bf16_bytes if bf16 else q8_bytes
    total = mb(d.vocab, H)
    for i in range(d.n_layers):
        total += 2 * mb(F, H) + mb(H, F)
        if d.layer_type(i) == L.LAYER_CONV:
            total += mb(3 * H, H) + mb(H, H)
        else:
            total += mb(d.heads * D, H) + 2 * mb(d.kv_heads * D, H)
            total += mb(d.heads, H) + mb(H, d.heads * D)
    return total


def round_bytes(d: L.Dims, positions, bf16: bool = False) -> int:
    """Algorithmic HBM bytes of one round at the given positions: weights,
    K/V rows read (keys [first, p]) and written, conv histories read and
    written."""
    kv_row = 2 * d.kv_heads * d.head_dim * 2  # K + V, F16
    total = weight_bytes(d, bf16)
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


def bf16_gemv_roofline(batch: int, copies: int, passes: int):
    """The exact BF16 GEMV at the single-GEMV shape (W 8192 x 2048 BF16, `batch`
    FP32 rows) over `copies` rotated weight buffers (32 MB each, past the
    MALL), replayed from a HIP graph."""
    M, K = 8192, 2048
    h = L.bf16(L.SEED, "bf16.gemv.W", M, K)
    tiles = np.zeros(L.lib().lfm3_bf16_tiled_bytes(M, K) // 2, np.uint16)
    L.check(L.lib().lfm3_bf16_pack_host(L.ptr(h), M, K, L.ptr(tiles), 0, 1))
    mats = [L.DeviceBuffer.of(tiles) for _ in range(copies)]
    x = L.DeviceBuffer.of(L.normal(L.SEED, f"bf16.gemv.X{batch}", batch * K))
    y = L.DeviceBuffer(batch * M * 4)
    us = time_launches(lambda i, st: L.check(L.lib().lfm3_bf16_gemv(
        mats[i].addr, M, K, x.addr, K, y.addr, M, batch, 1, 0, st)), copies, passes)
    nbytes = bf16_bytes(M, K) + batch * K * 4 + batch * M * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"kernel": "exact BF16 x FP32 GEMV, W 8192 x 2048 BF16", "batch": batch,
            "us": round(us, 3), "bytes": nbytes, "GBps": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def packed_copies(parts, rows_total: int, cols: int, copies: int):
    """`copies` device copies of a tiled Q8_0 matrix packed from
    (gguf blob, rows, tile_offset, tile_stride) sources."""
    import ctypes as C
    cb, sb = C.c_size_t(), C.c_size_t()
    L.lib().lfm3_q8_tiled_bytes(rows_total, cols, C.byref(cb), C.byref(sb))
    codes = np.zeros(cb.value, np.uint8)
    scales = np.zeros(sb.value, np.uint8)
    for blob, rows, off, stride in parts:
        L.check(L.lib().lfm3_q8_pack_host(L.ptr(blob), rows, cols, L.ptr(codes), L.ptr(scales),
                                          off, stride))
    return [(L.DeviceBuffer.of(codes), L.DeviceBuffer.of(scales)) for _ in range(copies)]


def time_launches(launch, copies: int, passes: int, seqs: bool = False) -> float:
    """Microseconds per launch of launch(copy, stream) replayed from a HIP
    graph (one pass launches every copy once), timed with HIP events on the
    stream the kernels run on. With seqs, launch(copy, stream, seq) is a
    fused norm + GEMV launch, whose rows' flags must see a new sequence
    number at every launch: two graphs with disjoint numbers (1..copies and
    copies + 1..2 copies) replay alternately, so no launch finds its own
    number left in the flags by the one before it."""
    stream = L.Stream()
    graphs = []
    for g in range(2 if seqs else 1):
        def one_pass(base=g * copies + 1):
            for i in range(copies):
                if seqs:
                    launch(i, stream.handle, base + i)
                else:
                    launch(i, stream.handle)
        graphs.append(L.Graph(stream, one_pass))
    for graph in graphs:
        graph.launch()
    stream.synchronize()
    a, b = L.Event(), L.Event()
    a.record(stream.handle)
    for p in range(passes):
        graphs[p % len(graphs)].launch()
    b.record(stream.handle)
    b.synchronize()
    us = a.elapsed_ms(b) * 1000.0 / (passes * copies)
    for graph in graphs:
        graph.close()
    a.close()
    b.close()
    stream.close()
    return us


def norm_bytes(d: L.Dims, parts: int) -> int:
    """Algorithmic bytes of the round's residual norm over 8 rows: x read and
    written, the branch's K parts read, the norm and post-norm weights (the
    operand image it hands to the GEMV is not counted, as the GEMV's operand
    rows are counted once, as FP32 rows)."""
    return SESSIONS * d.hidden * 4 * (2 + parts) + 2 * d.hidden * 4


def round_kernels(d: L.Dims, positions=None, passes: int = 6):
    """Each kind of launch of the decode round alone at its round shape (8
    rows; weight and K/V copies rotated past the 256 MB MALL): microseconds,
    the algorithmic HBM bytes it moves and their fraction of 8 TB/s, and
    its launches per round. The round runs each residual norm inside the
    launch of the GEMV that consumes its image (lfm3_q8_gemv_image_norm,
    lfm3_q8_gemv_conv_image_norm), so those launches are timed fused, their
    bytes the GEMV's plus the norm's. The first entry, the fused norm +
    SwiGLU GEMV, is the round's dominant kernel. With `positions` (the rows'
    positions) the fused heads + decode attention of a global and of a
    sliding layer are timed too."""
    H, F, V, B = d.hidden, d.intermediate, d.vocab, SESSIONS
    lib = L.lib()
    seed = L.SEED
    out = []

    def entry(name, us, nbytes, per_round):
        gbs = nbytes / (us * 1e-6) / 1e9
        out.append({"kernel": name, "us": round(us, 3), "bytes": int(nbytes),
                    "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                    "per_round": per_round})

    # An operand image of 8 normed rows (the norm the round runs).
    x = L.DeviceBuffer.of(L.normal(seed, "rk.x", B * H))
    branch = L.DeviceBuffer.of(L.normal(seed, "rk.b", 4 * B * H))
    wts = L.DeviceBuffer.of(L.normal(seed, "rk.w", H, 1, 0.02))
    image = L.DeviceBuffer(lib.lfm3_operand_image_bytes(H))
    exps = L.DeviceBuffer(8 * 4)
    L.check(lib.lfm3_residual_norm_image(branch.addr, 1, B * H, wts.addr, x.addr, wts.addr, None,
                                         image.addr, exps.addr, B, H, d.eps, None))
    # The fused launches' flags and wait-error word.
    flags = L.DeviceBuffer(lib.lfm3_norm_flags_bytes())
    L.hip_check(L.hip().hipMemset(flags.addr, 0, flags.nbytes))
    werr = L.DeviceBuffer(4)
    L.hip_check(L.hip().hipMemset(werr.addr, 0, 4))
    L.synchronize()

    def norm_args(parts, seq):
        return (branch.addr, parts, B * H, wts.addr, x.addr, wts.addr, d.eps, image.addr,
                exps.addr, flags.addr, seq, werr.addr)

    n_conv = sum(1 for i in range(d.n_layers) if d.layer_type(i) == L.LAYER_CONV)
    n_attn = d.n_layers - n_conv
    mixer_parts = lib.lfm3_q8_gemv_parts(H, H)
    ffn_parts = lib.lfm3_q8_gemv_parts(H, F)
    # The FFN norm and SwiGLU (gate/up interleaved) on its operand image.
    g, u = L.q8(seed, "rk.gate", F, H), L.q8(seed, "rk.up", F, H)
    mats = packed_copies([(g, F, 0, 2), (u, F, 1, 2)], 2 * F, H, 12)
    hid = L.DeviceBuffer(B * F * 4)
    us = time_launches(lambda i, s, q: L.check(lib.lfm3_q8_gemv_image_norm(
        *norm_args(mixer_parts, q), mats[i][0].addr, mats[i][1].addr, F, H, 1, B, hid.addr, F,
        s)), len(mats), passes, seqs=True)
    entry(f"residual norm ({mixer_parts} K parts) + SwiGLU GEMV on its image, 2 x 7680 x 2048",
          us, 2 * q8_bytes(F, H) + B * H * 4 + B * F * 4 + norm_bytes(d, mixer_parts),
          d.n_layers)
    # The same GEMV as a launch of its own (its operand image ready).
    us = time_launches(lambda i, s: L.check(lib.lfm3_q8_gemv_swiglu_image(
        mats[i][0].addr, mats[i][1].addr, F, H, image.addr, exps.addr, B, hid.addr, F, s)),
        len(mats), passes)
    entry("(the SwiGLU GEMV alone on a ready image, 2 x 7680 x 2048; not a launch of the round)",
          us, 2 * q8_bytes(F, H) + B * H * 4 + B * F * 4, 0)
    del mats
    # Down projection in K parts from the FP32 hidden rows.
    mats = packed_copies([(L.q8(seed, "rk.down", H, F), H, 0, 1)], H, F, 20)
    parts = lib.lfm3_q8_gemv_parts(H, F)
    y = L.DeviceBuffer(parts * B * H * 4)
    us = time_launches(lambda i, s: L.check(lib.lfm3_q8_gemv_partials(
        mats[i][0].addr, mats[i][1].addr, H, F, hid.addr, F, y.addr, H, B, parts, s)),
        len(mats), passes)
    entry(f"down GEMV in {parts} K parts, 2048 x 7680", us,
          q8_bytes(H, F) + B * F * 4 + parts * B * H * 4, d.n_layers)
    del mats
    # Attention output / convolution output projection (2048 x 2048).
    mats = packed_copies([(L.q8(seed, "rk.out", H, H), H, 0, 1)], H, H, 72)
    parts = lib.lfm3_q8_gemv_parts(H, H)
    us = time_launches(lambda i, s: L.check(lib.lfm3_q8_gemv_partials(
        mats[i][0].addr, mats[i][1].addr, H, H, x.addr, H, y.addr, H, B, parts, s)),
        len(mats), passes)
    entry(f"out / attn_out GEMV in {parts} K parts, 2048 x 2048", us,
          q8_bytes(H, H) + B * H * 4 + parts * B * H * 4, d.n_layers)
    del mats
    # The convolution layer's in projection with the step in its epilogue.
    mats = packed_copies([(L.q8(seed, "rk.in", 3 * H, H), 3 * H, 0, 1)], 3 * H, H, 24)
    taps = L.DeviceBuffer.of(L.normal(seed, "rk.taps", H * d.conv_width, 0, 0.1))
    hists = [L.DeviceBuffer.of(L.normal(seed, f"rk.h{r}", H * (d.conv_width - 1)))
             for r in range(B)]
    table = L.DeviceBuffer.of(np.array([h.addr for h in hists], np.uint64))
    a = L.DeviceBuffer(B * H * 4)
    us = time_launches(lambda i, s, q: L.check(lib.lfm3_q8_gemv_conv_image_norm(
        *norm_args(ffn_parts, q), mats[i][0].addr, mats[i][1].addr, H, B, taps.addr, table.addr,
        d.conv_width, a.addr, H, s)), len(mats), passes, seqs=True)
    entry(f"residual norm ({ffn_parts} K parts) + convolution in_proj GEMV + step, 6144 x 2048",
          us, q8_bytes(3 * H, H) + B * H * 4 * (2 + 2 * (d.conv_width - 1))
          + norm_bytes(d, ffn_parts), n_conv)
    del mats
    # q | k | v | gate of an attention layer on the operand image.
    qr, kr = d.heads * d.head_dim, d.kv_heads * d.head_dim
    tq, tk, tg = -(-qr // 16), -(-kr // 16), -(-d.heads // 16)
    rows = (tq + 2 * tk + tg) * 16
    mats = packed_copies([(L.q8(seed, "rk.q", qr, H), qr, 0, 1),
                          (L.q8(seed, "rk.k", kr, H), kr, tq, 1),
                          (L.q8(seed, "rk.v", kr, H), kr, tq + tk, 1),
                          (L.q8(seed, "rk.g", d.heads, H), d.heads, tq + 2 * tk, 1)],
                         rows, H, 48)
    proj = L.DeviceBuffer(B * rows * 4)
    us = time_launches(lambda i, s, q: L.check(lib.lfm3_q8_gemv_image_norm(
        *norm_args(ffn_parts, q), mats[i][0].addr, mats[i][1].addr, rows, H, 0, B, proj.addr,
        rows, s)), len(mats), passes, seqs=True)
    entry(f"residual norm ({ffn_parts} K parts) + q | k | v | gate GEMV, 3088 x 2048", us,
          q8_bytes(qr + 2 * kr + d.heads, H) + B * H * 4 + B * rows * 4
          + norm_bytes(d, ffn_parts), n_attn)
    del mats
    # The vocabulary head (the round's own launch also keeps greedy keys).
    mats = packed_copies([(L.q8(seed, "rk.head", V, H), V, 0, 1)], V, H, 2)
    logits = L.DeviceBuffer(B * V * 4)
    us = time_launches(lambda i, s, q: L.check(lib.lfm3_q8_gemv_image_norm(
        *norm_args(ffn_parts, q), mats[i][0].addr, mats[i][1].addr, V, H, 0, B, logits.addr, V,
        s)), len(mats), max(2, passes // 2), seqs=True)
    entry(f"final norm ({ffn_parts} K parts) + vocabulary head GEMV, 128000 x 2048", us,
          q8_bytes(V, H) + B * H * 4 + B * V * 4 + norm_bytes(d, ffn_parts), 1)
    del mats
    assert int(werr.download(np.uint32, 1)[0]) == 0, "a fused launch's wait timed out"
    if positions is not None:
        for window in (0, d.window):
            out.append(attention_launch(d, positions, window, proj, rows, passes))
    return out


def attention_launch(d: L.Dims, positions, window: int, proj, ld: int, passes: int):
    """The fused heads + ragged decode attention of one layer of the round
    (global when window is 0, else sliding): rows at `positions` over F16
    rings of N(0, 1) bytes, copies rotated past the MALL. Bytes: the K/V rows
    read (keys [first, position]) and the one written a row."""
    lib = L.lib()
    B, D, kv, heads = len(positions), d.head_dim, d.kv_heads, d.heads
    stride = kv * D
    caps = [min(p + 1, window) if window else p + 1 for p in positions]
    keys = sum(min(p + 1, window) if window else p + 1 for p in positions)
    nbytes = keys * stride * 2 * 2 + B * stride * 2 * 2
    copies = max(2, min(64, (300 << 20) // max(nbytes, 1)))
    pos = np.asarray(positions, np.uint32)
    cap_items = lib.lfm3_attention_max_items(B, int(pos.max()))
    items = (L.AttentionItem * cap_items)()
    count = L.check(lib.lfm3_attention_plan(L.ptr(pos), B, window, items, cap_items))
    ditems = L.DeviceBuffer(count * L.C.sizeof(L.AttentionItem))
    L.hip_check(L.hip().hipMemcpy(ditems.addr, L.C.addressof(items),
                                  count * L.C.sizeof(L.AttentionItem), L.H2D))
    ws_bytes = lib.lfm3_attention_workspace_bytes(count, B, heads, kv, D)
    ws = L.DeviceBuffer(max(ws_bytes, 4))
    dpos = L.DeviceBuffer.of(pos)
    dcap = L.DeviceBuffer.of(np.array(caps, np.uint32))
    norm = L.DeviceBuffer.of(L.normal(L.SEED, "ra.norm", D, 1, 0.02))
    freq = L.DeviceBuffer.of(L.normal(L.SEED, "ra.freq", D // 2, 0.5, 0.1))
    outb = L.DeviceBuffer(B * heads * D * 4)
    sets = []
    for c in range(copies):
        ks = [L.DeviceBuffer(cap * stride * 2) for cap in caps]
        vs = [L.DeviceBuffer(cap * stride * 2) for cap in caps]
        for r in range(B):
            L.hip_check(L.hip().hipMemset(ks[r].addr, 0x3c, ks[r].nbytes))
            L.hip_check(L.hip().hipMemset(vs[r].addr, 0x3c, vs[r].nbytes))
        tk = L.DeviceBuffer.of(np.array([b.addr for b in ks], np.uint64))
        tv = L.DeviceBuffer.of(np.array([b.addr for b in vs], np.uint64))
        sets.append((ks, vs, tk, tv))
    q_off, k_off = 0, heads * D
    v_off, g_off = k_off + stride, k_off + 2 * stride

    def launch(i, stream):
        _, _, tk, tv = sets[i]
        L.check(lib.lfm3_decode_heads_attention_ragged(
            proj.addr + 4 * q_off, proj.addr + 4 * k_off, proj.addr + 4 * v_off, ld,
            proj.addr + 4 * g_off, ld, norm.addr, norm.addr, freq.addr, 0, tk.addr, tv.addr,
            dpos.addr, dcap.addr, ditems.addr, count, outb.addr, heads * D, B, heads, kv, D,
            d.eps, ws.addr, ws_bytes, stream))

    us = time_launches(launch, copies, passes)
    gbs = nbytes / (us * 1e-6) / 1e9
    n_layers = sum(1 for i in range(d.n_layers)
                   if d.layer_type(i) == (L.LAYER_SLIDING if window else L.LAYER_FULL))
    kind = f"sliding-{window}" if window else "global"
    return {"kernel": f"heads + decode attention, {kind} layer ({count} spans; merge included)",
            "us": round(us, 3), "bytes": int(nbytes), "GBps": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "per_round": n_layers}


def config_attention(ctx, heads: int, kv: int, D: int, window: int, passes: int, sets: int = 8):
    """Config 2: the fused heads + ragged decode attention of one layer over
    8 sessions at contexts `ctx` (positions ctx - 1), Q/K RMSNorm, paired
    RoPE at theta 1e6, the sigmoid per-head gate; F16 K/V rings of N(0, 1)
    values, capacity 4096 (global) or 256 (sliding, window 256); at least
    `sets` independent cache sets rotated per timed pass. Bytes: the K/V
    rows read (keys [first, position]), the current row written, and the
    q / k / v / gate rows read and the output written."""
    lib = L.lib()
    B = len(ctx)
    stride = kv * D
    cap = window if window else 4096
    pos = (np.asarray(ctx, np.uint32) - 1).astype(np.uint32)
    keys = sum(min(int(p) + 1, window) if window else int(p) + 1 for p in pos)
    ld = (heads + 2 * kv) * D + heads
    nbytes = keys * stride * 2 * 2 + B * stride * 2 * 2 + B * ld * 4 + B * heads * D * 4
    ring_bytes = cap * stride * 2
    copies = max(sets, min(64, (300 << 20) // max(B * 2 * ring_bytes, 1)))
    cap_items = lib.lfm3_attention_max_items(B, int(pos.max()))
    items = (L.AttentionItem * cap_items)()
    count = L.check(lib.lfm3_attention_plan(L.ptr(pos), B, window, items, cap_items))
    ditems = L.DeviceBuffer(count * L.C.sizeof(L.AttentionItem))
    L.hip_check(L.hip().hipMemcpy(ditems.addr, L.C.addressof(items),
                                  count * L.C.sizeof(L.AttentionItem), L.H2D))
    ws_bytes = lib.lfm3_attention_workspace_bytes(count, B, heads, kv, D)
    ws = L.DeviceBuffer(max(ws_bytes, 4))
    dpos = L.DeviceBuffer.of(pos)
    dcap = L.DeviceBuffer.of(np.full(B, cap, np.uint32))
    qn = L.DeviceBuffer.of(L.normal(L.SEED, f"c2.qn{D}", D, 1, 0.02))
    kn = L.DeviceBuffer.of(L.normal(L.SEED, f"c2.kn{D}", D, 1, 0.02))
    i = np.arange(D // 2, dtype=np.float64)
    freq = L.DeviceBuffer.of(np.power(1e6, -2.0 * i / D).astype(np.float32))
    factors = L.DeviceBuffer.of(np.ones(D // 2, np.float32))
    proj = L.DeviceBuffer.of(L.normal(L.SEED, f"c2.proj{heads}.{D}", B * ld))
    outb = L.DeviceBuffer(B * heads * D * 4)
    # one ring of N(0, 1) halves, copied into every ring of every set
    src = L.DeviceBuffer.of(L.half_normal(L.SEED, f"c2.kv{D}.{window}", cap * stride))
    rings = []
    for c in range(copies):
        ks = [L.DeviceBuffer(ring_bytes) for _ in range(B)]
        vs = [L.DeviceBuffer(ring_bytes) for _ in range(B)]
        for b in ks + vs:
            L.hip_check(L.hip().hipMemcpy(b.addr, src.addr, ring_bytes, 3))  # D2D
        tk = L.DeviceBuffer.of(np.array([b.addr for b in ks], np.uint64))
        tv = L.DeviceBuffer.of(np.array([b.addr for b in vs], np.uint64))
        rings.append((ks, vs, tk, tv))
    L.synchronize()
    k_off, v_off, g_off = heads * D, heads * D + stride, heads * D + 2 * stride

    def launch(c, stream):
        _, _, tk, tv = rings[c]
        L.check(lib.lfm3_decode_heads_attention_ragged(
            proj.addr, proj.addr + 4 * k_off, proj.addr + 4 * v_off, ld, proj.addr + 4 * g_off,
            ld, qn.addr, kn.addr, freq.addr, 0 if window else factors.addr, tk.addr, tv.addr,
            dpos.addr, dcap.addr, ditems.addr, count, outb.addr, heads * D, B, heads, kv, D,
            1e-5, ws.addr, ws_bytes, stream))

    us = time_launches(launch, copies, passes)
    gbs = nbytes / (us * 1e-6) / 1e9
    kind = f"sliding-{window}" if window else "global"
    return {"kernel": f"heads + decode attention, {heads}q/{kv}kv x {D}, {kind}, 8 rows "
                      f"({count} spans; {copies} cache sets rotated)",
            "us": round(us, 3), "bytes": int(nbytes), "GBps": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def config_conv(passes: int):
    """Config 3: the gated width-7 short-convolution block of 8 sessions
    (hidden 2048; in projection 6144 x 2048 with the step in its epilogue,
    from the normed rows' operand image; out projection 2048 x 2048 in K
    parts; FP32 histories [8][2048][6] N(0, 1), taps N(0, 0.1)), two launches
    a block, 24 rotated weight copies; and the prefill variant, the packed
    prompt convolution over segments of {512, 37, 300, 1} rows (850 rows,
    each continuing its own session's history), from their in-projection
    rows."""
    lib = L.lib()
    seed = L.SEED
    H, B, W = 2048, SESSIONS, 7
    x = L.DeviceBuffer.of(L.normal(seed, "c3.x", B * H))
    wts = L.DeviceBuffer.of(np.ones(H, np.float32))
    image = L.DeviceBuffer(lib.lfm3_operand_image_bytes(H))
    exps = L.DeviceBuffer(32)
    L.check(lib.lfm3_residual_norm_image(None, 1, 0, None, x.addr, wts.addr, None, image.addr,
                                         exps.addr, B, H, 1e-5, None))
    taps = L.DeviceBuffer.of(L.normal(seed, "c3.taps", H * W, 0, 0.1))
    hists = [L.DeviceBuffer.of(L.normal(seed, f"c3.h{r}", H * (W - 1))) for r in range(B)]
    table = L.DeviceBuffer.of(np.array([h.addr for h in hists], np.uint64))
    copies = 24
    ins = packed_copies([(L.q8(seed, "c3.in", 3 * H, H), 3 * H, 0, 1)], 3 * H, H, copies)
    outs = packed_copies([(L.q8(seed, "c3.out", H, H), H, 0, 1)], H, H, copies)
    a = L.DeviceBuffer(B * H * 4)
    parts = lib.lfm3_q8_gemv_parts(H, H)
    y = L.DeviceBuffer(parts * B * H * 4)

    def block(i, s):
        L.check(lib.lfm3_q8_gemv_conv_image(ins[i][0].addr, ins[i][1].addr, H, image.addr,
                                            exps.addr, B, taps.addr, table.addr, W, a.addr, H,
                                            s))
        L.check(lib.lfm3_q8_gemv_partials(outs[i][0].addr, outs[i][1].addr, H, H, a.addr, H,
                                          y.addr, H, B, parts, s))

    us = time_launches(block, copies, passes)
    nbytes = (q8_bytes(3 * H, H) + q8_bytes(H, H) + B * H * 4  # weights, normed rows
              + B * H * (W - 1) * 4 * 2                        # histories read and written
              + B * H * 4 * 2 + parts * B * H * 4)             # y written and read, out parts
    gbs = nbytes / (us * 1e-6) / 1e9
    block_line = {"kernel": f"convolution block, 8 rows: in projection 6144 x 2048 + step, out "
                            f"projection 2048 x 2048 in {parts} K parts (two launches)",
                  "us": round(us, 3), "bytes": int(nbytes), "GBps": round(gbs, 1),
                  "frac": round(gbs / HBM_PEAK_GBS, 4)}
    del ins, outs
    # the packed prompt convolution
    seg = [512, 37, 300, 1]
    n = sum(seg)
    begins = np.cumsum([0] + seg[:-1]).astype(np.uint32)
    p = L.DeviceBuffer.of(L.normal(seed, "c3.p", n * 3 * H))
    yp = L.DeviceBuffer(n * H * 4)
    phist = [L.DeviceBuffer.of(L.normal(seed, f"c3.ph{r}", H * (W - 1))) for r in range(4)]
    hp = (L.C.c_void_p * 4)(*[h.addr for h in phist])
    rows = np.asarray(seg, np.uint32)

    def conv(i, s):
        L.check(lib.lfm3_conv_prompt(p.addr, 3 * H, taps.addr, hp, L.ptr(begins), L.ptr(rows), 4,
                                     yp.addr, H, H, W, 0, s))

    us = time_launches(conv, 8, passes)
    nbytes = n * H * 4 * 4 + 4 * H * (W - 1) * 4
    gbs = nbytes / (us * 1e-6) / 1e9
    prefill_line = {"kernel": "packed prompt convolution, segments {512, 37, 300, 1} (850 rows), "
                              "hidden 2048, width 7",
                    "us": round(us, 3), "bytes": int(nbytes), "GBps": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4)}
    return block_line, prefill_line


def projection_weights(d: L.Dims) -> int:
    """Weight elements of every projection a token's row goes through (the
    vocabulary head excluded)."""
    H, F, D = d.hidden, d.intermediate, d.head_dim
    total = 0
    for i in range(d.n_layers):
        total += 3 * F * H
        if d.layer_type(i) == L.LAYER_CONV:
            total += 3 * H * H + H * H
        else:
            total += (d.heads * D + 2 * d.kv_heads * D + d.heads) * H + H * d.heads * D
    return total


def pass_flops(d: L.Dims, n: int, depth: int, pruned: bool) -> int:
    """Algorithmic FLOPs of an n-row prompt pass at `depth`: 2 n W for the
    projections and 4 D h keys for QK^T and PV per query row. With the
    reference's trailing-row pruning (engine.cpp:304-323) a last global
    layer runs its attention output, attention and FFN on the frontier row
    only."""
    H, F, D = d.hidden, d.intermediate, d.head_dim
    flops = 2 * n * projection_weights(d)
    for i in range(d.n_layers):
        t = d.layer_type(i)
        if t == L.LAYER_CONV:
            continue
        keys = [depth + r + 1 if t == L.LAYER_FULL else min(depth + r + 1, d.window)
                for r in range(n)]
        flops += 4 * D * d.heads * sum(keys)
    if pruned and d.layer_type(d.n_layers - 1) == L.LAYER_FULL:
        last_keys = sum(depth + r + 1 for r in range(n - 1))
        flops -= 2 * (n - 1) * (H * d.heads * D + 3 * F * H) + 4 * D * d.heads * last_keys
    return flops


def gemm_roofline(copies: int, passes: int):
    """The prompt pass's dominant kernel: the gate/up SwiGLU GEMM (7680 gate
    + 7680 up rows x 2048, Q8_0 on FP16 tiles) on 512 FP16 rows, launched as
    the pass launches it (lfm3_q8_gemm_swiglu_h16_rows: its trailing blocks
    write the down projection's FP16 rows), over `copies` rotated weight
    buffers, replayed from HIP graphs and timed with HIP events on the
    stream it runs on. The same GEMM without the trailing blocks
    (lfm3_q8_gemm_swiglu_h16, its row maxima for a separate conversion) is
    timed beside it."""
    import ctypes as C
    lib = L.lib()
    F, H, n = 7680, 2048, PASS_ROWS
    cb, sb = C.c_size_t(), C.c_size_t()
    lib.lfm3_q8_tiled_bytes(2 * F, H, C.byref(cb), C.byref(sb))
    codes = np.zeros(cb.value, np.uint8)
    scales = np.zeros(sb.value, np.uint8)
    g = L.q8(L.SEED, "gemm.gate", F, H)
    u = L.q8(L.SEED, "gemm.up", F, H)
    L.check(lib.lfm3_q8_pack_host(L.ptr(g), F, H, L.ptr(codes), L.ptr(scales), 0, 2))
    L.check(lib.lfm3_q8_pack_host(L.ptr(u), F, H, L.ptr(codes), L.ptr(scales), 1, 2))
    # The pass reads FP16 tiles: decoded once from the codes, as the model does.
    dcodes = L.DeviceBuffer.of(codes)
    mats = []
    for _ in range(copies):
        halves = L.DeviceBuffer(lib.lfm3_q8_half_tiles_bytes(2 * F, H))
        L.check(lib.lfm3_q8_half_tiles(dcodes.addr, 2 * F, H, halves.addr, None))
        mats.append((halves, L.DeviceBuffer.of(scales)))
    L.synchronize()
    dcodes.close()
    x = L.DeviceBuffer.of(L.normal(L.SEED, "gemm.x", n * H))
    a16 = L.DeviceBuffer(n * H * 2)
    scale = L.DeviceBuffer(n * 4)
    L.check(lib.lfm3_half_rows(x.addr, H, None, 0, a16.addr, H, scale.addr, n, H, None))
    y = L.DeviceBuffer(n * F * 4)
    max_blocks = lib.lfm3_q8_gemm_swiglu_max_blocks(F)
    row_max = L.DeviceBuffer(max_blocks * n * 4)
    hld = (F + 63) // 64 * 64
    hid16 = L.DeviceBuffer(n * hld * 2)
    hscale = L.DeviceBuffer(n * 4)
    flags = L.DeviceBuffer(lib.lfm3_q8_gemm_swiglu_flags_bytes(F, n))
    L.hip_check(L.hip().hipMemset(flags.addr, 0, flags.nbytes))
    err = L.DeviceBuffer(4)
    L.hip_check(L.hip().hipMemset(err.addr, 0, 4))
    L.synchronize()
    us = time_launches(lambda i, s, q: L.check(lib.lfm3_q8_gemm_swiglu_h16_rows(
        mats[i][0].addr, mats[i][1].addr, F, H, a16.addr, H, scale.addr, n, y.addr, F,
        row_max.addr, hid16.addr, hld, hscale.addr, flags.addr, q, err.addr, s)),
        copies, passes, seqs=True)
    if int(err.download(np.uint32, 1)[0]):
        raise RuntimeError("the SwiGLU GEMM's trailing blocks timed out waiting")
    gemm_us = time_launches(lambda i, s: L.check(lib.lfm3_q8_gemm_swiglu_h16(
        mats[i][0].addr, mats[i][1].addr, F, H, a16.addr, H, scale.addr, n, y.addr, F,
        row_max.addr, s)), copies, passes)
    flops = 2 * n * 2 * F * H
    # FP16 weights (2 bytes each) and their fp16 block scales, the FP16
    # rows with their scales, the FP32 outputs and row maxima, and the FP16
    # hidden rows with their scales (the trailing blocks' re-read of the
    # FP32 outputs is not counted).
    gemm_bytes = (2 * F * H * 2 + 2 * F * (H // 32) * 2 + n * H * 2 + n * 4 + n * F * 4
                  + max_blocks * n * 4)
    nbytes = gemm_bytes + n * hld * 2 + n * 4
    return {"flops": flops, "bytes": nbytes, "us": us, "tflops": flops / (us * 1e-6) / 1e12,
            "gemm_only_us": gemm_us, "gemm_only_bytes": gemm_bytes,
            "gemm_only_tflops": flops / (gemm_us * 1e-6) / 1e12}


def copy_calibration(nbytes: int, reps: int):
    """Plain device-to-device copies of `nbytes` (the runtime's blit
    kernel): the known-size launch that FETCH_SIZE and WRITE_SIZE are
    scaled by when the roofline kernels' HBM traffic is counted."""
    src, dst = L.DeviceBuffer(nbytes), L.DeviceBuffer(nbytes)
    stream = L.Stream()
    for _ in range(reps):
        L.hip_check(L.hip().hipMemcpyAsync(dst.addr, src.addr, nbytes, L.D2D, stream.handle))
    stream.synchronize()
    stream.close()
    src.close()
    dst.close()


def device_ceilings(read_bytes: int = 2 << 30, reps: int = 8):
    """What this MI355X delivers to a kernel, beside the published peaks: a
    plain streaming read of a 2 GiB buffer (lfm3_measure_stream_read, best
    of four grid sizes) and a register-only f16 MFMA loop
    (lfm3_measure_mfma_f16, 4 waves a SIMD), each timed with HIP events over
    `reps` back-to-back launches on its own stream after one untimed
    launch."""
    lib = L.lib()
    stream = L.Stream()

    def timed(launch) -> float:
        launch()
        stream.synchronize()
        a, b = L.Event(), L.Event()
        a.record(stream.handle)
        for _ in range(reps):
            launch()
        b.record(stream.handle)
        b.synchronize()
        ms = a.elapsed_ms(b) / reps
        a.close()
        b.close()
        return ms

    buf = L.DeviceBuffer(read_bytes)
    L.hip_check(L.hip().hipMemset(buf.addr, 0x5a, read_bytes))
    sink = L.DeviceBuffer(65535 * 4 * 4)
    best, best_blocks = 0.0, 0
    for blocks in (1024, 2048, 4096, 8192):
        ms = timed(lambda: L.check(lib.lfm3_measure_stream_read(
            buf.addr, read_bytes, sink.addr, blocks, stream.handle)))
        if read_bytes / (ms * 1e-3) / 1e9 > best:
            best, best_blocks = read_bytes / (ms * 1e-3) / 1e9, blocks
    buf.close()
    iters, blocks = 4096, 1024
    ms = timed(lambda: L.check(lib.lfm3_measure_mfma_f16(iters, blocks, sink.addr,
                                                         stream.handle)))
    tflops = lib.lfm3_measure_mfma_f16_flops(iters, blocks) / (ms * 1e-3) / 1e12
    sink.close()
    stream.close()
    return {"stream_read_GBps": round(best, 1), "stream_read_bytes": read_bytes,
            "stream_read_blocks": best_blocks,
            "mfma_f16_TFLOPs": round(tflops, 1),
            "stream_read_frac_of_peak": round(best / HBM_PEAK_GBS, 4),
            "mfma_f16_frac_of_peak": round(tflops / MFMA_PEAK_TFLOPS, 4)}


def roofline_only():
    """The roofline kernels and the copy calibration, nothing else: the
    program that rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE run (the
    decode round's kernels at their round shapes, the attention at the
    bench's contexts included, the 8192 x 2048 GEMV at 8 rows, the prompt
    pass's SwiGLU GEMM)."""
    copy_bytes = 256 << 20
    copy_calibration(copy_bytes, 4)
    ctx = L.uniform_u32(L.SEED, "bench.ctx", SESSIONS, CTX_LO, CTX_HI)
    kernels = round_kernels(L.Dims(), [int(c) - 1 for c in ctx], passes=2)
    g = gemv_roofline(8, 32, 2)
    m = gemm_roofline(8, 2)
    print(json.dumps({"copy_bytes": copy_bytes, "round_kernels": kernels,
                      "gemv_bytes": g["bytes"], "gemv_us": g["us"],
                      "gemm_flops": m["flops"], "gemm_us": m["us"]}), flush=True)


def variant_round(dims: L.Dims, seed, ctx, tokens0, steps: int, warmup: int, workload: str,
                  bf16: bool = False):
    """The decode round of 8 sessions at the same contexts on another model:
    its own random-init weights (Q8_0, or BF16 with bf16) and synthesized
    state, greedy ids fed back."""
    model = L.Model(L.synth_weights(dims, seed=seed, bf16_weights=bf16))
    sessions = []
    for sid, c in enumerate(ctx):
        s = model.session(int(c) + warmup + steps + 8)
        L.inject_synth_state(s, dims, seed, sid, int(c) - 1)
        sessions.append(s)
    toks = tokens0 % dims.vocab
    for _ in range(warmup):
        toks = model.forward_batch_greedy(sessions, toks)
    L.synchronize()
    positions = [[s.position + k for s in sessions] for k in range(steps)]
    t0 = time.perf_counter()
    for _ in range(steps):
        toks = model.forward_batch_greedy(sessions, toks)
    L.synchronize()
    ms = (time.perf_counter() - t0) * 1000.0 / steps
    nbytes = statistics.mean(round_bytes(dims, p, bf16) for p in positions)
    for s in sessions:
        s.close()
    model.close()
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {
        "workload": workload,
        "ms": round(ms, 4),
        "tok_s": round(SESSIONS / (ms * 1e-3), 1),
        "bytes": int(nbytes),
        "weight_bytes": weight_bytes(dims, bf16),
        "achieved_GBps": round(gbs, 1),
        "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4),
    }


def prefill_and_mixed(model, dims, seed, reps: int, warmup: int):
    """The 512-token pass at depth 24576 alone, then the mixed round (7
    decode sessions at contexts in [16384, 32768] plus the pass). Each
    repetition rewinds the prompt session to the depth, so every pass does
    the same work."""
    prompt = model.session(PASS_DEPTH + PASS_ROWS)
    L.inject_synth_state(prompt, dims, seed, 100, PASS_DEPTH)
    tokens = L.uniform_u32(seed, "bench.pass.tokens", PASS_ROWS, 0, dims.vocab - 1)

    def one_pass():
        prompt.set_position(PASS_DEPTH)
        prompt.forward(tokens)

    for _ in range(warmup):
        one_pass()
    L.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        one_pass()
    L.synchronize()
    pass_ms = (time.perf_counter() - t0) * 1000.0 / reps

    ctx = L.uniform_u32(seed, "bench.mixed.ctx", MIXED_DECODE, MIXED_LO, MIXED_HI)
    decode = []
    for sid, c in enumerate(ctx):
        s = model.session(int(c) + 3 * (warmup + reps) + 8)
        L.inject_synth_state(s, dims, seed, 200 + sid, int(c) - 1)
        decode.append(s)
    toks = L.uniform_u32(seed, "bench.mixed.tokens", MIXED_DECODE, 0, dims.vocab - 1)

    def overlapped(toks):
        prompt.set_position(PASS_DEPTH)
        ids, _, _ = model.scheduler_round(decode, toks, prompt, tokens)
        return ids

    def serial(toks):
        toks = model.forward_batch_greedy(decode, toks)
        one_pass()
        return toks

    def decode_only(toks):
        return model.forward_batch_greedy(decode, toks)

    times = {}
    for name, fn in (("decode", decode_only), ("serial", serial), ("overlapped", overlapped)):
        for _ in range(warmup):
            toks = fn(toks)
        L.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            toks = fn(toks)
        L.synchronize()
        times[name] = (time.perf_counter() - t0) * 1000.0 / reps
    return pass_ms, times, [int(c) for c in ctx]


def usable_cores(hw: int) -> int:
    """The cores this process may run on: its CPU affinity, capped by a
    cgroup CPU quota where one is set (cgroup v2 cpu.max, or v1
    cfs_quota_us / cfs_period_us)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else hw
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
            if q != "max":
                quota = int(q) / int(period)
    except (OSError, ValueError):
        try:
            with open("/sys/fs/cgroup/cpu/cpu.cfs_quota_us") as f:
                q = int(f.read())
            with open("/sys/fs/cgroup/cpu/cpu.cfs_period_us") as f:
                period = int(f.read())
            if q > 0:
                quota = q / period
        except (OSError, ValueError):
            pass
    if quota is not None:
        n = min(n, max(1, int(quota)))
    return max(1, n)


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(dims, weights, ctx, tokens, seed):
    """The CPU oracle (a scalar FP32 restatement of reference.cpp) decoding
    the same eight sessions from the same synthesized state, each session's
    greedy id fed back as its next token, in three modes:

      faithful      one round, sessions one after another on one thread
                    (reference.cpp has no threads);
      per_session   rounds with one thread per session;
      row_parallel  rounds with sessions in turn and each matrix-vector
                    product's rows (and each attention read's heads) split
                    over the host's cores, in the style of npu/host_ops.hpp
                    Parallel.

    Every mode computes identical logits (each output row keeps its
    sequential sum). About 10 s of wall time each. Returns (result dict,
    per-session greedy ids of the first round, their top-2 margins)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    hw = O.hardware_concurrency()
    usable = usable_cores(hw)
    cores = usable
    om = O.Model(dims, weights)

    def fresh_sessions(extra):
        out = []
        for sid, c in enumerate(ctx):
            position = int(c) - 1
            s = om.session(int(c) + extra + 256, f16=True)
            for l in range(dims.n_layers):
                if dims.layer_type(l) == L.LAYER_CONV:
                    s.conv(l)[:] = L.synth_conv_state(seed, sid, l, dims)
                else:
                    rows = L.live_slots(position, s.capacity(l))
                    n = rows * dims.kv_heads * dims.head_dim
                    for view, tag in ((s.k, "k"), (s.v, "v")):
                        view(l)[:n] = O.half_to_float(
                            L.synth_kv_state(seed, sid, l, tag, rows, dims))
            s.set_position(position)
            out.append(s)
        return out

    first = [None] * len(ctx)

    def run(mode, rounds):
        sessions = fresh_sessions(rounds)
        toks = [int(t) for t in tokens]

        def session_rounds(i):
            for r in range(rounds):
                logits = sessions[i].step(toks[i])
                toks[i] = O.argmax(logits)
                if r == 0 and first[i] is None:
                    first[i] = logits

        t0 = time.perf_counter()
        if mode == "per_session":
            O.set_threads(1)
            workers = [threading.Thread(target=session_rounds, args=(i,))
                       for i in range(len(sessions))]
            for w in workers:
                w.start()
            for w in workers:
                w.join()
            used = len(sessions)
        else:
            O.set_threads(cores if mode == "row_parallel" else 1)
            for r in range(rounds):
                for i in range(len(sessions)):
                    logits = sessions[i].step(toks[i])
                    toks[i] = O.argmax(logits)
                    if r == 0 and first[i] is None:
                        first[i] = logits
            used = cores if mode == "row_parallel" else 1
        wall = time.perf_counter() - t0
        O.set_threads(1)
        for s in sessions:
            s.close()
        return {"mode": mode, "value": round(rounds * len(ctx) / wall, 4), "cores": used,
                "rounds": rounds, "wall_s": round(wall, 2)}

    modes = [run("faithful", 1), run("per_session", 6), run("row_parallel", 4)]
    om.close()
    best = max(modes, key=lambda m: m["value"])
    ids = [O.argmax(o) for o in first]
    margins = [float(np.diff(np.sort(o)[-2:])[0]) for o in first]
    res = {"value": best["value"], "unit": "tok/s", "cores": best["cores"], "kind": "port",
           "sample": (f"decode rounds of {len(ctx)} sessions (one token each, greedy ids fed "
                      f"back) through the full model from the same contexts and state; value "
                      f"is the fastest mode ({best['mode']}: {best['rounds']} rounds, "
                      f"{best['cores']} threads, {best['wall_s']} s)"),
           "modes": modes, "hardware_concurrency": hw, "usable_cores": usable,
           "cpu_model": cpu_model()}
    return res, ids, margins


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--gemv-copies", type=int, default=32)
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the 512-token pass and the mixed round")
    ap.add_argument("--prefill-reps", type=int, default=5)
    ap.add_argument("--roofline-only", action="store_true",
                    help="run only the roofline kernels and a plain copy (for rocprofv3 --pmc)")
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
    if args.roofline_only:
        roofline_only()
        return

    seed = L.SEED
    dims = L.Dims(context=MIXED_HI + 1024)
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
        s = model.session(int(c) + 2 * (args.warmup + args.steps) + 8)
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
    step_ms = []
    for _ in range(args.steps):
        ts = time.perf_counter()
        toks = model.forward_batch_greedy(sessions, toks)  # returns after the ids land
        step_ms.append((time.perf_counter() - ts) * 1000.0)
    L.synchronize()
    wall = time.perf_counter() - t0
    ev1.record(stream)
    ev1.synchronize()
    ms_per_step = wall * 1000.0 / args.steps
    value = SESSIONS / (ms_per_step / 1000.0)
    rbytes = statistics.mean(round_bytes(dims, p) for p in positions)
    round_gbs = rbytes / (ms_per_step / 1000.0) / 1e9
    log(f"round {ms_per_step:.3f} ms, {value:.1f} tok/s, {round_gbs:.0f} GB/s")

    # The same rounds with the serving loop's sampler (runner.cpp:31-35
    # defaults) in place of the greedy pick: the last 64 ids of each session
    # as its penalty list, seeded uniforms.
    params = L.Sampling(0.1, 50, 1.1)
    rng = np.random.default_rng(seed)
    recent = np.full((SESSIONS, 64), dims.vocab, np.uint32)  # ids >= vocab pad
    for k in range(args.warmup):  # untimed, as for the greedy rounds
        recent[:, k % 64] = toks
        toks = model.forward_batch_sample(sessions, toks, params,
                                          rng.random(SESSIONS, dtype=np.float32), recent)
    t0 = time.perf_counter()
    for k in range(args.warmup, args.warmup + args.steps):
        recent[:, k % 64] = toks
        toks = model.forward_batch_sample(sessions, toks, params,
                                          rng.random(SESSIONS, dtype=np.float32), recent)
    L.synchronize()
    sampled_ms = (time.perf_counter() - t0) * 1000.0 / args.steps
    log(f"sampled round {sampled_ms:.3f} ms")

    # The round's kernels alone at their round shapes; the first (the
    # residual norm fused with the SwiGLU operand-image GEMV, the largest
    # share of the round) is the roofline.
    kernels = round_kernels(dims, [int(c) - 1 for c in ctx])
    top = kernels[0]
    for k in kernels:
        log(f"{k['kernel']}: {k['us']:.2f} us, {k['GBps']:.0f} GB/s ({100 * k['frac']:.1f}%), "
            f"x{k['per_round']} a round")
    # The single Q8_0 GEMV, W 8192 x 2048 on FP32 rows, B = 1, 2, 4, 8.
    sweep = [gemv_roofline(b, args.gemv_copies, 8) for b in (1, 2, 4, 8)]
    for g in sweep:
        log(f"gemv B={g['batch']}: {g['us']:.2f} us/launch, "
            f"{g['bytes'] / (g['us'] * 1e-6) / 1e9:.0f} GB/s")
    # Config 2: one layer's ragged decode attention at contexts U[1, 4096],
    # both head shapes, global and sliding; config 3: the convolution block
    # and the packed prompt convolution.
    ctx2 = L.uniform_u32(seed, "bench.attn.ctx", SESSIONS, 1, 4096)
    config2 = [config_attention(ctx2, h, kv, D, w, 6)
               for h, kv, D in ((32, 8, 64), (16, 4, 128)) for w in (0, 256)]
    conv_block, conv_prompt = config_conv(6)
    for k in config2 + [conv_block, conv_prompt]:
        log(f"{k['kernel']}: {k['us']:.2f} us, {k['GBps']:.0f} GB/s ({100 * k['frac']:.1f}%)")

    result = {
        "metric": "decode tok/s @8 sessions (HBM GB/s % peak); 512-tok prefill pass ms (MFMA %)",
        "value": round(value, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 x f32 (activations as two fp16 planes, hi and lo each truncated to 11 "
                 "bits: within 2^-20 of each value; fp32 accumulate)",
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
            "kernel": top["kernel"] + ", 8 rows (the round's dominant launch)",
            "achieved": top["GBps"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": top["frac"],
            "traffic": (SWIGLU_TRAFFIC["read"] + SWIGLU_TRAFFIC["write"]
                        if SWIGLU_TRAFFIC["read"] is not None else None),
            "traffic_read_write": [SWIGLU_TRAFFIC["read"], SWIGLU_TRAFFIC["write"]],
            "bytes_per_launch": top["bytes"],
            "us_per_launch": top["us"],
        },
        "round_kernels": kernels,
        "round": {
            "bytes": int(rbytes),
            "achieved_GBps": round(round_gbs, 1),
            "frac_of_peak": round(round_gbs / HBM_PEAK_GBS, 4),
            "gpu_ms_per_step": round(ev0.elapsed_ms(ev1) / args.steps, 4),
            "step_ms_median": round(float(np.median(step_ms)), 4),
            "step_ms_p10": round(float(np.percentile(step_ms, 10)), 4),
            "step_ms_p90": round(float(np.percentile(step_ms, 90)), 4),
        },
        "sampled_round": {
            "workload": ("the same round with lfm3_forward_batch_sample at the serving "
                         "loop's defaults (temperature 0.1, top_k 50, repeat_penalty 1.1 "
                         "over the last 64 ids) instead of the greedy pick"),
            "ms": round(sampled_ms, 4),
            "tok_s": round(SESSIONS / (sampled_ms * 1e-3), 1),
        },
        "gemv_8192x2048": {
            "kernel": "Q8_0 skinny GEMV, W 8192 x 2048 on FP32 rows (single-GEMV workload)",
            "sweep": [{"batch": g["batch"], "us": round(g["us"], 3), "bytes": g["bytes"],
                       "GBps": round(g["bytes"] / (g["us"] * 1e-6) / 1e9, 1),
                       "frac": round(g["bytes"] / (g["us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
                      for g in sweep],
            "traffic_read_write": [GEMV_TRAFFIC["read"], GEMV_TRAFFIC["write"]],
        },
        "attention_one_layer": {
            "workload": ("one layer's fused Q/K norm, RoPE (theta 1e6), gate and ragged decode "
                         "attention, 8 sessions at contexts uniform in [1, 4096], F16 K/V rings "
                         "(capacity 4096 global, 256 sliding)"),
            "contexts": [int(c) for c in ctx2],
            "lines": config2,
        },
        "conv_block": conv_block,
        "conv_prompt_packed": conv_prompt,
    }
    ceilings = device_ceilings()
    log(f"measured ceilings: streaming read {ceilings['stream_read_GBps']:.0f} GB/s, "
        f"f16 MFMA loop {ceilings['mfma_f16_TFLOPs']:.0f} TFLOP/s")
    result["measured_ceilings"] = ceilings
    result["roofline"]["frac_of_measured"] = round(top["GBps"] / ceilings["stream_read_GBps"], 4)
    result["round"]["frac_of_measured"] = round(round_gbs / ceilings["stream_read_GBps"], 4)
    span = CTX_HI + args.warmup + args.steps + 64
    nominal = variant_round(
        L.Dims(intermediate=8192, heads=32, kv_heads=8, head_dim=64, vocab=65536, context=span),
        seed, ctx, tokens0, args.steps, args.warmup,
        "the same round on the nominal dims: FFN 8192, 32q/8kv heads x 64, vocab 65536 "
        "(hidden 2048, 24 layers 13/5/6, Q8_0)")
    log(f"nominal-dims round {nominal['ms']:.3f} ms, {nominal['tok_s']:.0f} tok/s, "
        f"{nominal['achieved_GBps']:.0f} GB/s")
    result["nominal_round"] = nominal
    bf16 = variant_round(
        L.Dims(context=span), seed, ctx, tokens0, args.steps, args.warmup,
        "the same round with BF16 weights (the reference precision: exact BF16 x FP32 "
        "projections), reference dims", bf16=True)
    log(f"BF16-weights round {bf16['ms']:.3f} ms, {bf16['tok_s']:.0f} tok/s, "
        f"{bf16['achieved_GBps']:.0f} GB/s")
    bf16["gemv"] = bf16_gemv_roofline(8, 16, 6)
    log(f"BF16 GEMV 8192 x 2048, 8 rows: {bf16['gemv']['us']:.2f} us, "
        f"{bf16['gemv']['GBps']:.0f} GB/s")
    result["bf16_round"] = bf16
    if not args.no_prefill:
        log("512-token prompt pass at depth 24576 and the mixed round ...")
        pass_ms, mixed, mixed_ctx = prefill_and_mixed(model, dims, seed, args.prefill_reps, 2)
        mixed_ms = mixed["overlapped"]
        flops = pass_flops(dims, PASS_ROWS, PASS_DEPTH, pruned=True)
        flops_full = pass_flops(dims, PASS_ROWS, PASS_DEPTH, pruned=False)
        tflops = flops / (pass_ms * 1e-3) / 1e12
        gemm = gemm_roofline(8, 4)
        log(f"pass {pass_ms:.2f} ms, {tflops:.0f} TFLOP/s; mixed round {mixed_ms:.2f} ms "
            f"(serial {mixed['serial']:.2f}, decode alone {mixed['decode']:.2f}); "
            f"swiglu GEMM {gemm['us']:.1f} us, {gemm['tflops']:.0f} TFLOP/s "
            f"(without its trailing blocks {gemm['gemm_only_us']:.1f} us)")
        result["prefill"] = {
            "workload": (f"one {PASS_ROWS}-token prompt pass (Session::Forward) at depth "
                         f"{PASS_DEPTH} of a synthesized session, same model"),
            "ms": round(pass_ms, 3),
            "flops": int(flops),
            "flops_without_pruning": int(flops_full),
            "tflops": round(tflops, 1),
            "mfma_frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
            "mfma_frac_of_measured": round(tflops / ceilings["mfma_f16_TFLOPs"], 4),
            "reps": args.prefill_reps,
            "roofline": {
                "bound": "mfma",
                "kernel": ("Q8_0 x FP16 SwiGLU GEMM, 15360 x 2048 on 512 rows, with its "
                           "trailing blocks writing the 512 x 7680 FP16 hidden rows"),
                "achieved": round(gemm["tflops"], 1),
                "peak": MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(gemm["tflops"] / MFMA_PEAK_TFLOPS, 4),
                "frac_of_measured": round(gemm["tflops"] / ceilings["mfma_f16_TFLOPs"], 4),
                "traffic": GEMM_TRAFFIC["read"] + GEMM_TRAFFIC["write"],
                "traffic_read_write": [GEMM_TRAFFIC["read"], GEMM_TRAFFIC["write"]],
                "algorithmic_bytes": gemm["bytes"],
                "flops_per_launch": gemm["flops"],
                "us_per_launch": round(gemm["us"], 2),
                "gemm_only_us_per_launch": round(gemm["gemm_only_us"], 2),
                "gemm_only_frac": round(gemm["gemm_only_tflops"] / MFMA_PEAK_TFLOPS, 4),
            },
        }
        result["mixed_round"] = {
            "workload": (f"{MIXED_DECODE} decode sessions at contexts in [{MIXED_LO}, {MIXED_HI}] "
                         f"plus the {PASS_ROWS}-token pass (lfm3_scheduler_round: the decode "
                         f"round and the pass on two streams)"),
            "ms": round(mixed_ms, 3),
            "serial_ms": round(mixed["serial"], 3),
            "decode_round_ms": round(mixed["decode"], 3),
            "pass_ms": round(pass_ms, 3),
            "decode_contexts": mixed_ctx,
        }
    if not args.no_cpu:
        log("CPU oracle rounds (faithful, per-session and row-parallel modes) ...")
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
