"""The full-dims decode round and the mixed round's depths at their own
sizes on the GPU, against the CPU oracle (reference.cpp restated).

The decode round: the full 24-layer model at the reference checkpoint's dims (13
conv, 5 sliding-256, 6 global; hidden 2048, FFN 7680, 16q/4kv x 128, vocab
128000, random-init Q8_0) with 8 sessions at the benchmark's contexts,
uniform in [128, 8192]: one ForwardBatch round. Logits within 2e-3 of the
oracle and the same greedy id for every session, unconditionally (each
session's oracle top-2 margin is printed beside it).

The mixed round's depths: decode attention of 7 rows at contexts uniform in
[16384, 32768] (sliding and global), the 512-row prompt attention at depth
24576 (16/4 heads x 128, sliding and global) against an FP64 softmax over
the F16-rounded keys at 1e-3 (ops_test.cpp:203), and a full-dims
Session::Forward of a 513-token prompt on a session at depth 24576 against
the oracle stepping the same tokens and against 513 GPU decode rounds, at
session_test.cpp:120-143's gate (KL < 1e-6, max |logit| < 0.02, the same
argmax)."""
import math
import threading

import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import (kl_divergence, oracle_prompt, oracle_twin, pointer_table,
                      prompt_gate_pair, same_greedy, within)

pytestmark = pytest.mark.gpu
SEED = L.SEED
C_ITEM = L.C.sizeof(L.AttentionItem)


def inject_both(g, o, dims, seed, sid, position):
    """Synthesized state at `position` (conv history, the ring slots of
    positions [0, position)), identical on the GPU and oracle sessions."""
    L.inject_synth_state(g, dims, seed, sid, position)
    for l in range(dims.n_layers):
        if dims.layer_type(l) == L.LAYER_CONV:
            o.conv(l)[:] = L.synth_conv_state(seed, sid, l, dims)
        else:
            assert g.capacity(l) == o.capacity(l)
            rows = L.live_slots(position, o.capacity(l))
            n = rows * dims.kv_heads * dims.head_dim
            for view, tag in ((o.k, "k"), (o.v, "v")):
                view(l)[:n] = O.half_to_float(L.synth_kv_state(seed, sid, l, tag, rows, dims))
    o.set_position(position)


def test_full_dims_round_eight_sessions():
    ctx = L.uniform_u32(SEED, "bench.ctx", 8, 128, 8192)
    dims = L.Dims(context=8192 + 64)
    w = L.synth_weights(dims, seed=SEED)
    gm, om = L.Model(w), O.Model(dims, w)
    gs, os_ = [], []
    for sid, c in enumerate(ctx):
        g = gm.session(int(c) + 8)
        o = om.session(int(c) + 8, f16=True)
        inject_both(g, o, dims, SEED, sid, int(c) - 1)
        gs.append(g)
        os_.append(o)
    toks = L.uniform_u32(SEED, "bench.tokens", 8, 0, dims.vocab - 1)
    got = gm.forward_batch(gs, toks)
    want = [None] * 8

    def step(i):
        want[i] = os_[i].step(int(toks[i]))

    O.set_threads(1)
    workers = [threading.Thread(target=step, args=(i,)) for i in range(8)]
    for t in workers:
        t.start()
    for t in workers:
        t.join()
    for i in range(8):
        err = same_greedy(got[i], want[i], f"session {i} ctx {int(ctx[i])}")
        assert err < 2e-3, (i, err)
        assert gs[i].position == os_[i].position == int(ctx[i])
    for x in gs + os_:
        x.close()
    gm.close()
    om.close()


@pytest.mark.parametrize("window", [0, 256])
def test_decode_attention_at_depth(window):
    """Seven rows at contexts U[16384, 32768]: fused heads + ragged decode
    attention against orc_attention_step (reference.cpp:102-146), 16/4
    heads x 128, RoPE theta 1e6."""
    n, heads, kv, D = 7, 16, 4, 128
    ctx = L.uniform_u32(SEED, f"depth.ctx.{window}", n, 16384, 32768)
    positions = (ctx - 1).astype(np.uint32)
    stride = kv * D
    caps = [window if window else int(c) for c in ctx]
    ld = (heads + 2 * kv) * D + heads
    qkv = L.normal(SEED, f"depth.qkv.{window}", n * ld).reshape(n, ld)
    q_off, k_off, v_off, g_off = 0, heads * D, (heads + kv) * D, (heads + 2 * kv) * D
    qn = L.normal(SEED, "depth.qn", D, 1, 0.02)
    kn = L.normal(SEED, "depth.kn", D, 1, 0.02)
    factors = np.ones(D // 2, np.float32)
    rings_k = [L.half_normal(SEED, f"depth.k{r}.{window}", caps[r] * stride) for r in range(n)]
    rings_v = [L.half_normal(SEED, f"depth.v{r}.{window}", caps[r] * stride) for r in range(n)]
    dk = [L.DeviceBuffer.of(x) for x in rings_k]
    dv = [L.DeviceBuffer.of(x) for x in rings_v]
    tk = pointer_table([b.addr for b in dk])
    tv = pointer_table([b.addr for b in dv])
    dcap = L.DeviceBuffer.of(np.array(caps, np.uint32))
    dpos = L.DeviceBuffer.of(positions)
    from test_oracle import powf
    i = np.arange(D // 2, dtype=np.float32)
    freq = powf(1e6, np.float32(-2.0) * i / np.float32(D))
    dfreq, dfac = L.DeviceBuffer.of(freq), L.DeviceBuffer.of(factors)
    dq = L.DeviceBuffer.of(qkv)
    dqn, dkn = L.DeviceBuffer.of(qn), L.DeviceBuffer.of(kn)
    cap_items = L.lib().lfm3_attention_max_items(n, int(positions.max()))
    items = (L.AttentionItem * cap_items)()
    count = L.check(L.lib().lfm3_attention_plan(L.ptr(positions), n, window, items, cap_items))
    ditems = L.DeviceBuffer(count * C_ITEM)
    L.hip_check(L.hip().hipMemcpy(ditems.addr, L.C.addressof(items), count * C_ITEM, L.H2D))
    ws_bytes = L.lib().lfm3_attention_workspace_bytes(count, n, heads, kv, D)
    ws = L.DeviceBuffer(max(ws_bytes, 4))
    dout = L.DeviceBuffer(n * heads * D * 4)
    print(f"[depth] contexts {ctx.tolist()} window {window}: {count} items", flush=True)
    L.check(L.lib().lfm3_decode_heads_attention_ragged(
        dq.addr + 4 * q_off, dq.addr + 4 * k_off, dq.addr + 4 * v_off, ld, dq.addr + 4 * g_off,
        ld, dqn.addr, dkn.addr, dfreq.addr, 0 if window else dfac.addr, tk.addr, tv.addr,
        dpos.addr, dcap.addr, ditems.addr, count, dout.addr, heads * D, n, heads, kv, D, 1e-5,
        ws.addr, ws_bytes, None))
    L.synchronize()
    out = dout.download(np.float32, n * heads * D).reshape(n, heads * D)
    O.set_threads(8)
    try:
        for r in range(n):
            p = int(positions[r])
            want, _, _ = O.attention_step(
                qkv[r, q_off:k_off], qkv[r, k_off:v_off], qkv[r, v_off:g_off],
                qkv[r, g_off:g_off + heads], qn, kn, None if window else factors,
                O.half_to_float(rings_k[r]), O.half_to_float(rings_v[r]), heads, kv, D, p,
                caps[r], window, 1e6, bool(window), 1e-5, True)
            ok, err = within(out[r], want)
            assert ok, (r, p, err)
            slot = p % caps[r]
            gv = dv[r].download(np.uint16, caps[r] * stride).reshape(caps[r], stride)
            assert np.array_equal(gv[slot], O.float_to_half(qkv[r, v_off:g_off]))
    finally:
        O.set_threads(1)


def prompt_attention_fp64_blocked(q, gates, kc, vc, kr, vr, n, H, KH, D, P, cap, window):
    """The FP64 softmax of ops_test.cpp:142-220 over the F16-rounded keys,
    vectorized per head over all rows: keys before P from ring slot t % cap,
    the rest from the chunk; row r sees keys [first, P + r]."""
    stride = KH * D
    kc = kc.reshape(n, stride).astype(np.float64)
    vc = vc.reshape(n, stride).astype(np.float64)
    kr = kr.reshape(-1, stride).astype(np.float64)
    vr = vr.reshape(-1, stride).astype(np.float64)
    out = np.zeros((n, H * D))
    gate_div = 1.0 + np.exp(-gates.astype(np.float64))
    rows = np.arange(n)
    if window:
        # Row r: keys P + r - window + 1 .. P + r (window slots, oldest first).
        t = P + rows[:, None] - window + 1 + np.arange(window)[None, :]
        valid = t >= 0
        tc = np.clip(t, 0, None)
        own = tc >= P
        ring_idx = tc % cap
        chunk_idx = np.clip(tc - P, 0, n - 1)
        for kh in range(KH):
            ks = np.where(own[..., None], kc[chunk_idx, kh * D:(kh + 1) * D],
                          kr[ring_idx, kh * D:(kh + 1) * D])
            vs = np.where(own[..., None], vc[chunk_idx, kh * D:(kh + 1) * D],
                          vr[ring_idx, kh * D:(kh + 1) * D])
            for h in range(kh * (H // KH), (kh + 1) * (H // KH)):
                s = np.einsum("rwd,rd->rw", ks, q[:, h * D:(h + 1) * D].astype(np.float64))
                s = np.where(valid, s / math.sqrt(D), -np.inf)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                p /= p.sum(axis=1, keepdims=True)
                out[:, h * D:(h + 1) * D] = np.einsum("rw,rwd->rd", p, vs) / gate_div[:, h:h + 1]
        return out
    keys = np.concatenate([kr[np.arange(P) % cap], kc])     # P + n keys in order
    vals = np.concatenate([vr[np.arange(P) % cap], vc])
    mask = np.arange(P + n)[None, :] <= (P + rows)[:, None]
    for h in range(H):
        kh = h // (H // KH)
        s = (q[:, h * D:(h + 1) * D].astype(np.float64) @ keys[:, kh * D:(kh + 1) * D].T)
        s = np.where(mask, s / math.sqrt(D), -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, h * D:(h + 1) * D] = (p @ vals[:, kh * D:(kh + 1) * D]) / gate_div[:, h:h + 1]
    return out


@pytest.mark.parametrize("window", [0, 256])
def test_prompt_attention_at_depth(window):
    """512 prompt rows at depth 24576, 16/4 heads x 128 (the pass of config
    5): spans split and merged on the global layer; max |error| < 1e-3."""
    from test_gpu_prefill import data, run_prompt_attention
    n, H, KH, D, P = 512, 16, 4, 128, 24576
    cap = window if window else P + n
    stride = KH * D
    q = data(n * H * D, 0.7).reshape(n, H * D)
    gates = data(n * H, 0.7).reshape(n, H)
    kbits = O.float_to_half(data(n * stride, 0.5))
    vbits = O.float_to_half(data(n * stride, 0.9))
    ckbits = L.half_normal(SEED, f"pdepth.k.{window}", cap * stride)
    cvbits = L.half_normal(SEED, f"pdepth.v.{window}", cap * stride)
    print(f"[depth] prompt attention n {n} P {P} window {window}", flush=True)
    out, ws_bytes = run_prompt_attention(q, gates, kbits, vbits, ckbits, cvbits, n, H, KH, D, P,
                                         cap, window)
    if not window:
        assert ws_bytes > 0
    want = prompt_attention_fp64_blocked(q, gates, O.half_to_float(kbits),
                                         O.half_to_float(vbits), O.half_to_float(ckbits),
                                         O.half_to_float(cvbits), n, H, KH, D, P, cap, window)
    assert np.all(np.isfinite(out))
    err = float(np.max(np.abs(out - want)))
    print(f"max |error| {err:.3g}")
    assert err < 1e-3


def test_session_forward_full_dims_at_depth():
    """Session::Forward (engine.cpp:882-938) of a 513-token prompt on a
    full-dims session at depth 24576 (injected state; 512 rows and then a
    one-row chunk, the pass of config 5 plus its continuation): FP16 prompt
    projections, packed convolution, prompt heads and MFMA prompt attention
    at depth, gated as session_test.cpp:120-143 gates a batched prompt
    against serial steps (KL < 1e-6, max |logit| < 0.02, the same argmax):
    against the oracle stepping the same tokens (layer-major steps,
    bit-identical to token steps), and against the same tokens run one
    decode round each on the GPU (the reference test's own pair)."""
    depth, n = 24576, 513
    dims = L.Dims(context=depth + 1024)
    w = L.synth_weights(dims, seed=SEED)
    gm, om = L.Model(w), O.Model(dims, w)
    g, serial = gm.session(depth + 640), gm.session(depth + 640)
    o = om.session(depth + 640, f16=True)
    inject_both(g, o, dims, SEED, 300, depth)
    oh = oracle_twin(om, o, depth + 640)
    L.inject_synth_state(serial, dims, SEED, 300, depth)
    tokens = L.uniform_u32(SEED, "depth.prompt.513", n, 0, dims.vocab - 1)
    print(f"[depth] Session::Forward {n} tokens at depth {depth}", flush=True)
    got = g.forward(tokens)
    O.set_threads(max(1, min(16, len(__import__("os").sched_getaffinity(0)))))
    try:
        want = oracle_prompt(o, tokens)
        want_prompt = oracle_prompt(oh, tokens, prompt=True)
    finally:
        O.set_threads(1)
    oh.close()
    prompt_gate_pair(got, want, want_prompt, f"{n}-token pass")
    assert g.position == o.position == depth + n
    gs_logits = None
    for t in tokens:
        gs_logits = gm.forward_batch([serial], np.array([t], np.uint32))[0]
    # the reference test's own pair: the pass against the same tokens one
    # decode round each (FP32 GEMVs), at the FP32 oracle's gate
    err = float(np.max(np.abs(got.astype(np.float64) - gs_logits)))
    kl = kl_divergence(gs_logits, got)
    print(f"{n}-token pass vs {n} GPU decode rounds: max |Δ| {err:.3g}, kl {kl:.3g}", flush=True)
    assert err < 0.02 and kl < kl_divergence(want, want_prompt) + 5e-7
    assert int(np.argmax(got)) == int(np.argmax(gs_logits))
    assert serial.position == depth + n
    # One decode round continues from the prompt's state.
    tok = L.uniform_u32(SEED, "depth.next", 1, 0, dims.vocab - 1)
    got = gm.forward_batch([g], tok)[0]
    O.set_threads(16)
    try:
        want = o.step(int(tok[0]))
    finally:
        O.set_threads(1)
    assert float(np.max(np.abs(got - want))) < 0.02
    same_greedy(got, want, "decode round after the pass")
    for x in (g, serial, o):
        x.close()
    gm.close()
    om.close()


def test_mixed_round_full_dims_at_depth():
    """Config 5 as one workload, the bench's own: one lfm3_scheduler_round of
    the full-dims model with 7 decode sessions at contexts uniform in
    [16384, 32768] beside a 512-token pass at depth 24576 (the two on two
    streams), against the oracle: every decode row's logits within 2e-3 with
    the same greedy id, and the pass's last logits at session_test.cpp:
    120-143's gate (the oracle's layer-major steps of the same tokens)."""
    depth, n = 24576, 512
    ctx = L.uniform_u32(SEED, "bench.mixed.ctx", 7, 16384, 32768)
    dims = L.Dims(context=int(ctx.max()) + 64)
    w = L.synth_weights(dims, seed=SEED)
    gm, om = L.Model(w), O.Model(dims, w)
    print(f"[depth] mixed round: contexts {ctx.tolist()}, pass of {n} at {depth}", flush=True)
    gs, os_ = [], []
    for sid, c in enumerate(ctx):
        g = gm.session(int(c) + 8)
        o = om.session(int(c) + 8, f16=True)
        inject_both(g, o, dims, SEED, 200 + sid, int(c) - 1)
        gs.append(g)
        os_.append(o)
    gp = gm.session(depth + n)
    op = om.session(depth + n, f16=True)
    inject_both(gp, op, dims, SEED, 100, depth)
    oph = oracle_twin(om, op, depth + n)
    toks = L.uniform_u32(SEED, "bench.mixed.tokens", 7, 0, dims.vocab - 1)
    ptoks = L.uniform_u32(SEED, "bench.pass.tokens", n, 0, dims.vocab - 1)
    ids, logits, plog = gm.scheduler_round(gs, toks, gp, ptoks, want_logits=True)
    O.set_threads(max(1, min(16, len(__import__("os").sched_getaffinity(0)))))
    try:
        for i, o in enumerate(os_):
            want = o.step(int(toks[i]))
            err = same_greedy(logits[i], want, f"decode row {i} ctx {int(ctx[i])}")
            assert err < 2e-3, (i, err)
            assert ids[i] == O.argmax(want)
            assert gs[i].position == o.position == int(ctx[i])
        prompt_gate_pair(plog, op.steps(ptoks), oph.steps(ptoks, prompt_path=True),
                         f"{n}-token pass at depth {depth}")
    finally:
        O.set_threads(1)
    assert gp.position == op.position == depth + n
    for x in gs + os_ + [gp, op, oph]:
        x.close()
    gm.close()
    om.close()
