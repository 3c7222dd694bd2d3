"""Prompt chunk rows on the GPU against the CPU oracle and the reference's
own formulas, through the C-ABI: packed ragged prompt convolution (outputs
and history bit-exact against decode steps), prompt heads (Q/K norm, RoPE,
F16 K/V rows), the K/V ring store (slots exact), and causal MFMA prompt
attention (ops_test.cpp:142-220's FP64 formula, gate 1e-3 for prompts).

Gates follow tests/ops_test.cpp: prompt attention 1e-3 absolute against
FP64 over F16-rounded K/V; convolution history exact; ring contents exact."""
import math

import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from test_oracle import data, powf

pytestmark = pytest.mark.gpu
SEED = L.SEED


def host_u32(values):
    return np.ascontiguousarray(values, np.uint32)


def host_ptrs(addrs):
    return (L.C.c_void_p * len(addrs))(*addrs)


# ------------------------------------------------------------ convolution

def run_conv_prompt(p, ldp, taps, hists, begins, rows, H, Lw, update=True):
    dp, dt = L.DeviceBuffer.of(p), L.DeviceBuffer.of(taps)
    dh = [L.DeviceBuffer.of(h) for h in hists]
    n = int(sum(rows))
    dy = L.DeviceBuffer(n * H * 4)
    b, r = host_u32(begins), host_u32(rows)
    L.check(L.lib().lfm3_conv_prompt(dp.addr, ldp, dt.addr, host_ptrs([d.addr for d in dh]),
                                     L.ptr(b), L.ptr(r), len(rows), dy.addr, H, H, Lw,
                                     int(update), None))
    L.synchronize()
    y = dy.download(np.float32, n * H).reshape(n, H)
    return y, [d.download(np.float32, H * (Lw - 1)) for d in dh]


@pytest.mark.parametrize("Lw", [7, 4, 20])
def test_conv_prompt_packed_segments_bit_exact(Lw):
    """The packed ragged prefill variant: prompts of 512, 37, 300 and 1 rows
    in one launch, each continuing its own session history; every output
    and history equals sequential decode steps (the oracle) bit for bit.
    Width 20 reaches past one 16-row group, where the history moves in a
    launch of its own."""
    H = 2048
    seg_rows = [512, 37, 300, 1]
    begins = np.cumsum([0] + seg_rows[:-1])
    n = sum(seg_rows)
    ldp = 3 * H + 8
    p = L.normal(SEED, f"pconv.p{Lw}", n * ldp).reshape(n, ldp)
    taps = L.normal(SEED, f"pconv.taps{Lw}", H * Lw, 0, 0.1)
    hists = [L.normal(SEED, f"pconv.h{s}.{Lw}", H * (Lw - 1)) for s in range(len(seg_rows))]
    y, got_h = run_conv_prompt(p, ldp, taps, hists, begins, seg_rows, H, Lw)
    for s, (b, r) in enumerate(zip(begins, seg_rows)):
        h = hists[s]
        for i in range(b, b + r):
            want, h = O.conv_step(p[i, :3 * H], taps, h, H, Lw)
            assert np.array_equal(y[i], want), (s, i)
        assert np.array_equal(got_h[s], h), s


@pytest.mark.parametrize("n", [1, 8, 9, 15, 16, 29, 32, 33, 128, 512])
def test_conv_prompt_reference_vectors(n):
    """ops_test.cpp:90-116: H = 37, L = 7, sin-formula inputs; outputs within
    1e-7 of the FP64 sequential scan and the history exact."""
    H, Lw = 37, 7
    proj = data(n * 3 * H)
    weight = data(H * Lw, 0.3)
    history = data(H * (Lw - 1))
    expected = np.zeros((n, H))
    expected_h = history.copy()
    for c in range(H):
        seq = [float(history[c * (Lw - 1) + j]) for j in range(Lw - 1)]
        for t in range(n):
            seq.append(float(np.float32(proj[t * 3 * H + c] * proj[t * 3 * H + 2 * H + c])))
            s = sum(float(weight[c * Lw + j]) * seq[t + j] for j in range(Lw))
            expected[t, c] = s * float(proj[t * 3 * H + H + c])
        for j in range(Lw - 1):
            expected_h[c * (Lw - 1) + j] = seq[n + j]
    y, got_h = run_conv_prompt(proj.reshape(n, 3 * H), 3 * H, weight, [history], [0], [n], H, Lw)
    assert np.max(np.abs(y - expected)) <= 1e-7
    assert np.array_equal(got_h[0], expected_h)


def test_conv_prompt_without_history_update_leaves_it():
    H, Lw, n = 256, 7, 20
    p = L.normal(SEED, "pconv.keep.p", n * 3 * H).reshape(n, 3 * H)
    taps = L.normal(SEED, "pconv.keep.t", H * Lw, 0, 0.1)
    hist = L.normal(SEED, "pconv.keep.h", H * (Lw - 1))
    y, got_h = run_conv_prompt(p, 3 * H, taps, [hist], [0], [n], H, Lw, update=False)
    assert np.array_equal(got_h[0], hist)
    h = hist
    for i in range(n):
        want, h = O.conv_step(p[i], taps, h, H, Lw)
        assert np.array_equal(y[i], want)


@pytest.mark.parametrize("H,n,skip,Lw", [(2048, 512, 0, 7), (2048, 300, 13, 7), (2048, 37, 0, 7),
                                          (256, 20, 5, 7), (256, 5, 2, 7), (2048, 100, 50, 4),
                                          (2048, 40, 9, 5), (96, 17, 0, 2)])
def test_conv_prompt_half_is_conv_then_half_rows(H, n, skip, Lw):
    """The convolution fused with its output's FP16 row-scaled activations
    against the oracle's decode steps followed by its FP16 row conversion
    (hip/q8_prefill.hpp:27-51): rows skip.. of the FP16 output, their
    scales and the new history bit-exact; chunk tails zero; nothing written
    past the live rows or the chunk tail. Covers a prompt shorter than the
    window (the history moves within it), a skip past the first row block,
    other widths and a hidden size that is not a whole chunk."""
    p = L.normal(SEED, f"pch.p.{H}.{n}", n * 3 * H).reshape(n, 3 * H)
    taps = L.normal(SEED, f"pch.t.{H}.{Lw}", H * Lw, 0, 0.1)
    hist = L.normal(SEED, f"pch.h.{H}.{Lw}", H * (Lw - 1))
    lda = (H + 63) // 64 * 64 + 64
    live = n - skip
    dp, dt, dh = L.DeviceBuffer.of(p), L.DeviceBuffer.of(taps), L.DeviceBuffer.of(hist)
    sentinel = np.full((live + 1) * lda, 0x7e00, np.uint16)
    da = L.DeviceBuffer.of(sentinel)
    ds = L.DeviceBuffer.of(np.full(live + 1, -1.0, np.float32))
    L.check(L.lib().lfm3_conv_prompt_half(dp.addr, 3 * H, dt.addr, dh.addr, n, skip, da.addr,
                                          lda, ds.addr, H, Lw, 1, None))
    L.synchronize()
    a = da.download(np.uint16, (live + 1) * lda).reshape(live + 1, lda)
    scale = ds.download(np.float32, live + 1)
    y = np.zeros((n, H), np.float32)
    h = hist
    for i in range(n):
        y[i], h = O.conv_step(p[i], taps, h, H, Lw)
    inputs, exps = O.half_rows(y[skip:])
    want = O.float_to_half(np.ldexp(y[skip:], exps[:, None]).astype(np.float32))
    assert np.array_equal(a[:live, :H], want)
    assert np.array_equal(scale[:live], np.ldexp(np.float32(1), -exps).astype(np.float32))
    padded = (H + 63) // 64 * 64
    assert not a[:live, H:padded].any()
    assert np.all(a[:live, padded:] == 0x7e00) and np.all(a[live] == 0x7e00)
    assert scale[live] == -1.0
    assert np.array_equal(dh.download(np.float32, H * (Lw - 1)), h)


# ------------------------------------------------------------------ heads

@pytest.mark.parametrize("heads,kv,D", [(16, 4, 128), (32, 8, 64)])
@pytest.mark.parametrize("sliding", [False, True])
def test_prompt_heads(heads, kv, D, sliding):
    """Rows at position + r: per-head RMSNorm and RoPE (theta 1e6, masked
    tail factors on global layers, ops_test.cpp:117-141) against the oracle;
    V rows stored bit-exact, K rows the exact F16 rounding of the rotated
    rows written back."""
    n, position, theta, eps = 77, 3000, 1e6, 1e-5
    ld = (heads + 2 * kv) * D + heads
    qkv = L.normal(SEED, f"ph.qkv.{D}.{sliding}", n * ld).reshape(n, ld)
    q_off, k_off, v_off = 0, heads * D, (heads + kv) * D
    qn = L.normal(SEED, "ph.qn", D, 1, 0.02)
    kn = L.normal(SEED, "ph.kn", D, 1, 0.02)
    factors = np.ones(D // 2, np.float32)
    factors[D // 4:] = 1e30
    i = np.arange(D // 2, dtype=np.float32)
    freq = powf(theta, np.float32(-2.0) * i / np.float32(D))
    dq = L.DeviceBuffer.of(qkv)
    dqn, dkn = L.DeviceBuffer.of(qn), L.DeviceBuffer.of(kn)
    dfreq, dfac = L.DeviceBuffer.of(freq), L.DeviceBuffer.of(factors)
    k16, v16 = L.DeviceBuffer(n * kv * D * 2), L.DeviceBuffer(n * kv * D * 2)
    L.check(L.lib().lfm3_prompt_heads(dq.addr, dq.addr + 4 * k_off, dq.addr + 4 * v_off, ld,
                                      dqn.addr, dkn.addr, dfreq.addr,
                                      0 if sliding else dfac.addr, k16.addr, v16.addr, n,
                                      heads, kv, D, position, eps, None))
    L.synchronize()
    got = dq.download(np.float32, n * ld).reshape(n, ld)
    gk = k16.download(np.uint16, n * kv * D).reshape(n, kv * D)
    gv = v16.download(np.uint16, n * kv * D).reshape(n, kv * D)
    fac = None if sliding else factors
    for r in range(n):
        pos = position + r
        for h in range(heads):
            want = O.rope(O.norm(qkv[r, h * D:(h + 1) * D], qn, eps), D, pos, theta, sliding, fac)
            np.testing.assert_allclose(got[r, h * D:(h + 1) * D], want, rtol=1e-4, atol=2e-5)
        for h in range(kv):
            kr = O.rope(O.norm(qkv[r, k_off + h * D:k_off + (h + 1) * D], kn, eps), D, pos,
                        theta, sliding, fac)
            got_k = got[r, k_off + h * D:k_off + (h + 1) * D]
            np.testing.assert_allclose(got_k, kr, rtol=1e-4, atol=2e-5)
            # the stored K row is exactly the F16 rounding of the rotated row
            assert np.array_equal(gk[r, h * D:(h + 1) * D], O.float_to_half(got_k))
        assert np.array_equal(gv[r], O.float_to_half(qkv[r, v_off:v_off + kv * D]))


# ------------------------------------------------------------- ring store

@pytest.mark.parametrize("n,position,capacity", [(5, 0, 256), (37, 250, 256), (512, 3000, 256),
                                                 (300, 1000, 4096), (1, 255, 256)])
def test_store_kv_ring_slots(n, position, capacity):
    """Row r lands in slot (position + r) % capacity; only the last
    min(n, capacity) rows are written; every other slot keeps its bits."""
    stride = 2 * 128
    chunk_k = L.half_normal(SEED, f"skv.k.{n}", n * stride)
    chunk_v = L.half_normal(SEED, f"skv.v.{n}", n * stride)
    ring_k = L.half_normal(SEED, f"skv.rk.{capacity}", capacity * stride)
    ring_v = L.half_normal(SEED, f"skv.rv.{capacity}", capacity * stride)
    dck, dcv = L.DeviceBuffer.of(chunk_k), L.DeviceBuffer.of(chunk_v)
    drk, drv = L.DeviceBuffer.of(ring_k), L.DeviceBuffer.of(ring_v)
    L.check(L.lib().lfm3_store_kv(dck.addr, dcv.addr, drk.addr, drv.addr, n, stride, position,
                                  capacity, None))
    L.synchronize()
    want_k = ring_k.reshape(capacity, stride).copy()
    want_v = ring_v.reshape(capacity, stride).copy()
    for r in range(n):
        want_k[(position + r) % capacity] = chunk_k.reshape(n, stride)[r]
        want_v[(position + r) % capacity] = chunk_v.reshape(n, stride)[r]
    assert np.array_equal(drk.download(np.uint16, capacity * stride).reshape(capacity, stride),
                          want_k)
    assert np.array_equal(drv.download(np.uint16, capacity * stride).reshape(capacity, stride),
                          want_v)


# -------------------------------------------------------- prompt attention

def prompt_attention_fp64(q, gates, k, v, ck, cv, n, H, KH, D, P, cap, window):
    """ops_test.cpp:142-220: FP64 softmax over the F16-rounded keys of each
    row; keys at or after P come from the chunk, earlier ones from the ring."""
    stride = KH * D
    out = np.zeros((n, H * D))
    kc, vc = k.reshape(n, stride).astype(np.float64), v.reshape(n, stride).astype(np.float64)
    kr, vr = ck.reshape(-1, stride).astype(np.float64), cv.reshape(-1, stride).astype(np.float64)
    for row in range(n):
        last = P + row
        first = max(0, last + 1 - window) if window else 0
        ts = np.arange(first, last + 1)
        keys = np.where((ts >= P)[:, None], kc[np.clip(ts - P, 0, n - 1)], kr[ts % cap])
        vals = np.where((ts >= P)[:, None], vc[np.clip(ts - P, 0, n - 1)], vr[ts % cap])
        for h in range(H):
            kh = h // (H // KH)
            s = keys[:, kh * D:(kh + 1) * D] @ q[row, h * D:(h + 1) * D].astype(np.float64)
            s /= math.sqrt(D)
            p = np.exp(s - s.max())
            p /= p.sum()
            out[row, h * D:(h + 1) * D] = (p @ vals[:, kh * D:(kh + 1) * D]) / (
                1 + math.exp(-float(gates[row, h])))
    return out


def run_prompt_attention(q, gates, kbits, vbits, ckbits, cvbits, n, H, KH, D, P, cap, window,
                         ldq=None, ldg=None):
    ldq = ldq or H * D
    ldg = ldg or H
    dq = L.DeviceBuffer.of(np.ascontiguousarray(q, np.float32))
    dg = L.DeviceBuffer.of(np.ascontiguousarray(gates, np.float32))
    dk, dv = L.DeviceBuffer.of(kbits), L.DeviceBuffer.of(vbits)
    dck, dcv = L.DeviceBuffer.of(ckbits), L.DeviceBuffer.of(cvbits)
    ws_bytes = L.lib().lfm3_prompt_attention_workspace_bytes(n, H, D, P, window)
    ws = L.DeviceBuffer(max(ws_bytes, 4))
    dout = L.DeviceBuffer(n * H * D * 4)
    L.check(L.lib().lfm3_prompt_attention(dq.addr, ldq, dk.addr, dv.addr, dg.addr, ldg,
                                          dck.addr, dcv.addr, dout.addr, H * D, n, H, KH, D, P,
                                          cap, window, ws.addr, ws_bytes, None))
    L.synchronize()
    return dout.download(np.float32, n * H * D).reshape(n, H * D), ws_bytes


def reference_case(n, window, P, H, KH, D=128):
    """ops_test.cpp:146-155 inputs: sin-formula Q, K, V, gates and ring."""
    cap = window if window else P + n
    stride = KH * D
    q = data(n * H * D, 0.7).reshape(n, H * D)
    gates = data(n * H, 0.7).reshape(n, H)
    kbits = O.float_to_half(data(n * stride, 0.5))
    vbits = O.float_to_half(data(n * stride, 0.9))
    ckbits = O.float_to_half(data(cap * stride, 0.6))
    cvbits = O.float_to_half(data(cap * stride, 0.8))
    return q, gates, kbits, vbits, ckbits, cvbits, cap


CASES = ([(n, w, 259, 4, 2) for n in (2, 8, 9, 15, 16, 29, 32, 33, 128, 512) for w in (0, 256)]
         + [(40, 0, 17000, 4, 2), (40, 256, 17000, 4, 2)]
         + [(n, w, 3000, 16, 4) for n in (77, 512) for w in (0, 256)])


@pytest.mark.parametrize("n,window,P,H,KH", CASES)
def test_prompt_attention_reference_vectors(n, window, P, H, KH):
    """ops_test.cpp:142-253 for n > 1: short and long (split) histories, the
    sliding ring, and the model's 16 query / 4 KV heads; max |error| < 1e-3
    against the FP64 formula; then the sliding ring holds exactly the
    chunk's rounded rows (StoreKV)."""
    D = 128
    q, gates, kbits, vbits, ckbits, cvbits, cap = reference_case(n, window, P, H, KH, D)
    out, ws_bytes = run_prompt_attention(q, gates, kbits, vbits, ckbits, cvbits, n, H, KH, D, P,
                                         cap, window)
    if P + n > 2048 and not window:
        assert ws_bytes > 0  # spans split and merged
    want = prompt_attention_fp64(q, gates, O.half_to_float(kbits), O.half_to_float(vbits),
                                 O.half_to_float(ckbits), O.half_to_float(cvbits), n, H, KH, D,
                                 P, cap, window)
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out - want)) < 1e-3
    if window:
        stride = KH * D
        dck, dcv = L.DeviceBuffer.of(ckbits), L.DeviceBuffer.of(cvbits)
        dk, dv = L.DeviceBuffer.of(kbits), L.DeviceBuffer.of(vbits)
        L.check(L.lib().lfm3_store_kv(dk.addr, dv.addr, dck.addr, dcv.addr, n, stride, P, cap,
                                      None))
        L.synchronize()
        ring_k = ckbits.reshape(cap, stride).copy()
        for r in range(n):
            ring_k[(P + r) % cap] = kbits.reshape(n, stride)[r]
        assert np.array_equal(dck.download(np.uint16, cap * stride).reshape(cap, stride), ring_k)


@pytest.mark.parametrize("n,window,P,H,KH,D", [(512, 0, 24576, 16, 4, 128), (512, 256, 24576, 16, 4, 128),
                                               (77, 0, 3000, 16, 4, 128), (16, 0, 259, 4, 2, 128),
                                               (37, 256, 300, 32, 8, 64), (200, 0, 0, 32, 8, 64)])
def test_prompt_attention_half_is_attention_then_half_rows(n, window, P, H, KH, D):
    """The attention output as the output projection's FP16 rows: every
    row equals lfm3_prompt_attention's FP32 row converted by the oracle's
    FP16 row rule (hip/q8_prefill.hpp:27-51) bit for bit, with its scale,
    for a global history split into spans (depth 24576), the sliding
    window (one span), a short history and the 32 x 64 head shape; nothing
    is written past the row's heads x dim halves."""
    cap = window if window else P + n
    stride = KH * D
    tag = f"{n}.{window}.{P}.{H}.{D}"
    q = L.normal(SEED, f"pah.q.{tag}", n * H * D).reshape(n, H * D)
    gates = L.normal(SEED, f"pah.g.{tag}", n * H).reshape(n, H)
    kbits = L.half_normal(SEED, f"pah.k.{tag}", n * stride)
    vbits = L.half_normal(SEED, f"pah.v.{tag}", n * stride)
    ckbits = L.half_normal(SEED, f"pah.ck.{tag}", cap * stride)
    cvbits = L.half_normal(SEED, f"pah.cv.{tag}", cap * stride)
    print(f"[prompt attention half] {tag}", flush=True)
    out, _ = run_prompt_attention(q, gates, kbits, vbits, ckbits, cvbits, n, H, KH, D, P, cap,
                                  window)
    lda = H * D + 64
    dq = L.DeviceBuffer.of(np.ascontiguousarray(q, np.float32))
    dg = L.DeviceBuffer.of(np.ascontiguousarray(gates, np.float32))
    dk, dv = L.DeviceBuffer.of(kbits), L.DeviceBuffer.of(vbits)
    dck, dcv = L.DeviceBuffer.of(ckbits), L.DeviceBuffer.of(cvbits)
    ws_bytes = L.lib().lfm3_prompt_attention_half_workspace_bytes(n, H, D, P, window)
    assert ws_bytes >= n * H * (D + 2) * 4
    ws = L.DeviceBuffer(ws_bytes)
    da = L.DeviceBuffer.of(np.full((n + 1) * lda, 0x7e00, np.uint16))
    ds = L.DeviceBuffer.of(np.full(n + 1, -1.0, np.float32))
    L.check(L.lib().lfm3_prompt_attention_half(dq.addr, H * D, dk.addr, dv.addr, dg.addr, H,
                                               dck.addr, dcv.addr, da.addr, lda, ds.addr, n, H,
                                               KH, D, P, cap, window, ws.addr, ws_bytes, None))
    L.synchronize()
    a = da.download(np.uint16, (n + 1) * lda).reshape(n + 1, lda)
    scale = ds.download(np.float32, n + 1)
    _, exps = O.half_rows(out)
    want = O.float_to_half(np.ldexp(out, exps[:, None]).astype(np.float32))
    assert np.array_equal(a[:n, :H * D], want)
    assert np.array_equal(scale[:n], np.ldexp(np.float32(1), -exps).astype(np.float32))
    assert np.all(a[:n, H * D:] == 0x7e00) and np.all(a[n] == 0x7e00) and scale[n] == -1.0


@pytest.mark.parametrize("n,window,P,cap,D", [(9, 256, 37, 46, 128), (8, 0, 40, 50, 128),
                                               (5, 256, 30, 35, 64), (33, 0, 20, 60, 128),
                                               (70, 256, 100, 171, 64), (40, 256, 300, 340, 128)])
def test_prompt_attention_short_rings(n, window, P, cap, D):
    """Sessions whose context is below the window (or a tile) keep rings of
    fewer than 64 slots or of an odd size: ring slots t % cap past a tile's
    worth of keys, tiles straddling the first chunk key, against the FP64
    formula at 1e-3."""
    H, KH = 16, 4
    stride = KH * D
    tag = f"{n}.{window}.{P}.{cap}.{D}"
    q = L.normal(SEED, f"pring.q.{tag}", n * H * D).reshape(n, H * D)
    gates = L.normal(SEED, f"pring.g.{tag}", n * H).reshape(n, H)
    kbits = L.half_normal(SEED, f"pring.k.{tag}", n * stride)
    vbits = L.half_normal(SEED, f"pring.v.{tag}", n * stride)
    ckbits = L.half_normal(SEED, f"pring.ck.{tag}", cap * stride)
    cvbits = L.half_normal(SEED, f"pring.cv.{tag}", cap * stride)
    print(f"[prompt attention] short ring {tag}", flush=True)
    out, _ = run_prompt_attention(q, gates, kbits, vbits, ckbits, cvbits, n, H, KH, D, P, cap,
                                  window)
    want = prompt_attention_fp64(q, gates, O.half_to_float(kbits), O.half_to_float(vbits),
                                 O.half_to_float(ckbits), O.half_to_float(cvbits), n, H, KH, D,
                                 P, cap, window)
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out - want)) < 1e-3


@pytest.mark.parametrize("window", [0, 256])
@pytest.mark.parametrize("P", [0, 700])
def test_prompt_attention_baseline_heads_dim64(window, P):
    """The nominal LFM3-1.7B heads (32 query / 8 KV x 64) on random inputs,
    against the FP64 formula and, row by row, the oracle's FP32 attention
    read over the same keys (reference.cpp:117-144), both within the
    prompt gate of 1e-3."""
    n, H, KH, D = 96, 32, 8, 64
    stride = KH * D
    cap = window if window else P + n
    q = L.normal(SEED, f"pa64.q.{P}", n * H * D).reshape(n, H * D)
    gates = L.normal(SEED, f"pa64.g.{P}", n * H).reshape(n, H)
    kbits = L.half_normal(SEED, f"pa64.k.{P}", n * stride)
    vbits = L.half_normal(SEED, f"pa64.v.{P}", n * stride)
    ckbits = L.half_normal(SEED, f"pa64.ck.{P}.{window}", max(cap, 1) * stride)
    cvbits = L.half_normal(SEED, f"pa64.cv.{P}.{window}", max(cap, 1) * stride)
    out, _ = run_prompt_attention(q, gates, kbits, vbits, ckbits, cvbits, n, H, KH, D, P,
                                  max(cap, 1), window)
    want = prompt_attention_fp64(q, gates, O.half_to_float(kbits), O.half_to_float(vbits),
                                 O.half_to_float(ckbits), O.half_to_float(cvbits), n, H, KH, D,
                                 P, max(cap, 1), window)
    assert np.max(np.abs(out - want)) < 1e-3
    # The oracle reads one row at a time from a ring holding every key of
    # the row (history then chunk), so each prompt row is one decode read.
    full = P + n
    keys_k = np.zeros((full, stride), np.float32)
    keys_v = np.zeros((full, stride), np.float32)
    ring_k = O.half_to_float(ckbits).reshape(-1, stride)
    ring_v = O.half_to_float(cvbits).reshape(-1, stride)
    for t in range(P):
        keys_k[t], keys_v[t] = ring_k[t % max(cap, 1)], ring_v[t % max(cap, 1)]
    keys_k[P:] = O.half_to_float(kbits).reshape(n, stride)
    keys_v[P:] = O.half_to_float(vbits).reshape(n, stride)
    for r in range(0, n, 7):
        ref = O.attention_read(q[r], gates[r], keys_k.reshape(-1), keys_v.reshape(-1), H, KH, D,
                               P + r, full, window)
        # the prompt gate (F16 Q and probabilities), as against FP64
        assert np.max(np.abs(out[r] - ref)) < 1e-3, r


def test_prompt_attention_strided_rows_from_projection():
    """q and gate read from the fused projection rows (stride ld), as the
    engine lays them out; same result as contiguous rows."""
    n, H, KH, D, P = 64, 16, 4, 128, 500
    ld = (H + 2 * KH) * D + H + 4
    proj = L.normal(SEED, "pa.proj", n * ld).reshape(n, ld)
    q = proj[:, :H * D]
    gates = proj[:, (H + 2 * KH) * D:(H + 2 * KH) * D + H]
    stride = KH * D
    kbits = L.half_normal(SEED, "pa.proj.k", n * stride)
    vbits = L.half_normal(SEED, "pa.proj.v", n * stride)
    ckbits = L.half_normal(SEED, "pa.proj.ck", (P + n) * stride)
    cvbits = L.half_normal(SEED, "pa.proj.cv", (P + n) * stride)
    dproj = L.DeviceBuffer.of(proj)
    dk, dv = L.DeviceBuffer.of(kbits), L.DeviceBuffer.of(vbits)
    dck, dcv = L.DeviceBuffer.of(ckbits), L.DeviceBuffer.of(cvbits)
    dout = L.DeviceBuffer(n * H * D * 4)
    L.check(L.lib().lfm3_prompt_attention(dproj.addr, ld, dk.addr, dv.addr,
                                          dproj.addr + 4 * (H + 2 * KH) * D, ld, dck.addr,
                                          dcv.addr, dout.addr, H * D, n, H, KH, D, P, P + n, 0,
                                          None, 0, None))
    L.synchronize()
    strided = dout.download(np.float32, n * H * D).reshape(n, H * D)
    dense, _ = run_prompt_attention(q, gates, kbits, vbits, ckbits, cvbits, n, H, KH, D, P,
                                    P + n, 0)
    assert np.array_equal(strided, dense)
