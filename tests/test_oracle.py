"""Pins the CPU oracle before anything is checked against it.

Sources of truth, none of them a retyping of the oracle's own loops:
  * the reference's operator tests (tests/ops_test.cpp): deterministic
    inputs Data(n, s) = s * sin(0.73 i), formula Q8_0 weights, FP64
    expectations and their tolerances (projection 1e-4, conv 1e-7 with
    exact history, RoPE 2e-5, decode attention 2e-6);
  * numpy's IEEE binary16 conversions;
  * closed forms (RMSNorm of a constant row, RoPE at position 0 and its
    norm preservation, attention over identical keys);
  * an independent float64 numpy model (tests/numpy_model.py) for the
    composition of the full step.
"""
import math

import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from numpy_model import NumpySession


_libm = __import__("ctypes").CDLL("libm.so.6")
_libm.powf.restype = __import__("ctypes").c_float
_libm.powf.argtypes = [__import__("ctypes").c_float] * 2


def powf(base, exponents):
    """glibc powf, the std::pow(float, float) of reference.cpp and ops_test.cpp."""
    return np.array([_libm.powf(base, float(e)) for e in np.asarray(exponents, np.float32)],
                    np.float32)


def data(n, scale=0.1):
    """ops_test.cpp:30-35: scale * sin(float(i) * 0.73F), in float32."""
    i = np.arange(n, dtype=np.float32)
    return (np.float32(scale) * np.sin((i * np.float32(0.73)).astype(np.float32))).astype(np.float32)


def formula_q8(M, K):
    """ops_test.cpp:48-53: d = 0x2400 + 32 (i % 10), q = (17 i + 37 j) % 255 - 127."""
    blocks = M * K // 32
    out = np.zeros((blocks, 34), np.uint8)
    i = np.arange(blocks)
    d = (0x2400 + 32 * (i % 10)).astype(np.uint16)
    out[:, 0:2] = d.view(np.uint8).reshape(blocks, 2)
    j = np.arange(32)
    q = ((i[:, None] * 17 + j[None, :] * 37) % 255 - 127).astype(np.int8)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


# ------------------------------------------------------------------ halves

def test_half_to_float_all_patterns():
    bits = np.arange(65536, dtype=np.uint16)
    got = O.half_to_float(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_round_to_nearest_even():
    rng = np.random.default_rng(1)
    cases = [rng.standard_normal(200000).astype(np.float32),
             (rng.standard_normal(50000) * 1e-5).astype(np.float32),   # subnormal range
             (rng.standard_normal(50000) * 7e4).astype(np.float32),    # overflow edge
             np.array([0.0, -0.0, 65504, 65520, 65519.99, 6.1e-5, 5.96e-8, 2.98e-8,
                       2.99e-8, np.inf, -np.inf], np.float32)]
    # Exact ties between adjacent halves round to even.
    h = np.arange(0x3c00, 0x3c40, dtype=np.uint16).view(np.float16).astype(np.float32)
    cases.append(((h[:-1].astype(np.float64) + h[1:]) / 2).astype(np.float32))
    for x in cases:
        got = O.float_to_half(x)
        want = x.astype(np.float16).view(np.uint16)
        assert np.array_equal(got, want)


# ------------------------------------------------------- rows and products

def test_decode_row_is_d_times_q():
    M, K = 37, 2048
    w = formula_q8(M, K)
    t = O.q8_tensor(w, M, K)
    want = L.q8_dequant(w, M, K).astype(np.float32)
    for r in (0, 1, 17, 36):
        assert np.array_equal(O.decode_row(t, r), want[r])


@pytest.mark.parametrize("n", [1, 8, 9])
def test_mat_matches_reference_projection_vectors(n):
    """ops_test.cpp:46-89 at FP32 input rows: FP64 expectation, gate 1e-4."""
    M, K = 37, 2048
    w = formula_q8(M, K)
    x = data(n * K, 0.07).reshape(n, K)
    want = x.astype(np.float64) @ L.q8_dequant(w, M, K).T
    got = O.mat(O.q8_tensor(w, M, K), x)
    assert np.max(np.abs(got - want)) < 1e-4


def test_mat_transposition_and_row_order():
    """A non-square, asymmetric case: swapping operands or rows fails."""
    rng = np.random.default_rng(2)
    M, K = 48, 96
    w = L.q8(5, "mat", M, K)
    x = rng.standard_normal(K).astype(np.float32)
    want = L.q8_dequant(w, M, K) @ x.astype(np.float64)
    got = O.mat(O.q8_tensor(w, M, K), x)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


# -------------------------------------------------------------------- norm

def test_norm_fp64_and_constant_row():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(2048).astype(np.float32) * 3
    w = (1 + 0.02 * rng.standard_normal(2048)).astype(np.float32)
    got = O.norm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 ** 2) + 1e-5) * w
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)
    c = np.full(256, -2.5, np.float32)
    got = O.norm(c, np.ones(256, np.float32), 1e-5)
    closed = -2.5 / math.sqrt(6.25 + 1e-5)
    np.testing.assert_allclose(got, closed, rtol=1e-6)


# -------------------------------------------------------------------- rope

@pytest.mark.parametrize("n", [1, 8, 33])
def test_rope_matches_reference_rotary_vectors(n):
    """ops_test.cpp:117-141: D = 128, 3 heads, P = 12001, factors 1e30 on
    pairs 32..63 (unchanged), gate 2e-5."""
    D, H, P = 128, 3, 12001
    x = data(n * H * D).reshape(n, H * D)
    factors = np.ones(D // 2, np.float32)
    factors[32:] = 1e30
    for row in range(n):
        got = O.rope(x[row], D, P + row, 1e6, False, factors).reshape(H, D)
        xr = x[row].reshape(H, D).astype(np.float64)
        i = np.arange(D // 2)
        freq = powf(1e6, np.float32(-2.0) * i.astype(np.float32) / np.float32(D))
        ang = (np.float32(P + row) * freq / factors).astype(np.float32).astype(np.float64)
        want = np.concatenate([xr[:, :64] * np.cos(ang) - xr[:, 64:] * np.sin(ang),
                               xr[:, 64:] * np.cos(ang) + xr[:, :64] * np.sin(ang)], 1)
        assert np.max(np.abs(got - want)) < 2e-5
        assert np.array_equal(got[:, 32:64], x[row].reshape(H, D)[:, 32:64])


def test_rope_position_zero_and_norm():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(4 * 64).astype(np.float32)
    assert np.array_equal(O.rope(x, 64, 0, 1e4, True, None), x)
    y = O.rope(x, 64, 777, 1e4, True, None).reshape(4, 64)
    xr = x.reshape(4, 64)
    pair_in = xr[:, :32] ** 2 + xr[:, 32:] ** 2
    pair_out = y[:, :32].astype(np.float64) ** 2 + y[:, 32:] ** 2
    np.testing.assert_allclose(pair_out, pair_in, rtol=1e-5)


# -------------------------------------------------------------------- conv

@pytest.mark.parametrize("n", [1, 8, 9, 33])
def test_conv_matches_reference_scan(n):
    """ops_test.cpp:90-116: FP64 sequential scan, outputs 1e-7, history exact."""
    H, Lw = 37, 7
    proj = data(n * 3 * H).reshape(n, 3 * H)
    taps = data(H * Lw, 0.3)
    hist = data(H * (Lw - 1))
    expected_hist = hist.copy()
    expected = np.zeros((n, H))
    for c in range(H):
        seq = [float(v) for v in hist[c * (Lw - 1):(c + 1) * (Lw - 1)]]
        for t in range(n):
            seq.append(float(np.float32(proj[t, c] * proj[t, 2 * H + c])))
            s = sum(float(taps[c * Lw + j]) * seq[t + j] for j in range(Lw))
            expected[t, c] = s * float(proj[t, H + c])
        expected_hist[c * (Lw - 1):(c + 1) * (Lw - 1)] = seq[n:n + Lw - 1]
    h = hist
    for t in range(n):
        y, h = O.conv_step(proj[t], taps, h, H, Lw)
        assert np.max(np.abs(y - expected[t])) < 1e-7
    assert np.array_equal(h, expected_hist)


# --------------------------------------------------------------- attention

def attention_fp64(q, gate, ck, cv, H, KH, D, P, cap, window):
    first = max(0, P + 1 - window) if window else 0
    out = np.zeros(H * D)
    stride = KH * D
    for h in range(H):
        kh = h // (H // KH)
        ts = np.arange(first, P + 1)
        keys = ck.reshape(-1, stride)[ts % cap, kh * D:(kh + 1) * D].astype(np.float64)
        vals = cv.reshape(-1, stride)[ts % cap, kh * D:(kh + 1) * D].astype(np.float64)
        s = keys @ q[h * D:(h + 1) * D].astype(np.float64) / math.sqrt(D)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h * D:(h + 1) * D] = (p @ vals) / (1 + math.exp(-float(gate[h])))
    return out


@pytest.mark.parametrize("P,H,KH,window", [(259, 4, 2, 0), (259, 4, 2, 256), (4999, 4, 2, 0),
                                           (4999, 4, 2, 256), (3000, 16, 4, 0), (3000, 16, 4, 256)])
def test_attention_matches_reference_decode_vectors(P, H, KH, window):
    """ops_test.cpp:142-220 at n = 1: F16-rounded K/V, FP64 softmax, gate 2e-6."""
    D = 128
    cap = window if window else P + 1
    stride = KH * D
    q = data(H * D, 0.7)
    gates = data(H, 0.7)
    ck = O.half_to_float(O.float_to_half(data(cap * stride, 0.6)))
    cv = O.half_to_float(O.float_to_half(data(cap * stride, 0.8)))
    ck[(P % cap) * stride:(P % cap + 1) * stride] = O.half_to_float(O.float_to_half(data(stride, 0.5)))
    cv[(P % cap) * stride:(P % cap + 1) * stride] = O.half_to_float(O.float_to_half(data(stride, 0.9)))
    got = O.attention_read(q, gates, ck, cv, H, KH, D, P, cap, window)
    want = attention_fp64(q, gates, ck, cv, H, KH, D, P, cap, window)
    assert np.max(np.abs(got - want)) < 2e-6


def test_attention_identical_keys_average_values():
    """Equal scores: the output is the mean of the values, gated."""
    H, KH, D, P = 4, 2, 64, 40
    cap = P + 1
    ck = np.tile(np.linspace(-1, 1, KH * D, dtype=np.float32), cap)
    cv = np.random.default_rng(5).standard_normal(cap * KH * D).astype(np.float32)
    q = np.random.default_rng(6).standard_normal(H * D).astype(np.float32)
    gate = np.zeros(H, np.float32)
    got = O.attention_read(q, gate, ck, cv, H, KH, D, P, cap, 0).reshape(H, D)
    mean = cv.reshape(cap, KH, D).astype(np.float64).mean(0)
    for h in range(H):
        np.testing.assert_allclose(got[h], mean[h // 2] / 2, rtol=1e-5, atol=1e-6)


def test_swiglu_and_argmax():
    rng = np.random.default_rng(7)
    g = rng.standard_normal(1000).astype(np.float32) * 4
    u = rng.standard_normal(1000).astype(np.float32)
    want = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    np.testing.assert_allclose(O.swiglu(g, u), want, rtol=1e-6, atol=1e-7)
    x = np.array([1, 3, 2, 3, -1], np.float32)
    assert O.argmax(x) == 1  # first of equal maxima, as std::max_element


# ------------------------------------------------------------ composition

def tiny_dims(**kw):
    base = dict(hidden=128, intermediate=192, vocab=300, context=64, heads=4, head_dim=64,
                kv_heads=2, window=8, pattern="CSGCG")
    base.update(kw)
    return L.Dims(**base)


def test_step_matches_independent_fp64_model():
    dims = tiny_dims()
    w = L.synth_weights(dims, seed=11)
    model = O.Model(dims, w)
    # FP32 K/V on both sides: binary16 rounding would turn FP32 noise near a
    # rounding boundary into half-ulp jumps (the switch is pinned below).
    s = model.session(64, f16=False)
    ref = NumpySession(dims, w, 64, f16=False)
    tokens = L.uniform_u32(11, "tokens", 14, 0, dims.vocab - 1)
    for tok in tokens:   # crosses the sliding window (8) several times
        got = s.step(int(tok))
        want = ref.step(int(tok))
        scale = np.max(np.abs(want))
        assert np.max(np.abs(got - want)) < 2e-5 * max(1.0, scale)
    s.close()
    model.close()


def test_state_injection_reproduces_stepping():
    """A session restored at position p with the state of another session
    continues identically (bit for bit)."""
    dims = tiny_dims()
    w = L.synth_weights(dims, seed=12)
    model = O.Model(dims, w)
    a = model.session(64)
    for tok in range(9):
        a.step(tok * 7 % dims.vocab, logits=False)
    b = model.session(64)
    for i in range(dims.n_layers):
        if dims.layer_type(i) == L.LAYER_CONV:
            b.conv(i)[:] = a.conv(i)
        else:
            b.k(i)[:] = a.k(i)
            b.v(i)[:] = a.v(i)
    b.set_position(a.position)
    assert np.array_equal(a.step(5), b.step(5))
    with pytest.raises(ValueError):
        a.step(dims.vocab)       # token out of range is refused
    assert a.position == 10
    model.close()


def test_parallel_rows_and_heads_give_identical_steps():
    """The row-parallel matrix-vector products and head-parallel attention
    (orc_set_threads) keep every output row's sequential sum: logits are
    bit-identical to the serial reference loops for any thread count."""
    dims = tiny_dims()
    w = L.synth_weights(dims, seed=14)
    model = O.Model(dims, w)
    runs = []
    for threads in (1, 3, 8):
        O.set_threads(threads)
        s = model.session(64)
        runs.append([s.step(tok * 5 % dims.vocab) for tok in range(6)])
        s.close()
    O.set_threads(1)
    assert O.threads() == 1
    for other in runs[1:]:
        for a, b in zip(runs[0], other):
            assert np.array_equal(a, b)
    model.close()


@pytest.mark.parametrize("n,start", [(1, 0), (13, 0), (21, 9)])
def test_layer_major_prompt_steps_are_the_token_steps(n, start):
    """orc_session_steps (n rows a layer at a time) against n calls of the
    token step: the same logits and the same state, bit for bit, across the
    sliding window (8) and from a session already at a position."""
    dims = tiny_dims()
    w = L.synth_weights(dims, seed=15)
    model = O.Model(dims, w)
    O.set_threads(3)
    try:
        a, b = model.session(64), model.session(64)
        for tok in range(start):
            a.step(tok * 11 % dims.vocab, logits=False)
            b.step(tok * 11 % dims.vocab, logits=False)
        tokens = L.uniform_u32(15, f"steps.{n}", n, 0, dims.vocab - 1)
        want = None
        for tok in tokens:
            want = a.step(int(tok))
        got = b.steps(tokens)
        assert np.array_equal(got, want)
        assert a.position == b.position == start + n
        for i in range(dims.n_layers):
            if dims.layer_type(i) == L.LAYER_CONV:
                assert np.array_equal(a.conv(i), b.conv(i))
            else:
                assert np.array_equal(a.k(i), b.k(i)) and np.array_equal(a.v(i), b.v(i))
        # refused without moving the state: past the context, a bad token
        with pytest.raises(ValueError):
            b.steps(np.zeros(64, np.uint32))
        with pytest.raises(ValueError):
            b.steps(np.array([0, dims.vocab], np.uint32))
        assert b.position == start + n
        a.close()
        b.close()
    finally:
        O.set_threads(1)
    model.close()


def _tensor(entry):
    data, typ, cols, rows = entry
    return O.Tensor(data.ctypes.data, typ, cols, rows)


def prune_rows(dims, n):
    """engine.cpp:304-323 restated: (live_in, live_out) per layer."""
    live_in, live_out = [n] * dims.n_layers, [n] * dims.n_layers
    need = 1
    for i in reversed(range(dims.n_layers)):
        t = dims.layer_type(i)
        if t == L.LAYER_SLIDING:
            break
        live_out[i] = min(n, need)
        if t == L.LAYER_FULL:
            break
        need = min(n, need + dims.conv_width - 1)
        live_in[i] = need
    return live_in, live_out


def composed_prompt_chunk(dims, w, state, tokens, position):
    """A prompt chunk of n rows with the reference's prompt-path numerics,
    composed in Python from the oracle's pinned primitives (norm, RoPE, mat,
    conv step, half rows, both attention reads, SwiGLU), layer by layer:
    projections over 16 rows or more read FP16 row-scaled inputs
    (hip/ops.hpp:32, q8_prefill.hpp:27-51), the live row counts follow
    trailing-row pruning (engine.cpp:304-323), attention reads through the
    prompt read except a full-attention layer left with one row (FP32
    decode read). state holds per layer the conv history or the FP32 (K, V)
    rings (binary16 values), updated in place. Returns the last logits."""
    H, D, n = dims.hidden, dims.head_dim, len(tokens)
    live_in, live_out = prune_rows(dims, n)

    def inp(rows, live):
        rows = np.asarray(rows, np.float32)
        return O.half_rows(rows)[0] if live >= 16 else rows

    norm_rows = lambda rows, wt: np.stack([O.norm(r, wt, dims.eps) for r in rows])
    x = np.stack([O.decode_row(_tensor(w.globals[0]), int(t)) for t in tokens])
    for i in range(dims.n_layers):
        t = w.layers[i]
        z = inp(norm_rows(x, t[0][0]), live_in[i])
        if dims.layer_type(i) == L.LAYER_CONV:
            p = O.mat(_tensor(t[8]), z)
            y = np.empty((n, H), np.float32)
            for r in range(n):
                y[r], state[i] = O.conv_step(p[r], t[7][0], state[i], H, dims.conv_width)
            out = O.mat(_tensor(t[9]), inp(y, live_out[i]))
        else:
            sliding = dims.layer_type(i) == L.LAYER_SLIDING
            q, k, v, g = (O.mat(_tensor(t[j]), z) for j in (10, 11, 12, 15))
            ck, cv = state[i]
            stride = dims.kv_heads * D
            cap = ck.size // stride
            theta = dims.theta_swa if sliding else dims.theta
            prompt_read = not (live_out[i] == 1 and not sliding)
            a = np.empty((n, dims.heads * D), np.float32)
            for r in range(n):
                pos = position + r
                qr = np.concatenate([O.norm(h, t[13][0], dims.eps)
                                     for h in q[r].reshape(dims.heads, D)])
                kr = np.concatenate([O.norm(h, t[14][0], dims.eps)
                                     for h in k[r].reshape(dims.kv_heads, D)])
                qr = O.rope(qr, D, pos, theta, sliding, w.globals[3][0])
                kr = O.rope(kr, D, pos, theta, sliding, w.globals[3][0])
                slot = pos % cap
                ck[slot * stride:(slot + 1) * stride] = O.half_to_float(O.float_to_half(kr))
                cv[slot * stride:(slot + 1) * stride] = O.half_to_float(O.float_to_half(v[r]))
                read = O.attention_read_prompt if prompt_read else O.attention_read
                a[r] = read(qr, g[r], ck, cv, dims.heads, dims.kv_heads, D, pos, cap,
                            dims.window if sliding else 0)
            out = O.mat(_tensor(t[16]), inp(a, live_out[i]))
        if t[2] is not None and t[2][0] is not None:
            out = norm_rows(out, t[2][0])
        x = (x + out).astype(np.float32)
        z = inp(norm_rows(x, t[1][0]), live_out[i])
        h = O.swiglu(O.mat(_tensor(t[4]), z), O.mat(_tensor(t[5]), z))
        out = O.mat(_tensor(t[6]), inp(h, live_out[i]))
        if t[3] is not None and t[3][0] is not None:
            out = norm_rows(out, t[3][0])
        x = (x + out).astype(np.float32)
    last = O.norm(x[-1], w.globals[2][0], dims.eps)
    return O.mat(_tensor(w.globals[0]), last)


def test_prompt_read_matches_fp64_with_f16_points():
    """orc_attention_read_prompt against float64 numpy with the prompt
    path's three rounding points (F16 of q log2(e)/sqrt(D), F16 probabilities
    against the row maximum, the sum over the rounded probabilities): within
    2e-6 of the output scale, while the FP32 read differs by far more."""
    rng = np.random.default_rng(5)
    H, KH, D, P, cap = 8, 2, 64, 300, 512
    q = rng.standard_normal(H * D).astype(np.float32)
    gate = rng.standard_normal(H).astype(np.float32)
    ck = O.half_to_float(O.float_to_half(rng.standard_normal(cap * KH * D).astype(np.float32)))
    cv = O.half_to_float(O.float_to_half(rng.standard_normal(cap * KH * D).astype(np.float32)))
    for window in (0, 32):
        got = O.attention_read_prompt(q, gate, ck, cv, H, KH, D, P, cap, window)
        fp32 = O.attention_read(q, gate, ck, cv, H, KH, D, P, cap, window)
        first = max(0, P + 1 - window) if window else 0
        keys = ck.reshape(cap, KH, D).astype(np.float64)
        vals = cv.reshape(cap, KH, D).astype(np.float64)
        ts = np.arange(first, P + 1) % cap
        scale = np.float32(np.float32(1) / np.sqrt(np.float32(D))) * np.float32(1.4426950408889634)
        want = np.empty(H * D)
        for h in range(H):
            kh = h // (H // KH)
            qs = (q[h * D:(h + 1) * D] * scale).astype(np.float32).astype(np.float16)
            sc = keys[ts, kh] @ qs.astype(np.float64)
            p = np.exp2(sc - sc.max()).astype(np.float32).astype(np.float16).astype(np.float64)
            want[h * D:(h + 1) * D] = (p @ vals[ts, kh] / p.sum()) / (1 + np.exp(-float(gate[h])))
        sc_out = np.max(np.abs(want))
        err = np.max(np.abs(got - want)) / sc_out
        err32 = np.max(np.abs(fp32 - want)) / sc_out
        assert err < 2e-6 and err32 > 20 * err, (window, err, err32)


@pytest.mark.parametrize("n,pattern", [(5, "CSGCG"), (19, "CSGCG"), (40, "CSGCG"),
                                       (40, "GSCCC"), (2, "CSGCG")])
def test_prompt_path_steps_are_the_composed_chunk(n, pattern):
    """orc_session_steps with prompt_path against the same chunk composed in
    Python from the pinned primitives: the same logits bit for bit. Chunks
    below 16 rows (FP32 projections, F16 attention), above (FP16 row inputs),
    a last layer that is global (one live row: FP32 decode read, FP32 FFN)
    and trailing convolutions (7 then 13 live rows), across the sliding
    window (8); and different logits from the FP32 steps."""
    dims = tiny_dims(pattern=pattern)
    w = L.synth_weights(dims, seed=17)
    model = O.Model(dims, w)
    a, b = model.session(64), model.session(64)
    for tok in range(3):                 # start from position 3
        a.step(tok, logits=False)
        b.step(tok, logits=False)
    state = {}
    for i in range(dims.n_layers):
        if dims.layer_type(i) == L.LAYER_CONV:
            state[i] = a.conv(i).copy()
        else:
            state[i] = (a.k(i).copy(), a.v(i).copy())
    tokens = L.uniform_u32(17, f"prompt.{n}.{pattern}", n, 0, dims.vocab - 1)
    got = a.steps(tokens, prompt_path=True)
    full = b.steps(tokens)
    want = composed_prompt_chunk(dims, w, state, tokens, 3)
    assert np.array_equal(got, want)
    assert not np.array_equal(got, full)
    for i in range(dims.n_layers):
        if dims.layer_type(i) == L.LAYER_CONV:
            assert np.array_equal(a.conv(i), state[i])
        else:
            assert np.array_equal(a.k(i), state[i][0]) and np.array_equal(a.v(i), state[i][1])
    model.close()


def test_isa_builds_give_identical_steps():
    """The x86-64-v3 and x86-64-v4 builds of the oracle (vectorized only
    across independent sums) step to identical logits."""
    import ctypes
    if not O._has_avx512() or not __import__("os").path.exists(O.LIB_V4_PATH):
        pytest.skip("no AVX-512 on this CPU")
    dims = tiny_dims()
    w = L.synth_weights(dims, seed=16)
    model = O.Model(dims, w)
    outs = []
    for path in (O.LIB_PATH, O.LIB_V4_PATH):
        h = ctypes.CDLL(path)
        h.orc_model_create.restype = ctypes.c_void_p
        h.orc_model_create.argtypes = [ctypes.POINTER(O.Config), ctypes.POINTER(O.Tensor),
                                       ctypes.c_size_t]
        h.orc_session_create.restype = ctypes.c_void_p
        h.orc_session_create.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int]
        h.orc_session_step.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p,
                                       ctypes.c_void_p]
        h.orc_session_destroy.argtypes = [ctypes.c_void_p]
        h.orc_model_destroy.argtypes = [ctypes.c_void_p]
        m = h.orc_model_create(ctypes.byref(model.config), model._tensors,
                               len(model._tensors))
        s = h.orc_session_create(m, 64, 1)
        rows = []
        for tok in range(12):
            out = np.empty(dims.vocab, np.float32)
            assert h.orc_session_step(s, tok * 13 % dims.vocab, out.ctypes.data, None) == 0
            rows.append(out)
        h.orc_session_destroy(s)
        h.orc_model_destroy(m)
        outs.append(rows)
    for a, b in zip(*outs):
        assert np.array_equal(a, b)
    model.close()


def test_step_row_with_embedding_row_is_the_token_step():
    """ForwardBatchInputs' row path (engine.cpp:1217-1299 copies the row over
    the embedding): the step from the token's dequantized embedding row is
    the token step, bit for bit; the hidden row is the final-normed row the
    logits come from (the tied head applied to it gives the logits)."""
    dims = tiny_dims()
    w = L.synth_weights(dims, seed=13)
    model = O.Model(dims, w)
    a, b = model.session(64), model.session(64)
    emb = L.q8_dequant(w.globals[0][0], dims.vocab, dims.hidden).astype(np.float32)
    for tok in (3, 200, 17, 299, 0, 42, 8, 91, 150):
        want = a.step(tok)
        got, hidden = b.step_row(emb[tok])
        assert np.array_equal(got, want)
        head = emb.astype(np.float64) @ hidden.astype(np.float64)
        assert np.max(np.abs(head - want)) < 1e-4 * max(1.0, np.max(np.abs(want)))
    # a row that is no embedding row moves the state differently
    _, h1 = a.step_row(np.full(dims.hidden, 0.25, np.float32))
    _, h2 = b.step_row(np.full(dims.hidden, -0.25, np.float32))
    assert not np.array_equal(h1, h2)
    _, none = b.step_row(np.ones(dims.hidden, np.float32), logits=False)
    assert none.shape == (dims.hidden,) and a.position == b.position - 1
    model.close()


def test_f16_switch_stores_binary16_rows():
    dims = tiny_dims()
    w = L.synth_weights(dims, seed=13)
    model = O.Model(dims, w)
    s = model.session(64, f16=True)
    s.step(3, logits=False)
    for i in range(dims.n_layers):
        if dims.layer_type(i) != L.LAYER_CONV:
            row = s.k(i)[:dims.kv_heads * dims.head_dim]
            assert np.array_equal(row, row.astype(np.float16).astype(np.float32))
            assert np.any(row != 0)
    model.close()


def test_half_rows_matches_binary16_and_exponent_rule():
    """Prompt activations (q8_prefill.hpp:27-51): the row maximum lands in
    [2^14, 2^15) after scaling, each element is numpy's binary16 rounding of
    the scaled value, a zero row keeps exponent 0, and tiny and large rows
    keep 11 significant bits relative to the maximum."""
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (6, 300)).astype(np.float32)
    x[1] *= 1e-6
    x[2] *= 3e4
    x[3] = 0
    x[4, 7] = -65504.0 * 4
    inputs, exps = O.half_rows(x)
    for r in range(6):
        m = np.abs(x[r]).max()
        if m == 0:
            assert exps[r] == 0 and not inputs[r].any()
            continue
        scaled = np.ldexp(m, exps[r])
        assert 2.0 ** 14 <= scaled < 2.0 ** 15
        want = np.ldexp(np.ldexp(x[r], exps[r]).astype(np.float16).astype(np.float32), -exps[r])
        assert np.array_equal(inputs[r], want)
        assert np.max(np.abs(inputs[r] - x[r])) <= m * 2.0 ** -11
