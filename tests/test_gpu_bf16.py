"""BF16 weights on the GPU: the exact BF16 x FP32 GEMV (lfm3_bf16_gemv),
the BF16 embedding gather, and a BF16 model through the engine's decode
rounds and prompt passes, against the oracle's BF16 rows (weights.cpp:116-117)
and float64.

Gates:
  * the GEMV against float64 over the widened weights: |y - y64| <= 4e-6 *
    sum_k |w_k x_k| (the three-part split makes every product exact, so
    only FP32 summation remains; a dropped lo part would leave 2^-16 of the
    row's magnitude, a dropped mid part 2^-8); and within() of the
    oracle's scalar FP32 product;
  * an identity weight gives y == x bit for bit (the split reassembles x);
  * the embedding rows bit-exact;
  * model rounds and prompts at the same gates as the Q8_0 model (logits
    within 2e-3 of the oracle per decode step; prompt logits within 0.02)
    and greedy ids equal, unconditionally (prompts at session_test.cpp:
    120-143's gate: KL < 1e-6, max < 0.02, the same argmax).
"""
import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import inject_state, prompt_gate, same_greedy, within

pytestmark = pytest.mark.gpu
SEED = L.SEED


class Bf16Matrix:
    def __init__(self, h, rows, cols, pairs=None):
        if pairs is None:
            n = L.lib().lfm3_bf16_tiled_bytes(rows, cols)
            t = np.zeros(n // 2, np.uint16)
            L.check(L.lib().lfm3_bf16_pack_host(L.ptr(h), rows, cols, L.ptr(t), 0, 1))
        else:  # gate/up interleaved by row tile
            g, u = pairs
            n = L.lib().lfm3_bf16_tiled_bytes(2 * (-(-rows // 16)) * 16, cols)
            t = np.zeros(n // 2, np.uint16)
            L.check(L.lib().lfm3_bf16_pack_host(L.ptr(g), rows, cols, L.ptr(t), 0, 2))
            L.check(L.lib().lfm3_bf16_pack_host(L.ptr(u), rows, cols, L.ptr(t), 1, 2))
        self.buf = L.DeviceBuffer.of(t)
        self.rows, self.cols = rows, cols


def run(m, x, parts=1, swiglu=False, ldx=None):
    B, K = x.shape
    ldx = ldx or K
    host = np.zeros((B, ldx), np.float32)
    host[:, :K] = x
    dx = L.DeviceBuffer.of(host)
    dy = L.DeviceBuffer(parts * B * m.rows * 4)
    L.check(L.lib().lfm3_bf16_gemv(m.buf.addr, m.rows, m.cols, dx.addr, ldx, dy.addr, m.rows, B,
                                   parts, 1 if swiglu else 0, None))
    L.synchronize()
    y = dy.download(np.float32, parts * B * m.rows).reshape(parts, B, m.rows)
    return y.astype(np.float64).sum(axis=0) if parts > 1 else y[0]


def check_fp64(y, h, rows, cols, x):
    w64 = L.bf16_to_f32(h).reshape(rows, cols).astype(np.float64)
    x64 = x.astype(np.float64)
    want = x64 @ w64.T
    scale = np.abs(x64) @ np.abs(w64).T
    bad = np.abs(y - want) > 4e-6 * scale + 1e-30
    assert not bad.any(), float(np.max(np.abs(y - want) / (scale + 1e-30)))


@pytest.mark.parametrize("M,K,B", [(8192, 2048, 1), (8192, 2048, 8), (2048, 7680, 8),
                                   (128000, 2048, 4), (37, 96, 5), (3088, 2048, 8),
                                   (2048, 2048, 17), (1024, 256, 512), (16, 32, 1)])
def test_bf16_gemv_exact_products(M, K, B):
    h = L.bf16(SEED, f"bfg.{M}x{K}", M, K)
    m = Bf16Matrix(h, M, K)
    x = (3.0 * L.normal(SEED, f"bfg.x.{M}x{K}.{B}", B * K)).reshape(B, K).astype(np.float32)
    y = run(m, x)
    check_fp64(y, h, M, K, x)
    if M * K <= 8192 * 2048 and B <= 8:
        ok, err = within(y, O.mat(O.bf16_tensor(h, M, K), x))
        assert ok, err
    parts = L.lib().lfm3_bf16_gemv_parts(M, K, B)
    for p in sorted({2, parts}):
        if p <= K // 32:
            check_fp64(run(m, x, parts=p), h, M, K, x)


def test_bf16_identity_reassembles_fp32_inputs():
    """y = I x: the three BF16 parts of every FP32 input add back to it."""
    K = 256
    eye = np.zeros((K, K), np.float32)
    np.fill_diagonal(eye, 1.0)
    m = Bf16Matrix(L.to_bf16(eye), K, K)
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((8, K)) * np.exp2(rng.integers(-20, 20, (8, K)))).astype(np.float32)
    x[0, :4] = [1.0 + 2.0 ** -9 + 2.0 ** -17 + 2.0 ** -23, -np.float32(np.pi), 3e-30, 7e30]
    y = run(m, x)
    assert np.array_equal(y.view(np.uint32), x.view(np.uint32))


def test_bf16_swiglu_pairs():
    F, H, B = 768, 512, 8
    g, u = L.bf16(SEED, "bfs.g", F, H), L.bf16(SEED, "bfs.u", F, H)
    m = Bf16Matrix(None, F, H, pairs=(g, u))
    x = L.normal(SEED, "bfs.x", B * H).reshape(B, H).astype(np.float32)
    y = run(m, x, swiglu=True)
    gt, ut = O.bf16_tensor(g, F, H), O.bf16_tensor(u, F, H)
    want = np.stack([O.swiglu(O.mat(gt, x[b]), O.mat(ut, x[b])) for b in range(B)])
    ok, err = within(y, want)
    assert ok, err


def test_bf16_embed_rows():
    V, H, n = 1000, 256, 9
    h = L.bf16(SEED, "bfe", V, H)
    m = Bf16Matrix(h, V, H)
    toks = np.array([0, 999, 17, 16, 15, 500, 3, 1000, 2], np.uint32)   # 1000: past the table
    dt = L.DeviceBuffer.of(toks)
    out = L.DeviceBuffer(n * H * 4)
    L.check(L.lib().lfm3_bf16_embed(m.buf.addr, V, H, dt.addr, None, n, out.addr, None))
    L.synchronize()
    got = out.download(np.float32, n * H).reshape(n, H)
    table = L.bf16_to_f32(h).reshape(V, H)
    for i, t in enumerate(toks):
        want = table[t] if t < V else np.zeros(H, np.float32)
        assert np.array_equal(got[i], want), i


def test_bf16_gemv_refusals():
    lib = L.lib()
    buf = L.DeviceBuffer(1 << 16)
    assert lib.lfm3_bf16_gemv(buf.addr, 16, 48, buf.addr, 48, buf.addr, 16, 1, 1, 0,
                              None) == L.E_INVALID      # cols % 32
    assert lib.lfm3_bf16_gemv(buf.addr, 16, 64, buf.addr, 62, buf.addr, 16, 1, 1, 0,
                              None) == L.E_INVALID      # ldx % 4
    assert lib.lfm3_bf16_gemv(buf.addr, 16, 64, buf.addr, 64, buf.addr, 16, 1, 2, 1,
                              None) == L.E_INVALID      # parts with SwiGLU
    assert lib.lfm3_bf16_gemv(buf.addr, 16, 64, buf.addr, 64, buf.addr, 16, 1, 3, 0,
                              None) == L.E_INVALID      # more parts than column blocks


def small_dims(**kw):
    base = dict(hidden=256, intermediate=512, vocab=1000, context=1024, heads=8, head_dim=128,
                kv_heads=2, window=32, pattern="CSGCCSCG")
    base.update(kw)
    return L.Dims(**base)


@pytest.mark.parametrize("dims_kw", [{}, dict(heads=8, kv_heads=4, head_dim=64)])
def test_bf16_model_rounds_match_oracle(dims_kw):
    dims = small_dims(**dims_kw)
    n = 8
    w = L.synth_weights(dims, seed=81, bf16_weights=True)
    gm, om = L.Model(w), O.Model(dims, w)
    positions = L.uniform_u32(SEED, "bf.pos", n, 0, 600)
    gs, os_ = [], []
    for sid, p in enumerate(positions):
        g, o = gm.session(1024), om.session(1024, f16=True)
        inject_state(g, o, dims, 81, sid, int(p))
        gs.append(g)
        os_.append(o)
    worst = 0.0
    for step in range(3):
        toks = L.uniform_u32(SEED, f"bf.tok{step}", n, 0, dims.vocab - 1)
        if step == 1:
            ids = gm.forward_batch_greedy(gs, toks)
            logits = np.stack([s.read_logits() for s in gs])
            assert list(ids) == [O.argmax(r) for r in logits]
        else:
            logits = gm.forward_batch(gs, toks)
        for i in range(n):
            want = os_[i].step(int(toks[i]))
            err = same_greedy(logits[i], want, f"step {step} row {i}")
            worst = max(worst, err)
            assert err < 2e-3, (step, i, err)
    print(f"BF16 model: max |logit - oracle| = {worst:.3g}")
    for s in gs:
        s.close()
    gm.close()
    om.close()


@pytest.mark.parametrize("n", [1, 5, 40, 600])
def test_bf16_prompt_matches_oracle_steps(n):
    dims = small_dims()
    w = L.synth_weights(dims, seed=82, bf16_weights=True)
    gm, om = L.Model(w), O.Model(dims, w)
    g, o = gm.session(1024), om.session(1024, f16=True)
    inject_state(g, o, dims, 82, 0, 97)
    tokens = L.uniform_u32(SEED, f"bf.prompt.{n}", n, 0, dims.vocab - 1)
    got = g.forward(tokens)
    want = None
    for t in tokens:
        want = o.step(int(t))
    prompt_gate(got, want, f"BF16 {n}-token prompt")
    assert g.position == o.position == 97 + n
    # logits on demand after a round without the head
    tok = np.array([7], np.uint32)
    gm.forward_batch_inputs([g], tok, [None], want_logits=False)
    want = o.step(7)
    assert float(np.max(np.abs(g.read_logits() - want))) < 0.02
    g.close()
    gm.close()
    om.close()


def test_bf16_and_q8_matrices_do_not_mix():
    dims = small_dims()
    w = L.synth_weights(dims, seed=83, bf16_weights=True)
    q = L.synth_weights(dims, seed=83)
    w.layers[2][6] = q.layers[2][6]      # one Q8_0 down projection
    with pytest.raises(L.LFM3Error) as e:
        L.Model(w)
    assert e.value.status == L.E_INVALID
