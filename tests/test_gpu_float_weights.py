"""F16 and F32 weights on the GPU (the float formats the reference binds
besides Q8_0 and BF16, weights.cpp:30-37): lfm3_float_gemv, the float
embedding gather, and F16 / F32 models through decode rounds and prompt
passes, against float64 and the oracle's F16 / F32 rows
(weights.cpp:101-125).

Gates:
  * the GEMV against float64 over the widened weights: |y - y64| <=
    4e-6 * sum_k |w_k x_k| (every weight and input splits exactly into BF16
    parts, so every product is exact and only FP32 summation remains; a
    dropped weight part would leave 2^-8 of the row's magnitude);
  * an identity weight gives y == x bit for bit;
  * BF16 through lfm3_float_gemv equals lfm3_bf16_gemv bit for bit;
  * the embedding rows bit-exact;
  * model rounds and prompts at the BF16 model's gates (logits within 2e-3
    of the oracle per decode step; prompts at session_test.cpp:120-143's
    gate: KL < 1e-6, max < 0.02, the same argmax), greedy ids equal,
    unconditionally.
"""
import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import inject_state, prompt_gate, same_greedy, within

pytestmark = pytest.mark.gpu
SEED = L.SEED
TYPES = {"f16": L.TYPE_F16, "f32": L.TYPE_F32}


def synth(type_id, name, rows, cols, std=0.0116):
    return (L.f16 if type_id == L.TYPE_F16 else L.f32 if type_id == L.TYPE_F32 else L.bf16)(
        SEED, name, rows, cols, std)


class FloatMatrix:
    def __init__(self, type_id, data, rows, cols, pairs=None):
        lib = L.lib()
        if pairs is None:
            n = lib.lfm3_float_tiled_bytes(type_id, rows, cols)
            t = np.zeros(n, np.uint8)
            L.check(lib.lfm3_float_pack_host(type_id, L.ptr(data), rows, cols, L.ptr(t), 0, 1))
        else:
            g, u = pairs
            n = lib.lfm3_float_tiled_bytes(type_id, 2 * (-(-rows // 16)) * 16, cols)
            t = np.zeros(n, np.uint8)
            L.check(lib.lfm3_float_pack_host(type_id, L.ptr(g), rows, cols, L.ptr(t), 0, 2))
            L.check(lib.lfm3_float_pack_host(type_id, L.ptr(u), rows, cols, L.ptr(t), 1, 2))
        self.buf = L.DeviceBuffer.of(t)
        self.type, self.rows, self.cols = type_id, rows, cols


def run(m, x, parts=1, swiglu=False, generic=True):
    B, K = x.shape
    dx = L.DeviceBuffer.of(np.ascontiguousarray(x, np.float32))
    dy = L.DeviceBuffer(parts * B * m.rows * 4)
    if generic:
        L.check(L.lib().lfm3_float_gemv(m.type, m.buf.addr, m.rows, m.cols, dx.addr, K, dy.addr,
                                        m.rows, B, parts, 1 if swiglu else 0, None))
    else:
        L.check(L.lib().lfm3_bf16_gemv(m.buf.addr, m.rows, m.cols, dx.addr, K, dy.addr, m.rows,
                                       B, parts, 1 if swiglu else 0, None))
    L.synchronize()
    y = dy.download(np.float32, parts * B * m.rows).reshape(parts, B, m.rows)
    return y.astype(np.float64).sum(axis=0) if parts > 1 else y[0]


def check_fp64(y, w32, x):
    w64, x64 = w32.astype(np.float64), x.astype(np.float64)
    want = x64 @ w64.T
    scale = np.abs(x64) @ np.abs(w64).T
    bad = np.abs(y - want) > 4e-6 * scale + 1e-30
    assert not bad.any(), float(np.max(np.abs(y - want) / (scale + 1e-30)))


@pytest.mark.parametrize("kind", sorted(TYPES))
@pytest.mark.parametrize("M,K,B", [(8192, 2048, 8), (2048, 7680, 3), (37, 96, 5), (16, 32, 1),
                                   (1024, 256, 40)])
def test_float_gemv_exact_products(kind, M, K, B):
    tid = TYPES[kind]
    h = synth(tid, f"fw.{kind}.{M}x{K}", M, K)
    m = FloatMatrix(tid, h, M, K)
    x = (3.0 * L.normal(SEED, f"fw.x.{M}x{K}.{B}", B * K)).reshape(B, K).astype(np.float32)
    w32 = L.float_to_f32(h, tid).reshape(M, K)
    check_fp64(run(m, x), w32, x)
    if M * K <= 2048 * 7680 and B <= 8:
        t = O.f16_tensor(h, M, K) if tid == L.TYPE_F16 else O.f32_tensor(h, M, K)
        ok, err = within(run(m, x), O.mat(t, x))
        assert ok, err
    parts = L.lib().lfm3_bf16_gemv_parts(M, K, B)
    for p in sorted({2, parts}):
        if p <= K // 32:
            check_fp64(run(m, x, parts=p), w32, x)


@pytest.mark.parametrize("kind", sorted(TYPES))
def test_float_identity_reassembles_inputs(kind):
    tid = TYPES[kind]
    K = 256
    eye = np.eye(K, dtype=np.float32)
    data = eye.astype(np.float16).view(np.uint16).ravel() if tid == L.TYPE_F16 else eye.ravel()
    m = FloatMatrix(tid, data, K, K)
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((8, K)) * np.exp2(rng.integers(-20, 20, (8, K)))).astype(np.float32)
    x[0, :4] = [1.0 + 2.0 ** -9 + 2.0 ** -17 + 2.0 ** -23, -np.float32(np.pi), 3e-30, 7e30]
    y = run(m, x)
    assert np.array_equal(y.view(np.uint32), x.view(np.uint32))


def test_float_weights_not_representable_in_bf16_keep_every_bit():
    """F16 weights with all 11 significant bits and F32 weights with all 24
    times x = 1: y equals the weight exactly (the weight's BF16 parts add
    back to it)."""
    K = 64
    for tid in (L.TYPE_F16, L.TYPE_F32):
        w = np.zeros((16, K), np.float32)
        w[:, 0] = 1.0 + np.arange(16) * 2.0 ** -10 + 2.0 ** -10 - 2.0 ** -23 * (tid == L.TYPE_F32)
        w[:, 0] *= np.exp2(np.arange(16) - 8.0)
        data = w.astype(np.float16).view(np.uint16).ravel() if tid == L.TYPE_F16 else w.ravel()
        widened = L.float_to_f32(data, tid).reshape(16, K)
        m = FloatMatrix(tid, data, 16, K)
        x = np.zeros((1, K), np.float32)
        x[0, 0] = 1.0
        y = run(m, x)
        assert np.array_equal(y[0].astype(np.float32).view(np.uint32),
                              widened[:, 0].view(np.uint32)), tid


def test_bf16_through_the_generic_entry_is_the_same():
    M, K, B = 3088, 2048, 8
    h = L.bf16(SEED, "fw.same", M, K)
    m = FloatMatrix(L.TYPE_BF16, h, M, K)
    x = L.normal(SEED, "fw.same.x", B * K).reshape(B, K).astype(np.float32)
    a, b = run(m, x), run(m, x, generic=False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("kind", sorted(TYPES))
def test_float_swiglu_pairs(kind):
    tid = TYPES[kind]
    F, H, B = 768, 512, 8
    g, u = synth(tid, f"fws.g.{kind}", F, H), synth(tid, f"fws.u.{kind}", F, H)
    m = FloatMatrix(tid, None, F, H, pairs=(g, u))
    x = L.normal(SEED, f"fws.x.{kind}", B * H).reshape(B, H).astype(np.float32)
    y = run(m, x, swiglu=True)
    mk = O.f16_tensor if tid == L.TYPE_F16 else O.f32_tensor
    gt, ut = mk(g, F, H), mk(u, F, H)
    want = np.stack([O.swiglu(O.mat(gt, x[b]), O.mat(ut, x[b])) for b in range(B)])
    ok, err = within(y, want)
    assert ok, err


@pytest.mark.parametrize("kind", sorted(TYPES))
def test_float_embed_rows(kind):
    tid = TYPES[kind]
    V, H, n = 1000, 256, 9
    h = synth(tid, f"fwe.{kind}", V, H)
    m = FloatMatrix(tid, h, V, H)
    toks = np.array([0, 999, 17, 16, 15, 500, 3, 1000, 2], np.uint32)   # 1000: past the table
    dt = L.DeviceBuffer.of(toks)
    out = L.DeviceBuffer(n * H * 4)
    L.check(L.lib().lfm3_float_embed(tid, m.buf.addr, V, H, dt.addr, None, n, out.addr, None))
    L.synchronize()
    got = out.download(np.float32, n * H).reshape(n, H)
    table = L.float_to_f32(h, tid).reshape(V, H)
    for i, t in enumerate(toks):
        want = table[t] if t < V else np.zeros(H, np.float32)
        assert np.array_equal(got[i], want), i


def small_dims(**kw):
    base = dict(hidden=256, intermediate=512, vocab=1000, context=1024, heads=8, head_dim=128,
                kv_heads=2, window=32, pattern="CSGCCSCG")
    base.update(kw)
    return L.Dims(**base)


@pytest.mark.parametrize("kind", sorted(TYPES))
def test_float_model_rounds_match_oracle(kind):
    tid = TYPES[kind]
    dims = small_dims()
    n = 8
    w = L.synth_weights(dims, seed=91, weight_type=tid)
    gm, om = L.Model(w), O.Model(dims, w)
    positions = L.uniform_u32(SEED, f"fw.pos.{kind}", n, 0, 600)
    gs, os_ = [], []
    for sid, p in enumerate(positions):
        g, o = gm.session(1024), om.session(1024, f16=True)
        inject_state(g, o, dims, 91, sid, int(p))
        gs.append(g)
        os_.append(o)
    for step in range(3):
        toks = L.uniform_u32(SEED, f"fw.tok{step}.{kind}", n, 0, dims.vocab - 1)
        if step == 1:
            ids = gm.forward_batch_greedy(gs, toks)
            logits = np.stack([s.read_logits() for s in gs])
            assert list(ids) == [O.argmax(r) for r in logits]
        else:
            logits = gm.forward_batch(gs, toks)
        for i in range(n):
            want = os_[i].step(int(toks[i]))
            err = same_greedy(logits[i], want, f"step {step} row {i}")
            assert err < 2e-3, (step, i, err)
    for s in gs:
        s.close()
    gm.close()
    om.close()


@pytest.mark.parametrize("kind", sorted(TYPES))
@pytest.mark.parametrize("n", [5, 40])
def test_float_prompt_matches_oracle_steps(kind, n):
    tid = TYPES[kind]
    dims = small_dims()
    w = L.synth_weights(dims, seed=92, weight_type=tid)
    gm, om = L.Model(w), O.Model(dims, w)
    g, o = gm.session(1024), om.session(1024, f16=True)
    inject_state(g, o, dims, 92, 0, 97)
    tokens = L.uniform_u32(SEED, f"fw.prompt.{kind}.{n}", n, 0, dims.vocab - 1)
    got = g.forward(tokens)
    want = None
    for t in tokens:
        want = o.step(int(t))
    prompt_gate(got, want, f"{kind} {n}-token prompt")
    assert g.position == o.position == 97 + n
    g.close()
    gm.close()
    om.close()
