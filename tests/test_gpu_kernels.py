"""Kernel parity on the GPU: every HIP entry point against the CPU oracle on
the same seeded inputs, through the C-ABI.

Gates: the reference's own (ops_test.cpp: projection 1e-4 vs FP64, conv
1e-7 with exact history, decode attention 2e-6 vs FP64) where its vectors
apply, and the FP32 parity gates elsewhere (1e-3 relative / 1e-4 absolute for
FP32 GEMV and attention outputs; bit-exact for indexing, ring slots and
greedy ids)."""
import zlib

import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import DeviceMatrix, gemv, pointer_table, within
from test_oracle import attention_fp64, data, formula_q8

pytestmark = pytest.mark.gpu
SEED = L.SEED


# -------------------------------------------------------------------- GEMV

@pytest.mark.parametrize("B", [1, 2, 3, 8])
def test_gemv_reference_projection_vectors(B):
    """ops_test.cpp:46-89 (M = 37, K = 2048, formula weights, FP32 rows)."""
    M, K = 37, 2048
    w = formula_q8(M, K)
    x = data(B * K, 0.07).reshape(B, K)
    y = gemv(DeviceMatrix(w, M, K), x)
    want64 = x.astype(np.float64) @ L.q8_dequant(w, M, K).T
    assert np.max(np.abs(y - want64)) < 1e-4
    ok, err = within(y, O.mat(O.q8_tensor(w, M, K), x))
    assert ok, err


@pytest.mark.parametrize("B", [1, 2, 4, 8])
def test_gemv_decode_shape_8192x2048(B):
    """The config-1 matrix: W 8192 x 2048 Q8_0, X ~ N(0, 1) rows."""
    M, K = 8192, 2048
    w = L.q8(SEED, "gemv.W", M, K)
    x = L.normal(SEED, f"gemv.X{B}", B * K).reshape(B, K)
    y = gemv(DeviceMatrix(w, M, K), x)
    ok, err = within(y, O.mat(O.q8_tensor(w, M, K), x))
    assert ok, err
    want64 = x.astype(np.float64) @ L.q8_dequant(w, M, K).T
    assert np.max(np.abs(y - want64)) < 2e-5


def wide_range_rows(B, K, tag):
    """Rows whose magnitudes span 2^-20..1 inside every 64-column chunk:
    |x| = 2^(-20 u) with u uniform in [0, 1), random signs, and one entry of
    magnitude 1 per chunk, so every chunk's (and slice's) maximum is 1."""
    rng = np.random.default_rng(zlib.crc32(f"{SEED}.{tag}".encode()))
    u = rng.random((B, K))
    x = np.exp2(-20.0 * u) * rng.choice([-1.0, 1.0], (B, K))
    for c in range(0, K, 64):
        x[:, c + rng.integers(0, 64)] = rng.choice([-1.0, 1.0], B)
    return x.astype(np.float32)


def truncate_to_fp16_grid(x, e):
    """fp16(x 2^e) 2^-e truncated toward zero, for x 2^e in fp16's normal
    range: the float32 significand cut to 11 bits (the operand's hi plane)."""
    bits = (np.asarray(x, np.float32) * np.float32(2.0 ** e)).view(np.uint32) & np.uint32(0xffffe000)
    return bits.view(np.float32).astype(np.float64) * 2.0 ** -e


@pytest.mark.parametrize("B", [1, 2, 4, 8])
def test_gemv_operand_keeps_two_fp16_planes_over_a_wide_range(B):
    """The decode operand's precision (q8.hip SplitPair, norm_image.hpp) on
    the config-1 matrix (W 8192 x 2048 Q8_0) with rows spanning 2^-20..1
    inside every chunk, against FP64.

    Bound: with the slice's maximum in [2^14, 2^15) after scaling by 2^e, hi
    = fp16(x 2^e) truncated keeps 11 bits (|r| < 2^-10 |X|, X = x 2^e) and
    lo = fp16(r 2^11) truncated keeps 11 bits of r (an error below 2^-10
    |r|); X >= 2^-6 keeps both planes normal, so the operand is within
    2^-20 |x| of x. The FP32 sums add at most 128 u (u = 2^-24: 31
    roundings in a block's 32 exact products, 64 block FMAs, the hi + lo
    sum), so |y - y64| <= (2^-20 + 2^-17) S per output, S = sum |w| |x|.

    Tight check: the error's RMS stays within twice that of the reference's
    FP32 path (the oracle, reference.cpp's order) on the same rows; the same
    rows with the lo plane dropped (hi alone) are about 400 times worse, so
    a lost or shortened lo plane fails here.

    Both the FP32-row GEMV (an exponent per wave slice: every slice's
    maximum is 1, e = 14) and the image GEMV fed by the residual norm (an
    exponent per row) are checked."""
    M, K = 8192, 2048
    w = L.q8(SEED, "prec.W", M, K)
    wd = L.q8_dequant(w, M, K)
    x = wide_range_rows(B, K, f"prec.x{B}")
    m = DeviceMatrix(w, M, K)
    tensor = O.q8_tensor(w, M, K)

    def check(y, xin, label, e=None):
        x64 = np.asarray(xin, np.float64)
        want = x64 @ wd.T
        err = np.asarray(y, np.float64) - want
        bound = (2.0 ** -20 + 2.0 ** -17) * (np.abs(x64) @ np.abs(wd).T)
        ref = O.mat(tensor, xin) - want
        rms = lambda v: float(np.sqrt(np.mean(np.square(v))))
        print(f"[{label}] B={B} max |err| / bound {np.max(np.abs(err) / bound):.4f}, "
              f"rms err {rms(err):.3g} (FP32 reference {rms(ref):.3g})", flush=True)
        assert np.all(np.abs(err) <= bound), label
        assert rms(err) <= 2.0 * rms(ref), label
        if e is not None:
            hi_only = truncate_to_fp16_grid(xin, e) @ wd.T - want
            assert rms(hi_only) > 100.0 * rms(ref), label

    check(gemv(m, x), x, "fp32 rows", e=14)
    # The image path: the residual norm (no branch, unit weights) writes z
    # and its operand image; the GEMV reads the image.
    H = K
    dx = L.DeviceBuffer.of(x)
    dwn = L.DeviceBuffer.of(np.ones(H, np.float32))
    dz = L.DeviceBuffer(B * H * 4)
    img = L.DeviceBuffer(L.lib().lfm3_operand_image_bytes(H))
    ex = L.DeviceBuffer(32)
    L.check(L.lib().lfm3_residual_norm_image(None, 1, 0, None, dx.addr, dwn.addr, dz.addr,
                                             img.addr, ex.addr, B, H, 1e-5, None))
    dy = L.DeviceBuffer(B * M * 4)
    L.check(L.lib().lfm3_q8_gemv_image(m.codes.addr, m.scales.addr, M, H, img.addr, ex.addr, B,
                                       dy.addr, M, 1, None))
    L.synchronize()
    gz = dz.download(np.float32, B * H).reshape(B, H)
    zmax = np.abs(gz).max(axis=1)
    assert np.all(np.abs(gz).min(axis=1) >= zmax * 2.0 ** -21)  # the range survives the norm
    check(dy.download(np.float32, B * M).reshape(B, M), gz, "image")


@pytest.mark.parametrize("M,B", [(128000, 8), (128000, 3), (32784, 5)])
def test_image_gemv_loop_equals_group_blocks(M, B):
    """Past 1024 two-tile groups (the vocabulary head, 128000 x 2048) the
    operand-image GEMV runs as a grid-stride loop over one block a CU, each
    block issuing its next group's loads before it reduces the current one;
    per group it takes the loads, products and reductions of the one-group
    blocks that smaller matrices run. Its first and last 2048 rows equal,
    bit for bit, the same rows computed as 2048-row matrices (64 groups:
    one block a group) over the same tiles, and every row is within the
    FP64 gate. 32784 rows: 1025 groups, the last one a single tile."""
    K = 2048
    lib = L.lib()
    w = L.q8(SEED, f"loop.W.{M}", M, K)
    m = DeviceMatrix(w, M, K)
    x = L.normal(SEED, f"loop.x.{M}.{B}", B * K, 0, 2).reshape(B, K)
    dx = L.DeviceBuffer.of(x)
    dwn = L.DeviceBuffer.of(np.ones(K, np.float32))
    dz = L.DeviceBuffer(B * K * 4)
    img = L.DeviceBuffer(lib.lfm3_operand_image_bytes(K))
    ex = L.DeviceBuffer(32)
    L.check(lib.lfm3_residual_norm_image(None, 1, 0, None, dx.addr, dwn.addr, dz.addr, img.addr,
                                         ex.addr, B, K, 1e-5, None))
    print(f"[loop] M {M} B {B}", flush=True)
    dy = L.DeviceBuffer(B * M * 4)
    L.check(lib.lfm3_q8_gemv_image(m.codes.addr, m.scales.addr, M, K, img.addr, ex.addr, B,
                                   dy.addr, M, 1, None))
    L.synchronize()
    y = dy.download(np.float32, B * M).reshape(B, M)
    nchunks, sub = K // 64, 2048
    for first in (0, M - sub):
        tile = first // 16
        ds = L.DeviceBuffer(B * sub * 4)
        L.check(lib.lfm3_q8_gemv_image(m.codes.addr + tile * nchunks * 1024,
                                       m.scales.addr + tile * nchunks * 64, sub, K, img.addr,
                                       ex.addr, B, ds.addr, sub, 1, None))
        L.synchronize()
        assert np.array_equal(ds.download(np.float32, B * sub).reshape(B, sub),
                              y[:, first:first + sub]), first
    gz = dz.download(np.float32, B * K).reshape(B, K)
    ok, err = within(y, O.mat(O.q8_tensor(w, M, K), gz))
    assert ok, err


@pytest.mark.parametrize("M,B", [(128000, 1), (128000, 8), (32784, 3)])
def test_fp32_row_gemv_loop_equals_group_blocks(M, B):
    """The FP32-row GEMV (lfm3_q8_gemv) past 1024 two-tile groups with K in
    one slice (the prompt's vocabulary head on its frontier row) runs the
    same grid-stride loop as the operand-image GEMV; each wave stages its
    chunks of x once with the one-block-a-group kernel's exponents and
    operands. Its first and last 2048 rows equal, bit for bit, the same
    rows computed as 2048-row matrices (64 groups: one block a group) over
    the same tiles, and every row is within the FP32 gate of the oracle."""
    K = 2048
    lib = L.lib()
    w = L.q8(SEED, f"floop.W.{M}", M, K)
    m = DeviceMatrix(w, M, K)
    x = (3.0 * L.normal(SEED, f"floop.x.{M}.{B}", B * K)).reshape(B, K)
    print(f"[fp32 loop] M {M} B {B}", flush=True)
    y = gemv(m, x)
    dx = L.DeviceBuffer.of(np.ascontiguousarray(x, np.float32))
    nchunks, sub = K // 64, 2048
    for first in (0, M - sub):
        tile = first // 16
        ds = L.DeviceBuffer(B * sub * 4)
        L.check(lib.lfm3_q8_gemv(m.codes.addr + tile * nchunks * 1024,
                                 m.scales.addr + tile * nchunks * 64, sub, K, dx.addr, K,
                                 ds.addr, sub, B, None, 0, None))
        L.synchronize()
        assert np.array_equal(ds.download(np.float32, B * sub).reshape(B, sub),
                              y[:, first:first + sub]), first
    ok, err = within(y, O.mat(O.q8_tensor(w, M, K), x))
    assert ok, err


@pytest.mark.parametrize("M,K,B", [(2048, 7680, 8), (128000, 2048, 4), (16, 2048, 5),
                                   (3088, 2048, 8), (48, 96, 7), (512, 64, 8), (64, 64, 1), (6144, 2048, 8)])
def test_gemv_model_shapes(M, K, B):
    w = L.q8(SEED, f"shape.{M}x{K}", M, K)
    x = (3.0 * L.normal(SEED, f"shape.x.{M}x{K}", B * K)).reshape(B, K)
    y = gemv(DeviceMatrix(w, M, K), x)
    ok, err = within(y, O.mat(O.q8_tensor(w, M, K), x))
    assert ok, err


def test_gemv_rows_are_independent_and_ragged_scales():
    """Rows of very different magnitude share a launch; each row's result
    equals its single-row result bit for bit."""
    M, K = 2048, 2048
    w = L.q8(SEED, "indep", M, K)
    x = L.normal(SEED, "indep.x", 8 * K).reshape(8, K)
    x *= np.array([1e-3, 1, 1e3, 7, 0.5, 1e-6, 30, 2], np.float32)[:, None]
    m = DeviceMatrix(w, M, K)
    y = gemv(m, x)
    for b in (0, 2, 5):
        assert np.array_equal(gemv(m, x[b:b + 1])[0], y[b])


@pytest.mark.parametrize("F,K,B", [(7680, 2048, 8), (192, 128, 3), (8192, 2048, 1)])
def test_gemv_swiglu(F, K, B):
    g = L.q8(SEED, f"sw.g{F}", F, K)
    u = L.q8(SEED, f"sw.u{F}", F, K)
    x = L.normal(SEED, f"sw.x{F}", B * K).reshape(B, K)
    y = gemv(DeviceMatrix(g, F, K, interleave_with=u), x, swiglu=True)
    want = np.stack([O.swiglu(O.mat(O.q8_tensor(g, F, K), x[b]), O.mat(O.q8_tensor(u, F, K), x[b]))
                     for b in range(B)])
    ok, err = within(y, want)
    assert ok, err


def test_device_pack_matches_host_pack():
    import ctypes as C
    from gpu_util import packed
    for rows, cols in ((37, 96), (512, 2048), (16, 7680)):
        src = L.q8(SEED, f"dp{rows}", rows, cols)
        codes, scales = packed(src, rows, cols)
        dsrc = L.DeviceBuffer.of(src)
        dc, ds = L.DeviceBuffer(codes.nbytes), L.DeviceBuffer(scales.nbytes)
        L.check(L.lib().lfm3_q8_pack_device(dsrc.addr, rows, cols, dc.addr, ds.addr, 0, 1, None))
        L.synchronize()
        assert np.array_equal(dc.download(np.uint8, codes.size), codes)
        assert np.array_equal(ds.download(np.uint8, scales.size), scales)


def test_embed_is_exact_row_decode():
    V, H = 1000, 2048
    w = L.q8(SEED, "emb", V, H)
    m = DeviceMatrix(w, V, H)
    toks = np.array([0, 999, 17, 500, 17, 3], np.uint32)
    dt = L.DeviceBuffer.of(toks)
    out = L.DeviceBuffer(len(toks) * H * 4)
    L.check(L.lib().lfm3_embed(m.codes.addr, m.scales.addr, V, H, dt.addr, len(toks), out.addr, None))
    L.synchronize()
    got = out.download(np.float32, len(toks) * H).reshape(len(toks), H)
    t = O.q8_tensor(w, V, H)
    for i, tok in enumerate(toks):
        assert np.array_equal(got[i], O.decode_row(t, int(tok)))


# ------------------------------------------------------------------- norms

@pytest.mark.parametrize("H", [2048, 256, 4096])
def test_residual_norm(H):
    n = 8
    x = L.normal(SEED, f"rn.x{H}", n * H, 0, 5).reshape(n, H)
    br = L.normal(SEED, f"rn.b{H}", n * H, 0, 2).reshape(n, H)
    post = L.normal(SEED, f"rn.p{H}", H, 1, 0.02)
    wn = L.normal(SEED, f"rn.w{H}", H, 1, 0.02)
    dx, db = L.DeviceBuffer.of(x), L.DeviceBuffer.of(br)
    dp, dw = L.DeviceBuffer.of(post), L.DeviceBuffer.of(wn)
    dz = L.DeviceBuffer(n * H * 4)
    L.check(L.lib().lfm3_residual_norm(db.addr, dp.addr, dx.addr, dw.addr, dz.addr, n, H, 1e-5, None))
    L.synchronize()
    gx = dx.download(np.float32, n * H).reshape(n, H)
    gz = dz.download(np.float32, n * H).reshape(n, H)
    for r in range(n):
        wx = x[r] + O.norm(br[r], post, 1e-5)
        np.testing.assert_allclose(gx[r], wx, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(gz[r], O.norm(wx, wn, 1e-5), rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------- conv

def test_conv_step_ragged_bit_exact():
    """Per-row histories through a pointer table (rows in scrambled session
    order): outputs and histories equal the oracle's bit for bit given the
    same projection rows."""
    H, Lw, n = 2048, 7, 8
    order = [3, 0, 7, 5, 1, 6, 2, 4]
    ldp = 3 * H + 16
    p = L.normal(SEED, "conv.p", n * ldp).reshape(n, ldp)
    taps = L.normal(SEED, "conv.taps", H * Lw, 0, 0.1)
    hists = [L.normal(SEED, f"conv.h{s}", H * (Lw - 1)) for s in range(8)]
    dh = [L.DeviceBuffer.of(h) for h in hists]
    table = pointer_table([dh[order[r]].addr for r in range(n)])
    dp, dt = L.DeviceBuffer.of(p), L.DeviceBuffer.of(taps)
    dy = L.DeviceBuffer(n * H * 4)
    L.check(L.lib().lfm3_conv_step_ragged(dp.addr, ldp, dt.addr, table.addr, dy.addr, H, n, H, Lw, None))
    L.synchronize()
    y = dy.download(np.float32, n * H).reshape(n, H)
    for r in range(n):
        want_y, want_h = O.conv_step(p[r, :3 * H], taps, hists[order[r]], H, Lw)
        assert np.array_equal(y[r], want_y)
        assert np.array_equal(dh[order[r]].download(np.float32, H * (Lw - 1)), want_h)


# --------------------------------------------------- heads and attention

def ragged_case(heads, kv, D, window, ctx_hi=4096, n=8, tag="a", global_cap=4096):
    # A stable per-case seed (str hashes are salted per process).
    rng = np.random.default_rng(zlib.crc32(repr((heads, kv, D, window, tag)).encode()))
    ctx = L.uniform_u32(SEED, f"att.ctx.{tag}", n, 1, ctx_hi)
    positions = (ctx - 1).astype(np.uint32)
    cap = window if window else global_cap
    stride = kv * D
    order = list(rng.permutation(n))
    return ctx, positions, cap, stride, order


@pytest.mark.parametrize("heads,kv,D", [(32, 8, 64), (16, 4, 128), (16, 8, 128), (16, 2, 128)])
@pytest.mark.parametrize("window", [0, 256])
@pytest.mark.parametrize("fused", [False, True])
def test_heads_and_attention_ragged(heads, kv, D, window, fused):
    """Config-2 shape: 8 sessions, contexts U[1, 4096], Q/K RMSNorm, paired
    RoPE at theta 1e6, F16 ring store, gated GQA; sliding (256) and global.
    Unfused: the heads launch, then attention over the ring. Fused: one
    entry norms, rotates and stores inside the attention launch."""
    n = 8
    ctx, positions, cap, stride, order = ragged_case(heads, kv, D, window)
    theta = 1e6
    factors = np.ones(D // 2, np.float32)
    ld = (heads + 2 * kv) * D + heads + 4
    qkv = L.normal(SEED, f"att.qkv.{heads}.{D}.{window}", n * ld).reshape(n, ld)
    q_off, k_off, v_off, g_off = 0, heads * D, (heads + kv) * D, (heads + 2 * kv) * D
    qn = L.normal(SEED, "att.qn", D, 1, 0.02)
    kn = L.normal(SEED, "att.kn", D, 1, 0.02)
    rings_k = [L.half_normal(SEED, f"att.k{s}.{D}", cap * stride) for s in range(n)]
    rings_v = [L.half_normal(SEED, f"att.v{s}.{D}", cap * stride) for s in range(n)]
    dk = [L.DeviceBuffer.of(r) for r in rings_k]
    dv = [L.DeviceBuffer.of(r) for r in rings_v]
    # row r belongs to session order[r]; its position is that session's
    pos_rows = np.array([positions[order[r]] for r in range(n)], np.uint32)
    tk = pointer_table([dk[order[r]].addr for r in range(n)])
    tv = pointer_table([dv[order[r]].addr for r in range(n)])
    caps = L.DeviceBuffer.of(np.full(n, cap, np.uint32))
    dpos = L.DeviceBuffer.of(pos_rows)
    i = np.arange(D // 2, dtype=np.float32)
    from test_oracle import powf
    freq = powf(theta, np.float32(-2.0) * i / np.float32(D))
    dfreq, dfac = L.DeviceBuffer.of(freq), L.DeviceBuffer.of(factors)
    dq = L.DeviceBuffer.of(qkv)
    dqn, dkn = L.DeviceBuffer.of(qn), L.DeviceBuffer.of(kn)
    if not fused:
        L.check(L.lib().lfm3_decode_heads_ragged(
            dq.addr + 4 * q_off, dq.addr + 4 * k_off, dq.addr + 4 * v_off, ld, dqn.addr,
            dkn.addr, dfreq.addr, 0 if window else dfac.addr, tk.addr, tv.addr, dpos.addr,
            caps.addr, n, heads, kv, D, 1e-5, None))
    cap_items = 4096
    items = (L.AttentionItem * cap_items)()
    count = L.check(L.lib().lfm3_attention_plan(L.ptr(pos_rows), n, window, items, cap_items))
    ditems = L.DeviceBuffer(count * C_ITEM)
    L.hip_check(L.hip().hipMemcpy(ditems.addr, L.C.addressof(items), count * C_ITEM, L.H2D))
    ws_bytes = L.lib().lfm3_attention_workspace_bytes(count, n, heads, kv, D)
    ws = L.DeviceBuffer(ws_bytes)
    dout = L.DeviceBuffer(n * heads * D * 4)
    for repeat in range(2):  # the second call reuses the workspace
        if fused:
            L.check(L.lib().lfm3_decode_heads_attention_ragged(
                dq.addr + 4 * q_off, dq.addr + 4 * k_off, dq.addr + 4 * v_off, ld,
                dq.addr + 4 * g_off, ld, dqn.addr, dkn.addr, dfreq.addr,
                0 if window else dfac.addr, tk.addr, tv.addr, dpos.addr, caps.addr,
                ditems.addr, count, dout.addr, heads * D, n, heads, kv, D, 1e-5, ws.addr,
                ws_bytes, None))
        else:
            L.check(L.lib().lfm3_decode_attention_ragged(
                dq.addr + 4 * q_off, ld, dq.addr + 4 * g_off, ld, tk.addr, tv.addr, caps.addr,
                ditems.addr, count, dout.addr, heads * D, n, heads, kv, D, ws.addr, ws_bytes,
                None))
        L.synchronize()
        out = dout.download(np.float32, n * heads * D).reshape(n, heads * D)
        if repeat == 0:
            first = out
    assert np.array_equal(first, out)
    for r in range(n):
        s = order[r]
        p = int(pos_rows[r])
        ck = O.half_to_float(rings_k[s])
        cv = O.half_to_float(rings_v[s])
        want, qr, kr = O.attention_step(qkv[r, q_off:k_off], qkv[r, k_off:v_off],
                                        qkv[r, v_off:g_off], qkv[r, g_off:g_off + heads], qn, kn,
                                        None if window else factors, ck, cv, heads, kv, D, p, cap,
                                        window, theta, bool(window), 1e-5, True)
        ok, err = within(out[r], want)
        assert ok, (r, err)
        # ring: only slot p % cap changed; V bits exact; K within one ulp
        gk = dk[s].download(np.uint16, cap * stride).reshape(cap, stride)
        gv = dv[s].download(np.uint16, cap * stride).reshape(cap, stride)
        slot = p % cap
        keep = np.ones(cap, bool)
        keep[slot] = False
        assert np.array_equal(gk[keep], rings_k[s].reshape(cap, stride)[keep])
        assert np.array_equal(gv[keep], rings_v[s].reshape(cap, stride)[keep])
        assert np.array_equal(gv[slot], O.float_to_half(qkv[r, v_off:g_off]))
        ulps = np.abs(gk[slot].astype(np.int32) - O.float_to_half(kr).astype(np.int32))
        assert ulps.max() <= 1 and (ulps > 0).mean() < 0.02
        gq = dq.download(np.float32, n * ld).reshape(n, ld)
        if fused:  # the projection rows are left as they were
            assert np.array_equal(gq[r], qkv[r])
        else:  # rotated q/k written back in place, as the reference's heads kernel does
            np.testing.assert_allclose(gq[r, q_off:k_off], qr, rtol=1e-4, atol=2e-5)


C_ITEM = L.C.sizeof(L.AttentionItem)


@pytest.mark.parametrize("P,H,KH,window", [(259, 4, 2, 0), (259, 4, 2, 256), (4999, 4, 2, 0),
                                           (4999, 4, 2, 256), (3000, 16, 4, 0),
                                           (3000, 16, 4, 256)])
def test_attention_reference_decode_vectors(P, H, KH, window):
    """ops_test.cpp:142-220 at n = 1 through the ragged entry point."""
    D = 128
    cap = window if window else P + 1
    stride = KH * D
    q = data(H * D, 0.7)
    gates = data(H, 0.7)
    kbits = O.float_to_half(data(cap * stride, 0.6))
    vbits = O.float_to_half(data(cap * stride, 0.8))
    kbits[(P % cap) * stride:(P % cap + 1) * stride] = O.float_to_half(data(stride, 0.5))
    vbits[(P % cap) * stride:(P % cap + 1) * stride] = O.float_to_half(data(stride, 0.9))
    dk, dv = L.DeviceBuffer.of(kbits), L.DeviceBuffer.of(vbits)
    tk, tv = pointer_table([dk.addr]), pointer_table([dv.addr])
    caps = L.DeviceBuffer.of(np.array([cap], np.uint32))
    pos = np.array([P], np.uint32)
    cap_items = L.lib().lfm3_attention_max_items(1, int(pos[0]))
    items = (L.AttentionItem * cap_items)()
    count = L.check(L.lib().lfm3_attention_plan(L.ptr(pos), 1, window, items, cap_items))
    ditems = L.DeviceBuffer(count * C_ITEM)
    L.hip_check(L.hip().hipMemcpy(ditems.addr, L.C.addressof(items), count * C_ITEM, L.H2D))
    ws_bytes = L.lib().lfm3_attention_workspace_bytes(count, 1, H, KH, D)
    ws = L.DeviceBuffer(ws_bytes)
    dq, dg = L.DeviceBuffer.of(q), L.DeviceBuffer.of(gates)
    dout = L.DeviceBuffer(H * D * 4)
    L.check(L.lib().lfm3_decode_attention_ragged(dq.addr, H * D, dg.addr, H, tk.addr, tv.addr,
                                                 caps.addr, ditems.addr, count, dout.addr, H * D,
                                                 1, H, KH, D, ws.addr, ws_bytes, None))
    L.synchronize()
    out = dout.download(np.float32, H * D)
    want = attention_fp64(q, gates, O.half_to_float(kbits), O.half_to_float(vbits), H, KH, D, P,
                          cap, window)
    assert np.max(np.abs(out - want)) < 2e-6


# ------------------------------------------------------------------ argmax

def test_argmax_first_index_of_ties():
    rows, V = 8, 128000
    x = L.normal(SEED, "argmax", rows * V).reshape(rows, V)
    x[0, 5] = x[0, 70000] = 50.0          # tie: first index wins
    x[1, :] = -3.0                         # all equal: index 0
    x[2, 127999] = 99.0
    x[3, 8191] = x[3, 8192] = 9.0          # tie across block boundary
    x[4] = -np.abs(x[4]) - 1               # all negative
    dx = L.DeviceBuffer.of(x)
    ids = L.DeviceBuffer(rows * 4)
    ws = L.DeviceBuffer(L.lib().lfm3_argmax_workspace_bytes(rows))
    for _ in range(2):
        L.check(L.lib().lfm3_argmax(dx.addr, rows, V, ids.addr, ws.addr, ws.nbytes, None))
        L.synchronize()
        got = ids.download(np.uint32, rows)
        assert list(got) == [O.argmax(x[r]) for r in range(rows)]
    assert got[0] == 5 and got[1] == 0 and got[2] == 127999 and got[3] == 8191


def test_gemv_shapes_share_one_workspace():
    """Engine pattern: consecutive GEMVs of different shapes (different row
    group counts and K slices) reuse one workspace; each must match its own
    fresh-workspace result bit for bit."""
    shapes = [(768, 256, 8), (2048, 2048, 3), (256, 512, 8), (3088, 2048, 1), (64, 7680, 8),
              (2048, 7680, 2), (512, 2048, 8)]
    mats = {}
    most = 256
    for M, K, B in shapes:
        mats[(M, K)] = (L.q8(SEED, f"ws{M}x{K}", M, K), DeviceMatrix(L.q8(SEED, f"ws{M}x{K}", M, K), M, K))
        most = max(most, L.lib().lfm3_gemv_workspace_bytes(M, K, B))
    shared = L.DeviceBuffer(most)
    for rep in range(2):
        for M, K, B in shapes:
            src, m = mats[(M, K)]
            x = L.normal(SEED, f"wsx{M}x{K}", B * K).reshape(B, K)
            fresh = gemv(m, x)
            dx = L.DeviceBuffer.of(x)
            dy = L.DeviceBuffer(B * M * 4)
            L.check(L.lib().lfm3_q8_gemv(m.codes.addr, m.scales.addr, M, K, dx.addr, K, dy.addr,
                                         M, B, shared.addr, shared.nbytes, None))
            L.synchronize()
            assert np.array_equal(dy.download(np.float32, B * M).reshape(B, M), fresh), (M, K, B)


# ------------------------------------------------- partials, operand images

def decode_image(image: np.ndarray, exps: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Inverse of the operand-image layout: (hi + lo 2^-11) 2^-e per token.
    hi and lo are truncations, so the decoded row is within 2^-21 of the
    row maximum."""
    nch = (cols + 63) // 64
    lanes = image.view(np.float16).reshape(nch, 2, 4, 16, 8).astype(np.float64)  # c, b, g, m, i
    out = np.zeros((rows, nch * 64))
    for t in range(rows):
        hi, lo = lanes[:, :, :, t, :], lanes[:, :, :, 8 + t, :]
        val = (hi + lo / 2048.0) * 2.0 ** (-int(exps[t]))
        out[t] = val.reshape(nch * 64)  # c, b, g, i -> 64 c + 32 b + 8 g + i
    return out[:, :cols]


@pytest.mark.parametrize("B", [1, 3, 8])
def test_norm_image_feeds_gemv(B):
    """lfm3_residual_norm_image on K-part partial branches: x and z follow the
    oracle's residual + RMSNorm, the image decodes to z, and the image GEMV
    (plain, partials, SwiGLU) equals the FP32 GEMV of the same z up to the
    order of its chunk sums (a smaller grid takes 16 waves, two chunks
    each, where the FP32 GEMV's 8 waves take four): 1e-5 relative."""
    H, M, F, parts = 2048, 3088, 512, 4
    x = L.normal(SEED, f"ni.x{B}", B * H, 0, 3).reshape(B, H)
    br = L.normal(SEED, f"ni.b{B}", parts * B * H, 0, 1).reshape(parts, B, H)
    post = L.normal(SEED, "ni.post", H, 1, 0.02)
    wn = L.normal(SEED, "ni.w", H, 1, 0.02)
    dx, dbr = L.DeviceBuffer.of(x), L.DeviceBuffer.of(br)
    dpost, dwn = L.DeviceBuffer.of(post), L.DeviceBuffer.of(wn)
    dz = L.DeviceBuffer(B * H * 4)
    img = L.DeviceBuffer(L.lib().lfm3_operand_image_bytes(H))
    L.hip_check(L.hip().hipMemset(img.addr, 0x7f, img.nbytes))  # poison: every word is rewritten
    ex = L.DeviceBuffer(32)
    L.check(L.lib().lfm3_residual_norm_image(dbr.addr, parts, B * H, dpost.addr, dx.addr, dwn.addr,
                                             dz.addr, img.addr, ex.addr, B, H, 1e-5, None))
    L.synchronize()
    gx = dx.download(np.float32, B * H).reshape(B, H)
    gz = dz.download(np.float32, B * H).reshape(B, H)
    branch = br[0] + br[1] + br[2] + br[3]  # part order
    for r in range(B):
        wx = x[r] + O.norm(branch[r], post, 1e-5)
        np.testing.assert_allclose(gx[r], wx, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(gz[r], O.norm(wx, wn, 1e-5), rtol=1e-5, atol=1e-6)
    image = img.download(np.uint8, img.nbytes)
    exps = ex.download(np.int32, 8)
    dec = decode_image(image, exps, B, H)
    assert np.all(np.abs(dec - gz) <= np.abs(gz).max(axis=1, keepdims=True) * 2.0 ** -21)
    # plain and K-part image GEMVs against the FP32 GEMV of z
    w = L.q8(SEED, "ni.W", M, H)
    m = DeviceMatrix(w, M, H)
    want = gemv(m, gz)
    dy = L.DeviceBuffer(B * M * 4)
    L.check(L.lib().lfm3_q8_gemv_image(m.codes.addr, m.scales.addr, M, H, img.addr, ex.addr, B,
                                       dy.addr, M, 1, None))
    L.synchronize()
    ok, err = within(dy.download(np.float32, B * M).reshape(B, M), want, rtol=1e-5, atol=1e-6)
    assert ok, err
    k_parts = 4
    dp = L.DeviceBuffer(k_parts * B * M * 4)
    L.check(L.lib().lfm3_q8_gemv_image(m.codes.addr, m.scales.addr, M, H, img.addr, ex.addr, B,
                                       dp.addr, M, k_parts, None))
    L.synchronize()
    got = dp.download(np.float32, k_parts * B * M).reshape(k_parts, B, M).sum(axis=0, dtype=np.float64)
    ok, err = within(got, O.mat(O.q8_tensor(w, M, H), gz))
    assert ok, err
    # SwiGLU pair
    g, u = L.q8(SEED, "ni.g", F, H), L.q8(SEED, "ni.u", F, H)
    ms = DeviceMatrix(g, F, H, interleave_with=u)
    want = gemv(ms, gz, swiglu=True)
    dh = L.DeviceBuffer(B * F * 4)
    L.check(L.lib().lfm3_q8_gemv_swiglu_image(ms.codes.addr, ms.scales.addr, F, H, img.addr,
                                              ex.addr, B, dh.addr, F, None))
    L.synchronize()
    ok, err = within(dh.download(np.float32, B * F).reshape(B, F), want, rtol=1e-5, atol=1e-6)
    assert ok, err


@pytest.mark.parametrize("M,K,B", [(2048, 7680, 8), (2048, 2048, 5), (64, 96, 2)])
def test_gemv_partials_sum_to_the_product(M, K, B):
    parts = L.lib().lfm3_q8_gemv_parts(M, K)
    assert 1 <= parts <= 8
    w = L.q8(SEED, f"gp.{M}x{K}", M, K)
    m = DeviceMatrix(w, M, K)
    x = L.normal(SEED, f"gp.x{M}x{K}", B * K).reshape(B, K)
    dx = L.DeviceBuffer.of(x)
    want = O.mat(O.q8_tensor(w, M, K), x)
    for p in sorted({1, parts, min(3, (K + 63) // 64)}):
        dy = L.DeviceBuffer(p * B * M * 4)
        L.check(L.lib().lfm3_q8_gemv_partials(m.codes.addr, m.scales.addr, M, K, dx.addr, K,
                                              dy.addr, M, B, p, None))
        L.synchronize()
        got = dy.download(np.float32, p * B * M).reshape(p, B, M)
        acc = got[0].copy()
        for q in range(1, p):
            acc = acc + got[q]
        ok, err = within(acc, want)
        assert ok, (p, err)


def test_conv_row_image_bit_exact():
    """Row-per-block convolution writing the out projection's operand image:
    outputs and histories equal the oracle's bit for bit."""
    H, Lw, n = 2048, 7, 8
    p = L.normal(SEED, "cri.p", n * 3 * H).reshape(n, 3 * H)
    taps = L.normal(SEED, "cri.taps", H * Lw, 0, 0.1)
    hist = [L.normal(SEED, f"cri.h{i}", H * (Lw - 1)) for i in range(n)]
    dh = [L.DeviceBuffer.of(h) for h in hist]
    table = pointer_table([b.addr for b in dh])
    dp, dt = L.DeviceBuffer.of(p), L.DeviceBuffer.of(taps)
    dy = L.DeviceBuffer(n * H * 4)
    img = L.DeviceBuffer(L.lib().lfm3_operand_image_bytes(H))
    ex = L.DeviceBuffer(32)
    L.check(L.lib().lfm3_conv_step_ragged_image(dp.addr, 3 * H, dt.addr, table.addr, dy.addr, H,
                                                img.addr, ex.addr, n, H, Lw, None))
    L.synchronize()
    y = dy.download(np.float32, n * H).reshape(n, H)
    for r in range(n):
        want_y, want_h = O.conv_step(p[r], taps, hist[r], H, Lw)
        assert np.array_equal(y[r], want_y)
        assert np.array_equal(dh[r].download(np.float32, H * (Lw - 1)), want_h)
    dec = decode_image(img.download(np.uint8, img.nbytes), ex.download(np.int32, 8), n, H)
    assert np.all(np.abs(dec - y) <= np.abs(y).max(axis=1, keepdims=True) * 2.0 ** -21)


@pytest.mark.parametrize("H,B", [(2048, 8), (2048, 3), (256, 1)])
def test_projection_conv_image(H, B):
    """lfm3_q8_gemv_conv_image against the in projection's image GEMV followed
    by lfm3_conv_step_ragged (which equals the oracle's step bit for bit):
    outputs and histories agree up to the order of the projection's chunk
    sums (its 16-wave blocks add them differently): 1e-5 relative."""
    Lw = 7
    x = L.normal(SEED, f"pc.x{H}.{B}", B * H).reshape(B, H)
    dx, dw = L.DeviceBuffer.of(x), L.DeviceBuffer.of(np.ones(H, np.float32))
    dz = L.DeviceBuffer(B * H * 4)
    img = L.DeviceBuffer(L.lib().lfm3_operand_image_bytes(H))
    ex = L.DeviceBuffer(32)
    L.check(L.lib().lfm3_residual_norm_image(None, 1, 0, None, dx.addr, dw.addr, dz.addr, img.addr,
                                             ex.addr, B, H, 1e-5, None))
    w = L.q8(SEED, f"pc.W{H}", 3 * H, H)
    m = DeviceMatrix(w, 3 * H, H)
    taps = L.normal(SEED, f"pc.taps{H}", H * Lw, 0, 0.1)
    hist = [L.normal(SEED, f"pc.h{H}.{i}", H * (Lw - 1)) for i in range(B)]
    dt = L.DeviceBuffer.of(taps)
    # reference path: projection, then the step
    dp = L.DeviceBuffer(B * 3 * H * 4)
    L.check(L.lib().lfm3_q8_gemv_image(m.codes.addr, m.scales.addr, 3 * H, H, img.addr, ex.addr,
                                       B, dp.addr, 3 * H, 1, None))
    dh1 = [L.DeviceBuffer.of(h) for h in hist]
    t1 = pointer_table([b.addr for b in dh1])
    dy1 = L.DeviceBuffer(B * H * 4)
    L.check(L.lib().lfm3_conv_step_ragged(dp.addr, 3 * H, dt.addr, t1.addr, dy1.addr, H, B, H, Lw,
                                          None))
    # fused
    dh2 = [L.DeviceBuffer.of(h) for h in hist]
    t2 = pointer_table([b.addr for b in dh2])
    dy2 = L.DeviceBuffer(B * H * 4)
    L.check(L.lib().lfm3_q8_gemv_conv_image(m.codes.addr, m.scales.addr, H, img.addr, ex.addr, B,
                                            dt.addr, t2.addr, Lw, dy2.addr, H, None))
    L.synchronize()
    p = dp.download(np.float32, B * 3 * H).reshape(B, 3 * H)
    y1 = dy1.download(np.float32, B * H).reshape(B, H)
    y2 = dy2.download(np.float32, B * H).reshape(B, H)
    ok, err = within(y2, y1, rtol=1e-5, atol=1e-6)
    assert ok, err
    for r in range(B):
        h1 = dh1[r].download(np.float32, H * (Lw - 1))
        h2 = dh2[r].download(np.float32, H * (Lw - 1))
        want_y, want_h = O.conv_step(p[r], taps, hist[r], H, Lw)
        assert np.array_equal(y1[r], want_y) and np.array_equal(h1, want_h)
        ok, err = within(h2, h1, rtol=1e-5, atol=1e-6)
        assert ok, (r, err)
        # the shifted part of the window is copied, not recomputed
        keep = hist[r].reshape(H, Lw - 1)[:, 1:]
        assert np.array_equal(h2.reshape(H, Lw - 1)[:, :-1], keep)
