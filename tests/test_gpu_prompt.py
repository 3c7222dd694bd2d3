"""Prompt-pass kernels on the GPU against the oracle: FP16 row-scaled
activations (bit-exact), the Q8_0 x FP16 MFMA GEMM against FP64 over the
same rounded inputs (the reference's 1e-4 gate, ops_test.cpp:55-89, and the
1e-3 / 1e-4 gate), the SwiGLU epilogue and its row maxima."""
import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import DeviceMatrix, within
from test_oracle import data, formula_q8

pytestmark = pytest.mark.gpu
SEED = L.SEED


def half_rows_gpu(x, lda=None, row_max=None, max_blocks=0):
    n, K = x.shape
    lda = lda or (K + 63) // 64 * 64
    dx = L.DeviceBuffer.of(np.ascontiguousarray(x, np.float32))
    da = L.DeviceBuffer(n * lda * 2)
    ds = L.DeviceBuffer(n * 4)
    dm = None if row_max is None else L.DeviceBuffer.of(row_max)
    L.check(L.lib().lfm3_half_rows(dx.addr, K, 0 if dm is None else dm.addr, max_blocks, da.addr,
                                   lda, ds.addr, n, K, None))
    L.synchronize()
    return da, ds, lda


@pytest.mark.parametrize("n,K", [(16, 2048), (37, 96), (512, 7680)])
def test_half_rows_bit_exact(n, K):
    x = (L.normal(SEED, f"hr.{n}.{K}", n * K) * np.float32(3.0)).reshape(n, K)
    x[0] = 0
    da, ds, lda = half_rows_gpu(x)
    inputs, exps = O.half_rows(x)
    a = da.download(np.uint16, n * lda).reshape(n, lda)
    scale = ds.download(np.float32, n)
    assert np.array_equal(scale, np.ldexp(np.float32(1), -exps).astype(np.float32))
    want = O.float_to_half(np.ldexp(x, exps[:, None]).astype(np.float32))
    assert np.array_equal(a[:, :K], want)
    assert not a[:, K:(K + 63) // 64 * 64].any()  # the last chunk's zero tail
    # effective inputs match the oracle's
    got = np.ldexp(O.half_to_float(a[:, :K]), -exps[:, None])
    assert np.array_equal(got.astype(np.float32), inputs)


def half_tiles(m: DeviceMatrix, rows=None):
    """The FP16 tiles of a device matrix (lfm3_q8_half_tiles)."""
    rows = rows or m.rows
    out = L.DeviceBuffer(L.lib().lfm3_q8_half_tiles_bytes(rows, m.cols))
    L.check(L.lib().lfm3_q8_half_tiles(m.codes.addr, rows, m.cols, out.addr, None))
    L.synchronize()
    return out


def gemm(m: DeviceMatrix, x, parts=None, swiglu=False, half=False):
    n, K = x.shape
    da, ds, lda = half_rows_gpu(x)
    M = m.rows
    parts = parts or L.lib().lfm3_q8_gemm_parts(M, K, n, int(swiglu))
    w = half_tiles(m, 2 * M if swiglu else M) if half else m.codes
    if swiglu:
        dy = L.DeviceBuffer(n * M * 4)
        blocks = L.lib().lfm3_q8_gemm_swiglu_max_blocks(M)
        rm = L.DeviceBuffer(blocks * n * 4)
        fn = L.lib().lfm3_q8_gemm_swiglu_h16 if half else L.lib().lfm3_q8_gemm_swiglu
        L.check(fn(w.addr, m.scales.addr, M, K, da.addr, lda, ds.addr, n, dy.addr, M, rm.addr,
                   None))
        L.synchronize()
        return (dy.download(np.float32, n * M).reshape(n, M),
                rm.download(np.uint32, blocks * n).reshape(blocks, n))
    dy = L.DeviceBuffer(parts * n * M * 4)
    fn = L.lib().lfm3_q8_gemm_h16 if half else L.lib().lfm3_q8_gemm
    L.check(fn(w.addr, m.scales.addr, M, K, da.addr, lda, ds.addr, n, dy.addr, M, parts, None))
    L.synchronize()
    y = dy.download(np.float32, parts * n * M).reshape(parts, n, M)
    out = y[0].copy()
    for p in range(1, parts):
        out = out + y[p]
    return out


@pytest.mark.parametrize("n", [16, 29, 512])
def test_gemm_reference_projection_vectors(n):
    """ops_test.cpp:46-89: M = 37, K = 2048 formula weights, prompt rows as
    FP16 row-scaled inputs, FP64 expectation, gate 1e-4."""
    M, K = 37, 2048
    w = formula_q8(M, K)
    x = data(n * K, 0.07).reshape(n, K)
    y = gemm(DeviceMatrix(w, M, K), x)
    inputs, _ = O.half_rows(x)
    want = inputs.astype(np.float64) @ L.q8_dequant(w, M, K).T
    assert np.max(np.abs(y - want)) < 1e-4


@pytest.mark.parametrize("M,K,n,parts", [(2048, 2048, 512, None), (3088, 2048, 512, 1),
                                         (6144, 2048, 130, None), (2048, 7680, 512, None),
                                         (2048, 7680, 64, 3), (48, 96, 17, 2),
                                         (12288, 256, 512, None), (12288, 256, 500, 2)])
def test_gemm_model_shapes(M, K, n, parts):
    """Model projections (128-row blocks) and a tall matrix whose 256-row
    blocks fill the CUs (12288 rows x 500 or 512 tokens: the wide block shape)."""
    w = L.q8(SEED, f"pg.{M}.{K}", M, K)
    x = L.normal(SEED, f"pg.x.{M}.{K}.{n}", n * K).reshape(n, K)
    y = gemm(DeviceMatrix(w, M, K), x, parts)
    inputs, _ = O.half_rows(x)
    want = inputs.astype(np.float64) @ L.q8_dequant(w, M, K).T
    ok, err = within(y, want)
    assert ok, err


@pytest.mark.parametrize("F,K,n", [(7680, 2048, 512), (192, 128, 20)])
def test_gemm_swiglu_and_row_max(F, K, n):
    g = L.q8(SEED, f"ps.g{F}", F, K)
    u = L.q8(SEED, f"ps.u{F}", F, K)
    x = L.normal(SEED, f"ps.x{F}", n * K).reshape(n, K)
    y, rm = gemm(DeviceMatrix(g, F, K, interleave_with=u), x, swiglu=True)
    inputs, _ = O.half_rows(x)
    gv = inputs.astype(np.float64) @ L.q8_dequant(g, F, K).T
    uv = inputs.astype(np.float64) @ L.q8_dequant(u, F, K).T
    want = gv / (1 + np.exp(-gv)) * uv
    ok, err = within(y, want)
    assert ok, err
    # partial maxima per block of 128 output rows (16 interleaved gate/up
    # tiles); their maximum is the row's
    parts = rm.view(np.float32)
    assert parts.shape[0] == -(-F // 128)
    for b in range(parts.shape[0]):
        assert np.array_equal(parts[b], np.abs(y[:, 128 * b:128 * (b + 1)]).max(axis=1))
    assert np.array_equal(parts.max(axis=0), np.abs(y).max(axis=1))
    # and they stand in for the row scan of the down projection's FP16 rows
    da, ds, lda = half_rows_gpu(y)
    db, dt, _ = half_rows_gpu(y, row_max=rm.reshape(-1), max_blocks=parts.shape[0])
    assert np.array_equal(da.download(np.uint16, n * lda), db.download(np.uint16, n * lda))
    assert np.array_equal(ds.download(np.float32, n), dt.download(np.float32, n))


@pytest.mark.parametrize("M,K", [(37, 2048), (3088, 2048), (48, 96)])
def test_half_tiles_layout(M, K):
    """FP16 tile (t, c), lane L = 16 g + n: row 16 t + n, block 0's elements
    64 c + 8 g .. + 7 at byte 16 L, block 1's (64 c + 32 + 8 g ..) at
    1024 + 16 L, each the exact fp16 of the code; padding rows and columns
    are zero."""
    w = L.q8(SEED, f"ht.{M}.{K}", M, K)
    m = DeviceMatrix(w, M, K)
    got = half_tiles(m).download(np.uint16, L.lib().lfm3_q8_half_tiles_bytes(M, K) // 2)
    tiles, chunks = -(-M // 16), -(-K // 64)
    got = got.reshape(tiles, chunks, 2, 4, 16, 8)  # tile, chunk, block, g, n, element
    codes = np.zeros((tiles * 16, chunks * 64), np.float32)
    blocks = w.reshape(M, K // 32, 34)
    codes[:M, :K] = blocks[:, :, 2:].view(np.int8).reshape(M, K).astype(np.float32)
    want = codes.reshape(tiles, 16, chunks, 2, 4, 8).transpose(0, 2, 3, 4, 1, 5)
    assert np.array_equal(got, O.float_to_half(np.ascontiguousarray(want)))


@pytest.mark.parametrize("M,K,n,parts,swiglu", [(2048, 2048, 512, None, False),
                                                (3088, 2048, 512, 1, False),
                                                (6144, 2048, 130, None, False),
                                                (2048, 7680, 64, 3, False),
                                                (12288, 256, 500, 2, False),
                                                (48, 96, 17, 2, False),
                                                (7680, 2048, 512, None, True),
                                                (192, 128, 20, None, True)])
def test_gemm_half_tiles_identical(M, K, n, parts, swiglu):
    """The GEMM over FP16 tiles takes the same operands, products and block
    fmas as over code tiles: outputs (and SwiGLU row maxima) bit-exact, and
    within the gate of FP64 over the same rounded inputs."""
    g = L.q8(SEED, f"hg.{M}.{K}", M, K)
    u = L.q8(SEED, f"hu.{M}.{K}", M, K) if swiglu else None
    m = DeviceMatrix(g, M, K, interleave_with=u) if swiglu else DeviceMatrix(g, M, K)
    x = L.normal(SEED, f"hg.x.{M}.{K}.{n}", n * K).reshape(n, K)
    a = gemm(m, x, parts, swiglu=swiglu)
    b = gemm(m, x, parts, swiglu=swiglu, half=True)
    if swiglu:
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        return
    assert np.array_equal(a, b)
    inputs, _ = O.half_rows(x)
    ok, err = within(b, inputs.astype(np.float64) @ L.q8_dequant(g, M, K).T)
    assert ok, err


@pytest.mark.parametrize("F,K,ns", [(7680, 2048, (512, 300)), (192, 128, (20, 133)),
                                    (7680, 2048, (16, 512))])
def test_gemm_swiglu_rows_is_gemm_then_half_rows(F, K, ns):
    """The SwiGLU GEMM whose trailing blocks write the down projection's
    FP16 rows (lfm3_q8_gemm_swiglu_h16_rows) against the plain SwiGLU GEMM
    followed by lfm3_half_rows with its row maxima: y, the row maxima, the
    FP16 rows and their scales bit-exact, chunk tails zero, nothing past the
    last row; two calls in a row on the same flags (the second with another
    row count and the next sequence number), and no wait timed out."""
    lib = L.lib()
    g, u = L.q8(SEED, f"sr.g{F}", F, K), L.q8(SEED, f"sr.u{F}", F, K)
    m = DeviceMatrix(g, F, K, interleave_with=u)
    halves = half_tiles(m, 2 * F)
    flags = L.DeviceBuffer(lib.lfm3_q8_gemm_swiglu_flags_bytes(F, 512))
    L.hip_check(L.hip().hipMemset(flags.addr, 0, flags.nbytes))
    err = L.DeviceBuffer.of(np.zeros(1, np.uint32))
    blocks = lib.lfm3_q8_gemm_swiglu_max_blocks(F)
    out_ld = (F + 63) // 64 * 64 + 64
    for seq, n in enumerate(ns, start=1):
        print(f"[swiglu rows] F {F} K {K} n {n} seq {seq}", flush=True)
        x = L.normal(SEED, f"sr.x.{F}.{n}", n * K).reshape(n, K)
        da, ds, lda = half_rows_gpu(x)
        want_y, want_rm = gemm(m, x, swiglu=True, half=True)
        dy = L.DeviceBuffer(n * F * 4)
        rm = L.DeviceBuffer(blocks * n * 4)
        out = L.DeviceBuffer.of(np.full((n + 1) * out_ld, 0x7e00, np.uint16))
        sc = L.DeviceBuffer.of(np.full(n + 1, -1.0, np.float32))
        L.check(lib.lfm3_q8_gemm_swiglu_h16_rows(halves.addr, m.scales.addr, F, K, da.addr, lda,
                                                 ds.addr, n, dy.addr, F, rm.addr, out.addr,
                                                 out_ld, sc.addr, flags.addr, seq, err.addr,
                                                 None))
        L.synchronize()
        y = dy.download(np.float32, n * F).reshape(n, F)
        assert np.array_equal(y, want_y)
        assert np.array_equal(rm.download(np.uint32, blocks * n).reshape(blocks, n), want_rm)
        wa, ws, wlda = half_rows_gpu(want_y, row_max=want_rm.reshape(-1), max_blocks=blocks)
        want = wa.download(np.uint16, n * wlda).reshape(n, wlda)
        got = out.download(np.uint16, (n + 1) * out_ld).reshape(n + 1, out_ld)
        padded = (F + 63) // 64 * 64
        assert np.array_equal(got[:n, :padded], want[:, :padded])
        assert np.all(got[:n, padded:] == 0x7e00) and np.all(got[n] == 0x7e00)
        scale = sc.download(np.float32, n + 1)
        assert np.array_equal(scale[:n], ws.download(np.float32, n)) and scale[n] == -1.0
    assert err.download(np.uint32, 1)[0] == 0
