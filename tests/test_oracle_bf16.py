"""Pins the oracle's BF16 rows and the host-side BF16 tile pack.

BF16 is the reference's numerical-reference precision (README.md:24-27);
weights.cpp:116-117 widens a BF16 value to FP32 as the high half of the
word. The reference's tests hold no BF16 vectors, so the oracle is pinned
by the closed form of that widening (known patterns: 1, -2, infinity, the
smallest subnormal), by numpy's own widening of every pattern, and by a
float64 product over the widened rows; the pack is pinned by reading the
tile layout back with numpy's reshape of the documented lane order.
"""
import numpy as np

import lfm3amd as L
import oracle as O


def test_bf16_rows_are_the_high_half_of_fp32():
    pats = np.arange(65536, dtype=np.uint16).reshape(256, 256)
    t = O.bf16_tensor(pats.ravel(), 256, 256)
    got = np.stack([O.decode_row(t, r) for r in range(256)])
    want = (pats.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    row = O.decode_row(O.bf16_tensor(np.array([0x3F80, 0xC000, 0x7F80, 0x0001], np.uint16), 1, 4),
                       0)
    assert row[0] == 1.0 and row[1] == -2.0 and np.isposinf(row[2])
    assert row[3] == np.float32(2.0) ** -133


def test_bf16_mat_matches_fp64():
    rows, cols = 300, 2048
    h = L.bf16(L.SEED, "orc.bf16", rows, cols)
    x = L.normal(L.SEED, "orc.bf16.x", cols).astype(np.float32)
    y = O.mat(O.bf16_tensor(h, rows, cols), x)
    w64 = L.bf16_to_f32(h).reshape(rows, cols).astype(np.float64)
    want = w64 @ x.astype(np.float64)
    scale = np.abs(w64) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y - want) <= 1e-6 * scale)
    # rows of the same values as FP32 tensors give the same products
    wf = L.bf16_to_f32(h)        # kept alive: the tensor view borrows it
    assert np.array_equal(O.mat(O.f32_tensor(wf, rows, cols), x), y)


def test_bf16_round_to_nearest_even():
    # the unit in the last place at 1.0 is 2^-7
    x = np.array([1.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 3 * 2.0 ** -9], np.float32)
    assert list(L.to_bf16(x)) == [0x3F80, 0x3F80, 0x3F82, 0x3F81]  # ties to even; 0.75 up
    assert list(L.to_bf16(-x)) == [0xBF80, 0xBF80, 0xBF82, 0xBF81]


def test_bf16_pack_layout():
    """lfm3_bf16_pack_host: tile [row tile][column block] of 1 KB, lane
    16 g + n holding row n's columns 8g..8g+7; padding is zero; stride 2
    interleaves two matrices by row tile."""
    for rows, cols in ((37, 96), (16, 32), (100, 2048)):
        h = L.bf16(L.SEED, f"pack.{rows}", rows, cols)
        n = L.lib().lfm3_bf16_tiled_bytes(rows, cols)
        tiles = -(-rows // 16)
        assert n == tiles * (cols // 32) * 1024
        t = np.zeros(n // 2, np.uint16)
        L.check(L.lib().lfm3_bf16_pack_host(L.ptr(h), rows, cols, L.ptr(t), 0, 1))
        back = t.reshape(tiles, cols // 32, 4, 16, 8).transpose(0, 3, 1, 2, 4).reshape(-1, cols)
        assert np.array_equal(back[:rows], h.reshape(rows, cols))
        assert not back[rows:].any()
    a, b = L.bf16(1, "ia", 32, 64), L.bf16(1, "ib", 32, 64)
    t = np.zeros(L.lib().lfm3_bf16_tiled_bytes(64, 64) // 2, np.uint16)
    L.check(L.lib().lfm3_bf16_pack_host(L.ptr(a), 32, 64, L.ptr(t), 0, 2))
    L.check(L.lib().lfm3_bf16_pack_host(L.ptr(b), 32, 64, L.ptr(t), 1, 2))
    back = t.reshape(4, 2, 4, 16, 8).transpose(0, 3, 1, 2, 4).reshape(4, 16, 64)
    assert np.array_equal(back[0::2].reshape(32, 64), a.reshape(32, 64))
    assert np.array_equal(back[1::2].reshape(32, 64), b.reshape(32, 64))


def test_f16_rows_widen_as_ieee_binary16():
    """The oracle's F16 rows (weights.cpp:118-121, Fp16ToFloat) equal
    numpy's binary16 widening for every bit pattern (NaNs compared as
    NaN)."""
    pats = np.arange(65536, dtype=np.uint16).reshape(256, 256)
    t = O.f16_tensor(pats.ravel(), 256, 256)
    got = np.stack([O.decode_row(t, r) for r in range(256)])
    want = pats.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    row = O.decode_row(O.f16_tensor(np.array([0x3C00, 0xC000, 0x7C00, 0x0001], np.uint16), 1, 4),
                       0)
    assert row[0] == 1.0 and row[1] == -2.0 and np.isposinf(row[2])
    assert row[3] == np.float32(2.0) ** -24


def test_float_pack_layouts():
    """lfm3_float_pack_host: 16-bit formats as the BF16 tiles; F32 tiles in
    two 1 KB planes, lane 16 g + n holding row n's columns 8g..8g+3 in the
    first and 8g+4..8g+7 in the second; padding zero."""
    for rows, cols in ((37, 96), (16, 32), (100, 2048)):
        a = L.f32(L.SEED, f"fpack.{rows}", rows, cols)
        n = L.lib().lfm3_float_tiled_bytes(L.TYPE_F32, rows, cols)
        tiles = -(-rows // 16)
        assert n == tiles * (cols // 32) * 2048
        t = np.zeros(n // 4, np.float32)
        L.check(L.lib().lfm3_float_pack_host(L.TYPE_F32, L.ptr(a), rows, cols, L.ptr(t), 0, 1))
        # [tile][block][plane][g][n][4] -> rows x cols
        back = t.reshape(tiles, cols // 32, 2, 4, 16, 4).transpose(0, 4, 1, 3, 2, 5)
        back = back.reshape(-1, cols)
        assert np.array_equal(back[:rows], a.reshape(rows, cols))
        assert not back[rows:].any()
        h = L.f16(L.SEED, f"fpack16.{rows}", rows, cols)
        t16 = np.zeros(L.lib().lfm3_float_tiled_bytes(L.TYPE_F16, rows, cols) // 2, np.uint16)
        L.check(L.lib().lfm3_float_pack_host(L.TYPE_F16, L.ptr(h), rows, cols, L.ptr(t16), 0, 1))
        tb = np.zeros_like(t16)
        L.check(L.lib().lfm3_bf16_pack_host(L.ptr(h), rows, cols, L.ptr(tb), 0, 1))
        assert np.array_equal(t16, tb)   # the same 16-bit element layout
    assert L.lib().lfm3_float_tiled_bytes(L.TYPE_Q8_0, 16, 32) == 0
