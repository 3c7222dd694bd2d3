"""Helpers shared by the GPU parity tests (device buffers, packing, state
injection). The oracle gives the expected results; the library does the work."""
import ctypes as C

import numpy as np

import lfm3amd as L
import oracle as O


def packed(src: np.ndarray, rows: int, cols: int):
    cb, sb = C.c_size_t(), C.c_size_t()
    L.lib().lfm3_q8_tiled_bytes(rows, cols, C.byref(cb), C.byref(sb))
    codes = np.zeros(cb.value, np.uint8)
    scales = np.zeros(sb.value, np.uint8)
    L.check(L.lib().lfm3_q8_pack_host(L.ptr(src), rows, cols, L.ptr(codes), L.ptr(scales), 0, 1))
    return codes, scales


class DeviceMatrix:
    def __init__(self, src, rows, cols, interleave_with=None):
        self.rows, self.cols = rows, cols
        if interleave_with is None:
            codes, scales = packed(src, rows, cols)
        else:
            cb, sb = C.c_size_t(), C.c_size_t()
            L.lib().lfm3_q8_tiled_bytes(rows, cols, C.byref(cb), C.byref(sb))
            codes = np.zeros(2 * cb.value, np.uint8)
            scales = np.zeros(2 * sb.value, np.uint8)
            for off, part in ((0, src), (1, interleave_with)):
                L.check(L.lib().lfm3_q8_pack_host(L.ptr(part), rows, cols, L.ptr(codes),
                                                  L.ptr(scales), off, 2))
        self.codes = L.DeviceBuffer.of(codes)
        self.scales = L.DeviceBuffer.of(scales)


def gemv(m: DeviceMatrix, x: np.ndarray, swiglu=False, ldy=None):
    B, K = x.shape
    ldy = ldy or m.rows
    dx = L.DeviceBuffer.of(np.ascontiguousarray(x, np.float32))
    dy = L.DeviceBuffer(B * ldy * 4)
    ws_bytes = L.lib().lfm3_gemv_workspace_bytes(m.rows, m.cols, B)
    ws = L.DeviceBuffer(max(ws_bytes, 256))
    fn = L.lib().lfm3_q8_gemv_swiglu if swiglu else L.lib().lfm3_q8_gemv
    L.check(fn(m.codes.addr, m.scales.addr, m.rows, m.cols, dx.addr, K, dy.addr, ldy, B,
               ws.addr, ws.nbytes, None))
    L.synchronize()
    y = dy.download(np.float32, B * ldy).reshape(B, ldy)[:, :m.rows]
    # a second call reuses the workspace (its tickets must have been reset)
    L.check(fn(m.codes.addr, m.scales.addr, m.rows, m.cols, dx.addr, K, dy.addr, ldy, B,
               ws.addr, ws.nbytes, None))
    L.synchronize()
    y2 = dy.download(np.float32, B * ldy).reshape(B, ldy)[:, :m.rows]
    assert np.array_equal(y, y2), "GEMV is not deterministic across calls"
    return y


def within(got, want, rtol=1e-3, atol=1e-4):
    """FP32 parity gate: |got - want| <= atol + rtol |want| elementwise."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    bad = np.abs(got - want) > atol + rtol * np.abs(want)
    return not bad.any(), float(np.max(np.abs(got - want))) if got.size else 0.0


def pointer_table(addrs):
    return L.DeviceBuffer.of(np.asarray(addrs, np.uint64))


def inject_state(gs: L.Session, os_: O.Session, dims: L.Dims, seed: int, sid: int,
                 position: int):
    """Synthetic prefilled state: conv history N(0, 1), K/V rings F16 N(0, 1),
    identical on the GPU session and the oracle session."""
    H, D, kv = dims.hidden, dims.head_dim, dims.kv_heads
    for l in range(dims.n_layers):
        if dims.layer_type(l) == L.LAYER_CONV:
            h = L.normal(seed, f"s{sid}.l{l}.conv", H * (dims.conv_width - 1))
            addr, nbytes = gs.state(L.STATE_CONV, l)
            assert nbytes == h.nbytes
            L.upload_to(addr, h)
            os_.conv(l)[:] = h
        else:
            cap = gs.capacity(l)
            assert cap == os_.capacity(l)
            for kind, view, tag in ((L.STATE_KEY, os_.k, "k"), (L.STATE_VALUE, os_.v, "v")):
                bits = L.half_normal(seed, f"s{sid}.l{l}.{tag}", cap * kv * D)
                addr, nbytes = gs.state(kind, l)
                assert nbytes == bits.nbytes
                L.upload_to(addr, bits)
                view(l)[:] = O.half_to_float(bits)
    gs.set_position(position)
    os_.set_position(position)
