"""The decode round's residual norm fused into the launch of the GEMV that
consumes its operand image (lfm3_q8_gemv_image_norm,
lfm3_q8_gemv_conv_image_norm): the launch's first blocks run the norm and
publish each row through a flag; its GEMV blocks wait for the rows.

Against the same work as two launches (lfm3_residual_norm_image, then
lfm3_q8_gemv_image / lfm3_q8_gemv_swiglu_image): the GEMV outputs, the
updated residual rows, the image and its exponents equal bit for bit (the
same expressions; only the hand-over differs). The convolution projection's
fused launch runs 8 compute waves where the separate one runs 16, so its
chunk sums add in another order: 1e-5 relative, the history's shifted part
exact. Flags are reused across calls with new sequence numbers, and the
wait-error word stays clear."""
import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import DeviceMatrix, pointer_table, within

pytestmark = pytest.mark.gpu
SEED = L.SEED


class Flags:
    def __init__(self):
        self.buf = L.DeviceBuffer(L.lib().lfm3_norm_flags_bytes())
        L.hip_check(L.hip().hipMemset(self.buf.addr, 0, self.buf.nbytes))
        self.err = L.DeviceBuffer(4)
        L.hip_check(L.hip().hipMemset(self.err.addr, 0, 4))
        self.seq = 0

    def next(self):
        self.seq += 1
        return self.seq

    def error(self):
        return int(self.err.download(np.uint32, 1)[0])


def norm_inputs(tag, B, H, parts):
    x = L.normal(SEED, f"fu.x.{tag}", B * H, 0, 3).reshape(B, H)
    br = L.normal(SEED, f"fu.b.{tag}", max(parts, 1) * B * H).reshape(max(parts, 1), B, H)
    post = L.normal(SEED, f"fu.post.{tag}", H, 1, 0.02)
    wn = L.normal(SEED, f"fu.w.{tag}", H, 1, 0.02)
    return x, br, post, wn


@pytest.mark.parametrize("M,H,swiglu", [(3088, 2048, False), (7680, 2048, True),
                                        (2048, 2048, False), (64, 256, False),
                                        (512, 512, True), (8192, 2048, True)])
def test_fused_norm_gemv_equals_the_two_launches(M, H, swiglu):
    """The fused entry against the norm launch followed by the GEMV launch.
    8192 x 2048 SwiGLU (512 GEMV blocks + the norm's, more than two blocks
    a CU) takes the entry's own fallback to the two launches."""
    lib = L.lib()
    w = L.q8(SEED, f"fu.W.{M}.{H}", M, H)
    if swiglu:
        m = DeviceMatrix(w, M, H, interleave_with=L.q8(SEED, f"fu.U.{M}.{H}", M, H))
    else:
        m = DeviceMatrix(w, M, H)
    flags = Flags()
    for B, parts in ((8, 4), (3, 2), (1, 1), (8, 0)):
        print(f"[fused] M {M} H {H} swiglu {swiglu} B {B} parts {parts}", flush=True)
        x, br, post, wn = norm_inputs(f"{M}.{H}.{B}.{parts}", B, H, parts)
        dbr, dpost, dwn = L.DeviceBuffer.of(br), L.DeviceBuffer.of(post), L.DeviceBuffer.of(wn)
        branch = dbr.addr if parts else None
        n_parts = max(parts, 1)
        outs = []
        for fused in (False, True):
            dx = L.DeviceBuffer.of(x)
            img = L.DeviceBuffer(lib.lfm3_operand_image_bytes(H))
            L.hip_check(L.hip().hipMemset(img.addr, 0x7f, img.nbytes))
            ex = L.DeviceBuffer(32)
            dy = L.DeviceBuffer(B * M * 4)
            if fused:
                L.check(lib.lfm3_q8_gemv_image_norm(
                    branch, n_parts, B * H, dpost.addr, dx.addr, dwn.addr, 1e-5, img.addr,
                    ex.addr, flags.buf.addr, flags.next(), flags.err.addr, m.codes.addr,
                    m.scales.addr, M, H, int(swiglu), B, dy.addr, M, None))
            else:
                L.check(lib.lfm3_residual_norm_image(branch, n_parts, B * H, dpost.addr, dx.addr,
                                                     dwn.addr, None, img.addr, ex.addr, B, H,
                                                     1e-5, None))
                if swiglu:
                    L.check(lib.lfm3_q8_gemv_swiglu_image(m.codes.addr, m.scales.addr, M, H,
                                                          img.addr, ex.addr, B, dy.addr, M,
                                                          None))
                else:
                    L.check(lib.lfm3_q8_gemv_image(m.codes.addr, m.scales.addr, M, H, img.addr,
                                                   ex.addr, B, dy.addr, M, 1, None))
            L.synchronize()
            outs.append((dy.download(np.float32, B * M), dx.download(np.float32, B * H),
                         img.download(np.uint8, img.nbytes).reshape(-1, 64, 16),
                         ex.download(np.int32, B)))
        (y1, x1, i1, e1), (y2, x2, i2, e2) = outs
        assert np.array_equal(y1, y2) and np.array_equal(x1, x2) and np.array_equal(e1, e2)
        # the rows < B of every image word (lanes 16 g + r, r and r + 8 < 16)
        lanes = [16 * g + r for g in range(4) for r in list(range(B)) + list(range(8, 8 + B))]
        assert np.array_equal(i1[:, lanes], i2[:, lanes])
        # the residual rows follow the oracle (x += post(sum of parts))
        if parts:
            branch = br[0].copy()
            for p in range(1, parts):      # part order, FP32
                branch = branch + br[p]
            want = x + np.stack([O.norm(branch[r], post, 1e-5) for r in range(B)])
            np.testing.assert_allclose(x2.reshape(B, H), want, rtol=1e-5, atol=1e-5)
    assert flags.error() == 0


@pytest.mark.parametrize("H,B", [(2048, 8), (2048, 3), (256, 1)])
def test_fused_norm_conv_projection(H, B):
    lib = L.lib()
    Lw = 7
    w = L.q8(SEED, f"fc.W{H}", 3 * H, H)
    m = DeviceMatrix(w, 3 * H, H)
    taps = L.normal(SEED, f"fc.taps{H}", H * Lw, 0, 0.1)
    hist = [L.normal(SEED, f"fc.h{H}.{i}", H * (Lw - 1)) for i in range(B)]
    dt = L.DeviceBuffer.of(taps)
    x, br, post, wn = norm_inputs(f"c{H}.{B}", B, H, 4)
    dbr, dpost, dwn = L.DeviceBuffer.of(br), L.DeviceBuffer.of(post), L.DeviceBuffer.of(wn)
    flags = Flags()
    res = []
    for fused in (False, True):
        dx = L.DeviceBuffer.of(x)
        img = L.DeviceBuffer(lib.lfm3_operand_image_bytes(H))
        ex = L.DeviceBuffer(32)
        dh = [L.DeviceBuffer.of(h) for h in hist]
        tb = pointer_table([b.addr for b in dh])
        dy = L.DeviceBuffer(B * H * 4)
        if fused:
            L.check(lib.lfm3_q8_gemv_conv_image_norm(
                dbr.addr, 4, B * H, dpost.addr, dx.addr, dwn.addr, 1e-5, img.addr, ex.addr,
                flags.buf.addr, flags.next(), flags.err.addr, m.codes.addr, m.scales.addr, H, B,
                dt.addr, tb.addr, Lw, dy.addr, H, None))
        else:
            L.check(lib.lfm3_residual_norm_image(dbr.addr, 4, B * H, dpost.addr, dx.addr,
                                                 dwn.addr, None, img.addr, ex.addr, B, H, 1e-5,
                                                 None))
            L.check(lib.lfm3_q8_gemv_conv_image(m.codes.addr, m.scales.addr, H, img.addr,
                                                ex.addr, B, dt.addr, tb.addr, Lw, dy.addr, H,
                                                None))
        L.synchronize()
        res.append((dy.download(np.float32, B * H), dx.download(np.float32, B * H),
                    [b.download(np.float32, H * (Lw - 1)) for b in dh]))
    (y1, x1, h1), (y2, x2, h2) = res
    assert np.array_equal(x1, x2)
    ok, err = within(y2, y1, rtol=1e-5, atol=1e-6)
    assert ok, err
    for r in range(B):
        ok, err = within(h2[r], h1[r], rtol=1e-5, atol=1e-6)
        assert ok, (r, err)
        keep = hist[r].reshape(H, Lw - 1)[:, 1:]
        assert np.array_equal(h2[r].reshape(H, Lw - 1)[:, :-1], keep)
    assert flags.error() == 0
