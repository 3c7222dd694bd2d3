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


def top2_margin(logits) -> float:
    top = np.sort(np.asarray(logits, np.float32))[-2:]
    return float(top[1] - top[0])


def same_greedy(got, want, label=""):
    """The greedy id of the GPU logits is the oracle's, unconditionally
    (std::max_element's first maximum, session_test.cpp:32-34); the oracle's
    top-2 margin and the largest logit difference are printed beside it."""
    err = float(np.max(np.abs(np.asarray(got, np.float64) - want)))
    print(f"{label}: max |logit - oracle| {err:.3g}, oracle top-2 margin "
          f"{top2_margin(want):.3g}", flush=True)
    assert int(np.argmax(got)) == O.argmax(want), (label, err, top2_margin(want))
    return err


def kl_divergence(p_logits, q_logits) -> float:
    """session_test.cpp:19-31 Divergence: KL(softmax(p) || softmax(q)),
    log-softmax in float64."""
    def log_softmax(x):
        x = np.asarray(x, np.float64)
        m = x.max()
        return x - m - np.log(np.sum(np.exp(x - m)))
    lp, lq = log_softmax(p_logits), log_softmax(q_logits)
    return float(np.sum(np.exp(lp) * (lp - lq)))


def prompt_gate(got, want, label=""):
    """session_test.cpp:120-143's gate between a batched prompt pass and the
    same tokens stepped one at a time: KL(want || got) < 1e-6, max |Δlogit|
    < 0.02 and the same argmax, all unconditional."""
    got = np.asarray(got, np.float32)
    assert np.all(np.isfinite(got)) and np.all(np.isfinite(want)), label
    kl = kl_divergence(want, got)
    err = float(np.max(np.abs(got.astype(np.float64) - want)))
    print(f"{label}: max |logit - oracle| {err:.3g}, kl {kl:.3g}, oracle top-2 margin "
          f"{top2_margin(want):.3g}", flush=True)
    assert kl < 1e-6 and err < 0.02, (label, kl, err)
    assert int(np.argmax(got)) == O.argmax(want), (label, err, top2_margin(want))
    return err, kl


PROMPT_CHUNK = 512      # engine.hpp:47 kPrefillChunk


def oracle_twin(om: O.Model, o: O.Session, context: int, f16: bool = True) -> O.Session:
    """A second oracle session holding o's state and position."""
    t = om.session(context, f16=f16)
    d = om.dims
    for l in range(d.n_layers):
        if d.layer_type(l) == L.LAYER_CONV:
            t.conv(l)[:] = o.conv(l)
        else:
            t.k(l)[:] = o.k(l)
            t.v(l)[:] = o.v(l)
    t.set_position(o.position)
    return t


def oracle_prompt(o: O.Session, tokens=None, rows=None, prompt: bool = False):
    """The oracle over a prompt in the engine's 512-row chunks, layer-major
    (bit-identical to one step per token). With prompt, every chunk of two
    rows or more takes the reference's prompt-path numerics (FP16
    row-scaled projection inputs from 16 rows on, F16 attention arithmetic,
    trailing-row pruning), as the engine runs it; a one-row chunk is a
    decode row. Returns the last logits."""
    n = len(tokens) if tokens is not None else len(rows)
    out = None
    for i in range(0, n, PROMPT_CHUNK):
        m = min(PROMPT_CHUNK, n - i)
        if tokens is not None:
            out = o.steps(tokens[i:i + m], prompt_path=prompt)
        else:
            out, _ = o.steps_rows(rows[i:i + m], prompt_path=prompt)
    return out


def prompt_gate_pair(got, want, want_prompt, label=""):
    """A prompt pass against the oracle twice, with session_test.cpp:120-143's
    gate (KL < 1e-6, max |Δ| < 0.02, the same argmax) wherever the prompt
    path's own formats allow it:
    * want (reference.cpp's FP32 steps): max |Δ| < 0.02, the same argmax, and
      a KL above the prompt path's own cost, KL(want || want_prompt), by less
      than 5e-7 (half the reference gate's budget);
    * want_prompt (the oracle restating the prompt path's numerics: FP16
      row-scaled projection inputs, F16 attention query and probabilities,
      pruned rows in FP32): max |Δ| < 0.02, the same argmax, and KL below
      1e-6, or below the prompt path's own cost where that is larger. (The
      kernel rounds each probability against the running maximum of its key
      span; that rounding noise is independent of any fixed-order
      restatement, so two faithful implementations of these formats differ
      by about the formats' own cost.)"""
    got64 = np.asarray(got, np.float64)
    assert np.all(np.isfinite(got64)) and np.all(np.isfinite(want_prompt)), label
    kl_format = kl_divergence(want, want_prompt)
    err_p = float(np.max(np.abs(got64 - want_prompt)))
    kl_p = kl_divergence(want_prompt, got)
    err = float(np.max(np.abs(got64 - want)))
    kl = kl_divergence(want, got)
    print(f"{label}: vs prompt-path oracle max |Δ| {err_p:.3g}, kl {kl_p:.3g}; vs FP32 oracle "
          f"max |Δ| {err:.3g}, kl {kl:.3g}; the prompt path's own kl {kl_format:.3g}; oracle "
          f"top-2 margin {top2_margin(want):.3g}", flush=True)
    assert err_p < 0.02 and kl_p < max(1e-6, kl_format), (label, err_p, kl_p, kl_format)
    assert err < 0.02 and kl < kl_format + 5e-7, (label, err, kl, kl_format)
    assert int(np.argmax(got)) == O.argmax(want_prompt) == O.argmax(want), \
        (label, err, top2_margin(want))
