"""The boundary past token prompts, on the GPU through the C-ABI.

Session::ForwardEmbeddings (engine.cpp:939-985) and Session::ForwardInputs
(engine.cpp:986-1100): input rows in place of token embeddings, against the
oracle stepping from the same rows (reference.cpp with the row in place of
the embedding lookup), and mixed token/row runs sharing 512-row passes.
Continuation hooks (continuation_hooks.hpp:6-15, engine.cpp:888-1524) and
the state inventory (continuation_layout.cpp:6-46) against the session's
own state tables. gpu::RopeFrequencies / gpu::Rope (ops_test.cpp:117-141
vectors, 2e-5) and gpu::PackKV (binary16 round to nearest even, bit-exact
against the oracle's textbook rounding)."""
import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import oracle_prompt, oracle_twin, prompt_gate, prompt_gate_pair
from test_oracle import data, powf

pytestmark = pytest.mark.gpu
SEED = L.SEED


def small_dims(**kw):
    base = dict(hidden=256, intermediate=512, vocab=1000, context=1024, heads=8, head_dim=128,
                kv_heads=2, window=32, pattern="CSGCCSCG")
    base.update(kw)
    return L.Dims(**base)


@pytest.mark.parametrize("n", [1, 5, 40, 600])
def test_forward_rows_matches_oracle(n):
    """n input rows (host memory, and the same rows from device memory on a
    twin session): logits at the prompt gate against oracle steps from the
    rows, identical across the two paths; the hidden row is the oracle's
    final-normed row."""
    dims = small_dims()
    w = L.synth_weights(dims, seed=51)
    gm, om = L.Model(w), O.Model(dims, w)
    g, g2 = gm.session(1024), gm.session(1024)
    o = om.session(1024, f16=True)
    rows = L.normal(SEED, f"rows.{n}", n * dims.hidden).reshape(n, dims.hidden) * np.float32(0.05)
    got = g.forward_rows(rows)
    dev = L.DeviceBuffer.of(np.ascontiguousarray(rows))
    got2 = g2.forward_rows(n, device_addr=dev.addr)
    assert np.array_equal(got, got2)
    oh = oracle_twin(om, o, 1024)
    want_prompt = oracle_prompt(oh, rows=rows, prompt=True)
    oh.close()
    want, hidden = None, None
    for r in rows:
        want, hidden = o.step_row(r)
    prompt_gate_pair(got, want, want_prompt, f"{n} input rows")
    assert g.position == o.position == n
    front = g.read_hidden()
    assert np.max(np.abs(front - hidden)) < 0.02 * max(1.0, float(np.max(np.abs(hidden))))
    # Decoding continues from the rows' state.
    tok = L.uniform_u32(SEED, f"rows.next.{n}", 1, 0, dims.vocab - 1)
    assert np.max(np.abs(gm.forward_batch([g], tok)[0] - o.step(int(tok[0])))) < 0.02
    for x in (g, g2, o):
        x.close()
    gm.close()
    om.close()


def test_forward_inputs_mixed_runs_equal_token_prompt():
    """Runs of tokens and of their own embedding rows (d * q in FP32, the
    values the embedding gather writes) share the 512-row passes: the result
    equals a token prompt of the same ids bit for bit, across a pass
    boundary (700 rows: passes of 512 and 188)."""
    dims = small_dims()
    w = L.synth_weights(dims, seed=52)
    gm = L.Model(w)
    a, b = gm.session(1024), gm.session(1024)
    emb = L.q8_dequant(w.globals[0][0], dims.vocab, dims.hidden).astype(np.float32)
    toks = L.uniform_u32(SEED, "mixed.tok", 700, 0, dims.vocab - 1)
    runs = [("tokens", toks[:100]), ("rows", emb[toks[100:300]]), ("tokens", toks[300:511]),
            ("rows", emb[toks[511:513]]), ("tokens", np.zeros(0, np.uint32)),
            ("tokens", toks[513:700])]
    got = a.forward_inputs(runs)
    want = b.forward(toks)
    assert np.array_equal(got, want)
    assert a.position == b.position == 700
    # Logits skipped, then read from the frontier row.
    a2, b2 = gm.session(1024), gm.session(1024)
    assert a2.forward_inputs([("rows", emb[toks[:3]]), ("tokens", toks[3:20])],
                             want_logits=False) is None
    b2.forward(toks[:20])
    assert np.array_equal(a2.read_logits(), b2.read_logits())
    for x in (a, b, a2, b2):
        x.close()
    gm.close()


def test_forward_inputs_refusals_leave_state():
    dims = small_dims()
    gm = L.Model(L.synth_weights(dims, seed=53))
    s = gm.session(64)
    s.forward(np.arange(5, dtype=np.uint32))
    rows = np.zeros((2, dims.hidden), np.float32)
    arr = (L.Input * 1)()
    keep = (np.arange(3, dtype=np.uint32), rows)
    arr[0] = L.Input(L.ptr(keep[0]), 3, L.ptr(keep[1]), 2)        # tokens and rows
    with pytest.raises(L.LFM3Error) as e:
        L.check(L.lib().lfm3_session_forward_inputs(s.handle, arr, 1, None))
    assert e.value.status == L.E_INVALID
    with pytest.raises(L.LFM3Error):
        s.forward_inputs([("tokens", np.array([1, dims.vocab], np.uint32))])
    with pytest.raises(L.LFM3Error):
        s.forward_inputs([("tokens", np.zeros(0, np.uint32))])     # nothing to run
    with pytest.raises(L.LFM3Error):
        s.forward_inputs([("rows", np.zeros((60, dims.hidden), np.float32))])  # past context
    with pytest.raises(L.LFM3Error):
        s.forward_rows(np.zeros((0, dims.hidden), np.float32))
    assert s.position == 5 and s.coherent()
    s.close()
    gm.close()


def test_continuation_hooks_see_and_can_refuse_every_change():
    """BeforeWrite gets [position, position + n) before a prompt and
    [position, position + 1) before a batch round; a refusal leaves the
    session untouched (LFM3_E_REFUSED); BeforeReset and BeforeRestore run
    first in Reset and RestoreSnapshot."""
    dims = small_dims()
    gm = L.Model(L.synth_weights(dims, seed=54))
    a, b = gm.session(256), gm.session(256)
    calls = []
    refuse = {"write": False, "reset": False, "restore": False}

    def on_write(first, end):
        calls.append(("write", first, end))
        return 1 if refuse["write"] else 0

    def on_reset():
        calls.append(("reset",))
        return 1 if refuse["reset"] else 0

    def on_restore():
        calls.append(("restore",))
        return 1 if refuse["restore"] else 0

    a.set_hooks(on_write, on_reset, on_restore)
    a.forward(np.arange(30, dtype=np.uint32), want_logits=False)
    gm.forward_batch([b, a], np.array([1, 2], np.uint32))
    a.forward_rows(np.zeros((3, dims.hidden), np.float32), want_logits=False)
    assert calls == [("write", 0, 30), ("write", 30, 31), ("write", 31, 34)]
    snap = a.save_snapshot()
    before = a.read_logits()
    refuse["write"] = True
    with pytest.raises(L.LFM3Error) as e:
        a.forward(np.array([5], np.uint32))
    assert e.value.status == L.E_REFUSED
    with pytest.raises(L.LFM3Error):
        gm.forward_batch([b, a], np.array([1, 2], np.uint32))
    assert a.position == 34 and b.position == 1 and a.coherent() and b.coherent()
    assert a.save_snapshot() == snap
    refuse["reset"] = True
    with pytest.raises(L.LFM3Error) as e:
        a.reset()
    assert e.value.status == L.E_REFUSED
    assert a.position == 34 and a.save_snapshot() == snap
    refuse["restore"] = True
    with pytest.raises(L.LFM3Error) as e:
        a.restore_snapshot(b.save_snapshot())
    assert e.value.status == L.E_REFUSED and a.save_snapshot() == snap
    assert calls[-3:] == [("write", 34, 35), ("reset",), ("restore",)]
    refuse.update(write=False, reset=False, restore=False)
    a.restore_snapshot(snap)
    assert np.array_equal(a.read_logits(), before)
    a.reset()
    assert calls[-2:] == [("restore",), ("reset",)] and a.position == 0
    a.set_hooks()                                  # cleared: no more calls
    a.forward(np.arange(3, dtype=np.uint32))
    assert calls[-1] == ("reset",)
    a.close()
    b.close()
    gm.close()


@pytest.mark.parametrize("context", [20, 700])
def test_continuation_layout_matches_session_state(context):
    """Every private component's bytes equal the session's state table of
    that part; a full-attention K/V row component times the context equals
    the ring's bytes."""
    dims = small_dims()
    gm = L.Model(L.synth_weights(dims, seed=55))
    s = gm.session(context)
    for cid, part, layer, row, state in L.continuation_layout(dims, context):
        if part == L.PART_LOGITS:
            assert state == s.state(L.STATE_LOGITS)[1]
        elif part == L.PART_FRONTIER:
            assert state == s.state(L.STATE_FRONTIER)[1]
        elif part == L.PART_METADATA:
            assert state == 16
        elif part == L.PART_CONVOLUTION:
            assert state == s.state(L.STATE_CONV, layer)[1]
        elif part == L.PART_SLIDING_WINDOW:
            assert state == s.state(L.STATE_KEY, layer)[1] + s.state(L.STATE_VALUE, layer)[1]
            assert s.capacity(layer) == min(context, dims.window)
        else:
            kind = L.STATE_KEY if part == L.PART_KEY else L.STATE_VALUE
            assert row * context == s.state(kind, layer)[1] and state == 0
    s.close()
    gm.close()


@pytest.mark.parametrize("n", [1, 8, 33])
def test_rope_reference_vectors(n):
    """ops_test.cpp:117-141 through lfm3_rope_frequencies and lfm3_rope:
    D = 128, 3 heads, P = 12001, factors 1e30 on pairs 32..63 (unchanged),
    gate 2e-5 against the float angles of std::pow(1e6f, -2i/D)."""
    D, H, P = 128, 3, 12001
    x = data(n * H * D).reshape(n, H * D)
    factors = np.ones(D // 2, np.float32)
    factors[32:] = 1e30
    dx, dfac = L.DeviceBuffer.of(x), L.DeviceBuffer.of(factors)
    dfreq = L.DeviceBuffer(D // 2 * 4)
    L.check(L.lib().lfm3_rope_frequencies(dfreq.addr, D, 1e6, None))
    L.check(L.lib().lfm3_rope(dx.addr, dfreq.addr, dfac.addr, n, H, D, P, None))
    L.synchronize()
    freq = dfreq.download(np.float32, D // 2)
    i = np.arange(D // 2)
    exact = np.power(np.float64(1e6), (np.float32(-2.0) * i.astype(np.float32)
                                       / np.float32(D)).astype(np.float64)).astype(np.float32)
    ulps = np.abs(freq.view(np.int32) - exact.view(np.int32))
    assert ulps.max() <= 1
    got = dx.download(np.float32, n * H * D).reshape(n, H, D)
    for row in range(n):
        xr = x[row].reshape(H, D).astype(np.float64)
        f = powf(1e6, np.float32(-2.0) * i.astype(np.float32) / np.float32(D))
        ang = (np.float32(P + row) * f / factors).astype(np.float32).astype(np.float64)
        want = np.concatenate([xr[:, :64] * np.cos(ang) - xr[:, 64:] * np.sin(ang),
                               xr[:, 64:] * np.cos(ang) + xr[:, :64] * np.sin(ang)], 1)
        assert np.max(np.abs(got[row] - want)) < 2e-5
        assert np.array_equal(got[row][:, 32:64], x[row].reshape(H, D)[:, 32:64])


def test_pack_kv_rounds_to_nearest_even():
    """gpu::PackKV: every value rounded to binary16 exactly as the oracle's
    textbook rounding: normal values, ties, subnormals, overflow to
    infinity, NaN."""
    specials = np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25,
                         3 * 2.0 ** -26, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf,
                         np.nan], np.float32)
    k = np.concatenate([specials, L.normal(SEED, "pack.k", 100000, 0, 10)])
    v = np.concatenate([specials[::-1], L.normal(SEED, "pack.v", 100000, 0, 1e-3)])
    dk, dv = L.DeviceBuffer.of(k), L.DeviceBuffer.of(v)
    k16, v16 = L.DeviceBuffer(k.size * 2), L.DeviceBuffer(v.size * 2)
    L.check(L.lib().lfm3_pack_kv(dk.addr, dv.addr, k16.addr, v16.addr, k.size, None))
    L.synchronize()
    gk, gv = k16.download(np.uint16, k.size), v16.download(np.uint16, v.size)
    wk, wv = O.float_to_half(k), O.float_to_half(v)
    nan_k, nan_v = np.isnan(k), np.isnan(v)
    assert np.array_equal(gk[~nan_k], wk[~nan_k]) and np.array_equal(gv[~nan_v], wv[~nan_v])
    assert np.all((gk[nan_k] & 0x7c00) == 0x7c00) and np.all(gk[nan_k] & 0x3ff)
    assert L.lib().lfm3_pack_kv(None, None, None, None, 0, None) == 0


def test_prepare_logits_runs_the_head_on_the_frontier():
    """Session::PrepareLogits (engine.cpp:1369-1373): after a round and a
    prompt without the vocabulary head, the device logits row
    (LFM3_STATE_LOGITS) holds the head on the returned frontier row: the
    oracle's tied head applied to that row (within(); the GPU's head GEMV
    reads the row as fp16 hi/lo parts), and exactly what read_logits then
    returns; logits already current are left as they are; a session at
    position 0 (no frontier) is refused."""
    from gpu_util import within
    dims = small_dims()
    w = L.synth_weights(dims, seed=56)
    gm, om = L.Model(w), O.Model(dims, w)
    a, b = gm.session(256), gm.session(256)
    with pytest.raises(L.LFM3Error) as e:
        a.prepare_logits()
    assert e.value.status == L.E_INVALID
    head = O.q8_tensor(w.globals[0][0], dims.vocab, dims.hidden)
    addr, nbytes = a.state(L.STATE_LOGITS)
    assert nbytes == dims.vocab * 4
    # a decode round without the head (ForwardBatchInputs, want_logits 0)
    gm.forward_batch_inputs([a, b], np.array([3, 9], np.uint32), [0, 0], want_logits=False)
    # a prompt without logits
    b.forward(np.arange(40, dtype=np.uint32), want_logits=False)
    for s in (a, b):
        s.prepare_logits()
        addr, _ = s.state(L.STATE_LOGITS)
        dev = L.download_from(addr, np.float32, dims.vocab)
        want = O.mat(head, s.read_hidden())
        ok, err = within(dev, want)
        assert ok, err
        assert np.array_equal(s.read_logits(), dev)
        s.prepare_logits()                      # current: unchanged
        assert np.array_equal(L.download_from(addr, np.float32, dims.vocab), dev)
    a.close()
    b.close()
    gm.close()
    om.close()
