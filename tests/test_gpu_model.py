"""Engine parity on the GPU: ForwardBatch rounds of ragged sessions against
the CPU oracle stepping each session alone (reference.cpp), plus the
reference's session-level contracts (session_test.cpp:224-283: batched rows
equal independent serial sessions with the same greedy token; invalid
batches are refused without mutating state)."""
import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import inject_state, same_greedy, within

pytestmark = pytest.mark.gpu
SEED = L.SEED


def small_dims(**kw):
    base = dict(hidden=256, intermediate=512, vocab=1000, context=1024, heads=8, head_dim=128,
                kv_heads=2, window=32, pattern="CSGCCSCG")
    base.update(kw)
    return L.Dims(**base)


def build(dims, seed, positions, context):
    w = L.synth_weights(dims, seed=seed)
    gm = L.Model(w)
    om = O.Model(dims, w)
    gs, os_ = [], []
    for sid, p in enumerate(positions):
        g = gm.session(context)
        o = om.session(context, f16=True)
        inject_state(g, o, dims, seed, sid, int(p))
        gs.append(g)
        os_.append(o)
    return w, gm, om, gs, os_


@pytest.mark.parametrize("dims_kw", [{}, dict(heads=8, kv_heads=4, head_dim=64),
                                     dict(heads=16, kv_heads=2, head_dim=64, pattern="GSC")])
def test_forward_batch_matches_oracle(dims_kw):
    dims = small_dims(**dims_kw)
    n = 8
    positions = L.uniform_u32(SEED, "eng.pos", n, 0, 600)
    w, gm, om, gs, os_ = build(dims, 21, positions, 1024)
    worst = 0.0
    for step in range(3):
        toks = L.uniform_u32(SEED, f"eng.tok{step}", n, 0, dims.vocab - 1)
        logits = gm.forward_batch(gs, toks)
        for i in range(n):
            want = os_[i].step(int(toks[i]))
            err = same_greedy(logits[i], want, f"step {step} row {i}")
            worst = max(worst, err)
            assert err < 2e-3, (step, i, err)
            assert gs[i].position == os_[i].position == positions[i] + step + 1
            assert np.array_equal(gs[i].read_logits(), logits[i])
    print(f"max |logit - oracle| = {worst:.3g}")


def test_batch_rows_equal_serial_sessions():
    """session_test.cpp:224-283: C2..C8 batches equal independent sessions.
    Row arithmetic never depends on the other rows here, so equality is
    exact."""
    dims = small_dims()
    positions = [1, 33, 257, 513, 2, 40, 300, 700]
    w = L.synth_weights(dims, seed=22)
    gm = L.Model(w)
    om = O.Model(dims, w)
    lanes, controls = [], []
    for sid, p in enumerate(positions):
        a, b = gm.session(1024), gm.session(1024)
        o1, o2 = om.session(1024), om.session(1024)
        inject_state(a, o1, dims, 22, sid, p)
        inject_state(b, o2, dims, 22, sid, p)
        lanes.append(a)
        controls.append(b)
    for width in (2, 3, 4, 8):
        toks = L.uniform_u32(SEED, f"bs.tok{width}", width, 0, dims.vocab - 1)
        batch = gm.forward_batch(lanes[:width], toks)
        for i in range(width):
            alone = gm.forward_batch([controls[i]], toks[i:i + 1])[0]
            assert np.array_equal(batch[i], alone)
            assert lanes[i].position == controls[i].position
    ids = gm.forward_batch_greedy(lanes, np.arange(8, dtype=np.uint32))
    for i in range(8):
        assert ids[i] == int(np.argmax(lanes[i].read_logits()))


def test_invalid_batches_are_refused_without_mutation():
    dims = small_dims()
    w = L.synth_weights(dims, seed=23)
    gm = L.Model(w)
    a, b = gm.session(16), gm.session(16)
    toks = np.array([1, 2], np.uint32)
    for bad in ([a, a], ):
        with pytest.raises(L.LFM3Error) as e:
            gm.forward_batch(bad, toks)
        assert e.value.status == L.E_INVALID
    with pytest.raises(L.LFM3Error):
        gm.forward_batch([a, b], np.array([1, dims.vocab], np.uint32))
    with pytest.raises(L.LFM3Error):
        gm.forward_batch([a] * 9, np.zeros(9, np.uint32))
    assert a.position == 0 and b.position == 0 and a.coherent() and b.coherent()
    a.set_position(16)   # context exhausted
    with pytest.raises(L.LFM3Error):
        gm.forward_batch([a, b], toks)
    assert b.position == 0
    a.reset()
    gm.forward_batch([a, b], toks)
    assert a.position == 1 and b.position == 1


def test_batch_of_two_models_is_refused():
    """engine.cpp:1188-1192: every session of a batch must belong to the
    front session's model; a mixed batch is refused and nothing moves."""
    dims = small_dims()
    g1 = L.Model(L.synth_weights(dims, seed=31))
    g2 = L.Model(L.synth_weights(dims, seed=32))
    a, b = g1.session(16), g2.session(16)
    with pytest.raises(L.LFM3Error) as e:
        g1.forward_batch([a, b], np.array([1, 2], np.uint32))
    assert e.value.status == L.E_INVALID and "incompatible" in str(e.value)
    assert a.position == 0 and b.position == 0
    g1.forward_batch([a], np.array([1], np.uint32))
    assert a.position == 1


def test_sliding_ring_wraps_across_rounds():
    """Ten rounds past a 32-slot ring: logits keep matching the oracle."""
    dims = small_dims(pattern="SCS")
    positions = [29, 30, 31, 95]
    w, gm, om, gs, os_ = build(dims, 24, positions, 1024)
    for step in range(10):
        toks = L.uniform_u32(SEED, f"wrap{step}", 4, 0, dims.vocab - 1)
        logits = gm.forward_batch(gs, toks)
        for i in range(4):
            want = os_[i].step(int(toks[i]))
            assert np.max(np.abs(logits[i] - want)) < 2e-3


def test_full_reference_dims_round():
    """LFM3-1.7B dims (24 layers, 13 conv / 5 sliding / 6 global, FFN 7680,
    16/4 heads x 128, vocab 128000) with random-init Q8_0 weights: one
    two-session round against the oracle, greedy ids identical."""
    dims = L.Dims(context=4096)
    positions = [150, 700]
    w, gm, om, gs, os_ = build(dims, SEED, positions, 1024)
    toks = np.array([11, 90000], np.uint32)
    logits = gm.forward_batch(gs, toks)
    for i in range(2):
        want = os_[i].step(int(toks[i]))
        err = same_greedy(logits[i], want, f"row {i}")
        assert err < 2e-3


def test_forward_batch_inputs_rows_and_tokens():
    """Session::ForwardBatchInputs (engine.cpp:1217-1299): device FP32 rows
    stand in for some sessions' token embeddings. Rows equal to the token's
    dequantized embedding row give the token round exactly; arbitrary rows
    match the oracle stepping from the same row; out-of-range tokens are
    accepted where a row replaces them."""
    dims = small_dims()
    n = 6
    positions = L.uniform_u32(SEED, "inp.pos", n, 0, 600)
    w, gm, om, gs, os_ = build(dims, 31, positions, 1024)
    _, gm2, _, gs2, _ = build(dims, 31, positions, 1024)
    emb = L.q8_dequant(w.globals[0][0], dims.vocab, dims.hidden).astype(np.float32)
    toks = L.uniform_u32(SEED, "inp.tok", n, 0, dims.vocab - 1)
    # Embedding rows in place of tokens 0, 2, 4: identical to the token round.
    erows = [L.DeviceBuffer.of(emb[int(toks[i])]) if i % 2 == 0 else None for i in range(n)]
    want = gm2.forward_batch(gs2, toks)
    got = gm.forward_batch_inputs(gs, toks, [r.addr if r else 0 for r in erows])
    assert np.array_equal(got, want)
    for i in range(n):
        os_[i].step(int(toks[i]), logits=False)
    # Arbitrary rows (and a token id past the vocabulary under a row).
    rows = [L.normal(SEED, f"inp.row{i}", dims.hidden) * np.float32(0.05) for i in range(n)]
    drows = [L.DeviceBuffer.of(r) if i != 1 else None for i, r in enumerate(rows)]
    toks2 = L.uniform_u32(SEED, "inp.tok2", n, 0, dims.vocab - 1)
    toks2[0] = dims.vocab + 5
    got = gm.forward_batch_inputs(gs, toks2, [r.addr if r else 0 for r in drows])
    for i in range(n):
        if drows[i] is None:
            ref = os_[i].step(int(toks2[i]))
        else:
            ref, _ = os_[i].step_row(rows[i])
        err = float(np.max(np.abs(got[i] - ref)))
        assert err < 2e-3, (i, err)
        assert gs[i].position == os_[i].position
    # Without logits: positions and frontier rows advance; reading logits
    # then runs the head on the frontier row (EnsureLogits, engine.cpp:237-245).
    got = gm.forward_batch_inputs(gs, toks, [r.addr if r else 0 for r in drows],
                                  want_logits=False)
    assert got is None
    for i in range(n):
        if drows[i] is None:
            ref, hidden = os_[i].step(int(toks[i])), None
        else:
            ref, hidden = os_[i].step_row(rows[i])
        ptr, nbytes = gs[i].state(L.STATE_FRONTIER)
        front = L.download_from(ptr, np.float32, dims.hidden)
        if hidden is not None:
            assert np.max(np.abs(front - hidden)) < 2e-4 * max(1.0, np.max(np.abs(hidden)))
        assert gs[i].position == os_[i].position
        err = float(np.max(np.abs(gs[i].read_logits() - ref)))
        assert err < 2e-3, (i, err)
    # A token past the vocabulary without a row is refused, state untouched.
    before = [s.position for s in gs]
    bad = toks.copy()
    bad[3] = dims.vocab
    with pytest.raises(L.LFM3Error):
        gm.forward_batch_inputs(gs, bad, [0] * n)
    assert [s.position for s in gs] == before and all(s.coherent() for s in gs)


def test_two_host_threads_on_one_model():
    """Calls on sessions of one model from two host threads (the model's
    lock serializes them; ctypes releases the GIL, so the calls really
    overlap on the host) give the single-threaded results bit for bit:
    thread 1 runs decode rounds of two sessions, thread 2 prompts and
    snapshots of a third, against twins run one after the other."""
    import threading
    dims = L.Dims(hidden=256, intermediate=512, vocab=1000, context=2048, heads=8,
                  head_dim=128, kv_heads=2, window=32, pattern="CSGCCSCG")
    w = L.synth_weights(dims, seed=57)
    gm = L.Model(w)
    dec = [gm.session(1024) for _ in range(2)]
    dec2 = [gm.session(1024) for _ in range(2)]
    p, p2 = gm.session(1024), gm.session(1024)
    prompts = [L.uniform_u32(SEED, f"threads.p{i}", 40 + 37 * i, 0, dims.vocab - 1)
               for i in range(4)]
    toks = L.uniform_u32(SEED, "threads.d", 2, 0, dims.vocab - 1)
    got_dec, got_p, errors = [], [], []

    def decode():
        try:
            t = toks
            for _ in range(12):
                got_dec.append(gm.forward_batch(dec, t))
                t = np.array([O.argmax(r) for r in got_dec[-1]], np.uint32)
        except Exception as e:          # noqa: BLE001 - reported below
            errors.append(e)

    def prompt():
        try:
            for toks_p in prompts:
                got_p.append((p.forward(toks_p), p.save_snapshot()))
        except Exception as e:          # noqa: BLE001
            errors.append(e)

    workers = [threading.Thread(target=decode), threading.Thread(target=prompt)]
    for t in workers:
        t.start()
    for t in workers:
        t.join()
    assert not errors, errors
    t = toks
    for r in range(12):
        want = gm.forward_batch(dec2, t)
        assert np.array_equal(got_dec[r], want), r
        t = np.array([O.argmax(x) for x in want], np.uint32)
    for i, toks_p in enumerate(prompts):
        want = p2.forward(toks_p)
        assert np.array_equal(got_p[i][0], want), i
        assert got_p[i][1] == p2.save_snapshot(), i
    for s in dec + dec2 + [p, p2]:
        s.close()
    gm.close()
