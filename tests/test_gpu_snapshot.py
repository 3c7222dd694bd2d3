"""Snapshot v2 on the GPU (Session::SaveSnapshot / RestoreSnapshot,
engine.cpp:1387-1574), following session_test.cpp:181-223: a snapshot of a
wrapped sliding ring restores exactly into the same and into a fresh
session, every corrupted header word and a truncated payload are refused
without mutation, forked continuations agree bit for bit, an intermediate
prompt snapshot computes its logits from the frontier row, and an empty
snapshot restores position 0. The bytes follow the reference's layout
(header words, FNV-1a configuration signature, sections)."""
import numpy as np
import pytest

import lfm3amd as L
from snapshot_format import HEADER_BYTES, MAGIC, VERSION, header, sections, signature, state_bytes

pytestmark = pytest.mark.gpu
SEED = L.SEED


def dims(**kw):
    base = dict(hidden=256, intermediate=512, vocab=1000, context=1024, heads=8, head_dim=128,
                kv_heads=2, window=32, pattern="CSGCCSCG")
    base.update(kw)
    return L.Dims(**base)


@pytest.fixture(scope="module")
def model():
    d = dims()
    m = L.Model(L.synth_weights(d, seed=41))
    yield d, m
    m.close()


def tokens(n, tag):
    return L.uniform_u32(SEED, f"snap.{tag}", n, 0, 999)


def test_snapshot_layout_and_exact_restore(model):
    d, m = model
    a, b = m.session(1024), m.session(1024)
    toks = tokens(400, "t")
    a.forward(toks[:300], want_logits=False)   # prompt: wraps the 32-slot sliding rings
    a.forward(toks[300:301])                   # a decode row
    data = a.save_snapshot()
    pos = a.position
    assert pos == 301 and len(data) == state_bytes(d, pos)
    assert header(data) == (MAGIC, VERSION, 1024, pos, d.hidden, d.vocab, d.n_layers,
                            signature(d))
    caps = [a.capacity(i) for i in range(d.n_layers)]
    frontier, logits, layers = sections(d, data, caps)
    want_logits = a.read_logits()
    assert np.array_equal(logits, want_logits)
    fp, _ = a.state(L.STATE_FRONTIER)
    assert np.array_equal(frontier, L.download_from(fp, np.float32, d.hidden))
    for i in range(d.n_layers):
        if d.layer_type(i) == L.LAYER_CONV:
            cp, nb = a.state(L.STATE_CONV, i)
            assert np.array_equal(layers[i], L.download_from(cp, np.float32, nb // 4))
        else:
            n = min(pos, caps[i]) * d.kv_heads * d.head_dim
            kp, _ = a.state(L.STATE_KEY, i)
            vp, _ = a.state(L.STATE_VALUE, i)
            assert np.array_equal(layers[i][0], L.download_from(kp, np.uint16, n))
            assert np.array_equal(layers[i][1], L.download_from(vp, np.uint16, n))
    # dirty the state, then restore into it and into a fresh session
    a.forward(toks[301:318], want_logits=False)
    a.restore_snapshot(data)
    b.restore_snapshot(data)
    assert a.position == b.position == pos
    assert np.array_equal(a.read_logits(), want_logits)
    assert b.save_snapshot() == data
    # every header word corrupted, and a truncated payload: refused, no mutation
    for word in range(8):
        bad = bytearray(data)
        bad[word * 4] ^= 0x80
        with pytest.raises(L.LFM3Error):
            a.restore_snapshot(bytes(bad))
        assert a.position == pos and a.coherent()
    with pytest.raises(L.LFM3Error):
        a.restore_snapshot(data[:-1])
    assert np.array_equal(a.read_logits(), want_logits)
    # forked continuations agree bit for bit, as prompts and as decode rounds
    assert np.array_equal(a.forward(toks[318:321]), b.forward(toks[318:321]))
    ra = m.forward_batch([a], toks[321:322])
    rb = m.forward_batch([b], toks[321:322])
    assert np.array_equal(ra, rb)
    a.close()
    b.close()


def test_intermediate_and_empty_snapshots(model):
    d, m = model
    a, b = m.session(1024), m.session(1024)
    toks = tokens(400, "p")
    a.forward(toks[:257], want_logits=False)
    partial = a.save_snapshot()                 # logits from the frontier row
    serial = b.forward(toks[:257])
    assert np.array_equal(a.read_logits(), serial)
    _, logits, _ = sections(d, partial, [a.capacity(i) for i in range(d.n_layers)])
    assert np.array_equal(logits, serial)
    a.forward(toks[257:276], want_logits=False)
    a.restore_snapshot(partial)
    assert np.array_equal(a.forward(toks[257:]), b.forward(toks[257:]))
    a.reset()
    empty = a.save_snapshot()
    assert len(empty) == state_bytes(d, 0) and header(empty)[3] == 0
    assert not any(empty[HEADER_BYTES:HEADER_BYTES + (d.hidden + d.vocab) * 4])
    b.restore_snapshot(empty)
    assert b.position == 0 and b.coherent()
    with pytest.raises(L.LFM3Error):
        b.read_logits()                          # no frontier at position 0
    a.close()
    b.close()


def test_reset_reproduces_exact_logits(model):
    """session_test.cpp:145-147: after a reset the same prompt gives the
    same logits bit for bit, and so does the decode row that follows."""
    d, m = model
    a = m.session(1024)
    toks = tokens(300, "reset")
    first = a.forward(toks[:290])
    step = m.forward_batch([a], toks[290:291])
    a.reset()
    assert a.position == 0
    assert np.array_equal(a.forward(toks[:290]), first)
    assert np.array_equal(m.forward_batch([a], toks[290:291]), step)
    a.close()


def test_batch_lane_snapshot_restores_its_row(model):
    """session_test.cpp:274-283: the snapshot of a batch lane, restored into
    a fresh session, serves exactly the logits row the batch returned, and
    both continue identically."""
    d, m = model
    lanes = [m.session(1024) for _ in range(3)]
    for i, s in enumerate(lanes):
        s.forward(tokens(20 + 7 * i, f"lane{i}"), want_logits=False)
    rows = m.forward_batch(lanes, tokens(3, "batchrow"))
    saved = lanes[1].save_snapshot()
    control = m.session(1024)
    control.restore_snapshot(saved)
    assert control.position == lanes[1].position
    assert np.array_equal(control.read_logits(), rows[1])
    nxt = tokens(2, "after")
    assert np.array_equal(m.forward_batch([control], nxt[:1]),
                          m.forward_batch([lanes[1]], nxt[:1]))
    for s in lanes + [control]:
        s.close()


def test_snapshot_of_another_configuration_is_refused(model):
    d, m = model
    other_dims = dims(theta_swa=2e4)             # same sizes, another signature
    other = L.Model(L.synth_weights(other_dims, seed=41))
    s = other.session(1024)
    s.forward(tokens(20, "o"))
    data = s.save_snapshot()
    assert header(data)[7] == signature(other_dims) != signature(d)
    t = m.session(1024)
    t.forward(tokens(5, "q"))
    with pytest.raises(L.LFM3Error):
        t.restore_snapshot(data)
    assert t.position == 5 and t.coherent()
    short = m.session(512)                       # another context
    with pytest.raises(L.LFM3Error):
        short.restore_snapshot(s.save_snapshot())
    for x in (s, t, short):
        x.close()
    other.close()


def test_restore_through_state_rows_serves_the_written_logits(model):
    """Session::BeginRestore / FinishRestore (engine.cpp:1372-1384): a
    continuation written row by row through the state pointers resumes with
    the logits row it carried, bit for bit, and decodes as the original."""
    d, m = model
    a, b = m.session(1024), m.session(1024)
    toks = tokens(80, "r")
    a.forward(toks[:40], want_logits=False)
    a.forward(toks[40:41])
    want = a.read_logits()
    b.forward(tokens(7, "other"))                 # dirty state to overwrite
    b.begin_restore()
    assert not b.coherent()
    with pytest.raises(L.LFM3Error):
        b.forward(toks[41:42])                    # refused while restoring
    kinds = [(L.STATE_LOGITS, 0), (L.STATE_FRONTIER, 0)]
    for i in range(d.n_layers):
        if d.layer_type(i) == L.LAYER_CONV:
            kinds.append((L.STATE_CONV, i))
        else:
            kinds += [(L.STATE_KEY, i), (L.STATE_VALUE, i)]
    for kind, layer in kinds:
        src, nbytes = a.state(kind, layer)
        dst, nbytes_b = b.state(kind, layer)
        assert nbytes == nbytes_b
        L.upload_to(dst, L.download_from(src, np.uint8, nbytes))
    b.set_position(a.position)
    assert b.coherent() and b.position == a.position
    assert np.array_equal(b.read_logits(), want)
    assert np.array_equal(b.forward(toks[41:44]), a.forward(toks[41:44]))
    a.close()
    b.close()
