"""One scheduler round (lfm3_scheduler_round): a decode batch beside a
prompt pass on two streams. Its results are checked against the oracle
(every decode row's logits at 2e-3 with the same greedy id; the pass's last
logits at session_test.cpp:120-143's prompt gate) and against the two run
one after the other (lfm3_forward_batch and lfm3_session_forward on twin
sessions, bit for bit), for prompts that overlap the round, a prompt whose
last chunk is one row (run after the round), and rounds with only one of the
two; invalid rounds are refused before any work."""
import numpy as np
import pytest

import lfm3amd as L
from gpu_util import inject_state, oracle_prompt, prompt_gate_pair, same_greedy
import oracle as O

pytestmark = pytest.mark.gpu
SEED = L.SEED


def small_dims(**kw):
    base = dict(hidden=256, intermediate=512, vocab=1000, context=2048, heads=8, head_dim=128,
                kv_heads=2, window=32, pattern="CSGCCSCG")
    base.update(kw)
    return L.Dims(**base)


def twins(gm, om, dims, positions, seed):
    """Two GPU sessions and one oracle session per position, all three at
    the same injected state."""
    a, b, o = [], [], []
    for sid, p in enumerate(positions):
        x, y = gm.session(2048), gm.session(2048)
        o1, o2 = om.session(2048), om.session(2048)
        inject_state(x, o1, dims, seed, sid, p)
        inject_state(y, o2, dims, seed, sid, p)
        o2.close()
        a.append(x)
        b.append(y)
        o.append(o1)
    return a, b, o


@pytest.mark.parametrize("n_prompt", [40, 513, 600])
def test_scheduler_round_equals_serial_work(n_prompt):
    dims = small_dims()
    w = L.synth_weights(dims, seed=61)
    gm, om = L.Model(w), O.Model(dims, w)
    positions = [3, 100, 700, 1500]
    dec, dec2, orc = twins(gm, om, dims, positions, 61)
    p1, p2 = gm.session(2048), gm.session(2048)
    po, poh = om.session(2048), om.session(2048)
    ptoks = L.uniform_u32(SEED, f"mixed.p.{n_prompt}", n_prompt, 0, dims.vocab - 1)
    toks = L.uniform_u32(SEED, "mixed.d", 4, 0, dims.vocab - 1)
    for rnd in range(2):
        ids, logits, plog = gm.scheduler_round(dec, toks, p1, ptoks, want_logits=True)
        # the oracle: each decode row one step, the prompt layer-major steps
        for i, o in enumerate(orc):
            want = o.step(int(toks[i]))
            err = same_greedy(logits[i], want, f"round {rnd} decode row {i}")
            assert err < 2e-3, (rnd, i, err)
            assert ids[i] == O.argmax(want)
        prompt_gate_pair(plog, oracle_prompt(po, ptoks), oracle_prompt(poh, ptoks, prompt=True),
                         f"round {rnd} {n_prompt}-token pass")
        # the same work one after the other, bit for bit
        want = gm.forward_batch(dec2, toks)
        pwant = p2.forward(ptoks)
        assert np.array_equal(logits, want), rnd
        assert np.array_equal(ids, np.array([O.argmax(r) for r in want], np.uint32))
        assert np.array_equal(plog, pwant), rnd
        assert [s.position for s in dec] == [s.position for s in dec2] == \
            [o.position for o in orc]
        assert p1.position == p2.position == po.position == (rnd + 1) * n_prompt
        toks = ids
    for x in dec + dec2 + [p1, p2]:
        x.close()
    for o in orc + [po, poh]:
        o.close()
    gm.close()
    om.close()


def test_scheduler_round_one_side_and_refusals():
    dims = small_dims()
    w = L.synth_weights(dims, seed=62)
    gm = L.Model(w)
    a, b, p, q = (gm.session(2048) for _ in range(4))
    toks = np.array([1, 2], np.uint32)
    ids, _, plog = gm.scheduler_round([a, b], toks)                 # decode only
    assert plog is None and a.position == b.position == 1
    _, _, plog = gm.scheduler_round([], None, p, np.arange(20, dtype=np.uint32))  # prompt only
    assert p.position == 20 and np.array_equal(plog, p.read_logits())
    q.forward(np.arange(20, dtype=np.uint32))
    assert np.array_equal(plog, q.read_logits())
    # refused before any work: a session that decodes and prefills, an
    # out-of-range prompt token, an empty round
    for bad in (lambda: gm.scheduler_round([a, p], toks, p, np.arange(5, dtype=np.uint32)),
                lambda: gm.scheduler_round([a], toks[:1], p,
                                           np.array([dims.vocab], np.uint32)),
                lambda: gm.scheduler_round([], None)):
        with pytest.raises(L.LFM3Error) as e:
            bad()
        assert e.value.status == L.E_INVALID
    assert (a.position, b.position, p.position) == (1, 1, 20)
    # a refusing prompt hook stops the whole round
    p.set_hooks(before_write=lambda first, end: 1)
    with pytest.raises(L.LFM3Error) as e:
        gm.scheduler_round([a, b], toks, p, np.arange(5, dtype=np.uint32))
    assert e.value.status == L.E_REFUSED
    assert (a.position, b.position, p.position) == (1, 1, 20)
    p.set_hooks()
    for x in (a, b, p, q):
        x.close()
    gm.close()
