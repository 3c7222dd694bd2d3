"""Session::Forward on the GPU (engine.cpp:882-938): a prompt of n tokens in
chunks of 512 rows against the CPU oracle stepping the same tokens one at a
time (reference.cpp), then decode rounds continuing from the prompt's state.

The prompt path rounds activations to FP16 (per-row power-of-two scales)
and attention probabilities to F16, where the oracle keeps FP32; the gate
on the last token's logits is session_test.cpp:120-143's (KL < 1e-6, max
|logit| < 0.02, the same argmax, unconditionally) against the oracle with
the prompt path's FP16 row-scaled projection inputs, and against the FP32
oracle max |logit| < 0.02, the same argmax, and a KL within 5e-7 of the
FP16 format's own. Invalid calls are refused
without touching state (engine.cpp:904-913)."""
import numpy as np
import pytest

import lfm3amd as L
import oracle as O
from gpu_util import inject_state, oracle_prompt, oracle_twin, prompt_gate_pair

pytestmark = pytest.mark.gpu
SEED = L.SEED


def small_dims(**kw):
    base = dict(hidden=256, intermediate=512, vocab=1000, context=1024, heads=8, head_dim=128,
                kv_heads=2, window=32, pattern="CSGCCSCG")
    base.update(kw)
    return L.Dims(**base)


@pytest.mark.parametrize("n", [2, 5, 15, 16, 40, 300, 600])
@pytest.mark.parametrize("start", [0, 97])
def test_prompt_matches_oracle_steps(n, start):
    """Prompts below 16 rows (FP32 projections), at 16 and above (FP16
    prompt path), and past one 512-row chunk, from an empty session and
    from an injected state at position 97."""
    dims = small_dims()
    w = L.synth_weights(dims, seed=31)
    gm, om = L.Model(w), O.Model(dims, w)
    g, o = gm.session(1024), om.session(1024, f16=True)
    if start:
        inject_state(g, o, dims, 31, 0, start)
    oh = oracle_twin(om, o, 1024)
    tokens = L.uniform_u32(SEED, f"prompt.tok.{n}.{start}", n, 0, dims.vocab - 1)
    got = g.forward(tokens)
    want = oracle_prompt(o, tokens)
    prompt_gate_pair(got, want, oracle_prompt(oh, tokens, prompt=True),
                     f"{n}-token prompt from {start}")
    oh.close()
    assert g.position == o.position == start + n
    assert np.array_equal(g.read_logits(), got)
    # Decode continues from the prompt's state.
    for step in range(3):
        tok = L.uniform_u32(SEED, f"prompt.next.{n}.{start}.{step}", 1, 0, dims.vocab - 1)
        got = gm.forward_batch([g], tok)[0]
        want = o.step(int(tok[0]))
        err = float(np.max(np.abs(got - want)))
        assert err < 0.02, (step, err)


@pytest.mark.parametrize("dims_kw", [dict(heads=8, kv_heads=4, head_dim=64),
                                     dict(heads=16, kv_heads=2, head_dim=64, pattern="GSC"),
                                     dict(pattern="CCSCGCCSCGCCSCGCSCGCSCGG", hidden=256,
                                          intermediate=512),
                                     dict(hidden=512, intermediate=1024)])
def test_prompt_other_shapes(dims_kw):
    """Other head shapes, a prompt ending on a convolution layer, the
    24-layer pattern (13 conv, 5 sliding, 6 global; last layer global, so
    the last layer's FFN runs on the frontier row only), and a hidden size
    of 512, where the attention input projection runs in two K parts that
    the heads kernel adds."""
    dims = small_dims(**dims_kw)
    if dims.hidden == 512:
        qkvg = dims.heads * dims.head_dim + 2 * dims.kv_heads * dims.head_dim + dims.heads
        assert L.lib().lfm3_q8_gemm_parts(qkvg, dims.hidden, 200, 0) == 2
    w = L.synth_weights(dims, seed=32)
    gm, om = L.Model(w), O.Model(dims, w)
    g, o = gm.session(1024), om.session(1024, f16=True)
    oh = om.session(1024, f16=True)
    tokens = L.uniform_u32(SEED, f"prompt.shapes.{dims.pattern}", 200, 0, dims.vocab - 1)
    got = g.forward(tokens)
    prompt_gate_pair(got, oracle_prompt(o, tokens), oracle_prompt(oh, tokens, prompt=True),
                     f"200-token prompt, {dims.pattern}")


def test_prompt_state_matches_oracle():
    """After a 300-token prompt: every convolution history and every K/V
    ring (global rows 0..299, the sliding ring's last window rows) is within
    the prompt gate of the oracle's state."""
    dims = small_dims()
    w = L.synth_weights(dims, seed=33)
    gm, om = L.Model(w), O.Model(dims, w)
    g, o = gm.session(1024), om.session(1024, f16=True)
    n = 300
    tokens = L.uniform_u32(SEED, "prompt.state", n, 0, dims.vocab - 1)
    g.forward(tokens, want_logits=False)
    oracle_prompt(o, tokens)
    def read(kind, layer, dtype):
        addr, nbytes = g.state(kind, layer)
        return L.download_from(addr, dtype, nbytes // np.dtype(dtype).itemsize)

    for layer, kind in enumerate(dims.pattern):
        if kind == "C":
            got = read(L.STATE_CONV, layer, np.float32)
            assert np.max(np.abs(got - o.conv(layer))) < 0.02, layer
        else:
            cap = g.capacity(layer)
            rows = min(n, cap)
            gk = O.half_to_float(read(L.STATE_KEY, layer, np.uint16))
            gv = O.half_to_float(read(L.STATE_VALUE, layer, np.uint16))
            slots = [(t % cap) for t in range(n - rows, n)]
            assert np.max(np.abs(gk.reshape(cap, -1)[slots] - o.k(layer).reshape(cap, -1)[slots])) < 0.02
            assert np.max(np.abs(gv.reshape(cap, -1)[slots] - o.v(layer).reshape(cap, -1)[slots])) < 0.02


def test_prompt_refusals_leave_state():
    dims = small_dims()
    w = L.synth_weights(dims, seed=34)
    gm = L.Model(w)
    g = gm.session(64)
    with pytest.raises(L.LFM3Error) as e:
        g.forward(np.zeros(0, np.uint32))
    assert e.value.status == L.E_INVALID
    with pytest.raises(L.LFM3Error):
        g.forward(np.zeros(65, np.uint32))  # more than the context holds
    with pytest.raises(L.LFM3Error):
        g.forward(np.array([1, 2, dims.vocab], np.uint32))
    assert g.position == 0
    g.forward(np.arange(40, dtype=np.uint32))
    assert g.position == 40
    with pytest.raises(L.LFM3Error):
        g.forward(np.zeros(25, np.uint32))  # 40 + 25 > 64
    assert g.position == 40 and g.coherent()
