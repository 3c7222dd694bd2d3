"""lfm3_decode_heads_attention_ragged_noalloc against the workspace entry
point it mirrors (lfm3_decode_heads_attention_ragged), through the C-ABI:
identical outputs and ring rows on two calls in a row, the second with
fewer rows and shorter contexts, and a plan too large for the library's
scratch refused before any device work."""
import zlib

import numpy as np
import pytest

import lfm3amd as L
from gpu_util import pointer_table

pytestmark = pytest.mark.gpu
SEED = L.SEED
C_ITEM = L.C.sizeof(L.AttentionItem)


def run_case(n, ctx_hi, heads, kv, D, window, tag):
    """Both entry points on the same inputs (each on its own copy of the
    rings, which the fused launch writes); returns both outputs and rings."""
    ctx = L.uniform_u32(SEED, f"noalloc.ctx.{tag}", n, 1, ctx_hi)
    positions = (ctx - 1).astype(np.uint32)
    cap = window if window else ctx_hi
    stride = kv * D
    ld = (heads + 2 * kv) * D + heads
    qkv = L.normal(SEED, f"noalloc.qkv.{tag}", n * ld).reshape(n, ld)
    q_off, k_off, v_off, g_off = 0, heads * D, (heads + kv) * D, (heads + 2 * kv) * D
    qn = L.normal(SEED, "noalloc.qn", D, 1, 0.02)
    kn = L.normal(SEED, "noalloc.kn", D, 1, 0.02)
    freq = L.normal(SEED, "noalloc.freq", D // 2, 0.5, 0.1)
    rings = [(L.half_normal(SEED, f"noalloc.k{r}.{tag}", cap * stride),
              L.half_normal(SEED, f"noalloc.v{r}.{tag}", cap * stride)) for r in range(n)]
    order = np.random.default_rng(zlib.crc32(tag.encode())).permutation(n)
    cap_items = L.lib().lfm3_attention_max_items(n, int(positions.max()))
    items = (L.AttentionItem * cap_items)()
    count = L.check(L.lib().lfm3_attention_plan(L.ptr(positions), n, window, items, cap_items))
    ditems = L.DeviceBuffer(count * C_ITEM)
    L.hip_check(L.hip().hipMemcpy(ditems.addr, L.C.addressof(items), count * C_ITEM, L.H2D))
    dq = L.DeviceBuffer.of(qkv)
    dqn, dkn, dfreq = L.DeviceBuffer.of(qn), L.DeviceBuffer.of(kn), L.DeviceBuffer.of(freq)
    dpos = L.DeviceBuffer.of(positions)
    dcap = L.DeviceBuffer.of(np.full(n, cap, np.uint32))
    results = []
    for noalloc in (False, True):
        dk = [L.DeviceBuffer.of(rings[order[r]][0]) for r in range(n)]
        dv = [L.DeviceBuffer.of(rings[order[r]][1]) for r in range(n)]
        tk = pointer_table([b.addr for b in dk])
        tv = pointer_table([b.addr for b in dv])
        dout = L.DeviceBuffer(n * heads * D * 4)
        common = (dq.addr + 4 * q_off, dq.addr + 4 * k_off, dq.addr + 4 * v_off, ld,
                  dq.addr + 4 * g_off, ld, dqn.addr, dkn.addr, dfreq.addr, 0, tk.addr, tv.addr,
                  dpos.addr, dcap.addr, ditems.addr, count, dout.addr, heads * D, n, heads, kv,
                  D, 1e-5)
        if noalloc:
            L.check(L.lib().lfm3_decode_heads_attention_ragged_noalloc(*common, None))
        else:
            ws_bytes = L.lib().lfm3_attention_workspace_bytes(count, n, heads, kv, D)
            ws = L.DeviceBuffer(max(ws_bytes, 4))
            L.check(L.lib().lfm3_decode_heads_attention_ragged(*common, ws.addr, ws_bytes, None))
        L.synchronize()
        out = dout.download(np.float32, n * heads * D)
        ring_rows = [(dk[r].download(np.uint16, cap * stride), dv[r].download(np.uint16,
                                                                               cap * stride))
                     for r in range(n)]
        results.append((out, ring_rows))
    multi = any(items[i].parts > 1 for i in range(count))
    return results, multi


@pytest.mark.parametrize("heads,kv,D", [(16, 4, 128), (32, 8, 64)])
def test_noalloc_matches_workspace_entry(heads, kv, D):
    # First call: 8 rows over long histories (rows split into spans, so the
    # partials live in the scratch array); second: 3 rows, shorter.
    for n, ctx_hi, tag in ((8, 4096, f"a{heads}"), (3, 700, f"b{heads}")):
        results, multi = run_case(n, ctx_hi, heads, kv, D, 0, tag)
        (ref, ref_rings), (got, got_rings) = results
        assert multi
        assert np.all(np.isfinite(got))
        assert np.array_equal(got, ref), (n, tag)
        for (rk, rv), (gk, gv) in zip(ref_rings, got_rings):
            assert np.array_equal(rk, gk) and np.array_equal(rv, gv)


def test_noalloc_refuses_a_plan_past_its_scratch():
    heads, kv, D = 32, 8, 128
    per_item = heads * (D + 2) * 4
    items = (8 << 20) // per_item + 1
    assert L.lib().lfm3_attention_workspace_bytes(items, 8, heads, kv, D) > (8 << 20)
    dummy = L.DeviceBuffer(4096)
    with pytest.raises(L.LFM3Error) as e:
        L.check(L.lib().lfm3_decode_heads_attention_ragged_noalloc(
            dummy.addr, dummy.addr, dummy.addr, 64, dummy.addr, 64, dummy.addr, dummy.addr,
            dummy.addr, 0, dummy.addr, dummy.addr, dummy.addr, dummy.addr, dummy.addr, items,
            dummy.addr, heads * D, 8, heads, kv, D, 1e-5, None))
    assert e.value.status == L.E_INVALID and "scratch" in str(e.value)
