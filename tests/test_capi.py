"""CPU checks of the C-ABI library: it loads, exports every declared entry
point, and its host-side logic (tile packing, attention work lists,
synthetic inputs, input validation) follows its integer closed forms. No
kernel runs here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import lfm3amd as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lfm3_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lfm3_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding covers all of them
    assert set(names) <= set(L._SIGS)


def test_synthetic_inputs_are_deterministic():
    a = L.normal(L.SEED, "x", 300000)
    b = L.normal(L.SEED, "x", 300000)
    c = L.normal(L.SEED, "y", 300000)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    # element i does not depend on how many were drawn
    assert np.array_equal(L.normal(L.SEED, "x", 1000), a[:1000])
    w = L.q8(L.SEED, "w", 64, 256)
    blocks = w.reshape(-1, 34)
    q = blocks[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127 and len(np.unique(q)) > 250
    d = blocks[:, :2].copy().view(np.float16).astype(np.float64)
    assert (d >= 0).all() and abs(np.mean(d) * 127 - 0.02 * np.sqrt(2 / np.pi)) < 2e-3
    u = L.uniform_u32(L.SEED, "u", 100000, 1, 4096)
    assert u.min() >= 1 and u.max() <= 4096 and abs(u.mean() - 2048.5) < 30


def unpack_tiles(codes, scales, rows, cols, tile_offset=0, tile_stride=1, tiles=None):
    """Inverse of the documented tile layout: lane 16 g + n of tile
    (r / 16, chunk) holds row n, bytes [0,8) block 2c elements 8g.., [8,16)
    block 2c + 1 elements 8g..; codes stored biased (q ^ 0x80); scales
    [row][block] per tile."""
    nchunks = (cols + 63) // 64
    q = np.zeros((rows, nchunks * 64), np.int8)
    d = np.zeros((rows, nchunks * 2), np.uint16)
    t = (codes ^ 0x80).reshape(-1, nchunks, 4, 16, 16)      # tile, chunk, g, n, byte
    s = scales.view(np.uint16).reshape(-1, nchunks, 16, 2)
    for r in range(rows):
        tile = tile_offset + (r // 16) * tile_stride
        n = r % 16
        for c in range(nchunks):
            for g in range(4):
                q[r, c * 64 + 8 * g:c * 64 + 8 * g + 8] = t[tile, c, g, n, :8].view(np.int8)
                q[r, c * 64 + 32 + 8 * g:c * 64 + 32 + 8 * g + 8] = t[tile, c, g, n, 8:].view(np.int8)
            d[r, 2 * c:2 * c + 2] = s[tile, c, n]
    return q[:, :cols], d[:, :cols // 32], q[:, cols:], d[:, cols // 32:]


@pytest.mark.parametrize("rows,cols", [(37, 96), (16, 64), (48, 2048), (5, 32)])
def test_host_pack_round_trip(rows, cols):
    src = L.q8(3, f"p{rows}x{cols}", rows, cols)
    cb, sb = C.c_size_t(), C.c_size_t()
    L.lib().lfm3_q8_tiled_bytes(rows, cols, C.byref(cb), C.byref(sb))
    tiles = (rows + 15) // 16
    nchunks = (cols + 63) // 64
    assert cb.value == tiles * nchunks * 1024 and sb.value == tiles * nchunks * 64
    codes = np.full(cb.value, 0x5a, np.uint8)
    scales = np.full(sb.value, 0x5a, np.uint8)
    L.check(L.lib().lfm3_q8_pack_host(L.ptr(src), rows, cols, L.ptr(codes), L.ptr(scales), 0, 1))
    q, d, q_pad, d_pad = unpack_tiles(codes, scales, rows, cols)
    blocks = src.reshape(rows, cols // 32, 34)
    assert np.array_equal(q, blocks[:, :, 2:].view(np.int8).reshape(rows, cols))
    assert np.array_equal(d, blocks[:, :, :2].copy().view(np.uint16).reshape(rows, cols // 32))
    assert not q_pad.any() and not d_pad.any()
    # padding rows of the last tile hold the code of zero too
    t = (codes ^ 0x80).reshape(tiles, nchunks, 4, 16, 16)
    if rows % 16:
        assert not t[-1, :, :, rows % 16:, :].any()


def test_host_pack_interleave_and_concat():
    rows, cols = 32, 128
    a = L.q8(4, "a", rows, cols)
    b = L.q8(4, "b", rows, cols)
    nchunks = 2
    codes = np.zeros(4 * nchunks * 1024, np.uint8)
    scales = np.zeros(4 * nchunks * 64, np.uint8)
    L.check(L.lib().lfm3_q8_pack_host(L.ptr(a), rows, cols, L.ptr(codes), L.ptr(scales), 0, 2))
    L.check(L.lib().lfm3_q8_pack_host(L.ptr(b), rows, cols, L.ptr(codes), L.ptr(scales), 1, 2))
    qa, _, _, _ = unpack_tiles(codes, scales, rows, cols, 0, 2)
    qb, _, _, _ = unpack_tiles(codes, scales, rows, cols, 1, 2)
    assert np.array_equal(qa, a.reshape(rows, -1, 34)[:, :, 2:].view(np.int8).reshape(rows, cols))
    assert np.array_equal(qb, b.reshape(rows, -1, 34)[:, :, 2:].view(np.int8).reshape(rows, cols))


def plan(positions, window, capacity=4096):
    pos = np.ascontiguousarray(positions, np.uint32)
    items = (L.AttentionItem * capacity)()
    n = L.check(L.lib().lfm3_attention_plan(L.ptr(pos), len(pos), window, items, capacity))
    return [items[i] for i in range(n)]


@pytest.mark.parametrize("window", [0, 256])
def test_attention_plan_covers_each_row_exactly(window):
    positions = L.uniform_u32(L.SEED, "ctx", 8, 1, 4096) - 1
    positions = np.concatenate([positions, [0, 255, 256, 257, 511, 512]]).astype(np.uint32)
    items = plan(positions, window)
    # one span length per call: a multiple of 64 in [64, 1024], about a
    # 128th of the keys; a window of at most 256 keys is a single span
    keys = [int(p) + 1 - (max(0, int(p) + 1 - window) if window else 0) for p in positions]
    span = max(it.key_end - it.key_begin for it in items)
    assert span % 64 == 0 and 64 <= span <= 1024
    per_item = -(-sum(keys) // 128)
    want = min(1024, max(64, (per_item + 63) // 64 * 64))
    if 0 < window <= 256:
        want = max(want, window)
        assert len(items) == len(positions)
    assert span == want
    assert len(items) <= L.lib().lfm3_attention_max_items(len(positions), int(max(positions)))
    by_row = {}
    for idx, it in enumerate(items):
        by_row.setdefault(it.row, []).append((idx, it))
    assert sorted(by_row) == list(range(len(positions)))
    for r, lst in by_row.items():
        p = int(positions[r])
        first = max(0, p + 1 - window) if window else 0
        spans = [(it.key_begin, it.key_end) for _, it in lst]
        assert spans[0][0] == first and spans[-1][1] == p + 1
        for (b0, e0), (b1, e1) in zip(spans, spans[1:]):
            assert e0 == b1
        assert all(0 < e - b <= span for b, e in spans)
        assert all(e - b == span for b, e in spans[:-1])
        assert all(it.parts == len(lst) and it.first_item == lst[0][0] for _, it in lst)
        assert len(lst) <= 256


def test_attention_plan_refuses_overflow():
    with pytest.raises(L.LFM3Error):
        plan([10000], 0, capacity=8)


def test_model_load_rejects_bad_inputs_before_device_work():
    dims = L.Dims(hidden=128, intermediate=192, vocab=300, context=64, heads=4, head_dim=64,
                  kv_heads=2, window=8, pattern="CSG")
    w = L.synth_weights(dims, seed=1)
    bad = L.Dims(**{**dims.__dict__, "head_dim": 96})
    with pytest.raises(L.LFM3Error) as e:
        L.Model(L.Weights(bad, w.globals, w.layers))
    assert e.value.status == L.E_INVALID
    # a Q8 tensor with the wrong row count
    layers = [list(t) for t in w.layers]
    data, typ, cols, rows = layers[0][8]
    layers[0][8] = (data, typ, cols, rows - 16)
    with pytest.raises(L.LFM3Error) as e:
        L.Model(L.Weights(dims, w.globals, layers))
    assert e.value.status == L.E_INVALID and "in_proj" in str(e.value)
    # a non-positive RoPE factor (weights.cpp:59-63)
    g = list(w.globals)
    g[3] = (np.zeros(32, np.float32), L.TYPE_F32, 32, 1)
    with pytest.raises(L.LFM3Error) as e:
        L.Model(L.Weights(dims, g, w.layers))
    assert "RoPE" in str(e.value)


def test_kernel_entry_points_refuse_unsupported_shapes():
    lib = L.lib()
    # Q8_0 needs cols % 32 == 0 and 1..8 rows; attention needs dim 64/128.
    assert lib.lfm3_q8_gemv(1, 1, 16, 40, 16, 40, 1, 16, 1, None, 0, None) == L.E_INVALID
    assert lib.lfm3_q8_gemv(1, 1, 16, 64, 16, 64, 1, 16, 9, None, 0, None) == L.E_INVALID
    assert lib.lfm3_decode_attention_ragged(1, 8, 1, 8, 1, 1, 1, 1, 1, 1, 8, 1, 6, 2, 96,
                                            1, 1 << 20, None) == L.E_INVALID
    assert lib.lfm3_decode_attention_ragged(1, 8, 1, 8, 1, 1, 1, 1, 1, 1, 8, 1, 6, 2, 128,
                                            1, 1 << 20, None) == L.E_INVALID  # group 3
    assert b"attention" in lib.lfm3_last_error()


def test_prompt_attention_rejects_bad_shapes():
    """Unsupported dimension or group, and a split history without its
    workspace, are refused before any launch."""
    lib = L.lib()
    assert lib.lfm3_prompt_attention(1, 512, 1, 1, 1, 4, 1, 1, 1, 512, 8, 4, 2, 96, 0, 1, 0,
                                     None, 0, None) == L.E_INVALID
    assert lib.lfm3_prompt_attention(1, 768, 1, 1, 1, 6, 1, 1, 1, 768, 8, 6, 2, 128, 0, 1, 0,
                                     None, 0, None) == L.E_INVALID  # group 3
    # a split history without its workspace
    assert lib.lfm3_prompt_attention(1, 512, 1, 1, 1, 4, 1, 1, 1, 512, 40, 4, 2, 128, 17000,
                                     17040, 0, None, 0, None) == L.E_INVALID
    # a ring of 2 GiB (2^21 slots x 4 KV heads x 128 dims x 2 bytes): the
    # kernel addresses rings with 32-bit buffer offsets
    assert lib.lfm3_prompt_attention(1, 2048, 1, 1, 1, 16, 1, 1, 1, 2048, 40, 16, 4, 128, 100,
                                     1 << 21, 256, None, 0, None) == L.E_INVALID
    # a sliding ring shorter than the window - 1 keys the first row reads
    # (here 254 < min(255, 300)): the older of them would be overwritten
    assert lib.lfm3_prompt_attention(1, 2048, 1, 1, 1, 16, 1, 1, 1, 2048, 40, 16, 4, 128, 300,
                                     254, 256, None, 0, None) == L.E_INVALID
    assert b"prompt attention" in lib.lfm3_last_error()


def test_model_load_refuses_rings_past_2gib():
    """A context whose full K/V ring of one layer reaches 2 GiB is refused
    before any device work."""
    dims = L.Dims(hidden=128, intermediate=192, vocab=300, context=64, heads=4, head_dim=64,
                  kv_heads=2, window=8, pattern="CSG")
    w = L.synth_weights(dims, seed=1)
    huge = L.Dims(**{**dims.__dict__, "context": 1 << 23})  # 2^23 x 2 x 64 x 2 B = 2 GiB
    with pytest.raises(L.LFM3Error) as e:
        L.Model(L.Weights(huge, w.globals, w.layers))
    assert e.value.status == L.E_INVALID and "context" in str(e.value)


def test_projection_conv_rejects_bad_shapes():
    """Missing operands, a width outside [2, 32] or a hidden size that is not
    a whole number of 16-row tiles are refused before any launch."""
    lib = L.lib()
    assert lib.lfm3_q8_gemv_conv_image(None, None, 2048, None, None, 1, None, None, 7, None, 2048,
                                       None) == L.E_INVALID
    assert lib.lfm3_q8_gemv_conv_image(1, 1, 2048, 16, 1, 1, 1, 1, 1, 1, 2048,
                                       None) == L.E_INVALID  # width 1
    assert lib.lfm3_q8_gemv_conv_image(1, 1, 2056, 16, 1, 1, 1, 1, 7, 1, 2056,
                                       None) == L.E_INVALID  # 2056 % 16


def test_conv_prompt_half_rejects_bad_shapes():
    """The convolution with FP16 rows out refuses, before any launch: skip
    not below rows, a hidden size that is not a multiple of 4 or past 2048,
    a width outside [2, 7], a row stride that is not a whole number of
    64-column chunks."""
    lib = L.lib()
    f = 64
    ok = dict(p=f, ldp=3 * 2048, taps=f, hist=f, rows=40, skip=3, out=f, lda=2048, scale=f,
              hidden=2048, width=7)

    def call(**kw):
        a = dict(ok, **kw)
        return lib.lfm3_conv_prompt_half(a["p"], a["ldp"], a["taps"], a["hist"], a["rows"],
                                         a["skip"], a["out"], a["lda"], a["scale"], a["hidden"],
                                         a["width"], 1, None)
    assert call(skip=40) == L.E_INVALID
    assert call(hidden=2050, ldp=3 * 2050, lda=2112) == L.E_INVALID
    assert call(hidden=2052, ldp=3 * 2052, lda=2112) == L.E_INVALID
    assert call(width=8) == L.E_INVALID
    assert call(width=1) == L.E_INVALID
    assert call(lda=2080) == L.E_INVALID
    assert call(ldp=3 * 2048 - 1) == L.E_INVALID
    assert call(out=None) == L.E_INVALID


def test_swiglu_rows_rejects_bad_arguments():
    """The SwiGLU GEMM with FP16 hidden rows refuses, before any launch: a
    missing output, scale, row-maximum or flags buffer, sequence number 0,
    rows not a multiple of 4 or past 8192, an output stride that is not a
    whole number of 64-column chunks."""
    lib = L.lib()
    f = 4096
    ok = dict(h=f, s=f, rows=7680, cols=2048, a=f, lda=2048, asc=f, tokens=512, y=f, ldy=7680,
              rm=f, out=f, out_ld=7680, osc=f, flags=f, seq=1)

    def call(**kw):
        a = dict(ok, **kw)
        return lib.lfm3_q8_gemm_swiglu_h16_rows(a["h"], a["s"], a["rows"], a["cols"], a["a"],
                                                a["lda"], a["asc"], a["tokens"], a["y"],
                                                a["ldy"], a["rm"], a["out"], a["out_ld"],
                                                a["osc"], a["flags"], a["seq"], None, None)
    assert call(out=None) == L.E_INVALID
    assert call(osc=None) == L.E_INVALID
    assert call(rm=None) == L.E_INVALID
    assert call(flags=None) == L.E_INVALID
    assert call(seq=0) == L.E_INVALID
    assert call(rows=7682, ldy=7682, out_ld=7744) == L.E_INVALID
    assert call(rows=8196, ldy=8196, out_ld=8256) == L.E_INVALID
    assert call(out_ld=7700) == L.E_INVALID
    assert lib.lfm3_q8_gemm_swiglu_flags_bytes(7680, 512) == 60 * 4 * 4


def test_snapshot_signature_is_fnv1a32():
    """The snapshot's configuration signature is 32-bit FNV-1a
    (engine.cpp ConfigSignature): the published test vectors, and the word
    order of the configuration bytes."""
    import struct

    from snapshot_format import fnv1a32, signature
    assert fnv1a32(b"") == 0x811C9DC5
    assert fnv1a32(b"a") == 0xE40C292C
    assert fnv1a32(b"foobar") == 0xBF9CF968
    d = L.Dims(hidden=256, intermediate=512, vocab=1000, context=64, heads=8, head_dim=128,
               kv_heads=2, window=32, pattern="CG")
    raw = struct.pack("<7I3f", 256, 512, 1000, 8, 128, 32, 7, d.eps, d.theta, d.theta_swa)
    raw += struct.pack("<4I", L.LAYER_CONV, 0, L.LAYER_FULL, 2)
    assert signature(d) == fnv1a32(raw)


def test_continuation_layout_follows_the_state_inventory():
    """continuation_layout.cpp:6-46 restated from the config: logits,
    frontier and a 16-byte metadata part, then per layer its convolution
    history, its sliding ring (K and V of min(context, window) slots) or a
    K and a V row component; ids count from 1. RowBytes(p) is p times the
    row bytes; invalid geometry and frontiers are refused."""
    d = L.Dims(context=8192)
    ctx = 3000
    comps = L.continuation_layout(d, ctx)
    want = [(L.PART_LOGITS, 0, 0, d.vocab * 4), (L.PART_FRONTIER, 0, 0, d.hidden * 4),
            (L.PART_METADATA, 0, 0, 16)]
    row = d.kv_heads * d.head_dim * 2
    for l in range(d.n_layers):
        t = d.layer_type(l)
        if t == L.LAYER_CONV:
            want.append((L.PART_CONVOLUTION, l, 0, d.hidden * (d.conv_width - 1) * 4))
        elif t == L.LAYER_SLIDING:
            want.append((L.PART_SLIDING_WINDOW, l, 0, 2 * row * min(ctx, d.window)))
        else:
            want += [(L.PART_KEY, l, row, 0), (L.PART_VALUE, l, row, 0)]
    assert [c[1:] for c in comps] == want
    assert [c[0] for c in comps] == list(range(1, len(want) + 1))
    assert len(comps) == 3 + 13 + 5 + 2 * 6
    private, rows = L.continuation_bytes(d, ctx, 1234)
    assert private == sum(w[3] for w in want)
    assert rows == 1234 * 2 * 6 * row
    assert L.continuation_bytes(d, ctx, 0)[1] == 0
    for bad_ctx in (0, d.context + 1):
        with pytest.raises(L.LFM3Error):
            L.continuation_layout(d, bad_ctx)
    with pytest.raises(L.LFM3Error):
        L.continuation_bytes(d, ctx, ctx + 1)
    # A context below the window shrinks the sliding rings to the context.
    small = L.continuation_layout(d, 100)
    assert all(c[4] == 2 * row * 100 for c in small if c[1] == L.PART_SLIDING_WINDOW)


def test_measurement_probes_refuse_bad_arguments():
    """Refused before any launch: no device memory is touched."""
    lib = L.lib()
    fake = C.c_void_p(1 << 20)
    assert lib.lfm3_measure_stream_read(fake, 40, fake, 4, None) == L.E_INVALID  # bytes % 16
    assert lib.lfm3_measure_stream_read(C.c_void_p((1 << 20) + 4), 64, fake, 4,
                                        None) == L.E_INVALID                    # alignment
    assert lib.lfm3_measure_stream_read(fake, 64, fake, 0, None) == L.E_INVALID
    assert lib.lfm3_measure_mfma_f16(1 << 15, 4, fake, None) == L.E_INVALID       # exactness cap
    assert lib.lfm3_measure_mfma_f16(0, 4, fake, None) == L.E_INVALID

def test_batch_entries_refuse_empty_and_oversized_batches():
    """engine.cpp:1178-1180: an empty batch or one past kMaxBatch (8) is an
    invalid shape, refused before any device work, by every batch entry."""
    lib = L.lib()
    toks = (C.c_uint32 * 9)()
    ids = (C.c_uint32 * 9)()
    sessions = (C.c_void_p * 9)()
    for n in (0, 9):
        assert lib.lfm3_forward_batch(sessions, n, toks, None) == L.E_INVALID
        assert b"decode batch shape" in lib.lfm3_last_error()
        assert lib.lfm3_forward_batch_greedy(sessions, n, toks, ids) == L.E_INVALID
    # null session pointers are refused too
    assert lib.lfm3_forward_batch_greedy(sessions, 2, toks, ids) == L.E_INVALID
    assert b"null" in lib.lfm3_last_error()


def test_fused_norm_gemv_refusals():
    """The fused norm + GEMV entries refuse a zero sequence number, missing
    flags, more than 8 rows and an unsupported GEMV shape before any launch."""
    lib = L.lib()
    assert lib.lfm3_norm_flags_bytes() >= 8 * 8 * 4
    args = lambda seq, flags, batch, cols: (None, 1, 0, None, 1, 1, 1e-5, 16, 16, flags, seq, None,
                                            16, 16, 64, cols, 0, batch, 16, 64, None)
    assert lib.lfm3_q8_gemv_image_norm(*args(0, 16, 8, 256)) == L.E_INVALID     # seq 0
    assert lib.lfm3_q8_gemv_image_norm(*args(1, None, 8, 256)) == L.E_INVALID   # no flags
    assert lib.lfm3_q8_gemv_image_norm(*args(1, 16, 9, 256)) == L.E_INVALID     # 9 rows
    assert lib.lfm3_q8_gemv_image_norm(*args(1, 16, 8, 200)) == L.E_INVALID     # cols % 32
    assert lib.lfm3_q8_gemv_conv_image_norm(None, 1, 0, None, 1, 1, 1e-5, 16, 16, 16, 0, None,
                                            16, 16, 256, 8, 16, 16, 7, 16, 256,
                                            None) == L.E_INVALID
