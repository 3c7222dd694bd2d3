"""Snapshot v2 layout as the reference writes it (engine.cpp:1387-1574),
restated for the tests: the header words and the configuration signature
(FNV-1a, 32-bit, over the little-endian bytes of the configuration words)."""
import struct

import numpy as np

import lfm3amd as L

MAGIC, VERSION, HEADER_BYTES = 0x334D464C, 2, 32


def fnv1a32(data: bytes) -> int:
    h = 2166136261
    for b in data:
        h = ((h ^ b) * 16777619) & 0xFFFFFFFF
    return h


def signature(d: L.Dims) -> int:
    words = [d.hidden, d.intermediate, d.vocab, d.heads, d.head_dim, d.window, d.conv_width]
    raw = struct.pack("<7I", *words) + struct.pack("<3f", d.eps, d.theta, d.theta_swa)
    for i in range(d.n_layers):
        t = d.layer_type(i)
        raw += struct.pack("<2I", t, 0 if t == L.LAYER_CONV else d.kv_heads)
    return fnv1a32(raw)


def state_bytes(d: L.Dims, position: int) -> int:
    n = HEADER_BYTES + (d.hidden + d.vocab) * 4
    for i in range(d.n_layers):
        t = d.layer_type(i)
        if t == L.LAYER_CONV:
            n += d.hidden * (d.conv_width - 1) * 4
        else:
            slots = min(position, d.window) if t == L.LAYER_SLIDING else position
            n += 2 * slots * d.kv_heads * d.head_dim * 2
    return n


def header(data: bytes):
    return struct.unpack("<8I", data[:HEADER_BYTES])


def sections(d: L.Dims, data: bytes, capacities):
    """(frontier, logits, per-layer arrays) of a snapshot."""
    pos = header(data)[3]
    off = HEADER_BYTES
    frontier = np.frombuffer(data, np.float32, d.hidden, off)
    off += d.hidden * 4
    logits = np.frombuffer(data, np.float32, d.vocab, off)
    off += d.vocab * 4
    layers = []
    for i in range(d.n_layers):
        if d.layer_type(i) == L.LAYER_CONV:
            n = d.hidden * (d.conv_width - 1)
            layers.append(np.frombuffer(data, np.float32, n, off))
            off += n * 4
        else:
            n = min(pos, capacities[i]) * d.kv_heads * d.head_dim
            k = np.frombuffer(data, np.uint16, n, off)
            v = np.frombuffer(data, np.uint16, n, off + n * 2)
            layers.append((k, v))
            off += n * 4
    assert off == len(data)
    return frontier, logits, layers
