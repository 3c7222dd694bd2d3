"""ctypes binding of the CPU oracle (liboracle.so): TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline use this
module, to compare the library's results with; the product never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")
LIB_V4_PATH = os.path.join(ORACLE_DIR, "liboracle_v4.so")


def _has_avx512() -> bool:
    """x86-64-v4's AVX-512 subsets, from the kernel's CPU flags."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    flags = set(line.split(":", 1)[1].split())
                    return {"avx512f", "avx512bw", "avx512cd", "avx512dq",
                            "avx512vl"} <= flags
    except OSError:
        pass
    return False


def lib_path() -> str:
    """The oracle build this CPU runs: x86-64-v4 where AVX-512 is present,
    else x86-64-v3 (identical results; only the speed differs)."""
    if _has_avx512() and os.path.exists(LIB_V4_PATH):
        return LIB_V4_PATH
    return LIB_PATH

F32, F16, Q8_0, BF16 = 0, 1, 8, 30
CONV, FULL, SLIDING = 0, 1, 2
vp, u32, f32, sz, i32 = C.c_void_p, C.c_uint32, C.c_float, C.c_size_t, C.c_int


class Config(C.Structure):
    _fields_ = [("hidden", u32), ("intermediate", u32), ("vocab", u32), ("context", u32),
                ("heads", u32), ("head_dim", u32), ("window", u32), ("conv_width", u32),
                ("n_layers", u32), ("eps", f32), ("theta", f32), ("theta_swa", f32),
                ("kv_heads", C.POINTER(u32)), ("layer_type", C.POINTER(C.c_uint8))]


class Tensor(C.Structure):
    _fields_ = [("data", vp), ("type", u32), ("cols", u32), ("rows", u32)]


_SIGS = {
    "orc_set_threads": (None, [u32]),
    "orc_threads": (u32, []),
    "orc_hardware_concurrency": (u32, []),
    "orc_half_to_float": (f32, [C.c_uint16]),
    "orc_float_to_half": (C.c_uint16, [f32]),
    "orc_halves_to_floats": (None, [vp, vp, sz]),
    "orc_floats_to_halves": (None, [vp, vp, sz]),
    "orc_decode_row": (i32, [C.POINTER(Tensor), u32, vp]),
    "orc_mat": (i32, [C.POINTER(Tensor), vp, vp]),
    "orc_mat_batch": (i32, [C.POINTER(Tensor), vp, vp, u32]),
    "orc_norm": (None, [vp, sz, vp, f32]),
    "orc_rope": (None, [vp, sz, u32, u32, f32, i32, vp]),
    "orc_conv_step": (None, [vp, vp, vp, vp, u32, u32]),
    "orc_attention_step": (None, [vp, vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32,
                                  u32, u32, f32, i32, f32, i32, vp]),
    "orc_attention_read": (None, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, vp]),
    "orc_half_rows": (None, [vp, sz, sz, vp, vp]),
    "orc_swiglu": (None, [vp, vp, sz]),
    "orc_argmax": (u32, [vp, sz]),
    "orc_sample": (u32, [vp, sz, f32, u32, f32, vp, sz, f32]),
    "orc_model_create": (vp, [C.POINTER(Config), C.POINTER(Tensor), sz]),
    "orc_model_destroy": (None, [vp]),
    "orc_session_create": (vp, [vp, u32, i32]),
    "orc_session_destroy": (None, [vp]),
    "orc_session_reset": (None, [vp]),
    "orc_session_position": (u32, [vp]),
    "orc_session_set_position": (None, [vp, u32]),
    "orc_session_capacity": (u32, [vp, u32]),
    "orc_session_conv": (C.POINTER(C.c_float), [vp, u32]),
    "orc_session_k": (C.POINTER(C.c_float), [vp, u32]),
    "orc_session_v": (C.POINTER(C.c_float), [vp, u32]),
    "orc_session_step": (i32, [vp, u32, vp, vp]),
    "orc_session_step_row": (i32, [vp, vp, vp, vp]),
    "orc_session_steps": (i32, [vp, vp, u32, vp, vp, i32]),
    "orc_session_steps_rows": (i32, [vp, vp, u32, vp, vp, i32]),
    "orc_attention_read_prompt": (None, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, vp]),
}

_lib = None


def build():
    subprocess.run(["make", "-C", ORACLE_DIR, "-B"], check=True, capture_output=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = C.CDLL(lib_path())
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags.c_contiguous
    return a.ctypes.data


def q8_tensor(blob: np.ndarray, rows: int, cols: int) -> Tensor:
    return Tensor(_p(blob), Q8_0, cols, rows)


def bf16_tensor(h: np.ndarray, rows: int, cols: int) -> Tensor:
    """GGUF BF16 rows (uint16 bit patterns)."""
    assert h.dtype == np.uint16 and h.size == rows * cols
    return Tensor(_p(h), BF16, cols, rows)


def f16_tensor(h: np.ndarray, rows: int, cols: int) -> Tensor:
    """GGUF F16 rows (uint16 bit patterns)."""
    assert h.dtype == np.uint16 and h.size == rows * cols
    return Tensor(_p(h), F16, cols, rows)


def f32_tensor(a: np.ndarray, rows: int, cols: int) -> Tensor:
    assert a.dtype == np.float32
    return Tensor(_p(a), F32, cols, rows)


def set_threads(n: int):
    """Worker threads per matrix-vector product / attention read (1 = the
    reference's serial loops; results are identical for any count)."""
    lib().orc_set_threads(max(1, int(n)))


def threads() -> int:
    return int(lib().orc_threads())


def hardware_concurrency() -> int:
    return int(lib().orc_hardware_concurrency())


def half_to_float(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_halves_to_floats(_p(h), _p(out), h.size)
    return out


def float_to_half(f: np.ndarray) -> np.ndarray:
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().orc_floats_to_halves(_p(f), _p(out), f.size)
    return out


def decode_row(t: Tensor, row: int) -> np.ndarray:
    out = np.empty(t.cols, np.float32)
    if lib().orc_decode_row(C.byref(t), row, _p(out)) != 0:
        raise ValueError("invalid row")
    return out


def mat(t: Tensor, x: np.ndarray) -> np.ndarray:
    """reference.cpp Mat over one or more input rows."""
    x = np.ascontiguousarray(x, np.float32)
    batch = 1 if x.ndim == 1 else x.shape[0]
    y = np.empty((batch, t.rows), np.float32)
    if lib().orc_mat_batch(C.byref(t), _p(x), _p(y), batch) != 0:
        raise ValueError("invalid tensor")
    return y[0] if x.ndim == 1 else y


def norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    out = np.array(x, np.float32, copy=True)
    lib().orc_norm(_p(out), out.size, _p(np.ascontiguousarray(weight, np.float32)), eps)
    return out


def rope(x: np.ndarray, dim: int, position: int, theta: float, sliding: bool,
         factors) -> np.ndarray:
    out = np.array(x, np.float32, copy=True)
    fac = None if factors is None else np.ascontiguousarray(factors, np.float32)
    lib().orc_rope(_p(out), out.size // dim, dim, position, theta, int(sliding),
                   0 if fac is None else _p(fac))
    return out


def conv_step(p: np.ndarray, taps: np.ndarray, history: np.ndarray, hidden: int, width: int):
    """One row; returns (y, new_history)."""
    hist = np.array(history, np.float32, copy=True)
    y = np.empty(hidden, np.float32)
    lib().orc_conv_step(_p(np.ascontiguousarray(p, np.float32)),
                        _p(np.ascontiguousarray(taps, np.float32)), _p(hist), _p(y), hidden, width)
    return y, hist


def attention_read(q, gate, cache_k, cache_v, heads, kv_heads, dim, position, capacity,
                   window) -> np.ndarray:
    out = np.empty(heads * dim, np.float32)
    lib().orc_attention_read(_p(np.ascontiguousarray(q, np.float32)),
                             _p(np.ascontiguousarray(gate, np.float32)),
                             _p(np.ascontiguousarray(cache_k, np.float32)),
                             _p(np.ascontiguousarray(cache_v, np.float32)),
                             heads, kv_heads, dim, position, capacity, window, _p(out))
    return out


def attention_step(q, k, v, gate, q_norm, k_norm, factors, cache_k, cache_v, heads, kv_heads,
                   dim, position, capacity, window, theta, sliding, eps, f16=True):
    """Norm + RoPE + store + read; cache_k / cache_v (float32) are updated in place."""
    q = np.array(q, np.float32, copy=True)
    k = np.array(k, np.float32, copy=True)
    out = np.empty(heads * dim, np.float32)
    fac = 0 if factors is None else _p(np.ascontiguousarray(factors, np.float32))
    lib().orc_attention_step(_p(q), _p(k), _p(np.ascontiguousarray(v, np.float32)),
                             _p(np.ascontiguousarray(gate, np.float32)),
                             _p(np.ascontiguousarray(q_norm, np.float32)),
                             _p(np.ascontiguousarray(k_norm, np.float32)), fac,
                             _p(cache_k), _p(cache_v), heads, kv_heads, dim, position, capacity,
                             window, theta, int(sliding), eps, int(f16), _p(out))
    return out, q, k


def attention_read_prompt(q, gate, cache_k, cache_v, heads, kv_heads, dim, position, capacity,
                          window) -> np.ndarray:
    """The prompt path's attention read (F16 scaled query and probabilities)."""
    out = np.empty(heads * dim, np.float32)
    lib().orc_attention_read_prompt(_p(np.ascontiguousarray(q, np.float32)),
                                    _p(np.ascontiguousarray(gate, np.float32)),
                                    _p(np.ascontiguousarray(cache_k, np.float32)),
                                    _p(np.ascontiguousarray(cache_v, np.float32)),
                                    heads, kv_heads, dim, position, capacity, window, _p(out))
    return out


def half_rows(x: np.ndarray):
    """Prompt activations: (effective inputs, exponent per row)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    inputs = np.empty_like(x)
    exps = np.empty(rows, np.int32)
    lib().orc_half_rows(_p(x), rows, cols, _p(inputs), _p(exps))
    return inputs, exps


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.array(gate, np.float32, copy=True)
    lib().orc_swiglu(_p(g), _p(np.ascontiguousarray(up, np.float32)), g.size)
    return g


def argmax(x: np.ndarray) -> int:
    return int(lib().orc_argmax(_p(np.ascontiguousarray(x, np.float32)), x.size))


def sample(x: np.ndarray, temperature: float, top_k: int, repeat_penalty: float = 1.0,
           penalty_ids=None, u: float = 0.0) -> int:
    """orc_sample: one row's pick (runner.cpp:300-325 SelectNext semantics)."""
    x = np.ascontiguousarray(x, np.float32)
    pen = (np.zeros(0, np.uint32) if penalty_ids is None
           else np.ascontiguousarray(penalty_ids, np.uint32))
    return int(lib().orc_sample(_p(x), x.size, temperature, top_k, repeat_penalty,
                                _p(pen) if pen.size else None, pen.size, u))


class Model:
    """Oracle model over GGUF-layout host tensors (the same arrays the GPU loads)."""

    def __init__(self, dims, weights):
        self.dims = dims
        n = dims.n_layers
        self._kv = (u32 * n)(*[0 if dims.layer_type(i) == CONV else dims.kv_heads
                               for i in range(n)])
        self._lt = (C.c_uint8 * n)(*[dims.layer_type(i) for i in range(n)])
        self.config = Config(dims.hidden, dims.intermediate, dims.vocab, dims.context, dims.heads,
                             dims.head_dim, dims.window, dims.conv_width, n, dims.eps, dims.theta,
                             dims.theta_swa, self._kv, self._lt)
        entries = weights.tensor_list()
        entries[1] = entries[0]  # tied vocabulary head (weights.cpp:56-57)
        self._tensors = (Tensor * len(entries))()
        for i, e in enumerate(entries):
            if e is not None:
                data, typ, cols, rows = e
                self._tensors[i] = Tensor(_p(data), typ, cols, rows)  # GGML type ids
        self._weights = weights
        self.handle = lib().orc_model_create(C.byref(self.config), self._tensors, len(entries))
        if not self.handle:
            raise ValueError("oracle model rejected")

    def close(self):
        if self.handle:
            lib().orc_model_destroy(self.handle)
            self.handle = None

    def session(self, context: int, f16: bool = True) -> "Session":
        return Session(self, context, f16)


class Session:
    def __init__(self, model: Model, context: int, f16: bool):
        self.model = model
        self.handle = lib().orc_session_create(model.handle, context, int(f16))
        if not self.handle:
            raise ValueError("invalid oracle context")

    def close(self):
        if self.handle:
            lib().orc_session_destroy(self.handle)
            self.handle = None

    @property
    def position(self) -> int:
        return lib().orc_session_position(self.handle)

    def set_position(self, p: int):
        lib().orc_session_set_position(self.handle, p)

    def capacity(self, layer: int) -> int:
        return lib().orc_session_capacity(self.handle, layer)

    def _view(self, fn, layer, count):
        p = fn(self.handle, layer)
        return np.ctypeslib.as_array(p, shape=(count,))

    def conv(self, layer: int) -> np.ndarray:
        d = self.model.dims
        return self._view(lib().orc_session_conv, layer, d.hidden * (d.conv_width - 1))

    def k(self, layer: int) -> np.ndarray:
        d = self.model.dims
        return self._view(lib().orc_session_k, layer,
                          self.capacity(layer) * d.kv_heads * d.head_dim)

    def v(self, layer: int) -> np.ndarray:
        d = self.model.dims
        return self._view(lib().orc_session_v, layer,
                          self.capacity(layer) * d.kv_heads * d.head_dim)

    def step(self, token: int, logits: bool = True):
        out = np.empty(self.model.dims.vocab, np.float32) if logits else None
        if lib().orc_session_step(self.handle, token, 0 if out is None else _p(out), 0) != 0:
            raise ValueError("invalid oracle step")
        return out

    def steps(self, tokens, logits: bool = True, prompt_path: bool = False):
        """A prompt of n tokens, layer-major over the n rows: bit-identical to
        n calls of step(); returns the last row's logits (or None). With
        prompt_path, the n rows are one prompt chunk with the reference's
        prompt-path numerics (FP16 row-scaled projection inputs, F16
        attention arithmetic, trailing-row pruning)."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.model.dims.vocab, np.float32) if logits else None
        if lib().orc_session_steps(self.handle, _p(toks), toks.size,
                                   0 if out is None else _p(out), 0, int(prompt_path)) != 0:
            raise ValueError("invalid oracle steps")
        return out

    def steps_rows(self, rows, logits: bool = True, prompt_path: bool = False):
        """steps() from FP32 input rows (n, hidden) in place of embedding
        rows; returns (last logits or None, last final-normed hidden row)."""
        rows = np.ascontiguousarray(rows, np.float32)
        n = rows.shape[0]
        out = np.empty(self.model.dims.vocab, np.float32) if logits else None
        hidden = np.empty(self.model.dims.hidden, np.float32)
        if lib().orc_session_steps_rows(self.handle, _p(rows), n, 0 if out is None else _p(out),
                                        _p(hidden), int(prompt_path)) != 0:
            raise ValueError("invalid oracle steps")
        return out, hidden

    def step_row(self, row, logits: bool = True):
        """One step from an FP32 input row in place of a token's embedding
        row; returns (logits or None, final-normed hidden row)."""
        row = np.ascontiguousarray(row, np.float32)
        out = np.empty(self.model.dims.vocab, np.float32) if logits else None
        hidden = np.empty(self.model.dims.hidden, np.float32)
        if lib().orc_session_step_row(self.handle, _p(row), 0 if out is None else _p(out),
                                      _p(hidden)) != 0:
            raise ValueError("invalid oracle step")
        return out, hidden
