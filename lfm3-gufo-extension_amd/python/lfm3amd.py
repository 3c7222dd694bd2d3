"""ctypes binding of liblfm3_amd.so (the gfx950 LFM3 step) for tests and the
benchmark. Device buffers come straight from the HIP runtime (plumbing
only); every computation runs in the HIP library, and loading fails loudly
when the library is missing.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "liblfm3_amd.so")

OK, E_INVALID, E_HIP, E_STATE, E_NOMEM, E_REFUSED = 0, -1, -2, -3, -4, -5
LAYER_CONV, LAYER_FULL, LAYER_SLIDING = 0, 1, 2
TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_BF16 = 0, 1, 8, 30
STATE_LOGITS, STATE_FRONTIER, STATE_CONV, STATE_KEY, STATE_VALUE = range(5)
GLOBAL_TENSORS, LAYER_TENSORS = 4, 17
MAX_BATCH = 8

vp, u32, u64, f32, sz, i32 = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_size_t, C.c_int


class LFM3Error(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


class Config(C.Structure):
    _fields_ = [("hidden", u32), ("intermediate", u32), ("vocab", u32), ("context", u32),
                ("heads", u32), ("head_dim", u32), ("window", u32), ("conv_width", u32),
                ("n_layers", u32), ("eps", f32), ("theta", f32), ("theta_swa", f32),
                ("kv_heads", C.POINTER(u32)), ("layer_type", C.POINTER(C.c_uint8))]


class Tensor(C.Structure):
    _fields_ = [("data", vp), ("type", u32), ("cols", u32), ("rows", u32)]


class Input(C.Structure):
    """lfm3_input: a run of token ids or of FP32 input rows."""
    _fields_ = [("tokens", vp), ("n_tokens", C.c_size_t), ("rows", vp), ("n_rows", C.c_size_t)]


WRITE_HOOK = C.CFUNCTYPE(C.c_int, vp, C.c_uint32, C.c_uint32)
EVENT_HOOK = C.CFUNCTYPE(C.c_int, vp)


class Hooks(C.Structure):
    """lfm3_hooks: continuation callbacks (a nonzero return refuses)."""
    _fields_ = [("user", vp), ("before_write", WRITE_HOOK), ("before_reset", EVENT_HOOK),
                ("before_restore", EVENT_HOOK)]


class Component(C.Structure):
    """lfm3_continuation_component."""
    _fields_ = [("id", C.c_uint32), ("part", C.c_uint32), ("layer", C.c_uint32),
                ("reserved", C.c_uint32), ("row_bytes", C.c_size_t),
                ("state_bytes", C.c_size_t)]


class Sampling(C.Structure):
    """lfm3_sampling (runner.cpp:31-35 defaults: 0.1, 50, 1.1)."""
    _fields_ = [("temperature", f32), ("top_k", u32), ("repeat_penalty", f32)]


SAMPLE_MAX_TOP_K, SAMPLE_MAX_PENALTY, SAMPLE_MAX_COLS = 1024, 4096, 262144


class AttentionItem(C.Structure):
    _fields_ = [("row", u32), ("key_begin", u32), ("key_end", u32),
                ("first_item", u32), ("parts", u32), ("reserved", u32 * 3)]


_SIGS = {
    "lfm3_last_error": (C.c_char_p, []),
    "lfm3_q8_tiled_bytes": (None, [u32, u32, C.POINTER(sz), C.POINTER(sz)]),
    "lfm3_q8_pack_host": (i32, [vp, u32, u32, vp, vp, u32, u32]),
    "lfm3_q8_pack_device": (i32, [vp, u32, u32, vp, vp, u32, u32, vp]),
    "lfm3_gemv_workspace_bytes": (sz, [u32, u32, u32]),
    "lfm3_q8_gemv": (i32, [vp, vp, u32, u32, vp, u32, vp, u32, u32, vp, sz, vp]),
    "lfm3_q8_gemv_parts": (u32, [u32, u32]),
    "lfm3_q8_gemv_partials": (i32, [vp, vp, u32, u32, vp, u32, vp, u32, u32, u32, vp]),
    "lfm3_residual_norm_parts": (i32, [vp, u32, sz, vp, vp, vp, vp, u32, u32, f32, vp]),
    "lfm3_operand_image_bytes": (sz, [u32]),
    "lfm3_q8_gemv_image": (i32, [vp, vp, u32, u32, vp, vp, u32, vp, u32, u32, vp]),
    "lfm3_q8_gemv_swiglu_image": (i32, [vp, vp, u32, u32, vp, vp, u32, vp, u32, vp]),
    "lfm3_q8_gemv_conv_image": (i32, [vp, vp, u32, vp, vp, u32, vp, vp, u32, vp, u32, vp]),
    "lfm3_residual_norm_image": (i32, [vp, u32, sz, vp, vp, vp, vp, vp, vp, u32, u32, f32, vp]),
    "lfm3_norm_flags_bytes": (sz, []),
    "lfm3_q8_gemv_image_norm": (i32, [vp, u32, sz, vp, vp, vp, f32, vp, vp, vp, u32, vp,
                                      vp, vp, u32, u32, i32, u32, vp, u32, vp]),
    "lfm3_q8_gemv_conv_image_norm": (i32, [vp, u32, sz, vp, vp, vp, f32, vp, vp, vp, u32, vp,
                                           vp, vp, u32, u32, vp, vp, u32, vp, u32, vp]),
    "lfm3_conv_step_ragged_image": (i32, [vp, u32, vp, vp, vp, u32, vp, vp, u32, u32, u32, vp]),
    "lfm3_half_rows": (i32, [vp, u32, vp, u32, vp, u32, vp, u32, u32, vp]),
    "lfm3_q8_gemm_swiglu_max_blocks": (u32, [u32]),
    "lfm3_residual_norm_half": (i32, [vp, u32, sz, vp, vp, vp, vp, vp, u32, vp, u32, u32, f32,
                                      vp]),
    "lfm3_q8_gemm_parts": (u32, [u32, u32, u32, i32]),
    "lfm3_q8_gemm": (i32, [vp, vp, u32, u32, vp, u32, vp, u32, vp, u32, u32, vp]),
    "lfm3_q8_gemm_swiglu": (i32, [vp, vp, u32, u32, vp, u32, vp, u32, vp, u32, vp, vp]),
    "lfm3_q8_half_tiles_bytes": (sz, [u32, u32]),
    "lfm3_q8_half_tiles": (i32, [vp, u32, u32, vp, vp]),
    "lfm3_q8_gemm_h16": (i32, [vp, vp, u32, u32, vp, u32, vp, u32, vp, u32, u32, vp]),
    "lfm3_q8_gemm_swiglu_h16": (i32, [vp, vp, u32, u32, vp, u32, vp, u32, vp, u32, vp, vp]),
    "lfm3_q8_gemm_swiglu_flags_bytes": (sz, [u32, u32]),
    "lfm3_q8_gemm_swiglu_h16_rows": (i32, [vp, vp, u32, u32, vp, u32, vp, u32, vp, u32, vp, vp,
                                           u32, vp, vp, u32, vp, vp]),
    "lfm3_q8_gemv_swiglu": (i32, [vp, vp, u32, u32, vp, u32, vp, u32, u32, vp, sz, vp]),
    "lfm3_bf16_tiled_bytes": (sz, [u32, u32]),
    "lfm3_bf16_pack_host": (i32, [vp, u32, u32, vp, u32, u32]),
    "lfm3_bf16_gemv_parts": (u32, [u32, u32, u32]),
    "lfm3_bf16_gemv": (i32, [vp, u32, u32, vp, u32, vp, u32, u32, u32, i32, vp]),
    "lfm3_bf16_embed": (i32, [vp, u32, u32, vp, vp, u32, vp, vp]),
    "lfm3_float_tiled_bytes": (sz, [u32, u32, u32]),
    "lfm3_float_pack_host": (i32, [u32, vp, u32, u32, vp, u32, u32]),
    "lfm3_float_gemv": (i32, [u32, vp, u32, u32, vp, u32, vp, u32, u32, u32, i32, vp]),
    "lfm3_float_embed": (i32, [u32, vp, u32, u32, vp, vp, u32, vp, vp]),
    "lfm3_residual_norm": (i32, [vp, vp, vp, vp, vp, u32, u32, f32, vp]),
    "lfm3_embed": (i32, [vp, vp, u32, u32, vp, u32, vp, vp]),
    "lfm3_argmax_workspace_bytes": (sz, [u32]),
    "lfm3_argmax": (i32, [vp, u32, u32, vp, vp, sz, vp]),
    "lfm3_sample_workspace_bytes": (sz, [u32, u32, u32]),
    "lfm3_sample": (i32, [vp, u32, u32, u32, vp, vp, u32, vp, vp, vp, sz, vp]),
    "lfm3_conv_step_ragged": (i32, [vp, u32, vp, vp, vp, u32, u32, u32, u32, vp]),
    "lfm3_decode_heads_ragged": (i32, [vp, vp, vp, u32, vp, vp, vp, vp, vp, vp, vp, vp,
                                       u32, u32, u32, u32, f32, vp]),
    "lfm3_sum_parts": (i32, [vp, sz, u32, u32, u32, u32, vp]),
    "lfm3_conv_prompt": (i32, [vp, u32, vp, vp, vp, vp, u32, vp, u32, u32, u32, i32, vp]),
    "lfm3_conv_prompt_half": (i32, [vp, u32, vp, vp, u32, u32, vp, u32, vp, u32, u32, i32, vp]),
    "lfm3_prompt_heads": (i32, [vp, vp, vp, u32, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32,
                                u32, f32, vp]),
    "lfm3_store_kv": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, vp]),
    "lfm3_prompt_attention_workspace_bytes": (sz, [u32, u32, u32, u32, u32]),
    "lfm3_prompt_attention": (i32, [vp, u32, vp, vp, vp, u32, vp, vp, vp, u32, u32, u32, u32,
                                    u32, u32, u32, u32, vp, sz, vp]),
    "lfm3_prompt_attention_half_workspace_bytes": (sz, [u32, u32, u32, u32, u32]),
    "lfm3_prompt_attention_half": (i32, [vp, u32, vp, vp, vp, u32, vp, vp, vp, u32, vp, u32, u32,
                                         u32, u32, u32, u32, u32, vp, sz, vp]),
    "lfm3_attention_plan": (i32, [vp, u32, u32, vp, u32]),
    "lfm3_attention_max_items": (sz, [u32, u32]),
    "lfm3_attention_workspace_bytes": (sz, [u32, u32, u32, u32, u32]),
    "lfm3_decode_attention_ragged": (i32, [vp, u32, vp, u32, vp, vp, vp, vp, u32, vp, u32,
                                           u32, u32, u32, u32, vp, sz, vp]),
    "lfm3_decode_heads_attention_ragged": (i32, [vp, vp, vp, u32, vp, u32, vp, vp, vp, vp, vp,
                                                 vp, vp, vp, vp, u32, vp, u32, u32, u32, u32,
                                                 u32, f32, vp, sz, vp]),
    "lfm3_decode_heads_attention_ragged_noalloc": (i32, [vp, vp, vp, u32, vp, u32, vp, vp, vp,
                                                         vp, vp, vp, vp, vp, vp, u32, vp, u32,
                                                         u32, u32, u32, u32, f32, vp]),
    "lfm3_model_load": (i32, [C.POINTER(Config), C.POINTER(Tensor), sz, C.POINTER(vp)]),
    "lfm3_model_destroy": (None, [vp]),
    "lfm3_model_stream": (vp, [vp]),
    "lfm3_session_create": (i32, [vp, u32, C.POINTER(vp)]),
    "lfm3_session_destroy": (None, [vp]),
    "lfm3_session_position": (u32, [vp]),
    "lfm3_session_reset": (i32, [vp]),
    "lfm3_session_is_coherent": (i32, [vp]),
    "lfm3_session_ring_capacity": (u32, [vp, u32]),
    "lfm3_session_state": (i32, [vp, i32, u32, C.POINTER(vp), C.POINTER(sz)]),
    "lfm3_session_set_position": (i32, [vp, u32]),
    "lfm3_session_begin_restore": (i32, [vp]),
    "lfm3_scheduler_round": (i32, [vp, sz, vp, vp, vp, vp, vp, sz, vp]),
    "lfm3_session_forward_rows": (i32, [vp, vp, sz, i32, vp]),
    "lfm3_session_forward_inputs": (i32, [vp, vp, sz, vp]),
    "lfm3_session_read_hidden": (i32, [vp, vp]),
    "lfm3_session_set_hooks": (i32, [vp, vp]),
    "lfm3_continuation_layout": (i32, [vp, u32, vp, sz, C.POINTER(sz)]),
    "lfm3_continuation_bytes": (i32, [vp, u32, u32, C.POINTER(sz), C.POINTER(sz)]),
    "lfm3_rope_frequencies": (i32, [vp, u32, f32, vp]),
    "lfm3_rope": (i32, [vp, vp, vp, u32, u32, u32, u32, vp]),
    "lfm3_pack_kv": (i32, [vp, vp, vp, vp, sz, vp]),
    "lfm3_session_forward": (i32, [vp, vp, sz, vp]),
    "lfm3_forward_batch": (i32, [vp, sz, vp, vp]),
    "lfm3_forward_batch_greedy": (i32, [vp, sz, vp, vp]),
    "lfm3_forward_batch_sample": (i32, [vp, sz, vp, vp, vp, u32, vp, vp]),
    "lfm3_forward_batch_inputs": (i32, [vp, sz, vp, vp, i32, vp]),
    "lfm3_session_read_logits": (i32, [vp, vp]),
    "lfm3_session_prepare_logits": (i32, [vp]),
    "lfm3_session_snapshot_bytes": (sz, [vp]),
    "lfm3_session_save_snapshot": (i32, [vp, vp, sz]),
    "lfm3_session_restore_snapshot": (i32, [vp, vp, sz]),
    "lfm3_synth_key": (u64, [u64, C.c_char_p]),
    "lfm3_synth_normal": (None, [u64, f32, f32, vp, sz]),
    "lfm3_synth_uniform_u32": (None, [u64, u32, u32, vp, sz]),
    "lfm3_synth_half_normal": (None, [u64, vp, sz]),
    "lfm3_synth_q8": (None, [u64, u32, u32, f32, vp]),
    "lfm3_measure_stream_read": (i32, [vp, sz, vp, u32, vp]),
    "lfm3_measure_mfma_f16": (i32, [u32, u32, vp, vp]),
    "lfm3_measure_mfma_f16_flops": (u64, [u32, u32]),
}

_lib = None


def lib():
    """The loaded library; raises if it was not built (no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it (python -c 'import __graft_entry__ as g; g.build()')")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> int:
    if status < 0:
        raise LFM3Error(status, lib().lfm3_last_error().decode())
    return status


def ptr(a) -> int:
    """Address of a numpy array or a DeviceBuffer (0 for None)."""
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    if a is None:
        return 0
    return a.addr


# ---------------------------------------------------------------- synthetic

def key(seed: int, name: str) -> int:
    return lib().lfm3_synth_key(seed, name.encode())


def normal(seed: int, name: str, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().lfm3_synth_normal(key(seed, name), mean, std, ptr(out), n)
    return out


def uniform_u32(seed: int, name: str, n: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().lfm3_synth_uniform_u32(key(seed, name), lo, hi, ptr(out), n)
    return out


def half_normal(seed: int, name: str, n: int) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().lfm3_synth_half_normal(key(seed, name), ptr(out), n)
    return out


def q8(seed: int, name: str, rows: int, cols: int, d_std=0.02) -> np.ndarray:
    out = np.empty(rows * (cols // 32) * 34, np.uint8)
    lib().lfm3_synth_q8(key(seed, name), rows, cols, d_std, ptr(out))
    return out


def bf16(seed: int, name: str, rows: int, cols: int, std=0.0116) -> np.ndarray:
    """Random BF16 matrix (GGUF row-major uint16 bit patterns), N(0, std)
    rounded to nearest even; std matches the synthetic Q8_0 weights."""
    return to_bf16(normal(seed, name, rows * cols, 0.0, std))


def to_bf16(x: np.ndarray) -> np.ndarray:
    """FP32 -> BF16 bit patterns, round to nearest even."""
    b = np.array(x, np.float32).view(np.uint32)   # a copy, rounded in place
    r = (b >> 16) & 1
    r += 0x7FFF
    b += r          # finite values cannot carry out of 32 bits
    b >>= 16
    return b.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16(seed: int, name: str, rows: int, cols: int, std=0.0116) -> np.ndarray:
    """Random F16 matrix (GGUF row-major uint16 bit patterns), N(0, std)
    rounded to nearest even by numpy."""
    return normal(seed, name, rows * cols, 0.0, std).astype(np.float16).view(np.uint16)


def f32(seed: int, name: str, rows: int, cols: int, std=0.0116) -> np.ndarray:
    """Random F32 matrix (GGUF row-major), N(0, std)."""
    return normal(seed, name, rows * cols, 0.0, std).astype(np.float32)


def float_to_f32(data: np.ndarray, type_id: int) -> np.ndarray:
    """FP32 values of a float-format matrix's elements (BF16, F16 or F32)."""
    if type_id == TYPE_BF16:
        return bf16_to_f32(data)
    if type_id == TYPE_F16:
        return np.asarray(data, np.uint16).view(np.float16).astype(np.float32)
    return np.asarray(data, np.float32)


def q8_dequant(blob: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """float64 d * q of GGUF Q8_0 rows (test helper)."""
    blocks = blob.reshape(rows, cols // 32, 34)
    d = blocks[:, :, :2].copy().view(np.float16).astype(np.float64)
    q = blocks[:, :, 2:].view(np.int8).astype(np.float64)
    return (d * q).reshape(rows, cols)


SEED = 20261201


@dataclass
class Dims:
    """LFM3 text dims. Defaults: the reference checkpoint (config_test.cpp:82-92)."""
    hidden: int = 2048
    intermediate: int = 7680
    vocab: int = 128000
    context: int = 262144
    heads: int = 16
    head_dim: int = 128
    kv_heads: int = 4
    window: int = 256
    conv_width: int = 7
    eps: float = 1e-5
    theta: float = 1e6
    theta_swa: float = 1e4
    # C conv, S sliding, G global: 13 / 5 / 6, last layer global.
    pattern: str = "CCSCGCCSCGCCSCGCSCGCSCGG"

    @property
    def n_layers(self) -> int:
        return len(self.pattern)

    def layer_type(self, i: int) -> int:
        return {"C": LAYER_CONV, "G": LAYER_FULL, "S": LAYER_SLIDING}[self.pattern[i]]


NOMINAL = dict(intermediate=8192, vocab=65536, heads=32, head_dim=64, kv_heads=8)


@dataclass
class Weights:
    dims: Dims
    globals: list = field(default_factory=list)   # 4 (array|None, type, cols, rows)
    layers: list = field(default_factory=list)    # per layer: 17 entries

    def tensor_list(self):
        return self.globals + [t for layer in self.layers for t in layer]


def synth_weights(dims: Dims, seed: int = SEED, masked_rope=True, bf16_weights=False,
                  weight_type=None) -> Weights:
    """Random-init model of the given dims (GGUF layouts): Q8_0 matrices, or
    BF16 ones with bf16_weights, or any of TYPE_Q8_0 / TYPE_BF16 / TYPE_F16
    / TYPE_F32 as weight_type."""
    H, F, D, V = dims.hidden, dims.intermediate, dims.head_dim, dims.vocab
    w = Weights(dims)
    mtype = weight_type if weight_type is not None else TYPE_BF16 if bf16_weights else TYPE_Q8_0
    mat = {TYPE_Q8_0: q8, TYPE_BF16: bf16, TYPE_F16: f16, TYPE_F32: f32}[mtype]
    factors = np.ones(D // 2, np.float32)
    if masked_rope:
        factors[D // 4:] = 1e30
    w.globals = [(mat(seed, "token_embd", V, H), mtype, H, V), None,
                 (normal(seed, "output_norm", H, 1.0, 0.02), TYPE_F32, H, 1),
                 (factors, TYPE_F32, D // 2, 1)]
    for i in range(dims.n_layers):
        p = f"blk.{i}."
        t = [None] * LAYER_TENSORS
        for j, name in enumerate(["attn_norm", "ffn_norm", "post_attention_norm", "post_ffw_norm"]):
            t[j] = (normal(seed, p + name, H, 1.0, 0.02), TYPE_F32, H, 1)
        t[4] = (mat(seed, p + "ffn_gate", F, H), mtype, H, F)
        t[5] = (mat(seed, p + "ffn_up", F, H), mtype, H, F)
        t[6] = (mat(seed, p + "ffn_down", H, F), mtype, F, H)
        if dims.layer_type(i) == LAYER_CONV:
            t[7] = (normal(seed, p + "shortconv.conv", H * dims.conv_width, 0.0, 0.1), TYPE_F32,
                    dims.conv_width, H)
            t[8] = (mat(seed, p + "shortconv.in_proj", 3 * H, H), mtype, H, 3 * H)
            t[9] = (mat(seed, p + "shortconv.out_proj", H, H), mtype, H, H)
        else:
            kv = dims.kv_heads
            t[10] = (mat(seed, p + "attn_q", dims.heads * D, H), mtype, H, dims.heads * D)
            t[11] = (mat(seed, p + "attn_k", kv * D, H), mtype, H, kv * D)
            t[12] = (mat(seed, p + "attn_v", kv * D, H), mtype, H, kv * D)
            t[13] = (normal(seed, p + "attn_q_norm", D, 1.0, 0.02), TYPE_F32, D, 1)
            t[14] = (normal(seed, p + "attn_k_norm", D, 1.0, 0.02), TYPE_F32, D, 1)
            t[15] = (mat(seed, p + "attn_gate", dims.heads, H), mtype, H, dims.heads)
            t[16] = (mat(seed, p + "attn_output", H, dims.heads * D), mtype, dims.heads * D, H)
        w.layers.append(t)
    return w


def make_config(dims: Dims):
    kv = (u32 * dims.n_layers)(*[0 if dims.layer_type(i) == LAYER_CONV else dims.kv_heads
                                 for i in range(dims.n_layers)])
    lt = (C.c_uint8 * dims.n_layers)(*[dims.layer_type(i) for i in range(dims.n_layers)])
    cfg = Config(dims.hidden, dims.intermediate, dims.vocab, dims.context, dims.heads,
                 dims.head_dim, dims.window, dims.conv_width, dims.n_layers, dims.eps,
                 dims.theta, dims.theta_swa, kv, lt)
    return cfg, (kv, lt)


PART_LOGITS, PART_FRONTIER, PART_METADATA, PART_CONVOLUTION = 0, 1, 2, 3
PART_SLIDING_WINDOW, PART_KEY, PART_VALUE = 4, 5, 6


def continuation_layout(dims: Dims, context: int):
    """lfm3_continuation_layout: [(id, part, layer, row_bytes, state_bytes)]."""
    cfg, keep = make_config(dims)
    n = sz()
    check(lib().lfm3_continuation_layout(C.byref(cfg), context, None, 0, C.byref(n)))
    arr = (Component * n.value)()
    check(lib().lfm3_continuation_layout(C.byref(cfg), context, arr, n.value, C.byref(n)))
    return [(c.id, c.part, c.layer, c.row_bytes, c.state_bytes) for c in arr]


def continuation_bytes(dims: Dims, context: int, position: int):
    """lfm3_continuation_bytes: (private bytes, append-row bytes at position)."""
    cfg, keep = make_config(dims)
    a, b = sz(), sz()
    check(lib().lfm3_continuation_bytes(C.byref(cfg), context, position, C.byref(a), C.byref(b)))
    return a.value, b.value


def tensor_array(entries):
    arr = (Tensor * len(entries))()
    for i, e in enumerate(entries):
        if e is not None:
            data, typ, cols, rows = e
            arr[i] = Tensor(ptr(data), typ, cols, rows)
    return arr


class Model:
    """lfm3_model: device weights of one checkpoint (Model::Load)."""

    def __init__(self, weights: Weights):
        self.dims = weights.dims
        cfg, self._keep = make_config(weights.dims)
        self._tensors = tensor_array(weights.tensor_list())
        handle = vp()
        check(lib().lfm3_model_load(C.byref(cfg), self._tensors, len(self._tensors),
                                    C.byref(handle)))
        self.handle = handle

    def close(self):
        if self.handle:
            lib().lfm3_model_destroy(self.handle)
            self.handle = None

    def stream(self) -> int:
        return lib().lfm3_model_stream(self.handle) or 0

    def session(self, context: int) -> "Session":
        return Session(self, context)

    def forward_batch(self, sessions, tokens, want_logits=True):
        """Session::ForwardBatch: returns (n, vocab) float32 logits."""
        n = len(sessions)
        toks = np.ascontiguousarray(tokens, np.uint32)
        handles = (vp * max(n, 1))(*[s.handle for s in sessions])
        if want_logits:
            out = np.empty((n, self.dims.vocab), np.float32)
            rows = (vp * max(n, 1))(*[out[i].ctypes.data for i in range(n)])
            check(lib().lfm3_forward_batch(handles, n, ptr(toks), rows))
            return out
        ids = np.empty(n, np.uint32)
        check(lib().lfm3_forward_batch_greedy(handles, n, ptr(toks), ptr(ids)))
        return ids

    def forward_batch_greedy(self, sessions, tokens):
        return self.forward_batch(sessions, tokens, want_logits=False)

    def forward_batch_sample(self, sessions, tokens, params, uniforms=None, penalty=None):
        """lfm3_forward_batch_sample: one round, then the sampler's pick per
        row. penalty: (n, m) uint32 recent-token lists (ids >= vocab pad)."""
        n = len(sessions)
        toks = np.ascontiguousarray(tokens, np.uint32)
        handles = (vp * max(n, 1))(*[s.handle for s in sessions])
        ids = np.empty(n, np.uint32)
        uni = None if uniforms is None else np.ascontiguousarray(uniforms, np.float32)
        pen = None if penalty is None else np.ascontiguousarray(penalty, np.uint32).reshape(n, -1)
        check(lib().lfm3_forward_batch_sample(
            handles, n, ptr(toks), C.byref(params), ptr(pen) if pen is not None else None,
            pen.shape[1] if pen is not None else 0, ptr(uni) if uni is not None else None,
            ptr(ids)))
        return ids

    def scheduler_round(self, sessions, tokens, prompt=None, prompt_tokens=None,
                        want_logits=False, want_prompt_logits=True):
        """lfm3_scheduler_round: decode rows of `sessions` beside a prompt
        pass of `prompt`. Returns (greedy ids, decode logits or None, prompt
        logits or None)."""
        n = len(sessions)
        toks = np.ascontiguousarray(tokens if n else np.zeros(0), np.uint32)
        handles = (vp * max(n, 1))(*[s.handle for s in sessions])
        ids = np.zeros(n, np.uint32)
        out = np.empty((n, self.dims.vocab), np.float32) if want_logits and n else None
        dst = (vp * max(n, 1))(*[out[i].ctypes.data for i in range(n)]) if out is not None else None
        ptoks = np.ascontiguousarray(prompt_tokens if prompt is not None else np.zeros(0),
                                     np.uint32)
        pout = (np.empty(self.dims.vocab, np.float32)
                if prompt is not None and want_prompt_logits else None)
        check(lib().lfm3_scheduler_round(handles, n, ptr(toks) if n else None,
                                         ptr(ids) if n else None, dst,
                                         prompt.handle if prompt is not None else None,
                                         ptr(ptoks) if ptoks.size else None, ptoks.size,
                                         ptr(pout) if pout is not None else None))
        return ids, out, pout

    def forward_batch_inputs(self, sessions, tokens, rows, want_logits=True):
        """Session::ForwardBatchInputs: rows[i] is a device address of an
        FP32 hidden row standing in for token i, or 0 to use the token.
        Returns (n, vocab) float32 logits, or None without logits."""
        n = len(sessions)
        toks = np.ascontiguousarray(tokens, np.uint32)
        handles = (vp * max(n, 1))(*[s.handle for s in sessions])
        inputs = (vp * max(n, 1))(*[r or None for r in rows])
        out, dst = None, None
        if want_logits:
            out = np.empty((n, self.dims.vocab), np.float32)
            dst = (vp * max(n, 1))(*[out[i].ctypes.data for i in range(n)])
        check(lib().lfm3_forward_batch_inputs(handles, n, ptr(toks), inputs, int(want_logits),
                                              dst))
        return out


class Session:
    def __init__(self, model: Model, context: int):
        self.model = model
        handle = vp()
        check(lib().lfm3_session_create(model.handle, context, C.byref(handle)))
        self.handle = handle
        self.context = context

    def close(self):
        if self.handle:
            lib().lfm3_session_destroy(self.handle)
            self.handle = None

    @property
    def position(self) -> int:
        return lib().lfm3_session_position(self.handle)

    def set_position(self, p: int):
        check(lib().lfm3_session_set_position(self.handle, p))

    def begin_restore(self):
        check(lib().lfm3_session_begin_restore(self.handle))

    def reset(self):
        check(lib().lfm3_session_reset(self.handle))

    def coherent(self) -> bool:
        return bool(lib().lfm3_session_is_coherent(self.handle))

    def capacity(self, layer: int) -> int:
        return lib().lfm3_session_ring_capacity(self.handle, layer)

    def state(self, kind: int, layer: int = 0):
        data, nbytes = vp(), sz()
        check(lib().lfm3_session_state(self.handle, kind, layer, C.byref(data), C.byref(nbytes)))
        return data.value, nbytes.value

    def forward(self, tokens, want_logits=True):
        """Session::Forward: the last token's logits (or None)."""
        toks = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.model.dims.vocab, np.float32) if want_logits else None
        check(lib().lfm3_session_forward(self.handle, ptr(toks), len(toks),
                                         ptr(out) if want_logits else None))
        return out

    def read_logits(self) -> np.ndarray:
        out = np.empty(self.model.dims.vocab, np.float32)
        check(lib().lfm3_session_read_logits(self.handle, ptr(out)))
        return out

    def prepare_logits(self):
        """Session::PrepareLogits: the head on the frontier row, into the
        device logits row (no host copy)."""
        check(lib().lfm3_session_prepare_logits(self.handle))

    def read_hidden(self) -> np.ndarray:
        out = np.empty(self.model.dims.hidden, np.float32)
        check(lib().lfm3_session_read_hidden(self.handle, ptr(out)))
        return out

    def forward_rows(self, rows, want_logits=True, device_addr=None):
        """Session::ForwardEmbeddings: host rows (n, hidden) float32, or
        device_addr of n rows (rows is then the row count)."""
        out = np.empty(self.model.dims.vocab, np.float32) if want_logits else None
        if device_addr is not None:
            check(lib().lfm3_session_forward_rows(self.handle, device_addr, int(rows), 1,
                                                  ptr(out) if want_logits else None))
        else:
            r = np.ascontiguousarray(rows, np.float32).reshape(-1, self.model.dims.hidden)
            check(lib().lfm3_session_forward_rows(self.handle, ptr(r), r.shape[0], 0,
                                                  ptr(out) if want_logits else None))
        return out

    def forward_inputs(self, runs, want_logits=True):
        """Session::ForwardInputs: runs of ("tokens", ids) or ("rows", (n,
        hidden) float32), in order."""
        keep = []
        arr = (Input * max(len(runs), 1))()
        for i, (kind, data) in enumerate(runs):
            if kind == "tokens":
                t = np.ascontiguousarray(data, np.uint32)
                keep.append(t)
                arr[i] = Input(ptr(t) if t.size else None, t.size, None, 0)
            else:
                r = np.ascontiguousarray(data, np.float32).reshape(-1, self.model.dims.hidden)
                keep.append(r)
                arr[i] = Input(None, 0, ptr(r) if r.size else None, r.shape[0])
        out = np.empty(self.model.dims.vocab, np.float32) if want_logits else None
        check(lib().lfm3_session_forward_inputs(self.handle, arr, len(runs),
                                                ptr(out) if want_logits else None))
        return out

    def set_hooks(self, before_write=None, before_reset=None, before_restore=None):
        """Continuation hooks: Python callables returning 0 (allow) or
        nonzero (refuse); None clears them all when every one is None."""
        if before_write is None and before_reset is None and before_restore is None:
            self._hooks = None
            check(lib().lfm3_session_set_hooks(self.handle, None))
            return
        h = Hooks(None,
                  WRITE_HOOK(lambda u, a, b: int(before_write(a, b))) if before_write
                  else WRITE_HOOK(),
                  EVENT_HOOK(lambda u: int(before_reset())) if before_reset else EVENT_HOOK(),
                  EVENT_HOOK(lambda u: int(before_restore())) if before_restore
                  else EVENT_HOOK())
        self._hooks = h  # the callbacks must outlive the session's use
        check(lib().lfm3_session_set_hooks(self.handle, C.byref(h)))

    def save_snapshot(self) -> bytes:
        """Session::SaveSnapshot: the snapshot v2 bytes."""
        out = np.empty(lib().lfm3_session_snapshot_bytes(self.handle), np.uint8)
        check(lib().lfm3_session_save_snapshot(self.handle, ptr(out), out.size))
        return out.tobytes()

    def restore_snapshot(self, data: bytes):
        """Session::RestoreSnapshot."""
        buf = np.frombuffer(data, np.uint8).copy()
        check(lib().lfm3_session_restore_snapshot(self.handle, ptr(buf) if buf.size else None,
                                                  buf.size))


# ------------------------------------------------------------ device memory

_hip = None


def hip():
    """The HIP runtime (libamdhip64) for allocations and copies."""
    global _hip
    if _hip is None:
        h = C.CDLL("libamdhip64.so")
        h.hipMalloc.argtypes = [C.POINTER(vp), sz]
        h.hipFree.argtypes = [vp]
        h.hipMemcpy.argtypes = [vp, vp, sz, i32]
        h.hipMemset.argtypes = [vp, i32, sz]
        h.hipDeviceSynchronize.argtypes = []
        h.hipGetErrorString.restype = C.c_char_p
        h.hipGetErrorString.argtypes = [i32]
        h.hipGetDeviceCount.argtypes = [C.POINTER(i32)]
        h.hipStreamSynchronize.argtypes = [vp]
        h.hipStreamCreate.argtypes = [C.POINTER(vp)]
        h.hipStreamDestroy.argtypes = [vp]
        h.hipEventCreate.argtypes = [C.POINTER(vp)]
        h.hipEventDestroy.argtypes = [vp]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventSynchronize.argtypes = [vp]
        h.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), vp, vp]
        h.hipMemcpyAsync.argtypes = [vp, vp, sz, i32, vp]
        h.hipStreamBeginCapture.argtypes = [vp, i32]
        h.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        h.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, C.c_char_p, sz]
        h.hipGraphLaunch.argtypes = [vp, vp]
        h.hipGraphExecDestroy.argtypes = [vp]
        h.hipGraphDestroy.argtypes = [vp]
        _hip = h
    return _hip


def hip_check(e: int):
    if e != 0:
        raise LFM3Error(E_HIP, hip().hipGetErrorString(e).decode())


H2D, D2H, D2D = 1, 2, 3


class DeviceBuffer:
    """hipMalloc'd bytes, zeroed, freed on close/GC."""

    def __init__(self, nbytes: int):
        self.nbytes = max(int(nbytes), 1)
        p = vp()
        hip_check(hip().hipMalloc(C.byref(p), self.nbytes))
        self.addr = p.value
        hip_check(hip().hipMemset(self.addr, 0, self.nbytes))

    @classmethod
    def of(cls, host: np.ndarray) -> "DeviceBuffer":
        host = np.ascontiguousarray(host)
        b = cls(host.nbytes)
        b.upload(host)
        return b

    def upload(self, host: np.ndarray, offset: int = 0):
        host = np.ascontiguousarray(host)
        assert offset + host.nbytes <= self.nbytes
        hip_check(hip().hipMemcpy(self.addr + offset, host.ctypes.data, host.nbytes, H2D))

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.empty(count, dtype)
        assert offset + out.nbytes <= self.nbytes
        hip_check(hip().hipMemcpy(out.ctypes.data, self.addr + offset, out.nbytes, D2H))
        return out

    def close(self):
        if self.addr:
            hip().hipFree(self.addr)
            self.addr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def upload_to(addr: int, host: np.ndarray):
    host = np.ascontiguousarray(host)
    hip_check(hip().hipMemcpy(addr, host.ctypes.data, host.nbytes, H2D))


def download_from(addr: int, dtype, count: int) -> np.ndarray:
    out = np.empty(count, dtype)
    hip_check(hip().hipMemcpy(out.ctypes.data, addr, out.nbytes, D2H))
    return out


def synchronize():
    hip_check(hip().hipDeviceSynchronize())


def gpu_count() -> int:
    n = i32(0)
    try:
        if hip().hipGetDeviceCount(C.byref(n)) != 0:
            return 0
    except OSError:
        return 0
    return n.value


class Stream:
    """A default-priority HIP stream."""

    def __init__(self):
        p = vp()
        hip_check(hip().hipStreamCreate(C.byref(p)))
        self.handle = p.value

    def synchronize(self):
        hip_check(hip().hipStreamSynchronize(self.handle))

    def close(self):
        if self.handle:
            hip().hipStreamDestroy(self.handle)
            self.handle = None


class Event:
    """hipEvent recorded on a given stream (the stream the kernels run on)."""

    def __init__(self):
        p = vp()
        hip_check(hip().hipEventCreate(C.byref(p)))
        self.handle = p.value

    def record(self, stream=None):
        hip_check(hip().hipEventRecord(self.handle, stream))

    def synchronize(self):
        hip_check(hip().hipEventSynchronize(self.handle))

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float()
        hip_check(hip().hipEventElapsedTime(C.byref(ms), self.handle, end.handle))
        return ms.value

    def close(self):
        if self.handle:
            hip().hipEventDestroy(self.handle)
            self.handle = None


class Graph:
    """A HIP graph captured from the launches `record()` makes on `stream`
    (for timing back-to-back launches without host launch overhead)."""

    def __init__(self, stream: Stream, record):
        h = hip()
        hip_check(h.hipStreamBeginCapture(stream.handle, 0))
        try:
            record()
        finally:
            graph = vp()
            hip_check(h.hipStreamEndCapture(stream.handle, C.byref(graph)))
        self.graph = graph.value
        exec_ = vp()
        hip_check(h.hipGraphInstantiate(C.byref(exec_), self.graph, None, None, 0))
        self.exec = exec_.value
        self.stream = stream

    def launch(self):
        hip_check(hip().hipGraphLaunch(self.exec, self.stream.handle))

    def close(self):
        if self.exec:
            hip().hipGraphExecDestroy(self.exec)
            hip().hipGraphDestroy(self.graph)
            self.exec = None


# ------------------------------------------------------- synthetic sessions

def synth_conv_state(seed: int, sid: int, layer: int, dims: Dims) -> np.ndarray:
    """Convolution history [hidden][width - 1] of session sid, N(0, 1)."""
    return normal(seed, f"s{sid}.l{layer}.conv", dims.hidden * (dims.conv_width - 1))


def synth_kv_state(seed: int, sid: int, layer: int, tag: str, rows: int, dims: Dims) -> np.ndarray:
    """The first `rows` slots of a K ("k") or V ("v") ring, F16 N(0, 1) bits."""
    return half_normal(seed, f"s{sid}.l{layer}.{tag}", rows * dims.kv_heads * dims.head_dim)


def live_slots(position: int, capacity: int) -> int:
    """Ring slots holding positions before `position` (slot = t % capacity)."""
    return min(position, capacity)


def inject_synth_state(session: Session, dims: Dims, seed: int, sid: int, position: int):
    """Prefilled state of a session at `position`: every conv history and the
    ring slots of positions [0, position) are synthesized; later slots stay
    zero and are written before any round reads them."""
    for l in range(dims.n_layers):
        if dims.layer_type(l) == LAYER_CONV:
            addr, nbytes = session.state(STATE_CONV, l)
            h = synth_conv_state(seed, sid, l, dims)
            assert nbytes == h.nbytes
            upload_to(addr, h)
        else:
            rows = live_slots(position, session.capacity(l))
            for kind, tag in ((STATE_KEY, "k"), (STATE_VALUE, "v")):
                addr, nbytes = session.state(kind, l)
                bits = synth_kv_state(seed, sid, l, tag, rows, dims)
                assert bits.nbytes <= nbytes
                upload_to(addr, bits)
    session.set_position(position)
