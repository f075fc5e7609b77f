"""ctypes binding of libwillamette_hip.so (the C ABI in include/willamette_hip.h).

Python-side mirror of project-willamette's Rust API for the BitNet decode
path, for tests and benchmarks:

    bitlinear_i2s_matvec_f32(weight, input) -> output   src/model/bitlinear.rs:67
    compute_logits(hidden, token_embd) -> logits        src/model/lm_head.rs:29
    argmax(logits) -> id | None                         src/model/lm_head.rs:161
    Model / KVCache / forward_with_cache / greedy_generate
                                  src/model/{graph,kv_cache,cached_forward,generate}.rs

Errors raise WillametteError carrying the C status, mirroring the Rust
`Result<_, WillametteError>` (src/error.rs:9-57).  There is no CPU
fallback: if the shared library is missing this module fails to import.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref
from pathlib import Path

import numpy as np

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("WILLAMETTE_HIP_LIB", _PKG / "libwillamette_hip.so"))

if not LIB_PATH.exists():
    raise ImportError(
        f"{LIB_PATH} is missing: build it with `python project-willamette_amd/build.py` "
        "(or __graft_entry__.build()); there is no CPU fallback"
    )

lib = C.CDLL(str(LIB_PATH))

WM_OK = 0
STATUS = {
    1: "UnsupportedTensorType",
    2: "Shape",
    3: "NonFinite",
    4: "OutOfMemory",
    5: "Hip",
    6: "Arg",
    7: "State",
    8: "GgufParse",
    9: "InvalidMagic",
    10: "UnsupportedVersion",
    11: "UnsupportedArchitecture",
    12: "MissingMetadata",
    13: "TensorOutOfBounds",
    14: "Io",
    15: "NotImplemented",
}
TYPE_I2S = 36
TYPE_Q6K = 14


class WillametteError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{STATUS.get(status, status)}] {message}")
        self.status = status
        self.kind = STATUS.get(status, str(status))


_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_u32p = C.POINTER(C.c_uint32)
_vp = C.c_void_p


class ModelConfig(C.Structure):
    _fields_ = [
        ("n_layers", C.c_uint32),
        ("n_embd", C.c_uint32),
        ("n_ff", C.c_uint32),
        ("n_heads", C.c_uint32),
        ("n_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("n_rot", C.c_uint32),
        ("vocab_size", C.c_uint32),
        ("context_length", C.c_uint32),
        ("rms_eps", C.c_float),
        ("rope_freq_base", C.c_float),
    ]


class SamplingParams(C.Structure):
    """wm_sampling_params: SamplingParams (src/model/sampler.rs:40-79) with
    each Option as a has_* flag."""
    _fields_ = [("temperature", C.c_float), ("has_top_k", C.c_uint32), ("top_k", C.c_uint64),
                ("top_p", C.c_float), ("has_top_p", C.c_uint32),
                ("repetition_penalty", C.c_float), ("has_repetition_penalty", C.c_uint32)]

    @classmethod
    def make(cls, temperature=0.0, top_k=None, top_p=None, repetition_penalty=None):
        return cls(temperature, top_k is not None, top_k or 0, 0.0 if top_p is None else top_p,
                   top_p is not None, 0.0 if repetition_penalty is None else repetition_penalty,
                   repetition_penalty is not None)


def _sig(name, restype, *argtypes):
    f = getattr(lib, name)
    f.restype = restype
    f.argtypes = list(argtypes)
    return f


# Every symbol the header declares.
EXPORTS = {
    "wm_ctx_create": (C.c_int, C.c_int, C.POINTER(_vp)),
    "wm_ctx_destroy": (None, _vp),
    "wm_last_error": (C.c_char_p, _vp),
    "wm_ctx_stream": (_vp, _vp),
    "wm_ctx_synchronize": (C.c_int, _vp),
    "wm_version": (C.c_char_p,),
    "wm_dev_alloc": (C.c_int, _vp, C.c_size_t, C.POINTER(_vp)),
    "wm_dev_free": (C.c_int, _vp, _vp),
    "wm_memcpy_h2d": (C.c_int, _vp, _vp, _vp, C.c_size_t),
    "wm_memcpy_d2h": (C.c_int, _vp, _vp, _vp, C.c_size_t),
    "wm_tensor_upload_i2s": (C.c_int, _vp, _u8p, C.c_size_t, _u8p, C.c_size_t, C.c_uint64,
                             C.c_uint64, C.POINTER(_vp)),
    "wm_tensor_upload_q6k": (C.c_int, _vp, _u8p, C.c_size_t, C.c_uint64, C.c_uint64,
                             C.POINTER(_vp)),
    "wm_tensor_destroy": (None, _vp),
    "wm_tensor_info": (C.c_int, _vp, C.POINTER(C.c_uint64), C.POINTER(C.c_int), _f32p),
    "wm_bitlinear_i2s_matvec_f32": (C.c_int, _vp, _vp, _f32p, C.c_size_t, _f32p, C.c_size_t),
    "wm_bitlinear_i2s_matvec_f32_debug": (C.c_int, _vp, _vp, _f32p, C.c_size_t, _f32p,
                                          C.c_size_t, _i8p, _f32p, _i32p),
    "wm_bitlinear_i2s_matvec_f32_dev": (C.c_int, _vp, _vp, _vp, _vp),
    "wm_ffn_block_forward": (C.c_int, _vp, _vp, C.c_size_t, _vp, C.c_size_t, _vp, _vp, _vp, _vp,
                             C.c_size_t, C.c_float, _vp, C.c_size_t),
    "wm_ffn_block_forward_dev": (C.c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_float, _vp),
    "wm_bitlinear_i2s_matvec_f32_scalar": (C.c_int, _vp, _vp, _f32p, C.c_size_t, _f32p, C.c_size_t),
    "wm_bitlinear_i2s_matvec_f32_scalar_dev": (C.c_int, _vp, _vp, _vp, _vp),
    "wm_bitlinear_i2s_matvec_f32_dev_noalloc": (C.c_int, _vp, _vp, _vp, _vp),
    "wm_debug_rerun_role": (C.c_int, _vp, _vp, C.c_uint32, C.c_uint32, C.c_uint32),
    "wm_debug_set_fused_flags": (C.c_int, _vp, C.c_uint32),
    "wm_bitlinear_i2s_matvec_f32_multi_dev": (C.c_int, _vp, C.POINTER(_vp), C.c_uint32, _vp, _vp),
    "wm_bitlinear_i2s_matmul_f32_dev": (C.c_int, _vp, _vp, _vp, C.c_uint32, _vp),
    "wm_bitlinear_i2s_matmul_f32": (C.c_int, _vp, _vp, _f32p, C.c_size_t, C.c_uint32, _f32p,
                                    C.c_size_t),
    "wm_q6k_dequantize_row": (C.c_int, _vp, _vp, C.c_uint64, _f32p, C.c_size_t),
    "wm_compute_logits": (C.c_int, _vp, _vp, _f32p, C.c_size_t, _f32p, C.c_size_t),
    "wm_logits_argmax": (C.c_int, _vp, _vp, _f32p, C.c_size_t, _f32p, _u32p),
    "wm_logits_argmax_dev": (C.c_int, _vp, _vp, _vp, _vp, _vp),
    "wm_argmax": (C.c_int, _f32p, C.c_size_t, _u32p),
    "wm_model_create": (C.c_int, _vp, C.POINTER(ModelConfig), C.POINTER(_vp)),
    "wm_model_destroy": (None, _vp),
    "wm_model_set_layer": (C.c_int, _vp, C.c_uint32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f32p,
                           _f32p, _f32p, _f32p),
    "wm_model_set_output": (C.c_int, _vp, _vp, _f32p),
    "wm_kv_cache_create": (C.c_int, _vp, C.c_uint32, C.POINTER(_vp)),
    "wm_kv_cache_destroy": (None, _vp),
    "wm_kv_cache_position": (C.c_uint32, _vp),
    "wm_kv_cache_rollback": (C.c_int, _vp, C.c_uint32),
    "wm_kv_cache_append_position": (C.c_int, _vp, _f32p, _f32p),
    "wm_kv_cache_append_positions": (C.c_int, _vp, _f32p, _f32p, C.c_uint32),
    "wm_kv_cache_read_raw": (C.c_int, _vp, C.c_uint32, _i8p, _f32p, _i8p, _f32p, C.c_uint32),
    "wm_forward_with_cache": (C.c_int, _vp, _vp, C.c_uint32, C.c_uint32, _f32p, _f32p),
    "wm_forward_single_token_position_zero": (C.c_int, _vp, C.c_uint32, _f32p),
    "wm_kv_cache_read_into": (C.c_int, _vp, C.c_uint32, _f32p, _f32p),
    "wm_decode_step": (C.c_int, _vp, _vp, C.c_uint32, C.c_uint32, _f32p, _f32p, _u32p),
    "wm_greedy_generate": (C.c_int, _vp, _vp, _u32p, C.c_uint32, C.c_uint32, C.c_int64, _u32p,
                           _u32p),
    "wm_batch_forward": (C.c_int, _vp, C.POINTER(_vp), C.c_uint32, _u32p, _u32p, _f32p, _u32p),
    "wm_prefill": (C.c_int, _vp, _vp, _u32p, C.c_uint32, _f32p),
    "wm_sampler_create": (C.c_int, _vp, C.POINTER(SamplingParams), C.c_uint64, C.POINTER(_vp)),
    "wm_sampler_destroy": (None, _vp),
    "wm_sampler_observe": (C.c_int, _vp, C.c_uint32),
    "wm_sampler_checkpoint": (C.c_int, _vp, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)),
    "wm_sampler_rollback": (C.c_int, _vp, C.c_uint64, C.c_uint64),
    "wm_sampler_sample": (C.c_int, _vp, _f32p, C.c_size_t, _u32p),
    "wm_sampler_sample_dev": (C.c_int, _vp, _vp, C.c_size_t, _u32p),
    "wm_generate_with_sampler": (C.c_int, _vp, _vp, _u32p, C.c_uint32, C.c_uint32, C.c_int64,
                                 _u32p, C.c_uint32, _vp, _u32p, _u32p),
    "wm_server_create": (C.c_int, _vp, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(_vp)),
    "wm_server_destroy": (None, _vp),
    "wm_server_submit": (C.c_int, _vp, _u32p, C.c_uint32, C.c_uint32, C.c_int64, _u32p, C.c_uint32,
                         C.POINTER(SamplingParams), C.c_uint64, C.POINTER(C.c_uint64)),
    "wm_server_step": (C.c_int, _vp, _u32p),
    "wm_server_result": (C.c_int, _vp, C.c_uint64, _u32p, C.c_uint32, _u32p, C.POINTER(C.c_int)),
    "wm_server_release": (C.c_int, _vp, C.c_uint64),
    "wm_debug_seq_sum": (C.c_int, _vp, _f32p, C.c_size_t, _f32p),
    "wm_debug_q6k_bounded_logits": (C.c_int, _vp, _vp, _f32p, C.c_size_t, _f32p, _f32p),
    "wm_debug_q6k_bounded_logits_dev": (C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_int),
    "wm_gguf_parse": (C.c_int, _u8p, C.c_size_t, C.POINTER(_vp), C.c_char_p, C.c_size_t),
    "wm_gguf_open": (C.c_int, C.c_char_p, C.POINTER(_vp), C.c_char_p, C.c_size_t),
    "wm_gguf_close": (None, _vp),
    "wm_gguf_version": (C.c_uint32, _vp),
    "wm_gguf_alignment": (C.c_uint64, _vp),
    "wm_gguf_tensor_count": (C.c_uint64, _vp),
    "wm_gguf_data_offset": (C.c_uint64, _vp),
    "wm_gguf_find_tensor": (C.c_int64, _vp, C.c_char_p),
    "wm_gguf_tensor_info": (C.c_int, _vp, C.c_uint64, C.POINTER(C.c_char_p), _u32p, _u32p,
                            C.POINTER(C.c_uint64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                            C.POINTER(_u8p), C.POINTER(_u8p)),
    "wm_gguf_meta_u64": (C.c_int, _vp, C.c_char_p, C.POINTER(C.c_uint64)),
    "wm_gguf_meta_f32": (C.c_int, _vp, C.c_char_p, _f32p),
    "wm_gguf_meta_str": (C.c_int, _vp, C.c_char_p, C.POINTER(C.c_char_p)),
    "wm_gguf_bitnet_config": (C.c_int, _vp, C.POINTER(ModelConfig), C.c_char_p, C.c_size_t),
    "wm_gguf_bitnet_check": (C.c_int, _vp, C.c_char_p, C.c_size_t),
    "wm_model_from_gguf": (C.c_int, _vp, _vp, C.c_uint32, C.POINTER(_vp)),
    "wm_synth_stream_seed": (C.c_uint64, C.c_uint64, C.c_uint64),
    "wm_synth_i2s": (None, C.c_uint64, C.c_uint64, _u8p, C.c_size_t),
    "wm_synth_normal": (None, C.c_uint64, C.c_uint64, _f32p, C.c_size_t, C.c_double),
    "wm_synth_uniform": (None, C.c_uint64, C.c_uint64, _f32p, C.c_size_t, C.c_double, C.c_double),
    "wm_synth_q6k": (None, C.c_uint64, C.c_uint64, _u8p, C.c_size_t, C.c_double),
}

for _name, (_res, *_args) in EXPORTS.items():
    _sig(_name, _res, *_args)


def _ptr(a: np.ndarray, ct):
    return a.ctypes.data_as(C.POINTER(ct))


# ---------------------------------------------------------------------------
# synthetic inputs (src/synth.rs role; host only, no GPU needed)
# ---------------------------------------------------------------------------

def synth_i2s(seed: int, tag: int, in_dim: int, out_dim: int) -> np.ndarray:
    out = np.empty(in_dim // 4 * out_dim, dtype=np.uint8)
    lib.wm_synth_i2s(seed, tag, _ptr(out, C.c_uint8), out.size)
    return out


def synth_normal(seed: int, tag: int, n: int, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib.wm_synth_normal(seed, tag, _ptr(out, C.c_float), n, sigma)
    return out


def synth_uniform(seed: int, tag: int, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib.wm_synth_uniform(seed, tag, _ptr(out, C.c_float), n, lo, hi)
    return out


def synth_q6k(seed: int, tag: int, n_rows: int, row_len: int, d_sigma: float = 1e-3) -> np.ndarray:
    n_blocks = n_rows * (row_len // 256)
    out = np.empty(n_blocks * 210, dtype=np.uint8)
    lib.wm_synth_q6k(seed, tag, _ptr(out, C.c_uint8), n_blocks, d_sigma)
    return out


def scale_block(scale: float) -> np.ndarray:
    """The 32-byte I2_S trailing block: LE f32 scale + 28 zero bytes."""
    b = np.zeros(32, dtype=np.uint8)
    b[:4] = np.frombuffer(np.float32(scale).tobytes(), dtype=np.uint8)
    return b


def argmax(logits: np.ndarray):
    """src/model/lm_head.rs:161-174 (None for an empty slice)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    out = C.c_uint32()
    st = lib.wm_argmax(_ptr(logits, C.c_float), logits.size, C.byref(out))
    return None if st else int(out.value)


# ---------------------------------------------------------------------------
# context / tensors
# ---------------------------------------------------------------------------

class Context:
    def __init__(self, device: int = 0):
        h = _vp()
        st = lib.wm_ctx_create(device, C.byref(h))
        if st:
            raise WillametteError(st, f"wm_ctx_create(device={device}) failed")
        self.h = h
        self._children = weakref.WeakSet()  # tensors, buffers, models, caches

    def adopt(self, child):
        self._children.add(child)
        return child

    def check(self, st: int):
        if st:
            raise WillametteError(st, lib.wm_last_error(self.h).decode())

    def close(self):
        """Destroys every live object made on this context, then the context."""
        if self.h:
            for c in sorted(list(self._children), key=lambda c: getattr(c, "_close_rank", 0)):
                c.close()
            lib.wm_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self):
        self.check(lib.wm_ctx_synchronize(self.h))

    @property
    def stream(self) -> int:
        return lib.wm_ctx_stream(self.h) or 0

    # device buffers
    def alloc(self, nbytes: int) -> "DeviceBuffer":
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = DeviceBuffer(self, a.nbytes)
        self.check(lib.wm_memcpy_h2d(self.h, b.ptr, a.ctypes.data, a.nbytes))
        return b

    # tensors
    def upload_i2s(self, packed: np.ndarray, scale, in_dim: int, out_dim: int) -> "Tensor":
        packed = np.ascontiguousarray(packed, dtype=np.uint8)
        sb = scale if isinstance(scale, np.ndarray) else scale_block(float(scale))
        sb = np.ascontiguousarray(sb, dtype=np.uint8)
        h = _vp()
        self.check(lib.wm_tensor_upload_i2s(self.h, _ptr(packed, C.c_uint8), packed.size,
                                            _ptr(sb, C.c_uint8), sb.size, in_dim, out_dim,
                                            C.byref(h)))
        return Tensor(self, h)

    def upload_q6k(self, blocks: np.ndarray, row_len: int, n_rows: int) -> "Tensor":
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        h = _vp()
        self.check(lib.wm_tensor_upload_q6k(self.h, _ptr(blocks, C.c_uint8), blocks.size, row_len,
                                            n_rows, C.byref(h)))
        return Tensor(self, h)


class Sampler:
    """Sampler (src/model/sampler.rs:81-149) whose sample() runs on the device."""
    _close_rank = 0

    def __init__(self, ctx: Context, params: SamplingParams, seed: int):
        self.ctx, self.params = ctx, params
        h = _vp()
        ctx.check(lib.wm_sampler_create(ctx.h, C.byref(params), seed, C.byref(h)))
        self.h = h
        ctx.adopt(self)

    def close(self):
        if self.h:
            lib.wm_sampler_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def observe(self, tok: int):
        self.ctx.check(lib.wm_sampler_observe(self.h, tok))

    def checkpoint(self):
        st, n = C.c_uint64(), C.c_uint64()
        self.ctx.check(lib.wm_sampler_checkpoint(self.h, C.byref(st), C.byref(n)))
        return st.value, n.value

    def rollback(self, cp):
        self.ctx.check(lib.wm_sampler_rollback(self.h, cp[0], cp[1]))

    def sample(self, logits: np.ndarray) -> int:
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        out = C.c_uint32()
        self.ctx.check(lib.wm_sampler_sample(self.h, _ptr(logits, C.c_float), logits.size,
                                             C.byref(out)))
        return int(out.value)

    def sample_dev(self, buf: "DeviceBuffer", n: int) -> int:
        out = C.c_uint32()
        self.ctx.check(lib.wm_sampler_sample_dev(self.h, buf.ptr, n, C.byref(out)))
        return int(out.value)


class DeviceBuffer:
    _close_rank = 2

    def __init__(self, ctx: Context, nbytes: int):
        self.ctx = ctx
        p = _vp()
        ctx.check(lib.wm_dev_alloc(ctx.h, nbytes, C.byref(p)))
        self.ptr = p.value
        self.nbytes = nbytes
        ctx.adopt(self)

    def to_host(self, dtype, count=None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        self.ctx.check(lib.wm_memcpy_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr and self.ctx.h:
            lib.wm_dev_free(self.ctx.h, self.ptr)
        self.ptr = None

    close = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Tensor:
    _close_rank = 2

    def __init__(self, ctx: Context, h):
        self.ctx, self.h = ctx, h
        ctx.adopt(self)
        shape = (C.c_uint64 * 2)()
        t = C.c_int()
        s = C.c_float()
        ctx.check(lib.wm_tensor_info(h, shape, C.byref(t), C.byref(s)))
        self.shape = (int(shape[0]), int(shape[1]))
        self.type = t.value
        self.scale = s.value

    def close(self):
        if self.h:
            lib.wm_tensor_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# kernels (host-slice API, mirrors the Rust signatures)
# ---------------------------------------------------------------------------

def bitlinear_i2s_matvec_f32(ctx: Context, w: Tensor, x: np.ndarray, debug: bool = False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(w.shape[1], dtype=np.float32)
    if not debug:
        ctx.check(lib.wm_bitlinear_i2s_matvec_f32(ctx.h, w.h, _ptr(x, C.c_float), x.size,
                                                  _ptr(y, C.c_float), y.size))
        return y
    act = np.empty(w.shape[0], dtype=np.int8)
    acc = np.empty(w.shape[1], dtype=np.int32)
    sc = C.c_float()
    ctx.check(lib.wm_bitlinear_i2s_matvec_f32_debug(ctx.h, w.h, _ptr(x, C.c_float), x.size,
                                                    _ptr(y, C.c_float), y.size, _ptr(act, C.c_int8),
                                                    C.byref(sc), _ptr(acc, C.c_int32)))
    return y, act, float(np.float32(sc.value)), acc


def ffn_block_forward(ctx: Context, x, ffn_norm_weight, gate: Tensor, up: Tensor, down: Tensor,
                      ffn_sub_norm_weight, eps: float = 1e-5) -> np.ndarray:
    """ffn_block_forward (src/model/ffn.rs:73-136): ffn_norm, gate and up,
    relu(gate)^2 * up, ffn_sub_norm, down; no residual add."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    nw = np.ascontiguousarray(ffn_norm_weight, dtype=np.float32)
    sw = np.ascontiguousarray(ffn_sub_norm_weight, dtype=np.float32)
    y = np.empty(gate.shape[0], dtype=np.float32)
    ctx.check(lib.wm_ffn_block_forward(ctx.h, _ptr(x, C.c_float), x.size, _ptr(nw, C.c_float), nw.size,
                                       gate.h, up.h, down.h, _ptr(sw, C.c_float), sw.size, eps,
                                       _ptr(y, C.c_float), y.size))
    return y


def bitlinear_i2s_matvec_f32_scalar(ctx: Context, w: Tensor, x: np.ndarray) -> np.ndarray:
    """bitlinear_i2s_matvec_f32_scalar (src/model/bitlinear.rs:146-233): f32
    inputs, no int8 quantiser."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(w.shape[1], dtype=np.float32)
    ctx.check(lib.wm_bitlinear_i2s_matvec_f32_scalar(ctx.h, w.h, _ptr(x, C.c_float), x.size,
                                                     _ptr(y, C.c_float), y.size))
    return y


def bitlinear_i2s_matmul_f32(ctx: Context, w: Tensor, x: np.ndarray) -> np.ndarray:
    """Rows of x (m x in_dim) through the batched BitLinear: row r equals
    bitlinear_i2s_matvec_f32 on x[r]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    m = x.shape[0]
    y = np.empty((m, w.shape[1]), dtype=np.float32)
    ctx.check(lib.wm_bitlinear_i2s_matmul_f32(ctx.h, w.h, _ptr(x, C.c_float), x.size, m,
                                              _ptr(y, C.c_float), y.size))
    return y


def debug_seq_sum(ctx: Context, values: np.ndarray) -> np.float32:
    """The device's exact left-to-right f32 sum (test hook)."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    out = C.c_float()
    ctx.check(lib.wm_debug_seq_sum(ctx.h, _ptr(values, C.c_float), values.size, C.byref(out)))
    return np.float32(out.value)


def q6k_dequantize_row(ctx: Context, t: Tensor, row: int) -> np.ndarray:
    out = np.empty(t.shape[0], dtype=np.float32)
    ctx.check(lib.wm_q6k_dequantize_row(ctx.h, t.h, row, _ptr(out, C.c_float), out.size))
    return out


def compute_logits(ctx: Context, t: Tensor, hidden: np.ndarray) -> np.ndarray:
    hidden = np.ascontiguousarray(hidden, dtype=np.float32)
    out = np.empty(t.shape[1], dtype=np.float32)
    ctx.check(lib.wm_compute_logits(ctx.h, t.h, _ptr(hidden, C.c_float), hidden.size,
                                    _ptr(out, C.c_float), out.size))
    return out


def logits_argmax(ctx: Context, t: Tensor, hidden: np.ndarray, want_logits: bool = True):
    hidden = np.ascontiguousarray(hidden, dtype=np.float32)
    out = np.empty(t.shape[1], dtype=np.float32) if want_logits else None
    a = C.c_uint32()
    ctx.check(lib.wm_logits_argmax(ctx.h, t.h, _ptr(hidden, C.c_float), hidden.size,
                                   _ptr(out, C.c_float) if out is not None else None, C.byref(a)))
    return out, int(a.value)


def q6k_bounded_logits(ctx: Context, t: Tensor, hidden: np.ndarray):
    """The id-only lm-head's bounded pass (test hook): per row the
    fixed-point dot and a bound on its distance from the reference's logit."""
    hidden = np.ascontiguousarray(hidden, dtype=np.float32)
    approx = np.empty(t.shape[1], dtype=np.float32)
    bound = np.empty(t.shape[1], dtype=np.float32)
    ctx.check(lib.wm_debug_q6k_bounded_logits(ctx.h, t.h, _ptr(hidden, C.c_float), hidden.size,
                                              _ptr(approx, C.c_float), _ptr(bound, C.c_float)))
    return approx, bound


# ---------------------------------------------------------------------------
# GGUF files (src/gguf/reader.rs; host only, no GPU needed)
# ---------------------------------------------------------------------------

class GgufFile:
    """GgufFile (src/gguf/reader.rs:120-415) over bytes (parse) or a path
    (open).  Tensor data is read in place; `data` must outlive the object."""

    def __init__(self, h, keep=None):
        self.h = h
        self._keep = keep

    @staticmethod
    def _raise(st: int, err) -> None:
        raise WillametteError(st, err.value.decode("utf-8", "replace"))

    @classmethod
    def parse(cls, data) -> "GgufFile":
        buf = np.frombuffer(bytes(data), dtype=np.uint8) if not isinstance(data, np.ndarray) else data
        buf = np.ascontiguousarray(buf, dtype=np.uint8)
        h, err = _vp(), C.create_string_buffer(512)
        st = lib.wm_gguf_parse(_ptr(buf, C.c_uint8), buf.size, C.byref(h), err, 512)
        if st:
            cls._raise(st, err)
        return cls(h, buf)

    @classmethod
    def open(cls, path) -> "GgufFile":
        h, err = _vp(), C.create_string_buffer(512)
        st = lib.wm_gguf_open(str(path).encode(), C.byref(h), err, 512)
        if st:
            cls._raise(st, err)
        return cls(h)

    def close(self):
        if self.h:
            lib.wm_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def version(self) -> int:
        return int(lib.wm_gguf_version(self.h))

    @property
    def alignment(self) -> int:
        return int(lib.wm_gguf_alignment(self.h))

    @property
    def data_offset(self) -> int:
        return int(lib.wm_gguf_data_offset(self.h))

    def __len__(self) -> int:
        return int(lib.wm_gguf_tensor_count(self.h))

    def find(self, name: str) -> int:
        return int(lib.wm_gguf_find_tensor(self.h, name.encode()))

    def tensor(self, index: int) -> dict:
        name, typ, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
        shape = (C.c_uint64 * 4)()
        off, nb = C.c_uint64(), C.c_uint64()
        data, sb = _u8p(), _u8p()
        st = lib.wm_gguf_tensor_info(self.h, index, C.byref(name), C.byref(typ), C.byref(nd), shape,
                                     C.byref(off), C.byref(nb), C.byref(data), C.byref(sb))
        if st:
            raise WillametteError(st, f"tensor index {index}")
        n = nb.value
        raw = np.ctypeslib.as_array(data, shape=(n,)).copy() if n else np.empty(0, np.uint8)
        scale = np.ctypeslib.as_array(sb, shape=(32,)).copy() if sb else None
        return {"name": name.value.decode(), "type": typ.value,
                "shape": [int(shape[d]) for d in range(nd.value)], "offset": off.value,
                "bytes": n, "data": raw, "scale_block": scale}

    def meta_u64(self, key: str):
        v = C.c_uint64()
        return int(v.value) if lib.wm_gguf_meta_u64(self.h, key.encode(), C.byref(v)) == 0 else None

    def meta_f32(self, key: str):
        v = C.c_float()
        return float(v.value) if lib.wm_gguf_meta_f32(self.h, key.encode(), C.byref(v)) == 0 else None

    def meta_str(self, key: str):
        v = C.c_char_p()
        return v.value.decode() if lib.wm_gguf_meta_str(self.h, key.encode(), C.byref(v)) == 0 else None

    def bitnet_check(self) -> None:
        err = C.create_string_buffer(512)
        st = lib.wm_gguf_bitnet_check(self.h, err, 512)
        if st:
            self._raise(st, err)

    def bitnet_config(self) -> ModelConfig:
        cfg, err = ModelConfig(), C.create_string_buffer(512)
        st = lib.wm_gguf_bitnet_config(self.h, C.byref(cfg), err, 512)
        if st:
            self._raise(st, err)
        return cfg
