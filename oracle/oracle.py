"""ctypes loader for the parity oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY.  Importable by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, where it is the checker or the timed CPU
baseline; the product (project-willamette_amd/) never imports it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


if not LIB.exists():
    build()

lib = C.CDLL(str(LIB))

_u8p, _i8p = C.POINTER(C.c_uint8), C.POINTER(C.c_int8)
_f32p, _i32p, _u32p = C.POINTER(C.c_float), C.POINTER(C.c_int32), C.POINTER(C.c_uint32)
_vp, _sz = C.c_void_p, C.c_size_t

_SIGS = {
    "or_f16_to_f32": (C.c_float, C.c_uint16),
    "or_ternary_from_code": (C.c_int8, C.c_uint8),
    "or_expf": (C.c_float, C.c_float),
    "or_quantize_input_absmax_i8": (C.c_float, _f32p, _sz, _i8p),
    "or_i2s_unpack_row": (C.c_int, _u8p, _sz, _sz, _sz, _i8p),
    "or_bitlinear_i2s_matvec_f32_sse2_i8": (C.c_int, _u8p, _sz, C.c_float, _sz, _sz, _f32p, _f32p,
                                            _i8p, _f32p, _i32p),
    "or_bitlinear_i2s_matvec_f32_scalar": (C.c_int, _u8p, _sz, C.c_float, _sz, _sz, _f32p, _f32p),
    "or_i2s_scale": (C.c_int, _u8p, _sz, _f32p),
    "or_q6k_dequantize_row": (C.c_int, _u8p, _sz, _f32p, _sz),
    "or_q6k_dot_row_sse2": (C.c_float, _u8p, _f32p, _sz),
    "or_q6k_dot_row_scalar": (C.c_float, _u8p, _f32p, _sz),
    "or_compute_logits_q6k": (C.c_int, _u8p, _sz, _sz, _f32p, _f32p, C.c_int),
    "or_argmax": (C.c_int64, _f32p, _sz),
    "or_rms_norm": (None, _f32p, _f32p, _sz, C.c_float, _f32p),
    "or_rope_neox": (None, _f32p, _sz, _sz, C.c_uint32, C.c_float),
    "or_softmax_inplace": (None, _f32p, _sz),
    "or_relu_square_mul": (None, _f32p, _f32p, _sz, _f32p),
    "or_kv_quantise": (C.c_float, _f32p, _sz, _i8p),
    "or_ffn_block_forward": (C.c_int, _f32p, _sz, _sz, _f32p, _u8p, C.c_float, _u8p, C.c_float,
                             _u8p, C.c_float, _f32p, C.c_float, _f32p),
    "or_model_create": (_vp, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                        C.c_uint32, C.c_uint32, C.c_float, C.c_float),
    "or_model_destroy": (None, _vp),
    "or_model_set_layer": (C.c_int, _vp, C.c_uint32, _u8p, C.c_float, _u8p, C.c_float, _u8p,
                           C.c_float, _u8p, C.c_float, _u8p, C.c_float, _u8p, C.c_float, _u8p,
                           C.c_float, _f32p, _f32p, _f32p, _f32p),
    "or_model_set_output": (C.c_int, _vp, _u8p, _f32p),
    "or_model_set_threads": (None, _vp, C.c_int),
    "or_sdpa": (None, _f32p, _f32p, _f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _f32p,
                _f32p),
    "or_kv_create": (_vp, C.c_uint32, C.c_uint32, C.c_uint32),
    "or_kv_destroy": (None, _vp),
    "or_kv_position": (C.c_uint32, _vp),
    "or_kv_rollback": (None, _vp, C.c_uint32),
    "or_kv_append_position": (C.c_int, _vp, _f32p, _f32p),
    "or_kv_read_raw": (C.c_int, _vp, C.c_uint32, _i8p, _f32p, _i8p, _f32p, C.c_uint32),
    "or_forward_with_cache": (C.c_int, _vp, _vp, C.c_uint32, C.c_uint32, _f32p, _f32p),
    "or_logits_argmax": (C.c_int, _vp, _f32p, _f32p, _u32p),
    "or_forward_single_token_position_zero": (C.c_int, _vp, C.c_uint32, _f32p, _f32p),
    "or_greedy_generate": (C.c_int, _vp, _vp, _u32p, C.c_uint32, C.c_uint32, C.c_int64, _u32p,
                           _u32p, _f32p),
    "or_xorshift64_seed": (C.c_uint64, C.c_uint64),
    "or_xorshift64_next": (C.c_uint64, C.POINTER(C.c_uint64)),
    "or_xorshift64_next_unit": (C.c_float, C.POINTER(C.c_uint64)),
    "or_apply_repetition_penalty": (None, _f32p, _sz, _u32p, _sz, C.c_float),
    "or_apply_temperature": (None, _f32p, _sz, C.c_float),
    "or_apply_top_k": (None, _f32p, _sz, C.c_uint64),
    "or_softmax_to_probs": (None, _f32p, _sz, _f32p),
    "or_apply_top_p": (None, _f32p, _sz, C.c_float),
    "or_sample": (C.c_int, _vp, C.POINTER(C.c_uint64), _u32p, _sz, _f32p, _sz, _u32p, _f32p),
}
for _n, (_r, *_a) in _SIGS.items():
    _f = getattr(lib, _n)
    _f.restype, _f.argtypes = _r, list(_a)


def P(a: np.ndarray, ct):
    return a.ctypes.data_as(C.POINTER(ct)) if a is not None else None


# ---- convenience wrappers ------------------------------------------------

def quantize_input_absmax_i8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, dtype=np.int8)
    s = lib.or_quantize_input_absmax_i8(P(x, C.c_float), x.size, P(q, C.c_int8))
    return q, np.float32(s)


def bitlinear_i8(packed: np.ndarray, scale: float, in_dim: int, out_dim: int, x: np.ndarray):
    """SSE2-i8 BitLinear; returns (y, act, act_scale, acc) or raises on error."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.size != in_dim:  # input.len() != in_dim (bitlinear_sse2.rs:145-151)
        raise ValueError("input length != in_dim")
    y = np.empty(out_dim, dtype=np.float32)
    act = np.empty(in_dim, dtype=np.int8)
    acc = np.empty(out_dim, dtype=np.int32)
    sc = C.c_float()
    rc = lib.or_bitlinear_i2s_matvec_f32_sse2_i8(P(packed, C.c_uint8), packed.size, scale, in_dim,
                                                 out_dim, P(x, C.c_float), P(y, C.c_float),
                                                 P(act, C.c_int8), C.byref(sc), P(acc, C.c_int32))
    if rc:
        raise ValueError(f"oracle bitlinear rejected input (rc={rc})")
    return y, act, np.float32(sc.value), acc


def bitlinear_scalar(packed, scale, in_dim, out_dim, x):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.size != in_dim:  # bitlinear.rs:165-172
        raise ValueError("input length != in_dim")
    y = np.empty(out_dim, dtype=np.float32)
    rc = lib.or_bitlinear_i2s_matvec_f32_scalar(P(packed, C.c_uint8), packed.size, scale, in_dim,
                                                out_dim, P(x, C.c_float), P(y, C.c_float))
    if rc:
        raise ValueError(f"oracle scalar bitlinear rejected input (rc={rc})")
    return y


def unpack_row(packed, in_dim, out_dim, row):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(in_dim, dtype=np.int8)
    rc = lib.or_i2s_unpack_row(P(packed, C.c_uint8), in_dim, out_dim, row, P(out, C.c_int8))
    if rc:
        raise ValueError(rc)
    return out


def q6k_dequantize_row(row: np.ndarray, n: int):
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    rc = lib.or_q6k_dequantize_row(P(row, C.c_uint8), row.size, P(out, C.c_float), n)
    if rc:
        raise ValueError(rc)
    return out


def q6k_dot_sse2(row, x):
    row = np.ascontiguousarray(row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.float32(lib.or_q6k_dot_row_sse2(P(row, C.c_uint8), P(x, C.c_float), x.size))


def q6k_dot_scalar(row, x):
    row = np.ascontiguousarray(row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    return np.float32(lib.or_q6k_dot_row_scalar(P(row, C.c_uint8), P(x, C.c_float), x.size))


def compute_logits(embd, n_embd, vocab, hidden, threads=1):
    embd = np.ascontiguousarray(embd, dtype=np.uint8)
    hidden = np.ascontiguousarray(hidden, dtype=np.float32)
    out = np.empty(vocab, dtype=np.float32)
    rc = lib.or_compute_logits_q6k(P(embd, C.c_uint8), n_embd, vocab, P(hidden, C.c_float),
                                   P(out, C.c_float), threads)
    if rc:
        raise ValueError(rc)
    return out


def argmax(logits):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    r = lib.or_argmax(P(logits, C.c_float), logits.size)
    return None if r < 0 else int(r)


def rms_norm(x, w, eps=1e-5):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    lib.or_rms_norm(P(x, C.c_float), P(w, C.c_float), x.size, eps, P(out, C.c_float))
    return out


def ffn_block(x, ffn_norm_w, gate, gate_scale, up, up_scale, down, down_scale, ffn_sub_norm_w,
              n_ff, eps=1e-5):
    """ffn_block_forward (src/model/ffn.rs:73-136): n_embd = x.size; gate and
    up are I2_S packed [n_embd -> n_ff], down [n_ff -> n_embd]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    E = x.size
    nw = np.ascontiguousarray(ffn_norm_w, dtype=np.float32)
    sw = np.ascontiguousarray(ffn_sub_norm_w, dtype=np.float32)
    g, u, d = (np.ascontiguousarray(t, dtype=np.uint8) for t in (gate, up, down))
    if nw.size != E or sw.size != n_ff or g.size < E // 4 * n_ff or u.size < E // 4 * n_ff \
            or d.size < n_ff // 4 * E:
        raise ValueError("ffn_block: length mismatch")
    out = np.empty(E, dtype=np.float32)
    rc = lib.or_ffn_block_forward(P(x, C.c_float), E, n_ff, P(nw, C.c_float), P(g, C.c_uint8),
                                  C.c_float(gate_scale), P(u, C.c_uint8), C.c_float(up_scale),
                                  P(d, C.c_uint8), C.c_float(down_scale), P(sw, C.c_float),
                                  C.c_float(eps), P(out, C.c_float))
    if rc:
        raise ValueError(f"oracle ffn_block rejected input (rc={rc})")
    return out


def rope_neox(x, head_dim, n_rot, pos, base):
    x = np.array(x, dtype=np.float32)
    lib.or_rope_neox(P(x, C.c_float), head_dim, n_rot, pos, base)
    return x


def softmax(x):
    x = np.array(x, dtype=np.float32)
    lib.or_softmax_inplace(P(x, C.c_float), x.size)
    return x


def sdpa(q, kd, vd, n_heads: int, n_kv_heads: int, head_dim: int):
    """Attention of q [n_heads*head_dim] over f32 K/V rows kd, vd
    [n_past][n_kv_heads*head_dim] (src/model/cached_forward.rs:417-449)."""
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
    kd = np.ascontiguousarray(kd, dtype=np.float32)
    vd = np.ascontiguousarray(vd, dtype=np.float32)
    kvd = n_kv_heads * head_dim
    assert q.size == n_heads * head_dim and kd.size % kvd == 0 and kd.shape == vd.shape
    n_past = kd.size // kvd
    out = np.empty(n_heads * head_dim, np.float32)
    scores = np.empty(max(n_past, 1), np.float32)
    lib.or_sdpa(P(q, C.c_float), P(kd, C.c_float), P(vd, C.c_float), n_past, n_heads, n_kv_heads,
                head_dim, P(out, C.c_float), P(scores, C.c_float))
    return out


def kv_quantise(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.size, dtype=np.int8)
    s = lib.or_kv_quantise(P(x, C.c_float), x.size, P(q, C.c_int8))
    return q, np.float32(s)


# ---- sampler (src/model/sampler.rs) --------------------------------------

class SamplingParams(C.Structure):
    """SamplingParams (sampler.rs:40-79) with the Option fields as flags;
    the same layout as the library's wm_sampling_params."""
    _fields_ = [("temperature", C.c_float), ("has_top_k", C.c_uint32), ("top_k", C.c_uint64),
                ("top_p", C.c_float), ("has_top_p", C.c_uint32),
                ("repetition_penalty", C.c_float), ("has_repetition_penalty", C.c_uint32)]

    @classmethod
    def make(cls, temperature=0.0, top_k=None, top_p=None, repetition_penalty=None):
        return cls(temperature, top_k is not None, top_k or 0, 0.0 if top_p is None else top_p,
                   top_p is not None, 0.0 if repetition_penalty is None else repetition_penalty,
                   repetition_penalty is not None)


class Sampler:
    """Sampler (sampler.rs:81-149) over the oracle's restatement."""

    def __init__(self, params: SamplingParams, seed: int):
        self.params = params
        self.state = C.c_uint64(lib.or_xorshift64_seed(seed))
        self.history: list[int] = []

    def observe(self, tok: int):
        self.history.append(int(tok))

    def checkpoint(self):
        return self.state.value, len(self.history)

    def rollback(self, cp):
        self.state.value, n = cp
        del self.history[n:]

    def sample(self, logits):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        hist = np.ascontiguousarray(self.history, dtype=np.uint32)
        out, total = C.c_uint32(), C.c_float()
        rc = lib.or_sample(C.byref(self.params), C.byref(self.state), P(hist, C.c_uint32), hist.size,
                           P(logits, C.c_float), logits.size, C.byref(out), C.byref(total))
        if rc:
            raise ValueError(f"oracle sample failed rc={rc} total={total.value}")
        return int(out.value)


def apply_top_k(logits, k):
    x = np.array(logits, dtype=np.float32)
    lib.or_apply_top_k(P(x, C.c_float), x.size, k)
    return x


def apply_top_p(probs, p):
    x = np.array(probs, dtype=np.float32)
    lib.or_apply_top_p(P(x, C.c_float), x.size, p)
    return x


def softmax_to_probs(logits):
    x = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty_like(x)
    lib.or_softmax_to_probs(P(x, C.c_float), x.size, P(out, C.c_float))
    return out


def apply_repetition_penalty(logits, history, r):
    x = np.array(logits, dtype=np.float32)
    h = np.ascontiguousarray(history, dtype=np.uint32)
    lib.or_apply_repetition_penalty(P(x, C.c_float), x.size, P(h, C.c_uint32), h.size, r)
    return x
