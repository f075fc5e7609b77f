"""Seeded BitNet b1.58 models with random-init weights (the role of the
reference's src/synth.rs, at BitNet-b1.58-2B shape).

Every tensor is drawn from its own counter-based SplitMix64 stream
(wm_synth_* in libwillamette_hip.so), keyed by (master seed, tag), so the
same weights can be produced on any host and fed identically to the device
model and to the oracle.

Distributions (per workload definition):
  I2_S weights   each of {-1, 0, +1} with probability 1/3, I2_S byte layout
  I2_S scales    U(0.5, 2) per tensor
  norm weights   U(0.9, 1.1)
  token_embd     Q6_K: ql/qh uniform bytes, sub-scales uniform in [-32, 31],
                 d = f16(|N(0, 1e-3)|)
  KV prefill     N(0, 1) per (position, layer) K and V vector
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import willamette_hip as wh


def master_seed(config_index: int) -> int:
    """Seed of workload k: 0x5749_4C4C_0000_000k ("WILL" + k)."""
    return 0x5749_4C4C_0000_0000 | config_index


@dataclass(frozen=True)
class BitNetConfig:
    n_layers: int = 30
    n_embd: int = 2560
    n_ff: int = 6912
    n_heads: int = 20
    n_kv_heads: int = 5
    head_dim: int = 128
    vocab: int = 128256
    context_length: int = 4096
    rms_eps: float = 1e-5
    rope_base: float = 500000.0

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    def c_config(self) -> wh.ModelConfig:
        return wh.ModelConfig(self.n_layers, self.n_embd, self.n_ff, self.n_heads, self.n_kv_heads,
                              self.head_dim, self.head_dim, self.vocab, self.context_length,
                              self.rms_eps, self.rope_base)

    def weight_bytes(self) -> dict:
        """Algorithmic bytes of the weights one decode token streams."""
        E, F, KV = self.n_embd, self.n_ff, self.kv_dim
        i2s = self.n_layers * (E * E + 2 * E * KV + E * E + 3 * E * F) // 4
        norms = self.n_layers * (3 * E + F) * 4 + E * 4
        lm = self.vocab * (E // 256) * 210
        return {"i2s": i2s, "norms": norms, "lm_head": lm}


BITNET_2B = BitNetConfig()

ROLES = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
NORMS = ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm")


def role_shape(cfg: BitNetConfig, role: str):
    """(in_dim, out_dim) in GGUF order (docs/BITLINEAR_I2S_MATVEC.md:26-34)."""
    E, F, KV = cfg.n_embd, cfg.n_ff, cfg.kv_dim
    return {"attn_q": (E, E), "attn_k": (E, KV), "attn_v": (E, KV), "attn_output": (E, E),
            "ffn_gate": (E, F), "ffn_up": (E, F), "ffn_down": (F, E)}[role]


def _tag(layer: int, kind: int, idx: int) -> int:
    return (layer << 16) | (kind << 8) | idx


@dataclass
class HostLayer:
    packed: dict = field(default_factory=dict)  # role -> uint8[in/4*out]
    scales: dict = field(default_factory=dict)  # role -> float
    norms: dict = field(default_factory=dict)   # name -> float32[n]


@dataclass
class HostModel:
    cfg: BitNetConfig
    seed: int
    layers: list
    token_embd: np.ndarray  # Q6_K bytes, vocab x (n_embd/256*210)
    output_norm: np.ndarray


def make_host_model(cfg: BitNetConfig, seed: int) -> HostModel:
    layers = []
    for l in range(cfg.n_layers):
        hl = HostLayer()
        for i, role in enumerate(ROLES):
            ind, outd = role_shape(cfg, role)
            hl.packed[role] = wh.synth_i2s(seed, _tag(l, 1, i), ind, outd)
            hl.scales[role] = float(wh.synth_uniform(seed, _tag(l, 2, i), 1, 0.5, 2.0)[0])
        for i, name in enumerate(NORMS):
            n = cfg.n_ff if name == "ffn_sub_norm" else cfg.n_embd
            hl.norms[name] = wh.synth_uniform(seed, _tag(l, 3, i), n, 0.9, 1.1)
        layers.append(hl)
    embd = wh.synth_q6k(seed, _tag(0xFFFF, 4, 0), cfg.vocab, cfg.n_embd, 1e-3)
    out_norm = wh.synth_uniform(seed, _tag(0xFFFF, 5, 0), cfg.n_embd, 0.9, 1.1)
    return HostModel(cfg, seed, layers, embd, out_norm)


def kv_prefill(cfg: BitNetConfig, seed: int, n_pos: int):
    """N(0,1) K and V for n_pos positions, shaped [n_pos][n_layers][kv_dim]."""
    n = n_pos * cfg.n_layers * cfg.kv_dim
    k = wh.synth_normal(seed, _tag(0xFFFE, 6, 0), n).reshape(n_pos, cfg.n_layers, cfg.kv_dim)
    v = wh.synth_normal(seed, _tag(0xFFFE, 6, 1), n).reshape(n_pos, cfg.n_layers, cfg.kv_dim)
    return k, v


def load_device_model(ctx: wh.Context, hm: HostModel) -> "DeviceModel":
    return DeviceModel(ctx, hm)


class DeviceModel:
    """wm_model built from a HostModel (ModelGraph::from_gguf role)."""

    _close_rank = 1

    def __init__(self, ctx: wh.Context, hm: HostModel):
        self.ctx, self.cfg = ctx, hm.cfg
        cc = hm.cfg.c_config()
        h = wh._vp()
        ctx.check(wh.lib.wm_model_create(ctx.h, wh.C.byref(cc), wh.C.byref(h)))
        self.h = h
        ctx.adopt(self)
        for l, hl in enumerate(hm.layers):
            ts = []
            for role in ROLES:
                ind, outd = role_shape(hm.cfg, role)
                ts.append(ctx.upload_i2s(hl.packed[role], hl.scales[role], ind, outd))
            nrm = [np.ascontiguousarray(hl.norms[n], dtype=np.float32) for n in NORMS]
            ctx.check(wh.lib.wm_model_set_layer(self.h, l, *[t.h for t in ts],
                                                *[wh._ptr(a, wh.C.c_float) for a in nrm]))
            for t in ts:
                t.close()
        emb = ctx.upload_q6k(hm.token_embd, hm.cfg.n_embd, hm.cfg.vocab)
        on = np.ascontiguousarray(hm.output_norm, dtype=np.float32)
        ctx.check(wh.lib.wm_model_set_output(self.h, emb.h, wh._ptr(on, wh.C.c_float)))
        emb.close()

    @classmethod
    def from_gguf(cls, ctx: wh.Context, gf: "wh.GgufFile", max_context: int = 0) -> "DeviceModel":
        """ModelGraph::from_gguf (src/model/graph.rs:79-237) through
        wm_model_from_gguf: config, checks and upload in the library."""
        c = gf.bitnet_config()
        self = cls.__new__(cls)
        self.ctx = ctx
        self.cfg = BitNetConfig(c.n_layers, c.n_embd, c.n_ff, c.n_heads, c.n_kv_heads, c.head_dim,
                                c.vocab_size,
                                min(c.context_length, max_context) if max_context else c.context_length,
                                c.rms_eps, c.rope_freq_base)
        h = wh._vp()
        ctx.check(wh.lib.wm_model_from_gguf(ctx.h, gf.h, max_context, wh.C.byref(h)))
        self.h = h
        ctx.adopt(self)
        return self

    def close(self):
        if self.h:
            wh.lib.wm_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def kv_cache(self, max_seq: int) -> "DeviceKV":
        return DeviceKV(self, max_seq)

    def forward_position_zero(self, token: int) -> np.ndarray:
        """forward_single_token_position_zero (src/model/forward.rs:29): the
        hidden after output_norm, no cache."""
        hidden = np.empty(self.cfg.n_embd, np.float32)
        self.ctx.check(wh.lib.wm_forward_single_token_position_zero(self.h, token,
                                                                    wh._ptr(hidden, wh.C.c_float)))
        return hidden

    def batch_forward(self, kvs, seqs, want_hidden: bool = True, want_next: bool = True):
        """Ragged step: seqs[i] (token ids) appended to kvs[i] in one batch.
        Returns (last hidden per sequence, next token per sequence)."""
        n = len(kvs)
        arr = (wh._vp * n)(*[kv.h.value for kv in kvs])
        n_new = np.array([len(t) for t in seqs], np.uint32)
        toks = np.ascontiguousarray(np.concatenate([np.asarray(t, np.uint32) for t in seqs]))
        hidden = np.empty((n, self.cfg.n_embd), np.float32) if want_hidden else None
        nxt = np.empty(n, np.uint32) if want_next else None
        self.ctx.check(wh.lib.wm_batch_forward(
            self.h, arr, n, wh._ptr(n_new, wh.C.c_uint32), wh._ptr(toks, wh.C.c_uint32),
            wh._ptr(hidden, wh.C.c_float) if want_hidden else None,
            wh._ptr(nxt, wh.C.c_uint32) if want_next else None))
        return hidden, (nxt.tolist() if want_next else None)


class DeviceKV:
    _close_rank = 0

    def __init__(self, model: DeviceModel, max_seq: int):
        self.model, self.ctx = model, model.ctx
        h = wh._vp()
        self.ctx.check(wh.lib.wm_kv_cache_create(model.h, max_seq, wh.C.byref(h)))
        self.h = h
        self.ctx.adopt(self)

    def close(self):
        if self.h:
            wh.lib.wm_kv_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def position(self) -> int:
        return int(wh.lib.wm_kv_cache_position(self.h))

    def rollback(self, pos: int):
        self.ctx.check(wh.lib.wm_kv_cache_rollback(self.h, pos))

    def append_positions(self, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        n_pos = k.shape[0]
        self.ctx.check(wh.lib.wm_kv_cache_append_positions(self.h, wh._ptr(k, wh.C.c_float),
                                                           wh._ptr(v, wh.C.c_float), n_pos))

    def read_raw(self, layer: int, n_pos: int):
        kvd = self.model.cfg.kv_dim
        k = np.empty(n_pos * kvd, np.int8)
        v = np.empty(n_pos * kvd, np.int8)
        ks = np.empty(n_pos, np.float32)
        vs = np.empty(n_pos, np.float32)
        self.ctx.check(wh.lib.wm_kv_cache_read_raw(self.h, layer, wh._ptr(k, wh.C.c_int8),
                                                   wh._ptr(ks, wh.C.c_float), wh._ptr(v, wh.C.c_int8),
                                                   wh._ptr(vs, wh.C.c_float), n_pos))
        return k.reshape(n_pos, kvd), ks, v.reshape(n_pos, kvd), vs

    def read_into(self, layer: int):
        """KVCache::read_into: (K, V) dequantised, [position][kv_dim] f32."""
        n = self.position * self.model.cfg.kv_dim
        k = np.empty(n, np.float32)
        v = np.empty(n, np.float32)
        self.ctx.check(wh.lib.wm_kv_cache_read_into(self.h, layer, wh._ptr(k, wh.C.c_float),
                                                    wh._ptr(v, wh.C.c_float)))
        return k.reshape(-1, self.model.cfg.kv_dim), v.reshape(-1, self.model.cfg.kv_dim)

    def forward(self, token: int, pos: int, trace: bool = False):
        cfg = self.model.cfg
        hidden = np.empty(cfg.n_embd, np.float32)
        tr = np.empty((cfg.n_layers, cfg.n_embd), np.float32) if trace else None
        self.ctx.check(wh.lib.wm_forward_with_cache(self.model.h, self.h, token, pos,
                                                    wh._ptr(hidden, wh.C.c_float),
                                                    wh._ptr(tr, wh.C.c_float) if trace else None))
        return (hidden, tr) if trace else hidden

    def decode_step(self, token: int, pos: int, want_logits: bool = True):
        cfg = self.model.cfg
        hidden = np.empty(cfg.n_embd, np.float32)
        logits = np.empty(cfg.vocab, np.float32) if want_logits else None
        nxt = wh.C.c_uint32()
        self.ctx.check(wh.lib.wm_decode_step(self.model.h, self.h, token, pos,
                                             wh._ptr(hidden, wh.C.c_float),
                                             wh._ptr(logits, wh.C.c_float) if want_logits else None,
                                             wh.C.byref(nxt)))
        return hidden, logits, int(nxt.value)

    def greedy(self, prompt, max_new: int, eos: int = -1):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = wh.C.c_uint32()
        self.ctx.check(wh.lib.wm_greedy_generate(self.model.h, self.h, wh._ptr(prompt, wh.C.c_uint32),
                                                 prompt.size, max_new, eos,
                                                 wh._ptr(out, wh.C.c_uint32), wh.C.byref(n)))
        return out[: n.value].tolist()

    def prefill(self, tokens, want_hidden: bool = True):
        """Batched prefill of `tokens` at the cache's position; the last
        token's hidden after output_norm."""
        tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
        hidden = np.empty(self.model.cfg.n_embd, np.float32) if want_hidden else None
        self.ctx.check(wh.lib.wm_prefill(self.model.h, self.h, wh._ptr(tokens, wh.C.c_uint32),
                                         tokens.size,
                                         wh._ptr(hidden, wh.C.c_float) if want_hidden else None))
        return hidden

    def generate_sampled(self, prompt, max_new: int, sampler, eos: int = -1, stop_ids=()):
        """generate_with_cache_and_sampler (src/model/generate.rs:195-277)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        stops = np.ascontiguousarray(list(stop_ids) or [0], dtype=np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = wh.C.c_uint32()
        self.ctx.check(wh.lib.wm_generate_with_sampler(
            self.model.h, self.h, wh._ptr(prompt, wh.C.c_uint32), prompt.size, max_new, eos,
            wh._ptr(stops, wh.C.c_uint32), len(stop_ids), sampler.h, wh._ptr(out, wh.C.c_uint32),
            wh.C.byref(n)))
        return out[: n.value].tolist()


class Server:
    """Continuous-batching driver (wm_server_*) over a DeviceModel."""
    _close_rank = -1

    def __init__(self, model: DeviceModel, max_seqs: int, max_seq_len: int, step_tokens: int):
        self.model, self.ctx = model, model.ctx
        h = wh._vp()
        self.ctx.check(wh.lib.wm_server_create(model.h, max_seqs, max_seq_len, step_tokens,
                                               wh.C.byref(h)))
        self.h = h
        self.ctx.adopt(self)

    def close(self):
        if self.h:
            wh.lib.wm_server_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def submit(self, prompt, max_new: int, params, seed: int, eos: int = -1, stop_ids=()) -> int:
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        stops = np.ascontiguousarray(list(stop_ids) or [0], dtype=np.uint32)
        rid = wh.C.c_uint64()
        self.ctx.check(wh.lib.wm_server_submit(self.h, wh._ptr(prompt, wh.C.c_uint32), prompt.size,
                                               max_new, eos, wh._ptr(stops, wh.C.c_uint32),
                                               len(stop_ids), wh.C.byref(params), seed,
                                               wh.C.byref(rid)))
        return rid.value

    def step(self) -> int:
        n = wh.C.c_uint32()
        self.ctx.check(wh.lib.wm_server_step(self.h, wh.C.byref(n)))
        return n.value

    def result(self, rid: int):
        """(ids so far, finished); raises the request's error if it failed."""
        n, fin = wh.C.c_uint32(), wh.C.c_int()
        self.ctx.check(wh.lib.wm_server_result(self.h, rid, None, 0, wh.C.byref(n), wh.C.byref(fin)))
        out = np.empty(max(n.value, 1), np.uint32)
        self.ctx.check(wh.lib.wm_server_result(self.h, rid, wh._ptr(out, wh.C.c_uint32), n.value,
                                               wh.C.byref(n), wh.C.byref(fin)))
        return out[: n.value].tolist(), bool(fin.value)

    def release(self, rid: int):
        self.ctx.check(wh.lib.wm_server_release(self.h, rid))


@dataclass(frozen=True)
class RaggedWorkload:
    """A continuous-batching step: sequence i holds contexts[i] pre-filled
    positions (N(0,1) K/V through the int8 KV quantiser, stream seed
    prefill_seeds[i]) and appends the token ids new_tokens[i]."""
    contexts: tuple
    new_tokens: tuple
    prefill_seeds: tuple

    @property
    def n_tokens(self) -> int:
        return sum(len(t) for t in self.new_tokens)


def ragged_workload(cfg: BitNetConfig, n_seq: int = 16, ctx_lo: int = 128, ctx_hi: int = 4064,
                    new_lo: int = 1, new_hi: int = 32) -> RaggedWorkload:
    """The ragged multi-sequence batch at BitNet-2B shape: n_seq sequences
    with contexts ~U[ctx_lo, ctx_hi] and ~U[new_lo, new_hi] new tokens each
    (ids uniform over the vocabulary), all drawn from master seed 5."""
    rng = np.random.default_rng(master_seed(5))
    ctxs = tuple(int(c) for c in rng.integers(ctx_lo, ctx_hi + 1, n_seq))
    news = [int(n) for n in rng.integers(new_lo, new_hi + 1, n_seq)]
    seqs = tuple(tuple(int(t) for t in rng.integers(0, cfg.vocab, n)) for n in news)
    seeds = tuple(master_seed(5) + 1 + i for i in range(n_seq))
    return RaggedWorkload(ctxs, seqs, seeds)


# ---------------------------------------------------------------------------
# GGUF images of host models (the file format src/gguf/reader.rs reads)
# ---------------------------------------------------------------------------

GGUF_MAGIC = 0x46554747
_GGUF_U32, _GGUF_F32, _GGUF_STR, _GGUF_ARR, _GGUF_U64 = 4, 6, 8, 9, 10


def _gguf_str(s: str) -> bytes:
    b = s.encode()
    return len(b).to_bytes(8, "little") + b


def _gguf_kv(key: str, vtype: int, value) -> bytes:
    out = _gguf_str(key) + vtype.to_bytes(4, "little")
    if vtype == _GGUF_U32:
        return out + int(value).to_bytes(4, "little")
    if vtype == _GGUF_U64:
        return out + int(value).to_bytes(8, "little")
    if vtype == _GGUF_F32:
        return out + np.float32(value).tobytes()
    if vtype == _GGUF_STR:
        return out + _gguf_str(value)
    if vtype == _GGUF_ARR:  # array of strings
        return out + _GGUF_STR.to_bytes(4, "little") + len(value).to_bytes(8, "little") + \
            b"".join(_gguf_str(v) for v in value)
    raise ValueError(vtype)


def gguf_tensors(hm: HostModel):
    """(name, GGUF shape, GGML type, bytes) of every tensor, token_embd and
    output_norm first, then each layer's roles; I2_S data is followed by its
    32-byte trailing scale block (src/gguf/tensor.rs:278-309)."""
    cfg = hm.cfg
    out = [("token_embd.weight", [cfg.n_embd, cfg.vocab], wh.TYPE_Q6K, hm.token_embd.tobytes()),
           ("output_norm.weight", [cfg.n_embd], 0, np.ascontiguousarray(hm.output_norm, np.float32).tobytes())]
    for l, hl in enumerate(hm.layers):
        for name in ("attn_norm", "attn_sub_norm"):
            out.append((f"blk.{l}.{name}.weight", [hl.norms[name].size], 0, hl.norms[name].tobytes()))
        for role in ROLES:
            ind, outd = role_shape(cfg, role)
            blk = hl.packed[role].tobytes() + wh.scale_block(hl.scales[role]).tobytes()
            out.append((f"blk.{l}.{role}.weight", [ind, outd], wh.TYPE_I2S, blk))
        for name in ("ffn_norm", "ffn_sub_norm"):
            out.append((f"blk.{l}.{name}.weight", [hl.norms[name].size], 0, hl.norms[name].tobytes()))
    return out


def gguf_metadata(cfg: BitNetConfig, arch: str = "bitnet-b1.58", alignment=None) -> list:
    """The metadata keys ModelConfig::from_gguf_metadata_with_prefix reads
    (src/model/config.rs:81-160), prefixed by the architecture string."""
    kv = [("general.architecture", _GGUF_STR, arch),
          ("general.name", _GGUF_STR, "synthetic BitNet b1.58"),
          (f"{arch}.block_count", _GGUF_U32, cfg.n_layers),
          (f"{arch}.embedding_length", _GGUF_U32, cfg.n_embd),
          (f"{arch}.feed_forward_length", _GGUF_U32, cfg.n_ff),
          (f"{arch}.context_length", _GGUF_U32, cfg.context_length),
          (f"{arch}.attention.head_count", _GGUF_U32, cfg.n_heads),
          (f"{arch}.attention.head_count_kv", _GGUF_U32, cfg.n_kv_heads),
          (f"{arch}.attention.layer_norm_rms_epsilon", _GGUF_F32, cfg.rms_eps),
          (f"{arch}.rope.dimension_count", _GGUF_U32, cfg.head_dim),
          (f"{arch}.rope.freq_base", _GGUF_F32, cfg.rope_base),
          (f"{arch}.vocab_size", _GGUF_U32, cfg.vocab),
          ("tokenizer.ggml.model", _GGUF_STR, "gpt2"),
          ("tokenizer.ggml.tokens", _GGUF_ARR, ["<s>", "</s>", "a", "b"])]
    if alignment is not None:
        kv.append(("general.alignment", _GGUF_U32, alignment))
    return kv


def gguf_image(tensors, metadata, alignment: int = 32, version: int = 3):
    """Yield the bytes of a GGUF file: header, metadata, tensor directory,
    padding to the alignment, tensor data (each tensor's offset aligned)."""
    head = [GGUF_MAGIC.to_bytes(4, "little"), version.to_bytes(4, "little"),
            len(tensors).to_bytes(8, "little"), len(metadata).to_bytes(8, "little")]
    head += [_gguf_kv(*kv) for kv in metadata]
    off = 0
    offsets = []
    for name, shape, typ, data in tensors:
        offsets.append(off)
        head.append(_gguf_str(name) + len(shape).to_bytes(4, "little") +
                    b"".join(int(d).to_bytes(8, "little") for d in shape) +
                    typ.to_bytes(4, "little") + off.to_bytes(8, "little"))
        off += len(data)
        off += -off % alignment
    h = b"".join(head)
    yield h + bytes(-len(h) % alignment)
    for name, shape, typ, data in tensors:
        yield data
        yield bytes(-len(data) % alignment)


def gguf_bytes(hm: HostModel, arch: str = "bitnet-b1.58", alignment: int = 32, version: int = 3) -> bytes:
    meta = gguf_metadata(hm.cfg, arch, None if alignment == 32 else alignment)
    return b"".join(gguf_image(gguf_tensors(hm), meta, alignment, version))


def write_gguf(path, hm: HostModel, arch: str = "bitnet-b1.58", alignment: int = 32) -> None:
    meta = gguf_metadata(hm.cfg, arch, None if alignment == 32 else alignment)
    with open(path, "wb") as f:
        for chunk in gguf_image(gguf_tensors(hm), meta, alignment):
            f.write(chunk)
