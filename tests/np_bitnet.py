"""An independent float64 numpy restatement of the BitNet b1.58 forward with
the int8 KV cache (test infrastructure: it checks the oracle's composition).

Written from the reference's description of the step, vectorised over
whole vectors and heads, not from the oracle's loops:
  embedding      Q6_K row dequantised (src/model/q6_k.rs:25-69)
  per layer      src/model/cached_forward.rs:308-415 and :451-502:
                 attn_norm -> Q, K, V BitLinears -> NEOX RoPE on Q and K ->
                 K/V appended through the int8 KV quantiser
                 (src/model/kv_cache.rs:245-259) -> GQA attention over the
                 dequantised cache, query head h reading kv head h // group
                 (src/model/primitives.rs:377) -> attn_sub_norm -> O ->
                 hidden += O -> ffn_norm -> gate, up -> relu(gate)^2 * up ->
                 ffn_sub_norm -> down -> hidden += down
  output         output_norm; logits = dequantised Q6_K rows . hidden
BitLinear is the int8 activation path of src/model/bitlinear_sse2.rs:285-342
(per-vector absmax codes, an exact integer dot with the ternary matrix, the
two scales), evaluated in float64.

The knobs in `Mistakes` plant one plausible composition error each; the
tests use them to show that the tolerance they compare the oracle with is
tight enough to catch such an error.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def unpack_ternary(packed: np.ndarray, in_dim: int, out_dim: int) -> np.ndarray:
    """I2_S bytes -> int8 [out_dim, in_dim] (codes 00 -1, 01 0, 10 +1, 11 0;
    byte g of a 32-byte block holds columns g, 32+g, 64+g, 96+g from the top
    bit pair down, docs/BITLINEAR_I2S_MATVEC.md)."""
    b = packed[: in_dim // 4 * out_dim].reshape(out_dim, in_dim // 128, 32)
    codes = np.stack([(b >> 6) & 3, (b >> 4) & 3, (b >> 2) & 3, b & 3], axis=2)
    return np.array([-1, 0, 1, 0], np.int8)[codes].reshape(out_dim, in_dim)


def q6k_dequant(rows: np.ndarray, n: int) -> np.ndarray:
    """Q6_K rows (210-byte blocks) -> float64 [n_rows, n]."""
    blk = rows.reshape(-1, 210)
    nb = blk.shape[0]
    d = (blk[:, 208].astype(np.uint16) | (blk[:, 209].astype(np.uint16) << 8)).view(np.float16)
    d = d.astype(np.float64)
    out = np.empty((nb, 256), np.float64)
    for h in range(2):
        ql = blk[:, h * 64:(h + 1) * 64].astype(np.int32)
        qh = blk[:, 128 + h * 32:128 + (h + 1) * 32].astype(np.int32)
        sc = blk[:, 192 + h * 8:192 + (h + 1) * 8].view(np.int8).astype(np.float64)
        lo, hi = ql[:, :32], ql[:, 32:]
        q = [(lo & 15) | ((qh & 3) << 4), (hi & 15) | (((qh >> 2) & 3) << 4),
             (lo >> 4) | (((qh >> 4) & 3) << 4), (hi >> 4) | (((qh >> 6) & 3) << 4)]
        l = np.arange(32)
        for k in range(4):
            s = sc[:, l // 16 + 2 * k]
            out[:, h * 128 + 32 * k: h * 128 + 32 * k + 32] = d[:, None] * s * (q[k] - 32)
    return out.reshape(-1, n)


def round_half_away(v: np.ndarray) -> np.ndarray:
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def bitlinear(t: np.ndarray, w_scale: float, x: np.ndarray) -> np.ndarray:
    m = np.abs(x).max()
    if m == 0:
        return np.zeros(t.shape[0])
    q = np.clip(round_half_away(x * (127.0 / m)), -127, 127).astype(np.int64)
    return (w_scale * (m / 127.0)) * (t.astype(np.int64) @ q)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    return x / np.sqrt(np.mean(x * x) + eps) * w


def kv_round_trip(x: np.ndarray) -> np.ndarray:
    m = np.abs(x).max()
    if m == 0 or not np.isfinite(m):
        return np.zeros_like(x)
    return np.clip(round_half_away(x * (127.0 / m)), -127, 127) * (m / 127.0)


@dataclass
class Mistakes:
    kv_head_of: str = "div"      # "div": h // group (correct); "mod": h % n_kv_heads
    sub_norm: bool = True        # attn_sub_norm before O
    o_residual: bool = True      # hidden += O
    rope_pairs: str = "neox"     # "neox": (j, j + hd/2); "adjacent": (2j, 2j + 1)
    relu_square: bool = True     # relu(gate)^2 * up; False: relu(gate) * up
    rope_on_k: bool = True
    ffn_sub_norm: bool = True    # ffn_sub_norm before down
    gate_up_swapped: bool = False  # relu(up)^2 * gate


def ffn_block(t_gate, s_gate, t_up, s_up, t_down, s_down, norm_w, sub_norm_w, eps, x,
              mk: Mistakes | None = None) -> np.ndarray:
    """ffn_block_forward (src/model/ffn.rs:73-136), no residual: ffn_norm ->
    gate, up -> relu(gate)^2 * up -> ffn_sub_norm -> down."""
    mk = mk or Mistakes()
    xf = rms_norm(x, norm_w, eps)
    g = bitlinear(t_gate, s_gate, xf)
    u = bitlinear(t_up, s_up, xf)
    if mk.gate_up_swapped:
        g, u = u, g
    r = np.maximum(g, 0.0)
    f = (r * r if mk.relu_square else r) * u
    fn = rms_norm(f, sub_norm_w, eps) if mk.ffn_sub_norm else f
    return bitlinear(t_down, s_down, fn)


class NpModel:
    def __init__(self, hm, mistakes: Mistakes | None = None):
        self.hm, self.cfg = hm, hm.cfg
        self.mk = mistakes or Mistakes()
        cfg = self.cfg
        shapes = {"attn_q": (cfg.n_embd, cfg.n_embd), "attn_k": (cfg.n_embd, cfg.kv_dim),
                  "attn_v": (cfg.n_embd, cfg.kv_dim), "attn_output": (cfg.n_embd, cfg.n_embd),
                  "ffn_gate": (cfg.n_embd, cfg.n_ff), "ffn_up": (cfg.n_embd, cfg.n_ff),
                  "ffn_down": (cfg.n_ff, cfg.n_embd)}
        self.t = [{r: unpack_ternary(hl.packed[r], *shapes[r]) for r in shapes} for hl in hm.layers]
        self.embd_bytes = hm.token_embd.reshape(cfg.vocab, -1)
        self.k = [[] for _ in range(cfg.n_layers)]  # dequantised cache rows per layer
        self.v = [[] for _ in range(cfg.n_layers)]

    def embed(self, tok: int) -> np.ndarray:
        return q6k_dequant(self.embd_bytes[tok], self.cfg.n_embd)[0]

    def append_prefill(self, k: np.ndarray, v: np.ndarray):
        """k, v: [n_pos][n_layers][kv_dim] f32, through the KV quantiser."""
        for p in range(k.shape[0]):
            for l in range(self.cfg.n_layers):
                self.k[l].append(kv_round_trip(k[p, l].astype(np.float64)))
                self.v[l].append(kv_round_trip(v[p, l].astype(np.float64)))

    def rope(self, x: np.ndarray, pos: int) -> np.ndarray:
        hd = self.cfg.head_dim
        x = x.reshape(-1, hd).copy()
        j = np.arange(hd // 2)
        th = pos * self.cfg.rope_base ** (-2.0 * j / hd)
        c, s = np.cos(th), np.sin(th)
        if self.mk.rope_pairs == "neox":
            a, b = x[:, :hd // 2].copy(), x[:, hd // 2:].copy()
            x[:, :hd // 2], x[:, hd // 2:] = a * c - b * s, a * s + b * c
        else:
            a, b = x[:, 0::2].copy(), x[:, 1::2].copy()
            x[:, 0::2], x[:, 1::2] = a * c - b * s, a * s + b * c
        return x.reshape(-1)

    def attention(self, q: np.ndarray, l: int) -> np.ndarray:
        cfg = self.cfg
        hd, group = cfg.head_dim, cfg.n_heads // cfg.n_kv_heads
        K = np.stack(self.k[l]).reshape(-1, cfg.n_kv_heads, hd)
        V = np.stack(self.v[l]).reshape(-1, cfg.n_kv_heads, hd)
        qh = q.reshape(cfg.n_heads, hd)
        h = np.arange(cfg.n_heads)
        kvh = h // group if self.mk.kv_head_of == "div" else h % cfg.n_kv_heads
        s = np.einsum("hd,phd->hp", qh, K[:, kvh, :]) / np.sqrt(hd)
        w = np.exp(s - s.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        return np.einsum("hp,phd->hd", w, V[:, kvh, :]).reshape(-1)

    def layer(self, l: int, x: np.ndarray, pos: int, kv_row=None):
        """One layer at `pos` on hidden x; appends this position's K/V to the
        cache (kv_row = (k, v) dequantised rows to append instead of this
        model's own, for teacher-forced checks).  Returns (hidden after the
        layer, this model's own K after RoPE, its own V)."""
        eps = self.cfg.rms_eps
        T, sc = self.t[l], self.hm.layers[l].scales
        nm = {k: v.astype(np.float64) for k, v in self.hm.layers[l].norms.items()}
        xn = rms_norm(x, nm["attn_norm"], eps)
        q = self.rope(bitlinear(T["attn_q"], sc["attn_q"], xn), pos)
        k = bitlinear(T["attn_k"], sc["attn_k"], xn)
        if self.mk.rope_on_k:
            k = self.rope(k, pos)
        v = bitlinear(T["attn_v"], sc["attn_v"], xn)
        kr, vr = kv_row if kv_row is not None else (kv_round_trip(k), kv_round_trip(v))
        self.k[l].append(np.asarray(kr, np.float64))
        self.v[l].append(np.asarray(vr, np.float64))
        a = self.attention(q, l)
        if self.mk.sub_norm:
            a = rms_norm(a, nm["attn_sub_norm"], eps)
        o = bitlinear(T["attn_output"], sc["attn_output"], a)
        if self.mk.o_residual:
            x = x + o
        y = ffn_block(T["ffn_gate"], sc["ffn_gate"], T["ffn_up"], sc["ffn_up"], T["ffn_down"],
                      sc["ffn_down"], nm["ffn_norm"], nm["ffn_sub_norm"], eps, x, self.mk)
        return x + y, k, v

    def output(self, x: np.ndarray) -> np.ndarray:
        return rms_norm(x, self.hm.output_norm.astype(np.float64), self.cfg.rms_eps)

    def forward(self, tok: int, pos: int):
        """Returns (final hidden after output_norm, hidden after each layer)."""
        x = self.embed(tok)
        trace = []
        for l in range(self.cfg.n_layers):
            x, _, _ = self.layer(l, x, pos)
            trace.append(x.copy())
        return self.output(x), np.stack(trace)

    def layer_position_zero(self, l: int, x: np.ndarray) -> np.ndarray:
        """forward_single_token_position_zero's layer (src/model/block.rs:38-105):
        position 0, no cache: the attention sees only this token's own K and V
        as computed (no int8 round trip)."""
        saved = self.k[l], self.v[l]
        self.k[l], self.v[l] = [], []
        T, sc = self.t[l], self.hm.layers[l].scales
        xn = rms_norm(x, self.hm.layers[l].norms["attn_norm"].astype(np.float64), self.cfg.rms_eps)
        k = self.rope(bitlinear(T["attn_k"], sc["attn_k"], xn), 0) if self.mk.rope_on_k else \
            bitlinear(T["attn_k"], sc["attn_k"], xn)
        v = bitlinear(T["attn_v"], sc["attn_v"], xn)
        out, _, _ = self.layer(l, x, 0, kv_row=(k, v))
        self.k[l], self.v[l] = saved
        return out

    def logits(self, hidden: np.ndarray) -> np.ndarray:
        return q6k_dequant(self.hm.token_embd, self.cfg.n_embd) @ hidden
