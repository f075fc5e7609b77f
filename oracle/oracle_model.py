"""Oracle-side twin of bitnet_synth.DeviceModel: the same HostModel loaded
into oracle/wm_oracle.c's model (test infrastructure)."""
from __future__ import annotations

import ctypes as C

import numpy as np

import bitnet_synth as bs
import oracle.oracle as orc


class OracleModel:
    def __init__(self, hm: bs.HostModel, threads: int = 8):
        cfg = hm.cfg
        self.cfg, self.hm = cfg, hm
        self.h = orc.lib.or_model_create(cfg.n_layers, cfg.n_embd, cfg.n_ff, cfg.n_heads,
                                         cfg.n_kv_heads, cfg.head_dim, cfg.vocab, cfg.rms_eps,
                                         cfg.rope_base)
        assert self.h
        self._keep = []
        for l, hl in enumerate(hm.layers):
            args = []
            for role in bs.ROLES:
                a = np.ascontiguousarray(hl.packed[role])
                self._keep.append(a)
                args += [orc.P(a, C.c_uint8), hl.scales[role]]
            norms = []
            for n in bs.NORMS:
                a = np.ascontiguousarray(hl.norms[n], np.float32)
                self._keep.append(a)
                norms.append(orc.P(a, C.c_float))
            assert orc.lib.or_model_set_layer(self.h, l, *args, *norms) == 0
        self._keep += [hm.token_embd, hm.output_norm]
        assert orc.lib.or_model_set_output(self.h, orc.P(hm.token_embd, C.c_uint8),
                                           orc.P(hm.output_norm, C.c_float)) == 0
        orc.lib.or_model_set_threads(self.h, threads)

    def close(self):
        if self.h:
            orc.lib.or_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def kv(self, max_seq: int) -> "OracleKV":
        return OracleKV(self, max_seq)

    def forward_position_zero(self, token: int, trace: bool = False):
        """forward_single_token_position_zero: (hidden after output_norm[,
        hidden after each layer]); RuntimeError on a non-finite layer."""
        cfg = self.cfg
        hidden = np.empty(cfg.n_embd, np.float32)
        tr = np.empty((cfg.n_layers, cfg.n_embd), np.float32) if trace else None
        rc = orc.lib.or_forward_single_token_position_zero(self.h, token, orc.P(hidden, C.c_float),
                                                           orc.P(tr, C.c_float) if trace else None)
        if rc:
            raise RuntimeError(f"oracle position-zero forward failed rc={rc}")
        return (hidden, tr) if trace else hidden


class OracleKV:
    def __init__(self, m: OracleModel, max_seq: int):
        self.m = m
        self.h = orc.lib.or_kv_create(m.cfg.n_layers, m.cfg.kv_dim, max_seq)
        assert self.h

    def close(self):
        if self.h:
            orc.lib.or_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def position(self):
        return int(orc.lib.or_kv_position(self.h))

    def rollback(self, pos: int):
        orc.lib.or_kv_rollback(self.h, pos)

    def append_positions(self, k: np.ndarray, v: np.ndarray):
        for p in range(k.shape[0]):
            kp = np.ascontiguousarray(k[p], np.float32)
            vp = np.ascontiguousarray(v[p], np.float32)
            assert orc.lib.or_kv_append_position(self.h, orc.P(kp, C.c_float), orc.P(vp, C.c_float)) == 0

    def read_raw(self, layer: int, n_pos: int):
        kvd = self.m.cfg.kv_dim
        k = np.empty(n_pos * kvd, np.int8)
        v = np.empty(n_pos * kvd, np.int8)
        ks = np.empty(n_pos, np.float32)
        vs = np.empty(n_pos, np.float32)
        assert orc.lib.or_kv_read_raw(self.h, layer, orc.P(k, C.c_int8), orc.P(ks, C.c_float),
                                      orc.P(v, C.c_int8), orc.P(vs, C.c_float), n_pos) == 0
        return k.reshape(n_pos, kvd), ks, v.reshape(n_pos, kvd), vs

    def forward(self, token: int, pos: int, trace: bool = False):
        cfg = self.m.cfg
        hidden = np.empty(cfg.n_embd, np.float32)
        tr = np.empty((cfg.n_layers, cfg.n_embd), np.float32) if trace else None
        rc = orc.lib.or_forward_with_cache(self.m.h, self.h, token, pos, orc.P(hidden, C.c_float),
                                           orc.P(tr, C.c_float) if trace else None)
        if rc:
            raise RuntimeError(f"oracle forward failed rc={rc}")
        return (hidden, tr) if trace else hidden

    def logits_argmax(self, hidden: np.ndarray):
        logits = np.empty(self.m.cfg.vocab, np.float32)
        nxt = C.c_uint32()
        hidden = np.ascontiguousarray(hidden, np.float32)
        assert orc.lib.or_logits_argmax(self.m.h, orc.P(hidden, C.c_float), orc.P(logits, C.c_float),
                                        C.byref(nxt)) == 0
        return logits, int(nxt.value)

    def greedy(self, prompt, max_new: int, eos: int = -1, want_logits: bool = False):
        prompt = np.ascontiguousarray(prompt, np.uint32)
        out = np.empty(max(max_new, 1), np.uint32)
        n = C.c_uint32()
        lt = np.empty((max_new, self.m.cfg.vocab), np.float32) if want_logits else None
        rc = orc.lib.or_greedy_generate(self.m.h, self.h, orc.P(prompt, C.c_uint32), prompt.size,
                                        max_new, eos, orc.P(out, C.c_uint32), C.byref(n),
                                        orc.P(lt, C.c_float) if want_logits else None)
        if rc:
            raise RuntimeError(f"oracle greedy failed rc={rc}")
        ids = out[: n.value].tolist()
        return (ids, lt) if want_logits else ids
