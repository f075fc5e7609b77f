"""Writes tests/golden/bitnet2b_ragged16.json with the oracle (oracle/).

The ragged multi-sequence batch at BitNet-2B shape, as the benchmark runs
it: the decode model (random-init weights from master seed
0x5749_4C4C_0000_0004), 16 sequences whose caches are pre-filled to
contexts ~U[128, 4064] with N(0,1) K/V, each appending 1-32 new tokens
(bitnet_synth.ragged_workload).  The oracle runs every sequence token by
token through forward_with_cache (the sequential prefill of
src/model/generate.rs:151-160) and, after its last token, the lm-head and
argmax.  Recorded per sequence:
  next_id        argmax of the last token's logits
  hidden_sha256  SHA-256 of the last token's f32 hidden after output_norm
  kv_sha256      SHA-256 over layers of the new positions' K codes, K
                 scales, V codes and V scales (layer-major, in that order)

    python tests/golden/make_ragged_golden.py      (a few minutes on 8 cores)
"""
import hashlib
import json
import multiprocessing as mp
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (ROOT, ROOT / "project-willamette_amd", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import bitnet_synth as bs  # noqa: E402

OUT = HERE / "bitnet2b_ragged16.json"


def kv_digest(rows) -> str:
    """rows: per layer (k codes, k scales, v codes, v scales) of the new positions."""
    h = hashlib.sha256()
    for k, ks, v, vs in rows:
        for a in (k, ks, v, vs):
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def run_sequence(i: int):
    from oracle.oracle_model import OracleModel
    cfg = bs.BITNET_2B
    wl = bs.ragged_workload(cfg)
    hm = bs.make_host_model(cfg, bs.master_seed(4))
    orm = OracleModel(hm, threads=1)
    okv = orm.kv(cfg.context_length)
    c = wl.contexts[i]
    k, v = bs.kv_prefill(cfg, wl.prefill_seeds[i], c)
    okv.append_positions(k, v)
    del k, v
    hidden = None
    for j, tok in enumerate(wl.new_tokens[i]):
        hidden = okv.forward(tok, c + j)
    _, nxt = okv.logits_argmax(hidden)
    n = len(wl.new_tokens[i])
    rows = []
    for layer in range(cfg.n_layers):
        kk, ks, vv, vs = okv.read_raw(layer, c + n)
        rows.append((kk[c:], ks[c:], vv[c:], vs[c:]))
    out = {"context": c, "new_tokens": list(wl.new_tokens[i]), "next_id": int(nxt),
           "hidden_sha256": hashlib.sha256(np.ascontiguousarray(hidden, np.float32).tobytes()).hexdigest(),
           "kv_sha256": kv_digest(rows)}
    okv.close()
    orm.close()
    return i, out


def main():
    cfg = bs.BITNET_2B
    wl = bs.ragged_workload(cfg)
    t0 = time.time()
    seqs = [None] * len(wl.contexts)
    with mp.get_context("spawn").Pool(8) as pool:
        for i, rec in pool.imap_unordered(run_sequence, range(len(wl.contexts))):
            seqs[i] = rec
            print(f"sequence {i}: context {rec['context']}, {len(rec['new_tokens'])} tokens, "
                  f"next {rec['next_id']} ({time.time() - t0:.0f}s)", flush=True)
    out = {
        "workload": "ragged 16-sequence batch, BitNet-2B shape, random-init weights",
        "model_seed": hex(bs.master_seed(4)),
        "workload_seed": hex(bs.master_seed(5)),
        "sequences": seqs,
        "next_id_xor": int(np.bitwise_xor.reduce(np.array([s["next_id"] for s in seqs], np.uint64))),
    }
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {OUT.name}: {wl.n_tokens} tokens in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
