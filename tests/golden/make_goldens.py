"""Writes tests/golden/bitnet2b_decode64.json with the oracle (oracle/).

The BitNet-2B-shaped greedy decode: 30 layers, n_embd 2560, n_ff 6912,
20/5 heads, vocab 128256, random-init weights from master seed
0x5749_4C4C_0000_0004, KV cache pre-filled to 1024 positions with N(0,1),
start token 15339 at position 1024 (the reference's bench token,
src/main.rs:1293-1297), 64 greedy steps.  Records the ids and, per step,
the sha256 of the f32 logits, the maximum logit and the top-5 ids.

    python tests/golden/make_goldens.py      (about two minutes on 8 cores)
"""
import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (ROOT, ROOT / "project-willamette_amd", ROOT / "tests"):
    sys.path.insert(0, str(p))

import bitnet_synth as bs  # noqa: E402
from oracle.oracle_model import OracleModel  # noqa: E402

PREFILL, START, STEPS = 1024, 15339, 64


def main():
    cfg = bs.BITNET_2B
    seed = bs.master_seed(4)
    t0 = time.time()
    hm = bs.make_host_model(cfg, seed)
    orm = OracleModel(hm, threads=8)
    okv = orm.kv(cfg.context_length)
    k, v = bs.kv_prefill(cfg, seed, PREFILL)
    okv.append_positions(k, v)
    del k, v
    print(f"setup {time.time() - t0:.1f}s", flush=True)
    ids, logits = okv.greedy([START], STEPS, want_logits=True)
    print(f"decode {time.time() - t0:.1f}s", flush=True)
    out = {
        "workload": "BitNet-2B-shaped greedy decode, random-init weights",
        "seed": hex(seed),
        "prefill": PREFILL,
        "start_token": START,
        "steps": STEPS,
        "ids": [int(i) for i in ids],
        "logits_sha256": [hashlib.sha256(np.ascontiguousarray(l).tobytes()).hexdigest() for l in logits],
        "logits_max": [float(l.max()) for l in logits],
        "top5": [[int(i) for i in np.argsort(-l, kind="stable")[:5]] for l in logits],
    }
    (HERE / "bitnet2b_decode64.json").write_text(json.dumps(out, indent=1) + "\n")
    print("ids", out["ids"][:16], "...")


if __name__ == "__main__":
    main()
