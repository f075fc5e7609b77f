"""GPU parity of the norm-fused matvecs' rarer paths.

The fused matvecs quantise speculatively from the rsqrt of the float64
total of the squares while the exact sequential sum runs, then redo exactly
the codes that the exact rsqrt and max|y| could change, or every code when
too many could, or when max|y| cannot come from the candidate lists.  On
ordinary inputs the first path almost always suffices; the test hook
wm_debug_set_fused_flags forces the others (the approximate max|y| skewed
by 2^-12 or 2^-7, the candidate lists treated as failed).  Bar: the same bits
as without the hook, i.e. the oracle's: the FFN block (config 3's own
inputs), small models' decode steps, and the BitNet-2B decode's first steps
(ids and logits SHA-256 of tests/golden/bitnet2b_decode64.json).
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import bitnet_synth as bs
import oracle.oracle as orc
import willamette_hip as wh
from oracle.oracle_model import OracleModel

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
FLAGS = {"skew_small": 1, "skew_large": 2, "no_candidates": 4, "skew_small+no_candidates": 5}
SMALL = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=512, n_heads=2, n_kv_heads=1, head_dim=128,
                        vocab=1000, context_length=64)


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


class fused_flags:
    def __init__(self, ctx, flags):
        self.ctx, self.flags = ctx, flags

    def __enter__(self):
        self.ctx.check(wh.lib.wm_debug_set_fused_flags(self.ctx.h, self.flags))

    def __exit__(self, *exc):
        self.ctx.check(wh.lib.wm_debug_set_fused_flags(self.ctx.h, 0))


def test_unknown_flags_rejected(ctx):
    with pytest.raises(wh.WillametteError) as e:
        ctx.check(wh.lib.wm_debug_set_fused_flags(ctx.h, 32))
    assert e.value.status == 6  # WM_E_ARG


@pytest.mark.parametrize("name", list(FLAGS))
def test_ffn_block_exact_on_forced_paths(ctx, name):
    E, F = 2560, 6912
    s = bs.master_seed(3)
    g, u, d = wh.synth_i2s(s, 1, E, F), wh.synth_i2s(s, 2, E, F), wh.synth_i2s(s, 3, F, E)
    sc = wh.synth_uniform(s, 4, 3, 0.5, 2.0)
    nw, sw = wh.synth_uniform(s, 5, E, 0.9, 1.1), wh.synth_uniform(s, 6, F, 0.9, 1.1)
    x = wh.synth_normal(s, 7, E)
    tg, tu, td = (ctx.upload_i2s(g, float(sc[0]), E, F), ctx.upload_i2s(u, float(sc[1]), E, F),
                  ctx.upload_i2s(d, float(sc[2]), F, E))
    ref = orc.ffn_block(x, nw, g, sc[0], u, sc[1], d, sc[2], sw, F)
    print(f"ffn block, flags {name}", flush=True)
    with fused_flags(ctx, FLAGS[name]):
        for f in (1.0, 1000.0, 1e-3):
            xs = (x * np.float32(f)).astype(np.float32)
            want = ref if f == 1.0 else orc.ffn_block(xs, nw, g, sc[0], u, sc[1], d, sc[2], sw, F)
            assert same_bits(wh.ffn_block_forward(ctx, xs, nw, tg, tu, td, sw), want)


@pytest.mark.parametrize("name", list(FLAGS))
def test_small_model_decode_exact_on_forced_paths(ctx, name):
    hm = bs.make_host_model(SMALL, seed=1234 + SMALL.n_layers)
    dev, orm = bs.load_device_model(ctx, hm), OracleModel(hm)
    dkv, okv = dev.kv_cache(SMALL.context_length), orm.kv(SMALL.context_length)
    print(f"small model decode, flags {name}", flush=True)
    with fused_flags(ctx, FLAGS[name]):
        tok = 3
        for pos in range(10):
            h, logits, nxt = dkv.decode_step(tok, pos)
            rh = okv.forward(tok, pos)
            rlogits, rnxt = okv.logits_argmax(rh)
            assert same_bits(h, rh) and same_bits(logits, rlogits) and nxt == rnxt, f"pos {pos}"
            tok = nxt
    dkv.close()
    dev.close()
    orm.close()


@pytest.fixture(scope="module")
def bitnet2b(ctx):
    gold = json.loads((GOLDEN / "bitnet2b_decode64.json").read_text())
    cfg = bs.BITNET_2B
    seed = bs.master_seed(4)
    hm = bs.make_host_model(cfg, seed)
    dev = bs.load_device_model(ctx, hm)
    k, v = bs.kv_prefill(cfg, seed, gold["prefill"])
    dkv = dev.kv_cache(cfg.context_length)
    dkv.append_positions(k, v)
    del k, v, hm
    yield gold, dkv
    dkv.close()
    dev.close()


@pytest.mark.parametrize("name", list(FLAGS))
def test_bitnet2b_decode_exact_on_forced_paths(ctx, bitnet2b, name):
    """Every fused matvec of the BitNet-2B step on the forced path (QKV with
    RoPE and split heads, O, gate/up, down): 6 steps, ids and logits."""
    gold, dkv = bitnet2b
    dkv.rollback(gold["prefill"])
    tok, pos = gold["start_token"], gold["prefill"]
    print(f"bitnet2b decode, flags {name}", flush=True)
    with fused_flags(ctx, FLAGS[name]):
        for step in range(6):
            _, logits, nxt = dkv.decode_step(tok, pos)
            assert hashlib.sha256(np.ascontiguousarray(logits, np.float32).tobytes()).hexdigest() == \
                gold["logits_sha256"][step], f"step {step}"
            assert nxt == gold["ids"][step]
            tok, pos = nxt, pos + 1


ATTN_NO_WAIT = 8


def test_attention_wait_gives_up_without_hanging(ctx):
    """Decode attention's workgroups of a kv head meet once their scores are
    out (a bounded wait).  With the hook every wait gives up at once: the
    step must fail (WM_E_HIP, the layer named), leave the cache where it
    was, and the following steps must be the oracle's bit for bit (the
    arrival counters stay consistent after a failed launch)."""
    hm = bs.make_host_model(SMALL, seed=77)
    dev, orm = bs.load_device_model(ctx, hm), OracleModel(hm)
    dkv, okv = dev.kv_cache(SMALL.context_length), orm.kv(SMALL.context_length)
    tok = 5
    for pos in range(3):
        h, _, nxt = dkv.decode_step(tok, pos)
        assert same_bits(h, okv.forward(tok, pos)), f"pos {pos}"
        tok = nxt
    print("attention wait hook: failing step at position 3", flush=True)
    with fused_flags(ctx, ATTN_NO_WAIT):
        with pytest.raises(wh.WillametteError) as e:
            dkv.decode_step(tok, 3)
    assert e.value.status == 5 and "attention workgroups stopped waiting" in str(e.value)
    assert dkv.position == 3
    for pos in range(3, 8):
        h, logits, nxt = dkv.decode_step(tok, pos)
        rh = okv.forward(tok, pos)
        rlogits, rnxt = okv.logits_argmax(rh)
        assert same_bits(h, rh) and same_bits(logits, rlogits) and nxt == rnxt, f"pos {pos}"
        tok = nxt
    print("attention wait hook: greedy with every wait failing", flush=True)
    before = dkv.position
    with fused_flags(ctx, ATTN_NO_WAIT):
        with pytest.raises(wh.WillametteError) as e:
            dkv.greedy([tok], 4)
    assert e.value.status == 5 and dkv.position == before
    dkv.close()
    dev.close()
    orm.close()


ATTN_LOOSE_COUNT = 16


@pytest.mark.parametrize("cfg_name", ["small", "medium"])
def test_attention_restarts_scores_on_the_device_count(ctx, cfg_name):
    """The greedy loop sizes each attention launch for the count the host
    expects, and the kernel's first loads go out for it before the device's
    position arrives.  With the hook the launches are sized for up to 9
    positions more, so every launch starts its scores again with the
    device's count (and workgroups with no positions under the host's count
    get some): the ids must still be the oracle's, and the cache ends where
    the oracle's does."""
    cfg = SMALL if cfg_name == "small" else MEDIUM
    hm = bs.make_host_model(cfg, seed=606)
    dev, orm = bs.load_device_model(ctx, hm), OracleModel(hm)
    dkv, okv = dev.kv_cache(cfg.context_length), orm.kv(cfg.context_length)
    print(f"attention loose count, {cfg_name}", flush=True)
    with fused_flags(ctx, ATTN_LOOSE_COUNT):
        ids = dkv.greedy([3, 1, 4], max_new=20)
    assert ids == okv.greedy([3, 1, 4], max_new=20) and len(ids) == 20
    assert dkv.position == okv.position
    dkv.close()
    dev.close()
    orm.close()


MEDIUM = bs.BitNetConfig(n_layers=2, n_embd=1024, n_ff=1536, n_heads=8, n_kv_heads=2, head_dim=128,
                         vocab=1000, context_length=64)


@pytest.mark.parametrize("name", ["none"] + list(FLAGS))
def test_medium_model_decode_exact(ctx, name):
    """A 1024 / 1536 model (8 query heads over 2 kv heads; 16-wave fused
    matvecs with 8 lanes per row for Q/K/V, O and down): decode steps
    bit-exact against the oracle, on the fused matvecs' forced paths too."""
    hm = bs.make_host_model(MEDIUM, seed=4321)
    dev, orm = bs.load_device_model(ctx, hm), OracleModel(hm)
    dkv, okv = dev.kv_cache(MEDIUM.context_length), orm.kv(MEDIUM.context_length)
    print(f"medium model decode, flags {name}", flush=True)
    with fused_flags(ctx, FLAGS.get(name, 0)):
        tok = 9
        for pos in range(8):
            h, logits, nxt = dkv.decode_step(tok, pos)
            rh = okv.forward(tok, pos)
            rlogits, rnxt = okv.logits_argmax(rh)
            assert same_bits(h, rh) and same_bits(logits, rlogits) and nxt == rnxt, f"pos {pos}"
            tok = nxt
    dkv.close()
    dev.close()
    orm.close()
