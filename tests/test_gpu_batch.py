"""GPU parity: the ragged multi-sequence batch (int8 MFMA BitLinear GEMMs,
per-token norms, attention of every token over its own sequence cache) vs
the oracle run token by token.

Reference semantics: multi_token_forward (src/model/multi_forward.rs:49-243)
with a pre-filled int8 KV cache, which is the sequential prefill of
src/model/generate.rs:151-160: every token of every sequence goes through
forward_with_cache in order.  Bar: every row of the batched BitLinear equals
the single-row SSE2-i8 path bit for bit; each sequence's last hidden, its
next greedy token and the new cache codes equal the oracle's bit for bit.
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


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


# --------------------------------------------------------------------------
# batched BitLinear (one GEMM over m token rows)
# --------------------------------------------------------------------------

# up to 512 output tiles of 64 x 64: the kernel whose waves split K; more
# (the last two): the kernel whose waves split the tokens
MATMUL_SHAPES = [(128, 64, 1), (256, 100, 5), (2560, 640, 16), (2560, 2560, 63), (2560, 2560, 64),
                 (2560, 2560, 65), (2560, 6912, 200), (6912, 2560, 37), (640, 65, 130),
                 (2560, 13824, 200), (1024, 13000, 150)]


@pytest.mark.parametrize("in_dim,out_dim,m", MATMUL_SHAPES)
def test_matmul_rows_equal_single_row_path(ctx, in_dim, out_dim, m):
    rng = np.random.default_rng(in_dim * 7 + out_dim * 3 + m)
    packed = rng.integers(0, 256, out_dim * in_dim // 4, dtype=np.uint8)
    scale = np.float32(rng.uniform(0.5, 2.0))
    x = rng.standard_normal((m, in_dim)).astype(np.float32) * np.float32(rng.uniform(0.1, 30))
    x[m // 2] = 0.0  # an all-zero row: scale 1, output exactly 0
    w = ctx.upload_i2s(packed, scale, in_dim, out_dim)
    y = wh.bitlinear_i2s_matmul_f32(ctx, w, x)
    for r in range(m):
        ry, _, _, _ = orc.bitlinear_i8(packed, scale, in_dim, out_dim, x[r])
        assert bits_equal(y[r], ry), f"row {r} of {m} differs from the SSE2-i8 path"
    w.close()


def test_matmul_rejects_bad_lengths(ctx):
    rng = np.random.default_rng(5)
    w = ctx.upload_i2s(rng.integers(0, 256, 64 * 128 // 4, dtype=np.uint8), 1.0, 128, 64)
    x = np.zeros(3 * 128 + 1, np.float32)
    y = np.zeros(3 * 64, np.float32)
    with pytest.raises(wh.WillametteError) as e:
        ctx.check(wh.lib.wm_bitlinear_i2s_matmul_f32(ctx.h, w.h, wh._ptr(x, wh.C.c_float), x.size, 3,
                                                     wh._ptr(y, wh.C.c_float), y.size))
    assert e.value.kind == "Shape"
    w.close()


# --------------------------------------------------------------------------
# ragged batch forward
# --------------------------------------------------------------------------

SMALL = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=512, n_heads=2, n_kv_heads=1, head_dim=128,
                        vocab=1000, context_length=96)
GQA4 = bs.BitNetConfig(n_layers=3, n_embd=256, n_ff=384, n_heads=4, n_kv_heads=1, head_dim=64,
                       vocab=777, context_length=128)


@pytest.fixture(scope="module", params=[SMALL, GQA4], ids=["small", "gqa4"])
def pair(request, ctx):
    cfg = request.param
    hm = bs.make_host_model(cfg, seed=4321 + cfg.n_layers)
    dev = bs.load_device_model(ctx, hm)
    orm = OracleModel(hm)
    yield cfg, hm, dev, orm
    dev.close()
    orm.close()


def run_case(cfg, dev, orm, prefill, new_tokens, seed):
    """prefill[i] positions of N(0,1) K/V, then new_tokens[i] appended to
    sequence i in one batch; compared with the oracle token by token."""
    dkvs, okvs = [], []
    for i, n_pre in enumerate(prefill):
        dkv, okv = dev.kv_cache(cfg.context_length), orm.kv(cfg.context_length)
        if n_pre:
            k, v = bs.kv_prefill(cfg, seed=seed + i, n_pos=n_pre)
            dkv.append_positions(k, v)
            okv.append_positions(k, v)
        dkvs.append(dkv)
        okvs.append(okv)
    hidden, nxt = dev.batch_forward(dkvs, new_tokens)
    for i, toks in enumerate(new_tokens):
        okv = okvs[i]
        for tok in toks:
            rh = okv.forward(int(tok), okv.position)
        _, rnext = okv.logits_argmax(rh)
        assert bits_equal(hidden[i], rh), f"sequence {i}: last hidden differs"
        assert nxt[i] == rnext, f"sequence {i}: next token {nxt[i]} != {rnext}"
        assert dkvs[i].position == okv.position == prefill[i] + len(toks)
        n_pos = okv.position
        for l in range(cfg.n_layers):
            dk, dks, dv, dvs = dkvs[i].read_raw(l, n_pos)
            ok, oks, ov, ovs = okv.read_raw(l, n_pos)
            assert np.array_equal(dk, ok) and np.array_equal(dv, ov), f"seq {i} layer {l}: cache codes"
            assert bits_equal(dks, oks) and bits_equal(dvs, ovs), f"seq {i} layer {l}: cache scales"
    for kv in dkvs + okvs:
        kv.close()


def test_batch_single_sequence_from_empty_cache(pair):
    cfg, hm, dev, orm = pair
    run_case(cfg, dev, orm, [0], [[3, 17, 42, 7, 1]], seed=10)


def test_batch_ragged_sequences(pair):
    cfg, hm, dev, orm = pair
    rng = np.random.default_rng(cfg.n_layers)
    prefill = [0, 5, 40, 1, 63, 17]
    new = [[int(t) for t in rng.integers(0, cfg.vocab, n)] for n in (4, 1, 7, 2, 3, 1)]
    run_case(cfg, dev, orm, prefill, new, seed=20)


def test_batch_decode_step_all_single_tokens(pair):
    cfg, hm, dev, orm = pair
    rng = np.random.default_rng(7)
    prefill = [int(p) for p in rng.integers(1, cfg.context_length - 2, 9)]
    new = [[int(rng.integers(0, cfg.vocab))] for _ in prefill]
    run_case(cfg, dev, orm, prefill, new, seed=30)


DENSE = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=384, n_heads=2, n_kv_heads=1, head_dim=128,
                        vocab=500, context_length=4096)


def test_batch_dense_softmax_long_rows(ctx):
    """attn_q scaled down to 1e-6: every score is tiny and no softmax weight
    underflows, so each row's exact exp sum crosses many binades and runs
    over several 512-term steps with ragged tails (rows of 1 to ~3000
    positions), every tile live; ragged batch against the oracle token by
    token."""
    hm = bs.make_host_model(DENSE, seed=43)
    for hl in hm.layers:
        hl.scales["attn_q"] = 1e-6
    dev = bs.load_device_model(ctx, hm)
    orm = OracleModel(hm)
    rng = np.random.default_rng(12)
    prefill = [2999, 1030, 511, 0, 64]
    new = [[int(t) for t in rng.integers(0, DENSE.vocab, n)] for n in (3, 2, 4, 1, 6)]
    run_case(DENSE, dev, orm, prefill, new, seed=50)
    dev.close()
    orm.close()


def test_batch_over_64_tokens(pair):
    # more than one 64-token GEMM tile, tiles shared by several sequences
    cfg, hm, dev, orm = pair
    rng = np.random.default_rng(11)
    prefill = [2, 0, 30]
    new = [[int(t) for t in rng.integers(0, cfg.vocab, n)] for n in (33, 29, 20)]
    run_case(cfg, dev, orm, prefill, new, seed=40)


def test_batch_rejects(pair):
    cfg, hm, dev, orm = pair
    a, b = dev.kv_cache(8), dev.kv_cache(8)
    for kvs, seqs in (([a, a], [[1], [2]]),            # the same cache twice
                      ([a, b], [[1], []]),             # an empty sequence
                      ([a], [[1] * 9]),                # past max_seq_len
                      ([a], [[cfg.vocab]])):           # token out of range
        with pytest.raises(wh.WillametteError):
            dev.batch_forward(kvs, seqs)
        assert a.position == 0 and b.position == 0
    a.close()
    b.close()


def test_batch_nonfinite_leaves_caches_untouched(ctx):
    cfg = SMALL
    hm = bs.make_host_model(cfg, seed=77)
    hm.layers[1].norms["ffn_sub_norm"][:] = np.inf
    dev = bs.load_device_model(ctx, hm)
    a, b = dev.kv_cache(cfg.context_length), dev.kv_cache(cfg.context_length)
    k, v = bs.kv_prefill(cfg, seed=3, n_pos=4)
    a.append_positions(k, v)
    with pytest.raises(wh.WillametteError) as e:
        dev.batch_forward([a, b], [[1, 2], [3]])
    assert e.value.kind == "NonFinite"
    assert a.position == 4 and b.position == 0
    a.close()
    b.close()
    dev.close()


def test_batch_bitnet2b_shape(ctx):
    """BitNet-2B shape: three sequences with contexts of 100, 1024 and 37
    pre-filled positions append 3, 1 and 2 tokens."""
    cfg = bs.BITNET_2B
    hm = bs.make_host_model(cfg, bs.master_seed(5))
    dev = bs.load_device_model(ctx, hm)
    orm = OracleModel(hm)
    try:
        run_case(cfg, dev, orm, [100, 1024, 37], [[15339, 11, 500], [128000], [7, 9]], seed=50)
    finally:
        dev.close()
        orm.close()


GOLDEN = Path(__file__).resolve().parent / "golden"


def test_batch_bitnet2b_ragged16_matches_oracle_fixture(ctx):
    """The benchmark's ragged step at its own size: BitNet-2B shape, 16
    sequences with contexts 1002-3842 appending 3-25 tokens each (257 in
    all), one wm_batch_forward.  Each sequence's next id, the SHA-256 of its
    last hidden and of its new cache rows must equal the oracle's
    token-by-token run recorded in tests/golden/bitnet2b_ragged16.json."""
    gold = json.loads((GOLDEN / "bitnet2b_ragged16.json").read_text())
    cfg = bs.BITNET_2B
    wl = bs.ragged_workload(cfg)
    assert [s["context"] for s in gold["sequences"]] == list(wl.contexts)
    hm = bs.make_host_model(cfg, bs.master_seed(4))
    dev = bs.load_device_model(ctx, hm)
    kvs = []
    for i, c in enumerate(wl.contexts):
        kv = dev.kv_cache(cfg.context_length)
        k, v = bs.kv_prefill(cfg, wl.prefill_seeds[i], c)
        kv.append_positions(k, v)
        del k, v
        kvs.append(kv)
    hidden, nxt = dev.batch_forward(kvs, wl.new_tokens)
    for i, rec in enumerate(gold["sequences"]):
        c, n = wl.contexts[i], len(wl.new_tokens[i])
        assert kvs[i].position == c + n
        assert nxt[i] == rec["next_id"], f"sequence {i}: next id"
        assert hashlib.sha256(np.ascontiguousarray(hidden[i], np.float32).tobytes()).hexdigest() == \
            rec["hidden_sha256"], f"sequence {i}: last hidden"
        h = hashlib.sha256()
        for layer in range(cfg.n_layers):
            k, ks, v, vs = kvs[i].read_raw(layer, c + n)
            for a in (k[c:], ks[c:], v[c:], vs[c:]):
                h.update(np.ascontiguousarray(a).tobytes())
        assert h.hexdigest() == rec["kv_sha256"], f"sequence {i}: new cache rows"
    for kv in kvs:
        kv.close()
    dev.close()
