"""GPU parity: the full decode step (embedding, 30-layer forward with KV
cache, output norm, lm-head, argmax) vs the oracle.

Bar: hidden states after every layer, final hidden, logits and KV cache
codes bit-identical to the oracle on the same seeded inputs, so greedy ids
are identical; the BitNet-2B-shaped 64-step greedy decode is checked against
committed oracle fixtures (tests/golden/bitnet2b_decode64.json).
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import bitnet_synth as bs
import willamette_hip as wh
from oracle.oracle_model import OracleModel

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"

SMALL = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=512, n_heads=2, n_kv_heads=1, head_dim=128,
                        vocab=1000, context_length=64)
GQA4 = bs.BitNetConfig(n_layers=3, n_embd=256, n_ff=384, n_heads=4, n_kv_heads=1, head_dim=64,
                       vocab=777, context_length=96)


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module", params=[SMALL, GQA4], ids=["small", "gqa4"])
def pair(request, ctx):
    cfg = request.param
    hm = bs.make_host_model(cfg, seed=1234 + cfg.n_layers)
    dev = bs.load_device_model(ctx, hm)
    orm = OracleModel(hm)
    yield cfg, hm, dev, orm
    dev.close()
    orm.close()


def test_forward_positions_bit_exact(pair):
    cfg, hm, dev, orm = pair
    dkv, okv = dev.kv_cache(cfg.context_length), orm.kv(cfg.context_length)
    tokens = [3, 17, 999 % cfg.vocab, 0, 42, 42, 7, 500 % cfg.vocab, 1, 2, 3, 4]
    for pos, tok in enumerate(tokens):
        h, tr = dkv.forward(tok, pos, trace=True)
        rh, rtr = okv.forward(tok, pos, trace=True)
        for l in range(cfg.n_layers):
            assert bits_equal(tr[l], rtr[l]), f"pos {pos}: hidden after layer {l} differs"
        assert bits_equal(h, rh), f"pos {pos}: final hidden differs"
    assert dkv.position == okv.position == len(tokens)
    for l in range(cfg.n_layers):
        dk, dks, dv, dvs = dkv.read_raw(l, len(tokens))
        ok, oks, ov, ovs = okv.read_raw(l, len(tokens))
        assert np.array_equal(dk, ok) and np.array_equal(dv, ov)
        assert bits_equal(dks, oks) and bits_equal(dvs, ovs)


def test_prefill_then_greedy_bit_exact(pair):
    cfg, hm, dev, orm = pair
    n_pre = cfg.context_length // 2
    k, v = bs.kv_prefill(cfg, seed=99, n_pos=n_pre)
    dkv, okv = dev.kv_cache(cfg.context_length), orm.kv(cfg.context_length)
    dkv.append_positions(k, v)
    okv.append_positions(k, v)
    for l in range(cfg.n_layers):
        dk, dks, _, dvs = dkv.read_raw(l, n_pre)
        ok, oks, _, ovs = okv.read_raw(l, n_pre)
        assert np.array_equal(dk, ok) and bits_equal(dks, oks) and bits_equal(dvs, ovs)
    # step by step: logits and next token
    tok, pos = 5, n_pre
    for step in range(6):
        h, logits, nxt = dkv.decode_step(tok, pos)
        rh = okv.forward(tok, pos)
        rlogits, rnxt = okv.logits_argmax(rh)
        assert bits_equal(h, rh) and bits_equal(logits, rlogits), f"step {step}"
        assert nxt == rnxt
        tok, pos = nxt, pos + 1
    # greedy loop on both from here
    ids = dkv.greedy([tok], max_new=cfg.context_length - pos - 2)
    rids = okv.greedy([tok], max_new=cfg.context_length - pos - 2)
    assert ids == rids and len(ids) > 0


def test_greedy_eos_stops(pair):
    cfg, hm, dev, orm = pair
    dkv, okv = dev.kv_cache(cfg.context_length), orm.kv(cfg.context_length)
    ids = dkv.greedy([1, 2, 3], max_new=8)
    eos = ids[3]
    dkv2 = dev.kv_cache(cfg.context_length)
    ids2 = dkv2.greedy([1, 2, 3], max_new=8, eos=eos)
    assert ids2 == ids[: ids.index(eos)]
    assert ids == okv.greedy([1, 2, 3], max_new=8)


def test_position_zero_forward_bit_exact(pair):
    """forward_single_token_position_zero: no cache, each head attends to the
    token's own f32 K/V; the final hidden is bit-identical to the oracle's,
    and differs from the cached step at position 0 (whose V goes through
    the int8 cache)."""
    cfg, hm, dev, orm = pair
    for tok in [0, 3, 17, cfg.vocab - 1]:
        h = dev.forward_position_zero(tok)
        assert bits_equal(h, orm.forward_position_zero(tok)), f"token {tok}"
    dkv = dev.kv_cache(cfg.context_length)
    assert not bits_equal(dev.forward_position_zero(3), dkv.forward(3, 0))


def test_kv_read_into_dequantises(pair):
    """KVCache::read_into: every cached row as code * the row's scale, for
    positions [0, position), equal to the raw codes and scales dequantised
    on the host; a layer out of range is rejected."""
    cfg, hm, dev, orm = pair
    dkv = dev.kv_cache(cfg.context_length)
    k, v = bs.kv_prefill(cfg, seed=8, n_pos=9)
    dkv.append_positions(k, v)
    dkv.forward(4, 9)
    for l in range(cfg.n_layers):
        K, V = dkv.read_into(l)
        kk, ks, vv, vs = dkv.read_raw(l, 10)
        assert K.shape == (10, cfg.kv_dim)
        assert bits_equal(K, kk.astype(np.float32) * ks[:, None])
        assert bits_equal(V, vv.astype(np.float32) * vs[:, None])
    with pytest.raises(wh.WillametteError) as e:
        dkv.read_into(cfg.n_layers)
    assert e.value.kind == "Shape"
    assert dev.kv_cache(cfg.context_length).read_into(0)[0].shape == (0, cfg.kv_dim)


def test_position_protocol_and_nonfinite_rollback(ctx):
    cfg = SMALL
    hm = bs.make_host_model(cfg, seed=5)
    dev = bs.load_device_model(ctx, hm)
    dkv = dev.kv_cache(cfg.context_length)
    dkv.forward(1, 0)
    with pytest.raises(wh.WillametteError) as e:
        dkv.forward(1, 5)  # tokens must be processed in order
    assert e.value.kind == "State"
    with pytest.raises(wh.WillametteError) as e:
        dkv.forward(cfg.vocab, 1)  # token out of vocab
    assert e.value.kind == "Shape"
    assert dkv.position == 1
    # An infinite ffn_sub_norm weight: the down projection's int8 quantiser
    # sees absmax = inf, every code becomes 0 and its scale inf, so the
    # projection yields inf * 0 = NaN and layer 0's hidden is non-finite
    # -> error + rollback (src/model/cached_forward.rs:256-259, :511-521).
    # (An infinite ffn_norm would not do: the NaN gate is zeroed by ReLU and
    # the sub-norm's quantiser drops NaN, so the hidden stays finite.)
    hm.layers[0].norms["ffn_sub_norm"][:] = np.inf
    bad = bs.load_device_model(ctx, hm)
    bkv = bad.kv_cache(cfg.context_length)
    with pytest.raises(wh.WillametteError) as e:
        bkv.forward(1, 0)
    assert e.value.kind == "NonFinite" and bkv.position == 0
    orm = OracleModel(hm)
    okv = orm.kv(cfg.context_length)
    with pytest.raises(RuntimeError):
        okv.forward(1, 0)
    assert okv.position == 0
    # the no-cache position-0 forward fails the same way, then leaves the
    # error flag clear for the next call
    with pytest.raises(wh.WillametteError) as e:
        bad.forward_position_zero(1)
    assert e.value.kind == "NonFinite"
    with pytest.raises(RuntimeError):
        orm.forward_position_zero(1)
    h = dev.forward_position_zero(2)
    assert np.all(np.isfinite(h))


def test_greedy_nonfinite_step_with_steps_in_flight(ctx):
    """The greedy loop enqueues steps ahead of the host.  Token T's
    embedding row has an infinite Q6_K d, so the step that embeds T makes
    layer 1's residual non-finite: the call fails with NonFinite, the cache
    is back at its starting position although later steps were already
    enqueued, and the error flag is cleared, so the next call decodes like
    the oracle."""
    cfg = SMALL
    hm = bs.make_host_model(cfg, seed=6)
    T = 77
    nb = cfg.n_embd // 256
    row0 = T * nb * 210
    hm.token_embd.reshape(-1)[row0 + 208:row0 + 210] = [0x00, 0x7C]  # d = +inf (f16)
    dev = bs.load_device_model(ctx, hm)
    dkv = dev.kv_cache(cfg.context_length)
    dkv.forward(1, 0)
    with pytest.raises(wh.WillametteError) as e:
        dkv.greedy([2, T], max_new=12)
    assert e.value.kind == "NonFinite" and dkv.position == 1
    ids = dkv.greedy([3], max_new=10)
    orm = OracleModel(hm)
    okv = orm.kv(cfg.context_length)
    okv.forward(1, 0)
    assert T not in ids and ids == okv.greedy([3], max_new=10)
    assert dkv.position == okv.position == 11
    dev.close()
    orm.close()


def _inf_embedding_model(cfg, seed, token):
    """The host model with an infinite Q6_K d in block 0 of `token`'s
    embedding row: the step that embeds it goes non-finite, and its tied
    lm-head logit is +-inf."""
    hm = bs.make_host_model(cfg, seed=seed)
    row0 = token * (cfg.n_embd // 256) * 210
    hm.token_embd.reshape(-1)[row0 + 208:row0 + 210] = [0x00, 0x7C]  # d = +inf (f16)
    return hm


def test_greedy_eos_clears_error_flag_of_steps_in_flight(ctx):
    """Steps queued past an EOS stop still run.  Here EOS is id 0 and row 0
    of the tied embedding has an infinite d: its logit is NaN, which wins
    the argmax at index 0 (lm_head.rs:161-174), so every step yields 0, and
    the steps queued behind the first one embed token 0 and raise the
    cumulative error flag.  The call still ends cleanly at EOS, and the next
    calls decode like the oracle instead of failing with NonFinite."""
    cfg = SMALL
    hm = _inf_embedding_model(cfg, 6, 0)
    orm = OracleModel(hm)
    okv = orm.kv(cfg.context_length)
    okv.forward(1, 0)
    dev = bs.load_device_model(ctx, hm)
    dkv = dev.kv_cache(cfg.context_length)
    dkv.forward(1, 0)
    assert dkv.greedy([2, 5], max_new=10, eos=0) == okv.greedy([2, 5], max_new=10, eos=0) == []
    assert dkv.position == okv.position == 3
    # the flag left by the steps past EOS must not fail these
    assert dkv.greedy([3], max_new=6, eos=0) == okv.greedy([3], max_new=6, eos=0) == []
    assert bits_equal(dkv.forward(4, dkv.position), okv.forward(4, okv.position))
    # generate_with_sampler (greedy parameters, no EOS) samples 0 and fails
    # on the step that embeds it: the cache goes back to where the call
    # found it
    dkv2 = dev.kv_cache(cfg.context_length)
    dkv2.forward(1, 0)
    with pytest.raises(wh.WillametteError) as e:
        dkv2.generate_sampled([2, 5], 10, wh.Sampler(ctx, wh.SamplingParams.make(), 7))
    assert e.value.kind == "NonFinite" and dkv2.position == 1
    okv2 = orm.kv(cfg.context_length)
    okv2.forward(1, 0)
    assert bits_equal(dkv2.forward(3, 1), okv2.forward(3, 1))
    dev.close()
    orm.close()


def test_zero_weight_model_closed_form(ctx):
    """tests/synthetic_model.rs analogue: all-zero ternary weights, unit norms,
    an all-ones embedding -> every BitLinear outputs 0, the hidden stays the
    embedding, output = 1/sqrt(1 + eps), all logits tie -> token 0."""
    cfg = SMALL
    hm = bs.make_host_model(cfg, seed=6)
    for hl in hm.layers:
        for r in bs.ROLES:
            hl.packed[r][:] = 0x55
        for n in bs.NORMS:
            hl.norms[n][:] = 1.0
    ones = np.concatenate([np.full(128, 0x11, np.uint8), np.full(64, 0xAA, np.uint8),
                           np.full(16, 1, np.uint8), np.array([0x00, 0x3C], np.uint8)])
    hm.token_embd = np.tile(ones, cfg.vocab * (cfg.n_embd // 256))
    hm.output_norm[:] = 1.0
    dev = bs.load_device_model(ctx, hm)
    dkv = dev.kv_cache(cfg.context_length)
    h, logits, nxt = dkv.decode_step(3, 0)
    expect = np.float32(1.0) * (np.float32(1.0) / np.sqrt(np.float32(1.0) + np.float32(1e-5)))
    assert np.all(h == expect)
    assert np.all(logits == logits[0]) and nxt == 0


def _sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def test_bitnet2b_decode64_matches_oracle_fixture(ctx):
    """Full BitNet-2B shape: 30 layers, 2560/6912, 20/5 heads, vocab 128256,
    KV pre-filled to 1024 positions with N(0,1), start token 15339, 64
    greedy steps.  Ids and every step's logits (sha256) must match the
    oracle's run recorded in tests/golden/bitnet2b_decode64.json."""
    gold = json.loads((GOLDEN / "bitnet2b_decode64.json").read_text())
    cfg = bs.BITNET_2B
    seed = bs.master_seed(4)
    hm = bs.make_host_model(cfg, seed)
    dev = bs.load_device_model(ctx, hm)
    k, v = bs.kv_prefill(cfg, seed, gold["prefill"])
    dkv = dev.kv_cache(cfg.context_length)
    dkv.append_positions(k, v)
    del k, v
    tok, pos = gold["start_token"], gold["prefill"]
    ids, shas = [], []
    for step in range(gold["steps"]):
        _, logits, nxt = dkv.decode_step(tok, pos)
        shas.append(_sha(logits))
        ids.append(nxt)
        tok, pos = nxt, pos + 1
    assert ids == gold["ids"]
    assert shas == gold["logits_sha256"]
    # the id-only lm-head (bounded pass + exact rescoring), the path the
    # benchmark times, over the same 64 steps from the rolled-back cache
    dkv.rollback(gold["prefill"])
    tok, pos = gold["start_token"], gold["prefill"]
    fast = []
    for step in range(gold["steps"]):
        _, _, nxt = dkv.decode_step(tok, pos, want_logits=False)
        fast.append(nxt)
        tok, pos = nxt, pos + 1
    assert fast == gold["ids"]
    # the library's greedy loop (steps enqueued ahead of the host), the
    # benchmark's timed call: the start token as a one-token prompt
    dkv.rollback(gold["prefill"])
    ids = dkv.greedy([gold["start_token"]], gold["steps"])
    assert ids == gold["ids"] and dkv.position == gold["prefill"] + gold["steps"]
    # EOS inside the window of steps in flight: the loop stops at it and the
    # cache ends one past the EOS step, whatever was enqueued after it
    dkv.rollback(gold["prefill"])
    eos_at = 5
    ids = dkv.greedy([gold["start_token"]], gold["steps"], eos=gold["ids"][eos_at])
    first = gold["ids"].index(gold["ids"][eos_at])
    assert ids == gold["ids"][:first] and dkv.position == gold["prefill"] + first + 1


LONG = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=384, n_heads=2, n_kv_heads=1, head_dim=128,
                       vocab=500, context_length=4096)


@pytest.mark.parametrize("n_pre", [3500, 4092])
def test_long_context_decode_bit_exact(ctx, n_pre):
    """Positions past 2048, up to the 4096-position context (the attention
    kernels' largest instantiation, above 64 KB of LDS), with a stale cache
    row at the decoded position: the row is first written with other values
    and rolled back, so the step must use this token's K/V, not the row's
    old contents (n_pre % 1024 is in [64, 1024): the row is loaded by a
    wave other than the one that writes the new V)."""
    cfg = LONG
    hm = bs.make_host_model(cfg, seed=31)
    dev = bs.load_device_model(ctx, hm)
    orm = OracleModel(hm)
    k, v = bs.kv_prefill(cfg, seed=32, n_pos=n_pre + 1)
    dkv, okv = dev.kv_cache(cfg.context_length), orm.kv(cfg.context_length)
    dkv.append_positions(k, v)  # one row past the prefill ...
    dkv.rollback(n_pre)         # ... left behind as a stale row
    okv.append_positions(k[:n_pre], v[:n_pre])
    tok, pos = 17, n_pre
    while pos < min(n_pre + 12, cfg.context_length):
        h, logits, nxt = dkv.decode_step(tok, pos)
        rh = okv.forward(tok, pos)
        rlogits, rnxt = okv.logits_argmax(rh)
        assert bits_equal(h, rh) and bits_equal(logits, rlogits), f"position {pos}"
        assert nxt == rnxt
        tok, pos = nxt, pos + 1
    for l in range(cfg.n_layers):
        dk, dks, dv, dvs = dkv.read_raw(l, pos)
        ok, oks, ov, ovs = okv.read_raw(l, pos)
        assert np.array_equal(dk[n_pre:], ok[n_pre:]) and np.array_equal(dv[n_pre:], ov[n_pre:])
        assert bits_equal(dks, oks) and bits_equal(dvs, ovs)
    dev.close()
    orm.close()


def test_greedy_across_attention_sizes(ctx):
    """The greedy loop's steps read their position on the device: 24 tokens
    from position 2040 cross from the attention instantiation for up to
    2048 positions to the larger one in one call, then more run after a
    rollback, against the oracle."""
    cfg = LONG
    hm = bs.make_host_model(cfg, seed=51)
    dev = bs.load_device_model(ctx, hm)
    orm = OracleModel(hm)
    n_pre = 2040
    k, v = bs.kv_prefill(cfg, seed=52, n_pos=n_pre)
    dkv, okv = dev.kv_cache(cfg.context_length), orm.kv(cfg.context_length)
    dkv.append_positions(k, v)
    okv.append_positions(k, v)
    ids = dkv.greedy([9], max_new=24)
    assert ids == okv.greedy([9], max_new=24) and dkv.position == okv.position == n_pre + 24
    for kv in (dkv, okv):
        kv.rollback(2050)
    ids = dkv.greedy([4, 5], max_new=10)
    assert ids == okv.greedy([4, 5], max_new=10) and dkv.position == okv.position == 2050 + 11
    dev.close()
    orm.close()


@pytest.mark.parametrize("n_pre", [40, 300, 1500, 3000])
def test_dense_softmax_decode_bit_exact(ctx, n_pre):
    """attn_q scaled down to 1e-6, so every score is tiny and no softmax
    weight underflows: the attention sums run over every position (the
    workgroup's exact exp sum, above 64 terms), against the oracle."""
    cfg = LONG
    hm = bs.make_host_model(cfg, seed=41)
    for hl in hm.layers:
        hl.scales["attn_q"] = 1e-6
    dev = bs.load_device_model(ctx, hm)
    orm = OracleModel(hm)
    k, v = bs.kv_prefill(cfg, seed=42, n_pos=n_pre)
    dkv, okv = dev.kv_cache(cfg.context_length), orm.kv(cfg.context_length)
    dkv.append_positions(k, v)
    okv.append_positions(k, v)
    tok, pos = 3, n_pre
    for _ in range(4):
        h, tr = dkv.forward(tok, pos, trace=True)
        rh, rtr = okv.forward(tok, pos, trace=True)
        for l in range(cfg.n_layers):
            assert bits_equal(tr[l], rtr[l]), f"position {pos}: layer {l}"
        assert bits_equal(h, rh)
        tok, pos = (tok * 7 + 1) % cfg.vocab, pos + 1
    dev.close()
    orm.close()
