"""CPU tests that pin the oracle's composition: its attention (or_sdpa), the
layer order inside or_forward_with_cache, and the greedy loop.

The leaves (quantisers, BitLinear, Q6_K, RMSNorm, RoPE, softmax, KV
quantiser) are pinned in test_oracle.py.  Here the oracle's model is checked
against the reference's own known answers (attention at position 0 returns V
of each query head's kv head, src/model/attention.rs:397-414; the zero-weight
closed form and the EOS / position / rollback rules of
tests/synthetic_model.rs:378-550 and src/model/cached_forward.rs:256-259) and
against tests/np_bitnet.py, an independent float64 restatement of the
forward.  Each comparison with np_bitnet also runs with one planted
composition mistake (wrong kv-head map, attn_sub_norm skipped, O residual
dropped, adjacent RoPE pairs, ReLU instead of ReLU^2, no RoPE on K) and
requires that mistake to miss the tolerance by a wide margin, so the
tolerance is known to be tight enough to catch it.
"""
import numpy as np
import pytest

import bitnet_synth as bs
import np_bitnet as nb
import oracle.oracle as orc
import willamette_hip as wh
from oracle.oracle_model import OracleModel

f32 = np.float32

GQA4 = bs.BitNetConfig(n_layers=3, n_embd=256, n_ff=384, n_heads=8, n_kv_heads=2, head_dim=32,
                       vocab=300, context_length=64)
MHA1 = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=512, n_heads=4, n_kv_heads=1, head_dim=64,
                       vocab=257, context_length=64)

MISTAKES = {
    "kv_head_mod": nb.Mistakes(kv_head_of="mod"),
    "no_attn_sub_norm": nb.Mistakes(sub_norm=False),
    "no_o_residual": nb.Mistakes(o_residual=False),
    "adjacent_rope_pairs": nb.Mistakes(rope_pairs="adjacent"),
    "relu_not_squared": nb.Mistakes(relu_square=False),
    "no_rope_on_k": nb.Mistakes(rope_on_k=False),
}


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def test_sdpa_position_zero_returns_v_per_kv_head():
    """src/model/attention.rs:397-414: 4 query heads, 2 kv heads, head_dim 2;
    one position, so every softmax is [1.0] and head h returns V of kv head
    h // 2 exactly."""
    q = np.ones(8, np.float32)
    k = np.full(4, 0.1, np.float32)
    v = np.array([5.0, 6.0, 70.0, 80.0], np.float32)
    out = orc.sdpa(q, k, v, n_heads=4, n_kv_heads=2, head_dim=2)
    assert out.tolist() == [5.0, 6.0, 5.0, 6.0, 70.0, 80.0, 70.0, 80.0]


def np_attention(q, K, V, n_heads, n_kv_heads, hd, head_of=lambda h, g, nkv: h // g):
    g = n_heads // n_kv_heads
    K = K.astype(np.float64).reshape(-1, n_kv_heads, hd)
    V = V.astype(np.float64).reshape(-1, n_kv_heads, hd)
    out = np.empty((n_heads, hd))
    for h in range(n_heads):
        kvh = head_of(h, g, n_kv_heads)
        s = K[:, kvh, :] @ q.astype(np.float64).reshape(n_heads, hd)[h] / np.sqrt(hd)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ V[:, kvh, :]
    return out.reshape(-1)


@pytest.mark.parametrize("n_heads,n_kv,hd,n_past", [(8, 2, 16, 37), (20, 5, 128, 300), (4, 4, 32, 1)])
def test_sdpa_matches_float64_attention(n_heads, n_kv, hd, n_past):
    rng = np.random.default_rng(n_heads * 100 + n_past)
    q = rng.standard_normal(n_heads * hd).astype(np.float32) * np.float32(2.0)
    K = rng.standard_normal((n_past, n_kv * hd)).astype(np.float32)
    V = rng.standard_normal((n_past, n_kv * hd)).astype(np.float32)
    got = orc.sdpa(q, K, V, n_heads, n_kv, hd).astype(np.float64)
    ref = np_attention(q, K, V, n_heads, n_kv, hd)
    tol = 1e-5 * np.abs(ref).max()
    assert np.abs(got - ref).max() <= tol
    if n_kv > 1 and n_heads > n_kv:  # the mapping h % n_kv would not pass
        wrong = np_attention(q, K, V, n_heads, n_kv, hd, head_of=lambda h, g, nkv: h % nkv)
        assert np.abs(got - wrong).max() > 1000 * tol


def test_sdpa_peaked_softmax_and_zero_query():
    """A zero query gives equal weights (the mean of V); a dominant score
    gives that position's V."""
    rng = np.random.default_rng(3)
    V = rng.standard_normal((10, 8)).astype(np.float32)
    K = rng.standard_normal((10, 8)).astype(np.float32)
    out = orc.sdpa(np.zeros(8, np.float32), K, V, 1, 1, 8)
    assert np.allclose(out, V.astype(np.float64).mean(axis=0), atol=1e-6)
    K2 = np.zeros((10, 8), np.float32)
    K2[6] = 1000.0
    out = orc.sdpa(np.ones(8, np.float32), K2, V, 1, 1, 8)
    assert np.array_equal(out, V[6])


# ---------------------------------------------------------------------------
# layer composition against the float64 restatement
# ---------------------------------------------------------------------------

def teacher_forced_deviation(hm, mistakes, n_pre, tokens):
    """Runs the oracle, then every layer of np_bitnet on the oracle's input
    hidden and cache rows.  Returns (largest relative deviation of a layer's
    output or the final hidden, largest distance in codes between np_bitnet's
    new K/V before quantisation and the oracle's new cache row)."""
    cfg = hm.cfg
    orm = OracleModel(hm)
    okv = orm.kv(cfg.context_length)
    if n_pre:
        k, v = bs.kv_prefill(cfg, seed=17, n_pos=n_pre)
        okv.append_positions(k, v)
    npm = nb.NpModel(hm, mistakes)
    dev, kv_codes = 0.0, 0.0
    for i, tok in enumerate(tokens):
        pos = n_pre + i
        rh, rtr = okv.forward(tok, pos, trace=True)
        x = npm.embed(tok)
        for l in range(cfg.n_layers):
            kk, ks, vv, vs = okv.read_raw(l, pos + 1)
            K = kk.astype(np.float64) * ks[:, None]
            V = vv.astype(np.float64) * vs[:, None]
            npm.k[l], npm.v[l] = list(K[:pos]), list(V[:pos])
            xo, kn, vn = npm.layer(l, x, pos, kv_row=(K[pos], V[pos]))
            dev = max(dev, np.abs(xo - rtr[l]).max() / np.abs(rtr[l]).max())
            kv_codes = max(kv_codes, np.abs(kn - K[pos]).max() / ks[pos],
                           np.abs(vn - V[pos]).max() / vs[pos])
            x = rtr[l].astype(np.float64)
        dev = max(dev, np.abs(npm.output(x) - rh).max() / np.abs(rh).max())
    orm.close()
    return dev, kv_codes


LAYER_TOL = 1e-5     # relative max-abs deviation of a layer's output
KV_CODE_TOL = 0.501  # a value rounds to its nearest code: at most half a step away


@pytest.mark.parametrize("cfg,n_pre", [(GQA4, 12), (MHA1, 5)], ids=["gqa4_prefill12", "mha1_prefill5"])
def test_layer_composition_matches_float64_model(cfg, n_pre):
    hm = bs.make_host_model(cfg, seed=4242)
    dev, kv_codes = teacher_forced_deviation(hm, None, n_pre, [5, 77, 123, 9, 250, 1])
    assert dev <= LAYER_TOL, f"oracle layer output off the float64 model by {dev:.3g}"
    assert kv_codes <= KV_CODE_TOL, f"new K/V row {kv_codes:.3f} codes from the float64 model"


@pytest.mark.parametrize("name", list(MISTAKES))
def test_planted_composition_mistake_is_caught(name):
    hm = bs.make_host_model(GQA4, seed=4242)
    dev, kv_codes = teacher_forced_deviation(hm, MISTAKES[name], 12, [5, 77, 123])
    assert dev > 1000 * LAYER_TOL or kv_codes > 10 * KV_CODE_TOL, name


def test_forward_from_empty_cache_matches_float64_model():
    """Free-running (no teacher forcing) from an empty cache: every layer's
    hidden and the final hidden agree with the float64 model."""
    hm = bs.make_host_model(GQA4, seed=4242)
    orm = OracleModel(hm)
    okv = orm.kv(GQA4.context_length)
    npm = nb.NpModel(hm)
    for pos, tok in enumerate([5, 77, 123, 9, 250, 1]):
        rh, rtr = okv.forward(tok, pos, trace=True)
        h, tr = npm.forward(tok, pos)
        for l in range(GQA4.n_layers):
            assert np.abs(tr[l] - rtr[l]).max() <= LAYER_TOL * np.abs(rtr[l]).max(), (pos, l)
        assert np.abs(h - rh).max() <= LAYER_TOL * np.abs(rh).max()
    orm.close()


def test_logits_match_float64_lm_head():
    hm = bs.make_host_model(GQA4, seed=4242)
    orm = OracleModel(hm)
    okv = orm.kv(GQA4.context_length)
    h = okv.forward(11, 0)
    logits, nxt = okv.logits_argmax(h)
    ref = nb.NpModel(hm).logits(h.astype(np.float64))
    assert np.abs(logits - ref).max() <= 1e-5 * np.abs(ref).max()
    top2 = np.sort(ref)[-2:]
    assert top2[1] - top2[0] > 1e-3 * np.abs(ref).max() and nxt == int(np.argmax(ref))
    orm.close()


# ---------------------------------------------------------------------------
# generation loop, positions, EOS, rollback
# ---------------------------------------------------------------------------

def test_greedy_equals_forward_logits_argmax_loop():
    """or_greedy_generate is the loop of generate.rs:111-189: prefill the
    prompt, then logits -> argmax -> forward on the new token."""
    hm = bs.make_host_model(GQA4, seed=99)
    orm = OracleModel(hm)
    a, b = orm.kv(GQA4.context_length), orm.kv(GQA4.context_length)
    ids = a.greedy([3, 1, 4], max_new=10)
    pos = 0
    for t in [3, 1, 4]:
        h = b.forward(t, pos)
        pos += 1
    loop = []
    for _ in range(10):
        _, nxt = b.logits_argmax(h)
        loop.append(nxt)
        h = b.forward(nxt, pos)
        pos += 1
    assert ids == loop and len(ids) == 10
    assert a.position == 3 + 9  # the last id is returned, not fed back
    orm.close()


def test_greedy_eos_rules():
    """tests/synthetic_model.rs:530-550: an EOS first token yields nothing; an
    EOS later truncates the ids before it."""
    hm = bs.make_host_model(GQA4, seed=99)
    orm = OracleModel(hm)
    ids = orm.kv(64).greedy([3, 1, 4], max_new=10)
    assert orm.kv(64).greedy([3, 1, 4], max_new=10, eos=ids[0]) == []
    k = next(i for i in range(1, 10) if ids[i] not in ids[:i])
    assert orm.kv(64).greedy([3, 1, 4], max_new=10, eos=ids[k]) == ids[:k]
    orm.close()


def test_positions_and_rollback():
    """tests/synthetic_model.rs:393-411 (two positions advance the cache to 2),
    cached_forward.rs:271-305 (tokens in order), :256-259 and :511-521
    (a non-finite hidden rolls the cache back)."""
    hm = bs.make_host_model(GQA4, seed=5)
    orm = OracleModel(hm)
    kv = orm.kv(8)
    h0 = kv.forward(0, 0)
    h1 = kv.forward(1, 1)
    assert kv.position == 2 and np.all(np.isfinite(h0)) and np.all(np.isfinite(h1))
    with pytest.raises(RuntimeError):
        kv.forward(1, 5)
    with pytest.raises(RuntimeError):
        kv.forward(GQA4.vocab, 2)
    assert kv.position == 2
    orm.close()
    hm.layers[1].norms["ffn_sub_norm"][:] = np.inf
    bad = OracleModel(hm)
    bkv = bad.kv(8)
    with pytest.raises(RuntimeError):
        bkv.forward(0, 0)
    assert bkv.position == 0
    bad.close()


def test_zero_weight_model_closed_form():
    """tests/synthetic_model.rs:378-391 with values: all-zero ternary weights
    and unit norms make every BitLinear output exactly 0, so the hidden stays
    the all-ones embedding row and output_norm gives 1/sqrt(1 + eps); every
    logit is then equal and the argmax is token 0."""
    cfg = GQA4
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
    orm = OracleModel(hm)
    kv = orm.kv(8)
    expect = f32(1.0) * (f32(1.0) / np.sqrt(f32(1.0) + f32(1e-5)))
    for pos in range(3):
        h, tr = kv.forward(3, pos, trace=True)
        assert np.all(tr == 1.0) and np.all(h == expect)
    logits, nxt = kv.logits_argmax(h)
    assert np.all(logits == logits[0]) and nxt == 0
    orm.close()


# ---------------------------------------------------------------------------
# forward_single_token_position_zero (no cache, f32 K/V at position 0)
# ---------------------------------------------------------------------------

def position_zero_deviation(hm, mistakes, tokens, quantised_v=False):
    """The oracle's no-cache position-0 forward against np_bitnet's
    layer_position_zero, teacher-forced layer by layer; with quantised_v the
    float64 side runs the cached layer instead (K/V through the int8 round
    trip), the mistake of treating position zero like a cached step."""
    cfg = hm.cfg
    orm = OracleModel(hm)
    npm = nb.NpModel(hm, mistakes)
    dev = 0.0
    for tok in tokens:
        rh, rtr = orm.forward_position_zero(tok, trace=True)
        x = npm.embed(tok)
        for l in range(cfg.n_layers):
            if quantised_v:
                npm.k[l], npm.v[l] = [], []
                xo, _, _ = npm.layer(l, x, 0)
            else:
                xo = npm.layer_position_zero(l, x)
            dev = max(dev, np.abs(xo - rtr[l]).max() / np.abs(rtr[l]).max())
            x = rtr[l].astype(np.float64)
        dev = max(dev, np.abs(npm.output(x) - rh).max() / np.abs(rh).max())
    orm.close()
    return dev


def test_position_zero_matches_float64_model():
    hm = bs.make_host_model(GQA4, seed=808)
    assert position_zero_deviation(hm, None, [5, 77, 299]) <= LAYER_TOL


@pytest.mark.parametrize("name", ["kv_head_mod", "no_attn_sub_norm", "no_o_residual", "relu_not_squared"])
def test_position_zero_planted_mistake_is_caught(name):
    hm = bs.make_host_model(GQA4, seed=808)
    assert position_zero_deviation(hm, MISTAKES[name], [5, 77]) > 1000 * LAYER_TOL, name


def test_position_zero_is_not_the_cached_step():
    """The no-cache path attends to the f32 K/V it just computed; the cached
    step at position 0 attends to their int8 round trip.  Comparing the
    oracle's position-zero forward with the cached layer misses the
    tolerance by far, so the comparison above would catch an oracle that
    quantised V here."""
    hm = bs.make_host_model(GQA4, seed=808)
    assert position_zero_deviation(hm, None, [5, 77], quantised_v=True) > 100 * LAYER_TOL


def test_position_zero_zero_weights_agree_with_cache():
    """tests/synthetic_model.rs:497-523: with all-zero ternary weights both
    paths compute the same hidden (every BitLinear returns exact 0)."""
    hm = bs.make_host_model(GQA4, seed=6)
    for hl in hm.layers:
        for r in bs.ROLES:
            hl.packed[r][:] = 0x55
    orm = OracleModel(hm)
    h0 = orm.forward_position_zero(3)
    h1 = orm.kv(8).forward(3, 0)
    assert np.array_equal(h0, h1) and np.all(np.isfinite(h0))
    orm.close()


def test_position_zero_nonfinite_fails():
    """forward.rs:47-55: a non-finite hidden after a layer fails the call."""
    hm = bs.make_host_model(GQA4, seed=5)
    hm.layers[1].norms["ffn_sub_norm"][:] = np.inf
    orm = OracleModel(hm)
    with pytest.raises(RuntimeError):
        orm.forward_position_zero(1)
    orm.close()


# ---------------------------------------------------------------------------
# the FFN block on its own (ffn_block_forward, src/model/ffn.rs:73-136)
# ---------------------------------------------------------------------------

FFN_MISTAKES = {
    "relu_not_squared": nb.Mistakes(relu_square=False),
    "no_ffn_sub_norm": nb.Mistakes(ffn_sub_norm=False),
    "gate_up_swapped": nb.Mistakes(gate_up_swapped=True),
}


def ffn_inputs(E, F, seed):
    """The FFN block's own inputs: I2_S gate/up [E -> F] and down [F -> E]
    with uniform ternary codes, per-tensor scales ~U(0.5, 2), norm weights
    ~U(0.9, 1.1), x ~N(0, 1) fed straight into ffn_norm."""
    g, u, d = wh.synth_i2s(seed, 1, E, F), wh.synth_i2s(seed, 2, E, F), wh.synth_i2s(seed, 3, F, E)
    sc = wh.synth_uniform(seed, 4, 3, 0.5, 2.0)
    nw, sw = wh.synth_uniform(seed, 5, E, 0.9, 1.1), wh.synth_uniform(seed, 6, F, 0.9, 1.1)
    return g, u, d, sc, nw, sw, wh.synth_normal(seed, 7, E)


def ffn_twin(E, F, g, u, d, sc, nw, sw, x, mk=None):
    return nb.ffn_block(nb.unpack_ternary(g, E, F), float(sc[0]), nb.unpack_ternary(u, E, F),
                        float(sc[1]), nb.unpack_ternary(d, F, E), float(sc[2]),
                        nw.astype(np.float64), sw.astype(np.float64), 1e-5, x.astype(np.float64), mk)


@pytest.mark.parametrize("E,F", [(2560, 6912), (256, 384)], ids=["bitnet2b", "small"])
def test_ffn_block_matches_float64_twin_and_catches_mistakes(E, F):
    g, u, d, sc, nw, sw, x = ffn_inputs(E, F, bs.master_seed(3) + E)
    y = orc.ffn_block(x, nw, g, sc[0], u, sc[1], d, sc[2], sw, F)
    r = ffn_twin(E, F, g, u, d, sc, nw, sw, x)
    assert np.abs(y - r).max() <= LAYER_TOL * np.abs(r).max()
    for name, mk in FFN_MISTAKES.items():
        bad = ffn_twin(E, F, g, u, d, sc, nw, sw, x, mk)
        assert np.abs(bad - r).max() > 1000 * LAYER_TOL * np.abs(r).max(), name


def test_ffn_block_zero_input_and_determinism():
    """tests/ffn.rs: zero input gives exactly zero output (RMSNorm of zeros is
    zeros, every quantiser sees absmax 0), and two calls agree bit for bit."""
    E, F = 2560, 6912
    g, u, d, sc, nw, sw, x = ffn_inputs(E, F, 11)
    z = orc.ffn_block(np.zeros(E, np.float32), nw, g, sc[0], u, sc[1], d, sc[2], sw, F)
    assert np.array_equal(z.view(np.uint32), np.zeros(E, np.uint32))
    a = orc.ffn_block(x, nw, g, sc[0], u, sc[1], d, sc[2], sw, F)
    b = orc.ffn_block(x, nw, g, sc[0], u, sc[1], d, sc[2], sw, F)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)) and np.all(np.isfinite(a))
    assert np.count_nonzero(a) > E // 2


def test_ffn_block_is_the_models_ffn():
    """The model's layer runs the same block: a one-layer model whose
    attention weights are all zero (codes 01) adds nothing before the FFN, so
    its hidden after the layer is embedding + ffn_block(embedding)."""
    cfg = bs.BitNetConfig(n_layers=1, n_embd=256, n_ff=384, n_heads=2, n_kv_heads=1, head_dim=128,
                          vocab=50, context_length=8)
    hm = bs.make_host_model(cfg, seed=77)
    L = hm.layers[0]
    for r in ("attn_q", "attn_k", "attn_v", "attn_output"):
        L.packed[r][:] = 0x55
    orm = OracleModel(hm)
    okv = orm.kv(cfg.context_length)
    _, tr = okv.forward(7, 0, trace=True)
    x = nb.q6k_dequant(hm.token_embd.reshape(cfg.vocab, -1)[7], cfg.n_embd)[0].astype(np.float32)
    y = orc.ffn_block(x, L.norms["ffn_norm"], L.packed["ffn_gate"], L.scales["ffn_gate"],
                      L.packed["ffn_up"], L.scales["ffn_up"], L.packed["ffn_down"],
                      L.scales["ffn_down"], L.norms["ffn_sub_norm"], cfg.n_ff, cfg.rms_eps)
    # hidden += O (all zeros: turns a -0 of the embedding into +0), then += down
    h = (x + np.zeros_like(x)) + y
    assert np.array_equal(h.view(np.uint32), tr[0].view(np.uint32))
    orm.close()
