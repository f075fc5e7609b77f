"""GPU parity of the device sampler, the batched prefill and the sampled
generation loop against the oracle.

Bar: every sampled id and the xorshift64 state after each draw identical to
the oracle's Sampler::sample restatement (src/model/sampler.rs:133-196) on
the same logits, parameters and history, over repetition penalty,
temperature, top-k, top-p, their edge values and 128256-entry logits; the
same error kinds (multinomial error, NaN under top-p) with the state
untouched; the batched prefill bit-identical to token-by-token decode
(hidden and raw cache bytes); generate_with_cache_and_sampler's ids equal to
the oracle composition of forward, logits and sampler.
"""
import numpy as np
import pytest

import bitnet_synth as bs
import oracle.oracle as orc
import willamette_hip as wh
from oracle.oracle_model import OracleModel

pytestmark = pytest.mark.gpu

NAN = float("nan")


def pair_samplers(ctx, seed, **kw):
    return (wh.Sampler(ctx, wh.SamplingParams.make(**kw), seed),
            orc.Sampler(orc.SamplingParams.make(**kw), seed))


PARAMS = [
    dict(temperature=1.0),
    dict(temperature=0.7),
    dict(temperature=1.3, top_k=40),
    dict(temperature=0.8, top_k=1),
    dict(temperature=1.0, top_p=0.9),
    dict(temperature=0.6, top_p=0.5),
    dict(temperature=1.0, top_k=1000, top_p=0.95),
    dict(temperature=0.9, top_p=0.0),
    dict(temperature=1.0, top_p=1.0),
    dict(temperature=1.0, top_p=NAN),
    dict(temperature=1.1, repetition_penalty=1.3),
    dict(temperature=0.7, top_k=50, top_p=0.9, repetition_penalty=1.1),
    dict(temperature=0.0, top_k=20),           # temperature skipped, not greedy
    dict(temperature=0.0),                     # greedy
    dict(temperature=0.0, repetition_penalty=0.5),
]


@pytest.mark.parametrize("n", [7, 1000, 128256])
@pytest.mark.parametrize("pi", range(len(PARAMS)))
def test_sample_matches_oracle(ctx, n, pi):
    kw = PARAMS[pi]
    print(f"sampler n={n} params={kw}", flush=True)
    rng = np.random.default_rng(1000 * pi + n)
    dev, ref = pair_samplers(ctx, 1234 + pi, **kw)
    for tok in rng.integers(0, n, 30):
        dev.observe(int(tok))
        ref.observe(int(tok))
    for step in range(6 if n == 128256 else 12):
        logits = (rng.standard_normal(n) * rng.uniform(0.5, 4)).astype(np.float32)
        got, want = dev.sample(logits), ref.sample(logits)
        assert got == want, f"step {step}"
        assert dev.checkpoint()[0] == ref.state.value
        dev.observe(got)
        ref.observe(want)


def test_sample_dev_logits_and_ties(ctx):
    """Logits on the device; equal probabilities at the top-p cut (lowest
    indices kept) and at the top-k threshold (all kept)."""
    n = 4096
    logits = np.zeros(n, np.float32)
    logits[::3] = 2.0
    for kw in (dict(temperature=1.0, top_p=0.3), dict(temperature=1.0, top_k=5),
               dict(temperature=1.0, top_k=5, top_p=0.5)):
        dev, ref = pair_samplers(ctx, 77, **kw)
        buf = ctx.to_device(logits)
        for _ in range(20):
            assert dev.sample_dev(buf, n) == ref.sample(logits)
        buf.free()


@pytest.mark.parametrize("case", ["all_neg_inf", "top_k_zero", "nan_plain", "nan_top_p",
                                  "nan_top_p_one_hot", "nan_top_k", "nan_top_k_all", "inf",
                                  "tiny_temperature", "empty"])
def test_sample_errors_match(ctx, case):
    logits = np.array([0.5, -1.0, 2.0, 0.25], np.float32)
    kw = dict(temperature=1.0)
    if case == "all_neg_inf":
        logits[:] = -np.inf
    elif case == "top_k_zero":
        kw["top_k"] = 0
    elif case == "nan_plain":
        logits[1] = np.nan
    elif case == "nan_top_p":
        logits[1] = np.nan
        kw["top_p"] = 0.5
    elif case == "nan_top_k":  # top-k sorts: a NaN leaves its k-th largest open
        logits[1] = np.nan
        kw["top_k"] = 2
    elif case == "nan_top_k_all":  # k >= n sorts nothing: the NaN reaches the multinomial
        logits[1] = np.nan
        kw["top_k"] = 4
    elif case == "nan_top_p_one_hot":
        logits[:] = -np.inf
        kw["top_p"] = 0.0
    elif case == "inf":
        logits[2] = np.inf
    elif case == "tiny_temperature":
        kw["temperature"] = 1e-30
    elif case == "empty":
        logits = logits[:0]
    dev, ref = pair_samplers(ctx, 5, **kw)
    st0 = dev.checkpoint()[0]
    try:
        want = ref.sample(logits)
    except ValueError as e:
        want = e
    if isinstance(want, int):
        assert dev.sample(logits) == want
        assert dev.checkpoint()[0] == ref.state.value
        return
    with pytest.raises(wh.WillametteError) as ei:
        dev.sample(logits)
    if "rc=-3" in str(want):
        assert ei.value.kind == "NonFinite"
    else:
        assert ei.value.kind == "GgufParse" and "multinomial" in str(ei.value)
    assert dev.checkpoint()[0] == st0 == ref.state.value


def test_greedy_sampler_is_argmax(ctx):
    dev = wh.Sampler(ctx, wh.SamplingParams.make(), 0xABAD1DEA)
    assert dev.sample([0.1, 0.5, 0.3, 0.9]) == 3
    assert dev.sample([np.nan, 5.0]) == 0
    assert dev.sample([1.0, np.nan, 3.0, 3.0]) == 2
    with pytest.raises(wh.WillametteError):
        dev.sample(np.zeros(0, np.float32))


def test_rollback_restores_history_and_rng(ctx):  # sampler.rs:348-372 on the device
    kw = dict(temperature=1.0, repetition_penalty=1.1)
    logits = np.full(16, 0.1, np.float32)
    s = wh.Sampler(ctx, wh.SamplingParams.make(**kw), 12345)
    s.observe(2)
    cp = s.checkpoint()
    s.observe(s.sample(logits))
    s.rollback(cp)
    clean = wh.Sampler(ctx, wh.SamplingParams.make(**kw), 12345)
    clean.observe(2)
    assert s.sample(logits) == clean.sample(logits)


# ---- batched prefill and the sampled loop --------------------------------

LONG = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=384, n_heads=4, n_kv_heads=2, head_dim=64,
                       vocab=600, context_length=1100)


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.fixture(scope="module")
def long_pair(ctx):
    hm = bs.make_host_model(LONG, seed=0x5A11)
    dev = bs.load_device_model(ctx, hm)
    orm = OracleModel(hm)
    yield hm, dev, orm
    dev.close()
    orm.close()


def test_prefill_matches_token_by_token(long_pair):
    """600 tokens after a 40-position prefill: two batched chunks (512 + 88)
    give the same last hidden and cache bytes as 600 decode steps."""
    hm, dev, orm = long_pair
    rng = np.random.default_rng(8)
    k, v = bs.kv_prefill(LONG, seed=9, n_pos=40)
    toks = rng.integers(0, LONG.vocab, 600).tolist()
    a, b = dev.kv_cache(LONG.context_length), dev.kv_cache(LONG.context_length)
    a.append_positions(k, v)
    b.append_positions(k, v)
    ha = a.prefill(toks)
    for i, t in enumerate(toks):
        hb = b.forward(t, 40 + i)
    assert a.position == b.position == 640
    assert bits_equal(ha, hb)
    for l in range(LONG.n_layers):
        ra, rb = a.read_raw(l, 640), b.read_raw(l, 640)
        assert all(np.array_equal(x, y) for x, y in zip(ra, rb))
    # and the oracle agrees on the last hidden
    okv = orm.kv(LONG.context_length)
    okv.append_positions(k, v)
    for i, t in enumerate(toks[:-1]):
        okv.forward(t, 40 + i)
    assert bits_equal(okv.forward(toks[-1], 639), ha)
    a.close()
    b.close()


@pytest.mark.parametrize("kw,eos,stops", [
    (dict(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.1), -1, ()),
    (dict(temperature=1.2), -1, (3, 5)),
    (dict(temperature=0.0), 7, ()),
])
def test_generate_with_sampler_matches_oracle(long_pair, ctx, kw, eos, stops):
    """generate_with_cache_and_sampler (generate.rs:195-277): the oracle
    composition (forward, logits, Sampler::sample, observe) gives the same
    ids; greedy parameters give the greedy loop's ids."""
    hm, dev, orm = long_pair
    prompt = [11, 250, 3, 499, 42]
    max_new = 16
    dkv = dev.kv_cache(LONG.context_length)
    ds = wh.Sampler(ctx, wh.SamplingParams.make(**kw), 99)
    got = dkv.generate_sampled(prompt, max_new, ds, eos=eos, stop_ids=stops)
    # the oracle's loop
    okv = orm.kv(LONG.context_length)
    rs = orc.Sampler(orc.SamplingParams.make(**kw), 99)
    for t in prompt:
        rs.observe(t)
    for i, t in enumerate(prompt):
        h = okv.forward(t, i)
    want, pos = [], len(prompt)
    for step in range(max_new):
        logits, _ = okv.logits_argmax(h)
        nxt = rs.sample(logits)
        if nxt == eos or nxt in stops:
            break
        want.append(nxt)
        rs.observe(nxt)
        if step + 1 < max_new:
            h = okv.forward(nxt, pos)
            pos += 1
    assert got == want
    assert ds.checkpoint() == (rs.state.value, len(rs.history))
    assert dkv.position == okv.position
    if kw == dict(temperature=0.0):
        gkv = dev.kv_cache(LONG.context_length)
        assert gkv.greedy(prompt, max_new, eos=eos) == got
        gkv.close()
    dkv.close()
