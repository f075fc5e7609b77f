"""GPU test of the continuous-batching driver (wm_server_*).

Bar: every request's ids equal those of generate_with_cache_and_sampler run
on its own (wm_generate_with_sampler; wm_greedy_generate for greedy
parameters) with the same prompt, parameters and seed, while requests are
queued, admitted, prefilled in chunks and decoded together; the budget and
prompt checks of the reference reject bad requests.
"""
import numpy as np
import pytest

import bitnet_synth as bs
import willamette_hip as wh

pytestmark = pytest.mark.gpu

CFG = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=384, n_heads=4, n_kv_heads=2, head_dim=64,
                      vocab=600, context_length=256)
SP = wh.SamplingParams.make


@pytest.fixture(scope="module")
def model(ctx):
    hm = bs.make_host_model(CFG, seed=0x5E7)
    dev = bs.load_device_model(ctx, hm)
    yield dev
    dev.close()


REQUESTS = [
    ([11, 250, 3, 499, 42], 12, dict(temperature=0.8, top_k=50, top_p=0.9, repetition_penalty=1.1), 1, -1, ()),
    (list(range(1, 60)), 9, dict(temperature=0.0), 2, -1, ()),
    ([7], 20, dict(temperature=1.2), 3, -1, (5, 9)),
    ([300, 301, 302] * 10, 5, dict(temperature=0.7, top_p=0.5), 4, -1, ()),
    ([1, 2, 3], 0, dict(temperature=1.0), 5, -1, ()),
    (list(range(100, 180)), 15, dict(temperature=0.0), 6, 17, ()),
    ([599, 0, 599], 1, dict(temperature=0.9, top_k=3), 7, -1, ()),
]


def solo(ctx, model, prompt, max_new, kw, seed, eos, stops):
    kv = model.kv_cache(CFG.context_length)
    s = wh.Sampler(ctx, SP(**kw), seed)
    ids = kv.generate_sampled(prompt, max_new, s, eos=eos, stop_ids=stops)
    if kw == dict(temperature=0.0):
        g = model.kv_cache(CFG.context_length)
        assert g.greedy(prompt, max_new, eos=eos) == ids
        g.close()
    kv.close()
    s.close()
    return ids


@pytest.mark.parametrize("max_seqs,step_tokens", [(3, 16), (8, 512), (1, 1)])
def test_server_matches_solo_generation(ctx, model, max_seqs, step_tokens):
    print(f"server max_seqs={max_seqs} step_tokens={step_tokens}", flush=True)
    want = [solo(ctx, model, *r) for r in REQUESTS]
    srv = bs.Server(model, max_seqs=max_seqs, max_seq_len=CFG.context_length, step_tokens=step_tokens)
    ids = [srv.submit(p, mn, SP(**kw), seed, eos=eos, stop_ids=st)
           for p, mn, kw, seed, eos, st in REQUESTS]
    steps = 0
    while srv.step():
        steps += 1
        assert steps < 5000
    for rid, w in zip(ids, want):
        got, fin = srv.result(rid)
        assert fin and got == w, f"request {rid}"
    # a request submitted after the others finished reuses a pooled cache
    rid = srv.submit(*REQUESTS[0][:2], SP(**REQUESTS[0][2]), REQUESTS[0][3])
    while srv.step():
        pass
    assert srv.result(rid) == (want[0], True)
    for rid in ids:
        srv.release(rid)
    srv.close()


def test_server_rejects_and_releases(ctx, model):
    srv = bs.Server(model, max_seqs=2, max_seq_len=64, step_tokens=8)
    with pytest.raises(wh.WillametteError):
        srv.submit([], 3, SP(temperature=1.0), 1)
    with pytest.raises(wh.WillametteError):
        srv.submit([CFG.vocab], 3, SP(temperature=1.0), 1)
    with pytest.raises(wh.WillametteError):
        srv.submit(list(range(60)), 6, SP(temperature=1.0), 1)  # 60 + 5 > 64
    a = srv.submit(list(range(60)), 5, SP(temperature=1.0), 1)    # 60 + 4 = 64 fits
    b = srv.submit([4, 5, 6], 30, SP(temperature=0.0), 2)
    srv.step()
    srv.release(b)  # cancel while active
    while srv.step():
        pass
    got, fin = srv.result(a)
    assert fin and len(got) <= 5
    with pytest.raises(wh.WillametteError):
        srv.result(b)
    with pytest.raises(wh.WillametteError):
        bs.Server(model, max_seqs=4, max_seq_len=64, step_tokens=2)
    with pytest.raises(wh.WillametteError):
        bs.Server(model, max_seqs=1, max_seq_len=CFG.context_length + 1, step_tokens=8)
    srv.close()
