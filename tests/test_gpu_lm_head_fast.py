"""GPU parity: the id-only lm-head (bounded fixed-point pass + exact rescoring).

Bar: the returned id is the oracle's argmax (first index of the maximum,
NaN rules) on every input, exactly.  That rests on one property, checked
directly on every row: the bounded pass's value lies within its bound of the
oracle's SSE2-order f32 logit, |approx - logit| <= bound.  When more than
one row's bounds reach the largest lower bound, those rows are recomputed in
the exact order; when a single row's do, it is the argmax as it stands.
"""
import numpy as np
import pytest

import oracle.oracle as orc
import willamette_hip as wh

pytestmark = pytest.mark.gpu

BITNET_SEED = 0x5749_4C4C_0000_0002


def random_q6k(rng, n_rows, n_embd, finite=True):
    t = rng.integers(0, 256, n_rows * (n_embd // 256) * 210, dtype=np.uint8).reshape(-1, 210)
    if finite:
        t[:, 209] &= 0x3B  # |d| < 2^15, finite
    return t.ravel()


def synth_rows(rng, n_rows, n_embd, d_sigma=1e-3):
    raw = wh.synth_q6k(int(rng.integers(1 << 62)), 1, n_rows, n_embd, d_sigma)
    return raw


def check_bound(ctx, t, raw, n_embd, n_rows, h):
    approx, bound = wh.q6k_bounded_logits(ctx, t, h)
    ref = orc.compute_logits(raw, n_embd, n_rows, h, threads=16)
    fin = np.isfinite(ref)
    err = np.abs(approx.astype(np.float64) - ref.astype(np.float64))
    ok = (err <= bound) | ~fin | ~np.isfinite(bound)
    assert ok.all(), f"bound violated on {np.count_nonzero(~ok)} rows, e.g. row {np.argmax(~ok)}"
    return approx, bound, ref


@pytest.fixture(scope="module")
def bitnet_lm_head(ctx):
    raw = wh.synth_q6k(BITNET_SEED, 1, 128256, 2560, 1e-3)
    return raw, ctx.upload_q6k(raw, 2560, 128256)


def test_bound_holds_full_size(ctx, bitnet_lm_head):
    """128256 x 2560 (BitNet-2B tied lm-head), hidden ~ N(0,1)."""
    raw, t = bitnet_lm_head
    h = wh.synth_normal(BITNET_SEED, 2, 2560)
    approx, bound, ref = check_bound(ctx, t, raw, 2560, 128256, h)
    # the bound is useful: far below the spread of the logits
    assert np.median(bound) < 0.02 * np.std(ref)
    _, a = wh.logits_argmax(ctx, t, h, want_logits=False)
    assert a == orc.argmax(ref)


@pytest.mark.parametrize("tag", [3, 4, 5, 6, 7])
def test_argmax_only_full_size_many_hidden(ctx, bitnet_lm_head, tag):
    raw, t = bitnet_lm_head
    h = wh.synth_normal(BITNET_SEED, tag, 2560, 0.3 * tag)
    ref = orc.compute_logits(raw, 2560, 128256, h, threads=16)
    _, a = wh.logits_argmax(ctx, t, h, want_logits=False)
    assert a == orc.argmax(ref)


@pytest.mark.parametrize("n_rows,n_embd", [(1, 256), (2, 256), (3, 512), (5, 768), (7, 1024),
                                           (333, 1280), (1000, 2048), (4099, 4096), (600, 8192)])
def test_bound_and_argmax_shapes(ctx, n_rows, n_embd):
    rng = np.random.default_rng(n_rows * 7 + n_embd)
    raw = random_q6k(rng, n_rows, n_embd)
    h = rng.standard_normal(n_embd).astype(np.float32)
    t = ctx.upload_q6k(raw, n_embd, n_rows)
    _, _, ref = check_bound(ctx, t, raw, n_embd, n_rows, h)
    _, a = wh.logits_argmax(ctx, t, h, want_logits=False)
    assert a == orc.argmax(ref)


def test_ties_and_near_ties_resolved_exactly(ctx):
    """Duplicate rows (equal logits: the first index wins) and rows one quant
    apart (logits closer than the bound: only the exact order decides)."""
    rng = np.random.default_rng(11)
    n_rows, n_embd = 2000, 2560
    raw = wh.synth_q6k(77, 1, n_rows, n_embd, 1e-3).reshape(n_rows, -1)
    h = rng.standard_normal(n_embd).astype(np.float32)
    ref = orc.compute_logits(raw.ravel(), n_embd, n_rows, h)
    top = int(orc.argmax(ref))
    # copies of the best row after it (ties -> first index) and a one-quant
    # variant before it
    for dst in (top + 1, n_rows - 1):
        if dst < n_rows:
            raw[dst] = raw[top]
    if top > 0:
        v = raw[top].copy()
        v[5] ^= 0x01  # one low-nibble bit of one quant
        raw[top - 1] = v
    raw = raw.ravel()
    ref = orc.compute_logits(raw, n_embd, n_rows, h)
    t = ctx.upload_q6k(raw, n_embd, n_rows)
    _, a = wh.logits_argmax(ctx, t, h, want_logits=False)
    assert a == orc.argmax(ref)
    # all rows identical: every row ties, index 0
    same = np.tile(raw.reshape(n_rows, -1)[top], 64)
    t2 = ctx.upload_q6k(same, n_embd, 64)
    _, a2 = wh.logits_argmax(ctx, t2, h, want_logits=False)
    assert a2 == 0


@pytest.mark.parametrize("kind", ["zeros", "nan", "inf", "huge", "tiny", "one_hot", "row_copy"])
def test_special_hidden_vectors(ctx, kind):
    rng = np.random.default_rng(5)
    n_rows, n_embd = 3001, 2560
    raw = random_q6k(rng, n_rows, n_embd)
    h = rng.standard_normal(n_embd).astype(np.float32)
    if kind == "zeros":
        h[:] = 0
    elif kind == "nan":
        h[17] = np.nan
    elif kind == "inf":
        h[1000] = np.inf
    elif kind == "huge":
        h *= np.float32(1e30)
    elif kind == "tiny":
        h *= np.float32(1e-38)
    elif kind == "one_hot":
        h[:] = 0
        h[123] = 1
    elif kind == "row_copy":  # hidden = a row's own values: that row's logit stands out
        h = orc.q6k_dequantize_row(raw[2 * 10 * 210:3 * 10 * 210], n_embd)
    t = ctx.upload_q6k(raw, n_embd, n_rows)
    with np.errstate(all="ignore"):
        ref = orc.compute_logits(raw, n_embd, n_rows, h)
    _, a = wh.logits_argmax(ctx, t, h, want_logits=False)
    assert a == orc.argmax(ref)


def test_nonfinite_scales_id_only(ctx):
    rng = np.random.default_rng(9)
    raw = random_q6k(rng, 64, 512).reshape(-1, 210)
    raw[3, 208:210] = [0x00, 0x7C]   # d = +inf: that row's logit is +-inf or NaN
    raw[10, 208:210] = [0x00, 0xFC]  # d = -inf
    raw[17, 208:210] = [0x01, 0x7E]  # d = NaN
    raw = raw.ravel()
    h = rng.standard_normal(512).astype(np.float32)
    t = ctx.upload_q6k(raw, 512, 64)
    ref = orc.compute_logits(raw, 512, 64, h)
    _, a = wh.logits_argmax(ctx, t, h, want_logits=False)
    assert a == orc.argmax(ref)
    # NaN in row 0 wins, as in the reference's scan
    raw2 = raw.reshape(-1, 210).copy()
    raw2[0, 208:210] = [0x01, 0x7E]
    t2 = ctx.upload_q6k(raw2.ravel(), 512, 64)
    _, a2 = wh.logits_argmax(ctx, t2, h, want_logits=False)
    assert a2 == 0


def test_subnormal_scales(ctx):
    """Every block's d an f16 subnormal: the bounded pass must convert them
    exactly (a flushed d would drop whole rows and break the bound)."""
    rng = np.random.default_rng(21)
    n_rows, n_embd = 512, 2560
    raw = random_q6k(rng, n_rows, n_embd).reshape(-1, 210)
    raw[:, 209] &= 0x83  # exponent bits 0 -> subnormal (or zero)
    raw = raw.ravel()
    h = rng.standard_normal(n_embd).astype(np.float32)
    t = ctx.upload_q6k(raw, n_embd, n_rows)
    approx, bound, ref = check_bound(ctx, t, raw, n_embd, n_rows, h)
    assert np.count_nonzero(ref) > n_rows // 2
    _, a = wh.logits_argmax(ctx, t, h, want_logits=False)
    assert a == orc.argmax(ref)
