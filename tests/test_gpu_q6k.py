"""GPU parity: Q6_K dequantisation and the tied lm-head (logits + argmax).

Bar: dequantised values bit-identical (they are exact products); logits
bit-identical to the oracle's SSE2-order row dots (the device keeps the
reference's 16 partial sums per row); argmax equal, with the reference's
first-index / NaN rules.
"""
import numpy as np
import pytest

import oracle.oracle as orc
import willamette_hip as wh

pytestmark = pytest.mark.gpu


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return a.shape == b.shape and bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | nan))


def random_q6k(rng, n_rows, n_embd, finite=True):
    t = rng.integers(0, 256, n_rows * (n_embd // 256) * 210, dtype=np.uint8).reshape(-1, 210)
    if finite:
        t[:, 209] &= 0x3B  # |d| < 2^15, finite
    return t.ravel()


def ones_block(scale=1):
    return np.concatenate([np.full(128, 0x11, np.uint8), np.full(64, 0xAA, np.uint8),
                           np.full(16, scale, np.uint8), np.array([0x00, 0x3C], np.uint8)])


def test_dequant_kats(ctx):
    t = ctx.upload_q6k(ones_block(), 256, 1)  # src/model/q6_k.rs:253-257
    assert np.all(wh.q6k_dequantize_row(ctx, t, 0) == 1.0)
    b = np.zeros(210, np.uint8)  # src/model/q6_k.rs:260-280
    b[0], b[32], b[128] = 0xF0, 0xE1, 0xE4
    b[192:208] = np.arange(1, 17, dtype=np.uint8)
    b[200] = 0xFE
    b[64], b[160] = 0x0F, 0x03
    b[208:210] = [0x00, 0x3C]
    out = wh.q6k_dequantize_row(ctx, ctx.upload_q6k(b, 256, 1), 0)
    assert (out[0], out[32], out[64], out[96], out[128]) == (-32.0, -45.0, 75.0, 210.0, -62.0)


@pytest.mark.parametrize("n_rows,n_embd", [(5, 256), (37, 512), (1000, 2560)])
def test_dequant_rows_bit_exact(ctx, n_rows, n_embd):
    rng = np.random.default_rng(n_rows)
    raw = random_q6k(rng, n_rows, n_embd, finite=False)
    t = ctx.upload_q6k(raw, n_embd, n_rows)
    rb = n_embd // 256 * 210
    for r in sorted({0, 1, n_rows // 2, n_rows - 1}):
        assert bits_equal(wh.q6k_dequantize_row(ctx, t, r), orc.q6k_dequantize_row(raw[r * rb:(r + 1) * rb], n_embd))


def test_constant_rows_matvec(ctx):  # src/model/linear.rs:406-421
    t = ctx.upload_q6k(np.concatenate([ones_block(1), ones_block(2)]), 256, 2)
    logits, a = wh.logits_argmax(ctx, t, np.ones(256, np.float32))
    assert list(logits) == [256.0, 512.0] and a == 1


@pytest.mark.parametrize("n_rows,n_embd", [(1, 256), (7, 256), (333, 512), (4096, 2560)])
def test_logits_bit_exact_small(ctx, n_rows, n_embd):
    rng = np.random.default_rng(n_rows + n_embd)
    raw = random_q6k(rng, n_rows, n_embd)
    h = rng.standard_normal(n_embd).astype(np.float32)
    t = ctx.upload_q6k(raw, n_embd, n_rows)
    logits, a = wh.logits_argmax(ctx, t, h)
    ref = orc.compute_logits(raw, n_embd, n_rows, h, threads=8)
    assert bits_equal(logits, ref)
    assert a == orc.argmax(ref)


def test_lm_head_bitnet2b_full_size(ctx):
    """Config: Q6_K tied lm-head 128256 x 2560, d ~ |N(0,1e-3)|, h ~ N(0,1)."""
    seed = 0x5749_4C4C_0000_0002
    raw = wh.synth_q6k(seed, 1, 128256, 2560, 1e-3)
    h = wh.synth_normal(seed, 2, 2560)
    t = ctx.upload_q6k(raw, 2560, 128256)
    logits, a = wh.logits_argmax(ctx, t, h)
    ref = orc.compute_logits(raw, 2560, 128256, h, threads=16)
    assert bits_equal(logits, ref)
    assert a == orc.argmax(ref)
    _, a2 = wh.logits_argmax(ctx, t, h, want_logits=False)
    assert a2 == a


def test_argmax_rules_on_device(ctx):
    # every row identical -> ties -> index 0
    t = ctx.upload_q6k(np.tile(ones_block(), 9), 256, 9)
    _, a = wh.logits_argmax(ctx, t, np.ones(256, np.float32))
    assert a == 0
    # rows 3 and 6 share the maximum -> first (3)
    blocks = [ones_block(1)] * 9
    blocks[3] = ones_block(3)
    blocks[6] = ones_block(3)
    t = ctx.upload_q6k(np.concatenate(blocks), 256, 9)
    _, a = wh.logits_argmax(ctx, t, np.ones(256, np.float32))
    assert a == 3
    # a NaN logit at index 0 wins (the scan starts from logits[0]); elsewhere NaN never wins
    nan_row = ones_block(1).copy()
    nan_row[208:210] = [0x00, 0x7E]  # d = NaN
    t = ctx.upload_q6k(np.concatenate([nan_row] + [ones_block(2)] * 4), 256, 5)
    logits, a = wh.logits_argmax(ctx, t, np.ones(256, np.float32))
    assert np.isnan(logits[0]) and a == 0
    t = ctx.upload_q6k(np.concatenate([ones_block(1), nan_row, ones_block(2), nan_row]), 256, 4)
    logits, a = wh.logits_argmax(ctx, t, np.ones(256, np.float32))
    assert a == 2


def test_nonfinite_scale_blocks_match_oracle(ctx):
    rng = np.random.default_rng(9)
    raw = random_q6k(rng, 64, 512, finite=True).reshape(-1, 210)
    raw[3, 208:210] = [0x00, 0x7C]   # d = +inf
    raw[10, 208:210] = [0x00, 0xFC]  # d = -inf
    raw[17, 208:210] = [0x01, 0x7E]  # d = NaN
    raw = raw.ravel()
    h = rng.standard_normal(512).astype(np.float32)
    t = ctx.upload_q6k(raw, 512, 64)
    logits, _ = wh.logits_argmax(ctx, t, h)
    assert bits_equal(logits, orc.compute_logits(raw, 512, 64, h))


def test_q6k_rejects(ctx):
    with pytest.raises(wh.WillametteError) as e:
        ctx.upload_q6k(np.zeros(209, np.uint8), 256, 1)
    assert e.value.kind == "Shape"
    with pytest.raises(wh.WillametteError) as e:
        ctx.upload_q6k(np.zeros(210, np.uint8), 128, 1)
    assert e.value.kind == "Shape"
    t = ctx.upload_q6k(np.zeros(420, np.uint8), 256, 2)
    with pytest.raises(wh.WillametteError) as e:
        wh.q6k_dequantize_row(ctx, t, 2)
    assert e.value.kind == "Shape"
    with pytest.raises(wh.WillametteError):
        wh.logits_argmax(ctx, t, np.zeros(255, np.float32))
