"""CPU tests that pin the oracle (oracle/wm_oracle.c) to the reference.

Each check is either one of the reference's own known-answer tests (cited
file:line in project-willamette), a brute-force restatement computed a
different way (numpy int64 / float64), or a closed form chosen so that a
plausible mistake (wrong code map, dropped term, wrong pairing, wrong
reduction order) fails it.
"""
import math

import numpy as np
import pytest

import oracle.oracle as orc

f32 = np.float32


def scale_block(s):
    b = np.zeros(32, np.uint8)
    b[:4] = np.frombuffer(np.float32(s).tobytes(), np.uint8)
    return b


# ---------------------------------------------------------------------------
# independent numpy restatements used as brute-force cross-checks
# ---------------------------------------------------------------------------

def np_unpack_ternary(packed, in_dim, out_dim):
    """I2_S bytes -> int8 ternary matrix [out_dim, in_dim] (docs/BITLINEAR_I2S_MATVEC.md §3)."""
    b = packed[: in_dim // 4 * out_dim].reshape(out_dim, in_dim // 128, 32)
    codes = np.stack([(b >> 6) & 3, (b >> 4) & 3, (b >> 2) & 3, b & 3], axis=2)  # [o, blk, 4, 32]
    lut = np.array([-1, 0, 1, 0], np.int8)
    return lut[codes].reshape(out_dim, in_dim)


def np_quantize(x):
    x = x.astype(np.float32)
    a = np.abs(x)
    a = np.where(np.isnan(a), 0, a)
    m = f32(a.max()) if a.size else f32(0)
    if m == 0:
        return np.zeros(x.size, np.int8), f32(1.0)
    inv = f32(127.0) / m
    v = (x * inv).astype(np.float64)
    r = np.sign(v) * np.floor(np.abs(v) + 0.5)
    r = np.clip(r, -127, 127)
    r = np.where(np.isnan(r), 0, r)
    return r.astype(np.int8), f32(m / f32(127.0))


def np_q6k_dequant(row, n):
    blk = row.reshape(n // 256, 210)
    out = np.empty((n // 256, 256), np.float64)
    d = blk[:, 208].astype(np.uint16) | (blk[:, 209].astype(np.uint16) << 8)
    dval = d.view(np.float16).astype(np.float64)
    for h in range(2):
        ql = blk[:, h * 64:(h + 1) * 64].astype(np.int32)
        qh = blk[:, 128 + h * 32:128 + (h + 1) * 32].astype(np.int32)
        sc = blk[:, 192 + h * 8:192 + (h + 1) * 8].view(np.int8).astype(np.float64)
        for l in range(32):
            q = [(ql[:, l] & 15) | ((qh[:, l] & 3) << 4),
                 (ql[:, l + 32] & 15) | (((qh[:, l] >> 2) & 3) << 4),
                 (ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4),
                 (ql[:, l + 32] >> 4) | (((qh[:, l] >> 6) & 3) << 4)]
            for k in range(4):
                out[:, h * 128 + l + 32 * k] = dval * sc[:, l // 16 + 2 * k] * (q[k] - 32)
    return out.reshape(-1)


# ---------------------------------------------------------------------------
# BitLinear I2_S
# ---------------------------------------------------------------------------

def test_ternary_code_table():  # src/model/bitlinear.rs:334-340
    assert [orc.lib.or_ternary_from_code(c) for c in range(4)] == [-1, 0, 1, 0]


def test_matvec_all_plus_one():  # bitlinear.rs:343-360
    x = (np.arange(128) * 0.1).astype(np.float32)
    y = orc.bitlinear_scalar(np.full(32, 0xAA, np.uint8), 1.0, 128, 1, x)
    assert abs(y[0] - x.sum()) < 1e-4


def test_matvec_all_minus_one():  # bitlinear.rs:363-380
    x = (np.arange(128) * 0.1).astype(np.float32)
    y = orc.bitlinear_scalar(np.zeros(32, np.uint8), 1.0, 128, 1, x)
    assert abs(y[0] + x.sum()) < 1e-4


@pytest.mark.parametrize("path", ["scalar", "i8"])
def test_matvec_all_zero_weights_exact(path):  # bitlinear.rs:383-397
    x = (1.0 + np.arange(128) * 0.01).astype(np.float32)
    w = np.full(32, 0x55, np.uint8)
    y = orc.bitlinear_scalar(w, 1.0, 128, 1, x) if path == "scalar" else orc.bitlinear_i8(w, 1.0, 128, 1, x)[0]
    assert y[0] == 0.0


@pytest.mark.parametrize("path", ["scalar", "i8"])
def test_matvec_scale_applied_at_end(path):  # bitlinear.rs:400-411: 3.5 * 128 * 2 = 896
    x = np.full(128, 2.0, np.float32)
    w = np.full(32, 0xAA, np.uint8)
    y = orc.bitlinear_scalar(w, 3.5, 128, 1, x) if path == "scalar" else orc.bitlinear_i8(w, 3.5, 128, 1, x)[0]
    assert abs(y[0] - 896.0) < 1e-3


def test_matvec_two_rows():  # bitlinear.rs:414-428
    w = np.concatenate([np.full(32, 0xAA, np.uint8), np.zeros(32, np.uint8)])
    y = orc.bitlinear_scalar(w, 1.0, 128, 2, np.ones(128, np.float32))
    assert abs(y[0] - 128) < 1e-4 and abs(y[1] + 128) < 1e-4


def test_matvec_column_stride_32_mapping():  # bitlinear.rs:431-465 -> 991
    w = np.full(32, 0x55, np.uint8)
    w[0] = 0x86
    x = np.zeros(128, np.float32)
    x[[0, 32, 64, 96]] = [1.0, 10.0, 100.0, 1000.0]
    assert abs(orc.bitlinear_scalar(w, 1.0, 128, 1, x)[0] - 991.0) < 1e-4


def test_unpack_row_positions():  # bitlinear.rs:527-548
    w = np.full(32, 0x55, np.uint8)
    w[0] = 0x86
    row = orc.unpack_row(w, 128, 1, 0)
    assert (row[0], row[32], row[64], row[96]) == (1, -1, 0, 1)
    assert all(row[i] == 0 for i in [1, 31, 33, 63, 65, 95, 97, 127])


@pytest.mark.parametrize("in_dim,out_dim,n", [(64, 1, 64), (128, 1, 64), (128, 2, 128)])
def test_matvec_rejects(in_dim, out_dim, n):  # bitlinear.rs:467-512
    w = np.full(32, 0xAA, np.uint8)
    with pytest.raises(ValueError):
        if in_dim == 64:
            orc.bitlinear_i8(w, 1.0, in_dim, out_dim, np.zeros(n, np.float32))
        else:
            orc.bitlinear_scalar(w, 1.0, in_dim, out_dim, np.zeros(n, np.float32))


def test_zero_input_gives_exact_zero():  # tests/bitlinear_sse2_i8.rs:150-161
    rng = np.random.default_rng(1)
    w = rng.integers(0, 256, 640 * 64, dtype=np.uint8)
    y, act, s, acc = orc.bitlinear_i8(w, 1.3, 2560, 64, np.zeros(2560, np.float32))
    assert np.all(y == 0) and np.all(act == 0) and s == 1.0 and np.all(acc == 0)


def test_quantize_extremes_map_to_127():
    x = np.array([0.5, -3.0, 3.0, 0.0, 1.5], np.float32)
    q, s = orc.quantize_input_absmax_i8(x)
    assert q[1] == -127 and q[2] == 127 and q[3] == 0
    assert s == f32(3.0) / f32(127.0)


def test_quantize_matches_numpy_restatement():
    rng = np.random.default_rng(2)
    for n in (128, 2560, 6912):
        x = rng.standard_normal(n).astype(np.float32) * rng.uniform(0.01, 100)
        # values that land exactly on .5 after scaling exercise half-away-from-zero
        x[:8] = np.array([0.5, -0.5, 1.5, -2.5, 2.5, 126.5, -126.5, 127], np.float32) * (f32(np.abs(x).max()) / f32(127))
        q, s = orc.quantize_input_absmax_i8(x)
        q2, s2 = np_quantize(x)
        assert s == s2
        assert np.array_equal(q, q2)


def test_quantize_nan_ignored_and_zeroed():
    x = np.array([1.0, np.nan, -2.0, 0.25], np.float32)
    q, s = orc.quantize_input_absmax_i8(x)
    assert s == f32(2.0) / f32(127.0) and q[1] == 0 and q[2] == -127


@pytest.mark.parametrize("in_dim,out_dim", [(128, 3), (256, 17), (2560, 64), (6912, 8)])
def test_i8_matvec_bruteforce_int64(in_dim, out_dim):
    """a1+a3+a4: the i32 dot is an integer sum, so int64 brute force fixes it."""
    rng = np.random.default_rng(in_dim + out_dim)
    w = rng.integers(0, 256, in_dim // 4 * out_dim, dtype=np.uint8)  # includes code 11
    x = rng.standard_normal(in_dim).astype(np.float32)
    y, act, s, acc = orc.bitlinear_i8(w, 0.75, in_dim, out_dim, x)
    q, s2 = np_quantize(x)
    assert s == s2 and np.array_equal(act, q)
    t = np_unpack_ternary(w, in_dim, out_dim).astype(np.int64)
    dot = t @ q.astype(np.int64)
    assert np.array_equal(acc.astype(np.int64), dot)
    assert np.array_equal(y, f32(f32(0.75) * s) * dot.astype(np.float32))


def test_i8_vs_scalar_f32_tolerance():  # tests/bitlinear_sse2_i8.rs:31-36, :100-112
    rng = np.random.default_rng(3)
    w = rng.integers(0, 3, 2560 * 2560).astype(np.uint8)
    packed = ((w[0::4] << 6) | (w[1::4] << 4) | (w[2::4] << 2) | w[3::4]).astype(np.uint8)
    x = rng.standard_normal(2560).astype(np.float32)
    yi = orc.bitlinear_i8(packed, 1.0, 2560, 2560, x)[0]
    ys = orc.bitlinear_scalar(packed, 1.0, 2560, 2560, x)
    cos = float(yi @ ys / (np.linalg.norm(yi) * np.linalg.norm(ys)))
    assert cos > 0.999
    assert np.abs(yi - ys).max() / np.abs(ys).max() <= 0.05


def test_i2s_scale_block():  # src/gguf/tensor.rs:564-581, :612-638
    s = f32()
    import ctypes as C
    out = C.c_float()
    b = scale_block(1.5)
    assert orc.lib.or_i2s_scale(orc.P(b, C.c_uint8), 32, C.byref(out)) == 0 and out.value == 1.5
    for bad in (np.nan, np.inf, -np.inf):
        b = scale_block(bad)
        assert orc.lib.or_i2s_scale(orc.P(b, C.c_uint8), 32, C.byref(out)) != 0


# ---------------------------------------------------------------------------
# f16 / Q6_K
# ---------------------------------------------------------------------------

def test_f16_known_values():  # src/model/primitives.rs:460-483
    f = orc.lib.or_f16_to_f32
    assert f(0x0000) == 0.0 and math.copysign(1, f(0x8000)) < 0
    assert (f(0x3C00), f(0xBC00), f(0x4000), f(0x3800)) == (1.0, -1.0, 2.0, 0.5)
    assert math.isinf(f(0x7C00)) and f(0x7C00) > 0 and math.isinf(f(0xFC00)) and f(0xFC00) < 0
    assert math.isnan(f(0x7E00))
    assert f(0x0001) == 2.0 ** -24


def test_f16_all_bit_patterns_match_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.lib.or_f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    r = ref[::7]
    same = (got.view(np.uint32) == r.view(np.uint32)) | (np.isnan(got) & np.isnan(r))
    assert same.all()


def ones_block(scale=1):
    return np.concatenate([np.full(128, 0x11, np.uint8), np.full(64, 0xAA, np.uint8),
                           np.full(16, scale, np.uint8), np.array([0x00, 0x3C], np.uint8)])


def test_q6k_ones_block():  # src/model/q6_k.rs:253-257
    assert np.all(orc.q6k_dequantize_row(ones_block(), 256) == 1.0)


def test_q6k_pinned_mapping():  # src/model/q6_k.rs:260-280
    b = np.zeros(210, np.uint8)
    b[0], b[32], b[128] = 0xF0, 0xE1, 0xE4
    b[192:208] = np.arange(1, 17, dtype=np.uint8)
    b[200] = np.uint8(np.int8(-2).view(np.uint8))
    b[64], b[160] = 0x0F, 0x03
    b[208:210] = [0x00, 0x3C]
    out = orc.q6k_dequantize_row(b, 256)
    assert (out[0], out[32], out[64], out[96], out[128]) == (-32.0, -45.0, 75.0, 210.0, -62.0)


def test_q6k_constant_rows_matvec():  # src/model/linear.rs:406-421 -> [256, 512]
    t = np.concatenate([ones_block(1), ones_block(2)])
    ones = np.ones(256, np.float32)
    assert orc.q6k_dot_sse2(t[:210], ones) == 256.0 and orc.q6k_dot_sse2(t[210:], ones) == 512.0
    assert list(orc.compute_logits(t, 256, 2, ones)) == [256.0, 512.0]


def test_q6k_direct_dot_equals_dequantized_dot():  # src/model/q6_k.rs:283-292
    x = (np.arange(256) / 32.0 - 4.0).astype(np.float32)
    deq = orc.q6k_dequantize_row(ones_block(), 256)
    expected = f32(0)
    for a, b in zip(deq, x):
        expected = f32(expected + f32(a * b))
    assert orc.q6k_dot_scalar(ones_block(), x) == expected
    assert abs(orc.q6k_dot_sse2(ones_block(), x) - expected) < 1e-3


def test_q6k_dequant_matches_numpy_restatement():
    rng = np.random.default_rng(4)
    row = rng.integers(0, 256, 210 * 10, dtype=np.uint8)
    for b in range(10):  # finite d
        row[b * 210 + 209] &= 0x3B
    got = orc.q6k_dequantize_row(row, 2560)
    ref = np_q6k_dequant(row, 2560)
    assert np.array_equal(got.astype(np.float64), ref)  # (d*sc)*q is exact in f32


def test_q6k_sse2_vs_scalar_and_float64():  # src/model/q6_k.rs:296-324 tolerance
    rng = np.random.default_rng(5)
    for _ in range(20):
        row = rng.integers(0, 256, 210 * 10, dtype=np.uint8)
        for b in range(10):
            row[b * 210 + 209] &= 0x1F  # |d| < 2^-3
        x = rng.standard_normal(2560).astype(np.float32)
        w = np_q6k_dequant(row, 2560)
        tol = 1e-5 * max(float(np.abs(w * x).sum()), 1.0)
        s, c = orc.q6k_dot_sse2(row, x), orc.q6k_dot_scalar(row, x)
        assert abs(s - c) <= tol and abs(float(s) - float(w @ x.astype(np.float64))) <= tol


def test_q6k_sse2_accumulation_order_closed_form():
    """All weights 1, x[0] = 2^24, other x = 1: the 16-partial SSE2 order gives
    lane (k=0,l=0) = 2^24 (each +1 absorbed), 15 lanes of 160, then
    ((2^24+160)+320 + 640) + (640+640) = 16779616 -- not the sequential
    16777216 nor the exact 16779775."""
    row = ones_block()  # d=1, sc=1, q=1
    x = np.ones(256 * 10, np.float32)
    row10 = np.tile(row, 10)
    x[0] = 2.0 ** 24
    assert orc.q6k_dot_sse2(row10, x) == 16779616.0
    assert orc.q6k_dot_scalar(row10, x) == 16777216.0


def test_argmax():  # src/model/lm_head.rs:221-226
    assert orc.argmax(np.array([0.1, 0.5, 0.3], np.float32)) == 1
    assert orc.argmax(np.array([], np.float32)) is None
    assert orc.argmax(np.array([0.5], np.float32)) == 0
    assert orc.argmax(np.array([1.0, 1.0], np.float32)) == 0
    assert orc.argmax(np.array([np.nan, 5.0], np.float32)) == 0
    assert orc.argmax(np.array([1.0, np.nan, 2.0], np.float32)) == 2


# ---------------------------------------------------------------------------
# f32 primitives
# ---------------------------------------------------------------------------

def test_rms_norm_known_value():  # src/model/primitives.rs:486-503
    x = np.array([1, 2, 3, 4], np.float32)
    out = orc.rms_norm(x, np.ones(4, np.float32), 1e-5)
    assert np.all(np.abs(out - x / np.sqrt(f32(7.5) + f32(1e-5))) < 1e-6)


def test_rms_norm_float64_and_sequential_order():
    rng = np.random.default_rng(6)
    x = rng.standard_normal(6912).astype(np.float32) * 30
    w = rng.uniform(0.9, 1.1, 6912).astype(np.float32)
    got = orc.rms_norm(x, w, 1e-5).astype(np.float64)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd @ xd) / 6912 + 1e-5) * w
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    # order: x^2 = [2^24, 1, 1, ...] sums to exactly 2^24 left to right
    x = np.ones(4096, np.float32)
    x[0] = 4096.0
    out = orc.rms_norm(x, np.ones(4096, np.float32), 0.0)
    rs = f32(1.0) / np.sqrt(f32(2.0 ** 24) / f32(4096))
    assert out[1] == f32(1.0) * rs


def test_rope_neox_pairing_and_values():  # primitives.rs:514-565
    x = orc.rope_neox(np.array([0.1, 0.2, 0.3, 0.4], np.float32), 4, 4, 0, 10000.0)
    assert np.allclose(x, [0.1, 0.2, 0.3, 0.4], atol=1e-6)
    x = orc.rope_neox(np.array([1.0, 0, 0, 0], np.float32), 4, 4, 1, 10000.0)
    # NEOX pairs (0, 2): sin lands at index 2 (Norm would put it at index 1)
    assert abs(x[0] - math.cos(1.0)) < 1e-6 and abs(x[2] - math.sin(1.0)) < 1e-6 and x[1] == 0
    rng = np.random.default_rng(7)
    v = rng.standard_normal(128).astype(np.float32)
    out = orc.rope_neox(v, 128, 128, 77, 500000.0)
    j = np.arange(64)
    th = 77 * 500000.0 ** (-2.0 * j / 128)
    a, b = v[:64].astype(np.float64), v[64:].astype(np.float64)
    assert np.allclose(out[:64], a * np.cos(th) - b * np.sin(th), atol=1e-4)
    assert np.allclose(out[64:], a * np.sin(th) + b * np.cos(th), atol=1e-4)
    assert np.allclose(out[:64] ** 2 + out[64:] ** 2, a ** 2 + b ** 2, rtol=1e-5)


def test_softmax():  # src/model/attention.rs:322-366
    assert list(orc.softmax([1.25])) == [1.0]
    assert np.allclose(orc.softmax([0, 0, 0, 0]), 0.25, atol=1e-6)
    s = orc.softmax([-np.inf, 0.0])
    assert s[0] == 0.0 and abs(s[1] - 1) < 1e-6
    s = orc.softmax([1, 2, 3, 4, 5])
    assert abs(s.sum() - 1) < 1e-6 and np.all(np.diff(s) > 0)
    assert np.all(orc.softmax([-np.inf] * 4) == 0)


def test_kv_quantise():  # src/model/kv_cache.rs:291-317
    k = np.array([0.1, -0.2, 0.3, -0.4], np.float32)
    q, s = orc.kv_quantise(k)
    assert np.all(np.abs(q.astype(np.float32) * s - k) <= 0.4 / 200)
    q, s = orc.kv_quantise(np.zeros(4, np.float32))
    assert s == 0.0 and np.all(q == 0)
    q, s = orc.kv_quantise(np.array([1.0, np.nan, -2.0], np.float32))
    assert s == f32(2.0) / f32(127.0) and q[1] == 0
    q, s = orc.kv_quantise(np.array([1.0, np.inf], np.float32))
    assert s == 0.0 and np.all(q == 0)


def test_relu_square_mul():  # src/model/ffn.rs:143-155
    g = np.array([-2, -0.5, 0, 0.5, 2, 3, -np.inf, np.inf], np.float32)
    out = np.empty(8, np.float32)
    orc.lib.or_relu_square_mul(orc.P(g, orc.C.c_float), orc.P(np.ones(8, np.float32), orc.C.c_float),
                               8, orc.P(out, orc.C.c_float))
    assert list(out[:6]) == [0, 0, 0, 0.25, 4, 9] and out[6] == 0 and np.isinf(out[7])
