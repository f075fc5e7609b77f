"""GPU parity: BitLinear I2_S matvec (gfx950) vs the oracle's SSE2-i8 path.

Bar: int8 activations, activation scale, i32 accumulators and f32 outputs
bit-identical to the oracle on the same inputs.
"""
import numpy as np
import pytest

import oracle.oracle as orc
import willamette_hip as wh

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def run_both(ctx, packed, scale, in_dim, out_dim, x):
    w = ctx.upload_i2s(packed, scale, in_dim, out_dim)
    y, act, s, acc = wh.bitlinear_i2s_matvec_f32(ctx, w, x, debug=True)
    ry, ract, rs, racc = orc.bitlinear_i8(packed, np.float32(scale), in_dim, out_dim, x)
    return (y, act, s, acc), (ry, ract, rs, racc)


def assert_parity(got, ref):
    (y, act, s, acc), (ry, ract, rs, racc) = got, ref
    assert np.array_equal(act, ract), "int8 activations differ"
    assert np.float32(s) == rs, "activation scale differs"
    assert np.array_equal(acc, racc), "i32 accumulators differ"
    assert same_bits(y, ry), "f32 outputs differ"


# 16384 is the widest input the one-launch matvec takes (256 chunks of 64
# columns); 16512 goes through the split quantise / dots / finalise path
SHAPES = [(128, 1), (128, 3), (256, 100), (640, 65), (2560, 2560), (2560, 640), (2560, 6912),
          (6912, 2560), (128, 64), (4096, 128), (16384, 100), (16512, 70)]


@pytest.mark.parametrize("in_dim,out_dim", SHAPES)
def test_matvec_random_bytes_bit_exact(ctx, in_dim, out_dim):
    rng = np.random.default_rng(in_dim * 7 + out_dim)
    packed = rng.integers(0, 256, in_dim // 4 * out_dim, dtype=np.uint8)  # includes code 11
    x = (rng.standard_normal(in_dim) * rng.uniform(0.1, 10)).astype(np.float32)
    assert_parity(*run_both(ctx, packed, 1.37, in_dim, out_dim, x))


def test_matvec_bitnet_attn_q_synth(ctx):
    """Config: 2560x2560 attn_q, ternary 1/3 each, scale ~U(0.5,2), x ~N(0,1)."""
    seed = 0x5749_4C4C_0000_0001
    packed = wh.synth_i2s(seed, 1, 2560, 2560)
    scale = float(wh.synth_uniform(seed, 2, 1, 0.5, 2.0)[0])
    x = wh.synth_normal(seed, 3, 2560)
    assert_parity(*run_both(ctx, packed, scale, 2560, 2560, x))


@pytest.mark.parametrize("kind", ["zeros", "all_plus", "all_minus", "all_zero_w", "one_hot",
                                  "nan", "inf", "tiny", "huge"])
def test_matvec_edge_inputs(ctx, kind):
    rng = np.random.default_rng(11)
    in_dim, out_dim = 256, 70
    packed = rng.integers(0, 256, in_dim // 4 * out_dim, dtype=np.uint8)
    x = rng.standard_normal(in_dim).astype(np.float32)
    if kind == "zeros":
        x[:] = 0
    elif kind == "all_plus":
        packed[:] = 0xAA
    elif kind == "all_minus":
        packed[:] = 0x00
    elif kind == "all_zero_w":
        packed[:] = 0x55
    elif kind == "one_hot":
        x[:] = 0
        x[37] = -3.5
    elif kind == "nan":
        x[5] = np.nan
    elif kind == "inf":
        x[9] = np.inf
    elif kind == "tiny":
        x *= np.float32(1e-40)  # subnormal activations
    elif kind == "huge":
        x *= np.float32(1e37)
    got, ref = run_both(ctx, packed, 0.9, in_dim, out_dim, x)
    (y, act, s, acc), (ry, ract, rs, racc) = got, ref
    assert np.array_equal(act, ract) and np.array_equal(acc, racc)
    assert np.array_equal(y.view(np.uint32), ry.view(np.uint32)) or (
        np.array_equal(np.isnan(y), np.isnan(ry)) and np.array_equal(y[~np.isnan(y)], ry[~np.isnan(ry)]))


def test_reference_kats_through_device(ctx):
    # all-zero weights -> exactly 0 (src/model/bitlinear.rs:383-397)
    w = ctx.upload_i2s(np.full(32, 0x55, np.uint8), 1.0, 128, 1)
    assert wh.bitlinear_i2s_matvec_f32(ctx, w, 1.0 + np.arange(128, dtype=np.float32) * 0.01)[0] == 0.0
    # all +1, x = 2, scale 3.5 -> 896 (bitlinear.rs:400-411)
    w = ctx.upload_i2s(np.full(32, 0xAA, np.uint8), 3.5, 128, 1)
    assert abs(wh.bitlinear_i2s_matvec_f32(ctx, w, np.full(128, 2.0, np.float32))[0] - 896.0) < 1e-3
    # two rows +-128 (bitlinear.rs:414-428)
    w = ctx.upload_i2s(np.concatenate([np.full(32, 0xAA, np.uint8), np.zeros(32, np.uint8)]), 1.0, 128, 2)
    y = wh.bitlinear_i2s_matvec_f32(ctx, w, np.ones(128, np.float32))
    assert abs(y[0] - 128) < 1e-3 and abs(y[1] + 128) < 1e-3


def test_rejects_like_reference(ctx):
    ok = np.full(32, 0xAA, np.uint8)
    with pytest.raises(wh.WillametteError) as e:
        ctx.upload_i2s(ok, 1.0, 64, 1)  # in_dim not a multiple of 128
    assert e.value.kind == "Shape"
    with pytest.raises(wh.WillametteError) as e:
        ctx.upload_i2s(ok, 1.0, 128, 2)  # packed too short
    assert e.value.kind == "Shape"
    for bad in (np.nan, np.inf):
        with pytest.raises(wh.WillametteError) as e:
            ctx.upload_i2s(ok, bad, 128, 1)
        assert e.value.kind == "NonFinite"
    w = ctx.upload_i2s(ok, 1.0, 128, 1)
    for n in (64, 129):
        with pytest.raises(wh.WillametteError) as e:
            wh.bitlinear_i2s_matvec_f32(ctx, w, np.zeros(n, np.float32))
        assert e.value.kind == "Shape"
    out = np.empty(2, np.float32)
    x = np.zeros(128, np.float32)
    st = wh.lib.wm_bitlinear_i2s_matvec_f32(ctx.h, w.h, wh._ptr(x, wh.C.c_float), 128,
                                             wh._ptr(out, wh.C.c_float), 2)
    assert st == 2
    q = ctx.upload_q6k(np.zeros(210, np.uint8), 256, 1)
    with pytest.raises(wh.WillametteError) as e:
        wh.bitlinear_i2s_matvec_f32(ctx, q, np.zeros(256, np.float32))
    assert e.value.kind == "UnsupportedTensorType"


def test_device_and_multi_entry_points_agree(ctx):
    rng = np.random.default_rng(5)
    in_dim, out_dim, n = 2560, 640, 11
    xs = rng.standard_normal(in_dim).astype(np.float32)
    ws, refs = [], []
    for i in range(n):
        p = rng.integers(0, 256, in_dim // 4 * out_dim, dtype=np.uint8)
        s = float(rng.uniform(0.5, 2))
        ws.append(ctx.upload_i2s(p, s, in_dim, out_dim))
        refs.append(orc.bitlinear_i8(p, np.float32(s), in_dim, out_dim, xs)[0])
    dx = ctx.to_device(xs)
    dy = ctx.alloc(n * out_dim * 4)
    arr = (wh._vp * n)(*[w.h.value for w in ws])
    ctx.check(wh.lib.wm_bitlinear_i2s_matvec_f32_multi_dev(ctx.h, arr, n, dx.ptr, dy.ptr))
    got = dy.to_host(np.float32).reshape(n, out_dim)
    for i in range(n):
        assert same_bits(got[i], refs[i])
    dy1 = ctx.alloc(out_dim * 4)
    ctx.check(wh.lib.wm_bitlinear_i2s_matvec_f32_dev(ctx.h, ws[3].h, dx.ptr, dy1.ptr))
    assert same_bits(dy1.to_host(np.float32), refs[3])


def test_multi_entry_point_many_copies(ctx):
    """More tensors than fit in one launch's argument block (64): the
    pointers go through a device table."""
    rng = np.random.default_rng(9)
    in_dim, out_dim, n = 512, 128, 150
    xs = rng.standard_normal(in_dim).astype(np.float32)
    ws, refs = [], []
    for i in range(n):
        p = rng.integers(0, 256, in_dim // 4 * out_dim, dtype=np.uint8)
        s = float(rng.uniform(0.5, 2))
        ws.append(ctx.upload_i2s(p, s, in_dim, out_dim))
        refs.append(orc.bitlinear_i8(p, np.float32(s), in_dim, out_dim, xs)[0])
    dx = ctx.to_device(xs)
    dy = ctx.alloc(n * out_dim * 4)
    arr = (wh._vp * n)(*[w.h.value for w in ws])
    ctx.check(wh.lib.wm_bitlinear_i2s_matvec_f32_multi_dev(ctx.h, arr, n, dx.ptr, dy.ptr))
    got = dy.to_host(np.float32).reshape(n, out_dim)
    for i in range(n):
        assert same_bits(got[i], refs[i]), f"copy {i}"


# ---- the scalar f32 path (src/model/bitlinear.rs:146-233) -----------------

def same_bits_nan(a, b):
    """Bit-identical except that any NaN matches any NaN: IEEE 754 leaves a
    NaN result's sign and payload open (x86 passes the operand's through,
    the GPU returns the canonical one), and the reference never inspects
    them."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return a.shape == b.shape and np.array_equal(na, nb) and \
        np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


SCALAR_SHAPES = [(128, 1), (128, 64), (256, 100), (1152, 65), (2560, 2560), (6912, 2560),
                 (4096, 128)]


@pytest.mark.parametrize("in_dim,out_dim", SCALAR_SHAPES)
def test_scalar_matvec_bit_exact(ctx, in_dim, out_dim):
    """f32 outputs bit-identical to the oracle's scalar restatement; random
    bytes include the degenerate code 11; 1152 columns leave a partial LDS
    round of x."""
    rng = np.random.default_rng(in_dim * 13 + out_dim)
    packed = rng.integers(0, 256, in_dim // 4 * out_dim, dtype=np.uint8)
    x = (rng.standard_normal(in_dim) * rng.uniform(0.1, 10)).astype(np.float32)
    scale = float(rng.uniform(0.5, 2))
    w = ctx.upload_i2s(packed, scale, in_dim, out_dim)
    y = wh.bitlinear_i2s_matvec_f32_scalar(ctx, w, x)
    ry = orc.bitlinear_scalar(packed, np.float32(scale), in_dim, out_dim, x)
    assert same_bits(y, ry)


@pytest.mark.parametrize("kind", ["kat_aa", "kat_00", "kat_55", "nan_skipped", "nan_used", "inf",
                                  "neg_zero", "huge"])
def test_scalar_matvec_edges(ctx, kind):
    """Reference KATs (0xAA -> scale * Σx, 0x00 -> -scale * Σx, 0x55 -> 0,
    bitlinear.rs:343-428) and non-finite inputs: a NaN under a 0 code is
    skipped, under a +-1 code it reaches the output; -0.0 inputs leave +0.0
    sums."""
    rng = np.random.default_rng(5)
    in_dim, out_dim = 256, 70
    x = rng.standard_normal(in_dim).astype(np.float32)
    packed = rng.integers(0, 256, in_dim // 4 * out_dim, dtype=np.uint8)
    if kind.startswith("kat"):
        packed[:] = {"kat_aa": 0xAA, "kat_00": 0x00, "kat_55": 0x55}[kind]
    elif kind == "nan_skipped":
        packed[:] = 0x55
        packed[1::7] = 0xAA
        x[0] = np.nan  # column 0: bits 7:6 of byte 0 of each row, code 01 unless byte 0 was set
    elif kind == "nan_used":
        x[37] = np.nan
    elif kind == "inf":
        x[3], x[200] = np.inf, -np.inf
    elif kind == "neg_zero":
        x[:] = -0.0
    elif kind == "huge":
        x *= np.float32(3e37)
    w = ctx.upload_i2s(packed, 1.5, in_dim, out_dim)
    y = wh.bitlinear_i2s_matvec_f32_scalar(ctx, w, x)
    ry = orc.bitlinear_scalar(packed, np.float32(1.5), in_dim, out_dim, x)
    assert same_bits_nan(y, ry)
    if kind in ("kat_aa", "kat_00"):
        # the block walk's column order: byte gp of block bk, then its four codes
        order = [128 * bk + gp + 32 * q for bk in range(in_dim // 128) for gp in range(32)
                 for q in range(4)]
        s = np.float32(0)
        for j in order:
            s = np.float32(s + x[j])
        want = np.float32(1.5) * (s if kind == "kat_aa" else np.float32(np.float32(0) - s))
        assert np.all(y == want)
    if kind in ("kat_55", "neg_zero"):
        assert np.all(y == 0) and not np.any(np.signbit(y))
    if kind == "nan_skipped":
        assert np.all(np.isfinite(y[(packed.reshape(out_dim, -1)[:, 0] >> 6) != 2]))


def test_scalar_matvec_rejects(ctx):
    """Length and type checks of bitlinear.rs:157-199, before any launch."""
    w = ctx.upload_i2s(np.zeros(256 // 4 * 8, np.uint8), 1.0, 256, 8)
    y = np.empty(8, np.float32)
    for xn, yn in ((255, 8), (256, 7)):
        x = np.zeros(xn, np.float32)
        yy = np.empty(yn, np.float32)
        with pytest.raises(wh.WillametteError) as ei:
            ctx.check(wh.lib.wm_bitlinear_i2s_matvec_f32_scalar(
                ctx.h, w.h, wh._ptr(x, wh.C.c_float), x.size, wh._ptr(yy, wh.C.c_float), yy.size))
        assert ei.value.kind == "Shape"
    q = ctx.upload_q6k(np.zeros(210, np.uint8), 256, 1)
    with pytest.raises(wh.WillametteError) as ei:
        wh.bitlinear_i2s_matvec_f32_scalar(ctx, q, np.zeros(256, np.float32))
    assert ei.value.kind == "UnsupportedTensorType"
