"""GPU parity: the FFN block on its own (ffn_block_forward,
src/model/ffn.rs:73-136) vs the oracle, on the block's own inputs.

The BitNet-2B FFN shape: x ~ N(0, 1) fed straight into ffn_norm (2560, eps
1e-5, weight ~U(0.9, 1.1)), gate and up I2_S 6912x2560, relu(gate)^2 * up,
ffn_sub_norm (6912), down I2_S 2560x6912, uniform ternary weights with
per-tensor scales ~U(0.5, 2).  Bar: the f32 output bit-identical to the
oracle's (the norms' sums in the reference's order, the BitLinears exact).
"""
import numpy as np
import pytest

import bitnet_synth as bs
import oracle.oracle as orc
import willamette_hip as wh

pytestmark = pytest.mark.gpu


def ffn_inputs(E, F, seed):
    g, u, d = wh.synth_i2s(seed, 1, E, F), wh.synth_i2s(seed, 2, E, F), wh.synth_i2s(seed, 3, F, E)
    sc = wh.synth_uniform(seed, 4, 3, 0.5, 2.0)
    nw, sw = wh.synth_uniform(seed, 5, E, 0.9, 1.1), wh.synth_uniform(seed, 6, F, 0.9, 1.1)
    return g, u, d, sc, nw, sw, wh.synth_normal(seed, 7, E)


def upload(ctx, E, F, g, u, d, sc):
    return (ctx.upload_i2s(g, float(sc[0]), E, F), ctx.upload_i2s(u, float(sc[1]), E, F),
            ctx.upload_i2s(d, float(sc[2]), F, E))


def same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("E,F,seed", [(2560, 6912, 0), (2560, 6912, 1), (2560, 6912, 2),
                                      (256, 384, 0), (128, 1024, 0), (1024, 128, 0)])
def test_ffn_block_bit_exact(ctx, E, F, seed):
    s = bs.master_seed(3) + seed
    g, u, d, sc, nw, sw, x = ffn_inputs(E, F, s)
    print(f"ffn block {E}x{F} seed {seed}", flush=True)
    tg, tu, td = upload(ctx, E, F, g, u, d, sc)
    y = wh.ffn_block_forward(ctx, x, nw, tg, tu, td, sw)
    ry = orc.ffn_block(x, nw, g, sc[0], u, sc[1], d, sc[2], sw, F)
    assert same_bits(y, ry)
    # scaled inputs: the same block on 1000 * x and on 1e-3 * x
    for f in (1000.0, 1e-3):
        xs = (x * np.float32(f)).astype(np.float32)
        assert same_bits(wh.ffn_block_forward(ctx, xs, nw, tg, tu, td, sw),
                         orc.ffn_block(xs, nw, g, sc[0], u, sc[1], d, sc[2], sw, F))


def test_ffn_block_edges(ctx):
    """tests/ffn.rs: zero input -> exactly zero output; a single non-zero
    input; the reference's length checks, in its order (ffn.rs:87-114)."""
    E, F = 2560, 6912
    g, u, d, sc, nw, sw, x = ffn_inputs(E, F, 5)
    tg, tu, td = upload(ctx, E, F, g, u, d, sc)
    z = wh.ffn_block_forward(ctx, np.zeros(E, np.float32), nw, tg, tu, td, sw)
    assert np.array_equal(z.view(np.uint32), np.zeros(E, np.uint32))
    one = np.zeros(E, np.float32)
    one[1234] = -3.5
    assert same_bits(wh.ffn_block_forward(ctx, one, nw, tg, tu, td, sw),
                     orc.ffn_block(one, nw, g, sc[0], u, sc[1], d, sc[2], sw, F))
    for bad in (dict(x=np.zeros(E - 1, np.float32)), dict(nw=nw[:-1]), dict(sw=sw[1:])):
        with pytest.raises(wh.WillametteError) as e:
            wh.ffn_block_forward(ctx, bad.get("x", x), bad.get("nw", nw), tg, tu, td, bad.get("sw", sw))
        assert e.value.kind == "Shape"
    with pytest.raises(wh.WillametteError) as e:  # down of the wrong shape
        wh.ffn_block_forward(ctx, x, nw, tg, tu, tg, sw)
    assert e.value.kind == "Shape"


def test_ffn_block_dev_equals_host_form(ctx):
    E, F = 2560, 6912
    g, u, d, sc, nw, sw, x = ffn_inputs(E, F, 9)
    tg, tu, td = upload(ctx, E, F, g, u, d, sc)
    bx, bn, bsw, bo = ctx.to_device(x), ctx.to_device(nw), ctx.to_device(sw), ctx.alloc(E * 4)
    for _ in range(2):
        ctx.check(wh.lib.wm_ffn_block_forward_dev(ctx.h, bx.ptr, bn.ptr, tg.h, tu.h, td.h, bsw.ptr,
                                                  1e-5, bo.ptr))
        assert same_bits(bo.to_host(np.float32), wh.ffn_block_forward(ctx, x, nw, tg, tu, td, sw))
    for b in (bx, bn, bsw, bo):
        b.free()
