"""GPU check of wm_bitlinear_i2s_matvec_f32_dev_noalloc, the allocation-free
form of wm_bitlinear_i2s_matvec_f32_dev: through the C ABI, two calls in a
row (the second on a smaller tensor, so it runs on what the first left in
the shared scratch array), each bit-identical to the allocating entry point
on the same inputs; and a shape above the scratch limit is rejected."""
import numpy as np
import pytest

import willamette_hip as wh

pytestmark = pytest.mark.gpu


def run_dev(ctx, fn, w, x_host, out_dim):
    x = ctx.to_device(np.ascontiguousarray(x_host, np.float32))
    y = ctx.alloc(out_dim * 4)
    ctx.check(fn(ctx.h, w.h, x.ptr, y.ptr))
    ctx.synchronize()
    out = y.to_host(np.float32, out_dim)
    x.free()
    y.free()
    return out


def test_noalloc_matvec_equals_dev_entry_point(ctx):
    rng = np.random.default_rng(2024)
    for in_dim, out_dim in ((2560, 6912), (256, 128)):  # the second call is smaller
        packed = rng.integers(0, 256, out_dim * in_dim // 4, dtype=np.uint8)
        scale = float(rng.uniform(0.5, 2.0))
        w = ctx.upload_i2s(packed, scale, in_dim, out_dim)
        x = rng.standard_normal(in_dim).astype(np.float32) * np.float32(rng.uniform(0.5, 20))
        got = run_dev(ctx, wh.lib.wm_bitlinear_i2s_matvec_f32_dev_noalloc, w, x, out_dim)
        ref = run_dev(ctx, wh.lib.wm_bitlinear_i2s_matvec_f32_dev, w, x, out_dim)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (in_dim, out_dim)
        w.close()


def test_noalloc_rejects_shape_above_scratch_limit(ctx):
    # 1048576 output rows of 128 values: one partial dot per row is 4 MiB,
    # which with the activation codes and their record is above the 4 MiB array
    in_dim, out_dim = 128, 1 << 20
    w = ctx.upload_i2s(np.full(out_dim * in_dim // 4, 0x55, np.uint8), 1.0, in_dim, out_dim)
    x = ctx.to_device(np.ones(in_dim, np.float32))
    y = ctx.alloc(out_dim * 4)
    with pytest.raises(wh.WillametteError) as e:
        ctx.check(wh.lib.wm_bitlinear_i2s_matvec_f32_dev_noalloc(ctx.h, w.h, x.ptr, y.ptr))
    assert e.value.kind == "Shape"
    x.free()
    y.free()
    w.close()
