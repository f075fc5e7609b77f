"""GPU: the exact wave-parallel evaluation of a left-to-right f32 sum
(project-willamette_amd/csrc/wm_seqsum.h) against numpy's sequential float32
accumulation, on inputs built to hit its special cases: round-half-even
ties, binade crossings, absorbed terms, zeros, subnormals, overflow, NaN."""
import numpy as np
import pytest

import willamette_hip as wh

pytestmark = pytest.mark.gpu


def seq_ref(a: np.ndarray) -> np.float32:
    a = np.asarray(a, np.float32)
    if a.size == 0:
        return np.float32(0.0)
    return np.add.accumulate(a, dtype=np.float32)[-1]


def same(x, y):
    x, y = np.float32(x), np.float32(y)
    return (np.isnan(x) and np.isnan(y)) or x.view(np.uint32) == y.view(np.uint32)


def cases():
    rng = np.random.default_rng(0)
    out = []
    for n in (0, 1, 2, 31, 32, 33, 63, 100, 255, 256, 257, 289, 2560, 6912, 65536):
        out.append((f"sq{n}", (rng.standard_normal(n).astype(np.float32) ** 2)))
    # RMSNorm-like inputs at decode scale
    out.append(("hidden2560", (rng.standard_normal(2560).astype(np.float32) * 300) ** 2))
    out.append(("ffn6912", (rng.standard_normal(6912) ** 3 * 1e3).astype(np.float32) ** 2))
    # softmax-like: exp of non-positive scores
    s = rng.standard_normal(1088).astype(np.float32) * 4
    out.append(("softmax1088", np.exp(s - s.max()).astype(np.float32)))
    # ties: s = 2^24 (ulp 2); odd integers are exact halfway cases
    t = np.concatenate([[2.0 ** 24], rng.integers(0, 4, 5000).astype(np.float32)])
    out.append(("ties_ulp2", t))
    t = np.concatenate([[3.0 * 2 ** 23], np.tile(np.float32([1, 1, 3, 0.5, 1.5, 1]), 700)])
    out.append(("ties_mixed", t))
    # every term absorbed, then growth across many binades
    out.append(("absorbed", np.concatenate([[2.0 ** 30], np.full(3000, 1.0)]).astype(np.float32)))
    out.append(("growth", (2.0 ** (np.arange(600) / 8.0)).astype(np.float32)))
    out.append(("powers", np.float32(2.0) ** rng.integers(-30, 30, 4000).astype(np.float32)))
    # zeros, tiny and subnormal terms
    z = np.zeros(3000, np.float32)
    z[1500] = 1e-3
    out.append(("zeros_then_one", z))
    out.append(("subnormal", np.full(4000, 1e-40, np.float32)))
    sub = rng.standard_normal(4000).astype(np.float32) ** 2
    sub[::7] = 1e-42
    out.append(("mixed_subnormal", sub))
    # overflow to inf and NaN terms
    out.append(("overflow", np.full(300, 3e37, np.float32)))
    nan = rng.standard_normal(700).astype(np.float32) ** 2
    nan[400] = np.nan
    out.append(("nan", nan))
    inf = rng.standard_normal(700).astype(np.float32) ** 2
    inf[10] = np.inf
    out.append(("inf", inf))
    # s reaches a significand of all ones (N = 2^24 - 1) after the leading
    # terms; zero-increment terms there must not end the run
    out.append(("allones_significand", np.concatenate(
        [[16777215.0], np.zeros(127), [0.25, 0, 0, 1.0, 0.5, 3.0], np.full(600, 0.25)]).astype(np.float32)))
    # long random runs with many ties: values on a coarse grid
    g = (rng.integers(0, 64, 20000) * 0.25).astype(np.float32)
    out.append(("grid", np.concatenate([[2.0 ** 22], g]).astype(np.float32)))
    # exact prefix 2^-52 below 4096 at a thread boundary while the f32 sum
    # lags 3 ulps behind (absorbed terms), then 2^-11, a tie and zeros
    head = [4096.0 - 3 * 2.0 ** -12] + [2.0 ** -14] * 11 + [2.0 ** -i for i in range(15, 41)]
    out.append(("prefix_at_power_of_two",
                np.array(head + [2.0 ** -11, 2.0 ** -12] + [0.0] * 1460, np.float32)))
    # the same with the boundary prefixes on many powers of two (m = 4)
    ones = np.ones(4000, np.float32)
    ones[::7] = np.float32(2.0 ** -30)
    out.append(("ones_on_powers", ones))
    # runs of exact zeros: a softmax whose older positions underflow (zero
    # prefix, then the live terms), a zero lead-in, a sparse vector
    for n, live in ((1088, 64), (4000, 5), (2049, 1)):
        sc = np.concatenate([rng.standard_normal(n - live) * 4.0 - 200.0, rng.standard_normal(live) * 3.0])
        out.append((f"softmax_underflow{n}_{live}", np.exp((sc - sc.max()).astype(np.float32)).astype(np.float32)))
    out.append(("zero_lead", np.concatenate([np.zeros(700), rng.random(388) + 0.5]).astype(np.float32)))
    sp = (rng.standard_normal(3000) ** 2).astype(np.float32)
    sp[rng.random(3000) < 0.9] = 0.0
    out.append(("sparse", sp))
    return out


@pytest.mark.parametrize("name,a", cases(), ids=[c[0] for c in cases()])
def test_seq_sum_matches_sequential_f32(ctx, name, a):
    got = wh.debug_seq_sum(ctx, a)
    ref = seq_ref(a)
    assert same(got, ref), f"{name}: device {got!r} vs sequential {ref!r}"


def test_seq_sum_random_fuzz(ctx):
    rng = np.random.default_rng(42)
    for i in range(300):
        n = int(rng.integers(1, 3000))
        scale = float(2.0 ** rng.integers(-20, 20))
        kind = i % 3
        if kind == 0:
            a = (rng.standard_normal(n) * scale).astype(np.float32) ** 2
        elif kind == 1:
            a = (rng.integers(0, 8, n) * scale).astype(np.float32)
        else:
            a = rng.exponential(scale, n).astype(np.float32)
        if i % 5 == 4:  # runs of zeros
            a[rng.random(n) < rng.random()] = 0.0
        got, ref = wh.debug_seq_sum(ctx, a), seq_ref(a)
        assert same(got, ref), f"case {i} n={n} kind={kind}: {got!r} vs {ref!r}"
