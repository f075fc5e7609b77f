"""CPU checks of the C ABI: the library loads, exports every entry point
include/willamette_hip.h declares, and its host-only functions behave.  No
GPU compute runs here."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import willamette_hip as wh

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    text = (ROOT / "include" / "willamette_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wm_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    names = declared_functions()
    assert len(names) > 30
    lib = C.CDLL(str(wh.LIB_PATH))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares a signature for each of them
    assert set(names) == set(wh.EXPORTS), set(names) ^ set(wh.EXPORTS)


def test_version_string():
    assert b"gfx950" in wh.lib.wm_version()


def test_synth_streams_are_deterministic_and_counter_based():
    a = wh.synth_i2s(7, 3, 256, 64)
    b = wh.synth_i2s(7, 3, 256, 64)
    c = wh.synth_i2s(7, 4, 256, 64)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    big = wh.synth_i2s(7, 3, 2560, 2560)  # many threads
    assert np.array_equal(big[: a.size], a)  # prefix does not depend on the split
    codes = np.stack([(big >> 6) & 3, (big >> 4) & 3, (big >> 2) & 3, big & 3]).ravel()
    assert codes.max() == 2  # never the degenerate 11 code (src/synth.rs:209-212)
    frac = np.bincount(codes, minlength=3) / codes.size
    assert np.all(np.abs(frac - 1 / 3) < 0.005)


def test_synth_distributions():
    u = wh.synth_uniform(1, 1, 100000, 0.5, 2.0)
    assert u.min() >= 0.5 and u.max() < 2.0 and abs(u.mean() - 1.25) < 0.01
    n = wh.synth_normal(1, 2, 200000)
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1) < 0.01
    q = wh.synth_q6k(1, 3, 64, 256).reshape(64, 210)
    sc = q[:, 192:208].view(np.int8)
    assert sc.min() >= -32 and sc.max() <= 31
    d = q[:, 208:210].copy().view(np.float16).astype(np.float32).ravel()
    assert np.all(d >= 0) and 2e-4 < float(np.median(d)) < 2e-3


def test_host_argmax_matches_reference_rule():  # src/model/lm_head.rs:161-174
    assert wh.argmax(np.array([0.1, 0.5, 0.3], np.float32)) == 1
    assert wh.argmax(np.array([], np.float32)) is None
    assert wh.argmax(np.array([1.0, 1.0], np.float32)) == 0


def test_scale_block_layout():
    b = wh.scale_block(1.5)
    assert b.size == 32 and np.frombuffer(b[:4].tobytes(), np.float32)[0] == 1.5 and not b[4:].any()
