"""CPU tests of the GGUF reader and BitNet graph checks (wm_gguf_*), against
the reference's own reader test vectors and oracle/gguf_ref.py.

- The reference's reader tests (src/gguf/reader.rs:820-930) are restated one
  by one and run on both the library and the oracle: each must reject with
  the reference's message fragments.
- The oracle is further pinned by round trips through this file's
  independent GGUF builder and bitnet_synth's writer, by the synthetic-model
  layout of tests/synthetic_model.rs:172-305 (2 layers, n_embd 128, 2+11*2
  tensors) and by edge cases whose outcome the format fixes (alignment,
  EOF, UTF-8, nesting depth).
- Then the library and the oracle are compared on every prefix and on
  seeded byte mutations of real images: same accept/reject, same error kind,
  same message, and for accepted images the same directory and metadata.

No device calls: wm_gguf_parse / _open / _bitnet_config / _bitnet_check are
host-only.
"""
import struct

import numpy as np
import pytest

import bitnet_synth as bs
import willamette_hip as wh
from oracle import gguf_ref as gr

MAGIC = 0x46554747


def u32(v):
    return struct.pack("<I", v)


def u64(v):
    return struct.pack("<Q", v)


def gstr(s):
    b = s.encode() if isinstance(s, str) else s
    return u64(len(b)) + b


def header(n_tensors, n_kv, version=3):
    return u32(MAGIC) + u32(version) + u64(n_tensors) + u64(n_kv)


def build(infos, data, meta=b"", n_kv=0, align=32):
    """The reference tests' build_gguf (src/gguf/reader.rs:797-814): header,
    directory, zero padding to 32, raw tensor bytes."""
    buf = header(len(infos), n_kv) + meta
    for name, shape, typ, off in infos:
        buf += gstr(name) + u32(len(shape)) + b"".join(u64(d) for d in shape) + u32(typ) + u64(off)
    buf += bytes(-len(buf) % align)
    return buf + bytes(data)


def kv_u32(key, v):
    return gstr(key) + u32(4) + u32(v)


def lib_parse(data):
    """(kind, message) of the library's rejection, or the parsed file."""
    try:
        return wh.GgufFile.parse(data)
    except wh.WillametteError as e:
        return (e.kind, str(e).split("] ", 1)[1])


def ref_parse(data):
    try:
        return gr.parse(data)
    except gr.GgufRefError as e:
        # the library's message is a C string: a name's NULs drop out of it
        return (e.kind, e.message.replace("\x00", ""))


# --------------------------------------------------------------------------
# the reference's reader tests (src/gguf/reader.rs:820-930)
# --------------------------------------------------------------------------

REFERENCE_VECTORS = {
    # name: (image, fragments that must all appear in the message)
    "unknown_byte_layout": (build([("unknown", [7], 999, 0)], [1, 2, 3, 4, 5, 6, 7]),
                            ["unsupported type", "byte length is unknown"]),
    "overlapping_known_tensors": (build([("first", [2], 0, 0), ("second", [1], 0, 4)], bytes(8)),
                                  ["overlaps next tensor"]),
    "i2s_scale_block_overlap": (build([("i2s", [128], 36, 0), ("next", [1], 0, 48)], bytes(64)),
                                ["scale block ends", "overlapping next tensor"]),
    "shape_product_overflow": (build([("bad", [2**64 - 1, 2], 24, 0)], b""),
                               ["shape product overflow"]),
    "byte_length_overflow": (build([("bad", [2**64 - 1], 28, 0)], b""), ["byte length overflow"]),
    "incomplete_quantized_block": (build([("bad", [31], 2, 0)], b""), ["Q4_0 row length 31"]),
    "q8_0_row_alignment": (build([("bad", [16, 2], 8, 0)], bytes(34)), ["Q8_0 row length 16"]),
    "q4_0_row_alignment": (build([("bad", [16, 2], 2, 0)], bytes(18)), ["Q4_0 row length 16"]),
    "q4k_row_alignment": (build([("bad", [128, 2], 12, 0)], bytes(144)), ["Q4_K row length 128"]),
    "excessive_tensor_count": (header(1_000_001, 0), ["tensor_count", "safety limit"]),
    "excessive_kv_count": (header(0, 1_000_001), ["metadata_kv_count", "safety limit"]),
    "excessive_dims": (header(1, 0) + gstr("bad") + u32(5) + bytes(24), ["n_dims 5 exceeds 4"]),
    "excessive_array_count": (header(0, 1) + gstr("array") + u32(9) + u32(0) + u64(1_000_001),
                              ["array count", "safety limit"]),
}


@pytest.mark.parametrize("name", sorted(REFERENCE_VECTORS))
def test_reference_reader_vectors(name):
    data, fragments = REFERENCE_VECTORS[name]
    for got in (lib_parse(data), ref_parse(data)):
        assert isinstance(got, tuple), f"{name}: accepted"
        kind, msg = got
        assert kind == "GgufParse", (name, kind, msg)
        for f in fragments:
            assert f in msg, (name, msg)


# --------------------------------------------------------------------------
# header-level errors and format rules
# --------------------------------------------------------------------------

def test_magic_version_and_truncation():
    bad_magic = u32(0x12345678) + u32(3) + u64(0) + u64(0)
    for got in (lib_parse(bad_magic), ref_parse(bad_magic)):
        assert got == ("InvalidMagic", "Invalid GGUF magic (expected 0x46554747, got 0x12345678)")
    for v in (1, 4):
        data = header(0, 0, version=v)
        for got in (lib_parse(data), ref_parse(data)):
            assert got == ("UnsupportedVersion", f"Unsupported GGUF version: {v} (supported: 2, 3)")
    for data in (b"", u32(MAGIC)[:3], u32(MAGIC), u32(MAGIC) + u32(3) + u64(0)):
        for got in (lib_parse(data), ref_parse(data)):
            assert got[0] == "GgufParse" and "unexpected end of data" in got[1], got
    # an empty file has no tensors: v2 and v3 both parse
    for v in (2, 3):
        g = wh.GgufFile.parse(header(0, 0, version=v))
        assert (g.version, len(g), g.alignment) == (v, 0, 32)


def test_alignment_rules():
    # general.alignment = 64 moves the data section and every offset
    meta = kv_u32("general.alignment", 64)
    data = build([("t", [4], 0, 0)], struct.pack("<4f", 1, 2, 3, 4), meta, 1, align=64)
    g = wh.GgufFile.parse(data)
    r = gr.parse(data)
    assert g.alignment == r["alignment"] == 64
    assert g.data_offset == r["data_start"] and g.data_offset % 64 == 0
    t = g.tensor(0)
    assert np.frombuffer(t["data"].tobytes(), "<f4").tolist() == [1, 2, 3, 4]
    # non power of two, or zero
    for a in (0, 48):
        data = build([], b"", kv_u32("general.alignment", a), 1)
        for got in (lib_parse(data), ref_parse(data)):
            assert got == ("GgufParse", f"invalid alignment value: {a}")
    # a negative i32 alignment is not a u64: the default applies
    meta = gstr("general.alignment") + u32(5) + struct.pack("<i", -64)
    g = wh.GgufFile.parse(build([("t", [1], 0, 0)], bytes(4), meta, 1))
    assert g.alignment == 32


def test_tensor_bounds_and_offsets():
    # data past EOF: TensorOutOfBounds with the byte range
    data = build([("t", [8], 0, 0)], bytes(16))
    for got in (lib_parse(data), ref_parse(data)):
        assert got[0] == "TensorOutOfBounds" and 'tensor "t" requires bytes' in got[1], got
    # I2_S with its codes in the file but not its 32-byte scale block
    data = build([("w", [128, 1], 36, 0)], bytes(32 + 31))
    for got in (lib_parse(data), ref_parse(data)):
        assert got[0] == "TensorOutOfBounds" and "(scale block)" in got[1], got
    data = build([("w", [128, 1], 36, 0)], bytes(64))
    g = wh.GgufFile.parse(data)
    assert g.tensor(0)["bytes"] == 32 and g.tensor(0)["scale_block"].size == 32
    # two tensors at one offset
    data = build([("a", [1], 0, 0), ("b", [1], 0, 0)], bytes(8))
    for got in (lib_parse(data), ref_parse(data)):
        assert got == ("GgufParse", 'tensor "a" shares data offset 0 with another tensor')
    # a tensor directory that points past EOF before any data
    data = header(1, 0) + gstr("t") + u32(1) + u64(1) + u32(0) + u64(0)
    for got in (lib_parse(data), ref_parse(data)):
        assert got[0] == "GgufParse" and "starts beyond EOF" in got[1], got
    # zero-element tensors take no bytes, whatever the type
    g = wh.GgufFile.parse(build([("z", [0, 5], 999, 0)], b""))
    assert g.tensor(0)["bytes"] == 0


def test_strings_and_arrays():
    # a string above 1 MiB
    data = header(0, 1) + u64(1_048_577) + bytes(16)
    for got in (lib_parse(data), ref_parse(data)):
        assert got[0] == "GgufParse" and "exceeds 1 MiB safety limit" in got[1], got
    # invalid UTF-8 (overlong, surrogate, lone continuation, past U+10FFFF,
    # cut short, bad third byte): Rust's Utf8Error text
    cases = {b"\xc0\xaf": "invalid utf-8 sequence of 1 bytes from index 0",
             b"\xed\xa0\x80": "invalid utf-8 sequence of 1 bytes from index 0",
             b"\x80": "invalid utf-8 sequence of 1 bytes from index 0",
             b"\xf4\x90\x80\x80": "invalid utf-8 sequence of 1 bytes from index 0",
             b"ab\xe2\x82": "incomplete utf-8 byte sequence from index 2",
             b"ab\xe2\x82x": "invalid utf-8 sequence of 2 bytes from index 2",
             b"\xf0\x9f\x99z": "invalid utf-8 sequence of 3 bytes from index 0"}
    for bad, text in cases.items():
        data = header(0, 1) + gstr(bad) + u32(4) + u32(1)
        for got in (lib_parse(data), ref_parse(data)):
            assert got == ("GgufParse", f"metadata[0] key: invalid UTF-8: {text}"), (bad, got)
    good = "κλειδί-🙂"
    g = wh.GgufFile.parse(header(0, 1) + gstr(good) + u32(8) + gstr("ok"))
    assert g.meta_str(good) == "ok"
    # nesting: 16 levels parse, 17 do not
    def nested(depth):
        v = u32(4) + u64(1) + u32(7)  # innermost: array of one u32
        for _ in range(depth - 1):
            v = u32(9) + u64(1) + v
        return header(0, 1) + gstr("deep") + u32(9) + v
    assert isinstance(lib_parse(nested(16)), wh.GgufFile)
    assert isinstance(ref_parse(nested(16)), dict)
    for got in (lib_parse(nested(17)), ref_parse(nested(17))):
        assert got[0] == "GgufParse" and "nesting depth 17 exceeds 16" in got[1], got
    # an array whose minimum size exceeds the bytes left
    data = header(0, 1) + gstr("a") + u32(9) + u32(10) + u64(100) + bytes(16)
    for got in (lib_parse(data), ref_parse(data)):
        assert got[0] == "GgufParse" and "cannot fit in" in got[1], got


def test_oracle_utf8_matches_python_decoder():
    """The oracle's UTF-8 rule against CPython's strict decoder on random
    and structured byte strings: valid exactly when CPython decodes, the
    same start index, and the same maximal-subpart length (CPython's
    invalid-start / invalid-continuation / unexpected-end reasons)."""
    rng = np.random.default_rng(7)
    pool = [0x00, 0x41, 0x7F, 0x80, 0xBF, 0xC0, 0xC1, 0xC2, 0xDF, 0xE0, 0xED, 0xEF, 0xF0, 0xF4,
            0xF5, 0xFF, 0x9F, 0xA0, 0x8F, 0x90]
    for _ in range(20000):
        n = int(rng.integers(0, 7))
        b = bytes(int(rng.choice(pool)) if rng.random() < 0.8 else int(rng.integers(0, 256))
                  for _ in range(n))
        err = gr.utf8_error(b)
        try:
            b.decode("utf-8")
            assert err is None, b
        except UnicodeDecodeError as e:
            if e.reason == "unexpected end of data":
                assert err == f"incomplete utf-8 byte sequence from index {e.start}", (b, err)
            else:
                assert err == f"invalid utf-8 sequence of {e.end - e.start} bytes from index {e.start}", (b, err, e)


def test_metadata_getters():
    meta = (gstr("u8") + u32(0) + b"\x07" + gstr("i32n") + u32(5) + struct.pack("<i", -3) +
            gstr("i64") + u32(11) + struct.pack("<q", 9) + gstr("f64") + u32(12) + struct.pack("<d", 0.1) +
            gstr("s") + u32(8) + gstr("text"))
    g = wh.GgufFile.parse(header(0, 5) + meta)
    assert g.meta_u64("u8") == 7 and g.meta_u64("i64") == 9
    assert g.meta_u64("i32n") is None                       # as_u64 of a negative
    assert g.meta_f32("f64") == float(np.float32(0.1))      # as_f32 narrows f64
    assert g.meta_f32("u8") is None and g.meta_str("s") == "text" and g.meta_u64("missing") is None


# --------------------------------------------------------------------------
# BitNet models: round trips, config and graph checks
# --------------------------------------------------------------------------

TINY = bs.BitNetConfig(n_layers=2, n_embd=256, n_ff=384, n_heads=4, n_kv_heads=2, head_dim=64,
                       vocab=300, context_length=128)


@pytest.fixture(scope="module")
def tiny():
    hm = bs.make_host_model(TINY, 0x5EED)
    return hm, bs.gguf_bytes(hm)


def _directory(g):
    return [(t["name"], t["type"], t["shape"], t["offset"], t["bytes"]) for t in
            (g.tensor(i) for i in range(len(g)))]


def test_writer_round_trip(tiny, tmp_path):
    hm, data = tiny
    r = gr.parse(data)
    g = wh.GgufFile.parse(data)
    assert g.version == 3 and len(g) == 2 + 11 * TINY.n_layers == len(r["tensors"])
    assert _directory(g) == [(t["name"], t["type"], t["shape"], t["offset"], t["bytes"]) for t in r["tensors"]]
    # every tensor's bytes are the host model's
    expect = {n: d for n, _, _, d in bs.gguf_tensors(hm)}
    for i in range(len(g)):
        t = g.tensor(i)
        blob = expect[t["name"]]
        if t["type"] == wh.TYPE_I2S:
            assert t["data"].tobytes() + t["scale_block"].tobytes() == blob
        else:
            assert t["data"].tobytes() == blob and t["scale_block"] is None
        assert t["offset"] % 32 == 0
    cfg = g.bitnet_config()
    ref = gr.bitnet_config(r)
    for f, _ in wh.ModelConfig._fields_:
        assert getattr(cfg, f) == pytest.approx(ref[f], rel=0, abs=0), f
    assert (cfg.n_layers, cfg.n_embd, cfg.n_ff, cfg.head_dim, cfg.vocab_size) == (2, 256, 384, 64, 300)
    g.bitnet_check()
    gr.bitnet_graph(r)
    # the same through a file mapping
    p = tmp_path / "tiny.gguf"
    bs.write_gguf(p, hm)
    assert p.read_bytes() == data
    gf = wh.GgufFile.open(p)
    assert _directory(gf) == _directory(g)
    gf.close()


def test_reference_synthetic_layout():
    """tests/synthetic_model.rs:172-330: 2 layers, n_embd 128, vocab 4,
    head_dim 64 (2 heads, 1 kv head), n_ff 256, F16 embedding; parses to a
    complete graph with 2 + 2*11 tensors.  The library accepts the file
    and its config but reports the F16 embedding as unsupported (its
    embedding and lm-head kernels read Q6_K)."""
    E, F, V, L, HD = 128, 256, 4, 2, 64
    tensors = [("token_embd.weight", [E, V], 1, np.full(E * V, 0x3C00, "<u2").tobytes()),
               ("output_norm.weight", [E], 0, np.ones(E, "<f4").tobytes())]
    i2s = lambda i, o: bytes([0x55]) * (i * o // 4) + struct.pack("<f", 1.0) + bytes(28)
    for il in range(L):
        tensors += [(f"blk.{il}.attn_norm.weight", [E], 0, np.ones(E, "<f4").tobytes()),
                    (f"blk.{il}.attn_sub_norm.weight", [E], 0, np.ones(E, "<f4").tobytes()),
                    (f"blk.{il}.attn_q.weight", [E, E], 36, i2s(E, E)),
                    (f"blk.{il}.attn_k.weight", [E, HD], 36, i2s(E, HD)),
                    (f"blk.{il}.attn_v.weight", [E, HD], 36, i2s(E, HD)),
                    (f"blk.{il}.attn_output.weight", [E, E], 36, i2s(E, E)),
                    (f"blk.{il}.ffn_norm.weight", [E], 0, np.ones(E, "<f4").tobytes()),
                    (f"blk.{il}.ffn_sub_norm.weight", [F], 0, np.ones(F, "<f4").tobytes()),
                    (f"blk.{il}.ffn_gate.weight", [E, F], 36, i2s(E, F)),
                    (f"blk.{il}.ffn_up.weight", [E, F], 36, i2s(E, F)),
                    (f"blk.{il}.ffn_down.weight", [F, E], 36, i2s(F, E))]
    cfg = bs.BitNetConfig(n_layers=L, n_embd=E, n_ff=F, n_heads=2, n_kv_heads=1, head_dim=HD, vocab=V,
                          context_length=64)
    data = b"".join(bs.gguf_image(tensors, bs.gguf_metadata(cfg)))
    r = gr.parse(data)
    assert r["version"] == 3 and len(r["tensors"]) == 2 + L * 11
    graph = gr.bitnet_graph(r)
    assert graph["config"]["head_dim"] == HD and len(graph["layers"]) == L
    g = wh.GgufFile.parse(data)
    assert g.bitnet_config().head_dim == HD
    with pytest.raises(wh.WillametteError) as ei:
        g.bitnet_check()
    assert ei.value.kind == "UnsupportedTensorType" and "F16" in str(ei.value)


def _meta_without(cfg, drop=None, arch="bitnet-b1.58", replace=None):
    kv = [x for x in bs.gguf_metadata(cfg, arch) if x[0] != drop]
    if replace:
        kv = [replace.get(k, (k, t, v)) for k, t, v in kv]
    return kv


@pytest.mark.parametrize("case,kind,fragment", [
    ("arch_llama", "UnsupportedArchitecture", 'Unsupported architecture: "llama"'),
    ("no_arch", "MissingMetadata", "general.architecture"),
    ("no_block_count", "MissingMetadata", "bitnet-b1.58.block_count (u32/u64)"),
    ("no_eps", "MissingMetadata", "layer_norm_rms_epsilon (f32)"),
    ("eps_as_u32", "MissingMetadata", "layer_norm_rms_epsilon (f32)"),
    ("vocab_too_big", "GgufParse", "does not fit in u32"),
    ("heads_not_dividing", "GgufParse", "not divisible by head_count 3"),
    ("kv_not_dividing", "GgufParse", "GQA ratio must be integer"),
    ("rope_dim", "GgufParse", "rope.dimension_count (32) must equal head_dim (64)"),
    ("zero_layers", "GgufParse", "block_count must be > 0"),
])
def test_config_errors(tiny, case, kind, fragment):
    hm, _ = tiny
    a = "bitnet-b1.58"
    meta = {
        "arch_llama": _meta_without(TINY, replace={"general.architecture": ("general.architecture", 8, "llama")}),
        "no_arch": _meta_without(TINY, "general.architecture"),
        "no_block_count": _meta_without(TINY, f"{a}.block_count"),
        "no_eps": _meta_without(TINY, f"{a}.attention.layer_norm_rms_epsilon"),
        "eps_as_u32": _meta_without(TINY, replace={f"{a}.attention.layer_norm_rms_epsilon":
                                                   (f"{a}.attention.layer_norm_rms_epsilon", 4, 1)}),
        "vocab_too_big": _meta_without(TINY, replace={f"{a}.vocab_size": (f"{a}.vocab_size", 10, 2**32)}),
        "heads_not_dividing": _meta_without(TINY, replace={f"{a}.attention.head_count":
                                                           (f"{a}.attention.head_count", 4, 3)}),
        "kv_not_dividing": _meta_without(TINY, replace={f"{a}.attention.head_count_kv":
                                                        (f"{a}.attention.head_count_kv", 4, 3)}),
        "rope_dim": _meta_without(TINY, replace={f"{a}.rope.dimension_count":
                                                 (f"{a}.rope.dimension_count", 4, 32)}),
        "zero_layers": _meta_without(TINY, replace={f"{a}.block_count": (f"{a}.block_count", 4, 0)}),
    }[case]
    data = b"".join(bs.gguf_image(bs.gguf_tensors(hm), meta))
    g = wh.GgufFile.parse(data)
    with pytest.raises(wh.WillametteError) as ei:
        g.bitnet_config()
    assert ei.value.kind == kind and fragment in str(ei.value), str(ei.value)
    with pytest.raises(gr.GgufRefError) as er:
        gr.bitnet_config(gr.parse(data))
    assert er.value.kind == kind and fragment in er.value.message


@pytest.mark.parametrize("arch", ["bitnet-b1.58", "bitnet-25", "bitnet"])
def test_architecture_aliases(tiny, arch):
    """bitnet.rs:29-43: the three strings share the graph; each is its own
    metadata prefix."""
    hm, _ = tiny
    g = wh.GgufFile.parse(bs.gguf_bytes(hm, arch=arch))
    assert g.meta_str("general.architecture") == arch
    assert g.bitnet_config().n_layers == TINY.n_layers
    g.bitnet_check()


def _mutated_tensors(hm, how):
    ts = bs.gguf_tensors(hm)
    if how == "missing_role":
        return [t for t in ts if t[0] != "blk.1.ffn_sub_norm.weight"]
    if how == "missing_embd":
        return [t for t in ts if t[0] != "token_embd.weight"]
    if how == "bias":
        return ts + [("blk.0.attn_q.bias", [TINY.n_embd], 0, bytes(4 * TINY.n_embd))]
    if how == "duplicate":
        return ts + [ts[1]]
    if how == "q_as_f32":
        return [(n, s, 0, bytes(4 * s[0] * s[1])) if n == "blk.0.attn_q.weight" else (n, s, t, d)
                for n, s, t, d in ts]
    if how == "k_shape":
        return [(n, [s[0], s[1] // 2], t, d[: len(d) // 2 - 16] + d[-32:]) if n == "blk.1.attn_k.weight"
                else (n, s, t, d) for n, s, t, d in ts]
    if how == "output_weight_q4":
        E, V = TINY.n_embd, TINY.vocab
        return ts + [("output.weight", [E, V], 2, bytes(E // 32 * 18 * V))]
    raise ValueError(how)


@pytest.mark.parametrize("how,kind,fragment", [
    ("missing_role", "MissingMetadata", "tensor blk.1.ffn_sub_norm.weight"),
    ("missing_embd", "MissingMetadata", "tensor token_embd.weight"),
    ("bias", "NotImplemented", "blk.0.attn_q.bias"),
    ("duplicate", "GgufParse", "duplicate tensor names"),
    ("q_as_f32", "GgufParse", "blk.0.attn_q.weight"),
    ("k_shape", "Shape", "blk.1.attn_k.weight"),
    ("output_weight_q4", "GgufParse", "output.weight"),
])
def test_graph_errors(tiny, how, kind, fragment):
    hm, _ = tiny
    tensors = _mutated_tensors(hm, how)
    if how == "duplicate":
        # the directory holds the name twice at different offsets
        data = b"".join(bs.gguf_image(tensors, bs.gguf_metadata(TINY)))
    else:
        data = b"".join(bs.gguf_image(tensors, bs.gguf_metadata(TINY)))
    g = wh.GgufFile.parse(data)
    with pytest.raises(wh.WillametteError) as ei:
        g.bitnet_check()
    assert ei.value.kind == kind and fragment in str(ei.value), str(ei.value)
    with pytest.raises(gr.GgufRefError) as er:
        gr.bitnet_graph(gr.parse(data))
    assert er.value.kind == kind and fragment in er.value.message, er.value.message


# --------------------------------------------------------------------------
# library vs oracle on prefixes and byte mutations
# --------------------------------------------------------------------------

def _compare(data):
    a, b = lib_parse(data), ref_parse(data)
    if isinstance(a, tuple) or isinstance(b, tuple):
        assert a == b, (a, b)
        return False
    assert (a.version, a.alignment, a.data_offset) == (b["version"], b["alignment"], b["data_start"])
    # names come back as C strings: compared up to a NUL
    assert _directory(a) == [(t["name"].split("\x00")[0], t["type"], t["shape"], t["offset"], t["bytes"])
                             for t in b["tensors"]]
    for k, (t, v) in b["meta"].items():
        if "\x00" in k:  # a NUL inside a key cannot be named through a C string
            continue
        if t in (gr.U8, gr.U16, gr.U32, gr.U64) or (t in (gr.I32, gr.I64) and v >= 0):
            assert a.meta_u64(k) == v
        elif t == gr.STR:
            assert a.meta_str(k) == v
        elif t in (gr.F32, gr.F64):
            x = a.meta_f32(k)
            assert x == gr.as_f32((t, v)) or (x != x and v != v)
    return True


def test_prefixes_match_oracle(tiny):
    """Every truncation of a small image through its header and the first
    tensors: same outcome and message."""
    _, data = tiny
    g = wh.GgufFile.parse(data)
    first = g.tensor(1)
    cut = first["offset"] + first["bytes"] + 8
    for n in range(0, cut):
        _compare(data[:n])


def test_mutations_match_oracle(tiny):
    """Seeded single-byte and u64 overwrites of the header, metadata and
    directory: same outcome, kind and message, and the same directory when
    accepted."""
    _, data = tiny
    head = wh.GgufFile.parse(data).data_offset
    rng = np.random.default_rng(20261202)
    accepted = 0
    for _ in range(1500):
        b = bytearray(data)
        pos = int(rng.integers(0, head))
        mode = rng.integers(0, 3)
        if mode == 0:
            b[pos] = int(rng.integers(0, 256))
        elif mode == 1 and pos + 8 <= len(b):
            vals = [0, 1, 2, 5, 7, 31, 36, 2**31, 2**63, 2**64 - 1]
            b[pos:pos + 8] = struct.pack("<Q", vals[int(rng.integers(0, len(vals)))])
        else:
            b[pos] ^= 1 << int(rng.integers(0, 8))
        accepted += _compare(bytes(b))
    assert accepted > 50  # some mutations land in values that still parse
