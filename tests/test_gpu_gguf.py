"""GPU parity of the GGUF loader: a model built by wm_model_from_gguf decodes
bit-identically to the oracle on the same weights.

The GGUF images come from bitnet_synth's writer (the tensor layout of
tests/synthetic_model.rs:172-305 with random ternary weights, per-tensor
I2_S scales in the trailing 32-byte blocks, Q6_K token_embd), parsed from
memory and from a file mapping.  Bar: final hidden, logits and greedy ids
bit-identical to the oracle model over the same host weights, and to the
model uploaded tensor by tensor.
"""
import numpy as np
import pytest

import bitnet_synth as bs
import willamette_hip as wh
from oracle.oracle_model import OracleModel

pytestmark = pytest.mark.gpu

GQA = bs.BitNetConfig(n_layers=3, n_embd=256, n_ff=384, n_heads=4, n_kv_heads=2, head_dim=64,
                      vocab=600, context_length=96)


def bits_equal(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("source", ["bytes", "file"])
def test_gguf_model_decodes_like_oracle(ctx, tmp_path, source):
    hm = bs.make_host_model(GQA, seed=0x6607)
    if source == "bytes":
        gf = wh.GgufFile.parse(bs.gguf_bytes(hm))
    else:
        p = tmp_path / "gqa.gguf"
        bs.write_gguf(p, hm, alignment=64)
        gf = wh.GgufFile.open(p)
    print(f"gguf {source}: {len(gf)} tensors", flush=True)
    dev = bs.DeviceModel.from_gguf(ctx, gf)
    gf.close()  # the device model owns its copies
    orm = OracleModel(hm)
    n_pre = 40
    k, v = bs.kv_prefill(GQA, seed=5, n_pos=n_pre)
    dkv, okv = dev.kv_cache(GQA.context_length), orm.kv(GQA.context_length)
    dkv.append_positions(k, v)
    okv.append_positions(k, v)
    tok = 11
    for pos in range(n_pre, n_pre + 8):
        h, logits, nxt = dkv.decode_step(tok, pos)
        rh = okv.forward(tok, pos)
        rlogits, rnxt = okv.logits_argmax(rh)
        assert bits_equal(h, rh), f"pos {pos}: hidden differs"
        assert bits_equal(logits, rlogits), f"pos {pos}: logits differ"
        assert nxt == rnxt
        tok = nxt
    dev.close()
    orm.close()


def test_gguf_model_matches_uploaded_model_2b(ctx, tmp_path):
    """BitNet-b1.58-2B shape through a 792 MB GGUF file: the file-loaded
    model and the tensor-by-tensor model give identical hidden states,
    logits and ids over a prefilled cache."""
    cfg = bs.BITNET_2B
    hm = bs.make_host_model(cfg, seed=bs.master_seed(1))
    p = tmp_path / "bitnet2b.gguf"
    bs.write_gguf(p, hm)
    gf = wh.GgufFile.open(p)
    print("gguf 2b: opened", flush=True)
    a = bs.DeviceModel.from_gguf(ctx, gf, max_context=1024)
    gf.close()
    p.unlink()
    b = bs.load_device_model(ctx, hm)
    n_pre = 300
    k, v = bs.kv_prefill(cfg, seed=3, n_pos=n_pre)
    ka, kb = a.kv_cache(1024), b.kv_cache(1024)
    ka.append_positions(k, v)
    kb.append_positions(k, v)
    tok = 128000
    for pos in range(n_pre, n_pre + 4):
        ha, la, na = ka.decode_step(tok, pos)
        hb, lb, nb = kb.decode_step(tok, pos)
        assert bits_equal(ha, hb) and bits_equal(la, lb) and na == nb, f"pos {pos}"
        tok = na
    # the cap on the cache length holds
    with pytest.raises(wh.WillametteError):
        a.kv_cache(1025)
    a.close()
    b.close()


def test_gguf_rejections_leave_no_model(ctx):
    """A graph error is reported before any device memory is taken; the
    context stays usable."""
    hm = bs.make_host_model(GQA, seed=1)
    ts = [t for t in bs.gguf_tensors(hm) if t[0] != "blk.2.ffn_down.weight"]
    gf = wh.GgufFile.parse(b"".join(bs.gguf_image(ts, bs.gguf_metadata(GQA))))
    with pytest.raises(wh.WillametteError) as ei:
        bs.DeviceModel.from_gguf(ctx, gf)
    assert ei.value.kind == "MissingMetadata" and "blk.2.ffn_down.weight" in str(ei.value)
    # a corrupt I2_S scale (NaN) is caught by the upload's finiteness check
    ts = bs.gguf_tensors(hm)
    bad = []
    for n, s, t, d in ts:
        if n == "blk.0.attn_v.weight":
            d = d[:-32] + np.float32(np.nan).tobytes() + d[-28:]
        bad.append((n, s, t, d))
    gf = wh.GgufFile.parse(b"".join(bs.gguf_image(bad, bs.gguf_metadata(GQA))))
    with pytest.raises(wh.WillametteError) as ei:
        bs.DeviceModel.from_gguf(ctx, gf)
    assert ei.value.kind == "NonFinite"
    ok = bs.DeviceModel.from_gguf(ctx, wh.GgufFile.parse(bs.gguf_bytes(hm)))
    ok.close()
