"""GGUF ingestion (ts_model::load_backend, src/common/ts_model.cpp:13-41):
the library's reader against fixtures written by tests/gguf_writer.py, and
the DiT / T5 loaders against the same weights set tensor by tensor.
The reader tests are host-only; the loader tests run the drivers on the GPU."""
import numpy as np
import pytest

import gguf_writer as gw


@pytest.fixture(scope="module")
def tsk():
    from __graft_entry__ import ensure_built, load_tsk
    ensure_built()
    return load_tsk()


def q8_blocks(rng, rows, K, d=0.01):
    qs = rng.integers(-127, 128, size=(rows, K // 32, 32), dtype=np.int8)
    dh = np.full((rows, K // 32, 1), np.float16(d)).view(np.uint8)
    return np.ascontiguousarray(np.concatenate([dh, qs.view(np.uint8)], axis=2))


def test_reader_types_and_metadata(tsk, tmp_path, orc):
    rng = np.random.default_rng(3)
    a32 = rng.standard_normal((5, 64)).astype(np.float32)
    v32 = rng.standard_normal(7).astype(np.float32)
    a16 = rng.standard_normal((3, 32)).astype(np.float16)
    bfb = orc.f32_to_bf16_bits(rng.standard_normal((4, 40)).astype(np.float32))
    q8 = q8_blocks(rng, 6, 96)
    path = tmp_path / "t.gguf"
    gw.write_gguf(path, {"dit.hidden_dim": (gw.U32, 1024), "dit.rope_theta": (gw.F32, 10000.0),
                         "general.name": (gw.STRING, "fixture"), "x.flag": (gw.BOOL, True)},
                  [gw.f32_tensor("a32", a32), gw.f32_tensor("v32", v32), gw.f16_tensor("a16", a16),
                   gw.bf16_tensor("abf", bfb), gw.q8_0_tensor("q8", q8, 96)])
    g = tsk.Gguf(path)
    names = {n: (ne, t) for n, ne, t in g.tensors()}
    assert names["a32"] == ((64, 5, 1, 1), 0) and names["v32"] == ((7, 1, 1, 1), 0)
    assert names["a16"] == ((32, 3, 1, 1), 1) and names["abf"] == ((40, 4, 1, 1), 30)
    assert names["q8"] == ((96, 6, 1, 1), 8)
    np.testing.assert_array_equal(g.read("a32"), a32)
    np.testing.assert_array_equal(g.read("v32"), v32)
    np.testing.assert_array_equal(g.read("a16"), a16.astype(np.float32))
    np.testing.assert_array_equal(g.read("abf"), orc.bf16_bits_to_f32(bfb))
    np.testing.assert_array_equal(g.read("q8"), orc.dequantize_q8_0(q8).reshape(6, 96))
    assert g.read("q8", as_f32=False).tobytes() == q8.tobytes()
    assert g.u32("dit.hidden_dim") == 1024 and g.f32("dit.rope_theta") == 10000.0
    assert g.str("general.name") == "fixture" and g.u32("x.flag") == 1
    c = g.dit_config()
    assert c.hidden == 1024 and c.rope_theta == 10000.0
    with pytest.raises(tsk.TskError):
        g.read("missing")
    with pytest.raises(tsk.TskError):
        g.u32("general.name")
    g.close()


def test_reader_rejects_bad_files(tsk, tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + b"\0" * 60)
    with pytest.raises(tsk.TskError):
        tsk.Gguf(bad)
    good = tmp_path / "good.gguf"
    gw.write_gguf(good, {}, [gw.f32_tensor("w", np.ones((64, 64), np.float32))])
    raw = good.read_bytes()
    trunc = tmp_path / "trunc.gguf"
    trunc.write_bytes(raw[:-100])                       # tensor data cut short
    with pytest.raises(tsk.TskError):
        tsk.Gguf(trunc)
    head = tmp_path / "head.gguf"
    head.write_bytes(raw[:20])                          # header only
    with pytest.raises(tsk.TskError):
        tsk.Gguf(head)
    with pytest.raises(tsk.TskError):
        tsk.Gguf(tmp_path / "none.gguf")


@pytest.mark.gpu
def test_dit_load_gguf_matches_set_tensor(tsk, tmp_path, orc):
    tsk.init(0)
    cfg = tsk.dit_config(depth=3, fused_depth=1, max_latent=64)
    a, b = tsk.Dit(cfg), tsk.Dit(cfg)
    W = tsk.synthetic_weights(a.tensors(), seed=21)
    tensors = []
    for i, (name, w) in enumerate(W.items()):
        a.set_tensor(name, w)
        if w.ndim == 2 and i % 3 == 0:
            tensors.append(gw.bf16_tensor(name, orc.f32_to_bf16_bits(w)))   # the bf16 GGUF's matrices
        else:
            tensors.append(gw.f32_tensor(name, w))                        # the f32 GGUF
    path = tmp_path / "dit.gguf"
    gw.write_gguf(path, {"dit.depth": (gw.U32, 3), "dit.fused_depth": (gw.U32, 1)}, tensors)
    g = tsk.Gguf(path)
    c2 = g.dit_config(max_latent=64)
    assert c2.depth == 3 and c2.fused_depth == 1
    g.load_into(b)
    rng = np.random.default_rng(5)
    lat = rng.standard_normal((2, 64, 40), dtype=np.float32)     # ne = [T, latent_dim, B]
    txt = rng.standard_normal((2, 77, 1024), dtype=np.float32)
    t = np.array([0.7, 0.7], np.float32)
    np.testing.assert_array_equal(a.forward(lat, t, txt), b.forward(lat, t, txt))
    g.close()
    # a Q8_0 matrix is refused: this driver runs BF16 weights
    qname = next(n for n, w in W.items() if w.ndim == 2 and w.shape[1] % 32 == 0)
    qt = [gw.q8_0_tensor(qname, orc.quantize_q8_0(W[qname]), W[qname].shape[1]) if tt[0] == qname else tt
          for tt in tensors]
    path_q = tmp_path / "dit_q8.gguf"
    gw.write_gguf(path_q, {"dit.depth": (gw.U32, 3), "dit.fused_depth": (gw.U32, 1)}, qt)
    gq = tsk.Gguf(path_q)
    with pytest.raises(tsk.TskError) as ei:
        gq.load_into(b)
    assert ei.value.status == -2
    gq.close()
    a.close()
    b.close()


@pytest.mark.gpu
def test_t5_load_gguf_matches_set_tensor(tsk, tmp_path):
    tsk.init(0)
    cfg = tsk.t5_config(n_layers=1, max_tokens=64)
    a, b = tsk.T5(cfg), tsk.T5(cfg)
    rng = np.random.default_rng(8)
    tensors = []
    for name, ne, ty in a.tensors():
        if ty == 8:
            blk = q8_blocks(rng, ne[1], ne[0], d=1e-3)
            a.set_tensor(name, blk)
            tensors.append(gw.q8_0_tensor(name, blk, ne[0]))
        else:
            v = rng.standard_normal(ne[0] * ne[1]).astype(np.float32).reshape(ne[1], ne[0])
            a.set_tensor(name, v)
            tensors.append(gw.f32_tensor(name, v if ne[1] > 1 else v[0]))
    path = tmp_path / "t5.gguf"
    gw.write_gguf(path, {"t5.n_layers": (gw.U32, 1)}, tensors)
    g = tsk.Gguf(path)
    assert g.t5_config().n_layers == 1
    g.load_into(b)
    x = rng.standard_normal((50, 2048)).astype(np.float32)
    ids = np.arange(1, 51, dtype=np.int32)
    ids[-5:] = 0
    np.testing.assert_array_equal(a.encode(x, ids), b.encode(x, ids))
    g.close()
    a.close()
    b.close()
