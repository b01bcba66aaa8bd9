"""GGUF model files (gnc-x_amd/gguf.py, decode.write_model_gguf / load_model_gguf)
against the layout the reference's loader parses (lua/gncx_gguf.lua:223-306).
CPU only."""
from __future__ import annotations

import struct

import numpy as np

import gguf as G


def _s(text: str) -> bytes:
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def test_known_answer_file(tmp_path):
    """One u32 key, one string array key, one 3-float F32 tensor and one 2-block
    Q8_0 tensor, assembled here byte by byte from the format description."""
    f32 = np.array([1.5, -2.0, 0.25], np.float32)
    q8 = bytes(range(68))
    specs = [G.TensorSpec("a", G.F32, (3,), lambda f: f.write(f32.tobytes())),
             G.TensorSpec("b.weight", G.Q8_0, (32, 2), lambda f: f.write(q8))]
    meta = [("k", G.UINT32, 7), ("toks", G.ARRAY, (G.STRING, ["x", "yz"]))]
    offs = G.write_gguf(tmp_path / "t.gguf", meta, specs)
    head = (b"GGUF" + struct.pack("<IQQ", 3, 2, 2)
            + _s("k") + struct.pack("<II", G.UINT32, 7)
            + _s("toks") + struct.pack("<IIQ", G.ARRAY, G.STRING, 2) + _s("x") + _s("yz")
            + _s("a") + struct.pack("<IQIQ", 1, 3, G.F32, 0)
            + _s("b.weight") + struct.pack("<IQQIQ", 2, 32, 2, G.Q8_0, 32))  # 12 bytes padded to 32
    data0 = (len(head) + 31) // 32 * 32
    want = head + b"\0" * (data0 - len(head)) + f32.tobytes() + b"\0" * 20 + q8 + b"\0" * 28
    got = (tmp_path / "t.gguf").read_bytes()
    assert got == want
    assert offs == {"a": data0, "b.weight": data0 + 32}
    meta_r, tens, d0 = G.read_gguf(got)
    assert d0 == data0 and meta_r["k"] == 7 and meta_r["toks"] == ["x", "yz"] and meta_r["__version__"] == 3
    assert tens["b.weight"].dims == (32, 2) and tens["b.weight"].byte_size == 68
    assert tens["b.weight"].abs_file_offset == data0 + 32 and tens["a"].byte_size == 12


def test_alignment_key_and_all_value_types(tmp_path):
    meta = [("general.alignment", G.UINT32, 64), ("u8", G.UINT8, 200), ("i8", G.INT8, -3), ("u16", G.UINT16, 60000),
            ("i16", G.INT16, -2), ("i32", G.INT32, -7), ("f32", G.FLOAT32, 0.5), ("b", G.BOOL, True),
            ("u64", G.UINT64, 2**40), ("i64", G.INT64, -(2**40)), ("f64", G.FLOAT64, 0.1),
            ("fa", G.ARRAY, (G.FLOAT32, [1.0, 2.0])), ("ia", G.ARRAY, (G.INT32, [-1, 2, 3]))]
    specs = [G.TensorSpec("t", G.F32, (5,), lambda f: f.write(np.arange(5, dtype=np.float32).tobytes()))]
    G.write_gguf(tmp_path / "a.gguf", meta, specs)
    buf = (tmp_path / "a.gguf").read_bytes()
    m, t, d0 = G.read_gguf(buf)
    assert d0 % 64 == 0 and t["t"].abs_file_offset == d0
    for k, _, v in meta:
        got = m[k]
        assert got == (list(v[1]) if isinstance(v, tuple) else v), k
    assert np.array_equal(np.frombuffer(buf[d0:d0 + 20], np.float32), np.arange(5, dtype=np.float32))


def test_model_file_round_trip(tmp_path):
    import gncx_amd.decode as dec
    sh = dec.Qwen3Shape(n_layers=2, embed=256, n_heads=4, n_kv=2, head_dim=64, ffn=512, vocab=600)
    offs = dec.write_model_gguf(tmp_path / "m.gguf", sh, seed=3)
    m = dec.load_model_gguf(tmp_path / "m.gguf")
    assert (m.shape.n_layers, m.shape.embed, m.shape.n_heads, m.shape.n_kv, m.shape.head_dim, m.shape.ffn,
            m.shape.vocab, m.shape.layer_type, m.shape.embd_type) == (2, 256, 4, 2, 64, 512, 600, G.Q4_K, G.Q6_K)
    assert np.float32(m.shape.eps) == np.float32(1e-6) and m.shape.rope_base == 1e6
    assert m.offsets == offs and all(o % 32 == 0 for o in offs.values())
    meta, tens, _ = G.read_gguf(m.blob)
    assert meta["general.architecture"] == "qwen3" and len(meta["tokenizer.ggml.tokens"]) == 600
    # tensors lie inside the file without overlap, each the size its type gives
    spans = sorted((t.abs_file_offset, t.abs_file_offset + t.byte_size) for t in tens.values())
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])) and spans[-1][1] <= m.blob.size
    q = tens["blk.1.ffn_down.weight"]
    assert q.dims == (512, 256) and q.byte_size == 256 * (512 // 256) * 144
    # Q4_K super-block scales are |N(0, 0.02)| halves; Q6_K sub-block scales lie in [-32, 31]
    blk = np.asarray(m.blob[q.abs_file_offset:q.abs_file_offset + q.byte_size]).reshape(-1, 144)
    d = blk[:, 0:4].copy().view(np.float16).astype(np.float32)
    assert (d >= 0).all() and 0.005 < d.mean() < 0.03
    e = tens["token_embd.weight"]
    sc = np.asarray(m.blob[e.abs_file_offset:e.abs_file_offset + e.byte_size]).reshape(-1, 210)[:, 192:208]
    assert sc.view(np.int8).min() >= -32 and sc.view(np.int8).max() <= 31
