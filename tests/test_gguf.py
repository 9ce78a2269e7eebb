"""GGUF reader, qwen35 loaders and writer (yuuka_amd/gguf.py) against the
cases of gguf/reader_test.go (valid files, nested metadata arrays, every
malformed file it rejects, split shards) and model/qwen35/load.go (tensor
names, shapes, dtypes, tied output). Files are written here: by the module's
writer, or, for malformed files, by a raw encoder with explicit offsets."""
from __future__ import annotations

import struct
from dataclasses import replace

import numpy as np
import pytest

from yuuka_amd import gguf as G
from yuuka_amd import model as Mdl


def _raw(version=3, meta=(), tensors=(), data=b"", align=32):
    """Header + directory + data with explicit tensor offsets (relative to the
    aligned data start). meta: (key, type, packed value bytes); tensors:
    (name, dims, dtype, offset)."""
    out = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(meta))]
    for k, t, vb in meta:
        kb = k.encode()
        out.append(struct.pack("<Q", len(kb)) + kb + struct.pack("<I", t) + vb)
    for name, dims, dtype, off in tensors:
        nb = name.encode()
        out.append(struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims)) +
                   b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", dtype, off))
    head = b"".join(out)
    pad = (-len(head)) % align
    return head + b"\0" * pad + data


def _u32(v):
    return struct.pack("<I", v)


def _write_raw(tmp_path, raw, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(raw)
    return str(p)


def test_valid_file_metadata_and_tensors(tmp_path):
    """reader_test.go TestReaderValidF32: header, every metadata type, tensor
    bytes and GGML shapes (dims[0] is the row width), alignment 64."""
    rng = np.random.default_rng(0)
    f32 = rng.normal(size=(3, 8)).astype(np.float32)
    f16 = rng.normal(size=(2, 32)).astype(np.float16)
    q4 = rng.integers(0, 256, 2 * 144, dtype=np.uint8)
    q6 = rng.integers(0, 256, 3 * 210, dtype=np.uint8)
    meta = {"general.architecture": G.Value(G.STRING, "test"), "a.u8": G.Value(G.U8, 7),
            "a.i8": G.Value(G.I8, -7), "a.u16": G.Value(G.U16, 700), "a.i16": G.Value(G.I16, -700),
            "a.u32": G.Value(G.U32, 70000), "a.i32": G.Value(G.I32, -70000), "a.f32": G.Value(G.F32V, 0.5),
            "a.bool": G.Value(G.BOOL, True), "a.u64": G.Value(G.U64, 1 << 40), "a.i64": G.Value(G.I64, -(1 << 40)),
            "a.f64": G.Value(G.F64V, 1e-300),
            "a.strs": G.Value(G.ARRAY, [G.Value(G.STRING, s) for s in ("x", "yy", "")], G.STRING)}
    path = str(tmp_path / "v.gguf")
    G.write(path, meta, [("w", (8, 3), G.F32, f32.view(np.uint8)), ("h", (32, 2), G.F16, f16.view(np.uint8)),
                         ("q4", (256, 2), G.Q4_K, q4), ("q6", (768,), G.Q6_K, q6)], alignment=64)
    with G.Reader(path) as r:
        assert r.version == 3 and r.alignment == 64
        assert r.metadata["a.i8"].as_int() == -7 and r.metadata["a.u64"].as_uint() == 1 << 40
        assert r.metadata["a.f32"].as_float() == 0.5 and r.metadata["a.bool"].value is True
        assert r.metadata["a.f64"].as_float() == 1e-300
        assert r.metadata["a.strs"].as_strs() == ["x", "yy", ""]
        assert r.get_str("general.architecture") == "test"
        assert [t.name for t in r.order] == ["w", "h", "q4", "q6"]
        w = r.tensors["w"]
        assert w.dims == (8, 3) and w.rows == 3 and w.cols == 8 and w.nbytes == 96
        assert np.array_equal(w.data().view(np.float32).reshape(3, 8), f32)
        assert np.array_equal(r.tensors["h"].data().view(np.float16).reshape(2, 32), f16)
        assert np.array_equal(r.tensors["q4"].data(), q4) and np.array_equal(r.tensors["q6"].data(), q6)
        for t in r.order:
            assert t.offset % 64 == 0
        with pytest.raises(G.GGUFInvalidModel):
            r.get_int("a.missing")
        with pytest.raises(G.GGUFInvalidModel):
            r.get_int("a.f32")
        assert r.metadata["a.i32"].as_int() == -70000
        with pytest.raises(G.GGUFError):
            r.metadata["a.i32"].as_uint()  # negative


def test_nested_metadata_array(tmp_path):
    """reader_test.go TestReaderNestedMetadataArray: an array of arrays."""
    inner = [G.Value(G.ARRAY, [G.Value(G.I32, i), G.Value(G.I32, -i)], G.I32) for i in range(3)]
    path = str(tmp_path / "n.gguf")
    G.write(path, {"nest": G.Value(G.ARRAY, inner, G.ARRAY)}, [])
    with G.Reader(path) as r:
        v = r.metadata["nest"]
        assert v.elem_type == G.ARRAY and [x.as_ints() for x in v.value] == [[0, 0], [1, -1], [2, -2]]


MALFORMED = [
    ("bad magic", lambda: b"XGUF" + _raw()[4:], G.GGUFMalformed),
    ("truncated header", lambda: _raw()[:8], G.GGUFMalformed),
    ("unsupported version", lambda: _raw(version=1), G.GGUFUnsupported),
    ("tensor rank exceeds limit", lambda: _raw(tensors=[("w", [1] * 9, G.F32, 0)], data=bytes(64)), G.GGUFMalformed),
    ("unknown metadata type", lambda: _raw(meta=[("a", 99, _u32(1))]), G.GGUFMalformed),
    ("duplicate metadata", lambda: _raw(meta=[("a", G.U32, _u32(1)), ("a", G.U32, _u32(2))]), G.GGUFMalformed),
    ("duplicate tensor", lambda: _raw(tensors=[("w", [2], G.F32, 0), ("w", [2], G.F32, 32)], data=bytes(64)),
     G.GGUFMalformed),
    ("zero dimension", lambda: _raw(tensors=[("w", [0], G.F32, 0)]), G.GGUFMalformed),
    ("quant width not divisible", lambda: _raw(tensors=[("w", [31, 2], G.Q8_0, 0)], data=bytes(128)),
     G.GGUFMalformed),
    ("range outside file", lambda: _raw(tensors=[("w", [2], G.F32, 1 << 20)], data=bytes(32)), G.GGUFMalformed),
    ("unaligned tensor offset", lambda: _raw(tensors=[("w", [2], G.F32, 8)], data=bytes(64)), G.GGUFMalformed),
    ("overlapping tensors", lambda: _raw(tensors=[("a", [4], G.F32, 0), ("b", [4], G.F32, 0)], data=bytes(32)),
     G.GGUFMalformed),
    ("alignment not a power of two", lambda: _raw(meta=[("general.alignment", G.U32, _u32(24))]), G.GGUFMalformed),
    ("unknown dtype", lambda: _raw(tensors=[("w", [2], 99, 0)], data=bytes(32)), G.GGUFUnsupported),
    ("bool out of range", lambda: _raw(meta=[("b", G.BOOL, b"\x02")]), G.GGUFMalformed),
    ("empty file", lambda: b"", G.GGUFMalformed),
]


@pytest.mark.parametrize("name,make,err", MALFORMED, ids=[m[0] for m in MALFORMED])
def test_rejects_malformed(tmp_path, name, make, err):
    """reader_test.go TestReaderRejectsMalformed (plus alignment, dtype,
    bool and empty-file cases): each raises the reference's error class."""
    path = _write_raw(tmp_path, make())
    with pytest.raises(err):
        G.Reader(path)


def _shard(tmp_path, i, n, tensors, name="model"):
    path = str(tmp_path / f"{name}-{i + 1:05d}-of-{n:05d}.gguf")
    G.write(path, {"split.no": G.Value(G.U16, i), "split.count": G.Value(G.U16, n)}, tensors)
    return path


def test_split_shards(tmp_path):
    """reader_test.go TestReaderSplitShards: tensors of every shard by name,
    each read from its own file."""
    a = np.arange(8, dtype=np.float32)
    b = np.arange(16, dtype=np.float32) * 2
    p0 = _shard(tmp_path, 0, 2, [("a", (8,), G.F32, a.view(np.uint8))])
    _shard(tmp_path, 1, 2, [("b", (16,), G.F32, b.view(np.uint8))])
    with G.Reader(p0) as r:
        assert r.tensors["a"].shard == 0 and r.tensors["b"].shard == 1
        assert np.array_equal(r.tensors["b"].data().view(np.float32), b)


def test_split_shard_errors(tmp_path):
    """reader_test.go TestReaderRejectsMissingShard, ...DuplicateShardTensor,
    ...SplitCountMismatch."""
    a = np.zeros(8, np.float32).view(np.uint8)
    d1 = tmp_path / "missing"
    d1.mkdir()
    with pytest.raises(G.GGUFError):
        G.Reader(_shard(d1, 0, 2, [("a", (8,), G.F32, a)]))
    d2 = tmp_path / "dup"
    d2.mkdir()
    p = _shard(d2, 0, 2, [("a", (8,), G.F32, a)])
    _shard(d2, 1, 2, [("a", (8,), G.F32, a)])
    with pytest.raises(G.GGUFMalformed):
        G.Reader(p)
    d3 = tmp_path / "count"
    d3.mkdir()
    p = str(d3 / "model-00001-of-00003.gguf")
    G.write(p, {"split.no": G.Value(G.U16, 0), "split.count": G.Value(G.U16, 2)}, [("a", (8,), G.F32, a)])
    with pytest.raises(G.GGUFMalformed):
        G.Reader(p)


def _same_weights(w, v):
    def same(x, y):
        if isinstance(x, dict):
            assert (x["rows"], x["cols"], x["dtype"]) == (y["rows"], y["cols"], y["dtype"])
            assert np.array_equal(np.asarray(x["data"]).view(np.uint8), np.asarray(y["data"]).view(np.uint8))
        else:
            assert np.array_equal(np.asarray(x, np.float32), np.asarray(y, np.float32))
    for k in ("embedding", "output", "output_norm"):
        same(w[k], v[k])
    assert len(w["layers"]) == len(v["layers"])
    for L, M in zip(w["layers"], v["layers"]):
        assert set(L) == set(M)
        for k in L:
            same(L[k], M[k])


@pytest.mark.parametrize("which", ["dense", "moe"])
def test_qwen35_round_trip(tmp_path, which):
    """model/qwen35/config.go LoadConfig and load.go Load on a file written by
    write_q35: the same configuration and byte-identical weights (views of the
    mapping) as the model written."""
    cfg = replace(Mdl.TINY if which == "dense" else Mdl.TINY_MOE, n_layers=4)
    w = Mdl.make_weights(cfg, seed=3)
    path = str(tmp_path / f"{which}.gguf")
    G.write_q35(path, cfg, w)
    with G.Reader(path) as r:
        got = G.load_config(r, capacity=cfg.capacity)
        assert got == replace(cfg, eps=float(np.float32(cfg.eps)))
        v = G.load_weights(r, got)
        _same_weights(w, v)
        del v


def test_qwen35_tied_output_and_vocab_from_tokens(tmp_path):
    """load.go:93-102: without output.weight the LM head is the token
    embedding; config.go:158-166: the vocabulary size comes from
    tokenizer.ggml.tokens when present."""
    cfg = Mdl.TINY
    w = Mdl.make_weights(cfg, seed=4)
    path = str(tmp_path / "tied.gguf")
    G.write_q35(path, cfg, w, tie_output=True)
    with G.Reader(path) as r:
        v = G.load_weights(r, G.load_config(r))
        assert v["output"] is v["embedding"]
        assert np.array_equal(np.asarray(v["output"]["data"]), np.asarray(w["embedding"]["data"]))
        del v
    # vocabulary from the token list (the writer's vocab_size key removed)
    with G.Reader(path) as r:
        meta = dict(r.metadata)
        ts = [(t.name, t.dims, t.dtype, np.array(t.data())) for t in r.order]
    del meta["qwen35.vocab_size"]
    meta["tokenizer.ggml.tokens"] = G.Value(G.ARRAY, [G.Value(G.STRING, f"t{i}") for i in range(cfg.vocab)], G.STRING)
    p2 = str(tmp_path / "tokens.gguf")
    G.write(p2, meta, ts)
    with G.Reader(p2) as r:
        assert G.load_config(r).vocab == cfg.vocab


def test_qwen35_loader_rejects_bad_models(tmp_path):
    """load.go loadMatrix / loadVector / loadF32 and config.go validate: a
    wrong shape, a missing tensor, a non-F32 vector, an unexecutable matrix
    dtype and a wrong architecture are errors."""
    cfg = Mdl.TINY
    w = Mdl.make_weights(cfg, seed=5)
    path = str(tmp_path / "ok.gguf")
    G.write_q35(path, cfg, w)
    with G.Reader(path) as r:
        meta = dict(r.metadata)
        ts = [(t.name, t.dims, t.dtype, np.array(t.data())) for t in r.order]

    def variant(name, fix_meta=None, fix_ts=None):
        m, t = dict(meta), list(ts)
        if fix_meta:
            fix_meta(m)
        if fix_ts:
            t = fix_ts(t)
        p = str(tmp_path / name)
        G.write(p, m, t)
        return p

    def swap(name, dims=None, dtype=None, data=None):
        def f(t):
            return [(n, dims or d, dt if dtype is None else dtype, data if (data is not None and n == name) else b)
                    if n == name else (n, d, dt, b) for n, d, dt, b in t]
        return f

    cases = [
        (variant("shape.gguf", fix_ts=swap("blk.0.attn_qkv.weight", dims=(cfg.hidden, cfg.conv_dim // 2),
                                           data=np.zeros(cfg.conv_dim // 2 * cfg.hidden // 256 * 144, np.uint8))),
         G.GGUFInvalidModel),
        (variant("missing.gguf", fix_ts=lambda t: [x for x in t if x[0] != "blk.3.ffn_down.weight"]), G.GGUFInvalidModel),
        (variant("vecdtype.gguf", fix_ts=swap("output_norm.weight", dims=(cfg.hidden,), dtype=G.F16,
                                              data=np.zeros(cfg.hidden, np.float16).view(np.uint8))),
         G.GGUFInvalidModel),
        (variant("q8.gguf", fix_ts=swap("blk.0.ssm_beta.weight", dims=(cfg.hidden, cfg.rank), dtype=G.Q8_0,
                                        data=np.zeros(cfg.rank * cfg.hidden // 32 * 34, np.uint8))),
         G.GGUFUnsupported),
        (variant("arch.gguf", fix_meta=lambda m: m.update({"general.architecture": G.Value(G.STRING, "llama")})),
         G.GGUFInvalidModel),
        (variant("heads.gguf", fix_meta=lambda m: m.update({"qwen35.attention.head_count_kv": G.Value(G.U32, 3)})),
         G.GGUFInvalidModel),
    ]
    for p, err in cases:
        with G.Reader(p) as r:
            with pytest.raises(err):
                G.load_weights(r, G.load_config(r))
