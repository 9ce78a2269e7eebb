"""GGUF model files: a validating reader (zero-copy tensor views over a
read-only memory map), the qwen35 / qwen35moe configuration and weight
loaders that produce the engine's weight dictionary (model.make_weights
layout, ready for yuuka_q35_create), and a small writer.

Follows gguf/reader.go (header, metadata, tensor directory, alignment,
shards, range and overlap checks), gguf/metadata.go (value types and
conversions), model/qwen35/config.go:48-178 (LoadConfig) and
model/qwen35/load.go:79-322 (Load: tensor names, shapes and dtypes).
Errors are GGUFMalformed / GGUFUnsupported / GGUFInvalidModel, the
reference's ErrMalformed / ErrUnsupported / ErrInvalidModel.
"""
from __future__ import annotations

import mmap
import os
import re
import struct
from dataclasses import dataclass, field

import numpy as np

MAGIC = b"GGUF"
MIN_VERSION, MAX_VERSION = 2, 3
DEFAULT_ALIGN = 32
MAX_METADATA_KEYS = 1 << 20
MAX_TENSORS = 1 << 24
MAX_STRING_BYTES = 1 << 30
MAX_RANK = 8

# gguf/metadata.go:10-24 value types
U8, I8, U16, I16, U32, I32, F32V, BOOL, STRING, ARRAY, U64, I64, F64V = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32V: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64V: "<d"}
_MIN_SIZE = {U8: 1, I8: 1, BOOL: 1, U16: 2, I16: 2, U32: 4, I32: 4, F32V: 4, U64: 8, I64: 8, F64V: 8,
             STRING: 8, ARRAY: 16}

# tensor/dtype.go:13-35 dtype codes and :102-148 storage blocks (elements, bytes)
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 0, 1, 2, 3, 6, 7, 8, 9
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 10, 11, 12, 13, 14, 15
BLOCKS = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24),
          Q8_0: (32, 34), Q8_1: (32, 40), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144),
          Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292), 16: (256, 66), 17: (256, 74),
          18: (256, 98), 19: (256, 50), 20: (32, 18), 21: (256, 110), 22: (256, 82), 23: (256, 136)}
# dtypes the verify engine executes for 2-D weights (the router is F32)
ENGINE_DTYPES = (F32, Q4_K, Q6_K)


class GGUFError(ValueError):
    pass


class GGUFMalformed(GGUFError):
    pass


class GGUFUnsupported(GGUFError):
    pass


class GGUFInvalidModel(GGUFError):
    pass


@dataclass
class Value:
    """One metadata value (gguf/metadata.go Value): `type`, the element type
    of an array, and the decoded Python value (list of Value for arrays)."""
    type: int
    value: object
    elem_type: int = -1

    def as_uint(self) -> int:
        if self.type in (U8, U16, U32, U64):
            return int(self.value)
        if self.type in (I8, I16, I32, I64):
            if self.value < 0:
                raise GGUFError(f"metadata value {self.value} is negative")
            return int(self.value)
        raise GGUFError(f"metadata type {self.type} is not an integer")

    def as_int(self) -> int:
        if self.type in (I8, I16, I32, I64, U8, U16, U32):
            return int(self.value)
        if self.type == U64:
            if self.value > (1 << 63) - 1:
                raise GGUFError(f"metadata value {self.value} overflows int64")
            return int(self.value)
        raise GGUFError(f"metadata type {self.type} is not an integer")

    def as_float(self) -> float:
        if self.type in (F32V, F64V):
            return float(self.value)
        raise GGUFError(f"metadata type {self.type} is not a float")

    def as_str(self) -> str:
        if self.type != STRING:
            raise GGUFError(f"metadata type {self.type} is not a string")
        return self.value

    def as_ints(self) -> list:
        if self.type != ARRAY:
            raise GGUFError(f"metadata type {self.type} is not an array")
        return [v.as_int() for v in self.value]

    def as_strs(self) -> list:
        if self.type != ARRAY or self.elem_type != STRING:
            raise GGUFError("metadata value is not a string array")
        return [v.value for v in self.value]


@dataclass
class Tensor:
    """One tensor of the directory (gguf/reader.go Tensor): GGML dimension
    order (dims[0] is the contiguous row width)."""
    name: str
    dims: tuple
    dtype: int
    offset: int          # relative to its shard's data section
    nbytes: int
    shard: int = 0
    absolute: int = 0    # absolute file offset in its shard
    _reader: object = field(default=None, repr=False)

    @property
    def rows(self) -> int:
        r = 1
        for d in self.dims[1:]:
            r *= d
        return r

    @property
    def cols(self) -> int:
        return self.dims[0]

    def data(self) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view of the mapping."""
        return self._reader._view(self)


class _Cursor:
    def __init__(self, path, buf):
        self.path, self.buf, self.off = path, buf, 0

    def need(self, n):
        if n < 0 or self.off + n > len(self.buf):
            raise GGUFMalformed(f"{self.path}: unexpected end of file at byte {self.off}")

    def unpack(self, fmt):
        n = struct.calcsize(fmt)
        self.need(n)
        v = struct.unpack_from(fmt, self.buf, self.off)[0]
        self.off += n
        return v

    def raw(self, n):
        self.need(n)
        v = bytes(self.buf[self.off:self.off + n])
        self.off += n
        return v

    def str(self):
        n = self.unpack("<Q")
        if n > MAX_STRING_BYTES:
            raise GGUFMalformed(f"{self.path}: string length {n} exceeds limit")
        try:
            return self.raw(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GGUFMalformed(f"{self.path}: string is not UTF-8: {e}") from None


def _read_value(c: _Cursor, typ: int, depth: int) -> Value:
    """gguf/reader.go readRawValue."""
    if depth > 4:
        raise GGUFMalformed(f"{c.path}: metadata nesting exceeds limit")
    if typ in _SCALAR:
        v = c.unpack(_SCALAR[typ])
        if typ == BOOL:
            if v > 1:
                raise GGUFMalformed(f"{c.path}: invalid bool value {v}")
            v = bool(v)
        return Value(typ, v)
    if typ == STRING:
        return Value(typ, c.str())
    if typ == ARRAY:
        et = c.unpack("<I")
        count = c.unpack("<Q")
        if et not in _MIN_SIZE:
            raise GGUFMalformed(f"{c.path}: unknown array element type {et}")
        if et != STRING and count > (len(c.buf) - c.off) // _MIN_SIZE[et]:
            raise GGUFMalformed(f"{c.path}: array length {count} exceeds remaining bytes")
        if count > 1 << 31:
            raise GGUFMalformed(f"{c.path}: array length {count} exceeds limit")
        items = []
        for i in range(count):
            if et == ARRAY:  # a nested array repeats its own type tag, which must be an array
                tag = c.unpack("<I")
                if tag != ARRAY:
                    raise GGUFMalformed(f"{c.path}: array element {i} has type {tag}, not array")
                item = _read_value(c, tag, depth + 1)
            else:
                item = _read_value(c, et, depth + 1)
            items.append(item)
        return Value(ARRAY, items, et)
    raise GGUFMalformed(f"{c.path}: unknown metadata type {typ}")


def _align_up(v, a):
    return v if a <= 1 or v % a == 0 else v + (a - v % a)


@dataclass
class _FileMeta:
    version: int
    alignment: int
    metadata: dict
    tensors: list
    data_start: int


def _parse(path, buf) -> _FileMeta:
    """gguf/reader.go parseFile: header, metadata, tensor directory."""
    c = _Cursor(path, buf)
    if c.raw(4) != MAGIC:
        raise GGUFMalformed(f"{path}: bad magic")
    version = c.unpack("<I")
    if not MIN_VERSION <= version <= MAX_VERSION:
        raise GGUFUnsupported(f"{path}: version {version} is not supported (want {MIN_VERSION}..{MAX_VERSION})")
    n_tensors = c.unpack("<Q")
    n_meta = c.unpack("<Q")
    if n_tensors > MAX_TENSORS:
        raise GGUFMalformed(f"{path}: tensor count {n_tensors} exceeds limit")
    if n_meta > MAX_METADATA_KEYS:
        raise GGUFMalformed(f"{path}: metadata count {n_meta} exceeds limit")
    meta = {}
    for _ in range(n_meta):
        key = c.str()
        if not key:
            raise GGUFMalformed(f"{path}: empty metadata key")
        if key in meta:
            raise GGUFMalformed(f"{path}: duplicate metadata key {key!r}")
        meta[key] = _read_value(c, c.unpack("<I"), 0)
    align = DEFAULT_ALIGN
    if "general.alignment" in meta:
        try:
            align = meta["general.alignment"].as_uint()
        except GGUFError as e:
            raise GGUFMalformed(f"{path}: general.alignment: {e}") from None
        if align == 0 or align > 1 << 20 or align & (align - 1):
            raise GGUFMalformed(f"{path}: general.alignment {align} is not a power of two")
    tensors, seen = [], set()
    for _ in range(n_tensors):
        name = c.str()
        if not name:
            raise GGUFMalformed(f"{path}: empty tensor name")
        if name in seen:
            raise GGUFMalformed(f"{path}: duplicate tensor name {name!r}")
        seen.add(name)
        rank = c.unpack("<I")
        if rank == 0 or rank > MAX_RANK:
            raise GGUFMalformed(f"{path}: tensor {name!r} has invalid rank {rank}")
        dims, elements = [], 1
        for _ in range(rank):
            d = c.unpack("<Q")
            if d == 0:
                raise GGUFMalformed(f"{path}: tensor {name!r} has zero dimension")
            if elements > ((1 << 64) - 1) // d:
                raise GGUFMalformed(f"{path}: tensor {name!r} element count overflows")
            elements *= d
            dims.append(d)
        dtype = c.unpack("<I")
        offset = c.unpack("<Q")
        if dtype not in BLOCKS:
            raise GGUFUnsupported(f"{path}: tensor {name!r}: unsupported dtype {dtype}")
        be, bb = BLOCKS[dtype]
        if be > 1 and dims[0] % be:
            raise GGUFMalformed(f"{path}: tensor {name!r} row width {dims[0]} is not a multiple of {be}")
        tensors.append(Tensor(name, tuple(dims), dtype, offset, elements // be * bb))
    data_start = _align_up(c.off, align)
    if data_start > len(buf):
        if n_tensors:
            raise GGUFMalformed(f"{path}: tensor data starts beyond end of file")
        data_start = len(buf)
    return _FileMeta(version, align, meta, tensors, data_start)


_SPLIT = re.compile(r"^(.*)-([0-9]{5})-of-([0-9]{5})\.gguf$")


class Reader:
    """A validated GGUF model (gguf/reader.go Open): every shard mapped
    read-only, tensor byte ranges inside their shard, aligned and disjoint."""

    def __init__(self, path: str):
        self.path = os.path.abspath(path)
        self._maps = []
        try:
            buf = self._map(self.path)
            meta = _parse(self.path, buf)
            self.version, self.alignment, self.metadata = meta.version, meta.alignment, meta.metadata
            count = 1
            if "split.count" in meta.metadata:
                try:
                    count = meta.metadata["split.count"].as_uint()
                except GGUFError as e:
                    raise GGUFMalformed(f"{self.path}: split.count: {e}") from None
                if count == 0 or count > 1 << 20:
                    raise GGUFMalformed(f"{self.path}: invalid split.count {count}")
            paths = [self.path] if count == 1 else self._split_paths(count)
            self.tensors, self.order = {}, []
            for i, p in enumerate(paths):
                if i == 0:
                    sbuf, smeta = buf, meta
                else:
                    sbuf = self._map(p)
                    smeta = _parse(p, sbuf)
                if smeta.version != meta.version or smeta.alignment != meta.alignment:
                    raise GGUFMalformed(f"split shard {i} header differs from shard 0")
                if count > 1:
                    no, cnt = smeta.metadata.get("split.no"), smeta.metadata.get("split.count")
                    if no is None or no.as_uint() != i:
                        raise GGUFMalformed(f"split shard {i} has no matching split.no")
                    if cnt is None or cnt.as_uint() != count:
                        raise GGUFMalformed(f"split shard {i} has split.count != {count}")
                for t in smeta.tensors:
                    if t.name in self.tensors:
                        raise GGUFMalformed(f"tensor {t.name!r} appears in more than one shard")
                    if t.offset % meta.alignment:
                        raise GGUFMalformed(f"tensor {t.name!r} offset {t.offset} is not aligned to "
                                            f"{meta.alignment}")
                    t.absolute = smeta.data_start + t.offset
                    if t.absolute + t.nbytes > len(sbuf):
                        raise GGUFMalformed(f"tensor {t.name!r} range [{t.absolute},{t.absolute + t.nbytes}) "
                                            f"exceeds shard size {len(sbuf)}")
                    t.shard, t._reader = i, self
                    self.tensors[t.name] = t
                    self.order.append(t)
            self._check_overlaps()
        except BaseException:
            self.close()
            raise

    def _map(self, p):
        try:
            f = open(p, "rb")
        except OSError as e:
            raise GGUFError(f"open {p}: {e}") from None
        with f:
            size = os.fstat(f.fileno()).st_size
            if size <= 0:
                raise GGUFMalformed(f"{p}: empty file")
            m = mmap.mmap(f.fileno(), size, access=mmap.ACCESS_READ)
        self._maps.append(m)
        return m

    def _split_paths(self, count):
        mt = _SPLIT.match(self.path)
        if not mt:
            raise GGUFMalformed(f"split model path {self.path!r} does not use -NNNNN-of-NNNNN.gguf")
        if int(mt.group(3)) != count:
            raise GGUFMalformed(f"split count {count} does not match file name")
        return [f"{mt.group(1)}-{i + 1:05d}-of-{count:05d}.gguf" for i in range(count)]

    def _check_overlaps(self):
        by_shard = {}
        for t in self.order:
            by_shard.setdefault(t.shard, []).append((t.absolute, t.absolute + t.nbytes, t.name))
        for s, spans in by_shard.items():
            spans.sort()
            for a, b in zip(spans, spans[1:]):
                if b[0] < a[1]:
                    raise GGUFMalformed(f"shard {s}: tensors {a[2]!r} and {b[2]!r} overlap")

    def _view(self, t: Tensor) -> np.ndarray:
        return np.frombuffer(self._maps[t.shard], dtype=np.uint8, count=t.nbytes, offset=t.absolute)

    def close(self):
        for m in self._maps:
            try:
                m.close()
            except BufferError:  # a numpy view still references the mapping; it closes when freed
                pass
        self._maps = []

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- metadata accessors (gguf/reader.go String / Uint / Int / Float)
    def _get(self, key) -> Value:
        if key not in self.metadata:
            raise GGUFInvalidModel(f"missing metadata key {key!r}")
        return self.metadata[key]

    def get_str(self, key):
        try:
            return self._get(key).as_str()
        except GGUFInvalidModel:
            raise
        except GGUFError as e:
            raise GGUFInvalidModel(f"{key!r}: {e}") from None

    def get_int(self, key):
        try:
            return self._get(key).as_int()
        except GGUFInvalidModel:
            raise
        except GGUFError as e:
            raise GGUFInvalidModel(f"{key!r}: {e}") from None

    def get_float(self, key):
        try:
            return self._get(key).as_float()
        except GGUFInvalidModel:
            raise
        except GGUFError as e:
            raise GGUFInvalidModel(f"{key!r}: {e}") from None


# ------------------------------------------------------------- qwen35 loader

ARCH, MOE_ARCH = "qwen35", "qwen35moe"


def load_config(r: Reader, **session):
    """model/qwen35/config.go:48-178 LoadConfig, as a model.Q35Config (the
    keyword arguments set the session geometry: capacity, max_rows, ...)."""
    from .model import Q35Config
    arch = r.get_str("general.architecture")
    if arch not in (ARCH, MOE_ARCH):
        raise GGUFInvalidModel(f"model architecture {arch!r} is not {ARCH!r} or {MOE_ARCH!r}")
    sc = r.metadata.get(arch + ".rope.scaling.type")
    if sc is not None and sc.as_str().strip().lower() not in ("", "none", "default"):
        raise GGUFInvalidModel(f"{arch}.rope.scaling.type {sc.as_str()!r} is not supported")

    def ikey(name):
        v = r.get_int(f"{arch}.{name}")
        if v <= 0 or v > 1 << 31:
            raise GGUFInvalidModel(f"metadata {arch}.{name} has invalid value {v}")
        return v

    kw = dict(n_layers=ikey("block_count"), hidden=ikey("embedding_length"), heads=ikey("attention.head_count"),
              kv_heads=ikey("attention.head_count_kv"), head_dim=ikey("attention.key_length"),
              rope_dim=ikey("rope.dimension_count"), rope_base=r.get_float(f"{arch}.rope.freq_base"),
              eps=float(np.float32(r.get_float(f"{arch}.attention.layer_norm_rms_epsilon"))),
              conv_kernel=ikey("ssm.conv_kernel"), state_size=ikey("ssm.state_size"),
              groups=ikey("ssm.group_count"), rank=ikey("ssm.time_step_rank"),
              full_interval=ikey("full_attention_interval"))
    ikey("context_length")
    value_dim = ikey("attention.value_length")
    inner = ikey("ssm.inner_size")
    if arch == MOE_ARCH:
        kw.update(ffn=0, n_experts=ikey("expert_count"), n_experts_used=ikey("expert_used_count"))
        ef = r._get(f"{arch}.expert_feed_forward_length")
        if ef.type == ARRAY:
            widths = ef.as_ints()
            if not widths or any(w != widths[0] for w in widths):
                raise GGUFInvalidModel(f"{arch}.expert_feed_forward_length is empty or varies by layer")
            kw["expert_ffn"] = widths[0]
        else:
            kw["expert_ffn"] = ef.as_int()
        key = f"{arch}.expert_shared_feed_forward_length"
        kw["shared_ffn"] = ikey("expert_shared_feed_forward_length") if key in r.metadata else kw["expert_ffn"]
    else:
        kw["ffn"] = ikey("feed_forward_length")
    if "tokenizer.ggml.tokens" in r.metadata:
        kw["vocab"] = len(r.metadata["tokenizer.ggml.tokens"].as_strs())
    else:
        try:
            kw["vocab"] = ikey("vocab_size")
        except GGUFInvalidModel:
            raise GGUFInvalidModel("vocabulary size is unavailable") from None
    # config.go validate(): the checks this engine relies on
    if kw["heads"] % kw["kv_heads"]:
        raise GGUFInvalidModel(f"head count {kw['heads']} is not a multiple of KV head count {kw['kv_heads']}")
    if value_dim != kw["head_dim"]:
        raise GGUFInvalidModel(f"key head dim {kw['head_dim']} differs from value head dim {value_dim}")
    if kw["rope_dim"] % 2 or kw["rope_dim"] > kw["head_dim"]:
        raise GGUFInvalidModel(f"rope dimension {kw['rope_dim']} is invalid for head dim {kw['head_dim']}")
    if inner != kw["rank"] * kw["state_size"]:
        raise GGUFInvalidModel(f"ssm inner size {inner} is not time_step_rank x state_size")
    kw.update(session)
    return Q35Config(**kw)


def _matrix(r: Reader, name, rows, cols):
    """load.go loadMatrix: rank 2, GGML shape [cols, rows], an executable dtype."""
    t = r.tensors.get(name)
    if t is None:
        raise GGUFInvalidModel(f"missing required tensor {name!r}")
    if len(t.dims) != 2:
        raise GGUFInvalidModel(f"tensor {name!r} has rank {len(t.dims)}, want 2")
    if t.dims != (cols, rows):
        raise GGUFInvalidModel(f"tensor {name!r} has shape {list(t.dims)}, want [{cols}, {rows}]")
    if t.dtype not in ENGINE_DTYPES:
        raise GGUFUnsupported(f"tensor {name!r} uses dtype {t.dtype}, which the verify engine does not execute")
    return dict(data=t.data(), rows=rows, cols=cols, dtype=t.dtype)


def _experts(r: Reader, name, rows, cols, experts):
    """load.go loadExperts: rank 3 [cols, rows, experts], one expert's rows
    contiguous (exposed as an experts*rows x cols matrix)."""
    t = r.tensors.get(name)
    if t is None:
        raise GGUFInvalidModel(f"missing required tensor {name!r}")
    if t.dims != (cols, rows, experts):
        raise GGUFInvalidModel(f"tensor {name!r} has shape {list(t.dims)}, want [{cols}, {rows}, {experts}]")
    if t.dtype not in ENGINE_DTYPES:
        raise GGUFUnsupported(f"tensor {name!r} uses dtype {t.dtype}, which the verify engine does not execute")
    return dict(data=t.data(), rows=experts * rows, cols=cols, dtype=t.dtype)


def _f32(r: Reader, name, count, vector=True):
    """load.go loadVector / loadF32: F32 data of `count` elements."""
    t = r.tensors.get(name)
    if t is None:
        raise GGUFInvalidModel(f"missing required tensor {name!r}")
    if vector and t.dims != (count,):
        raise GGUFInvalidModel(f"tensor {name!r} has shape {list(t.dims)}, want [{count}]")
    if t.dtype != F32:
        raise GGUFInvalidModel(f"tensor {name!r} uses dtype {t.dtype}, want F32")
    if t.nbytes != count * 4:
        raise GGUFInvalidModel(f"tensor {name!r} has {t.nbytes} bytes, want {count * 4}")
    return t.data().view(np.float32)


def load_weights(r: Reader, cfg) -> dict:
    """model/qwen35/load.go:79-228 Load: every tensor by name and shape into
    the engine's weight dictionary (views of the mapping, nothing copied);
    no output.weight means the LM head is the token embedding."""
    H = cfg.hidden
    w = dict(embedding=_matrix(r, "token_embd.weight", cfg.vocab, H))
    w["output"] = _matrix(r, "output.weight", cfg.vocab, H) if "output.weight" in r.tensors else w["embedding"]
    w["output_norm"] = _f32(r, "output_norm.weight", H)
    q_dim, kv_dim, o_dim = cfg.heads * cfg.head_dim * 2, cfg.kv_heads * cfg.head_dim, cfg.heads * cfg.head_dim
    layers = []
    for i in range(cfg.n_layers):
        p = f"blk.{i}."
        L = dict(attn_norm=_f32(r, p + "attn_norm.weight", H), post_norm=_f32(r, p + "post_attention_norm.weight", H))
        if cfg.is_recurrent(i):
            L.update(qkv=_matrix(r, p + "attn_qkv.weight", cfg.conv_dim, H),
                     gate=_matrix(r, p + "attn_gate.weight", cfg.inner, H),
                     out=_matrix(r, p + "ssm_out.weight", H, cfg.inner),
                     beta=_matrix(r, p + "ssm_beta.weight", cfg.rank, H),
                     alpha=_matrix(r, p + "ssm_alpha.weight", cfg.rank, H),
                     conv=_f32(r, p + "ssm_conv1d.weight", cfg.conv_kernel * cfg.conv_dim, vector=False),
                     dt=_f32(r, p + "ssm_dt.bias", cfg.rank), a=_f32(r, p + "ssm_a", cfg.rank),
                     ssm_norm=_f32(r, p + "ssm_norm.weight", cfg.state_size))
        else:
            L.update(q=_matrix(r, p + "attn_q.weight", q_dim, H), k=_matrix(r, p + "attn_k.weight", kv_dim, H),
                     v=_matrix(r, p + "attn_v.weight", kv_dim, H), o=_matrix(r, p + "attn_output.weight", H, o_dim),
                     q_norm=_f32(r, p + "attn_q_norm.weight", cfg.head_dim),
                     k_norm=_f32(r, p + "attn_k_norm.weight", cfg.head_dim))
        if cfg.n_experts:
            E, ef, sf = cfg.n_experts, cfg.expert_ffn, cfg.shared_ffn
            L.update(router=_matrix(r, p + "ffn_gate_inp.weight", E, H),
                     shared_gate_vec=_f32(r, p + "ffn_gate_inp_shexp.weight", H),
                     shared_gate=_matrix(r, p + "ffn_gate_shexp.weight", sf, H),
                     shared_up=_matrix(r, p + "ffn_up_shexp.weight", sf, H),
                     shared_down=_matrix(r, p + "ffn_down_shexp.weight", H, sf),
                     gate_exps=_experts(r, p + "ffn_gate_exps.weight", ef, H, E),
                     up_exps=_experts(r, p + "ffn_up_exps.weight", ef, H, E),
                     down_exps=_experts(r, p + "ffn_down_exps.weight", H, ef, E))
        else:
            L.update(ffn_gate=_matrix(r, p + "ffn_gate.weight", cfg.ffn, H),
                     ffn_up=_matrix(r, p + "ffn_up.weight", cfg.ffn, H),
                     ffn_down=_matrix(r, p + "ffn_down.weight", H, cfg.ffn))
        layers.append(L)
    w["layers"] = layers
    return w


# --------------------------------------------------------------- the writer

def _enc_value(v: Value) -> bytes:
    if v.type in _SCALAR:
        return struct.pack(_SCALAR[v.type], int(v.value) if v.type == BOOL else v.value)
    if v.type == STRING:
        b = v.value.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    if v.type == ARRAY:
        out = [struct.pack("<IQ", v.elem_type, len(v.value))]
        for item in v.value:
            out.append((struct.pack("<I", item.type) if v.elem_type == ARRAY else b"") + _enc_value(item))
        return b"".join(out)
    raise GGUFError(f"cannot encode metadata type {v.type}")


def write(path: str, metadata: dict, tensors: list, version: int = 3, alignment: int = DEFAULT_ALIGN) -> None:
    """Writes a GGUF file. `metadata`: name -> Value (general.alignment is
    added when `alignment` is not the default); `tensors`: (name, dims in
    GGML order, dtype, bytes) in file order, each placed at the next aligned
    offset of the data section."""
    meta = dict(metadata)
    if alignment != DEFAULT_ALIGN:
        meta.setdefault("general.alignment", Value(U32, alignment))
    head = [MAGIC, struct.pack("<IQQ", version, len(tensors), len(meta))]
    for k, v in meta.items():
        kb = k.encode("utf-8")
        head.append(struct.pack("<Q", len(kb)) + kb + struct.pack("<I", v.type) + _enc_value(v))
    tensors = [(name, dims, dtype, np.ascontiguousarray(data).reshape(-1).view(np.uint8))
               for name, dims, dtype, data in tensors]
    offsets, off = [], 0
    for name, dims, dtype, data in tensors:
        be, bb = BLOCKS[dtype]
        n = 1
        for d in dims:
            n *= d
        if len(data) != n // be * bb:
            raise GGUFError(f"tensor {name!r}: {len(data)} bytes, want {n // be * bb}")
        off = _align_up(off, alignment)
        offsets.append(off)
        off += len(data)
        nb = name.encode("utf-8")
        head.append(struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims)) +
                    b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", dtype, offsets[-1]))
    header = b"".join(head)
    start = _align_up(len(header), alignment)
    with open(path, "wb") as f:
        f.write(header + b"\0" * (start - len(header)))
        pos = 0
        for (name, dims, dtype, data), o in zip(tensors, offsets):
            f.write(b"\0" * (o - pos))
            f.write(data.tobytes())
            pos = o + len(data)


def write_q35(path: str, cfg, w: dict, tie_output: bool = False) -> None:
    """Writes a qwen35 / qwen35moe model (config and weight dictionary in the
    model.make_weights layout) under the names and shapes load_weights reads."""
    arch = MOE_ARCH if cfg.n_experts else ARCH
    ui = lambda v: Value(U32, int(v))  # noqa: E731
    meta = {"general.architecture": Value(STRING, arch), f"{arch}.block_count": ui(cfg.n_layers),
            f"{arch}.context_length": ui(max(cfg.capacity, 1)), f"{arch}.embedding_length": ui(cfg.hidden),
            f"{arch}.attention.head_count": ui(cfg.heads), f"{arch}.attention.head_count_kv": ui(cfg.kv_heads),
            f"{arch}.attention.key_length": ui(cfg.head_dim), f"{arch}.attention.value_length": ui(cfg.head_dim),
            f"{arch}.rope.dimension_count": ui(cfg.rope_dim), f"{arch}.rope.freq_base": Value(F32V, cfg.rope_base),
            f"{arch}.attention.layer_norm_rms_epsilon": Value(F32V, cfg.eps),
            f"{arch}.ssm.conv_kernel": ui(cfg.conv_kernel), f"{arch}.ssm.state_size": ui(cfg.state_size),
            f"{arch}.ssm.group_count": ui(cfg.groups), f"{arch}.ssm.time_step_rank": ui(cfg.rank),
            f"{arch}.ssm.inner_size": ui(cfg.inner), f"{arch}.full_attention_interval": ui(cfg.full_interval),
            f"{arch}.vocab_size": ui(cfg.vocab)}
    if cfg.n_experts:
        meta.update({f"{arch}.expert_count": ui(cfg.n_experts), f"{arch}.expert_used_count": ui(cfg.n_experts_used),
                     f"{arch}.expert_feed_forward_length": ui(cfg.expert_ffn),
                     f"{arch}.expert_shared_feed_forward_length": ui(cfg.shared_ffn)})
    else:
        meta[f"{arch}.feed_forward_length"] = ui(cfg.ffn)
    ts = []

    def mat(name, m):
        ts.append((name, (m["cols"], m["rows"]), m["dtype"], np.asarray(m["data"]).view(np.uint8)))

    def vec(name, v, dims=None):
        v = np.asarray(v, np.float32)
        ts.append((name, dims or (v.size,), F32, v.view(np.uint8)))

    mat("token_embd.weight", w["embedding"])
    if not tie_output:
        mat("output.weight", w["output"])
    vec("output_norm.weight", w["output_norm"])
    for i, L in enumerate(w["layers"]):
        p = f"blk.{i}."
        vec(p + "attn_norm.weight", L["attn_norm"])
        vec(p + "post_attention_norm.weight", L["post_norm"])
        if cfg.is_recurrent(i):
            for n, k in (("attn_qkv", "qkv"), ("attn_gate", "gate"), ("ssm_out", "out"), ("ssm_beta", "beta"),
                         ("ssm_alpha", "alpha")):
                mat(p + n + ".weight", L[k])
            vec(p + "ssm_conv1d.weight", L["conv"], (cfg.conv_kernel, cfg.conv_dim))
            vec(p + "ssm_dt.bias", L["dt"])
            vec(p + "ssm_a", L["a"])
            vec(p + "ssm_norm.weight", L["ssm_norm"])
        else:
            for n, k in (("attn_q", "q"), ("attn_k", "k"), ("attn_v", "v"), ("attn_output", "o")):
                mat(p + n + ".weight", L[k])
            vec(p + "attn_q_norm.weight", L["q_norm"])
            vec(p + "attn_k_norm.weight", L["k_norm"])
        if cfg.n_experts:
            E = cfg.n_experts
            mat(p + "ffn_gate_inp.weight", L["router"])
            vec(p + "ffn_gate_inp_shexp.weight", L["shared_gate_vec"])
            mat(p + "ffn_gate_shexp.weight", L["shared_gate"])
            mat(p + "ffn_up_shexp.weight", L["shared_up"])
            mat(p + "ffn_down_shexp.weight", L["shared_down"])
            for n, k in (("ffn_gate_exps", "gate_exps"), ("ffn_up_exps", "up_exps"), ("ffn_down_exps", "down_exps")):
                m = L[k]
                ts.append((p + n + ".weight", (m["cols"], m["rows"] // E, E), m["dtype"],
                           np.asarray(m["data"]).view(np.uint8)))
        else:
            for n, k in (("ffn_gate", "ffn_gate"), ("ffn_up", "ffn_up"), ("ffn_down", "ffn_down")):
                mat(p + n + ".weight", L[k])
    write(path, meta, ts)
