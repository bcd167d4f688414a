"""GGUF on the host: the container bc-infer reads a model from (crates/bc-infer/src/gguf.rs),
and the loading of one stage's tensors into GpuLayers (model.rs:44-70 Config::from_header,
86-108 needed, 176-217 Part::new).

parse() restates gguf.rs:157-200: the magic, version 2 or 3, tensor and key counts, typed
metadata (gguf.rs:126-155: integers widen to u64/i64, f32 to f64, arrays nest at most twice),
tensor descriptions (name, at most 4 dims, ggml type, offset), the data start aligned to
general.alignment (32 by default), and each tensor's absolute byte range from its type's block
size. A header cut short raises NeedMore (read more bytes and try again, as Source does).
write_gguf() restates the fixture writer (gguf.rs:233-296): version 3, tensors at offsets
rounded up to 32 bytes, the data start padded to 32."""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from layers import Config, Matrix

# (weights, bytes) per block of each ggml type (quant.rs:69-82).
BLOCKS = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
          12: (256, 144), 13: (256, 176), 14: (256, 210)}


class NeedMore(Exception):
    """The header continues past the bytes given (gguf.rs:88-97)."""


@dataclass
class TensorInfo:
    name: str
    dims: list            # ggml order: dims[0] is the row length
    ty: int
    range: tuple          # absolute [start, end) in the file
    file: int = 0

    def elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n

    def shape2(self) -> tuple[int, int]:
        """(row length, rows), extra dimensions counted as more rows (gguf.rs:70-75)."""
        cols = int(self.dims[0]) if self.dims else 1
        return cols, self.elements() // max(cols, 1)


@dataclass
class Header:
    version: int
    meta: dict = field(default_factory=dict)
    tensors: list = field(default_factory=list)
    data_start: int = 0

    def get(self, key):
        return self.meta.get(key)

    def tensor(self, name: str):
        for t in self.tensors:
            if t.name == name:
                return t
        return None

    def arch(self) -> str:
        a = self.get("general.architecture")
        return a if isinstance(a, str) else "llama"

    def arch_u64(self, key: str):
        v = self.get(f"{self.arch()}.{key}")
        return v if isinstance(v, int) and not isinstance(v, bool) and v >= 0 else None

    def arch_f64(self, key: str):
        v = self.get(f"{self.arch()}.{key}")
        return float(v) if isinstance(v, (int, float)) and not isinstance(v, bool) else None


class _Cursor:
    def __init__(self, b: bytes):
        self.b, self.at = b, 0

    def take(self, n: int) -> bytes:
        if self.at + n > len(self.b):
            raise NeedMore()
        s = self.b[self.at:self.at + n]
        self.at += n
        return s

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def u64(self) -> int:
        return struct.unpack("<Q", self.take(8))[0]

    def string(self) -> str:
        n = self.u64()
        if n > 1 << 24:
            raise ValueError(f"GGUF header string of {n} bytes is past the limit")
        return self.take(n).decode("utf-8", errors="replace")

    def value(self, ty: int, depth: int):
        """gguf.rs:126-155."""
        if ty == 0:
            return self.take(1)[0]
        if ty == 1:
            return struct.unpack("<b", self.take(1))[0]
        if ty == 2:
            return struct.unpack("<H", self.take(2))[0]
        if ty == 3:
            return struct.unpack("<h", self.take(2))[0]
        if ty == 4:
            return self.u32()
        if ty == 5:
            return struct.unpack("<i", self.take(4))[0]
        if ty == 6:
            return float(struct.unpack("<f", self.take(4))[0])
        if ty == 7:
            return self.take(1)[0] != 0
        if ty == 8:
            return self.string()
        if ty == 9:
            if depth > 2:
                raise ValueError("GGUF metadata array holds arrays (not accepted)")
            item, n = self.u32(), self.u64()
            if n > 1 << 24:
                raise ValueError(f"GGUF metadata array of {n} items is past the limit")
            return [self.value(item, depth + 1) for _ in range(n)]
        if ty == 10:
            return self.u64()
        if ty == 11:
            return struct.unpack("<q", self.take(8))[0]
        if ty == 12:
            return struct.unpack("<d", self.take(8))[0]
        raise ValueError(f"GGUF metadata value type {ty} is not defined")


def parse(data: bytes) -> Header:
    """gguf.rs:157-200: the header from the start of a file."""
    c = _Cursor(bytes(data))
    if c.take(4) != b"GGUF":
        raise ValueError("bad magic: the bytes do not start a GGUF container")
    version = c.u32()
    if version not in (2, 3):
        raise ValueError(f"GGUF container version {version} (2 and 3 are read)")
    n_tensors, n_meta = c.u64(), c.u64()
    if n_tensors > 1 << 20 or n_meta > 1 << 20:
        raise ValueError(f"GGUF counts past the limits: {n_tensors} tensors, {n_meta} metadata keys")
    meta = {}
    for _ in range(n_meta):
        key = c.string()
        meta[key] = c.value(c.u32(), 0)
    raw = []
    for _ in range(n_tensors):
        name = c.string()
        nd = c.u32()
        if nd > 4:
            raise ValueError(f"tensor {name}: {nd} dimensions is past the limit")
        dims = [c.u64() for _ in range(nd)]
        raw.append((name, dims, c.u32(), c.u64()))
    align = meta.get("general.alignment")
    align = max(align if isinstance(align, int) and not isinstance(align, bool) and align >= 0 else 32, 1)
    data_start = (c.at + align - 1) // align * align
    tensors = []
    for name, dims, ty, offset in raw:
        if ty not in BLOCKS:
            raise ValueError(f"tensor {name}: ggml type {ty} is not one this loader reads")
        n, size = BLOCKS[ty]
        elements = 1
        for d in dims:
            elements *= d
        if elements % n:
            raise ValueError(f"tensor {name}: {elements} elements do not fill whole {n}-weight blocks")
        start = data_start + offset
        tensors.append(TensorInfo(name, dims, ty, (start, start + elements // n * size)))
    return Header(version, meta, tensors, data_start)


def _string(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(meta, tensors) -> bytes:
    """gguf.rs:233-296 (test fixtures only). meta: [(key, kind, value)] with kind one of
    "u32", "f32", "str", "strs", "f32s", "i32s"; tensors: [(name, dims, ggml type, bytes)]."""
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(meta)))
    codes = {"u32": (4, "<I"), "f32": (6, "<f")}
    arrays = {"strs": 8, "f32s": 6, "i32s": 5}
    for key, kind, v in meta:
        out += _string(key)
        if kind in codes:
            code, fmt = codes[kind]
            out += struct.pack("<I", code) + struct.pack(fmt, v)
        elif kind == "str":
            out += struct.pack("<I", 8) + _string(v)
        else:
            item = arrays[kind]
            out += struct.pack("<IIQ", 9, item, len(v))
            for x in v:
                out += _string(x) if item == 8 else struct.pack("<f" if item == 6 else "<i", x)
    offset, offsets = 0, []
    for name, dims, ty, data in tensors:
        out += _string(name) + struct.pack("<I", len(dims))
        for d in dims:
            out += struct.pack("<Q", d)
        out += struct.pack("<IQ", ty, offset)
        offsets.append(offset)
        offset = (offset + len(data) + 31) // 32 * 32
    while len(out) % 32:
        out.append(0)
    base = len(out)
    for (_, _, _, data), off in zip(tensors, offsets):
        out += bytes(base + off - len(out))
        out += bytes(data)
    return bytes(out)


def config_from_header(h: Header) -> Config:
    """Config::from_header (model.rs:44-70)."""
    arch = h.arch()
    if arch not in ("llama", "qwen2", "mistral"):
        raise ValueError(f"model architecture {arch!r}: only llama, mistral and qwen2 layouts load")

    def need(key):
        v = h.arch_u64(key)
        if v is None:
            raise ValueError(f"no {key}")
        return v

    def dflt(v, d):
        return d if v is None else v

    n_embd, n_head = need("embedding_length"), need("attention.head_count")
    head_dim = dflt(h.arch_u64("attention.key_length"), n_embd // max(n_head, 1))
    embd = h.tensor("token_embd.weight")
    if embd is None:
        raise ValueError("no token_embd.weight")
    f32 = lambda x: float(np.float32(x))
    return Config(n_embd=n_embd, n_layer=need("block_count"), n_head=n_head,
                  n_head_kv=dflt(h.arch_u64("attention.head_count_kv"), n_head), head_dim=head_dim,
                  rope_dim=dflt(h.arch_u64("rope.dimension_count"), head_dim),
                  rope_base=f32(dflt(h.arch_f64("rope.freq_base"), 10000.0)), rope_neox=arch == "qwen2",
                  eps=f32(dflt(h.arch_f64("attention.layer_norm_rms_epsilon"), 1e-5)), vocab=embd.shape2()[1],
                  context=dflt(h.arch_u64("context_length"), 4096))


def needed(h: Header, lo: int, hi: int, first: bool, last: bool) -> list:
    """model.rs:86-108: the tensors a stage of layers [lo, hi) reads."""
    has_output = h.tensor("output.weight") is not None
    out = []
    for t in h.tensors:
        if t.name.startswith("blk."):
            part = t.name[4:].split(".")[0]
            if part.isdigit() and lo <= int(part) < hi:
                out.append(t)
        elif t.name == "token_embd.weight":
            if first or (last and not has_output):
                out.append(t)
        elif t.name in ("output_norm.weight", "output.weight"):
            if last:
                out.append(t)
        elif t.name == "rope_freqs.weight" and hi > lo:
            out.append(t)
    return out


def _vector(data: bytes, t: TensorInfo) -> np.ndarray:
    """A norm or bias vector as f32 (QTensor::to_f32 of an f32 tensor)."""
    if t.ty != 0:
        raise ValueError(f"{t.name}: vectors are read as f32 here, not ggml type {t.ty}")
    return np.frombuffer(data[t.range[0]:t.range[1]], np.float32).copy()


def _matrix(data: bytes, t: TensorInfo) -> Matrix:
    cols, rows = t.shape2()
    return Matrix(t.ty, bytes(data[t.range[0]:t.range[1]]), rows, cols)


def load_stage(data: bytes, lo: int, hi: int, first: bool, last: bool):
    """Part::new's tensor lookup (model.rs:176-200) over one GGUF file: (Config, the layer
    dicts GpuLayers takes, the head (output_norm, output) or None, the embedding Matrix or
    None, the rope_freqs factors or None)."""
    h = parse(data)
    cfg = config_from_header(h)
    if hi > cfg.n_layer:
        raise ValueError(f"layers {lo}..{hi} are past the model's {cfg.n_layer}")
    ts = {t.name: t for t in needed(h, lo, hi, first, last)}

    def get(name):
        if name not in ts:
            raise ValueError(f"missing tensor {name}")
        return ts[name]

    layers = []
    for l in range(lo, hi):
        p = lambda s: f"blk.{l}.{s}"
        d = {"attn_norm": _vector(data, get(p("attn_norm.weight"))),
             "ffn_norm": _vector(data, get(p("ffn_norm.weight")))}
        for key, name in (("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"),
                          ("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
            d[key] = _matrix(data, get(p(f"{name}.weight")))
        for key, name in (("bq", "attn_q"), ("bk", "attn_k"), ("bv", "attn_v")):
            t = ts.get(p(f"{name}.bias"))
            d[key] = None if t is None else _vector(data, t)
        layers.append(d)
    embd = _matrix(data, get("token_embd.weight")) if first else None
    head = None
    if last:
        out = ts.get("output.weight") or get("token_embd.weight")
        head = (_vector(data, get("output_norm.weight")), _matrix(data, out))
    factors = ts.get("rope_freqs.weight")
    return cfg, layers, head, embd, None if factors is None else _vector(data, factors)
