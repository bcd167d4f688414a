"""The GGUF container on the host (borrowed-compute_amd/gguf.py, crates/bc-infer/src/gguf.rs):
the reference's own round-trip test (gguf.rs:308-334), the byte layout of the published GGUF
format (version 3: magic, counts, typed metadata, tensor descriptions, 32-byte aligned data)
written out by hand, every cut inside a header, and a stage's tensor choice (model.rs:86-108)
and Config (model.rs:44-70) over the reference's small model file (fixtures.rs:7-60)."""
import struct

import numpy as np
import pytest

import gguf
from tiny_model import tiny_model_file


def test_round_trips_and_asks_for_more():
    """gguf.rs:308-334, word for word."""
    file = gguf.write_gguf(
        [("general.architecture", "str", "llama"), ("llama.block_count", "u32", 2),
         ("tokenizer.ggml.tokens", "strs", ["a", "b"])],
        [("w", [32, 2], 0, bytes([1]) * 256), ("v", [32], 8, bytes([2]) * 34)])
    h = gguf.parse(file)
    assert h.arch() == "llama"
    assert h.arch_u64("block_count") == 2
    w = h.tensor("w")
    assert w.shape2() == (32, 2)
    assert file[w.range[0]:w.range[1]] == bytes([1]) * 256
    v = h.tensor("v")
    assert file[v.range[0]:v.range[1]] == bytes([2]) * 34
    with pytest.raises(gguf.NeedMore):
        gguf.parse(file[:40])
    with pytest.raises(ValueError):
        gguf.parse(b"NOPE0000")


def test_the_published_byte_layout():
    """One key and one tensor, laid out by hand from the GGUF format: "GGUF", version 3 (u32),
    tensor and key counts (u64), key (u64 length + bytes), value type 4 (u32) and value,
    tensor name, n_dims (u32), dims (u64), type (u32), offset (u64), zeros to 32 bytes, data."""
    data = bytes(range(16))
    got = gguf.write_gguf([("a", "u32", 7)], [("t", [4], 0, data)])
    want = b"GGUF" + struct.pack("<IQQ", 3, 1, 1)
    want += struct.pack("<Q", 1) + b"a" + struct.pack("<II", 4, 7)
    want += struct.pack("<Q", 1) + b"t" + struct.pack("<IQIQ", 1, 4, 0, 0)
    want += bytes(-len(want) % 32) + data
    assert got == want
    h = gguf.parse(want)
    assert len(want) == 96 + 16  # a 74-byte header padded to 96
    assert h.version == 3 and h.meta == {"a": 7} and h.data_start == 96
    assert h.tensor("t").range == (96, 112)


def test_every_value_type_and_alignment():
    """gguf.rs:126-155: each typed value, nested arrays, and general.alignment."""
    body = b""
    keys = []

    def kv(k, ty, payload):
        nonlocal body
        body += struct.pack("<Q", len(k)) + k.encode() + struct.pack("<I", ty) + payload
        keys.append(k)

    kv("u8", 0, b"\xff")
    kv("i8", 1, b"\xff")
    kv("u16", 2, struct.pack("<H", 65535))
    kv("i16", 3, struct.pack("<h", -2))
    kv("i32", 5, struct.pack("<i", -7))
    kv("f32", 6, struct.pack("<f", 0.5))
    kv("bool", 7, b"\x01")
    kv("u64", 10, struct.pack("<Q", 1 << 40))
    kv("i64", 11, struct.pack("<q", -(1 << 40)))
    kv("f64", 12, struct.pack("<d", 0.25))
    kv("nest", 9, struct.pack("<IQ", 9, 1) + struct.pack("<IQ", 4, 2) + struct.pack("<II", 3, 4))
    kv("general.alignment", 4, struct.pack("<I", 64))
    head = b"GGUF" + struct.pack("<IQQ", 3, 0, len(keys)) + body
    h = gguf.parse(head)
    assert h.meta == {"u8": 255, "i8": -1, "u16": 65535, "i16": -2, "i32": -7, "f32": 0.5, "bool": True,
                      "u64": 1 << 40, "i64": -(1 << 40), "f64": 0.25, "nest": [[3, 4]], "general.alignment": 64}
    assert h.data_start == (len(head) + 63) // 64 * 64
    deep = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"x" + struct.pack("<I", 9)
    deep += struct.pack("<IQ", 9, 1) * 3 + struct.pack("<IQ", 4, 0)
    with pytest.raises(ValueError):
        gguf.parse(deep)


def test_a_cut_header_asks_for_more_at_every_byte():
    file = tiny_model_file(1, False)
    h = gguf.parse(file)
    for cut in range(0, h.data_start - 31, 7):
        with pytest.raises(gguf.NeedMore):
            gguf.parse(file[:cut])
    # Past the header only the tensor data is missing: the header parses.
    assert len(gguf.parse(file[:h.data_start]).tensors) == len(h.tensors)


@pytest.mark.parametrize("neox", [False, True])
def test_the_small_model_file(neox):
    """fixtures.rs:7-60 read back: tensor order, shapes, types, 32-byte aligned data, metadata,
    and Config::from_header."""
    file = tiny_model_file(3, neox)
    h = gguf.parse(file)
    arch = "qwen2" if neox else "llama"
    assert h.version == 3 and h.arch() == arch and h.data_start % 32 == 0
    names = [t.name for t in h.tensors]
    per = ["attn_norm.weight", "attn_q.weight", "attn_k.weight", "attn_v.weight", "attn_q.bias",
           "attn_output.weight", "ffn_norm.weight", "ffn_gate.weight", "ffn_up.weight", "ffn_down.weight"]
    assert names == ["token_embd.weight"] + [f"blk.{l}.{p}" for l in range(3) for p in per] + \
        ["output_norm.weight", "output.weight"]
    for t in h.tensors:
        assert (t.range[0] - h.data_start) % 32 == 0 and t.range[1] <= len(file)
    assert h.tensor("blk.1.attn_k.weight").dims == [64, 32] and h.tensor("blk.1.attn_k.weight").ty == 8
    assert h.tensor("blk.0.ffn_down.weight").shape2() == (128, 64)
    assert len(h.get("tokenizer.ggml.tokens")) == 96 and h.get("tokenizer.ggml.tokens")[3] == " "
    c = gguf.config_from_header(h)
    assert (c.n_embd, c.n_layer, c.n_head, c.n_head_kv, c.head_dim, c.rope_dim, c.vocab, c.context) == \
        (64, 3, 4, 2, 16, 16, 96, 2048)
    assert c.rope_neox == neox and c.rope_base == 10000.0 and c.eps == float(np.float32(1e-5))
    norm = h.tensor("output_norm.weight")
    assert np.array_equal(np.frombuffer(file[norm.range[0]:norm.range[1]], "<f4"), np.ones(64, np.float32))


def test_a_stage_reads_only_its_tensors():
    """model.rs:86-108: its layers, the embeddings when first, the head when last (the
    embeddings again when the model ties them), rope factors whenever it holds a layer."""
    h = gguf.parse(tiny_model_file(4, False))
    mid = {t.name for t in gguf.needed(h, 1, 3, False, False)}
    assert mid == {t.name for t in h.tensors if t.name.startswith(("blk.1.", "blk.2."))}
    assert "token_embd.weight" in {t.name for t in gguf.needed(h, 0, 1, True, False)}
    last = {t.name for t in gguf.needed(h, 3, 4, False, True)}
    assert {"output_norm.weight", "output.weight"} <= last and "token_embd.weight" not in last
    tied = gguf.write_gguf([("general.architecture", "str", "llama")],
                           [("token_embd.weight", [32, 4], 0, bytes(512)), ("output_norm.weight", [32], 0, bytes(128)),
                            ("rope_freqs.weight", [4], 0, bytes(16))])
    ht = gguf.parse(tied)
    assert {t.name for t in gguf.needed(ht, 0, 1, False, True)} == {"token_embd.weight", "output_norm.weight",
                                                                   "rope_freqs.weight"}
    assert {t.name for t in gguf.needed(ht, 0, 0, False, False)} == set()
