"""Test fixture: the reference's small random Llama-shaped model (crates/bc-infer/src/
fixtures.rs:7-60), restated as the same GGUF file: width 64, feed-forward 128, vocabulary 96,
4 query and 2 KV heads, Q8_0 matrices (quantised by the oracle's restatement of
quant.rs:634-646), f32 norms and q bias, the weights drawn from one xorshift stream in the
file's tensor order, the metadata and tokens of fixtures.rs:38-56, written by gguf.write_gguf
(gguf.rs:233-296) and read back by gguf.load_stage (the loader the GPU layers take their
weights from). Also an f64 forward of the same model (model.rs:297-352 with dequantised
weights and exact arithmetic) to check the GPU layers against."""
from __future__ import annotations

import numpy as np

import oracle as O
from gguf import load_stage, write_gguf
from layers import Config, Matrix, inv_freq

M64 = (1 << 64) - 1


def tiny_model_file(n_layer: int, neox: bool) -> bytes:
    """fixtures.rs:7-60: the GGUF file's bytes."""
    d, ff, vocab, heads, kv_heads = 64, 128, 96, 4, 2
    state = [0x9E3779B97F4A7C15]

    def rnd(n: int, scale: float) -> np.ndarray:
        s = state[0]
        out = np.empty(n, np.float32)
        for i in range(n):
            s ^= (s << 13) & M64
            s ^= s >> 7
            s ^= (s << 17) & M64
            out[i] = (np.float32(s % 2001) / np.float32(1000.0) - np.float32(1.0)) * np.float32(scale)
        state[0] = s
        return out

    q8 = lambda v: O.quantize_q8_0(v).tobytes()
    f32b = lambda v: np.asarray(v, "<f4").tobytes()
    kvd = d // heads * kv_heads
    tensors = [("token_embd.weight", [d, vocab], 8, q8(rnd(d * vocab, 1.0)))]
    for l in range(n_layer):
        p = lambda s: f"blk.{l}.{s}"
        tensors += [
            (p("attn_norm.weight"), [d], 0, f32b(rnd(d, 0.2) + np.float32(1.0))),
            (p("attn_q.weight"), [d, d], 8, q8(rnd(d * d, 0.15))),
            (p("attn_k.weight"), [d, kvd], 8, q8(rnd(d * kvd, 0.15))),
            (p("attn_v.weight"), [d, kvd], 8, q8(rnd(d * kvd, 0.15))),
            (p("attn_q.bias"), [d], 0, f32b(rnd(d, 0.1))),
            (p("attn_output.weight"), [d, d], 8, q8(rnd(d * d, 0.15))),
            (p("ffn_norm.weight"), [d], 0, f32b(rnd(d, 0.2) + np.float32(1.0))),
            (p("ffn_gate.weight"), [d, ff], 8, q8(rnd(d * ff, 0.15))),
            (p("ffn_up.weight"), [d, ff], 8, q8(rnd(d * ff, 0.15))),
            (p("ffn_down.weight"), [ff, d], 8, q8(rnd(ff * d, 0.15))),
        ]
    tensors.append(("output_norm.weight", [d], 0, f32b(np.ones(d, np.float32))))
    tensors.append(("output.weight", [d, vocab], 8, q8(rnd(d * vocab, 0.3))))
    arch = "qwen2" if neox else "llama"
    tokens = ["<unk>", "<s>", "</s>"] + [chr(32 + i % 95) for i in range(vocab - 3)]
    meta = [("general.architecture", "str", arch), ("general.name", "str", "tiny"),
            (f"{arch}.embedding_length", "u32", d), (f"{arch}.block_count", "u32", n_layer),
            (f"{arch}.attention.head_count", "u32", heads), (f"{arch}.attention.head_count_kv", "u32", kv_heads),
            (f"{arch}.feed_forward_length", "u32", ff), (f"{arch}.context_length", "u32", 2048),
            ("tokenizer.ggml.model", "str", "llama"), ("tokenizer.ggml.tokens", "strs", tokens),
            ("tokenizer.ggml.scores", "f32s", [0.0] * vocab), ("tokenizer.ggml.bos_token_id", "u32", 1),
            ("tokenizer.ggml.eos_token_id", "u32", 2)]
    return write_gguf(meta, tensors)


def tiny_model(n_layer: int, neox: bool):
    """The fixture loaded as a whole model: (Config, layer dicts for GpuLayers, head,
    embedding Matrix)."""
    cfg, layers, head, embd, _ = load_stage(tiny_model_file(n_layer, neox), 0, n_layer, True, True)
    return cfg, layers, head, embd


def embed(embd: Matrix, tokens) -> np.ndarray:
    """Part::embed (model.rs:270-281): the tokens' rows of token_embd, dequantised."""
    table = O.dequant(embd.type, np.frombuffer(embd.data, np.uint8), embd.rows, embd.cols)
    return table[np.asarray(tokens, np.int64)].astype(np.float32)


class RefModel:
    """The same layers in f64 over dequantised weights: the reference's CPU forward
    (model.rs:297-352) with exact arithmetic, its cache a list of rows per layer."""

    def __init__(self, cfg: Config, layers, head):
        self.cfg = cfg
        deq = lambda m: O.dequant(m.type, np.frombuffer(m.data, np.uint8), m.rows, m.cols).astype(np.float64)
        self.layers = []
        for l in layers:
            w = {k: deq(l[k]) for k in ("wq", "wk", "wv", "wo", "gate", "up", "down")}
            for k in ("attn_norm", "ffn_norm"):
                w[k] = np.asarray(l[k], np.float64)
            w["bq"] = None if l["bq"] is None else np.asarray(l["bq"], np.float64)
            self.layers.append(w)
        self.norm, self.out = np.asarray(head[0], np.float64), deq(head[1])
        self.freq = inv_freq(cfg).astype(np.float64)

    def new_cache(self):
        return {"k": [np.zeros((0, self.cfg.n_head_kv * self.cfg.head_dim)) for _ in self.layers],
                "v": [np.zeros((0, self.cfg.n_head_kv * self.cfg.head_dim)) for _ in self.layers]}

    def _norm(self, x, w):
        return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + self.cfg.eps) * w

    def _rope(self, t, heads, positions):
        c = self.cfg
        t = t.reshape(len(positions), heads, c.head_dim).copy()
        half = c.rope_dim // 2
        th = np.asarray(positions, np.float64)[:, None] * self.freq[None, :half]
        cos, sin = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
        if c.rope_neox:
            a, b = t[:, :, :half].copy(), t[:, :, half:2 * half].copy()
            t[:, :, :half], t[:, :, half:2 * half] = a * cos - b * sin, a * sin + b * cos
        else:
            a, b = t[:, :, 0:2 * half:2].copy(), t[:, :, 1:2 * half:2].copy()
            t[:, :, 0:2 * half:2], t[:, :, 1:2 * half:2] = a * cos - b * sin, a * sin + b * cos
        return t.reshape(len(positions), heads * c.head_dim)

    def forward(self, x, pos: int, tree, cache) -> np.ndarray:
        c = self.cfg
        rows = len(x)
        positions, visible, base = O.shape(rows, pos, tree)
        x = np.asarray(x, np.float64).copy()
        hd, nh, nkv = c.head_dim, c.n_head, c.n_head_kv
        g = nh // nkv
        for li, w in enumerate(self.layers):
            n = self._norm(x, w["attn_norm"])
            q, k, v = n @ w["wq"].T, n @ w["wk"].T, n @ w["wv"].T
            if w["bq"] is not None:
                q = q + w["bq"]
            q, k = self._rope(q, nh, positions), self._rope(k, nkv, positions)
            kc = np.concatenate([cache["k"][li][:pos], k])
            vc = np.concatenate([cache["v"][li][:pos], v])
            cache["k"][li], cache["v"][li] = kc, vc
            att = np.zeros((rows, nh * hd))
            for r in range(rows):
                if visible is None:
                    slots = np.arange(pos + r + 1)
                else:
                    bits = [j for j in range(64) if (int(visible[r]) >> j) & 1]
                    slots = np.concatenate([np.arange(base), base + np.asarray(bits, np.int64)]).astype(np.int64)
                for h in range(nh):
                    kv = h // g
                    qs = q[r, h * hd:(h + 1) * hd]
                    s = kc[slots, kv * hd:(kv + 1) * hd] @ qs / np.sqrt(hd)
                    p = np.exp(s - s.max())
                    att[r, h * hd:(h + 1) * hd] = (p / p.sum()) @ vc[slots, kv * hd:(kv + 1) * hd]
            x = x + att @ w["wo"].T
            n = self._norm(x, w["ffn_norm"])
            gt, up = n @ w["gate"].T, n @ w["up"].T
            x = x + (gt / (1.0 + np.exp(-gt)) * up) @ w["down"].T
        return x

    def logits(self, x) -> np.ndarray:
        return self._norm(np.asarray(x, np.float64), self.norm) @ self.out.T


def wide_model_file(n_layer: int, neox: bool, seed: int = 7) -> bytes:
    """A random model at the widths the measured kernels take (no reference counterpart; the
    reference's fixture is the small one above): width 512, 4 query and 2 KV heads of head_dim
    128, feed-forward 1024, vocabulary 256. The attention matrices and the head are Q8_0
    (quantised from N(0, 1/width) draws by the oracle's quantiser), gate and up Q4K, down Q6K
    (random blocks, their scales set so the weights stay modest), so every product of more
    than one row runs on the matrix cores (widths a multiple of 256) and a one-row product on
    the VALU. Weights from numpy's seeded generator, written by gguf.write_gguf."""
    d, ff, vocab, heads, kv_heads = 512, 1024, 256, 4, 2
    rng = np.random.default_rng(seed)
    q8 = lambda rows, cols, s: O.quantize_q8_0(rng.standard_normal(rows * cols).astype(np.float32) * np.float32(s)).tobytes()
    f32b = lambda v: np.asarray(v, "<f4").tobytes()

    def kquant(wtype: int, rows: int, cols: int) -> bytes:
        n, size = {12: (256, 144), 14: (256, 210)}[wtype]
        data = rng.integers(0, 256, rows * cols // n * size, dtype=np.uint8).reshape(-1, size)
        f16 = lambda x: np.frombuffer(np.float16(x).tobytes(), np.uint8)
        if wtype == 12:  # Q4K: w = d sc q - dmin m, q in 0..15, sc and m in 0..63
            data[:, 0:2] = f16(2.0 ** -12)
            data[:, 2:4] = f16(7.5 * 2.0 ** -12)  # about centres the weights
        else:  # Q6K: w = d sc (q - 32), sc an int8
            data[:, 208:210] = f16(2.0 ** -14)
        return data.tobytes()

    kvd = d // heads * kv_heads
    tensors = [("token_embd.weight", [d, vocab], 8, q8(vocab, d, 1.0))]
    for l in range(n_layer):
        p = lambda s: f"blk.{l}.{s}"
        tensors += [
            (p("attn_norm.weight"), [d], 0, f32b(rng.standard_normal(d).astype(np.float32) * 0.2 + 1.0)),
            (p("attn_q.weight"), [d, d], 8, q8(d, d, d ** -0.5)),
            (p("attn_k.weight"), [d, kvd], 8, q8(kvd, d, d ** -0.5)),
            (p("attn_v.weight"), [d, kvd], 8, q8(kvd, d, d ** -0.5)),
            (p("attn_q.bias"), [d], 0, f32b(rng.standard_normal(d).astype(np.float32) * 0.1)),
            (p("attn_output.weight"), [d, d], 8, q8(d, d, d ** -0.5)),
            (p("ffn_norm.weight"), [d], 0, f32b(rng.standard_normal(d).astype(np.float32) * 0.2 + 1.0)),
            (p("ffn_gate.weight"), [d, ff], 12, kquant(12, ff, d)),
            (p("ffn_up.weight"), [d, ff], 12, kquant(12, ff, d)),
            (p("ffn_down.weight"), [ff, d], 14, kquant(14, d, ff)),
        ]
    tensors.append(("output_norm.weight", [d], 0, f32b(np.ones(d, np.float32))))
    tensors.append(("output.weight", [d, vocab], 8, q8(vocab, d, d ** -0.5)))
    arch = "qwen2" if neox else "llama"
    tokens = ["<unk>", "<s>", "</s>"] + [f"t{i}" for i in range(vocab - 3)]
    meta = [("general.architecture", "str", arch), ("general.name", "str", "wide"),
            (f"{arch}.embedding_length", "u32", d), (f"{arch}.block_count", "u32", n_layer),
            (f"{arch}.attention.head_count", "u32", heads), (f"{arch}.attention.head_count_kv", "u32", kv_heads),
            (f"{arch}.feed_forward_length", "u32", ff), (f"{arch}.context_length", "u32", 4096),
            (f"{arch}.rope.freq_base", "f32", 500000.0 if not neox else 1000000.0),
            ("tokenizer.ggml.model", "str", "llama"), ("tokenizer.ggml.tokens", "strs", tokens),
            ("tokenizer.ggml.scores", "f32s", [0.0] * vocab), ("tokenizer.ggml.bos_token_id", "u32", 1),
            ("tokenizer.ggml.eos_token_id", "u32", 2)]
    return write_gguf(meta, tensors)


def wide_model(n_layer: int, neox: bool):
    """wide_model_file loaded as a whole model, as tiny_model."""
    cfg, layers, head, embd, _ = load_stage(wide_model_file(n_layer, neox), 0, n_layer, True, True)
    return cfg, layers, head, embd
