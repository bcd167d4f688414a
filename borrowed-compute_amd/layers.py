"""One pipeline stage's layers on the GPU: bc-infer's Layers::forward
(crates/bc-infer/src/gpu/mod.rs:428-495), its logits head (mod.rs:499-508, the product
of model.rs:361-370) and the sampler after it (sample.rs, engine.rs:341-350), issued as this
library's entry points instead of a Cmd list.

Per layer, in the reference's order: RMSNorm, the q/k/v products, their biases, RoPE of q
and k with the append of k and v at slot `pos` (the four commands at mod.rs:464-475 as one
bchip_rope_append), attention over the cache (for a line pass, with the append as one
call: bchip_rope_append_attention or its multi-row form), the output product and the
residual add,
RMSNorm, gate and up products, SiLU-mul, the down product and the residual add. Weights
stay in their ggml blocks (bchip_matmul). The cache is a bchip.KvCache (Gpu::reserve's
growth, mod.rs:404-423); positions and the tree's visibility masks come from the caller's
Shape (model.rs:405-443), as in the reference."""
from __future__ import annotations

import ctypes
import ctypes.util
import math
from dataclasses import dataclass

import numpy as np

import bchip


@dataclass
class Config:
    """model.rs:27-80 (the fields the layers read)."""
    n_embd: int
    n_layer: int
    n_head: int
    n_head_kv: int
    head_dim: int
    rope_dim: int
    rope_base: float = 10000.0
    rope_neox: bool = False
    eps: float = 1e-5
    vocab: int = 0
    context: int = 4096


_libm = None


def _powf(x: float, y: float) -> float:
    """The C library's single-precision pow, the one the reference's f32::powf calls
    (numpy's float32 power differs from it in the last bit for many of these arguments)."""
    global _libm
    if _libm is None:
        _libm = ctypes.CDLL(ctypes.util.find_library("m") or "libm.so.6")
        _libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
        _libm.powf.restype = ctypes.c_float
    return _libm.powf(x, y)


def inv_freq(cfg: Config, factors=None) -> np.ndarray:
    """model.rs:208-211: rope_base^(-2i / rope_dim) in f32 (the exponent rounded to f32
    first), over the optional per-pair factors (rope_freqs.weight)."""
    half = cfg.rope_dim // 2
    f = np.empty(half, np.float32)
    for i in range(half):
        e = np.float32(np.float32(-2.0) * np.float32(i)) / np.float32(cfg.rope_dim)
        f[i] = _powf(np.float32(cfg.rope_base), e)
    if factors is not None:
        f = (f / np.asarray(factors, np.float32)[:half]).astype(np.float32)
    return f


@dataclass
class Matrix:
    """A weight matrix as stored: `rows` rows of `cols` weights in ggml blocks of `type`."""
    type: int
    data: bytes
    rows: int
    cols: int


class GpuLayers:
    """The layers of one stage (and the head, on the last stage), resident on the device.

    `layers` holds per layer: attn_norm, ffn_norm (f32 vectors), wq, wk, wv, wo, gate, up,
    down (Matrix), and bq, bk, bv (f32 vectors or None). `head` is (output_norm, output)
    or None."""

    def __init__(self, ctx: bchip.Ctx, cfg: Config, layers: list[dict], head=None, kv_type: int = bchip.F32):
        self.ctx, self.cfg, self.kv_type = ctx, cfg, kv_type
        up = lambda a: ctx.upload(np.ascontiguousarray(a, np.float32))
        self.layers = []
        for l in layers:
            d = {k: up(l[k]) for k in ("attn_norm", "ffn_norm")}
            for k in ("wq", "wk", "wv", "wo", "gate", "up", "down"):
                m: Matrix = l[k]
                d[k] = (ctx.upload(np.frombuffer(m.data, np.uint8)), m.type, m.rows, m.cols)
            for k in ("bq", "bk", "bv"):
                d[k] = up(l[k]) if l.get(k) is not None else None
            self.layers.append(d)
        self.head = None
        if head is not None:
            norm, out = head
            self.head = (up(norm), ctx.upload(np.frombuffer(out.data, np.uint8)), out.type, out.rows, out.cols)
        self.freq = up(inv_freq(cfg))
        self.ff = layers[0]["gate"].rows if layers else 0
        self.scratch_rows = 0
        self.scratch: dict[str, bchip.Buf] = {}

    def new_cache(self) -> bchip.KvCache:
        """Gpu::new_cache (mod.rs:398-400)."""
        return bchip.KvCache(self.ctx, len(self.layers), self.cfg.n_head_kv * self.cfg.head_dim, self.kv_type)

    def _scratch(self, rows: int) -> dict:
        """Working buffers of at least `rows` rows, kept between calls (mod.rs:444-449)."""
        if rows > self.scratch_rows:
            c = self.cfg
            qd, kvd = c.n_head * c.head_dim, c.n_head_kv * c.head_dim
            for b in self.scratch.values():
                b.free()
            sizes = {"x": c.n_embd, "n": c.n_embd, "q": qd, "k": kvd, "v": kvd, "att": qd, "o": c.n_embd,
                     "gate": self.ff, "up": self.ff, "pos": 1, "mask": 2}
            self.scratch = {k: self.ctx.zeros(max(rows * w, 1) * 4) for k, w in sizes.items()}
            self.scratch_rows = rows
        return self.scratch

    def _matmul(self, w, x, out, rows: int, nrows: int | None = None) -> None:
        buf, ty, wr, wc = w
        self.ctx.matmul(buf, ty, x, out, wr if nrows is None else nrows, wc, rows)

    def forward(self, x: np.ndarray, pos: int, positions, masks, cache: bchip.KvCache) -> np.ndarray:
        """mod.rs:428-495: `rows` hidden states at positions `positions` (slots pos..), with
        `masks` = (base, visible) for a tree; returns the updated states."""
        c, ctx = self.cfg, self.ctx
        rows = len(positions)
        cache.reserve(pos + rows, pos, c.context)
        e, hd, nh, nkv = c.n_embd, c.head_dim, c.n_head, c.n_head_kv
        qd, kvd = nh * hd, nkv * hd
        s = self._scratch(rows)
        ctx.upload(np.ascontiguousarray(x, np.float32), s["x"])
        ctx.upload(np.ascontiguousarray(positions, np.uint32), s["pos"])
        mb, seen = None, pos
        if masks is not None:
            seen, visible = masks
            ctx.upload(bchip.masks_words(visible), s["mask"])
            mb = s["mask"]
        scale = 1.0 / math.sqrt(hd)
        for l, kc, vc in zip(self.layers, cache.k, cache.v):
            ctx.rms_norm(s["x"], l["attn_norm"], s["n"], rows, e, c.eps)
            self._matmul(l["wq"], s["n"], s["q"], rows)
            self._matmul(l["wk"], s["n"], s["k"], rows)
            self._matmul(l["wv"], s["n"], s["v"], rows)
            for bias, out, dim in ((l["bq"], s["q"], qd), (l["bk"], s["k"], kvd), (l["bv"], s["v"], kvd)):
                if bias is not None:
                    ctx.bias_add(out, bias, rows * dim, dim)
            if rows == 1 and masks is None:
                # A one-token line step: the five commands as one launch (same bits).
                ctx.rope_append_attention(s["q"], s["k"], s["v"], kc, vc, self.kv_type, self.freq, s["pos"], nh, nkv,
                                          hd, c.rope_dim, c.rope_neox, pos, scale, s["att"])
            elif masks is None:
                # A line pass of several rows: one call (one launch where the library can, else
                # its two calls; the same bits either way).
                ctx.rope_append_attention_rows(s["q"], s["k"], s["v"], kc, vc, self.kv_type, self.freq, s["pos"], rows,
                                               nh, nkv, hd, c.rope_dim, c.rope_neox, pos, scale, s["att"])
            else:
                ctx.rope_append(s["q"], s["k"], s["v"], kc, vc, self.kv_type, self.freq, s["pos"], rows, nh, nkv, hd,
                                c.rope_dim, c.rope_neox, pos)
                ctx.attention(s["q"], kc, vc, self.kv_type, s["att"], mb, masks is not None, rows, nh, nkv, hd, seen,
                              scale)
            self._matmul(l["wo"], s["att"], s["o"], rows)
            ctx.add(s["x"], s["o"], rows * e)
            ctx.rms_norm(s["x"], l["ffn_norm"], s["n"], rows, e, c.eps)
            self._matmul(l["gate"], s["n"], s["gate"], rows)
            self._matmul(l["up"], s["n"], s["up"], rows)
            ctx.silu_mul(s["gate"], s["up"], rows * self.ff)
            self._matmul(l["down"], s["gate"], s["o"], rows)
            ctx.add(s["x"], s["o"], rows * e)
        return ctx.read(s["x"], (rows, e))

    def logits(self, x: np.ndarray, rows: int, upto: int | None = None) -> np.ndarray:
        """Next-token scores of each row for the first `upto` tokens (mod.rs:499-508):
        RMSNorm with output_norm, then the product against the first `upto` rows of the
        output matrix (Gpu::matmul_rows)."""
        if self.head is None:
            raise ValueError("this stage has no output head")
        norm, out, ty, vr, vc = self.head
        upto = vr if upto is None else min(upto, vr)
        s = self._scratch(rows)
        ctx = self.ctx
        ctx.upload(np.ascontiguousarray(x, np.float32), s["x"])
        ctx.rms_norm(s["x"], norm, s["n"], rows, self.cfg.n_embd, self.cfg.eps)
        scores = ctx.zeros(rows * upto * 4)
        ctx.matmul(out, ty, s["n"], scores, upto, vc, rows)
        got = ctx.read(scores, (rows, upto))
        scores.free()
        return got

    def sample(self, x: np.ndarray, rows: int, temperature: float, top_p: float, seed: int, step0: int,
               upto: int | None = None) -> np.ndarray:
        """The last stage's next tokens (engine.rs:341-350): the logits head, then sample.rs's
        pick for each row on the device (bchip_sample; row r at step step0 + r). Only the ids
        come back to the host, not the rows x vocab scores."""
        if self.head is None:
            raise ValueError("this stage has no output head")
        norm, out, ty, vr, vc = self.head
        upto = vr if upto is None else min(upto, vr)
        s = self._scratch(rows)
        ctx = self.ctx
        ctx.upload(np.ascontiguousarray(x, np.float32), s["x"])
        ctx.rms_norm(s["x"], norm, s["n"], rows, self.cfg.n_embd, self.cfg.eps)
        scores, ids = ctx.zeros(rows * upto * 4), ctx.zeros(rows * 4)
        ctx.matmul(out, ty, s["n"], scores, upto, vc, rows)
        ctx.sample(scores, rows, upto, temperature, top_p, seed, step0, ids)
        got = ctx.read(ids, (rows,), np.uint32)
        scores.free()
        ids.free()
        return got

    def free(self) -> None:
        for l in self.layers:
            for k, v in l.items():
                if isinstance(v, bchip.Buf):
                    v.free()
                elif isinstance(v, tuple):
                    v[0].free()
        if self.head is not None:
            self.head[0].free()
            self.head[1].free()
        self.freq.free()
        for b in self.scratch.values():
            b.free()
        self.scratch, self.scratch_rows = {}, 0
