"""ctypes face of libbchip.so (include/bchip.h): bc-infer's attention path on one MI355X.

A thin host mirror of the reference's backend calls (crates/bc-infer/src/gpu/cuda.rs:31-94:
new, name, memory, unified, upload, zeros, read, run) plus the attention operators, for
tests and benchmarks. Every compute call goes to the HIP library; there is no CPU path
here, and loading fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbchip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "bchip.h")

F32, F16 = 0, 1
OK, E_ARG, E_HIP, E_NODEV, E_DISABLED, E_UNSUPPORTED, E_OOM = 0, -1, -2, -3, -4, -5, -6
CHUNK_MULTI = 192
# ggml weight types (quant.rs:35-49) and (weights, bytes) per block (quant.rs:69-82).
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_1, GGML_Q5_0, GGML_Q5_1, GGML_Q8_0 = 0, 1, 2, 3, 6, 7, 8
GGML_Q4K, GGML_Q5K, GGML_Q6K, GGML_BF16 = 12, 13, 14, 30
GGML_BLOCKS = {GGML_F32: (1, 4), GGML_F16: (1, 2), GGML_BF16: (1, 2), GGML_Q4_0: (32, 18), GGML_Q4_1: (32, 20),
               GGML_Q5_0: (32, 22), GGML_Q5_1: (32, 24), GGML_Q8_0: (32, 34), GGML_Q4K: (256, 144),
               GGML_Q5K: (256, 176), GGML_Q6K: (256, 210)}


def ggml_row_bytes(wtype: int, cols: int) -> int:
    n, b = GGML_BLOCKS[wtype]
    return cols // n * b

_lib = None


class BchipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"bchip error {code}: {msg}")
        self.code = code


def declared_functions(header: str = HEADER) -> list[str]:
    """Names of the functions include/bchip.h declares."""
    text = open(header).read()
    return sorted(set(re.findall(r"\b(bchip_[a-z_0-9]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    P, u32, u64, f32, sz, i32 = (ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float,
                                 ctypes.c_size_t, ctypes.c_int)
    sig = {
        "bchip_last_error": ([], ctypes.c_char_p),
        "bchip_abi_version": ([], i32),
        "bchip_init": ([i32, P], i32),
        "bchip_destroy": ([P], i32),
        "bchip_device_name": ([P, ctypes.c_char_p, sz], i32),
        "bchip_mem_free": ([P, P], i32),
        "bchip_unified": ([P, P], i32),
        "bchip_alloc": ([P, sz, P], i32),
        "bchip_free": ([P, P], i32),
        "bchip_upload": ([P, P, sz, P, sz], i32),
        "bchip_download": ([P, P, sz, P, sz], i32),
        "bchip_sync": ([P], i32),
        "bchip_stream": ([P, P], i32),
        "bchip_rope": ([P, P, P, P, u32, u32, u32, u32, u32], i32),
        "bchip_copy": ([P, P, u32, P, u32, u64, u64], i32),
        "bchip_move": ([P, P, u32, u64, u64, u64], i32),
        "bchip_keep": ([P, P, u32, u32, u32, u64, P, u32], i32),
        "bchip_cache_grow": ([P, P, P, u32, u32, u64, u64], i32),
        "bchip_rope_append": ([P, P, P, P, P, P, u32, P, P, u32, u32, u32, u32, u32, u32, u64], i32),
        "bchip_attention": ([P, P, P, P, u32, P, P, u32, u32, u32, u32, u32, u32, f32], i32),
        "bchip_rope_append_attention": ([P, P, P, P, P, P, u32, P, P, u32, u32, u32, u32, u32, u32, f32, P], i32),
        "bchip_rope_append_attention_noalloc": ([P, P, P, P, P, P, u32, P, P, u32, u32, u32, u32, u32, u32, f32,
                                                 P], i32),
        "bchip_rope_append_attention_rows": ([P, P, P, P, P, P, u32, P, P, u32, u32, u32, u32, u32, u32, u32, f32,
                                              P], i32),
        "bchip_attention_ragged": ([P, P, P, P, u32, P, P, P, u32, u32, u32, u32, f32], i32),
        "bchip_rope_append_ragged": ([P, P, P, P, P, P, u32, P, P, P, P, u32, u32, u32, u32, u32, u32], i32),
        "bchip_rope_append_attention_ragged": ([P, P, P, P, P, P, u32, P, P, P, P, u32, u32, u32, u32, u32, u32, f32,
                                                P], i32),
        "bchip_fill_normal": ([P, P, u32, u64, u64], i32),
        "bchip_sample": ([P, P, u32, u32, f32, f32, u64, u64, P], i32),
        "bchip_matmul": ([P, P, u32, P, P, u32, u32, u32], i32),
        "bchip_rms_norm": ([P, P, P, P, u32, u32, f32], i32),
        "bchip_bias_add": ([P, P, P, u64, u32], i32),
        "bchip_silu_mul": ([P, P, P, u64], i32),
        "bchip_add": ([P, P, P, u64], i32),
        "bchip_timer_start": ([P], i32),
        "bchip_timer_stop": ([P, P], i32),
        "bchip_timer_arm": ([P, P, P], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def last_error() -> str:
    return lib().bchip_last_error().decode()


def check(code: int) -> None:
    if code != OK:
        raise BchipError(code, last_error())


def esize(t: int) -> int:
    return 2 if t == F16 else 4


class Buf:
    """Device memory from bchip_alloc, freed with its context (or by free())."""

    def __init__(self, ctx: "Ctx", nbytes: int):
        self.ctx = ctx
        self.nbytes = nbytes
        p = ctypes.c_void_p()
        check(lib().bchip_alloc(ctx.h, nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def offset(self, nbytes: int) -> int:
        return self.ptr + nbytes

    def free(self) -> None:
        if self.ptr:
            check(lib().bchip_free(self.ctx.h, self.ptr))
            self.ptr = None


class Ctx:
    """One device context: the reference's Backend (cuda.rs:21-25)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(lib().bchip_init(device, ctypes.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            lib().bchip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # Backend::name / memory / unified
    def name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        check(lib().bchip_device_name(self.h, buf, 256))
        return buf.value.decode()

    def memory(self) -> int:
        v = ctypes.c_uint64()
        check(lib().bchip_mem_free(self.h, ctypes.byref(v)))
        return v.value

    def unified(self) -> bool:
        v = ctypes.c_int()
        check(lib().bchip_unified(self.h, ctypes.byref(v)))
        return bool(v.value)

    # Backend::zeros / upload / read
    def zeros(self, nbytes: int) -> Buf:
        return Buf(self, nbytes)

    def upload(self, arr: np.ndarray, buf: Buf | None = None, off: int = 0) -> Buf:
        a = np.ascontiguousarray(arr)
        if buf is None:
            buf = Buf(self, max(a.nbytes, 1))
        check(lib().bchip_upload(self.h, buf.ptr, off, a.ctypes.data_as(ctypes.c_void_p), a.nbytes))
        return buf

    def read(self, buf: Buf | int, shape, dtype=np.float32, off: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        ptr = buf.ptr if isinstance(buf, Buf) else buf
        check(lib().bchip_download(self.h, ptr, off, out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def sync(self) -> None:
        check(lib().bchip_sync(self.h))

    def stream(self) -> int:
        p = ctypes.c_void_p()
        check(lib().bchip_stream(self.h, ctypes.byref(p)))
        return p.value

    # operators
    def rope(self, x, inv_freq, positions, rows, heads, hd, rope_dim, neox) -> None:
        check(lib().bchip_rope(self.h, _ptr(x), _ptr(inv_freq), _ptr(positions), rows, heads, hd, rope_dim,
                               int(neox)))

    def copy(self, src, st, dst, dt, off, n) -> None:
        check(lib().bchip_copy(self.h, _ptr(src), st, _ptr(dst), dt, off, n))

    def move(self, buf, t, frm, to, n) -> None:
        check(lib().bchip_move(self.h, _ptr(buf), t, frm, to, n))

    def keep(self, bufs, t, width, base, rows) -> None:
        arr = (ctypes.c_void_p * len(bufs))(*[_ptr(b) for b in bufs])
        r = np.ascontiguousarray(rows, np.uint32)
        check(lib().bchip_keep(self.h, arr, len(bufs), t, width, base, r.ctypes.data_as(ctypes.c_void_p), len(r)))

    def cache_grow(self, srcs, dsts, t, keep, total) -> None:
        n = len(dsts)
        sa = (ctypes.c_void_p * n)(*[_ptr(b) for b in srcs]) if srcs else None
        da = (ctypes.c_void_p * n)(*[_ptr(b) for b in dsts])
        check(lib().bchip_cache_grow(self.h, sa, da, n, t, keep, total))

    def rope_append(self, q, k, v, kc, vc, kv_type, inv_freq, positions, rows, nh, nkv, hd, rope_dim, neox,
                    slot0) -> None:
        check(lib().bchip_rope_append(self.h, _ptr(q), _ptr(k), _ptr(v), _ptr(kc), _ptr(vc), kv_type,
                                      _ptr(inv_freq), _ptr(positions), rows, nh, nkv, hd, rope_dim, int(neox),
                                      slot0))

    def attention(self, q, kc, vc, kv_type, out, masks, tree, rows, nh, nkv, hd, pos, scale) -> None:
        check(lib().bchip_attention(self.h, _ptr(q), _ptr(kc), _ptr(vc), kv_type, _ptr(out), _ptr(masks),
                                    int(tree), rows, nh, nkv, hd, pos, scale))

    def rope_append_attention(self, q, k, v, kc, vc, kv_type, inv_freq, positions, nh, nkv, hd, rope_dim, neox,
                              pos, scale, out) -> None:
        check(lib().bchip_rope_append_attention(self.h, _ptr(q), _ptr(k), _ptr(v), _ptr(kc), _ptr(vc), kv_type,
                                                _ptr(inv_freq), _ptr(positions), nh, nkv, hd, rope_dim, int(neox),
                                                pos, scale, _ptr(out)))

    def rope_append_attention_rows(self, q, k, v, kc, vc, kv_type, inv_freq, positions, rows, nh, nkv, hd, rope_dim,
                                   neox, pos, scale, out) -> None:
        """rope_append of `rows` rows at slot pos, then attention of those rows at pos, in one call."""
        check(lib().bchip_rope_append_attention_rows(self.h, _ptr(q), _ptr(k), _ptr(v), _ptr(kc), _ptr(vc), kv_type,
                                                     _ptr(inv_freq), _ptr(positions), rows, nh, nkv, hd, rope_dim,
                                                     int(neox), pos, scale, _ptr(out)))

    def rope_append_attention_noalloc(self, q, k, v, kc, vc, kv_type, inv_freq, positions, nh, nkv, hd, rope_dim,
                                      neox, pos, scale, out) -> None:
        """bchip_rope_append_attention with the library's fixed scratch: no device allocation."""
        check(lib().bchip_rope_append_attention_noalloc(self.h, _ptr(q), _ptr(k), _ptr(v), _ptr(kc), _ptr(vc),
                                                        kv_type, _ptr(inv_freq), _ptr(positions), nh, nkv, hd,
                                                        rope_dim, int(neox), pos, scale, _ptr(out)))

    def attention_ragged(self, q, kc, vc, kv_type, out, seq_lens, kv_offsets, nh, nkv, hd, scale) -> None:
        lens = np.ascontiguousarray(seq_lens, np.uint32)
        offs = np.ascontiguousarray(kv_offsets, np.uint64)
        check(lib().bchip_attention_ragged(self.h, _ptr(q), _ptr(kc), _ptr(vc), kv_type, _ptr(out),
                                           lens.ctypes.data_as(ctypes.c_void_p),
                                           offs.ctypes.data_as(ctypes.c_void_p), len(lens), nh, nkv, hd, scale))

    def rope_append_ragged(self, q, k, v, kc, vc, kv_type, inv_freq, positions, seq_lens, kv_offsets, nh, nkv, hd,
                           rope_dim, neox) -> None:
        lens = np.ascontiguousarray(seq_lens, np.uint32)
        offs = np.ascontiguousarray(kv_offsets, np.uint64)
        check(lib().bchip_rope_append_ragged(self.h, _ptr(q), _ptr(k), _ptr(v), _ptr(kc), _ptr(vc), kv_type,
                                             _ptr(inv_freq), _ptr(positions), lens.ctypes.data_as(ctypes.c_void_p),
                                             offs.ctypes.data_as(ctypes.c_void_p), len(lens), nh, nkv, hd, rope_dim,
                                             int(neox)))

    def rope_append_attention_ragged(self, q, k, v, kc, vc, kv_type, inv_freq, positions, seq_lens, kv_offsets, nh,
                                     nkv, hd, rope_dim, neox, scale, out) -> None:
        lens = np.ascontiguousarray(seq_lens, np.uint32)
        offs = np.ascontiguousarray(kv_offsets, np.uint64)
        check(lib().bchip_rope_append_attention_ragged(self.h, _ptr(q), _ptr(k), _ptr(v), _ptr(kc), _ptr(vc),
                                                       kv_type, _ptr(inv_freq), _ptr(positions),
                                                       lens.ctypes.data_as(ctypes.c_void_p),
                                                       offs.ctypes.data_as(ctypes.c_void_p), len(lens), nh, nkv, hd,
                                                       rope_dim, int(neox), scale, _ptr(out)))

    def matmul(self, w, wtype, x, out, rows, cols, n) -> None:
        check(lib().bchip_matmul(self.h, _ptr(w), wtype, _ptr(x), _ptr(out), rows, cols, n))

    def rms_norm(self, x, w, out, rows, cols, eps) -> None:
        check(lib().bchip_rms_norm(self.h, _ptr(x), _ptr(w), _ptr(out), rows, cols, eps))

    def bias_add(self, x, b, n, dim) -> None:
        check(lib().bchip_bias_add(self.h, _ptr(x), _ptr(b), n, dim))

    def silu_mul(self, g, u, n) -> None:
        check(lib().bchip_silu_mul(self.h, _ptr(g), _ptr(u), n))

    def add(self, x, y, n) -> None:
        check(lib().bchip_add(self.h, _ptr(x), _ptr(y), n))

    def sample(self, scores, rows, vocab, temperature, top_p, seed, step0, ids) -> None:
        """sample.rs on the device: ids (device u32 [rows]) from scores (device f32 [rows][vocab])."""
        check(lib().bchip_sample(self.h, _ptr(scores), rows, vocab, temperature, top_p, seed & 0xFFFFFFFFFFFFFFFF,
                                 step0 & 0xFFFFFFFFFFFFFFFF, _ptr(ids)))

    def fill_normal(self, dst, t, n, seed) -> None:
        check(lib().bchip_fill_normal(self.h, _ptr(dst), t, n, seed))

    def timer_start(self) -> None:
        check(lib().bchip_timer_start(self.h))

    def timer_arm(self, before, after) -> None:
        """The next attention call records these hipEvent_t around its main kernel."""
        check(lib().bchip_timer_arm(self.h, before, after))

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        check(lib().bchip_timer_stop(self.h, ctypes.byref(ms)))
        return ms.value


def grown_capacity(cap: int, need: int, context: int) -> int:
    """Gpu::reserve's new capacity in tokens (gpu/mod.rs:409): what is needed, at least twice
    the old capacity and at least 256, but no more than the context (or what is needed, when
    that is more)."""
    return min(max(need, cap * 2, 256), max(context, need))


class KvCache:
    """A model's KV cache on the device, the reference's Cache (gpu/mod.rs:300-337) with
    Gpu::new_cache and Gpu::reserve (mod.rs:398-423): per layer a K and a V buffer of
    cap x kvd elements of kv_type (kvd = n_head_kv * head_dim), grown by doubling, the kept
    prefix copied for every layer in one launch (bchip_cache_grow), and Cache::keep in one
    launch (bchip_keep)."""

    def __init__(self, ctx: "Ctx", n_layer: int, kvd: int, kv_type: int = F16):
        self.ctx, self.n_layer, self.kvd, self.kv_type = ctx, n_layer, kvd, kv_type
        self.k: list[Buf] = []
        self.v: list[Buf] = []
        self.cap = 0

    def reserve(self, need: int, keep: int, context: int) -> None:
        """Grows the cache to hold `need` tokens, keeping its first `keep` (mod.rs:403-423)."""
        if need <= self.cap:
            return
        if keep > self.cap:
            raise ValueError(f"keep {keep} past the cache's {self.cap} tokens")
        cap = grown_capacity(self.cap, need, context)
        nbytes = cap * self.kvd * esize(self.kv_type)
        k = [Buf(self.ctx, nbytes) for _ in range(self.n_layer)]
        v = [Buf(self.ctx, nbytes) for _ in range(self.n_layer)]
        old = self.k + self.v
        if keep > 0 and old:
            self.ctx.cache_grow(old, k + v, self.kv_type, keep * self.kvd, cap * self.kvd)
        for b in old:
            b.free()
        self.k, self.v, self.cap = k, v, cap

    def keep(self, base: int, rows) -> None:
        """Cache::keep (mod.rs:322-337): the accepted rows move down to base, base + 1, ..."""
        if self.k:
            self.ctx.keep(self.k + self.v, self.kv_type, self.kvd, base, rows)

    def bytes(self) -> int:
        """Cache::bytes: device bytes the cache holds."""
        return len(self.k) * 2 * self.cap * self.kvd * esize(self.kv_type)

    def free(self) -> None:
        for b in self.k + self.v:
            b.free()
        self.k, self.v, self.cap = [], [], 0


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, Buf):
        return x.ptr
    return int(x)


def masks_words(visible) -> np.ndarray:
    """64-bit visibility masks as the two u32 words per row the kernels read (mod.rs:438)."""
    v = np.asarray(visible, np.uint64)
    out = np.empty(2 * len(v), np.uint32)
    out[0::2] = (v & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    out[1::2] = (v >> np.uint64(32)).astype(np.uint32)
    return out


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, np.float32).astype(np.float16)
