"""ctypes face of the CPU oracle (oracle/bc_oracle.c): TEST INFRASTRUCTURE ONLY.

Imported only by tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline``
leg, as the checker. The product library never touches it. Each wrapper names the
reference lines its C function restates (paths inside Harshil089/Borrowed-Compute).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
ROOT = 0xFFFFFFFF  # model.rs:406
MAX_TREE = 64  # model.rs:408

_lib = None


def build() -> str:
    """Compiles liboracle.so from bc_oracle.c (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        u32, u64, f32, sz = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_size_t
        L.bco_inv_freq.argtypes = [P, u32, f32, P]
        L.bco_rope.argtypes = [P, u32, u32, u32, ctypes.c_int, u64, P]
        L.bco_shape.argtypes = [u32, u64, P, u32, P, P, P]
        L.bco_shape.restype = ctypes.c_int
        L.bco_dot.argtypes = [P, P, sz]
        L.bco_dot.restype = f32
        L.bco_attention.argtypes = [P, P, P, P, u32, u64, P, u64, u32, u32, u32, f32]
        L.bco_keep.argtypes = [P, u64, P, u64, P, u32]
        L.bco_keep.restype = ctypes.c_int
        L.bco_f32_to_f16.argtypes = [f32]
        L.bco_f32_to_f16.restype = ctypes.c_uint16
        L.bco_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.bco_f16_to_f32.restype = f32
        L.bco_round_f16.argtypes = [P, sz]
        L.bco_splitmix64.argtypes = [P]
        L.bco_splitmix64.restype = u64
        L.bco_normal.argtypes = [u64, P, sz]
        L.bcl_block.argtypes = [u32, P, P]
        L.bcl_block.restype = ctypes.c_int
        L.bcl_ref_f32_to_f16.argtypes = [f32]
        L.bcl_ref_f32_to_f16.restype = ctypes.c_uint16
        L.bcl_scale_min_k4.argtypes = [u32, P, P, P]
        L.bcl_dequant_block.argtypes = [u32, P, P]
        L.bcl_dequant.argtypes = [u32, P, u64, u64, P]
        L.bcl_dequant.restype = ctypes.c_int
        L.bcl_random_tensor.argtypes = [u32, u64, u64, u64, P]
        L.bcl_random_tensor.restype = ctypes.c_int
        L.bcl_quantize_q8_0.argtypes = [P, u64, P]
        L.bcl_matmul_f64.argtypes = [u32, P, u64, u64, P, u64, P]
        L.bcl_matmul_f64.restype = ctypes.c_int
        L.bcl_rms_norm.argtypes = [P, P, P, u64, u64, f32]
        L.bcl_silu_mul.argtypes = [P, P, u64]
        L.bcl_bias_add.argtypes = [P, P, u64, u64]
        L.bcl_add.argtypes = [P, P, u64]
        L.bcs_argmax.argtypes = [P, u32]
        L.bcs_argmax.restype = u32
        L.bcs_uniform.argtypes = [u64]
        L.bcs_uniform.restype = f32
        L.bcs_exp.argtypes = [f32]
        L.bcs_exp.restype = f32
        L.bcs_sample.argtypes = [P, u32, f32, f32, u64, u64]
        L.bcs_sample.restype = u32
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def inv_freq(rope_dim: int, base: float, factors=None) -> np.ndarray:
    """model.rs:208-211."""
    out = np.zeros(rope_dim // 2, np.float32)
    f = None if factors is None else _f32(factors)
    lib().bco_inv_freq(_p(out), rope_dim, base, _p(f))
    return out


def rope(x, heads: int, head_dim: int, rope_dim: int, neox: bool, pos: int, inv: np.ndarray) -> np.ndarray:
    """model.rs:391-403 on one row (heads x head_dim); returns a rotated copy."""
    y = _f32(x).copy()
    lib().bco_rope(_p(y), heads, head_dim, rope_dim, int(neox), pos, _p(_f32(inv)))
    return y


def rope_rows(x, positions, heads: int, head_dim: int, rope_dim: int, neox: bool, inv) -> np.ndarray:
    """model.rs:330-333: row i rotated to positions[i]; x is [rows][heads*head_dim]."""
    y = _f32(x).reshape(len(positions), heads * head_dim).copy()
    inv = _f32(inv)
    for i, p in enumerate(positions):
        row = np.ascontiguousarray(y[i])
        lib().bco_rope(_p(row), heads, head_dim, rope_dim, int(neox), int(p), _p(inv))
        y[i] = row
    return y


class ShapeError(ValueError):
    pass


def shape(rows: int, pos: int, tree=None):
    """model.rs:421-443: (positions, visible or None, base)."""
    positions = np.zeros(rows, np.uint64)
    if tree is None:
        lib().bco_shape(rows, pos, None, 0, _p(positions), None, None)
        return positions, None, pos
    t = np.ascontiguousarray(tree, dtype=np.uint32)
    visible = np.zeros(rows, np.uint64)
    base = np.zeros(1, np.uint64)
    if lib().bco_shape(rows, pos, _p(t), len(t), _p(positions), _p(visible), _p(base)) != 0:
        raise ShapeError(f"a tree of {len(t)} nodes for {rows} rows at {pos}")
    return positions, visible, int(base[0])


def dot(a, b) -> float:
    """quant.rs:617-631."""
    a, b = _f32(a), _f32(b)
    return float(lib().bco_dot(_p(a), _p(b), a.size))


def attention(q, kc, vc, rows: int, pos: int, nh: int, nkv: int, hd: int, scale: float | None = None,
              visible=None, base: int | None = None) -> np.ndarray:
    """model.rs:448-481. q [rows][nh][hd]; kc, vc [slots][nkv*hd] (f32); returns out."""
    q, kc, vc = _f32(q), _f32(kc), _f32(vc)
    need = pos + rows
    assert q.size == rows * nh * hd, "q is not rows x nh x hd"
    assert kc.size >= need * nkv * hd and vc.size >= need * nkv * hd, "cache shorter than pos + rows"
    out = np.zeros((rows, nh, hd), np.float32)
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    vis = None if visible is None else np.ascontiguousarray(visible, dtype=np.uint64)
    b = pos if base is None else base
    lib().bco_attention(_p(q), _p(kc), _p(vc), _p(out), rows, pos, _p(vis), b, nh, nkv, hd, scale)
    return out


def keep(cache: np.ndarray, width: int, length: int, base: int, rows) -> int:
    """model.rs:146-166 on one buffer (modified in place); returns the new length."""
    assert cache.dtype == np.float32 and cache.flags.c_contiguous
    r = np.ascontiguousarray(rows, dtype=np.uint32)
    n = np.array([length], np.uint64)
    if lib().bco_keep(_p(cache), width, _p(n), base, _p(r), len(r)) != 0:
        raise ValueError(f"rows {list(rows)} at {base} are not an ascending path within {length}")
    return int(n[0])


def f16_round(x) -> np.ndarray:
    y = _f32(x).copy()
    lib().bco_round_f16(_p(y), y.size)
    return y


def f32_to_f16_bits(x: float) -> int:
    return int(lib().bco_f32_to_f16(x))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().bco_f16_to_f32(h))


def splitmix64(seed: int, n: int) -> list[int]:
    s = np.array([seed], np.uint64)
    return [int(lib().bco_splitmix64(_p(s))) for _ in range(n)]


def normal(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().bco_normal(seed, _p(out), n)
    return out


# ---- The rest of the layer (bc_layer.c). ----
# ggml type numbers (quant.rs:35-49).
F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4K, Q5K, Q6K, BF16 = 0, 1, 2, 3, 6, 7, 8, 12, 13, 14, 30
GGML_TYPES = (F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q4K, Q5K, Q6K)
TYPE_NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q4_0: "Q4_0", Q4_1: "Q4_1", Q5_0: "Q5_0", Q5_1: "Q5_1",
              Q8_0: "Q8_0", Q4K: "Q4K", Q5K: "Q5K", Q6K: "Q6K"}


def block(ty: int) -> tuple[int, int]:
    """quant.rs:69-82: (weights, bytes) per block."""
    n, b = np.zeros(1, np.uint32), np.zeros(1, np.uint32)
    if not lib().bcl_block(ty, _p(n), _p(b)):
        raise ValueError(f"ggml type {ty}")
    return int(n[0]), int(b[0])


def row_bytes(ty: int, cols: int) -> int:
    n, b = block(ty)
    assert cols % n == 0
    return cols // n * b


def f16_to_f32(h: int) -> np.float32:
    """quant.rs:93-112 (IEEE binary16 to f32, exact)."""
    return np.float32(lib().bco_f16_to_f32(int(h)))


def ref_f32_to_f16(x: float) -> int:
    """quant.rs:114-131 (half up, subnormals flushed)."""
    return int(lib().bcl_ref_f32_to_f16(float(x)))


def scale_min_k4(j: int, q) -> tuple[float, float]:
    """quant.rs:136-146."""
    qb = np.ascontiguousarray(q, dtype=np.uint8)
    sc, mn = np.zeros(1, np.float32), np.zeros(1, np.float32)
    lib().bcl_scale_min_k4(j, _p(qb), _p(sc), _p(mn))
    return float(sc[0]), float(mn[0])


def dequant_block(ty: int, src) -> np.ndarray:
    """quant.rs:150-259."""
    n, b = block(ty)
    sb = np.ascontiguousarray(src, dtype=np.uint8)
    assert sb.size >= b
    out = np.zeros(n, np.float32)
    lib().bcl_dequant_block(ty, _p(sb), _p(out))
    return out


def dequant(ty: int, data, rows: int, cols: int) -> np.ndarray:
    """quant.rs:349-362: the tensor as f32 rows."""
    d = np.ascontiguousarray(data, dtype=np.uint8)
    assert d.size == rows * row_bytes(ty, cols)
    out = np.zeros((rows, cols), np.float32)
    assert lib().bcl_dequant(ty, _p(d), rows, cols, _p(out)) == 0
    return out


def random_tensor(ty: int, rows: int, cols: int, seed: int) -> np.ndarray:
    """fixtures.rs:66-92: the tensor's bytes (rows x row_bytes)."""
    out = np.zeros(rows * row_bytes(ty, cols), np.uint8)
    assert lib().bcl_random_tensor(ty, rows, cols, seed, _p(out)) == 0
    return out


def quantize_q8_0(values) -> np.ndarray:
    """quant.rs:634-646."""
    v = _f32(values)
    assert v.size % 32 == 0
    out = np.zeros(v.size // 32 * 34, np.uint8)
    lib().bcl_quantize_q8_0(_p(v), v.size, _p(out))
    return out


def matmul_f64(ty: int, data, rows: int, cols: int, x, n: int) -> np.ndarray:
    """gpu/mod.rs:193-196: out[i][r] = sum_c W[r][c] x[i][c] in f64 over dequantized weights,
    for the first `rows` weight rows; returns [n][rows] float64."""
    d = np.ascontiguousarray(data, dtype=np.uint8)
    xv = _f32(x)
    assert xv.size == n * cols
    out = np.zeros((n, rows), np.float64)
    assert lib().bcl_matmul_f64(ty, _p(d), rows, cols, _p(xv), n, _p(out)) == 0
    return out


def rms_norm(x, w, eps: float) -> np.ndarray:
    """model.rs:381-388; x [rows][cols], w [cols]."""
    w = _f32(w)
    xv = _f32(x).reshape(-1, w.size)
    out = np.zeros_like(xv)
    lib().bcl_rms_norm(_p(xv), _p(w), _p(out), xv.shape[0], w.size, float(eps))
    return out


def silu_mul(g, u) -> np.ndarray:
    """model.rs:343."""
    gv = _f32(g).copy()
    lib().bcl_silu_mul(_p(gv), _p(_f32(u)), gv.size)
    return gv


def bias_add(x, b) -> np.ndarray:
    """model.rs:371-377."""
    xv = _f32(x).copy()
    bv = _f32(b)
    lib().bcl_bias_add(_p(xv), _p(bv), xv.size, bv.size)
    return xv


def add(x, y) -> np.ndarray:
    """model.rs:337."""
    xv = _f32(x).copy()
    lib().bcl_add(_p(xv), _p(_f32(y)), xv.size)
    return xv


# ---- The sampler (bc_sample.c). ----
def argmax(scores) -> int:
    """sample.rs:24-32."""
    s = _f32(scores)
    return int(lib().bcs_argmax(_p(s), s.size))


def uniform(seed: int) -> float:
    """sample.rs:74-81."""
    return float(lib().bcs_uniform(seed & 0xFFFFFFFFFFFFFFFF))


def sample(scores, temperature: float, top_p: float, seed: int, step: int) -> int:
    """sample.rs:35-71 (exp correctly rounded)."""
    s = _f32(scores)
    return int(lib().bcs_sample(_p(s), s.size, temperature, top_p, seed & 0xFFFFFFFFFFFFFFFF,
                                step & 0xFFFFFFFFFFFFFFFF))
