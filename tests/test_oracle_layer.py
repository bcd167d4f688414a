"""CPU checks of the layer oracle (oracle/bc_layer.c) before it checks the HIP product:
the reference's known-answer block tests (crates/bc-infer/src/quant.rs:650-729), an
independent vectorised numpy dequantisation of every ggml format built from the block
layouts (a different derivation from the C loops: whole-array bit slicing), and the
norm / elementwise ops against numpy."""
import numpy as np
import pytest

import oracle as O


def f16b(v: float) -> list[int]:
    h = O.ref_f32_to_f16(v)
    return [h & 255, h >> 8]


def test_f16_conversions():
    """quant.rs:650-662."""
    for h, f in [(0x3C00, 1.0), (0xC000, -2.0), (0x0000, 0.0), (0x7BFF, 65504.0), (0x0001, 5.9604645e-8),
                 (0x3555, 0.33325195)]:
        assert O.f16_to_f32(h) == np.float32(f), hex(h)
    for v in [1.0, -0.5, 1234.0, 0.1]:
        assert abs(O.f16_to_f32(O.ref_f32_to_f16(v)) - v) <= abs(v) * 1e-3


def test_q4_0_and_q8_0_blocks():
    """quant.rs:664-676."""
    b = np.array(f16b(0.5) + [j | ((15 - j) << 4) for j in range(16)], np.uint8)
    out = O.dequant_block(O.Q4_0, b)
    assert out[0] == -4.0 and out[15] == 3.5 and out[16] == 3.5
    q8 = O.quantize_q8_0(np.arange(32, dtype=np.float32) - 16.0)
    out = O.dequant_block(O.Q8_0, q8)
    assert abs(out[0] + 16.0) < 0.1 and abs(out[31] - 15.0) < 0.1


def test_q5_0_uses_the_fifth_bit():
    """quant.rs:678-689."""
    b = np.array(f16b(1.0) + list((0x00010001).to_bytes(4, "little")) + [0] * 16, np.uint8)
    out = O.dequant_block(O.Q5_0, b)
    assert out[0] == 0.0 and out[1] == -16.0 and out[16] == 0.0 and out[20] == -16.0


def test_k_quant_scales_unpack():
    """quant.rs:691-700."""
    s = np.zeros(12, np.uint8)
    s[0], s[4], s[8] = 0b11_000101, 7, 0x2A
    assert O.scale_min_k4(0, s) == (5.0, 7.0)
    assert O.scale_min_k4(4, s) == (float(0xA | (3 << 4)), 2.0)


def test_q4k_block_is_d_sc_q_minus_dmin_m():
    """quant.rs:702-716."""
    scales = [0] * 12
    scales[0], scales[4] = 2, 4
    b = np.array(f16b(0.5) + f16b(0.25) + scales + [0x31] * 128, np.uint8)
    out = O.dequant_block(O.Q4K, b)
    assert out[0] == 0.5 * 2.0 * 1.0 - 0.25 * 4.0
    assert out[32] == 0.0


def test_q6k_block():
    """quant.rs:718-729."""
    b = np.zeros(210, np.uint8)
    b[0], b[128], b[192] = 0x05, 0x02, 3
    b[208:210] = f16b(0.5)
    out = O.dequant_block(O.Q6K, b)
    assert out[0] == 0.5 * 3.0 * (37.0 - 32.0)
    assert out[1] == 0.5 * 3.0 * -32.0


# ---- An independent numpy dequantisation (whole tensors, bit slicing per layout). ----

def _f16(u8: np.ndarray) -> np.ndarray:
    return u8.copy().view(np.float16).astype(np.float32)


def np_dequant(ty: int, data: np.ndarray, rows: int, cols: int) -> np.ndarray:
    n, size = O.block(ty)
    blk = data.reshape(-1, size)
    if ty == O.F32:
        return blk.copy().view(np.float32).reshape(rows, cols)
    if ty == O.F16:
        return _f16(blk).reshape(rows, cols)
    if ty == O.BF16:
        return (blk.copy().view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(rows, cols)
    if ty in (O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1, O.Q8_0):
        d = _f16(blk[:, 0:2]).reshape(-1, 1)
        if ty == O.Q8_0:
            q = blk[:, 2:34].view(np.int8).astype(np.float32)
            return (q * d).reshape(rows, cols)
        has_m = ty in (O.Q4_1, O.Q5_1)
        m = _f16(blk[:, 2:4]).reshape(-1, 1) if has_m else np.float32(0.0)
        at = 4 if has_m else 2
        five = ty in (O.Q5_0, O.Q5_1)
        qs = blk[:, at + 4 * five:at + 4 * five + 16].astype(np.uint32)
        q = np.concatenate([qs & 15, qs >> 4], axis=1)  # element j: low nibble, j + 16: high
        if five:
            qh = blk[:, at:at + 4].copy().view("<u4").astype(np.uint32).reshape(-1, 1)
            q = q | (((qh >> np.arange(32, dtype=np.uint32)) & 1) << 4)  # element i takes bit i
        off = np.float32(8.0 if ty == O.Q4_0 else 16.0 if ty == O.Q5_0 else 0.0)
        return ((q.astype(np.float32) - off) * d + m).reshape(rows, cols)
    if ty in (O.Q4K, O.Q5K):
        d = _f16(blk[:, 0:2]).reshape(-1, 1)
        dmin = _f16(blk[:, 2:4]).reshape(-1, 1)
        s = blk[:, 4:16].astype(np.uint32)
        sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)], axis=1)
        mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        qs = blk[:, 16:144] if ty == O.Q4K else blk[:, 48:176]
        qs = qs.astype(np.uint32).reshape(-1, 4, 32)
        q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32)  # sub-block 2c: low, 2c+1: high
        if ty == O.Q5K:
            qh = blk[:, 16:48].astype(np.uint32).reshape(-1, 1, 32)
            q = q + (((qh >> np.arange(8, dtype=np.uint32).reshape(1, 8, 1)) & 1) << 4)
        w = (d.reshape(-1, 1, 1) * sc.astype(np.float32).reshape(-1, 8, 1)) * q.astype(np.float32) \
            - (dmin.reshape(-1, 1, 1) * mn.astype(np.float32).reshape(-1, 8, 1))
        return w.reshape(rows, cols)
    if ty == O.Q6K:
        ql = blk[:, 0:128].astype(np.int32).reshape(-1, 2, 64)
        qh = blk[:, 128:192].astype(np.int32).reshape(-1, 2, 32)
        sc = blk[:, 192:208].view(np.int8).astype(np.float32).reshape(-1, 2, 8)
        d = _f16(blk[:, 208:210]).reshape(-1, 1, 1)
        q = np.stack([(ql[:, :, :32] & 15) | ((qh & 3) << 4), (ql[:, :, 32:] & 15) | (((qh >> 2) & 3) << 4),
                      (ql[:, :, :32] >> 4) | (((qh >> 4) & 3) << 4), (ql[:, :, 32:] >> 4) | (((qh >> 6) & 3) << 4)],
                     axis=2) - 32  # [blk][half][quarter][l]
        s = sc.reshape(-1, 2, 4, 2)[:, :, :, :, None].repeat(16, axis=4).reshape(-1, 2, 4, 32)  # l // 16
        return ((d.reshape(-1, 1, 1, 1) * s) * q.astype(np.float32)).reshape(rows, cols)
    raise ValueError(ty)


@pytest.mark.parametrize("ty", O.GGML_TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_dequant_matches_independent_numpy(ty):
    rows, cols = 5, 512
    data = O.random_tensor(ty, rows, cols, 3)
    got = O.dequant(ty, data, rows, cols)
    want = np_dequant(ty, data, rows, cols)
    np.testing.assert_array_equal(got, want, err_msg=O.TYPE_NAMES[ty])


@pytest.mark.parametrize("ty", O.GGML_TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_random_tensor_fixture(ty):
    """fixtures.rs:66-92: seeded, deterministic, modest scales (so products stay finite)."""
    a = O.random_tensor(ty, 3, 256, 7)
    assert a.size == 3 * O.row_bytes(ty, 256)
    np.testing.assert_array_equal(a, O.random_tensor(ty, 3, 256, 7))
    assert not np.array_equal(a, O.random_tensor(ty, 3, 256, 8))
    w = O.dequant(ty, a, 3, 256)
    assert np.isfinite(w).all()
    lim = 1.0 if ty in (O.F32, O.F16, O.BF16) else 0.025 * 64 * 64
    assert np.abs(w).max() <= lim


def test_matmul_f64_is_the_dequantized_product():
    for ty in (O.Q8_0, O.Q4K, O.Q6K, O.F16):
        rows, cols, n = 7, 512, 3
        data = O.random_tensor(ty, rows, cols, 11)
        x = (np.arange(n * cols, dtype=np.float32) * 31 % 97 - 48) / 50
        got = O.matmul_f64(ty, data, rows, cols, x, n)
        w = np_dequant(ty, data, rows, cols).astype(np.float64)
        want = x.reshape(n, cols).astype(np.float64) @ w.T
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_rms_norm_silu_bias_add():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    w = rng.standard_normal(96).astype(np.float32)
    got = O.rms_norm(x, w, 1e-5)
    ms = (x.astype(np.float64) ** 2).mean(axis=1, keepdims=True)
    want = x / np.sqrt(ms + 1e-5) * w
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-6)
    g, u = rng.standard_normal(300).astype(np.float32) * 4, rng.standard_normal(300).astype(np.float32)
    np.testing.assert_allclose(O.silu_mul(g, u), g / (1 + np.exp(-g.astype(np.float64))) * u, rtol=1e-6, atol=1e-7)
    b = rng.standard_normal(96).astype(np.float32)
    np.testing.assert_array_equal(O.bias_add(x, b), x + b)
    np.testing.assert_array_equal(O.add(x, w.reshape(1, 96).repeat(3, 0)), x + w)
