"""The rest of a layer on the GPU against the oracle: the GGUF block-format product in
every format (k_matmul, gpu/kernels.h:51-214, checked as Gpu::self_check checks it,
gpu/mod.rs:181-206: within 1e-3 * (1 + |want|) of the f64 dequantized product), on the VALU
for one input row and on the matrix cores for batches of 2 or more (the reference's own
batched product from MM_FROM = 2 rows, gpu/mod.rs:33-41), its batch invariance and determinism
(kernels.h:9-11), matmul_rows (gpu/mod.rs:163-178), RMSNorm (model.rs:381-388) and the
elementwise ops (model.rs:337, 343, 371-377)."""
import numpy as np
import pytest

import bchip
import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = bchip.Ctx(0)
    yield c
    c.close()


def selfcheck_x(n: int, cols: int) -> np.ndarray:
    """gpu/mod.rs:188: the self-check's input rows."""
    i = np.arange(n * cols, dtype=np.int64)
    return (((i * 31 % 97).astype(np.float32) - 48.0) / 50.0).reshape(n, cols)


def product(ctx, ty, data, rows, cols, x, n):
    wb, xb, ob = ctx.upload(data), ctx.upload(np.ascontiguousarray(x, np.float32)), ctx.zeros(n * rows * 4)
    ctx.matmul(wb, ty, xb, ob, rows, cols, n)
    got = ctx.read(ob, (n, rows))
    for b in (wb, xb, ob):
        b.free()
    return got


def within_selfcheck(got, want, what):
    err = np.abs(got.astype(np.float64) - want)
    bound = 1e-3 * (1.0 + np.abs(want))
    worst = np.unravel_index(np.argmax(err / bound), err.shape)
    assert (err <= bound).all(), f"{what}: got {got[worst]}, want {want[worst]} at {worst}"


MM_TYPES = [O.F16, O.Q8_0, O.Q4_0, O.Q4_1, O.Q5_0, O.Q5_1, O.Q4K, O.Q5K, O.Q6K]  # matrix cores for n >= 2


@pytest.mark.parametrize("ty", O.GGML_TYPES, ids=lambda t: O.TYPE_NAMES[t])
def test_product_matches_self_check(ctx, ty):
    """Gpu::self_check's shapes (37 x 512, seed 7) and bound, at n = 1 and 3 (the self-check's)
    and n = 8 and 17 (batches: the matrix-core product where the format has one)."""
    rows, cols = 37, 512
    data = O.random_tensor(ty, rows, cols, 7)
    for n in (1, 3, 8, 17):
        x = selfcheck_x(n, cols)
        got = product(ctx, ty, data, rows, cols, x, n)
        within_selfcheck(got, O.matmul_f64(ty, data, rows, cols, x, n), f"{O.TYPE_NAMES[ty]} n={n}")


@pytest.mark.parametrize("ty", MM_TYPES + [O.BF16, O.F32], ids=lambda t: O.TYPE_NAMES[t])
def test_product_at_model_widths(ctx, ty):
    """Model-width rows (4096 weights: 128 groups), a row count that is not a multiple of a
    workgroup's 16, and 13 and 5 input rows (the matrix cores; BF16 and F32 in VALU passes of
    8)."""
    rows, cols = 301, 4096
    data = O.random_tensor(ty, rows, cols, 5)
    for n in (13, 5):
        x = np.random.default_rng(3 + n).standard_normal((n, cols)).astype(np.float32)
        got = product(ctx, ty, data, rows, cols, x, n)
        within_selfcheck(got, O.matmul_f64(ty, data, rows, cols, x, n), f"{O.TYPE_NAMES[ty]} n={n}")


@pytest.mark.parametrize("ty", [O.Q4K, O.Q4_0, O.Q6K, O.F16, O.BF16], ids=lambda t: O.TYPE_NAMES[t])
def test_product_rows_do_not_depend_on_the_batch(ctx, ty):
    """kernels.h:9-11: a row's result never depends on how many rows share the batch, and
    reruns give the same bits: among batches of 2 or more (the matrix-core product: the same
    row at another place of another batch), and one-row passes among themselves. A batch row
    agrees with the same row passed alone within rounding, as the reference's does
    (gpu/mod.rs:35-37: its batched product sums in another order too); BF16 (no matrix-core
    form) gives the same bits either way."""
    rows, cols, n = 70, 1024, 19
    data = O.random_tensor(ty, rows, cols, 9)
    x = np.random.default_rng(4).standard_normal((n, cols)).astype(np.float32)
    whole = product(ctx, ty, data, rows, cols, x, n)
    np.testing.assert_array_equal(whole, product(ctx, ty, data, rows, cols, x, n))
    np.testing.assert_array_equal(product(ctx, ty, data, rows, cols, x[3:11], 8), whole[3:11])
    np.testing.assert_array_equal(product(ctx, ty, data, rows, cols, x[5:19], 14), whole[5:19])
    np.testing.assert_array_equal(product(ctx, ty, data, rows, cols, x[3:10], 7), whole[3:10])
    np.testing.assert_array_equal(product(ctx, ty, data, rows, cols, x[4:6], 2), whole[4:6])
    alone = np.stack([product(ctx, ty, data, rows, cols, x[i:i + 1], 1)[0] for i in range(3, 10)])
    np.testing.assert_array_equal(product(ctx, ty, data, rows, cols, x[5:6], 1)[0], alone[2])
    if ty not in MM_TYPES:
        np.testing.assert_array_equal(alone, whole[3:10])
        return
    # Both are f32 sums of the same terms in other orders (each within ~3e-7 of the f64
    # product, relative to the row's largest output): bound the difference by the row's scale.
    top = 1.0 + np.abs(whole[3:10].astype(np.float64)).max(axis=1, keepdims=True)
    d = np.abs(alone.astype(np.float64) - whole[3:10]) / top
    print(f"{O.TYPE_NAMES[ty]}: a batch row against the same row passed alone: {d.max():.3g} of the row's scale",
          flush=True)
    assert d.max() <= 2e-6


@pytest.mark.parametrize("ty", [O.Q4K, O.Q8_0, O.Q6K], ids=lambda t: O.TYPE_NAMES[t])
def test_product_k_splits_serial_and_parallel_agree(ctx, ty):
    """The matrix-core product splits K the same way whatever n is; few tiles run the splits
    in parallel and the last workgroup of a tile adds them, many tiles run them one after
    another in one workgroup: the same bits either way (1100 rows x 456 inputs is past the
    parallel limit of 1024 tiles of 64 rows x 8 inputs; 8 and 16 inputs are within it)."""
    rows, cols, n = 1100, 512, 456
    data = O.random_tensor(ty, rows, cols, 11)
    x = np.random.default_rng(8).standard_normal((n, cols)).astype(np.float32)
    whole = product(ctx, ty, data, rows, cols, x, n)
    np.testing.assert_array_equal(product(ctx, ty, data, rows, cols, x[:8], 8), whole[:8])
    np.testing.assert_array_equal(product(ctx, ty, data, rows, cols, x[440:456], 16), whole[440:456])
    within_selfcheck(whole[::57], O.matmul_f64(ty, data, rows, cols, x[::57], len(x[::57])), O.TYPE_NAMES[ty])


def test_f16_subnormal_weights_on_the_matrix_cores(ctx):
    """F16 weights below 2^-14 (subnormal) count in the matrix-core product as they do on the
    VALU: a batch of 8 against one-row passes over weights of scale 2e-5 (most subnormal)."""
    rows, cols = 64, 1024
    w = (np.random.default_rng(12).standard_normal((rows, cols)) * 2e-5).astype(np.float16)
    assert (np.abs(w) < 2.0 ** -14).mean() > 0.9
    x = np.random.default_rng(13).standard_normal((8, cols)).astype(np.float32)
    wb = w.view(np.uint8).reshape(-1)
    batch = product(ctx, O.F16, wb, rows, cols, x, 8)
    small = np.stack([product(ctx, O.F16, wb, rows, cols, x[i:i + 1], 1)[0] for i in range(7)])
    top = np.abs(small.astype(np.float64)).max(axis=1, keepdims=True)
    d = np.abs(batch[:7].astype(np.float64) - small) / top
    print(f"F16 subnormal weights: batch against VALU pass {d.max():.3g} of the row's scale", flush=True)
    assert d.max() <= 2e-6


def test_matmul_rows_is_the_first_rows(ctx):
    """gpu/mod.rs:163-178: the product against the first `rows` weight rows only."""
    ty, rows, cols, n = O.Q6K, 50, 512, 2
    data = O.random_tensor(ty, rows, cols, 2)
    x = selfcheck_x(n, cols)
    whole = product(ctx, ty, data, rows, cols, x, n)
    part = product(ctx, ty, data[:17 * O.row_bytes(ty, cols)], 17, cols, x, n)
    np.testing.assert_array_equal(part, whole[:, :17])


def test_product_refuses_bad_shapes(ctx):
    wb, xb, ob = ctx.zeros(4096), ctx.zeros(4096), ctx.zeros(4096)
    with pytest.raises(bchip.BchipError):
        ctx.matmul(wb, 5, xb, ob, 1, 32, 1)  # not a ggml type this library takes
    with pytest.raises(bchip.BchipError):
        ctx.matmul(wb, O.Q4K, xb, ob, 1, 128, 1)  # K-quant rows are whole 256-blocks
    with pytest.raises(bchip.BchipError):
        ctx.matmul(wb, O.F32, xb, ob, 1, 48, 1)  # groups of 32
    with pytest.raises(bchip.BchipError):
        ctx.matmul(wb, O.Q8_0, xb, ob, 200, 256, 1)  # weights pass the end of their buffer
    with pytest.raises(bchip.BchipError):
        ctx.matmul(wb, O.F32, xb, ob, 1, 32, 8 * 65535 + 1)  # more input rows than a call takes
    for b in (wb, xb, ob):
        b.free()


@pytest.mark.parametrize("rows,cols", [(3, 4096), (5, 896), (2, 37)])
def test_rms_norm_matches_oracle(ctx, rows, cols):
    rng = np.random.default_rng(cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    w = (1.0 + 0.2 * rng.standard_normal(cols)).astype(np.float32)
    xb, wb, ob = ctx.upload(x), ctx.upload(w), ctx.zeros(x.nbytes)
    ctx.rms_norm(xb, wb, ob, rows, cols, 1e-5)
    got = ctx.read(ob, x.shape)
    # The sum of squares is a different f32 order from the reference's 8-lane dot.
    np.testing.assert_allclose(got, O.rms_norm(x, w, 1e-5), rtol=2e-6, atol=1e-6)
    for b in (xb, wb, ob):
        b.free()


def test_elementwise_ops_match_oracle(ctx):
    rng = np.random.default_rng(7)
    n, dim = 3 * 1000 + 7, 1000
    x = rng.standard_normal(n).astype(np.float32) * 4
    y = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(dim).astype(np.float32)
    xb, yb, bb = ctx.upload(x), ctx.upload(y), ctx.upload(b)
    ctx.bias_add(xb, bb, n, dim)
    np.testing.assert_array_equal(ctx.read(xb, n), O.bias_add(x, b))
    ctx.upload(x, xb)
    ctx.add(xb, yb, n)
    np.testing.assert_array_equal(ctx.read(xb, n), O.add(x, y))
    ctx.upload(x, xb)
    ctx.silu_mul(xb, yb, n)
    # e^-v on the hardware's exp2 (the reference GPU's EXP, cuda.cu:66) against libm's expf.
    np.testing.assert_allclose(ctx.read(xb, n), O.silu_mul(x, y), rtol=4e-6, atol=1e-7)
    for buf in (xb, yb, bb):
        buf.free()
