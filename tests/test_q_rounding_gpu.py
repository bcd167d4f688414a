"""Every kernel rounds a query element the same way on its way to the f16 MFMA operand:
q * sc rounded to f32, then to f16 (sc = scale * log2(e) in f32). A single rounding of the
exact product (what a mixed-precision FMA, v_fma_mixlo_f16, gives) differs from the two
roundings where the f32 product falls exactly between two f16 values; the compiler chose
one form or the other per kernel, so queries carrying such elements are what the bit-exact
invariants between kernels need: the fused step against its two calls (gpu/mod.rs:464-482),
tree rows against their lines (model.rs:538-579), a split verify against a larger pass."""
import math

import numpy as np
import pytest

import bchip
import oracle as O

LOG2E = np.float32(1.4426950408889634)


def sc32(scale):
    """The kernels' score scale: scale * log2(e), one f32 multiplication."""
    return np.float32(np.float32(scale) * LOG2E)


def midpoint_values(scale, count, seed):
    """f32 values x of about unit size whose f32 product with sc32(scale) lies exactly
    between two f16 values, with the exact product on the side that makes f16(f32(x sc))
    and f16(x sc) differ: for midpoints m of random adjacent f16 pairs, x = m / sc and its
    two f32 neighbours, kept where they qualify."""
    sc = sc32(scale)
    rng = np.random.default_rng(seed)
    found, total = [], 0
    while total < count:
        a = np.abs(rng.standard_normal(2 * count + 64) * float(sc)).astype(np.float16)
        a = a[a >= np.float16(2.0 ** -14)]  # normal f16
        b = np.nextafter(a, np.float16(np.inf))
        m = (a.astype(np.float32) + b.astype(np.float32)) / np.float32(2)  # exact
        m = np.where(rng.random(m.size) < 0.5, -m, m).astype(np.float32)
        x0 = (m.astype(np.float64) / np.float64(sc)).astype(np.float32)
        for x in (x0, np.nextafter(x0, np.float32(np.inf)), np.nextafter(x0, np.float32(-np.inf))):
            p = x * sc  # float32 * float32: rounded to f32
            exact = x.astype(np.float64) * np.float64(sc)  # exact: 24 x 24 bits
            ok = (p == m) & (exact.astype(np.float16) != p.astype(np.float16))
            found.append(x[ok])
            total += int(ok.sum())
    return np.concatenate(found)[:count]


def plant(q, scale, seed, every=4, dims=slice(None)):
    """q with every `every`-th element of the given dims replaced by a midpoint value."""
    q = q.copy()
    view = q[..., dims]
    flat = view.reshape(-1)
    idx = np.arange(0, flat.size, every)
    flat[idx] = midpoint_values(scale, idx.size, seed)
    q[..., dims] = flat.reshape(view.shape)
    return q


def test_midpoint_values_round_differently():
    """The values the GPU tests plant: for each, the two roundings give different f16."""
    scale = 1.0 / math.sqrt(128)
    x = midpoint_values(scale, 256, 1)
    p = x * sc32(scale)
    assert x.size == 256 and np.all(np.abs(x) < 8)
    assert np.all(p.astype(np.float16) != (x.astype(np.float64) * np.float64(sc32(scale))).astype(np.float16))
    # the f32 product sits exactly on an f16 midpoint: half an f16 unit from both neighbours
    lo = p.astype(np.float16)
    ulp = np.spacing(np.abs(lo)).astype(np.float64)
    assert np.all(np.abs(np.abs(p.astype(np.float64) - lo.astype(np.float64)) - ulp / 2) == 0)


@pytest.fixture(scope="module")
def ctx():
    c = bchip.Ctx(0)
    yield c
    c.close()


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("pos", [63, 4096])
def test_fused_step_and_its_two_calls_round_q_alike(ctx, pos):
    """RoPE over the first 64 of 128 dims leaves dims 64-127 as given: they carry the
    planted values into both paths (the fused kernel's q conversion, the two-call path's)."""
    nh, nkv, hd, rd = 32, 8, 128, 64
    kvd = nkv * hd
    scale = 1.0 / math.sqrt(hd)
    q = plant(rand((1, nh, hd), 1), scale, 2, dims=slice(rd, hd)).reshape(1, nh * hd)
    k, v = rand((1, kvd), 3), rand((1, kvd), 4)
    kc0, vc0 = rand((pos + 1, kvd), 5).astype(np.float16), rand((pos + 1, kvd), 6).astype(np.float16)
    ib, pb = ctx.upload(O.inv_freq(rd, 5e5)), ctx.upload(np.array([pos], np.uint32))
    kb, vb = ctx.upload(k), ctx.upload(v)
    outs = []
    for fused in (False, True):
        qb, kcb, vcb, ob = ctx.upload(q), ctx.upload(kc0), ctx.upload(vc0), ctx.zeros(nh * hd * 4)
        if fused:
            ctx.rope_append_attention(qb, kb, vb, kcb, vcb, bchip.F16, ib, pb, nh, nkv, hd, rd, False, pos, scale, ob)
        else:
            ctx.rope_append(qb, kb, vb, kcb, vcb, bchip.F16, ib, pb, 1, nh, nkv, hd, rd, False, pos)
            ctx.attention(qb, kcb, vcb, bchip.F16, ob, None, False, 1, nh, nkv, hd, pos, scale)
        outs.append(ctx.read(ob, (nh, hd)))
        for b in (qb, kcb, vcb, ob):
            b.free()
    np.testing.assert_array_equal(outs[1], outs[0])
    for b in (ib, pb, kb, vb):
        b.free()


def run(ctx, q, kc, vc, rows, pos, nh, nkv, hd, scale, visible=None):
    qb, kb, vb = ctx.upload(np.ascontiguousarray(q)), ctx.upload(kc), ctx.upload(vc)
    ob = ctx.zeros(rows * nh * hd * 4)
    mb = ctx.upload(bchip.masks_words(visible)) if visible is not None else None
    ctx.attention(qb, kb, vb, bchip.F16, ob, mb, visible is not None, rows, nh, nkv, hd, pos, scale)
    got = ctx.read(ob, (rows, nh, hd))
    for b in (qb, kb, vb, ob) + ((mb,) if mb is not None else ()):
        b.free()
    return got


@pytest.mark.gpu
def test_tree_rows_and_their_lines_round_q_alike(ctx):
    """Tree rows (attn_decode) against the lines their paths are (chunked multi-row passes)."""
    nh, nkv, hd, prefix = 32, 8, 128, 700
    scale = 1.0 / math.sqrt(hd)
    tree = [O.ROOT, 0, 0, 1, O.ROOT]
    rows = len(tree)
    _, visible, base = O.shape(rows, prefix, tree)
    n = prefix + rows
    q = plant(rand((rows, nh, hd), 11), scale, 12)
    kc, vc = rand((n, nkv * hd), 13).astype(np.float16), rand((n, nkv * hd), 14).astype(np.float16)
    got = run(ctx, q, kc, vc, rows, base, nh, nkv, hd, scale, visible)
    for row, path in enumerate([[0], [0, 1], [0, 2], [0, 1, 3], [4]]):
        m = prefix + len(path)
        lk = np.concatenate([kc[:prefix], kc[[prefix + p for p in path]]])
        lv = np.concatenate([vc[:prefix], vc[[prefix + p for p in path]]])
        lq = rand((m, nh, hd), 15)
        lq[-1] = q[row]
        want = run(ctx, lq, lk, lv, m, 0, nh, nkv, hd, scale)
        np.testing.assert_array_equal(got[row], want[-1], err_msg=f"row {row}, path {path}")


@pytest.mark.gpu
def test_verify_rows_and_a_larger_pass_round_q_alike(ctx):
    """8 verify rows (four-wave kernel, split by chunk) against the same rows in a pass of 200
    (eight-wave kernel) at 64/8 heads."""
    nh, nkv, hd, pos = 64, 8, 128, 3000
    scale = 1.0 / math.sqrt(hd)
    n = pos + 200
    q = plant(rand((200, nh, hd), 21), scale, 22)
    kc, vc = rand((n, nkv * hd), 23).astype(np.float16), rand((n, nkv * hd), 24).astype(np.float16)
    whole = run(ctx, q, kc, vc, 200, pos, nh, nkv, hd, scale)
    for v0 in (0, 96, 192):
        part = run(ctx, q[v0:v0 + 8], kc, vc, 8, pos + v0, nh, nkv, hd, scale)
        np.testing.assert_array_equal(part, whole[v0:v0 + 8], err_msg=f"rows {v0}..")
