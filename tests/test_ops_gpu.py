"""The cache-side operators on the GPU against the oracle and the reference semantics:
k_rope (kernels.h:235-248), the fused RoPE + KV append (gpu/mod.rs:464-475), k_copy /
k_move (kernels.h:332-334), Cache::keep (gpu/mod.rs:322-337) and the seeded generator."""
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


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("neox,hd,rd,theta", [(False, 128, 128, 5e5), (True, 64, 64, 1e6), (True, 128, 96, 1e4),
                                              (False, 16, 16, 1e4)])
def test_rope_matches_oracle(ctx, neox, hd, rd, theta):
    rows, heads = 6, 5
    positions = np.array([0, 1, 511, 4097, 32767, 40000], np.uint32)
    x = rand((rows, heads * hd), 1)
    inv = O.inv_freq(rd, theta)
    xb, ib, pb = ctx.upload(x), ctx.upload(inv), ctx.upload(positions)
    ctx.rope(xb, ib, pb, rows, heads, hd, rd, neox)
    got = ctx.read(xb, x.shape)
    want = O.rope_rows(x, positions, heads, hd, rd, neox, inv)
    # theta and the products round as the reference does; sin/cos may differ in the last bit.
    np.testing.assert_allclose(got, want, atol=2e-6, rtol=0)
    np.testing.assert_array_equal(got[0], x[0])  # position 0 is the identity
    for b in (xb, ib, pb):
        b.free()


@pytest.mark.parametrize("kv_type", [bchip.F32, bchip.F16])
@pytest.mark.parametrize("neox,rd", [(False, 128), (True, 64)])
def test_rope_append_is_the_four_reference_launches(ctx, kv_type, neox, rd):
    rows, nh, nkv, hd, slot0, cap = 4, 32, 8, 128, 37, 64
    positions = np.arange(slot0, slot0 + rows, dtype=np.uint32)
    q, k, v = rand((rows, nh * hd), 2), rand((rows, nkv * hd), 3), rand((rows, nkv * hd), 4)
    inv = O.inv_freq(rd, 5e5)
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    kc0 = rand((cap, nkv * hd), 5).astype(dt)
    vc0 = rand((cap, nkv * hd), 6).astype(dt)
    qb, kb, vb = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    kcb, vcb = ctx.upload(kc0), ctx.upload(vc0)
    ib, pb = ctx.upload(inv), ctx.upload(positions)
    ctx.rope_append(qb, kb, vb, kcb, vcb, kv_type, ib, pb, rows, nh, nkv, hd, rd, neox, slot0)
    gq = ctx.read(qb, q.shape)
    gk = ctx.read(kcb, kc0.shape, dt).astype(np.float32)
    gv = ctx.read(vcb, vc0.shape, dt).astype(np.float32)
    # The same rotation as bchip_rope, bit for bit (one code path).
    q2 = ctx.upload(q)
    ctx.rope(q2, ib, pb, rows, nh, hd, rd, neox)
    np.testing.assert_array_equal(gq, ctx.read(q2, q.shape))
    np.testing.assert_allclose(gq, O.rope_rows(q, positions, nh, hd, rd, neox, inv), atol=2e-6, rtol=0)
    kr = O.rope_rows(k, positions, nkv, hd, rd, neox, inv)
    want_k = kc0.astype(np.float32).copy()
    want_v = vc0.astype(np.float32).copy()
    want_k[slot0:slot0 + rows] = kr.astype(dt).astype(np.float32)
    want_v[slot0:slot0 + rows] = v.astype(dt).astype(np.float32)
    tol = 2e-6 if kv_type == bchip.F32 else 1e-3
    np.testing.assert_allclose(gk, want_k, atol=tol, rtol=0)
    np.testing.assert_array_equal(gv, want_v)
    np.testing.assert_array_equal(ctx.read(kb, k.shape), k)  # k and v are read only
    for b in (qb, kb, vb, kcb, vcb, ib, pb, q2):
        b.free()


def test_copy_converts_and_offsets(ctx):
    x = rand(1000, 7)
    src = ctx.upload(x)
    for dt, npt in ((bchip.F32, np.float32), (bchip.F16, np.float16)):
        dst = ctx.zeros(1200 * (4 if dt == bchip.F32 else 2))
        ctx.copy(src, bchip.F32, dst, dt, 150, 1000)
        got = ctx.read(dst, 1200, npt)
        np.testing.assert_array_equal(got[150:1150], x.astype(npt))
        assert not got[:150].any() and not got[1150:].any()
        back = ctx.zeros(4000)
        ctx.copy(dst.ptr + 150 * bchip.esize(dt), dt, back, bchip.F32, 0, 1000)
        np.testing.assert_array_equal(ctx.read(back, 1000), x.astype(npt).astype(np.float32))
        dst.free()
        back.free()
    src.free()


@pytest.mark.parametrize("dt,npt", [(bchip.F32, np.float32), (bchip.F16, np.float16)])
def test_move_including_overlap(ctx, dt, npt):
    for frm, to, n in ((500, 100, 300), (130, 100, 300), (101, 100, 50), (100, 100, 10)):
        x = rand(1000, frm + to).astype(npt)
        b = ctx.upload(x)
        ctx.move(b, dt, frm, to, n)
        want = x.copy()
        want[to:to + n] = x[frm:frm + n].copy()
        np.testing.assert_array_equal(ctx.read(b, 1000, npt), want, err_msg=f"{frm}->{to} x{n}")
        b.free()


@pytest.mark.parametrize("dt,npt", [(bchip.F32, np.float32), (bchip.F16, np.float16)])
def test_keep_matches_kv_keep(ctx, dt, npt):
    width, slots, base = 256, 20, 6
    rows = [0, 2, 3, 7, 9]
    layers = [rand((slots, width), 11 + i).astype(npt) for i in range(6)]
    bufs = [ctx.upload(x) for x in layers]
    ctx.keep(bufs, dt, width, base, rows)
    for x, b in zip(layers, bufs):
        want = x.astype(np.float32).ravel().copy()
        n = O.keep(want, width, slots, base, rows)
        got = ctx.read(b, x.shape, npt).astype(np.float32)
        np.testing.assert_array_equal(got[:n], want.reshape(slots, width)[:n])
        b.free()


def test_fill_normal_is_the_oracle_generator(ctx):
    n = 100001
    b = ctx.zeros(n * 4)
    ctx.fill_normal(b, bchip.F32, n, 77)
    got = ctx.read(b, n)
    want = O.normal(77, n)
    np.testing.assert_allclose(got, want, rtol=2e-7, atol=1e-7)
    assert (got == want).mean() > 0.99
    b.free()


def test_offsets_that_overflow_are_refused_before_any_launch(ctx):
    """Slot offsets whose byte spans overflow 64 bits, or wrap the address space, must fail the
    argument checks (BCHIP_E_ARG) rather than wrap into a span that passes them. Nothing is
    launched: each call is refused on the host."""
    nh, nkv, hd, rd = 4, 2, 64, 64
    kvd = nkv * hd
    q, k, v = rand((2, nh * hd), 11), rand((2, kvd), 12), rand((2, kvd), 13)
    qb, kb, vb = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    kc, vc = ctx.zeros(64 * kvd * 2), ctx.zeros(64 * kvd * 2)
    ib = ctx.upload(O.inv_freq(rd, 1e4))
    pb = ctx.upload(np.array([5, 6], np.uint32))
    out = ctx.zeros(2 * nh * hd * 4)
    # (offset + rows) * kvd * 2 wraps to a small number for these offsets.
    wraps = [(1 << 64) // (kvd * 2) - 1, (1 << 63) + 1, (1 << 64) - 2]

    def refused(fn):
        with pytest.raises(bchip.BchipError) as e:
            fn()
        assert e.value.code == bchip.E_ARG, bchip.last_error()

    for off in wraps:
        refused(lambda: ctx.rope_append(qb, kb, vb, kc, vc, bchip.F16, ib, pb, 1, nh, nkv, hd, rd, True, off))
        refused(lambda: ctx.rope_append_ragged(qb, kb, vb, kc, vc, bchip.F16, ib, pb, [3], [off], nh, nkv, hd, rd,
                                               True))
        refused(lambda: ctx.rope_append_attention_ragged(qb, kb, vb, kc, vc, bchip.F16, ib, pb, [3], [off], nh, nkv,
                                                         hd, rd, True, 0.125, out))
        refused(lambda: ctx.attention_ragged(qb, kc, vc, bchip.F16, out, [3], [off], nh, nkv, hd, 0.125))
        refused(lambda: ctx.copy(kb, bchip.F32, kc, bchip.F16, off, 8))
        refused(lambda: ctx.move(kc, bchip.F16, off, 0, 8))
        refused(lambda: ctx.fill_normal(kc, bchip.F16, off, 1))
    with pytest.raises(bchip.BchipError):
        ctx.read(kc, (4,), np.float16, off=(1 << 64) - 4)
    # The caches are untouched: every call above was refused before it launched anything.
    np.testing.assert_array_equal(ctx.read(kc, (64 * kvd,), np.float16), 0)
    for b in (qb, kb, vb, kc, vc, ib, pb, out):
        b.free()
