"""KV-cache management on the GPU: the growth step of Gpu::reserve (gpu/mod.rs:404-423) for
every layer's K and V in one launch (bchip_cache_grow), and the host mirror of the
reference's Cache (mod.rs:300-337, 398-423): capacity by doubling, the kept prefix carried
over bit for bit, the new tail zero, Cache::keep after a growth, and attention over a grown
cache giving the bits of the same tokens in a fresh one."""
import math

import numpy as np
import pytest

import bchip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = bchip.Ctx(0)
    yield c
    c.close()


@pytest.mark.parametrize("t,dtype", [(bchip.F16, np.float16), (bchip.F32, np.float32)])
def test_grow_keeps_the_prefix_and_zeroes_the_tail(ctx, t, dtype):
    rng = np.random.default_rng(3)
    keep, total = 1001, 4999  # neither a whole 16-byte piece: the straddling piece goes byte by byte
    srcs = [rng.standard_normal(keep).astype(dtype) for _ in range(3)]
    sb = [ctx.upload(s) for s in srcs]
    db = [ctx.upload(np.full(total, 7, dtype)) for _ in range(3)]
    ctx.cache_grow(sb, db, t, keep, total)
    for s, d in zip(srcs, db):
        got = ctx.read(d, total, dtype)
        np.testing.assert_array_equal(got[:keep].view(np.uint8), s.view(np.uint8))
        assert not got[keep:].any()
    # Nothing kept: no source, every element zero.
    ctx.cache_grow(None, db[:1], t, 0, total)
    assert not ctx.read(db[0], total, dtype).any()
    for b in sb + db:
        b.free()


def test_grow_refuses_bad_arguments(ctx):
    a, b = ctx.zeros(4096), ctx.zeros(4096)
    with pytest.raises(bchip.BchipError):
        ctx.cache_grow([a], [b], bchip.F32, 11, 10)  # keep past total
    with pytest.raises(bchip.BchipError):
        ctx.cache_grow([a], [a], bchip.F32, 10, 20)  # a buffer onto itself
    with pytest.raises(bchip.BchipError):
        ctx.cache_grow([a], [b.ptr + 4], bchip.F32, 10, 20)  # not 16-byte aligned
    with pytest.raises(bchip.BchipError):
        ctx.cache_grow([a], [b], bchip.F32, 10, 2000)  # past the destination's end
    with pytest.raises(bchip.BchipError):
        ctx.cache_grow([a], [b], 2, 10, 20)  # not f32 or f16
    for x in (a, b):
        x.free()


def test_cache_reserve_keep_and_attention(ctx):
    """A cache filled to 300 tokens, grown for 400 (capacity 600, the first 300 kept), then
    Cache::keep of an accepted path, then attention over the grown cache against the same
    tokens uploaded into a fresh buffer: the same bits."""
    n_layer, nh, nkv, hd, context = 2, 8, 2, 64, 4096
    kvd = nkv * hd
    rng = np.random.default_rng(11)
    cache = bchip.KvCache(ctx, n_layer, kvd, bchip.F16)
    cache.reserve(300, 0, context)
    assert cache.cap == 300 and cache.bytes() == n_layer * 2 * 300 * kvd * 2
    data = [rng.standard_normal((300, kvd)).astype(np.float16) for _ in range(2 * n_layer)]
    for buf, d in zip(cache.k + cache.v, data):
        ctx.upload(d, buf)
    cache.reserve(400, 300, context)
    assert cache.cap == 600
    for buf, d in zip(cache.k + cache.v, data):
        got = ctx.read(buf, (600, kvd), np.float16)
        np.testing.assert_array_equal(got[:300].view(np.uint16), d.view(np.uint16))
        assert not got[300:].any()
    # The reference's keep: rows 290 + [0, 2, 5] move to 290, 291, 292.
    cache.keep(290, [0, 2, 5])
    for i, (buf, d) in enumerate(zip(cache.k + cache.v, data)):
        want = d.copy()
        want[291], want[292] = d[292], d[295]
        got = ctx.read(buf, (600, kvd), np.float16)[:300]
        np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16), err_msg=f"buffer {i}")
        data[i] = want
    # Attention of 7 rows at positions 286..292 over the grown cache and over a fresh copy.
    rows, pos, scale = 7, 286, 1.0 / math.sqrt(hd)
    q = rng.standard_normal((rows, nh, hd)).astype(np.float32)
    qb, out = ctx.upload(q), ctx.zeros(q.nbytes)
    ctx.attention(qb, cache.k[1], cache.v[1], bchip.F16, out, None, False, rows, nh, nkv, hd, pos, scale)
    grown = ctx.read(out, q.shape)
    kf, vf = ctx.upload(data[1][:pos + rows]), ctx.upload(data[n_layer + 1][:pos + rows])
    ctx.attention(qb, kf, vf, bchip.F16, out, None, False, rows, nh, nkv, hd, pos, scale)
    np.testing.assert_array_equal(grown, ctx.read(out, q.shape))
    for b in (qb, out, kf, vf):
        b.free()
    cache.free()
