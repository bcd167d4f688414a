"""bchip_rope_append_attention_noalloc, through the C ABI, against bchip_rope_append_attention:
the same step on the same inputs must give the same bits (output, q left rotated, both
caches), on two calls in a row on one context, the second smaller than the first (the fixed
scratch keeps the first call's contents). A step too big for the scratch is refused before
anything is launched, and leaves its inputs untouched."""
import math

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


def step(ctx, noalloc, nh, nkv, hd, rd, neox, theta, kv_type, pos, seed):
    kvd = nkv * hd
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    q, k, v = rand((1, nh * hd), seed), rand((1, kvd), seed + 1), rand((1, kvd), seed + 2)
    kc0, vc0 = rand((pos + 1, kvd), seed + 3).astype(dt), rand((pos + 1, kvd), seed + 4).astype(dt)
    bufs = [ctx.upload(O.inv_freq(rd, theta)), ctx.upload(np.array([pos], np.uint32)), ctx.upload(k), ctx.upload(v),
            ctx.upload(q), ctx.upload(kc0), ctx.upload(vc0), ctx.zeros(nh * hd * 4)]
    ib, pb, kb, vb, qb, kcb, vcb, ob = bufs
    call = ctx.rope_append_attention_noalloc if noalloc else ctx.rope_append_attention
    call(qb, kb, vb, kcb, vcb, kv_type, ib, pb, nh, nkv, hd, rd, neox, pos, 1.0 / math.sqrt(hd), ob)
    res = (ctx.read(ob, (nh, hd)), ctx.read(qb, q.shape), ctx.read(kcb, kc0.shape, dt), ctx.read(vcb, vc0.shape, dt))
    for b in bufs:
        b.free()
    return res


# Pairs of steps, the second smaller: nh, nkv, hd, rope_dim, neox, theta, kv_type, pos
PAIRS = [
    ((32, 8, 128, 128, False, 5e5, bchip.F16, 32767), (32, 8, 128, 128, False, 5e5, bchip.F16, 1000)),
    ((8, 8, 256, 256, False, 1e4, bchip.F16, 20000), (28, 4, 128, 128, True, 1e6, bchip.F16, 3000)),
    # f32 caches (attn_f32 rotating q and appending the row itself); 60001 slots take more
    # chunk states than the scratch holds (then unsplit, q written back by the kernel: the
    # same bits as the split pass of the allocating entry point, q rotated by its fold).
    ((32, 8, 128, 128, False, 5e5, bchip.F32, 60000), (14, 2, 64, 64, True, 1e6, bchip.F32, 511)),
    # Shapes the fused kernel does not take: rope_append, then the one-row kernel.
    ((16, 1, 128, 128, False, 5e5, bchip.F16, 9000), (32, 8, 128, 96, True, 5e5, bchip.F16, 100)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_step_gives_the_bits_of_the_allocating_one(ctx, first, second):
    for i, case in enumerate((first, second)):
        print(f"no-alloc step {i}: {case}", flush=True)
        want = step(ctx, False, *case, seed=10 * i + 1)
        got = step(ctx, True, *case, seed=10 * i + 1)
        for name, a, b in zip(("out", "rotated q", "K cache", "V cache"), got, want):
            np.testing.assert_array_equal(a, b, err_msg=f"{case}: {name}")


def test_noalloc_refuses_a_step_past_its_scratch(ctx):
    """512 query heads of 256 dims: 128K floats of staged q, past the 64K the scratch holds."""
    nh, nkv, hd, pos = 512, 64, 256, 100
    kvd = nkv * hd
    q, k, v = rand((1, nh * hd), 1), rand((1, kvd), 2), rand((1, kvd), 3)
    kc0 = rand((pos + 1, kvd), 4).astype(np.float16)
    bufs = [ctx.upload(O.inv_freq(hd, 5e5)), ctx.upload(np.array([pos], np.uint32)), ctx.upload(k), ctx.upload(v),
            ctx.upload(q), ctx.upload(kc0), ctx.upload(kc0), ctx.zeros(nh * hd * 4)]
    ib, pb, kb, vb, qb, kcb, vcb, ob = bufs
    with pytest.raises(bchip.BchipError) as e:
        ctx.rope_append_attention_noalloc(qb, kb, vb, kcb, vcb, bchip.F16, ib, pb, nh, nkv, hd, hd, False, pos,
                                          0.0625, ob)
    assert "no-allocation" in str(e.value)
    np.testing.assert_array_equal(ctx.read(qb, q.shape), q)
    np.testing.assert_array_equal(ctx.read(kcb, kc0.shape, np.float16), kc0)
    for b in bufs:
        b.free()
