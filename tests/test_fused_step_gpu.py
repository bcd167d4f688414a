"""bchip_rope_append_attention: one decode step of one layer as a single call, against the
two calls it stands for (bchip_rope_append with rows = 1, then bchip_attention at the new
slot), which in turn are the reference's k_rope(q), k_rope(k), k_copy(k), k_copy(v),
k_attention sequence (crates/bc-infer/src/gpu/mod.rs:464-482). The fused call must give the
same bits everywhere: the output, q (left rotated), and both caches; and the output must
pass the oracle gate."""
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


CASES = [
    # nh, nkv, hd, rope_dim, neox, theta, kv_type, pos
    (32, 8, 128, 128, False, 5e5, bchip.F16, 0),       # the first token: one slot
    (32, 8, 128, 128, False, 5e5, bchip.F16, 1),
    (32, 8, 128, 128, False, 5e5, bchip.F16, 63),      # one chunk (written by the unit)
    (32, 8, 128, 128, False, 5e5, bchip.F16, 64),      # the new row opens a block
    (32, 8, 128, 128, False, 5e5, bchip.F16, 4096),    # many chunks (q written by the fold)
    (32, 8, 128, 128, False, 5e5, bchip.F16, 32767),   # configs[1] at 32768 slots
    (14, 2, 64, 64, True, 1e6, bchip.F32, 511),        # configs[0]: Qwen2.5-0.5B, f32 cache
    (28, 4, 128, 128, True, 1e6, bchip.F16, 3000),     # configs[3] heads, neox
    (64, 8, 128, 128, False, 5e5, bchip.F16, 6136),    # configs[4] heads
    (8, 8, 256, 256, False, 1e4, bchip.F16, 700),      # head_dim 256
    (32, 8, 128, 96, True, 5e5, bchip.F16, 100),       # neox pairs 48 apart: the two-call path
    (4, 2, 16, 16, False, 1e4, bchip.F32, 6),          # tiny_model shape (hd 16), f32 cache
    (32, 8, 128, 128, False, 5e5, bchip.F32, 0),       # f32 cache: the first token (unsplit, q by the kernel)
    (32, 8, 128, 128, False, 5e5, bchip.F32, 192),     # f32: the new row alone in the last chunk
    (32, 8, 128, 128, False, 5e5, bchip.F32, 4000),    # f32: split, q rotated by attn_combine
    (32, 8, 128, 128, False, 5e5, bchip.F32, 32767),   # configs[1] over an f32 cache (attn_combine_long)
    (28, 4, 128, 96, True, 1e6, bchip.F32, 3000),      # f32: neox pairs 48 apart, partial rotary
    (8, 8, 256, 128, False, 1e4, bchip.F32, 700),      # f32: head_dim 256, partial rotary
    (14, 2, 64, 32, True, 1e6, bchip.F32, 300),        # f32: hd 64, neox over half the dims
    (16, 1, 64, 64, False, 1e4, bchip.F32, 100),       # f32: 16 query heads per KV head
    (16, 1, 128, 128, False, 5e5, bchip.F16, 200),     # 16 query heads per KV head: the two-call path
    (16, 2, 128, 128, False, 5e5, bchip.F16, 256),     # 8 per KV head, the last chunk holds the new row alone
]


@pytest.mark.parametrize("nh,nkv,hd,rd,neox,theta,kv_type,pos", CASES)
def test_fused_step_is_rope_append_then_attention(ctx, nh, nkv, hd, rd, neox, theta, kv_type, pos):
    seed = nh * 7 + pos
    kvd = nkv * hd
    cap = pos + 1 + 3
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    q, k, v = rand((1, nh * hd), seed), rand((1, kvd), seed + 1), rand((1, kvd), seed + 2)
    kc0, vc0 = rand((cap, kvd), seed + 3).astype(dt), rand((cap, kvd), seed + 4).astype(dt)
    inv = O.inv_freq(rd, theta)
    positions = np.array([pos], np.uint32)
    scale = 1.0 / math.sqrt(hd)
    ib, pb, kb, vb = ctx.upload(inv), ctx.upload(positions), ctx.upload(k), ctx.upload(v)
    runs = []
    for fused in (False, True):
        qb, kcb, vcb = ctx.upload(q), ctx.upload(kc0), ctx.upload(vc0)
        ob = ctx.zeros(nh * hd * 4)
        if fused:
            ctx.rope_append_attention(qb, kb, vb, kcb, vcb, kv_type, ib, pb, nh, nkv, hd, rd, neox, pos, scale, ob)
        else:
            ctx.rope_append(qb, kb, vb, kcb, vcb, kv_type, ib, pb, 1, nh, nkv, hd, rd, neox, pos)
            ctx.attention(qb, kcb, vcb, kv_type, ob, None, False, 1, nh, nkv, hd, pos, scale)
        runs.append((ctx.read(ob, (1, nh, hd)), ctx.read(qb, q.shape), ctx.read(kcb, kc0.shape, dt),
                     ctx.read(vcb, vc0.shape, dt)))
        for b in (qb, kcb, vcb, ob):
            b.free()
    (o0, q0, k0, v0), (o1, q1, k1, v1) = runs
    what = f"{nh}/{nkv}/{hd} rope {rd} {'neox' if neox else 'adjacent'} at {pos}"
    np.testing.assert_array_equal(o1, o0, err_msg=what + ": out")
    np.testing.assert_array_equal(q1, q0, err_msg=what + ": rotated q")
    np.testing.assert_array_equal(k1, k0, err_msg=what + ": K cache")
    np.testing.assert_array_equal(v1, v0, err_msg=what + ": V cache")
    # Only slot pos changed in the caches, and the output passes the oracle gate on them.
    np.testing.assert_array_equal(np.delete(k1, pos, axis=0), np.delete(kc0, pos, axis=0))
    np.testing.assert_array_equal(np.delete(v1, pos, axis=0), np.delete(vc0, pos, axis=0))
    want = O.attention(q1.reshape(1, nh, hd), k1[:pos + 1].astype(np.float32), v1[:pos + 1].astype(np.float32),
                       1, pos, nh, nkv, hd, scale)
    got = o1.astype(np.float64).ravel()
    ref = np.asarray(want, np.float64).ravel()
    err = float(np.abs(got - ref).max())
    cos = float(got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref)))
    assert err <= 5e-3 and cos >= 0.9999, f"{what}: max abs {err:.3g}, cosine {cos:.8f}"
    for b in (ib, pb, kb, vb):
        b.free()


def test_fused_step_repeats_bit_for_bit(ctx):
    """Run-to-run determinism of the fused step (model.rs:648 asks it of every pass)."""
    nh, nkv, hd, pos = 32, 8, 128, 9000
    kvd = nkv * hd
    q, k, v = rand((1, nh * hd), 1), rand((1, kvd), 2), rand((1, kvd), 3)
    kc0, vc0 = rand((pos + 1, kvd), 4).astype(np.float16), rand((pos + 1, kvd), 5).astype(np.float16)
    ib, pb = ctx.upload(O.inv_freq(hd, 5e5)), ctx.upload(np.array([pos], np.uint32))
    kb, vb = ctx.upload(k), ctx.upload(v)
    outs = []
    for _ in range(3):
        qb, kcb, vcb, ob = ctx.upload(q), ctx.upload(kc0), ctx.upload(vc0), ctx.zeros(nh * hd * 4)
        ctx.rope_append_attention(qb, kb, vb, kcb, vcb, bchip.F16, ib, pb, nh, nkv, hd, hd, False, pos,
                                  1 / math.sqrt(hd), ob)
        outs.append(ctx.read(ob, (nh, hd)))
        for b in (qb, kcb, vcb, ob):
            b.free()
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(outs[0], outs[2])
    for b in (ib, pb, kb, vb):
        b.free()
