"""bchip_rope_append_attention_rows: one layer of a multi-row pass (a speculative verify step,
llm.rs:655-667) as a single call, against the two calls it stands for (bchip_rope_append
with slot0 = pos, then bchip_attention of the same rows at pos), which in turn are the
reference's k_rope(q), k_rope(k), k_copy(k), k_copy(v), k_attention sequence for a pass of
several rows (crates/bc-infer/src/gpu/mod.rs:464-482). The single call must give the same
bits everywhere: the output, q (left rotated), and both caches; the output must pass the
oracle gate. The cases cover the fused launch (a split pass folded in its launch: configs[4]'s
verify at 4096 and 6136 slots, new rows crossing a block and a chunk boundary, adjacent and
neox pairs, partial rotary dims) and the shapes that run as the two calls."""
import math
import os

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
    # rows, nh, nkv, hd, rope_dim, neox, theta, kv_type, pos
    (8, 64, 8, 128, 128, False, 5e5, bchip.F16, 4096),   # configs[4]'s verify (fused)
    (8, 64, 8, 128, 128, False, 5e5, bchip.F16, 6136),   # its last step (fused)
    (8, 32, 8, 128, 128, False, 5e5, bchip.F16, 190),    # new rows across a chunk boundary (fused)
    (5, 32, 8, 128, 128, False, 5e5, bchip.F16, 1000),   # new rows across a block boundary (fused)
    (3, 32, 8, 128, 128, False, 5e5, bchip.F16, 2049),   # a few rows (fused)
    (9, 28, 4, 128, 128, True, 1e6, bchip.F16, 3000),    # neox, 7 query heads a KV head (fused)
    (8, 32, 8, 128, 64, True, 1e4, bchip.F16, 800),      # partial rotary, neox (fused)
    (8, 32, 8, 128, 96, False, 1e4, bchip.F16, 800),     # partial rotary, adjacent pairs (fused)
    (8, 32, 8, 128, 96, True, 1e4, bchip.F16, 800),      # neox pairs 48 dims apart: the two calls
    (16, 64, 16, 128, 128, False, 5e5, bchip.F16, 500),  # 16 rows, 4 query heads a KV head (fused)
    (4, 16, 1, 128, 128, False, 5e5, bchip.F16, 3000),   # 16 query heads a KV head, 4 rows (fused)
    (16, 32, 8, 128, 64, True, 1e4, bchip.F16, 2500),    # 16 rows, neox over half the dims (fused)
    (8, 64, 8, 128, 128, False, 5e5, bchip.F16, 100),    # one chunk: the two calls
    (20, 32, 8, 128, 128, False, 5e5, bchip.F16, 700),   # 80 slots a KV head: the two calls
    (8, 16, 16, 128, 128, False, 5e5, bchip.F16, 900),   # one query head a KV head (fused)
    (8, 32, 8, 64, 64, True, 1e6, bchip.F16, 900),       # head_dim 64: the two calls
    (4, 14, 2, 64, 64, True, 1e6, bchip.F32, 511),       # f32 cache: the two calls
    (1, 32, 8, 128, 128, False, 5e5, bchip.F16, 4096),   # one row: the two calls
    # f32 caches (attn_f32 rotating q and appending the rows itself, up to 8 rows)
    (8, 64, 8, 128, 128, False, 5e5, bchip.F32, 4096),   # configs[4]'s verify, split (q by the fold)
    (8, 32, 8, 128, 128, False, 5e5, bchip.F32, 100),    # one chunk (q by the kernel)
    (5, 32, 8, 128, 96, True, 1e4, bchip.F32, 190),      # new rows across a chunk boundary, partial neox
    (8, 16, 16, 64, 64, True, 1e6, bchip.F32, 700),      # 8 rows, one query head a KV head
    (7, 28, 4, 128, 128, True, 1e6, bchip.F32, 3000),    # four row blocks share the new rows' chunk
    (9, 28, 4, 128, 128, True, 1e6, bchip.F32, 3000),    # 9 rows: the two calls
    (3, 14, 2, 64, 64, True, 1e6, bchip.F32, 8000),      # configs[0] heads, a long list (the long fold)
    (20, 32, 8, 128, 128, False, 5e5, bchip.F32, 700),   # 20 rows: the two calls
]


@pytest.mark.parametrize("rows,nh,nkv,hd,rd,neox,theta,kv_type,pos", CASES)
def test_rows_step_is_rope_append_then_attention(ctx, rows, nh, nkv, hd, rd, neox, theta, kv_type, pos):
    seed = rows * 31 + nh * 7 + pos
    kvd = nkv * hd
    cap = pos + rows + 3
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    q, k, v = rand((rows, nh * hd), seed), rand((rows, kvd), seed + 1), rand((rows, kvd), seed + 2)
    kc0, vc0 = rand((cap, kvd), seed + 3).astype(dt), rand((cap, kvd), seed + 4).astype(dt)
    inv = O.inv_freq(rd, theta)
    positions = (pos + np.arange(rows)).astype(np.uint32)
    scale = 1.0 / math.sqrt(hd)
    ib, pb, kb, vb = ctx.upload(inv), ctx.upload(positions), ctx.upload(k), ctx.upload(v)
    runs = []
    for fused in (False, True):
        qb, kcb, vcb = ctx.upload(q), ctx.upload(kc0), ctx.upload(vc0)
        ob = ctx.zeros(rows * nh * hd * 4)
        if fused:
            ctx.rope_append_attention_rows(qb, kb, vb, kcb, vcb, kv_type, ib, pb, rows, nh, nkv, hd, rd, neox, pos,
                                           scale, ob)
        else:
            ctx.rope_append(qb, kb, vb, kcb, vcb, kv_type, ib, pb, rows, nh, nkv, hd, rd, neox, pos)
            ctx.attention(qb, kcb, vcb, kv_type, ob, None, False, rows, nh, nkv, hd, pos, scale)
        runs.append((ctx.read(ob, (rows, nh, hd)), ctx.read(qb, q.shape), ctx.read(kcb, kc0.shape, dt),
                     ctx.read(vcb, vc0.shape, dt)))
        for b in (qb, kcb, vcb, ob):
            b.free()
    (o0, q0, k0, v0), (o1, q1, k1, v1) = runs
    what = f"{rows} rows {nh}/{nkv}/{hd} rope {rd} {'neox' if neox else 'adjacent'} at {pos}"
    np.testing.assert_array_equal(o1, o0, err_msg=what + ": out")
    np.testing.assert_array_equal(q1, q0, err_msg=what + ": rotated q")
    np.testing.assert_array_equal(k1, k0, err_msg=what + ": K cache")
    np.testing.assert_array_equal(v1, v0, err_msg=what + ": V cache")
    # Only the new slots changed in the caches, and the output passes the oracle gate on them.
    new = list(range(pos, pos + rows))
    np.testing.assert_array_equal(np.delete(k1, new, axis=0), np.delete(kc0, new, axis=0))
    np.testing.assert_array_equal(np.delete(v1, new, axis=0), np.delete(vc0, new, axis=0))
    want = O.attention(q1.reshape(rows, nh, hd), k1[:pos + rows].astype(np.float32),
                       v1[:pos + rows].astype(np.float32), rows, pos, nh, nkv, hd, scale)
    got = o1.astype(np.float64).ravel()
    ref = np.asarray(want, np.float64).ravel()
    err = float(np.abs(got - ref).max())
    cos = float(got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref)))
    assert err <= 5e-3 and cos >= 0.9999, f"{what}: max abs {err:.3g}, cosine {cos:.8f}"
    for b in (ib, pb, kb, vb):
        b.free()


def test_rows_step_takes_each_rows_position(ctx):
    """The rotation angles come from positions[r], which need not be the rows' slots (a
    pipeline stage or a tree numbers its tokens as it likes): rows with scattered positions,
    fused (configs[4]'s shape) against the two calls, bit for bit."""
    rows, nh, nkv, hd, pos = 8, 64, 8, 128, 3000
    kvd = nkv * hd
    q, k, v = rand((rows, nh * hd), 31), rand((rows, kvd), 32), rand((rows, kvd), 33)
    kc0, vc0 = rand((pos + rows, kvd), 34).astype(np.float16), rand((pos + rows, kvd), 35).astype(np.float16)
    inv = O.inv_freq(hd, 5e5)
    positions = np.array([7, 100000, 3000, 3001, 12, 65535, 40000, 2999], np.uint32)
    want = _step(ctx, False, q, k, v, kc0, vc0, inv, positions, rows, nh, nkv, hd, pos)
    got = _step(ctx, True, q, k, v, kc0, vc0, inv, positions, rows, nh, nkv, hd, pos)
    for name, a, b in zip(("out", "rotated q", "K cache", "V cache"), got, want):
        np.testing.assert_array_equal(a, b, err_msg=name)


def test_rows_step_with_unaligned_new_rows(ctx):
    """k and v 4 bytes past a 16-byte boundary: the one-launch form loads them 16 bytes a lane,
    so the call runs as its two calls; the same bits as those."""
    rows, nh, nkv, hd, pos = 8, 64, 8, 128, 4096
    kvd = nkv * hd
    q, k, v = rand((rows, nh * hd), 41), rand((rows, kvd), 42), rand((rows, kvd), 43)
    kc0, vc0 = rand((pos + rows, kvd), 44).astype(np.float16), rand((pos + rows, kvd), 45).astype(np.float16)
    ib = ctx.upload(O.inv_freq(hd, 5e5))
    pb = ctx.upload((pos + np.arange(rows)).astype(np.uint32))
    kb, vb = ctx.zeros(k.nbytes + 16), ctx.zeros(v.nbytes + 16)
    ctx.upload(k, kb, 4)
    ctx.upload(v, vb, 4)
    outs = []
    for fused in (False, True):
        qb, kcb, vcb, ob = ctx.upload(q), ctx.upload(kc0), ctx.upload(vc0), ctx.zeros(rows * nh * hd * 4)
        args = (qb, kb.ptr + 4, vb.ptr + 4, kcb, vcb, bchip.F16, ib, pb, rows, nh, nkv, hd, hd, False, pos)
        if fused:
            ctx.rope_append_attention_rows(*args, 1 / math.sqrt(hd), ob)
        else:
            ctx.rope_append(*args)
            ctx.attention(qb, kcb, vcb, bchip.F16, ob, None, False, rows, nh, nkv, hd, pos, 1 / math.sqrt(hd))
        outs.append((ctx.read(ob, (rows, nh, hd)), ctx.read(qb, q.shape), ctx.read(kcb, kc0.shape, np.float16)))
        for b in (qb, kcb, vcb, ob):
            b.free()
    for name, a, b in zip(("out", "rotated q", "K cache"), outs[1], outs[0]):
        np.testing.assert_array_equal(a, b, err_msg=name)
    for b in (ib, pb, kb, vb):
        b.free()


def test_rows_step_repeats_bit_for_bit(ctx):
    """Run-to-run determinism of the fused multi-row step (model.rs:648 asks it of every pass)."""
    rows, nh, nkv, hd, pos = 8, 64, 8, 128, 5000
    kvd = nkv * hd
    q, k, v = rand((rows, nh * hd), 1), rand((rows, kvd), 2), rand((rows, kvd), 3)
    kc0, vc0 = rand((pos + rows, kvd), 4).astype(np.float16), rand((pos + rows, kvd), 5).astype(np.float16)
    ib = ctx.upload(O.inv_freq(hd, 5e5))
    pb = ctx.upload((pos + np.arange(rows)).astype(np.uint32))
    kb, vb = ctx.upload(k), ctx.upload(v)
    outs = []
    for _ in range(3):
        qb, kcb, vcb, ob = ctx.upload(q), ctx.upload(kc0), ctx.upload(vc0), ctx.zeros(rows * nh * hd * 4)
        ctx.rope_append_attention_rows(qb, kb, vb, kcb, vcb, bchip.F16, ib, pb, rows, nh, nkv, hd, hd, False, pos,
                                       1 / math.sqrt(hd), ob)
        outs.append(ctx.read(ob, (rows, nh, hd)))
        for b in (qb, kcb, vcb, ob):
            b.free()
    np.testing.assert_array_equal(outs[0], outs[1])
    np.testing.assert_array_equal(outs[0], outs[2])
    for b in (ib, pb, kb, vb):
        b.free()


def _ctx_with(env):
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return bchip.Ctx(0)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


def _step(c, fused, q, k, v, kc0, vc0, inv, positions, rows, nh, nkv, hd, pos):
    ib, pb, kb, vb = c.upload(inv), c.upload(positions), c.upload(k), c.upload(v)
    qb, kcb, vcb, ob = c.upload(q), c.upload(kc0), c.upload(vc0), c.zeros(rows * nh * hd * 4)
    args = (qb, kb, vb, kcb, vcb, bchip.F16, ib, pb, rows, nh, nkv, hd, hd, False, pos)
    if fused:
        c.rope_append_attention_rows(*args, 1 / math.sqrt(hd), ob)
    else:
        c.rope_append(*args)
        c.attention(qb, kcb, vcb, bchip.F16, ob, None, False, rows, nh, nkv, hd, pos, 1 / math.sqrt(hd))
    got = (c.read(ob, (rows, nh, hd)), c.read(qb, q.shape), c.read(kcb, kc0.shape, np.float16),
           c.read(vcb, vc0.shape, np.float16))
    for b in (ib, pb, kb, vb, qb, kcb, vcb, ob):
        b.free()
    return got


@pytest.mark.parametrize("env", [{"BCHIP_GROUP_FOLD": "spread"}, {"BCHIP_GROUP_FOLD": "0"}])
def test_rows_step_under_the_fold_switches(ctx, env):
    """The fused step with the group fold's spread path forced (every state published again
    write-through, a second count), and with the group fold off (the call then runs as its two
    calls): the same bits as the two calls on the default context, three calls in a row."""
    rows, nh, nkv, hd, pos = 8, 64, 8, 128, 4096
    kvd = nkv * hd
    q, k, v = rand((rows, nh * hd), 21), rand((rows, kvd), 22), rand((rows, kvd), 23)
    kc0, vc0 = rand((pos + rows, kvd), 24).astype(np.float16), rand((pos + rows, kvd), 25).astype(np.float16)
    inv = O.inv_freq(hd, 5e5)
    positions = (pos + np.arange(rows)).astype(np.uint32)
    want = _step(ctx, False, q, k, v, kc0, vc0, inv, positions, rows, nh, nkv, hd, pos)
    other = _ctx_with(env)
    try:
        for _ in range(3):
            got = _step(other, True, q, k, v, kc0, vc0, inv, positions, rows, nh, nkv, hd, pos)
            for name, a, b in zip(("out", "rotated q", "K cache", "V cache"), got, want):
                np.testing.assert_array_equal(a, b, err_msg=f"{env}: {name}")
    finally:
        other.close()
