"""A seeded sweep over attention shapes the named configurations do not reach: head dims that
are not powers of two, one to sixteen query heads a KV head, line and tree rows at random
positions, f16 and f32 caches, each against the oracle (model.rs:448-481) at the north
star's gate; and the one-call steps (a decode step, a verify step's rows) against their two
calls, bit for bit, at random shapes. The shapes come from a fixed seed, so every run checks
the same ones."""
import math

import numpy as np
import pytest

import bchip
import oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 5e-3
MIN_COS = 0.9999


@pytest.fixture(scope="module")
def ctx():
    c = bchip.Ctx(0)
    yield c
    c.close()


def _attention_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        hd = int(rng.choice([32, 48, 64, 80, 96, 112, 128, 192, 256]))
        nkv = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.integers(1, 17))
        rows = int(rng.choice([1, 1, 2, 5, 8, 16, 33]))
        pos = int(rng.integers(0, 2500))
        tree = bool(rows > 1 and rng.random() < 0.3)
        kv_type = bchip.F16 if rng.random() < 0.7 else bchip.F32
        if rows * g * nkv * (pos + rows) * hd > 1.5e8:  # keep the oracle's share to a second or so
            continue
        cases.append((rows, pos, g * nkv, nkv, hd, tree, kv_type, int(rng.integers(1 << 30))))
    return cases


# Long lists beside the sweep: a verify pass past the group fold's reach (more than 32 chunks:
# the long fold), the same over f32, a tree at 9000 slots, a line of 100 rows at 12000.
LONG = [(8, 35000, 64, 8, 128, False, bchip.F16, 1), (8, 35000, 64, 8, 128, False, bchip.F32, 2),
        (40, 9000, 32, 8, 128, True, bchip.F16, 3), (100, 12000, 8, 2, 128, False, bchip.F16, 4)]


@pytest.mark.parametrize("rows,pos,nh,nkv,hd,tree,kv_type,seed", LONG + _attention_cases(120, 20261202))
def test_attention_against_the_oracle(ctx, rows, pos, nh, nkv, hd, tree, kv_type, seed):
    rng = np.random.default_rng(seed)
    kvd = nkv * hd
    slots = pos + rows
    kc = rng.standard_normal((slots, kvd)).astype(np.float32)
    vc = rng.standard_normal((slots, kvd)).astype(np.float32)
    q = rng.standard_normal((rows, nh, hd)).astype(np.float32)
    if kv_type == bchip.F16:
        kc, vc = O.f16_round(kc).reshape(kc.shape), O.f16_round(vc).reshape(vc.shape)
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    visible = None
    if tree:
        parents = [O.ROOT] + [int(rng.integers(-1, j)) if j else O.ROOT for j in range(1, rows)]
        parents = [O.ROOT if p < 0 else p for p in parents]
        _, visible, _ = O.shape(rows, pos, parents)
    scale = 1.0 / math.sqrt(hd)
    kb, vb = ctx.upload(kc.astype(dt)), ctx.upload(vc.astype(dt))
    qb, ob = ctx.upload(q), ctx.zeros(q.nbytes)
    mb = None if visible is None else ctx.upload(bchip.masks_words(visible))
    ctx.attention(qb, kb, vb, kv_type, ob, mb, tree, rows, nh, nkv, hd, pos, scale)
    got = ctx.read(ob, q.shape)
    want = O.attention(q, kc, vc, rows, pos, nh, nkv, hd, scale, visible=visible, base=pos if tree else None)
    g64, w64 = got.astype(np.float64).ravel(), np.asarray(want, np.float64).ravel()
    err = float(np.abs(g64 - w64).max())
    cos = float(g64 @ w64 / (np.linalg.norm(g64) * np.linalg.norm(w64)))
    what = f"{rows} {'tree' if tree else 'line'} rows at {pos}, {nh}/{nkv} heads of {hd}, " \
           f"{'f16' if kv_type == bchip.F16 else 'f32'}"
    assert np.isfinite(got).all(), what
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max abs {err:.3g}, cosine {cos:.8f}"
    for b in [kb, vb, qb, ob] + ([mb] if mb is not None else []):
        b.free()


def _step_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        hd = int(rng.choice([64, 96, 128, 128, 128, 256]))
        nkv = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.choice([1, 2, 4, 7, 8, 16]))
        rows = int(rng.choice([1, 2, 3, 8, 9, 16]))
        pos = int(rng.integers(0, 5000))
        rd = int(rng.choice([hd, hd, hd // 2]))
        rd -= rd % 2
        neox = bool(rng.random() < 0.5)
        kv_type = bchip.F16 if rng.random() < 0.7 else bchip.F32
        cases.append((rows, g * nkv, nkv, hd, rd, neox, kv_type, pos, int(rng.integers(1 << 30))))
    return cases


@pytest.mark.parametrize("rows,nh,nkv,hd,rd,neox,kv_type,pos,seed", _step_cases(60, 777))
def test_one_call_steps_against_their_two_calls(ctx, rows, nh, nkv, hd, rd, neox, kv_type, pos, seed):
    """bchip_rope_append_attention (one row) and bchip_rope_append_attention_rows (several) at
    random shapes: the same bits as bchip_rope_append then bchip_attention (out, q left
    rotated, both caches), whichever form the library picks for the shape."""
    rng = np.random.default_rng(seed)
    kvd = nkv * hd
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    q = rng.standard_normal((rows, nh * hd)).astype(np.float32)
    k = rng.standard_normal((rows, kvd)).astype(np.float32)
    v = rng.standard_normal((rows, kvd)).astype(np.float32)
    kc0 = rng.standard_normal((pos + rows, kvd)).astype(dt)
    vc0 = rng.standard_normal((pos + rows, kvd)).astype(dt)
    inv = O.inv_freq(rd, 1e4) if rd else np.zeros(1, np.float32)
    positions = (pos + np.arange(rows)).astype(np.uint32)
    scale = 1.0 / math.sqrt(hd)
    ib, pb, kb, vb = ctx.upload(inv), ctx.upload(positions), ctx.upload(k), ctx.upload(v)
    runs = []
    for fused in (False, True):
        qb, kcb, vcb, ob = ctx.upload(q), ctx.upload(kc0), ctx.upload(vc0), ctx.zeros(q.nbytes)
        if fused and rows == 1:
            ctx.rope_append_attention(qb, kb, vb, kcb, vcb, kv_type, ib, pb, nh, nkv, hd, rd, neox, pos, scale, ob)
        elif fused:
            ctx.rope_append_attention_rows(qb, kb, vb, kcb, vcb, kv_type, ib, pb, rows, nh, nkv, hd, rd, neox, pos,
                                           scale, ob)
        else:
            ctx.rope_append(qb, kb, vb, kcb, vcb, kv_type, ib, pb, rows, nh, nkv, hd, rd, neox, pos)
            ctx.attention(qb, kcb, vcb, kv_type, ob, None, False, rows, nh, nkv, hd, pos, scale)
        runs.append((ctx.read(ob, (rows, nh, hd)), ctx.read(qb, q.shape), ctx.read(kcb, kc0.shape, dt),
                     ctx.read(vcb, vc0.shape, dt)))
        for b in (qb, kcb, vcb, ob):
            b.free()
    what = f"{rows} rows at {pos}, {nh}/{nkv} heads of {hd}, rope {rd} {'neox' if neox else 'adjacent'}, " \
           f"{'f16' if kv_type == bchip.F16 else 'f32'}"
    for name, a, b in zip(("out", "rotated q", "K cache", "V cache"), runs[1], runs[0]):
        np.testing.assert_array_equal(a, b, err_msg=f"{what}: {name}")
    for b in (ib, pb, kb, vb):
        b.free()
