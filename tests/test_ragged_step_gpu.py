"""A decode step of several conversations in one cache pool (the up-to-16 streams a stage
keeps, crates/bc-mesh/src/engine.rs:25, 305-314): bchip_rope_append_attention_ragged (one
launch: RoPE of every sequence's q and k, its K/V append, attention) against the two ragged
calls it stands for (bchip_rope_append_ragged, bchip_attention_ragged) and against each
sequence's own one-token step (bchip_rope_append_attention on its slice of the pool), bit
for bit: output, q left rotated, the caches; and every sequence against the oracle's rope and
attention (model.rs:391-403, 448-481)."""
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


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


def gate(got, want, what):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    err = float(np.abs(got - want).max())
    cos = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want)))
    print(f"{what}: max abs {err:.3g}, cosine {cos:.8f}", flush=True)
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max abs {err:.3g}, cosine {cos:.8f}"


def run_step(ctx, kind, pool_k, pool_v, q, k, v, lens, offs, kv_type, nh, nkv, hd, rd, neox, theta, scale):
    """One step on fresh device copies; kind: fused | two | single. Returns (out, q, kc, vc)."""
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    kvd = nkv * hd
    n = len(lens)
    kb, vb = ctx.upload(pool_k.astype(dt)), ctx.upload(pool_v.astype(dt))
    qb, knb, vnb = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    ib = ctx.upload(O.inv_freq(rd, theta))
    pb = ctx.upload(np.asarray(lens, np.uint32) - 1)
    ob = ctx.zeros(n * nh * hd * 4)
    if kind == "fused":
        ctx.rope_append_attention_ragged(qb, knb, vnb, kb, vb, kv_type, ib, pb, lens, offs, nh, nkv, hd, rd, neox,
                                         scale, ob)
    elif kind == "two":
        ctx.rope_append_ragged(qb, knb, vnb, kb, vb, kv_type, ib, pb, lens, offs, nh, nkv, hd, rd, neox)
        ctx.attention_ragged(qb, kb, vb, kv_type, ob, lens, offs, nh, nkv, hd, scale)
    else:
        es = bchip.esize(kv_type)
        for i, (L, off) in enumerate(zip(lens, offs)):
            L, off = int(L), int(off)
            ctx.rope_append_attention(qb.offset(i * nh * hd * 4), knb.offset(i * kvd * 4), vnb.offset(i * kvd * 4),
                                      kb.offset(off * kvd * es), vb.offset(off * kvd * es), kv_type, ib,
                                      pb.offset(4 * i), nh, nkv, hd, rd, neox, L - 1, scale, ob.offset(i * nh * hd * 4))
    res = (ctx.read(ob, (n, nh, hd)), ctx.read(qb, q.shape), ctx.read(kb, pool_k.shape, dt),
           ctx.read(vb, pool_v.shape, dt))
    for b in (kb, vb, qb, knb, vnb, ib, pb, ob):
        b.free()
    return res


def ragged_step(ctx, lens, kv_type, nh, nkv, hd, rd, neox, theta, seed):
    kvd = nkv * hd
    lens = np.asarray(lens, np.uint32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    total = int(lens.sum())
    scale = 1.0 / math.sqrt(hd)
    pool_k, pool_v = rand((total, kvd), seed), rand((total, kvd), seed + 1)
    q, k, v = rand((len(lens), nh * hd), seed + 2), rand((len(lens), kvd), seed + 3), rand((len(lens), kvd), seed + 4)
    args = (pool_k, pool_v, q, k, v, lens, offs, kv_type, nh, nkv, hd, rd, neox, theta, scale)
    print(f"ragged step: {len(lens)} sequences, {total} slots, kv_type {kv_type}", flush=True)
    fused = run_step(ctx, "fused", *args)
    for kind in ("two", "single"):
        other = run_step(ctx, kind, *args)
        for name, a, b in zip(("out", "rotated q", "K pool", "V pool"), fused, other):
            np.testing.assert_array_equal(a, b, err_msg=f"fused against {kind}: {name}")
    out, q_dev, kc_dev, vc_dev = fused
    inv = O.inv_freq(rd, theta)
    for i, (L, off) in enumerate(zip(lens, offs)):
        L, off = int(L), int(off)
        pos = L - 1
        q_ref = O.rope(q[i], nh, hd, rd, neox, pos, inv)
        k_ref = O.rope(k[i], nkv, hd, rd, neox, pos, inv)
        assert np.abs(q_dev[i] - q_ref).max() <= 1e-4 * (1 + np.abs(q_ref).max()), f"sequence {i}: rotated q"
        kc = kc_dev[off:off + L].astype(np.float32)
        vc = vc_dev[off:off + L].astype(np.float32)
        gate(out[i:i + 1], O.attention(q_dev[i].reshape(1, nh, hd), kc, vc, 1, pos, nh, nkv, hd, scale),
             f"sequence {i} ({L} slots, kernel error)")
        k32, v32 = pool_k[off:off + L].copy(), pool_v[off:off + L].copy()
        k32[pos], v32[pos] = k_ref, v[i]
        gate(out[i:i + 1], O.attention(q_ref.reshape(1, nh, hd), k32, v32, 1, pos, nh, nkv, hd, scale),
             f"sequence {i} ({L} slots, total error)")
    # The slots outside each sequence's new row are untouched.
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    new = (offs + lens - 1).astype(np.int64)
    keep = np.setdiff1d(np.arange(int(lens.sum())), new)
    np.testing.assert_array_equal(kc_dev[keep], pool_k.astype(dt)[keep])
    np.testing.assert_array_equal(vc_dev[keep], pool_v.astype(dt)[keep])


def test_qwen7b_ragged_decode_step_16_streams(ctx):
    """16 conversations, lengths U[1024, 32768] (seed 4, as the benchmark draws
    them), 28/4 heads, hd 128, f16 pool, RoPE theta 1e6 neox."""
    lens = np.random.default_rng(4).integers(1024, 32769, size=16)
    ragged_step(ctx, lens, bchip.F16, 28, 4, 128, 128, True, 1e6, 40)


def test_ragged_decode_step_short_and_mixed(ctx):
    """Lists of one slot, one block, a chunk boundary; more than 64 sequences (two launches)."""
    lens = [1, 2, 63, 64, 65, 288, 289, 1000] * 9
    ragged_step(ctx, lens, bchip.F16, 32, 8, 128, 128, False, 5e5, 50)


def test_ragged_decode_step_f32_and_unfused_shapes(ctx):
    """f32 pools, and shapes the fused kernel does not take, run as the two calls."""
    ragged_step(ctx, [7, 300, 5, 129], bchip.F32, 14, 2, 64, 64, True, 1e6, 60)
    ragged_step(ctx, [7, 300, 5, 129], bchip.F16, 16, 1, 128, 128, False, 5e5, 70)


def _ragged_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        nseq = int(rng.integers(1, 25))
        lens = [int(x) for x in rng.integers(1, 6000, nseq)]
        hd = int(rng.choice([64, 128, 128, 256]))
        nkv = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.choice([1, 2, 4, 7, 8]))
        rd = int(rng.choice([hd, hd // 2]))
        neox = bool(rng.random() < 0.5)
        kv_type = bchip.F16 if rng.random() < 0.75 else bchip.F32
        cases.append((lens, kv_type, g * nkv, nkv, hd, rd, neox, int(rng.integers(1 << 30))))
    return cases


@pytest.mark.parametrize("lens,kv_type,nh,nkv,hd,rd,neox,seed", _ragged_cases(12, 4242))
def test_ragged_decode_step_seeded_sweep(ctx, lens, kv_type, nh, nkv, hd, rd, neox, seed):
    """Random pools (1-24 sequences of 1-6000 slots), heads, head dims and rotary shapes: the
    one launch against the two calls and each sequence's own step bit for bit, and every
    sequence against the oracle."""
    ragged_step(ctx, lens, kv_type, nh, nkv, hd, rd, neox, 1e4, seed % 100000)
