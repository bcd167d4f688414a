"""One-row launches with a unit a run of chunks against a unit a chunk (BCHIP_ROW_RUNS=2 and
=0 at init; the default takes runs from 4096 chunk units, a ragged batch of long lists).

The fold of a one-row list's chunk states is fixed by the list alone: runs of eight
consecutive chunks, each folded left to right from a cleared state, then attn_row_fold's
order over the runs. With runs, the decode wave that streams a run folds its chunks itself
and writes one state; without, attn_row_fold folds the run from the chunk states. Outputs,
the rotated q and the caches must be the same bits either way, for single steps (fused and
unfused) and ragged batches, at lengths with one chunk, whole and partial runs, and at
every head dim the one-row kernel takes; and within tolerance of the oracle
(model.rs:448-481).
"""
import math
import os

import numpy as np
import pytest

import bchip
import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctxs():
    made = []
    old = os.environ.get("BCHIP_ROW_RUNS")
    try:
        for mode in ("2", "0"):
            os.environ["BCHIP_ROW_RUNS"] = mode
            made.append(bchip.Ctx(0))
    finally:
        if old is None:
            os.environ.pop("BCHIP_ROW_RUNS", None)
        else:
            os.environ["BCHIP_ROW_RUNS"] = old
    yield made
    for c in made:
        c.close()


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


def step(ctx, kind, lens, nh, nkv, hd, seed):
    """kind: fused (the fused ragged step), plain (attention over the pool as it is) or
    single (each list's own fused step). Returns (out, q, K pool, V pool)."""
    kvd = nkv * hd
    lens = np.asarray(lens, np.uint32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    total = int(lens.sum())
    n = len(lens)
    scale = 1.0 / math.sqrt(hd)
    kb = ctx.upload(rand((total, kvd), seed).astype(np.float16))
    vb = ctx.upload(rand((total, kvd), seed + 1).astype(np.float16))
    q = rand((n, nh * hd), seed + 2)
    qb, knb, vnb = ctx.upload(q), ctx.upload(rand((n, kvd), seed + 3)), ctx.upload(rand((n, kvd), seed + 4))
    ib = ctx.upload(O.inv_freq(hd, 1e6))
    pb = ctx.upload(lens - 1)
    ob = ctx.zeros(n * nh * hd * 4)
    if kind == "fused":
        ctx.rope_append_attention_ragged(qb, knb, vnb, kb, vb, bchip.F16, ib, pb, lens, offs, nh, nkv, hd, hd, True,
                                         scale, ob)
    elif kind == "plain":
        ctx.attention_ragged(qb, kb, vb, bchip.F16, ob, lens, offs, nh, nkv, hd, scale)
    else:
        for i, (L, off) in enumerate(zip(lens, offs)):
            L, off = int(L), int(off)
            ctx.rope_append_attention(qb.offset(i * nh * hd * 4), knb.offset(i * kvd * 4), vnb.offset(i * kvd * 4),
                                      kb.offset(off * kvd * 2), vb.offset(off * kvd * 2), bchip.F16, ib,
                                      pb.offset(4 * i), nh, nkv, hd, hd, True, L - 1, scale, ob.offset(i * nh * hd * 4))
    res = (ctx.read(ob, (n, nh, hd)), ctx.read(qb, q.shape), ctx.read(kb, (total, kvd), np.float16),
           ctx.read(vb, (total, kvd), np.float16))
    for b in (kb, vb, qb, knb, vnb, ib, pb, ob):
        b.free()
    return res


CASES = [
    # lens, nh, nkv, hd: one chunk, a partial last run, whole runs, the longest lists
    ([1, 64, 65, 300, 1000, 5000], 32, 8, 128),
    ([32768], 32, 8, 128),
    ([20000, 777, 3], 28, 4, 128),
    ([4097, 129, 12345], 14, 2, 64),
    ([6000, 70], 16, 4, 256),
    ([3000, 2500], 8, 2, 96),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_runs_give_the_chunk_units_bits(ctxs, case):
    lens, nh, nkv, hd = CASES[case]
    runs, chunks = ctxs
    print(f"row runs: lens {lens}, heads {nh}/{nkv}, hd {hd}", flush=True)
    for kind in ("fused", "plain", "single"):
        a = step(runs, kind, lens, nh, nkv, hd, 80 + case)
        b = step(chunks, kind, lens, nh, nkv, hd, 80 + case)
        for name, x, y in zip(("out", "q", "K pool", "V pool"), a, b):
            np.testing.assert_array_equal(x, y, err_msg=f"{kind}: {name}")


def test_runs_against_the_oracle(ctxs):
    """A unit a run, plain attention over an f16 pool, each list against the oracle."""
    lens, nh, nkv, hd = [5000, 1300, 2], 16, 4, 128
    runs = ctxs[0]
    out, q, kc, vc = step(runs, "plain", lens, nh, nkv, hd, 90)
    off = 0
    for i, L in enumerate(lens):
        want = O.attention(q[i].reshape(1, nh, hd), kc[off:off + L].astype(np.float32),
                           vc[off:off + L].astype(np.float32), 1, L - 1, nh, nkv, hd, 1.0 / math.sqrt(hd))
        err = float(np.abs(out[i:i + 1] - want).max())
        print(f"list {i} ({L} slots): max abs {err:.3g}", flush=True)
        assert err <= 5e-3
        off += L
