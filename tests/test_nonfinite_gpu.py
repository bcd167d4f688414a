"""Non-finite inputs stay where they are.

The f16 attention kernels are built with -fno-honor-nans (a masked entry is -inf, so a max
needs no NaN-quieting of its operands), which leaves unspecified the output of a (row,
query head) whose q holds a NaN, or whose visible list holds a K or V element that is
infinite or NaN. What the build does fix, and what these tests check bit for bit over f16
and f32 caches, is that no other output moves: every slot's max, sum and weighted values
are its own, in the decode step, the split verify rows (the group fold), the wide prefill
and the chunked line, so one bad value cannot spread to another head, another KV group or
an earlier row. (The
reference's kernel computes the same products in IEEE arithmetic, kernels.h:271-324, where a
non-finite input likewise reaches only the outputs that read it.)

One difference from that kernel is checked as it stands: the multi-row kernels multiply a
whole block of V by P (64 entries over f16 caches, 32 over f32), and an entry a row does not
see has P = 0 there, so a V element that is NaN or infinite (0 x inf is NaN) also reaches,
in its own dimension, the rows of its KV group that stream its block without seeing it;
the reference's loop, bounded by each row's length, does not touch such an entry. A K
element does not: masked scores are replaced, not multiplied."""
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


def _run(ctx, q, kc, vc, rows, pos, nh, nkv, hd, kv_type):
    kb, vb = ctx.upload(kc), ctx.upload(vc)
    qb, ob = ctx.upload(q), ctx.zeros(q.nbytes)
    ctx.attention(qb, kb, vb, kv_type, ob, None, False, rows, nh, nkv, hd, pos, 1.0 / math.sqrt(hd))
    out = ctx.read(ob, (rows, nh, hd))
    for b in (kb, vb, qb, ob):
        b.free()
    return out


# (rows, pos, nh, nkv): a decode step at 4096 slots, a verify pass split over chunks and
# folded in the same launch, a 300-row line (chunked kernel), a 2048-row prefill (wide).
SHAPES = [(1, 4095, 32, 8), (8, 4096, 64, 8), (300, 700, 32, 8), (2048, 0, 32, 8)]


@pytest.mark.parametrize("rows,pos,nh,nkv", SHAPES)
@pytest.mark.parametrize("what", ["q_nan", "k_inf", "v_nan"])
@pytest.mark.parametrize("kv_type", [bchip.F16, bchip.F32], ids=["f16", "f32"])
def test_a_non_finite_input_reaches_only_its_own_outputs(ctx, rows, pos, nh, nkv, what, kv_type):
    hd = 128
    rng = np.random.default_rng(rows + pos + len(what))
    kvd, slots, G = nkv * hd, pos + rows, nh // nkv
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    q = rng.standard_normal((rows, nh * hd)).astype(np.float32)
    kc = rng.standard_normal((slots, kvd)).astype(dt)
    vc = rng.standard_normal((slots, kvd)).astype(dt)
    clean = _run(ctx, q, kc, vc, rows, pos, nh, nkv, hd, kv_type)
    assert np.isfinite(clean).all()
    # Which outputs may move: a q element moves its own (row, head); a K/V entry at slot s of
    # KV head j moves the heads of group j in the rows that see s (row r sees pos + r + 1).
    may = np.zeros((rows, nh), bool)
    r0, h0 = rows // 2, nh // 2 + 1
    if what == "q_nan":
        q = q.copy()
        q[r0, h0 * hd + 7] = np.nan
        may[r0, h0] = True
    else:
        j, s = nkv - 2, min(pos + rows // 3, slots - 1)
        cache = (kc if what == "k_inf" else vc).copy()
        cache[s, j * hd + 33] = np.inf if what == "k_inf" else np.nan
        if what == "k_inf":
            kc = cache
        else:
            vc = cache
        # A row sees s, or (V) streams the block that holds it: 64 entries (f16 caches, MFMA
        # tiles), 32 (f32 caches, attn_f32's blocks).
        blk = 64 if kv_type == bchip.F16 else 32
        first = s if what == "k_inf" else s - s % blk
        seen = pos + np.arange(rows) + 1 > first
        may[np.ix_(seen, np.arange(j * G, (j + 1) * G))] = True
    planted = _run(ctx, q, kc, vc, rows, pos, nh, nkv, hd, kv_type)
    keep = ~may
    np.testing.assert_array_equal(planted[keep].view(np.uint32), clean[keep].view(np.uint32),
                                  err_msg=f"{what}: an output that does not read the planted value moved")
    assert may.any()
