"""The long-list fold (attn_combine_long) against attn_combine (selected for every list with
BCHIP_COMBINE_LONG=0 at init).

Split passes whose lists run past CMB_RUN chunks (an f32 cache's decode and short passes,
tree rows at long contexts) fold their chunk states in attn_combine_long: a workgroup per
output slot stages the slot's states in LDS, takes each chunk's weights from the prefix
maximum of the chunk maxima, and runs the serial recurrence in chunk order with
attn_combine's expressions. The outputs must be the same bits as attn_combine's. The cases
cover one segment and several (the LDS holds 224 chunk states at hd 128, 256 at hd 64, 112
at hd 256), a padded head dim, line passes of several rows (row blocks of G heads), and tree
rows on f16 and f32 caches (the decode kernels' state layout).
"""
import os

import numpy as np
import pytest

import bchip
import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctxs():
    one = bchip.Ctx(0)
    old = os.environ.get("BCHIP_COMBINE_LONG")
    os.environ["BCHIP_COMBINE_LONG"] = "0"
    try:
        two = bchip.Ctx(0)
    finally:
        if old is None:
            del os.environ["BCHIP_COMBINE_LONG"]
        else:
            os.environ["BCHIP_COMBINE_LONG"] = old
    yield one, two
    one.close()
    two.close()


def run(ctx, q, kc, vc, kv_type, rows, pos, nh, nkv, hd, visible=None):
    dt = np.float16 if kv_type == bchip.F16 else np.float32
    qb, kb, vb = ctx.upload(q), ctx.upload(kc.astype(dt)), ctx.upload(vc.astype(dt))
    out = ctx.zeros(q.nbytes)
    mb = ctx.upload(bchip.masks_words(visible)) if visible is not None else None
    ctx.attention(qb, kb, vb, kv_type, out, mb, visible is not None, rows, nh, nkv, hd, pos, 1.0 / np.sqrt(hd))
    got = ctx.read(out, (rows, nh, hd))
    for b in (qb, kb, vb, out, mb):
        if b is not None:
            b.free()
    return got


CASES = [
    # kv_type, rows, pos, nh, nkv, hd: every one a split pass of more than 32 chunks
    (bchip.F32, 1, 8000, 32, 8, 128),    # 42 chunks, one segment
    (bchip.F32, 1, 50000, 14, 2, 64),    # 261 chunks at hd 64: two segments of up to 256
    (bchip.F32, 1, 30000, 16, 4, 256),   # 157 chunks at hd 256: two segments of up to 112
    (bchip.F32, 1, 45000, 32, 8, 128),   # 235 chunks: a full segment of 224 and 11 more
    (bchip.F32, 1, 7000, 8, 2, 96),      # hd 96, padded to 128
    (bchip.F32, 5, 7000, 28, 4, 128),    # five rows, G = 7: row blocks of 2 rows
    (bchip.F16, 8, 7000, 16, 4, 64),     # an f16 line pass at hd 64 (split, folded by the combine)
    (bchip.F16, 5, 9000, 32, 8, 128),    # f16 tree rows: the decode kernel's state layout
    (bchip.F32, 5, 7000, 16, 4, 64),     # f32 tree rows
]


@pytest.mark.parametrize("kv_type,rows,pos,nh,nkv,hd", CASES)
def test_long_fold_gives_the_bits_of_attn_combine(ctxs, kv_type, rows, pos, nh, nkv, hd):
    one, two = ctxs
    print(f"case {'f16' if kv_type == bchip.F16 else 'f32'} rows {rows} pos {pos} heads {nh}/{nkv} hd {hd}", flush=True)
    rng = np.random.default_rng(pos + hd)
    q = rng.standard_normal((rows, nh, hd)).astype(np.float32)
    n = pos + rows
    kc = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    visible = base = None
    if rows == 5 and (kv_type == bchip.F16 or hd == 64):
        tree = [O.ROOT, 0, 0, 1, O.ROOT]
        _, visible, base = O.shape(rows, pos, tree)
    p = base if visible is not None else pos
    got = run(one, q, kc, vc, kv_type, rows, p, nh, nkv, hd, visible)
    want = run(two, q, kc, vc, kv_type, rows, p, nh, nkv, hd, visible)
    np.testing.assert_array_equal(got, want)
    assert np.isfinite(got).all()
    if visible is None and rows == 1 and pos <= 8000:
        ref = O.attention(q, kc, vc, rows, pos, nh, nkv, hd, 1.0 / np.sqrt(hd))
        assert float(np.abs(got - ref).max()) <= 1e-4
