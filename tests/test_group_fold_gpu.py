"""The single-launch fold of split passes (group fold) against the two-launch fold.

A multi-row pass with few workgroups is split by chunk across CUs. Its chunk states are
folded left to right, either by the split launch's own workgroups once their group is
complete (the group fold: one launch), or by attn_combine after the split launch has
drained (two launches, which BCHIP_GROUP_FOLD=0 at init selects). Both folds take the states
in chunk order with the same expressions, so the outputs must be the same bits. The cases
cover both kernels that split (four waves for verify-sized passes, eight for wider ones),
groups of 2 to 32 chunks (the last filling all 256 CUs), query groups of 4, 7, 8 and 16, and
row blocks that end inside a group.
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
    one = bchip.Ctx(0)
    old = os.environ.get("BCHIP_GROUP_FOLD")
    os.environ["BCHIP_GROUP_FOLD"] = "0"
    try:
        two = bchip.Ctx(0)
    finally:
        if old is None:
            del os.environ["BCHIP_GROUP_FOLD"]
        else:
            os.environ["BCHIP_GROUP_FOLD"] = old
    yield one, two
    one.close()
    two.close()


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


class Pass:
    def __init__(self, ctx, q, kc, vc, nh, nkv, hd):
        self.ctx, self.nh, self.nkv, self.hd = ctx, nh, nkv, hd
        self.q = ctx.upload(q)
        self.kc = ctx.upload(kc.astype(np.float16))
        self.vc = ctx.upload(vc.astype(np.float16))
        self.out = ctx.zeros(q.nbytes)

    def run(self, rows, pos):
        ctx = self.ctx
        ctx.attention(self.q, self.kc, self.vc, bchip.F16, self.out, None, False, rows, self.nh, self.nkv, self.hd,
                      pos, 1.0 / math.sqrt(self.hd))
        return ctx.read(self.out, (rows, self.nh, self.hd))

    def free(self):
        for b in (self.q, self.kc, self.vc, self.out):
            b.free()


CASES = [
    # rows, pos, nh, nkv, hd
    (8, 4096, 64, 8, 128),   # configs[4]'s verify: 22 chunks x 8 KV heads, four-wave kernel
    (8, 6136, 64, 8, 128),   # its last step: 32 chunks x 8 = 256 workgroups, every CU
    (8, 4096, 32, 8, 128),   # G = 4
    (3, 2000, 28, 4, 128),   # G = 7, a row block of 3 rows
    (8, 1000, 16, 1, 128),   # one KV head, G = 16
    (2, 200, 32, 8, 128),    # 2 chunks
    (100, 700, 28, 4, 128),  # eight-wave kernel: 6 row blocks x 4 KV heads x 5 chunks
    (64, 1000, 32, 8, 128),  # eight-wave kernel: 2 row blocks x 8 KV heads x 6 chunks
]


@pytest.mark.parametrize("rows,pos,nh,nkv,hd", CASES)
def test_group_fold_gives_the_bits_of_the_two_launch_fold(ctxs, rows, pos, nh, nkv, hd):
    one, two = ctxs
    n = pos + rows
    q = rand((rows, nh, hd), rows + pos)
    kc, vc = rand((n, nkv * hd), pos + 1), rand((n, nkv * hd), pos + 2)
    a, b = Pass(one, q, kc, vc, nh, nkv, hd), Pass(two, q, kc, vc, nh, nkv, hd)
    got, want = a.run(rows, pos), b.run(rows, pos)
    a.free()
    b.free()
    np.testing.assert_array_equal(got, want)
    # And within the north star's bound of the oracle on the f16-rounded caches.
    ref = O.attention(q, O.f16_round(kc), O.f16_round(vc), rows, pos, nh, nkv, hd, 1.0 / math.sqrt(hd))
    assert float(np.abs(got - ref).max()) <= 5e-3


def test_group_counters_start_over_between_calls(ctxs):
    """Passes of different chunk counts over the same groups, queued back to back with no sync
    between them: each call's group counters must be back at zero for the next. Every call
    equals the same pass run alone, bit for bit."""
    one, _ = ctxs
    nh, nkv, hd = 64, 8, 128
    n = 6200
    q = rand((8, nh, hd), 3)
    kc, vc = rand((n, nkv * hd), 4), rand((n, nkv * hd), 5)
    p = Pass(one, q, kc, vc, nh, nkv, hd)
    positions = [4096, 200, 6136, 1000, 5000, 190, 3000]
    alone = {pos: p.run(8, pos) for pos in positions}
    outs = [(pos, one.zeros(8 * nh * hd * 4)) for rep in range(4) for pos in positions]
    one.sync()
    for pos, out in outs:
        one.attention(p.q, p.kc, p.vc, bchip.F16, out, None, False, 8, nh, nkv, hd, pos, 1.0 / math.sqrt(hd))
    one.sync()
    for pos, out in outs:
        np.testing.assert_array_equal(one.read(out, (8, nh, hd)), alone[pos], err_msg=f"pos {pos}")
        out.free()
    p.free()


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


@pytest.mark.parametrize("rows,pos,nh,nkv,hd", [(8, 4096, 64, 8, 128), (100, 700, 28, 4, 128)])
def test_spread_groups_give_the_same_bits(ctxs, rows, pos, nh, nkv, hd):
    """The path of a group whose workgroups ran on several XCDs (each state published again
    write-through, a second count, an agent-scope acquire), forced from the host: the same
    bits as the two-launch fold."""
    _, two = ctxs
    spread = _ctx_with({"BCHIP_GROUP_FOLD": "spread"})
    try:
        n = pos + rows
        q = rand((rows, nh, hd), rows + pos)
        kc, vc = rand((n, nkv * hd), pos + 1), rand((n, nkv * hd), pos + 2)
        a, b = Pass(spread, q, kc, vc, nh, nkv, hd), Pass(two, q, kc, vc, nh, nkv, hd)
        for _ in range(3):  # and its counters start over between calls
            np.testing.assert_array_equal(a.run(rows, pos), b.run(rows, pos))
        a.free()
        b.free()
    finally:
        spread.close()


def test_a_wait_that_runs_out_is_reported_and_the_next_call_recovers(ctxs):
    """A group fold whose bound on waiting runs out (forced from the host: a bound of one poll,
    so workgroups that arrive before the last stop waiting) writes NaN for its outputs and sets
    the context's error word: the next bchip_sync reports it, and a call after that, with the
    counters cleared, is right again. Every kernel still exits normally."""
    _, two = ctxs
    short = _ctx_with({"BCHIP_GROUP_FOLD_SPINS": "1"})
    try:
        rows, pos, nh, nkv, hd = 8, 4096, 64, 8, 128
        n = pos + rows
        q = rand((rows, nh, hd), 9)
        kc, vc = rand((n, nkv * hd), 10), rand((n, nkv * hd), 11)
        a, b = Pass(short, q, kc, vc, nh, nkv, hd), Pass(two, q, kc, vc, nh, nkv, hd)
        want = b.run(rows, pos)
        reported = 0
        for _ in range(20):
            short.attention(a.q, a.kc, a.vc, bchip.F16, a.out, None, False, rows, nh, nkv, hd, pos,
                            1.0 / math.sqrt(hd))
            try:
                short.sync()
            except bchip.BchipError as e:
                assert e.code == bchip.E_HIP and "timed out" in str(e)
                reported += 1
                got = short.read(a.out, (rows, nh, hd))
                assert np.isnan(got).any()
                continue
            np.testing.assert_array_equal(short.read(a.out, (rows, nh, hd)), want)
        print(f"{reported} of 20 calls ran out of their one poll", flush=True)
        assert reported > 0
        a.free()
        b.free()
    finally:
        short.close()
    # The other contexts are unaffected.
    one, _ = ctxs
    p = Pass(one, q, kc, vc, nh, nkv, hd)
    np.testing.assert_array_equal(p.run(rows, pos), want)
    p.free()
