"""Parity of the HIP attention (libbchip.so, through its C ABI) with the CPU oracle, and the
reference's bit-exact invariants (crates/bc-infer/src/model.rs:538-650).

Gate: max abs error <= 5e-3 and cosine >= 0.9999 against the
f32 oracle. For an f16 cache both the kernel error (oracle fed the f16-rounded K/V) and the
total error (oracle fed the unrounded f32 values) must pass.
"""
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
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def gate(got, want, what):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    err = float(np.abs(got - want).max())
    cos = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want)))
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max abs {err:.3g}, cosine {cos:.8f}"
    return err, cos


class Attn:
    """Device buffers for one attention problem: cache of `slots`, q and out of `rows`."""

    def __init__(self, ctx, kc, vc, kv_type, nh, nkv, hd):
        self.ctx, self.kv_type, self.nh, self.nkv, self.hd = ctx, kv_type, nh, nkv, hd
        dt = np.float16 if kv_type == bchip.F16 else np.float32
        self.kc = ctx.upload(np.ascontiguousarray(kc, np.float32).astype(dt))
        self.vc = ctx.upload(np.ascontiguousarray(vc, np.float32).astype(dt))

    def run(self, q, rows, pos, scale, visible=None):
        ctx = self.ctx
        qb = ctx.upload(np.ascontiguousarray(q, np.float32))
        out = ctx.zeros(rows * self.nh * self.hd * 4)
        mb = None
        if visible is not None:
            mb = ctx.upload(bchip.masks_words(visible))
        ctx.attention(qb, self.kc, self.vc, self.kv_type, out, mb, visible is not None, rows, self.nh, self.nkv,
                      self.hd, pos, scale)
        res = ctx.read(out, (rows, self.nh, self.hd))
        qb.free()
        out.free()
        if mb is not None:
            mb.free()
        return res

    def free(self):
        self.kc.free()
        self.vc.free()


def check_against_oracle(got, q, kc, vc, kv_type, rows, pos, nh, nkv, hd, scale, visible=None, base=None, what=""):
    if kv_type == bchip.F16:
        kr, vr = O.f16_round(kc), O.f16_round(vc)
        gate(got, O.attention(q, kr, vr, rows, pos, nh, nkv, hd, scale, visible, base), what + " (kernel error)")
    gate(got, O.attention(q, kc, vc, rows, pos, nh, nkv, hd, scale, visible, base), what + " (total error)")


DECODE = [
    # nh, nkv, hd, slots, kv_type
    (14, 2, 64, 512, bchip.F32),   # config 1 shape
    (32, 8, 128, 1, bchip.F16),
    (32, 8, 128, 2, bchip.F16),
    (32, 8, 128, 63, bchip.F16),
    (32, 8, 128, 65, bchip.F16),
    (32, 8, 128, 1024, bchip.F16),  # config 2 contexts
    (32, 8, 128, 4096, bchip.F16),
    (32, 8, 128, 16385, bchip.F16),
    (28, 4, 128, 3001, bchip.F16),  # Qwen2.5-7B shape
    (4, 2, 16, 7, bchip.F32),       # the reference's tiny_model shape (fixtures.rs:8)
    (8, 8, 256, 300, bchip.F16),
    (16, 1, 128, 200, bchip.F16),   # a group of 16
    (12, 3, 40, 150, bchip.F32),    # head_dim padded inside the kernel
    # The one-row kernel takes a list's last entry as a block of its own after the last
    # chunk's stream: lists whose last chunk holds that entry alone (chunks of 64 entries).
    (32, 8, 128, 257, bchip.F16),
    (32, 8, 128, 4097, bchip.F16),
    (28, 4, 128, 8193, bchip.F16),
    (14, 2, 64, 129, bchip.F32),
    (32, 8, 128, 32769, bchip.F16),  # configs[1]'s step: 114 chunks of 288, the last of 225
]


@pytest.mark.parametrize("nh,nkv,hd,slots,kv_type", DECODE)
def test_decode_matches_oracle(ctx, nh, nkv, hd, slots, kv_type):
    seed = nh * 1000 + slots
    q = rand((1, nh, hd), seed)
    kc, vc = rand((slots, nkv * hd), seed + 1), rand((slots, nkv * hd), seed + 2)
    scale = 1.0 / math.sqrt(hd)
    a = Attn(ctx, kc, vc, kv_type, nh, nkv, hd)
    got = a.run(q, 1, slots - 1, scale)
    a.free()
    check_against_oracle(got, q, kc, vc, kv_type, 1, slots - 1, nh, nkv, hd, scale, what=f"decode {slots}")


def test_qwen05b_config1_decode_24_layers(ctx):
    """14/2 heads, hd 64, 512 slots, f32 K/V with RoPE (theta 1e6, neox)
    pre-applied (K at positions 0..511, Q at 511), scale 1/8, 24 layers of seeds base+layer."""
    nh, nkv, hd, L = 14, 2, 64, 512
    inv = O.inv_freq(hd, 1.0e6)
    for layer in range(24):
        seed = 1000 + layer
        q = O.normal(seed * 3, nh * hd).reshape(1, nh * hd)
        kc = O.normal(seed * 3 + 1, L * nkv * hd).reshape(L, nkv * hd)
        vc = O.normal(seed * 3 + 2, L * nkv * hd).reshape(L, nkv * hd)
        q = O.rope_rows(q, [L - 1], nh, hd, hd, True, inv)
        kc = O.rope_rows(kc, np.arange(L), nkv, hd, hd, True, inv)
        a = Attn(ctx, kc, vc, bchip.F32, nh, nkv, hd)
        got = a.run(q, 1, L - 1, 0.125)
        a.free()
        gate(got, O.attention(q, kc, vc, 1, L - 1, nh, nkv, hd, 0.125), f"layer {layer}")


PREFILL = [
    # rows, pos, nh, nkv, hd, kv_type
    (2, 0, 32, 8, 128, bchip.F16),
    (17, 0, 32, 8, 128, bchip.F16),
    (300, 0, 32, 8, 128, bchip.F16),
    (64, 100, 32, 8, 128, bchip.F16),   # a chunk of a chunked prefill
    (9, 0, 4, 2, 16, bchip.F32),
    (33, 5, 14, 2, 64, bchip.F32),
    (100, 700, 28, 4, 128, bchip.F16),  # G = 7: workgroups straddle heads
    (40, 3, 8, 8, 256, bchip.F16),
    (8, 4096, 64, 8, 128, bchip.F16),   # config 5 verify: split across chunks
    (8, 1000, 16, 1, 128, bchip.F16),
    (5, 600, 14, 2, 64, bchip.F32),     # short line, G = 7: units of 2 rows, f32 cache
    (3, 2000, 28, 4, 128, bchip.F16),   # short line over 8 chunks, G = 7
    (2, 190, 32, 8, 128, bchip.F16),    # lists of 191 and 192: the second ends a chunk
    (4, 381, 28, 4, 128, bchip.F16),    # lists 382..385 across the second chunk's end
    (300, 0, 28, 4, 128, bchip.F16),    # packed-V^T prefill with G = 7 (workgroups straddle heads)
    (2, 190, 32, 8, 128, bchip.F32),    # f32 path: lists of 191 and 192
    (40, 370, 8, 2, 64, bchip.F32),     # f32 path: a row block across the second chunk's end
]


@pytest.mark.parametrize("rows,pos,nh,nkv,hd,kv_type", PREFILL)
def test_multirow_matches_oracle(ctx, rows, pos, nh, nkv, hd, kv_type):
    seed = rows * 7 + pos
    n = pos + rows
    q = rand((rows, nh, hd), seed)
    kc, vc = rand((n, nkv * hd), seed + 1), rand((n, nkv * hd), seed + 2)
    scale = 1.0 / math.sqrt(hd)
    a = Attn(ctx, kc, vc, kv_type, nh, nkv, hd)
    got = a.run(q, rows, pos, scale)
    a.free()
    check_against_oracle(got, q, kc, vc, kv_type, rows, pos, nh, nkv, hd, scale, what=f"rows {rows} at {pos}")


def test_golden_fixtures_on_gpu(ctx):
    import os
    gdir = os.path.join(os.path.dirname(__file__), "golden")
    for f in sorted(x for x in os.listdir(gdir) if x.endswith(".npz")):
        z = np.load(os.path.join(gdir, f))
        rows, pos, nh, nkv, hd = (int(x) for x in z["shape"])
        vis = z["visible"] if z["visible"].size else None
        a = Attn(ctx, z["kc"], z["vc"], bchip.F32, nh, nkv, hd)
        got = a.run(z["q"], rows, pos if vis is None else int(z["base"]), float(z["scale"]), vis)
        a.free()
        gate(got, z["out"], f)


def test_batch_invariance_and_determinism(ctx):
    """A row's bits depend only on its q and its visible slots, not on the batch
    (model.rs:592-594, 646): one 40-row pass against the same rows in passes of 2, 7, 31,
    and the wide (128-slot) and narrow (64-slot) workgroups; and reruns give the same bits
    (model.rs:648)."""
    nh, nkv, hd, pos = 32, 8, 128, 10
    rows = 40
    n = pos + rows
    q = rand((rows, nh, hd), 5)
    kc, vc = rand((n, nkv * hd), 6), rand((n, nkv * hd), 7)
    a = Attn(ctx, kc, vc, bchip.F16, nh, nkv, hd)
    whole = a.run(q, rows, pos, 0.0884)
    again = a.run(q, rows, pos, 0.0884)
    np.testing.assert_array_equal(whole, again)
    start = 0
    for size in (2, 7, 31):
        part = a.run(q[start:start + size], size, pos + start, 0.0884)
        np.testing.assert_array_equal(part, whole[start:start + size], err_msg=f"batch of {size} at {start}")
        start += size
    a.free()


def test_split_and_unsplit_give_the_same_bits(ctx):
    """8 verify rows at a long context, split across CUs by chunk, against the same rows in
    passes of 200 (too few workgroups to run unsplit: the transposing-read kernel, split by
    chunk, combined): identical bits, the chunk fold being fixed. Every row of a large pass
    (enough workgroups for the wide kernel: one online softmax over each row's whole list)
    against those passes: within 1e-4, the reference's bound for a batch row against a
    one-token pass (model.rs:641-642); reruns of the large pass give the same bits
    (model.rs:648)."""
    nh, nkv, hd = 32, 8, 128
    pos = 3000
    big = 2100  # 8 kv heads x 66 row blocks of 32: enough workgroups to run unsplit
    n = pos + big
    q = rand((big, nh, hd), 15)
    kc, vc = rand((n, nkv * hd), 16), rand((n, nkv * hd), 17)
    a = Attn(ctx, kc, vc, bchip.F16, nh, nkv, hd)
    whole = a.run(q, big, pos, 0.0884)
    for _ in range(3):
        np.testing.assert_array_equal(a.run(q, big, pos, 0.0884), whole, err_msg="wide pass rerun")
    worst = 0.0
    for r0 in range(0, big, 200):
        n = min(200, big - r0)
        part = a.run(q[r0:r0 + n], n, pos + r0, 0.0884)
        for v0 in (r0, r0 + n - 8):
            verify = a.run(q[v0:v0 + 8], 8, pos + v0, 0.0884)
            np.testing.assert_array_equal(verify, part[v0 - r0:v0 - r0 + 8], err_msg=f"rows {v0}.. in a pass of {n}")
        worst = max(worst, float(np.abs(part - whole[r0:r0 + n]).max()))
    print(f"wide pass against passes of 200: max abs {worst:.3g}", flush=True)
    assert worst < 1e-4
    a.free()


def test_decode_against_a_batch_row(ctx):
    """A one-row pass against the same row in a batch: within 1e-4 (model.rs:641-642). The
    one-row pass folds its chunks in groups (a two-level fold), a batch row in one left
    fold, so they agree within rounding."""
    nh, nkv, hd = 32, 8, 128
    for slots in (700, 16400):
        q = rand((3, nh, hd), slots)
        kc, vc = rand((slots + 2, nkv * hd), 1), rand((slots + 2, nkv * hd), 2)
        a = Attn(ctx, kc, vc, bchip.F16, nh, nkv, hd)
        batch = a.run(q, 3, slots - 1, 0.0884)
        one = a.run(q[:1], 1, slots - 1, 0.0884)
        again = a.run(q[:1], 1, slots - 1, 0.0884)
        a.free()
        np.testing.assert_array_equal(one, again)
        assert np.abs(one[0] - batch[0]).max() < 1e-4


def test_decode_rows_are_independent_of_their_launch(ctx):
    """Decode workgroups take (chunk, KV head) units dynamically, in whatever order they
    finish; a row's chunk states are combined by a tree fixed by its length. So the same
    row gets the same bits in a launch of 64 rows as alone."""
    nh, nkv, hd = 16, 16, 64
    lens = [200] * 60 + [1, 64, 65, 3000]
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    total = int(sum(lens))
    kc, vc = rand((total, nkv * hd), 31), rand((total, nkv * hd), 32)
    q = rand((len(lens), nh, hd), 33)
    kb, vb, qb = ctx.upload(kc.astype(np.float16)), ctx.upload(vc.astype(np.float16)), ctx.upload(q)
    out = ctx.zeros(q.nbytes)
    ctx.attention_ragged(qb, kb, vb, bchip.F16, out, lens, offs, nh, nkv, hd, 0.125)  # 64 x 16 units: in registers
    got = ctx.read(out, q.shape)
    for i in (0, 59, 60, 61, 62, 63):
        off, L = int(offs[i]), lens[i]
        a = Attn(ctx, kc[off:off + L], vc[off:off + L], bchip.F16, nh, nkv, hd)
        one = a.run(q[i:i + 1], 1, L - 1, 0.125)  # a single row: split across CUs
        a.free()
        np.testing.assert_array_equal(got[i], one[0], err_msg=f"sequence {i} ({L} slots)")
    check_against_oracle(got[62:63], q[62:63], kc[int(offs[62]):int(offs[62]) + 65], vc[int(offs[62]):int(offs[62]) + 65],
                         bchip.F16, 1, 64, nh, nkv, hd, 0.125, what="65 slots")
    for b in (kb, vb, qb, out):
        b.free()


def tree_setup(nh, nkv, hd, prefix, seed):
    tree = [O.ROOT, 0, 0, 1, O.ROOT]
    rows = len(tree)
    positions, visible, base = O.shape(rows, prefix, tree)
    n = prefix + rows
    q = rand((rows, nh, hd), seed)
    kc, vc = rand((n, nkv * hd), seed + 1), rand((n, nkv * hd), seed + 2)
    return tree, visible, base, q, kc, vc


@pytest.mark.parametrize("prefix,kv_type", [(3, bchip.F32), (3, bchip.F16), (700, bchip.F16), (1030, bchip.F32)])
def test_tree_rows_equal_their_line(ctx, prefix, kv_type):
    """model.rs:538-579: each tree row gets exactly the bits of the line its path is (the
    path fed alone after the prefix, as one multi-row pass), and matches the oracle."""
    nh, nkv, hd = 4, 2, 16
    tree, visible, base, q, kc, vc = tree_setup(nh, nkv, hd, prefix, prefix)
    rows = len(tree)
    a = Attn(ctx, kc, vc, kv_type, nh, nkv, hd)
    got = a.run(q, rows, base, 0.25, visible)
    a.free()
    check_against_oracle(got, q, kc, vc, kv_type, rows, prefix, nh, nkv, hd, 0.25, visible, base, "tree")
    paths = [[0], [0, 1], [0, 2], [0, 1, 3], [4]]
    for row, path in enumerate(paths):
        n = prefix + len(path)
        lk = np.concatenate([kc[:prefix], kc[[prefix + p for p in path]]])
        lv = np.concatenate([vc[:prefix], vc[[prefix + p for p in path]]])
        lq = rand((n, nh, hd), 99)
        lq[-1] = q[row]
        line = Attn(ctx, lk, lv, kv_type, nh, nkv, hd)
        want = line.run(lq, n, 0, 0.25)
        line.free()
        np.testing.assert_array_equal(got[row], want[-1], err_msg=f"row {row}, path {path}")


def test_tree_grown_a_level_at_a_time(ctx):
    """model.rs:580-594: the same tree fed a level at a time gives every multi-row node the
    same bits; the last level is a one-row pass and agrees within rounding."""
    nh, nkv, hd, prefix = 8, 2, 64, 40
    order_parents = [O.ROOT, O.ROOT, 0, 0, 2]
    n = prefix + 5
    q = rand((5, nh, hd), 3)
    kc, vc = rand((n, nkv * hd), 4), rand((n, nkv * hd), 5)
    a = Attn(ctx, kc, vc, bchip.F16, nh, nkv, hd)
    _, vis_all, base = O.shape(5, prefix, order_parents)
    whole = a.run(q, 5, base, 0.125, vis_all)
    for lo, hi in ((0, 2), (2, 4), (4, 5)):
        _, vis, b = O.shape(hi - lo, prefix + lo, order_parents[:hi])
        part = a.run(q[lo:hi], hi - lo, b, 0.125, vis)
        if hi - lo >= 2:
            np.testing.assert_array_equal(part, whole[lo:hi])
        else:
            assert np.abs(part - whole[lo:hi]).max() < 1e-4
    a.free()


@pytest.mark.parametrize("prefix,kv_type", [(190, bchip.F16), (191, bchip.F16), (190, bchip.F32)])
def test_grown_tree_level_whose_list_passes_its_rows(ctx, prefix, kv_type):
    """A tree fed a level at a time (model.rs:580-594): the last level of [ROOT, ROOT, 0, 0,
    2] is one row that sees the prefix and nodes 0, 2 and 4, so its list (prefix + 3) runs
    past prefix + rows, across the first 192-entry chunk's end. Against the oracle, and bit
    for bit against the line its path is."""
    nh, nkv, hd = 8, 2, 64
    parents = [O.ROOT, O.ROOT, 0, 0, 2]
    n = prefix + len(parents)
    q = rand((len(parents), nh, hd), prefix)
    kc, vc = rand((n, nkv * hd), prefix + 1), rand((n, nkv * hd), prefix + 2)
    a = Attn(ctx, kc, vc, kv_type, nh, nkv, hd)
    _, vis, base = O.shape(1, prefix + 4, parents)
    assert base == prefix and int(vis[0]) == 0b10101
    got = a.run(q[4:5], 1, base, 0.125, vis)
    a.free()
    check_against_oracle(got, q[4:5], kc, vc, kv_type, 1, prefix + 4, nh, nkv, hd, 0.125, vis, base, "grown level")
    path = [0, 2, 4]
    lk = np.concatenate([kc[:prefix], kc[[prefix + j for j in path]]])
    lv = np.concatenate([vc[:prefix], vc[[prefix + j for j in path]]])
    lq = rand((prefix + 3, nh, hd), 98)
    lq[-1] = q[4]
    line = Attn(ctx, lk, lv, kv_type, nh, nkv, hd)
    want = line.run(lq, prefix + 3, 0, 0.125)
    line.free()
    np.testing.assert_array_equal(got[0], want[-1])


@pytest.mark.parametrize("kv_type", [bchip.F16, bchip.F32])
def test_grown_tree_level_across_the_second_chunk(ctx, kv_type):
    """A chain of 8 nodes after 380 slots, fed as two levels of 4: the second level's rows see
    lists of 385..388 entries, across the second chunk's end (384), while the pass's rows end
    at 384. Every row against the oracle and against the same rows of the whole tree in one
    pass, bit for bit."""
    nh, nkv, hd, prefix = 4, 2, 16, 380
    parents = [O.ROOT, 0, 1, 2, 3, 4, 5, 6]
    n = prefix + 8
    q = rand((8, nh, hd), 11)
    kc, vc = rand((n, nkv * hd), 12), rand((n, nkv * hd), 13)
    a = Attn(ctx, kc, vc, kv_type, nh, nkv, hd)
    _, vis_all, base = O.shape(8, prefix, parents)
    whole = a.run(q, 8, base, 0.25, vis_all)
    _, vis, b2 = O.shape(4, prefix + 4, parents)
    assert b2 == base
    part = a.run(q[4:], 4, b2, 0.25, vis)
    a.free()
    check_against_oracle(part, q[4:], kc, vc, kv_type, 4, prefix + 4, nh, nkv, hd, 0.25, vis, b2, "second level")
    np.testing.assert_array_equal(part, whole[4:])


def test_ragged_matches_single_sequence_decode(ctx):
    """Config 4's layout: sequences of different lengths in one pool, one launch; each
    sequence's result is its own one-row pass, bit for bit, and matches the oracle."""
    nh, nkv, hd = 28, 4, 128
    lens = [1, 64, 65, 1000, 4097, 20000, 300, 17]
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64) + 5
    total = int(offs[-1]) + lens[-1]
    kc, vc = rand((total, nkv * hd), 1), rand((total, nkv * hd), 2)
    q = rand((len(lens), nh, hd), 3)
    dt = np.float16
    kb, vb = ctx.upload(kc.astype(dt)), ctx.upload(vc.astype(dt))
    qb = ctx.upload(q)
    out = ctx.zeros(q.nbytes)
    ctx.attention_ragged(qb, kb, vb, bchip.F16, out, lens, offs, nh, nkv, hd, 0.0884)
    got = ctx.read(out, q.shape)
    for i, (L, off) in enumerate(zip(lens, offs)):
        off = int(off)
        a = Attn(ctx, kc[off:off + L], vc[off:off + L], bchip.F16, nh, nkv, hd)
        one = a.run(q[i:i + 1], 1, L - 1, 0.0884)
        a.free()
        np.testing.assert_array_equal(got[i], one[0], err_msg=f"sequence {i}")
        if L <= 4097:
            check_against_oracle(got[i:i + 1], q[i:i + 1], kc[off:off + L], vc[off:off + L], bchip.F16, 1, L - 1,
                                 nh, nkv, hd, 0.0884, what=f"sequence {i}")
    for b in (kb, vb, qb, out):
        b.free()


def test_long_conversation_in_chunks(ctx):
    """model.rs:652-674: 1100 tokens fed in chunks of 300 cross the reference's 1024 tile;
    every chunk matches the oracle."""
    nh, nkv, hd, total = 4, 2, 16, 1100
    q = rand((total, nh, hd), 8)
    kc, vc = rand((total, nkv * hd), 9), rand((total, nkv * hd), 10)
    a = Attn(ctx, kc, vc, bchip.F32, nh, nkv, hd)
    for start in range(0, total, 300):
        rows = min(300, total - start)
        got = a.run(q[start:start + rows], rows, start, 0.25)
        want = O.attention(q[start:start + rows], kc, vc, rows, start, nh, nkv, hd, 0.25)
        gate(got, want, f"chunk at {start}")
    a.free()


def test_bad_arguments_are_refused_before_launch(ctx):
    kc = ctx.zeros(10 * 8 * 128 * 2)
    q = ctx.zeros(32 * 128 * 4)
    out = ctx.zeros(32 * 128 * 4)
    with pytest.raises(bchip.BchipError) as e:  # the cache holds 10 slots, not 20
        ctx.attention(q, kc, kc, bchip.F16, out, None, False, 1, 32, 8, 128, 19, 0.1)
    assert "kc" in str(e.value)
    with pytest.raises(bchip.BchipError):  # 32 heads over 5 KV heads
        ctx.attention(q, kc, kc, bchip.F16, out, None, False, 1, 32, 5, 128, 0, 0.1)
    with pytest.raises(bchip.BchipError):  # a tree without masks
        ctx.attention(q, kc, kc, bchip.F16, out, None, True, 1, 32, 8, 128, 0, 0.1)
    # bchip_rope_append: an inv_freq buffer shorter than rope_dim / 2 floats.
    inv = ctx.zeros(16 * 4)
    pos = ctx.zeros(4)
    kn = ctx.zeros(8 * 128 * 4)
    with pytest.raises(bchip.BchipError) as e:
        ctx.rope_append(q, kn, kn, kc, kc, bchip.F16, inv, pos, 1, 32, 8, 128, 128, False, 0)
    assert "inv_freq" in str(e.value)
    for b in (kc, q, out, inv, pos, kn):
        b.free()
