"""Pins the CPU oracle (oracle/bc_oracle.c) before anything is checked against it.

Each oracle function is checked against something that is not its own formula retyped:
an f64 brute force over an explicit visibility matrix, torch's scaled_dot_product_attention
in f64, closed forms, the reference's own tests (crates/bc-infer/src/model.rs:538-611,
676-688), numpy's IEEE float16, and the published splitmix64 sequence. Plausible mistakes
(a wrong KV-head mapping, a wrong tree slot, a dropped scale, sequential instead of
8-lane dot order) each fail at least one of these; test_mutants_are_caught shows it.
"""
import math
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def visibility(rows, pos, visible=None, base=None):
    """[rows][pos+rows] booleans from the definition (model.rs:445-447, 458-459)."""
    n = pos + rows
    m = np.zeros((rows, n), bool)
    for i in range(rows):
        if visible is None:
            m[i, : pos + i + 1] = True
        else:
            m[i, :base] = True
            for j in range(n - base):
                if (int(visible[i]) >> j) & 1:
                    m[i, base + j] = True
    return m


def brute(q, kc, vc, rows, pos, nh, nkv, hd, scale, visible=None, base=None):
    """f64 attention over an explicit mask, heads mapped h -> h // (nh // nkv)."""
    vis = visibility(rows, pos, visible, base)
    n = vis.shape[1]
    q = q.reshape(rows, nh, hd).astype(np.float64)
    k = kc[: n * nkv * hd].reshape(n, nkv, hd).astype(np.float64)
    v = vc[: n * nkv * hd].reshape(n, nkv, hd).astype(np.float64)
    grp = nh // nkv
    out = np.zeros((rows, nh, hd))
    for h in range(nh):
        s = q[:, h, :] @ k[:, h // grp, :].T * scale
        s = np.where(vis, s, -np.inf)
        s = s - s.max(axis=1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h, :] = p @ v[:, h // grp, :]
    return out


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


CASES = [
    # rows, pos, nh, nkv, hd
    (1, 0, 4, 2, 16),
    (1, 511, 14, 2, 64),
    (4, 3, 4, 2, 16),
    (5, 40, 8, 8, 32),
    (3, 100, 28, 4, 128),
    (7, 9, 32, 8, 24),  # hd not a multiple of 8: the remainder path of dot
]


@pytest.mark.parametrize("rows,pos,nh,nkv,hd", CASES)
def test_attention_matches_f64_brute_force(rows, pos, nh, nkv, hd):
    n = pos + rows
    q = rand((rows, nh, hd), 1)
    kc, vc = rand((n, nkv * hd), 2), rand((n, nkv * hd), 3)
    scale = 1.0 / math.sqrt(hd)
    got = O.attention(q, kc, vc, rows, pos, nh, nkv, hd, scale)
    want = brute(q, kc, vc, rows, pos, nh, nkv, hd, scale)
    np.testing.assert_allclose(got, want, atol=2e-5, rtol=1e-4)


def test_attention_matches_torch_sdpa_f64():
    torch = pytest.importorskip("torch")
    rows, pos, nh, nkv, hd = 6, 50, 32, 8, 64
    n = pos + rows
    q = rand((rows, nh, hd), 11)
    kc, vc = rand((n, nkv * hd), 12), rand((n, nkv * hd), 13)
    scale = 1.0 / math.sqrt(hd)
    got = O.attention(q, kc, vc, rows, pos, nh, nkv, hd, scale)
    grp = nh // nkv
    tq = torch.from_numpy(q).double().permute(1, 0, 2)  # [nh][rows][hd]
    tk = torch.from_numpy(kc).double().view(n, nkv, hd).permute(1, 0, 2).repeat_interleave(grp, 0)
    tv = torch.from_numpy(vc).double().view(n, nkv, hd).permute(1, 0, 2).repeat_interleave(grp, 0)
    mask = torch.from_numpy(visibility(rows, pos))
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=scale)
    np.testing.assert_allclose(got, ref.permute(1, 0, 2).numpy(), atol=2e-5, rtol=1e-4)


def test_tree_attention_matches_brute_force_and_sdpa():
    torch = pytest.importorskip("torch")
    tree = [O.ROOT, 0, 0, 1, O.ROOT]
    rows, pos, nh, nkv, hd = 5, 3, 4, 2, 16
    positions, visible, base = O.shape(rows, pos, tree)
    n = pos + rows
    q = rand((rows, nh, hd), 21)
    kc, vc = rand((n, nkv * hd), 22), rand((n, nkv * hd), 23)
    got = O.attention(q, kc, vc, rows, pos, nh, nkv, hd, 0.25, visible=visible, base=base)
    np.testing.assert_allclose(got, brute(q, kc, vc, rows, pos, nh, nkv, hd, 0.25, visible, base), atol=2e-5)
    grp = nh // nkv
    tq = torch.from_numpy(q).double().permute(1, 0, 2)
    tk = torch.from_numpy(kc).double().view(n, nkv, hd).permute(1, 0, 2).repeat_interleave(grp, 0)
    tv = torch.from_numpy(vc).double().view(n, nkv, hd).permute(1, 0, 2).repeat_interleave(grp, 0)
    mask = torch.from_numpy(visibility(rows, pos, visible, base))
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=0.25)
    np.testing.assert_allclose(got, ref.permute(1, 0, 2).numpy(), atol=2e-5)


@pytest.mark.parametrize("prefix", [190, 191, 380])
def test_grown_tree_level_sees_nodes_past_its_rows(prefix):
    """A tree fed a level at a time (model.rs:421-443, 580-594): the last level of
    [ROOT, ROOT, 0, 0, 2] is one row at position prefix + 4 whose list is the prefix and
    nodes 0, 2 and 4 (prefix + 3 entries: past prefix + rows). The oracle's row against the
    f64 brute force and against its path fed as a line."""
    nh, nkv, hd = 8, 2, 64
    parents = [O.ROOT, O.ROOT, 0, 0, 2]
    n = prefix + 5
    q = rand((1, nh, hd), 71)
    kc, vc = rand((n, nkv * hd), 72), rand((n, nkv * hd), 73)
    _, vis, base = O.shape(1, prefix + 4, parents)
    assert base == prefix and int(vis[0]) == 0b10101
    got = O.attention(q, kc, vc, 1, prefix + 4, nh, nkv, hd, 0.125, visible=vis, base=base)
    np.testing.assert_allclose(got, brute(q, kc, vc, 1, prefix + 4, nh, nkv, hd, 0.125, vis, base), atol=2e-5)
    idx = list(range(prefix)) + [prefix + j for j in (0, 2, 4)]
    line = O.attention(q, kc[idx], vc[idx], 1, prefix + 2, nh, nkv, hd, 0.125)
    np.testing.assert_array_equal(got, line)


def test_golden_fixtures():
    """Vectors written by tests/golden/make_golden.py from torch SDPA in f64."""
    files = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))
    assert files, "no golden fixtures"
    for f in files:
        z = np.load(os.path.join(GOLDEN, f))
        rows, pos, nh, nkv, hd = (int(x) for x in z["shape"])
        vis = z["visible"] if z["visible"].size else None
        base = int(z["base"])
        got = O.attention(z["q"], z["kc"], z["vc"], rows, pos, nh, nkv, hd, float(z["scale"]),
                          visible=vis, base=base)
        np.testing.assert_allclose(got, z["out"], atol=2e-5, rtol=1e-4, err_msg=f)


def test_closed_forms():
    nh, nkv, hd = 8, 2, 32
    # One visible key: the output is that key's value row, exactly.
    q = rand((1, nh, hd), 31)
    kc, vc = rand((1, nkv * hd), 32), rand((1, nkv * hd), 33)
    out = O.attention(q, kc, vc, 1, 0, nh, nkv, hd)
    for h in range(nh):
        np.testing.assert_array_equal(out[0, h], vc[0].reshape(nkv, hd)[h // 4])
    # Identical keys: the mean of the values.
    n = 37
    kc = np.tile(rand((1, nkv * hd), 34), (n, 1))
    vc = rand((n, nkv * hd), 35)
    out = O.attention(q, kc, vc, 1, n - 1, nh, nkv, hd)
    mean = vc.reshape(n, nkv, hd).astype(np.float64).mean(axis=0)
    for h in range(nh):
        np.testing.assert_allclose(out[0, h], mean[h // 4], atol=1e-5)
    # Constant values: that constant.
    vc = np.full((n, nkv * hd), 0.625, np.float32)
    kc = rand((n, nkv * hd), 36)
    out = O.attention(q, kc, vc, 1, n - 1, nh, nkv, hd)
    np.testing.assert_allclose(out, 0.625, atol=1e-6)
    # q = lambda * k_j with large lambda: the output tends to v_j.
    kc = rand((n, nkv * hd), 37)
    kc /= np.linalg.norm(kc.reshape(n, nkv, hd), axis=2).repeat(hd, axis=1).reshape(n, nkv * hd)
    vc = rand((n, nkv * hd), 38)
    j = 17
    q = np.zeros((1, nh, hd), np.float32)
    for h in range(nh):
        q[0, h] = 400.0 * kc[j].reshape(nkv, hd)[h // 4]
    out = O.attention(q, kc, vc, 1, n - 1, nh, nkv, hd, scale=1.0)
    for h in range(nh):
        np.testing.assert_allclose(out[0, h], vc[j].reshape(nkv, hd)[h // 4], atol=1e-4)


def test_gqa_equals_mha_with_replicated_heads():
    rows, pos, nh, nkv, hd = 3, 20, 12, 3, 16
    n = pos + rows
    q = rand((rows, nh, hd), 41)
    kc, vc = rand((n, nkv * hd), 42), rand((n, nkv * hd), 43)
    got = O.attention(q, kc, vc, rows, pos, nh, nkv, hd)
    rep = lambda c: np.repeat(c.reshape(n, nkv, hd), nh // nkv, axis=1).reshape(n, nh * hd)
    want = O.attention(q, rep(kc), rep(vc), rows, pos, nh, nh, hd)
    np.testing.assert_array_equal(got, want)


def test_softmax_weights_sum_to_one_and_permutation():
    # With V = all ones the output is sum(p/sum) in slot order: 1 within rounding.
    rows, pos, nh, nkv, hd = 2, 300, 4, 1, 16
    n = pos + rows
    q = rand((rows, nh, hd), 51)
    kc = rand((n, nkv * hd), 52)
    out = O.attention(q, kc, np.ones((n, hd), np.float32), rows, pos, nh, nkv, hd)
    np.testing.assert_allclose(out, 1.0, atol=2e-6)
    # Permuting the first row's visible slots (all of 0..pos) leaves it within rounding.
    vc = rand((n, nkv * hd), 53)
    perm = np.random.default_rng(54).permutation(pos + 1)
    kp, vp = kc.copy(), vc.copy()
    kp[: pos + 1], vp[: pos + 1] = kc[perm], vc[perm]
    a = O.attention(q, kc, vc, rows, pos, nh, nkv, hd)[0]
    b = O.attention(q, kp, vp, rows, pos, nh, nkv, hd)[0]
    np.testing.assert_allclose(a, b, atol=1e-5)


def test_dot_uses_eight_lanes():
    # 2^24 + 1 rounds back to 2^24 in lane 0; lane 1 holds -2^24: the lanes sum to 0, while
    # a sequential sum would give 1 (quant.rs:617-631 sums lanes, then the remainder).
    a = np.zeros(16, np.float32)
    b = np.ones(16, np.float32)
    a[0], a[8], a[1] = 2.0**24, 1.0, -(2.0**24)
    assert O.dot(a, b) == 0.0
    # The remainder is added after the lanes.
    a = np.zeros(9, np.float32)
    a[0], a[1], a[8] = 2.0**24, -(2.0**24), 1.0
    assert O.dot(a, np.ones(9, np.float32)) == 1.0
    x, y = rand(1000, 61), rand(1000, 62)
    assert abs(O.dot(x, y) - float(np.dot(x.astype(np.float64), y.astype(np.float64)))) < 1e-3


def test_rope_reference_test():
    """model.rs:676-688."""
    inv = O.inv_freq(4, 10000.0)
    x = O.rope([1.0, 0.0, 1.0, 0.0], 1, 4, 4, False, 0, inv)
    assert list(x) == [1.0, 0.0, 1.0, 0.0], "position 0 is the identity"
    x = O.rope(x, 1, 4, 4, False, 1, inv)
    assert abs(x[0] - math.cos(1.0)) < 1e-6 and abs(x[1] - math.sin(1.0)) < 1e-6
    assert abs(math.hypot(x[2], x[3]) - 1.0) < 1e-6, "rotations keep length"


@pytest.mark.parametrize("neox", [False, True])
def test_rope_rotates_the_right_pairs(neox):
    hd, rd, heads = 64, 48, 3
    inv = O.inv_freq(rd, 500000.0)
    f64 = 500000.0 ** (-2.0 * np.arange(rd // 2) / rd)
    np.testing.assert_allclose(inv, f64, rtol=2e-6)
    x = rand((heads, hd), 71)
    pos = 30011
    y = O.rope(x, heads, hd, rd, neox, pos, inv).reshape(heads, hd)
    half = rd // 2
    for h in range(heads):
        for i in range(half):
            a, b = (i, i + half) if neox else (2 * i, 2 * i + 1)
            th = np.float64(np.float32(pos) * inv[i])  # theta as the reference forms it, in f32
            c, s = math.cos(th), math.sin(th)
            assert abs(y[h, a] - (x[h, a] * c - x[h, b] * s)) < 2e-6
            assert abs(y[h, b] - (x[h, a] * s + x[h, b] * c)) < 2e-6
        np.testing.assert_array_equal(y[h, rd:], x[h, rd:])
        np.testing.assert_allclose(np.linalg.norm(y[h]), np.linalg.norm(x[h]), rtol=1e-6)


def test_shape_reference_tree():
    """The tree of model.rs:561-567 at position 3: 40 -> (41 -> 43, 42), and 44."""
    positions, visible, base = O.shape(5, 3, [O.ROOT, 0, 0, 1, O.ROOT])
    assert base == 3
    assert list(positions) == [3, 4, 4, 5, 3]
    assert [int(v) for v in visible] == [0b1, 0b11, 0b101, 0b1011, 0b10000]
    # Grown a level at a time (model.rs:582-591): the last call's rows only.
    parents = [O.ROOT, O.ROOT, 0, 0, 2]
    p, v, b = O.shape(2, 3 + 2, parents[:4])
    assert b == 3 and list(p) == [4, 4] and [int(x) for x in v] == [0b101, 0b1001]
    p, v, b = O.shape(1, 3 + 4, parents)
    assert b == 3 and list(p) == [5] and [int(x) for x in v] == [0b10101]
    # Parents must come first (model.rs:604), trees are at most 64 nodes, and earlier
    # nodes must fit before pos.
    for args in [(2, 0, [1, O.ROOT]), (1, 100, [O.ROOT] * 65), (1, 0, [O.ROOT, 0])]:
        with pytest.raises(O.ShapeError):
            O.shape(*args)
    p, v, b = O.shape(3, 7, None)
    assert list(p) == [7, 8, 9] and v is None and b == 7


def test_keep_reference_cases():
    """model.rs:146-166 and the checks of model.rs:595-610."""
    width = 6
    cache = np.arange(8 * width, dtype=np.float32)
    n = O.keep(cache, width, 8, 3, [0, 1, 3])
    assert n == 6
    rows = cache.reshape(8, width)
    np.testing.assert_array_equal(rows[:5], np.arange(5 * width).reshape(5, width))
    np.testing.assert_array_equal(rows[5], np.arange(6 * width, 7 * width))
    small = np.zeros(3 * width, np.float32)
    for bad in ([2, 1], [0, 5]):
        with pytest.raises(ValueError):
            O.keep(small, width, 3, 0, bad)


def test_f16_rounding_matches_numpy():
    rng = np.random.default_rng(81)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),  # subnormal range
        np.array([65504, 65519, 65520, 1e6, -1e6, np.inf, -np.inf, 2.0**-24, 2.0**-25, 3 * 2.0**-26, 0.0,
                  -0.0], np.float32),
        # exact ties between two f16 values
        (np.arange(1, 2000, dtype=np.float32) * 2.0**-10 + 2.0**-11).astype(np.float32),
    ])
    want = x.astype(np.float16).astype(np.float32)
    got = O.f16_round(x)
    np.testing.assert_array_equal(got, want)
    assert math.isnan(O.f16_round(np.array([np.nan], np.float32))[0])
    for h in [0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xFC00, 0x8001]:
        assert O.f16_bits_to_f32(h) == float(np.array([h], np.uint16).view(np.float16)[0])


def test_splitmix64_published_sequence_and_normal_draws():
    # The sequence from seed 1234567 published with splitmix64 (Vigna's reference test).
    assert O.splitmix64(1234567, 5) == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                                        4593380528125082431, 16408922859458223821]
    stats = pytest.importorskip("scipy.stats")
    z = O.normal(2024, 200000)
    assert abs(float(z.mean())) < 0.01 and abs(float(z.std()) - 1.0) < 0.01
    assert stats.kstest(z[:20000], "norm").pvalue > 1e-3
    np.testing.assert_array_equal(O.normal(5, 1001)[:1000], O.normal(5, 1000))


def test_mutants_are_caught():
    """Plausible mistakes, planted in numpy copies of the oracle's algorithm, each differ
    from the brute force by far more than the tolerances above: the checks bite."""
    rows, pos, nh, nkv, hd = 3, 30, 8, 2, 16
    n = pos + rows
    q = rand((rows, nh, hd), 91)
    kc, vc = rand((n, nkv * hd), 92), rand((n, nkv * hd), 93)
    want = brute(q, kc, vc, rows, pos, nh, nkv, hd, 0.25)

    def variant(head_map=lambda h: h // (nh // nkv), scale=0.25, extra=0):
        out = np.zeros((rows, nh, hd))
        k = kc.reshape(n, nkv, hd).astype(np.float64)
        v = vc.reshape(n, nkv, hd).astype(np.float64)
        for i in range(rows):
            upto = pos + i + 1 + extra
            for h in range(nh):
                s = k[:upto, head_map(h)] @ q[i, h] * scale
                p = np.exp(s - s.max())
                out[i, h] = (p / p.sum()) @ v[:upto, head_map(h)]
        return out

    assert np.abs(variant() - want).max() < 1e-9
    assert np.abs(variant(head_map=lambda h: h % nkv) - want).max() > 1e-2
    assert np.abs(variant(scale=1.0) - want).max() > 1e-2
    assert np.abs(variant(extra=1)[:2] - want[:2]).max() > 1e-3
