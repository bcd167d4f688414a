"""bchip_sample (the device sampler) against the CPU restatement of sample.rs
(oracle/bc_sample.c): token ids are index results, so they must be equal, row for row, at
Qwen2.5's and Llama-3's vocabulary sizes, greedy and nucleus, with the reference's own test
(sample.rs:78-89) on the device."""
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


def device_ids(ctx, scores, temperature, top_p, seed, step0):
    rows, vocab = scores.shape
    sb, ib = ctx.upload(np.ascontiguousarray(scores, np.float32)), ctx.zeros(rows * 4)
    ctx.sample(sb, rows, vocab, temperature, top_p, seed, step0, ib)
    ids = ctx.read(ib, (rows,), np.uint32)
    sb.free()
    ib.free()
    return ids


def check(ctx, scores, temperature, top_p, seed, step0, what):
    got = device_ids(ctx, scores, temperature, top_p, seed, step0)
    want = [O.sample(scores[r], temperature, top_p, seed, step0 + r) for r in range(scores.shape[0])]
    print(f"{what}: {list(got[:8])}", flush=True)
    np.testing.assert_array_equal(got, np.array(want, np.uint32), err_msg=what)


def test_reference_greedy_and_nucleus_on_the_device(ctx):
    scores = np.array([[0.1, 3.0, 2.9, -5.0]], np.float32)
    assert device_ids(ctx, scores, 0.0, 1.0, 0, 0)[0] == 1
    tight = np.repeat(scores, 20, axis=0)
    assert (device_ids(ctx, tight, 1.0, 0.01, 7, 0) == 1).all()
    wide = np.repeat(scores, 200, axis=0)
    picks = device_ids(ctx, wide, 1.0, 0.95, 7, 0)
    assert 1 in picks and 2 in picks and 3 not in picks
    np.testing.assert_array_equal(picks, [O.sample(scores[0], 1.0, 0.95, 7, i) for i in range(200)])


@pytest.mark.parametrize("vocab", [151936, 128256, 37, 1])
def test_greedy_is_the_restatements_argmax(ctx, vocab):
    rng = np.random.default_rng(vocab)
    s = rng.standard_normal((6, vocab)).astype(np.float32) * 3
    if vocab > 10:
        s[1, [7, vocab // 2, vocab - 1]] = s[1].max() + 1.0  # a three-way tie for the top
        s[2, 0] = np.nan                                 # a NaN first: index 0
        s[3, 5] = np.nan                                 # a NaN elsewhere is passed over
        s[4, :] = -np.inf
    check(ctx, s, 0.0, 1.0, 0, 0, f"greedy, vocab {vocab}")


@pytest.mark.parametrize("temperature,top_p", [(1.0, 0.95), (0.7, 0.9), (1.5, 1.0), (0.3, 0.5), (1.0, 0.01)])
def test_nucleus_is_the_restatements(ctx, temperature, top_p):
    rng = np.random.default_rng(int(temperature * 100 + top_p * 10))
    for vocab in (151936, 1000):
        s = (rng.standard_normal((4, vocab)) * 2.5).astype(np.float32)
        check(ctx, s, temperature, top_p, 12345, 100, f"T {temperature} top_p {top_p} vocab {vocab}")


def test_flat_scores_keep_the_whole_vocabulary(ctx):
    """Equal scores: every p is 1, the nucleus runs over many staging chunks, ties go by index."""
    s = np.zeros((3, 20000), np.float32)
    check(ctx, s, 1.0, 1.0, 9, 0, "flat")
    check(ctx, s, 1.0, 0.5, 9, 7, "flat, half")
