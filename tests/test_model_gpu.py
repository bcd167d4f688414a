"""The reference's end-to-end model tests (crates/bc-infer/src/model.rs:509-675) on the GPU
layers: the small random model of fixtures.rs (tests/tiny_model.py) run through
layers.GpuLayers, every layer op a call into this library, checked against an exact f64
forward of the same weights and against itself: a model split in stages computes what the
whole does, a tree pass scores every path as if fed alone (also grown a level at a time),
Cache::keep keeps the accepted path, and a long conversation grows the cache.

The bounds are the reference's own: prompt-then-step against the whole sequence < 1e-4
(model.rs:531), a batch row against a one-token pass < 1e-4 (model.rs:641-642), the next
step after keep within 1e-4 x (1 + the largest score) of the text fed whole (model.rs:548,
601), and the GPU against the CPU within 0.02 x (1 + the largest score) (model.rs:626-632;
held here at 5e-3 against an exact forward). The stage's cache is f32 (the reference's), and
every pass over an f32 cache takes one f32 arithmetic whatever its rows (attention_f32.hip),
so the first three hold with room to spare."""
import numpy as np
import pytest

import bchip
from layers import GpuLayers
from tiny_model import RefModel, embed, tiny_model

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = bchip.Ctx(0)
    yield c
    c.close()


class Part:
    """Part (model.rs:176-370) over GPU layers: layers [lo, hi) and the head on the last."""

    def __init__(self, ctx, model, lo, hi, last):
        cfg, layers, head, self.embd = model
        self.cfg = cfg
        self.g = GpuLayers(ctx, cfg, layers[lo:hi], head if last else None)

    def forward(self, x, pos, tree, cache):
        positions, visible, base = O.shape(len(x), pos, tree)
        masks = None if visible is None else (base, visible)
        return self.g.forward(x, pos, positions, masks, cache)


def run(parts, caches, tokens, pos):
    """model.rs:495-507: embed, every stage's layers, the last stage's scores (rows x vocab)."""
    x = embed(parts[0].embd, tokens)
    for p, c in zip(parts, caches):
        x = p.forward(x, pos, None, c)
    return parts[-1].g.logits(x, len(tokens))


def close(got, want, bar, what):
    """Within bar x (1 + the largest score), the reference's relative bound (model.rs:545-548, 626-632)."""
    err = np.abs(got.astype(np.float64) - want).max()
    top = np.abs(want).max()
    print(f"{what}: max error {err:.3g} against scores up to {top:.3g}")
    assert err <= bar * (1.0 + top), f"{what}: max error {err} against scores up to {top}"


def within(got, want, bound, what):
    """Every score within `bound` absolute (model.rs:531, 641-642)."""
    err = float(np.abs(got.astype(np.float64) - np.asarray(want, np.float64)).max())
    print(f"{what}: max error {err:.3g}")
    assert err < bound, f"{what}: max error {err}"


@pytest.mark.parametrize("neox", [False, True])
def test_the_gpu_layers_compute_what_an_exact_forward_does(ctx, neox):
    """model.rs:613-650 (the_gpu_computes_what_the_cpu_does), against an exact forward."""
    model = tiny_model(4, neox)
    cfg, layers, head, embd = model
    part = Part(ctx, model, 0, 4, True)
    ref = RefModel(cfg, layers, head)
    cache, rc = part.g.new_cache(), ref.new_cache()
    prompt = [5, 9, 13, 2, 7, 1]
    got = run([part], [cache], prompt, 0)
    want = ref.logits(ref.forward(embed(embd, prompt), 0, None, rc))
    close(got, want, 5e-3, "prompt")
    got = run([part], [cache], [40], 6)
    want = ref.logits(ref.forward(embed(embd, [40]), 6, None, rc))
    close(got, want, 5e-3, "one-token step")
    # A batch row against a one-token pass (model.rs:641-642).
    fresh = part.g.new_cache()
    whole = run([part], [fresh], prompt + [40], 0)
    within(got[0], whole[6], 1e-4, "one-token pass against the batch row")
    # Going back cuts the cache: rerunning position 6 gives the same bits.
    np.testing.assert_array_equal(run([part], [cache], [40], 6), got)
    for c in (cache, fresh):
        c.free()
    part.g.free()


@pytest.mark.parametrize("neox", [False, True])
def test_a_split_model_computes_what_the_whole_one_does(ctx, neox):
    """model.rs:509-536: stages [0, 1), [1, 3), [3, 4) against the whole 4 layers, bit for
    bit, a prompt then a step; prompt-then-step against the whole sequence at once."""
    model = tiny_model(4, neox)
    whole = Part(ctx, model, 0, 4, True)
    parts = [Part(ctx, model, 0, 1, False), Part(ctx, model, 1, 3, False), Part(ctx, model, 3, 4, True)]
    kv1 = [whole.g.new_cache()]
    kv3 = [p.g.new_cache() for p in parts]
    one = run([whole], kv1, [5, 9, 13, 2], 0)
    np.testing.assert_array_equal(run(parts, kv3, [5, 9, 13, 2], 0), one)
    one = run([whole], kv1, [40], 4)
    np.testing.assert_array_equal(run(parts, kv3, [40], 4), one)
    fresh = [whole.g.new_cache()]
    all5 = run([whole], fresh, [5, 9, 13, 2, 40], 0)
    within(all5[4], one[0], 1e-4, "the whole sequence's last row against prompt then step")
    np.testing.assert_array_equal(run([whole], kv1, [40], 4), one)
    for c in kv1 + kv3 + fresh:
        c.free()
    for p in parts + [whole]:
        p.g.free()


@pytest.mark.parametrize("neox", [False, True])
def test_a_tree_pass_scores_every_path_as_if_fed_alone(ctx, neox):
    """model.rs:538-611 on the GPU: tree rows equal their lines bit for bit; the same tree
    grown a level at a time scores every node the same, bit for bit where the level is a
    batch and within 1e-4 x (1 + the largest score) for the lone-row level (whose products
    run on the VALU, the reference's `!on_gpu || node < 4`, model.rs:593); after Cache::keep
    of the accepted path the next step matches the text fed whole within 1e-4 x (1 + the
    largest score) (model.rs:595-601)."""
    model = tiny_model(3, neox)
    part = Part(ctx, model, 0, 3, True)
    prefix = [5, 9, 13]
    tokens = [40, 41, 42, 43, 44]
    tree = [O.ROOT, 0, 0, 1, O.ROOT]
    kv = part.g.new_cache()
    run([part], [kv], prefix, 0)
    x = part.forward(embed(part.embd, tokens), len(prefix), tree, kv)
    scores = part.g.logits(x, len(tokens))
    paths = [[40], [40, 41], [40, 42], [40, 41, 43], [44]]
    for row, path in enumerate(paths):
        alone = part.g.new_cache()
        line = prefix + path
        want = run([part], [alone], line, 0)
        alone.free()
        np.testing.assert_array_equal(scores[row], want[len(line) - 1], err_msg=f"row {row}, path {path}")
    grown = part.g.new_cache()
    run([part], [grown], prefix, 0)
    order = [40, 44, 41, 42, 43]
    parents = [O.ROOT, O.ROOT, 0, 0, 2]
    seen = []
    for lo, hi in [(0, 2), (2, 4), (4, 5)]:
        x = part.forward(embed(part.embd, order[lo:hi]), len(prefix) + lo, parents[:hi], grown)
        seen.extend(part.g.logits(x, hi - lo))
    for node, row in [(0, 0), (1, 4), (2, 1), (3, 2), (4, 3)]:
        if node < 4:
            np.testing.assert_array_equal(seen[node], scores[row], err_msg=f"node {node}")
        else:
            close(seen[node], scores[row].astype(np.float64), 1e-4, f"node {node} (a lone-row level)")
    # Accept 40 -> 41 -> 43 (rows 0, 1, 3).
    kv.keep(len(prefix), [0, 1, 3])
    nxt = run([part], [kv], [50], 6)
    fresh = part.g.new_cache()
    want = run([part], [fresh], [5, 9, 13, 40, 41, 43, 50], 0)
    close(nxt[0], want[6].astype(np.float64), 1e-4, "after keep")
    for c in (kv, grown, fresh):
        c.free()
    part.g.free()


def test_the_last_stage_samples_on_the_device(ctx):
    """engine.rs:341-350: the last stage samples every row (sample.rs). On the device, the ids
    equal the restatement's picks from the same stage's scores, greedy and nucleus."""
    model = tiny_model(2, False)
    part = Part(ctx, model, 0, 2, True)
    kv = part.g.new_cache()
    x = part.forward(embed(part.embd, [5, 9, 13, 2, 7]), 0, None, kv)
    scores = part.g.logits(x, 5)
    for temperature, top_p, seed in ((0.0, 1.0, 0), (0.8, 0.9, 42), (1.3, 1.0, 7)):
        ids = part.g.sample(x, 5, temperature, top_p, seed, 10)
        want = [O.sample(scores[r], temperature, top_p, seed, 10 + r) for r in range(5)]
        np.testing.assert_array_equal(ids, want, err_msg=f"T {temperature} top_p {top_p}")
    kv.free()
    part.g.free()


def test_a_long_conversation_grows_the_gpu_cache(ctx):
    """model.rs:652-675: 1100 tokens in passes of 300 (past the first 256-slot allocation
    and past one 1024-slot tile of the reference's kernel), against the exact forward."""
    model = tiny_model(2, True)
    cfg, layers, head, embd = model
    part = Part(ctx, model, 0, 2, True)
    ref = RefModel(cfg, layers, head)
    prompt = [(i * 7 % 90) + 1 for i in range(1100)]
    kg, kc = part.g.new_cache(), ref.new_cache()
    for i in range(0, 1100, 300):
        chunk = prompt[i:i + 300]
        g = run([part], [kg], chunk, i)
        x = ref.forward(embed(embd, chunk), i, None, kc)
    want = ref.logits(x[-1:])
    close(g[-1:], want, 5e-3, "last row after 1100 tokens")
    assert kg.bytes() >= 1100 * 2 * 2 * 32 * 4
    kg.free()
    part.g.free()
