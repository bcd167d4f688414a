"""The reference's end-to-end invariants (crates/bc-infer/src/model.rs:509-650) on the kernels
the benchmark times: a random model at head_dim 128 and width 512 (tests/tiny_model.py
wide_model: 4 query and 2 KV heads, Q8_0 attention matrices, Q4K gate and up, Q6K down) run
through layers.GpuLayers with an f16 KV cache, so that

- one-token steps take the fused decode kernel (attn_decode_row, f16 MFMA tiles),
- lines of several rows take the chunked MFMA kernels (attn_prefill, split by chunk and
  folded in one launch when they are few workgroups),
- tree rows take the tree-row kernel (attn_decode),
- products of several rows take the matrix-core block-format product (k_matmul_mm) and
  one-row products the VALU one.

Checked, as in the reference:
- the scores against an exact f64 forward of the same weights within 5e-3 x (1 + the largest
  score) (model.rs:626-632 allows 0.02);
- a model split in stages computes what the whole does, bit for bit (model.rs:509-536);
- tree rows equal their lines bit for bit (model.rs:578);
- a batch row against the same token as a one-token pass (model.rs:641-642): within the
  reference's 1e-4 on an f32 cache; on an f16 cache within one f16 step of the largest score,
  2^-11 x (1 + top). The f16 cache rounds every q, K and V element to 11 bits, so a
  difference in the last f32 bit upstream (the one-row product on the VALU against the
  batch's on the matrix cores) can move an element by one f16 step; measured 2.5e-4 to
  3.2e-4 against scores up to 4.9, where the f32 cache stays under 1e-5;
- after Cache::keep of an accepted path, the next step against the text fed whole within
  1e-4 x (1 + the largest score) (model.rs:548, 601).
The same model with an f32 cache (the reference's cache type) is checked against the exact
forward too.
"""
import numpy as np
import pytest

import bchip
from layers import GpuLayers
from tiny_model import RefModel, embed, wide_model

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = bchip.Ctx(0)
    yield c
    c.close()


class Part:
    """Part (model.rs:176-370) over GPU layers: layers [lo, hi) and the head on the last."""

    def __init__(self, ctx, model, lo, hi, last, kv_type):
        cfg, layers, head, self.embd = model
        self.cfg = cfg
        self.g = GpuLayers(ctx, cfg, layers[lo:hi], head if last else None, kv_type=kv_type)

    def forward(self, x, pos, tree, cache):
        positions, visible, base = O.shape(len(x), pos, tree)
        masks = None if visible is None else (base, visible)
        return self.g.forward(x, pos, positions, masks, cache)


def run(parts, caches, tokens, pos):
    x = embed(parts[0].embd, tokens)
    for p, c in zip(parts, caches):
        x = p.forward(x, pos, None, c)
    return parts[-1].g.logits(x, len(tokens))


def close(got, want, bar, what):
    err = np.abs(got.astype(np.float64) - want).max()
    top = np.abs(want).max()
    print(f"{what}: max error {err:.3g} against scores up to {top:.3g}", flush=True)
    assert err <= bar * (1.0 + top), f"{what}: max error {err} against scores up to {top}"


def within(got, want, bound, what):
    err = float(np.abs(got.astype(np.float64) - np.asarray(want, np.float64)).max())
    print(f"{what}: max error {err:.3g}", flush=True)
    assert err < bound, f"{what}: max error {err}"


PROMPT = [(i * 37 + 11) % 250 + 3 for i in range(40)]


@pytest.fixture(scope="module", params=[False, True], ids=["llama", "qwen2"])
def model(request):
    return wide_model(3, request.param)


@pytest.mark.parametrize("kv_type", [bchip.F16, bchip.F32], ids=["f16", "f32"])
def test_wide_stage_computes_what_an_exact_forward_does(ctx, model, kv_type):
    cfg, layers, head, embd = model
    assert cfg.head_dim == 128 and cfg.n_embd == 512
    part = Part(ctx, model, 0, 3, True, kv_type)
    ref = RefModel(cfg, layers, head)
    cache, rc = part.g.new_cache(), ref.new_cache()
    got = run([part], [cache], PROMPT, 0)
    want = ref.logits(ref.forward(embed(embd, PROMPT), 0, None, rc))
    close(got, want, 5e-3, "prompt of 40")
    for i, tok in enumerate([17, 99, 201]):
        got = run([part], [cache], [tok], len(PROMPT) + i)
        want = ref.logits(ref.forward(embed(embd, [tok]), len(PROMPT) + i, None, rc))
        close(got, want, 5e-3, f"one-token step {i}")
    cache.free()
    part.g.free()


F16_STEP = 2.0 ** -11


@pytest.mark.parametrize("kv_type", [bchip.F16, bchip.F32], ids=["f16", "f32"])
def test_wide_stage_split_equals_whole_and_batch_row_equals_step(ctx, model, kv_type):
    """model.rs:509-536 and 641-642: stages [0, 1) and [1, 3) against the whole 3 layers bit
    for bit (a prompt, then one-token steps); the whole sequence's rows against
    prompt-then-steps within 1e-4 (f32 cache) or one f16 step of the largest score (f16)."""
    whole = Part(ctx, model, 0, 3, True, kv_type)
    parts = [Part(ctx, model, 0, 1, False, kv_type), Part(ctx, model, 1, 3, True, kv_type)]
    kv1 = [whole.g.new_cache()]
    kv2 = [p.g.new_cache() for p in parts]
    one = run([whole], kv1, PROMPT, 0)
    np.testing.assert_array_equal(run(parts, kv2, PROMPT, 0), one)
    steps = []
    for i, tok in enumerate([17, 99, 201]):
        s = run([whole], kv1, [tok], len(PROMPT) + i)
        np.testing.assert_array_equal(run(parts, kv2, [tok], len(PROMPT) + i), s)
        steps.append(s[0])
    fresh = [whole.g.new_cache()]
    every = run([whole], fresh, PROMPT + [17, 99, 201], 0)
    for i in range(3):
        what = f"batch row {len(PROMPT) + i} against its one-token step"
        if kv_type == bchip.F32:
            within(every[len(PROMPT) + i], steps[i], 1e-4, what)
        else:
            close(every[len(PROMPT) + i], steps[i].astype(np.float64), F16_STEP, what)
    for c in kv1 + kv2 + fresh:
        c.free()
    for p in parts + [whole]:
        p.g.free()


def test_wide_stage_f16_tree_rows_equal_their_lines_and_keep(ctx, model):
    """model.rs:538-611 on the f16 kernels: every tree row equals its line bit for bit; after
    Cache::keep of the accepted path the next step matches the text fed whole within
    1e-4 x (1 + the largest score)."""
    part = Part(ctx, model, 0, 3, True, bchip.F16)
    prefix = PROMPT[:20]
    tokens = [40, 41, 42, 43, 44, 45]
    tree = [O.ROOT, 0, 0, 1, 3, O.ROOT]
    kv = part.g.new_cache()
    run([part], [kv], prefix, 0)
    x = part.forward(embed(part.embd, tokens), len(prefix), tree, kv)
    scores = part.g.logits(x, len(tokens))
    paths = [[40], [40, 41], [40, 42], [40, 41, 43], [40, 41, 43, 44], [45]]
    for row, path in enumerate(paths):
        alone = part.g.new_cache()
        line = prefix + path
        want = run([part], [alone], line, 0)
        alone.free()
        np.testing.assert_array_equal(scores[row], want[len(line) - 1], err_msg=f"row {row}, path {path}")
    kv.keep(len(prefix), [0, 1, 3, 4])  # accept 40 -> 41 -> 43 -> 44
    nxt = run([part], [kv], [50], len(prefix) + 4)
    fresh = part.g.new_cache()
    want = run([part], [fresh], prefix + [40, 41, 43, 44, 50], 0)
    close(nxt[0], want[-1].astype(np.float64), 1e-4, "after keep")
    for c in (kv, fresh):
        c.free()
    part.g.free()


def test_wide_stage_f16_verify_rows_after_a_long_prefix(ctx, model):
    """A verify step's draft rows (llm.rs:655-667) after a prefix longer than one 192-slot
    chunk, so that each layer's rows run as one call of RoPE, append and split attention in
    one launch: fed as a line and as a chain tree (each row sees the prefix and the rows
    before it), the same bits row for row (model.rs:578); the line's last row against the
    text fed whole within one f16 step of the largest score."""
    part = Part(ctx, model, 0, 3, True, bchip.F16)
    prefix = [(i * 53 + 7) % 250 + 3 for i in range(230)]
    drafts = [40, 41, 42, 43, 44, 45, 46, 47]
    kv_line, kv_tree = part.g.new_cache(), part.g.new_cache()
    run([part], [kv_line], prefix, 0)
    run([part], [kv_tree], prefix, 0)
    line = run([part], [kv_line], drafts, len(prefix))
    chain = [O.ROOT] + list(range(len(drafts) - 1))
    x = part.forward(embed(part.embd, drafts), len(prefix), chain, kv_tree)
    tree = part.g.logits(x, len(drafts))
    for row in range(len(drafts)):
        np.testing.assert_array_equal(line[row], tree[row], err_msg=f"draft row {row}")
    fresh = part.g.new_cache()
    whole = run([part], [fresh], prefix + drafts, 0)
    close(line[-1], whole[-1].astype(np.float64), F16_STEP, "verify rows against the text fed whole")
    for c in (kv_line, kv_tree, fresh):
        c.free()
    part.g.free()
