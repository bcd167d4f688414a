"""BASELINE.json's configurations, each run at its full size through the C ABI and checked
against the CPU oracle (bc-infer's attention, crates/bc-infer/src/model.rs:448-481).

The oracle is a single-thread restatement, so the big passes are checked on sampled rows
(the first, middle and last rows of a prefill; the first, middle and last steps of the verify
loop; every sequence of the ragged batch in full) and, in full, through properties the
reference's tests demand: the last rows of a prefill recomputed as a speculative verify agree
within LINE_TOL (the reference's bound for a batch row against a one-token pass, model.rs:642;
the wide prefill takes one online softmax over a row's whole list, the verify pass folds
192-entry chunks, so the two round differently), and one sequence of a ragged batch gives the
bits of the sequence alone.

Gate (north star): max abs error <= 5e-3 and cosine >= 0.9999 against the f32 oracle, both
on the f16-rounded cache (the kernel's error) and on the unrounded f32 values (total)."""
import math

import numpy as np
import pytest

import bchip
import oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 5e-3
MIN_COS = 0.9999
LINE_TOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = bchip.Ctx(0)
    yield c
    c.close()


def say(msg):
    print(msg, flush=True)


def gate(got, want, what):
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    err = float(np.abs(got - want).max())
    cos = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want)))
    say(f"{what}: max abs {err:.3g}, cosine {cos:.8f}")
    assert err <= MAX_ABS and cos >= MIN_COS, f"{what}: max abs {err:.3g}, cosine {cos:.8f}"


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


def sampled_rows(rows, n=16):
    return [(0, n), (rows // 2 - n // 2, rows // 2 + n // 2), (rows - n, rows)]


def check_rows(got, q, kc, vc, r0, r1, nh, nkv, hd, scale, what):
    """Rows r0..r1 of a causal pass from position 0 (row r sees slots 0..r)."""
    kr, vr = O.f16_round(kc[:r1]), O.f16_round(vc[:r1])
    gate(got[r0:r1], O.attention(q[r0:r1], kr, vr, r1 - r0, r0, nh, nkv, hd, scale), what + " (kernel error)")
    gate(got[r0:r1], O.attention(q[r0:r1], kc[:r1], vc[:r1], r1 - r0, r0, nh, nkv, hd, scale), what + " (total error)")


def causal_prefill(ctx, S, nh, nkv, hd, seed):
    """One layer's causal prefill of S tokens from position 0 (f16 cache), checked on sampled
    rows against the oracle and its last 8 rows against an 8-row verify pass (within
    LINE_TOL)."""
    say(f"prefill S={S} heads {nh}/{nkv} hd {hd}")
    q = rand((S, nh, hd), seed)
    kc, vc = rand((S, nkv * hd), seed + 1), rand((S, nkv * hd), seed + 2)
    scale = 1.0 / math.sqrt(hd)
    kb, vb = ctx.upload(kc.astype(np.float16)), ctx.upload(vc.astype(np.float16))
    qb, ob = ctx.upload(q), ctx.zeros(q.nbytes)
    ctx.attention(qb, kb, vb, bchip.F16, ob, None, False, S, nh, nkv, hd, 0, scale)
    got = ctx.read(ob, q.shape)
    assert np.isfinite(got).all()
    for r0, r1 in sampled_rows(S):
        check_rows(got, q, kc, vc, r0, r1, nh, nkv, hd, scale, f"S={S} rows {r0}..{r1}")
    # The last rows again as a speculative verify (8 rows at S-8: split over CUs by chunk).
    q8, o8 = ctx.upload(q[S - 8:]), ctx.zeros(8 * nh * hd * 4)
    ctx.attention(q8, kb, vb, bchip.F16, o8, None, False, 8, nh, nkv, hd, S - 8, scale)
    d = float(np.abs(ctx.read(o8, (8, nh, hd)) - got[S - 8:]).max())
    say(f"S={S}: verify of the last rows against the prefill: max abs {d:.3g}")
    assert d < LINE_TOL, f"S={S}: verify of the last rows differs by {d}"
    for b in (kb, vb, qb, ob, q8, o8):
        b.free()


@pytest.mark.parametrize("S", [2048, 8192])
def test_llama8b_causal_prefill(ctx, S):
    """Llama-3-8B prefill of S prompt tokens (32/8 heads, hd 128, f16)."""
    causal_prefill(ctx, S, 32, 8, 128, S)


def test_llama70b_share_prefill_4096(ctx):
    """configs[4]'s prefill: 4096 tokens at 64/8 heads (a group of 8 per KV head)."""
    causal_prefill(ctx, 4096, 64, 8, 128, 70)


def test_qwen7b_shape_prefill_group_of_7(ctx):
    """A prefill large enough for the packed-V^T kernel with a group of 7 (Qwen2.5-7B,
    28/4): its workgroups hold rows of several heads."""
    causal_prefill(ctx, 300, 28, 4, 128, 7)


def test_llama70b_share_verify_loop_256_steps(ctx):
    """configs[4]'s decode: after a 4096-token context, 256 speculative-verify steps of 8 rows
    (all accepted), each step RoPE + K/V append of its 8 rows (bchip_rope_append, theta 5e5,
    adjacent pairs) then attention of the 8 rows over ctx + 8 slots; ctx 4096 -> 6136. Steps
    0, 128 and 255 against the oracle's rope and attention."""
    nh, nkv, hd, ctx0, steps, R = 64, 8, 128, 4096, 256, 8
    kvd = nkv * hd
    cap = ctx0 + steps * R
    theta = 5e5
    scale = 1.0 / math.sqrt(hd)
    inv = O.inv_freq(hd, theta)
    k0, v0 = rand((ctx0, kvd), 401), rand((ctx0, kvd), 402)
    kb, vb = ctx.zeros(cap * kvd * 2), ctx.zeros(cap * kvd * 2)
    ctx.upload(k0.astype(np.float16), kb)
    ctx.upload(v0.astype(np.float16), vb)
    ib = ctx.upload(inv)
    qb, knb, vnb = ctx.zeros(R * nh * hd * 4), ctx.zeros(R * kvd * 4), ctx.zeros(R * kvd * 4)
    pb, ob = ctx.zeros(R * 4), ctx.zeros(R * nh * hd * 4)
    # The f32 history the total error is measured on: rotated K rows as the oracle rotates them.
    k32, v32 = np.zeros((cap, kvd), np.float32), np.zeros((cap, kvd), np.float32)
    k32[:ctx0], v32[:ctx0] = k0, v0
    check = {0, 128, steps - 1}
    for step in range(steps):
        pos = ctx0 + step * R
        q = rand((R, nh * hd), 1000 + step)
        kn, vn = rand((R, kvd), 2000 + step), rand((R, kvd), 3000 + step)
        positions = np.arange(pos, pos + R, dtype=np.uint32)
        ctx.upload(q, qb)
        ctx.upload(kn, knb)
        ctx.upload(vn, vnb)
        ctx.upload(positions, pb)
        ctx.rope_append(qb, knb, vnb, kb, vb, bchip.F16, ib, pb, R, nh, nkv, hd, hd, False, pos)
        ctx.attention(qb, kb, vb, bchip.F16, ob, None, False, R, nh, nkv, hd, pos, scale)
        k32[pos:pos + R] = O.rope_rows(kn, positions, nkv, hd, hd, False, inv)
        v32[pos:pos + R] = vn
        if step not in check:
            continue
        say(f"verify step {step}: 8 rows at {pos}")
        got = ctx.read(ob, (R, nh, hd))
        q_dev = ctx.read(qb, (R, nh * hd))
        q_ref = O.rope_rows(q, positions, nh, hd, hd, False, inv)
        assert np.abs(q_dev - q_ref).max() <= 1e-4 * (1 + np.abs(q_ref).max()), "rotated q"
        kc_dev = ctx.read(kb, (pos + R, kvd), np.float16).astype(np.float32)
        vc_dev = ctx.read(vb, (pos + R, kvd), np.float16).astype(np.float32)
        np.testing.assert_array_equal(vc_dev[pos:], O.f16_round(vn), err_msg="appended V rows")
        # The device's sin/cos and the host's may differ in the last bit, so a rotated K value
        # may round to the neighbouring f16 value: within one f16 spacing.
        kref = O.f16_round(k32[pos:pos + R])
        assert np.all(np.abs(kc_dev[pos:] - kref) <= np.abs(kref) * 2.0 ** -10 + 1e-7), "appended K rows"
        gate(got, O.attention(q_dev.reshape(R, nh, hd), kc_dev, vc_dev, R, pos, nh, nkv, hd, scale),
             f"verify step {step} (kernel error)")
        gate(got, O.attention(q_ref.reshape(R, nh, hd), k32[:pos + R], v32[:pos + R], R, pos, nh, nkv, hd, scale),
             f"verify step {step} (total error)")
    for b in (kb, vb, ib, qb, knb, vnb, pb, ob):
        b.free()


def test_qwen7b_ragged_16_sequences(ctx):
    """16 concurrent sequences, lengths drawn as the benchmark draws them
    (U[1024, 32768], seed 4), 28/4 heads, hd 128, one f16 pool; each sequence against the
    oracle in full and against its own one-row pass bit for bit."""
    nh, nkv, hd = 28, 4, 128
    kvd = nkv * hd
    scale = 1.0 / math.sqrt(hd)
    lens = np.random.default_rng(4).integers(1024, 32769, size=16).astype(np.uint32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    total = int(lens.sum())
    kb, vb = ctx.zeros(total * kvd * 2), ctx.zeros(total * kvd * 2)
    for i, (L, off) in enumerate(zip(lens, offs)):
        ctx.upload(rand((int(L), kvd), 500 + i).astype(np.float16), kb, int(off) * kvd * 2)
        ctx.upload(rand((int(L), kvd), 600 + i).astype(np.float16), vb, int(off) * kvd * 2)
    q = rand((16, nh, hd), 700)
    qb, ob = ctx.upload(q), ctx.zeros(q.nbytes)
    ctx.attention_ragged(qb, kb, vb, bchip.F16, ob, lens, offs, nh, nkv, hd, scale)
    got = ctx.read(ob, q.shape)
    for i, (L, off) in enumerate(zip(lens, offs)):
        L, off = int(L), int(off)
        say(f"ragged sequence {i}: {L} slots at {off}")
        kc, vc = rand((L, kvd), 500 + i), rand((L, kvd), 600 + i)
        gate(got[i:i + 1], O.attention(q[i:i + 1], O.f16_round(kc), O.f16_round(vc), 1, L - 1, nh, nkv, hd, scale),
             f"sequence {i} (kernel error)")
        gate(got[i:i + 1], O.attention(q[i:i + 1], kc, vc, 1, L - 1, nh, nkv, hd, scale), f"sequence {i} (total error)")
        q1, o1 = ctx.upload(q[i:i + 1]), ctx.zeros(nh * hd * 4)
        ctx.attention(q1, kb.offset(off * kvd * 2), vb.offset(off * kvd * 2), bchip.F16, o1, None, False, 1, nh, nkv,
                      hd, L - 1, scale)
        np.testing.assert_array_equal(ctx.read(o1, (1, nh, hd))[0], got[i], err_msg=f"sequence {i} alone")
        q1.free()
        o1.free()
    for b in (kb, vb, qb, ob):
        b.free()
