"""Benchmark of the MI355X attention path (libbchip.so) on BASELINE.json's configurations.

Headline (`value`): configs[1], Llama-3-8B-shaped decode: batch 1, 32 query / 8 KV heads,
head_dim 128, f16 KV cache at 32768 visible slots, RoPE theta 5e5 with the one-row K/V
append, 32 layers with distinct caches. A step is one token through all 32 layers, each
layer one bchip_rope_append_attention call (k_rope(q), k_rope(k), k_copy(k), k_copy(v) and
k_attention of the reference's per-layer sequence, the same bits as bchip_rope_append then
bchip_attention); value = tokens/s of those steps, inputs resident in HBM. Extras: decode
at 1024 and 4096 slots (their 32 layers' caches fit the 256 MB MALL: labelled so), causal
prefill at 2048 and 8192 tokens (TFLOP/s, configs[2]), the Llama-3-70B stage share's
prefill and verify steps, Qwen2.5-7B ragged batched decode with each
conversation's RoPE and K/V append in the same launch.

roofline: the dominant kernel, the decode attention kernel (attn_decode_row): algorithmic
bytes per launch (2 * L * n_kv * hd * 2 bytes of f16 K and V, each read once) over its mean
duration, from HIP events the library records on its stream right before and after that
kernel (bchip_timer_arm) on every 8th layer's call of the timed region. roofline.call gives
the same bytes over the whole per-layer call (decode kernel, chunk fold, launch gaps: the
step time over the layers). traffic: measured HBM bytes per launch from the committed
rocprofv3 counter summary.

cpu_baseline: bc-infer's CPU attention as the oracle's C restatement (single thread, as
the reference runs it: crates/bc-infer/src/model.rs:391-403, 448-481), timed on this
host on a bounded sample of the same workload: a few layers of one decode token at 32768
slots, median per layer, scaled to tokens/s for 32 layers. extra.cpu_per_config holds the
same baseline beside every other configuration (each on a stated bounded sample).
"""
import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "borrowed-compute_amd"))

import numpy as np  # noqa: E402

import bchip  # noqa: E402

HBM_PEAK_GBS = 8000.0
EVENT_EVERY = 8  # decode: HIP events bracket the attention call of every 8th layer
MFMA_F16_PEAK_TFLOPS = 2516.6
METRIC = "attn decode GB/s & prefill TFLOP/s on 1 MI355X, % of roofline; tokens/s"


class Hip:
    """hipEvent timing on a given stream (the library's), through the HIP runtime."""

    def __init__(self):
        path = None
        for cand in ("/opt/rocm/lib/libamdhip64.so", "libamdhip64.so"):
            try:
                self.lib = ctypes.CDLL(cand)
                path = cand
                break
            except OSError:
                continue
        if path is None:
            raise RuntimeError("libamdhip64.so not found")
        L = self.lib
        L.hipEventCreate.argtypes = [ctypes.c_void_p]
        L.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        L.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        L.hipEventElapsedTime.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def events(self, n):
        out = []
        for _ in range(n):
            e = ctypes.c_void_p()
            assert self.lib.hipEventCreate(ctypes.byref(e)) == 0
            out.append(e.value)
        return out

    def record(self, e, stream):
        assert self.lib.hipEventRecord(e, stream) == 0

    def elapsed(self, a, b):
        assert self.lib.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.lib.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value

    def destroy(self, evs):
        for e in evs:
            self.lib.hipEventDestroy(e)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class DecodeModel:
    """n_layer layers' caches and per-step inputs on the device, all generated there."""

    def __init__(self, ctx, nh, nkv, hd, theta, neox, n_layer, ctx_len, steps, seed=1, kv_type=bchip.F16):
        self.ctx, self.nh, self.nkv, self.hd, self.n_layer = ctx, nh, nkv, hd, n_layer
        self.ctx_len, self.steps, self.kv_type = ctx_len, steps, kv_type
        kvd = nkv * hd
        cap = ctx_len + steps + 1
        self.kc, self.vc = [], []
        for layer in range(n_layer):
            k = ctx.zeros(cap * kvd * bchip.esize(kv_type))
            v = ctx.zeros(cap * kvd * bchip.esize(kv_type))
            ctx.fill_normal(k, kv_type, ctx_len * kvd, seed * 1000 + 2 * layer)
            ctx.fill_normal(v, kv_type, ctx_len * kvd, seed * 1000 + 2 * layer + 1)
            self.kc.append(k)
            self.vc.append(v)
        # q, k, v of every (step, layer), positions of every step.
        per = (nh + 2 * nkv) * hd
        self.qkv = ctx.zeros(steps * n_layer * per * 4)
        ctx.fill_normal(self.qkv, bchip.F32, steps * n_layer * per, seed * 7919)
        self.out = ctx.zeros(nh * hd * 4)
        self.pos = ctx.upload(np.arange(ctx_len, ctx_len + steps, dtype=np.uint32))
        inv = np.array([theta ** (-2.0 * i / hd) for i in range(hd // 2)], np.float32)
        self.inv = ctx.upload(inv)
        self.neox = neox
        self.per = per
        ctx.sync()

    def layer_ptrs(self, step, layer):
        base = self.qkv.ptr + (step * self.n_layer + layer) * self.per * 4
        q = base
        k = base + self.nh * self.hd * 4
        v = k + self.nkv * self.hd * 4
        return q, k, v

    def step(self, step, hip=None, evs=None, every=EVENT_EVERY):
        """One token through every layer: the layer's RoPE + K/V append + attention as one
        bchip_rope_append_attention call (the same bits as bchip_rope_append followed by
        bchip_attention). With evs, the calls of every `every`-th layer record a pair of HIP
        events around their attention kernel (bchip_timer_arm: the library records them on
        its stream right before and after the kernel); a pair costs a few microseconds of
        stream time, so it is not put on every call of the step being timed."""
        ctx = self.ctx
        slot = self.ctx_len + step
        for layer in range(self.n_layer):
            q, k, v = self.layer_ptrs(step, layer)
            if evs is not None and layer % every == 0:
                ctx.timer_arm(evs[2 * (layer // every)], evs[2 * (layer // every) + 1])
            ctx.rope_append_attention(q, k, v, self.kc[layer], self.vc[layer], self.kv_type, self.inv,
                                      self.pos.ptr + 4 * step, self.nh, self.nkv, self.hd, self.hd, self.neox, slot,
                                      1.0 / math.sqrt(self.hd), self.out)

    def free(self):
        for b in self.kc + self.vc + [self.qkv, self.out, self.pos, self.inv]:
            b.free()


def bench_decode(ctx, hip, ctx_len, steps, warmup, n_layer=32, nh=32, nkv=8, hd=128, theta=5e5, neox=False,
                 kv_type=bchip.F16):
    m = DecodeModel(ctx, nh, nkv, hd, theta, neox, n_layer, ctx_len, steps + warmup, kv_type=kv_type)
    m.stream = ctx.stream()
    for s in range(warmup):
        m.step(s)
    ctx.sync()
    per_step = n_layer // EVENT_EVERY
    evs = hip.events(2 * per_step * steps)
    ctx.timer_start()
    for s in range(steps):
        m.step(warmup + s, hip, evs[2 * per_step * s: 2 * per_step * (s + 1)])
    total_ms = ctx.timer_stop()
    kernel_ms = [hip.elapsed(evs[2 * i], evs[2 * i + 1]) for i in range(per_step * steps)]
    hip.destroy(evs)
    m.free()
    mean_kernel_ms = statistics.fmean(kernel_ms)
    # Visible slots grow by one per step: average algorithmic bytes over the timed launches.
    mean_len = ctx_len + warmup + (steps - 1) / 2 + 1
    bytes_per_launch = 2 * mean_len * nkv * hd * bchip.esize(kv_type)
    gbs = bytes_per_launch / (mean_kernel_ms * 1e-3) / 1e9
    call_ms = total_ms / steps / n_layer  # one layer's whole call: decode kernel, fold, gaps
    return {
        "ctx": ctx_len, "layers": n_layer, "steps": steps, "ms_per_step": total_ms / steps,
        "tokens_per_s": steps / (total_ms * 1e-3), "attn_kernel_us": mean_kernel_ms * 1e3,
        "attn_bytes_per_launch": bytes_per_launch, "attn_GBps": gbs, "hbm_frac": gbs / HBM_PEAK_GBS,
        "call_us": call_ms * 1e3, "call_GBps": bytes_per_launch / (call_ms * 1e-3) / 1e9,
        "call_hbm_frac": bytes_per_launch / (call_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
    }


def bench_multirow(ctx, hip, rows, pos, nh, nkv, hd, reps, n_layer=1, verify=False):
    """Causal multi-row attention over n_layer distinct caches (prefill: pos 0)."""
    kvd = nkv * hd
    slots = pos + rows
    kcs, vcs = [], []
    for layer in range(n_layer):
        k, v = ctx.zeros(slots * kvd * 2), ctx.zeros(slots * kvd * 2)
        ctx.fill_normal(k, bchip.F16, slots * kvd, 50 + 2 * layer)
        ctx.fill_normal(v, bchip.F16, slots * kvd, 51 + 2 * layer)
        kcs.append(k)
        vcs.append(v)
    q = ctx.zeros(rows * nh * hd * 4)
    ctx.fill_normal(q, bchip.F32, rows * nh * hd, 49)
    out = ctx.zeros(rows * nh * hd * 4)
    scale = 1.0 / math.sqrt(hd)
    for layer in range(n_layer):
        ctx.attention(q, kcs[layer], vcs[layer], bchip.F16, out, None, False, rows, nh, nkv, hd, pos, scale)
    ctx.sync()
    # The call figure is the stream time of the whole timed region over the calls (no event
    # inside it but those of the main kernel, armed on every EVENT_EVERY-th call: a pair of
    # stream events costs a few microseconds, comparable to a verify call).
    every = 1 if rows >= 256 else EVENT_EVERY  # prefill kernels take milliseconds
    armed = [j for j in range(reps * n_layer) if j % every == 0]
    evs = hip.events(2 * len(armed))
    j = 0
    ctx.timer_start()
    for r in range(reps):
        for layer in range(n_layer):
            if j % every == 0:
                k = 2 * (j // every)
                ctx.timer_arm(evs[k], evs[k + 1])
            ctx.attention(q, kcs[layer], vcs[layer], bchip.F16, out, None, False, rows, nh, nkv, hd, pos, scale)
            j += 1
    total_ms = ctx.timer_stop()
    per_call = [total_ms / (reps * n_layer)]
    per_kernel = [hip.elapsed(evs[2 * k], evs[2 * k + 1]) for k in range(len(armed))]
    hip.destroy(evs)
    for b in kcs + vcs + [q, out]:
        b.free()
    pairs = rows * pos + rows * (rows + 1) / 2  # unmasked (query, key) pairs
    flops = 4.0 * hd * nh * pairs
    kv_bytes = 2.0 * slots * kvd * 2
    us = statistics.fmean(per_kernel) * 1e3
    call_us = statistics.fmean(per_call) * 1e3
    res = {"rows": rows, "pos": pos, "heads": [nh, nkv, hd], "layers": n_layer, "kernel_us": us, "call_us": call_us,
           "ms_per_pass": total_ms / reps, "TFLOPs": flops / (us * 1e-6) / 1e12,
           "mfma_frac": flops / (us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS,
           "call_TFLOPs": flops / (call_us * 1e-6) / 1e12,
           "call_mfma_frac": flops / (call_us * 1e-6) / 1e12 / MFMA_F16_PEAK_TFLOPS}
    if verify:
        res["GBps"] = kv_bytes / (us * 1e-6) / 1e9
        res["hbm_frac"] = res["GBps"] / HBM_PEAK_GBS
        res["call_GBps"] = kv_bytes / (call_us * 1e-6) / 1e9
    return res


def bench_verify_loop(ctx, steps=256, ctx0=4096, n_layer=20, nh=64, nkv=8, hd=128, rows=8, fused=False,
                      kv_type=bchip.F16):
    """configs[4]'s speculative decode as configured: 256 steps, each a pass of 8 draft rows
    through the stage's 20 layers, every layer the reference's attention sub-sequence
    (gpu/mod.rs:464-482) for 8 rows: bchip_rope_append (RoPE of q and k, the K/V append at the
    rows' slots) then bchip_attention over the line, or (fused) the one call that stands for
    both, bchip_rope_append_attention_rows (the same bits); all drafts accepted, so the context
    grows 4096 -> 6136 by 8 a step. Timed as one region: the stream time of all 256 x 20
    layer-steps. kv_type: the cache's element type (f16 as configured; f32 is the reference's
    own cache, what an unmodified binding passes)."""
    kvd = nkv * hd
    cap = ctx0 + steps * rows
    es = 2 if kv_type == bchip.F16 else 4
    kcs, vcs = [], []
    for layer in range(n_layer):
        k, v = ctx.zeros(cap * kvd * es), ctx.zeros(cap * kvd * es)
        ctx.fill_normal(k, kv_type, ctx0 * kvd, 700 + 2 * layer)
        ctx.fill_normal(v, kv_type, ctx0 * kvd, 701 + 2 * layer)
        kcs.append(k)
        vcs.append(v)
    per = rows * (nh + 2 * nkv) * hd  # a layer's q [rows][nh*hd], then k and v [rows][kvd]
    qkv = ctx.zeros(n_layer * per * 4)
    ctx.fill_normal(qkv, bchip.F32, n_layer * per, 699)
    pos = ctx.upload(np.arange(ctx0, cap, dtype=np.uint32))
    inv = ctx.upload(np.array([5e5 ** (-2.0 * i / hd) for i in range(hd // 2)], np.float32))
    out = ctx.zeros(rows * nh * hd * 4)
    scale = 1.0 / math.sqrt(hd)

    def step(s):
        base = ctx0 + s * rows
        for layer in range(n_layer):
            q = qkv.ptr + layer * per * 4
            k = q + rows * nh * hd * 4
            v = k + rows * kvd * 4
            if fused:
                ctx.rope_append_attention_rows(q, k, v, kcs[layer], vcs[layer], kv_type, inv, pos.ptr + 4 * s * rows,
                                               rows, nh, nkv, hd, hd, False, base, scale, out)
                continue
            ctx.rope_append(q, k, v, kcs[layer], vcs[layer], kv_type, inv, pos.ptr + 4 * s * rows, rows, nh, nkv,
                            hd, hd, False, base)
            ctx.attention(q, kcs[layer], vcs[layer], kv_type, out, None, False, rows, nh, nkv, hd, base, scale)

    step(0)  # warm (the step's appends are rewritten by the timed step 0)
    ctx.sync()
    ctx.timer_start()
    for s in range(steps):
        step(s)
    total_ms = ctx.timer_stop()
    for b in kcs + vcs + [qkv, pos, inv, out]:
        b.free()
    kv_bytes = sum(2.0 * (ctx0 + (s + 1) * rows) * kvd * es for s in range(steps)) * n_layer
    layer_steps = steps * n_layer
    return {"steps": steps, "rows": rows, "ctx": [ctx0, ctx0 + steps * rows], "layers": n_layer,
            "cache": "f16" if kv_type == bchip.F16 else "f32",
            "calls_per_layer_step": "bchip_rope_append_attention_rows" if fused else "bchip_rope_append + bchip_attention",
            "total_ms": total_ms,
            "us_per_layer_step": total_ms * 1e3 / layer_steps,
            "tokens_per_s": rows * steps / (total_ms * 1e-3),
            "kv_GBps": kv_bytes / (total_ms * 1e-3) / 1e9, "kv_hbm_frac": kv_bytes / (total_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "note": "tokens_per_s: accepted draft tokens per second through the 20-layer stage's attention path"}


def bench_ragged(ctx, hip, reps):
    """16 conversations in one pool, lengths U[1024, 32768] (seeded) counting the new
    token, 28/4 heads, hd 128, RoPE theta 1e6 (neox), 28 layers. A step is one token of every
    conversation through every layer, each layer one bchip_rope_append_attention_ragged call:
    the RoPE of each conversation's new q and k, its K/V append at its last slot and the
    attention of all 16, in one launch."""
    nh, nkv, hd, n_layer, nseq = 28, 4, 128, 28, 16
    rng = np.random.default_rng(4)
    lens = rng.integers(1024, 32769, size=nseq).astype(np.uint32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.uint64)
    total = int(lens.sum())
    kvd = nkv * hd
    kcs, vcs = [], []
    for layer in range(n_layer):
        k, v = ctx.zeros(total * kvd * 2), ctx.zeros(total * kvd * 2)
        ctx.fill_normal(k, bchip.F16, total * kvd, 300 + 2 * layer)
        ctx.fill_normal(v, bchip.F16, total * kvd, 301 + 2 * layer)
        kcs.append(k)
        vcs.append(v)
    per = nseq * (nh + 2 * nkv) * hd  # q [16][nh*hd], then k and v [16][kvd], per layer
    qkv = ctx.zeros(n_layer * per * 4)
    ctx.fill_normal(qkv, bchip.F32, n_layer * per, 299)
    pos = ctx.upload(lens - 1)
    inv = ctx.upload(np.array([1e6 ** (-2.0 * i / hd) for i in range(hd // 2)], np.float32))
    out = ctx.zeros(nseq * nh * hd * 4)
    scale = 1.0 / math.sqrt(hd)

    def call(layer):
        q = qkv.ptr + layer * per * 4
        k = q + nseq * nh * hd * 4
        v = k + nseq * kvd * 4
        ctx.rope_append_attention_ragged(q, k, v, kcs[layer], vcs[layer], bchip.F16, inv, pos, lens, offs, nh, nkv,
                                         hd, hd, True, scale, out)

    for layer in range(n_layer):
        call(layer)
    ctx.sync()
    # Call figure: the timed region's stream time over the calls; the main kernel's events are
    # armed on every EVENT_EVERY-th call only (as in bench_decode).
    armed = [j for j in range(reps * n_layer) if j % EVENT_EVERY == 0]
    evs = hip.events(2 * len(armed))
    j = 0
    ctx.timer_start()
    for r in range(reps):
        for layer in range(n_layer):
            if j % EVENT_EVERY == 0:
                k = 2 * (j // EVENT_EVERY)
                ctx.timer_arm(evs[k], evs[k + 1])
            call(layer)
            j += 1
    total_ms = ctx.timer_stop()
    per_call = [total_ms / (reps * n_layer)]
    per_kernel = [hip.elapsed(evs[2 * k], evs[2 * k + 1]) for k in range(len(armed))]
    hip.destroy(evs)
    for b in kcs + vcs + [qkv, pos, inv, out]:
        b.free()
    us = statistics.fmean(per_kernel) * 1e3
    call_us = statistics.fmean(per_call) * 1e3
    bytes_ = 2.0 * total * kvd * 2
    return {"seqs": nseq, "total_slots": total, "layers": n_layer, "step": "bchip_rope_append_attention_ragged",
            "kernel_us": us, "call_us": call_us, "ms_per_step": total_ms / reps,
            "tokens_per_s": nseq * reps / (total_ms * 1e-3),
            "GBps": bytes_ / (us * 1e-6) / 1e9, "hbm_frac": bytes_ / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "call_GBps": bytes_ / (call_us * 1e-6) / 1e9,
            "call_hbm_frac": bytes_ / (call_us * 1e-6) / 1e9 / HBM_PEAK_GBS}


def bench_copy_calibration(ctx, hip, mib=256, reps=4):
    """A plain f16 copy of known size (bchip_copy): the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters of a profiling run, and achievable copy bandwidth."""
    n = mib * 1024 * 1024 // 2
    src, dst = ctx.zeros(n * 2), ctx.zeros(n * 2)
    ctx.copy(src, bchip.F16, dst, bchip.F16, 0, n)
    ctx.sync()
    ctx.timer_start()
    for _ in range(reps):
        ctx.copy(src, bchip.F16, dst, bchip.F16, 0, n)
    ms = ctx.timer_stop()
    src.free()
    dst.free()
    return {"bytes_read_per_copy": n * 2, "bytes_written_per_copy": n * 2, "copies": reps + 1,
            "copy_GBps": 2 * n * 2 * reps / (ms * 1e-3) / 1e9}


def synthetic_weights(wtype, rows, cols, seed):
    """Random ggml blocks with finite, modest scales (every scale field 1/1024), as bytes."""
    n, size = bchip.GGML_BLOCKS[wtype]
    rng = np.random.default_rng(seed)
    data = rng.integers(0, 256, rows * cols // n * size, dtype=np.uint8).reshape(-1, size)
    if wtype in (bchip.GGML_F16, bchip.GGML_BF16, bchip.GGML_F32):
        vals = rng.standard_normal(rows * cols).astype(np.float32)
        if wtype == bchip.GGML_F16:
            return vals.astype(np.float16).view(np.uint8)
        if wtype == bchip.GGML_BF16:
            return (vals.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
        return vals.view(np.uint8)
    scale = np.frombuffer(np.float16(1.0 / 1024).tobytes(), np.uint8)
    fields = [208] if wtype == bchip.GGML_Q6K else [0, 2] if wtype in (bchip.GGML_Q4_1, bchip.GGML_Q5_1,
                                                                        bchip.GGML_Q4K, bchip.GGML_Q5K) else [0]
    for f in fields:
        data[:, f:f + 2] = scale
    return data.reshape(-1)


def bench_products(ctx, reps=20):
    """The GGUF block-format product (bchip_matmul) on Llama-3-8B's largest per-layer shapes:
    the FFN gate/up (14336 x 4096) and down (4096 x 14336) matrices, decode (one input row) and
    an 8-row batch, in the formats real GGUF files use. Weight bytes per call / call time
    (back-to-back calls on the stream, so launch gaps included) against 8 TB/s."""
    out = {}
    shapes = (("gate_14336x4096", 14336, 4096), ("down_4096x14336", 4096, 14336))
    for wtype, name in ((bchip.GGML_Q4K, "Q4K"), (bchip.GGML_Q6K, "Q6K"), (bchip.GGML_Q8_0, "Q8_0"),
                        (bchip.GGML_F16, "F16")):
        for shape, rows, cols in shapes:
            data = synthetic_weights(wtype, rows, cols, rows + cols + wtype)
            wb = ctx.upload(data)
            for n in (1, 8):
                xb = ctx.upload(np.random.default_rng(n).standard_normal((n, cols)).astype(np.float32))
                ob = ctx.zeros(n * rows * 4)
                ctx.matmul(wb, wtype, xb, ob, rows, cols, n)
                ctx.sync()
                ctx.timer_start()
                for _ in range(reps):
                    ctx.matmul(wb, wtype, xb, ob, rows, cols, n)
                ms = ctx.timer_stop()
                us = ms * 1e3 / reps
                gbps = data.nbytes / (us * 1e-6) / 1e9
                out[f"{name}_{shape}_n{n}"] = {"weight_bytes": int(data.nbytes), "call_us": us, "GBps": gbps,
                                              "hbm_frac": gbps / HBM_PEAK_GBS}
                xb.free()
                ob.free()
            wb.free()
    return out


def cpu_baseline(layers=5, ctx_len=32768, nh=32, nkv=8, hd=128):
    """The oracle's single-thread attention (+ rope of the new q and k rows) per layer of one
    decode token at ctx_len slots; median over `layers` layers, scaled to 32 layers."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    O.lib()
    inv = O.inv_freq(hd, 5e5)
    times = []
    for layer in range(layers):
        q = O.normal(10 + layer, nh * hd).reshape(1, nh, hd)
        kc = O.normal(20 + layer, (ctx_len + 1) * nkv * hd).reshape(ctx_len + 1, nkv * hd)
        vc = O.normal(30 + layer, (ctx_len + 1) * nkv * hd).reshape(ctx_len + 1, nkv * hd)
        t0 = time.perf_counter()
        qr = O.rope(q, nh, hd, hd, False, ctx_len, inv)
        kc[ctx_len] = O.rope(kc[ctx_len], nkv, hd, hd, False, ctx_len, inv)
        O.attention(qr, kc, vc, 1, ctx_len, nh, nkv, hd, 1.0 / math.sqrt(hd))
        times.append(time.perf_counter() - t0)
    per_layer = statistics.median(times)
    return {"value": 1.0 / (32 * per_layer), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{layers} layers of one Llama-3-8B decode token at {ctx_len} slots (f32 oracle, "
                      f"model.rs:391-403+448-481 restated in C, 1 thread); median {per_layer * 1e3:.1f} ms/layer, "
                      f"scaled to 32 layers",
            "cpu": _cpu_model(), "nproc": os.cpu_count()}


def cpu_per_config():
    """bc-infer's CPU attention (the oracle's C restatement of model.rs:391-403, 448-481, one
    thread, as the reference runs it) beside every configuration, each timed on this host on a
    bounded sample and scaled by its count of (query, key) pairs or of layers, as stated in each
    entry's "sample"."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    O.lib()
    rng = np.random.default_rng(11)
    out = {}

    def rnd(*shape):
        return rng.standard_normal(shape, dtype=np.float32)

    # Qwen2.5-0.5B decode at 512 slots, f32, 24 layers: the whole workload.
    nh, nkv, hd, L = 14, 2, 64, 512
    inv = O.inv_freq(hd, 1e6)
    t = 0.0
    for layer in range(24):
        q, kc, vc = rnd(1, nh, hd), rnd(L, nkv * hd), rnd(L, nkv * hd)
        t0 = time.perf_counter()
        qr = O.rope(q, nh, hd, hd, True, L - 1, inv)
        kc[L - 1] = O.rope(kc[L - 1], nkv, hd, hd, True, L - 1, inv)
        O.attention(qr, kc, vc, 1, L - 1, nh, nkv, hd, 0.125)
        t += time.perf_counter() - t0
    out["configs0_qwen05b_decode_512"] = {"tokens_per_s": 1.0 / t, "ms_per_token": t * 1e3, "cores": 1,
                                          "sample": "the whole workload: 24 layers of one token (rope + attention)"}

    def prefill(S, nh, nkv, hd, stride, name, layers):
        # Rows r = stride-1, 2*stride-1, ... of one layer, one row a call (row r sees r+1 slots);
        # scaled by the (query, key) pairs of all S rows.
        q, kc, vc = rnd(S, nh, hd), rnd(S, nkv * hd), rnd(S, nkv * hd)
        rows = list(range(stride - 1, S, stride))
        t0 = time.perf_counter()
        for r in rows:
            O.attention(q[r:r + 1], kc, vc, 1, r, nh, nkv, hd, 1.0 / math.sqrt(hd))
        t = time.perf_counter() - t0
        per_pair = t / sum(r + 1 for r in rows)
        res = {}
        for s_full in ((S,) if name != "configs2_llama8b_prefill" else (2048, 8192)):
            pairs = s_full * (s_full + 1) / 2
            layer_s = per_pair * pairs
            res[f"S{s_full}"] = {"s_per_layer": layer_s, "TFLOPs": 4.0 * hd * nh * pairs / layer_s / 1e12,
                                 "tokens_per_s": s_full / (layer_s * layers)}
        res.update({"cores": 1, "sample": f"{len(rows)} rows (every {stride}th) of one {S}-row layer, "
                                          f"{nh}/{nkv} heads; time per (query, key) pair scaled to every row and "
                                          f"{layers} layers" + ("; S=8192 extrapolated from S=2048's per-pair time"
                                                                if S == 2048 else "")})
        out[name] = res

    prefill(2048, 32, 8, 128, 8, "configs2_llama8b_prefill", 32)
    prefill(4096, 64, 8, 128, 32, "configs4_llama70b_prefill", 20)

    # 16 conversations' one-token steps; 4 of them timed, scaled by slots.
    nh, nkv, hd = 28, 4, 128
    lens = np.random.default_rng(4).integers(1024, 32769, size=16)
    picked = [int(x) for x in lens[:4]]
    t = 0.0
    for L in picked:
        q, kc, vc = rnd(1, nh, hd), rnd(L, nkv * hd), rnd(L, nkv * hd)
        t0 = time.perf_counter()
        O.attention(q, kc, vc, 1, L - 1, nh, nkv, hd, 1.0 / math.sqrt(hd))
        t += time.perf_counter() - t0
    layer_s = t * float(lens.sum()) / sum(picked)
    out["configs3_qwen7b_ragged"] = {"s_per_layer": layer_s, "tokens_per_s": 16 / (layer_s * 28), "cores": 1,
                                     "sample": "4 of the 16 conversations, one layer, scaled by slots to all 16 and 28 "
                                               "layers"}
    # one verify step of 8 rows at 4096 slots, one layer, scaled to 20 layers.
    nh, nkv, hd, ctx0 = 64, 8, 128, 4096
    q, kc, vc = rnd(8, nh, hd), rnd(ctx0 + 8, nkv * hd), rnd(ctx0 + 8, nkv * hd)
    t0 = time.perf_counter()
    O.attention(q, kc, vc, 8, ctx0, nh, nkv, hd, 1.0 / math.sqrt(hd))
    layer_s = time.perf_counter() - t0
    out["configs4_llama70b_verify_4096"] = {"s_per_layer_step": layer_s, "tokens_per_s": 8 / (layer_s * 20),
                                            "cores": 1, "sample": "one layer of one 8-row verify step at 4096 slots, "
                                                                  "scaled to 20 layers (all 8 drafts accepted)"}
    return out


def profiled_traffic(ctx_len):
    """HBM bytes per decode attention call (decode + fold kernels) from the committed counter
    summary: FETCH_SIZE and WRITE_SIZE passes of rocprofv3 over this script, scaled by the
    same counters' reading for a copy of known size. None when the summary is absent or was
    taken at another context length."""
    path = os.path.join(ROOT, "profiles", "attn_decode_row_llama8b_32k.txt")
    if ctx_len != 32768 or not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--ctx", type=int, default=32768, help="visible slots of the headline decode")
    ap.add_argument("--only", default="", help="comma list of sections: decode,short,prefill,verify,loop,f32,"
                                               "ragged,calib,products,cpu")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this build runs on one GPU; the attention path's "
                                   "split over several GPUs (by KV head or by sequence chunk) is a design, not run here"}))
        sys.exit(2)
    want = set(args.only.split(",")) if args.only else {"decode", "short", "prefill", "verify", "loop", "f32",
                                                         "ragged", "calib", "products", "cpu"}
    hip = Hip()
    extra = {}
    with bchip.Ctx(0) as ctx:
        log(f"device: {ctx.name()}")
        head = None
        if "decode" in want:
            log(f"decode: 32 layers at {args.ctx} slots, {args.warmup}+{args.steps} steps")
            head = bench_decode(ctx, hip, args.ctx, args.steps, args.warmup)
            log(json.dumps(head))
        if "short" in want:
            for L in (1024, 4096):
                log(f"decode at {L} slots (all 32 layers' caches fit the 256 MB MALL)")
                r = bench_decode(ctx, hip, L, args.steps, args.warmup)
                r["note"] = "MALL-resident and launch-bound: reported, not a roofline figure"
                extra[f"decode_{L}"] = r
                log(json.dumps(r))
        if "prefill" in want:
            for S, layers, reps in ((2048, 32, 2), (8192, 4, 2)):
                log(f"prefill {S} tokens, {layers} layers x {reps}")
                r = bench_multirow(ctx, hip, S, 0, 32, 8, 128, reps, n_layer=layers)
                extra[f"prefill_{S}"] = r
                log(json.dumps(r))
        if "verify" in want:
            log("Llama-3-70B share: 4096-token prefill, verify 8 rows at 4096 and 6136 slots, 20 layers")
            extra["prefill_70b_4096"] = bench_multirow(ctx, hip, 4096, 0, 64, 8, 128, 1, n_layer=20)
            log(json.dumps(extra["prefill_70b_4096"]))
            for ctx_len in (4096, 6136):
                r = bench_multirow(ctx, hip, 8, ctx_len, 64, 8, 128, 10, n_layer=20, verify=True)
                extra[f"verify_70b_{ctx_len}"] = r
                log(json.dumps(r))
        if "loop" in want:
            log("Llama-3-70B share: 256 verify steps of 8 rows, 20 layers, rope_append + attention a layer-step")
            extra["verify_loop_70b_256"] = bench_verify_loop(ctx)
            log(json.dumps(extra["verify_loop_70b_256"]))
            log("the same loop through the single call for the layer's rotations, appends and attention")
            extra["verify_loop_70b_256_fused"] = bench_verify_loop(ctx, fused=True)
            log(json.dumps(extra["verify_loop_70b_256_fused"]))
        if "f32" in want:
            # The drop-in default: an unmodified binding passes the reference's f32 cache
            # (bchip_rope_append_attention with BCHIP_F32: attn_f32 with the rotation and the append).
            log(f"f32-cache decode (the reference's cache type): configs[1] at {args.ctx} slots, configs[0]")
            r = bench_decode(ctx, hip, args.ctx, 10, 2, kv_type=bchip.F32)
            r["note"] = "f32 cache, f32 arithmetic (attn_f32): the path an unmodified binding runs"
            extra[f"decode_f32_{args.ctx}"] = r
            log(json.dumps(r))
            r = bench_decode(ctx, hip, 512, args.steps, args.warmup, n_layer=24, nh=14, nkv=2, hd=64, theta=1e6,
                             neox=True, kv_type=bchip.F32)
            r["note"] = "configs[0]: Qwen2.5-0.5B-shaped, f32 cache at 512 slots, 24 layers; cache-resident"
            extra["decode_qwen05b_512_f32"] = r
            log(json.dumps(r))
            log("configs[4]'s verify loop over f32 caches (one call a layer-step)")
            r = bench_verify_loop(ctx, fused=True, kv_type=bchip.F32)
            extra["verify_loop_70b_256_f32"] = r
            log(json.dumps(r))
        if "calib" in want:
            extra["copy_calibration"] = bench_copy_calibration(ctx, hip)
            log(json.dumps(extra["copy_calibration"]))
        if "ragged" in want:
            log("ragged: 16 Qwen2.5-7B sequences, 28 layers")
            extra["ragged_qwen7b"] = bench_ragged(ctx, hip, 5)
            log(json.dumps(extra["ragged_qwen7b"]))
        if "products" in want:
            log("GGUF block-format products at Llama-3-8B FFN shapes (the rest of the layer)")
            extra["products"] = bench_products(ctx)
            log(json.dumps(extra["products"]))
    cpu = None
    if "cpu" in want:
        log("cpu baseline (oracle, 1 thread)")
        cpu = cpu_baseline()
        log(json.dumps(cpu))
        extra["cpu_per_config"] = cpu_per_config()
        log(json.dumps(extra["cpu_per_config"]))
    # The rate a plain copy reaches in the same run (bytes read + written over its time):
    # the measured ceiling the kernel and the call are also reported against.
    ceil_gbs = (extra.get("copy_calibration") or {}).get("copy_GBps")
    if ceil_gbs and "ragged_qwen7b" in extra:
        rg = extra["ragged_qwen7b"]
        rg["frac_of_copy"], rg["call_frac_of_copy"] = rg["GBps"] / ceil_gbs, rg["call_GBps"] / ceil_gbs
    if head is None:
        print(json.dumps({"extra": extra, "cpu_baseline": cpu}))
        return
    measured = None
    if ceil_gbs:
        measured = {"what": "a plain 256 MiB f16 copy (bchip_copy) in the same run, read + write bytes over its time",
                    "GBps": ceil_gbs, "kernel_frac": head["attn_GBps"] / ceil_gbs,
                    "call_frac": head["call_GBps"] / ceil_gbs}
    line = {
        "metric": METRIC,
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: seeded N(0,1) q/k/v and KV cache (splitmix64 + Box-Muller, generated on the device)",
        "config": {"workload": "configs[1]: Llama-3-8B decode attention, batch 1, 32/8 heads, head_dim 128, "
                               f"f16 KV at {args.ctx} slots, RoPE theta 5e5 fused with the K/V append, 32 layers",
                   "ctx": args.ctx, "layers": 32},
        "roofline": {"bound": "hbm", "achieved": head["attn_GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": head["hbm_frac"], "traffic": profiled_traffic(args.ctx),
                     "traffic_source": "profiles/attn_decode_row_llama8b_32k.txt (rocprofv3 FETCH_SIZE x 2.0 + "
                                       "WRITE_SIZE x 1.0, factors from a 256 MiB copy)",
                     "kernel": "attn_decode_row<128, f16, fused> (bchip_rope_append_attention's attention kernel)",
                     "bytes_per_launch": head["attn_bytes_per_launch"], "launch_us": head["attn_kernel_us"],
                     "call": {"what": "the whole per-layer call: decode kernel, chunk fold, launch gaps",
                              "us": head["call_us"], "GBps": head["call_GBps"], "frac": head["call_hbm_frac"]},
                     "measured_ceiling": measured},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
