"""Writes the attention golden vectors in this directory (run from the repo root:
python tests/golden/make_golden.py).

The reference holds no attention fixtures (crates/bc-infer/src/model.rs:483-689 checks only
relative properties), so these come from a library routine instead of the reference:
torch.nn.functional.scaled_dot_product_attention in f64 on the CPU, with KV heads expanded
by repeat_interleave (query head h reads KV head h // (nh/nkv), model.rs:463) and the
visibility of model.rs:458-459 as an explicit boolean mask. Inputs are float32 seeded
N(0,1) draws; expected outputs are rounded to float32.
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = 0xFFFFFFFF


def tree_shape(rows, pos, parents):
    base = pos + rows - len(parents)
    depth, vis = [], []
    for i, p in enumerate(parents):
        d, seen = (0, 0) if p == ROOT else (depth[p] + 1, vis[p])
        depth.append(d)
        vis.append(seen | (1 << i))
    skip = len(parents) - rows
    return np.array(vis[skip:], np.uint64), base


def mask_of(rows, pos, visible, base):
    n = pos + rows
    m = np.zeros((rows, n), bool)
    for i in range(rows):
        if visible is None:
            m[i, : pos + i + 1] = True
        else:
            m[i, :base] = True
            for j in range(n - base):
                m[i, base + j] = bool((int(visible[i]) >> j) & 1)
    return m


def write(name, rows, pos, nh, nkv, hd, seed, parents=None, scale=None):
    rng = np.random.default_rng(seed)
    n = pos + rows
    q = rng.standard_normal((rows, nh, hd)).astype(np.float32)
    kc = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd))) if scale is None else scale
    visible, base = (None, pos) if parents is None else tree_shape(rows, pos, parents)
    g = nh // nkv
    tq = torch.from_numpy(q).double().permute(1, 0, 2)
    tk = torch.from_numpy(kc).double().view(n, nkv, hd).permute(1, 0, 2).repeat_interleave(g, 0)
    tv = torch.from_numpy(vc).double().view(n, nkv, hd).permute(1, 0, 2).repeat_interleave(g, 0)
    mask = torch.from_numpy(mask_of(rows, pos, visible, base))
    out = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=scale)
    np.savez_compressed(os.path.join(HERE, name), q=q, kc=kc, vc=vc, out=out.permute(1, 0, 2).float().numpy(),
                        shape=np.array([rows, pos, nh, nkv, hd]), scale=np.float32(scale),
                        visible=np.zeros(0, np.uint64) if visible is None else visible, base=np.int64(base))


if __name__ == "__main__":
    write("decode_qwen05b_l64.npz", 1, 63, 14, 2, 64, 1, scale=0.125)
    write("prefill_tiny_s9.npz", 9, 0, 4, 2, 16, 2)
    write("chunked_gqa_r5_p20.npz", 5, 20, 16, 4, 128, 3)
    write("tree_reference_shape.npz", 5, 3, 4, 2, 16, 4, parents=[ROOT, 0, 0, 1, ROOT])
    write("tree_grown_last_level.npz", 1, 7, 4, 2, 16, 5, parents=[ROOT, ROOT, 0, 0, 2])
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
