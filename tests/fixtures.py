"""Inputs of the reference's own known-answer fixtures, restated in numpy.

* kat_inputs: tests/sparse_numeric_fixture.cpp:23-156 (10 points, 2 batches,
  affine sequences);
* block_kat: tests/sparse_transformer_numeric_fixture.cpp:36-135 (one cross
  block, C=12, 2 heads x 6, MLP 18, context 5, projection 7).
The expected outputs are the reference binaries' printed values, committed as
tests/golden/*.json.
"""

import numpy as np


def kat_inputs():
    coords = np.array([[0, 0, 0, 0], [0, 0, 0, 1], [0, 0, 1, 0], [0, 1, 1, 1], [0, 2, 2, 2],
                       [1, 0, 0, 0], [1, 0, 1, 0], [1, 1, 1, 1], [1, 2, 1, 2], [1, 3, 3, 3]],
                      np.int32)
    n = 10
    f32 = np.float32
    feats = np.array([f32(-0.31) + f32(0.047) * f32(i) for i in range(n * 3)], f32).reshape(n, 3)
    lw = np.array([f32(-0.11) + f32(0.013) * f32(i) for i in range(12)], f32).reshape(4, 3)
    lb = np.array([-0.07, 0.02, 0.11, 0.20], f32)
    cw = np.array([f32(-0.021) + f32(0.0017) * f32(i) for i in range(27 * 12)], f32).reshape(27, 4, 3)
    cb = np.array([-0.03, 0.01, 0.05, 0.09], f32)
    q = np.array([f32(-0.23) + f32(0.017) * f32(i) for i in range(n * 12)], f32).reshape(n, 12)
    k = np.array([f32(0.17) - f32(0.021) * f32(i) for i in range(n * 12)], f32).reshape(n, 12)
    v = np.array([f32(-0.13) + f32(0.031) * f32(i) for i in range(n * 12)], f32).reshape(n, 12)
    ck = np.array([f32(0.09) - f32(0.014) * f32(i) for i in range(60)], f32).reshape(5, 12)
    cv = np.array([f32(-0.18) + f32(0.022) * f32(i) for i in range(60)], f32).reshape(5, 12)
    rg = np.array([f32(0.7) + f32(0.013) * f32(i) for i in range(12)], f32)
    pc = np.array([[0, 0, 0, 0], [0, 1, 0, 1], [1, 0, 1, 0]], np.int32)
    pf = np.array([f32(-0.17) + f32(0.011) * f32(i) for i in range(48)], f32).reshape(3, 16)
    sub = np.array([[1, 0, 1, 0, 0, 1, 0, 0], [0, 1, 1, 0, 1, 0, 0, 1], [1, 1, 0, 0, 0, 0, 1, 0]], f32)
    return dict(coords=coords, feats=feats, lw=lw, lb=lb, cw=cw, cb=cb, q=q, k=k, v=v, ck=ck,
                cv=cv, rg=rg, pc=pc, pf=pf, sub=sub)


def stable_param(name, count):
    """tests/sparse_transformer_numeric_fixture.cpp:36-50 (hash-of-name values)."""
    stable = sum((i + 1) * ord(ch) for i, ch in enumerate(name))
    out = np.array([(np.float32((i + stable) % 29) - np.float32(14.0)) * np.float32(0.018)
                    for i in range(count)], np.float32)
    if name.endswith("gamma"):
        out = np.abs(out) + np.float32(0.5)
    return out


def block_kat():
    C, H, M, CC, PC, n = 12, 2, 18, 5, 7, 10
    names = [("modulation", 6 * C), ("self_attn.to_qkv.weight", 3 * C * C),
             ("self_attn.to_qkv.bias", 3 * C), ("self_attn.q_rms_norm.gamma", C),
             ("self_attn.k_rms_norm.gamma", C), ("self_attn.to_out.weight", C * C),
             ("self_attn.to_out.bias", C), ("norm2.weight", C), ("norm2.bias", C),
             ("cross_attn.cross_attn_block.to_q.weight", C * C),
             ("cross_attn.cross_attn_block.to_q.bias", C),
             ("cross_attn.cross_attn_block.to_kv.weight", 2 * C * CC),
             ("cross_attn.cross_attn_block.to_kv.bias", 2 * C),
             ("cross_attn.cross_attn_block.q_rms_norm.gamma", C),
             ("cross_attn.cross_attn_block.k_rms_norm.gamma", C),
             ("cross_attn.cross_attn_block.to_out.weight", C * C),
             ("cross_attn.cross_attn_block.to_out.bias", C),
             ("cross_attn.proj_linear.weight", C * PC), ("cross_attn.proj_linear.bias", C),
             ("mlp.mlp.0.weight", M * C), ("mlp.mlp.0.bias", M), ("mlp.mlp.2.weight", C * M),
             ("mlp.mlp.2.bias", C)]
    ws = [stable_param(nm, cnt) for nm, cnt in names]
    seq = lambda cnt, off, step: np.array([np.float32(off) + np.float32(step) * np.float32(i)  # noqa: E731
                                           for i in range(cnt)], np.float32)
    coords = kat_inputs()["coords"]
    x = seq(n * C, -0.27, 0.013).reshape(n, C)
    proj = seq(n * PC, 0.19, -0.017).reshape(n, PC)
    ctx = seq(5 * CC, -0.11, 0.021).reshape(5, CC)
    tmod = seq(2 * 6 * C, 0.07, -0.009)
    return dict(coords=coords, x=x, proj=proj, ctx=ctx, tmod=tmod, weights=ws,
                cfg_i=[C, H, M, CC, PC, 1, 1, 1, 1], cfg_f=[1e-6, 1.0, 10000.0])
