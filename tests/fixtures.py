"""Inputs of the reference's own known-answer fixtures, restated in numpy.

* kat_inputs: tests/sparse_numeric_fixture.cpp:23-156 (10 points, 2 batches,
  affine sequences);
* block_kat: tests/sparse_transformer_numeric_fixture.cpp:36-135 (one cross
  block, C=12, 2 heads x 6, MLP 18, context 5, projection 7);
* flow_case: seeded SLat-flow inputs and weights (this build's, for the
  oracle-vs-reference and GPU-vs-oracle flow checks).
The expected outputs are the reference binaries' printed values, committed as
tests/golden/*.json.
"""

import os
import sys
import tempfile

import numpy as np

import workloads as W


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


def flow_case(seed, n_items, grid, C, H, nblocks, ctx_tokens, in_ch=8, out_ch=8, mlp_ratio=4):
    coords = W.shell_coords(grid, n_items, seed)
    n = coords.shape[0]
    M, CC = C * mlp_ratio, C
    rng_std = 0.02
    x = W.normal(seed, n * in_ch, 1).reshape(n, in_ch)
    t = (W.uniform(seed, len(n_items), 2) * 1000.0).astype(np.float32)
    ctx = W.normal(seed, ctx_tokens * len(n_items) * CC, 3).reshape(-1, CC)
    ctx_off = np.arange(len(n_items) + 1, dtype=np.int64) * ctx_tokens
    fw = [W.normal(seed, C * in_ch, 10, std=rng_std).reshape(C, in_ch), np.zeros(C, np.float32),
          W.normal(seed, C * 256, 11, std=rng_std).reshape(C, 256), np.zeros(C, np.float32),
          W.normal(seed, C * C, 12, std=rng_std).reshape(C, C), np.zeros(C, np.float32),
          W.normal(seed, 6 * C * C, 13, std=rng_std).reshape(6 * C, C),
          np.zeros(6 * C, np.float32),
          W.normal(seed, out_ch * C, 14, std=rng_std).reshape(out_ch, C),
          np.zeros(out_ch, np.float32)]
    shapes = [6 * C, 3 * C * C, 3 * C, C, C, C * C, C, C, C, C * C, C, 2 * C * CC, 2 * C, C, C,
              C * C, C, None, None, M * C, M, C * M, C]
    blocks = []
    for b in range(nblocks):
        ws = []
        for i, s in enumerate(shapes):
            if s is None:
                ws.append(None)
                continue
            w = W.normal(seed + 100 * (b + 1), s, i, std=rng_std)
            if i in (3, 4, 7, 13, 14):  # RMS gammas and the norm2 weight
                w = np.ones(s, np.float32)
            ws.append(w)
        blocks.append(ws)
    dims = [in_ch, C, out_ch, nblocks, H, M, CC, 1, 1]
    return dict(coords=coords, x=x, t=t, ctx=ctx, ctx_off=ctx_off, fw=fw, blocks=blocks,
                dims=dims, C=C, H=H, M=M, CC=CC, n=n)


def flow_velocity(coords, channels, seed=5):
    """A deterministic stand-in for the flow model (numpy float32): the
    velocity of state s at model time T for condition c is
    tanh(s * a_c) * (T / 1000 + 0.5) + m_c[item] + 0.01 * x-coordinate,
    with different a_c, m_c for the conditional and unconditional branch."""
    coords = np.asarray(coords, np.int32).reshape(-1, 4)
    items = coords[:, 0]
    nb = int(items.max()) + 1 if items.size else 1
    m = {True: W.normal(seed, nb * channels, 1, std=0.3).reshape(nb, channels),
         False: W.normal(seed, nb * channels, 2, std=0.3).reshape(nb, channels)}
    a = {True: np.float32(0.9), False: np.float32(-0.4)}
    xo = (np.float32(0.01) * coords[:, 1].astype(np.float32))[:, None]

    def fn(state, t_model, conditional):
        s = np.asarray(state, np.float32)
        scale = np.float32(t_model) / np.float32(1000.0) + np.float32(0.5)
        return (np.tanh(s * a[conditional]) * scale + m[conditional][items] + xo).astype(np.float32)

    return fn


def child_slots_brute_force(coords, out_coords):
    """Slot c of output (b, X, Y, Z) holds the input row at
    (b, 2X + (c & 1), 2Y + ((c >> 1) & 1), 2Z + (c >> 2)), or -1: the
    little-endian child order of the reference's factor-2 subdivision
    (src/sparse.cpp:676-690), found by dictionary lookup."""
    where = {tuple(r): i for i, r in enumerate(coords.tolist())}
    expect = np.full((out_coords.shape[0], 8), -1, np.int32)
    for q, (b, x, y, z) in enumerate(out_coords.tolist()):
        for c in range(8):
            expect[q, c] = where.get((b, 2 * x + (c & 1), 2 * y + ((c >> 1) & 1),
                                      2 * z + (c >> 2)), -1)
    return expect


def subdivided_parents(seed, channels, masked):
    """Parents on a 10^3 grid (two batch items) with 8*channels features and,
    when masked, a +-1 subdivision mask with at least one child per parent."""
    parents = W.shell_coords(10, [[(2.0, 4.0)], [(1.5, 3.5)]], seed)
    m = parents.shape[0]
    pf = W.normal(seed, m * 8 * channels, 1).reshape(m, 8 * channels)
    sub = None
    if masked:
        sub = np.where(W.uniform(seed, m * 8, 2).reshape(m, 8) < 0.5, 1.0, -1.0).astype(np.float32)
        sub[np.arange(m), np.arange(m) % 8] = 1.0
    return parents, pf, sub


# Flow-sampler runs whose PIXAL3D_FLOW_NONFINITE_TRACE lines the compiled
# reference wrote to tests/golden/flow_trace_lines.json (make_trace_golden.py).
# name: (steps, [sigma_min, rescale_t, strength, rescale, interval_min, interval_max], record)
TRACE_CASES = {
    "guided_rescale": (2, [1e-5, 3.0, 7.5, 0.7, 0.0, 1.0], True),
    "unguided": (2, [1e-5, 1.0, 1.0, 0.0, 0.0, 1.0], True),
    "blend_overflow": (2, [1e-5, 1.0, 3.0, 0.0, 0.0, 1.0], False),
}


def overflow_velocity(state, t_model, conditional):
    """+-3e38 velocities: their CFG blend overflows to infinity."""
    return np.full_like(state, 3e38 if conditional else -3e38)


def capture_stderr(fn):
    """Run fn with file descriptor 2 redirected to a file; -> (result, text)."""
    sys.stderr.flush()
    saved = os.dup(2)
    with tempfile.TemporaryFile(mode="w+b") as tmp:
        os.dup2(tmp.fileno(), 2)
        try:
            result = fn()
        finally:
            os.dup2(saved, 2)
            os.close(saved)
        tmp.seek(0)
        return result, tmp.read().decode()
