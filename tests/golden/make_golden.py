#!/usr/bin/env python3
"""Write the golden vectors that pin the oracle to the compiled reference.

Runs in the build container only (it needs /root/reference to build
oracle/_ref).  It writes:

* sparse_numeric_fixture.json       - the 11 outputs printed by the reference's
  own KAT binary tests/sparse_numeric_fixture.cpp (built from its sources into
  oracle/_ref/sparse_fixture), parsed as in scripts/compare_sparse.py:17-36.
* sparse_transformer_fixture.json   - the output of the reference's
  tests/sparse_transformer_numeric_fixture.cpp.
* ref_vectors.npz                   - seeded inputs and the reference library's
  outputs (oracle/_ref/libpixal3d_ref.so) for every primitive at small sizes.
* ref_conv_64.json                  - the SHA-256 and sampled rows of the
  reference sparse_submanifold_conv3d on the 64^3 fp32 workload.

Usage:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "pixal3d.cpp_amd" / "python"))

import oracle as O  # noqa: E402
import workloads as W  # noqa: E402

OUT = Path(__file__).resolve().parent


def parse_fixture(text: str) -> dict:
    out = {}
    for line in text.splitlines():
        fields = line.split()
        if len(fields) < 2:
            continue
        count = int(fields[1])
        values = [float(v) for v in fields[2:]]
        assert len(values) == count, fields[0]
        out[fields[0]] = values
    return out


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<f4").tobytes()).hexdigest()


def small_shell(grid, items, seed):
    return W.shell_coords(grid, items, seed)


def main() -> int:
    O.build_oracle()
    ref = O.Reference()
    ref.set_threads(4)

    text = subprocess.run([str(ROOT / "oracle" / "_ref" / "sparse_fixture")], check=True,
                          capture_output=True, text=True).stdout
    kat = parse_fixture(text)
    assert len(kat) == 11
    (OUT / "sparse_numeric_fixture.json").write_text(json.dumps(kat, indent=0) + "\n")

    text = subprocess.run([str(ROOT / "oracle" / "_ref" / "sparse_transformer_fixture")],
                          check=True, capture_output=True, text=True).stdout
    (OUT / "sparse_transformer_fixture.json").write_text(json.dumps(parse_fixture(text)) + "\n")

    v = {}
    # Submanifold conv on a 2-item shell set on 16^3.
    coords = small_shell(16, [[(4.0, 7.0)], [(3.0, 6.0), (5.0, 7.0)]], 11)
    n = coords.shape[0]
    feats = W.normal(11, n * 8, 1).reshape(n, 8)
    weight = W.normal(11, 27 * 12 * 8, 2, std=0.2).reshape(27, 12, 8)
    bias = W.normal(11, 12, 3)
    t = ref.sparse(coords, feats, 2, (16, 16, 16))
    v["conv_coords"], v["conv_feats"], v["conv_w"], v["conv_b"] = coords, feats, weight, bias
    v["conv_out"] = ref.subm_conv3d(t, weight, bias).read()[1]

    # Linear, varlen linear.
    x = W.normal(12, 200 * 24, 1).reshape(200, 24)
    lw = W.normal(12, 40 * 24, 2, std=0.3).reshape(40, 24)
    lb = W.normal(12, 40, 3)
    lc = np.stack([np.zeros(200, np.int32), np.arange(200) // 100, (np.arange(200) // 10) % 10,
                   np.arange(200) % 10], axis=1).astype(np.int32)
    v["lin_x"], v["lin_w"], v["lin_b"], v["lin_coords"] = x, lw, lb, lc
    v["lin_out"] = ref.linear(ref.sparse(lc, x, 1, (10, 10, 10)), lw, lb).read()[1]
    offs = np.array([0, 70, 70, 200], np.int64)
    v["vlin_offsets"] = offs
    v["vlin_out"] = ref.varlen_linear(ref.varlen(offs, x), lw, lb).read()

    # Layer norm (affine and plain).
    g, b = W.normal(13, 24, 1), W.normal(13, 24, 2)
    xs = x * 3.0 + 0.5
    v["ln_x"], v["ln_g"], v["ln_b"] = xs, g, b
    tl = ref.sparse(lc, xs, 1, (10, 10, 10))
    v["ln_out_affine"] = ref.layer_norm(tl, 1e-6, g, b).read()[1]
    v["ln_out_plain"] = ref.layer_norm(tl, 1e-5).read()[1]

    # Multi-head RMS norm and RoPE (4 heads x 64, coordinates up to 63).
    rc = small_shell(64, [[(16.0, 30.0)]], 14)[::160].copy()
    m = rc.shape[0]
    rx = W.normal(14, m * 256, 1).reshape(m, 256)
    rg = np.abs(W.normal(14, 256, 2)) + 0.5
    tr = ref.sparse(rc, rx, 1, (64, 64, 64))
    v["rms_coords"], v["rms_x"], v["rms_g"] = rc, rx, rg
    v["rms_out"] = ref.mh_rms_norm(tr, 4, 64, rg).read()[1]
    v["rope_out"] = ref.rope(tr, 4, 64, 1.0, 10000.0).read()[1]
    v["vrms_out"] = ref.varlen_mh_rms_norm(ref.varlen(np.array([0, m], np.int64), rx), 4, 64,
                                           rg).read()

    # Varlen self-attention: 3 batches of 37, 64, 5 rows, 2 heads x 16.
    lens = [37, 64, 5]
    ac = np.concatenate([np.stack([np.full(L, bi), np.arange(L) // 16, np.arange(L) % 16,
                                   np.zeros(L)], axis=1) for bi, L in enumerate(lens)])
    ac = ac.astype(np.int32)
    na = ac.shape[0]
    q = W.normal(15, na * 32, 1).reshape(na, 32)
    k = W.normal(15, na * 32, 2).reshape(na, 32)
    vv = W.normal(15, na * 32, 3).reshape(na, 32)
    sc = 0.25
    v["attn_coords"], v["attn_q"], v["attn_k"], v["attn_v"] = ac, q, k, vv
    shp = (16, 16, 16)
    v["attn_out"] = ref.sdpa(ref.sparse(ac, q, 3, shp), ref.sparse(ac, k, 3, shp),
                             ref.sparse(ac, vv, 3, shp), 2, 16, sc).read()[1]
    # Cross attention against 3 context sequences of 4, 9, 1 tokens.
    coffs = np.array([0, 4, 13, 14], np.int64)
    ck = W.normal(15, 14 * 32, 4).reshape(14, 32)
    cv = W.normal(15, 14 * 32, 5).reshape(14, 32)
    v["cross_offsets"], v["cross_k"], v["cross_v"] = coffs, ck, cv
    v["cross_out"] = ref.cross_attention(ref.sparse(ac, q, 3, shp), ref.varlen(coffs, ck),
                                         ref.varlen(coffs, cv), 2, 16, sc).read()[1]

    # Downsample mean (factor 2) and channel-to-spatial with a subdivision.
    dc = small_shell(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 16)
    nd = dc.shape[0]
    df = W.normal(16, nd * 16, 1).reshape(nd, 16)
    td = ref.sparse(dc, df, 2, (16, 16, 16))
    dco, dfo = ref.downsample_mean(td, 2).read()
    v["ds_coords"], v["ds_feats"], v["ds_out_coords"], v["ds_out_feats"] = dc, df, dco, dfo
    sub = (W.uniform(16, nd * 8, 2) > 0.5).astype(np.float32).reshape(nd, 8)
    c2o, c2f = ref.channel_to_spatial(td, 2, ref.sparse(dc, sub, 2, (16, 16, 16))).read()
    v["c2s_sub"], v["c2s_out_coords"], v["c2s_out_feats"] = sub, c2o, c2f
    c2o_all, c2f_all = ref.channel_to_spatial(td, 2).read()
    v["c2s_all_coords"], v["c2s_all_feats"] = c2o_all, c2f_all

    # One transformer block: C=32, 4 heads x 8, MLP 64, context 6 channels,
    # projection 5 channels, 2 batches.
    bc = small_shell(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 17)
    nb = bc.shape[0]
    Cc, H, Mh, CC, PC = 32, 4, 64, 6, 5
    shapes = [6 * Cc, 3 * Cc * Cc, 3 * Cc, Cc, Cc, Cc * Cc, Cc, Cc, Cc, Cc * Cc, Cc, 2 * Cc * CC,
              2 * Cc, Cc, Cc, Cc * Cc, Cc, Cc * PC, Cc, Mh * Cc, Mh, Cc * Mh, Cc]
    ws = []
    for i, s in enumerate(shapes):
        w = W.normal(17, s, 10 + i, std=0.15)
        if i in (3, 4, 7, 13, 14):  # gammas / norm2 weight
            w = np.abs(w) + 0.5
        ws.append(w)
    bx = W.normal(17, nb * Cc, 1).reshape(nb, Cc)
    tmod = W.normal(17, 2 * 6 * Cc, 2, std=0.1)
    ctx_off = np.array([0, 3, 7], np.int64)
    ctx = W.normal(17, 7 * CC, 3).reshape(7, CC)
    proj = W.normal(17, nb * PC, 4).reshape(nb, PC)
    cfg_i = [Cc, H, Mh, CC, PC, 1, 1, 1, 1]
    cfg_f = [1e-6, 1.0, 10000.0]
    out = ref.transformer_block(ref.sparse(bc, bx, 2, (16, 16, 16)), tmod, ref.varlen(ctx_off, ctx),
                                cfg_i, cfg_f, ws, projected=ref.sparse(bc, proj, 2, (16, 16, 16)))
    v["blk_coords"], v["blk_x"], v["blk_tmod"], v["blk_ctx"], v["blk_ctx_off"] = bc, bx, tmod, ctx, ctx_off
    v["blk_proj"] = proj
    for i, w in enumerate(ws):
        v[f"blk_w{i}"] = w
    v["blk_out"] = out.read()[1]
    # Same block with no projection and cross mode (as the flow uses it).
    cfg_i2 = [Cc, H, Mh, CC, PC, 1, 1, 1, 0]
    v["blk_out_noproj"] = ref.transformer_block(ref.sparse(bc, bx, 2, (16, 16, 16)), tmod,
                                                ref.varlen(ctx_off, ctx), cfg_i2, cfg_f,
                                                ws).read()[1]

    # Timestep embedding MLP (256 -> 32).
    ts = np.array([0.0, 137.5, 999.0], np.float32)
    tw0 = W.normal(18, 32 * 256, 1, std=0.05).reshape(32, 256)
    tb0 = W.normal(18, 32, 2)
    tw2 = W.normal(18, 32 * 32, 3, std=0.1).reshape(32, 32)
    tb2 = W.normal(18, 32, 4)
    v["temb_t"], v["temb_w0"], v["temb_b0"], v["temb_w2"], v["temb_b2"] = ts, tw0, tb0, tw2, tb2
    v["temb_out"] = ref.timestep_embed_mlp(ts, 32, 256, tw0, tb0, tw2, tb2)
    v["temb_freq"] = ref.timestep_embedding(ts, 256)

    np.savez_compressed(OUT / "ref_vectors.npz", **v)

    # Full-size fp32 conv (64^3, ~16k voxels, 64 -> 64): hash + samples.
    wl = W.conv_fp32_64()
    t = ref.sparse(wl["coords"], wl["feats"], 1, wl["shape"])
    cout = ref.subm_conv3d(t, wl["weight"], wl["bias"]).read()[1]
    rows = np.linspace(0, cout.shape[0] - 1, 64).astype(np.int64)
    (OUT / "ref_conv_64.json").write_text(json.dumps({
        "points": int(cout.shape[0]),
        "sha256": sha(cout),
        "rows": rows.tolist(),
        "values": cout[rows].tolist(),
    }) + "\n")
    print("golden vectors written to", OUT)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
