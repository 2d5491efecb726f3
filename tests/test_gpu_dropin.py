"""The C++ drop-in (include/pixal3d/sparse.h and sparse_transformer.h on
libpxs.so), called through the same C shim that drives the compiled reference.

Each test runs the reference's own inputs through the drop-in and compares
with what the reference produced for them:
* the reference KAT binaries' printed outputs (tests/golden/*.json,
  tests/sparse_numeric_fixture.cpp and tests/sparse_transformer_numeric_fixture.cpp);
* the compiled reference library's outputs on seeded inputs
  (tests/golden/ref_vectors.npz);
* the oracle for inputs the fixtures do not cover (other factors, aliasing).
fp32 results must be within 1e-5 of the reference, as max|g - r| / max|r|;
coordinates and error messages must match exactly.
"""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
import workloads as W
from fixtures import block_kat, kat_inputs
from gpu_common import FP32_TOL, max_rel

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def di():
    return O.DropIn()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


@pytest.fixture(scope="module")
def vec():
    return dict(np.load(GOLD / "ref_vectors.npz"))


def close(got, ref, what, tol=FP32_TOL):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    e = max_rel(got, ref)
    assert e <= tol, f"{what}: max rel error {e:.3e} > {tol}"


def test_dropin_reference_kat(di):
    """The 11 outputs of tests/sparse_numeric_fixture.cpp."""
    gold = {k: np.array(v, np.float32) for k, v in
            json.loads((GOLD / "sparse_numeric_fixture.json").read_text()).items()}
    a = kat_inputs()
    c = a["coords"]
    print("dropin KAT: 10 points, 2 batches", flush=True)
    t = di.sparse(c, a["feats"], 2, (4, 4, 4))
    close(di.linear(t, a["lw"], a["lb"]).read()[1].ravel(), gold["sparse_linear_output"], "linear")
    close(di.subm_conv3d(t, a["cw"], a["cb"]).read()[1].ravel(), gold["sparse_conv_output"], "conv")
    close(di.layer_norm(t, 1e-5, [0.8, 1.1, 1.4], [-0.2, 0.03, 0.17]).read()[1].ravel(),
          gold["sparse_norm_output"], "layer norm")
    dco, dfo = di.downsample_mean(t, 2).read()
    np.testing.assert_array_equal(dco.ravel().astype(np.float32), gold["sparse_downsample_coords"])
    close(dfo.ravel(), gold["sparse_downsample_output"], "downsample")
    q = di.sparse(c, a["q"], 2, (4, 4, 4))
    k = di.sparse(c, a["k"], 2, (4, 4, 4))
    v = di.sparse(c, a["v"], 2, (4, 4, 4))
    close(di.sdpa(q, k, v, 2, 6, 0.37).read()[1].ravel(), gold["sparse_attention_output"], "sdpa")
    close(di.rope(q, 2, 6).read()[1].ravel(), gold["sparse_rope_output"], "rope")
    close(di.mh_rms_norm(q, 2, 6, a["rg"]).read()[1].ravel(), gold["sparse_rms_output"], "rms")
    ck = di.varlen([0, 3, 5], a["ck"])
    cv = di.varlen([0, 3, 5], a["cv"])
    close(di.cross_attention(q, ck, cv, 2, 6, 0.29).read()[1].ravel(),
          gold["sparse_cross_output"], "cross attention")
    p = di.sparse(a["pc"], a["pf"], 2, (2, 2, 2))
    sub = di.sparse(a["pc"], a["sub"], 2, (2, 2, 2))
    sco, sfo = di.channel_to_spatial(p, 2, sub).read()
    np.testing.assert_array_equal(sco.ravel().astype(np.float32),
                                  gold["sparse_channel_to_spatial_coords"])
    close(sfo.ravel(), gold["sparse_channel_to_spatial_output"], "channel to spatial")


def block_handles(di, k):
    t = di.sparse(k["coords"], k["x"], 2, (4, 4, 4))
    ctx = di.varlen([0, 3, 5], k["ctx"])
    proj = di.sparse(k["coords"], k["proj"], 2, (4, 4, 4))
    return t, ctx, proj


def test_dropin_reference_block_kat(di):
    """tests/sparse_transformer_numeric_fixture.cpp: one block, C=12, 2 heads x 6."""
    gold = np.array(json.loads((GOLD / "sparse_transformer_fixture.json").read_text())
                    ["sparse_transformer_output"], np.float32)
    k = block_kat()
    t, ctx, proj = block_handles(di, k)
    out = di.transformer_block(t, k["tmod"], ctx, k["cfg_i"], k["cfg_f"], k["weights"],
                               projected=proj)
    coords, feats = out.read()
    np.testing.assert_array_equal(coords, k["coords"])
    close(feats.ravel(), gold, "block KAT")


# The binary-fraction fixtures of tests/sparse_linear_cuda_benchmark.cpp:53-57
# (points, input and output channels, batch size, spatial extent, bias) with
# the inputs of its fill_fixture_values (:200-216) and coordinates of its
# make_coords (:166-186): every product and partial sum is exact, so the
# drop-in's sparse_linear must equal the compiled reference bit for bit
# whatever its summation order (the 4-channel case runs the dense MFMA
# kernel, the others the gather-GEMM fallback).
@pytest.mark.parametrize("points,cin,cout,batch,spatial,with_bias", [
    (11, 3, 5, 2, 8, True), (13, 4, 4, 2, 8, False), (17, 5, 2, 1, 8, True)])
def test_dropin_linear_binary_fixtures(di, points, cin, cout, batch, spatial, with_bias):
    per = (points + batch - 1) // batch
    p = np.arange(points)
    local = p % per
    coords = np.stack([p // per, local % spatial, (local % (spatial * spatial)) // spatial,
                       local // (spatial * spatial)], 1).astype(np.int32)
    x = (0.125 * ((np.arange(points * cin) % 13) + 1)).astype(np.float32).reshape(points, cin)
    w = (0.0625 * ((np.arange(cout * cin) % 11) + 1)).astype(np.float32).reshape(cout, cin)
    b = (0.25 * (np.arange(cout) + 1)).astype(np.float32) if with_bias else np.zeros(cout, np.float32)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    shape = (spatial, spatial, spatial)
    got = di.linear(di.sparse(coords, x, batch, shape), w, b).read()
    np.testing.assert_array_equal(got[0], coords)
    np.testing.assert_array_equal(got[1], want.astype(np.float32))
    if O.REF_LIB.exists():  # the compiled reference, where it was built
        ref = O.Reference()
        np.testing.assert_array_equal(got[1], ref.linear(ref.sparse(coords, x, batch, shape), w, b).read()[1])


def test_dropin_block_alias_safe(di):
    """Callers pass the same tensor as input and output (src/slat_flow.cpp:238-241)."""
    gold = np.array(json.loads((GOLD / "sparse_transformer_fixture.json").read_text())
                    ["sparse_transformer_output"], np.float32)
    k = block_kat()
    t, ctx, proj = block_handles(di, k)
    di.transformer_block(t, k["tmod"], ctx, k["cfg_i"], k["cfg_f"], k["weights"],
                         projected=proj, out=t)
    close(t.read()[1].ravel(), gold, "block aliased")
    lin = di.linear(t, np.eye(12, dtype=np.float32), np.zeros(12, np.float32), out=t)
    close(lin.read()[1].ravel(), gold, "linear aliased")


def test_dropin_reference_vectors(di, vec):
    """Seeded inputs and the compiled reference library's outputs."""
    v = vec
    print("dropin vectors: conv/linear/norm/rope/attention/downsample/c2s", flush=True)
    t = di.sparse(v["conv_coords"], v["conv_feats"], 2, (16, 16, 16))
    close(di.subm_conv3d(t, v["conv_w"], v["conv_b"]).read()[1], v["conv_out"], "conv")
    tl = di.sparse(v["lin_coords"], v["lin_x"], 1, (10, 10, 10))
    close(di.linear(tl, v["lin_w"], v["lin_b"]).read()[1], v["lin_out"], "linear")
    vl = di.varlen(v["vlin_offsets"], v["lin_x"])
    close(di.varlen_linear(vl, v["lin_w"], v["lin_b"]).read(), v["vlin_out"], "varlen linear")
    tn = di.sparse(v["lin_coords"], v["ln_x"], 1, (10, 10, 10))
    close(di.layer_norm(tn, 1e-6, v["ln_g"], v["ln_b"]).read()[1], v["ln_out_affine"], "ln affine")
    close(di.layer_norm(tn, 1e-5).read()[1], v["ln_out_plain"], "ln plain")
    tr = di.sparse(v["rms_coords"], v["rms_x"], 1, (64, 64, 64))
    close(di.mh_rms_norm(tr, 4, 64, v["rms_g"]).read()[1], v["rms_out"], "rms")
    close(di.rope(tr, 4, 64).read()[1], v["rope_out"], "rope")
    vr = di.varlen(np.array([0, v["rms_x"].shape[0]]), v["rms_x"])
    close(di.varlen_mh_rms_norm(vr, 4, 64, v["rms_g"]).read(), v["vrms_out"], "varlen rms")
    shp = (16, 16, 16)
    q = di.sparse(v["attn_coords"], v["attn_q"], 3, shp)
    k = di.sparse(v["attn_coords"], v["attn_k"], 3, shp)
    vv = di.sparse(v["attn_coords"], v["attn_v"], 3, shp)
    close(di.sdpa(q, k, vv, 2, 16, 0.25).read()[1], v["attn_out"], "sdpa")
    ck = di.varlen(v["cross_offsets"], v["cross_k"])
    cv = di.varlen(v["cross_offsets"], v["cross_v"])
    close(di.cross_attention(q, ck, cv, 2, 16, 0.25).read()[1], v["cross_out"], "cross")
    td = di.sparse(v["ds_coords"], v["ds_feats"], 2, (16, 16, 16))
    dco, dfo = di.downsample_mean(td, 2).read()
    np.testing.assert_array_equal(dco, v["ds_out_coords"])
    close(dfo, v["ds_out_feats"], "downsample")
    sub = di.sparse(v["ds_coords"], v["c2s_sub"], 2, (16, 16, 16))
    co, cf = di.channel_to_spatial(td, 2, sub).read()
    np.testing.assert_array_equal(co, v["c2s_out_coords"])
    close(cf, v["c2s_out_feats"], "c2s subdivided")
    co, cf = di.channel_to_spatial(td, 2).read()
    np.testing.assert_array_equal(co, v["c2s_all_coords"])
    close(cf, v["c2s_all_feats"], "c2s all")


@pytest.mark.parametrize("proj", [True, False])
def test_dropin_block_vectors(di, vec, proj):
    v = vec
    ws = [v[f"blk_w{i}"] for i in range(23)]
    shp = (16, 16, 16)
    t = di.sparse(v["blk_coords"], v["blk_x"], 2, shp)
    ctx = di.varlen(v["blk_ctx_off"], v["blk_ctx"])
    cfg_i = [32, 4, 64, 6, 5, 1, 1, 1, 1 if proj else 0]
    p = di.sparse(v["blk_coords"], v["blk_proj"], 2, shp) if proj else None
    out = di.transformer_block(t, v["blk_tmod"], ctx, cfg_i, [1e-6, 1.0, 10000.0], ws,
                               projected=p)
    close(out.read()[1], v["blk_out"] if proj else v["blk_out_noproj"], f"block proj={proj}")


@pytest.mark.parametrize("factor", [1, 3])
def test_dropin_other_factors(di, orc, factor):
    """Factors the fixtures do not cover, against the oracle (which follows
    src/sparse.cpp:536-702 for any factor)."""
    coords = W.shell_coords(18, [[(4.0, 8.0)], [(3.0, 7.0)]], 21)
    n = coords.shape[0]
    cc = factor ** 3
    x = W.normal(21, n * 2 * cc, 1).reshape(n, 2 * cc)
    t = di.sparse(coords, x, 2, (18, 18, 18))
    dco, dfo = di.downsample_mean(t, factor).read()
    rco, rfo = orc.downsample_mean(coords, x, factor)
    np.testing.assert_array_equal(dco, rco)
    close(dfo, rfo, f"downsample f={factor}")
    sub = (W.uniform(21, n * cc, 2) > 0.4).astype(np.float32).reshape(n, cc)
    co, cf = di.channel_to_spatial(t, factor, di.sparse(coords, sub, 2, (18, 18, 18))).read()
    rco, rcf = orc.channel_to_spatial(coords, x, factor, sub)
    np.testing.assert_array_equal(co, rco)
    close(cf, rcf, f"c2s f={factor}")


def test_dropin_conv_full_size(di):
    """The 64^3 fp32 SubMConv3d workload (about 16k voxels, 64 -> 64) against the
    reference's sampled output rows (tests/golden/ref_conv_64.json)."""
    gold = json.loads((GOLD / "ref_conv_64.json").read_text())
    wl = W.conv_fp32_64()
    t = di.sparse(wl["coords"], wl["feats"], 1, wl["shape"])
    out = di.subm_conv3d(t, wl["weight"], wl["bias"]).read()[1]
    assert out.shape[0] == gold["points"]
    close(out[np.array(gold["rows"])], np.array(gold["values"], np.float32), "conv 64^3")


# ---- error behaviour ------------------------------------------------------------------

def expect_error(fn, message):
    with pytest.raises(O.ReferenceError) as e:
        fn()
    assert str(e.value) == message


def test_dropin_validation_messages(di):
    """SparseTensorF32::valid's messages (src/sparse.cpp:241-335), first failing row first."""
    c = np.array([[0, 0, 0, 0], [0, 1, 0, 0], [1, 0, 0, 0]], np.int32)
    f = np.ones((3, 2), np.float32)
    ok, msg = di.valid(di.sparse(c, f, 2, (4, 4, 4)))
    assert ok and msg == ""
    cases = [
        (di.sparse(c, f, 0, (4, 4, 4)), "invalid sparse tensor shape"),
        (di.sparse(c + [[0, 4, 0, 0]] * 3, f, 2, (4, 4, 4)), "sparse coordinate is outside its shape"),
        (di.sparse(np.array([[0, 0, 0, 0], [0, 0, 0, 0], [1, 0, 0, 0]], np.int32), f, 2, (4, 4, 4)),
         "sparse coordinates contain a duplicate point"),
        (di.sparse(c[::-1].copy(), f, 2, (4, 4, 4)), "sparse coordinates must be contiguous by batch"),
        (di.sparse(c, np.array([[1, 1], [1, np.nan], [1, 1]], np.float32), 2, (4, 4, 4)),
         "sparse features contain a non-finite value"),
    ]
    for t, message in cases:
        ok, msg = di.valid(t)
        assert not ok and msg == message
    # A duplicate after a non-finite row: the earlier row's error wins.
    c2 = np.array([[0, 0, 0, 0], [0, 1, 0, 0], [0, 1, 0, 0]], np.int32)
    ok, msg = di.valid(di.sparse(c2, np.array([[1, 1], [np.inf, 1], [1, 1]], np.float32), 1,
                                 (4, 4, 4)))
    assert msg == "sparse features contain a non-finite value"
    ok, msg = di.varlen_valid(di.varlen([0, 1, 3], np.array([[1.0], [2.0], [np.nan]], np.float32)))
    assert msg == "variable-length tensor contains a non-finite value"


def test_dropin_argument_errors(di):
    c = np.array([[0, 0, 0, 0], [1, 0, 0, 0]], np.int32)
    t = di.sparse(c, np.ones((2, 4), np.float32), 2, (4, 4, 4))
    w = np.ones((3, 4), np.float32)
    expect_error(lambda: di.linear(t, w, np.ones(3, np.float32)[:0]),
                 "sparse output channel count must be positive")
    expect_error(lambda: di.layer_norm(t, 0.0), "sparse layer norm epsilon must be finite and positive")
    expect_error(lambda: di.layer_norm(t, 1e-5, np.ones(4, np.float32), None),
                 "sparse layer norm affine parameters must be both null or non-null")
    expect_error(lambda: di.downsample_mean(t, 0), "sparse downsample factor must be positive")
    expect_error(lambda: di.channel_to_spatial(t, 2),
                 "sparse channel-to-spatial channels are not divisible by factor^3")
    expect_error(lambda: di.rope(t, 2, 3), "sparse RoPE head dimensions are invalid")
    expect_error(lambda: di.rope(t, 2, 2, 0.0), "sparse RoPE frequencies must be finite and positive")
    expect_error(lambda: di.sdpa(t, t, t, 3, 2, 0.5),
                 "sparse attention channel/head dimensions are invalid")
    expect_error(lambda: di.sdpa(t, t, t, 2, 2, -1.0),
                 "sparse attention scale must be finite and positive")
    only0 = di.sparse(c[:1], np.ones((1, 4), np.float32), 2, (4, 4, 4))
    expect_error(lambda: di.sdpa(t, only0, only0, 2, 2, 0.5),
                 "sparse attention has no keys or mismatched key/value rows")
    kv = di.varlen([0, 2, 2], np.ones((2, 4), np.float32))
    expect_error(lambda: di.cross_attention(t, kv, kv, 2, 2, 0.5),
                 "sparse cross-attention has an empty key sequence")
    kv2 = di.varlen([0, 1, 2], np.ones((2, 4), np.float32))
    expect_error(lambda: di.cross_attention(t, kv2, kv2, 2, 2, 0.0),
                 "sparse cross-attention scale must be finite and positive")
    expect_error(lambda: di.mh_rms_norm(t, 3, 2, np.ones(4, np.float32)),
                 "sparse RMS norm head dimensions are invalid")


def test_dropin_attention_wide_heads(di, orc):
    """sparse_scaled_dot_product_attention and sparse_cross_attention with
    heads wider than 64 (128-wide q/k, 96-wide v) against the oracle, which
    follows src/sparse.cpp:704-859."""
    coords = W.shell_coords(12, [[(3.0, 5.0)], [(2.0, 4.0)]], 67)
    n = coords.shape[0]
    heads, hd, vd = 2, 128, 96
    q = W.normal(67, n * heads * hd, 1).reshape(n, heads * hd)
    k = W.normal(67, n * heads * hd, 2).reshape(n, heads * hd)
    v = W.normal(67, n * heads * vd, 3).reshape(n, heads * vd)
    shp = (12, 12, 12)
    out = di.sdpa(di.sparse(coords, q, 2, shp), di.sparse(coords, k, 2, shp),
                  di.sparse(coords, v, 2, shp), heads, hd, 0.09).read()[1]
    cu = orc.batch_cu_seqlens(coords, 2)
    close(out, orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(0.09)), "sdpa wide")
    off = np.array([0, 7, 20], np.int64)
    ck = W.normal(67, 20 * heads * hd, 4).reshape(20, heads * hd)
    cv = W.normal(67, 20 * heads * vd, 5).reshape(20, heads * vd)
    out = di.cross_attention(di.sparse(coords, q, 2, shp), di.varlen(off, ck), di.varlen(off, cv),
                             heads, hd, 0.09).read()[1]
    close(out, orc.varlen_attention(q, ck, cv, cu, off, heads, hd, np.float32(0.09)), "cross wide")
