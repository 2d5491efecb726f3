"""GPU parity: submanifold conv (fp32 and bf16 MFMA), stride-2 conv, downsample."""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
import workloads as W
from gpu_common import assert_bf16, assert_fp32, host, t32, tbf, ti32

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def px():
    import pxs
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


def run_conv(px, coords, x, w, b, dtype):
    c = ti32(coords)
    nbr, masks = px.neighbor_map(c)
    conv = tbf if dtype == "bf16" else t32
    return px.subm_conv3d(conv(x), conv(w), t32(b), nbr, masks)


def test_conv_fp32_reference_kat(px):
    """The reference's own KAT (tests/sparse_numeric_fixture.cpp): 10 points, 3 -> 4."""
    from fixtures import kat_inputs

    a = kat_inputs()
    gold = np.array(json.loads((GOLD / "sparse_numeric_fixture.json").read_text())
                    ["sparse_conv_output"], np.float32)
    y = run_conv(px, a["coords"], a["feats"], a["cw"], a["cb"], "f32")
    assert_fp32(host(y).ravel(), gold, what="KAT conv")


def test_conv_fp32_64_full_size(px, orc):
    wl = W.conv_fp32_64()
    print(f"[conv fp32 64^3] n={wl['coords'].shape[0]}", flush=True)
    y = run_conv(px, wl["coords"], wl["feats"], wl["weight"], wl["bias"], "f32")
    ref = orc.subm_conv3d(wl["coords"], wl["feats"], wl["weight"], wl["bias"])
    assert_fp32(host(y), ref, what="conv fp32 64^3")


@pytest.mark.parametrize("cin,cout", [(8, 12), (3, 4), (64, 64), (96, 160), (128, 128)])
def test_conv_fp32_shapes(px, orc, cin, cout):
    coords = W.shell_coords(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 41)
    n = coords.shape[0]
    x = W.normal(41, n * cin, 1).reshape(n, cin)
    w = W.normal(41, 27 * cout * cin, 2, std=0.1).reshape(27, cout, cin)
    b = W.normal(41, cout, 3)
    print(f"[conv fp32] cin={cin} cout={cout}", flush=True)
    y = run_conv(px, coords, x, w, b, "f32")
    assert_fp32(host(y), orc.subm_conv3d(coords, x, w, b), what=f"conv {cin}->{cout}")


@pytest.mark.parametrize("cin,cout", [(128, 128), (256, 256), (64, 48), (40, 24)])
def test_conv_bf16_vs_oracle(px, orc, cin, cout):
    coords = W.shell_coords(24, [[(6.0, 10.0)], [(5.0, 9.0)]], 42)
    n = coords.shape[0]
    x = W.bf16_round(W.normal(42, n * cin, 1).reshape(n, cin))
    w = W.bf16_round(W.normal(42, 27 * cout * cin, 2, std=float(np.sqrt(2 / (27 * cin)))).reshape(27, cout, cin))
    b = W.normal(42, cout, 3, std=0.1)
    print(f"[conv bf16] cin={cin} cout={cout} n={n}", flush=True)
    y = run_conv(px, coords, x, w, b, "bf16")
    assert_bf16(host(y), orc.subm_conv3d(coords, x, w, b), what=f"bf16 conv {cin}->{cout}")


def test_conv_bf16_unet_full_size_sampled_rows(px):
    """The U-Net stage's op A at full size (~160k voxels, 128 -> 128): sampled output rows
    recomputed in float64 from the GPU neighbor map (itself bit-exact vs the
    oracle), plus the centre-identity property on every row."""
    wl = W.unet_stage_128()
    coords, x, w = wl["coords"], wl["feats"], wl["w_a"]
    n = coords.shape[0]
    print(f"[conv bf16 unet A] n={n}", flush=True)
    c = ti32(coords)
    nbr, masks = px.neighbor_map(c)
    xb, wb = tbf(x), tbf(w)
    y = host(px.subm_conv3d(xb, wb, t32(wl["b_a"]), nbr, masks))
    idx = nbr.cpu().numpy()
    rows = np.linspace(0, n - 1, 1500).astype(np.int64)
    ref = np.zeros((rows.size, 128))
    for k in range(27):
        src = idx[k, rows]
        ok = src != n
        ref[ok] += x[src[ok]].astype(np.float64) @ w[k].astype(np.float64).T
    assert_bf16(y[rows], ref, what="unet A sampled")
    # centre identity: W_13 = I, others 0, bias 0 -> y == x exactly (bf16 products by 1.0)
    eye = np.zeros((27, 128, 128), np.float32)
    eye[13] = np.eye(128, dtype=np.float32)
    yi = px.subm_conv3d(xb, tbf(eye), t32(np.zeros(128)), nbr, masks)
    np.testing.assert_array_equal(host(yi), host(xb))


def plane_spans(idx, n, bm=128):
    """Per (tile of bm rows, x-plane) span of the input rows the plane's nine
    offsets read."""
    spans = []
    for t in range(0, n, bm):
        sub = idx[:, t:t + bm]
        for kd in range(3):
            v = sub[9 * kd:9 * kd + 9].ravel()
            v = v[v != n]
            spans.append(int(v.max() - v.min() + 1) if v.size else 0)
    return np.array(spans)


@pytest.mark.parametrize("masks", [True, False])
def test_conv_bf16_staged_and_gathered_planes(px, orc, masks):
    """A 3 x 72 x 72 slab plus a shell in a second batch: dense tiles whose
    planes read rows hundreds apart next to thin shell tiles; both must agree
    with the oracle, with and without the neighbour masks."""
    slab = np.array([(0, x, y, z) for x in range(3) for y in range(72) for z in range(72)],
                    np.int32)
    shell = W.shell_coords(24, [[(6.0, 10.0)]], 45)
    shell[:, 0] = 1
    coords = np.concatenate([slab, shell])
    n = coords.shape[0]
    spans = plane_spans(orc.neighbor_map(coords), n)
    assert (spans > 256).any() and ((spans > 0) & (spans <= 256)).any()
    cin, cout = 64, 128
    x = W.bf16_round(W.normal(45, n * cin, 1).reshape(n, cin))
    w = W.bf16_round(W.normal(45, 27 * cout * cin, 2, std=float(np.sqrt(2 / (27 * cin))))
                     .reshape(27, cout, cin))
    b = W.normal(45, cout, 3, std=0.1)
    print(f"[conv bf16 slab] n={n} masks={masks}", flush=True)
    nbr, mk = px.neighbor_map(ti32(coords))
    y = px.subm_conv3d(tbf(x), tbf(w), t32(b), nbr, mk if masks else None)
    assert_bf16(host(y), orc.subm_conv3d(coords, x, w, b), what="bf16 conv slab")


def test_conv_masks_optional(px, orc):
    coords = W.shell_coords(16, [[(4.0, 7.0)]], 43)
    n = coords.shape[0]
    x = W.normal(43, n * 32, 1).reshape(n, 32)
    w = W.normal(43, 27 * 32 * 32, 2, std=0.1).reshape(27, 32, 32)
    b = W.normal(43, 32, 3)
    nbr, masks = px.neighbor_map(ti32(coords))
    y1 = px.subm_conv3d(t32(x), t32(w), t32(b), nbr, masks)
    y2 = px.subm_conv3d(t32(x), t32(w), t32(b), nbr, None)
    np.testing.assert_array_equal(host(y1), host(y2))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_strided_conv_s2(px, orc, dtype):
    coords = W.shell_coords(24, [[(6.0, 10.0)], [(5.0, 9.0)]], 44)
    n = coords.shape[0]
    cin, cout = 64, 96
    x = W.bf16_round(W.normal(44, n * cin, 1).reshape(n, cin))
    w = W.bf16_round(W.normal(44, 8 * cout * cin, 2, std=float(np.sqrt(2 / (8 * cin)))).reshape(8, cout, cin))
    b = W.normal(44, cout, 3, std=0.1)
    print(f"[conv s2] dtype={dtype}", flush=True)
    oc, child, m = px.downsample_s2(ti32(coords), 2, (24, 24, 24))
    conv = tbf if dtype == "bf16" else t32
    y = host(px.sparse_conv3d_s2(conv(x), conv(w), t32(b), child, m))
    roc, rchild = orc.downsample_coords_s2(coords)
    ref = orc.sparse_conv3d_s2(rchild, x, w, b)
    (assert_bf16 if dtype == "bf16" else assert_fp32)(y, ref, what=f"s2 conv {dtype}")


def test_strided_conv_identity_invariant(px, orc):
    """W_c = I, bias 0 => output = child count x mean pool (oracle's downsample_mean)."""
    coords = W.shell_coords(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 45)
    n = coords.shape[0]
    x = W.normal(45, n * 16, 1).reshape(n, 16)
    oc, child, m = px.downsample_s2(ti32(coords), 2, (16, 16, 16))
    w = np.tile(np.eye(16, dtype=np.float32), (8, 1, 1))
    y = host(px.sparse_conv3d_s2(t32(x), t32(w), t32(np.zeros(16)), child, m))
    _, mean = orc.downsample_mean(coords, x, 2)
    counts = (child.cpu().numpy()[:, :m] >= 0).sum(0)[:, None]
    assert_fp32(y, counts * mean, what="identity s2")


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_strided_conv_one_hot_inverts_subdivision(px, orc, dtype, masked):
    """Children from the oracle's sparse_channel_to_spatial (factor 2, pinned to
    the reference's child order c = cx + 2cy + 4cz): the device child map equals
    the brute-force slots, and the device stride-2 conv with W_c0 = I, every other
    W_c = 0, bias 0 hands back slice c0 of every parent (0 where the mask dropped
    child c0), exactly, for each of the 8 slots."""
    from fixtures import child_slots_brute_force, subdivided_parents

    cp = 16
    parents, pf, sub = subdivided_parents(30, cp, masked)
    if dtype == "bf16":
        pf = W.bf16_round(pf)
    cc, cf = orc.channel_to_spatial(parents, pf, 2, sub)
    print(f"[s2 one-hot] dtype={dtype} masked={masked} children={cc.shape[0]}", flush=True)
    oc, child, m = px.downsample_s2(ti32(cc), 2, (20, 20, 20))
    np.testing.assert_array_equal(oc.cpu().numpy(), parents)
    cm = child.cpu().numpy()[:, :m].T
    np.testing.assert_array_equal(cm, child_slots_brute_force(cc, parents))
    conv = tbf if dtype == "bf16" else t32
    keep = np.ones((m, 8), np.float32) if sub is None else (sub > 0).astype(np.float32)
    for c0 in range(8):
        w = np.zeros((8, cp, cp), np.float32)
        w[c0] = np.eye(cp, dtype=np.float32)
        y = host(px.sparse_conv3d_s2(conv(cf), conv(w), t32(np.zeros(cp)), child, m))
        np.testing.assert_array_equal(y, pf[:, c0 * cp:(c0 + 1) * cp] * keep[:, c0:c0 + 1])


def test_downsample_mean_matches_reference_vectors(px):
    v = dict(np.load(GOLD / "ref_vectors.npz"))
    oc, off, rows, m = px.downsample(ti32(v["ds_coords"]), 2, (16, 16, 16), 2)
    y = host(px.downsample_mean(t32(v["ds_feats"]), off, rows, m))
    np.testing.assert_array_equal(oc.cpu().numpy(), v["ds_out_coords"])
    assert_fp32(y, v["ds_out_feats"], what="downsample mean")


def test_unet_stage_strided_full_size(px):
    """The U-Net stage's op B (stride-2 conv 128 -> 256) at full size, sampled outputs in float64."""
    wl = W.unet_stage_128()
    coords, x, w = wl["coords"], wl["feats"], wl["w_b"]
    oc, child, m = px.downsample_s2(ti32(coords), 2, (128, 128, 128))
    y = host(px.sparse_conv3d_s2(tbf(x), tbf(w), t32(wl["b_b"]), child, m))
    cm = child.cpu().numpy()[:, :m]
    rows = np.linspace(0, m - 1, 1500).astype(np.int64)
    ref = np.zeros((rows.size, 256))
    for c in range(8):
        src = cm[c, rows]
        ok = src >= 0
        ref[ok] += x[src[ok]].astype(np.float64) @ w[c].astype(np.float64).T
    assert_bf16(y[rows], ref, what="unet B sampled")


def test_unet_stage_conv_c_full_size(px):
    """The U-Net stage's op C at full size (SubMConv3d 256 -> 256 on the ~40k coarse
    voxels, 128 x 256 tiles): sampled rows in float64, plus the exact centre
    identity on every row."""
    wl = W.unet_stage_128()
    oc, _, m = px.downsample_s2(ti32(wl["coords"]), 2, (128, 128, 128))
    coords = oc[:m].contiguous()
    print(f"[conv bf16 unet C] m={m}", flush=True)
    x = W.bf16_round(W.normal(95, m * 256, 1).reshape(m, 256))
    w = wl["w_c"]
    nbr, masks = px.neighbor_map(coords)
    xb = tbf(x)
    y = host(px.subm_conv3d(xb, tbf(w), t32(wl["b_c"]), nbr, masks))
    idx = nbr.cpu().numpy()
    rows = np.linspace(0, m - 1, 1500).astype(np.int64)
    ref = np.tile(wl["b_c"].astype(np.float64), (rows.size, 1))
    for k in range(27):
        src = idx[k, rows]
        ok = src != m
        ref[ok] += x[src[ok]].astype(np.float64) @ w[k].astype(np.float64).T
    assert_bf16(y[rows], ref, what="unet C sampled")
    eye = np.zeros((27, 256, 256), np.float32)
    eye[13] = np.eye(256, dtype=np.float32)
    yi = px.subm_conv3d(xb, tbf(eye), t32(np.zeros(256)), nbr, masks)
    np.testing.assert_array_equal(host(yi), host(xb))
