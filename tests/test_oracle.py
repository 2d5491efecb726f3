"""Pin the CPU oracle (oracle/pxs_oracle.cpp) before trusting it.

Checks, per oracle function:
* the reference's own KAT outputs (tests/sparse_numeric_fixture.cpp and
  tests/sparse_transformer_numeric_fixture.cpp, run from oracle/_ref and
  committed as tests/golden/*.json);
* seeded vectors from the compiled reference library (tests/golden/ref_vectors.npz);
* closed forms and brute force that a plausible mistake would fail.
All comparisons against the reference are bit-exact: the oracle follows the
reference's accumulation order and is built with its Release flags.
"""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
import workloads as W
from fixtures import block_kat, child_slots_brute_force, kat_inputs, subdivided_parents

GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


@pytest.fixture(scope="module")
def vec():
    return dict(np.load(GOLD / "ref_vectors.npz"))


# --- the reference's own KAT (tests/sparse_numeric_fixture.cpp:23-170) ----------

def test_kat_sparse_numeric_fixture(orc):
    gold = {k: np.array(v, np.float32) for k, v in
            json.loads((GOLD / "sparse_numeric_fixture.json").read_text()).items()}
    a = kat_inputs()
    c = a["coords"]
    np.testing.assert_array_equal(orc.linear(a["feats"], a["lw"], a["lb"]).ravel(),
                                  gold["sparse_linear_output"])
    np.testing.assert_array_equal(orc.subm_conv3d(c, a["feats"], a["cw"], a["cb"]).ravel(),
                                  gold["sparse_conv_output"])
    np.testing.assert_array_equal(
        orc.layer_norm(a["feats"], 1e-5, np.array([0.8, 1.1, 1.4], np.float32),
                       np.array([-0.2, 0.03, 0.17], np.float32)).ravel(),
        gold["sparse_norm_output"])
    dco, dfo = orc.downsample_mean(c, a["feats"], 2)
    np.testing.assert_array_equal(dco.ravel().astype(np.float32), gold["sparse_downsample_coords"])
    np.testing.assert_array_equal(dfo.ravel(), gold["sparse_downsample_output"])
    cu = orc.batch_cu_seqlens(c, 2)
    np.testing.assert_array_equal(
        orc.varlen_attention(a["q"], a["k"], a["v"], cu, cu, 2, 6, np.float32(0.37)).ravel(),
        gold["sparse_attention_output"])
    np.testing.assert_array_equal(orc.rope(c, a["q"], 2, 6).ravel(), gold["sparse_rope_output"])
    np.testing.assert_array_equal(orc.mh_rms_norm(a["q"], 2, 6, a["rg"]).ravel(),
                                  gold["sparse_rms_output"])
    np.testing.assert_array_equal(
        orc.varlen_attention(a["q"], a["ck"], a["cv"], cu, np.array([0, 3, 5]), 2, 6,
                             np.float32(0.29)).ravel(),
        gold["sparse_cross_output"])
    sco, sfo = orc.channel_to_spatial(a["pc"], a["pf"], 2, a["sub"])
    np.testing.assert_array_equal(sco.ravel().astype(np.float32),
                                  gold["sparse_channel_to_spatial_coords"])
    np.testing.assert_array_equal(sfo.ravel(), gold["sparse_channel_to_spatial_output"])


def test_kat_transformer_block(orc):
    gold = np.array(json.loads((GOLD / "sparse_transformer_fixture.json").read_text())
                    ["sparse_transformer_output"], np.float32)
    k = block_kat()
    out = orc.transformer_block(k["coords"], 2, k["x"], k["tmod"], k["ctx"], [0, 3, 5],
                                k["cfg_i"], k["cfg_f"], k["weights"], projected=k["proj"])
    np.testing.assert_array_equal(out.ravel(), gold)


# --- seeded vectors from the compiled reference --------------------------------

def test_ref_vectors_primitives(orc, vec):
    v = vec
    np.testing.assert_array_equal(orc.subm_conv3d(v["conv_coords"], v["conv_feats"], v["conv_w"],
                                                  v["conv_b"]), v["conv_out"])
    np.testing.assert_array_equal(orc.linear(v["lin_x"], v["lin_w"], v["lin_b"]), v["lin_out"])
    np.testing.assert_array_equal(orc.linear(v["lin_x"], v["lin_w"], v["lin_b"]), v["vlin_out"])
    np.testing.assert_array_equal(orc.layer_norm(v["ln_x"], 1e-6, v["ln_g"], v["ln_b"]),
                                  v["ln_out_affine"])
    np.testing.assert_array_equal(orc.layer_norm(v["ln_x"], 1e-5), v["ln_out_plain"])
    np.testing.assert_array_equal(orc.mh_rms_norm(v["rms_x"], 4, 64, v["rms_g"]), v["rms_out"])
    np.testing.assert_array_equal(orc.mh_rms_norm(v["rms_x"], 4, 64, v["rms_g"]), v["vrms_out"])
    np.testing.assert_array_equal(orc.rope(v["rms_coords"], v["rms_x"], 4, 64), v["rope_out"])
    cu = orc.batch_cu_seqlens(v["attn_coords"], 3)
    np.testing.assert_array_equal(
        orc.varlen_attention(v["attn_q"], v["attn_k"], v["attn_v"], cu, cu, 2, 16,
                             np.float32(0.25)), v["attn_out"])
    np.testing.assert_array_equal(
        orc.varlen_attention(v["attn_q"], v["cross_k"], v["cross_v"], cu, v["cross_offsets"], 2,
                             16, np.float32(0.25)), v["cross_out"])
    dco, dfo = orc.downsample_mean(v["ds_coords"], v["ds_feats"], 2)
    np.testing.assert_array_equal(dco, v["ds_out_coords"])
    np.testing.assert_array_equal(dfo, v["ds_out_feats"])
    co, cf = orc.channel_to_spatial(v["ds_coords"], v["ds_feats"], 2, v["c2s_sub"])
    np.testing.assert_array_equal(co, v["c2s_out_coords"])
    np.testing.assert_array_equal(cf, v["c2s_out_feats"])
    co, cf = orc.channel_to_spatial(v["ds_coords"], v["ds_feats"], 2)
    np.testing.assert_array_equal(co, v["c2s_all_coords"])
    np.testing.assert_array_equal(cf, v["c2s_all_feats"])


def test_ref_vectors_block_and_timestep(orc, vec):
    v = vec
    ws = [v[f"blk_w{i}"] for i in range(23)]
    cfg_f = [1e-6, 1.0, 10000.0]
    out = orc.transformer_block(v["blk_coords"], 2, v["blk_x"], v["blk_tmod"], v["blk_ctx"],
                                v["blk_ctx_off"], [32, 4, 64, 6, 5, 1, 1, 1, 1], cfg_f, ws,
                                projected=v["blk_proj"])
    np.testing.assert_array_equal(out, v["blk_out"])
    out = orc.transformer_block(v["blk_coords"], 2, v["blk_x"], v["blk_tmod"], v["blk_ctx"],
                                v["blk_ctx_off"], [32, 4, 64, 6, 5, 1, 1, 1, 0], cfg_f, ws)
    np.testing.assert_array_equal(out, v["blk_out_noproj"])
    np.testing.assert_array_equal(orc.timestep_embedding(v["temb_t"], 256), v["temb_freq"])
    np.testing.assert_array_equal(
        orc.timestep_embed_mlp(v["temb_t"], 32, 256, v["temb_w0"], v["temb_b0"], v["temb_w2"],
                               v["temb_b2"]), v["temb_out"])


@pytest.mark.parametrize("proj", [True, False])
def test_row_sampled_block_matches_full(orc, vec, proj):
    """Row sampling (the CPU baseline and the parity check for large configs:
    linears and attentions on the sampled rows, keys and values on all rows)
    is exact per sampled row, against the compiled reference's block."""
    v = vec
    ws = [v[f"blk_w{i}"] for i in range(23)]
    rows = np.array([0, 5, 17, 40, v["blk_coords"].shape[0] - 1])
    out = orc.transformer_block(v["blk_coords"], 2, v["blk_x"], v["blk_tmod"], v["blk_ctx"],
                                v["blk_ctx_off"], [32, 4, 64, 6, 5, 1, 1, 1, int(proj)],
                                [1e-6, 1.0, 10000.0], ws, rows=rows,
                                projected=v["blk_proj"] if proj else None)
    want = v["blk_out"] if proj else v["blk_out_noproj"]
    np.testing.assert_array_equal(out[rows], want[rows])


def test_ref_conv_full_size(orc):
    """The oracle reproduces the reference conv on the 64^3 fp32 workload bit for bit."""
    import hashlib

    gold = json.loads((GOLD / "ref_conv_64.json").read_text())
    wl = W.conv_fp32_64()
    out = orc.subm_conv3d(wl["coords"], wl["feats"], wl["weight"], wl["bias"])
    assert out.shape[0] == gold["points"]
    np.testing.assert_array_equal(out[gold["rows"]], np.array(gold["values"], np.float32))
    assert hashlib.sha256(np.ascontiguousarray(out, "<f4").tobytes()).hexdigest() == gold["sha256"]


# --- closed forms / brute force ---------------------------------------------------

def brute_neighbors(coords):
    index = {tuple(c): i for i, c in enumerate(coords.tolist())}
    n = len(coords)
    idx = np.full((27, n), n, np.int32)
    for p, (b, x, y, z) in enumerate(coords.tolist()):
        for k in range(27):
            kd, kh, kw = k // 9, (k // 3) % 3, k % 3
            idx[k, p] = index.get((b, x + kd - 1, y + kh - 1, z + kw - 1), n)
    return idx


def test_neighbor_map_brute_force_and_invariants(orc):
    coords = W.shell_coords(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 21)
    idx = orc.neighbor_map(coords)
    np.testing.assert_array_equal(idx, brute_neighbors(coords))
    n = coords.shape[0]
    np.testing.assert_array_equal(idx[13], np.arange(n))
    # symmetry: idx[k][p] = q  <=>  idx[26-k][q] = p
    for k in range(27):
        present = idx[k] != n
        p = np.nonzero(present)[0]
        np.testing.assert_array_equal(idx[26 - k][idx[k][p]], p)
    pin, pout, offs = orc.neighbor_pairs(idx)
    assert offs[27] == int((idx != n).sum())
    for k in range(27):
        seg = slice(offs[k], offs[k + 1])
        assert np.all(np.diff(pout[seg]) > 0)
        np.testing.assert_array_equal(idx[k][pout[seg]], pin[seg])


def test_neighbor_map_batches_do_not_mix(orc):
    coords = np.array([[0, 1, 1, 1], [1, 1, 1, 2], [1, 1, 1, 1]], np.int32)
    idx = orc.neighbor_map(coords)
    assert idx[13 + 1][0] == 3  # (0,1,1,2) absent in batch 0
    assert idx[13 + 1][2] == 1 and idx[13 - 1][1] == 2


def test_conv_centre_identity_closed_form(orc):
    coords = W.shell_coords(16, [[(4.0, 7.0)]], 22)
    n = coords.shape[0]
    x = W.normal(22, n * 8, 1).reshape(n, 8)
    w = np.zeros((27, 8, 8), np.float32)
    w[13] = np.eye(8, dtype=np.float32)
    b = W.normal(22, 8, 2)
    np.testing.assert_array_equal(orc.subm_conv3d(coords, x, w, b), x + b)


def test_conv_brute_force_small(orc):
    coords = W.shell_coords(8, [[(2.0, 3.5)]], 23)
    n = coords.shape[0]
    x = W.normal(23, n * 3, 1).reshape(n, 3).astype(np.float64)
    w = W.normal(23, 27 * 5 * 3, 2).reshape(27, 5, 3).astype(np.float64)
    b = W.normal(23, 5, 3).astype(np.float64)
    idx = brute_neighbors(coords)
    ref = np.tile(b, (n, 1))
    for k in range(27):
        for p in range(n):
            if idx[k, p] != n:
                ref[p] += w[k] @ x[idx[k, p]]
    got = orc.subm_conv3d(coords, x, w, b)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


def test_attention_closed_forms(orc):
    n, H, D = 12, 2, 8
    q = W.normal(24, n * H * D, 1).reshape(n, H * D)
    k = np.tile(W.normal(24, H * D, 2), (n, 1))  # identical keys -> uniform weights
    v = W.normal(24, n * H * D, 3).reshape(n, H * D)
    cu = np.array([0, n])
    out = orc.varlen_attention(q, k, v, cu, cu, H, D, 0.3)
    np.testing.assert_allclose(out, np.tile(v.mean(0), (n, 1)), rtol=1e-5, atol=1e-6)
    out1 = orc.varlen_attention(q, k[:1], v[:1], cu, np.array([0, 1]), H, D, 0.3)
    np.testing.assert_allclose(out1, np.tile(v[:1], (n, 1)), rtol=0, atol=0)


def test_layer_norm_constant_row_gives_beta(orc):
    x = np.full((3, 16), 2.5, np.float32)
    g, b = W.normal(25, 16, 1), W.normal(25, 16, 2)
    np.testing.assert_array_equal(orc.layer_norm(x, 1e-6, g, b), np.tile(b, (3, 1)))


def test_strided_conv_identity_is_count_times_mean(orc):
    coords = W.shell_coords(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 26)
    n = coords.shape[0]
    x = W.normal(26, n * 6, 1).reshape(n, 6)
    oc, child = orc.downsample_coords_s2(coords)
    dco, dfo = orc.downsample_mean(coords, x, 2)
    np.testing.assert_array_equal(oc, dco)
    w = np.tile(np.eye(6, dtype=np.float32), (8, 1, 1))
    out = orc.sparse_conv3d_s2(child, x, w, np.zeros(6, np.float32))
    counts = (child >= 0).sum(1).astype(np.float32)[:, None]
    np.testing.assert_allclose(out, counts * dfo, rtol=1e-5, atol=1e-5)
    # every input row is a child of exactly one output row
    rows = np.sort(child[child >= 0])
    np.testing.assert_array_equal(rows, np.arange(n))


def test_strided_conv_child_slots_brute_force(orc):
    coords = W.shell_coords(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 28)
    oc, child = orc.downsample_coords_s2(coords)
    np.testing.assert_array_equal(child, child_slots_brute_force(coords, oc))
    # a big-endian or axis-swapped order would differ on this input
    assert (child[:, 1] != child[:, 4]).any() and (child[:, 2] != child[:, 4]).any()


@pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref is built only where /root/reference exists")
@pytest.mark.parametrize("masked", [False, True])
def test_strided_conv_one_hot_inverts_reference_subdivision(orc, masked):
    """The compiled reference's sparse_channel_to_spatial (factor 2) moves parent
    channel slice c to child c = cx + 2cy + 4cz (src/sparse.cpp:676-690).  A
    stride-2 conv over those children with W_c0 = I, every other W_c = 0 and
    bias 0 must hand back slice c0 of every parent, or 0 where the mask dropped
    child c0, for each of the 8 slots: any other child order fails."""
    ref = O.Reference()
    cp = 5
    parents, pf, sub = subdivided_parents(29, cp, masked)
    sub_h = None if sub is None else ref.sparse(parents, sub, 2, (10, 10, 10))
    cc, cf = ref.channel_to_spatial(ref.sparse(parents, pf, 2, (10, 10, 10)), 2, sub_h).read()
    oc, child = orc.downsample_coords_s2(cc)
    np.testing.assert_array_equal(oc, parents)
    np.testing.assert_array_equal(child, child_slots_brute_force(cc, oc))
    keep = np.ones((parents.shape[0], 8), np.float32) if sub is None else (sub > 0)
    for c0 in range(8):
        w = np.zeros((8, cp, cp), np.float32)
        w[c0] = np.eye(cp, dtype=np.float32)
        out = orc.sparse_conv3d_s2(child, cf, w, np.zeros(cp, np.float32))
        np.testing.assert_array_equal(out, pf[:, c0 * cp:(c0 + 1) * cp] * keep[:, c0:c0 + 1])


def test_window_partition_brute_force(orc):
    coords = W.shell_coords(24, [[(6.0, 10.0)], [(5.0, 9.0)]], 27)
    for shift in (0, 4):
        fwd, bwd, cu = orc.window_partition(coords, (24, 24, 24), 8, shift)
        n = coords.shape[0]
        np.testing.assert_array_equal(np.sort(fwd), np.arange(n))
        np.testing.assert_array_equal(bwd[fwd], np.arange(n))
        nw = -(-(24 + shift) // 8)
        wkey = [(b, (x + shift) // 8, (y + shift) // 8, (z + shift) // 8)
                for b, x, y, z in coords.tolist()]
        wid = [((b * nw + a) * nw + c) * nw + d for b, a, c, d in wkey]
        expect = sorted(range(n), key=lambda i: (wid[i], i))
        np.testing.assert_array_equal(fwd, expect)
        for s in range(len(cu) - 1):
            members = fwd[cu[s]:cu[s + 1]]
            assert len({wid[i] for i in members}) == 1
        assert len(cu) - 1 == len(set(wid))


def test_validation_first_error_order(orc):
    coords = np.array([[0, 0, 0, 0], [0, 0, 0, 1], [0, 0, 0, 0], [0, 9, 0, 0]], np.int32)
    f = np.zeros((4, 2), np.float32)
    assert orc.sparse_valid(coords, 1, (4, 4, 4), f, 2) == (5, 2)
    coords2 = coords.copy()
    coords2[1] = [0, 0, 5, 0]
    assert orc.sparse_valid(coords2, 1, (4, 4, 4), f, 2) == (4, 1)
    f2 = f.copy()
    f2[0, 1] = np.nan
    assert orc.sparse_valid(coords, 1, (4, 4, 4), f2, 2) == (7, 0)
    c3 = np.array([[1, 0, 0, 0], [0, 0, 0, 1]], np.int32)
    assert orc.sparse_valid(c3, 2, (4, 4, 4), np.zeros((2, 2), np.float32), 2) == (6, 1)
    assert orc.sparse_valid(c3, 0, (4, 4, 4), np.zeros((2, 2), np.float32), 2)[0] == 1
    assert orc.sparse_valid(c3, 2, (4, 4, 4), np.zeros(3, np.float32), 2)[0] == 3


@pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref is built only where /root/reference exists")
def test_validation_messages_match_compiled_reference(orc):
    ref = O.Reference()
    cases = [
        (np.array([[0, 0, 0, 0], [0, 0, 0, 1], [0, 0, 0, 0]], np.int32), 1, np.zeros((3, 2))),
        (np.array([[0, 0, 0, 0], [0, 0, 5, 0]], np.int32), 1, np.zeros((2, 2))),
        (np.array([[1, 0, 0, 0], [0, 0, 0, 1]], np.int32), 2, np.zeros((2, 2))),
        (np.array([[0, 0, 0, 0], [0, 0, 0, 1]], np.int32), 1, np.array([[0, 1], [np.inf, 0]])),
    ]
    for coords, batch, feats in cases:
        ok, msg = ref.valid(ref.sparse(coords, feats, batch, (4, 4, 4)))
        code, _ = orc.sparse_valid(coords, batch, (4, 4, 4), feats, 2)
        assert not ok and code and O.VALID_MESSAGES[code] == msg


# --- decoder blocks: compositions of compiled reference primitives ---------------

def _silu(v):
    """silu_in_place (src/slat_decoder.cpp:68-78)."""
    v = np.asarray(v, np.float32)
    return v * (np.float32(1.0) / (np.float32(1.0) + np.exp(-v)))


@pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref is built only where /root/reference exists")
def test_decoder_blocks_compose_reference_primitives(orc):
    """orc_convnext_block and orc_resblock_c2s against the compiled reference's
    conv / layer norm / linear / channel_to_spatial chained in the order of
    src/slat_decoder.cpp:185-288, with SiLU and repeat_channels
    (src/slat_decoder.cpp:68-107) applied between the calls."""
    ref = O.Reference()
    seed, G, C, M, O_ = 51, 12, 16, 32, 8
    coords = W.shell_coords(G, [[(3.0, 4.5)], [(2.5, 4.0)]], seed)
    n = coords.shape[0]
    x = W.normal(seed, n * C, 1).reshape(n, C)
    g, b = 1.0 + W.normal(seed, C, 2, std=0.1), W.normal(seed, C, 3, std=0.1)
    cw = W.normal(seed, 27 * C * C, 4, std=0.05).reshape(27, C, C)
    cb = W.normal(seed, C, 5, std=0.1)
    w0, b0 = W.normal(seed, M * C, 6, std=0.2).reshape(M, C), W.normal(seed, M, 7, std=0.1)
    w2, b2 = W.normal(seed, C * M, 8, std=0.2).reshape(C, M), W.normal(seed, C, 9, std=0.1)
    sp = lambda c, f, shape=(G, G, G): ref.sparse(c, f, 2, shape)

    # ConvNeXt.
    conv = ref.subm_conv3d(sp(coords, x), cw, cb)
    h = ref.linear(ref.layer_norm(conv, 1e-6, g, b), w0, b0).read()[1]
    r = ref.linear(sp(coords, _silu(h)), w2, b2).read()[1]
    expect = r + x
    got = orc.convnext_block(coords, x, M, 1e-6, [g, b, cw, cb, w0, b0, w2, b2])
    assert np.max(np.abs(got - expect)) <= 1e-6 * np.max(np.abs(expect))

    # Channel-to-spatial residual block with a given subdivision.
    P = 8 * O_
    c1w = W.normal(seed, 27 * P * C, 10, std=0.05).reshape(27, P, C)
    c1b = W.normal(seed, P, 11, std=0.1)
    c2w = W.normal(seed, 27 * O_ * O_, 12, std=0.1).reshape(27, O_, O_)
    c2b = W.normal(seed, O_, 13, std=0.1)
    sub = W.normal(seed, n * 8, 14).reshape(n, 8)
    sub_t = sp(coords, sub)
    normed = _silu(ref.layer_norm(sp(coords, x), 1e-6, g, b).read()[1])
    packed = ref.subm_conv3d(sp(coords, normed), c1w, c1b)
    oc, hidden = ref.channel_to_spatial(packed, 2, sub_t).read()
    _, skip = ref.channel_to_spatial(sp(coords, x), 2, sub_t).read()
    S2 = (2 * G,) * 3
    hn = _silu(ref.layer_norm(sp(oc, hidden, S2), 1e-6).read()[1])
    y = ref.subm_conv3d(sp(oc, hn, S2), c2w, c2b).read()[1]
    expect = y + np.repeat(skip, O_ // (C // 8), axis=1)
    got_c, got = orc.resblock_c2s(coords, x, O_, 1e-6, [g, b, c1w, c1b, c2w, c2b],
                                  subdivision=sub)
    np.testing.assert_array_equal(got_c, oc)
    assert np.max(np.abs(got - expect)) <= 1e-6 * np.max(np.abs(expect))


def test_decoder_block_closed_forms(orc):
    """mlp2 = 0 makes the ConvNeXt block the identity; conv2 = 0 leaves the C2S
    block's output equal to the repeated subdivided input."""
    seed, C, M, O_ = 52, 16, 32, 8
    coords = W.shell_coords(12, [[(3.0, 4.5)]], seed)
    n = coords.shape[0]
    x = W.normal(seed, n * C, 1).reshape(n, C)
    ones, zeros = np.ones(C, np.float32), np.zeros(C, np.float32)
    cw = W.normal(seed, 27 * C * C, 4, std=0.05).reshape(27, C, C)
    w0 = W.normal(seed, M * C, 6, std=0.2).reshape(M, C)
    out = orc.convnext_block(coords, x, M, 1e-6, [ones, zeros, cw, zeros, w0, np.zeros(M),
                                                  np.zeros((C, M)), zeros])
    np.testing.assert_array_equal(out, x)
    P = 8 * O_
    c1w = W.normal(seed, 27 * P * C, 10, std=0.05).reshape(27, P, C)
    oc, y = orc.resblock_c2s(coords, x, O_, 1e-6, [ones, zeros, c1w, np.zeros(P),
                                                   np.zeros((27, O_, O_)), np.zeros(O_)])
    assert oc.shape[0] == 8 * n
    sc, skip = orc.channel_to_spatial(coords, x, 2)
    np.testing.assert_array_equal(oc, sc)
    # repeat_channels repeats each source channel consecutively.
    expect = np.repeat(skip, O_ // (C // 8), axis=1)
    np.testing.assert_array_equal(y, expect)
    assert y[0, 0] == y[0, 1] == skip[0, 0] and y[0, O_ // (C // 8)] == skip[0, 1]


def _silu_branch(v):
    """silu (src/slat_flow.cpp:79-83): the two-branch form."""
    v = np.asarray(v, np.float32)
    pos = v / (np.float32(1.0) + np.exp(-np.maximum(v, 0)))
    e = np.exp(np.minimum(v, 0))
    neg = v * e / (np.float32(1.0) + e)
    return np.where(v >= 0, pos, neg).astype(np.float32)


@pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref is built only where /root/reference exists")
def test_flow_composes_reference_primitives(orc):
    """orc_slat_flow_forward against the compiled reference's sparse_linear,
    timestep_embed_mlp (src/flow.cpp:125-180), the row linear's arithmetic
    (varlen_linear: bias first, inputs ascending), the transformer block and
    sparse_layer_norm, chained as src/slat_flow.cpp:201-248 does."""
    from fixtures import flow_case

    ref = O.Reference()
    C, H, B, G = 32, 2, 2, 12
    case = flow_case(33, [[(3.0, 4.5)], [(2.5, 4.0)]], G, C, H, 2, 5)
    fw, blocks = case["fw"], case["blocks"]
    h = ref.linear(ref.sparse(case["coords"], case["x"], B, (G, G, G)), fw[0], fw[1])
    temb = _silu_branch(ref.timestep_embed_mlp(case["t"], C, 256, fw[2], fw[3], fw[4], fw[5]))
    tmod = ref.varlen_linear(ref.varlen([0, B], temb), fw[6], fw[7]).read()
    ctx = ref.varlen(case["ctx_off"], case["ctx"])
    cfg_i = [C, H, case["M"], case["CC"], 0, 1, 1, 1, 0]
    for ws in blocks:
        h = ref.transformer_block(h, tmod, ctx, cfg_i, [1e-6, 1.0, 10000.0], ws)
    expect = ref.linear(ref.layer_norm(h, 1e-5), fw[8], fw[9]).read()[1]
    got = orc.slat_flow_forward(case["coords"], B, case["x"], case["t"], case["ctx"],
                                case["ctx_off"], case["dims"], [1e-6, 1.0, 10000.0], fw, blocks)
    assert np.max(np.abs(got - expect)) <= 1e-6 * np.max(np.abs(expect))


# --- flow Euler sampler (src/flow_sampler.cpp) -------------------------------------

SAMPLER_CASES = {
    # name: (steps, [sigma_min, rescale_t, strength, rescale, interval_min, interval_max])
    "unguided": (6, [1e-5, 1.0, 1.0, 0.0, 0.0, 1.0]),
    "guided": (5, [1e-5, 3.0, 3.0, 0.0, 0.0, 1.0]),
    "guided_rescale_interval": (7, [1e-5, 3.0, 7.5, 0.7, 0.2, 0.8]),
    "unconditional": (4, [1e-3, 1.0, 0.0, 0.0, 0.0, 1.0]),
    "full_rescale": (3, [1e-5, 1.0, 4.0, 1.0, 0.0, 1.0]),
}


def sampler_inputs(seed=61):
    from fixtures import flow_velocity
    coords = W.shell_coords(12, [[(3.0, 4.5)], [(2.5, 4.0)]], seed)
    noise = W.normal(seed, coords.shape[0] * 8, 1).reshape(-1, 8)
    return coords, noise, flow_velocity(coords, 8, seed)


@pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref is built only where /root/reference exists")
@pytest.mark.parametrize("case", list(SAMPLER_CASES))
def test_flow_sampler_matches_compiled_reference(orc, case):
    """orc_flow_euler_sample against the reference's flow_euler_sample_f32
    compiled from src/flow_sampler.cpp, both driven by the same velocity
    callback: samples and both trajectories bit for bit."""
    steps, cfg = SAMPLER_CASES[case]
    coords, noise, fn = sampler_inputs()
    ref = O.Reference()
    out, rxt, rx0 = ref.flow_euler_sample(ref.sparse(coords, noise, 2, (12, 12, 12)), steps, cfg,
                                          fn, record=True)
    got, xt, x0 = orc.flow_euler_sample(coords, 2, noise, steps, cfg, fn, record=True)
    np.testing.assert_array_equal(got, out.read()[1])
    np.testing.assert_array_equal(xt, rxt)
    np.testing.assert_array_equal(x0, rx0)


@pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref is built only where /root/reference exists")
def test_flow_sampler_errors_match_compiled_reference(orc):
    coords, noise, fn = sampler_inputs()
    ref = O.Reference()
    t = ref.sparse(coords, noise, 2, (12, 12, 12))
    for steps, cfg, msg in [
            (0, [1e-5, 1.0, 1.0, 0.0, 0.0, 1.0], "invalid flow Euler sampler configuration"),
            (3, [1e-5, 1.0, 1.0, -0.5, 0.0, 1.0], "invalid flow Euler sampler configuration"),
            (3, [1e-5, 1.0, 1.0, 0.0, 0.9, 0.1], "invalid flow Euler sampler configuration"),
            (3, [1.0, 1.0, 1.0, 0.0, 0.0, 1.0], "invalid flow Euler sampler configuration")]:
        with pytest.raises(O.ReferenceError, match=msg):
            ref.flow_euler_sample(t, steps, cfg, fn)
        assert orc.flow_schedule(steps, cfg, 0)[0] == 1
    with pytest.raises(O.ReferenceError, match="model callback is empty"):
        ref.flow_euler_sample(t, 3, [1e-5, 1.0, 1.0, 0.0, 0.0, 1.0], None)


def test_flow_sampler_closed_forms(orc):
    """Zero velocity keeps the noise; a constant velocity v moves the state by
    sum(t_i - t_{i+1}) v = (1 - 0) v; a unit guidance interval that excludes
    every step runs the conditional branch only."""
    coords, noise, fn = sampler_inputs()
    zero = lambda s, t, c: np.zeros_like(s)  # noqa: E731
    got, _, _ = orc.flow_euler_sample(coords, 2, noise, 5, [1e-5, 2.0, 3.0, 0.5, 0.0, 1.0], zero)
    np.testing.assert_array_equal(got, noise)
    v = W.normal(62, noise.size, 1).reshape(noise.shape)
    const = lambda s, t, c: v  # noqa: E731
    got, _, _ = orc.flow_euler_sample(coords, 2, noise, 8, [1e-5, 1.0, 1.0, 0.0, 0.0, 1.0], const)
    np.testing.assert_allclose(got, noise - v, rtol=0, atol=1e-5)
    a, _, _ = orc.flow_euler_sample(coords, 2, noise, 4, [1e-5, 1.0, 5.0, 0.7, 2.0, 3.0], fn)
    b, _, _ = orc.flow_euler_sample(coords, 2, noise, 4, [1e-5, 1.0, 1.0, 0.0, 0.0, 1.0], fn)
    np.testing.assert_array_equal(a, b)
    # Schedule with rescale_t = 1: t_i = 1 - i / steps.
    for i in range(4):
        rc, t, tn, g = orc.flow_schedule(4, [1e-5, 1.0, 2.0, 0.0, 0.0, 1.0], i)
        assert rc == 0 and t == np.float32(1.0) - np.float32(i) / np.float32(4.0) and g == 2.0


@pytest.mark.skipif(not O.REF_LIB.exists(), reason="oracle/_ref is built only where /root/reference exists")
def test_decoder_closed_form_helper_matches_compiled_reference(orc):
    """The decoder closed form (residual branches zero) built from the oracle's
    primitives equals the same chain built from the compiled reference's
    primitives (sparse_linear, sparse_channel_to_spatial, sparse_layer_norm)
    bit for bit; the channel repeat is repeat_channels (src/slat_decoder.cpp:
    84-107: each channel `repeats` times in a row)."""
    ref = O.Reference()
    coords = W.shell_coords(12, [[(3.0, 4.5)], [(2.5, 4.0)]], 90)
    n, latent, ch = coords.shape[0], 8, (256, 32, 16)  # 4 distinct values per final row
    x = W.normal(90, n * latent, 1).reshape(n, latent)
    fl_w = W.normal(90, ch[0] * latent, 2).reshape(ch[0], latent)
    fl_b = W.normal(90, ch[0], 3)
    ow = W.normal(90, 24 * ch[-1], 4).reshape(24, ch[-1])
    ob = W.normal(90, 24, 5)
    g0 = W.normal(91, n * 8, 1).reshape(n, 8)
    n1 = int((g0 > 0).sum())
    guides = [g0, W.normal(92, n1 * 8, 1).reshape(n1, 8)]
    # oracle primitives
    c, h = coords, orc.linear(x, fl_w, fl_b)
    for lv in range(2):
        c, sub = orc.channel_to_spatial(c, h, 2, guides[lv])
        h = np.repeat(sub, ch[lv + 1] // (ch[lv] // 8), axis=1)
    want = orc.linear(orc.layer_norm(h, 1e-5), ow, ob)
    # reference primitives
    shape = 12
    t = ref.linear(ref.sparse(coords, x, 2, (shape,) * 3), fl_w, fl_b)
    for lv in range(2):
        cc, _ = t.read()
        t = ref.channel_to_spatial(t, 2, ref.sparse(cc, guides[lv], 2, (shape,) * 3))
        shape *= 2
        rc, rf = t.read()
        t = ref.sparse(rc, np.repeat(rf, ch[lv + 1] // (ch[lv] // 8), axis=1), 2, (shape,) * 3)
    got = ref.linear(ref.layer_norm(t, 1e-5), ow, ob).read()
    np.testing.assert_array_equal(got[0], c)
    np.testing.assert_array_equal(got[1], want)
