"""Device-resident SLat-decoder blocks (pxs_convnext_block, pxs_resblock_c2s)
against the oracle's restatement of src/slat_decoder.cpp:185-288.

fp32: within 1e-5 (max|g - r| / max|r|); bf16 convolution and MLP operands
with fp32 accumulation: within 1e-2 relative L2, against the oracle run in
fp32 on the same bf16-rounded weights.  Output coordinates are bit-exact.
"""

import numpy as np
import pytest
import torch

import oracle as O
import pxs
import workloads as W
from gpu_common import assert_bf16, assert_fp32, host, t32, ti32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def px():
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


def convnext_case(seed, C, M, grid=16, items=((4.0, 6.0),)):
    coords = W.shell_coords(grid, [list(items)], seed)
    n = coords.shape[0]
    x = W.normal(seed, n * C, 1).reshape(n, C)
    w = {"norm_weight": 1.0 + W.normal(seed, C, 2, std=0.1),
         "norm_bias": W.normal(seed, C, 3, std=0.1),
         "conv1_weight": W.normal(seed, 27 * C * C, 4, std=(1.0 / (27 * C)) ** 0.5)
         .reshape(27, C, C),
         "conv1_bias": W.normal(seed, C, 5, std=0.1),
         "mlp0_weight": W.normal(seed, M * C, 6, std=C ** -0.5).reshape(M, C),
         "mlp0_bias": W.normal(seed, M, 7, std=0.1),
         "mlp2_weight": W.normal(seed, C * M, 8, std=M ** -0.5).reshape(C, M),
         "mlp2_bias": W.normal(seed, C, 9, std=0.1)}
    return coords, x, w


ORC_CONVNEXT = ("norm_weight", "norm_bias", "conv1_weight", "conv1_bias", "mlp0_weight",
                "mlp0_bias", "mlp2_weight", "mlp2_bias")
ORC_C2S = ("norm1_weight", "norm1_bias", "conv1_weight", "conv1_bias", "conv2_weight",
           "conv2_bias")


def device_decoder_weights(w, dtype):
    tdt = torch.bfloat16 if dtype == pxs.PXS_BF16 else torch.float32
    dev = {k: (t32(v).to(tdt) if k in pxs.DECODER_DTYPE_WEIGHTS else t32(v)) for k, v in w.items()}
    return dev, pxs.decoder_block_weights(dev)


def rounded(w, dtype):
    if dtype != pxs.PXS_BF16:
        return w
    return {k: (W.bf16_round(v) if k in pxs.DECODER_DTYPE_WEIGHTS else v) for k, v in w.items()}


@pytest.mark.parametrize("dtype", [pxs.PXS_F32, pxs.PXS_BF16])
def test_convnext_block(px, orc, dtype):
    C, M = (64, 256) if dtype == pxs.PXS_F32 else (128, 512)
    coords, x, w = convnext_case(41, C, M)
    print(f"convnext dtype={dtype} n={coords.shape[0]} C={C}", flush=True)
    keep, dw = device_decoder_weights(w, dtype)
    got = host(px.convnext_block(ti32(coords), t32(x), M, 1e-6, dw, dtype))
    wr = rounded(w, dtype)
    ref = orc.convnext_block(coords, x, M, 1e-6, [wr[k] for k in ORC_CONVNEXT])
    if dtype == pxs.PXS_F32:
        assert_fp32(got, ref, what="convnext fp32")
    else:
        assert_bf16(got, ref, what="convnext bf16")


def test_convnext_block_in_place_with_given_map(px, orc):
    """y aliasing x and a caller-built neighbor map give the same result."""
    C, M = 32, 128
    coords, x, w = convnext_case(42, C, M, items=((3.0, 5.0), (5.0, 7.0)))
    keep, dw = device_decoder_weights(w, pxs.PXS_F32)
    c = ti32(coords)
    nbr, masks = px.neighbor_map(c)
    ref = px.convnext_block(c, t32(x), M, 1e-6, dw, pxs.PXS_F32)
    h = t32(x)
    px.convnext_block(c, h, M, 1e-6, dw, pxs.PXS_F32, nbr=nbr, masks=masks, out=h)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(h), host(ref))


def c2s_case(seed, C, O_, grid=16):
    coords = W.shell_coords(grid, [[(4.0, 6.0)], [(3.0, 5.0)]], seed)
    n = coords.shape[0]
    x = W.normal(seed, n * C, 1).reshape(n, C)
    P = 8 * O_
    w = {"norm1_weight": 1.0 + W.normal(seed, C, 2, std=0.1),
         "norm1_bias": W.normal(seed, C, 3, std=0.1),
         "conv1_weight": W.normal(seed, 27 * P * C, 4, std=(1.0 / (27 * C)) ** 0.5)
         .reshape(27, P, C),
         "conv1_bias": W.normal(seed, P, 5, std=0.1),
         "conv2_weight": W.normal(seed, 27 * O_ * O_, 6, std=(1.0 / (27 * O_)) ** 0.5)
         .reshape(27, O_, O_),
         "conv2_bias": W.normal(seed, O_, 7, std=0.1),
         "to_subdiv_weight": W.normal(seed, 8 * C, 8, std=C ** -0.5).reshape(8, C),
         "to_subdiv_bias": W.normal(seed, 8, 9, std=0.5)}
    return coords, x, w


@pytest.mark.parametrize("dtype", [pxs.PXS_F32, pxs.PXS_BF16])
@pytest.mark.parametrize("mode", ["all", "given", "predicted"])
def test_resblock_c2s(px, orc, dtype, mode):
    C, O_ = 64, 32
    coords, x, w = c2s_case(43, C, O_)
    n = coords.shape[0]
    print(f"c2s dtype={dtype} mode={mode} n={n}", flush=True)
    keep, dw = device_decoder_weights(w, dtype)
    sub = W.normal(44, n * 8, 1).reshape(n, 8) if mode == "given" else None
    oc, y, pred = px.resblock_c2s(ti32(coords), t32(x), O_, 1e-6, dw, dtype,
                                  subdivision=None if sub is None else t32(sub),
                                  pred_subdiv=(mode == "predicted"))
    torch.cuda.synchronize()
    if mode == "predicted":
        # to_subdiv runs in sparse_linear's own order: the logits are bit-equal.
        ref_pred = orc.linear(x, w["to_subdiv_weight"], w["to_subdiv_bias"])
        np.testing.assert_array_equal(host(pred), ref_pred)
        # The oracle selects children with the device's own logits, so a logit
        # within rounding of zero cannot split the two topologies.
        sub = host(pred)
    wr = rounded(w, dtype)
    ref_c, ref_y = orc.resblock_c2s(coords, x, O_, 1e-6, [wr[k] for k in ORC_C2S],
                                    subdivision=sub)
    np.testing.assert_array_equal(host(oc).astype(np.int32), ref_c)
    if dtype == pxs.PXS_F32:
        assert_fp32(host(y), ref_y, what=f"c2s fp32 {mode}")
    else:
        assert_bf16(host(y), ref_y, what=f"c2s bf16 {mode}")


def test_resblock_c2s_zero_conv_is_repeated_skip(px, orc):
    """conv2 = 0 leaves y = repeat_channels(channel_to_spatial(x)) exactly."""
    C, O_ = 32, 16
    coords, x, w = c2s_case(45, C, O_)
    w["conv2_weight"] = np.zeros_like(w["conv2_weight"])
    w["conv2_bias"] = np.zeros_like(w["conv2_bias"])
    keep, dw = device_decoder_weights(w, pxs.PXS_F32)
    oc, y, _ = px.resblock_c2s(ti32(coords), t32(x), O_, 1e-6, dw, pxs.PXS_F32)
    torch.cuda.synchronize()
    _, skip = orc.channel_to_spatial(coords, x, 2)
    np.testing.assert_array_equal(host(y), np.repeat(skip, O_ // (C // 8), axis=1))


def test_add_repeat(px):
    a = torch.randn(37, 24, device="cuda")
    skip = torch.randn(37, 6, device="cuda")
    got = px.add_repeat(a, skip)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(got), host(a) + np.repeat(host(skip), 4, axis=1))
    ab = a.to(torch.bfloat16)
    got = px.add_repeat(ab, skip)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(got), host(ab) + np.repeat(host(skip), 4, axis=1))


# --- the decoder stack (slat_decoder_forward_f32, src/slat_decoder.cpp:290-440) -----

def convnext_weights(seed, C, M):
    return convnext_case(seed, C, M)[2]


def c2s_weights(seed, C, O_):
    return c2s_case(seed, C, O_)[2]


def decoder_case(seed, latent=8, out=24, channels=(64, 32, 16), nblocks=(1, 1, 1)):
    coords = W.shell_coords(12, [[(3.0, 4.5)], [(2.5, 4.0)]], seed)
    n = coords.shape[0]
    x = W.normal(seed, n * latent, 1).reshape(n, latent)
    fl_w = W.normal(seed, channels[0] * latent, 2, std=latent ** -0.5).reshape(channels[0], latent)
    fl_b = W.normal(seed, channels[0], 3, std=0.1)
    out_w = W.normal(seed, out * channels[-1], 4, std=channels[-1] ** -0.5).reshape(out, channels[-1])
    out_b = W.normal(seed, out, 5, std=0.1)
    blocks = []  # (kind, C, out, mlp, weights)
    k = 0
    for level, C in enumerate(channels):
        for _ in range(nblocks[level]):
            k += 1
            blocks.append((pxs.PXS_DECODER_CONVNEXT, C, C, 4 * C, convnext_weights(seed + k, C, 4 * C)))
        if level + 1 < len(channels):
            k += 1
            blocks.append((pxs.PXS_DECODER_C2S, C, channels[level + 1], 0,
                           c2s_weights(seed + k, C, channels[level + 1])))
    return dict(coords=coords, x=x, fl=(fl_w, fl_b), out=(out_w, out_b), blocks=blocks,
                channels=channels, nblocks=nblocks, latent=latent, out_ch=out)


def run_decoder(px, case, dtype, pred_subdiv, guide=None, upsample_times=-1):
    keep = []
    blocks = []
    for kind, C, O_, M, w in case["blocks"]:
        dev, dw = device_decoder_weights(w, dtype)
        keep.append(dev)
        blocks.append(pxs.DecoderBlock(kind, C, O_, M, dw))
    cfg = pxs.decoder_config(case["latent"], case["out_ch"], 1e-6, pred_subdiv,
                             list(case["channels"]), list(case["nblocks"]))
    fl = [t32(a) for a in case["fl"]]
    ow = [t32(a) for a in case["out"]]
    res = px.slat_decoder_forward(dtype, cfg, fl[0], fl[1], ow[0], ow[1], blocks,
                                  ti32(case["coords"]), t32(case["x"]),
                                  guide=None if guide is None else [t32(g) for g in guide],
                                  predict=pred_subdiv and upsample_times < 0,
                                  upsample_times=upsample_times)
    torch.cuda.synchronize()
    return res


def oracle_decoder(orc, case, dtype, select, stop=None):
    """slat_decoder_forward_f32 composed from the oracle's pieces in the
    reference's order (src/slat_decoder.cpp:332-372): select(level, hidden) gives
    the subdivision of each C2S; stop = upsample_times returns the hidden
    state of that level (src/slat_decoder.cpp:419-423)."""
    coords = case["coords"]
    h = orc.linear(case["x"], *case["fl"])
    bi = 0
    for level, C in enumerate(case["channels"]):
        if stop is not None and level == stop:
            return coords, h
        for _ in range(case["nblocks"][level]):
            kind, C_, O_, M, w = case["blocks"][bi]
            wr = rounded(w, dtype)
            h = orc.convnext_block(coords, h, M, 1e-6, [wr[k] for k in ORC_CONVNEXT])
            bi += 1
        if level + 1 < len(case["channels"]):
            kind, C_, O_, M, w = case["blocks"][bi]
            wr = rounded(w, dtype)
            coords, h = orc.resblock_c2s(coords, h, O_, 1e-6, [wr[k] for k in ORC_C2S],
                                         subdivision=select(level, h, w))
            bi += 1
    return coords, orc.linear(orc.layer_norm(h, 1e-5), *case["out"])


def test_decoder_stack_predicted_fp32(px, orc):
    """Three levels (64 -> 32 -> 16 channels, one ConvNeXt block each) with
    predicted subdivisions.  The oracle subdivides with the device's logits
    (a logit within rounding of zero could otherwise split the topologies),
    and those logits must equal the oracle's to_subdiv linear of the oracle's
    own hidden state to the fp32 bar."""
    case = decoder_case(81)
    oc, y, level_rows, preds = run_decoder(px, case, pxs.PXS_F32, True)
    print(f"[decoder stack fp32] level rows {level_rows}", flush=True)
    got_logits = [host(p) for p in preds]

    def select(level, h, w):
        ref = orc.linear(h, w["to_subdiv_weight"], w["to_subdiv_bias"])
        assert_fp32(got_logits[level], ref, what=f"level {level} logits")
        return got_logits[level]

    rc, ry = oracle_decoder(orc, case, pxs.PXS_F32, select)
    assert level_rows[-1] == rc.shape[0] and 0 < level_rows[1] < 8 * level_rows[0]
    np.testing.assert_array_equal(host(oc).astype(np.int32), rc)
    assert_fp32(host(y), ry, what="decoder stack fp32")


@pytest.mark.parametrize("dtype", [pxs.PXS_F32, pxs.PXS_BF16])
def test_decoder_stack_guided(px, orc, dtype):
    """Guide subdivisions fix the topology, so bf16 compares too."""
    case = decoder_case(82, nblocks=(2, 1, 1))
    n0 = case["coords"].shape[0]
    g0 = W.normal(83, n0 * 8, 1).reshape(n0, 8)
    guides = [g0]
    # The second level's guide needs its row count: the children g0 keeps.
    n1 = int((g0 > 0).sum())
    guides.append(W.normal(84, n1 * 8, 1).reshape(n1, 8))
    oc, y, level_rows, _ = run_decoder(px, case, dtype, False, guide=guides)
    print(f"[decoder stack guided] dtype={dtype} level rows {level_rows}", flush=True)
    rc, ry = oracle_decoder(orc, case, dtype, lambda level, h, w: guides[level])
    assert level_rows[1] == n1
    np.testing.assert_array_equal(host(oc).astype(np.int32), rc)
    if dtype == pxs.PXS_F32:
        assert_fp32(host(y), ry, what="decoder stack guided fp32")
    else:
        assert_bf16(host(y), ry, what="decoder stack guided bf16")


def test_decoder_upsample_coords(px, orc):
    """upsample_times = 1: the coordinates and hidden state after one C2S
    level (slat_decoder_upsample_coords_f32); upsample_times = 0 returns the
    latent projection on the input coordinates."""
    case = decoder_case(85)
    oc, y, _, _ = run_decoder(px, case, pxs.PXS_F32, True, upsample_times=0)
    np.testing.assert_array_equal(host(oc).astype(np.int32), case["coords"])
    assert_fp32(host(y), orc.linear(case["x"], *case["fl"]), what="upsample 0")
    oc1, y1, _, _ = run_decoder(px, case, pxs.PXS_F32, True, upsample_times=1)
    full_c, _, _, preds = run_decoder(px, case, pxs.PXS_F32, True)
    logits = host(preds[0])
    rc, rh = oracle_decoder(orc, case, pxs.PXS_F32, lambda level, h, w: logits, stop=1)
    np.testing.assert_array_equal(host(oc1).astype(np.int32), rc)
    assert_fp32(host(y1), rh, what="upsample 1")


def test_decoder_stack_errors(px):
    case = decoder_case(86)
    with pytest.raises(pxs.PxsError, match="weight block count"):
        bad = dict(case, blocks=case["blocks"][:-1])
        run_decoder(px, bad, pxs.PXS_F32, True)
    with pytest.raises(pxs.PxsError, match="coordinate-upsample configuration"):
        run_decoder(px, case, pxs.PXS_F32, False, upsample_times=1)
    with pytest.raises(pxs.PxsError, match="expected ConvNeXt block"):
        swapped = list(case["blocks"])
        swapped[0], swapped[1] = swapped[1], swapped[0]
        run_decoder(px, dict(case, blocks=swapped), pxs.PXS_F32, True)


def without_residual_branches(case):
    """Every ConvNeXt MLP-2 and every C2S conv2 (weight and bias) set to zero:
    each ConvNeXt block becomes the identity and each C2S block its
    subdivided, channel-repeated skip (src/slat_decoder.cpp:210-222, 262-287)."""
    blocks = []
    for kind, C, O_, M, w in case["blocks"]:
        w = dict(w)
        names = ("mlp2_weight", "mlp2_bias") if kind == pxs.PXS_DECODER_CONVNEXT else \
            ("conv2_weight", "conv2_bias")
        for k in names:
            w[k] = np.zeros_like(w[k])
        blocks.append((kind, C, O_, M, w))
    return dict(case, blocks=blocks)


def closed_form_decoder(orc, case, guides):
    """slat_decoder_forward_f32 (src/slat_decoder.cpp:332-376) with the residual
    branches zeroed: out_linear(LN_1e-5(R_L( ... R_1(from_latent(x)) ... ))),
    R_l = repeat each channel of channel_to_spatial(h, guide_l) to the next
    level's width.  Built from the pinned primitives only, not from the
    decoder composition."""
    coords, h = case["coords"], orc.linear(case["x"], *case["fl"])
    ch = case["channels"]
    for level in range(len(ch) - 1):
        coords, sub = orc.channel_to_spatial(coords, h, 2, guides[level])
        h = np.repeat(sub, ch[level + 1] // (ch[level] // 8), axis=1)
    return coords, orc.linear(orc.layer_norm(h, 1e-5), *case["out"])


@pytest.mark.parametrize("dtype", [pxs.PXS_F32, pxs.PXS_BF16])
def test_decoder_stack_closed_form(px, orc, dtype):
    """The device stack and the oracle's chained blocks both reduce to the
    closed form when the residual branches are zero: this pins the chain (the
    latent projection first, the levels' subdivisions in order, the skip's
    channel repeat, the final affine-free layer norm at eps 1e-5 and the
    output linear) independently of the chained restatement.  256 -> 32 -> 16
    channels: a level-1 child's 4 channels come from 4 different level-0
    channels, so the final norm sees 4 distinct values per row (with 64 -> 32
    every child would hold one value repeated, a zero-variance norm input whose
    output is rounding noise times 1/sqrt(eps))."""
    case = without_residual_branches(decoder_case(87, channels=(256, 32, 16), nblocks=(2, 1, 1)))
    n0 = case["coords"].shape[0]
    g0 = W.normal(88, n0 * 8, 1).reshape(n0, 8)
    n1 = int((g0 > 0).sum())
    guides = [g0, W.normal(89, n1 * 8, 1).reshape(n1, 8)]
    rc, ry = closed_form_decoder(orc, case, guides)
    print(f"[decoder closed form] dtype={dtype} rows={rc.shape[0]}", flush=True)
    oc, y, _, _ = run_decoder(px, case, dtype, False, guide=guides)
    np.testing.assert_array_equal(host(oc).astype(np.int32), rc)
    assert_fp32(host(y), ry, what=f"decoder closed form dtype={dtype}")
    oc2, oy = oracle_decoder(orc, case, pxs.PXS_F32, lambda level, h, w: guides[level])
    np.testing.assert_array_equal(oc2, rc)
    assert_fp32(oy, ry, what="chained oracle blocks vs closed form")


def _bench_scale_decoder(dtype):
    """The decoder stack at the reference's decode scale (the decoder bench
    workload): ~10.6k latent voxels at 64^3, levels of 1024, 512, 256, 128, 64
    channels, one ConvNeXt block each, predicted subdivisions; random weights
    drawn on the device (conv and MLP operands in the call's dtype)."""
    wl = W.decoder_64()
    dev = torch.device("cuda")
    coords = torch.from_numpy(wl["coords"]).to(dev)
    chans, nblk = wl["model_channels"], wl["num_blocks"]
    wdt = torch.bfloat16 if dtype == pxs.PXS_BF16 else torch.float32
    g = torch.Generator(device=dev).manual_seed(17)

    def rnd(*s, std=0.02, dt=torch.float32):
        return (torch.randn(*s, generator=g, device=dev) * std).to(dt)

    keep, blocks = [], []
    for level, C in enumerate(chans):
        for _ in range(nblk[level]):
            w = {"norm_weight": 1.0 + rnd(C), "norm_bias": rnd(C),
                 "conv1_weight": rnd(27, C, C, std=(27 * C) ** -0.5, dt=wdt), "conv1_bias": rnd(C),
                 "mlp0_weight": rnd(4 * C, C, std=C ** -0.5, dt=wdt), "mlp0_bias": rnd(4 * C),
                 "mlp2_weight": rnd(C, 4 * C, std=(4 * C) ** -0.5, dt=wdt), "mlp2_bias": rnd(C)}
            keep.append(w)
            blocks.append(pxs.DecoderBlock(pxs.PXS_DECODER_CONVNEXT, C, C, 4 * C,
                                           pxs.decoder_block_weights(w)))
        if level + 1 < len(chans):
            O_ = chans[level + 1]
            w = {"norm1_weight": torch.ones(C, device=dev), "norm1_bias": rnd(C),
                 "conv1_weight": rnd(27, 8 * O_, C, std=(27 * C) ** -0.5, dt=wdt),
                 "conv1_bias": rnd(8 * O_),
                 "conv2_weight": rnd(27, O_, O_, std=(27 * O_) ** -0.5, dt=wdt), "conv2_bias": rnd(O_),
                 "to_subdiv_weight": rnd(8, C, std=C ** -0.5), "to_subdiv_bias": rnd(8, std=0.0)}
            keep.append(w)
            blocks.append(pxs.DecoderBlock(pxs.PXS_DECODER_C2S, C, O_, 0, pxs.decoder_block_weights(w)))
    cfg = pxs.decoder_config(wl["latent_channels"], wl["out_channels"], 1e-6, True, chans, nblk)
    head = (rnd(chans[0], wl["latent_channels"], std=0.2), rnd(chans[0]),
            rnd(wl["out_channels"], chans[-1], std=0.1), rnd(wl["out_channels"]))
    x = torch.randn(coords.shape[0], wl["latent_channels"], generator=g, device=dev)
    return wl, cfg, blocks, keep, head, coords, x


@pytest.mark.parametrize("dtype", [pxs.PXS_BF16])
def test_decoder_stack_production_scale(px, orc, dtype):
    """The 5-level stack at the reference's decode scale (troubleshooting
    history of 9,857 -> 4,005,638 rows; here 10,624 -> ~2.5M), predicted
    subdivisions: every level's coordinates and row count bit-exact against the
    oracle's channel-to-spatial chain driven by the device's logits; the last
    level's ConvNeXt block, final layer norm and output linear on 300 sampled
    rows against float64, from the device's level-4 hidden state (the same
    stack stopped there); and a second decode bit-equal to the first."""
    wl, cfg, blocks, keep, (fl_w, fl_b, out_w, out_b), coords, x = _bench_scale_decoder(dtype)
    max_rows = 8_000_000
    oc, y, level_rows, preds = px.slat_decoder_forward(dtype, cfg, fl_w, fl_b, out_w, out_b, blocks,
                                                      coords, x, predict=True, max_rows=max_rows)
    torch.cuda.synchronize()
    print(f"[decoder production scale] level rows {level_rows}", flush=True)
    assert level_rows[-1] > 1_000_000 and torch.isfinite(y).all().item()
    # coordinates: the oracle's channel-to-spatial chain with the device's logits
    c = wl["coords"]
    for level, logits in enumerate(preds):
        lg = host(logits)
        c, _ = orc.channel_to_spatial(c, np.zeros((c.shape[0], 8), np.float32), 2, lg)
        assert c.shape[0] == level_rows[level + 1], f"level {level + 1} rows"
    np.testing.assert_array_equal(host(oc).astype(np.int32), c)
    # the last level from the device's level-4 hidden state
    oc4, h4, _, _ = px.slat_decoder_forward(dtype, cfg, fl_w, fl_b, out_w, out_b, blocks, coords, x,
                                            upsample_times=4, max_rows=max_rows)
    np.testing.assert_array_equal(host(oc4), host(oc))
    n4, C = h4.shape
    nbr, _ = px.neighbor_map(oc4.contiguous())
    sel = np.unique(np.linspace(0, n4 - 1, 300).astype(np.int64))
    idx = nbr[:, torch.from_numpy(sel).cuda()].cpu().numpy()
    hh = host(h4)
    rnd = W.bf16_round if dtype == pxs.PXS_BF16 else (lambda a: a)
    w = {k: v.float().cpu().numpy().astype(np.float64) for k, v in keep[-1].items()}
    xin = rnd(hh).astype(np.float64)
    conv = np.tile(w["conv1_bias"], (sel.size, 1))
    for k in range(27):
        ok = idx[k] != n4
        conv[ok] += xin[idx[k][ok]] @ w["conv1_weight"][k].T

    def ln(v, eps, gamma=None, beta=None):
        mu = v.mean(1, keepdims=True)
        var = ((v - mu) ** 2).mean(1, keepdims=True)
        out = (v - mu) / np.sqrt(var + eps)
        return out if gamma is None else out * gamma + beta

    hid = ln(conv, 1e-6, w["norm_weight"], w["norm_bias"]) @ w["mlp0_weight"].T + w["mlp0_bias"]
    hid = hid / (1.0 + np.exp(-hid))
    blk = hh[sel].astype(np.float64) + hid @ w["mlp2_weight"].T + w["mlp2_bias"]
    ref = ln(blk, 1e-5) @ host(out_w).astype(np.float64).T + host(out_b).astype(np.float64)
    assert_bf16(host(y)[sel], ref, what="decoder last level, sampled rows")
    oc2, y2, _, _ = px.slat_decoder_forward(dtype, cfg, fl_w, fl_b, out_w, out_b, blocks, coords, x,
                                            predict=True, max_rows=max_rows)
    np.testing.assert_array_equal(host(oc2), host(oc))
    np.testing.assert_array_equal(host(y2), host(y))
