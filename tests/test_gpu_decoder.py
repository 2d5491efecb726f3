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
        ref_pred = orc.linear(x, w["to_subdiv_weight"], w["to_subdiv_bias"])
        assert_fp32(host(pred), ref_pred, what="to_subdiv logits")
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
