"""GPU parity: sparse linear (fp32/bf16, activations, gate-residual epilogue),
layer norm (+modulation), multi-head RMS norm, RoPE, the QKV prologue."""

import numpy as np
import pytest

import oracle as O
import workloads as W
from gpu_common import assert_bf16, assert_fp32, host, t32, tbf, ti32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def px():
    import pxs
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


@pytest.mark.parametrize("rows,cin,cout", [(200, 24, 40), (1000, 64, 64), (777, 256, 384),
                                          (300, 8, 1024), (513, 1024, 8), (5, 3, 4)])
def test_linear_fp32(px, orc, rows, cin, cout):
    x = W.normal(51, rows * cin, 1).reshape(rows, cin)
    w = W.normal(51, cout * cin, 2, std=0.2).reshape(cout, cin)
    b = W.normal(51, cout, 3)
    print(f"[linear fp32] {rows}x{cin}->{cout}", flush=True)
    y = host(px.linear(t32(x), t32(w), t32(b)))
    assert_fp32(y, orc.linear(x, w, b), what="linear fp32")


def test_linear_reference_vectors(px):
    from pathlib import Path
    v = dict(np.load(Path(__file__).resolve().parent / "golden" / "ref_vectors.npz"))
    y = host(px.linear(t32(v["lin_x"]), t32(v["lin_w"]), t32(v["lin_b"])))
    assert_fp32(y, v["lin_out"], what="linear vs reference")


@pytest.mark.parametrize("rows,cin,cout", [(4096, 1024, 3072), (2000, 4096, 1024), (1500, 256, 200)])
def test_linear_bf16(px, rows, cin, cout):
    x = W.bf16_round(W.normal(52, rows * cin, 1).reshape(rows, cin))
    w = W.bf16_round(W.normal(52, cout * cin, 2, std=0.02).reshape(cout, cin))
    b = W.normal(52, cout, 3, std=0.1)
    print(f"[linear bf16] {rows}x{cin}->{cout}", flush=True)
    y = host(px.linear(tbf(x), tbf(w), t32(b)))
    ref = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert_bf16(y, ref, what="linear bf16")


@pytest.mark.parametrize("act", [1, 2])
def test_linear_activation_epilogue(px, orc, act):
    x = W.normal(53, 300 * 48, 1).reshape(300, 48)
    w = W.normal(53, 96 * 48, 2, std=0.2).reshape(96, 48)
    b = W.normal(53, 96, 3)
    y = host(px.linear(t32(x), t32(w), t32(b), act=act))
    ref = orc.linear(x, w, b)
    ref = orc.gelu_tanh(ref) if act == 1 else orc.silu(ref)
    assert_fp32(y, ref, what=f"act {act}")


def test_linear_gate_residual(px, orc):
    coords = np.concatenate([np.zeros((70, 4), np.int32), np.ones((50, 4), np.int32)])
    coords[:, 1:] = 0
    x = W.normal(54, 120 * 32, 1).reshape(120, 32)
    w = W.normal(54, 32 * 32, 2, std=0.2).reshape(32, 32)
    b = W.normal(54, 32, 3)
    bmod = W.normal(54, 6 * 32, 4)
    tmod = W.normal(54, 2 * 6 * 32, 5)
    res = W.normal(54, 120 * 32, 6).reshape(120, 32)
    r = t32(res)
    px.linear_gate_residual(t32(x), t32(w), t32(b), ti32(coords), t32(bmod), t32(tmod), 64, r)
    lin = orc.gate(coords, orc.linear(x, w, b), bmod, tmod, 64)
    assert_fp32(host(r), res + lin, what="gate residual")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_layer_norm(px, orc, dtype):
    x = (W.normal(55, 400 * 1024, 1) * 3 + 0.5).reshape(400, 1024)
    g, b = W.normal(55, 1024, 2), W.normal(55, 1024, 3)
    conv = t32 if dtype == "f32" else tbf
    xr = x if dtype == "f32" else W.bf16_round(x)
    for gamma, beta, eps in ((g, b, 1e-6), (None, None, 1e-5)):
        y = host(px.layer_norm(conv(x), eps, None if gamma is None else t32(gamma),
                               None if beta is None else t32(beta)))
        ref = orc.layer_norm(xr, eps, gamma, beta)
        (assert_fp32 if dtype == "f32" else assert_bf16)(y, ref, what=f"ln {dtype}")


@pytest.mark.parametrize("channels", [4, 8, 64, 96, 128, 256, 512, 2048])
@pytest.mark.parametrize("xd,yd", [("f32", "f32"), ("bf16", "bf16"), ("f32", "bf16"), ("bf16", "f32")])
def test_layer_norm_row_layouts(px, orc, channels, xd, yd):
    """Every row layout of the layer norm against the oracle: rows of 1 to 64
    16-byte vectors (4 fp32 or 8 bf16 channels each) share a wave, 64/L rows
    per wave; 128 and 256 vectors take 2 or 4 per lane; other widths (96
    channels, 4 bf16 channels, 2048 fp32 channels) one wave per row.  1,237
    rows leave the last wave part empty."""
    import torch
    rows = 1237
    x = (W.normal(57, rows * channels, 1) * 2 - 0.3).reshape(rows, channels)
    g, b = W.normal(57, channels, 2), W.normal(57, channels, 3)
    conv = t32 if xd == "f32" else tbf
    xr = x if xd == "f32" else W.bf16_round(x)
    out = torch.float32 if yd == "f32" else torch.bfloat16
    check = assert_fp32 if yd == "f32" else assert_bf16
    print(f"[ln layouts] channels={channels} {xd}->{yd}", flush=True)
    for gamma, beta, eps in ((g, b, 1e-6), (None, None, 1e-5)):
        y = host(px.layer_norm(conv(x), eps, None if gamma is None else t32(gamma),
                               None if beta is None else t32(beta), out_dtype=out))
        check(y, orc.layer_norm(xr, eps, gamma, beta), what=f"ln {channels} {xd}->{yd}")


def test_layer_norm_small_channels_and_kat(px):
    import json
    from pathlib import Path
    from test_oracle import kat_inputs
    gold = json.loads((Path(__file__).resolve().parent / "golden" /
                       "sparse_numeric_fixture.json").read_text())
    a = kat_inputs()
    y = host(px.layer_norm(t32(a["feats"]), 1e-5, t32(np.array([0.8, 1.1, 1.4])),
                           t32(np.array([-0.2, 0.03, 0.17]))))
    assert_fp32(y.ravel(), np.array(gold["sparse_norm_output"]), what="KAT layer norm")


def test_layer_norm_modulate_to_bf16(px, orc):
    coords = np.zeros((300, 4), np.int32)
    coords[150:, 0] = 1
    x = W.normal(56, 300 * 256, 1).reshape(300, 256)
    bmod = W.normal(56, 6 * 256, 2, std=0.1)
    tmod = W.normal(56, 2 * 6 * 256, 3, std=0.1)
    y = host(px.layer_norm_modulate(t32(x), 1e-6, ti32(coords), t32(bmod), t32(tmod), 3 * 256,
                                    out_dtype=__import__("torch").bfloat16))
    ref = orc.modulate(coords, orc.layer_norm(x, 1e-6), bmod, tmod, 3 * 256)
    assert_bf16(y, ref, tol=5e-3, what="ln modulate")
    y32 = host(px.layer_norm_modulate(t32(x), 1e-6, ti32(coords), t32(bmod), t32(tmod), 0))
    assert_fp32(y32, orc.modulate(coords, orc.layer_norm(x, 1e-6), bmod, tmod, 0), what="ln mod f32")


@pytest.mark.parametrize("heads,hd", [(4, 64), (2, 6), (3, 16)])
def test_rms_and_rope(px, orc, heads, hd):
    coords = W.shell_coords(64, [[(16.0, 30.0)]], 57)[::50].copy()
    n = coords.shape[0]
    x = W.normal(57, n * heads * hd, 1).reshape(n, heads * hd)
    g = np.abs(W.normal(57, heads * hd, 2)) + 0.5
    assert_fp32(host(px.mh_rms_norm(t32(x), heads, hd, t32(g))), orc.mh_rms_norm(x, heads, hd, g),
                what="rms")
    assert_fp32(host(px.rope(ti32(coords), t32(x), heads, hd)), orc.rope(coords, x, heads, hd),
                what="rope")


@pytest.mark.parametrize("dtype,hd,heads", [("f32", 64, 4), ("bf16", 64, 4), ("f32", 16, 4),
                                            ("bf16", 64, 12), ("f32", 64, 16)])
def test_qkv_prepare(px, orc, dtype, hd, heads):
    C = heads * hd
    coords = W.shell_coords(64, [[(16.0, 30.0)]], 58)[::30].copy()
    n = coords.shape[0]
    qkv = W.normal(58, n * 3 * C, 1).reshape(n, 3 * C)
    if dtype == "bf16":
        qkv = W.bf16_round(qkv)
    gq = np.abs(W.normal(58, C, 2)) + 0.5
    gk = np.abs(W.normal(58, C, 3)) + 0.5
    conv = t32 if dtype == "f32" else tbf
    q, k, v = px.qkv_prepare(conv(qkv), heads, hd, t32(gq), t32(gk), ti32(coords))
    rq = orc.rope(coords, orc.mh_rms_norm(qkv[:, :C], heads, hd, gq), heads, hd)
    rk = orc.rope(coords, orc.mh_rms_norm(qkv[:, C:2 * C], heads, hd, gk), heads, hd)
    check = assert_fp32 if dtype == "f32" else assert_bf16
    check(host(q), rq, what="q")
    check(host(k), rk, what="k")
    np.testing.assert_array_equal(host(v), qkv[:, 2 * C:])


@pytest.mark.parametrize("cin,cout,rows", [(64, 8, 1000), (37, 8, 1000), (128, 3, 1000),
                                           (96, 24, 1000), (2048, 8, 300), (5, 1, 70_001),
                                           (64, 7, 100_000)])
def test_linear_ordered_bit_exact(px, orc, cin, cout, rows):
    """pxs_linear_ordered reproduces sparse_linear's operation order: bit-equal
    to the oracle (itself bit-equal to the compiled reference).  Up to 8
    outputs run one thread per row over rows staged through LDS (16-byte loads
    when cin % 4 == 0, single floats otherwise; 2,048 inputs take the largest
    weight table); 24 outputs one thread per output."""
    x = W.normal(91, rows * cin, 1).reshape(rows, cin)
    w = W.normal(91, cout * cin, 2, std=cin ** -0.5).reshape(cout, cin)
    b = W.normal(91, cout, 3)
    got = px.linear_ordered(t32(x), t32(w), t32(b))
    np.testing.assert_array_equal(host(got), orc.linear(x, w, b))


@pytest.mark.parametrize("cin,cout", [(64, 7), (256, 8), (30, 2), (257, 8)])
def test_linear_fp32_few_outputs(px, orc, cin, cout):
    """fp32 linears with at most 8 outputs and at most 256 inputs run in the
    reference's own order (bit-equal to the oracle); 257 inputs take the MFMA
    path (the fp32 bar)."""
    rows = 20_011
    x = W.normal(92, rows * cin, 1).reshape(rows, cin)
    w = W.normal(92, cout * cin, 2, std=cin ** -0.5).reshape(cout, cin)
    b = W.normal(92, cout, 3)
    got = host(px.linear(t32(x), t32(w), t32(b)))
    ref = orc.linear(x, w, b)
    if cin <= 256:
        np.testing.assert_array_equal(got, ref)
    else:
        assert_fp32(got, ref, what="fp32 linear, 8 outputs")


@pytest.mark.parametrize("count", [0, 1, 777, 1_000_003])
def test_value_stats(px, count):
    """pxs_value_stats_f32 against numpy: finite min / max / max |v| exactly,
    the sum to double rounding, the non-finite count and the first one."""
    x = W.normal(68, count, 1) * np.float32(3.0)
    if count > 100:
        x[count // 3] = np.inf
        x[count // 2] = np.nan
        x[count - 1] = -np.inf
    print(f"[value stats] count={count}", flush=True)
    got = px.value_stats(t32(x))
    fin = x[np.isfinite(x)]
    bad = np.flatnonzero(~np.isfinite(x))
    assert got["nonfinite"] == bad.size
    assert got["first_bad"] == (bad[0] if bad.size else count)
    if bad.size:
        assert got["first_bad_value"] == x[bad[0]]
    assert got["min"] == (fin.min() if fin.size else np.inf)
    assert got["max"] == (fin.max() if fin.size else -np.inf)
    assert got["max_abs"] == (np.abs(fin).max() if fin.size else 0.0)
    assert abs(got["sum"] - fin.astype(np.float64).sum()) <= 1e-9 * max(1.0, np.abs(fin).sum())


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_elementwise_vector_paths_match_element_loops(px, dtype):
    """Activations, conversions and add_repeat run 8 elements per thread when
    the count is a multiple of 8 and the buffers are 16-byte aligned, one
    element per thread otherwise; both forms must give the same bits (and
    conversions torch's round-to-nearest-even)."""
    import torch
    import pxs
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    n = 8 * 40_000
    base = torch.from_numpy(W.normal(58, n, 1).reshape(-1) * 3).to("cuda")
    for act in (pxs.ACT_SILU, pxs.ACT_GELU_TANH):
        vec = base.to(tdt).clone()
        px.activation(vec, act)                   # multiple of 8, aligned
        tail = base.to(tdt)[: n - 1].clone()
        px.activation(tail, act)                  # n - 1 elements: the element loop
        torch.cuda.synchronize()
        assert torch.equal(vec[: n - 1], tail), f"activation {act} {dtype}"
    src = base if dtype == "f32" else base.to(torch.bfloat16)
    for out in (torch.float32, torch.bfloat16):
        want = src.to(out)
        assert torch.equal(px.convert(src, out), want), f"convert {dtype}->{out}"
        assert torch.equal(px.convert(src[1:], out), want[1:]), f"convert unaligned {dtype}->{out}"
    rows = 4_099
    for ch, sk in ((64, 8), (48, 48), (12, 3)):   # vector path, repeats 1, element loop
        a = torch.from_numpy(W.normal(59, rows * ch, 1).reshape(rows, ch)).to("cuda").to(tdt)
        skip = torch.from_numpy(W.normal(59, rows * sk, 2).reshape(rows, sk)).to("cuda")
        got = px.add_repeat(a, skip)
        torch.cuda.synchronize()
        want = a.float() + skip.repeat_interleave(ch // sk, dim=1)
        assert torch.equal(got, want), f"add_repeat {ch}/{sk} {dtype}"


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_head_norm_rope_64(px, orc, dtype):
    """pxs_mh_rms_norm and pxs_rope at head_dim 64 (one wavefront per row, 8
    lanes of 8 dims per head): 12 heads (the second pass of 8 heads half
    idle), a strided input (row stride 2C, as for the cross-attention keys)
    and an in-place call, against the oracle."""
    import torch
    import pxs
    rows, H, D = 3001, 12, 64
    C = H * D
    rng = np.random.default_rng(94)
    coords = np.concatenate([np.zeros((rows, 1), np.int32),
                             rng.integers(0, 64, (rows, 3)).astype(np.int32)], axis=1)
    x2 = (W.normal(93, rows * 2 * C, 1) * 2).reshape(rows, 2 * C)
    g = W.normal(93, C, 2) * np.float32(0.5) + np.float32(1.0)
    conv = t32 if dtype == "f32" else tbf
    check = assert_fp32 if dtype == "f32" else assert_bf16
    xr = (x2 if dtype == "f32" else W.bf16_round(x2))[:, :C]
    xd = conv(x2)
    check(host(px.mh_rms_norm(xd[:, :C], H, D, t32(g))), orc.mh_rms_norm(xr, H, D, g),
          what=f"rms strided {dtype}")
    check(host(px.rope(ti32(coords), xd[:, :C], H, D)), orc.rope(coords, xr, H, D),
          what=f"rope strided {dtype}")
    xc = conv(np.ascontiguousarray(x2[:, :C]))
    gd = t32(g)
    px._check(px.lib.pxs_mh_rms_norm(pxs._dtype_code(xc), pxs._ptr(xc), C, rows, H, D,
                                     pxs._ptr(gd), pxs._ptr(xc), C, px.stream()), "in place")
    check(host(xc), orc.mh_rms_norm(xr, H, D, g), what=f"rms in place {dtype}")


def _dense_case(px, orc, dtype, rows, cin, cout, seed):
    """Every epilogue of the plain linears at one shape against the oracle
    (sparse_linear's serial fp32 order) on the same (bf16-rounded) operands:
    bias with no activation, GELU, SiLU, no bias, the fp32 residual add and
    the adaLN gate with the residual add (two batch items)."""
    import torch
    import pxs
    conv = t32 if dtype == "f32" else tbf
    rnd = (lambda v: v) if dtype == "f32" else W.bf16_round
    check = assert_fp32 if dtype == "f32" else assert_bf16
    x = rnd(W.normal(seed, rows * cin, 1).reshape(rows, cin))
    w = rnd(W.normal(seed, cout * cin, 2, std=cin ** -0.5).reshape(cout, cin))
    b = W.normal(seed, cout, 3, std=0.1)
    lin = orc.linear(x, w, b)
    for act, f in ((pxs.ACT_NONE, lambda v: v), (pxs.ACT_GELU_TANH, orc.gelu_tanh),
                   (pxs.ACT_SILU, orc.silu)):
        y = host(px.linear(conv(x), conv(w), t32(b), act=act))
        check(y, f(lin), what=f"{dtype} linear act {act}")
    y = host(px.linear(conv(x), conv(w), None))
    check(y, orc.linear(x, w, np.zeros(cout, np.float32)), what=f"{dtype} linear, no bias")
    res0 = W.normal(seed, rows * cout, 4).reshape(rows, cout)
    res = t32(res0)
    px.linear_residual(conv(x), conv(w), t32(b), res)
    torch.cuda.synchronize()
    check(host(res), res0 + lin, what=f"{dtype} linear residual")
    coords = np.zeros((rows, 4), np.int32)
    coords[rows // 3:, 0] = 1
    bmod = W.normal(seed, 6 * cout, 5)
    tmod = W.normal(seed, 2 * 6 * cout, 6)
    res = t32(res0)
    px.linear_gate_residual(conv(x), conv(w), t32(b), ti32(coords), t32(bmod), t32(tmod), 2 * cout,
                            res)
    torch.cuda.synchronize()
    check(host(res), res0 + orc.gate(coords, lin, bmod, tmod, 2 * cout),
          what=f"{dtype} linear gate residual")


# Shapes for every tile of the dense kernels (256 x 256, 128 x 128, 128 x 64),
# K ragged against the 128-byte chunk (72, 136, 40), outputs not a multiple
# of 8 or 4 (the per-element epilogue), rows past one tile, and the
# gather-GEMM fallback (60 inputs: rows not whole 16-byte pieces).
@pytest.mark.parametrize("rows,cin,cout", [(4096, 256, 512), (300, 64, 96), (200, 64, 64),
                                           (1000, 60, 64), (1000, 72, 64), (257, 136, 130),
                                           (520, 40, 1000), (3000, 1024, 1024), (70000, 64, 256),
                                           (70000, 256, 64), (30000, 256, 256), (777, 128, 36)])
def test_linear_dense_bf16(px, orc, rows, cin, cout):
    print(f"[linear dense bf16] {rows}x{cin}->{cout}", flush=True)
    _dense_case(px, orc, "bf16", rows, cin, cout, 95)


@pytest.mark.parametrize("rows,cin,cout", [(2048, 512, 512), (1024, 768, 96), (4096, 136, 128),
                                           (20000, 128, 128), (20000, 64, 256), (333, 36, 70),
                                           (100, 8, 1024), (513, 1024, 12)])
def test_linear_dense_fp32(px, orc, rows, cin, cout):
    print(f"[linear dense fp32] {rows}x{cin}->{cout}", flush=True)
    _dense_case(px, orc, "f32", rows, cin, cout, 96)


def _sampled_rows(m, count=256, seed=0):
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([rng.integers(0, m, count), [0, m - 1]]))
    return rows


# The linears configs 3, 4 and 5 and the decoder run, at full size: inputs
# drawn on the device, sampled output rows recomputed in float64 on the host
# from the same bf16 operands (the gate and residual forms with fp32
# residuals), at the bf16 bar.
@pytest.mark.parametrize("rows,cin,cout,form", [
    (32768, 1024, 3072, "plain"), (32768, 1024, 1024, "gate"), (40960, 1024, 4096, "gelu"),
    (40960, 4096, 1024, "gate"), (40960, 1024, 1024, "residual"), (29700, 768, 2304, "plain"),
    (2492211, 64, 256, "silu"), (2492211, 256, 64, "residual")])
def test_linear_dense_config_shapes(px, rows, cin, cout, form):
    import torch
    import pxs
    print(f"[linear dense config] {rows}x{cin}->{cout} {form}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + cin + cout)
    x = torch.randn(rows, cin, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(cout, cin, device="cuda", generator=g) * cin ** -0.5).to(torch.bfloat16)
    b = torch.randn(cout, device="cuda", generator=g) * 0.1
    sel = _sampled_rows(rows, seed=rows)
    xs = x[torch.from_numpy(sel).cuda()].double().cpu().numpy()
    wd = w.double().cpu().numpy()
    lin = xs @ wd.T + b.double().cpu().numpy()
    if form in ("plain", "gelu", "silu"):
        act = {"plain": pxs.ACT_NONE, "gelu": pxs.ACT_GELU_TANH, "silu": pxs.ACT_SILU}[form]
        y = px.linear(x, w, b, act=act)
        got = host(y[torch.from_numpy(sel).cuda()])
        if form == "gelu":
            lin = 0.5 * lin * (1.0 + np.tanh(0.7978845608028654 * (lin + 0.044715 * lin ** 3)))
        elif form == "silu":
            lin = lin / (1.0 + np.exp(-lin))
        assert_bf16(got, lin, what=f"{form} {rows}x{cin}->{cout}")
        return
    res0 = torch.randn(rows, cout, device="cuda", generator=g)
    res = res0.clone()
    want = res0[torch.from_numpy(sel).cuda()].double().cpu().numpy()
    if form == "residual":
        px.linear_residual(x, w, b, res)
        want = want + lin
    else:
        batch = torch.zeros(rows, 4, dtype=torch.int32, device="cuda")
        batch[rows // 2:, 0] = 1
        bmod = torch.randn(6 * cout, device="cuda", generator=g)
        tmod = torch.randn(2 * 6 * cout, device="cuda", generator=g)
        px.linear_gate_residual(x, w, b, batch, bmod, tmod, 2 * cout, res)
        bsel = batch[torch.from_numpy(sel).cuda(), 0].cpu().numpy()
        gate = (bmod[2 * cout:3 * cout].double().cpu().numpy()[None, :] +
                tmod.double().cpu().numpy().reshape(2, 6 * cout)[bsel, 2 * cout:3 * cout])
        want = want + lin * gate
    got = host(res[torch.from_numpy(sel).cuda()])
    # the residual part is exact; the bar applies to the product's share
    assert_bf16(got - res0[torch.from_numpy(sel).cuda()].cpu().numpy(),
                want - res0[torch.from_numpy(sel).cuda()].double().cpu().numpy(),
                what=f"{form} {rows}x{cin}->{cout}")


# 256 x 256 tiles over hundreds of tiles: every output row of the three
# epilogues against a float32 product of the same bf16 operands on the
# device, row by row, so a tile stored at the wrong place or a K chunk
# carried into the wrong tile shows in the rows it touches.  Rows, K and
# outputs are ragged against the tile and the 64-element chunk.
@pytest.mark.parametrize("rows,cin,cout", [(16500, 520, 2000), (33000, 1024, 1024)])
def test_linear_dense_large_tiles_every_row(px, rows, cin, cout):
    import torch
    print(f"[linear dense 256x256 every row] {rows}x{cin}->{cout}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(rows + cin)
    x = torch.randn(rows, cin, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(cout, cin, device="cuda", generator=g) * cin ** -0.5).to(torch.bfloat16)
    b = torch.randn(cout, device="cuda", generator=g) * 0.1
    want = (x.float() @ w.float().t().contiguous()) + b

    def rows_ok(got, ref, what):
        err = (got.double() - ref.double()).norm(dim=1) / ref.double().norm(dim=1).clamp_min(1e-30)
        worst = int(err.argmax())
        assert float(err.max()) <= 1e-2, f"{what}: row {worst} rel L2 {float(err.max()):.3e}"

    rows_ok(px.linear(x, w, b).float(), want, "plain")
    res0 = torch.randn(rows, cout, device="cuda", generator=g)
    res = res0.clone()
    px.linear_residual(x, w, b, res)
    rows_ok(res - res0, want, "residual")
    batch = torch.zeros(rows, 4, dtype=torch.int32, device="cuda")
    batch[rows // 3:, 0] = 1
    bmod = torch.randn(6 * cout, device="cuda", generator=g)
    tmod = torch.randn(2 * 6 * cout, device="cuda", generator=g)
    res = res0.clone()
    px.linear_gate_residual(x, w, b, batch, bmod, tmod, cout, res)
    gate = bmod[cout:2 * cout][None, :] + tmod.view(2, 6 * cout)[batch[:, 0].long(), cout:2 * cout]
    rows_ok(res - res0, want * gate, "gate")


def _ref_bench_values(count, salt, scale, start=0):
    """tests/sparse_linear_cuda_benchmark.cpp:188-199 (deterministic_value):
    bucket = ((index * 6364136223846793005 + salt) >> 32) % 251 - 125, times
    scale, for indices start .. start + count - 1 (uint64 arithmetic)."""
    idx = np.arange(start, start + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        mixed = idx * np.uint64(6364136223846793005) + np.uint64(salt)
    bucket = ((mixed >> np.uint64(32)) % np.uint64(251)).astype(np.int64) - 125
    return (bucket.astype(np.float32) * np.float32(scale)).astype(np.float32)


# The reference's hot sparse_linear shapes
# (tests/sparse_linear_cuda_benchmark.cpp:42-52), fp32 as there, with its
# deterministic inputs (salts and scales of :228, :709-710): sampled rows
# against float64 at the fp32 bar; the 64 -> 7 shape takes the ordered-row
# kernel (bit-equal order) and is checked on every row of a prefix.
@pytest.mark.parametrize("points,cin,cout", [
    (46537, 2048, 512), (46537, 512, 2048), (206980, 1024, 256), (206980, 256, 1024),
    (909164, 512, 128), (909164, 128, 512), (9857, 4096, 1024), (9857, 1024, 4096),
    (4005638, 64, 7)])
def test_linear_reference_hot_shapes(px, points, cin, cout):
    import torch
    print(f"[linear reference hot shape] {points}x{cin}->{cout}", flush=True)
    # inputs generated on the device in chunks with the same integer recipe
    x = torch.empty(points, cin, dtype=torch.float32, device="cuda")
    total = points * cin
    step = 1 << 26
    flat = x.view(-1)
    for s0 in range(0, total, step):
        n = min(step, total - s0)
        flat[s0:s0 + n] = torch.from_numpy(_ref_bench_values(n, 0x13579bdf2468ace0, 0.00075, s0)).cuda()
    w = _ref_bench_values(cout * cin, 0x0f1e2d3c4b5a6978, 0.00055).reshape(cout, cin)
    b = _ref_bench_values(cout, 0xa5a5a5a55a5a5a5a, 0.0008)
    y = px.linear(x, t32(w), t32(b))
    sel = _sampled_rows(points, seed=points)
    xs = np.stack([_ref_bench_values(cin, 0x13579bdf2468ace0, 0.00075, int(r) * cin) for r in sel])
    ref = xs.astype(np.float64) @ w.astype(np.float64).T + b
    got = host(y[torch.from_numpy(sel).cuda()])
    assert_fp32(got, ref, what=f"hot shape {points}x{cin}->{cout}")

