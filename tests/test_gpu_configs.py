"""GPU parity at the full shapes of the attention and flow workloads.

* full-attention block, 12,288 + 20,480 tokens, width 1024 (16 x 64): QKV
  linear, per-head RMS norm on q and k, varlen attention, output linear;
* shifted-window attention, window 8, shift 0 and 4, 12 x 64, on the ~30k
  voxels of a 64^3 shell workload, and the subdivide up-conv 768 -> 8 x 192
  at 64^3 followed by channel-to-spatial to 128^3;
* one SLat-flow transformer block at width 1024 on ~42k voxels with 1,370
  context tokens, and the 24-block forward at that size.

The oracle runs on sampled rows (keys and values over every row, each sampled
query row exactly as in the full computation), in fp32 on the same
bf16-rounded inputs and weights; the device result must be within 1e-2
relative L2 on those rows (bf16 GEMM operands, fp32 accumulation).
"""

import numpy as np
import pytest
import torch

import oracle as O
import pxs
import workloads as W
from gpu_common import assert_bf16, dev, host, t32, tbf, ti32, ti64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def px():
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


def sampled(n, count, extra=()):
    rows = np.unique(np.concatenate([np.linspace(0, n - 1, count).astype(np.int64),
                                     np.asarray(extra, np.int64)]))
    return rows[(rows >= 0) & (rows < n)]


# --- full-attention block at 12,288 + 20,480 tokens -------------------------------

def test_attention_block_full_size_sampled_rows(px, orc):
    wl = W.attn_full()
    x, cu = wl["x"], wl["cu_seqlens"]
    n, C = x.shape
    H, D = wl["heads"], wl["head_dim"]
    print(f"[attn block full] n={n}", flush=True)
    qkv = px.linear(tbf(x), tbf(wl["w_qkv"]), t32(wl["b_qkv"]))
    q, k, v = px.qkv_prepare(qkv, H, D, t32(wl["gamma_q"]), t32(wl["gamma_k"]))
    o = px.varlen_attention(q, k, v, ti64(cu), ti64(cu), H, D, D ** -0.5)
    y = host(px.linear(o, tbf(wl["w_out"]), t32(wl["b_out"])))

    rows = sampled(n, 384, [0, 12287, 12288, n - 1])
    # oracle: q on the sampled rows, k and v on every row (src/sparse.cpp:337-451,
    # 919-954, 704-783), then the output projection on the sampled rows.
    w_qkv, b_qkv = wl["w_qkv"], wl["b_qkv"]
    qr = orc.mh_rms_norm(orc.linear(x[rows], w_qkv[:C], b_qkv[:C]), H, D, wl["gamma_q"])
    kv = orc.linear(x, w_qkv[C:], b_qkv[C:])
    kk = orc.mh_rms_norm(kv[:, :C], H, D, wl["gamma_k"])
    qf = np.zeros((n, C), np.float32)
    qf[rows] = qr
    att = orc.varlen_attention(qf, kk, kv[:, C:], cu, cu, H, D, np.float32(D ** -0.5), rows=rows)
    ref = orc.linear(att[rows], wl["w_out"], wl["b_out"])
    assert np.isfinite(y).all()
    assert_bf16(y[rows], ref, what="attention block full size")


# --- shifted-window attention and the subdivide up-conv at 64^3 -------------------

@pytest.mark.parametrize("shift", [0, 4])
def test_window_attention_full_size(px, orc, shift):
    """Window attention 12 x 64 over the full window partition of the ~30k-voxel
    shell workload: the device partition (bit-exact against the oracle's) drives
    the kernel through row_map; the oracle runs the reference attention window by
    window over the permuted rows.  Sampled rows cover windows of one key tile
    and of several, and the kernel's padded segment tail."""
    wl = W.swin_64()
    coords = wl["coords"]
    n = coords.shape[0]
    H, D = wl["heads"], wl["head_dim"]
    C = H * D
    q = W.bf16_round(W.normal(81, n * C, 1).reshape(n, C))
    k = W.bf16_round(W.normal(81, n * C, 2).reshape(n, C))
    v = W.bf16_round(W.normal(81, n * C, 3).reshape(n, C))
    print(f"[window attention full] n={n} shift={shift}", flush=True)
    fwd, bwd, cu, nwin = px.window_partition(ti32(coords), 1, wl["shape"], wl["window"], shift)
    rfwd, rbwd, rcu = orc.window_partition(coords, wl["shape"], wl["window"], shift)
    np.testing.assert_array_equal(fwd.cpu().numpy()[:n], rfwd)
    np.testing.assert_array_equal(cu.cpu().numpy()[:nwin + 1], rcu)
    lens = np.diff(rcu)
    assert nwin > 200 and lens.max() > 128 and (lens < 64).any()
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), cu, cu, H, D, 0.125, row_map=fwd,
                                 nseg=nwin))
    # permuted rows to check: every 4th, plus all rows of the longest window and
    # of the shortest multi-row window
    big, small = int(np.argmax(lens)), int(np.argmin(np.where(lens > 1, lens, n)))
    prow = sampled(n, n // 4, np.concatenate([np.arange(rcu[big], rcu[big + 1]),
                                              np.arange(rcu[small], rcu[small + 1])]))
    ro = orc.varlen_attention(q[rfwd], k[rfwd], v[rfwd], rcu, rcu, H, D, np.float32(0.125),
                              rows=prow)
    assert_bf16(o[rfwd[prow]], ro[prow], what=f"window attention shift {shift}")


def test_subdivide_upconv_full_size(px, orc):
    """SubMConv3d 768 -> 8 x 192 on the ~30k voxels at 64^3 (128 x 256 tiles):
    sampled rows in float64 and the exact centre identity; then the device
    channel-to-spatial to 128^3 equals the oracle's bit for bit."""
    wl = W.swin_64()
    coords = wl["coords"]
    n = coords.shape[0]
    x, w = wl["x"], wl["w_up"]
    cout = w.shape[1]
    print(f"[subdivide up-conv full] n={n} cout={cout}", flush=True)
    c = ti32(coords)
    nbr, masks = px.neighbor_map_grid(c, 1, wl["shape"])
    xb = tbf(x)
    y = px.subm_conv3d(xb, tbf(w), t32(wl["b_up"]), nbr, masks)
    yh = host(y)
    idx = nbr.cpu().numpy()
    np.testing.assert_array_equal(idx, orc.neighbor_map(coords))
    rows = sampled(n, 500)
    ref = np.tile(wl["b_up"].astype(np.float64), (rows.size, 1))
    for kk in range(27):
        src = idx[kk, rows]
        ok = src != n
        ref[ok] += x[src[ok]].astype(np.float64) @ w[kk].astype(np.float64).T
    assert_bf16(yh[rows], ref, what="up-conv sampled")
    eye = np.zeros((27, cout, 768), np.float32)
    eye[13, :768] = np.eye(768, dtype=np.float32)
    yi = host(px.subm_conv3d(xb, tbf(eye), t32(np.zeros(cout)), nbr, masks))
    np.testing.assert_array_equal(yi[:, :768], host(xb))
    assert not yi[:, 768:].any()
    oc, of = px.channel_to_spatial(c, y)
    rco, rcf = orc.channel_to_spatial(coords, yh, 2)
    np.testing.assert_array_equal(oc.cpu().numpy(), rco)
    np.testing.assert_array_equal(host(of), rcf)


# --- SLat-flow block and forward at width 1024 on ~42k voxels ---------------------

BLOCK_SHAPES = lambda C, M, CC: [  # noqa: E731  (SparseTransformerBlockWeightsF32 order)
    (6 * C,), (3 * C, C), (3 * C,), (C,), (C,), (C, C), (C,), (C,), (C,), (C, C), (C,),
    (2 * C, CC), (2 * C,), (C,), (C,), (C, C), (C,), None, None, (M, C), (M,), (C, M), (C,)]


def normal(rng, shape, std=1.0):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def flow_block_weights(rng, C, M, CC):
    """N(0, 0.02) linear weights (bf16-rounded), N(0, 0.02) biases and modulation,
    RMS / layer-norm gains 1 + N(0, 0.1)."""
    out = []
    for i, shape in enumerate(BLOCK_SHAPES(C, M, CC)):
        if shape is None:
            out.append(None)
            continue
        if i in (3, 4, 7, 13, 14):
            a = (1.0 + normal(rng, shape, 0.1)).astype(np.float32)
        else:
            a = normal(rng, shape, 0.02)
        out.append(W.bf16_round(a) if i in pxs.BLOCK_LINEAR_WEIGHTS else a)
    return out


def test_flow_block_full_size_sampled_rows(px, orc):
    """One transformer block of the SLat flow (width 1024, 16 x 64, MLP 4096,
    RoPE, q/k RMS norms, cross-attention to 1,370 tokens) on the ~42k voxels of
    the flow workload, bf16 GEMM operands: sampled rows against the oracle block
    (src/sparse_transformer.cpp:138-292)."""
    wl = W.flow_step_64()
    coords = wl["coords"]
    n, C, H, M, T = coords.shape[0], wl["width"], wl["heads"], wl["mlp_hidden"], wl["context_tokens"]
    rng = np.random.default_rng(91)  # host inputs shared by device and oracle
    ws = flow_block_weights(rng, C, M, C)
    x = normal(rng, (n, C))
    tmod = normal(rng, (1, 6 * C), 0.3)
    ctx = W.bf16_round(normal(rng, (T, C)))
    print(f"[flow block full] n={n} tokens={T}", flush=True)
    dws = [None if w is None else (tbf(w) if i in pxs.BLOCK_LINEAR_WEIGHTS else t32(w))
           for i, w in enumerate(ws)]
    cfg = pxs.BlockConfig(C, H, M, C, 0, 1e-6, 1.0, 10000.0, 1, 1, 1, 0)
    c = ti32(coords)
    hidden = t32(x).clone()
    px.transformer_block(cfg, pxs.block_weights(dws), c, 1, px.batch_cu_seqlens(c, 1), hidden,
                         t32(tmod), tbf(ctx), ti64([0, T]))
    got = host(hidden)
    assert np.isfinite(got).all()
    rows = sampled(n, 192, [0, n - 1])
    ref = orc.transformer_block(coords, 1, x, tmod, ctx, [0, T], [C, H, M, C, 0, 1, 1, 1, 0],
                                [1e-6, 1.0, 10000.0], ws, rows=rows)
    # the block adds its update to the residual stream: compare the update
    assert_bf16(got[rows] - x[rows], ref[rows] - x[rows], what="flow block update")


def test_flow_forward_full_size_24_blocks(px):
    """The 24-block SLat-flow forward (input 8 -> 1024, timestep MLP and adaLN,
    24 blocks, final layer norm, output 1024 -> 8) on ~42k voxels with 1,370
    context tokens and random N(0, 0.02) weights: finite, and bit-identical
    when run twice."""
    wl = W.flow_step_64()
    coords = ti32(wl["coords"])
    n, C, H, M, T, nb = (coords.shape[0], wl["width"], wl["heads"], wl["mlp_hidden"],
                         wl["context_tokens"], wl["blocks"])
    g = torch.Generator(device=dev()).manual_seed(93)
    rnd = lambda *s, dt=torch.bfloat16: (torch.randn(*s, generator=g, device=dev()) * 0.02).to(dt)  # noqa: E731
    one = lambda c: torch.ones(c, device=dev())  # noqa: E731
    zero = lambda c: torch.zeros(c, device=dev())  # noqa: E731
    keep, blocks = [], []
    for _ in range(nb):
        ws = [rnd(6 * C, dt=torch.float32), rnd(3 * C, C), zero(3 * C), one(C), one(C),
              rnd(C, C), zero(C), one(C), zero(C), rnd(C, C), zero(C), rnd(2 * C, C),
              zero(2 * C), one(C), one(C), rnd(C, C), zero(C), None, None, rnd(M, C), zero(M),
              rnd(C, M), zero(C)]
        keep.append(ws)
        blocks.append(pxs.block_weights(ws))
    fw = [rnd(C, 8, dt=torch.float32), zero(C), rnd(C, 256, dt=torch.float32), zero(C),
          rnd(C, C, dt=torch.float32), zero(C), rnd(6 * C, C, dt=torch.float32), zero(6 * C),
          rnd(8, C, dt=torch.float32), zero(8)]
    arr = (pxs.BlockWeights * nb)(*blocks)
    weights = pxs.FlowWeights(*[t.data_ptr() for t in fw], arr)
    cfg = pxs.FlowConfig(8, 8, C, C, nb, H, 0, M, 1e-6, 1.0, 10000.0, 1, 1, 0)
    ctx = torch.randn(T, C, generator=g, device=dev()).to(torch.bfloat16)
    x = torch.randn(n, 8, generator=g, device=dev())
    t = torch.tensor([437.5], device=dev())
    cu = px.batch_cu_seqlens(coords, 1)
    print(f"[flow forward full] n={n} blocks={nb}", flush=True)
    out1 = host(px.slat_flow_forward(cfg, weights, coords, 1, cu, x, t, ctx, ti64([0, T]),
                                     dtype=pxs.PXS_BF16))
    out2 = host(px.slat_flow_forward(cfg, weights, coords, 1, cu, x, t, ctx, ti64([0, T]),
                                     dtype=pxs.PXS_BF16))
    assert out1.shape == (n, 8) and np.isfinite(out1).all() and np.abs(out1).max() > 0
    np.testing.assert_array_equal(out1, out2)
