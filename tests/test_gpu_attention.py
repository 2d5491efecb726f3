"""GPU parity: varlen flash attention (fp32 and bf16), cross attention, window
attention over the GPU window partition."""

import json
from pathlib import Path

import numpy as np
import pytest

import oracle as O
import workloads as W
from gpu_common import assert_bf16, assert_fp32, host, t32, tbf, ti32, ti64

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def px():
    import pxs
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


def test_attention_reference_kat(px):
    from test_oracle import kat_inputs
    gold = json.loads((GOLD / "sparse_numeric_fixture.json").read_text())
    a = kat_inputs()
    cu = ti64([0, 5, 10])
    o = px.varlen_attention(t32(a["q"]), t32(a["k"]), t32(a["v"]), cu, cu, 2, 6, 0.37)
    assert_fp32(host(o).ravel(), np.array(gold["sparse_attention_output"]), what="KAT sdpa")
    o = px.varlen_attention(t32(a["q"]), t32(a["ck"]), t32(a["cv"]), cu, ti64([0, 3, 5]), 2, 6, 0.29)
    assert_fp32(host(o).ravel(), np.array(gold["sparse_cross_output"]), what="KAT cross")


def test_attention_reference_vectors(px):
    v = dict(np.load(GOLD / "ref_vectors.npz"))
    cu = ti64([0, 37, 101, 106])
    o = px.varlen_attention(t32(v["attn_q"]), t32(v["attn_k"]), t32(v["attn_v"]), cu, cu, 2, 16, 0.25)
    assert_fp32(host(o), v["attn_out"], what="sdpa vs reference")
    o = px.varlen_attention(t32(v["attn_q"]), t32(v["cross_k"]), t32(v["cross_v"]), cu,
                            ti64(v["cross_offsets"]), 2, 16, 0.25)
    assert_fp32(host(o), v["cross_out"], what="cross vs reference")


@pytest.mark.parametrize("lens,heads,hd", [((100, 300, 7), 3, 64), ((513, 64), 2, 32),
                                           ((1, 2, 129), 1, 8)])
def test_attention_fp32_random(px, orc, lens, heads, hd):
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n = int(cu[-1])
    C = heads * hd
    q = W.normal(61, n * C, 1).reshape(n, C)
    k = W.normal(61, n * C, 2).reshape(n, C)
    v = W.normal(61, n * C, 3).reshape(n, C)
    scale = 1.0 / np.sqrt(hd)
    print(f"[attn fp32] lens={lens} heads={heads} hd={hd}", flush=True)
    o = host(px.varlen_attention(t32(q), t32(k), t32(v), ti64(cu), ti64(cu), heads, hd, scale))
    assert_fp32(o, orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(scale)), what="attn")


def test_attention_bf16_random(px, orc):
    lens = (1000, 1536, 77)
    heads, hd = 4, 64
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n, C = int(cu[-1]), heads * hd
    q = W.bf16_round(W.normal(62, n * C, 1).reshape(n, C))
    k = W.bf16_round(W.normal(62, n * C, 2).reshape(n, C))
    v = W.bf16_round(W.normal(62, n * C, 3).reshape(n, C))
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), ti64(cu), ti64(cu), heads, hd, 0.125))
    assert_bf16(o, orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(0.125)), what="bf16 attn")


@pytest.mark.parametrize("jump", [4.0, 40.0, 400.0])
def test_attention_bf16_late_score_jump(px, orc, jump):
    """Keys after the first 64 score far above the first tile's maximum
    (scores scaled by `jump`): the kernel keeps the first tile's max as its
    reference and must renormalize when a later tile would overflow."""
    lens = (700, 260)
    heads, hd = 2, 64
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n, C = int(cu[-1]), heads * hd
    q = W.bf16_round(W.normal(64, n * C, 1).reshape(n, C))
    k = W.normal(64, n * C, 2).reshape(n, C)
    for b in range(len(lens)):
        k[cu[b] + 64:cu[b + 1]] *= jump
    k = W.bf16_round(k)
    v = W.bf16_round(W.normal(64, n * C, 3).reshape(n, C))
    print(f"[attn bf16 jump] jump={jump}", flush=True)
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), ti64(cu), ti64(cu), heads, hd, 0.125))
    assert np.isfinite(o).all()
    assert_bf16(o, orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(0.125)),
                what=f"bf16 attn jump {jump}")


def test_attention_bf16_full_size_sampled_rows(px, orc):
    """Full attention at full size (12,288 + 20,480 tokens, 16 x 64),
    checked exactly on sampled query rows by the oracle."""
    wl = W.attn_full()
    n, C = wl["x"].shape
    heads, hd = 16, 64
    # Post-RMS-norm-like inputs: unit-norm heads scaled by sqrt(d).
    q = W.bf16_round(W.normal(63, n * C, 1).reshape(n, C))
    k = W.bf16_round(W.normal(63, n * C, 2).reshape(n, C))
    v = W.bf16_round(W.normal(63, n * C, 3).reshape(n, C))
    cu = wl["cu_seqlens"]
    print(f"[attn bf16 full] n={n}", flush=True)
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), ti64(cu), ti64(cu), heads, hd, 0.125))
    rows = np.concatenate([np.arange(0, 12288, 97), np.arange(12288, n, 151), [12287, n - 1]])
    ref = orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(0.125), rows=rows)
    assert_bf16(o[rows], ref[rows], what="attn full sampled")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("shift", [0, 4])
def test_window_attention(px, orc, dtype, shift):
    coords = W.shell_coords(32, [[(8.0, 14.0)], [(6.0, 12.0)]], 64)
    n = coords.shape[0]
    heads, hd = 3, 64
    C = heads * hd
    q = W.bf16_round(W.normal(64, n * C, 1).reshape(n, C))
    k = W.bf16_round(W.normal(64, n * C, 2).reshape(n, C))
    v = W.bf16_round(W.normal(64, n * C, 3).reshape(n, C))
    fwd, bwd, cu, nwin = px.window_partition(ti32(coords), 2, (32, 32, 32), 8, shift)
    conv = t32 if dtype == "f32" else tbf
    o = host(px.varlen_attention(conv(q), conv(k), conv(v), cu, cu, heads, hd, 0.125,
                                 row_map=fwd, nseg=nwin))
    # Reference: permute rows by the oracle partition, run reference-order
    # attention per window, un-permute.
    rfwd, rbwd, rcu = orc.window_partition(coords, (32, 32, 32), 8, shift)
    ro = orc.varlen_attention(q[rfwd], k[rfwd], v[rfwd], rcu, rcu, heads, hd, np.float32(0.125))
    ref = ro[rbwd]
    (assert_fp32 if dtype == "f32" else assert_bf16)(o, ref, what=f"window {dtype}")


def test_attention_empty_key_segment_gives_zeros(px):
    q = W.normal(65, 10 * 64, 1).reshape(10, 64)
    k = W.normal(65, 4 * 64, 2).reshape(4, 64)
    o = host(px.varlen_attention(t32(q), t32(k), t32(k), ti64([0, 6, 10]), ti64([0, 4, 4]), 1, 64, 0.125))
    assert np.all(o[6:] == 0) and np.all(np.isfinite(o))


@pytest.mark.parametrize("jump", [1.0, 40.0])
def test_attention_bf16_hd128_tiled(px, orc, jump):
    """bf16 head_dim 128 on the tiled MFMA kernel (32-key tiles of two
    64-dim halves): segments ending mid-tile, one shorter than a tile, keys
    after the first tile scored up to 40x higher (the lazy-max rescale),
    against the oracle."""
    lens = (1000, 1536, 77, 31)
    heads, hd = 3, 128
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n, C = int(cu[-1]), heads * hd
    q = W.bf16_round(W.normal(67, n * C, 1).reshape(n, C))
    k = W.normal(67, n * C, 2).reshape(n, C)
    for b in range(len(lens)):
        k[cu[b] + 32:cu[b + 1]] *= jump
    k = W.bf16_round(k)
    v = W.bf16_round(W.normal(67, n * C, 3).reshape(n, C))
    scale = hd ** -0.5
    print(f"[attn bf16 hd128] jump={jump}", flush=True)
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), ti64(cu), ti64(cu), heads, hd, scale))
    assert np.isfinite(o).all()
    assert_bf16(o, orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(scale)),
                what=f"bf16 attn hd128 jump {jump}")


def test_attention_bf16_hd128_full_size_sampled_rows(px, orc):
    """Config 3's tokens (12,288 + 20,480) at 8 heads x 128, sampled query
    rows against the oracle."""
    wl = W.attn_full()
    n = wl["x"].shape[0]
    heads, hd = 8, 128
    C = heads * hd
    q = W.bf16_round(W.normal(68, n * C, 1).reshape(n, C))
    k = W.bf16_round(W.normal(68, n * C, 2).reshape(n, C))
    v = W.bf16_round(W.normal(68, n * C, 3).reshape(n, C))
    cu = wl["cu_seqlens"]
    scale = hd ** -0.5
    print(f"[attn bf16 hd128 full] n={n}", flush=True)
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), ti64(cu), ti64(cu), heads, hd, scale))
    rows = np.concatenate([np.arange(0, 12288, 131), np.arange(12288, n, 173), [12287, n - 1]])
    ref = orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(scale), rows=rows)
    assert_bf16(o[rows], ref[rows], what="attn hd128 full sampled")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("hd,vd", [(128, 128), (96, 160), (200, 40)])
def test_attention_wide_heads(px, orc, dtype, hd, vd):
    """Heads wider than 64 (the drop-in's reference API allows any width):
    self-attention over three segments, cross-attention with one empty key
    segment, and a permuted row order, against the oracle."""
    lens, klens = (300, 77, 1), (50, 0, 130)
    heads = 2
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    cuk = np.concatenate([[0], np.cumsum(klens)]).astype(np.int64)
    n, nk = int(cu[-1]), int(cuk[-1])
    rnd = lambda rows, w, s: W.bf16_round(W.normal(66, rows * w, s).reshape(rows, w))  # noqa: E731
    q, k, v = rnd(n, heads * hd, 1), rnd(n, heads * hd, 2), rnd(n, heads * vd, 3)
    ck, cv = rnd(nk, heads * hd, 4), rnd(nk, heads * vd, 5)
    conv = t32 if dtype == "f32" else tbf
    check = assert_fp32 if dtype == "f32" else assert_bf16
    scale = float(hd) ** -0.5
    print(f"[attn wide] dtype={dtype} hd={hd} vd={vd}", flush=True)
    o = host(px.varlen_attention(conv(q), conv(k), conv(v), ti64(cu), ti64(cu), heads, hd, scale,
                                 value_dim=vd))
    check(o, orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(scale)), what="wide self")
    o = host(px.varlen_attention(conv(q), conv(ck), conv(cv), ti64(cu), ti64(cuk), heads, hd,
                                 scale, value_dim=vd))
    ref = orc.varlen_attention(q, ck, cv, cu, cuk, heads, hd, np.float32(scale))
    assert np.all(o[cu[1]:cu[2]] == 0)
    check(o, ref, what="wide cross")
    perm = np.random.default_rng(7).permutation(n).astype(np.int32)
    o = host(px.varlen_attention(conv(q), conv(k), conv(v), ti64(cu), ti64(cu), heads, hd, scale,
                                 row_map=ti32(perm), value_dim=vd))
    ref = orc.varlen_attention(q[perm], k[perm], v[perm], cu, cu, heads, hd, np.float32(scale))
    check(o[perm], ref, what="wide permuted")


@pytest.mark.parametrize("permuted", [False, True])
def test_attention_bf16_short_segment_kernel(px, orc, permuted):
    """Segments whose mean length selects the short-segment kernel, with
    lengths on either side of its 64-key chunks and 128-query passes, an
    empty segment, a single row, and one segment longer than its 512-row
    staging (read through the row map in global memory)."""
    lens = (700, 1, 0, 63, 64, 65, 128, 129, 200, 511, 512)
    heads, hd = 3, 64
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n, C = int(cu[-1]), heads * hd
    assert n <= 512 * len(lens)
    q = W.bf16_round(W.normal(67, n * C, 1).reshape(n, C))
    k = W.bf16_round(W.normal(67, n * C, 2).reshape(n, C))
    v = W.bf16_round(W.normal(67, n * C, 3).reshape(n, C))
    perm = np.random.default_rng(8).permutation(n).astype(np.int32) if permuted else None
    print(f"[attn short segments] permuted={permuted}", flush=True)
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), ti64(cu), ti64(cu), heads, hd, 0.125,
                                 row_map=None if perm is None else ti32(perm)))
    if perm is None:
        ref = orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(0.125))
        assert_bf16(o, ref, what="short segments")
    else:
        ref = orc.varlen_attention(q[perm], k[perm], v[perm], cu, cu, heads, hd, np.float32(0.125))
        assert_bf16(o[perm], ref, what="short segments permuted")


def test_attention_bf16_many_short_segments(px, orc):
    """More segments than the short-segment kernel sorts by cost (65,536):
    the unsorted launch, over segments of 0 to 3 rows."""
    lens = np.random.default_rng(9).integers(0, 4, 70000)
    heads, hd = 1, 64
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n, C = int(cu[-1]), heads * hd
    q = W.bf16_round(W.normal(68, n * C, 1).reshape(n, C))
    k = W.bf16_round(W.normal(68, n * C, 2).reshape(n, C))
    v = W.bf16_round(W.normal(68, n * C, 3).reshape(n, C))
    print(f"[attn many segments] nseg={len(lens)} n={n}", flush=True)
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), ti64(cu), ti64(cu), heads, hd, 0.125))
    assert_bf16(o, orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(0.125)),
                what="many short segments")


def _peaked_qk(family, gain, n, C, seed):
    """Q and K whose logits are far sharper than unit Gaussians give: scaled
    Gaussians, rows RMS-normalised then scaled (as after a QK norm), and keys
    near one shared direction with a large norm (big common logit, small
    differences)."""
    rng = np.random.default_rng(seed)
    if family == "gaussian":
        q, k = rng.standard_normal((n, C)) * gain, rng.standard_normal((n, C)) * gain
    elif family == "rms":
        q, k = rng.standard_normal((n, C)), rng.standard_normal((n, C))
        q = gain * q / np.sqrt((q * q).mean(1, keepdims=True))
        k = gain * k / np.sqrt((k * k).mean(1, keepdims=True))
    else:
        u = rng.standard_normal(C)
        q = gain * (u + 0.1 * rng.standard_normal((n, C)))
        k = gain * (u + 0.1 * rng.standard_normal((n, C)))
    return W.bf16_round(q.astype(np.float32)), W.bf16_round(k.astype(np.float32))


@pytest.mark.parametrize("lens", [(1300, 200), (150, 90, 200)], ids=["long", "short"])
@pytest.mark.parametrize("family,gain", [("gaussian", 8.0), ("gaussian", 16.0), ("rms", 16.0),
                                         ("near_dup", 64.0)])
def test_attention_bf16_peaked_logits(px, orc, lens, family, gain):
    """Sharply peaked logits (scores tens to hundreds of units apart): the
    scores must reach the exponent at fp32 precision.  Rounding q * scale to
    bf16 before QK^T, for one, gives 1.1e-2 to 4.5e-2 relative L2 on such
    inputs, while exact fp32 scores give about 1e-4 plus the bf16 rounding of
    the output (about 1.1e-3), hence the bound of 5e-3 here.  The long
    segments run the long-segment kernel, the short ones the per-segment
    kernel."""
    heads, hd = 2, 64
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n, C = int(cu[-1]), heads * hd
    q, k = _peaked_qk(family, gain, n, C, 21)
    v = W.bf16_round(W.normal(69, n * C, 3).reshape(n, C))
    print(f"[attn peaked] {family} gain={gain} lens={lens}", flush=True)
    o = host(px.varlen_attention(tbf(q), tbf(k), tbf(v), ti64(cu), ti64(cu), heads, hd, 0.125))
    assert np.isfinite(o).all()
    assert_bf16(o, orc.varlen_attention(q, k, v, cu, cu, heads, hd, np.float32(0.125)),
                tol=5e-3, what=f"peaked {family} {gain}")
