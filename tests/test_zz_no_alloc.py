"""pxs_varlen_attention_noalloc, the attention entry point that allocates
nothing (its scratch is a static device array), against pxs_varlen_attention
with a caller workspace: bit-identical outputs on two calls in a row, the
second smaller, so a stale scratch from the first call cannot leak into it."""

import ctypes as C

import numpy as np
import pytest
import torch

import pxs
import workloads as W
from gpu_common import host, t32, tbf, ti32, ti64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def px():
    return pxs.Pxs()


def noalloc(px, q, k, v, cu_q, cu_k, heads, hd, scale, row_map=None, nseg=None):
    nseg = cu_q.shape[0] - 1 if nseg is None else nseg
    o = torch.empty((q.shape[0], heads * hd), dtype=q.dtype, device=q.device)
    p = lambda t: C.c_void_p(t.data_ptr() if t is not None else 0)  # noqa: E731
    dt = pxs.PXS_BF16 if q.dtype == torch.bfloat16 else pxs.PXS_F32
    rc = px.lib.pxs_varlen_attention_noalloc(dt, p(q), q.stride(0), p(k), k.stride(0), p(v),
                                             v.stride(0), p(cu_q), p(cu_k), nseg, q.shape[0],
                                             p(row_map), heads, hd, hd, scale, p(o), o.stride(0),
                                             px.stream())
    assert rc == 0, px.lib.pxs_last_error().decode()
    return o


def inputs(lens, heads, hd, seed, dtype):
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    n = int(cu[-1])
    conv = tbf if dtype == "bf16" else t32
    q, k, v = (conv(W.normal(seed, n * heads * hd, s).reshape(n, heads * hd)) for s in (1, 2, 3))
    return q, k, v, ti64(cu)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_noalloc_attention_matches_workspace_entry_point(px, dtype):
    heads, hd = 4, 64
    for lens, seed in (((3000, 700, 1, 4100, 64), 71), ((129, 5, 300), 72)):
        print(f"[noalloc attention] dtype={dtype} lens={lens}", flush=True)
        q, k, v, cu = inputs(lens, heads, hd, seed, dtype)
        got = noalloc(px, q, k, v, cu, cu, heads, hd, 0.125)
        want = px.varlen_attention(q, k, v, cu, cu, heads, hd, 0.125)
        np.testing.assert_array_equal(host(got), host(want))


def test_noalloc_window_attention_matches_workspace_entry_point(px):
    """Many segments (a window partition) and a permuted row order, then a
    smaller partition."""
    heads, hd = 3, 64
    for grid, seed in ((32, 73), (16, 74)):
        coords = W.shell_coords(grid, [[(grid / 4, grid / 2.3)]], seed)
        n = coords.shape[0]
        print(f"[noalloc window] n={n}", flush=True)
        fwd, bwd, cu, nwin = px.window_partition(ti32(coords), 1, (grid,) * 3, 8, 4)
        q, k, v = (tbf(W.normal(seed, n * heads * hd, s).reshape(n, heads * hd)) for s in (1, 2, 3))
        got = noalloc(px, q, k, v, cu, cu, heads, hd, 0.125, row_map=fwd, nseg=nwin)
        want = px.varlen_attention(q, k, v, cu, cu, heads, hd, 0.125, row_map=fwd, nseg=nwin)
        np.testing.assert_array_equal(host(got), host(want))


def test_noalloc_attention_rejects_too_many_segments(px):
    rc = px.lib.pxs_varlen_attention_noalloc(pxs.PXS_BF16, None, 64, None, 64, None, 64, None,
                                             None, pxs.PXS_ATTN_NOALLOC_MAX_SEGMENTS + 1, 1, None,
                                             1, 64, 64, 0.125, None, 64, None)
    assert rc == pxs.PXS_ERR_ARG
    assert "PXS_ATTN_NOALLOC_MAX_SEGMENTS" in px.lib.pxs_last_error().decode()
