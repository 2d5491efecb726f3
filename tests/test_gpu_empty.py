"""GPU: zero-row inputs.  The reference accepts empty sparse tensors (no
rows) in every primitive and returns empty outputs; each device entry point
must do the same (PXS_OK, nothing written, nothing launched that could fail).
Each case names the entry point it drives."""

import numpy as np
import pytest
import torch

import pxs
from gpu_common import dev, t32, ti32, ti64

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def px():
    return pxs.Pxs()


def empty(shape, dtype=torch.float32):
    return torch.empty(shape, dtype=dtype, device=dev())


CASES = {}


def case(fn):
    CASES[fn.__name__] = fn
    return fn


@case
def hash_validate_and_maps(px):
    c = empty((0, 4), torch.int32)
    assert px.validate(c, 1, (8, 8, 8)) == (0, -1)
    nbr, masks = px.neighbor_map(c)
    assert nbr.shape == (27, 0)
    nbr, masks = px.neighbor_map_grid(c, 1, (8, 8, 8))
    assert nbr.shape == (27, 0)
    _, _, offs = px.neighbor_pairs(nbr)
    assert offs.cpu().numpy().tolist() == [0] * 28


@case
def cu_seqlens(px):
    cu = px.batch_cu_seqlens(empty((0, 4), torch.int32), 3)
    assert cu.cpu().numpy().tolist() == [0, 0, 0, 0]


@case
def downsample_topologies(px):
    c = empty((0, 4), torch.int32)
    oc, child, m = px.downsample_s2(c, 1, (8, 8, 8))
    assert m == 0
    res = px.downsample(c, 1, (8, 8, 8), 2)
    assert res[-1] == 0


@case
def tagged_grid_topology(px):
    c = empty((0, 4), torch.int32)
    grid = px.tagged_grid(1, (8, 8, 8))
    px.tagged_insert(c, 1, (8, 8, 8), grid, 1)
    nbr, _ = px.neighbor_map_tagged(c, 1, (8, 8, 8), grid, 1)
    assert nbr.shape == (27, 0)
    coarse = empty((px.lib.pxs_voxel_grid_bytes(1, 4, 4, 4) // 4,), torch.int32)
    ws = px.s2_tagged_workspace(1, (8, 8, 8))
    assert px.downsample_s2_tagged(c, 1, (8, 8, 8), grid, 1, coarse, ws)[-1] == 0
    nbr, _, _, _, m = px.map_s2_tagged(c, 1, (8, 8, 8), grid, 1, coarse, ws)
    assert m == 0 and nbr.shape == (27, 0)


@case
def window_partition(px):
    res = px.window_partition(empty((0, 4), torch.int32), 1, (16, 16, 16), 8, 4)
    assert res is not None


@case
def convolutions(px):
    x = empty((0, 32), torch.bfloat16)
    w = torch.zeros((27, 48, 32), dtype=torch.bfloat16, device=dev())
    b = torch.zeros(48, device=dev())
    nbr = empty((27, 0), torch.int32)
    masks = empty((0,), torch.int32)
    y = px.subm_conv3d(x, w, b, nbr, masks)
    assert y.shape[0] == 0
    ws2 = torch.zeros((8, 48, 32), dtype=torch.bfloat16, device=dev())
    y = px.sparse_conv3d_s2(x, ws2, b, empty((8, 0), torch.int32), 0)
    assert y.shape[0] == 0


@case
def linears_and_norms(px):
    for dt in (torch.float32, torch.bfloat16):
        x = empty((0, 64), dt)
        w = torch.zeros((96, 64), dtype=dt, device=dev())
        assert px.linear(x, w, torch.zeros(96, device=dev())).shape == (0, 96)
        assert px.layer_norm(x, 1e-6).shape == (0, 64)
        assert px.mh_rms_norm(x, 2, 32, torch.ones(64, device=dev())).shape == (0, 64)
        px.activation(x, pxs.ACT_SILU)
    x = empty((0, 16))
    assert px.linear_ordered(x, torch.zeros((8, 16), device=dev())).shape == (0, 8)


@case
def rope_and_qkv(px):
    c = empty((0, 4), torch.int32)
    x = empty((0, 128), torch.bfloat16)
    assert px.rope(c, x, 2, 64).shape == (0, 128)
    qkv = empty((0, 384), torch.bfloat16)
    q, k, v = px.qkv_prepare(qkv, 2, 64, coords=c)
    assert q.shape == (0, 128)


@case
def attention(px):
    q = empty((0, 128), torch.bfloat16)
    cu = ti64(np.array([0, 0], np.int64))
    o = px.varlen_attention(q, q, q, cu, cu, 2, 64, 0.125)
    assert o.shape == (0, 128)


@case
def channel_to_spatial(px):
    res = px.channel_to_spatial(empty((0, 4), torch.int32), empty((0, 64)))
    assert res[0].shape[0] == 0


@pytest.mark.parametrize("name", list(CASES))
def test_zero_rows(px, name):
    print(f"[empty] {name}", flush=True)
    CASES[name](px)
    torch.cuda.synchronize()
