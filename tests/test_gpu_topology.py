"""GPU parity: voxel hash, validation, neighbor maps, pair lists, stride-2
topology, window partition, cu_seqlens, channel-to-spatial.  All integer
outputs must match the oracle bit for bit."""

import numpy as np
import torch
import pytest

import oracle as O
import workloads as W
from gpu_common import dev, host, t32, ti32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def px():
    import pxs
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


def coord_cases():
    return {
        "conv_fp32_64": (W.conv_fp32_64()["coords"], 1, (64, 64, 64)),
        "unet_stage_128": (W.shell_coords(128, W.UNET_ITEMS, 2), 2, (128, 128, 128)),
        "small_2batch": (W.shell_coords(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 31), 2, (16, 16, 16)),
        "single": (np.array([[0, 3, 3, 3]], np.int32), 1, (8, 8, 8)),
    }


@pytest.mark.parametrize("case", list(coord_cases()))
def test_neighbor_map_bit_exact(px, orc, case):
    coords, batch, shape = coord_cases()[case]
    print(f"[neighbor_map] case={case} n={coords.shape[0]}", flush=True)
    c = ti32(coords)
    nbr, masks = px.neighbor_map(c)
    got = host(nbr).astype(np.int64) if False else nbr.cpu().numpy()
    ref = orc.neighbor_map(coords)
    np.testing.assert_array_equal(got, ref)
    present = (ref != coords.shape[0])
    ref_masks = (present.astype(np.int64) << np.arange(27)[:, None]).sum(0)
    np.testing.assert_array_equal(masks.cpu().numpy().astype(np.int64) & 0x7FFFFFF, ref_masks)
    assert px.validate(c, batch, shape) == (0, -1)


@pytest.mark.parametrize("case", list(coord_cases()) + ["edges"])
def test_neighbor_map_grid_bit_exact(px, orc, case):
    """The dense-grid map equals the oracle's (and so the hash map's) bit for
    bit, including voxels on the grid faces and a coordinate outside the
    extents (never entered; its own row is still its centre)."""
    if case == "edges":
        coords = np.array([[0, 0, 0, 0], [0, 0, 0, 1], [0, 0, 1, 0], [0, 7, 7, 7], [0, 7, 7, 6],
                           [1, 0, 0, 0], [1, 7, 0, 7]], np.int32)
        batch, shape = 2, (8, 8, 8)
    else:
        coords, batch, shape = coord_cases()[case]
    print(f"[neighbor_map_grid] case={case} n={coords.shape[0]}", flush=True)
    nbr, masks = px.neighbor_map_grid(ti32(coords), batch, shape)
    ref = orc.neighbor_map(coords)
    np.testing.assert_array_equal(nbr.cpu().numpy(), ref)
    present = (ref != coords.shape[0])
    ref_masks = (present.astype(np.int64) << np.arange(27)[:, None]).sum(0)
    np.testing.assert_array_equal(masks.cpu().numpy().astype(np.int64) & 0x7FFFFFF, ref_masks)


def _brick_case(case):
    if case in coord_cases():
        return coord_cases()[case][0]
    if case == "edges":
        return np.array([[0, 0, 0, 0], [0, 0, 0, 1], [0, 0, 1, 0], [0, 7, 7, 7], [0, 7, 7, 6],
                         [1, 0, 0, 0], [1, 7, 0, 7], [1, 3, 4, 4], [1, 4, 4, 4], [1, 4, 3, 5]],
                        np.int32)
    if case == "offset_1024":  # the U-Net shells moved up to coordinates near 730
        return W.unet_stage_128()["coords"] + np.array([0, 600, 600, 600], np.int32)
    if case == "spaced":  # every third cell: bricks holding a few voxels, most neighbours absent
        return W.conv_fp32_64()["coords"] * np.array([1, 3, 3, 3], np.int32)
    rng = np.random.default_rng(5)  # "scattered": about one voxel per brick
    pts = np.unique(rng.integers(0, 200, size=(20000, 3)), axis=0)
    return np.ascontiguousarray(np.hstack([np.zeros((len(pts), 1), np.int64), pts]).astype(np.int32))


BRICK_CASES = ["conv_fp32_64", "unet_stage_128", "small_2batch", "single", "edges", "offset_1024",
               "spaced", "scattered"]


@pytest.mark.parametrize("case", BRICK_CASES)
def test_neighbor_map_bricks_bit_exact(px, orc, case):
    """The brick-table map equals the oracle's and the voxel hash's bit for
    bit: grid faces, brick faces in every direction, several batch items,
    coordinates near 730, sparse bricks and voxels about one per brick."""
    coords = _brick_case(case)
    print(f"[neighbor_map_bricks] case={case} n={coords.shape[0]}", flush=True)
    c = ti32(coords)
    nbr, masks = px.neighbor_map_bricks(c)
    ref = orc.neighbor_map(coords)
    np.testing.assert_array_equal(nbr.cpu().numpy(), ref)
    present = (ref != coords.shape[0])
    ref_masks = (present.astype(np.int64) << np.arange(27)[:, None]).sum(0)
    np.testing.assert_array_equal(masks.cpu().numpy().astype(np.int64) & 0x7FFFFFF, ref_masks)
    hnbr, hmasks = px.neighbor_map(c)
    np.testing.assert_array_equal(nbr.cpu().numpy(), hnbr.cpu().numpy())
    np.testing.assert_array_equal(masks.cpu().numpy(), hmasks.cpu().numpy())


def test_neighbor_map_bricks_duplicates_keep_smallest_row(px):
    """A repeated coordinate resolves to its smallest row, as in the voxel hash."""
    coords = np.array([[0, 5, 5, 5], [0, 5, 5, 6], [0, 5, 5, 5], [0, 6, 5, 5], [0, 5, 5, 6]],
                      np.int32)
    c = ti32(coords)
    nbr, masks = px.neighbor_map_bricks(c)
    hnbr, hmasks = px.neighbor_map(c)
    np.testing.assert_array_equal(nbr.cpu().numpy(), hnbr.cpu().numpy())
    np.testing.assert_array_equal(masks.cpu().numpy(), hmasks.cpu().numpy())


def test_neighbor_map_grid_skips_out_of_extent_rows(px):
    coords = np.array([[0, 1, 1, 1], [0, 1, 1, 2], [0, 9, 1, 1]], np.int32)  # x = 9 >= 8
    nbr, masks = px.neighbor_map_grid(ti32(coords), 1, (8, 8, 8))
    nb = nbr.cpu().numpy()
    assert nb[13].tolist() == [0, 1, 2]          # centres
    assert nb[14, 0] == 1 and nb[12, 1] == 0     # z neighbours inside the extents
    assert (np.delete(nb[:, 2], 13) == 3).all()  # the outside row sees no neighbour


@pytest.mark.parametrize("case", ["conv_fp32_64", "small_2batch"])
def test_neighbor_pairs_bit_exact(px, orc, case):
    coords, _, _ = coord_cases()[case]
    print(f"[neighbor_pairs] case={case}", flush=True)
    nbr, _ = px.neighbor_map(ti32(coords))
    pin, pout, offs = px.neighbor_pairs(nbr)
    rin, rout, roffs = orc.neighbor_pairs(orc.neighbor_map(coords))
    np.testing.assert_array_equal(offs.cpu().numpy(), roffs)
    np.testing.assert_array_equal(pin.cpu().numpy(), rin)
    np.testing.assert_array_equal(pout.cpu().numpy(), rout)


def test_validation_first_error_matches_oracle(px, orc):
    base = W.shell_coords(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 32)
    n = base.shape[0]
    feats = W.normal(32, n * 5, 1).reshape(n, 5)
    cases = []
    dup = base.copy(); dup[n // 2] = dup[n // 3]; cases.append(("duplicate", dup, feats))
    oob = base.copy(); oob[n // 4, 2] = 16; cases.append(("outside", oob, feats))
    neg = base.copy(); neg[7, 1] = -1; cases.append(("negative", neg, feats))
    cont = base.copy(); cont[n - 1, 0] = 0; cases.append(("contiguity", cont, feats))
    nanf = feats.copy(); nanf[n // 5, 3] = np.nan; cases.append(("nan", base, nanf))
    inff = feats.copy(); inff[2, 0] = np.inf; cases.append(("inf", base, inff))
    both = dup.copy(); both[n // 2 + 3, 1] = 99; cases.append(("dup_then_oob", both, nanf))
    for name, coords, f in cases:
        print(f"[validate] case={name}", flush=True)
        got = px.validate(ti32(coords), 2, (16, 16, 16), t32(f))
        ref = orc.sparse_valid(coords, 2, (16, 16, 16), f, 5)
        assert got == ref, (name, got, ref)


@pytest.mark.parametrize("case", ["unet_stage_128", "small_2batch", "single"])
def test_downsample_s2_topology(px, orc, case):
    coords, batch, shape = coord_cases()[case]
    print(f"[downsample_s2] case={case}", flush=True)
    oc, child, m = px.downsample_s2(ti32(coords), batch, shape)
    roc, rchild = orc.downsample_coords_s2(coords)
    assert m == roc.shape[0]
    np.testing.assert_array_equal(oc.cpu().numpy(), roc)
    np.testing.assert_array_equal(child.cpu().numpy()[:, :m], rchild.T)


@pytest.mark.parametrize("shift", [0, 4])
@pytest.mark.parametrize("case", ["swin_64", "small_2batch"])
def test_window_partition_bit_exact(px, orc, case, shift):
    if case == "swin_64":
        coords, batch, shape = W.shell_coords(64, [W.SWIN_SHELLS], 4), 1, (64, 64, 64)
    else:
        coords, batch, shape = coord_cases()[case]
    print(f"[window_partition] case={case} shift={shift}", flush=True)
    fwd, bwd, cu, nwin = px.window_partition(ti32(coords), batch, shape, 8, shift)
    rfwd, rbwd, rcu = orc.window_partition(coords, shape, 8, shift)
    assert nwin == len(rcu) - 1
    np.testing.assert_array_equal(fwd.cpu().numpy(), rfwd)
    np.testing.assert_array_equal(bwd.cpu().numpy(), rbwd)
    np.testing.assert_array_equal(cu.cpu().numpy(), rcu)


def test_window_partition_many_windows(px, orc):
    """Window 4 at 128^3, batch 2: 65,536 windows, past the single-workgroup
    scan (16,384 items), so the three-phase scan runs."""
    coords = W.shell_coords(128, W.UNET_ITEMS, 2)
    print(f"[window_partition] unet_stage_128 window=4 n={coords.shape[0]}", flush=True)
    fwd, bwd, cu, nwin = px.window_partition(ti32(coords), 2, (128, 128, 128), 4, 2)
    rfwd, rbwd, rcu = orc.window_partition(coords, (128, 128, 128), 4, 2)
    assert nwin == len(rcu) - 1
    np.testing.assert_array_equal(fwd.cpu().numpy(), rfwd)
    np.testing.assert_array_equal(bwd.cpu().numpy(), rbwd)
    np.testing.assert_array_equal(cu.cpu().numpy(), rcu)


@pytest.mark.parametrize("window,shift", [(8, 4), (4, 2)])
def test_window_partition_unsorted_rows(px, orc, window, shift):
    """Rows in random order (the stable order then differs from any
    coordinate order), with few windows (aggregated counts, one-workgroup
    offsets) and with 71,874 windows (the multi-kernel path)."""
    coords = W.shell_coords(128, W.UNET_ITEMS, 2)
    coords = coords[np.random.default_rng(10).permutation(coords.shape[0])]
    print(f"[window_partition unsorted] window={window} shift={shift}", flush=True)
    fwd, bwd, cu, nwin = px.window_partition(ti32(coords), 2, (128, 128, 128), window, shift)
    rfwd, rbwd, rcu = orc.window_partition(coords, (128, 128, 128), window, shift)
    assert nwin == len(rcu) - 1
    np.testing.assert_array_equal(fwd.cpu().numpy(), rfwd)
    np.testing.assert_array_equal(bwd.cpu().numpy(), rbwd)
    np.testing.assert_array_equal(cu.cpu().numpy(), rcu)


def test_window_partition_padded_segments(px, orc):
    """Without reading the window count, cu_seqlens up to min(n, windows) ends
    in empty segments, and attention over that bound equals attention over
    the exact count."""
    coords = W.shell_coords(64, [W.SWIN_SHELLS], 4)
    n = coords.shape[0]
    c = ti32(coords)
    fwd, bwd, cu, nwin = px.window_partition(c, 1, (64, 64, 64), 8, 4)
    _, _, cu_b, cap = px.window_partition(c, 1, (64, 64, 64), 8, 4, sync=False)
    assert cap == min(n, 9 ** 3) and cap >= nwin
    cb = cu_b.cpu().numpy()
    np.testing.assert_array_equal(cb[: nwin + 1], cu.cpu().numpy())
    assert (cb[nwin:] == n).all()
    H, D = 2, 64
    g = torch.Generator().manual_seed(5)
    q, k, v = [torch.randn(n, H * D, generator=g).to("cuda").to(torch.bfloat16) for _ in range(3)]
    o1 = px.varlen_attention(q, k, v, cu, cu, H, D, 0.125, row_map=fwd, nseg=nwin)
    o2 = px.varlen_attention(q, k, v, cu_b, cu_b, H, D, 0.125, row_map=fwd, nseg=cap)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(o1.float().cpu().numpy(), o2.float().cpu().numpy())


def test_batch_cu_seqlens(px, orc):
    coords = W.shell_coords(16, [[(4.0, 7.0)], [], [(3.0, 6.0)]], 33)
    cu = px.batch_cu_seqlens(ti32(coords), 4).cpu().numpy()
    np.testing.assert_array_equal(cu, orc.batch_cu_seqlens(coords, 4))


@pytest.mark.parametrize("with_sub", [False, True])
def test_channel_to_spatial(px, orc, with_sub):
    coords = W.shell_coords(16, [[(4.0, 7.0)], [(3.0, 6.0)]], 34)
    n = coords.shape[0]
    x = W.normal(34, n * 24, 1).reshape(n, 24)
    sub = (W.uniform(34, n * 8, 2) > 0.4).astype(np.float32).reshape(n, 8) if with_sub else None
    print(f"[c2s] sub={with_sub}", flush=True)
    oc, y = px.channel_to_spatial(ti32(coords), t32(x), None if sub is None else t32(sub))
    roc, ry = orc.channel_to_spatial(coords, x, 2, sub)
    np.testing.assert_array_equal(oc.cpu().numpy(), roc)
    np.testing.assert_array_equal(host(y), ry)


@pytest.mark.parametrize("factor", [1, 2, 3])
def test_downsample_any_factor(px, orc, factor):
    """Grouped topology and mean for any factor vs the oracle (src/sparse.cpp:536-602)."""
    coords = W.shell_coords(20, [[(5.0, 8.0)], [(4.0, 7.0)]], 35)
    n = coords.shape[0]
    x = W.normal(35, n * 40, 1).reshape(n, 40)
    print(f"[downsample] factor={factor} n={n}", flush=True)
    oc, off, rows, m = px.downsample(ti32(coords), 2, (20, 20, 20), factor)
    y = host(px.downsample_mean(t32(x), off, rows, m))
    roc, ry = orc.downsample_mean(coords, x, factor)
    np.testing.assert_array_equal(oc.cpu().numpy(), roc)
    # Same summation order as the reference: bit-exact.
    np.testing.assert_array_equal(y, ry)
    # Groups list their rows in ascending order.
    o, r = off.cpu().numpy(), rows.cpu().numpy()
    for q in range(m):
        assert np.all(np.diff(r[o[q]:o[q + 1]]) > 0)


def test_downsample_factor2_full_size(px, orc):
    """Factor-2 grouping and mean over the 162,263-row U-Net coordinates
    (group offsets scanned over more rows than one workgroup takes)."""
    coords = W.shell_coords(128, W.UNET_ITEMS, 2)
    n = coords.shape[0]
    x = W.normal(37, n * 8, 1).reshape(n, 8)
    print(f"[downsample] factor=2 n={n}", flush=True)
    oc, off, rows, m = px.downsample(ti32(coords), 2, (128, 128, 128), 2)
    y = host(px.downsample_mean(t32(x), off, rows, m))
    roc, ry = orc.downsample_mean(coords, x, 2)
    np.testing.assert_array_equal(oc.cpu().numpy(), roc)
    np.testing.assert_array_equal(y, ry)


def test_channel_to_spatial_factor3(px, orc):
    coords = W.shell_coords(12, [[(3.0, 5.0)], [(2.0, 4.0)]], 36)
    n = coords.shape[0]
    x = W.normal(36, n * 54, 1).reshape(n, 54)
    sub = (W.uniform(36, n * 27, 2) > 0.5).astype(np.float32).reshape(n, 27)
    oc, y = px.channel_to_spatial(ti32(coords), t32(x), t32(sub), factor=3)
    roc, ry = orc.channel_to_spatial(coords, x, 3, sub)
    np.testing.assert_array_equal(oc.cpu().numpy(), roc)
    np.testing.assert_array_equal(host(y), ry)


def max_extent_coords():
    """Rows at the edges of the largest extents the voxel key holds
    (PXS_MAX_EXTENT = 32768 per axis and for the batch): neighbours across
    x = 32767 / z = 32767 and in the last batch item."""
    M = 32767
    rows = [(0, 0, 0, 0), (0, 0, 0, 1), (0, 0, M, M - 1), (0, 0, M, M), (0, 1, M, M),
            (0, M, 0, 0), (0, M, M, M - 1), (0, M, M, M), (M, M - 1, M, M), (M, M, M, M)]
    return np.array(sorted(rows), np.int32)


def test_max_extent_coordinates(px, orc):
    coords = max_extent_coords()
    c = ti32(coords)
    nbr, masks = px.neighbor_map(c)
    ref = orc.neighbor_map(coords)
    np.testing.assert_array_equal(nbr.cpu().numpy(), ref)
    n = coords.shape[0]
    assert (ref != n).sum() > n  # the neighbours across the far faces are found
    shape = (32768, 32768, 32768)
    assert px.validate(c, 32768, shape) == (0, -1)
    f = W.normal(3, n * 2, 1).reshape(n, 2)
    assert orc.sparse_valid(coords, 32768, shape, f, 2) == (0, -1)
    # a z extent of 32767 puts the rows at z = 32767 outside the shape: the
    # first of them is reported, as the reference does
    got = px.validate(c, 32768, (32768, 32768, 32767), t32(f))
    assert got == orc.sparse_valid(coords, 32768, (32768, 32768, 32767), f, 2) == (4, 3)


@pytest.mark.parametrize("dims", [(32769, 8, 8, 8), (1, 8, 32769, 8), (1, 8, 8, 40000)])
def test_extents_beyond_the_key_are_rejected(px, dims):
    import pxs
    coords = ti32(np.array([[0, 1, 1, 1]], np.int32))
    with pytest.raises(pxs.PxsError, match="extent exceeds PXS_MAX_EXTENT"):
        px.validate(coords, dims[0], dims[1:])


# --- generation-tagged grids ---------------------------------------------------------

def test_tagged_grid_map_across_generations(px, orc):
    """One tagged grid, four builds with increasing generations over different
    coordinate sets (each a superset, a subset or a disjoint set of the last):
    each map equals the oracle's, so stale cells of earlier generations never
    leak into a later map."""
    shape, batch = (24, 24, 24), 2
    sets = [W.shell_coords(24, [[(6.0, 10.0)], [(5.0, 9.0)]], 51),
            W.shell_coords(24, [[(4.0, 11.0)], [(3.0, 10.0)]], 52),
            W.shell_coords(24, [[(8.0, 9.0)], [(2.0, 3.0)]], 53),
            W.shell_coords(24, [[(6.0, 10.0)], [(5.0, 9.0)]], 51)]
    grid = px.tagged_grid(batch, shape)
    for gen, coords in enumerate(sets, start=1):
        print(f"[tagged map] generation={gen} n={coords.shape[0]}", flush=True)
        c = ti32(coords)
        px.tagged_insert(c, batch, shape, grid, gen)
        nbr, masks = px.neighbor_map_tagged(c, batch, shape, grid, gen)
        ref = orc.neighbor_map(coords)
        np.testing.assert_array_equal(nbr.cpu().numpy(), ref)
        ref_masks = ((ref != coords.shape[0]).astype(np.int64) << np.arange(27)[:, None]).sum(0)
        np.testing.assert_array_equal(masks.cpu().numpy().astype(np.int64) & 0x7FFFFFF, ref_masks)


def test_tagged_grid_generation_cycle(px, orc):
    """Generations 254 and 255, a reset, then 1 and 2 again, over different
    coordinate sets: every map equals the oracle's.  Generations outside
    1..255 and row counts past 2^24 - 1 are rejected before any launch."""
    import ctypes as C
    import pxs
    shape, batch = (24, 24, 24), 2
    a = W.shell_coords(24, [[(6.0, 10.0)], [(5.0, 9.0)]], 55)
    b = W.shell_coords(24, [[(4.0, 7.0)], [(8.0, 11.0)]], 56)
    grid = px.tagged_grid(batch, shape)
    for gen, coords, reset in ((254, a, False), (255, b, False), (1, a, True), (2, b, False)):
        print(f"[tagged cycle] generation={gen} reset={reset} n={coords.shape[0]}", flush=True)
        if reset:
            px._check(px.lib.pxs_voxel_grid_tagged_reset(C.c_void_p(grid.data_ptr()), batch,
                                                         *shape, px.stream()),
                      "pxs_voxel_grid_tagged_reset")
        c = ti32(coords)
        px.tagged_insert(c, batch, shape, grid, gen)
        nbr, _ = px.neighbor_map_tagged(c, batch, shape, grid, gen)
        np.testing.assert_array_equal(nbr.cpu().numpy(), orc.neighbor_map(coords))
    c = ti32(a)
    for gen in (0, 256):
        with pytest.raises(pxs.PxsError, match="generation must be in 1..255"):
            px.tagged_insert(c, batch, shape, grid, gen)
    rc = px.lib.pxs_voxel_grid_tagged_insert(C.c_void_p(c.data_ptr()), 1 << 24, batch, *shape,
                                             C.c_void_p(grid.data_ptr()), 3, px.stream())
    assert rc != 0 and "2^24 - 1" in px.lib.pxs_last_error().decode()


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("case", ["unet_stage_128", "small_2batch", "single", "odd"])
def test_downsample_s2_tagged_bit_exact(px, orc, case, fused):
    """The tagged stride-2 topology equals the oracle's (coordinates, count,
    all 8 child slots), the coarse grid it writes gives the oracle's map over
    the output coordinates, and later calls on the same workspace and grids
    with other coordinates are exact too (the occupancy bitmap is left zero,
    stale fine-grid entries do not match, the coarse grid is rewritten whole).
    fused: insert, fine map and topology by pxs_map_s2_topology_tagged, whose
    fine map must equal the oracle's too."""
    if case == "odd":
        coords, batch, shape = (W.shell_coords(23, [[(5.0, 9.0)], [(4.0, 8.0)]], 54), 2,
                                (23, 23, 23))
    else:
        coords, batch, shape = coord_cases()[case]
    cshape = tuple((s + 1) // 2 for s in shape)
    fine = px.tagged_grid(batch, shape)
    coarse = torch.full((px.lib.pxs_voxel_grid_bytes(batch, *cshape) // 4,), 12345,
                        dtype=torch.int32, device=dev())  # garbage: every cell is written
    ws = px.s2_tagged_workspace(batch, shape)
    other = coords[::2].copy()
    for gen, cc in ((1, coords), (2, other), (3, coords)):
        print(f"[s2 tagged] case={case} fused={fused} generation={gen} n={cc.shape[0]}",
              flush=True)
        c = ti32(cc)
        if fused:
            fnbr, fmasks, oc, child, m = px.map_s2_tagged(c, batch, shape, fine, gen, coarse, ws)
            rmap = orc.neighbor_map(cc)
            np.testing.assert_array_equal(fnbr.cpu().numpy(), rmap)
            rmask = ((rmap != cc.shape[0]).astype(np.int64) << np.arange(27)[:, None]).sum(0)
            np.testing.assert_array_equal(fmasks.cpu().numpy().astype(np.int64) & 0x7FFFFFF, rmask)
        else:
            px.tagged_insert(c, batch, shape, fine, gen)
            oc, child, m = px.downsample_s2_tagged(c, batch, shape, fine, gen, coarse, ws)
        roc, rchild = orc.downsample_coords_s2(cc)
        assert m == roc.shape[0]
        np.testing.assert_array_equal(oc.cpu().numpy(), roc)
        np.testing.assert_array_equal(child.cpu().numpy()[:, :m], rchild.T)
        nbr, _ = px.neighbor_map_grid(oc.contiguous(), batch, cshape, grid=coarse)
        np.testing.assert_array_equal(nbr.cpu().numpy(), orc.neighbor_map(roc))
    # the occupancy bitmap (the workspace's first region) is left zero
    words = (batch * cshape[0] * cshape[1] * cshape[2] + 31) // 32
    assert not ws[:4 * words].any()
