"""GPU parity: SubMConv3d with the neighbours looked up in a dense voxel grid
inside the convolution (pxs_subm_conv3d_grid), against the same convolution
over the grid's neighbour map (bit for bit: same sources, same tiles, same
summation order) and against the oracle; the fused U-Net topology without
its map."""

import numpy as np
import pytest

import oracle as O
import workloads as W
from gpu_common import assert_bf16, assert_fp32, host, rel_l2, t32, tbf, ti32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def px():
    import pxs
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


def _bits(t):
    import torch
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16).cpu().numpy()


def _box_coords(seed, batch, shape, fill):
    """Random voxels of a small box, every face touched: lookups past the extents."""
    rng = np.random.default_rng(seed)
    cells = np.argwhere(rng.random((batch,) + shape) < fill).astype(np.int32)
    for b in range(batch):  # the box's corners, so every boundary is present
        for x in (0, shape[0] - 1):
            for y in (0, shape[1] - 1):
                for z in (0, shape[2] - 1):
                    cells = np.vstack([cells, [[b, x, y, z]]])
    cells = np.unique(cells, axis=0)
    return np.ascontiguousarray(cells, np.int32)


CASES = [
    # (name, coords builder, batch, extents, cin, cout, dtype)
    ("config1_f32", lambda: W.conv_fp32_64()["coords"], 1, (64, 64, 64), 64, 64, "f32"),
    ("config1_bf16", lambda: W.conv_fp32_64()["coords"], 1, (64, 64, 64), 64, 64, "bf16"),
    ("unet_a_bf16", lambda: W.unet_stage_128()["coords"], 2, (128, 128, 128), 128, 128, "bf16"),
    ("box_f32", lambda: _box_coords(7, 2, (6, 5, 7), 0.5), 2, (6, 5, 7), 16, 24, "f32"),
    ("box_bf16", lambda: _box_coords(8, 2, (6, 5, 7), 0.5), 2, (6, 5, 7), 32, 256, "bf16"),
    ("box_odd_f32", lambda: _box_coords(9, 1, (5, 9, 4), 0.6), 1, (5, 9, 4), 3, 5, "f32"),
    ("box_odd_bf16", lambda: _box_coords(10, 1, (5, 9, 4), 0.6), 1, (5, 9, 4), 12, 20, "bf16"),
    # neighbourhood ranges: four 64-channel chunks and 96 outputs (the last
    # weight rows of the 128-column tile repeat row 95); a grid only 2 deep
    # in z (each offset looked up on its own instead of three cells a load)
    ("ranges_cin256_bf16", lambda: _box_coords(16, 2, (20, 18, 22), 0.35), 2, (20, 18, 22), 256, 96,
     "bf16"),
    ("ranges_z2_bf16", lambda: _box_coords(17, 2, (30, 26, 2), 0.8), 2, (30, 26, 2), 64, 72, "bf16"),
]


def ranged(dtype, cin, cout):
    """Whether a grid convolution runs on neighbourhood ranges (bf16, inputs
    of a multiple of 64 channels, 65..256 outputs, a multiple of 8)."""
    return dtype == "bf16" and cin % 64 == 0 and 64 < cout <= 256 and cout % 8 == 0


@pytest.mark.parametrize("name,make,batch,shape,cin,cout,dtype", CASES, ids=[c[0] for c in CASES])
def test_conv_grid_matches_map(px, name, make, batch, shape, cin, cout, dtype):
    """Plain and tagged grids: bit-equal to pxs_subm_conv3d over the grid's map.
    The tagged grid first holds another coordinate set under an older
    generation, whose cells must read as absent."""
    coords = make()
    n = coords.shape[0]
    rng = np.random.default_rng(n + cin)
    x = rng.standard_normal((n, cin)).astype(np.float32)
    w = (rng.standard_normal((27, cout, cin)) * cin ** -0.5).astype(np.float32)
    b = rng.standard_normal(cout).astype(np.float32)
    conv = tbf if dtype == "bf16" else t32
    print(f"[conv grid] {name} n={n} {cin}->{cout} {dtype}", flush=True)
    c = ti32(coords)
    xd, wd, bd = conv(x), conv(w), t32(b)
    grid = px.grid_build(c, batch, shape)
    nbr, masks = px.neighbor_map_grid(c, batch, shape, grid=grid)
    y_map = px.subm_conv3d(xd, wd, bd, nbr.contiguous(), masks)
    y_grid = px.subm_conv3d_grid(xd, wd, bd, c, batch, shape, grid, 0)
    if ranged(dtype, cin, cout):
        # the grid form runs on neighbourhood ranges, which sum the same
        # products in another order: equal to a last bf16 rounding
        assert rel_l2(host(y_grid), host(y_map)) <= 4e-3
    else:
        np.testing.assert_array_equal(_bits(y_grid), _bits(y_map))
    tg = px.tagged_grid(batch, shape)
    other = _box_coords(11, batch, shape, 0.3) if max(shape) < 16 else coords[::-3].copy()
    other = np.ascontiguousarray(other[(other[:, 1:] < np.array(shape)).all(1)], np.int32)
    px.tagged_insert(ti32(other), batch, shape, tg, 3)
    px.tagged_insert(c, batch, shape, tg, 4)
    y_tag = px.subm_conv3d_grid(xd, wd, bd, c, batch, shape, tg, 4)
    np.testing.assert_array_equal(_bits(y_tag), _bits(y_grid))


def test_conv_grid_range_unet_full_size(px, orc):
    """The U-Net stage's conv A (162k voxels at 128^3, 128 -> 128, bf16) on
    neighbourhood ranges: 1,500 sampled rows against float64 sums over the
    oracle's neighbour map, and the centre identity (W_13 = I, every other
    W_k = 0, no bias) returning the input exactly."""
    wl = W.unet_stage_128()
    coords, x, w, b = wl["coords"], wl["feats"], wl["w_a"], wl["b_a"]
    n = coords.shape[0]
    print(f"[conv grid ranges, unet A] n={n}", flush=True)
    c = ti32(coords)
    grid = px.grid_build(c, 2, (128, 128, 128))
    xd = tbf(x)
    y = host(px.subm_conv3d_grid(xd, tbf(w), t32(b), c, 2, (128, 128, 128), grid, 0))
    idx = orc.neighbor_map(coords)
    rows = np.linspace(0, n - 1, 1500).astype(np.int64)
    ref = np.tile(b.astype(np.float64), (rows.size, 1))
    for k in range(27):
        src = idx[k, rows]
        ok = src != n
        ref[ok] += x[src[ok]].astype(np.float64) @ w[k].astype(np.float64).T
    assert_bf16(y[rows], ref, what="unet A on neighbourhood ranges")
    eye = np.zeros((27, 128, 128), np.float32)
    eye[13] = np.eye(128, dtype=np.float32)
    yi = px.subm_conv3d_grid(xd, tbf(eye), t32(np.zeros(128, np.float32)), c, 2, (128, 128, 128), grid, 0)
    np.testing.assert_array_equal(_bits(yi), _bits(xd))


@pytest.mark.parametrize("cin", [64, 128])
def test_conv_grid_range_gathered_planes(px, orc, cin):
    """A 3 x 72 x 72 slab next to a shell in a second batch item: dense tiles
    whose planes read rows hundreds apart (staged per kh row or per offset)
    beside thin shell tiles staged per plane; against the oracle."""
    slab = np.array([(0, x, y, z) for x in range(3) for y in range(72) for z in range(72)], np.int32)
    shell = W.shell_coords(24, [[(6.0, 10.0)]], 45)
    shell[:, 0] = 1
    coords = np.concatenate([slab, shell])
    n, cout = coords.shape[0], 128
    x = W.bf16_round(W.normal(46, n * cin, 1).reshape(n, cin))
    w = W.bf16_round(W.normal(46, 27 * cout * cin, 2, std=float(np.sqrt(2 / (27 * cin))))
                     .reshape(27, cout, cin))
    b = W.normal(46, cout, 3, std=0.1)
    print(f"[conv grid ranges, slab] n={n} cin={cin}", flush=True)
    c = ti32(coords)
    grid = px.grid_build(c, 2, (24, 72, 72))
    y = px.subm_conv3d_grid(tbf(x), tbf(w), t32(b), c, 2, (24, 72, 72), grid, 0)
    assert_bf16(host(y), orc.subm_conv3d(coords, x, w, b), what="slab on neighbourhood ranges")


@pytest.mark.parametrize("name,make,batch,shape,cin,cout", [
    ("cin256_cout96", lambda: _box_coords(16, 2, (20, 18, 22), 0.35), 2, (20, 18, 22), 256, 96),
    ("z2_cout72", lambda: _box_coords(17, 2, (30, 26, 2), 0.8), 2, (30, 26, 2), 64, 72),
    # the 256-column tile: 256 outputs, and 200 (a partial column tile)
    ("cin128_cout256", lambda: _box_coords(18, 2, (24, 20, 22), 0.35), 2, (24, 20, 22), 128, 256),
    ("z2_cout200", lambda: _box_coords(19, 1, (40, 36, 2), 0.7), 1, (40, 36, 2), 192, 200)])
def test_conv_grid_range_shapes_vs_oracle(px, orc, name, make, batch, shape, cin, cout):
    """Neighbourhood ranges over more K chunks, a partial column tile and the
    per-offset lookups of a grid under 3 cells deep, against the oracle."""
    coords = make()
    n = coords.shape[0]
    x = W.bf16_round(W.normal(47, n * cin, 1).reshape(n, cin))
    w = W.bf16_round(W.normal(47, 27 * cout * cin, 2, std=float(np.sqrt(2 / (27 * cin))))
                     .reshape(27, cout, cin))
    b = W.normal(47, cout, 3, std=0.1)
    print(f"[conv grid ranges] {name} n={n} {cin}->{cout}", flush=True)
    c = ti32(coords)
    grid = px.grid_build(c, batch, shape)
    y = px.subm_conv3d_grid(tbf(x), tbf(w), t32(b), c, batch, shape, grid, 0)
    assert_bf16(host(y), orc.subm_conv3d(coords, x, w, b), what=f"ranges {name}")


RANDOM_RANGE_CASES = [
    # (seed, batch, extents, density, cin, cout, tagged)
    (101, 1, (12, 40, 9), 0.5, 64, 128, False),
    (102, 3, (17, 13, 29), 0.15, 128, 72, True),
    (103, 2, (33, 9, 3), 0.9, 192, 104, False),
    (104, 1, (64, 64, 5), 0.05, 64, 128, True),
    (105, 2, (7, 70, 31), 0.3, 128, 128, False),
    (106, 2, (21, 30, 17), 0.6, 64, 256, True),
    (107, 1, (48, 11, 40), 0.12, 256, 136, False),
]


@pytest.mark.parametrize("seed,batch,shape,density,cin,cout,tagged", RANDOM_RANGE_CASES,
                         ids=[f"seed{c[0]}" for c in RANDOM_RANGE_CASES])
def test_conv_grid_range_random_boxes(px, orc, seed, batch, shape, density, cin, cout, tagged):
    """Neighbourhood ranges on random voxel sets: densities from 5% to 90%
    (planes staged whole, per kh row or per offset), thin and wide extents
    (z down to 3 cells), 1-3 batch items, 1-3 K chunks, partial column tiles,
    plain and tagged grids (the tagged grid first holding an older
    generation's voxels); against the oracle."""
    rng = np.random.default_rng(seed)
    coords = np.ascontiguousarray(np.argwhere(rng.random((batch,) + shape) < density).astype(np.int32))
    n = coords.shape[0]
    x = W.bf16_round(rng.standard_normal((n, cin)).astype(np.float32))
    w = W.bf16_round((rng.standard_normal((27, cout, cin)) * (2.0 / (27 * cin)) ** 0.5).astype(np.float32))
    b = (rng.standard_normal(cout) * 0.1).astype(np.float32)
    print(f"[conv grid ranges, random] seed={seed} n={n} {cin}->{cout} tagged={tagged}", flush=True)
    c = ti32(coords)
    if tagged:
        grid = px.tagged_grid(batch, shape)
        other = np.ascontiguousarray(coords[::2].copy())
        px.tagged_insert(ti32(other), batch, shape, grid, 5)
        px.tagged_insert(c, batch, shape, grid, 6)
        y = px.subm_conv3d_grid(tbf(x), tbf(w), t32(b), c, batch, shape, grid, 6)
    else:
        grid = px.grid_build(c, batch, shape)
        y = px.subm_conv3d_grid(tbf(x), tbf(w), t32(b), c, batch, shape, grid, 0)
    assert_bf16(host(y), orc.subm_conv3d(coords, x, w, b), what=f"random ranges seed {seed}")


def test_conv_grid_fp32_vs_oracle(px, orc):
    """The reference's CPU-runnable case through the grid convolution, against
    the oracle at the fp32 bar."""
    wl = W.conv_fp32_64()
    c = ti32(wl["coords"])
    grid = px.grid_build(c, 1, (64, 64, 64))
    y = px.subm_conv3d_grid(t32(wl["feats"]), t32(wl["weight"]), t32(wl["bias"]), c, 1,
                            (64, 64, 64), grid, 0)
    ref = orc.subm_conv3d(wl["coords"], wl["feats"], wl["weight"], wl["bias"])
    assert_fp32(host(y), ref, what="grid conv fp32 64^3")


def test_conv_grid_rejects_bad_arguments(px):
    import pxs
    c = ti32(_box_coords(12, 1, (4, 4, 4), 0.5))
    x = t32(np.ones((c.shape[0], 8), np.float32))
    w = t32(np.ones((27, 8, 8), np.float32))
    grid = px.grid_build(c, 1, (4, 4, 4))
    with pytest.raises(pxs.PxsError, match="generation"):
        px.subm_conv3d_grid(x, w, None, c, 1, (4, 4, 4), grid, 256)
    with pytest.raises(pxs.PxsError, match="extents"):
        px.subm_conv3d_grid(x, w, None, c, 1, (0, 4, 4), grid, 0)
    # zero rows: nothing to do, no error
    px._check(px.lib.pxs_subm_conv3d_grid(pxs.PXS_F32, x.data_ptr(), c.data_ptr(), 0, 8,
                                          w.data_ptr(), None, 8, 1, 4, 4, 4, grid.data_ptr(), 0,
                                          x.data_ptr(), px.stream()), "zero rows")


def test_map_s2_topology_without_map(px):
    """pxs_map_s2_topology_tagged with no map: the same coarse coordinates,
    child slots, count and coarse grid as with it."""
    import torch
    wl = W.unet_stage_128()
    c = ti32(wl["coords"])
    shape = (128, 128, 128)
    out = []
    for with_map in (True, False):
        tg = px.tagged_grid(2, shape)
        ws = px.s2_tagged_workspace(2, shape)
        cg = torch.empty(px.lib.pxs_voxel_grid_bytes(2, 64, 64, 64) // 4, dtype=torch.int32,
                         device=c.device)
        nbr, masks, oc, child, m = px.map_s2_tagged(c, 2, shape, tg, 1, cg, ws,
                                                    with_map=with_map)
        out.append((oc.cpu().numpy(), child[:, :m].cpu().numpy(), m, cg.cpu().numpy()))
    for a, b in zip(out[0], out[1]):
        np.testing.assert_array_equal(a, b)


def test_conv_bf16_square_tiles(px):
    """A gather wide enough for 256 x 256 tiles (2,112 outputs: a partial last
    column tile; 16,344 rows: a partial last row tile): sampled rows in float64
    from the GPU map, and the grid form bit-equal to the map form."""
    coords = W.shell_coords(48, [[(12.0, 22.0)], [(10.0, 20.0)]], 43)
    n, cin, cout = coords.shape[0], 128, 2112  # 54 K stages: the 256 x 256 tiles' condition
    x = W.bf16_round(W.normal(44, n * cin, 1).reshape(n, cin))
    w = W.bf16_round(W.normal(44, 27 * cout * cin, 2, std=float(np.sqrt(2 / (27 * cin))))
                     .reshape(27, cout, cin))
    b = W.normal(44, cout, 3, std=0.1)
    print(f"[conv bf16 256x256 tiles] n={n} {cin}->{cout}", flush=True)
    c = ti32(coords)
    grid = px.grid_build(c, 2, (48, 48, 48))
    nbr, masks = px.neighbor_map_grid(c, 2, (48, 48, 48), grid=grid)
    xd, wd, bd = tbf(x), tbf(w), t32(b)
    y_map = px.subm_conv3d(xd, wd, bd, nbr.contiguous(), masks)
    idx = nbr.cpu().numpy()
    rows = np.linspace(0, n - 1, 700).astype(np.int64)
    ref = np.tile(b.astype(np.float64), (rows.size, 1))
    for k in range(27):
        src = idx[k, rows]
        ok = src != n
        ref[ok] += x[src[ok]].astype(np.float64) @ w[k].astype(np.float64).T
    assert_bf16(host(y_map)[rows], ref, what="bf16 conv 256x256 tiles")
    y_grid = px.subm_conv3d_grid(xd, wd, bd, c, 2, (48, 48, 48), grid, 0)
    np.testing.assert_array_equal(_bits(y_grid), _bits(y_map))


def test_unet_conv_c_grid_from_topology(px):
    """The U-Net step's conv C exactly as the bench calls it: the 64^3 grid
    that pxs_map_s2_topology_tagged writes (no map), SubMConv3d 256 -> 256 in
    bf16 on 256-column neighbourhood-range tiles over the coarse rows; equal
    to a last bf16 rounding to the same convolution over the neighbour map of
    that grid (gather tiles), 1,000 sampled rows against float64 sums, and the
    coarse grid bit-equal to one built from the coarse coordinates."""
    import torch
    wl = W.unet_stage_128()
    c = ti32(wl["coords"])
    shape = (128, 128, 128)
    tg = px.tagged_grid(2, shape)
    ws = px.s2_tagged_workspace(2, shape)
    cg = torch.empty(px.lib.pxs_voxel_grid_bytes(2, 64, 64, 64) // 4, dtype=torch.int32,
                     device=c.device)
    _, _, oc, child, m = px.map_s2_tagged(c, 2, shape, tg, 1, cg, ws, with_map=False)
    oc = oc[:m].contiguous()
    print(f"[conv C over the topology's grid] m={m} 256->256 bf16", flush=True)
    built = px.grid_build(oc, 2, (64, 64, 64))
    np.testing.assert_array_equal(cg.cpu().numpy(), built.cpu().numpy()[:cg.numel()])
    rng = np.random.default_rng(m)
    x = tbf(rng.standard_normal((m, 256)).astype(np.float32))
    w = tbf((rng.standard_normal((27, 256, 256)) * (2.0 / (27 * 256)) ** 0.5).astype(np.float32))
    b = t32(rng.standard_normal(256).astype(np.float32) * 0.1)
    y_grid = px.subm_conv3d_grid(x, w, b, oc, 2, (64, 64, 64), cg, 0)
    nbr, masks = px.neighbor_map_grid(oc, 2, (64, 64, 64), grid=cg)
    y_map = px.subm_conv3d(x, w, b, nbr.contiguous(), masks)
    assert rel_l2(host(y_grid), host(y_map)) <= 4e-3
    idx = nbr.cpu().numpy()
    xh, wh = host(x).astype(np.float64), host(w).astype(np.float64)
    rows = np.linspace(0, m - 1, 1000).astype(np.int64)
    ref = np.tile(host(b).astype(np.float64), (rows.size, 1))
    for k in range(27):
        src = idx[k, rows]
        ok = src != m
        ref[ok] += xh[src[ok]] @ wh[k].T
    assert_bf16(host(y_grid)[rows], ref, what="conv C on 256-column ranges")


S2_CASES = [
    # (name, coords builder, batch, extents, cin, cout)
    ("unet_a", lambda: W.unet_stage_128()["coords"], 2, (128, 128, 128), 128, 128),
    ("box_odd", lambda: _box_coords(11, 1, (5, 9, 4), 0.6), 1, (5, 9, 4), 16, 24),
    ("box_wide", lambda: _box_coords(12, 3, (40, 22, 30), 0.3), 3, (40, 22, 30), 32, 64),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("name,make,batch,shape,cin,cout", S2_CASES, ids=[c[0] for c in S2_CASES])
def test_s2_emit_fused_matches_topology(px, name, make, batch, shape, cin, cout, dtype):
    """pxs_s2_tagged_insert then pxs_subm_conv3d_grid_s2_emit (bf16: the emit
    in extra workgroups of the convolution's launch; fp32: a launch after it)
    against pxs_map_s2_topology_tagged without a map then pxs_subm_conv3d_grid:
    the convolution, coarse coordinates, child slots, count and coarse grid
    bit-equal, and pxs_s2_tagged_emit alone the same.  Three successive
    generations over one grid and workspace, the second on a subset of the
    rows: each emit must clear the bitmap the next build marks."""
    import torch
    full = make()
    rng = np.random.default_rng(len(full))
    subset = full[np.sort(rng.choice(len(full), len(full) // 3, replace=False))]
    cx, cy, cz = [(s + 1) // 2 for s in shape]
    cells = px.lib.pxs_voxel_grid_bytes(batch, cx, cy, cz) // 4
    dev = torch.device("cuda")
    tg_ref, ws_ref = px.tagged_grid(batch, shape), px.s2_tagged_workspace(batch, shape)
    tg, ws = px.tagged_grid(batch, shape), px.s2_tagged_workspace(batch, shape)
    for gen, coords in ((1, full), (2, subset), (3, full)):
        n = len(coords)
        print(f"[s2 emit fused] {name} {dtype} gen={gen} n={n}", flush=True)
        c = ti32(coords)
        xr = rng.standard_normal((n, cin)).astype(np.float32)
        wr = (rng.standard_normal((27, cout, cin)) * (2.0 / (27 * cin)) ** 0.5).astype(np.float32)
        br = (rng.standard_normal(cout) * 0.1).astype(np.float32)
        x, w = (tbf(xr), tbf(wr)) if dtype == "bf16" else (t32(xr), t32(wr))
        b = t32(br)
        cg_ref = torch.full((cells,), 7, dtype=torch.int32, device=dev)
        _, _, oc_ref, child_ref, m_ref = px.map_s2_tagged(c, batch, shape, tg_ref, gen, cg_ref,
                                                          ws_ref, with_map=False)
        y_ref = px.subm_conv3d_grid(x, w, b, c, batch, shape, tg_ref, gen)
        cg = torch.full((cells,), 9, dtype=torch.int32, device=dev)
        px.s2_tagged_insert(c, batch, shape, tg, gen, ws)
        y, oc, child, m = px.subm_conv3d_grid_s2_emit(x, w, b, c, batch, shape, tg, gen, cg, ws)
        m = int(m.item())
        assert m == m_ref
        np.testing.assert_array_equal(_bits(y), _bits(y_ref))
        np.testing.assert_array_equal(oc[:m].cpu().numpy(), oc_ref.cpu().numpy())
        np.testing.assert_array_equal(child[:, :m].cpu().numpy(), child_ref[:, :m].cpu().numpy())
        np.testing.assert_array_equal(cg.cpu().numpy(), cg_ref.cpu().numpy())
        cg2 = torch.full((cells,), 5, dtype=torch.int32, device=dev)
        oc2, child2, m2 = px.s2_tagged_emit(n, batch, shape, tg, gen, cg2, ws)
        assert int(m2.item()) == m
        np.testing.assert_array_equal(oc2[:m].cpu().numpy(), oc_ref.cpu().numpy())
        np.testing.assert_array_equal(child2[:, :m].cpu().numpy(), child_ref[:, :m].cpu().numpy())
        np.testing.assert_array_equal(cg2.cpu().numpy(), cg_ref.cpu().numpy())


def test_s2_emit_rejects_bad_arguments(px):
    import pxs
    import torch
    c = ti32(np.zeros((4, 4), np.int32))
    grid = px.tagged_grid(1, (4, 4, 4))
    ws = px.s2_tagged_workspace(1, (4, 4, 4))
    with pytest.raises(pxs.PxsError, match="generation must be in 1..255"):
        px.s2_tagged_insert(c, 1, (4, 4, 4), grid, 0, ws)
    x = torch.zeros((4, 8), dtype=torch.bfloat16, device=c.device)
    w = torch.zeros((27, 8, 8), dtype=torch.bfloat16, device=c.device)
    cg = torch.zeros(8, dtype=torch.int32, device=c.device)
    outs = (torch.zeros((4, 4), dtype=torch.int32, device=c.device),
            torch.zeros((8, 2), dtype=torch.int32, device=c.device),
            torch.zeros(1, dtype=torch.int64, device=c.device))
    with pytest.raises(pxs.PxsError, match="child map stride below the row count"):
        px.subm_conv3d_grid_s2_emit(x, w, None, c, 1, (4, 4, 4), grid, 1, cg, ws, s2_out=outs)


LEVEL_CASES = [
    # (name, coords builder, batch, extents, cin, cout_a, cout_b, dtype): chained when bf16
    # with 65..128 SubMConv3d outputs and more than 64 strided outputs, and inputs of other
    # than a multiple of 64 channels (those run the SubMConv3d on neighbourhood ranges, in
    # two launches)
    ("unet_bf16", lambda: W.unet_stage_128()["coords"], 2, (128, 128, 128), 128, 128, 256, "bf16"),
    ("box_bf16_ranges", lambda: _box_coords(20, 2, (34, 21, 40), 0.3), 2, (34, 21, 40), 64, 96, 136,
     "bf16"),
    ("unet_bf16_cin96", lambda: W.unet_stage_128()["coords"], 2, (128, 128, 128), 96, 128, 256,
     "bf16"),
    ("box_bf16", lambda: _box_coords(13, 2, (40, 22, 30), 0.3), 2, (40, 22, 30), 32, 96, 72, "bf16"),
    ("box_bf16_unchained", lambda: _box_coords(14, 1, (9, 7, 11), 0.5), 1, (9, 7, 11), 16, 64, 32,
     "bf16"),
    ("box_f32", lambda: _box_coords(15, 1, (9, 7, 11), 0.5), 1, (9, 7, 11), 16, 24, 40, "f32"),
]


@pytest.mark.parametrize("name,make,batch,shape,cin,cout_a,cout_b,dtype", LEVEL_CASES,
                         ids=[c[0] for c in LEVEL_CASES])
def test_unet_s2_level_matches_two_calls(px, name, make, batch, shape, cin, cout_a, cout_b,
                                         dtype):
    """pxs_unet_s2_level (the strided conv's tiles waiting inside the launch
    for the emit and the SubMConv3d tiles they read) against
    pxs_subm_conv3d_grid_s2_emit then pxs_sparse_conv3d_s2: both convolutions,
    the coarse coordinates, child slots, count and coarse grid bit-equal, and
    no dependency wait given up; three successive generations on one grid and
    workspace, the second over a subset of the rows."""
    import torch
    full = make()
    rng = np.random.default_rng(len(full) + cout_b)
    subset = full[np.sort(rng.choice(len(full), len(full) // 3, replace=False))]
    cx, cy, cz = [(s + 1) // 2 for s in shape]
    cells = px.lib.pxs_voxel_grid_bytes(batch, cx, cy, cz) // 4
    dev = torch.device("cuda")
    tg_ref, ws_ref = px.tagged_grid(batch, shape), px.s2_tagged_workspace(batch, shape)
    tg, ws = px.tagged_grid(batch, shape), px.s2_tagged_workspace(batch, shape)
    for gen, coords in ((1, full), (2, subset), (3, full)):
        n = len(coords)
        c = ti32(coords)
        xr = rng.standard_normal((n, cin)).astype(np.float32)
        war = (rng.standard_normal((27, cout_a, cin)) * (2.0 / (27 * cin)) ** 0.5).astype(np.float32)
        wbr = (rng.standard_normal((8, cout_b, cout_a)) * (2.0 / (8 * cout_a)) ** 0.5).astype(np.float32)
        cast = tbf if dtype == "bf16" else t32
        x, wa, wb = cast(xr), cast(war), cast(wbr)
        ba = t32((rng.standard_normal(cout_a) * 0.1).astype(np.float32))
        bb = t32((rng.standard_normal(cout_b) * 0.1).astype(np.float32))
        cg_ref = torch.full((cells,), 3, dtype=torch.int32, device=dev)
        px.s2_tagged_insert(c, batch, shape, tg_ref, gen, ws_ref)
        ya_ref, oc_ref, child_ref, m_ref = px.subm_conv3d_grid_s2_emit(
            x, wa, ba, c, batch, shape, tg_ref, gen, cg_ref, ws_ref)
        m = int(m_ref.item())
        yb_ref = px.sparse_conv3d_s2(ya_ref, wb, bb, child_ref, m)
        print(f"[unet s2 level] {name} gen={gen} n={n} m={m}", flush=True)
        cg = torch.full((cells,), 4, dtype=torch.int32, device=dev)
        px.s2_tagged_insert(c, batch, shape, tg, gen, ws)
        ya, yb, oc, child, m_out = px.unet_s2_level(x, wa, ba, wb, bb, c, batch, shape, tg, gen,
                                                    m, cg, ws)
        assert px.unet_s2_level_error(ws, batch, shape) == 0
        assert int(m_out.item()) == m
        np.testing.assert_array_equal(_bits(ya), _bits(ya_ref))
        np.testing.assert_array_equal(_bits(yb), _bits(yb_ref))
        np.testing.assert_array_equal(oc[:m].cpu().numpy(), oc_ref[:m].cpu().numpy())
        np.testing.assert_array_equal(child[:, :m].cpu().numpy(), child_ref[:, :m].cpu().numpy())
        np.testing.assert_array_equal(cg.cpu().numpy(), cg_ref.cpu().numpy())
