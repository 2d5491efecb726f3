"""Device-resident transformer block and SLat-flow forward (pxs_transformer_block,
pxs_slat_flow_forward) against the compiled reference's vectors and the oracle.

fp32: within 1e-5 (max|g - r| / max|r|).  bf16 GEMM operands with fp32
accumulation and an fp32 residual stream: within 1e-2 relative L2, against the
oracle run in fp32 on the same bf16-rounded weights and inputs.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

import oracle as O
import pxs
import workloads as W
from fixtures import flow_case
from gpu_common import assert_bf16, assert_fp32, dev, host, rel_l2, t32, ti32, ti64

pytestmark = pytest.mark.gpu
GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def px():
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


def block_cfg(C, H, M, CC, PC, use_proj, eps=1e-6):
    return pxs.BlockConfig(C, H, M, CC, PC, eps, 1.0, 10000.0, 1, 1, 1, 1 if use_proj else 0)


def device_weights(ws, dtype):
    """Host arrays -> device tensors; linear weights in dtype, the rest fp32."""
    out = []
    for i, w in enumerate(ws):
        if w is None:
            out.append(None)
            continue
        t = t32(w)
        out.append(t.to(dtype) if (i in pxs.BLOCK_LINEAR_WEIGHTS and dtype != torch.float32) else t)
    return out


def bf16_round(ws):
    return [None if w is None else (W.bf16_round(w) if i in pxs.BLOCK_LINEAR_WEIGHTS else w)
            for i, w in enumerate(ws)]


@pytest.mark.parametrize("proj", [True, False])
def test_block_fp32_reference_vectors(px, proj):
    v = dict(np.load(GOLD / "ref_vectors.npz"))
    ws = [v[f"blk_w{i}"] for i in range(23)]
    if not proj:
        ws[17] = ws[18] = None
    dws = device_weights(ws, torch.float32)
    cfg = block_cfg(32, 4, 64, 6, 5, proj)
    coords = ti32(v["blk_coords"])
    cu = px.batch_cu_seqlens(coords, 2)
    hidden = t32(v["blk_x"]).clone()
    px.transformer_block(cfg, pxs.block_weights(dws), coords, 2, cu, hidden, t32(v["blk_tmod"]),
                         t32(v["blk_ctx"]), ti64(v["blk_ctx_off"]),
                         projected=t32(v["blk_proj"]) if proj else None)
    assert_fp32(host(hidden), v["blk_out"] if proj else v["blk_out_noproj"],
                what=f"block fp32 proj={proj}")


def run_flow(px, case, dtype):
    C, H, M, CC = case["C"], case["H"], case["M"], case["CC"]
    nb = len(case["blocks"])
    cfg = pxs.FlowConfig(case["dims"][0], case["dims"][2], C, CC, nb, H, 0, M, 1e-6, 1.0, 10000.0,
                         1, 1, 0)
    fw_dev = [t32(a) for a in case["fw"]]
    blk_dev = [device_weights(ws, dtype) for ws in case["blocks"]]
    arr = (pxs.BlockWeights * max(nb, 1))(*[pxs.block_weights(b) for b in blk_dev])
    weights = pxs.FlowWeights(*[a.data_ptr() for a in fw_dev], arr)
    coords = ti32(case["coords"])
    bsz = len(case["ctx_off"]) - 1
    cu = px.batch_cu_seqlens(coords, bsz)
    ctx = t32(case["ctx"]).to(dtype)
    out = px.slat_flow_forward(cfg, weights, coords, bsz, cu, t32(case["x"]), t32(case["t"]), ctx,
                               ti64(case["ctx_off"]))
    torch.cuda.synchronize()
    return host(out)


def oracle_flow(orc, case, bf16):
    blocks = [bf16_round(ws) for ws in case["blocks"]] if bf16 else case["blocks"]
    ctx = W.bf16_round(case["ctx"]) if bf16 else case["ctx"]
    return orc.slat_flow_forward(case["coords"], len(case["ctx_off"]) - 1, case["x"], case["t"],
                                 ctx, case["ctx_off"], case["dims"], [1e-6, 1.0, 10000.0],
                                 case["fw"], blocks)


def test_flow_fp32_small(px, orc):
    """Two blocks, C=64 (2 heads x 32), two batches of ~300 voxels; fp32 end to end."""
    case = flow_case(31, [[(4.0, 6.0)], [(3.0, 5.0)]], 16, 64, 2, 2, 7)
    print(f"flow fp32: n={case['n']}", flush=True)
    got = run_flow(px, case, torch.float32)
    ref = oracle_flow(orc, case, bf16=False)
    assert_fp32(got, ref, what="flow fp32")


def test_flow_bf16_reduced_config(px, orc):
    """The SLat-flow step at reduced size: 2 blocks of width 1024 (16 heads x 64,
    MLP 4096), 1,904 voxels in 2 batches, 137 context tokens each; bf16 GEMMs."""
    case = flow_case(32, [[(5.0, 7.0)], [(4.0, 6.0)]], 32, 1024, 16, 2, 137)
    print(f"flow bf16: n={case['n']}", flush=True)
    got = run_flow(px, case, torch.bfloat16)
    ref = oracle_flow(orc, case, bf16=True)
    assert np.isfinite(got).all()
    assert_bf16(got, ref, what="flow bf16 reduced")


def test_flow_bf16_full_depth(px, orc):
    """The SLat-flow step at its full depth and width: 24 blocks of width 1024
    (16 heads x 64, MLP 4096), 864 voxels in 2 batches, 137 context tokens
    each; bf16 GEMMs against the oracle's fp32 forward on the same
    bf16-rounded weights, so rounding that compounds over the 24 residual
    updates is held to the same 1e-2 relative L2 as one block."""
    case = flow_case(33, [[(4.0, 6.0)], [(3.0, 5.0)]], 24, 1024, 16, 24, 137)
    print(f"flow bf16 24 blocks: n={case['n']}", flush=True)
    got = run_flow(px, case, torch.bfloat16)
    ref = oracle_flow(orc, case, bf16=True)
    assert np.isfinite(got).all()
    print(f"flow bf16 24 blocks: rel L2 {rel_l2(got, ref):.3e}", flush=True)
    assert_bf16(got, ref, what="flow bf16 24 blocks")


def test_block_fp32_wide_heads(px, orc):
    """A block with 128-wide heads (C = 256, 2 heads; RoPE, q/k RMS norms,
    cross-attention), fp32, against the oracle block
    (src/sparse_transformer.cpp:138-292); the reference allows any head width."""
    from test_gpu_configs import flow_block_weights, normal
    rng = np.random.default_rng(94)
    coords = W.shell_coords(12, [[(3.0, 5.0)], [(2.0, 4.0)]], 94)
    n, C, H, M, CC, T = coords.shape[0], 256, 2, 512, 64, 9
    ws = flow_block_weights(rng, C, M, CC)
    x = normal(rng, (n, C))
    tmod = normal(rng, (2, 6 * C), 0.3)
    ctx = normal(rng, (2 * T, CC))
    off = np.array([0, T, 2 * T], np.int64)
    print(f"[block wide heads] n={n} head_dim={C // H}", flush=True)
    c = ti32(coords)
    hidden = t32(x).clone()
    dws = device_weights(ws, torch.float32)  # kept alive: the struct holds raw pointers
    px.transformer_block(block_cfg(C, H, M, CC, 0, False), pxs.block_weights(dws), c, 2,
                         px.batch_cu_seqlens(c, 2), hidden, t32(tmod), t32(ctx), ti64(off))
    ref = orc.transformer_block(coords, 2, x, tmod, ctx, off, [C, H, M, CC, 0, 1, 1, 1, 0],
                                [1e-6, 1.0, 10000.0], ws)
    assert_fp32(host(hidden), ref, what="block wide heads")
