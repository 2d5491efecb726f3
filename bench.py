#!/usr/bin/env python3
"""Throughput of the sparse-voxel hot path on one MI355X.

Default workload (one "step" = one pass over the batch, inputs resident in HBM):
  unet_stage_128 - batch 2 on a 128^3 grid (61,056 + 101,207 voxels, unions of
  three ellipsoid shells), bf16 features, fp32 accumulation:
    voxel hash + 3x3x3 neighbor map at 128^3
    SubMConv3d 3^3 128 -> 128
    stride-2 topology (coarse cells, child map)
    SparseConv3d 2^3 s2 128 -> 256
    voxel hash + neighbor map at 64^3
    SubMConv3d 3^3 256 -> 256
  value = sum over the three convs of (active pairs x Cin x Cout) / step time,
  in voxel-GMAC/s.

Also reported on the same line:
  roofline      - the dominant conv kernel: algorithmic FLOPs per launch /
                  its mean launch time (HIP events on its stream) vs the bf16
                  dense MFMA peak (2.5 PFLOP/s)
  attention     - the varlen flash-attention kernel on 12,288 + 20,480
                  tokens, 16 heads x 64 (2.336 TFLOP per call), TFLOP/s and
                  fraction of the bf16 MFMA peak
  cpu_baseline  - the reference CPU sparse_submanifold_conv3d (compiled from
                  the reference sources, oracle/_ref) on item 0 of the same
                  workload at fp32, all host threads, voxel-GMAC/s
--workload selects another configuration (conv_fp32_64, attn_full, swin_64).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for sub in ("pixal3d.cpp_amd/python", "oracle"):
    sys.path.insert(0, str(ROOT / sub))

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="unet_stage_128",
                    choices=["unet_stage_128", "conv_fp32_64", "attn_full", "swin_64"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-attention", action="store_true")
    return ap.parse_args()


class Timer:
    """Per-kernel HIP-event timing on torch's current stream."""

    def __init__(self, torch):
        self.torch = torch
        self.events = {}

    def run(self, name, fn):
        t = self.torch
        s, e = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        s.record()
        out = fn()
        e.record()
        self.events.setdefault(name, []).append((s, e))
        return out

    def mean_ms(self, name):
        ev = self.events.get(name, [])
        if not ev:
            return float("nan")
        return sum(s.elapsed_time(e) for s, e in ev) / len(ev)

    def reset(self):
        self.events = {}


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


# ---------------------------------------------------------------------------
def unet_stage(args, torch, px, W):
    import ctypes as C

    import numpy as np

    dev = torch.device("cuda:0")
    wl = W.unet_stage_128()
    coords_np = wl["coords"]
    n = coords_np.shape[0]
    coords = torch.from_numpy(coords_np).to(dev)
    x = torch.from_numpy(wl["feats"]).to(dev).to(torch.bfloat16)
    w_a = torch.from_numpy(wl["w_a"]).to(dev).to(torch.bfloat16)
    w_b = torch.from_numpy(wl["w_b"]).to(dev).to(torch.bfloat16)
    w_c = torch.from_numpy(wl["w_c"]).to(dev).to(torch.bfloat16)
    b_a = torch.from_numpy(wl["b_a"]).to(dev)
    b_b = torch.from_numpy(wl["b_b"]).to(dev)
    b_c = torch.from_numpy(wl["b_c"]).to(dev)
    lib = px.lib
    S = px.stream
    P = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731

    def ws(nbytes):
        return torch.empty(max(int(nbytes), 8), dtype=torch.uint8, device=dev)

    # Buffers sized once.
    table1 = ws(lib.pxs_voxel_hash_bytes(n))
    nbr1 = torch.empty((27, n), dtype=torch.int32, device=dev)
    mask1 = torch.empty(n, dtype=torch.int32, device=dev)
    y_a = torch.empty((n, 128), dtype=torch.bfloat16, device=dev)
    oc = torch.empty((n, 4), dtype=torch.int32, device=dev)
    child = torch.empty((8, n), dtype=torch.int32, device=dev)
    m_dev = torch.empty(1, dtype=torch.int64, device=dev)
    ds_ws = ws(lib.pxs_downsample_workspace_bytes(n, 2, 128, 128, 128, 2))
    # Topology size (deterministic for these coordinates): one sync here,
    # outside the timed region; every step recomputes the topology itself.
    _, _, m = px.downsample_s2(coords, 2, (128, 128, 128))
    y_b = torch.empty((m, 256), dtype=torch.bfloat16, device=dev)
    table2 = ws(lib.pxs_voxel_hash_bytes(m))
    nbr2 = torch.empty((27, m), dtype=torch.int32, device=dev)
    mask2 = torch.empty(m, dtype=torch.int32, device=dev)
    y_c = torch.empty((m, 256), dtype=torch.bfloat16, device=dev)
    timer = Timer(torch)

    def chk(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {lib.pxs_last_error().decode()}")

    def step():
        s = S()
        timer.run("hash_map_128", lambda: (
            chk(lib.pxs_voxel_hash_build(P(coords), n, P(table1), s), "hash"),
            chk(lib.pxs_neighbor_map_k3(P(coords), n, P(table1), P(nbr1), P(mask1), s), "map")))
        timer.run("subm_conv_a", lambda: chk(lib.pxs_subm_conv3d(
            1, P(x), n, 128, P(w_a), P(b_a), 128, P(nbr1), P(mask1), P(y_a), s), "conv a"))
        timer.run("downsample_s2", lambda: chk(lib.pxs_downsample_s2_topology(
            P(coords), n, 2, 128, 128, 128, P(oc), P(child), P(m_dev), P(ds_ws), s), "ds"))
        timer.run("sparse_conv_b", lambda: chk(lib.pxs_sparse_conv3d_s2(
            1, P(y_a), n, 128, P(w_b), P(b_b), 256, P(child), n, m, P(y_b), s), "conv b"))
        timer.run("hash_map_64", lambda: (
            chk(lib.pxs_voxel_hash_build(P(oc), m, P(table2), s), "hash2"),
            chk(lib.pxs_neighbor_map_k3(P(oc), m, P(table2), P(nbr2), P(mask2), s), "map2")))
        timer.run("subm_conv_c", lambda: chk(lib.pxs_subm_conv3d(
            1, P(y_b), m, 256, P(w_c), P(b_c), 256, P(nbr2), P(mask2), P(y_c), s), "conv c"))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Active pair counts (algorithmic work) from the neighbor masks.
    pa = int(np.unpackbits(mask1.cpu().numpy().view(np.uint8)).sum())
    pc = int(np.unpackbits(mask2.cpu().numpy().view(np.uint8)).sum())
    macs = {"subm_conv_a": pa * 128 * 128, "sparse_conv_b": n * 128 * 256,
            "subm_conv_c": pc * 256 * 256}
    timer.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1e3 / args.steps
    total_macs = sum(macs.values())
    value = total_macs / (dt / args.steps) / 1e9
    kern = {k: timer.mean_ms(k) for k in ("hash_map_128", "subm_conv_a", "downsample_s2",
                                         "sparse_conv_b", "hash_map_64", "subm_conv_c")}
    dom = max(macs, key=lambda k: kern[k])
    achieved = 2.0 * macs[dom] / (kern[dom] * 1e-3) / 1e12
    per_op = {k: {"ms": round(kern[k], 4),
                  "voxel_gmacs": round(macs[k] / (kern[k] * 1e-3) / 1e9, 1),
                  "tflops": round(2 * macs[k] / (kern[k] * 1e-3) / 1e12, 2)} for k in macs}
    # Map kernels are HBM-bound: coords in (16 B/row) + 27 int32 out + mask out.
    map_bytes = n * (16 + 27 * 4 + 4)
    per_op["hash_map_128"] = {"ms": round(kern["hash_map_128"], 4),
                              "gbs": round(map_bytes / (kern["hash_map_128"] * 1e-3) / 1e9, 1)}
    per_op["downsample_s2"] = {"ms": round(kern["downsample_s2"], 4)}
    per_op["hash_map_64"] = {"ms": round(kern["hash_map_64"], 4)}
    result = {
        "metric": "SubMConv3d voxel-GMAC/s & sparse-attn TFLOP/s vs roofline, 1 MI355X",
        "value": round(value, 2),
        "unit": "voxel-GMAC/s",
        "ms_per_step": round(ms, 4),
        "dtype": "bf16",
        "config": {"workload": "unet_stage_128: batch 2 on 128^3 (61,056 + 101,207 voxels, "
                               "3 ellipsoid shells each); hash+map, SubMConv3d 128->128, "
                               "s2 SparseConv3d 128->256, hash+map at 64^3, SubMConv3d 256->256",
                   "voxels": n, "voxels_64": m, "pairs_a": pa, "pairs_c": pc,
                   "per_op": per_op},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None},
    }
    return result


def attention_metric(args, torch, px, W):
    import numpy as np

    dev = torch.device("cuda:0")
    lens = (12288, 20480)
    heads, hd = 16, 64
    n = sum(lens)
    C = heads * hd
    q = torch.from_numpy(W.normal(71, n * C, 1).reshape(n, C)).to(dev).to(torch.bfloat16)
    k = torch.from_numpy(W.normal(71, n * C, 2).reshape(n, C)).to(dev).to(torch.bfloat16)
    v = torch.from_numpy(W.normal(71, n * C, 3).reshape(n, C)).to(dev).to(torch.bfloat16)
    cu = torch.tensor([0, lens[0], n], dtype=torch.int64, device=dev)
    o = torch.empty_like(q)
    timer = Timer(torch)
    for _ in range(args.warmup):
        px.varlen_attention(q, k, v, cu, cu, heads, hd, 0.125, out=o)
    torch.cuda.synchronize()
    steps = max(args.steps, 5)
    for _ in range(steps):
        timer.run("attn", lambda: px.varlen_attention(q, k, v, cu, cu, heads, hd, 0.125, out=o))
    torch.cuda.synchronize()
    flops = 4.0 * sum(L * L for L in lens) * hd * heads
    ms = timer.mean_ms("attn")
    tf = flops / (ms * 1e-3) / 1e12
    return {"workload": "varlen self-attention 12,288 + 20,480 tokens, 16 heads x 64, bf16",
            "ms": round(ms, 4), "tflops": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
            "frac": round(tf / PEAK_BF16_TFLOPS, 4), "flop_per_call": flops}


def cpu_baseline_conv():
    """Reference sparse_submanifold_conv3d (oracle/_ref) on item 0, fp32."""
    import numpy as np

    import oracle as O
    import workloads as W

    if not O.REF_LIB.exists():
        return None
    ref = O.Reference()
    threads = cpu_threads()
    ref.set_threads(threads)
    wl = W.unet_stage_128()
    item0 = wl["coords"][:, 0] == 0
    coords = wl["coords"][item0]
    feats = wl["feats"][item0]
    t = ref.sparse(coords, feats, 1, (128, 128, 128))
    orc = O.Oracle()
    idx = orc.neighbor_map(coords)
    pairs = int((idx != coords.shape[0]).sum())
    ref.subm_conv3d(t, wl["w_a"], wl["b_a"])  # warm
    t0 = time.perf_counter()
    reps = 2
    for _ in range(reps):
        ref.subm_conv3d(t, wl["w_a"], wl["b_a"])
    dt = (time.perf_counter() - t0) / reps
    return {"value": round(pairs * 128 * 128 / dt / 1e9, 3), "unit": "voxel-GMAC/s",
            "cores": threads, "kind": "reference",
            "sample": f"reference sparse_submanifold_conv3d fp32, SubMConv3d 128->128 on batch "
                      f"item 0 ({coords.shape[0]} voxels, {pairs} pairs) of the same workload, "
                      f"mean of {reps} calls ({dt:.2f} s each)"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              f"(the sparse path shards by segment and by spatial slab; see DESIGN.md)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import pxs
    import workloads as W

    px = pxs.Pxs()
    if args.workload != "unet_stage_128":
        from bench_workloads import run_workload
        result = run_workload(args, torch, px, W)
    else:
        result = unet_stage(args, torch, px, W)
        if not args.no_attention:
            result["attention"] = attention_metric(args, torch, px, W)
    base = {"metric": result.pop("metric"), "value": result.pop("value"),
            "unit": result.pop("unit"), "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": result.pop("ms_per_step"),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": result.pop("dtype"), "data": "synthetic (seeded ellipsoid shells, N(0,1) "
                                                  "features, Kaiming random weights)"}
    base.update(result)
    if not args.no_cpu_baseline and args.workload == "unet_stage_128":
        base["cpu_baseline"] = cpu_baseline_conv()
    print(json.dumps(base), flush=True)


if __name__ == "__main__":
    main()
