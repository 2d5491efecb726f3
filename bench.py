#!/usr/bin/env python3
"""Throughput of the sparse-voxel hot path on one MI355X.

Default workload (one "step" = one pass over the batch, inputs resident in HBM):
  unet_stage_128 - batch 2 on a 128^3 grid (61,056 + 101,207 voxels, unions of
  three ellipsoid shells), bf16 features, fp32 accumulation:
    generation-tagged voxel grid insert (with the stride-2 occupancy bits)
    SubMConv3d 3^3 128 -> 128, its 3x3x3 neighbours looked up in the 128^3
      grid inside its tiles (the neighbor map fused into the gather); extra
      workgroups of the same launch emit the stride-2 topology (coarse
      cells, child map, the 64^3 grid)
    SparseConv3d 2^3 s2 128 -> 256
    SubMConv3d 3^3 256 -> 256 over the 64^3 grid the topology wrote
  value = sum over the three convs of (active pairs x Cin x Cout) / step time,
  in voxel-GMAC/s.

Also reported on the same line:
  roofline      - the dominant conv kernel: algorithmic FLOPs per launch /
                  its mean launch time (HIP events on its stream) vs the bf16
                  dense MFMA peak (2.5 PFLOP/s)
  attention     - the varlen flash-attention kernel on 12,288 + 20,480
                  tokens, 16 heads x 64 (2.336 TFLOP per call), TFLOP/s and
                  fraction of the bf16 MFMA peak
  cpu_baseline  - the same three convs on the host cores at fp32: the
                  reference's sparse_submanifold_conv3d compiled from its
                  sources (oracle/_ref, OpenMP) for A and C, the oracle for B,
                  voxel-GMAC/s
--workload selects another configuration for profiling (conv_fp32_64,
attn_block, swin_64, flow_step); their lines are not the headline metric.
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
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--workload", default="unet_stage_128",
                    choices=["unet_stage_128", "conv_fp32_64", "attn_block", "swin_64",
                             "flow_step", "flow_sample", "decoder", "pack_load", "hash_map_128",
                             "linear_dense", "attn_wide"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-attention", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave configs 1 and 4 off the default line")
    ap.add_argument("--topology", default="fused", choices=["chained", "fused", "separate"],
                    help="U-Net step: conv A, the stride-2 emit and conv B in one launch "
                         "(chained), the emit inside conv A's launch (fused), or the "
                         "three-launch topology before conv A (separate)")
    return ap.parse_args()


class Timer:
    """Per-kernel HIP-event timing on torch's current stream.  Only the ops
    named in `only` (all when None) are bracketed by events: each event
    record is a packet of its own in the queue and costs the step time."""

    def __init__(self, torch):
        self.torch = torch
        self.events = {}
        self.only = None

    def run(self, name, fn):
        if self.only is not None and name not in self.only:
            return fn()
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


# Untimed warmup: the requested steps, continued until the GPU has run for
# at least this long (its clocks take a few hundred ms to settle).
MIN_WARMUP_S = 0.5


def warm_up(args, torch, step):
    """args.warmup untimed steps, then more until MIN_WARMUP_S has passed;
    returns the number of steps run."""
    t0 = time.perf_counter()
    done = 0
    for _ in range(args.warmup):
        step()
        done += 1
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < MIN_WARMUP_S:
        for _ in range(10):
            step()
        done += 10
        torch.cuda.synchronize()
    return done


def cpu_threads():
    """OpenMP threads for the CPU baseline and how they were chosen: the
    process's CPU affinity, capped by a cgroup CPU quota and by
    OMP_NUM_THREADS when either is set (a GPU box's CPU share can be smaller
    than the CPUs its affinity mask lists)."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    limits = {"affinity": affinity}
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if quota != "max":
            limits["cgroup_quota"] = max(1, int(int(quota) // int(period)))
    except (OSError, ValueError):
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        limits["OMP_NUM_THREADS"] = int(omp)
    return max(1, min(limits.values())), limits


def cpu_timing(fn, warmup=2, iterations=3):
    """The reference benchmark's method (tests/sparse_linear_cuda_benchmark.cpp:
    717-731): `warmup` untimed calls, then `iterations` timed ones; -> (median s,
    min s)."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(iterations):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], times[0]


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

    # Buffers sized once.  The 128^3 voxel grid is generation-tagged: reset
    # here, then every step inserts its rows under a new generation, so a
    # step refills it only once per 255 generations (O(rows) per build, not
    # O(cells)).
    grid1 = px.tagged_grid(2, (128, 128, 128))
    grid2 = ws(lib.pxs_voxel_grid_bytes(2, 64, 64, 64))  # rewritten whole by the s2 topology
    ds_ws = px.s2_tagged_workspace(2, (128, 128, 128))
    y_a = torch.empty((n, 128), dtype=torch.bfloat16, device=dev)
    oc = torch.empty((n, 4), dtype=torch.int32, device=dev)
    child = torch.empty((8, n), dtype=torch.int32, device=dev)
    m_dev = torch.empty(1, dtype=torch.int64, device=dev)
    # Topology size (deterministic for these coordinates): one sync here,
    # outside the timed region; every step recomputes the topology itself.
    _, _, m = px.downsample_s2(coords, 2, (128, 128, 128))
    y_b = torch.empty((m, 256), dtype=torch.bfloat16, device=dev)
    y_c = torch.empty((m, 256), dtype=torch.bfloat16, device=dev)
    # Active pair counts (the algorithmic work) from the neighbour maps of
    # both levels, built here once: the timed step builds no map (the
    # convolutions look their neighbours up in the grids).
    _, mask1 = px.neighbor_map_grid(coords, 2, (128, 128, 128))
    oc_host, _, _ = px.downsample_s2(coords, 2, (128, 128, 128))
    _, mask2 = px.neighbor_map_grid(oc_host[:m].contiguous(), 2, (64, 64, 64))
    pa = int(np.unpackbits(mask1.cpu().numpy().view(np.uint8)).sum())
    pc = int(np.unpackbits(mask2.cpu().numpy().view(np.uint8)).sum())
    del mask1, mask2, oc_host
    timer = Timer(torch)
    gen = [0]

    def chk(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {lib.pxs_last_error().decode()}")

    def step():
        s = S()
        # generations 1..255 between resets: the step after generation 255
        # refills the grid (and the s2 workspace's tagged bitmap) first (once
        # per 255 steps, inside the timed op)
        wrap = gen[0] == 255
        gen[0] = gen[0] % 255 + 1
        g = C.c_uint32(gen[0])

        def resets():
            if wrap:
                chk(lib.pxs_voxel_grid_tagged_reset(P(grid1), 2, 128, 128, 128, s), "reset")
                chk(lib.pxs_downsample_s2_tagged_workspace_reset(P(ds_ws), 2, 128, 128, 128, s),
                    "reset s2")
        # no neighbour maps: both SubMConv3d look their 27 neighbours up in the
        # grids inside their tiles
        if args.topology == "chained":
            # grid insert (+ the stride-2 occupancy bits), then one launch of
            # conv A, the coarse emit and conv B, whose tiles wait inside the
            # launch only for the conv A tiles (and the emit) they read
            timer.run("topology_128", lambda: (resets(), chk(lib.pxs_s2_tagged_insert(
                P(coords), n, 2, 128, 128, 128, P(grid1), g, P(ds_ws), s), "insert")))
            timer.run("conv_a_b_chained", lambda: chk(lib.pxs_unet_s2_level(
                1, P(x), P(coords), n, 128, P(w_a), P(b_a), 128, 2, 128, 128, 128, P(grid1), g,
                P(y_a), P(w_b), P(b_b), 256, m, P(y_b), P(oc), P(child), n, P(m_dev), P(grid2),
                P(ds_ws), s), "conv a + b"))
            timer.run("subm_conv_c", lambda: chk(lib.pxs_subm_conv3d_grid(
                1, P(y_b), P(oc), m, 256, P(w_c), P(b_c), 256, 2, 64, 64, 64, P(grid2), 0,
                P(y_c), s), "conv c"))
            return
        if args.topology == "fused":
            # grid insert (+ the stride-2 occupancy bits), then conv A, whose
            # launch also emits the coarse rows, child slots and 64^3 grid in
            # extra workgroups
            timer.run("topology_128", lambda: (resets(), chk(lib.pxs_s2_tagged_insert(
                P(coords), n, 2, 128, 128, 128, P(grid1), g, P(ds_ws), s), "insert")))
            timer.run("subm_conv_a", lambda: chk(lib.pxs_subm_conv3d_grid_s2_emit(
                1, P(x), P(coords), n, 128, P(w_a), P(b_a), 128, 2, 128, 128, 128, P(grid1), g,
                P(y_a), P(oc), P(child), n, P(m_dev), P(grid2), P(ds_ws), s), "conv a"))
        else:
            # grid insert and the stride-2 topology in three launches
            timer.run("topology_128", lambda: (resets(), chk(lib.pxs_map_s2_topology_tagged(
                P(coords), n, 2, 128, 128, 128, P(grid1), g, None, None, P(oc), P(child), n,
                P(m_dev), P(grid2), P(ds_ws), s), "topology")))
            timer.run("subm_conv_a", lambda: chk(lib.pxs_subm_conv3d_grid(
                1, P(x), P(coords), n, 128, P(w_a), P(b_a), 128, 2, 128, 128, 128, P(grid1), g,
                P(y_a), s), "conv a"))
        timer.run("sparse_conv_b", lambda: chk(lib.pxs_sparse_conv3d_s2(
            1, P(y_a), n, 128, P(w_b), P(b_b), 256, P(child), n, m, P(y_b), s), "conv b"))
        timer.run("subm_conv_c", lambda: chk(lib.pxs_subm_conv3d_grid(
            1, P(y_b), P(oc), m, 256, P(w_c), P(b_c), 256, 2, 64, 64, 64, P(grid2), 0, P(y_c), s),
            "conv c"))

    macs = {"subm_conv_a": pa * 128 * 128, "sparse_conv_b": n * 128 * 256,
            "subm_conv_c": pc * 256 * 256}
    if args.topology == "chained":
        macs = {"conv_a_b_chained": macs["subm_conv_a"] + macs["sparse_conv_b"],
                "subm_conv_c": macs["subm_conv_c"]}
    ops = ("topology_128",) + tuple(macs)
    timer.only = set()
    warm = warm_up(args, torch, step)
    # Per-op breakdown: a pass of its own with every op bracketed by events.
    timer.only = None
    timer.reset()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    kern = {k: timer.mean_ms(k) for k in ops}
    # The insert is a few microseconds of GPU work, shorter than the host's
    # issue of an event-bracketed op: its events would time the host.  It is
    # timed instead as a run of back-to-back inserts (same rows, same
    # generation: idempotent) between two events.
    if args.topology != "separate":
        g_last = C.c_uint32(gen[0])
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record()
        for _ in range(args.steps):
            chk(lib.pxs_s2_tagged_insert(P(coords), n, 2, 128, 128, 128, P(grid1), g_last,
                                         P(ds_ws), S()), "insert")
        ev1.record()
        torch.cuda.synchronize()
        kern["topology_128"] = ev0.elapsed_time(ev1) / args.steps
    dom = max(macs, key=lambda k: kern[k])
    # Timed region: only the dominant kernel carries events.
    timer.only = {dom}
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
    kern[dom] = timer.mean_ms(dom)
    achieved = 2.0 * macs[dom] / (kern[dom] * 1e-3) / 1e12
    traffic = measured_traffic(dom)
    per_op = {k: {"ms": round(kern[k], 4),
                  "voxel_gmacs": round(macs[k] / (kern[k] * 1e-3) / 1e9, 1),
                  "tflops": round(2 * macs[k] / (kern[k] * 1e-3) / 1e12, 2)} for k in macs}
    # The topology is HBM-bound: per fine row its coordinate (16 B) and one
    # 4-byte tagged cell written (and its bit in the occupancy bitmap); per
    # coarse cell one int32 of the 64^3 grid, per coarse row its coordinate
    # and 8 child slots (the child lookups read cells the insert just wrote).
    # With the fused topology the timed op is the insert alone (the emit's
    # bytes move inside conv A's launch).
    cells_64 = 2 * 64 * 64 * 64
    topo_bytes = n * (16 + 4) + (0 if args.topology != "separate" else cells_64 * 4 + m * (16 + 8 * 4))
    per_op["topology_128"] = {"ms": round(kern["topology_128"], 4),
                              "gbs": round(topo_bytes / (kern["topology_128"] * 1e-3) / 1e9, 1)}
    result = {
        "metric": "SubMConv3d voxel-GMAC/s & sparse-attn TFLOP/s vs roofline, 1 MI355X",
        "value": round(value, 2),
        "unit": "voxel-GMAC/s",
        "ms_per_step": round(ms, 4),
        "dtype": "bf16",
        "config": {"workload": "unet_stage_128: batch 2 on 128^3 (61,056 + 101,207 voxels, "
                               "3 ellipsoid shells each); tagged voxel grid and s2 topology "
                               "(+ 64^3 grid), SubMConv3d 128->128, SparseConv3d 128->256, "
                               "SubMConv3d 256->256; the SubMConv3d take their 27 neighbours "
                               "from the grids inside their tiles (no neighbour map)",
                   "topology": {"chained": "grid insert + stride-2 marks, then one launch of "
                                           "conv A, the coarse emit and conv B (conv B's tiles "
                                           "wait in the launch for the conv A tiles they read)",
                                "fused": "grid insert + stride-2 marks, then the coarse emit in "
                                         "extra workgroups of conv A's launch",
                                "separate": "three launches before conv A"}[args.topology],
                   "voxels": n, "voxels_64": m, "pairs_a": pa, "pairs_c": pc,
                   "warmup_steps_run": warm,
                   "per_op_note": "per-op times from a pass of args.steps steps with every op "
                                  "bracketed by HIP events; the dominant kernel's from the timed "
                                  "region, where only it carries events",
                   "per_op": per_op},
        "roofline": {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic, "traffic_source": traffic_note(dom),
                     "algorithmic_flop": 2 * macs[dom]},
    }
    return result


def measured_traffic(op):
    """HBM bytes per launch of `op` from the committed rocprofv3 --pmc summary
    (reads counted by L2 request size, writes by WRITE_SIZE), or None when the
    summary does not cover this kernel."""
    path = ROOT / "profiles" / "unet_stage_128_traffic.json"
    if not path.exists():
        return None
    rec = json.loads(path.read_text()).get(op)
    if not rec:
        return None
    return int(rec["read_bytes"] + rec["write_bytes"])


def kernel_source_digest(rec):
    """SHA-256 (first 16 hex digits) of the kernel sources a traffic record
    names, as they are in this tree."""
    import hashlib

    h = hashlib.sha256()
    for rel in rec.get("sources", []):
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()[:16]


def traffic_note(op):
    """Where the traffic figure of `op` comes from (it is not measured in the
    bench run: counters need the profiler), and whether the kernel sources
    are still the ones it was measured on."""
    path = ROOT / "profiles" / "unet_stage_128_traffic.json"
    rec = json.loads(path.read_text()).get(op) if path.exists() else None
    if not rec:
        return None
    same = rec.get("sources_sha16") == kernel_source_digest(rec)
    return (f"not measured in this run: rocprofv3 --pmc of {rec['kernel']} (grid {rec['grid']}) "
            f"at commit {rec['measured_at_commit']}, {rec['method']} ({rec['source']}); "
            + (f"{', '.join(rec['sources'])} unchanged since" if same else
               f"STALE: {', '.join(rec.get('sources', [])) or 'the kernel sources'} changed since"))


def attention_metric(args, torch, px, W, heads=16, hd=64):
    import numpy as np

    dev = torch.device("cuda:0")
    lens = (12288, 20480)
    n = sum(lens)
    C = heads * hd
    q = torch.from_numpy(W.normal(71, n * C, 1).reshape(n, C)).to(dev).to(torch.bfloat16)
    k = torch.from_numpy(W.normal(71, n * C, 2).reshape(n, C)).to(dev).to(torch.bfloat16)
    v = torch.from_numpy(W.normal(71, n * C, 3).reshape(n, C)).to(dev).to(torch.bfloat16)
    cu = torch.tensor([0, lens[0], n], dtype=torch.int64, device=dev)
    o = torch.empty_like(q)
    timer = Timer(torch)
    scale = hd ** -0.5
    warm_up(args, torch, lambda: px.varlen_attention(q, k, v, cu, cu, heads, hd, scale, out=o))
    steps = max(args.steps, 5)
    for _ in range(steps):
        timer.run("attn", lambda: px.varlen_attention(q, k, v, cu, cu, heads, hd, scale, out=o))
    torch.cuda.synchronize()
    flops = 4.0 * sum(L * L for L in lens) * hd * heads
    ms = timer.mean_ms("attn")
    tf = flops / (ms * 1e-3) / 1e12
    return {"workload": f"varlen self-attention 12,288 + 20,480 tokens, {heads} heads x {hd}, bf16",
            "ms": round(ms, 4), "tflops": round(tf, 2), "peak": PEAK_BF16_TFLOPS,
            "frac": round(tf / PEAK_BF16_TFLOPS, 4), "flop_per_call": flops}


def cpu_baseline_conv():
    """The U-Net stage on the host cores: SubMConv3d A (128 -> 128 at 128^3) and
    C (256 -> 256 at 64^3) by the reference's sparse_submanifold_conv3d compiled
    from its sources (oracle/_ref, OpenMP), the stride-2 conv B (which the
    reference does not have) by the oracle's restatement; the same inputs as the
    device stage, fp32."""
    import numpy as np

    import oracle as O
    import workloads as W

    if not O.REF_LIB.exists():
        return None
    ref, orc = O.Reference(), O.Oracle()
    threads, limits = cpu_threads()
    ref.set_threads(threads)
    wl = W.unet_stage_128()
    coords, feats = wl["coords"], wl["feats"]
    n = coords.shape[0]
    oc, child = orc.downsample_coords_s2(coords)
    m = oc.shape[0]
    pa = int((orc.neighbor_map(coords) != n).sum())
    pc = int((orc.neighbor_map(oc) != m).sum())
    t_a = ref.sparse(coords, feats, 2, (128, 128, 128))
    x_c = W.normal(95, m * 256, 1).reshape(m, 256)
    t_c = ref.sparse(oc, x_c, 2, (64, 64, 64))

    def stage():
        ref.subm_conv3d(t_a, wl["w_a"], wl["b_a"])
        orc.sparse_conv3d_s2(child, feats, wl["w_b"], wl["b_b"])
        ref.subm_conv3d(t_c, wl["w_c"], wl["b_c"])

    med, best = cpu_timing(stage)
    macs = pa * 128 * 128 + n * 128 * 256 + pc * 256 * 256
    return {"value": round(macs / med / 1e9, 3), "unit": "voxel-GMAC/s", "cores": threads,
            "kind": "reference",
            "sample": f"the whole stage on the host, fp32: SubMConv3d A ({n} voxels, {pa} pairs) "
                      f"and C ({m} voxels, {pc} pairs) by the reference sparse_submanifold_conv3d "
                      f"(compiled from its sources, OpenMP, {threads} threads; CPU limits "
                      f"{limits}), the stride-2 conv B by the oracle (no reference exists); "
                      f"warmup 2, iterations 3: median {med:.3f} s, min {best:.3f} s per stage",
            "median_s": round(med, 4), "min_s": round(best, 4)}


ATTN_CPU_ROWS = 32  # sampled query rows per segment


def cpu_baseline_attention():
    """The reference's sparse_scaled_dot_product_attention (single-threaded,
    src/sparse.cpp:704-783, compiled from its sources into oracle/_ref) on the
    12,288 + 20,480-token workload: ATTN_CPU_ROWS evenly spaced query rows per
    segment against every key of it, all 16 heads; the full-call time is
    extrapolated linearly in the queries (each row costs its segment's key
    count)."""
    import numpy as np

    import oracle as O
    import workloads as W

    if not O.REF_LIB.exists():
        return None
    ref = O.Reference()
    lens, heads, hd = (12288, 20480), 16, 64
    n, c = sum(lens), heads * hd
    coords = W.attn_full()["coords"]
    q = W.normal(71, n * c, 1).reshape(n, c)
    k = W.normal(71, n * c, 2).reshape(n, c)
    v = W.normal(71, n * c, 3).reshape(n, c)
    starts = np.cumsum((0,) + lens[:-1])
    rows = np.concatenate([s + np.linspace(0, L - 1, ATTN_CPU_ROWS).astype(np.int64)
                           for s, L in zip(starts, lens)])
    tq = ref.sparse(coords[rows], q[rows], 2, (32, 32, 32))
    tk, tv = ref.sparse(coords, k, 2, (32, 32, 32)), ref.sparse(coords, v, 2, (32, 32, 32))
    med, best = cpu_timing(lambda: ref.sdpa(tq, tk, tv, heads, hd, 0.125))
    scale = sum(L * L for L in lens) / (ATTN_CPU_ROWS * sum(lens))
    flops = 4.0 * sum(L * L for L in lens) * hd * heads
    full = med * scale
    return {"value": round(flops / full / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
            "kind": "reference",
            "sample": f"extrapolated: reference sparse_scaled_dot_product_attention (compiled "
                      f"from its sources; single-threaded, as the reference is) on "
                      f"{ATTN_CPU_ROWS} query rows per segment against all keys, 16 heads x 64; "
                      f"warmup 2, iterations 3: median {med:.3f} s, min {best:.3f} s per sample; "
                      f"the full call ({n} queries) extrapolated x{scale:.1f} to {full:.1f} s",
            "median_s": round(med, 4), "min_s": round(best, 4), "extrapolated_s": round(full, 2)}


# ---------------------------------------------------------------------------
# CPU baselines of the other configurations: the reference's own CPU
# primitives (compiled from its sources into oracle/_ref, OpenMP where the
# reference parallelises) timed by the reference benchmark's method (2
# untimed calls, median and min of 3).  Row-wise work (linears, norms) is
# timed on LIN_CPU_ROWS sampled rows and scaled by the row count (its cost is
# linear in rows); attention on ATTN_CPU_ROWS query rows per segment against
# every key and scaled by the query count; window attention on a sample of
# the windows, scaled by sum(L^2); a SubMConv3d on a slab of the voxels,
# scaled by active pairs.  Each result says what was sampled.
LIN_CPU_ROWS = 256


def _reference():
    import oracle as O

    if not O.REF_LIB.exists():
        return None, 0, {}
    ref = O.Reference()
    threads, limits = cpu_threads()
    ref.set_threads(threads)
    return ref, threads, limits


def _line_coords(rows):
    """rows distinct voxels of one item (valid coordinates for row-wise ops)."""
    import numpy as np

    i = np.arange(rows, dtype=np.int32)
    return np.stack([np.zeros_like(i), i % 64, (i // 64) % 64, i // 4096], 1).astype(np.int32)


def _cpu_rowwise(ref, rows, fn_of_tensor, cin, seed):
    """Seconds for `rows` rows of a row-wise op, from LIN_CPU_ROWS sampled rows."""
    import workloads as W

    r = min(rows, LIN_CPU_ROWS)
    t = ref.sparse(_line_coords(r), W.normal(seed, r * cin, 1).reshape(r, cin), 1, (64, 64, 64))
    med, _ = cpu_timing(lambda: fn_of_tensor(t))
    return med * rows / r


def _cpu_linear(ref, rows, cin, cout, seed):
    import workloads as W

    w = W.normal(seed, cout * cin, 2, std=cin ** -0.5).reshape(cout, cin)
    b = W.normal(seed, cout, 3, std=0.1)
    return _cpu_rowwise(ref, rows, lambda t: ref.linear(t, w, b), cin, seed)


def _cpu_attention(ref, coords, lens, heads, hd, seed, keys=None):
    """Seconds of the reference's sparse_scaled_dot_product_attention over
    segments of `lens` rows (batch items of `coords`), from ATTN_CPU_ROWS
    query rows per segment; with keys=(T, ctx) the reference's
    sparse_cross_attention against T context tokens per item instead."""
    import numpy as np

    import workloads as W

    c = heads * hd
    n = int(sum(lens))
    starts = np.cumsum((0,) + tuple(lens[:-1]))
    rows = np.concatenate([s + np.linspace(0, L - 1, min(ATTN_CPU_ROWS_BLOCK, L)).astype(np.int64)
                           for s, L in zip(starts, lens)])
    q = W.normal(seed, rows.size * c, 1).reshape(rows.size, c)
    b = len(lens)
    tq = ref.sparse(coords[rows], q, b, (64, 64, 64) if coords.max() < 64 else (128, 128, 128))
    if keys is None:
        k = W.normal(seed, n * c, 2).reshape(n, c)
        tk = ref.sparse(coords, k, b, (64, 64, 64) if coords.max() < 64 else (128, 128, 128))
        fn = lambda: ref.sdpa(tq, tk, tk, heads, hd, hd ** -0.5)  # noqa: E731
    else:
        T = keys
        kv = ref.varlen(np.arange(b + 1, dtype=np.int64) * T, W.normal(seed, b * T * c, 3).reshape(b * T, c))
        fn = lambda: ref.cross_attention(tq, kv, kv, heads, hd, hd ** -0.5)  # noqa: E731
    med, _ = cpu_timing(fn)
    return med * n / rows.size


ATTN_CPU_ROWS_BLOCK = 32  # sampled query rows per segment for the block baselines


def cpu_baseline_conv_fp32_64(wl, pairs):
    """Config 1 in full: the reference's sparse_submanifold_conv3d on the
    16k-voxel 64^3 shell, fp32, 64 -> 64."""
    ref, threads, limits = _reference()
    if ref is None:
        return None
    n = wl["coords"].shape[0]
    t = ref.sparse(wl["coords"], wl["feats"], 1, (64, 64, 64))
    med, best = cpu_timing(lambda: ref.subm_conv3d(t, wl["weight"], wl["bias"]))
    return {"value": round(pairs * 64 * 64 / med / 1e9, 3), "unit": "voxel-GMAC/s", "cores": threads,
            "kind": "reference",
            "sample": f"the whole call: reference sparse_submanifold_conv3d (compiled from its "
                      f"sources, OpenMP, {threads} threads; CPU limits {limits}) on {n} voxels, "
                      f"{pairs} pairs, fp32 64 -> 64; warmup 2, iterations 3: median {med:.4f} s, "
                      f"min {best:.4f} s",
            "median_s": round(med, 5), "min_s": round(best, 5)}


def cpu_baseline_attn_block(wl, flops):
    """Config 3's block on the host: QKV linear, per-head RMS of q and k,
    attention, output linear, by the reference's primitives (fp32)."""
    ref, threads, limits = _reference()
    if ref is None:
        return None
    n, C, H, D = wl["x"].shape[0], 1024, wl["heads"], wl["head_dim"]
    lens = tuple(int(v) for v in (wl["cu_seqlens"][1:] - wl["cu_seqlens"][:-1]))
    g = wl["gamma_q"]
    parts = {"qkv": _cpu_linear(ref, n, C, 3 * C, 81),
             "rms": 2 * _cpu_rowwise(ref, n, lambda t: ref.mh_rms_norm(t, H, D, g), C, 82),
             "attention": _cpu_attention(ref, wl["coords"], lens, H, D, 83),
             "out": _cpu_linear(ref, n, C, C, 84)}
    total = sum(parts.values())
    return {"value": round(flops / total / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "reference",
            "sample": f"extrapolated: reference sparse_linear, sparse_multi_head_rms_norm (on "
                      f"{LIN_CPU_ROWS} sampled rows, scaled by rows) and "
                      f"sparse_scaled_dot_product_attention ({ATTN_CPU_ROWS_BLOCK} query rows per "
                      f"segment against all keys, scaled by queries), {threads} threads (CPU limits "
                      f"{limits}), warmup 2, iterations 3 (median); the block's {n} rows take "
                      + ", ".join(f"{k} {v:.2f} s" for k, v in parts.items()) + f" = {total:.1f} s",
            "extrapolated_s": round(total, 3)}


def cpu_baseline_swin_64(wl, pairs, flops):
    """Config 4 on the host: per shift the window partition (the oracle: the
    reference has none), QKV and output linears and the reference's
    attention over the windows (each window a batch item); then the up-conv
    SubMConv3d 768 -> 1536 and the channel-to-spatial subdivision."""
    import numpy as np

    import oracle as O
    import workloads as W

    ref, threads, limits = _reference()
    if ref is None:
        return None
    orc = O.Oracle()
    coords = wl["coords"]
    n, C, H, D = coords.shape[0], 768, wl["heads"], wl["head_dim"]
    parts = {}
    for shift in wl["shifts"]:
        t0 = time.perf_counter()
        fwd, _, cu = orc.window_partition(coords, wl["shape"], wl["window"], shift)
        t_part = time.perf_counter() - t0
        lens = cu[1:] - cu[:-1]
        # every 16th window (by id), as batch items of their own
        pick = np.arange(0, lens.size, 16)
        rows = np.concatenate([fwd[cu[i]:cu[i + 1]] for i in pick])
        bidx = np.concatenate([np.full(lens[i], j, np.int32) for j, i in enumerate(pick)])
        wc = coords[rows].copy()
        wc[:, 0] = bidx
        q = W.normal(91 + shift, rows.size * C, 1).reshape(rows.size, C)
        t = ref.sparse(wc, q, pick.size, wl["shape"])
        med, _ = cpu_timing(lambda: ref.sdpa(t, t, t, H, D, D ** -0.5))
        scale = float((lens.astype(np.float64) ** 2).sum() / (lens[pick].astype(np.float64) ** 2).sum())
        parts[f"partition_{shift}"] = t_part
        parts[f"window_attention_{shift}"] = med * scale
        parts[f"qkv_{shift}"] = _cpu_linear(ref, n, C, 3 * C, 92 + shift)
        parts[f"out_{shift}"] = _cpu_linear(ref, n, C, C, 94 + shift)
    # the up-conv on the voxels of a slab (x below a cut holding ~1/64 of the
    # voxels), scaled by the pair count
    cut = int(np.quantile(coords[:, 1], 1.0 / 64))
    sub = np.ascontiguousarray(coords[coords[:, 1] < cut])
    sub_pairs = int((orc.neighbor_map(sub) != sub.shape[0]).sum())
    rng = np.random.default_rng(95)  # values do not change the reference's time
    w_up = (rng.standard_normal((27, 1536, C), dtype=np.float32) * 0.02).astype(np.float32)
    b_up = np.zeros(1536, np.float32)
    t_up = ref.sparse(sub, W.normal(96, sub.shape[0] * C, 1).reshape(-1, C), 1, wl["shape"])
    med, _ = cpu_timing(lambda: ref.subm_conv3d(t_up, w_up, b_up), warmup=1, iterations=3)
    parts["up_conv"] = med * pairs / sub_pairs
    t_c2s = ref.sparse(coords, rng.standard_normal((n, 1536), dtype=np.float32), 1, wl["shape"])
    med, _ = cpu_timing(lambda: ref.channel_to_spatial(t_c2s, 2))
    parts["c2s"] = med
    total = sum(parts.values())
    return {"value": round(flops / total / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "reference",
            "sample": f"extrapolated: reference sparse_linear ({LIN_CPU_ROWS} sampled rows, scaled "
                      f"by rows), sparse_scaled_dot_product_attention over every 16th window "
                      f"(scaled by sum L^2), sparse_submanifold_conv3d 768 -> 1536 on the voxels of "
                      f"a slab ({sub.shape[0]} voxels, {sub_pairs} of {pairs} pairs; scaled by "
                      f"pairs), sparse_channel_to_spatial in full; window partition by the oracle "
                      f"(no reference); {threads} threads (CPU limits {limits}), warmup 2 (1 for the "
                      f"conv), iterations 3 (median): "
                      + ", ".join(f"{k} {v:.2f} s" for k, v in parts.items()) + f" = {total:.1f} s",
            "extrapolated_s": round(total, 3)}


def cpu_baseline_flow_step(wl, flops):
    """Config 5 on the host: one transformer block's primitives (adaLN layer
    norms, QKV, RMS, RoPE, self-attention, output, cross-attention with its
    context linears, MLP) by the reference, times 24 blocks, plus the input and
    output linears."""
    ref, threads, limits = _reference()
    if ref is None:
        return None
    coords = wl["coords"]
    n, C, H, M, T = coords.shape[0], wl["width"], wl["heads"], wl["mlp_hidden"], wl["context_tokens"]
    D = C // H
    import numpy as np

    one = np.ones(C, np.float32)
    zero = np.zeros(C, np.float32)
    blk = {"layer_norms": 3 * _cpu_rowwise(ref, n, lambda t: ref.layer_norm(t, 1e-6, one, zero), C, 61),
           "qkv": _cpu_linear(ref, n, C, 3 * C, 62),
           "rms_rope": 2 * _cpu_rowwise(ref, n, lambda t: ref.mh_rms_norm(t, H, D, one), C, 63)
                       + 2 * _cpu_rowwise(ref, n, lambda t: ref.rope(t, H, D), C, 64),
           "self_attention": _cpu_attention(ref, coords, (n,), H, D, 65),
           "out": _cpu_linear(ref, n, C, C, 66),
           "cross_q": _cpu_linear(ref, n, C, C, 67),
           "cross_kv": _cpu_linear(ref, T, C, 2 * C, 68),
           "cross_attention": _cpu_attention(ref, coords, (n,), H, D, 69, keys=T),
           "cross_out": _cpu_linear(ref, n, C, C, 70),
           "mlp0": _cpu_linear(ref, n, C, M, 71),
           "mlp2": _cpu_linear(ref, n, M, C, 72)}
    per_block = sum(blk.values())
    io = _cpu_linear(ref, n, 8, C, 73) + _cpu_linear(ref, n, C, 8, 74)
    total = wl["blocks"] * per_block + io
    return {"value": round(flops / total / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": "reference",
            "sample": f"extrapolated: one block's reference primitives (row-wise ops on "
                      f"{LIN_CPU_ROWS} sampled rows scaled by rows; self- and cross-attention on "
                      f"{ATTN_CPU_ROWS_BLOCK} query rows scaled by queries), {threads} threads (CPU "
                      f"limits {limits}), warmup 2, iterations 3 (median); per block "
                      + ", ".join(f"{k} {v:.2f} s" for k, v in blk.items())
                      + f" = {per_block:.1f} s; x {wl['blocks']} blocks + input/output linears "
                        f"{io:.2f} s = {total:.0f} s per step",
            "extrapolated_s": round(total, 2)}


# ---------------------------------------------------------------------------
# The other configurations (parity cases; timed here for profiling).

def timed_steps(args, torch, step, timer=None):
    """Mean wall time of one step over args.steps after args.warmup untimed
    steps; the per-kernel timer restarts after the warmup."""
    warm_up(args, torch, step)
    if timer is not None:
        timer.reset()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / args.steps


def conv_fp32_64(args, torch, px, W):
    """One fp32 SubMConv3d 64 -> 64 on ~16k voxels at 64^3: voxel grid, then the
    convolution with its neighbours looked up in the grid."""
    import numpy as np

    dev = torch.device("cuda:0")
    wl = W.conv_fp32_64()
    coords = torch.from_numpy(wl["coords"]).to(dev)
    n = coords.shape[0]
    x = torch.from_numpy(wl["feats"]).to(dev)
    w = torch.from_numpy(wl["weight"]).to(dev)
    b = torch.from_numpy(wl["bias"]).to(dev)
    y = torch.empty((n, 64), dtype=torch.float32, device=dev)
    grid = torch.empty(px.lib.pxs_voxel_grid_bytes(1, 64, 64, 64) // 4, dtype=torch.int32,
                       device=dev)
    timer = Timer(torch)

    def build():
        px._check(px.lib.pxs_voxel_grid_build(coords.data_ptr(), n, 1, 64, 64, 64,
                                              grid.data_ptr(), px.stream()),
                  "pxs_voxel_grid_build")

    def step():
        timer.run("voxel_grid", build)
        timer.run("conv", lambda: px.subm_conv3d_grid(x, w, b, coords, 1, (64, 64, 64), grid, 0,
                                                      out=y))

    nbr, masks = px.neighbor_map(coords)
    pairs = int(np.unpackbits(masks.cpu().numpy().view(np.uint8)).sum())
    dt = timed_steps(args, torch, step, timer)
    macs = pairs * 64 * 64
    conv_ms = timer.mean_ms("conv")
    achieved = 2.0 * macs / (conv_ms * 1e-3) / 1e12
    cpu = None if args.no_cpu_baseline else cpu_baseline_conv_fp32_64(wl, pairs)
    return {"metric": "SubMConv3d voxel-GMAC/s, fp32 64->64 at 64^3", "value": round(macs / dt / 1e9, 2),
            "cpu_baseline": cpu,
            "unit": "voxel-GMAC/s", "ms_per_step": round(dt * 1e3, 4), "dtype": "f32",
            "config": {"workload": f"conv_fp32_64: {n} voxels, {pairs} pairs, voxel grid + "
                                   "SubMConv3d with its neighbours looked up in the grid",
                       "voxel_grid_ms": round(timer.mean_ms("voxel_grid"), 4),
                       "conv_ms": round(conv_ms, 4)},
            "roofline": {"bound": "mfma", "kernel": "conv", "achieved": round(achieved, 2),
                         "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": None}}


def attn_block(args, torch, px, W):
    """Attention block: QKV linear 1024->3072, per-head RMS on q/k, varlen attention on
    12,288 + 20,480 tokens (16 x 64), output linear 1024->1024, bf16."""
    dev = torch.device("cuda:0")
    wl = W.attn_full()
    n, C, H, D = wl["x"].shape[0], 1024, wl["heads"], wl["head_dim"]
    bf = lambda a: torch.from_numpy(a).to(dev).to(torch.bfloat16)  # noqa: E731
    f32 = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    x, w_qkv, w_out = bf(wl["x"]), bf(wl["w_qkv"]), bf(wl["w_out"])
    b_qkv, b_out, gq, gk = f32(wl["b_qkv"]), f32(wl["b_out"]), f32(wl["gamma_q"]), f32(wl["gamma_k"])
    cu = f32(wl["cu_seqlens"])
    qkv = torch.empty((n, 3 * C), dtype=torch.bfloat16, device=dev)
    o = torch.empty((n, C), dtype=torch.bfloat16, device=dev)
    y = torch.empty((n, C), dtype=torch.bfloat16, device=dev)
    timer = Timer(torch)

    def step():
        timer.run("qkv", lambda: px.linear(x, w_qkv, b_qkv, out=qkv))
        q, k, v = timer.run("prepare", lambda: px.qkv_prepare(qkv, H, D, gq, gk))
        timer.run("attention", lambda: px.varlen_attention(q, k, v, cu, cu, H, D, D ** -0.5, out=o))
        timer.run("out", lambda: px.linear(o, w_out, b_out, out=y))

    dt = timed_steps(args, torch, step, timer)
    lens = (wl["cu_seqlens"][1:] - wl["cu_seqlens"][:-1]).tolist()
    f_attn = 4.0 * sum(L * L for L in lens) * D * H
    flops = 2.0 * n * C * 3 * C + f_attn + 2.0 * n * C * C
    a_ms = timer.mean_ms("attention")
    achieved = f_attn / (a_ms * 1e-3) / 1e12
    per_op = {k: round(timer.mean_ms(k), 4) for k in ("qkv", "prepare", "attention", "out")}
    cpu = None if args.no_cpu_baseline else cpu_baseline_attn_block(wl, flops)
    return {"metric": "sparse full-attention block TFLOP/s, bf16", "value": round(flops / dt / 1e12, 2),
            "cpu_baseline": cpu,
            "unit": "TFLOP/s", "ms_per_step": round(dt * 1e3, 4), "dtype": "bf16",
            "config": {"workload": "attn_block: 12,288 + 20,480 tokens, width 1024, 16 x 64",
                       "per_op_ms": per_op, "flop_per_step": flops},
            "roofline": {"bound": "mfma", "kernel": "attention", "achieved": round(achieved, 2),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None}}


def swin_64(args, torch, px, W):
    """Two shifted-window attention blocks (window 8, shift 0 then 4,
    12 x 64, width 768) on ~28k voxels at 64^3, then the channel-to-spatial
    upsample: SubMConv3d 768 -> 8*192 at 64^3 and subdivision to 128^3."""
    dev = torch.device("cuda:0")
    wl = W.swin_64()
    coords = torch.from_numpy(wl["coords"]).to(dev)
    n, C, H, D = wl["x"].shape[0], 768, wl["heads"], wl["head_dim"]
    bf = lambda a: torch.from_numpy(a).to(dev).to(torch.bfloat16)  # noqa: E731
    f32 = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    x, w_qkv, w_out, w_up = bf(wl["x"]), bf(wl["w_qkv"]), bf(wl["w_out"]), bf(wl["w_up"])
    b_qkv, b_out, b_up = f32(wl["b_qkv"]), f32(wl["b_out"]), f32(wl["b_up"])
    h = x.clone()
    qkv = torch.empty((n, 3 * C), dtype=torch.bfloat16, device=dev)
    o = torch.empty((n, C), dtype=torch.bfloat16, device=dev)
    packed = torch.empty((n, 8 * 192), dtype=torch.bfloat16, device=dev)
    grid = torch.empty(px.lib.pxs_voxel_grid_bytes(1, *wl["shape"]) // 4, dtype=torch.int32,
                       device=dev)
    timer = Timer(torch)
    win_flops = []

    def build():
        px._check(px.lib.pxs_voxel_grid_build(coords.data_ptr(), n, 1, *wl["shape"],
                                              grid.data_ptr(), px.stream()),
                  "pxs_voxel_grid_build")

    def step():
        for shift in wl["shifts"]:
            fwd, bwd, cu, nw = timer.run(f"partition_{shift}", lambda: px.window_partition(
                coords, 1, wl["shape"], wl["window"], shift, sync=False))
            if len(win_flops) < len(wl["shifts"]):
                lens = (cu[1:] - cu[:-1]).cpu().double()
                win_flops.append(float(4.0 * (lens * lens).sum() * D * H))
            timer.run("qkv", lambda: px.linear(h, w_qkv, b_qkv, out=qkv))
            q, k, v = qkv[:, :C], qkv[:, C:2 * C], qkv[:, 2 * C:]
            timer.run("window_attention", lambda: px.varlen_attention(
                q, k, v, cu, cu, H, D, D ** -0.5, row_map=fwd, out=o, nseg=nw))
            timer.run("out", lambda: px.linear(o, w_out, b_out, out=h))
        # the up-conv looks its neighbours up in the voxel grid (no map)
        timer.run("voxel_grid", build)
        timer.run("up_conv", lambda: px.subm_conv3d_grid(h, w_up, b_up, coords, 1, wl["shape"],
                                                         grid, 0, out=packed))
        timer.run("c2s", lambda: px.channel_to_spatial(coords, packed))

    dt = timed_steps(args, torch, step, timer)
    nbr, masks = px.neighbor_map(coords)
    import numpy as np
    pairs = int(np.unpackbits(masks.cpu().numpy().view(np.uint8)).sum())
    f_win = sum(win_flops)
    f_lin = len(wl["shifts"]) * (2.0 * n * C * 3 * C + 2.0 * n * C * C)
    f_up = 2.0 * pairs * C * 8 * 192
    flops = f_win + f_lin + f_up
    per_op = {k: round(timer.mean_ms(k), 4) for k in ("qkv", "window_attention", "out", "voxel_grid",
                                                      "up_conv", "c2s", "partition_0", "partition_4")}
    up_tf = f_up / (timer.mean_ms("up_conv") * 1e-3) / 1e12
    # Window attention per shift reads Q, K, V (3C bf16 per row) and the
    # row map, and writes O (C bf16 per row): about 68 flop per byte here,
    # below the 312 flop/byte ridge of 2.5 PFLOP/s over 8 TB/s, so HBM bounds it.
    win_ms = timer.mean_ms("window_attention")
    win_bytes = n * (3 * C * 2 + C * 2 + 4)
    win_gbs = win_bytes / (win_ms * 1e-3) / 1e9
    cpu = None if args.no_cpu_baseline else cpu_baseline_swin_64(wl, pairs, flops)
    return {"metric": "shifted-window attention + C2S upsample TFLOP/s, bf16",
            "value": round(flops / dt / 1e12, 2), "unit": "TFLOP/s", "ms_per_step": round(dt * 1e3, 4),
            "cpu_baseline": cpu,
            "dtype": "bf16",
            "config": {"workload": f"swin_64: {n} voxels, window 8 shift 0/4, 12 x 64, "
                                   f"up-conv 768->1536 ({pairs} pairs) + C2S to 128^3",
                       "per_op_ms": per_op,
                       "window_attention_tflops": round(
                           f_win / len(wl["shifts"]) / (win_ms * 1e-3) / 1e12, 2),
                       "window_attention_roofline": {
                           "bound": "hbm", "achieved": round(win_gbs, 1), "peak": PEAK_HBM_GBS,
                           "unit": "GB/s", "frac": round(win_gbs / PEAK_HBM_GBS, 4),
                           "bytes_per_launch": win_bytes,
                           "flop_per_byte": round(f_win / len(wl["shifts"]) / win_bytes, 1)}},
            "roofline": {"bound": "mfma", "kernel": "up_conv", "achieved": round(up_tf, 2),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(up_tf / PEAK_BF16_TFLOPS, 4), "traffic": None}}


def flow_model(torch, px, W):
    """The 24-block SLat-flow model (width 1024, 16 x 64 heads, MLP 4096) on
    ~42k voxels at 64^3 with random N(0, 0.02) weights, bf16 GEMM operands."""
    import pxs as P

    dev = torch.device("cuda:0")
    wl = W.flow_step_64()
    coords = torch.from_numpy(wl["coords"]).to(dev)
    n, C, H, M, T = coords.shape[0], wl["width"], wl["heads"], wl["mlp_hidden"], wl["context_tokens"]
    nb = wl["blocks"]
    g = torch.Generator(device=dev).manual_seed(5)
    rnd = lambda *s, std=0.02, dt=torch.bfloat16: (torch.randn(*s, generator=g, device=dev) * std).to(dt)  # noqa: E731
    one = lambda c: torch.ones(c, device=dev)  # noqa: E731
    zero = lambda c: torch.zeros(c, device=dev)  # noqa: E731
    keep = []
    blocks = []
    for _ in range(nb):
        ws = [rnd(6 * C, dt=torch.float32), rnd(3 * C, C), zero(3 * C), one(C), one(C), rnd(C, C),
              zero(C), one(C), zero(C), rnd(C, C), zero(C), rnd(2 * C, C), zero(2 * C), one(C),
              one(C), rnd(C, C), zero(C), None, None, rnd(M, C), zero(M), rnd(C, M), zero(C)]
        keep.append(ws)
        blocks.append(P.block_weights(ws))
    fw = [rnd(C, 8, dt=torch.float32), zero(C), rnd(C, 256, dt=torch.float32), zero(C),
          rnd(C, C, dt=torch.float32), zero(C), rnd(6 * C, C, dt=torch.float32), zero(6 * C),
          rnd(8, C, dt=torch.float32), zero(8)]
    arr = (P.BlockWeights * nb)(*blocks)
    weights = P.FlowWeights(*[t.data_ptr() for t in fw], arr)
    cfg = P.FlowConfig(8, 8, C, C, nb, H, 0, M, 1e-6, 1.0, 10000.0, 1, 1, 0)
    ctx = torch.randn(T, C, generator=g, device=dev).to(torch.bfloat16)
    ctx_off = torch.tensor([0, T], dtype=torch.int64, device=dev)
    cu = px.batch_cu_seqlens(coords, 1)
    f_self = 4.0 * n * n * 64 * H
    f_lin = 2.0 * n * C * (3 * C + C + C + C + 2 * M)
    f_cross = 4.0 * n * T * 64 * H + 2.0 * T * C * 2 * C
    flops = nb * (f_self + f_lin + f_cross) + 2.0 * n * (8 * C + C * 8)
    return dict(cfg=cfg, weights=weights, keep=(keep, fw, arr), coords=coords, cu=cu, ctx=ctx,
                ctx_off=ctx_off, n=n, T=T, flops=flops, g=g, dev=dev)


def flow_step(args, torch, px, W):
    """One SLat-flow forward (24 blocks, width 1024) on ~42k voxels,
    device resident (pxs_slat_flow_forward), random N(0, 0.02) weights."""
    import pxs as P

    m = flow_model(torch, px, W)
    n, T, dev, g = m["n"], m["T"], m["dev"], m["g"]
    x = torch.randn(n, 8, generator=g, device=dev)
    tsteps = torch.rand(1, generator=g, device=dev) * 1000.0
    out = torch.empty((n, 8), dtype=torch.float32, device=dev)
    ws = torch.empty(px.flow_workspace_bytes(m["cfg"], n, T, 1, P.PXS_BF16), dtype=torch.uint8,
                     device=dev)

    def step():
        px.slat_flow_forward(m["cfg"], m["weights"], m["coords"], 1, m["cu"], x, tsteps, m["ctx"],
                             m["ctx_off"], out=out, workspace=ws, dtype=P.PXS_BF16)

    dt = timed_steps(args, torch, step)
    flops = m["flops"]
    assert torch.isfinite(out).all().item()
    cpu = None if args.no_cpu_baseline else cpu_baseline_flow_step(W.flow_step_64(), flops)
    return {"metric": "SLat-flow step TFLOP/s, bf16", "value": round(flops / dt / 1e12, 2),
            "cpu_baseline": cpu,
            "unit": "TFLOP/s", "ms_per_step": round(dt * 1e3, 4), "dtype": "bf16",
            "config": {"workload": f"flow_step: {n} voxels at 64^3, 24 blocks width 1024 "
                                   f"(16 x 64, MLP 4096), 1,370 context tokens",
                       "flop_per_step": flops},
            "roofline": {"bound": "mfma", "kernel": "whole forward", "achieved": round(flops / dt / 1e12, 2),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(flops / dt / 1e12 / PEAK_BF16_TFLOPS, 4), "traffic": None}}


def flow_sample(args, torch, px, W):
    """Guided flow-Euler sampling with the 24-block width-1024 SLat-flow model (pxs_flow_euler_sample):
    2 Euler steps at guidance 7.5 with CFG rescale 0.7, each step ONE forward
    over the doubled batch (conditional + unconditional, ~84k tokens); the same
    steps composed from two separate forwards are timed beside it."""
    import pxs as P

    m = flow_model(torch, px, W)
    n, T, dev, g = m["n"], m["T"], m["dev"], m["g"]
    noise = torch.randn(n, 8, generator=g, device=dev)
    uncond = torch.zeros_like(m["ctx"])
    out = torch.empty_like(noise)
    steps = 2
    scfg = P.SamplerConfig(steps, 1e-5, 3.0, 7.5, 0.7, 0.0, 1.0)

    def sample():
        px.flow_euler_sample(m["cfg"], m["weights"], scfg, m["coords"], 1, m["cu"], noise, m["ctx"],
                             m["ctx_off"], uncond, m["ctx_off"], dtype=P.PXS_BF16, out=out)

    state = torch.empty_like(noise)
    ws = torch.empty(px.flow_workspace_bytes(m["cfg"], n, T, 1, P.PXS_BF16), dtype=torch.uint8,
                     device=dev)
    sched = [px.flow_sampler_schedule(scfg, i) for i in range(steps)]
    tts = [torch.full((1,), 1000.0 * t, device=dev) for t, _, _ in sched]

    def separate():
        state.copy_(noise)
        for (t, tn, gd), tt in zip(sched, tts):
            pos = px.slat_flow_forward(m["cfg"], m["weights"], m["coords"], 1, m["cu"], state, tt,
                                       m["ctx"], m["ctx_off"], workspace=ws, dtype=P.PXS_BF16)
            neg = px.slat_flow_forward(m["cfg"], m["weights"], m["coords"], 1, m["cu"], state, tt,
                                       uncond, m["ctx_off"], workspace=ws, dtype=P.PXS_BF16)
            pred = px.flow_guidance(state, pos, neg, m["coords"], m["cu"], 1, t, 1e-5, gd, 0.7)
            px.flow_euler_update(state, pred, t - tn)

    dt = timed_steps(args, torch, sample)
    dt_sep = timed_steps(args, torch, separate)
    flops = 2 * steps * m["flops"]
    assert torch.isfinite(out).all().item()
    tf = flops / dt / 1e12
    return {"metric": "SLat-flow guided sampling TFLOP/s, bf16", "value": round(tf, 2),
            "unit": "TFLOP/s", "ms_per_step": round(dt * 1e3, 4), "dtype": "bf16",
            "config": {"workload": f"flow_sample: {n} voxels at 64^3, 24-block width-1024 model, {steps} "
                                   f"Euler steps, guidance 7.5, CFG rescale 0.7, 1,370 context "
                                   f"tokens (uncond: zeros)",
                       "ms_per_euler_step": round(dt * 1e3 / steps, 3),
                       "separate_forwards_ms": round(dt_sep * 1e3, 4),
                       "flop_per_call": flops},
            "roofline": {"bound": "mfma", "kernel": "whole sampler", "achieved": round(tf, 2),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None}}


def pack_load(args, torch, px, W):
    """GGUF ingestion of a SLat-flow component (width 1024, 24
    blocks, F32 storage as the deployed flow packs hold it, 1.6 GB):
    pxs_slat_flow_pack_load from a pack in the page cache into an HBM arena,
    block linears converted to bf16.  A step is one whole load; the pack is
    written once to a temporary file first (synthetic N(0, 0.02) values)."""
    import ctypes as C
    import os
    import tempfile

    import pxs as P

    dev = torch.device("cuda:0")
    tmpdir = os.environ.get("TMPDIR", tempfile.gettempdir())
    path = os.path.join(tmpdir, f"pxs_flow_pack_{os.getpid()}.gguf")
    try:
        payload = W.write_flow_pack(path)
        pack = px.pack_open(path)
        cfg, need = P.FlowConfig(), C.c_size_t()
        name = b"shape_flow_1024"
        px._check(px.lib.pxs_slat_flow_pack_plan(pack.handle, name, P.PXS_BF16, C.byref(cfg),
                                                 C.byref(need)), "pxs_slat_flow_pack_plan")
        arena = torch.empty(need.value, dtype=torch.uint8, device=dev)
        ws = torch.empty(px.lib.pxs_pack_upload_workspace_bytes(pack.handle), dtype=torch.uint8,
                         device=dev)
        blocks = (P.BlockWeights * cfg.num_blocks)()
        weights = P.FlowWeights()

        def step():
            px._check(px.lib.pxs_slat_flow_pack_load(
                pack.handle, name, P.PXS_BF16, C.c_void_p(arena.data_ptr()),
                C.c_size_t(arena.numel()), C.c_void_p(ws.data_ptr()), C.byref(weights), blocks,
                cfg.num_blocks, px.stream()), "pxs_slat_flow_pack_load")

        step()  # warm: page cache, pinned staging, first-touch of the arena
        steps = max(1, min(args.steps, 5))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        pack.close()
        # The bound: host -> HBM DMA from pinned memory on the same stream,
        # in the loader's 16 MiB pieces.
        chunk = 16 << 20
        pinned = torch.empty(chunk, dtype=torch.uint8, pin_memory=True)
        dst = torch.empty(chunk, dtype=torch.uint8, device=dev)
        for _ in range(8):
            dst.copy_(pinned, non_blocking=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(64):
            dst.copy_(pinned, non_blocking=True)
        torch.cuda.synchronize()
        dma = 64 * chunk / (time.perf_counter() - t0) / 1e9
    finally:
        if os.path.exists(path):
            os.remove(path)
    gbs = payload / dt / 1e9
    return {"metric": "SLat-flow pack ingestion GB/s (file payload -> HBM arena)",
            "value": round(gbs, 2), "unit": "GB/s", "ms_per_step": round(dt * 1e3, 3),
            "dtype": "f32->bf16", "steps": steps,
            "config": {"workload": f"pack_load: synthetic shape_flow_1024 pack, width 1024, "
                                   f"24 blocks, F32 payload {payload / 1e9:.3f} GB, page-cache "
                                   f"resident; block linears to bf16, the rest fp32",
                       "arena_bytes": int(need.value), "payload_bytes": int(payload)},
            "roofline": {"bound": "host link (pinned -> HBM DMA)", "kernel": "whole load",
                         "achieved": round(gbs, 2), "peak": round(dma, 2), "unit": "GB/s",
                         "frac": round(gbs / dma, 4), "traffic": None,
                         "peak_note": "measured DMA rate of 16 MiB pinned copies on the same "
                                      "stream (the PCIe gen5 x16 link's ~64 GB/s is the "
                                      "theoretical ceiling)"}}


def decoder(args, torch, px, W):
    """The SLat shape-decoder stack on the device (pxs_slat_decoder_forward):
    ~10.6k latent voxels at 64^3, 5 levels (1024 -> 64 channels), predicted
    subdivisions up to 1024^3, bf16 convolution and MLP operands."""
    import numpy as np

    import pxs as P

    dev = torch.device("cuda:0")
    wl = W.decoder_64()
    coords = torch.from_numpy(wl["coords"]).to(dev)
    n = coords.shape[0]
    chans, nblk = wl["model_channels"], wl["num_blocks"]
    g = torch.Generator(device=dev).manual_seed(7)
    rnd = lambda *s, std=0.02, dt=torch.float32: (torch.randn(*s, generator=g, device=dev) * std).to(dt)  # noqa: E731
    keep, blocks = [], []
    for level, C in enumerate(chans):
        for _ in range(nblk[level]):
            w = {"norm_weight": torch.ones(C, device=dev), "norm_bias": rnd(C),
                 "conv1_weight": rnd(27, C, C, std=(27 * C) ** -0.5, dt=torch.bfloat16),
                 "conv1_bias": rnd(C), "mlp0_weight": rnd(4 * C, C, std=C ** -0.5, dt=torch.bfloat16),
                 "mlp0_bias": rnd(4 * C), "mlp2_weight": rnd(C, 4 * C, std=0.02, dt=torch.bfloat16),
                 "mlp2_bias": rnd(C)}
            keep.append(w)
            blocks.append(P.DecoderBlock(P.PXS_DECODER_CONVNEXT, C, C, 4 * C,
                                         P.decoder_block_weights(w)))
        if level + 1 < len(chans):
            O_ = chans[level + 1]
            w = {"norm1_weight": torch.ones(C, device=dev), "norm1_bias": rnd(C),
                 "conv1_weight": rnd(27, 8 * O_, C, std=(27 * C) ** -0.5, dt=torch.bfloat16),
                 "conv1_bias": rnd(8 * O_),
                 "conv2_weight": rnd(27, O_, O_, std=(27 * O_) ** -0.5, dt=torch.bfloat16),
                 "conv2_bias": rnd(O_), "to_subdiv_weight": rnd(8, C, std=C ** -0.5),
                 "to_subdiv_bias": rnd(8, std=0.0)}
            keep.append(w)
            blocks.append(P.DecoderBlock(P.PXS_DECODER_C2S, C, O_, 0, P.decoder_block_weights(w)))
    cfg = P.decoder_config(wl["latent_channels"], wl["out_channels"], 1e-6, True, chans, nblk)
    fl_w, fl_b = rnd(chans[0], wl["latent_channels"], std=0.2), rnd(chans[0])
    out_w, out_b = rnd(wl["out_channels"], chans[-1], std=0.1), rnd(wl["out_channels"])
    x = torch.randn(n, wl["latent_channels"], generator=g, device=dev)
    # Capacity of every level: 8 x the largest pre-final level (about 4x
    # growth per predicted level here); the call fails loudly past it.
    max_rows = 8_000_000
    res = {}

    def step():
        res["out"] = px.slat_decoder_forward(P.PXS_BF16, cfg, fl_w, fl_b, out_w, out_b, blocks,
                                             coords, x, predict=False, max_rows=max_rows)

    dt = timed_steps(args, torch, step)
    oc, y, level_rows, _ = res["out"]
    assert torch.isfinite(y).all().item()
    # Algorithmic work: active conv pairs per level (from each level's map),
    # ConvNeXt MLPs, C2S convolutions, output linear.
    lvl_coords = [coords] + [px.slat_decoder_forward(P.PXS_BF16, cfg, fl_w, fl_b, out_w, out_b,
                                                     blocks, coords, x, upsample_times=u,
                                                     max_rows=max_rows)[0]
                             for u in range(1, len(chans))]
    macs = 0
    # (pair counts outside the timed region, from the decoder's own map path)
    for level, (c, C) in enumerate(zip(lvl_coords, chans)):
        _, masks = px.neighbor_map_bricks(c)
        pairs = int(np.unpackbits(masks.cpu().numpy().view(np.uint8)).sum())
        macs += nblk[level] * (pairs * C * C + 2 * c.shape[0] * C * 4 * C)
        if level + 1 < len(chans):
            O_ = chans[level + 1]
            _, m_next = px.neighbor_map_bricks(lvl_coords[level + 1])
            pairs_next = int(np.unpackbits(m_next.cpu().numpy().view(np.uint8)).sum())
            macs += pairs * C * 8 * O_ + pairs_next * O_ * O_
    macs += n * wl["latent_channels"] * chans[0] + level_rows[-1] * chans[-1] * wl["out_channels"]
    tf = 2.0 * macs / dt / 1e12
    return {"metric": "SLat decoder stack TFLOP/s, bf16", "value": round(tf, 2), "unit": "TFLOP/s",
            "ms_per_step": round(dt * 1e3, 4), "dtype": "bf16",
            "config": {"workload": f"decoder: {n} latent voxels at 64^3, channels {chans}, "
                                   f"one ConvNeXt block per level, predicted subdivisions",
                       "level_rows": level_rows,
                       "output_voxels_per_s": round(level_rows[-1] / dt, 1),
                       "flop_per_step": 2.0 * macs},
            "roofline": {"bound": "mfma", "kernel": "whole decoder", "achieved": round(tf, 2),
                         "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / PEAK_BF16_TFLOPS, 4), "traffic": None}}


def hash_map_128(args, torch, px, W):
    """The extent-free paths of the neighbour map on the U-Net stage's
    coordinates (162,263 voxels at 128^3, batch 2): the brick table
    (pxs_voxel_bricks_build + pxs_neighbor_map_k3_bricks, the decoder's path)
    and the voxel hash (pxs_voxel_hash_build + pxs_neighbor_map_k3).  Rates
    count the map's compulsory bytes: 16 B of coordinates read and 27 x 4 B of
    map + a 4 B mask written per row.  Also one 256 MiB device copy, the
    plain-copy reference for the FETCH_SIZE / WRITE_SIZE counters."""
    dev = torch.device("cuda:0")
    coords = torch.from_numpy(W.unet_stage_128()["coords"]).to(dev)
    n = coords.shape[0]
    table = torch.empty(px.lib.pxs_voxel_hash_bytes(n), dtype=torch.uint8, device=dev)
    bricks = torch.empty(px.lib.pxs_voxel_bricks_bytes(n), dtype=torch.uint8, device=dev)
    nbr = torch.empty((27, n), dtype=torch.int32, device=dev)
    masks = torch.empty(n, dtype=torch.int32, device=dev)
    timer = Timer(torch)
    src = torch.empty(1 << 28, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)  # the calibration copy (copyBuffer, 2^28 bytes each way)

    import ctypes as C

    lib = px.lib
    P = lambda t: C.c_void_p(t.data_ptr())  # noqa: E731

    def step():
        s = px.stream()
        timer.run("bricks_build", lambda: px._check(lib.pxs_voxel_bricks_build(
            P(coords), n, P(bricks), s), "pxs_voxel_bricks_build"))
        timer.run("neighbor_map_bricks", lambda: px._check(lib.pxs_neighbor_map_k3_bricks(
            P(coords), n, P(bricks), P(nbr), P(masks), s), "pxs_neighbor_map_k3_bricks"))
        timer.run("hash_build", lambda: px._check(lib.pxs_voxel_hash_build(
            P(coords), n, P(table), s), "pxs_voxel_hash_build"))
        timer.run("neighbor_map", lambda: px._check(lib.pxs_neighbor_map_k3(
            P(coords), n, P(table), P(nbr), P(masks), s), "pxs_neighbor_map_k3"))

    dt = timed_steps(args, torch, step, timer)
    ms = {k: timer.mean_ms(k) for k in ("bricks_build", "neighbor_map_bricks", "hash_build",
                                        "neighbor_map")}
    compulsory = n * (16 + 27 * 4 + 4)
    gbs = lambda b, t: round(b / (t * 1e-3) / 1e9, 1)  # noqa: E731
    brick_ms = ms["bricks_build"] + ms["neighbor_map_bricks"]
    return {"metric": "neighbour map GB/s (compulsory bytes), brick table",
            "value": gbs(compulsory, brick_ms), "unit": "GB/s",
            "ms_per_step": round(dt * 1e3, 4), "dtype": "int32",
            "config": {"workload": f"hash_map_128: {n} voxels at 128^3 (batch 2), brick table "
                                   "and voxel hash builds + 3x3x3 maps",
                       "compulsory_bytes_per_row": 16 + 27 * 4 + 4,
                       "per_op_ms": {k: round(v, 4) for k, v in ms.items()},
                       "bricks_build_plus_map_ms": round(brick_ms, 4),
                       "hash_build_plus_map_ms": round(ms["hash_build"] + ms["neighbor_map"], 4),
                       "neighbor_map_bricks_gbs": gbs(compulsory, ms["neighbor_map_bricks"]),
                       "neighbor_map_hash_gbs": gbs(compulsory, ms["neighbor_map"]),
                       "table_bytes": {"bricks": bricks.numel(), "hash": table.numel()}},
            "roofline": {"bound": "hbm", "kernel": "neighbor_map_bricks",
                         "achieved": gbs(compulsory, ms["neighbor_map_bricks"]),
                         "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(compulsory / (ms["neighbor_map_bricks"] * 1e-3) / 1e9
                                       / PEAK_HBM_GBS, 4),
                         "traffic": None}}


# Linear shapes: the configs' block linears (bf16) and the reference's hot
# sparse_linear shapes (tests/sparse_linear_cuda_benchmark.cpp:42-52, fp32).
LINEAR_SHAPES = [
    ("attn_block qkv", "bf16", 32768, 1024, 3072), ("attn_block out", "bf16", 32768, 1024, 1024),
    ("flow mlp0", "bf16", 40960, 1024, 4096), ("flow mlp2", "bf16", 40960, 4096, 1024),
    ("flow qkv", "bf16", 40960, 1024, 3072), ("swin qkv", "bf16", 29700, 768, 2304),
    ("swin out", "bf16", 29700, 768, 768), ("decoder mlp0", "bf16", 2492211, 64, 256),
    ("decoder mlp2", "bf16", 2492211, 256, 64),
    ("hot n46537 2048->512", "f32", 46537, 2048, 512), ("hot n46537 512->2048", "f32", 46537, 512, 2048),
    ("hot n206980 1024->256", "f32", 206980, 1024, 256), ("hot n206980 256->1024", "f32", 206980, 256, 1024),
    ("hot n909164 512->128", "f32", 909164, 512, 128), ("hot n909164 128->512", "f32", 909164, 128, 512),
    ("hot n9857 4096->1024", "f32", 9857, 4096, 1024), ("hot n9857 1024->4096", "f32", 9857, 1024, 4096),
]


def linear_dense(args, torch, px, W):
    """pxs_linear (the dense MFMA kernel) on each shape of LINEAR_SHAPES, timed
    with HIP events, next to torch's linear on the same operands (hipBLASLt:
    a comparison leg only).  value = all shapes' flops / all shapes' time."""
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    steps = max(5, min(args.steps, 50))
    rows_out, total_f, total_t = [], 0.0, 0.0
    qkv = None
    for name, dt, m, k, n in LINEAR_SHAPES:
        tdt = torch.bfloat16 if dt == "bf16" else torch.float32
        g = torch.Generator(device=dev).manual_seed(m + k + n)
        x = torch.randn(m, k, device=dev, generator=g).to(tdt)
        w = (torch.randn(n, k, device=dev, generator=g) * k ** -0.5).to(tdt)
        b = torch.randn(n, device=dev, generator=g) * 0.1
        y = torch.empty(m, n, device=dev, dtype=tdt)
        bt = b.to(tdt)

        def ours():
            px.linear(x, w, b, out=y)

        def lib():
            torch.nn.functional.linear(x, w, bt)

        res = {}
        for leg, fn in (("pxs", ours), ("hipblaslt", lib)):
            t0 = time.perf_counter()  # warm up for 0.2 s so the clocks settle
            while time.perf_counter() - t0 < 0.2:
                for _ in range(3):
                    fn()
                torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(steps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            res[leg] = e0.elapsed_time(e1) / steps
        flops = 2.0 * m * k * n
        total_f += flops
        total_t += res["pxs"] * 1e-3
        row = {"shape": name, "dtype": dt, "rows": m, "cin": k, "cout": n,
               "pxs_us": round(res["pxs"] * 1e3, 1), "hipblaslt_us": round(res["hipblaslt"] * 1e3, 1),
               "pxs_tflops": round(flops / (res["pxs"] * 1e-3) / 1e12, 1),
               "hipblaslt_tflops": round(flops / (res["hipblaslt"] * 1e-3) / 1e12, 1),
               "ratio": round(res["hipblaslt"] / res["pxs"], 3)}
        rows_out.append(row)
        if name == "attn_block qkv":
            qkv = row
        del x, w, y
        torch.cuda.empty_cache()
    achieved = qkv["pxs_tflops"]
    return {"metric": "dense linear TFLOP/s (pxs_linear), bf16 block shapes and fp32 reference shapes",
            "value": round(total_f / total_t / 1e12, 2), "unit": "TFLOP/s",
            "ms_per_step": round(total_t * 1e3, 4), "dtype": "bf16+f32",
            "config": {"workload": f"linear_dense: {len(LINEAR_SHAPES)} shapes, {steps} calls each, "
                                   "torch.nn.functional.linear (hipBLASLt) timed beside each",
                       "shapes": rows_out},
            "roofline": {"bound": "mfma", "kernel": "dense_gemm (attn_block qkv 32768x1024->3072)",
                         "achieved": achieved, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None}}


def attn_wide(args, torch, px, W):
    """Head dims above 64 (the wavefront-per-query kernel) against the tiled
    head_dim-64 kernel on config 3's tokens at the same width (1,024)."""
    res = {hd: attention_metric(args, torch, px, W, heads=1024 // hd, hd=hd) for hd in (64, 128)}
    wide = res[128]
    return {"metric": "varlen attention TFLOP/s, head_dim 128 (8 heads) vs 64 (16 heads)",
            "value": wide["tflops"], "unit": "TFLOP/s", "ms_per_step": wide["ms"], "dtype": "bf16",
            "config": {"workload": "attn_wide: 12,288 + 20,480 tokens, width 1,024",
                       "head_dim_128": wide, "head_dim_64": res[64]},
            "roofline": {"bound": "mfma", "kernel": "attention head_dim 128",
                         "achieved": wide["tflops"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                         "frac": wide["frac"], "traffic": None}}


OTHER_WORKLOADS = {"conv_fp32_64": conv_fp32_64, "attn_block": attn_block, "swin_64": swin_64,
                   "flow_sample": flow_sample, "decoder": decoder, "pack_load": pack_load,
                   "flow_step": flow_step, "hash_map_128": hash_map_128, "linear_dense": linear_dense,
                   "attn_wide": attn_wide}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              f"(the sparse path would shard by segment and by spatial slab)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    import pxs
    import workloads as W

    px = pxs.Pxs()
    if args.workload != "unet_stage_128":
        result = OTHER_WORKLOADS[args.workload](args, torch, px, W)
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
        if "attention" in base:
            base["attention"]["cpu_baseline"] = cpu_baseline_attention()
    if args.workload == "unet_stage_128" and not args.no_configs:
        # Configs 1 and 4 ride on the default line (with their CPU baselines),
        # each at up to 100 timed steps after 20 warm-up steps.
        sub = argparse.Namespace(**vars(args))
        sub.steps, sub.warmup = min(args.steps, 100), min(args.warmup, 20)
        for key, fn in (("config1_conv_fp32_64", conv_fp32_64), ("config4_swin_64", swin_64)):
            base[key] = fn(sub, torch, px, W)
    print(json.dumps(base), flush=True)


if __name__ == "__main__":
    main()
