"""CPU checks of bench.py's contract that need no GPU: one GPU only, the
measured traffic it reports for the roofline kernel, the CPU-baseline thread
count and timing method."""

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_traffic_comes_from_the_committed_summary():
    rec = json.loads((ROOT / "profiles" / "unet_stage_128_traffic.json").read_text())["subm_conv_a"]
    got = bench.measured_traffic("subm_conv_a")
    assert got == rec["read_bytes"] + rec["write_bytes"]
    # conv A's algorithmic bytes: features in and out, weights, map and masks
    n, cin, cout = 162263, 128, 128
    algorithmic = n * cin * 2 + n * cout * 2 + 27 * cout * cin * 2 + 27 * n * 4 + n * 4
    assert algorithmic < got < 2 * algorithmic
    assert bench.measured_traffic("not_a_kernel") is None


def test_traffic_note_flags_changed_kernel_sources(monkeypatch):
    """The note names the commit the traffic was measured at and says whether
    the kernel sources the record lists still hash as they did then."""
    rec = json.loads((ROOT / "profiles" / "unet_stage_128_traffic.json").read_text())["subm_conv_a"]
    assert rec["sources"] and all((ROOT / p).exists() for p in rec["sources"])
    assert rec["measured_at_commit"] in bench.traffic_note("subm_conv_a")
    monkeypatch.setattr(bench, "kernel_source_digest", lambda r: rec["sources_sha16"])
    assert "unchanged since" in bench.traffic_note("subm_conv_a")
    monkeypatch.setattr(bench, "kernel_source_digest", lambda r: "0" * 16)
    assert "STALE" in bench.traffic_note("subm_conv_a")


def test_cpu_threads_respect_every_limit(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "3")
    threads, limits = bench.cpu_threads()
    assert limits["OMP_NUM_THREADS"] == 3 and threads == min(limits.values()) and threads >= 1


def test_cpu_timing_is_median_and_min_after_warmup():
    calls = []
    durations = iter([0.0, 0.0, 0.03, 0.01, 0.02])

    def fn():
        import time
        calls.append(1)
        time.sleep(next(durations))

    med, lo = bench.cpu_timing(fn, warmup=2, iterations=3)
    assert len(calls) == 5
    assert lo <= med and 0.015 < med < 0.03 and lo < 0.02
