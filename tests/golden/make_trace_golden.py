#!/usr/bin/env python3
"""Write flow_trace_lines.json: the stderr lines and error of the reference's
flow_euler_sample_f32 with PIXAL3D_FLOW_NONFINITE_TRACE=1
(src/flow_sampler.cpp:20-83, 237-345), compiled from its sources into
oracle/_ref, for three runs driven by the seeded velocity callback of the
sampler tests:

* guided_rescale - 2 steps, guidance 7.5, CFG rescale 0.7, trajectories kept;
* unguided       - 2 steps, guidance 1, trajectories kept;
* blend_overflow - a callback returning +-3e38, whose CFG blend overflows: the
                   trace fails at step 0 with the reference's message.

Runs in the build container only (it needs /root/reference to build
oracle/_ref).  Usage:  python tests/golden/make_trace_golden.py
"""

from __future__ import annotations

import json
import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
for sub in ("oracle", "pixal3d.cpp_amd/python", "tests"):
    sys.path.insert(0, str(ROOT / sub))

import oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent


def main() -> int:
    from fixtures import TRACE_CASES, capture_stderr, overflow_velocity
    from test_oracle import sampler_inputs

    ref = O.Reference()
    coords, noise, fn = sampler_inputs()
    out = {}
    os.environ["PIXAL3D_FLOW_NONFINITE_TRACE"] = "1"
    try:
        for name, (steps, cfg, record) in TRACE_CASES.items():
            velocity = overflow_velocity if name == "blend_overflow" else fn

            def run():
                try:
                    ref.flow_euler_sample(ref.sparse(coords, noise, 2, (12, 12, 12)), steps, cfg,
                                          velocity, record=record)
                    return None
                except O.ReferenceError as e:
                    return str(e)

            error, text = capture_stderr(run)
            lines = [ln for ln in text.splitlines() if ln.startswith("pixal3d: flow trace")]
            out[name] = {"steps": steps, "cfg": cfg, "record": record, "lines": lines,
                         "error": error}
    finally:
        del os.environ["PIXAL3D_FLOW_NONFINITE_TRACE"]
    (OUT / "flow_trace_lines.json").write_text(json.dumps(out, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
