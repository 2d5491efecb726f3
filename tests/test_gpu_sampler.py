"""GPU parity: the flow-matching Euler sampler (src/flow_sampler.cpp).

* pxs_flow_guidance / pxs_flow_pred_to_xstart / pxs_flow_euler_update against
  the oracle (itself bit-exact against the compiled reference): bit for bit.
* The drop-in pixal3d::flow_euler_sample_f32 (device arithmetic, host model
  callback) against the oracle driven by the same callback: bit for bit,
  trajectories included, plus the reference's error messages.
* pxs_flow_euler_sample (the SLat-flow model on the device, conditional and
  unconditional forwards batched into one) against the same steps composed
  from separate forwards (bit for bit) and against the oracle sampler driving
  the oracle's flow forward (fp32 tolerance)."""

import numpy as np
import pytest
import torch

import oracle as O
import pxs
from gpu_common import FP32_TOL, host, max_rel, t32, ti32, ti64
from test_gpu_block import device_weights
from test_oracle import SAMPLER_CASES, sampler_inputs

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def px():
    return pxs.Pxs()


@pytest.fixture(scope="module")
def orc():
    return O.Oracle()


@pytest.mark.parametrize("t", [0.9, 0.15])
@pytest.mark.parametrize("guidance,rescale", [(3.0, 0.0), (7.5, 0.7), (4.0, 1.0), (0.5, 0.3)])
def test_guidance_bit_exact(px, orc, t, guidance, rescale):
    coords, state, _ = sampler_inputs(63)
    n = coords.shape[0]
    pos = (state * np.float32(0.7) + np.float32(0.2)).astype(np.float32)
    neg = np.tanh(state).astype(np.float32)
    print(f"[flow guidance] t={t} g={guidance} rescale={rescale} n={n}", flush=True)
    c = ti32(coords)
    cu = px.batch_cu_seqlens(c, 2)
    got = px.flow_guidance(t32(state), t32(pos), t32(neg), c, cu, 2, t, 1e-5, guidance, rescale)
    ref = orc.flow_guidance(state, pos, neg, coords, 2, t, 1e-5, guidance, rescale)
    np.testing.assert_array_equal(host(got), ref)


def test_euler_update_and_xstart_bit_exact(px):
    _, state, _ = sampler_inputs(64)
    pred = np.cos(state).astype(np.float32)
    t, sm = np.float32(0.37), np.float32(1e-5)
    a = np.float32(1.0) - sm
    b = sm + a * t
    x0 = host(px.flow_pred_to_xstart(t32(state), t32(pred), float(t), float(sm)))
    np.testing.assert_array_equal(x0, a * state - b * pred)
    s = t32(state)
    px.flow_euler_update(s, t32(pred), 0.125)
    np.testing.assert_array_equal(host(s), state - np.float32(0.125) * pred)


@pytest.mark.parametrize("case", list(SAMPLER_CASES))
def test_dropin_sampler_bit_exact(orc, case):
    steps, cfg = SAMPLER_CASES[case]
    coords, noise, fn = sampler_inputs()
    print(f"[drop-in sampler] case={case} steps={steps}", flush=True)
    d = O.DropIn()
    out, xt, x0 = d.flow_euler_sample(d.sparse(coords, noise, 2, (12, 12, 12)), steps, cfg, fn,
                                      record=True)
    ref, rxt, rx0 = orc.flow_euler_sample(coords, 2, noise, steps, cfg, fn, record=True)
    np.testing.assert_array_equal(out.read()[1], ref)
    np.testing.assert_array_equal(xt, rxt)
    np.testing.assert_array_equal(x0, rx0)


def test_dropin_sampler_errors():
    coords, noise, fn = sampler_inputs()
    d = O.DropIn()
    t = d.sparse(coords, noise, 2, (12, 12, 12))
    with pytest.raises(O.ReferenceError, match="invalid flow Euler sampler configuration"):
        d.flow_euler_sample(t, 3, [1e-5, 1.0, 1.0, 0.0, 0.9, 0.1], fn)
    with pytest.raises(O.ReferenceError, match="model callback is empty"):
        d.flow_euler_sample(t, 3, [1e-5, 1.0, 1.0, 0.0, 0.0, 1.0], None)
    bad = lambda s, tm, c: np.full_like(s, np.nan) if c else s  # noqa: E731
    with pytest.raises(O.ReferenceError, match="non-finite"):
        d.flow_euler_sample(t, 3, [1e-5, 1.0, 1.0, 0.0, 0.0, 1.0], bad)


# --- the device sampler over the SLat-flow model --------------------------------

def flow_setup(px, dtype, seed=71):
    from fixtures import flow_case
    case = flow_case(seed, [[(4.0, 6.0)], [(3.0, 5.0)]], 16, 64, 2, 2, 7)
    C, H, M, CC = case["C"], case["H"], case["M"], case["CC"]
    nb = len(case["blocks"])
    cfg = pxs.FlowConfig(8, 8, C, CC, nb, H, 0, M, 1e-6, 1.0, 10000.0, 1, 1, 0)
    fw_dev = [t32(a) for a in case["fw"]]
    blk_dev = [device_weights(ws, dtype) for ws in case["blocks"]]
    arr = (pxs.BlockWeights * max(nb, 1))(*[pxs.block_weights(b) for b in blk_dev])
    weights = pxs.FlowWeights(*[a.data_ptr() for a in fw_dev], arr)
    keep = (fw_dev, blk_dev, arr)
    rng = np.random.default_rng(seed)
    uncond = rng.standard_normal((2 * 3, CC)).astype(np.float32) * np.float32(0.5)
    return case, cfg, weights, keep, uncond


def test_device_sampler_batched_cfg_equals_separate_forwards(px):
    """Each guided step's single forward over the doubled batch gives the
    conditional and unconditional velocities the two separate forwards give,
    bit for bit, so the sampler equals its unbatched composition."""
    case, cfg, weights, keep, uncond = flow_setup(px, torch.float32)
    coords = ti32(case["coords"])
    cu = px.batch_cu_seqlens(coords, 2)
    ctx, ctx_off = t32(case["ctx"]), ti64(case["ctx_off"])
    unc, unc_off = t32(uncond), ti64(np.array([0, 3, 6], np.int64))
    noise = t32(np.random.default_rng(3).standard_normal((case["n"], 8)).astype(np.float32))
    scfg = pxs.SamplerConfig(3, 1e-5, 3.0, 5.0, 0.7, 0.0, 1.0)
    print(f"[device sampler] n={case['n']} steps=3", flush=True)
    got = px.flow_euler_sample(cfg, weights, scfg, coords, 2, cu, noise, ctx, ctx_off, unc,
                               unc_off)
    state = noise.clone()
    for step in range(3):
        t, tn, g = px.flow_sampler_schedule(scfg, step)
        tt = torch.full((2,), float(np.float32(1000.0) * np.float32(t)), dtype=torch.float32,
                        device="cuda")
        pos = px.slat_flow_forward(cfg, weights, coords, 2, cu, state, tt, ctx, ctx_off)
        neg = px.slat_flow_forward(cfg, weights, coords, 2, cu, state, tt, unc, unc_off)
        pred = px.flow_guidance(state, pos, neg, coords, cu, 2, t, 1e-5, g, 0.7)
        px.flow_euler_update(state, pred, float(np.float32(t) - np.float32(tn)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(got), host(state))


def test_device_sampler_matches_oracle(px, orc):
    """pxs_flow_euler_sample against orc_flow_euler_sample whose velocity is
    orc_slat_flow_forward (fp32 end to end), 3 guided steps with rescale."""
    case, cfg, weights, keep, uncond = flow_setup(px, torch.float32)
    coords = ti32(case["coords"])
    cu = px.batch_cu_seqlens(coords, 2)
    noise = np.random.default_rng(4).standard_normal((case["n"], 8)).astype(np.float32)
    steps, cfg_f = 3, [1e-5, 3.0, 5.0, 0.7, 0.0, 1.0]
    scfg = pxs.SamplerConfig(steps, *cfg_f)
    got = host(px.flow_euler_sample(cfg, weights, scfg, coords, 2, cu, t32(noise),
                                    t32(case["ctx"]), ti64(case["ctx_off"]), t32(uncond),
                                    ti64(np.array([0, 3, 6], np.int64))))
    unc_off = np.array([0, 3, 6], np.int64)

    def model(state, t_model, conditional):
        ctx, off = (case["ctx"], case["ctx_off"]) if conditional else (uncond, unc_off)
        return orc.slat_flow_forward(case["coords"], 2, state, np.full(2, t_model, np.float32),
                                     ctx, off, case["dims"], [1e-6, 1.0, 10000.0], case["fw"],
                                     case["blocks"])

    ref, _, _ = orc.flow_euler_sample(case["coords"], 2, noise, steps, cfg_f, model)
    e = max_rel(got, ref)
    print(f"[device sampler vs oracle] max rel {e:.2e}", flush=True)
    assert e <= FP32_TOL, f"device sampler: max rel error {e:.3e}"


@pytest.mark.parametrize("guidance,rescale", [(1.0, 0.0), (5.0, 0.0), (5.0, 0.7)])
def test_device_sampler_rejects_nonfinite_velocity(px, guidance, rescale):
    """A NaN output bias makes every velocity non-finite: the device sampler
    reports the reference's check (check_model_output -> valid(),
    src/flow_sampler.cpp:126-136) as PXS_ERR_DATA with its message, on the
    single-branch and the batched CFG paths; the same call with a finite bias
    succeeds."""
    case, cfg, weights, keep, uncond = flow_setup(px, torch.float32)
    coords = ti32(case["coords"])
    cu = px.batch_cu_seqlens(coords, 2)
    noise = t32(np.random.default_rng(5).standard_normal((case["n"], 8)).astype(np.float32))
    scfg = pxs.SamplerConfig(2, 1e-5, 3.0, guidance, rescale, 0.0, 1.0)
    args = (cfg, weights, scfg, coords, 2, cu, noise, t32(case["ctx"]), ti64(case["ctx_off"]),
            t32(uncond), ti64(np.array([0, 3, 6], np.int64)))
    print(f"[device sampler nan] guidance={guidance} rescale={rescale}", flush=True)
    assert np.isfinite(host(px.flow_euler_sample(*args))).all()
    out_bias = keep[0][9]
    out_bias[3] = float("nan")
    with pytest.raises(pxs.PxsError, match="sparse features contain a non-finite value"):
        px.flow_euler_sample(*args)
    out_bias[3] = 0.0
    assert np.isfinite(host(px.flow_euler_sample(*args))).all()


def trace_fields(line):
    head, _, rest = line.partition("pixal3d: flow trace ")
    return dict(kv.split("=", 1) for kv in rest.split())


@pytest.mark.parametrize("case", ["guided_rescale", "unguided", "blend_overflow"])
def test_dropin_sampler_trace_matches_reference(case, monkeypatch):
    """PIXAL3D_FLOW_NONFINITE_TRACE: the drop-in's stderr lines (figures from
    one device reduction per traced tensor) against the lines the compiled
    reference printed for the same run (tests/golden/flow_trace_lines.json):
    the same tensors in the same order with the same step, timestep, branch,
    counts, min, max, max_abs and first bad value, the mean within 1e-5
    (a double tree sum against a serial long-double sum), and the same error."""
    import json
    from pathlib import Path

    from fixtures import TRACE_CASES, capture_stderr, overflow_velocity

    gold = json.loads((Path(__file__).resolve().parent / "golden" / "flow_trace_lines.json")
                      .read_text())[case]
    steps, cfg, record = TRACE_CASES[case]
    coords, noise, fn = sampler_inputs()
    velocity = overflow_velocity if case == "blend_overflow" else fn
    d = O.DropIn()
    monkeypatch.setenv("PIXAL3D_FLOW_NONFINITE_TRACE", "1")
    print(f"[drop-in trace] case={case}", flush=True)

    def run():
        try:
            d.flow_euler_sample(d.sparse(coords, noise, 2, (12, 12, 12)), steps, cfg, velocity,
                                record=record)
            return None
        except O.ReferenceError as e:
            return str(e)

    error, text = capture_stderr(run)
    lines = [ln for ln in text.splitlines() if ln.startswith("pixal3d: flow trace")]
    assert error == gold["error"]
    assert len(lines) == len(gold["lines"])
    for got, want in zip(lines, gold["lines"]):
        g, w = trace_fields(got), trace_fields(want)
        assert g.keys() == w.keys(), (got, want)
        for key in g:
            if key == "mean":
                gm, wm = float(g[key]), float(w[key])
                assert abs(gm - wm) <= 1e-5 * max(abs(wm), 1e-3), (got, want)
            else:
                assert g[key] == w[key], (key, got, want)
