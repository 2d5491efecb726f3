// Drop-in declaration of the reference flow-matching Euler sampler
// (include/pixal3d/flow_sampler.h:14-52 of Pixal3D.cpp), implemented on the
// MI355X by libpxs.so (pixal3d.cpp_amd/csrc/dropin.cpp): the guidance blend,
// the CFG rescale and the Euler update run on the device, bit for bit equal
// to the reference's host arithmetic; the model stays a host callback.
//
// For the SLat-flow model itself, pxs_flow_euler_sample (include/pxs.h) runs
// the whole loop on the device with the conditional and unconditional
// forwards batched into one launch sequence per step.
#pragma once

#include "pixal3d/sparse.h"

#include <functional>
#include <string>
#include <vector>

namespace pixal3d {

struct FlowEulerSamplerConfig {
    int steps = 50;
    float sigma_min = 1e-5f;
    float rescale_t = 1.0f;
    float guidance_strength = 1.0f;
    float guidance_rescale = 0.0f;
    float guidance_interval_min = 0.0f;
    float guidance_interval_max = 1.0f;
    bool record_trajectory = false;
};

// model(state, 1000 * t, conditional, velocity, error): the velocity at the
// current state; conditional selects the positive or negative condition.
using FlowVelocityFn = std::function<bool(const SparseTensorF32 & state,
                                           float model_timestep,
                                           bool conditional,
                                           SparseTensorF32 & velocity,
                                           std::string * error)>;

struct FlowEulerSampleF32 {
    SparseTensorF32 samples;
    std::vector<SparseTensorF32> pred_x_t;
    std::vector<SparseTensorF32> pred_x_0;
};

bool flow_euler_sample_f32(
    const SparseTensorF32 & noise,
    const FlowEulerSamplerConfig & config,
    const FlowVelocityFn & model,
    FlowEulerSampleF32 & output,
    std::string * error = nullptr);

} // namespace pixal3d
