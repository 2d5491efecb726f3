// Flow-matching Euler sampler arithmetic on the device (src/flow_sampler.cpp).
//
// Every kernel here is elementwise over the fp32 state except the per-batch
// standard deviation of the CFG rescale.  The reference rounds each product
// and sum separately (an x86-64 build without FMA); this file switches
// floating-point contraction off (the pragma below), so every product and sum
// here rounds on its own too, and the results match the reference bit for
// bit (fp32 division and square root are correctly rounded).  The
// standard deviation keeps the reference's summation order: one thread per
// batch item walks that item's values in row order, the only order whose
// fp32 rounding reproduces the reference (a tree reduction would differ in
// the last bits, and the CFG rescale divides those bits by small timesteps).

#include "carve.h"
#include "pxs_common.h"

#include <algorithm>
#include <limits>
#include <cmath>

#pragma clang fp contract(off)

namespace pxs {
namespace {

constexpr int kThreads = 256;

// prediction = g * positive + (1 - g) * negative (src/flow_sampler.cpp:192-200).
__global__ void guidance_blend_kernel(const float * __restrict__ positive,
                                      const float * __restrict__ negative, int64_t count, float g,
                                      float * __restrict__ prediction) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const float nw = 1.0f - g;
    prediction[i] = g * positive[i] + nw * negative[i];
}

// x0 = a * state - b * prediction, a = 1 - sigma_min, b = sigma_min + a * t
// (src/flow_sampler.cpp:138-146).
__device__ __forceinline__ float to_xstart(float state, float pred, float a, float b) {
    return a * state - b * pred;
}

__global__ void pred_to_xstart_kernel(const float * __restrict__ state,
                                      const float * __restrict__ prediction, int64_t count,
                                      float a, float b, float * __restrict__ x0) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    x0[i] = to_xstart(state[i], prediction[i], a, b);
}

// Population standard deviation of the x0 of `pred` over every value of each
// batch item (src/flow_sampler.cpp:158-190), for pred = positive (slot 0) and
// pred = the blended prediction (slot 1).  One thread per (item, slot) walks
// the item's rows in order, like the reference loop; 16 values are loaded
// ahead of the serial sums.
__global__ void batch_std_kernel(const float * __restrict__ state,
                                 const float * __restrict__ positive,
                                 const float * __restrict__ prediction,
                                 const int64_t * __restrict__ cu_rows, int channels,
                                 int batch_size, float a, float b, float * __restrict__ stds) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= 2 * batch_size) return;
    const int item = t >> 1;
    const float * pred = (t & 1) ? prediction : positive;
    const int64_t begin = cu_rows[item] * channels, end = cu_rows[item + 1] * channels;
    float sum = 0.0f, sum_sq = 0.0f;
    for (int64_t i = begin; i < end; i += 16) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
            v[j] = i + j < end ? to_xstart(state[i + j], pred[i + j], a, b) : 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (i + j < end) {
                sum += v[j];
                sum_sq += v[j] * v[j];
            }
        }
    }
    const int64_t count = end - begin;
    float sd = 0.0f;
    if (count > 0) {
        const float n = static_cast<float>(count);
        const float mean = sum / n;
        const float mean_sq = sum_sq / n;
        sd = sqrtf(fmaxf(mean_sq - mean * mean, 0.0f));
    }
    stds[t] = sd;
}

// CFG rescale of the blended prediction (src/flow_sampler.cpp:202-235):
// x0_cfg scaled by std(x0_pos) / std(x0_cfg) (1 when that is 0), mixed with
// weight `rescale`, then converted back to a prediction.
__global__ void guidance_rescale_kernel(const float * __restrict__ state,
                                        const int32_t * __restrict__ coords, int64_t rows,
                                        int channels, const float * __restrict__ stds, float a,
                                        float b, float rescale, float * __restrict__ prediction) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * channels) return;
    const int64_t row = i / channels;
    const int item = coords[row * 4];
    const float sd_cfg = stds[2 * item + 1];
    const float ratio = sd_cfg != 0.0f ? stds[2 * item] / sd_cfg : 1.0f;
    const float x0 = to_xstart(state[i], prediction[i], a, b);
    const float rescaled = x0 * ratio;
    const float mixed = rescale * rescaled + (1.0f - rescale) * x0;
    prediction[i] = (a * state[i] - mixed) / b;
}

// state -= delta * prediction (src/flow_sampler.cpp:330-333).
__global__ void euler_update_kernel(float * __restrict__ state, const float * __restrict__ prediction,
                                    int64_t count, float delta) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    state[i] = state[i] - delta * prediction[i];
}

// Batched CFG inputs: rows [0, n) are the conditional items, rows [n, 2n)
// the same rows as items batch .. 2 batch - 1 (batch column shifted).
__global__ void cfg_coords_kernel(const int4 * __restrict__ coords, int64_t n, int batch,
                                  int4 * __restrict__ coords2) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    int4 c = coords[p];
    coords2[p] = c;
    c.x += batch;
    coords2[n + p] = c;
}

// offsets2 = offsets (batch + 1 entries) followed by offsets_b[1..] + shift,
// for the row bounds (shift = rows) and the context bounds (shift = cond
// tokens).
__global__ void cfg_offsets_kernel(const int64_t * __restrict__ a, const int64_t * __restrict__ b,
                                   int batch, int64_t shift, int64_t * __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i > 2 * batch) return;
    out[i] = i <= batch ? a[i] : b[i - batch] + shift;
}

__global__ void fill_f32_kernel(float * __restrict__ p, int count, float value) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) p[i] = value;
}

struct SamplerBuffers {
    int32_t * coords2;
    int64_t * cu2;
    int64_t * ctx_off2;
    float * x2;
    float * t2;
    void * ctx2;
    float * velocity;
    float * prediction;
    float * x0;
    int64_t * status;
    void * guide_ws;
    void * flow_ws;
};

SamplerBuffers carve_sampler(Carver & c, int dtype, const pxs_flow_config & f, int64_t rows,
                             int64_t cond_tokens, int64_t uncond_tokens, int batch) {
    const size_t r2 = static_cast<size_t>(2 * rows);
    const size_t tokens2 = static_cast<size_t>(cond_tokens + uncond_tokens);
    SamplerBuffers b{};
    b.coords2 = static_cast<int32_t *>(c.take(r2 * 4 * sizeof(int32_t)));
    b.cu2 = static_cast<int64_t *>(c.take((2 * batch + 1) * sizeof(int64_t)));
    b.ctx_off2 = static_cast<int64_t *>(c.take((2 * batch + 1) * sizeof(int64_t)));
    b.x2 = static_cast<float *>(c.take(r2 * f.in_channels * sizeof(float)));
    b.t2 = static_cast<float *>(c.take(2 * batch * sizeof(float)));
    b.ctx2 = c.take(std::max<size_t>(tokens2, 1) * f.cond_channels * dtype_bytes(dtype));
    b.velocity = static_cast<float *>(c.take(r2 * f.out_channels * sizeof(float)));
    b.prediction = static_cast<float *>(c.take(static_cast<size_t>(rows) * f.out_channels * sizeof(float)));
    b.x0 = static_cast<float *>(c.take(static_cast<size_t>(rows) * f.out_channels * sizeof(float)));
    b.status = static_cast<int64_t *>(c.take(sizeof(int64_t)));
    b.guide_ws = c.take(pxs_flow_guidance_workspace_bytes(batch));
    b.flow_ws = c.take(pxs_slat_flow_workspace_bytes(dtype, &f, 2 * rows,
                                                     std::max<int64_t>(cond_tokens + uncond_tokens, 1),
                                                     2 * batch));
    return b;
}

} // namespace
} // namespace pxs

using namespace pxs;

extern "C" {

int pxs_flow_sampler_schedule(const pxs_flow_sampler_config * cfg, int step, float * timestep,
                              float * next_timestep, float * guidance) {
    PXS_CHECK(cfg && timestep && next_timestep && guidance, PXS_ERR_ARG,
              "pxs_flow_sampler_schedule: null pointer");
    const pxs_flow_sampler_config & c = *cfg;
    PXS_CHECK(!(c.steps <= 0 || !(c.sigma_min >= 0.0f) || !(c.sigma_min < 1.0f) ||
                !std::isfinite(c.sigma_min) || !(c.rescale_t > 0.0f) || !std::isfinite(c.rescale_t) ||
                !std::isfinite(c.guidance_strength) || !std::isfinite(c.guidance_rescale) ||
                c.guidance_rescale < 0.0f || !std::isfinite(c.guidance_interval_min) ||
                !std::isfinite(c.guidance_interval_max) ||
                c.guidance_interval_min > c.guidance_interval_max),
              PXS_ERR_ARG, "invalid flow Euler sampler configuration");
    PXS_CHECK(step >= 0 && step < c.steps, PXS_ERR_ARG, "pxs_flow_sampler_schedule: bad step");
    // src/flow_sampler.cpp:270-285, in the same float operations.
    const float steps = static_cast<float>(c.steps);
    const float linear = 1.0f - static_cast<float>(step) / steps;
    const float denominator = 1.0f + (c.rescale_t - 1.0f) * linear;
    PXS_CHECK(denominator > 0.0f && std::isfinite(denominator), PXS_ERR_ARG,
              "flow Euler timestep schedule is not finite");
    const float t = c.rescale_t * linear / denominator;
    const float next_linear = 1.0f - static_cast<float>(step + 1) / steps;
    const float next_denominator = 1.0f + (c.rescale_t - 1.0f) * next_linear;
    PXS_CHECK(next_denominator > 0.0f && std::isfinite(next_denominator), PXS_ERR_ARG,
              "flow Euler timestep schedule is not finite");
    *timestep = t;
    *next_timestep = c.rescale_t * next_linear / next_denominator;
    const bool in_interval = t >= c.guidance_interval_min && t <= c.guidance_interval_max;
    *guidance = in_interval ? c.guidance_strength : 1.0f;
    return PXS_OK;
}

size_t pxs_flow_guidance_workspace_bytes(int batch_size) {
    return static_cast<size_t>(2 * std::max(batch_size, 1)) * sizeof(float) + 64;
}

int pxs_flow_guidance(const float * state, const float * positive, const float * negative,
                      const int32_t * coords, const int64_t * cu_rows, int64_t rows, int channels,
                      int batch_size, float timestep, float sigma_min, float guidance,
                      float guidance_rescale, float * prediction, void * workspace, void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_flow_guidance");
    PXS_CHECK(rows >= 0 && channels > 0 && batch_size > 0, PXS_ERR_ARG,
              "pxs_flow_guidance: bad shape");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(state && positive && negative && prediction, PXS_ERR_ARG,
              "pxs_flow_guidance: null pointer");
    PXS_CHECK(guidance_rescale <= 0.0f || (coords && cu_rows && workspace), PXS_ERR_ARG,
              "pxs_flow_guidance: the rescale needs coords, cu_rows and a workspace");
    hipStream_t s = as_stream(stream);
    const int64_t count = rows * channels;
    hipLaunchKernelGGL(guidance_blend_kernel, dim3(grid_for(count, kThreads)), dim3(kThreads), 0,
                       s, positive, negative, count, guidance, prediction);
    if (guidance_rescale > 0.0f) {
        const float a = 1.0f - sigma_min;
        const float b = sigma_min + a * timestep;
        float * stds = static_cast<float *>(workspace);
        hipLaunchKernelGGL(batch_std_kernel, dim3(grid_for(2 * batch_size, 64)), dim3(64), 0, s,
                           state, positive, prediction, cu_rows, channels, batch_size, a, b, stds);
        hipLaunchKernelGGL(guidance_rescale_kernel, dim3(grid_for(count, kThreads)), dim3(kThreads),
                           0, s, state, coords, rows, channels, stds, a, b, guidance_rescale,
                           prediction);
    }
    return check_launch("pxs_flow_guidance");
}

int pxs_flow_pred_to_xstart(const float * state, const float * prediction, int64_t count,
                            float timestep, float sigma_min, float * x0, void * stream) {
    PXS_CHECK(count >= 0, PXS_ERR_ARG, "pxs_flow_pred_to_xstart: bad count");
    if (count == 0) return PXS_OK;
    PXS_CHECK(state && prediction && x0, PXS_ERR_ARG, "pxs_flow_pred_to_xstart: null pointer");
    const float a = 1.0f - sigma_min;
    const float b = sigma_min + a * timestep;
    hipLaunchKernelGGL(pred_to_xstart_kernel, dim3(grid_for(count, kThreads)), dim3(kThreads), 0,
                       as_stream(stream), state, prediction, count, a, b, x0);
    return check_launch("pxs_flow_pred_to_xstart");
}

int pxs_flow_euler_update(float * state, const float * prediction, int64_t count, float delta,
                          void * stream) {
    PXS_CHECK(count >= 0, PXS_ERR_ARG, "pxs_flow_euler_update: bad count");
    if (count == 0) return PXS_OK;
    PXS_CHECK(state && prediction, PXS_ERR_ARG, "pxs_flow_euler_update: null pointer");
    hipLaunchKernelGGL(euler_update_kernel, dim3(grid_for(count, kThreads)), dim3(kThreads), 0,
                       as_stream(stream), state, prediction, count, delta);
    return check_launch("pxs_flow_euler_update");
}

size_t pxs_flow_euler_sample_workspace_bytes(int dtype, const pxs_flow_config * cfg,
                                             int64_t rows, int64_t cond_tokens,
                                             int64_t uncond_tokens, int batch_size) {
    if (!cfg || rows < 0 || batch_size <= 0) return 0;
    Carver c(nullptr);
    carve_sampler(c, dtype, *cfg, rows, cond_tokens, uncond_tokens, batch_size);
    return c.used();
}

int pxs_flow_euler_sample(int dtype, const pxs_flow_config * cfg, const pxs_flow_weights * w,
                          const pxs_flow_sampler_config * scfg, const int32_t * coords,
                          int64_t rows, int batch_size, const int64_t * cu_rows,
                          const float * noise, const void * cond, const int64_t * cond_offsets,
                          int64_t cond_tokens, const void * uncond,
                          const int64_t * uncond_offsets, int64_t uncond_tokens,
                          float * samples, void * workspace, void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_flow_euler_sample");
    PXS_CHECK(cfg && w && scfg, PXS_ERR_ARG, "pxs_flow_euler_sample: null config or weights");
    PXS_CHECK(rows >= 0 && batch_size > 0 && cond_tokens >= 0 && uncond_tokens >= 0, PXS_ERR_ARG,
              "pxs_flow_euler_sample: bad shape");
    PXS_CHECK(cfg->in_channels == cfg->out_channels, PXS_ERR_ARG,
              "pxs_flow_euler_sample: the velocity must have the state's channel count");
    PXS_CHECK(!cfg->use_projection, PXS_ERR_ARG,
              "pxs_flow_euler_sample: models with a projection input are not supported");
    {
        float t0, t1, g;  // the configuration checks of valid_config
        PXS_TRY(pxs_flow_sampler_schedule(scfg, 0, &t0, &t1, &g));
    }
    if (rows == 0) return PXS_OK;
    PXS_CHECK(coords && cu_rows && noise && cond && cond_offsets && uncond && uncond_offsets &&
                  samples && workspace,
              PXS_ERR_ARG, "pxs_flow_euler_sample: null pointer");
    hipStream_t s = as_stream(stream);
    Carver c(workspace);
    const SamplerBuffers b = carve_sampler(c, dtype, *cfg, rows, cond_tokens, uncond_tokens,
                                           batch_size);
    const int C = cfg->in_channels;
    const int64_t count = rows * C;
    const size_t ctx_row = static_cast<size_t>(cfg->cond_channels) * dtype_bytes(dtype);
    if (samples != noise) {
        PXS_TRY(check_hip(hipMemcpyAsync(samples, noise, count * sizeof(float),
                                         hipMemcpyDeviceToDevice, s),
                          "pxs_flow_euler_sample: state copy"));
    }
    // The doubled batch: coordinates, row bounds, context and its bounds.
    hipLaunchKernelGGL(cfg_coords_kernel, dim3(grid_for(rows, kThreads)), dim3(kThreads), 0, s,
                       reinterpret_cast<const int4 *>(coords), rows, batch_size,
                       reinterpret_cast<int4 *>(b.coords2));
    hipLaunchKernelGGL(cfg_offsets_kernel, dim3(grid_for(2 * batch_size + 1, 64)), dim3(64), 0, s,
                       cu_rows, cu_rows, batch_size, rows, b.cu2);
    hipLaunchKernelGGL(cfg_offsets_kernel, dim3(grid_for(2 * batch_size + 1, 64)), dim3(64), 0, s,
                       cond_offsets, uncond_offsets, batch_size, cond_tokens, b.ctx_off2);
    char * ctx2 = static_cast<char *>(b.ctx2);
    if (cond_tokens > 0) {
        PXS_TRY(check_hip(hipMemcpyAsync(ctx2, cond, cond_tokens * ctx_row, hipMemcpyDeviceToDevice, s),
                          "pxs_flow_euler_sample: context copy"));
    }
    if (uncond_tokens > 0) {
        PXS_TRY(check_hip(hipMemcpyAsync(ctx2 + cond_tokens * ctx_row, uncond, uncond_tokens * ctx_row,
                                         hipMemcpyDeviceToDevice, s),
                          "pxs_flow_euler_sample: context copy"));
    }
    PXS_TRY(check_launch("pxs_flow_euler_sample setup"));
    // One status word collects the reference's finiteness checks of every
    // step: the model velocity (check_model_output -> valid(),
    // src/flow_sampler.cpp:126-136) and, under CFG rescale, both x0 inputs of
    // sparse_batch_std (src/flow_sampler.cpp:168).  It is read once, after the
    // last step.
    PXS_TRY(pxs_status_reset(b.status, stream));

    for (int step = 0; step < scfg->steps; ++step) {
        float t = 0.0f, t_next = 0.0f, guidance = 1.0f;
        PXS_TRY(pxs_flow_sampler_schedule(scfg, step, &t, &t_next, &guidance));
        const float model_t = 1000.0f * t;
        const float * pred = nullptr;
        if (guidance == 1.0f || guidance == 0.0f) {
            // One branch only (src/flow_sampler.cpp:292-303).
            const bool conditional = guidance == 1.0f;
            hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(batch_size, 64)), dim3(64), 0, s, b.t2,
                               batch_size, model_t);
            PXS_TRY(pxs_slat_flow_forward(dtype, cfg, w, coords, rows, batch_size, cu_rows, samples,
                                          b.t2, conditional ? cond : uncond,
                                          conditional ? cond_offsets : uncond_offsets,
                                          conditional ? cond_tokens : uncond_tokens, nullptr,
                                          b.velocity, b.flow_ws, stream));
            PXS_TRY(pxs_check_finite(PXS_F32, b.velocity, rows, C, C, b.status, stream));
            pred = b.velocity;
        } else {
            // Both branches in one forward over the doubled batch.
            PXS_TRY(check_hip(hipMemcpyAsync(b.x2, samples, count * sizeof(float),
                                             hipMemcpyDeviceToDevice, s),
                              "pxs_flow_euler_sample: state copy"));
            PXS_TRY(check_hip(hipMemcpyAsync(b.x2 + count, samples, count * sizeof(float),
                                             hipMemcpyDeviceToDevice, s),
                              "pxs_flow_euler_sample: state copy"));
            hipLaunchKernelGGL(fill_f32_kernel, dim3(grid_for(2 * batch_size, 64)), dim3(64), 0, s,
                               b.t2, 2 * batch_size, model_t);
            PXS_TRY(pxs_slat_flow_forward(dtype, cfg, w, b.coords2, 2 * rows, 2 * batch_size, b.cu2,
                                          b.x2, b.t2, b.ctx2, b.ctx_off2,
                                          cond_tokens + uncond_tokens, nullptr, b.velocity,
                                          b.flow_ws, stream));
            PXS_TRY(pxs_check_finite(PXS_F32, b.velocity, 2 * rows, C, C, b.status, stream));
            if (scfg->guidance_rescale > 0.0f) {
                // x0 of the conditional prediction, then of the plain CFG blend.
                PXS_TRY(pxs_flow_pred_to_xstart(samples, b.velocity, count, t, scfg->sigma_min,
                                                b.x0, stream));
                PXS_TRY(pxs_check_finite(PXS_F32, b.x0, rows, C, C, b.status, stream));
                PXS_TRY(pxs_flow_guidance(samples, b.velocity, b.velocity + count, nullptr,
                                          nullptr, rows, C, batch_size, t, scfg->sigma_min,
                                          guidance, 0.0f, b.prediction, nullptr, stream));
                PXS_TRY(pxs_flow_pred_to_xstart(samples, b.prediction, count, t, scfg->sigma_min,
                                                b.x0, stream));
                PXS_TRY(pxs_check_finite(PXS_F32, b.x0, rows, C, C, b.status, stream));
            }
            PXS_TRY(pxs_flow_guidance(samples, b.velocity, b.velocity + count, coords, cu_rows, rows,
                                      C, batch_size, t, scfg->sigma_min, guidance,
                                      scfg->guidance_rescale, b.prediction, b.guide_ws, stream));
            pred = b.prediction;
        }
        PXS_TRY(pxs_flow_euler_update(samples, pred, count, t - t_next, stream));
    }
    PXS_TRY(check_launch("pxs_flow_euler_sample"));
    int64_t status = 0;
    PXS_TRY(check_hip(hipMemcpyAsync(&status, b.status, sizeof(status), hipMemcpyDeviceToHost, s),
                      "pxs_flow_euler_sample: status read"));
    PXS_TRY(check_hip(hipStreamSynchronize(s), "pxs_flow_euler_sample: status read"));
    PXS_CHECK(status == std::numeric_limits<int64_t>::max(), PXS_ERR_DATA,
              "sparse features contain a non-finite value");
    return PXS_OK;
}

} // extern "C"
