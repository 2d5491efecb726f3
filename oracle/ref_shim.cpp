// Test infrastructure only: a C-ABI shim over the pixal3d sparse API, so a
// C++ implementation of include/pixal3d/sparse.h and sparse_transformer.h can
// be driven from Python tests.  oracle/Makefile builds it twice:
//   * against the reference's own CPU primitives (compiled from their sources
//     under /root/reference into oracle/_ref/), the compiled reference that
//     pins the oracle and is timed as the reference CPU baseline;
//   * with PXS_DROPIN_SHIM against this repository's drop-in headers and
//     libpxs.so (into oracle/build/), so the same calls exercise the MI355X
//     drop-in.  The reference-only entry points (CPU threads, timestep
//     embedding) are left out of that build.
//
// Nothing in the shipped library links this file.  Each entry point forwards
// to the API function named in its comment; tensors cross the boundary as
// opaque handles so a timed call pays no marshalling cost.

#ifndef PXS_DROPIN_SHIM
#include "pixal3d/flow.h"
#include "pixal3d/cpu_threads.h"
#endif
#include "pixal3d/flow_sampler.h"
#ifdef PXS_DROPIN_SHIM
#include "pixal3d/pack.h"
#endif
#include "pixal3d/sparse.h"
#include "pixal3d/sparse_transformer.h"

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

using pixal3d::SparseTensorF32;
using pixal3d::VarLenTensorF32;

namespace {

int finish(bool ok, const std::string & message, char * err, int errlen) {
    if (!ok && err && errlen > 0) {
        std::strncpy(err, message.c_str(), static_cast<std::size_t>(errlen - 1));
        err[errlen - 1] = '\0';
    }
    return ok ? 1 : 0;
}

SparseTensorF32 * as_sparse(void * handle) { return static_cast<SparseTensorF32 *>(handle); }
VarLenTensorF32 * as_varlen(void * handle) { return static_cast<VarLenTensorF32 *>(handle); }

} // namespace

extern "C" {

// ---- tensor handles -------------------------------------------------------

void * ref_sparse_new(const int32_t * coords, int64_t points, int batch_size,
                      int sx, int sy, int sz, const float * feats, int channels) {
    auto * t = new SparseTensorF32();
    t->batch_size = batch_size;
    t->channels = channels;
    t->spatial_x = sx;
    t->spatial_y = sy;
    t->spatial_z = sz;
    t->coords.assign(coords, coords + points * 4);
    if (feats) t->feats.assign(feats, feats + points * static_cast<int64_t>(channels));
    return t;
}

void * ref_sparse_empty() { return new SparseTensorF32(); }
void ref_sparse_free(void * handle) { delete as_sparse(handle); }

// shape = {points, channels, batch_size, sx, sy, sz}
void ref_sparse_shape(void * handle, int64_t * shape) {
    const SparseTensorF32 * t = as_sparse(handle);
    shape[0] = static_cast<int64_t>(t->points());
    shape[1] = t->channels;
    shape[2] = t->batch_size;
    shape[3] = t->spatial_x;
    shape[4] = t->spatial_y;
    shape[5] = t->spatial_z;
}

void ref_sparse_read(void * handle, int32_t * coords, float * feats) {
    const SparseTensorF32 * t = as_sparse(handle);
    if (coords) std::memcpy(coords, t->coords.data(), t->coords.size() * sizeof(int32_t));
    if (feats) std::memcpy(feats, t->feats.data(), t->feats.size() * sizeof(float));
}

void * ref_varlen_new(int batch_size, int channels, const int64_t * offsets,
                      const float * feats) {
    auto * t = new VarLenTensorF32();
    t->batch_size = batch_size;
    t->channels = channels;
    t->offsets.resize(static_cast<std::size_t>(batch_size) + 1);
    for (int i = 0; i <= batch_size; ++i) t->offsets[i] = static_cast<std::size_t>(offsets[i]);
    const std::size_t count = t->offsets.back() * static_cast<std::size_t>(channels);
    if (feats) t->feats.assign(feats, feats + count);
    return t;
}

void * ref_varlen_empty() { return new VarLenTensorF32(); }
void ref_varlen_free(void * handle) { delete as_varlen(handle); }

void ref_varlen_shape(void * handle, int64_t * shape) {
    const VarLenTensorF32 * t = as_varlen(handle);
    shape[0] = static_cast<int64_t>(t->tokens());
    shape[1] = t->channels;
    shape[2] = t->batch_size;
}

void ref_varlen_read(void * handle, float * feats) {
    const VarLenTensorF32 * t = as_varlen(handle);
    std::memcpy(feats, t->feats.data(), t->feats.size() * sizeof(float));
}

#ifndef PXS_DROPIN_SHIM
// ---- threads (src/cpu_threads.cpp) ---------------------------------------

int ref_cpu_thread_count() { return pixal3d::cpu_thread_count(); }
void ref_set_cpu_threads(int threads) {
    if (threads > 0) pixal3d::set_cpu_thread_override(threads);
    else pixal3d::clear_cpu_thread_override();
}
#endif

// ---- primitives (src/sparse.cpp) -----------------------------------------

int ref_sparse_valid(void * in, char * err, int errlen) {
    std::string e;
    return finish(as_sparse(in)->valid(&e), e, err, errlen);
}

int ref_varlen_valid(void * in, char * err, int errlen) {
    std::string e;
    return finish(as_varlen(in)->valid(&e), e, err, errlen);
}

int ref_sparse_linear(void * in, const float * w, const float * b, int cout, void * out,
                      char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_linear(*as_sparse(in), w, b, cout, *as_sparse(out), &e),
                  e, err, errlen);
}

int ref_varlen_linear(void * in, const float * w, const float * b, int cout, void * out,
                      char * err, int errlen) {
    std::string e;
    return finish(pixal3d::varlen_linear(*as_varlen(in), w, b, cout, *as_varlen(out), &e),
                  e, err, errlen);
}

int ref_sparse_layer_norm(void * in, float eps, const float * gamma, const float * beta,
                          void * out, char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_layer_norm(*as_sparse(in), eps, gamma, beta,
                                             *as_sparse(out), &e), e, err, errlen);
}

int ref_sparse_downsample_mean(void * in, int factor, void * out, char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_downsample_mean(*as_sparse(in), factor, *as_sparse(out), &e),
                  e, err, errlen);
}

int ref_sparse_channel_to_spatial(void * in, int factor, void * subdivision, void * out,
                                  char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_channel_to_spatial(
                      *as_sparse(in), factor,
                      subdivision ? as_sparse(subdivision) : nullptr, *as_sparse(out), &e),
                  e, err, errlen);
}

int ref_sparse_sdpa(void * q, void * k, void * v, int heads, int head_dim, float scale,
                    void * out, char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_scaled_dot_product_attention(
                      *as_sparse(q), *as_sparse(k), *as_sparse(v), heads, head_dim, scale,
                      *as_sparse(out), &e), e, err, errlen);
}

int ref_sparse_cross_attention(void * q, void * k, void * v, int heads, int head_dim,
                               float scale, void * out, char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_cross_attention(
                      *as_sparse(q), *as_varlen(k), *as_varlen(v), heads, head_dim, scale,
                      *as_sparse(out), &e), e, err, errlen);
}

int ref_sparse_rope(void * in, int heads, int head_dim, float fmin, float fbase, void * out,
                    char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_rotary_position_embedding(
                      *as_sparse(in), heads, head_dim, fmin, fbase, *as_sparse(out), &e),
                  e, err, errlen);
}

int ref_sparse_mh_rms_norm(void * in, int heads, int head_dim, const float * gamma,
                           void * out, char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_multihead_rms_norm(*as_sparse(in), heads, head_dim, gamma,
                                                     *as_sparse(out), &e), e, err, errlen);
}

int ref_varlen_mh_rms_norm(void * in, int heads, int head_dim, const float * gamma,
                           void * out, char * err, int errlen) {
    std::string e;
    return finish(pixal3d::varlen_multihead_rms_norm(*as_varlen(in), heads, head_dim, gamma,
                                                     *as_varlen(out), &e), e, err, errlen);
}

int ref_sparse_submanifold_conv3d(void * in, const float * w, const float * b, int cout,
                                  void * out, char * err, int errlen) {
    std::string e;
    return finish(pixal3d::sparse_submanifold_conv3d(*as_sparse(in), w, b, cout,
                                                     *as_sparse(out), &e), e, err, errlen);
}

// ---- transformer block (src/sparse_transformer.cpp) ----------------------
// cfg_i = {channels, heads, mlp_hidden, context_channels, proj_in_channels,
//          use_rope, qk_rms_norm, qk_rms_norm_cross, use_projection}
// cfg_f = {norm_eps, rope_freq_min, rope_freq_base}
// weights = the 23 pointers of SparseTransformerBlockWeightsF32 in
//           declaration order.
int ref_transformer_block(void * in, const float * timestep_mod, void * context,
                          void * projected, const int * cfg_i, const float * cfg_f,
                          const float * const * weights, void * out, char * err, int errlen) {
    pixal3d::SparseTransformerBlockConfig c;
    c.channels = cfg_i[0];
    c.num_heads = cfg_i[1];
    c.mlp_hidden = cfg_i[2];
    c.context_channels = cfg_i[3];
    c.proj_in_channels = cfg_i[4];
    c.use_rope = cfg_i[5] != 0;
    c.qk_rms_norm = cfg_i[6] != 0;
    c.qk_rms_norm_cross = cfg_i[7] != 0;
    c.use_projection = cfg_i[8] != 0;
    c.norm_eps = cfg_f[0];
    c.rope_freq_min = cfg_f[1];
    c.rope_freq_base = cfg_f[2];
    pixal3d::SparseTransformerBlockWeightsF32 w;
    const float * const * p = weights;
    w.modulation = *p++;
    w.self_to_qkv_weight = *p++;
    w.self_to_qkv_bias = *p++;
    w.self_q_gamma = *p++;
    w.self_k_gamma = *p++;
    w.self_to_out_weight = *p++;
    w.self_to_out_bias = *p++;
    w.norm2_weight = *p++;
    w.norm2_bias = *p++;
    w.cross_to_q_weight = *p++;
    w.cross_to_q_bias = *p++;
    w.cross_to_kv_weight = *p++;
    w.cross_to_kv_bias = *p++;
    w.cross_q_gamma = *p++;
    w.cross_k_gamma = *p++;
    w.cross_to_out_weight = *p++;
    w.cross_to_out_bias = *p++;
    w.proj_weight = *p++;
    w.proj_bias = *p++;
    w.mlp0_weight = *p++;
    w.mlp0_bias = *p++;
    w.mlp2_weight = *p++;
    w.mlp2_bias = *p++;
    std::string e;
    return finish(pixal3d::sparse_transformer_cross_block_f32(
                      *as_sparse(in), timestep_mod, *as_varlen(context),
                      projected ? as_sparse(projected) : nullptr, c, w, *as_sparse(out), &e),
                  e, err, errlen);
}

// ---- flow Euler sampler (src/flow_sampler.cpp) ---------------------------
// model(state feats, rows, channels, 1000 t, conditional, velocity feats, user)
// returns nonzero on success; the velocity keeps the state's shape.
// cfg_i = {steps, record_trajectory}; cfg_f = {sigma_min, rescale_t,
// guidance_strength, guidance_rescale, interval_min, interval_max}.
// traj_xt / traj_x0 (nullable) receive steps x feats each.
typedef int (*ref_velocity_fn)(const float *, int64_t, int, float, int, float *, void *);

int ref_flow_euler_sample(void * noise, const int * cfg_i, const float * cfg_f,
                          ref_velocity_fn fn, void * user, void * out, float * traj_xt,
                          float * traj_x0, char * err, int errlen) {
    pixal3d::FlowEulerSamplerConfig c;
    c.steps = cfg_i[0];
    c.record_trajectory = cfg_i[1] != 0;
    c.sigma_min = cfg_f[0];
    c.rescale_t = cfg_f[1];
    c.guidance_strength = cfg_f[2];
    c.guidance_rescale = cfg_f[3];
    c.guidance_interval_min = cfg_f[4];
    c.guidance_interval_max = cfg_f[5];
    pixal3d::FlowVelocityFn model;
    if (fn) {
        model = [fn, user](const SparseTensorF32 & state, float t, bool cond,
                           SparseTensorF32 & velocity, std::string * error) {
            velocity = state;
            if (!fn(state.feats.data(), static_cast<int64_t>(state.points()), state.channels, t,
                    cond ? 1 : 0, velocity.feats.data(), user)) {
                if (error) *error = "velocity callback failed";
                return false;
            }
            return true;
        };
    }
    pixal3d::FlowEulerSampleF32 result;
    std::string e;
    const bool ok = pixal3d::flow_euler_sample_f32(*as_sparse(noise), c, model, result, &e);
    if (ok) {
        *as_sparse(out) = result.samples;
        const size_t count = result.samples.feats.size();
        for (size_t i = 0; traj_xt && i < result.pred_x_t.size(); ++i)
            std::memcpy(traj_xt + i * count, result.pred_x_t[i].feats.data(), count * sizeof(float));
        for (size_t i = 0; traj_x0 && i < result.pred_x_0.size(); ++i)
            std::memcpy(traj_x0 + i * count, result.pred_x_0[i].feats.data(), count * sizeof(float));
    }
    return finish(ok, e, err, errlen);
}

#ifndef PXS_DROPIN_SHIM
// ---- timestep embedding (src/flow.cpp) -----------------------------------

int ref_timestep_embedding(const float * t, int64_t batch, int dim, int max_period,
                           float * out, char * err, int errlen) {
    std::vector<float> v;
    std::string e;
    const bool ok = pixal3d::timestep_embedding(t, static_cast<std::size_t>(batch), dim,
                                                max_period, v, &e);
    if (ok) std::memcpy(out, v.data(), v.size() * sizeof(float));
    return finish(ok, e, err, errlen);
}

int ref_timestep_embed_mlp(const float * t, int64_t batch, int hidden, int freq,
                           const float * w0, const float * b0, const float * w2,
                           const float * b2, float * out, char * err, int errlen) {
    std::vector<float> v;
    std::string e;
    const bool ok = pixal3d::timestep_embed_mlp(t, static_cast<std::size_t>(batch), hidden,
                                                freq, w0, b0, w2, b2, v, &e);
    if (ok) std::memcpy(out, v.data(), v.size() * sizeof(float));
    return finish(ok, e, err, errlen);
}

#endif

#ifdef PXS_DROPIN_SHIM
// ---- pack reader (include/pixal3d/pack.h) -------------------------------------

// Drives pixal3d::load_pack_info and Pixal3DPackReader the way the
// reference's tests/test_pack_reader.cpp:53-69 drives them: open, inspect,
// read one tensor into out, read a missing tensor, read a u32 key, close,
// read after close.  Each result is one "key=value" line of report.
int dropin_pack_reader_case(const char * path, const char * tensor, const char * u32_key,
                            unsigned char * out, size_t cap, char * report, int reportlen) {
    std::string r, e;
    pixal3d::Pixal3DPackInfo info;
    const bool listed = pixal3d::load_pack_info(path, info, &e);
    r += "load_pack_info=" + std::to_string(listed) + ":" + (listed ? "" : e) + "\n";
    pixal3d::Pixal3DPackReader reader;
    e.clear();
    const bool opened = reader.open(path, &e);
    r += "open=" + std::to_string(opened) + ":" + (opened ? "" : e) + "\n";
    r += "is_open=" + std::to_string(reader.is_open()) + "\n";
    if (opened) {
        const pixal3d::Pixal3DPackInfo & in = reader.info();
        r += "tensors=" + std::to_string(in.tensors.size()) + "\n";
        r += "tensor_bytes=" + std::to_string(in.tensor_bytes()) + "\n";
        r += "has_tensor=" + std::to_string(in.has_tensor(tensor)) + "\n";
        for (const auto & t : in.tensors) {
            if (t.name == tensor) r += "offset=" + std::to_string(t.offset) + "\n";
        }
        std::vector<std::uint8_t> raw;
        e.clear();
        const bool read = reader.read_tensor(tensor, raw, &e);
        r += "read=" + std::to_string(read) + ":" + (read ? "" : e) + "\n";
        r += "bytes=" + std::to_string(raw.size()) + "\n";
        if (read && raw.size() <= cap) std::memcpy(out, raw.data(), raw.size());
        e.clear();
        const bool missing = reader.read_tensor("missing", raw, &e);
        r += "missing=" + std::to_string(missing) + ":" + e + "\n";
        std::uint32_t v = 0;
        e.clear();
        const bool meta = reader.metadata_u32(u32_key, v, true, &e);
        r += "meta=" + std::to_string(meta) + ":" + (meta ? std::to_string(v) : e) + "\n";
        reader.close();
        r += "closed_is_open=" + std::to_string(reader.is_open()) + "\n";
        e.clear();
        const bool after = reader.read_tensor(tensor, raw, &e);
        r += "closed_read=" + std::to_string(after) + ":" + e + "\n";
        e.clear();
        const bool meta_after = reader.metadata_u32(u32_key, v, true, &e);
        r += "closed_meta=" + std::to_string(meta_after) + ":" + e + "\n";
    }
    std::strncpy(report, r.c_str(), static_cast<std::size_t>(reportlen - 1));
    report[reportlen - 1] = '\0';
    return opened ? 1 : 0;
}
#endif

} // extern "C"
