// Drop-in declaration of the reference sparse CPU API (namespace pixal3d),
// implemented on the MI355X by libpxs.so (pixal3d.cpp_amd/csrc/dropin.cpp).
//
// The types and signatures are the reference's (include/pixal3d/sparse.h:12-154
// of Pixal3D.cpp) so existing callers recompile unchanged against this header
// and link libpxs.so instead of src/sparse.cpp.  Semantics, including the
// error strings written to *error, follow the reference; each call copies its
// host inputs to HBM, runs the HIP kernels, and copies the result back.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace pixal3d {

// Token rows of several sequences: offsets[batch_size + 1], feats [token, channel].
struct VarLenTensorF32 {
    int batch_size = 0;
    int channels = 0;
    std::vector<std::size_t> offsets;
    std::vector<float> feats;

    std::size_t tokens() const noexcept {
        return channels > 0 ? feats.size() / static_cast<std::size_t>(channels) : 0;
    }
    bool valid(std::string * error = nullptr) const;
};

// Sparse voxels: coords rows (batch, x, y, z), contiguous by batch; feats
// [point, channel].
struct SparseTensorF32 {
    int batch_size = 0;
    int channels = 0;
    int spatial_x = 0;
    int spatial_y = 0;
    int spatial_z = 0;
    std::vector<std::int32_t> coords;
    std::vector<float> feats;

    std::size_t points() const noexcept { return coords.size() / 4; }
    bool valid(std::string * error = nullptr) const;
};

bool sparse_linear(const SparseTensorF32 & input, const float * weight, const float * bias,
                   int out_channels, SparseTensorF32 & output, std::string * error = nullptr);

bool varlen_linear(const VarLenTensorF32 & input, const float * weight, const float * bias,
                   int out_channels, VarLenTensorF32 & output, std::string * error = nullptr);

bool sparse_layer_norm(const SparseTensorF32 & input, float epsilon, const float * gamma,
                       const float * beta, SparseTensorF32 & output,
                       std::string * error = nullptr);

bool sparse_downsample_mean(const SparseTensorF32 & input, int factor, SparseTensorF32 & output,
                            std::string * error = nullptr);

bool sparse_channel_to_spatial(const SparseTensorF32 & input, int factor,
                               const SparseTensorF32 * subdivision, SparseTensorF32 & output,
                               std::string * error = nullptr);

bool sparse_scaled_dot_product_attention(const SparseTensorF32 & query,
                                         const SparseTensorF32 & key,
                                         const SparseTensorF32 & value, int num_heads,
                                         int head_dim, float scale, SparseTensorF32 & output,
                                         std::string * error = nullptr);

bool sparse_cross_attention(const SparseTensorF32 & query, const VarLenTensorF32 & key,
                            const VarLenTensorF32 & value, int num_heads, int head_dim,
                            float scale, SparseTensorF32 & output,
                            std::string * error = nullptr);

bool sparse_rotary_position_embedding(const SparseTensorF32 & input, int num_heads,
                                      int head_dim, float frequency_min, float frequency_base,
                                      SparseTensorF32 & output, std::string * error = nullptr);

bool sparse_multihead_rms_norm(const SparseTensorF32 & input, int num_heads, int head_dim,
                               const float * gamma, SparseTensorF32 & output,
                               std::string * error = nullptr);

bool varlen_multihead_rms_norm(const VarLenTensorF32 & input, int num_heads, int head_dim,
                               const float * gamma, VarLenTensorF32 & output,
                               std::string * error = nullptr);

bool sparse_submanifold_conv3d(const SparseTensorF32 & input, const float * weight,
                               const float * bias, int out_channels, SparseTensorF32 & output,
                               std::string * error = nullptr);

} // namespace pixal3d
