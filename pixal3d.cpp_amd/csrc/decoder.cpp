// Device-resident composition of the SLat-decoder blocks out of the pxs
// kernels (src/slat_decoder.cpp:185-288).  The block input and output are fp32
// (the decoder's hidden stream); convolution and MLP operands are in the
// call's dtype with fp32 accumulation.
//
// ConvNeXt:  SubMConv3d -> LN(affine) -> Linear -> SiLU -> Linear -> + input.
// C2S:       [to_subdiv Linear] ; LN(affine) -> SiLU -> SubMConv3d(C -> 8 out)
//            -> channel_to_spatial ; LN -> SiLU -> SubMConv3d(out -> out)
//            -> + repeat_channels(channel_to_spatial(input)).

#include "carve.h"
#include "pxs_common.h"

#include <cmath>

namespace pxs {
namespace {

struct MapBuffers {
    void * table;
    int32_t * nbr;
    uint32_t * masks;
};

MapBuffers carve_map(Carver & c, int64_t rows) {
    const size_t r = static_cast<size_t>(std::max<int64_t>(rows, 1));
    MapBuffers m;
    m.table = c.take(pxs_voxel_hash_bytes(rows));
    m.nbr = static_cast<int32_t *>(c.take(27 * r * 4));
    m.masks = static_cast<uint32_t *>(c.take(r * 4));
    return m;
}

int build_map(const int32_t * coords, int64_t rows, const MapBuffers & m, void * stream) {
    PXS_TRY(pxs_voxel_hash_build(coords, rows, m.table, stream));
    return pxs_neighbor_map_k3(coords, rows, m.table, m.nbr, m.masks, stream);
}

struct ConvNextBuffers {
    void * xd;    // [rows, C] dtype copy of the input (bf16 only)
    void * conv;  // [rows, C]
    void * norm;  // [rows, C]
    void * hid;   // [rows, mlp_hidden]
    MapBuffers map;
};

ConvNextBuffers carve_convnext(Carver & c, int dtype, int64_t rows, int channels, int mlp_hidden,
                               bool have_map) {
    const size_t e = dtype_bytes(dtype);
    const size_t r = static_cast<size_t>(std::max<int64_t>(rows, 1));
    const size_t C = static_cast<size_t>(channels);
    ConvNextBuffers b{};
    b.xd = dtype == PXS_BF16 ? c.take(r * C * e) : nullptr;
    b.conv = c.take(r * C * e);
    b.norm = c.take(r * C * e);
    b.hid = c.take(r * static_cast<size_t>(mlp_hidden) * e);
    if (!have_map) b.map = carve_map(c, rows);
    return b;
}

struct C2SBuffers {
    float * pred;     // [rows, 8] subdivision logits when not returned to the caller
    void * norm;      // [rows, C]
    void * packed;    // [rows, 8 * out]
    void * hidden;    // [8 rows, out]
    void * hnorm;     // [8 rows, out]
    void * conv2;     // [8 rows, out] (bf16 only; fp32 writes y directly)
    float * skip;     // [8 rows, C / 8]
    int64_t * m_dev;  // child count
    void * c2s_ws;
    MapBuffers map1;
    MapBuffers map2;
};

C2SBuffers carve_c2s(Carver & c, int dtype, int64_t rows, int channels, int out_channels) {
    const size_t e = dtype_bytes(dtype);
    const size_t r = static_cast<size_t>(std::max<int64_t>(rows, 1));
    const size_t C = static_cast<size_t>(channels), O = static_cast<size_t>(out_channels);
    C2SBuffers b{};
    b.pred = static_cast<float *>(c.take(r * 8 * 4));
    b.norm = c.take(r * C * e);
    b.packed = c.take(r * 8 * O * e);
    b.hidden = c.take(8 * r * O * e);
    b.hnorm = c.take(8 * r * O * e);
    b.conv2 = dtype == PXS_BF16 ? c.take(8 * r * O * e) : nullptr;
    b.skip = static_cast<float *>(c.take(8 * r * (C / 8) * 4));
    b.m_dev = static_cast<int64_t *>(c.take(sizeof(int64_t)));
    b.c2s_ws = c.take(pxs_channel_to_spatial_workspace_bytes(rows, 2));
    b.map1 = carve_map(c, rows);
    b.map2 = carve_map(c, 8 * std::max<int64_t>(rows, 1));
    return b;
}

} // namespace
} // namespace pxs

using namespace pxs;

extern "C" {

size_t pxs_convnext_block_workspace_bytes(int dtype, int64_t rows, int channels, int mlp_hidden,
                                          int have_map) {
    if (rows < 0 || channels <= 0 || mlp_hidden <= 0) return 0;
    Carver c(nullptr);
    carve_convnext(c, dtype, rows, channels, mlp_hidden, have_map != 0);
    return c.used();
}

int pxs_convnext_block(int dtype, const int32_t * coords, int64_t rows, const float * x,
                       int channels, int mlp_hidden, float eps,
                       const pxs_decoder_block_weights * w, const int32_t * nbr,
                       const uint32_t * masks, float * y, void * workspace, void * stream) {
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG, "pxs_convnext_block: bad dtype");
    PXS_CHECK(eps > 0.0f && std::isfinite(eps), PXS_ERR_ARG,
              "SLat decoder norm epsilon must be finite and positive");
    PXS_CHECK(rows >= 0 && channels > 0 && mlp_hidden > 0, PXS_ERR_ARG,
              "invalid SLat ConvNeXt block dimensions");
    PXS_CHECK(w, PXS_ERR_ARG, "pxs_convnext_block: null weights");
    PXS_CHECK(w->norm_weight, PXS_ERR_ARG, "missing SLat decoder tensor: block.norm.weight");
    PXS_CHECK(w->norm_bias, PXS_ERR_ARG, "missing SLat decoder tensor: block.norm.bias");
    PXS_CHECK(w->conv1_weight, PXS_ERR_ARG, "missing SLat decoder tensor: block.conv.weight");
    PXS_CHECK(w->conv1_bias, PXS_ERR_ARG, "missing SLat decoder tensor: block.conv.bias");
    PXS_CHECK(w->mlp0_weight, PXS_ERR_ARG, "missing SLat decoder tensor: block.mlp.0.weight");
    PXS_CHECK(w->mlp0_bias, PXS_ERR_ARG, "missing SLat decoder tensor: block.mlp.0.bias");
    PXS_CHECK(w->mlp2_weight, PXS_ERR_ARG, "missing SLat decoder tensor: block.mlp.2.weight");
    PXS_CHECK(w->mlp2_bias, PXS_ERR_ARG, "missing SLat decoder tensor: block.mlp.2.bias");
    PXS_CHECK((nbr == nullptr) == (masks == nullptr), PXS_ERR_ARG,
              "pxs_convnext_block: pass both nbr and masks, or neither");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(coords && x && y && workspace, PXS_ERR_ARG, "pxs_convnext_block: null pointer");
    Carver c(workspace);
    const bool have_map = nbr != nullptr;
    const ConvNextBuffers b = carve_convnext(c, dtype, rows, channels, mlp_hidden, have_map);
    hipStream_t s = as_stream(stream);
    if (!have_map) {
        PXS_TRY(build_map(coords, rows, b.map, stream));
        nbr = b.map.nbr;
        masks = b.map.masks;
    }
    const void * xin = x;
    if (dtype == PXS_BF16) {
        PXS_TRY(pxs_convert(PXS_F32, x, rows * channels, PXS_BF16, b.xd, stream));
        xin = b.xd;
    }
    PXS_TRY(pxs_subm_conv3d(dtype, xin, rows, channels, w->conv1_weight, w->conv1_bias, channels,
                            nbr, masks, b.conv, stream));
    PXS_TRY(pxs_layer_norm(dtype, b.conv, rows, channels, eps, w->norm_weight, w->norm_bias, dtype,
                           b.norm, stream));
    PXS_TRY(pxs_linear(dtype, b.norm, rows, channels, w->mlp0_weight, w->mlp0_bias, mlp_hidden,
                       PXS_ACT_SILU, b.hid, stream));
    // The residual add is the epilogue of the second MLP linear; the input is
    // read by the convolution above, so y may alias x.
    if (y != x) {
        PXS_TRY(check_hip(hipMemcpyAsync(y, x, static_cast<size_t>(rows) * channels * 4,
                                         hipMemcpyDeviceToDevice, s),
                          "pxs_convnext_block: copy"));
    }
    return pxs_linear_residual(dtype, b.hid, rows, mlp_hidden, w->mlp2_weight, w->mlp2_bias,
                               channels, y, stream);
}

size_t pxs_resblock_c2s_workspace_bytes(int dtype, int64_t rows, int channels,
                                        int out_channels) {
    if (rows < 0 || channels <= 0 || out_channels <= 0) return 0;
    Carver c(nullptr);
    carve_c2s(c, dtype, rows, channels, out_channels);
    return c.used();
}

int pxs_resblock_c2s(int dtype, const int32_t * coords, int64_t rows, const float * x,
                     int channels, int out_channels, float eps,
                     const pxs_decoder_block_weights * w, int pred_subdiv,
                     const float * subdivision, float * predicted_subdiv, int32_t * out_coords,
                     float * y, int64_t * rows_out, void * workspace, void * stream) {
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG, "pxs_resblock_c2s: bad dtype");
    PXS_CHECK(eps > 0.0f && std::isfinite(eps), PXS_ERR_ARG,
              "SLat decoder norm epsilon must be finite and positive");
    PXS_CHECK(rows >= 0 && channels > 0 && out_channels > 0 && channels % 8 == 0, PXS_ERR_ARG,
              "invalid SLat channel-to-spatial block dimensions");
    PXS_CHECK(out_channels % (channels / 8) == 0, PXS_ERR_ARG,
              "SLat decoder skip channels are not repeatable");
    PXS_CHECK(8 * rows <= INT32_MAX, PXS_ERR_ARG, "pxs_resblock_c2s: too many rows");
    PXS_CHECK(w && rows_out, PXS_ERR_ARG, "pxs_resblock_c2s: null pointer");
    PXS_CHECK(w->norm1_weight, PXS_ERR_ARG, "missing SLat decoder tensor: up.norm1.weight");
    PXS_CHECK(w->norm1_bias, PXS_ERR_ARG, "missing SLat decoder tensor: up.norm1.bias");
    PXS_CHECK(w->conv1_weight, PXS_ERR_ARG, "missing SLat decoder tensor: up.conv1.weight");
    PXS_CHECK(w->conv1_bias, PXS_ERR_ARG, "missing SLat decoder tensor: up.conv1.bias");
    PXS_CHECK(w->conv2_weight, PXS_ERR_ARG, "missing SLat decoder tensor: up.conv2.weight");
    PXS_CHECK(w->conv2_bias, PXS_ERR_ARG, "missing SLat decoder tensor: up.conv2.bias");
    PXS_CHECK(!pred_subdiv || w->to_subdiv_weight, PXS_ERR_ARG,
              "missing SLat decoder tensor: up.to_subdiv.weight");
    PXS_CHECK(!pred_subdiv || w->to_subdiv_bias, PXS_ERR_ARG,
              "missing SLat decoder tensor: up.to_subdiv.bias");
    *rows_out = 0;
    if (rows == 0) return PXS_OK;
    PXS_CHECK(coords && x && out_coords && y && workspace, PXS_ERR_ARG,
              "pxs_resblock_c2s: null pointer");
    Carver c(workspace);
    const C2SBuffers b = carve_c2s(c, dtype, rows, channels, out_channels);
    hipStream_t s = as_stream(stream);
    const int packed_ch = 8 * out_channels;

    const float * selected = subdivision;
    if (pred_subdiv) {
        float * pred = predicted_subdiv ? predicted_subdiv : b.pred;
        PXS_TRY(pxs_linear(PXS_F32, x, rows, channels, w->to_subdiv_weight, w->to_subdiv_bias, 8,
                           PXS_ACT_NONE, pred, stream));
        selected = pred;
    }
    PXS_TRY(pxs_layer_norm(PXS_F32, x, rows, channels, eps, w->norm1_weight, w->norm1_bias, dtype,
                           b.norm, stream));
    PXS_TRY(pxs_activation(dtype, b.norm, rows * channels, PXS_ACT_SILU, stream));
    PXS_TRY(build_map(coords, rows, b.map1, stream));
    PXS_TRY(pxs_subm_conv3d(dtype, b.norm, rows, channels, w->conv1_weight, w->conv1_bias,
                            packed_ch, b.map1.nbr, b.map1.masks, b.packed, stream));
    PXS_TRY(pxs_channel_to_spatial(dtype, coords, rows, b.packed, packed_ch, 2, selected,
                                   out_coords, b.hidden, b.m_dev, b.c2s_ws, stream));
    // The skip path subdivides the fp32 input with the same selection; its
    // coordinates are identical, so they land in out_coords again.
    PXS_TRY(pxs_channel_to_spatial(PXS_F32, coords, rows, x, channels, 2, selected, out_coords,
                                   b.skip, b.m_dev, b.c2s_ws, stream));
    int64_t m = 8 * rows;
    if (selected) {
        PXS_TRY(check_hip(hipMemcpyAsync(&m, b.m_dev, sizeof(m), hipMemcpyDeviceToHost, s),
                          "pxs_resblock_c2s: read child count"));
        PXS_TRY(check_hip(hipStreamSynchronize(s), "pxs_resblock_c2s: read child count"));
    }
    *rows_out = m;
    if (m == 0) return PXS_OK;
    PXS_TRY(pxs_layer_norm(dtype, b.hidden, m, out_channels, eps, nullptr, nullptr, dtype, b.hnorm,
                           stream));
    PXS_TRY(pxs_activation(dtype, b.hnorm, m * out_channels, PXS_ACT_SILU, stream));
    PXS_TRY(build_map(out_coords, m, b.map2, stream));
    void * conv_out = dtype == PXS_BF16 ? b.conv2 : static_cast<void *>(y);
    PXS_TRY(pxs_subm_conv3d(dtype, b.hnorm, m, out_channels, w->conv2_weight, w->conv2_bias,
                            out_channels, b.map2.nbr, b.map2.masks, conv_out, stream));
    return pxs_add_repeat(dtype, conv_out, m, out_channels, b.skip, channels / 8, y, stream);
}

} // extern "C"
