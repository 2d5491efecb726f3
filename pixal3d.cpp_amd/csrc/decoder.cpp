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

#include <algorithm>
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
    m.table = c.take(pxs_voxel_bricks_bytes(rows));
    m.nbr = static_cast<int32_t *>(c.take(27 * r * 4));
    m.masks = static_cast<uint32_t *>(c.take(r * 4));
    return m;
}

// The level's map from the brick table: the decoder's levels reach 1024^3,
// where a dense grid would be gigabytes, and the voxel hash puts a row's 27
// neighbours in 27 unrelated lines.
int build_map(const int32_t * coords, int64_t rows, const MapBuffers & m, void * stream) {
    PXS_TRY(pxs_voxel_bricks_build(coords, rows, m.table, stream));
    return pxs_neighbor_map_k3_bricks(coords, rows, m.table, m.nbr, m.masks, stream);
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

// own_in / own_out: carve the block's own neighbour maps of its input and
// output coordinates (a caller that keeps maps per level passes them in).
C2SBuffers carve_c2s(Carver & c, int dtype, int64_t rows, int channels, int out_channels,
                     bool own_in = true, bool own_out = true) {
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
    if (own_in) b.map1 = carve_map(c, rows);
    if (own_out) b.map2 = carve_map(c, 8 * std::max<int64_t>(rows, 1));
    return b;
}

size_t c2s_shared_maps_bytes(int dtype, int64_t rows, int channels, int out_channels) {
    Carver c(nullptr);
    carve_c2s(c, dtype, rows, channels, out_channels, false, false);
    return c.used();
}

struct DecoderBuffers {
    float * hid[2];
    int32_t * crd[2];
    MapBuffers map[2];  // the current level's map and the next one's (built by the C2S block)
    void * block_ws;
};

int64_t grow8(int64_t n, int64_t cap) { return n > cap / 8 ? cap : 8 * n; }

// Buffers sized for each level's capacity min(max_rows, rows * 8^l): two
// hidden-state, two coordinate and two neighbour-map buffers (ping-pong across
// C2S levels), and the largest block workspace.  Blocks past n_blocks are
// not sized (the forward rejects such a configuration).
DecoderBuffers carve_decoder(Carver & c, int dtype, const pxs_decoder_config & cfg,
                             const pxs_decoder_block * blocks, int n_blocks, int64_t rows,
                             int64_t max_rows) {
    size_t hid = 0, ws = 0;
    int64_t cap = rows, cap_max = rows;
    int bi = 0;
    for (int l = 0; l < cfg.levels; ++l) {
        if (l > 0) cap = grow8(cap, max_rows);
        cap_max = std::max(cap_max, cap);
        const int C = cfg.model_channels[l];
        hid = std::max(hid, static_cast<size_t>(cap) * static_cast<size_t>(std::max(C, 1)));
        for (int k = 0; k < cfg.num_blocks[l] && bi < n_blocks; ++k, ++bi)
            ws = std::max(ws, pxs_convnext_block_workspace_bytes(dtype, cap, C, blocks[bi].mlp_hidden, 1));
        if (l + 1 < cfg.levels && bi < n_blocks) {
            ws = std::max(ws, c2s_shared_maps_bytes(dtype, cap, blocks[bi].channels,
                                                   blocks[bi].out_channels));
            ++bi;
        }
    }
    hid = std::max(hid, static_cast<size_t>(std::max<int64_t>(rows, 1)) *
                            static_cast<size_t>(std::max(cfg.latent_channels, 1)));
    DecoderBuffers b{};
    b.hid[0] = static_cast<float *>(c.take(hid * 4));
    b.hid[1] = static_cast<float *>(c.take(hid * 4));
    b.crd[0] = static_cast<int32_t *>(c.take(static_cast<size_t>(cap_max) * 16));
    b.crd[1] = static_cast<int32_t *>(c.take(static_cast<size_t>(cap_max) * 16));
    b.map[0] = carve_map(c, cap_max);
    b.map[1] = carve_map(c, cap_max);
    b.block_ws = c.take(ws);
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
    PXS_CHECK_WORKSPACE(workspace, "pxs_convnext_block");
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

// The C2S block; in_map (the map of coords, already built) and out_map
// (where to build the map of out_coords) come from a caller that keeps one
// map per level, or are null for the block's own in its workspace.
static int resblock_c2s(int dtype, const int32_t * coords, int64_t rows, const float * x,
                        int channels, int out_channels, float eps,
                        const pxs_decoder_block_weights * w, int pred_subdiv,
                        const float * subdivision, float * predicted_subdiv,
                        int32_t * out_coords, float * y, int64_t * rows_out, void * workspace,
                        void * stream, const MapBuffers * in_map, const MapBuffers * out_map) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_resblock_c2s");
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
    const C2SBuffers b = carve_c2s(c, dtype, rows, channels, out_channels, in_map == nullptr,
                                   out_map == nullptr);
    const MapBuffers & map1 = in_map ? *in_map : b.map1;
    const MapBuffers & map2 = out_map ? *out_map : b.map2;
    hipStream_t s = as_stream(stream);
    const int packed_ch = 8 * out_channels;

    const float * selected = subdivision;
    if (pred_subdiv) {
        float * pred = predicted_subdiv ? predicted_subdiv : b.pred;
        // In sparse_linear's own order: a logit's sign picks the children.
        PXS_TRY(pxs_linear_ordered(x, rows, channels, w->to_subdiv_weight, w->to_subdiv_bias, 8,
                                   pred, stream));
        selected = pred;
    }
    PXS_TRY(pxs_layer_norm(PXS_F32, x, rows, channels, eps, w->norm1_weight, w->norm1_bias, dtype,
                           b.norm, stream));
    PXS_TRY(pxs_activation(dtype, b.norm, rows * channels, PXS_ACT_SILU, stream));
    if (!in_map) PXS_TRY(build_map(coords, rows, map1, stream));
    PXS_TRY(pxs_subm_conv3d(dtype, b.norm, rows, channels, w->conv1_weight, w->conv1_bias,
                            packed_ch, map1.nbr, map1.masks, b.packed, stream));
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
    PXS_TRY(build_map(out_coords, m, map2, stream));
    void * conv_out = dtype == PXS_BF16 ? b.conv2 : static_cast<void *>(y);
    PXS_TRY(pxs_subm_conv3d(dtype, b.hnorm, m, out_channels, w->conv2_weight, w->conv2_bias,
                            out_channels, map2.nbr, map2.masks, conv_out, stream));
    return pxs_add_repeat(dtype, conv_out, m, out_channels, b.skip, channels / 8, y, stream);
}

int pxs_resblock_c2s(int dtype, const int32_t * coords, int64_t rows, const float * x,
                     int channels, int out_channels, float eps,
                     const pxs_decoder_block_weights * w, int pred_subdiv,
                     const float * subdivision, float * predicted_subdiv, int32_t * out_coords,
                     float * y, int64_t * rows_out, void * workspace, void * stream) {
    return resblock_c2s(dtype, coords, rows, x, channels, out_channels, eps, w, pred_subdiv,
                        subdivision, predicted_subdiv, out_coords, y, rows_out, workspace, stream,
                        nullptr, nullptr);
}

size_t pxs_slat_decoder_workspace_bytes(int dtype, const pxs_decoder_config * cfg,
                                        const pxs_decoder_block * blocks, int n_blocks,
                                        int64_t rows, int64_t max_rows) {
    if (!cfg || !blocks || cfg->levels <= 0 || !cfg->model_channels || !cfg->num_blocks ||
        rows < 0 || max_rows < rows) {
        return 0;
    }
    Carver c(nullptr);
    carve_decoder(c, dtype, *cfg, blocks, n_blocks, rows, max_rows);
    return c.used();
}

int pxs_slat_decoder_forward(int dtype, const pxs_decoder_config * cfg,
                             const float * from_latent_weight, const float * from_latent_bias,
                             const float * output_weight, const float * output_bias,
                             const pxs_decoder_block * blocks, int n_blocks,
                             const int32_t * coords, int64_t rows, const float * x,
                             const float * const * guide, float * const * predicted,
                             int upsample_times, int64_t max_rows, int32_t * out_coords,
                             float * y, int64_t * rows_out, int64_t * level_rows,
                             void * workspace, void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_slat_decoder_forward");
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG,
              "pxs_slat_decoder_forward: bad dtype");
    PXS_CHECK(cfg && rows_out, PXS_ERR_ARG, "pxs_slat_decoder_forward: null config");
    const bool upsample = upsample_times >= 0;
    // Configuration checks in the reference's order (src/slat_decoder.cpp:298-330, 385-410).
    PXS_CHECK(cfg->norm_eps > 0.0f && std::isfinite(cfg->norm_eps), PXS_ERR_ARG,
              "SLat decoder norm epsilon must be finite and positive");
    const bool shape_ok = cfg->latent_channels > 0 && cfg->out_channels > 0 && cfg->levels > 0 &&
                          cfg->model_channels && cfg->num_blocks;
    if (upsample) {
        PXS_CHECK(shape_ok && cfg->pred_subdiv && upsample_times < cfg->levels, PXS_ERR_ARG,
                  "invalid SLat decoder coordinate-upsample configuration");
    } else {
        PXS_CHECK(shape_ok, PXS_ERR_ARG, "invalid SLat decoder configuration");
    }
    const int levels = cfg->levels;
    int64_t expected = levels - 1;
    for (int l = 0; l < levels; ++l) {
        PXS_CHECK(cfg->num_blocks[l] >= 0, PXS_ERR_ARG, "invalid SLat decoder block count");
        expected += cfg->num_blocks[l];
    }
    PXS_CHECK(blocks && n_blocks == expected, PXS_ERR_ARG,
              "SLat decoder weight block count does not match configuration");
    PXS_CHECK(from_latent_weight, PXS_ERR_ARG, "missing SLat decoder tensor: from_latent.weight");
    PXS_CHECK(from_latent_bias, PXS_ERR_ARG, "missing SLat decoder tensor: from_latent.bias");
    if (!upsample) {
        PXS_CHECK(output_weight, PXS_ERR_ARG, "missing SLat decoder tensor: output_layer.weight");
        PXS_CHECK(output_bias, PXS_ERR_ARG, "missing SLat decoder tensor: output_layer.bias");
    }
    PXS_CHECK(!predicted || cfg->pred_subdiv, PXS_ERR_ARG,
              "pxs_slat_decoder_forward: predicted logits need pred_subdiv");
    PXS_CHECK(rows >= 0 && max_rows >= rows, PXS_ERR_ARG, "pxs_slat_decoder_forward: bad shape");
    PXS_CHECK(rows == 0 || (coords && x && out_coords && y && workspace), PXS_ERR_ARG,
              "pxs_slat_decoder_forward: null pointer");
    if (level_rows) level_rows[0] = rows;
    *rows_out = 0;
    if (rows == 0) return PXS_OK;
    hipStream_t s = as_stream(stream);
    Carver c(workspace);
    const DecoderBuffers b = carve_decoder(c, dtype, *cfg, blocks, n_blocks, rows, max_rows);
    const float eps = cfg->norm_eps;
    int cur = 0;
    int64_t n = rows;
    const int32_t * ccur = coords;
    PXS_TRY(pxs_linear(PXS_F32, x, rows, cfg->latent_channels, from_latent_weight, from_latent_bias,
                       cfg->model_channels[0], PXS_ACT_NONE, b.hid[0], stream));
    int bi = 0;
    // Each level's coordinates are hashed once: the C2S block builds the next
    // level's map into b.map[1 - mc] for its conv2, and the next level's
    // ConvNeXt blocks and C2S conv1 reuse it.
    int mc = 0;
    bool map_ready = false;
    for (int l = 0; l < levels; ++l) {
        const int C = cfg->model_channels[l];
        if (upsample && l == upsample_times) {
            // slat_decoder_upsample_coords_f32 returns the hidden state here.
            PXS_TRY(check_hip(hipMemcpyAsync(y, b.hid[cur], n * C * sizeof(float),
                                             hipMemcpyDeviceToDevice, s), "decoder output copy"));
            PXS_TRY(check_hip(hipMemcpyAsync(out_coords, ccur, n * 16, hipMemcpyDeviceToDevice, s),
                              "decoder coordinate copy"));
            *rows_out = n;
            return check_launch("pxs_slat_decoder_forward");
        }
        if ((cfg->num_blocks[l] > 0 || l + 1 < levels) && !map_ready) {
            PXS_TRY(build_map(ccur, n, b.map[mc], stream));
            map_ready = true;
        }
        for (int k = 0; k < cfg->num_blocks[l]; ++k, ++bi) {
            const pxs_decoder_block & blk = blocks[bi];
            PXS_CHECK(blk.kind == PXS_DECODER_CONVNEXT, PXS_ERR_ARG,
                      upsample ? "SLat decoder coordinate-upsample expected ConvNeXt block"
                               : "SLat decoder expected ConvNeXt block");
            PXS_CHECK(blk.channels == C, PXS_ERR_ARG,
                      "pxs_slat_decoder_forward: block channels do not match the level");
            PXS_TRY(pxs_convnext_block(dtype, ccur, n, b.hid[cur], C, blk.mlp_hidden, eps, &blk.w,
                                       b.map[mc].nbr, b.map[mc].masks, b.hid[cur], b.block_ws,
                                       stream));
        }
        if (l + 1 == levels) break;
        const pxs_decoder_block & blk = blocks[bi++];
        PXS_CHECK(blk.kind == PXS_DECODER_C2S, PXS_ERR_ARG,
                  upsample ? "SLat decoder coordinate-upsample expected C2S block"
                           : "SLat decoder expected channel-to-spatial block");
        PXS_CHECK(blk.channels == C && blk.out_channels == cfg->model_channels[l + 1], PXS_ERR_ARG,
                  "pxs_slat_decoder_forward: block channels do not match the level");
        PXS_CHECK(n <= max_rows / 8, PXS_ERR_ARG,
                  "pxs_slat_decoder_forward: a level may exceed max_rows (needs 8 * rows)");
        const int nxt = 1 - cur;
        const bool pred = upsample ? true : cfg->pred_subdiv != 0;
        const float * g = (!upsample && guide) ? guide[l] : nullptr;
        float * logits = (!upsample && predicted) ? predicted[l] : nullptr;
        int64_t m = 0;
        PXS_TRY(resblock_c2s(dtype, ccur, n, b.hid[cur], C, blk.out_channels, eps, &blk.w,
                             pred ? 1 : 0, g, logits, b.crd[nxt], b.hid[nxt], &m, b.block_ws,
                             stream, &b.map[mc], &b.map[1 - mc]));
        ccur = b.crd[nxt];
        cur = nxt;
        n = m;
        mc = 1 - mc;
        map_ready = m > 0;  // with no children the block returns before building it
        if (level_rows) level_rows[l + 1] = n;
    }
    // Final layer norm (eps 1e-5, no affine) and output linear
    // (src/slat_decoder.cpp:367-372).
    const int C = cfg->model_channels[levels - 1];
    PXS_TRY(pxs_layer_norm(PXS_F32, b.hid[cur], n, C, 1e-5f, nullptr, nullptr, PXS_F32,
                           b.hid[1 - cur], stream));
    PXS_TRY(pxs_linear(PXS_F32, b.hid[1 - cur], n, C, output_weight, output_bias, cfg->out_channels,
                       PXS_ACT_NONE, y, stream));
    if (n > 0 && ccur != out_coords) {
        PXS_TRY(check_hip(hipMemcpyAsync(out_coords, ccur, n * 16, hipMemcpyDeviceToDevice, s),
                          "decoder coordinate copy"));
    }
    *rows_out = n;
    return check_launch("pxs_slat_decoder_forward");
}

} // extern "C"
