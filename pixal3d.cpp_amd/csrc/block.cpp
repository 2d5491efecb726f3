// Device-resident composition of the sparse transformer block and the SLat
// flow forward out of the pxs kernels.  Every intermediate stays in HBM; the
// residual stream is fp32, GEMM operands are in the call's dtype.
//
// Block order follows src/sparse_transformer.cpp:195-290:
//   LN -> modulate(0) -> QKV -> [RMS q,k] -> [RoPE q,k] -> SDPA -> out-proj
//   -> gate(2C) + residual -> LN(norm2 affine) -> cross Q -> [RMS] ->
//   context KV -> [RMS k] -> cross attention -> out (+ projection) + residual
//   -> LN -> modulate(3C) -> MLP0 -> GELU-tanh -> MLP2 -> gate(5C) + residual.
// The adaLN modulate and the gates are fused into the layer-norm kernel and
// the GEMM epilogues; RMS norm and RoPE are fused into one QKV prologue.

#include "carve.h"
#include "pxs_common.h"
#include "scan.h"

#include <cmath>

namespace pxs {
namespace {

struct BlockBuffers {
    void * xm;    // [rows, C]       LN output fed to a GEMM
    void * big;   // [rows, max(3C, mlp)]  QKV, then MLP hidden
    void * q;     // [rows, C]
    void * k;     // [rows, C]
    void * v;     // [rows, C]
    void * att;   // [rows, C]       attention output
    void * ckv;   // [T, 2C]         context K | V
    void * ck;    // [T, C]          RMS-normed context K
    void * attn_ws;
};

BlockBuffers carve_block(Carver & c, int dtype, const pxs_block_config & cfg, int64_t rows,
                         int64_t tokens, int batch_size) {
    const size_t e = dtype_bytes(dtype);
    const size_t C = static_cast<size_t>(cfg.channels);
    const size_t wide = std::max<size_t>(3 * C, static_cast<size_t>(cfg.mlp_hidden));
    const size_t r = static_cast<size_t>(std::max<int64_t>(rows, 1));
    const size_t t = static_cast<size_t>(std::max<int64_t>(tokens, 1));
    BlockBuffers b;
    b.xm = c.take(r * C * e);
    b.big = c.take(r * wide * e);
    b.q = c.take(r * C * e);
    b.k = c.take(r * C * e);
    b.v = c.take(r * C * e);
    b.att = c.take(r * C * e);
    b.ckv = c.take(t * 2 * C * e);
    b.ck = c.take(t * C * e);
    b.attn_ws = c.take(pxs_attention_workspace_bytes(batch_size));
    return b;
}

int check_block_args(const pxs_block_config * cfg, const pxs_block_weights * w) {
    PXS_CHECK(cfg && w, PXS_ERR_ARG, "pxs_transformer_block: null config or weights");
    PXS_CHECK(cfg->channels > 0 && cfg->num_heads > 0 && cfg->mlp_hidden > 0 &&
                  cfg->context_channels > 0 && cfg->channels % cfg->num_heads == 0 &&
                  cfg->norm_eps > 0.0f && std::isfinite(cfg->norm_eps),
              PXS_ERR_ARG, "invalid sparse transformer block configuration");
    PXS_CHECK(cfg->channels / cfg->num_heads <= 192, PXS_ERR_ARG,
              "pxs_transformer_block: head_dim above 192 unsupported");
    PXS_CHECK(!cfg->use_projection || cfg->proj_in_channels > 0, PXS_ERR_ARG,
              "sparse transformer projection shape does not match query");
    PXS_CHECK(w->modulation && w->self_to_qkv_weight && w->self_to_qkv_bias &&
                  w->self_to_out_weight && w->self_to_out_bias && w->norm2_weight &&
                  w->norm2_bias && w->cross_to_q_weight && w->cross_to_q_bias &&
                  w->cross_to_kv_weight && w->cross_to_kv_bias && w->cross_to_out_weight &&
                  w->cross_to_out_bias && w->mlp0_weight && w->mlp0_bias && w->mlp2_weight &&
                  w->mlp2_bias,
              PXS_ERR_ARG, "missing sparse transformer tensor");
    PXS_CHECK(!cfg->qk_rms_norm || (w->self_q_gamma && w->self_k_gamma), PXS_ERR_ARG,
              "missing sparse transformer tensor: self_attn q/k rms gamma");
    PXS_CHECK(!cfg->qk_rms_norm_cross || (w->cross_q_gamma && w->cross_k_gamma), PXS_ERR_ARG,
              "missing sparse transformer tensor: cross_attn q/k rms gamma");
    PXS_CHECK(!cfg->use_projection || (w->proj_weight && w->proj_bias), PXS_ERR_ARG,
              "missing sparse transformer tensor: cross_attn.proj_linear");
    return PXS_OK;
}


int run_block(int dtype, const pxs_block_config & cfg, const pxs_block_weights & w,
              const int32_t * coords, int64_t rows, int batch_size, const int64_t * cu_rows,
              float * hidden, const float * time_mod, const void * context,
              const int64_t * context_offsets, int64_t tokens, const void * projected,
              const BlockBuffers & b, void * stream) {
    const int C = cfg.channels, H = cfg.num_heads, hd = C / H;
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    const size_t e = dtype_bytes(dtype);

    // Self-attention branch.
    PXS_TRY(pxs_layer_norm_modulate(PXS_F32, hidden, rows, C, cfg.norm_eps, coords, w.modulation,
                                    time_mod, 0, dtype, b.xm, stream));
    PXS_TRY(pxs_linear(dtype, b.xm, rows, C, w.self_to_qkv_weight, w.self_to_qkv_bias, 3 * C,
                       PXS_ACT_NONE, b.big, stream));
    PXS_TRY(pxs_qkv_prepare(dtype, b.big, rows, H, hd, cfg.qk_rms_norm ? w.self_q_gamma : nullptr,
                            cfg.qk_rms_norm ? w.self_k_gamma : nullptr,
                            cfg.use_rope ? coords : nullptr, cfg.rope_freq_min,
                            cfg.rope_freq_base, b.q, b.k, b.v, stream));
    PXS_TRY(pxs_varlen_attention(dtype, b.q, C, b.k, C, b.v, C, cu_rows, cu_rows, batch_size, rows,
                                 nullptr, H, hd, hd, scale, b.att, C, b.attn_ws, stream));
    PXS_TRY(pxs_linear_gate_residual(dtype, b.att, rows, C, w.self_to_out_weight,
                                     w.self_to_out_bias, C, coords, w.modulation, time_mod, 2 * C,
                                     hidden, stream));

    // Cross-attention branch.
    PXS_TRY(pxs_layer_norm(PXS_F32, hidden, rows, C, cfg.norm_eps, w.norm2_weight, w.norm2_bias,
                           dtype, b.xm, stream));
    PXS_TRY(pxs_linear(dtype, b.xm, rows, C, w.cross_to_q_weight, w.cross_to_q_bias, C,
                       PXS_ACT_NONE, b.q, stream));
    if (cfg.qk_rms_norm_cross) {
        PXS_TRY(pxs_mh_rms_norm(dtype, b.q, C, rows, H, hd, w.cross_q_gamma, b.q, C, stream));
    }
    PXS_TRY(pxs_linear(dtype, context, tokens, cfg.context_channels, w.cross_to_kv_weight,
                       w.cross_to_kv_bias, 2 * C, PXS_ACT_NONE, b.ckv, stream));
    const void * ck = b.ckv;
    int64_t ld_k = 2 * C;
    if (cfg.qk_rms_norm_cross) {
        PXS_TRY(pxs_mh_rms_norm(dtype, b.ckv, 2 * C, tokens, H, hd, w.cross_k_gamma, b.ck, C,
                                stream));
        ck = b.ck;
        ld_k = C;
    }
    const void * cv = static_cast<const char *>(b.ckv) + static_cast<size_t>(C) * e;
    PXS_TRY(pxs_varlen_attention(dtype, b.q, C, ck, ld_k, cv, 2 * C, cu_rows, context_offsets,
                                 batch_size, rows, nullptr, H, hd, hd, scale, b.att, C, b.attn_ws,
                                 stream));
    PXS_TRY(pxs_linear_residual(dtype, b.att, rows, C, w.cross_to_out_weight, w.cross_to_out_bias,
                                C, hidden, stream));
    if (cfg.use_projection) {
        PXS_TRY(pxs_linear_residual(dtype, projected, rows, cfg.proj_in_channels, w.proj_weight,
                                    w.proj_bias, C, hidden, stream));
    }

    // MLP branch.
    PXS_TRY(pxs_layer_norm_modulate(PXS_F32, hidden, rows, C, cfg.norm_eps, coords, w.modulation,
                                    time_mod, 3 * C, dtype, b.xm, stream));
    PXS_TRY(pxs_linear(dtype, b.xm, rows, C, w.mlp0_weight, w.mlp0_bias, cfg.mlp_hidden,
                       PXS_ACT_GELU_TANH, b.big, stream));
    PXS_TRY(pxs_linear_gate_residual(dtype, b.big, rows, cfg.mlp_hidden, w.mlp2_weight,
                                     w.mlp2_bias, C, coords, w.modulation, time_mod, 5 * C, hidden,
                                     stream));
    return PXS_OK;
}

pxs_block_config flow_block_config(const pxs_flow_config & f) {
    pxs_block_config c{};
    c.channels = f.model_channels;
    c.num_heads = f.num_heads;
    c.mlp_hidden = f.mlp_hidden;
    c.context_channels = f.cond_channels;
    c.proj_in_channels = f.proj_in_channels;
    c.norm_eps = f.norm_eps;
    c.rope_freq_min = f.rope_freq_min;
    c.rope_freq_base = f.rope_freq_base;
    c.use_rope = 1;  // src/slat_flow.cpp:233
    c.qk_rms_norm = f.qk_rms_norm;
    c.qk_rms_norm_cross = f.qk_rms_norm_cross;
    c.use_projection = f.use_projection;
    return c;
}

struct FlowBuffers {
    float * hidden;   // [rows, C] residual stream
    float * normed;   // [rows, C] final layer norm
    float * temb0;    // [batch, 256] sinusoid
    float * temb1;    // [batch, C]
    float * temb2;    // [batch, C]
    float * time_mod; // [batch, 6C]
    BlockBuffers block;
};

constexpr int kTimestepFreqDim = 256;  // src/slat_flow.cpp:209

FlowBuffers carve_flow(Carver & c, int dtype, const pxs_flow_config & f, int64_t rows,
                       int64_t tokens, int batch_size) {
    const size_t C = static_cast<size_t>(f.model_channels);
    const size_t r = static_cast<size_t>(std::max<int64_t>(rows, 1));
    const size_t bs = static_cast<size_t>(std::max(batch_size, 1));
    FlowBuffers b;
    b.hidden = static_cast<float *>(c.take(r * C * 4));
    b.normed = static_cast<float *>(c.take(r * C * 4));
    b.temb0 = static_cast<float *>(c.take(bs * kTimestepFreqDim * 4));
    b.temb1 = static_cast<float *>(c.take(bs * C * 4));
    b.temb2 = static_cast<float *>(c.take(bs * C * 4));
    b.time_mod = static_cast<float *>(c.take(bs * 6 * C * 4));
    const pxs_block_config bc = flow_block_config(f);
    b.block = carve_block(c, dtype, bc, rows, tokens, batch_size);
    return b;
}

} // namespace
} // namespace pxs

using namespace pxs;

extern "C" {

size_t pxs_transformer_block_workspace_bytes(int dtype, const pxs_block_config * cfg,
                                             int64_t rows, int64_t context_tokens,
                                             int batch_size) {
    if (!cfg) return 0;
    Carver c(nullptr);
    carve_block(c, dtype, *cfg, rows, context_tokens, batch_size);
    return c.used();
}

int pxs_transformer_block(int dtype, const pxs_block_config * cfg, const pxs_block_weights * w,
                          const int32_t * coords, int64_t rows, int batch_size,
                          const int64_t * cu_rows, float * hidden, const float * time_mod,
                          const void * context, const int64_t * context_offsets,
                          int64_t context_tokens, const void * projected, void * workspace,
                          void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_transformer_block");
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG,
              "pxs_transformer_block: bad dtype");
    PXS_TRY(check_block_args(cfg, w));
    PXS_CHECK(rows >= 0 && batch_size > 0 && context_tokens >= 0, PXS_ERR_ARG,
              "pxs_transformer_block: bad shape");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(coords && cu_rows && hidden && time_mod && context && context_offsets && workspace,
              PXS_ERR_ARG, "pxs_transformer_block: null pointer");
    PXS_CHECK(!cfg->use_projection || projected, PXS_ERR_ARG,
              "sparse transformer projection shape does not match query");
    Carver c(workspace);
    const BlockBuffers b = carve_block(c, dtype, *cfg, rows, context_tokens, batch_size);
    return run_block(dtype, *cfg, *w, coords, rows, batch_size, cu_rows, hidden, time_mod, context,
                     context_offsets, context_tokens, projected, b, stream);
}

size_t pxs_slat_flow_workspace_bytes(int dtype, const pxs_flow_config * cfg, int64_t rows,
                                     int64_t context_tokens, int batch_size) {
    if (!cfg) return 0;
    Carver c(nullptr);
    carve_flow(c, dtype, *cfg, rows, context_tokens, batch_size);
    return c.used();
}

int pxs_slat_flow_forward(int dtype, const pxs_flow_config * cfg, const pxs_flow_weights * w,
                          const int32_t * coords, int64_t rows, int batch_size,
                          const int64_t * cu_rows, const float * x, const float * timesteps,
                          const void * context, const int64_t * context_offsets,
                          int64_t context_tokens, const void * projected, float * out,
                          void * workspace, void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_slat_flow_forward");
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG,
              "pxs_slat_flow_forward: bad dtype");
    PXS_CHECK(cfg && w, PXS_ERR_ARG, "pxs_slat_flow_forward: null config or weights");
    PXS_CHECK(cfg->in_channels > 0 && cfg->out_channels > 0 && cfg->model_channels > 0 &&
                  cfg->num_blocks >= 0 && batch_size > 0 && rows >= 0,
              PXS_ERR_ARG, "pxs_slat_flow_forward: bad shape");
    PXS_CHECK(w->input_weight && w->input_bias && w->timestep_weight0 && w->timestep_bias0 &&
                  w->timestep_weight2 && w->timestep_bias2 && w->modulation_weight &&
                  w->modulation_bias && w->output_weight && w->output_bias &&
                  (cfg->num_blocks == 0 || w->blocks),
              PXS_ERR_ARG, "pxs_slat_flow_forward: missing weight");
    const pxs_block_config bc = flow_block_config(*cfg);
    for (int i = 0; i < cfg->num_blocks; ++i) PXS_TRY(check_block_args(&bc, &w->blocks[i]));
    if (rows == 0) return PXS_OK;
    PXS_CHECK(coords && cu_rows && x && timesteps && context && context_offsets && out && workspace,
              PXS_ERR_ARG, "pxs_slat_flow_forward: null pointer");
    PXS_CHECK(!cfg->use_projection || projected, PXS_ERR_ARG,
              "SLat flow projection context shape mismatch");
    Carver c(workspace);
    const FlowBuffers b = carve_flow(c, dtype, *cfg, rows, context_tokens, batch_size);
    hipStream_t s = as_stream(stream);
    const int C = cfg->model_channels;

    // hidden = input linear (src/slat_flow.cpp:204-205), accumulated into a
    // zeroed fp32 residual so the stream starts at full precision.
    PXS_TRY(fill_u32(reinterpret_cast<uint32_t *>(b.hidden), rows * C, 0u, s));
    PXS_TRY(pxs_linear_residual(PXS_F32, x, rows, cfg->in_channels, w->input_weight,
                                w->input_bias, C, b.hidden, stream));
    // Timestep embedding MLP, SiLU, adaLN linear (src/slat_flow.cpp:207-222).
    PXS_TRY(pxs_timestep_embedding(timesteps, batch_size, kTimestepFreqDim, 10000, b.temb0, stream));
    PXS_TRY(pxs_linear(PXS_F32, b.temb0, batch_size, kTimestepFreqDim, w->timestep_weight0,
                       w->timestep_bias0, C, PXS_ACT_SILU, b.temb1, stream));
    PXS_TRY(pxs_linear(PXS_F32, b.temb1, batch_size, C, w->timestep_weight2, w->timestep_bias2, C,
                       PXS_ACT_SILU, b.temb2, stream));
    PXS_TRY(pxs_linear(PXS_F32, b.temb2, batch_size, C, w->modulation_weight, w->modulation_bias,
                       6 * C, PXS_ACT_NONE, b.time_mod, stream));
    for (int i = 0; i < cfg->num_blocks; ++i) {
        PXS_TRY(run_block(dtype, bc, w->blocks[i], coords, rows, batch_size, cu_rows, b.hidden,
                          b.time_mod, context, context_offsets, context_tokens, projected, b.block,
                          stream));
    }
    // Final layer norm keeps eps 1e-5 (src/slat_flow.cpp:244-248).
    PXS_TRY(pxs_layer_norm(PXS_F32, b.hidden, rows, C, 1e-5f, nullptr, nullptr, PXS_F32, b.normed,
                           stream));
    return pxs_linear(PXS_F32, b.normed, rows, C, w->output_weight, w->output_bias,
                      cfg->out_channels, PXS_ACT_NONE, out, stream);
}

} // extern "C"
