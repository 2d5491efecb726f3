// Model loaders over an open pack: the SLat-flow and SLat-decoder weights of
// one component, uploaded into a caller-provided device arena in the layout
// and dtype pxs_slat_flow_forward / pxs_slat_decoder_forward take.
//
// SLatFlowModel::load (src/slat_flow.cpp:1239-1281, hyperparameters
// 397-429 checked by valid_hparams 113-138) and SLatDecoderModel::load
// (src/slat_decoder.cpp:3392-3467): the same component checks, metadata keys,
// defaults and messages in the same order; every tensor under the
// component's prefix is converted in table order, the first unsupported,
// misaligned or non-finite one failing the load with the reference's
// message.  The weight binding of SLatFlowModel::forward
// (src/slat_flow.cpp:1348-1395) and SLatDecoderModel::Impl::make_weights
// (src/slat_decoder.cpp:2911-2970) follows, at load time: a missing tensor
// fails with the reference's "missing ... tensor" message, and a tensor
// whose shape differs from the hyperparameters' fails too (the reference
// would read past it).
//
// The compact-v1 layouts are the kernels' operand layouts: a linear weight
// [out, in] and a convolution weight [27, out, in] keep the reduction axis
// contiguous, the B-operand rows the GEMMs stream.  Ingestion therefore
// converts and does not re-layout: GEMM operands (block linears, decoder
// convolutions and ConvNeXt MLPs) into the call's dtype (PXS_BF16 rounds to
// nearest even from the stored value, exact for BF16 payloads), everything
// else (norms, biases, gammas, modulations, the flow's embedding and
// output layers, the decoder's from_latent / output layers and subdivision
// head) into fp32.  Each tensor starts on a 256-byte boundary.

#include "ingest.h"
#include "pxs_common.h"

#include <cmath>
#include <cstring>
#include <string>
#include <vector>

namespace pxs {
namespace {

bool has_prefix(const std::string & s, const std::string & p) {
    return s.size() >= p.size() && s.compare(0, p.size(), p) == 0;
}

bool has_suffix(const std::string & s, const std::string & p) {
    return s.size() >= p.size() && s.compare(s.size() - p.size(), p.size(), p) == 0;
}

int argfail(const std::string & m) { return fail(PXS_ERR_ARG, m); }

// One component's tensors in table order with their arena placement.
struct Placement {
    const GgufTensor * t;
    int dtype;
    size_t offset;
    size_t bytes;
};

struct Layout {
    std::string prefix;  // "<alias>." of tensor names
    std::vector<Placement> items;
    size_t arena_bytes = 0;
};

int64_t elements_of(const GgufTensor & t) {
    if (t.type == kGgmlF32) return static_cast<int64_t>(t.n_bytes / 4);
    if (t.type == kGgmlF16 || t.type == kGgmlBf16) return static_cast<int64_t>(t.n_bytes / 2);
    return 0;
}

template <typename IsOperand>
void place(const GgufFile & f, const std::string & prefix, int dtype, IsOperand is_operand,
           Layout & out) {
    out.prefix = prefix;
    size_t off = 0;
    for (const GgufTensor & t : f.tensors) {
        if (!has_prefix(t.name, prefix)) continue;
        const int d = is_operand(t.name.substr(prefix.size())) ? dtype : PXS_F32;
        const size_t bytes = static_cast<size_t>(elements_of(t)) * (d == PXS_F32 ? 4 : 2);
        out.items.push_back({&t, d, off, bytes});
        off += (bytes + 255) / 256 * 256;
    }
    out.arena_bytes = off;
}

// Upload every placed tensor; `family` names the model in messages
// ("SLat flow" / "SLat decoder").  Error precedence is the reference's
// sequential one: the first tensor (in table order) that is unsupported,
// misaligned, unreadable or non-finite fails the load.
int upload_all(pxs_pack * pack, const Layout & layout, void * arena, void * workspace,
               hipStream_t stream, bool flow) {
    // Host checks in table order; the items before the first failing tensor
    // are uploaded, so a non-finite value in an earlier tensor still wins.
    int host_rc = PXS_OK;
    std::string host_msg;
    std::vector<IngestItem> items;
    size_t k = 0;
    for (; k < layout.items.size(); ++k) {
        const Placement & p = layout.items[k];
        const GgufTensor & t = *p.t;
        const bool wide = t.type == kGgmlF32, narrow = t.type == kGgmlF16 || t.type == kGgmlBf16;
        if (flow && (!(wide || narrow) || t.n_bytes % (wide ? 4 : 2) != 0)) {
            host_rc = PXS_ERR_ARG;
            host_msg = "unsupported or misaligned SLat flow tensor: " + t.name;
            break;
        }
        if (!flow && !(wide || narrow)) {
            host_rc = PXS_ERR_ARG;
            host_msg = "unsupported SLat decoder tensor type: " + t.name;
            break;
        }
        if (!flow && t.n_bytes % (wide ? 4 : 2) != 0) {
            host_rc = PXS_ERR_ARG;
            host_msg = "SLat decoder tensor payload is not element aligned: " + t.name;
            break;
        }
        if (p.bytes > 0) items.push_back({&t, p.dtype, static_cast<uint8_t *>(arena) + p.offset, k});
    }
    Ingest ingest(pack, workspace, layout.items.size(), stream);
    int rc = ingest.begin();
    if (rc != PXS_OK) return rc;
    rc = ingest.run(items);
    if (rc != PXS_OK) {
        // An I/O or runtime failure: still report an earlier non-finite
        // tensor first when the stream got that far.
        host_rc = rc;
        host_msg = pxs_last_error();
    }
    std::vector<int32_t> nonfinite;
    const int frc = ingest.finish(nonfinite);
    if (frc != PXS_OK) return frc;
    for (size_t j = 0; j < k; ++j) {
        if (nonfinite[j]) {
            return fail(PXS_ERR_DATA, std::string(flow ? "SLat flow" : "SLat decoder") +
                                          " tensor contains a non-finite value: " +
                                          layout.items[j].t->name);
        }
    }
    if (host_rc != PXS_OK) return fail(host_rc, host_msg);
    return PXS_OK;
}

std::string shape_text(const int64_t * ne) {
    return "[" + std::to_string(ne[0]) + ", " + std::to_string(ne[1]) + ", " +
           std::to_string(ne[2]) + ", " + std::to_string(ne[3]) + "]";
}

// Looks tensors up by local name and checks their shapes.
class Binder {
public:
    Binder(const Layout & layout, void * arena, const char * family)
        : layout_(layout), arena_(static_cast<uint8_t *>(arena)), family_(family) {}

    // A matrix [rows, cols] (GGUF ne = (cols, rows)), a convolution
    // [27, rows, cols] (ne = (cols, rows, 27)) or a vector of `count`
    // elements (any shape) when rows == 0.
    const void * get(const std::string & local, int64_t rows, int64_t cols, int64_t taps = 1,
                     int64_t count = 0) {
        if (rc_ != PXS_OK) return nullptr;
        const std::string full = layout_.prefix + local;
        const Placement * p = nullptr;
        for (const Placement & q : layout_.items) {
            if (q.t->name == full) {
                p = &q;
                break;
            }
        }
        if (!p) {
            rc_ = argfail("missing " + family_ + " tensor: " + full);
            return nullptr;
        }
        const int64_t * ne = p->t->ne;
        bool ok;
        std::string want;
        if (rows == 0) {
            ok = ne[0] * ne[1] * ne[2] * ne[3] == count;
            want = std::to_string(count) + " elements";
        } else {
            const int64_t w[4] = {cols, rows, taps, 1};
            ok = std::memcmp(ne, w, sizeof(w)) == 0;
            want = shape_text(w);
        }
        if (!ok) {
            rc_ = argfail(family_ + " tensor " + full + " has shape " + shape_text(ne) +
                          ", expected " + want);
            return nullptr;
        }
        return arena_ + p->offset;
    }
    const float * vec(const std::string & local, int64_t count) {
        return static_cast<const float *>(get(local, 0, 0, 1, count));
    }
    const float * mat32(const std::string & local, int64_t rows, int64_t cols) {
        return static_cast<const float *>(get(local, rows, cols));
    }
    int rc() const { return rc_; }

private:
    const Layout & layout_;
    uint8_t * arena_;
    std::string family_;
    int rc_ = PXS_OK;
};

// ---- SLat flow ------------------------------------------------------------------

// compact_prefix (src/slat_flow.cpp:354-359).
std::string flow_alias(const std::string & component) {
    if (component == "shape_flow_512") return "sh512";
    if (component == "shape_flow_1024") return "sh1024";
    if (component == "texture_flow_1024") return "tx1024";
    return {};
}

bool is_flow_operand(const std::string & local) {
    if (!has_prefix(local, "blocks.")) return false;
    static const char * kOperands[] = {
        ".self_attn.to_qkv.weight", ".self_attn.to_out.weight",
        ".cross_attn.cross_attn_block.to_q.weight", ".cross_attn.cross_attn_block.to_kv.weight",
        ".cross_attn.cross_attn_block.to_out.weight", ".cross_attn.proj_linear.weight",
        ".mlp.mlp.0.weight", ".mlp.mlp.2.weight"};
    for (const char * s : kOperands) {
        if (has_suffix(local, s)) return true;
    }
    return false;
}

int flow_plan(const pxs_pack * pack, const std::string & component, int dtype,
              pxs_flow_config & cfg, Layout & layout) {
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG, "SLat flow load: bad dtype");
    const std::string alias = flow_alias(component);
    if (alias.empty()) return argfail("unsupported SLat flow component: " + component);
    const GgufFile & f = pack->file;
    if (!f.tensor(alias + ".input_layer.weight")) {
        return argfail("GGUF pack does not contain SLat flow component: " + component);
    }
    // read_hparams (src/slat_flow.cpp:397-429).
    const std::string p = "pixal3d." + component + ".";
    std::string err, model_class, pe_mode, image_attn_mode;
    uint32_t resolution = 0, in_ch = 0, out_ch = 0, C = 0, cond = 0, blocks = 0, heads = 0,
             proj_in = 0;
    float mlp_ratio = 0.0f, rope_min = 1.0f, rope_base = 10000.0f;
    bool share_mod = false, qk = false, qk_cross = false;
    const float norm_eps = 1e-6f;  // SLatFlowHParams default; not a pack key
    if (!metadata_string(f, p + "model_class", model_class, true, &err) ||
        !metadata_u32(f, p + "resolution", resolution, true, &err) ||
        !metadata_u32(f, p + "in_channels", in_ch, true, &err) ||
        !metadata_u32(f, p + "out_channels", out_ch, true, &err) ||
        !metadata_u32(f, p + "model_channels", C, true, &err) ||
        !metadata_u32(f, p + "cond_channels", cond, true, &err) ||
        !metadata_u32(f, p + "num_blocks", blocks, true, &err) ||
        !metadata_u32(f, p + "num_heads", heads, true, &err) ||
        !metadata_f32(f, p + "mlp_ratio", mlp_ratio, true, &err) ||
        !metadata_string(f, p + "pe_mode", pe_mode, false, &err) ||
        !metadata_bool(f, p + "share_mod", share_mod, false, &err) ||
        !metadata_bool(f, p + "qk_rms_norm", qk, false, &err) ||
        !metadata_bool(f, p + "qk_rms_norm_cross", qk_cross, false, &err) ||
        !metadata_f32(f, p + "rope_freq_min", rope_min, false, &err) ||
        !metadata_f32(f, p + "rope_freq_base", rope_base, false, &err) ||
        !metadata_string(f, p + "image_attn_mode", image_attn_mode, false, &err) ||
        !metadata_u32(f, p + "proj_in_channels", proj_in, false, &err)) {
        return argfail(err);
    }
    if (pe_mode.empty()) pe_mode = "rope";
    if (image_attn_mode.empty()) image_attn_mode = "cross";
    const int proj = proj_in == 0 ? static_cast<int>(cond) : static_cast<int>(proj_in);
    // valid_hparams (src/slat_flow.cpp:113-138); the u32 values are read
    // into int as the reference does.
    const int ires = static_cast<int>(resolution), iin = static_cast<int>(in_ch),
              iout = static_cast<int>(out_ch), iC = static_cast<int>(C),
              icond = static_cast<int>(cond), iblocks = static_cast<int>(blocks),
              iheads = static_cast<int>(heads);
    const int head_dim = iheads > 0 ? iC / iheads : 0;
    if (ires <= 0 || iin <= 0 || iout <= 0 || iC <= 0 || icond <= 0 || iblocks <= 0 ||
        iheads <= 0 || iC % iheads != 0 || head_dim <= 0 || head_dim % 2 != 0 ||
        mlp_ratio <= 0.0f || !std::isfinite(mlp_ratio) || rope_min <= 0.0f ||
        rope_base <= 0.0f || !std::isfinite(rope_min) || !std::isfinite(rope_base)) {
        return argfail("invalid SLat flow hyperparameters");
    }
    if (pe_mode != "rope" || !share_mod) {
        return argfail("SLat flow currently requires pe_mode=rope and share_mod=true");
    }
    if (image_attn_mode != "cross" && image_attn_mode != "proj") {
        return argfail("SLat flow supports image_attn_mode cross or proj");
    }
    if (image_attn_mode == "proj" && proj <= 0) {
        return argfail("SLat flow projection channels must be positive");
    }
    place(f, alias + ".", dtype, is_flow_operand, layout);
    if (layout.items.empty()) return argfail("SLat flow component has no tensors: " + component);
    std::memset(&cfg, 0, sizeof(cfg));
    cfg.in_channels = iin;
    cfg.out_channels = iout;
    cfg.model_channels = iC;
    cfg.cond_channels = icond;
    cfg.num_blocks = iblocks;
    cfg.num_heads = iheads;
    cfg.proj_in_channels = proj;
    // block_config.mlp_hidden (src/slat_flow.cpp:227).
    cfg.mlp_hidden = static_cast<int>(static_cast<float>(iC) * mlp_ratio);
    cfg.norm_eps = norm_eps;
    cfg.rope_freq_min = rope_min;
    cfg.rope_freq_base = rope_base;
    cfg.qk_rms_norm = qk ? 1 : 0;
    cfg.qk_rms_norm_cross = qk_cross ? 1 : 0;
    cfg.use_projection = image_attn_mode == "proj" ? 1 : 0;
    return PXS_OK;
}

// ---- SLat decoder ---------------------------------------------------------------

bool is_decoder_operand(const std::string & local) {
    if (!has_prefix(local, "blocks.")) return false;
    return has_suffix(local, ".conv.weight") || has_suffix(local, ".conv1.weight") ||
           has_suffix(local, ".conv2.weight") || has_suffix(local, ".mlp.0.weight") ||
           has_suffix(local, ".mlp.2.weight");
}

int decoder_plan(const pxs_pack * pack, const std::string & component, int dtype,
                 pxs_decoder_hparams & hp, Layout & layout) {
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG,
              "SLat decoder load: bad dtype");
    if (component.empty() || component.find('.') != std::string::npos) {
        return argfail("invalid SLat decoder component name");
    }
    const GgufFile & f = pack->file;
    if (!f.tensor(component + ".from_latent.weight")) {
        return argfail("GGUF pack does not contain SLat decoder component: " + component);
    }
    const std::string p = "pixal3d." + component + ".";
    std::string err, model_class;
    uint32_t value = 0;
    std::memset(&hp, 0, sizeof(hp));
    if (!metadata_string(f, p + "model_class", model_class, true, &err) ||
        !metadata_u32(f, p + "resolution", value, false, &err)) {
        return argfail(err);
    }
    hp.resolution = static_cast<int>(value);
    if (!metadata_u32(f, p + "latent_channels", value, true, &err)) return argfail(err);
    hp.latent_channels = static_cast<int>(value);
    if (!metadata_u32(f, p + "out_channels", value, true, &err)) return argfail(err);
    hp.out_channels = static_cast<int>(value);
    if (!metadata_u32(f, p + "n_levels", value, true, &err)) return argfail(err);
    const int levels = static_cast<int>(value);
    float eps = 0.0f;
    if (!metadata_f32(f, p + "norm_eps", eps, false, &err)) return argfail(err);
    hp.norm_eps = eps > 0.0f && std::isfinite(eps) ? eps : 1e-6f;
    bool pred = false;
    if (!metadata_bool(f, p + "pred_subdiv", pred, false, &err)) return argfail(err);
    hp.pred_subdiv = pred ? 1 : 0;
    if (hp.resolution < 0 || hp.latent_channels <= 0 || hp.out_channels <= 0 || levels <= 0 ||
        levels > PXS_DECODER_MAX_LEVELS) {
        return argfail("invalid SLat decoder metadata");
    }
    hp.levels = levels;
    hp.n_blocks = levels - 1;
    for (int l = 0; l < levels; ++l) {
        if (!metadata_u32(f, p + "model_channels." + std::to_string(l), value, true, &err)) {
            return argfail(err);
        }
        hp.model_channels[l] = static_cast<int>(value);
        if (!metadata_u32(f, p + "num_blocks." + std::to_string(l), value, true, &err)) {
            return argfail(err);
        }
        hp.num_blocks[l] = static_cast<int>(value);
        if (hp.model_channels[l] <= 0 || hp.num_blocks[l] < 0) {
            return argfail("invalid SLat decoder level metadata");
        }
        hp.n_blocks += hp.num_blocks[l];
    }
    place(f, component + ".", dtype, is_decoder_operand, layout);
    if (layout.items.empty()) {
        return argfail("SLat decoder component has no tensors: " + component);
    }
    return PXS_OK;
}

int check_arena(void * arena, size_t arena_bytes, size_t need, void * workspace,
                const char * what) {
    PXS_CHECK(arena && workspace, PXS_ERR_ARG, std::string(what) + ": null arena or workspace");
    PXS_CHECK(reinterpret_cast<uintptr_t>(arena) % 256 == 0, PXS_ERR_ARG,
              std::string(what) + ": arena must be 256-byte aligned");
    PXS_CHECK(arena_bytes >= need, PXS_ERR_ARG,
              std::string(what) + ": arena holds " + std::to_string(arena_bytes) +
                  " bytes, the component needs " + std::to_string(need));
    return PXS_OK;
}

} // namespace
} // namespace pxs

using namespace pxs;

extern "C" {

int pxs_slat_flow_pack_plan(const pxs_pack * pack, const char * component, int dtype,
                            pxs_flow_config * cfg, size_t * arena_bytes) {
    return pxs::guarded("pxs_slat_flow_pack_plan", [&]() -> int {
        PXS_CHECK(pack && component && cfg && arena_bytes, PXS_ERR_ARG,
                  "pxs_slat_flow_pack_plan: null argument");
        Layout layout;
        int rc = flow_plan(pack, component, dtype, *cfg, layout);
        if (rc != PXS_OK) return rc;
        *arena_bytes = layout.arena_bytes;
        return PXS_OK;
    });
}

int pxs_slat_flow_pack_load(pxs_pack * pack, const char * component, int dtype, void * arena,
                            size_t arena_bytes, void * workspace, pxs_flow_weights * w,
                            pxs_block_weights * blocks, int max_blocks, void * stream) {
    return pxs::guarded("pxs_slat_flow_pack_load", [&]() -> int {
        PXS_CHECK(pack && component && w && blocks, PXS_ERR_ARG,
                  "pxs_slat_flow_pack_load: null argument");
        PXS_CHECK_WORKSPACE(workspace, "pxs_slat_flow_pack_load");
        pxs_flow_config cfg;
        Layout layout;
        int rc = flow_plan(pack, component, dtype, cfg, layout);
        if (rc != PXS_OK) return rc;
        rc = check_arena(arena, arena_bytes, layout.arena_bytes, workspace, "pxs_slat_flow_pack_load");
        if (rc != PXS_OK) return rc;
        PXS_CHECK(max_blocks >= cfg.num_blocks, PXS_ERR_ARG,
                  "pxs_slat_flow_pack_load: blocks holds " + std::to_string(max_blocks) +
                      " entries, the model has " + std::to_string(cfg.num_blocks));
        rc = upload_all(pack, layout, arena, workspace, as_stream(stream), true);
        if (rc != PXS_OK) return rc;
        const int64_t C = cfg.model_channels, CC = cfg.cond_channels, M = cfg.mlp_hidden;
        Binder b(layout, arena, "SLat flow");
        std::memset(w, 0, sizeof(*w));
        w->input_weight = b.mat32("input_layer.weight", C, cfg.in_channels);
        w->input_bias = b.vec("input_layer.bias", C);
        w->timestep_weight0 = b.mat32("t_embedder.mlp.0.weight", C, 256);
        w->timestep_bias0 = b.vec("t_embedder.mlp.0.bias", C);
        w->timestep_weight2 = b.mat32("t_embedder.mlp.2.weight", C, C);
        w->timestep_bias2 = b.vec("t_embedder.mlp.2.bias", C);
        w->modulation_weight = b.mat32("adaLN_modulation.1.weight", 6 * C, C);
        w->modulation_bias = b.vec("adaLN_modulation.1.bias", 6 * C);
        w->output_weight = b.mat32("out_layer.weight", cfg.out_channels, C);
        w->output_bias = b.vec("out_layer.bias", cfg.out_channels);
        for (int i = 0; i < cfg.num_blocks; ++i) {
            const std::string p = "blocks." + std::to_string(i);
            const std::string cross = p + ".cross_attn.cross_attn_block";
            pxs_block_weights & k = blocks[i];
            std::memset(&k, 0, sizeof(k));
            k.modulation = b.vec(p + ".modulation", 6 * C);
            k.self_to_qkv_weight = b.get(p + ".self_attn.to_qkv.weight", 3 * C, C);
            k.self_to_qkv_bias = b.vec(p + ".self_attn.to_qkv.bias", 3 * C);
            if (cfg.qk_rms_norm) {
                k.self_q_gamma = b.vec(p + ".self_attn.q_rms_norm.gamma", C);
                k.self_k_gamma = b.vec(p + ".self_attn.k_rms_norm.gamma", C);
            }
            k.self_to_out_weight = b.get(p + ".self_attn.to_out.weight", C, C);
            k.self_to_out_bias = b.vec(p + ".self_attn.to_out.bias", C);
            k.norm2_weight = b.vec(p + ".norm2.weight", C);
            k.norm2_bias = b.vec(p + ".norm2.bias", C);
            k.cross_to_q_weight = b.get(cross + ".to_q.weight", C, C);
            k.cross_to_q_bias = b.vec(cross + ".to_q.bias", C);
            k.cross_to_kv_weight = b.get(cross + ".to_kv.weight", 2 * C, CC);
            k.cross_to_kv_bias = b.vec(cross + ".to_kv.bias", 2 * C);
            if (cfg.qk_rms_norm_cross) {
                k.cross_q_gamma = b.vec(cross + ".q_rms_norm.gamma", C);
                k.cross_k_gamma = b.vec(cross + ".k_rms_norm.gamma", C);
            }
            k.cross_to_out_weight = b.get(cross + ".to_out.weight", C, C);
            k.cross_to_out_bias = b.vec(cross + ".to_out.bias", C);
            if (cfg.use_projection) {
                k.proj_weight = b.get(p + ".cross_attn.proj_linear.weight", C, cfg.proj_in_channels);
                k.proj_bias = b.vec(p + ".cross_attn.proj_linear.bias", C);
            }
            k.mlp0_weight = b.get(p + ".mlp.mlp.0.weight", M, C);
            k.mlp0_bias = b.vec(p + ".mlp.mlp.0.bias", M);
            k.mlp2_weight = b.get(p + ".mlp.mlp.2.weight", C, M);
            k.mlp2_bias = b.vec(p + ".mlp.mlp.2.bias", C);
        }
        w->blocks = blocks;
        return b.rc();
    });
}

int pxs_slat_decoder_pack_plan(const pxs_pack * pack, const char * component, int dtype,
                               pxs_decoder_hparams * hp, size_t * arena_bytes) {
    return pxs::guarded("pxs_slat_decoder_pack_plan", [&]() -> int {
        PXS_CHECK(pack && component && hp && arena_bytes, PXS_ERR_ARG,
                  "pxs_slat_decoder_pack_plan: null argument");
        Layout layout;
        int rc = decoder_plan(pack, component, dtype, *hp, layout);
        if (rc != PXS_OK) return rc;
        *arena_bytes = layout.arena_bytes;
        return PXS_OK;
    });
}

int pxs_slat_decoder_pack_load(pxs_pack * pack, const char * component, int dtype, void * arena,
                               size_t arena_bytes, void * workspace, pxs_decoder_block * blocks,
                               int max_blocks, const float ** io_weights, void * stream) {
    return pxs::guarded("pxs_slat_decoder_pack_load", [&]() -> int {
        PXS_CHECK(pack && component && blocks && io_weights, PXS_ERR_ARG,
                  "pxs_slat_decoder_pack_load: null argument");
        PXS_CHECK_WORKSPACE(workspace, "pxs_slat_decoder_pack_load");
        pxs_decoder_hparams hp;
        Layout layout;
        int rc = decoder_plan(pack, component, dtype, hp, layout);
        if (rc != PXS_OK) return rc;
        rc = check_arena(arena, arena_bytes, layout.arena_bytes, workspace,
                         "pxs_slat_decoder_pack_load");
        if (rc != PXS_OK) return rc;
        PXS_CHECK(max_blocks >= hp.n_blocks, PXS_ERR_ARG,
                  "pxs_slat_decoder_pack_load: blocks holds " + std::to_string(max_blocks) +
                      " entries, the model has " + std::to_string(hp.n_blocks));
        rc = upload_all(pack, layout, arena, workspace, as_stream(stream), false);
        if (rc != PXS_OK) return rc;
        // make_weights (src/slat_decoder.cpp:2911-2970).
        Binder b(layout, arena, "SLat decoder");
        const int L = hp.levels;
        io_weights[0] = b.mat32("from_latent.weight", hp.model_channels[0], hp.latent_channels);
        io_weights[1] = b.vec("from_latent.bias", hp.model_channels[0]);
        io_weights[2] = b.mat32("output_layer.weight", hp.out_channels, hp.model_channels[L - 1]);
        io_weights[3] = b.vec("output_layer.bias", hp.out_channels);
        int n = 0;
        for (int l = 0; l < L; ++l) {
            const int64_t C = hp.model_channels[l];
            for (int i = 0; i < hp.num_blocks[l]; ++i) {
                const std::string p = "blocks." + std::to_string(l) + "." + std::to_string(i);
                pxs_decoder_block & k = blocks[n++];
                std::memset(&k, 0, sizeof(k));
                k.kind = PXS_DECODER_CONVNEXT;
                k.channels = static_cast<int>(C);
                k.out_channels = static_cast<int>(C);
                k.mlp_hidden = static_cast<int>(4 * C);
                k.w.norm_weight = b.vec(p + ".norm.weight", C);
                k.w.norm_bias = b.vec(p + ".norm.bias", C);
                k.w.conv1_weight = b.get(p + ".conv.weight", C, C, 27);
                k.w.conv1_bias = b.vec(p + ".conv.bias", C);
                k.w.mlp0_weight = b.get(p + ".mlp.0.weight", 4 * C, C);
                k.w.mlp0_bias = b.vec(p + ".mlp.0.bias", 4 * C);
                k.w.mlp2_weight = b.get(p + ".mlp.2.weight", C, 4 * C);
                k.w.mlp2_bias = b.vec(p + ".mlp.2.bias", C);
            }
            if (l + 1 < L) {
                const int64_t O = hp.model_channels[l + 1];
                const std::string p =
                    "blocks." + std::to_string(l) + "." + std::to_string(hp.num_blocks[l]);
                pxs_decoder_block & k = blocks[n++];
                std::memset(&k, 0, sizeof(k));
                k.kind = PXS_DECODER_C2S;
                k.channels = static_cast<int>(C);
                k.out_channels = static_cast<int>(O);
                k.w.norm1_weight = b.vec(p + ".norm1.weight", C);
                k.w.norm1_bias = b.vec(p + ".norm1.bias", C);
                k.w.conv1_weight = b.get(p + ".conv1.weight", 8 * O, C, 27);
                k.w.conv1_bias = b.vec(p + ".conv1.bias", 8 * O);
                k.w.conv2_weight = b.get(p + ".conv2.weight", O, O, 27);
                k.w.conv2_bias = b.vec(p + ".conv2.bias", O);
                if (hp.pred_subdiv) {
                    k.w.to_subdiv_weight = b.mat32(p + ".to_subdiv.weight", 8, C);
                    k.w.to_subdiv_bias = b.vec(p + ".to_subdiv.bias", 8);
                }
            }
        }
        return b.rc();
    });
}

} // extern "C"
