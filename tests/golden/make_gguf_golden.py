#!/usr/bin/env python3
"""Write the golden GGUF packs with the reference's own converter.

Runs in the build container only: it imports the reference's
scripts/convert_pixal3d_to_gguf.py from /root/reference and drives the
converter's writer (_write_gguf, scripts/convert_pixal3d_to_gguf.py:881-919),
its key/value encoders and metadata builders (232-258, 692-846), its
precision policy (choose_flow_type / choose_decoder_type, 347-359), its
compact name prefixes (TENSOR_NAME_PREFIXES, 70-75) and its format-v1 storage
transform (_tensor_shape_and_value, 392-424: flex_gemm conv weights
[out, 3, 3, 3, in] become [27, out, in]) on small synthetic models, exactly as
convert_component (1080-1111) does for a real checkpoint, then runs the
converter's verify_gguf (952-987) on each file.  The synthetic checkpoints
are the only departure: a full model would not make a small fixture, and the
converter's fixed tensor-count checks (_tensor_specs, 656-666) belong to the
released checkpoints, so the specs are built here with the same helpers.

Outputs (tests/golden/):
  pack_flow_f16.gguf      ElasticSLatFlowModel (shape_flow_1024), ftype 1
                          (F16 matrices; F32 norms, gammas, modulations, vectors)
  pack_flow_bf16.gguf     the same model, ftype 2 (all BF16)
  pack_decoder_f16.gguf   SparseUnetVaeDecoder (texture_decoder), ftype 1
  pack_golden.npz         the float32 source tensors, keyed "flow/<source name>" and
                          "decoder/<source name>"
  pack_golden.json        per pack: component, model args, ftype, and the
                          tensor table the converter planned

Usage:  python tests/golden/make_gguf_golden.py
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

REF_SCRIPTS = Path("/root/reference/scripts")
OUT = Path(__file__).resolve().parent

sys.path.insert(0, str(REF_SCRIPTS))
import convert_pixal3d_to_gguf as cv  # noqa: E402


class Store:
    """The converter's TensorStore interface (keys() sorted, get(name))."""

    def __init__(self, tensors):
        self.tensors = tensors

    def keys(self):
        return tuple(sorted(self.tensors))

    def get(self, name):
        return torch.from_numpy(self.tensors[name].copy())


def normal(rng, shape, std):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def flow_sources(seed, C=16, H=2, CC=16, in_ch=8, out_ch=8, mlp_ratio=4):
    rng = np.random.default_rng(seed)
    M, D = C * mlp_ratio, C // H
    t = {"input_layer.weight": normal(rng, (C, in_ch), 0.3),
         "input_layer.bias": normal(rng, (C,), 0.1),
         "t_embedder.mlp.0.weight": normal(rng, (C, 256), 0.05),
         "t_embedder.mlp.0.bias": normal(rng, (C,), 0.1),
         "t_embedder.mlp.2.weight": normal(rng, (C, C), 0.2),
         "t_embedder.mlp.2.bias": normal(rng, (C,), 0.1),
         "adaLN_modulation.1.weight": normal(rng, (6 * C, C), 0.2),
         "adaLN_modulation.1.bias": normal(rng, (6 * C,), 0.1),
         "out_layer.weight": normal(rng, (out_ch, C), 0.2),
         "out_layer.bias": normal(rng, (out_ch,), 0.1)}
    b = "blocks.0."
    cross = b + "cross_attn.cross_attn_block."
    t.update({b + "modulation": normal(rng, (6 * C,), 0.25),
              b + "self_attn.to_qkv.weight": normal(rng, (3 * C, C), 0.25),
              b + "self_attn.to_qkv.bias": normal(rng, (3 * C,), 0.1),
              b + "self_attn.q_rms_norm.gamma": 1.0 + normal(rng, (H, D), 0.1),
              b + "self_attn.k_rms_norm.gamma": 1.0 + normal(rng, (H, D), 0.1),
              b + "self_attn.to_out.weight": normal(rng, (C, C), 0.25),
              b + "self_attn.to_out.bias": normal(rng, (C,), 0.1),
              b + "norm2.weight": 1.0 + normal(rng, (C,), 0.1),
              b + "norm2.bias": normal(rng, (C,), 0.1),
              cross + "to_q.weight": normal(rng, (C, C), 0.25),
              cross + "to_q.bias": normal(rng, (C,), 0.1),
              cross + "to_kv.weight": normal(rng, (2 * C, CC), 0.25),
              cross + "to_kv.bias": normal(rng, (2 * C,), 0.1),
              cross + "q_rms_norm.gamma": 1.0 + normal(rng, (H, D), 0.1),
              cross + "k_rms_norm.gamma": 1.0 + normal(rng, (H, D), 0.1),
              cross + "to_out.weight": normal(rng, (C, C), 0.25),
              cross + "to_out.bias": normal(rng, (C,), 0.1),
              b + "mlp.mlp.0.weight": normal(rng, (M, C), 0.25),
              b + "mlp.mlp.0.bias": normal(rng, (M,), 0.1),
              b + "mlp.mlp.2.weight": normal(rng, (C, M), 0.12),
              b + "mlp.mlp.2.bias": normal(rng, (C,), 0.1)})
    args = {"resolution": 64, "in_channels": in_ch, "out_channels": out_ch,
            "model_channels": C, "cond_channels": CC, "num_blocks": 1, "num_heads": H,
            "mlp_ratio": float(mlp_ratio), "pe_mode": "rope", "share_mod": True,
            "qk_rms_norm": True, "qk_rms_norm_cross": True, "rope_freq": [1.0, 10000.0],
            "image_attn_mode": "cross"}
    return t, args


def decoder_sources(seed, latent=8, channels=(8, 8), out=6):
    """Two levels: a ConvNeXt block at each level and a channel-to-spatial
    block between them (blocks.<level>.<index>), conv weights in flex_gemm's
    [out, 3, 3, 3, in] source layout."""
    rng = np.random.default_rng(seed)
    C0, C1 = channels
    t = {"from_latent.weight": normal(rng, (C0, latent), 0.3),
         "from_latent.bias": normal(rng, (C0,), 0.1),
         "output_layer.weight": normal(rng, (out, C1), 0.3),
         "output_layer.bias": normal(rng, (out,), 0.1)}
    for level, C in enumerate(channels):
        p = f"blocks.{level}.0."
        t.update({p + "norm.weight": 1.0 + normal(rng, (C,), 0.1),
                  p + "norm.bias": normal(rng, (C,), 0.1),
                  p + "conv.weight": normal(rng, (C, 3, 3, 3, C), (1.0 / (27 * C)) ** 0.5),
                  p + "conv.bias": normal(rng, (C,), 0.1),
                  p + "mlp.0.weight": normal(rng, (4 * C, C), C ** -0.5),
                  p + "mlp.0.bias": normal(rng, (4 * C,), 0.1),
                  p + "mlp.2.weight": normal(rng, (C, 4 * C), (4 * C) ** -0.5),
                  p + "mlp.2.bias": normal(rng, (C,), 0.1)})
    p = "blocks.0.1."
    t.update({p + "norm1.weight": 1.0 + normal(rng, (C0,), 0.1),
              p + "norm1.bias": normal(rng, (C0,), 0.1),
              p + "conv1.weight": normal(rng, (8 * C1, 3, 3, 3, C0), (1.0 / (27 * C0)) ** 0.5),
              p + "conv1.bias": normal(rng, (8 * C1,), 0.1),
              p + "conv2.weight": normal(rng, (C1, 3, 3, 3, C1), (1.0 / (27 * C1)) ** 0.5),
              p + "conv2.bias": normal(rng, (C1,), 0.1),
              p + "to_subdiv.weight": normal(rng, (8, C0), C0 ** -0.5),
              p + "to_subdiv.bias": normal(rng, (8,), 0.5)})
    args = {"model_channels": list(channels), "latent_channels": latent,
            "num_blocks": [1, 1], "block_type": ["SparseConvNeXtBlock3d"] * 2,
            "up_block_type": ["SparseResBlockC2S3d"], "out_channels": out,
            "pred_subdiv": True, "resolution": 16}
    return t, args


def specs_for(definition, store, ftype):
    """TensorSpec list as _tensor_specs (scripts/convert_pixal3d_to_gguf.py:
    623-667) builds it, without the released checkpoints' count checks."""
    specs = []
    prefix = definition.component + "."
    for source_name in store.keys():
        shape, _ = cv._tensor_shape_and_value(store.get(source_name), definition.kind,
                                              source_name)
        if definition.kind in ("ss-flow", "slat-flow"):
            ggml_type = cv.choose_flow_type(source_name, shape, ftype)
        else:
            ggml_type = cv.choose_decoder_type(shape, ftype)
        name = prefix + source_name
        for long_prefix, short in cv.TENSOR_NAME_PREFIXES:
            if name.startswith(long_prefix):
                name = short + name[len(long_prefix):]
                break
        specs.append(cv.TensorSpec(name, definition.key, source_name, definition.kind,
                                   ggml_type, tuple(reversed(shape)), shape,
                                   cv._element_count(shape) * cv._bytes_per_type(ggml_type)))
    return specs


def write_component(path, definition, store, args, ftype):
    """convert_component (scripts/convert_pixal3d_to_gguf.py:1080-1111)."""
    specs = specs_for(definition, store, ftype)
    metadata = cv._base_metadata(cv.PIXAL3D_ARCH, definition.stem, ftype)
    metadata += [cv.kv_u32(cv.PIXAL3D_PREFIX + "bundle_format", cv.PIXAL3D_BUNDLE_FORMAT),
                 cv.kv_str(cv.PIXAL3D_PREFIX + "tensor_name_scheme",
                           cv.PIXAL3D_TENSOR_NAME_SCHEME),
                 cv.kv_str(cv.PIXAL3D_PREFIX + "bundle_kind", "component"),
                 cv.kv_u32(cv.PIXAL3D_PREFIX + "component_count", 1),
                 cv.kv_str(cv.PIXAL3D_PREFIX + "component.0", definition.component)]
    metadata += cv._model_metadata(definition, args,
                                   cv.PIXAL3D_PREFIX + definition.component + ".")
    cv._write_gguf(path, metadata, specs, {definition.key: store}, True)
    cv.verify_gguf(path, specs)
    return specs


def main():
    flow_t, flow_args = flow_sources(11)
    dec_t, dec_args = decoder_sources(12)
    packs = [("pack_flow_f16", "flow", cv.MODELS["shape-flow-1024"], flow_t, flow_args, 1),
             ("pack_flow_bf16", "flow", cv.MODELS["shape-flow-1024"], flow_t, flow_args, 2),
             ("pack_decoder_f16", "decoder", cv.MODELS["tex-dec"], dec_t, dec_args, 1)]
    arrays, meta = {}, {}
    for stem, source, definition, tensors, args, ftype in packs:
        specs = write_component(OUT / (stem + ".gguf"), definition, Store(tensors), args, ftype)
        for name, a in tensors.items():
            arrays[f"{source}/{name}"] = a
        meta[stem] = {"file": stem + ".gguf", "sources": source,
                      "component": definition.component,
                      "stem": definition.stem, "model_class": definition.expected_class,
                      "variant": definition.variant, "ftype": ftype, "args": args,
                      "tensors": [{"name": s.name, "source": s.source_name,
                                   "ggml_type": s.ggml_type, "dims": list(s.dims),
                                   "nbytes": s.nbytes} for s in specs]}
        print(f"wrote {stem}.gguf ({(OUT / (stem + '.gguf')).stat().st_size} bytes, "
              f"{len(specs)} tensors)")
    np.savez_compressed(OUT / "pack_golden.npz", **arrays)
    (OUT / "pack_golden.json").write_text(json.dumps(meta, indent=1) + "\n")


if __name__ == "__main__":
    main()
