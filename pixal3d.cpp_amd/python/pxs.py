"""ctypes binding of libpxs.so (the C ABI in include/pxs.h) over torch tensors.

torch supplies device memory and the current HIP stream; every computation
runs in the HIP kernels of libpxs.so.  There is no fallback: if the library
is missing or a call fails, a PxsError is raised.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np
import torch

PKG = Path(__file__).resolve().parents[1]
LIB_PATH = Path(os.environ.get("PXS_LIB", PKG / "lib" / "libpxs.so"))

PXS_OK, PXS_ERR_ARG, PXS_ERR_HIP, PXS_ERR_DATA = 0, 1, 2, 3
PXS_F32, PXS_BF16 = 0, 1
PXS_ATTN_NOALLOC_MAX_SEGMENTS = 65536
ACT_NONE, ACT_GELU_TANH, ACT_SILU = 0, 1, 2

VALIDATION_MESSAGES = {
    4: "sparse coordinate is outside its shape",
    5: "sparse coordinates contain a duplicate point",
    6: "sparse coordinates must be contiguous by batch",
    7: "sparse features contain a non-finite value",
}


class PxsError(RuntimeError):
    pass


_vp, _i64, _i32, _f = C.c_void_p, C.c_int64, C.c_int, C.c_float

# name -> (restype, argtypes)
_SIGS = {
    "pxs_last_error": (C.c_char_p, []),
    "pxs_version": (_i32, []),
    "pxs_voxel_hash_bytes": (C.c_size_t, [_i64]),
    "pxs_voxel_hash_build": (_i32, [_vp, _i64, _vp, _vp]),
    "pxs_sparse_validate": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _vp]),
    "pxs_validation_message": (C.c_char_p, [_i32]),
    "pxs_neighbor_map_k3": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp]),
    "pxs_neighbor_pairs_workspace_bytes": (C.c_size_t, [_i64]),
    "pxs_neighbor_pairs": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _vp]),
    "pxs_subm_conv3d": (_i32, [_i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "pxs_subm_conv3d_grid": (_i32, [_i32, _vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _i32,
                                    _i32, _vp, C.c_uint32, _vp, _vp]),
    "pxs_status_reset": (_i32, [_vp, _vp]),
    "pxs_check_finite": (_i32, [_i32, _vp, _i64, _i32, _i64, _vp, _vp]),
    "pxs_value_stats_workspace_bytes": (C.c_size_t, [_i64]),
    "pxs_value_stats_f32": (_i32, [_vp, _i64, _vp, _vp, _vp]),
    "pxs_downsample_workspace_bytes": (C.c_size_t, [_i64, _i32, _i32, _i32, _i32, _i32]),
    "pxs_downsample_topology": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                       _vp, _vp]),
    "pxs_downsample_mean": (_i32, [_i32, _vp, _i32, _vp, _vp, _i64, _vp, _vp]),
    "pxs_downsample_s2_topology": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "pxs_sparse_conv3d_s2": (_i32, [_i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _i64, _i64, _vp, _vp]),
    "pxs_channel_to_spatial_workspace_bytes": (C.c_size_t, [_i64, _i32]),
    "pxs_channel_to_spatial": (_i32, [_i32, _vp, _i64, _vp, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                      _vp]),
    "pxs_linear_residual": (_i32, [_i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp]),
    "pxs_convert": (_i32, [_i32, _vp, _i64, _i32, _vp, _vp]),
    "pxs_timestep_embedding": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp]),
    "pxs_transformer_block_workspace_bytes": (C.c_size_t, [_i32, _vp, _i64, _i64, _i32]),
    "pxs_transformer_block": (_i32, [_i32, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp,
                                     _i64, _vp, _vp, _vp]),
    "pxs_slat_flow_workspace_bytes": (C.c_size_t, [_i32, _vp, _i64, _i64, _i32]),
    "pxs_linear_ordered": (_i32, [_vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp]),
    "pxs_slat_decoder_workspace_bytes": (C.c_size_t, [_i32, _vp, _vp, _i32, _i64, _i64]),
    "pxs_slat_decoder_forward": (_i32, [_i32, _vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _i64, _vp,
                                        _vp, _vp, _i32, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    "pxs_flow_sampler_schedule": (_i32, [_vp, _i32, _vp, _vp, _vp]),
    "pxs_flow_guidance_workspace_bytes": (C.c_size_t, [_i32]),
    "pxs_flow_guidance": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _f, _f, _f, _f, _vp,
                                 _vp, _vp]),
    "pxs_flow_pred_to_xstart": (_i32, [_vp, _vp, _i64, _f, _f, _vp, _vp]),
    "pxs_flow_euler_update": (_i32, [_vp, _vp, _i64, _f, _vp]),
    "pxs_flow_euler_sample_workspace_bytes": (C.c_size_t, [_i32, _vp, _i64, _i64, _i64, _i32]),
    "pxs_flow_euler_sample": (_i32, [_i32, _vp, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp,
                                     _i64, _vp, _vp, _i64, _vp, _vp, _vp]),
    "pxs_slat_flow_forward": (_i32, [_i32, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp,
                                     _i64, _vp, _vp, _vp, _vp]),
    "pxs_linear": (_i32, [_i32, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _vp, _vp]),
    "pxs_linear_gate_residual": (_i32, [_i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _vp, _vp]),
    "pxs_layer_norm": (_i32, [_i32, _vp, _i64, _i32, _f, _vp, _vp, _i32, _vp, _vp]),
    "pxs_layer_norm_modulate": (_i32, [_i32, _vp, _i64, _i32, _f, _vp, _vp, _vp, _i32, _i32, _vp, _vp]),
    "pxs_mh_rms_norm": (_i32, [_i32, _vp, _i64, _i64, _i32, _i32, _vp, _vp, _i64, _vp]),
    "pxs_rope": (_i32, [_i32, _vp, _vp, _i64, _i64, _i32, _i32, _f, _f, _vp, _i64, _vp]),
    "pxs_qkv_prepare": (_i32, [_i32, _vp, _i64, _i32, _i32, _vp, _vp, _vp, _f, _f, _vp, _vp, _vp, _vp]),
    "pxs_activation": (_i32, [_i32, _vp, _i64, _i32, _vp]),
    "pxs_attention_workspace_bytes": (C.c_size_t, [_i32]),
    "pxs_varlen_attention": (_i32, [_i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i32, _i64, _vp,
                                    _i32, _i32, _i32, _f, _vp, _i64, _vp, _vp]),
    "pxs_varlen_attention_noalloc": (_i32, [_i32, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i32,
                                            _i64, _vp, _i32, _i32, _i32, _f, _vp, _i64, _vp]),
    "pxs_batch_cu_seqlens": (_i32, [_vp, _i64, _i32, _vp, _vp]),
    "pxs_window_partition_workspace_bytes": (C.c_size_t, [_i32, _i32, _i32, _i32, _i32, _i32, _i64]),
    "pxs_window_partition": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                    _vp, _vp]),
    "pxs_voxel_grid_bytes": (C.c_size_t, [_i32, _i32, _i32, _i32]),
    "pxs_voxel_grid_tagged_bytes": (C.c_size_t, [_i32, _i32, _i32, _i32]),
    "pxs_voxel_grid_tagged_reset": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
    "pxs_voxel_grid_tagged_insert": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, C.c_uint32,
                                            _vp]),
    "pxs_neighbor_map_k3_grid_tagged": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, C.c_uint32,
                                               _vp, _vp, _vp]),
    "pxs_downsample_s2_tagged_workspace_bytes": (C.c_size_t, [_i32, _i32, _i32, _i32]),
    "pxs_downsample_s2_tagged_workspace_reset": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
    "pxs_downsample_s2_topology_tagged": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _vp,
                                                 C.c_uint32, _vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "pxs_map_s2_topology_tagged": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, C.c_uint32,
                                          _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "pxs_s2_tagged_insert": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, C.c_uint32, _vp,
                                    _vp]),
    "pxs_subm_conv3d_grid_s2_emit": (_i32, [_i32, _vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32,
                                            _i32, _i32, _i32, _vp, C.c_uint32, _vp, _vp, _vp,
                                            _i64, _vp, _vp, _vp, _vp]),
    "pxs_s2_tagged_emit": (_i32, [_i64, _i32, _i32, _i32, _i32, _vp, C.c_uint32, _vp, _vp, _i64,
                                  _vp, _vp, _vp, _vp]),
    "pxs_unet_s2_level": (_i32, [_i32, _vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _i32,
                                 _i32, _vp, C.c_uint32, _vp, _vp, _vp, _i32, _i64, _vp, _vp, _vp,
                                 _i64, _vp, _vp, _vp, _vp]),
    "pxs_unet_s2_level_error": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp, _vp]),
    "pxs_voxel_bricks_bytes": (C.c_size_t, [_i64]),
    "pxs_voxel_bricks_build": (_i32, [_vp, _i64, _vp, _vp]),
    "pxs_neighbor_map_k3_bricks": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp]),
    "pxs_voxel_grid_build": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp]),
    "pxs_neighbor_map_k3_grid": (_i32, [_vp, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "pxs_convnext_block_workspace_bytes": (C.c_size_t, [_i32, _i64, _i32, _i32, _i32]),
    "pxs_convnext_block": (_i32, [_i32, _vp, _i64, _vp, _i32, _i32, _f, _vp, _vp, _vp, _vp, _vp,
                                  _vp]),
    "pxs_resblock_c2s_workspace_bytes": (C.c_size_t, [_i32, _i64, _i32, _i32]),
    "pxs_resblock_c2s": (_i32, [_i32, _vp, _i64, _vp, _i32, _i32, _f, _vp, _i32, _vp, _vp, _vp,
                                _vp, _vp, _vp, _vp]),
    "pxs_add_repeat": (_i32, [_i32, _vp, _i64, _i32, _vp, _i32, _vp, _vp]),
    "pxs_pack_open": (_i32, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "pxs_pack_close": (None, [_vp]),
    "pxs_pack_describe": (C.c_size_t, [_vp, C.c_char_p, C.c_size_t]),
    "pxs_pack_metadata_u32": (_i32, [_vp, C.c_char_p, _i32, C.POINTER(C.c_uint32)]),
    "pxs_pack_metadata_f32": (_i32, [_vp, C.c_char_p, _i32, C.POINTER(C.c_float)]),
    "pxs_pack_metadata_bool": (_i32, [_vp, C.c_char_p, _i32, C.POINTER(C.c_int)]),
    "pxs_pack_metadata_string": (_i32, [_vp, C.c_char_p, _i32, C.c_char_p, C.c_size_t]),
    "pxs_pack_read_tensor": (_i32, [_vp, C.c_char_p, _vp, C.c_size_t, C.POINTER(C.c_size_t)]),
    "pxs_pack_upload_workspace_bytes": (C.c_size_t, [_vp]),
    "pxs_pack_upload": (_i32, [_vp, C.c_char_p, _i32, _vp, _i64, _vp, _vp]),
    "pxs_slat_flow_pack_plan": (_i32, [_vp, C.c_char_p, _i32, _vp, _vp]),
    "pxs_slat_flow_pack_load": (_i32, [_vp, C.c_char_p, _i32, _vp, C.c_size_t, _vp, _vp, _vp,
                                       _i32, _vp]),
    "pxs_slat_decoder_pack_plan": (_i32, [_vp, C.c_char_p, _i32, _vp, _vp]),
    "pxs_slat_decoder_pack_load": (_i32, [_vp, C.c_char_p, _i32, _vp, C.c_size_t, _vp, _vp,
                                          _i32, _vp, _vp]),
}


BLOCK_WEIGHT_FIELDS = (
    "modulation", "self_to_qkv_weight", "self_to_qkv_bias", "self_q_gamma", "self_k_gamma",
    "self_to_out_weight", "self_to_out_bias", "norm2_weight", "norm2_bias", "cross_to_q_weight",
    "cross_to_q_bias", "cross_to_kv_weight", "cross_to_kv_bias", "cross_q_gamma",
    "cross_k_gamma", "cross_to_out_weight", "cross_to_out_bias", "proj_weight", "proj_bias",
    "mlp0_weight", "mlp0_bias", "mlp2_weight", "mlp2_bias")
# Members that are linear weights (stored in the call's dtype); the rest are fp32.
BLOCK_LINEAR_WEIGHTS = frozenset({1, 5, 9, 11, 15, 17, 19, 21})


class BlockConfig(C.Structure):
    _fields_ = [("channels", C.c_int), ("num_heads", C.c_int), ("mlp_hidden", C.c_int),
                ("context_channels", C.c_int), ("proj_in_channels", C.c_int),
                ("norm_eps", C.c_float), ("rope_freq_min", C.c_float),
                ("rope_freq_base", C.c_float), ("use_rope", C.c_int), ("qk_rms_norm", C.c_int),
                ("qk_rms_norm_cross", C.c_int), ("use_projection", C.c_int)]


class BlockWeights(C.Structure):
    _fields_ = [(name, C.c_void_p) for name in BLOCK_WEIGHT_FIELDS]


class FlowConfig(C.Structure):
    _fields_ = [("in_channels", C.c_int), ("out_channels", C.c_int), ("model_channels", C.c_int),
                ("cond_channels", C.c_int), ("num_blocks", C.c_int), ("num_heads", C.c_int),
                ("proj_in_channels", C.c_int), ("mlp_hidden", C.c_int), ("norm_eps", C.c_float),
                ("rope_freq_min", C.c_float), ("rope_freq_base", C.c_float),
                ("qk_rms_norm", C.c_int), ("qk_rms_norm_cross", C.c_int),
                ("use_projection", C.c_int)]


class SamplerConfig(C.Structure):
    """pxs_flow_sampler_config (FlowEulerSamplerConfig without the trajectory flag)."""
    _fields_ = [("steps", C.c_int), ("sigma_min", C.c_float), ("rescale_t", C.c_float),
                ("guidance_strength", C.c_float), ("guidance_rescale", C.c_float),
                ("guidance_interval_min", C.c_float), ("guidance_interval_max", C.c_float)]


class FlowWeights(C.Structure):
    _fields_ = [(name, C.c_void_p) for name in (
        "input_weight", "input_bias", "timestep_weight0", "timestep_bias0", "timestep_weight2",
        "timestep_bias2", "modulation_weight", "modulation_bias", "output_weight",
        "output_bias")] + [("blocks", C.POINTER(BlockWeights))]


DECODER_WEIGHT_FIELDS = (
    "norm_weight", "norm_bias", "norm1_weight", "norm1_bias", "conv1_weight", "conv1_bias",
    "norm2_weight", "norm2_bias", "conv2_weight", "conv2_bias", "mlp0_weight", "mlp0_bias",
    "mlp2_weight", "mlp2_bias", "to_subdiv_weight", "to_subdiv_bias")
# Members stored in the call's dtype (convolution and ConvNeXt MLP weights).
DECODER_DTYPE_WEIGHTS = frozenset({"conv1_weight", "conv2_weight", "mlp0_weight", "mlp2_weight"})


class DecoderBlockWeights(C.Structure):
    _fields_ = [(name, C.c_void_p) for name in DECODER_WEIGHT_FIELDS]


PXS_DECODER_CONVNEXT = 0
PXS_DECODER_C2S = 1


class DecoderBlock(C.Structure):
    """pxs_decoder_block: one entry of SLatDecoderWeightsF32::blocks."""
    _fields_ = [("kind", C.c_int), ("channels", C.c_int), ("out_channels", C.c_int),
                ("mlp_hidden", C.c_int), ("w", DecoderBlockWeights)]


class DecoderConfig(C.Structure):
    """pxs_decoder_config (SLatDecoderConfig); keep the channel arrays alive."""
    _fields_ = [("latent_channels", C.c_int), ("out_channels", C.c_int), ("norm_eps", C.c_float),
                ("pred_subdiv", C.c_int), ("levels", C.c_int),
                ("model_channels", C.POINTER(C.c_int)), ("num_blocks", C.POINTER(C.c_int))]


def decoder_config(latent, out, eps, pred_subdiv, model_channels, num_blocks):
    mc = (C.c_int * len(model_channels))(*model_channels)
    nb = (C.c_int * len(num_blocks))(*num_blocks)
    cfg = DecoderConfig(latent, out, eps, int(pred_subdiv), len(model_channels), mc, nb)
    cfg._keep = (mc, nb)
    return cfg


def decoder_block_weights(tensors: dict) -> DecoderBlockWeights:
    """Device tensors by DECODER_WEIGHT_FIELDS name; missing names are NULL."""
    return DecoderBlockWeights(*[tensors[k].data_ptr() if tensors.get(k) is not None else None
                                 for k in DECODER_WEIGHT_FIELDS])


def block_weights(tensors) -> BlockWeights:
    """23 device tensors (or None) in BLOCK_WEIGHT_FIELDS order."""
    return BlockWeights(*[None if t is None else t.data_ptr() for t in tensors])


PXS_DECODER_MAX_LEVELS = 16


class DecoderHParams(C.Structure):
    """pxs_decoder_hparams (SLatDecoderHParams)."""
    _fields_ = [("resolution", C.c_int), ("latent_channels", C.c_int),
                ("out_channels", C.c_int), ("levels", C.c_int), ("pred_subdiv", C.c_int),
                ("n_blocks", C.c_int), ("norm_eps", C.c_float),
                ("model_channels", C.c_int * PXS_DECODER_MAX_LEVELS),
                ("num_blocks", C.c_int * PXS_DECODER_MAX_LEVELS)]


def load_library(path: Path = LIB_PATH) -> C.CDLL:
    if not Path(path).exists():
        raise PxsError(f"{path} is not built (run __graft_entry__.build())")
    lib = C.CDLL(str(path))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _ptr(t):
    """A device pointer argument: a tensor, a raw address (int) or None."""
    if t is None:
        return None
    return C.c_void_p(t if isinstance(t, int) else t.data_ptr())


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return PXS_F32
    if t.dtype == torch.bfloat16:
        return PXS_BF16
    raise PxsError(f"unsupported dtype {t.dtype}")


class Pxs:
    """Thin wrappers: allocate outputs with torch, call the C ABI on the current stream."""

    def __init__(self, path: Path = LIB_PATH):
        self.lib = load_library(path)
        self.path = Path(path)

    # -- plumbing ---------------------------------------------------------------
    @staticmethod
    def stream():
        return C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def _check(self, rc: int, what: str):
        if rc != 0:
            raise PxsError(f"{what}: {self.lib.pxs_last_error().decode()} (code {rc})")

    @staticmethod
    def _ws(nbytes: int, device) -> torch.Tensor:
        return torch.empty(max(int(nbytes), 8), dtype=torch.uint8, device=device)

    # -- topology -----------------------------------------------------------------
    def hash_build(self, coords: torch.Tensor) -> torch.Tensor:
        n = coords.shape[0]
        table = self._ws(self.lib.pxs_voxel_hash_bytes(n), coords.device)
        self._check(self.lib.pxs_voxel_hash_build(_ptr(coords), n, _ptr(table), self.stream()),
                    "pxs_voxel_hash_build")
        return table

    def validate(self, coords, batch_size, shape, feats=None, table=None):
        n = coords.shape[0]
        table = self.hash_build(coords) if table is None else table
        status = torch.empty(1, dtype=torch.int64, device=coords.device)
        dt = PXS_F32 if feats is None else _dtype_code(feats)
        ch = 0 if feats is None else feats.shape[1]
        self._check(self.lib.pxs_sparse_validate(_ptr(coords), n, batch_size, shape[0], shape[1],
                                                 shape[2], dt, _ptr(feats), ch, _ptr(table),
                                                 _ptr(status), self.stream()),
                    "pxs_sparse_validate")
        s = int(status.item())
        if s == (1 << 63) - 1:
            return 0, -1
        return s % 8, s // 8

    def neighbor_map(self, coords, table=None, want_masks=True):
        n = coords.shape[0]
        table = self.hash_build(coords) if table is None else table
        nbr = torch.empty((27, n), dtype=torch.int32, device=coords.device)
        masks = torch.empty(n, dtype=torch.int32, device=coords.device) if want_masks else None
        self._check(self.lib.pxs_neighbor_map_k3(_ptr(coords), n, _ptr(table), _ptr(nbr),
                                                 _ptr(masks), self.stream()),
                    "pxs_neighbor_map_k3")
        return nbr, masks

    def neighbor_map_bricks(self, coords, want_masks=True):
        """pxs_voxel_bricks_build + pxs_neighbor_map_k3_bricks -> (nbr [27, n], masks [n])."""
        n = coords.shape[0]
        table = self._ws(self.lib.pxs_voxel_bricks_bytes(n), coords.device)
        self._check(self.lib.pxs_voxel_bricks_build(_ptr(coords), n, _ptr(table), self.stream()),
                    "pxs_voxel_bricks_build")
        nbr = torch.empty((27, max(n, 1)), dtype=torch.int32, device=coords.device)
        masks = torch.empty(max(n, 1), dtype=torch.int32, device=coords.device) if want_masks \
            else None
        self._check(self.lib.pxs_neighbor_map_k3_bricks(_ptr(coords), n, _ptr(table), _ptr(nbr),
                                                        _ptr(masks), self.stream()),
                    "pxs_neighbor_map_k3_bricks")
        return nbr[:, :n], (masks[:n] if masks is not None else None)

    def grid_build(self, coords, batch_size, shape):
        nbytes = self.lib.pxs_voxel_grid_bytes(batch_size, *shape)
        grid = torch.empty(max(nbytes // 4, 1), dtype=torch.int32, device=coords.device)
        self._check(self.lib.pxs_voxel_grid_build(_ptr(coords), coords.shape[0], batch_size,
                                                  *shape, _ptr(grid), self.stream()),
                    "pxs_voxel_grid_build")
        return grid

    # -- generation-tagged grids ---------------------------------------------------
    def tagged_grid(self, batch_size, shape, device="cuda"):
        """A reset tagged voxel grid for these extents."""
        nbytes = self.lib.pxs_voxel_grid_tagged_bytes(batch_size, *shape)
        grid = torch.empty(max(nbytes // 8, 1), dtype=torch.int64, device=device)
        self._check(self.lib.pxs_voxel_grid_tagged_reset(_ptr(grid), batch_size, *shape,
                                                         self.stream()),
                    "pxs_voxel_grid_tagged_reset")
        return grid

    def tagged_insert(self, coords, batch_size, shape, grid, generation):
        self._check(self.lib.pxs_voxel_grid_tagged_insert(_ptr(coords), coords.shape[0],
                                                          batch_size, *shape, _ptr(grid),
                                                          generation, self.stream()),
                    "pxs_voxel_grid_tagged_insert")

    def map_s2_tagged(self, coords, batch_size, shape, grid, generation, coarse_grid, workspace,
                      sync=True, with_map=True):
        """pxs_map_s2_topology_tagged -> (nbr [27, n], masks [n], out_coords,
        child_map [8, n], m); m is the host count when sync (else the device
        int64).  with_map=False builds no map (nbr and masks None)."""
        n = coords.shape[0]
        dev = coords.device
        nbr = torch.empty((27, max(n, 1)), dtype=torch.int32, device=dev) if with_map else None
        masks = torch.empty(max(n, 1), dtype=torch.int32, device=dev) if with_map else None
        oc = torch.empty((max(n, 1), 4), dtype=torch.int32, device=dev)
        child = torch.empty((8, max(n, 1)), dtype=torch.int32, device=dev)
        m = torch.empty(1, dtype=torch.int64, device=dev)
        self._check(self.lib.pxs_map_s2_topology_tagged(
            _ptr(coords), n, batch_size, *shape, _ptr(grid), generation, _ptr(nbr), _ptr(masks),
            _ptr(oc), _ptr(child), child.shape[1], _ptr(m), _ptr(coarse_grid), _ptr(workspace),
            self.stream()), "pxs_map_s2_topology_tagged")
        if with_map:
            nbr, masks = nbr[:, :n], masks[:n]
        if not sync:
            return nbr, masks, oc, child, m
        mm = int(m.item())
        return nbr, masks, oc[:mm], child, mm

    def neighbor_map_tagged(self, coords, batch_size, shape, grid, generation):
        n = coords.shape[0]
        nbr = torch.empty((27, max(n, 1)), dtype=torch.int32, device=coords.device)
        masks = torch.empty(max(n, 1), dtype=torch.int32, device=coords.device)
        self._check(self.lib.pxs_neighbor_map_k3_grid_tagged(_ptr(coords), n, batch_size, *shape,
                                                             _ptr(grid), generation, _ptr(nbr),
                                                             _ptr(masks), self.stream()),
                    "pxs_neighbor_map_k3_grid_tagged")
        return nbr[:, :n], masks[:n]

    def s2_tagged_workspace(self, batch_size, shape, device="cuda"):
        """A workspace for pxs_downsample_s2_topology_tagged with its bitmap zeroed."""
        nbytes = self.lib.pxs_downsample_s2_tagged_workspace_bytes(batch_size, *shape)
        ws = self._ws(nbytes, device)
        self._check(self.lib.pxs_downsample_s2_tagged_workspace_reset(_ptr(ws), batch_size, *shape,
                                                                      self.stream()),
                    "pxs_downsample_s2_tagged_workspace_reset")
        return ws

    def downsample_s2_tagged(self, coords, batch_size, shape, fine_grid, fine_gen, coarse_grid,
                             workspace, sync=True):
        """-> (out_coords, child_map [8, n], m); m is the host count when sync
        (else the device int64).  coarse_grid (a plain voxel grid of the
        halved extents) is rewritten whole."""
        n = coords.shape[0]
        dev = coords.device
        oc = torch.empty((max(n, 1), 4), dtype=torch.int32, device=dev)
        child = torch.empty((8, max(n, 1)), dtype=torch.int32, device=dev)
        m = torch.empty(1, dtype=torch.int64, device=dev)
        self._check(self.lib.pxs_downsample_s2_topology_tagged(
            _ptr(coords), n, batch_size, *shape, _ptr(fine_grid), fine_gen, _ptr(oc), _ptr(child),
            child.shape[1], _ptr(m), _ptr(coarse_grid), _ptr(workspace),
            self.stream()), "pxs_downsample_s2_topology_tagged")
        if not sync:
            return oc, child, m
        mm = int(m.item())
        return oc[:mm], child, mm

    def neighbor_map_grid(self, coords, batch_size, shape, grid=None, want_masks=True):
        """pxs_voxel_grid_build + pxs_neighbor_map_k3_grid -> (nbr [27, n], masks [n])."""
        n = coords.shape[0]
        grid = self.grid_build(coords, batch_size, shape) if grid is None else grid
        nbr = torch.empty((27, max(n, 1)), dtype=torch.int32, device=coords.device)
        masks = torch.empty(max(n, 1), dtype=torch.int32, device=coords.device) if want_masks \
            else None
        self._check(self.lib.pxs_neighbor_map_k3_grid(_ptr(coords), n, batch_size, *shape,
                                                      _ptr(grid), _ptr(nbr), _ptr(masks),
                                                      self.stream()),
                    "pxs_neighbor_map_k3_grid")
        return nbr[:, :n], (masks[:n] if masks is not None else None)

    def neighbor_pairs(self, nbr):
        n = nbr.shape[1]
        dev = nbr.device
        pin = torch.empty(max(27 * n, 1), dtype=torch.int32, device=dev)
        pout = torch.empty(max(27 * n, 1), dtype=torch.int32, device=dev)
        offs = torch.empty(28, dtype=torch.int64, device=dev)
        ws = self._ws(self.lib.pxs_neighbor_pairs_workspace_bytes(n), dev)
        self._check(self.lib.pxs_neighbor_pairs(_ptr(nbr), n, _ptr(pin), _ptr(pout), _ptr(offs),
                                                _ptr(ws), self.stream()),
                    "pxs_neighbor_pairs")
        total = int(offs[27].item())
        return pin[:total], pout[:total], offs

    def batch_cu_seqlens(self, coords, batch_size):
        cu = torch.empty(batch_size + 1, dtype=torch.int64, device=coords.device)
        self._check(self.lib.pxs_batch_cu_seqlens(_ptr(coords), coords.shape[0], batch_size,
                                                  _ptr(cu), self.stream()),
                    "pxs_batch_cu_seqlens")
        return cu

    def downsample_s2(self, coords, batch_size, shape):
        n = coords.shape[0]
        dev = coords.device
        oc = torch.empty((max(n, 1), 4), dtype=torch.int32, device=dev)
        child = torch.empty((8, max(n, 1)), dtype=torch.int32, device=dev)
        m = torch.empty(1, dtype=torch.int64, device=dev)
        ws = self._ws(self.lib.pxs_downsample_workspace_bytes(n, batch_size, *shape, 2), dev)
        self._check(self.lib.pxs_downsample_s2_topology(_ptr(coords), n, batch_size, shape[0],
                                                        shape[1], shape[2], _ptr(oc), _ptr(child),
                                                        _ptr(m), _ptr(ws), self.stream()),
                    "pxs_downsample_s2_topology")
        mm = int(m.item())
        return oc[:mm], child, mm

    def downsample(self, coords, batch_size, shape, factor):
        """Factor-f output topology as groups: (coords, offsets, rows, m)."""
        n = coords.shape[0]
        dev = coords.device
        oc = torch.empty((max(n, 1), 4), dtype=torch.int32, device=dev)
        off = torch.empty(n + 1, dtype=torch.int64, device=dev)
        rows = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
        m = torch.empty(1, dtype=torch.int64, device=dev)
        ws = self._ws(self.lib.pxs_downsample_workspace_bytes(n, batch_size, *shape, factor), dev)
        self._check(self.lib.pxs_downsample_topology(_ptr(coords), n, batch_size, shape[0],
                                                     shape[1], shape[2], factor, _ptr(oc),
                                                     _ptr(off), _ptr(rows), _ptr(m), _ptr(ws),
                                                     self.stream()),
                    "pxs_downsample_topology")
        mm = int(m.item())
        return oc[:mm], off[: mm + 1], rows[:n], mm

    def window_partition(self, coords, batch_size, shape, window, shift, sync=True):
        """-> (fwd, bwd, cu, nseg).  sync=False skips reading the window count:
        nseg is then the host bound min(n, windows) and cu ends in empty
        segments."""
        n = coords.shape[0]
        dev = coords.device
        fwd = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
        bwd = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
        cu = torch.empty(n + 1, dtype=torch.int64, device=dev)
        nwin = torch.empty(1, dtype=torch.int64, device=dev)
        ws = self._ws(self.lib.pxs_window_partition_workspace_bytes(batch_size, *shape, window,
                                                                    shift, n), dev)
        self._check(self.lib.pxs_window_partition(_ptr(coords), n, batch_size, shape[0], shape[1],
                                                  shape[2], window, shift, _ptr(fwd), _ptr(bwd),
                                                  _ptr(cu), _ptr(nwin), _ptr(ws), self.stream()),
                    "pxs_window_partition")
        if not sync:
            grid = [(e + shift + window - 1) // window for e in shape]
            cap = min(n, batch_size * grid[0] * grid[1] * grid[2])
            return fwd[:n], bwd[:n], cu[: cap + 1], cap
        nw = int(nwin.item())
        return fwd[:n], bwd[:n], cu[: nw + 1], nw

    def channel_to_spatial(self, coords, x, subdivision=None, factor=2):
        n, ch = x.shape
        cc = factor ** 3
        dev = x.device
        oc = torch.empty((max(cc * n, 1), 4), dtype=torch.int32, device=dev)
        y = torch.empty((max(cc * n, 1), ch // cc), dtype=x.dtype, device=dev)
        m = torch.empty(1, dtype=torch.int64, device=dev)
        ws = self._ws(self.lib.pxs_channel_to_spatial_workspace_bytes(n, factor), dev)
        self._check(self.lib.pxs_channel_to_spatial(_dtype_code(x), _ptr(coords), n, _ptr(x), ch,
                                                    factor, _ptr(subdivision), _ptr(oc), _ptr(y),
                                                    _ptr(m), _ptr(ws), self.stream()),
                    "pxs_channel_to_spatial")
        mm = int(m.item())
        return oc[:mm], y[:mm]

    # -- GEMM family ----------------------------------------------------------------
    def subm_conv3d(self, x, weight, bias, nbr, masks=None, out=None):
        n, cin = x.shape
        cout = weight.shape[1]
        y = torch.empty((n, cout), dtype=x.dtype, device=x.device) if out is None else out
        self._check(self.lib.pxs_subm_conv3d(_dtype_code(x), _ptr(x), n, cin, _ptr(weight),
                                             _ptr(bias), cout, _ptr(nbr), _ptr(masks), _ptr(y),
                                             self.stream()),
                    "pxs_subm_conv3d")
        return y

    def subm_conv3d_grid(self, x, weight, bias, coords, batch_size, shape, grid, generation=0,
                         out=None):
        """pxs_subm_conv3d_grid: neighbours looked up in a dense voxel grid
        (generation 0: plain grid; 1..255: tagged)."""
        n, cin = x.shape
        cout = weight.shape[1]
        y = torch.empty((n, cout), dtype=x.dtype, device=x.device) if out is None else out
        self._check(self.lib.pxs_subm_conv3d_grid(_dtype_code(x), _ptr(x), _ptr(coords), n, cin,
                                                  _ptr(weight), _ptr(bias), cout, batch_size,
                                                  *shape, _ptr(grid), generation, _ptr(y),
                                                  self.stream()),
                    "pxs_subm_conv3d_grid")
        return y

    def s2_tagged_insert(self, coords, batch_size, shape, grid, generation, workspace):
        """pxs_s2_tagged_insert: rows into the tagged grid, their stride-2
        cells marked in the workspace's generation-tagged bitmap."""
        self._check(self.lib.pxs_s2_tagged_insert(_ptr(coords), coords.shape[0], batch_size,
                                                  *shape, _ptr(grid), generation, _ptr(workspace),
                                                  self.stream()), "pxs_s2_tagged_insert")

    def _s2_outputs(self, n, dev):
        oc = torch.empty((max(n, 1), 4), dtype=torch.int32, device=dev)
        child = torch.empty((8, max(n, 1)), dtype=torch.int32, device=dev)
        m = torch.empty(1, dtype=torch.int64, device=dev)
        return oc, child, m

    def subm_conv3d_grid_s2_emit(self, x, weight, bias, coords, batch_size, shape, grid,
                                 generation, coarse_grid, workspace, out=None, s2_out=None):
        """pxs_subm_conv3d_grid_s2_emit -> (y, out_coords, child_map [8, n],
        m as a device int64)."""
        n, cin = x.shape
        cout = weight.shape[1]
        y = torch.empty((n, cout), dtype=x.dtype, device=x.device) if out is None else out
        oc, child, m = self._s2_outputs(n, x.device) if s2_out is None else s2_out
        self._check(self.lib.pxs_subm_conv3d_grid_s2_emit(
            _dtype_code(x), _ptr(x), _ptr(coords), n, cin, _ptr(weight), _ptr(bias), cout,
            batch_size, *shape, _ptr(grid), generation, _ptr(y), _ptr(oc), _ptr(child),
            child.shape[1], _ptr(m), _ptr(coarse_grid), _ptr(workspace), self.stream()),
            "pxs_subm_conv3d_grid_s2_emit")
        return y, oc, child, m

    def s2_tagged_emit(self, n, batch_size, shape, grid, generation, coarse_grid, workspace):
        """pxs_s2_tagged_emit -> (out_coords, child_map [8, n], m as a device int64)."""
        oc, child, m = self._s2_outputs(n, grid.device)
        self._check(self.lib.pxs_s2_tagged_emit(n, batch_size, *shape, _ptr(grid), generation,
                                                _ptr(oc), _ptr(child), child.shape[1], _ptr(m),
                                                _ptr(coarse_grid), _ptr(workspace),
                                                self.stream()), "pxs_s2_tagged_emit")
        return oc, child, m

    def unet_s2_level(self, x, w_a, b_a, w_b, b_b, coords, batch_size, shape, grid, generation,
                      m, coarse_grid, workspace):
        """pxs_unet_s2_level -> (y_a, y_b [m rows], out_coords, child_map, m_out device int64)."""
        n, cin = x.shape
        cout_a, cout_b = w_a.shape[1], w_b.shape[1]
        y_a = torch.empty((n, cout_a), dtype=x.dtype, device=x.device)
        y_b = torch.empty((max(m, 1), cout_b), dtype=x.dtype, device=x.device)
        oc, child, m_out = self._s2_outputs(n, x.device)
        self._check(self.lib.pxs_unet_s2_level(
            _dtype_code(x), _ptr(x), _ptr(coords), n, cin, _ptr(w_a), _ptr(b_a), cout_a,
            batch_size, *shape, _ptr(grid), generation, _ptr(y_a), _ptr(w_b), _ptr(b_b), cout_b,
            m, _ptr(y_b), _ptr(oc), _ptr(child), child.shape[1], _ptr(m_out), _ptr(coarse_grid),
            _ptr(workspace), self.stream()), "pxs_unet_s2_level")
        return y_a, y_b[:m], oc, child, m_out

    def unet_s2_level_error(self, workspace, batch_size, shape):
        err = torch.zeros(1, dtype=torch.int32, device=workspace.device)
        self._check(self.lib.pxs_unet_s2_level_error(_ptr(workspace), batch_size, *shape, _ptr(err),
                                                     self.stream()), "pxs_unet_s2_level_error")
        return int(err.item())

    def sparse_conv3d_s2(self, x, weight, bias, child_map, m, out=None):
        n, cin = x.shape
        cout = weight.shape[1]
        y = torch.empty((m, cout), dtype=x.dtype, device=x.device) if out is None else out
        self._check(self.lib.pxs_sparse_conv3d_s2(_dtype_code(x), _ptr(x), n, cin, _ptr(weight),
                                                  _ptr(bias), cout, _ptr(child_map),
                                                  child_map.shape[1], m, _ptr(y), self.stream()),
                    "pxs_sparse_conv3d_s2")
        return y

    def downsample_mean(self, x, offsets, rows, m):
        y = torch.empty((max(m, 1), x.shape[1]), dtype=x.dtype, device=x.device)
        self._check(self.lib.pxs_downsample_mean(_dtype_code(x), _ptr(x), x.shape[1],
                                                 _ptr(offsets), _ptr(rows), m, _ptr(y),
                                                 self.stream()),
                    "pxs_downsample_mean")
        return y[:m]

    def linear_residual(self, x, weight, bias, residual):
        """pxs_linear_residual: residual (fp32) += x W^T + bias."""
        rows, cin = x.shape
        self._check(self.lib.pxs_linear_residual(_dtype_code(x), _ptr(x), rows, cin, _ptr(weight),
                                                 _ptr(bias), weight.shape[0], _ptr(residual),
                                                 self.stream()),
                    "pxs_linear_residual")
        return residual

    def linear(self, x, weight, bias=None, act=ACT_NONE, out=None):
        """pxs_linear: act(x W^T + bias) in x's dtype."""
        rows, cin = x.shape
        cout = weight.shape[0]
        y = torch.empty((rows, cout), dtype=x.dtype, device=x.device) if out is None else out
        self._check(self.lib.pxs_linear(_dtype_code(x), _ptr(x), rows, cin, _ptr(weight),
                                        _ptr(bias), cout, act, _ptr(y), self.stream()),
                    "pxs_linear")
        return y

    def linear_gate_residual(self, x, weight, bias, coords, block_mod, time_mod, gate_offset,
                             residual):
        rows, cin = x.shape
        cout = weight.shape[0]
        self._check(self.lib.pxs_linear_gate_residual(_dtype_code(x), _ptr(x), rows, cin,
                                                      _ptr(weight), _ptr(bias), cout,
                                                      _ptr(coords), _ptr(block_mod),
                                                      _ptr(time_mod), gate_offset,
                                                      _ptr(residual), self.stream()),
                    "pxs_linear_gate_residual")
        return residual

    # -- row-wise ---------------------------------------------------------------------
    def layer_norm(self, x, eps, gamma=None, beta=None, out_dtype=None):
        out_dtype = out_dtype or x.dtype
        y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
        self._check(self.lib.pxs_layer_norm(_dtype_code(x), _ptr(x), x.shape[0], x.shape[1], eps,
                                            _ptr(gamma), _ptr(beta), _dtype_code(y), _ptr(y),
                                            self.stream()),
                    "pxs_layer_norm")
        return y

    def layer_norm_modulate(self, x, eps, coords, block_mod, time_mod, offset, out_dtype=None):
        out_dtype = out_dtype or x.dtype
        y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
        self._check(self.lib.pxs_layer_norm_modulate(_dtype_code(x), _ptr(x), x.shape[0],
                                                     x.shape[1], eps, _ptr(coords),
                                                     _ptr(block_mod), _ptr(time_mod), offset,
                                                     _dtype_code(y), _ptr(y), self.stream()),
                    "pxs_layer_norm_modulate")
        return y

    def mh_rms_norm(self, x, heads, head_dim, gamma):
        y = torch.empty_like(x)
        self._check(self.lib.pxs_mh_rms_norm(_dtype_code(x), _ptr(x), x.stride(0), x.shape[0],
                                             heads, head_dim, _ptr(gamma), _ptr(y), y.stride(0),
                                             self.stream()),
                    "pxs_mh_rms_norm")
        return y

    def rope(self, coords, x, heads, head_dim, freq_min=1.0, freq_base=10000.0):
        y = torch.empty_like(x)
        self._check(self.lib.pxs_rope(_dtype_code(x), _ptr(coords), _ptr(x), x.stride(0),
                                      x.shape[0], heads, head_dim, freq_min, freq_base, _ptr(y),
                                      y.stride(0), self.stream()),
                    "pxs_rope")
        return y

    def qkv_prepare(self, qkv, heads, head_dim, q_gamma=None, k_gamma=None, coords=None,
                    freq_min=1.0, freq_base=10000.0):
        rows = qkv.shape[0]
        C = heads * head_dim
        q = torch.empty((rows, C), dtype=qkv.dtype, device=qkv.device)
        k, v = torch.empty_like(q), torch.empty_like(q)
        self._check(self.lib.pxs_qkv_prepare(_dtype_code(qkv), _ptr(qkv), rows, heads, head_dim,
                                             _ptr(q_gamma), _ptr(k_gamma), _ptr(coords), freq_min,
                                             freq_base, _ptr(q), _ptr(k), _ptr(v), self.stream()),
                    "pxs_qkv_prepare")
        return q, k, v

    def value_stats(self, x):
        """pxs_value_stats_f32 over an fp32 tensor -> dict of the summary."""
        count = x.numel()
        raw = torch.empty(40, dtype=torch.uint8, device=x.device)
        ws = self._ws(self.lib.pxs_value_stats_workspace_bytes(count), x.device)
        self._check(self.lib.pxs_value_stats_f32(_ptr(x), count, _ptr(raw), _ptr(ws),
                                                 self.stream()), "pxs_value_stats_f32")
        b = raw.cpu().numpy()
        i64, f64, f32 = b[:16].view(np.int64), b[16:24].view(np.float64), b[24:40].view(np.float32)
        return {"nonfinite": int(i64[0]), "first_bad": int(i64[1]), "sum": float(f64[0]),
                "first_bad_value": float(f32[0]), "min": float(f32[1]), "max": float(f32[2]),
                "max_abs": float(f32[3])}

    def convert(self, x, dtype):
        """x (fp32 or bf16, any shape) converted to dtype, elementwise."""
        y = torch.empty(x.shape, dtype=dtype, device=x.device)
        self._check(self.lib.pxs_convert(_dtype_code(x), _ptr(x), x.numel(), _dtype_code(y),
                                         _ptr(y), self.stream()),
                    "pxs_convert")
        return y

    def activation(self, x, act):
        self._check(self.lib.pxs_activation(_dtype_code(x), _ptr(x), x.numel(), act, self.stream()),
                    "pxs_activation")
        return x

    # -- attention --------------------------------------------------------------------
    def varlen_attention(self, q, k, v, cu_q, cu_k, heads, head_dim, scale, row_map=None,
                         out=None, nseg=None, value_dim=None):
        nseg = (cu_q.shape[0] - 1) if nseg is None else nseg
        value_dim = head_dim if value_dim is None else value_dim
        o = torch.empty((q.shape[0], heads * value_dim), dtype=q.dtype, device=q.device) \
            if out is None else out
        ws = self._ws(self.lib.pxs_attention_workspace_bytes(nseg), q.device)
        self._check(self.lib.pxs_varlen_attention(_dtype_code(q), _ptr(q), q.stride(0), _ptr(k),
                                                  k.stride(0), _ptr(v), v.stride(0), _ptr(cu_q),
                                                  _ptr(cu_k), nseg, q.shape[0], _ptr(row_map),
                                                  heads, head_dim, value_dim, scale, _ptr(o),
                                                  o.stride(0),
                                                  _ptr(ws), self.stream()),
                    "pxs_varlen_attention")
        return o

    # -- compositions ----------------------------------------------------------------------
    def transformer_block(self, cfg: BlockConfig, weights: BlockWeights, coords, batch_size, cu,
                          hidden, time_mod, context, ctx_offsets, projected=None, dtype=None):
        """pxs_transformer_block: hidden (fp32 [rows, C]) is updated in place."""
        dtype = _dtype_code(context) if dtype is None else dtype
        rows = coords.shape[0]
        tokens = context.shape[0]
        ws = self._ws(self.lib.pxs_transformer_block_workspace_bytes(
            dtype, C.byref(cfg), rows, tokens, batch_size), hidden.device)
        self._check(self.lib.pxs_transformer_block(
            dtype, C.byref(cfg), C.byref(weights), _ptr(coords), rows, batch_size, _ptr(cu),
            _ptr(hidden), _ptr(time_mod), _ptr(context), _ptr(ctx_offsets), tokens,
            _ptr(projected), _ptr(ws), self.stream()), "pxs_transformer_block")
        return hidden

    def slat_flow_forward(self, cfg: FlowConfig, weights: FlowWeights, coords, batch_size, cu, x,
                          timesteps, context, ctx_offsets, projected=None, dtype=None, out=None,
                          workspace=None):
        dtype = _dtype_code(context) if dtype is None else dtype
        rows = coords.shape[0]
        tokens = context.shape[0]
        y = torch.empty((rows, cfg.out_channels), dtype=torch.float32, device=x.device) \
            if out is None else out
        ws = workspace if workspace is not None else self._ws(
            self.flow_workspace_bytes(cfg, rows, tokens, batch_size, dtype), x.device)
        self._check(self.lib.pxs_slat_flow_forward(
            dtype, C.byref(cfg), C.byref(weights), _ptr(coords), rows, batch_size, _ptr(cu),
            _ptr(x), _ptr(timesteps), _ptr(context), _ptr(ctx_offsets), tokens, _ptr(projected),
            _ptr(y), _ptr(ws), self.stream()), "pxs_slat_flow_forward")
        return y

    def convnext_block(self, coords, x, mlp_hidden, eps, weights: DecoderBlockWeights, dtype,
                       nbr=None, masks=None, out=None):
        """pxs_convnext_block: x fp32 [rows, C] -> fp32 [rows, C] (out may be x)."""
        rows, ch = x.shape
        y = torch.empty_like(x) if out is None else out
        ws = self._ws(self.lib.pxs_convnext_block_workspace_bytes(
            dtype, rows, ch, mlp_hidden, int(nbr is not None)), x.device)
        self._check(self.lib.pxs_convnext_block(
            dtype, _ptr(coords), rows, _ptr(x), ch, mlp_hidden, eps, C.byref(weights), _ptr(nbr),
            _ptr(masks), _ptr(y), _ptr(ws), self.stream()), "pxs_convnext_block")
        return y

    def resblock_c2s(self, coords, x, out_channels, eps, weights: DecoderBlockWeights, dtype,
                     subdivision=None, pred_subdiv=False):
        """pxs_resblock_c2s -> (out_coords [m, 4], y fp32 [m, out], predicted [rows, 8] or None)."""
        rows, ch = x.shape
        dev = x.device
        oc = torch.empty((max(8 * rows, 1), 4), dtype=torch.int32, device=dev)
        y = torch.empty((max(8 * rows, 1), out_channels), dtype=torch.float32, device=dev)
        pred = torch.empty((max(rows, 1), 8), dtype=torch.float32, device=dev) if pred_subdiv \
            else None
        m = C.c_int64(0)
        ws = self._ws(self.lib.pxs_resblock_c2s_workspace_bytes(dtype, rows, ch, out_channels),
                      dev)
        self._check(self.lib.pxs_resblock_c2s(
            dtype, _ptr(coords), rows, _ptr(x), ch, out_channels, eps, C.byref(weights),
            int(pred_subdiv), _ptr(subdivision), _ptr(pred), _ptr(oc), _ptr(y), C.byref(m),
            _ptr(ws), self.stream()), "pxs_resblock_c2s")
        return oc[:m.value], y[:m.value], (pred[:rows] if pred is not None else None)

    def add_repeat(self, a, skip, out=None):
        rows, ch = a.shape
        y = torch.empty((rows, ch), dtype=torch.float32, device=a.device) if out is None else out
        self._check(self.lib.pxs_add_repeat(_dtype_code(a), _ptr(a), rows, ch, _ptr(skip),
                                            skip.shape[1], _ptr(y), self.stream()),
                    "pxs_add_repeat")
        return y

    def linear_ordered(self, x, weight, bias=None, out=None):
        """pxs_linear_ordered: fp32, the reference's summation order (bit-equal)."""
        rows, cin = x.shape
        cout = weight.shape[0]
        y = torch.empty((rows, cout), dtype=torch.float32, device=x.device) if out is None else out
        self._check(self.lib.pxs_linear_ordered(_ptr(x), rows, cin, _ptr(weight), _ptr(bias), cout,
                                                _ptr(y), self.stream()), "pxs_linear_ordered")
        return y

    def slat_decoder_forward(self, dtype, cfg: DecoderConfig, from_latent_w, from_latent_b,
                             output_w, output_b, blocks, coords, x, guide=None, predict=False,
                             upsample_times=-1, max_rows=None):
        """pxs_slat_decoder_forward -> (out_coords [m, 4], y [m, ch], level_rows list,
        predicted logits list or None)."""
        rows = coords.shape[0]
        levels = cfg.levels
        max_rows = rows * 8 ** (levels - 1) if max_rows is None else max_rows
        arr = (DecoderBlock * len(blocks))(*blocks)
        ws = self._ws(self.lib.pxs_slat_decoder_workspace_bytes(dtype, C.byref(cfg), arr,
                                                               len(blocks), rows, max_rows),
                      x.device)
        out_ch = cfg.out_channels if upsample_times < 0 else cfg.model_channels[upsample_times]
        out_coords = torch.empty((max_rows, 4), dtype=torch.int32, device=x.device)
        y = torch.empty((max_rows, out_ch), dtype=torch.float32, device=x.device)
        guide_arr = None
        if guide is not None:
            guide_arr = (C.c_void_p * (levels - 1))(*[g.data_ptr() for g in guide])
        preds = None
        pred_arr = None
        if predict:
            preds = [torch.empty((max_rows, 8), dtype=torch.float32, device=x.device)
                     for _ in range(levels - 1)]
            pred_arr = (C.c_void_p * (levels - 1))(*[t.data_ptr() for t in preds])
        m = C.c_int64()
        lvl = (C.c_int64 * levels)()
        self._check(self.lib.pxs_slat_decoder_forward(
            dtype, C.byref(cfg), _ptr(from_latent_w), _ptr(from_latent_b), _ptr(output_w),
            _ptr(output_b), arr, len(blocks), _ptr(coords), rows, _ptr(x), guide_arr, pred_arr,
            upsample_times, max_rows, _ptr(out_coords), _ptr(y), C.byref(m), lvl, _ptr(ws),
            self.stream()), "pxs_slat_decoder_forward")
        level_rows = list(lvl)
        if preds is not None:
            preds = [p[:level_rows[i]] for i, p in enumerate(preds)]
        return out_coords[:m.value], y[:m.value], level_rows, preds

    # -- flow Euler sampler -----------------------------------------------------
    def flow_sampler_schedule(self, scfg: SamplerConfig, step):
        """-> (t, t_next, guidance) of one step (host computation)."""
        t, tn, g = C.c_float(), C.c_float(), C.c_float()
        self._check(self.lib.pxs_flow_sampler_schedule(C.byref(scfg), step, C.byref(t),
                                                       C.byref(tn), C.byref(g)),
                    "pxs_flow_sampler_schedule")
        return t.value, tn.value, g.value

    def flow_guidance(self, state, positive, negative, coords, cu, batch_size, t, sigma_min,
                      guidance, rescale, out=None):
        rows, ch = state.shape
        y = torch.empty_like(state) if out is None else out
        ws = self._ws(self.lib.pxs_flow_guidance_workspace_bytes(batch_size), state.device)
        self._check(self.lib.pxs_flow_guidance(_ptr(state), _ptr(positive), _ptr(negative),
                                               _ptr(coords), _ptr(cu), rows, ch, batch_size, t,
                                               sigma_min, guidance, rescale, _ptr(y), _ptr(ws),
                                               self.stream()), "pxs_flow_guidance")
        return y

    def flow_pred_to_xstart(self, state, prediction, t, sigma_min):
        y = torch.empty_like(state)
        self._check(self.lib.pxs_flow_pred_to_xstart(_ptr(state), _ptr(prediction), state.numel(),
                                                     t, sigma_min, _ptr(y), self.stream()),
                    "pxs_flow_pred_to_xstart")
        return y

    def flow_euler_update(self, state, prediction, delta):
        """In place: state -= delta * prediction."""
        self._check(self.lib.pxs_flow_euler_update(_ptr(state), _ptr(prediction), state.numel(),
                                                   delta, self.stream()), "pxs_flow_euler_update")
        return state

    def flow_euler_sample(self, cfg: FlowConfig, weights: FlowWeights, scfg: SamplerConfig, coords,
                          batch_size, cu, noise, cond, cond_offsets, uncond, uncond_offsets,
                          dtype=None, out=None):
        dtype = _dtype_code(cond) if dtype is None else dtype
        rows = coords.shape[0]
        y = torch.empty_like(noise) if out is None else out
        ws = self._ws(self.lib.pxs_flow_euler_sample_workspace_bytes(
            dtype, C.byref(cfg), rows, cond.shape[0], uncond.shape[0], batch_size), noise.device)
        self._check(self.lib.pxs_flow_euler_sample(
            dtype, C.byref(cfg), C.byref(weights), C.byref(scfg), _ptr(coords), rows, batch_size,
            _ptr(cu), _ptr(noise), _ptr(cond), _ptr(cond_offsets), cond.shape[0], _ptr(uncond),
            _ptr(uncond_offsets), uncond.shape[0], _ptr(y), _ptr(ws), self.stream()),
            "pxs_flow_euler_sample")
        return y

    def flow_workspace_bytes(self, cfg: FlowConfig, rows, tokens, batch_size, dtype):
        return self.lib.pxs_slat_flow_workspace_bytes(dtype, C.byref(cfg), rows, tokens,
                                                      batch_size)

    # -- GGUF packs (f3) ----------------------------------------------------------
    def pack_open(self, path) -> "Pack":
        return Pack(self, path)

    def slat_flow_pack_load(self, pack: "Pack", component, dtype, device="cuda"):
        """pxs_slat_flow_pack_plan + _load -> PackedFlow (config, weights, arena)."""
        cfg, need = FlowConfig(), C.c_size_t()
        name = component.encode()
        self._check(self.lib.pxs_slat_flow_pack_plan(pack.handle, name, dtype, C.byref(cfg),
                                                     C.byref(need)), "pxs_slat_flow_pack_plan")
        arena = self._ws(need.value, device)
        ws = self._ws(self.lib.pxs_pack_upload_workspace_bytes(pack.handle), device)
        blocks = (BlockWeights * cfg.num_blocks)()
        weights = FlowWeights()
        self._check(self.lib.pxs_slat_flow_pack_load(
            pack.handle, name, dtype, _ptr(arena), C.c_size_t(arena.numel()), _ptr(ws),
            C.byref(weights), blocks, cfg.num_blocks, self.stream()), "pxs_slat_flow_pack_load")
        return PackedFlow(cfg, weights, blocks, arena, dtype)

    def slat_decoder_pack_load(self, pack: "Pack", component, dtype, device="cuda"):
        """pxs_slat_decoder_pack_plan + _load -> PackedDecoder."""
        hp, need = DecoderHParams(), C.c_size_t()
        name = component.encode()
        self._check(self.lib.pxs_slat_decoder_pack_plan(pack.handle, name, dtype, C.byref(hp),
                                                        C.byref(need)),
                    "pxs_slat_decoder_pack_plan")
        arena = self._ws(need.value, device)
        ws = self._ws(self.lib.pxs_pack_upload_workspace_bytes(pack.handle), device)
        blocks = (DecoderBlock * max(hp.n_blocks, 1))()
        io = (C.c_void_p * 4)()
        self._check(self.lib.pxs_slat_decoder_pack_load(
            pack.handle, name, dtype, _ptr(arena), C.c_size_t(arena.numel()), _ptr(ws), blocks,
            hp.n_blocks, io, self.stream()), "pxs_slat_decoder_pack_load")
        return PackedDecoder(hp, list(blocks)[:hp.n_blocks], [int(a) for a in io], arena, dtype)


class Pack:
    """An open GGUF pack (pxs_pack_open); close() it, or use it in a with."""

    def __init__(self, px: Pxs, path):
        self.px, self.lib = px, px.lib
        h = C.c_void_p()
        px._check(self.lib.pxs_pack_open(str(path).encode(), C.byref(h)), "pxs_pack_open")
        self.handle = h

    def close(self):
        if self.handle:
            self.lib.pxs_pack_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def describe(self) -> dict:
        import json
        n = self.lib.pxs_pack_describe(self.handle, None, 0)
        buf = C.create_string_buffer(n)
        self.lib.pxs_pack_describe(self.handle, buf, n)
        # Tensor names are bytes; keep ones that are not UTF-8 round-trippable.
        return json.loads(buf.value.decode("utf-8", errors="surrogateescape"))

    def metadata(self, key, kind, required=True):
        """kind: "u32", "f32", "bool" or "string"."""
        k = key.encode()
        if kind == "string":
            need = 1 << 16
            buf = C.create_string_buffer(need)
            self.px._check(self.lib.pxs_pack_metadata_string(self.handle, k, int(required), buf,
                                                             need), "pxs_pack_metadata_string")
            return buf.value.decode("utf-8")
        ctype = {"u32": C.c_uint32, "f32": C.c_float, "bool": C.c_int}[kind]
        v = ctype()
        fn = getattr(self.lib, f"pxs_pack_metadata_{kind}")
        self.px._check(fn(self.handle, k, int(required), C.byref(v)), f"pxs_pack_metadata_{kind}")
        return bool(v.value) if kind == "bool" else v.value

    def read_tensor(self, name) -> bytes:
        n = C.c_size_t()
        k = name.encode()
        info = {t["name"]: t for t in self.describe()["tensors"]}.get(name)
        size = info["n_bytes"] if info else 0
        buf = C.create_string_buffer(max(size, 1))
        self.px._check(self.lib.pxs_pack_read_tensor(self.handle, k, buf, size, C.byref(n)),
                       "pxs_pack_read_tensor")
        return buf.raw[:n.value]

    def upload(self, name, dtype, count, device="cuda", out=None):
        """pxs_pack_upload -> a 1-D device tensor of count elements in dtype."""
        tdt = torch.float32 if dtype == PXS_F32 else torch.bfloat16
        y = torch.empty(count, dtype=tdt, device=device) if out is None else out
        ws = self.px._ws(self.lib.pxs_pack_upload_workspace_bytes(self.handle), device)
        self.px._check(self.lib.pxs_pack_upload(self.handle, name.encode(), dtype, _ptr(y), count,
                                                _ptr(ws), self.px.stream()), "pxs_pack_upload")
        return y


class PackedFlow:
    """A SLat-flow component loaded into one device arena: cfg (FlowConfig),
    weights (FlowWeights over blocks) for slat_flow_forward / flow_euler_sample
    in `dtype`.  Keep this object alive while the weights are used."""

    def __init__(self, cfg, weights, blocks, arena, dtype):
        self.cfg, self.weights, self.blocks, self.arena, self.dtype = (cfg, weights, blocks,
                                                                         arena, dtype)


class PackedDecoder:
    """A SLat-decoder component in one device arena: hp (DecoderHParams),
    blocks (DecoderBlock list), io = [from_latent w, b, output w, b] device
    addresses; config() gives the DecoderConfig for slat_decoder_forward."""

    def __init__(self, hp, blocks, io, arena, dtype):
        self.hp, self.blocks, self.io, self.arena, self.dtype = hp, blocks, io, arena, dtype

    def config(self):
        L = self.hp.levels
        return decoder_config(self.hp.latent_channels, self.hp.out_channels, self.hp.norm_eps,
                              self.hp.pred_subdiv, list(self.hp.model_channels[:L]),
                              list(self.hp.num_blocks[:L]))
