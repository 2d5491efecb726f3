"""GPU parity: GGUF pack ingestion (pxs_pack_upload and the model loaders).

* pxs_pack_upload converts F32 / F16 / BF16 payloads on the device bit for
  bit as the oracle decodes them (every finite half, subnormals included;
  bf16 rounding equal to torch's), across the 16 MiB staging chunks, and
  rejects a non-finite value with the tensor's name.
* pxs_slat_flow_pack_load / pxs_slat_decoder_pack_load on the golden packs
  written by the reference's converter: every bound weight holds exactly the
  converter's value in the dtype its role takes, and the forward over the
  loaded arena equals, bit for bit, the forward over the same weights
  uploaded tensor by tensor.
* Load errors in the reference's precedence (table order) and wording."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import pack_oracle as G
import pxs
import workloads as W
from gpu_common import host, t32, ti32, ti64

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
META = json.loads((GOLD / "pack_golden.json").read_text())


@pytest.fixture(scope="module")
def px():
    return pxs.Pxs()


def golden(stem):
    return GOLD / META[stem]["file"]


def bits_of(t):
    if t.dtype == torch.float32:
        return t.cpu().view(torch.int32).numpy().view(np.uint32)
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def upload_pack(tmp_path):
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = halves[(halves & 0x7C00) != 0x7C00]           # every finite half
    rng = np.random.default_rng(9)
    f32 = np.concatenate([rng.standard_normal(1003).astype(np.float32) * 5,
                          np.array([0.0, -0.0, 1e-40, -3e-39, 3.38e38, -1.17549435e-38],
                                   np.float32),
                          ((np.arange(40, dtype=np.uint32) << 16) | 0x8000).view(np.float32)])
    bf = G.bf16_bits(rng.standard_normal(777).astype(np.float32) * 100)
    big = rng.standard_normal(9_000_011).astype(np.float16)  # > one 16 MiB chunk, odd tail
    tensors = [G.Tensor("f16_all", G.GGML_F16, (finite.size,), finite.tobytes()),
               G.f32_tensor("f32_mix", f32),
               G.Tensor("bf16_rand", G.GGML_BF16, (bf.size,), bf.tobytes()),
               G.Tensor("f16_big", G.GGML_F16, (big.size,), big.tobytes()),
               G.f32_tensor("f32_inf", np.array([1.0, 2.0, np.inf, 3.0], np.float32)),
               G.f32_tensor("f32_over_bf16", np.array([1.0, -3.4e38, 2.0], np.float32)),
               G.Tensor("f16_nan", G.GGML_F16, (3,), np.array([0x3C00, 0x7E00, 0], np.uint16)
                        .tobytes()),
               G.Tensor("q4", 2, (32,), bytes(18))]
    path = tmp_path / "upload.gguf"
    G.write_pack(path, G.pixal3d_kvs(), tensors)
    return path


def test_upload_conversions_bit_exact(px, tmp_path):
    path = upload_pack(tmp_path)
    info = G.load_pack_info(path)
    with px.pack_open(path) as pack:
        for name in ("f16_all", "f32_mix", "bf16_rand", "f16_big"):
            t = info.tensor(name)
            ref = G.decode_f32(G.read_tensor(info, name), t.ggml_type)
            print(f"[pack upload] {name} n={ref.size}", flush=True)
            got32 = pack.upload(name, pxs.PXS_F32, ref.size)
            np.testing.assert_array_equal(bits_of(got32), ref.view(np.uint32))
            got16 = pack.upload(name, pxs.PXS_BF16, ref.size)
            want16 = torch.from_numpy(ref).to(torch.bfloat16).view(torch.int16).numpy() \
                .view(np.uint16)
            np.testing.assert_array_equal(bits_of(got16), want16)
            np.testing.assert_array_equal(want16, G.bf16_bits(ref))
        # a destination with data around it: only the tensor's elements change
        buf = torch.full((1024 + 2000,), 7.0, device="cuda")
        pack.upload("f32_mix", pxs.PXS_F32, 1049, out=buf[512:512 + 1049])
        assert torch.all(buf[:512] == 7.0) and torch.all(buf[512 + 1049:] == 7.0)


def test_upload_errors(px, tmp_path):
    path = upload_pack(tmp_path)
    with px.pack_open(path) as pack:
        with pytest.raises(pxs.PxsError, match=r"tensor contains a non-finite value: f32_inf"):
            pack.upload("f32_inf", pxs.PXS_F32, 4)
        with pytest.raises(pxs.PxsError, match=r"non-finite value: f16_nan \(code 3\)"):
            pack.upload("f16_nan", pxs.PXS_BF16, 3)
        # a finite F32 beyond the bf16 range loads as fp32, but as bf16 it would
        # become an infinity: that load fails like a non-finite payload
        got = pack.upload("f32_over_bf16", pxs.PXS_F32, 3)
        assert float(got[1]) == float(np.float32(-3.4e38))
        with pytest.raises(pxs.PxsError, match=r"non-finite value: f32_over_bf16"):
            pack.upload("f32_over_bf16", pxs.PXS_BF16, 3)
        with pytest.raises(pxs.PxsError, match="has type q4_0, not f32, f16 or bf16"):
            pack.upload("q4", pxs.PXS_F32, 32)
        with pytest.raises(pxs.PxsError, match="holds 1049 elements, not 1048"):
            pack.upload("f32_mix", pxs.PXS_F32, 1048)
        with pytest.raises(pxs.PxsError, match="tensor not found: nope"):
            pack.upload("nope", pxs.PXS_F32, 1)
        ws = torch.empty(px.lib.pxs_pack_upload_workspace_bytes(pack.handle) + 16,
                         dtype=torch.uint8, device="cuda")
        y = torch.empty(777, dtype=torch.float32, device="cuda")
        rc = px.lib.pxs_pack_upload(pack.handle, b"bf16_rand", pxs.PXS_F32, y.data_ptr(), 777,
                                    ws.data_ptr() + 8, px.stream())
        assert rc == pxs.PXS_ERR_ARG
        assert px.lib.pxs_last_error().decode() == \
            "pxs_pack_upload: workspace must be 256-byte aligned"
        # the pack stays usable after an error
        got = pack.upload("bf16_rand", pxs.PXS_F32, 777)
        assert torch.isfinite(got).all()


# --- SLat flow ---------------------------------------------------------------------

FLOW_FIELDS = {
    "modulation": "modulation", "self_to_qkv_weight": "self_attn.to_qkv.weight",
    "self_to_qkv_bias": "self_attn.to_qkv.bias", "self_q_gamma": "self_attn.q_rms_norm.gamma",
    "self_k_gamma": "self_attn.k_rms_norm.gamma", "self_to_out_weight": "self_attn.to_out.weight",
    "self_to_out_bias": "self_attn.to_out.bias", "norm2_weight": "norm2.weight",
    "norm2_bias": "norm2.bias", "cross_to_q_weight": "cross_attn.cross_attn_block.to_q.weight",
    "cross_to_q_bias": "cross_attn.cross_attn_block.to_q.bias",
    "cross_to_kv_weight": "cross_attn.cross_attn_block.to_kv.weight",
    "cross_to_kv_bias": "cross_attn.cross_attn_block.to_kv.bias",
    "cross_q_gamma": "cross_attn.cross_attn_block.q_rms_norm.gamma",
    "cross_k_gamma": "cross_attn.cross_attn_block.k_rms_norm.gamma",
    "cross_to_out_weight": "cross_attn.cross_attn_block.to_out.weight",
    "cross_to_out_bias": "cross_attn.cross_attn_block.to_out.bias",
    "proj_weight": "cross_attn.proj_linear.weight", "proj_bias": "cross_attn.proj_linear.bias",
    "mlp0_weight": "mlp.mlp.0.weight", "mlp0_bias": "mlp.mlp.0.bias",
    "mlp2_weight": "mlp.mlp.2.weight", "mlp2_bias": "mlp.mlp.2.bias"}
FLOW_TOP = ["input_layer.weight", "input_layer.bias", "t_embedder.mlp.0.weight",
            "t_embedder.mlp.0.bias", "t_embedder.mlp.2.weight", "t_embedder.mlp.2.bias",
            "adaLN_modulation.1.weight", "adaLN_modulation.1.bias", "out_layer.weight",
            "out_layer.bias"]


def decoded(info, name):
    t = info.tensor(name)
    return G.decode_f32(G.read_tensor(info, name), t.ggml_type)


def arena_slice(packed, addr, count, dtype):
    off = addr - packed.arena.data_ptr()
    size = 4 if dtype == torch.float32 else 2
    assert 0 <= off and off + count * size <= packed.arena.numel() and off % 256 == 0
    return packed.arena[off:off + count * size].view(dtype)


def direct_flow(info, alias, nb, dtype):
    tdt = torch.bfloat16 if dtype == pxs.PXS_BF16 else torch.float32
    fw = [t32(decoded(info, f"{alias}.{n}")) for n in FLOW_TOP]
    blocks = []
    for b in range(nb):
        ws = []
        for i, field in enumerate(pxs.BLOCK_WEIGHT_FIELDS):
            name = f"{alias}.blocks.{b}.{FLOW_FIELDS[field]}"
            if info.tensor(name) is None:
                ws.append(None)
                continue
            t = t32(decoded(info, name))
            ws.append(t.to(tdt) if i in pxs.BLOCK_LINEAR_WEIGHTS else t)
        blocks.append(ws)
    arr = (pxs.BlockWeights * nb)(*[pxs.block_weights(ws) for ws in blocks])
    return pxs.FlowWeights(*[t.data_ptr() for t in fw], arr), (fw, blocks, arr)


def flow_inputs(cfg, tdt, seed=3):
    coords = W.shell_coords(16, [[(4.0, 6.0)], [(3.0, 5.0)]], seed)
    n = coords.shape[0]
    x = W.normal(seed, n * cfg.in_channels, 1).reshape(n, cfg.in_channels)
    ctx = W.normal(seed, 2 * 7 * cfg.cond_channels, 2).reshape(14, cfg.cond_channels)
    return (ti32(coords), t32(x), t32(np.array([731.5, 88.25], np.float32)),
            t32(ctx).to(tdt), ti64(np.array([0, 7, 14], np.int64)))


@pytest.mark.parametrize("stem", ["pack_flow_f16", "pack_flow_bf16"])
@pytest.mark.parametrize("dtype", [pxs.PXS_F32, pxs.PXS_BF16])
def test_flow_pack_load(px, stem, dtype):
    tdt = torch.bfloat16 if dtype == pxs.PXS_BF16 else torch.float32
    info = G.load_pack_info(golden(stem))
    print(f"[flow pack] {stem} dtype={dtype}", flush=True)
    with px.pack_open(golden(stem)) as pack:
        packed = px.slat_flow_pack_load(pack, "shape_flow_1024", dtype)
    cfg = packed.cfg
    # every bound weight: the converter's value in its role's dtype
    for i, name in enumerate(FLOW_TOP):
        ref = decoded(info, f"sh1024.{name}")
        got = arena_slice(packed, getattr(packed.weights, pxs.FlowWeights._fields_[i][0]),
                          ref.size, torch.float32)
        np.testing.assert_array_equal(bits_of(got), ref.view(np.uint32), err_msg=name)
    blk = packed.blocks[0]
    for i, field in enumerate(pxs.BLOCK_WEIGHT_FIELDS):
        name = f"sh1024.blocks.0.{FLOW_FIELDS[field]}"
        addr = getattr(blk, field)
        if info.tensor(name) is None or field.startswith("proj"):
            assert not addr, field
            continue
        ref = torch.from_numpy(decoded(info, name))
        want = ref.to(tdt) if i in pxs.BLOCK_LINEAR_WEIGHTS else ref
        got = arena_slice(packed, addr, ref.numel(), want.dtype)
        np.testing.assert_array_equal(bits_of(got), bits_of(want), err_msg=field)
    # the forward over the arena equals the forward over separately uploaded weights
    direct, keep = direct_flow(info, "sh1024", cfg.num_blocks, dtype)
    coords, x, t, ctx, ctx_off = flow_inputs(cfg, tdt)
    cu = px.batch_cu_seqlens(coords, 2)
    a = px.slat_flow_forward(cfg, packed.weights, coords, 2, cu, x, t, ctx, ctx_off, dtype=dtype)
    b = px.slat_flow_forward(cfg, direct, coords, 2, cu, x, t, ctx, ctx_off, dtype=dtype)
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    np.testing.assert_array_equal(bits_of(a), bits_of(b))


def edited_pack(src, dst, edit=None, drop=(), append=()):
    """Rewrite a golden pack with tensor payloads edited (name -> float32
    values), tensors dropped and extra tensors appended."""
    info = G.load_pack_info(src)
    kvs = [(k, vt, v) for k, (vt, v) in info.kv.items()]
    tensors = []
    for t in info.tensors:
        if t.name in drop:
            continue
        raw = G.read_tensor(info, t.name)
        dims = t.ne[:max(t.n_dims, 1)]
        if edit and t.name in edit:
            vals = np.asarray(edit[t.name], np.float32)
            if vals.size == int(np.prod(dims)):
                vals = vals.reshape(tuple(reversed(dims)))
            tensors.append(G.f32_tensor(t.name, vals))
        else:
            tensors.append(G.Tensor(t.name, t.ggml_type, dims, raw))
    tensors += list(append)
    G.write_pack(dst, kvs, tensors)
    return dst


def flow_load_error(px, path, dtype=pxs.PXS_F32, component="shape_flow_1024"):
    with px.pack_open(path) as pack:
        with pytest.raises(pxs.PxsError) as e:
            px.slat_flow_pack_load(pack, component, dtype)
    return str(e.value)


def test_flow_pack_load_errors(px, tmp_path):
    src = golden("pack_flow_f16")
    info = G.load_pack_info(src)
    names = [t.name for t in info.tensors]
    k = names.index("sh1024.blocks.0.norm2.bias")
    bad = decoded(info, names[k]).copy()
    bad[3] = np.nan
    late_q4 = G.Tensor("sh1024.zz_quant", 2, (32,), bytes(18))
    p = edited_pack(src, tmp_path / "a.gguf", {names[k]: bad}, append=[late_q4])
    assert flow_load_error(px, p) == \
        f"pxs_slat_flow_pack_load: SLat flow tensor contains a non-finite value: {names[k]} (code 3)"
    early_q4 = G.Tensor("sh1024.aa_quant", 2, (32,), bytes(18))
    info_tensors = [early_q4]
    p = edited_pack(src, tmp_path / "b.gguf", {names[k]: bad})
    G.write_pack(tmp_path / "c.gguf", [(kk, vt, v) for kk, (vt, v) in
                                       G.load_pack_info(p).kv.items()],
                 info_tensors + [G.Tensor(t.name, t.ggml_type, t.ne[:max(t.n_dims, 1)],
                                          G.read_tensor(G.load_pack_info(p), t.name))
                                 for t in G.load_pack_info(p).tensors])
    assert flow_load_error(px, tmp_path / "c.gguf") == \
        "pxs_slat_flow_pack_load: unsupported or misaligned SLat flow tensor: sh1024.aa_quant " \
        "(code 1)"
    p = edited_pack(src, tmp_path / "d.gguf", drop=("sh1024.blocks.0.mlp.mlp.2.bias",))
    assert flow_load_error(px, p) == \
        "pxs_slat_flow_pack_load: missing SLat flow tensor: sh1024.blocks.0.mlp.mlp.2.bias " \
        "(code 1)"
    w = decoded(info, "sh1024.out_layer.bias")
    p = edited_pack(src, tmp_path / "e.gguf", {"sh1024.out_layer.bias": np.append(w, 1.0)})
    assert flow_load_error(px, p) == \
        "pxs_slat_flow_pack_load: SLat flow tensor sh1024.out_layer.bias has shape " \
        "[9, 1, 1, 1], expected 8 elements (code 1)"


# --- SLat decoder --------------------------------------------------------------------

CONVNEXT_FIELDS = {"norm_weight": "norm.weight", "norm_bias": "norm.bias",
                   "conv1_weight": "conv.weight", "conv1_bias": "conv.bias",
                   "mlp0_weight": "mlp.0.weight", "mlp0_bias": "mlp.0.bias",
                   "mlp2_weight": "mlp.2.weight", "mlp2_bias": "mlp.2.bias"}
C2S_FIELDS = {"norm1_weight": "norm1.weight", "norm1_bias": "norm1.bias",
              "conv1_weight": "conv1.weight", "conv1_bias": "conv1.bias",
              "conv2_weight": "conv2.weight", "conv2_bias": "conv2.bias",
              "to_subdiv_weight": "to_subdiv.weight", "to_subdiv_bias": "to_subdiv.bias"}
DECODER_LAYOUT = [("blocks.0.0", CONVNEXT_FIELDS, pxs.PXS_DECODER_CONVNEXT),
                  ("blocks.0.1", C2S_FIELDS, pxs.PXS_DECODER_C2S),
                  ("blocks.1.0", CONVNEXT_FIELDS, pxs.PXS_DECODER_CONVNEXT)]


@pytest.mark.parametrize("dtype", [pxs.PXS_F32, pxs.PXS_BF16])
def test_decoder_pack_load(px, dtype):
    tdt = torch.bfloat16 if dtype == pxs.PXS_BF16 else torch.float32
    stem = "pack_decoder_f16"
    info = G.load_pack_info(golden(stem))
    print(f"[decoder pack] dtype={dtype}", flush=True)
    with px.pack_open(golden(stem)) as pack:
        packed = px.slat_decoder_pack_load(pack, "texture_decoder", dtype)
    assert len(packed.blocks) == 3
    keep, direct = [], []
    for blk, (prefix, fields, kind) in zip(packed.blocks, DECODER_LAYOUT):
        assert blk.kind == kind
        dev = {}
        for field, local in fields.items():
            ref = torch.from_numpy(decoded(info, f"texture_decoder.{prefix}.{local}"))
            want = ref.to(tdt) if field in pxs.DECODER_DTYPE_WEIGHTS else ref
            got = arena_slice(packed, getattr(blk.w, field), ref.numel(), want.dtype)
            np.testing.assert_array_equal(bits_of(got), bits_of(want), err_msg=prefix + field)
            dev[field] = want.cuda()
        keep.append(dev)
        direct.append(pxs.DecoderBlock(blk.kind, blk.channels, blk.out_channels, blk.mlp_hidden,
                                       pxs.decoder_block_weights(dev)))
    io_names = ["from_latent.weight", "from_latent.bias", "output_layer.weight",
                "output_layer.bias"]
    io = [t32(decoded(info, f"texture_decoder.{n}")) for n in io_names]
    for addr, t in zip(packed.io, io):
        np.testing.assert_array_equal(bits_of(arena_slice(packed, addr, t.numel(), torch.float32)),
                                      bits_of(t))
    coords = W.shell_coords(12, [[(3.0, 4.5)], [(2.5, 4.0)]], 21)
    x = t32(W.normal(21, coords.shape[0] * 8, 1).reshape(-1, 8))
    cfg = packed.config()
    a = px.slat_decoder_forward(dtype, cfg, *packed.io, packed.blocks, ti32(coords), x,
                                predict=True)
    b = px.slat_decoder_forward(dtype, cfg, *io, direct, ti32(coords), x, predict=True)
    torch.cuda.synchronize()
    assert a[2] == b[2] and a[2][-1] > a[2][0]
    np.testing.assert_array_equal(host(a[0]), host(b[0]))
    np.testing.assert_array_equal(bits_of(a[1]), bits_of(b[1]))
    for pa, pb in zip(a[3], b[3]):
        np.testing.assert_array_equal(bits_of(pa), bits_of(pb))


def test_decoder_pack_load_errors(px, tmp_path):
    src = golden("pack_decoder_f16")
    info = G.load_pack_info(src)
    name = "texture_decoder.blocks.0.1.conv2.bias"
    bad = decoded(info, name).copy()
    bad[0] = np.inf
    p = edited_pack(src, tmp_path / "a.gguf", {name: bad})
    with px.pack_open(p) as pack:
        with pytest.raises(pxs.PxsError, match=f"SLat decoder tensor contains a non-finite "
                                               f"value: {name}"):
            px.slat_decoder_pack_load(pack, "texture_decoder", pxs.PXS_F32)
    p = edited_pack(src, tmp_path / "b.gguf", drop=("texture_decoder.blocks.0.1.to_subdiv.bias",))
    with px.pack_open(p) as pack:
        with pytest.raises(pxs.PxsError, match="missing SLat decoder tensor: "
                                               "texture_decoder.blocks.0.1.to_subdiv.bias"):
            px.slat_decoder_pack_load(pack, "texture_decoder", pxs.PXS_BF16)
    p = edited_pack(src, tmp_path / "c.gguf",
                    append=[G.Tensor("texture_decoder.zz_quant", 2, (32,), bytes(18))])
    with px.pack_open(p) as pack:
        with pytest.raises(pxs.PxsError, match="unsupported SLat decoder tensor type: "
                                               "texture_decoder.zz_quant"):
            px.slat_decoder_pack_load(pack, "texture_decoder", pxs.PXS_F32)


def check_flow_arena(packed, info, alias, dtype):
    """Every weight pxs_slat_flow_pack_load bound holds the pack's value in
    its role's dtype."""
    tdt = torch.bfloat16 if dtype == pxs.PXS_BF16 else torch.float32
    for i, name in enumerate(FLOW_TOP):
        ref = decoded(info, f"{alias}.{name}")
        got = arena_slice(packed, getattr(packed.weights, pxs.FlowWeights._fields_[i][0]),
                          ref.size, torch.float32)
        np.testing.assert_array_equal(bits_of(got), ref.view(np.uint32), err_msg=name)
    for b in range(packed.cfg.num_blocks):
        blk = packed.blocks[b]
        for i, field in enumerate(pxs.BLOCK_WEIGHT_FIELDS):
            name = f"{alias}.blocks.{b}.{FLOW_FIELDS[field]}"
            if info.tensor(name) is None:
                continue
            ref = torch.from_numpy(decoded(info, name))
            want = ref.to(tdt) if i in pxs.BLOCK_LINEAR_WEIGHTS else ref
            got = arena_slice(packed, getattr(blk, field), ref.numel(), want.dtype)
            np.testing.assert_array_equal(bits_of(got), bits_of(want), err_msg=name)


@pytest.mark.parametrize("f16", [False, True])
def test_flow_pack_load_multichunk(px, tmp_path, f16):
    """Width 512, 3 blocks (~50 MB F32): tensors share and straddle the 16 MiB
    staging chunks; every bound weight is checked."""
    path = tmp_path / "wide.gguf"
    W.write_flow_pack(path, width=512, blocks=3, heads=8, cond=512, f16_matrices=f16)
    info = G.load_pack_info(path)
    for dtype in (pxs.PXS_F32, pxs.PXS_BF16):
        print(f"[flow pack multichunk] f16={f16} dtype={dtype}", flush=True)
        with px.pack_open(path) as pack:
            packed = px.slat_flow_pack_load(pack, "shape_flow_1024", dtype)
        torch.cuda.synchronize()
        check_flow_arena(packed, info, "sh1024", dtype)


def test_flow_pack_load_alignment_8(px, tmp_path):
    """general.alignment 8: payloads sit at 8-byte offsets, so pieces that are
    not 16-byte aligned in a chunk open a chunk of their own."""
    info = G.load_pack_info(golden("pack_flow_f16"))
    kvs = [(k, vt, (8 if k == "general.alignment" else v)) for k, (vt, v) in info.kv.items()]
    tensors = [G.Tensor(t.name, t.ggml_type, t.ne[:max(t.n_dims, 1)], G.read_tensor(info, t.name))
               for t in info.tensors]
    # a 2-byte tensor first shifts every later payload by 8 bytes
    tensors.insert(0, G.Tensor("sh1024.aaa_extra", G.GGML_F16, (1,), np.float16(0.5).tobytes()))
    path = tmp_path / "a8.gguf"
    G.write_pack(path, kvs, tensors, alignment=8)
    info8 = G.load_pack_info(path)
    assert any(t.offset % 16 for t in info8.tensors)
    for dtype in (pxs.PXS_F32, pxs.PXS_BF16):
        with px.pack_open(path) as pack:
            packed = px.slat_flow_pack_load(pack, "shape_flow_1024", dtype)
        torch.cuda.synchronize()
        check_flow_arena(packed, info8, "sh1024", dtype)


def test_flow_pack_load_projection_mode(px, tmp_path):
    """image_attn_mode proj: the block's proj_linear weights are bound (in
    the GEMM dtype) and the forward with a projection input equals the
    forward over the same weights uploaded directly."""
    info = G.load_pack_info(golden("pack_flow_f16"))
    C, PC = 16, 12
    rng = np.random.default_rng(31)
    pw = (rng.standard_normal((C, PC)) * 0.2).astype(np.float32)
    pb = (rng.standard_normal(C) * 0.1).astype(np.float32)
    kvs = [(k, vt, v) for k, (vt, v) in info.kv.items()
           if k != "pixal3d.shape_flow_1024.image_attn_mode"]
    kvs += [("pixal3d.shape_flow_1024.image_attn_mode", G.VT_STRING, "proj"),
            ("pixal3d.shape_flow_1024.proj_in_channels", G.VT_U32, PC)]
    tensors = [G.Tensor(t.name, t.ggml_type, t.ne[:max(t.n_dims, 1)], G.read_tensor(info, t.name))
               for t in info.tensors]
    tensors += [G.f32_tensor("sh1024.blocks.0.cross_attn.proj_linear.weight", pw, G.GGML_F16),
                G.f32_tensor("sh1024.blocks.0.cross_attn.proj_linear.bias", pb)]
    path = tmp_path / "proj.gguf"
    G.write_pack(path, kvs, tensors)
    info_p = G.load_pack_info(path)
    for dtype in (pxs.PXS_F32, pxs.PXS_BF16):
        tdt = torch.bfloat16 if dtype == pxs.PXS_BF16 else torch.float32
        with px.pack_open(path) as pack:
            packed = px.slat_flow_pack_load(pack, "shape_flow_1024", dtype)
        cfg = packed.cfg
        assert (cfg.use_projection, cfg.proj_in_channels) == (1, PC)
        check_flow_arena(packed, info_p, "sh1024", dtype)
        direct, keep = direct_flow(info_p, "sh1024", cfg.num_blocks, dtype)
        coords, x, t, ctx, ctx_off = flow_inputs(cfg, tdt)
        proj = t32(W.normal(5, coords.shape[0] * PC, 9).reshape(-1, PC)).to(tdt)
        cu = px.batch_cu_seqlens(coords, 2)
        a = px.slat_flow_forward(cfg, packed.weights, coords, 2, cu, x, t, ctx, ctx_off,
                                 projected=proj, dtype=dtype)
        b = px.slat_flow_forward(cfg, direct, coords, 2, cu, x, t, ctx, ctx_off, projected=proj,
                                 dtype=dtype)
        torch.cuda.synchronize()
        assert torch.isfinite(a).all()
        np.testing.assert_array_equal(bits_of(a), bits_of(b))


def test_decoder_pack_load_without_subdivision_head(px, tmp_path):
    """pred_subdiv false: the C2S block binds no to_subdiv tensors (the pack
    may omit them) and the decoder runs with given subdivisions."""
    info = G.load_pack_info(golden("pack_decoder_f16"))
    kvs = [(k, vt, (False if k == "pixal3d.texture_decoder.pred_subdiv" else v))
           for k, (vt, v) in info.kv.items()]
    tensors = [G.Tensor(t.name, t.ggml_type, t.ne[:max(t.n_dims, 1)], G.read_tensor(info, t.name))
               for t in info.tensors if "to_subdiv" not in t.name]
    path = tmp_path / "nosub.gguf"
    G.write_pack(path, kvs, tensors)
    with px.pack_open(path) as pack:
        packed = px.slat_decoder_pack_load(pack, "texture_decoder", pxs.PXS_F32)
    assert packed.hp.pred_subdiv == 0
    c2s = packed.blocks[1]
    assert not c2s.w.to_subdiv_weight and not c2s.w.to_subdiv_bias
    coords = W.shell_coords(12, [[(3.0, 4.5)], [(2.5, 4.0)]], 22)
    n = coords.shape[0]
    x = t32(W.normal(22, n * 8, 1).reshape(-1, 8))
    guide = t32((W.uniform(22, n * 8, 2).reshape(n, 8) > 0.5).astype(np.float32))
    out_coords, y, level_rows, _ = px.slat_decoder_forward(
        pxs.PXS_F32, packed.config(), *packed.io, packed.blocks, ti32(coords), x, guide=[guide])
    torch.cuda.synchronize()
    assert level_rows[0] == n and level_rows[1] == int(host(guide).sum())
    assert torch.isfinite(y).all() and y.shape[1] == packed.hp.out_channels
