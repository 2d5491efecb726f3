"""Seeded synthetic inputs for the sparse-voxel path.

Every random stream is a SplitMix64 counter generator (so the values do not
depend on numpy's generator versions), turned into U[0,1) doubles from the top
53 bits and into N(0,1) by Box-Muller.  Voxel sets are shells of random
axis-aligned ellipsoids of two-voxel thickness: a voxel v is active when
|rho - 1| * min(a) < 1 with rho = ||(v + 0.5 - c) / a||.  Rows are sorted
lexicographically by (batch, x, y, z).

Workloads (the sizes of the sparse path's benchmark workloads):
  conv_fp32_64     one 3x3x3 submanifold conv, fp32, 64^3 grid, one shell with
                   semi-axes U[16,30], C 64 -> 64
  unet_stage_128   batch 2 on a 128^3 grid, each item a union of 3 shells;
                   SubMConv3d 128->128, stride-2 conv 128->256, SubMConv3d at
                   64^3 256->256, bf16 features
  attn_full        varlen self-attention block, 12,288 + 20,480 tokens,
                   width 1024, 16 heads x 64
  swin_64          shifted-window attention, 64^3 grid ~30k voxels, windows of
                   8^3, shifts 0 and 4, 12 heads x 64, then the subdivide conv
  flow_step        one SLat-flow step, 24 blocks of width 1024 on ~40k voxels
"""

from __future__ import annotations

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(seed: int, count: int, stream: int = 0) -> np.ndarray:
    """count 64-bit outputs of SplitMix64 started at seed ^ (stream * golden)."""
    with np.errstate(over="ignore"):
        gamma = np.uint64(0x9E3779B97F4A7C15)
        start = np.uint64((seed ^ (stream * 0xD1B54A32D192ED03)) & 0xFFFFFFFFFFFFFFFF)
        z = start + gamma * (np.arange(1, count + 1, dtype=np.uint64))
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    return z


def uniform(seed: int, count: int, stream: int = 0) -> np.ndarray:
    """U[0,1) doubles."""
    return (splitmix64(seed, count, stream) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, count: int, stream: int = 0, std: float = 1.0) -> np.ndarray:
    """N(0, std^2) float32 by Box-Muller over pairs of uniforms."""
    pairs = (count + 1) // 2
    u = uniform(seed, 2 * pairs, stream)
    u1 = np.maximum(u[0::2], 1e-300)
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs, np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:count] * std).astype(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest bfloat16 (ties to even), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    rounded = (b + np.uint64(0x7FFF) + ((b >> np.uint64(16)) & np.uint64(1))) & np.uint64(0xFFFF0000)
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isfinite(x), out, x).astype(np.float32)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """bfloat16 bit patterns (uint16) of bf16_round(x)."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def ellipsoid_shell(grid: int, semi_lo: float, semi_hi: float, seed: int, stream: int = 0):
    """Boolean [grid]^3 mask of one two-voxel-thick ellipsoid shell."""
    u = uniform(seed, 6, stream)
    a = semi_lo + (semi_hi - semi_lo) * u[:3]
    jitter = np.floor(u[3:6] * 7.0) - 3.0
    c = grid / 2.0 + jitter
    ax = np.arange(grid, dtype=np.float64) + 0.5
    dx = ((ax - c[0]) / a[0])[:, None, None]
    dy = ((ax - c[1]) / a[1])[None, :, None]
    dz = ((ax - c[2]) / a[2])[None, None, :]
    rho = np.sqrt(dx * dx + dy * dy + dz * dz)
    return np.abs(rho - 1.0) * a.min() < 1.0


def shell_coords(grid: int, items, seed: int) -> np.ndarray:
    """int32 [N,4] rows (batch, x, y, z), lexicographically sorted.

    items: one entry per batch item, each a list of (semi_lo, semi_hi) shells
    whose union forms that item.
    """
    rows = []
    stream = 0
    for b, shells in enumerate(items):
        mask = np.zeros((grid, grid, grid), bool)
        for lo, hi in shells:
            mask |= ellipsoid_shell(grid, lo, hi, seed, stream)
            stream += 1
        xyz = np.argwhere(mask).astype(np.int32)  # C order == lexicographic
        rows.append(np.concatenate([np.full((xyz.shape[0], 1), b, np.int32), xyz], axis=1))
    return np.ascontiguousarray(np.concatenate(rows, axis=0), dtype=np.int32)


# ---------------------------------------------------------------------------
# Workload definitions.

def conv_fp32_64(seed: int = 2):
    """One SubMConv3d, fp32: 64^3, ~16k voxels, C 64 -> 64."""
    coords = shell_coords(64, [[(16.0, 30.0)]], seed)
    n = coords.shape[0]
    cin = cout = 64
    feats = normal(seed, n * cin, stream=101).reshape(n, cin)
    weight = normal(seed, 27 * cout * cin, stream=102,
                    std=float(np.sqrt(1.0 / (27 * 64)))).reshape(27, cout, cin)
    bias = np.zeros(cout, np.float32)
    return dict(coords=coords, batch_size=1, shape=(64, 64, 64), feats=feats, weight=weight,
                bias=bias)


UNET_ITEMS = [
    [(22.0, 36.0), (18.0, 30.0), (26.0, 40.0)],
    [(26.0, 44.0), (22.0, 38.0), (30.0, 50.0)],
]


def unet_stage_128(seed: int = 2):
    """Sparse conv U-Net stage, bf16, batch 2 on 128^3.

    Ops: SubMConv3d 3^3 128->128 at 128^3, stride-2 SparseConv3d 2^3 128->256,
    SubMConv3d 3^3 256->256 at 64^3.  Kaiming weights (std sqrt(2/fan_in)).
    """
    coords = shell_coords(128, UNET_ITEMS, seed)
    n = coords.shape[0]
    feats = bf16_round(normal(seed, n * 128, stream=201).reshape(n, 128))
    w_a = bf16_round(normal(seed, 27 * 128 * 128, stream=202,
                            std=float(np.sqrt(2.0 / (27 * 128)))).reshape(27, 128, 128))
    w_b = bf16_round(normal(seed, 8 * 256 * 128, stream=203,
                            std=float(np.sqrt(2.0 / (8 * 128)))).reshape(8, 256, 128))
    w_c = bf16_round(normal(seed, 27 * 256 * 256, stream=204,
                            std=float(np.sqrt(2.0 / (27 * 256)))).reshape(27, 256, 256))
    zeros = lambda c: np.zeros(c, np.float32)  # noqa: E731
    return dict(coords=coords, batch_size=2, shape=(128, 128, 128), feats=feats,
                w_a=w_a, b_a=zeros(128), w_b=w_b, b_b=zeros(256), w_c=w_c, b_c=zeros(256))


def attn_full(seed: int = 3, lengths=(12288, 20480), width: int = 1024, heads: int = 16):
    """Sparse full self-attention block, bf16, varlen batch (cu_seqlens)."""
    n = int(sum(lengths))
    # Only the batch column matters for full attention; coordinates are any
    # unique voxels per item (rows of a 32^3 lattice here).
    rows = []
    for b, length in enumerate(lengths):
        lin = np.arange(length, dtype=np.int64)
        xyz = np.stack([lin // 1024, (lin // 32) % 32, lin % 32], axis=1).astype(np.int32)
        rows.append(np.concatenate([np.full((length, 1), b, np.int32), xyz], axis=1))
    coords = np.concatenate(rows, axis=0)
    x = bf16_round(normal(seed, n * width, stream=301).reshape(n, width))
    w_qkv = bf16_round(normal(seed, 3 * width * width, stream=302, std=0.02).reshape(3 * width, width))
    b_qkv = np.zeros(3 * width, np.float32)
    w_out = bf16_round(normal(seed, width * width, stream=303, std=0.02).reshape(width, width))
    b_out = np.zeros(width, np.float32)
    gamma_q = np.ones(width, np.float32)
    gamma_k = np.ones(width, np.float32)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    return dict(coords=coords, batch_size=len(lengths), shape=(32, 32, 32), x=x, w_qkv=w_qkv,
                b_qkv=b_qkv, w_out=w_out, b_out=b_out, gamma_q=gamma_q, gamma_k=gamma_k,
                cu_seqlens=cu, heads=heads, head_dim=width // heads)


SWIN_SHELLS = [(20.0, 30.0), (14.0, 26.0)]


def swin_64(seed: int = 4, width: int = 768, heads: int = 12, up_out: int = 192):
    """Shifted-window sparse attention on 64^3 (~30k voxels) + subdivide conv."""
    coords = shell_coords(64, [SWIN_SHELLS], seed)
    n = coords.shape[0]
    x = bf16_round(normal(seed, n * width, stream=401).reshape(n, width))
    w_qkv = bf16_round(normal(seed, 3 * width * width, stream=402, std=0.02).reshape(3 * width, width))
    w_out = bf16_round(normal(seed, width * width, stream=403, std=0.02).reshape(width, width))
    w_up = bf16_round(normal(seed, 27 * 8 * up_out * width, stream=404,
                             std=0.02).reshape(27, 8 * up_out, width))
    return dict(coords=coords, batch_size=1, shape=(64, 64, 64), x=x, w_qkv=w_qkv,
                b_qkv=np.zeros(3 * width, np.float32), w_out=w_out,
                b_out=np.zeros(width, np.float32), w_up=w_up,
                b_up=np.zeros(8 * up_out, np.float32), heads=heads, head_dim=width // heads,
                window=8, shifts=(0, 4))


FLOW_SHELLS = [(24.0, 31.0), (18.0, 30.0), (12.0, 24.0)]


def flow_step_64(seed: int = 5):
    """One SLat-flow denoising step: ~42k voxels on 64^3 (three nested shells),
    24 blocks of width 1024 (16 heads x 64, MLP 4096), cross-attention to 1,370
    condition tokens of width 1024, input/output linears 8 -> 1024 -> 8."""
    coords = shell_coords(64, [FLOW_SHELLS], seed)
    return dict(coords=coords, batch_size=1, shape=(64, 64, 64), in_channels=8, out_channels=8,
                width=1024, heads=16, mlp_hidden=4096, blocks=24, context_tokens=1370)


DECODER_SHELLS = [(18.0, 22.0)]


def decoder_64(seed: int = 7):
    """A shape-decoder stack at the reference's decode scale: ~10.6k voxels at
    64^3, five levels of 1024, 512, 256, 128, 64 channels (the decoder shapes
    of tests/sparse_linear_cuda_benchmark.cpp:42-52: MLP 4C per level, output
    linear 64 -> 7), one ConvNeXt block per level, four predicted
    channel-to-spatial levels up to 1024^3."""
    coords = shell_coords(64, [DECODER_SHELLS], seed)
    return dict(coords=coords, latent_channels=32, out_channels=7,
                model_channels=[1024, 512, 256, 128, 64], num_blocks=[1, 1, 1, 1, 1])



def write_flow_pack(path, width=1024, blocks=24, heads=16, mlp_ratio=4, cond=1024,
                    in_ch=8, out_ch=8, seed=11, f16_matrices=False):
    """Write a synthetic SLat-flow component pack (shape_flow_1024, compact-v1
    names) in the converter's GGUF v3 layout: general / pixal3d keys, the
    flow hyperparameters, tensors in sorted name order, 32-byte alignment.
    Values are N(0, 0.02) (ones for norms and gammas); matrices are F16 when
    f16_matrices (the converter's ftype 1), else everything is F32 (the
    deployed flow policy).  Returns the payload bytes."""
    import struct

    C, M = width, width * mlp_ratio
    D = C // heads
    shapes = {"input_layer.weight": (C, in_ch), "input_layer.bias": (C,),
              "t_embedder.mlp.0.weight": (C, 256), "t_embedder.mlp.0.bias": (C,),
              "t_embedder.mlp.2.weight": (C, C), "t_embedder.mlp.2.bias": (C,),
              "adaLN_modulation.1.weight": (6 * C, C), "adaLN_modulation.1.bias": (6 * C,),
              "out_layer.weight": (out_ch, C), "out_layer.bias": (out_ch,)}
    for b in range(blocks):
        p, x = f"blocks.{b}.", f"blocks.{b}.cross_attn.cross_attn_block."
        shapes.update({p + "modulation": (6 * C,), p + "self_attn.to_qkv.weight": (3 * C, C),
                       p + "self_attn.to_qkv.bias": (3 * C,),
                       p + "self_attn.q_rms_norm.gamma": (heads, D),
                       p + "self_attn.k_rms_norm.gamma": (heads, D),
                       p + "self_attn.to_out.weight": (C, C), p + "self_attn.to_out.bias": (C,),
                       p + "norm2.weight": (C,), p + "norm2.bias": (C,),
                       x + "to_q.weight": (C, C), x + "to_q.bias": (C,),
                       x + "to_kv.weight": (2 * C, cond), x + "to_kv.bias": (2 * C,),
                       x + "q_rms_norm.gamma": (heads, D), x + "k_rms_norm.gamma": (heads, D),
                       x + "to_out.weight": (C, C), x + "to_out.bias": (C,),
                       p + "mlp.mlp.0.weight": (M, C), p + "mlp.mlp.0.bias": (M,),
                       p + "mlp.mlp.2.weight": (C, M), p + "mlp.mlp.2.bias": (C,)})

    def s(v):
        raw = v.encode()
        return struct.pack("<Q", len(raw)) + raw

    pre = "pixal3d.shape_flow_1024."
    kv = [(k, 8, s(v)) for k, v in (("general.architecture", "pixal3d"),
                                     ("general.name", "synthetic-flow"))]
    kv += [("general.file_type", 4, struct.pack("<I", 1 if f16_matrices else 0)),
           ("general.alignment", 4, struct.pack("<I", 32)),
           ("pixal3d.bundle_format", 4, struct.pack("<I", 1)),
           ("pixal3d.tensor_name_scheme", 8, s("compact-v1")),
           ("pixal3d.component.0", 8, s("shape_flow_1024")),
           (pre + "model_class", 8, s("ElasticSLatFlowModel"))]
    kv += [(pre + k, 4, struct.pack("<I", v)) for k, v in (
        ("resolution", 64), ("in_channels", in_ch), ("out_channels", out_ch),
        ("model_channels", C), ("cond_channels", cond), ("num_blocks", blocks),
        ("num_heads", heads))]
    kv += [(pre + "mlp_ratio", 6, struct.pack("<f", mlp_ratio)),
           (pre + "share_mod", 7, b"\x01"), (pre + "qk_rms_norm", 7, b"\x01"),
           (pre + "qk_rms_norm_cross", 7, b"\x01"),
           (pre + "rope_freq_min", 6, struct.pack("<f", 1.0)),
           (pre + "rope_freq_base", 6, struct.pack("<f", 10000.0))]
    names = sorted(shapes)
    types = {}
    for n in names:
        small = len(shapes[n]) < 2 or any(t in n for t in ("gamma", "modulation", "norm"))
        types[n] = 0 if (small or not f16_matrices) else 1
    align = lambda v: (v + 31) // 32 * 32  # noqa: E731
    head = bytearray(b"GGUF") + struct.pack("<IQQ", 3, len(names), len(kv))
    for k, t, v in kv:
        head += s(k) + struct.pack("<I", t) + v
    off, offsets = 0, []
    for n in names:
        offsets.append(off)
        off = align(off + int(np.prod(shapes[n])) * (2 if types[n] else 4))
    for n, o in zip(names, offsets):
        dims = tuple(reversed(shapes[n]))
        head += s("sh1024." + n) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", types[n], o)
    head += b"\0" * (align(len(head)) - len(head))
    rng = np.random.default_rng(seed)
    total = 0
    with open(path, "wb") as f:
        f.write(head)
        for n in names:
            count = int(np.prod(shapes[n]))
            if "gamma" in n or n.endswith("norm2.weight"):
                v = np.ones(count, np.float32)
            else:
                v = (rng.standard_normal(count, dtype=np.float32) * np.float32(0.02))
            raw = (v.astype(np.float16) if types[n] else v).tobytes()
            f.write(raw + b"\0" * (align(len(raw)) - len(raw)))
            total += len(raw)
    return total
