"""ctypes bindings for the CPU oracle and the compiled reference.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, to check and time against.  The shipped
library never imports this module.

* ``Oracle`` wraps build/liboracle.so, this repository's C++ restatement of
  the reference CPU path (pxs_oracle.cpp, with per-function citations).
* ``Reference`` wraps _ref/libpixal3d_ref.so, the reference's own
  src/{sparse,sparse_transformer,cpu_threads,flow}.cpp compiled from
  /root/reference by oracle/Makefile.  It exists only where that build ran.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "build" / "liboracle.so"
REF_LIB = HERE / "_ref" / "libpixal3d_ref.so"
DROPIN_LIB = HERE / "build" / "libdropin_shim.so"

# Validation codes of orc_sparse_valid -> the reference's messages
# (src/sparse.cpp:249-330).
VALID_MESSAGES = {
    1: "invalid sparse tensor shape",
    3: "sparse feature count does not match coordinates",
    4: "sparse coordinate is outside its shape",
    5: "sparse coordinates contain a duplicate point",
    6: "sparse coordinates must be contiguous by batch",
    7: "sparse features contain a non-finite value",
}

_i32p = C.POINTER(C.c_int32)
_i64p = C.POINTER(C.c_int64)
_f32p = C.POINTER(C.c_float)
_intp = C.POINTER(C.c_int)
_vp = C.c_void_p


def _p(a, ctype):
    if a is None:
        return None
    return a.ctypes.data_as(ctype)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _i64(a):
    return np.ascontiguousarray(a, dtype=np.int64)


# velocity(state*, rows, channels, 1000 t, conditional, velocity*, user) -> nonzero ok
VELOCITY_FN = C.CFUNCTYPE(C.c_int, _f32p, C.c_int64, C.c_int, C.c_float, C.c_int, _f32p, _vp)


def velocity_callback(fn):
    """Wrap fn(state [rows, ch] float32, t_model, conditional) -> velocity array
    as a C callback (keep the returned object alive while it is used)."""

    def cb(state_p, rows, channels, t_model, cond, out_p, _user):
        try:
            n = int(rows) * int(channels)
            state = np.ctypeslib.as_array(state_p, shape=(n,)).reshape(int(rows), int(channels))
            out = np.ctypeslib.as_array(out_p, shape=(n,)).reshape(int(rows), int(channels))
            out[...] = np.asarray(fn(state.copy(), np.float32(t_model), bool(cond)), np.float32)
            return 1
        except Exception:  # reported to the caller as a failed callback
            return 0

    return VELOCITY_FN(cb)


def build_oracle() -> None:
    """Compile build/liboracle.so (and _ref/ when /root/reference exists)."""
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE), "oracle"], check=True)
    if Path(os.environ.get("PXS_REFERENCE", "/root/reference"), "src", "sparse.cpp").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


class Oracle:
    """The C++ restatement of the reference CPU path (pxs_oracle.cpp)."""

    def __init__(self, path: Path = ORACLE_LIB):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} is not built; run make -C oracle")
        self.lib = L = C.CDLL(str(path))
        L.orc_sparse_valid.restype = C.c_int
        L.orc_sparse_valid.argtypes = [_i32p, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_int,
                                       _f32p, C.c_int64, C.c_int, _i64p]
        L.orc_neighbor_map_k3.argtypes = [_i32p, C.c_int64, _i32p]
        L.orc_neighbor_pairs.argtypes = [_i32p, C.c_int64, _i32p, _i32p, _i64p]
        L.orc_subm_conv3d.argtypes = [_i32p, C.c_int64, _f32p, C.c_int, _f32p, _f32p, C.c_int,
                                      _f32p]
        L.orc_downsample_coords_s2.restype = C.c_int64
        L.orc_downsample_coords_s2.argtypes = [_i32p, C.c_int64, _i32p, _i32p]
        L.orc_sparse_conv3d_s2.argtypes = [_i32p, C.c_int64, _f32p, C.c_int, _f32p, _f32p,
                                           C.c_int, _f32p]
        L.orc_downsample_mean.restype = C.c_int64
        L.orc_downsample_mean.argtypes = [_i32p, C.c_int64, _f32p, C.c_int, C.c_int, _i32p,
                                          _f32p]
        L.orc_channel_to_spatial.restype = C.c_int64
        L.orc_channel_to_spatial.argtypes = [_i32p, C.c_int64, _f32p, C.c_int, C.c_int, _f32p,
                                             _i32p, _f32p]
        L.orc_linear.argtypes = [_f32p, C.c_int64, C.c_int, _f32p, _f32p, C.c_int, _f32p]
        L.orc_layer_norm.argtypes = [_f32p, C.c_int64, C.c_int, C.c_float, _f32p, _f32p, _f32p]
        L.orc_mh_rms_norm.argtypes = [_f32p, C.c_int64, C.c_int, C.c_int, _f32p, _f32p]
        L.orc_rope.argtypes = [_i32p, _f32p, C.c_int64, C.c_int, C.c_int, C.c_float, C.c_float,
                               _f32p]
        L.orc_varlen_attention.argtypes = [_f32p, _f32p, _f32p, _i64p, _i64p, C.c_int, C.c_int,
                                           C.c_int, C.c_int, C.c_float, _f32p, _i64p, C.c_int64]
        L.orc_batch_cu_seqlens.argtypes = [_i32p, C.c_int64, C.c_int, _i64p]
        L.orc_window_partition.restype = C.c_int64
        L.orc_window_partition.argtypes = [_i32p, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_int,
                                           C.c_int, _i32p, _i32p, _i64p]
        L.orc_modulate.argtypes = [_i32p, _f32p, C.c_int64, C.c_int, _f32p, _f32p, C.c_int,
                                   _f32p]
        L.orc_gate.argtypes = [_i32p, _f32p, C.c_int64, C.c_int, _f32p, _f32p, C.c_int]
        L.orc_gelu_tanh.argtypes = [_f32p, C.c_int64]
        L.orc_silu.argtypes = [_f32p, C.c_int64]
        L.orc_transformer_block.argtypes = [_i32p, C.c_int64, C.c_int, _f32p, _f32p, _f32p,
                                            _i64p, _f32p, _intp, _f32p, C.POINTER(_f32p),
                                            _f32p, _i64p, C.c_int64]
        L.orc_timestep_embedding.argtypes = [_f32p, C.c_int64, C.c_int, C.c_int, _f32p]
        L.orc_timestep_embed_mlp.argtypes = [_f32p, C.c_int64, C.c_int, C.c_int, _f32p, _f32p,
                                             _f32p, _f32p, _f32p]
        L.orc_slat_flow_forward.argtypes = [_i32p, C.c_int64, C.c_int, _f32p, _f32p, _f32p,
                                            _i64p, _intp, _f32p, C.POINTER(_f32p),
                                            C.POINTER(_f32p), _f32p, _i64p, C.c_int64]
        L.orc_convnext_block.argtypes = [_i32p, C.c_int64, _f32p, C.c_int, C.c_int, C.c_float,
                                         C.POINTER(_f32p), _f32p]
        L.orc_resblock_c2s.restype = C.c_int64
        L.orc_resblock_c2s.argtypes = [_i32p, C.c_int64, _f32p, C.c_int, C.c_int, C.c_float,
                                       _f32p, C.POINTER(_f32p), _i32p, _f32p]
        L.orc_thread_count.restype = C.c_int
        L.orc_flow_schedule.restype = C.c_int
        L.orc_flow_schedule.argtypes = [C.c_int, _f32p, C.c_int, _f32p, _f32p, _f32p]
        L.orc_flow_guidance.restype = C.c_int
        L.orc_flow_guidance.argtypes = [_f32p, _f32p, _f32p, _i32p, C.c_int64, C.c_int, C.c_int,
                                        C.c_float, C.c_float, C.c_float, C.c_float, _f32p]
        L.orc_flow_euler_sample.restype = C.c_int
        L.orc_flow_euler_sample.argtypes = [_i32p, C.c_int64, C.c_int, C.c_int, _f32p, C.c_int,
                                            _f32p, VELOCITY_FN, _vp, _f32p, _f32p, _f32p]

    # -- validation and topology -------------------------------------------
    def sparse_valid(self, coords, batch_size, shape, feats, channels):
        coords, feats = _i32(coords).reshape(-1, 4), _f32(feats).reshape(-1)
        bad = C.c_int64(-1)
        code = self.lib.orc_sparse_valid(_p(coords, _i32p), coords.shape[0], batch_size,
                                         shape[0], shape[1], shape[2], _p(feats, _f32p),
                                         feats.size, channels, C.byref(bad))
        return code, bad.value

    def neighbor_map(self, coords):
        coords = _i32(coords).reshape(-1, 4)
        n = coords.shape[0]
        idx = np.empty((27, n), np.int32)
        self.lib.orc_neighbor_map_k3(_p(coords, _i32p), n, _p(idx, _i32p))
        return idx

    def neighbor_pairs(self, idx):
        idx = _i32(idx)
        n = idx.shape[1]
        offsets = np.zeros(28, np.int64)
        self.lib.orc_neighbor_pairs(_p(idx, _i32p), n, None, None, _p(offsets, _i64p))
        total = int(offsets[27])
        pin, pout = np.empty(total, np.int32), np.empty(total, np.int32)
        self.lib.orc_neighbor_pairs(_p(idx, _i32p), n, _p(pin, _i32p), _p(pout, _i32p),
                                    _p(offsets, _i64p))
        return pin, pout, offsets

    def batch_cu_seqlens(self, coords, batch_size):
        coords = _i32(coords).reshape(-1, 4)
        cu = np.zeros(batch_size + 1, np.int64)
        self.lib.orc_batch_cu_seqlens(_p(coords, _i32p), coords.shape[0], batch_size,
                                      _p(cu, _i64p))
        return cu

    def window_partition(self, coords, shape, window, shift):
        coords = _i32(coords).reshape(-1, 4)
        n = coords.shape[0]
        fwd, bwd = np.empty(n, np.int32), np.empty(n, np.int32)
        cu = np.zeros(n + 1, np.int64)
        nwin = self.lib.orc_window_partition(_p(coords, _i32p), n, shape[0], shape[1], shape[2],
                                             window, shift, _p(fwd, _i32p), _p(bwd, _i32p),
                                             _p(cu, _i64p))
        return fwd, bwd, cu[: nwin + 1].copy()

    # -- convolution --------------------------------------------------------
    def subm_conv3d(self, coords, feats, weight, bias):
        coords, feats = _i32(coords).reshape(-1, 4), _f32(feats)
        weight, bias = _f32(weight), _f32(bias)
        n, cin = feats.shape
        cout = bias.shape[0]
        assert weight.shape == (27, cout, cin)
        out = np.empty((n, cout), np.float32)
        self.lib.orc_subm_conv3d(_p(coords, _i32p), n, _p(feats, _f32p), cin, _p(weight, _f32p),
                                 _p(bias, _f32p), cout, _p(out, _f32p))
        return out

    def downsample_coords_s2(self, coords):
        coords = _i32(coords).reshape(-1, 4)
        n = coords.shape[0]
        oc = np.empty((n, 4), np.int32)
        child = np.empty((n, 8), np.int32)
        m = self.lib.orc_downsample_coords_s2(_p(coords, _i32p), n, _p(oc, _i32p),
                                              _p(child, _i32p))
        return oc[:m].copy(), child[:m].copy()

    def sparse_conv3d_s2(self, child_rows, feats, weight, bias):
        child_rows, feats = _i32(child_rows), _f32(feats)
        weight, bias = _f32(weight), _f32(bias)
        m = child_rows.shape[0]
        cin, cout = feats.shape[1], bias.shape[0]
        assert weight.shape == (8, cout, cin)
        out = np.empty((m, cout), np.float32)
        self.lib.orc_sparse_conv3d_s2(_p(child_rows, _i32p), m, _p(feats, _f32p), cin,
                                      _p(weight, _f32p), _p(bias, _f32p), cout, _p(out, _f32p))
        return out

    def downsample_mean(self, coords, feats, factor):
        coords, feats = _i32(coords).reshape(-1, 4), _f32(feats)
        n, ch = feats.shape
        oc = np.empty((n, 4), np.int32)
        of = np.empty((n, ch), np.float32)
        m = self.lib.orc_downsample_mean(_p(coords, _i32p), n, _p(feats, _f32p), ch, factor,
                                         _p(oc, _i32p), _p(of, _f32p))
        return oc[:m].copy(), of[:m].copy()

    def channel_to_spatial(self, coords, feats, factor, subdivision=None):
        coords, feats = _i32(coords).reshape(-1, 4), _f32(feats)
        n, ch = feats.shape
        children = factor ** 3
        sub = None if subdivision is None else _f32(subdivision)
        oc = np.empty((n * children, 4), np.int32)
        of = np.empty((n * children, ch // children), np.float32)
        m = self.lib.orc_channel_to_spatial(_p(coords, _i32p), n, _p(feats, _f32p), ch, factor,
                                            _p(sub, _f32p), _p(oc, _i32p), _p(of, _f32p))
        return oc[:m].copy(), of[:m].copy()

    # -- dense per-row ops ---------------------------------------------------
    def linear(self, x, weight, bias):
        x, weight, bias = _f32(x), _f32(weight), _f32(bias)
        rows, cin = x.shape
        cout = weight.shape[0]
        y = np.empty((rows, cout), np.float32)
        self.lib.orc_linear(_p(x, _f32p), rows, cin, _p(weight, _f32p), _p(bias, _f32p), cout,
                            _p(y, _f32p))
        return y

    def layer_norm(self, x, eps, gamma=None, beta=None):
        x = _f32(x)
        g = None if gamma is None else _f32(gamma)
        b = None if beta is None else _f32(beta)
        y = np.empty_like(x)
        self.lib.orc_layer_norm(_p(x, _f32p), x.shape[0], x.shape[1], eps, _p(g, _f32p),
                                _p(b, _f32p), _p(y, _f32p))
        return y

    def mh_rms_norm(self, x, heads, head_dim, gamma):
        x, gamma = _f32(x), _f32(gamma)
        y = np.empty_like(x)
        self.lib.orc_mh_rms_norm(_p(x, _f32p), x.shape[0], heads, head_dim, _p(gamma, _f32p),
                                 _p(y, _f32p))
        return y

    def rope(self, coords, x, heads, head_dim, freq_min=1.0, freq_base=10000.0):
        coords, x = _i32(coords).reshape(-1, 4), _f32(x)
        y = np.empty_like(x)
        self.lib.orc_rope(_p(coords, _i32p), _p(x, _f32p), x.shape[0], heads, head_dim, freq_min,
                          freq_base, _p(y, _f32p))
        return y

    def varlen_attention(self, q, k, v, cu_q, cu_k, heads, head_dim, scale, rows=None,
                         v_head_dim=None):
        q, k, v = _f32(q), _f32(k), _f32(v)
        cu_q, cu_k = _i64(cu_q), _i64(cu_k)
        vhd = v_head_dim or v.shape[1] // heads
        out = np.zeros((q.shape[0], heads * vhd), np.float32)
        r = None if rows is None else _i64(rows)
        self.lib.orc_varlen_attention(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), _p(cu_q, _i64p),
                                      _p(cu_k, _i64p), len(cu_q) - 1, heads, head_dim, vhd,
                                      scale, _p(out, _f32p), _p(r, _i64p),
                                      0 if r is None else r.size)
        return out

    def modulate(self, coords, x, block_mod, t_mod, offset):
        coords, x = _i32(coords).reshape(-1, 4), _f32(x)
        block_mod, t_mod = _f32(block_mod), _f32(t_mod)
        y = np.empty_like(x)
        self.lib.orc_modulate(_p(coords, _i32p), _p(x, _f32p), x.shape[0], x.shape[1],
                              _p(block_mod, _f32p), _p(t_mod, _f32p), offset, _p(y, _f32p))
        return y

    def gate(self, coords, x, block_mod, t_mod, offset):
        coords = _i32(coords).reshape(-1, 4)
        y = _f32(x).copy()
        block_mod, t_mod = _f32(block_mod), _f32(t_mod)
        self.lib.orc_gate(_p(coords, _i32p), _p(y, _f32p), y.shape[0], y.shape[1],
                          _p(block_mod, _f32p), _p(t_mod, _f32p), offset)
        return y

    def gelu_tanh(self, x):
        y = _f32(x).copy()
        self.lib.orc_gelu_tanh(_p(y, _f32p), y.size)
        return y

    def silu(self, x):
        y = _f32(x).copy()
        self.lib.orc_silu(_p(y, _f32p), y.size)
        return y

    # -- compositions ---------------------------------------------------------
    def transformer_block(self, coords, batch_size, x, t_mod, ctx, ctx_offsets, cfg_i, cfg_f,
                          weights, projected=None, rows=None):
        coords, x, t_mod, ctx = _i32(coords).reshape(-1, 4), _f32(x), _f32(t_mod), _f32(ctx)
        ctx_offsets = _i64(ctx_offsets)
        cfg_i_a = (C.c_int * 9)(*cfg_i)
        cfg_f_a = (C.c_float * 3)(*cfg_f)
        keep = [None if w is None else _f32(w) for w in weights]
        wp = (_f32p * 23)(*[_p(w, _f32p) if w is not None else None for w in keep])
        proj = None if projected is None else _f32(projected)
        r = None if rows is None else _i64(rows)
        out = np.empty_like(x)
        self.lib.orc_transformer_block(_p(coords, _i32p), coords.shape[0], batch_size,
                                       _p(x, _f32p), _p(t_mod, _f32p), _p(ctx, _f32p),
                                       _p(ctx_offsets, _i64p), _p(proj, _f32p), cfg_i_a, cfg_f_a,
                                       wp, _p(out, _f32p), _p(r, _i64p),
                                       0 if r is None else r.size)
        return out

    def timestep_embedding(self, t, dim, max_period=10000):
        t = _f32(t)
        out = np.empty((t.size, dim), np.float32)
        self.lib.orc_timestep_embedding(_p(t, _f32p), t.size, dim, max_period, _p(out, _f32p))
        return out

    def timestep_embed_mlp(self, t, hidden, freq_dim, w0, b0, w2, b2):
        t = _f32(t)
        ws = [_f32(a) for a in (w0, b0, w2, b2)]
        out = np.empty((t.size, hidden), np.float32)
        self.lib.orc_timestep_embed_mlp(_p(t, _f32p), t.size, hidden, freq_dim,
                                        *[_p(a, _f32p) for a in ws], _p(out, _f32p))
        return out

    def slat_flow_forward(self, coords, batch_size, x, timesteps, ctx, ctx_offsets, dims, cfg_f,
                          flow_weights, block_weights, rows=None):
        coords, x = _i32(coords).reshape(-1, 4), _f32(x)
        timesteps, ctx, ctx_offsets = _f32(timesteps), _f32(ctx), _i64(ctx_offsets)
        fw_keep = [_f32(a) for a in flow_weights]
        bw_keep = [None if a is None else _f32(a) for blk in block_weights for a in blk]
        fw = (_f32p * 10)(*[_p(a, _f32p) for a in fw_keep])
        bw = (_f32p * len(bw_keep))(*[None if a is None else _p(a, _f32p) for a in bw_keep])
        dims_a = (C.c_int * 9)(*dims)
        cfg_f_a = (C.c_float * 3)(*cfg_f)
        out = np.empty((x.shape[0], dims[2]), np.float32)
        r = None if rows is None else _i64(rows)
        self.lib.orc_slat_flow_forward(_p(coords, _i32p), coords.shape[0], batch_size,
                                       _p(x, _f32p), _p(timesteps, _f32p), _p(ctx, _f32p),
                                       _p(ctx_offsets, _i64p), dims_a, cfg_f_a, fw, bw,
                                       _p(out, _f32p), _p(r, _i64p), 0 if r is None else r.size)
        return out

    def convnext_block(self, coords, x, mlp_hidden, eps, weights):
        coords, x = _i32(coords).reshape(-1, 4), _f32(x)
        keep = [_f32(a) for a in weights]
        wp = (_f32p * 8)(*[_p(a, _f32p) for a in keep])
        out = np.empty_like(x)
        self.lib.orc_convnext_block(_p(coords, _i32p), coords.shape[0], _p(x, _f32p), x.shape[1],
                                    mlp_hidden, eps, wp, _p(out, _f32p))
        return out

    def resblock_c2s(self, coords, x, out_channels, eps, weights, subdivision=None):
        coords, x = _i32(coords).reshape(-1, 4), _f32(x)
        n = coords.shape[0]
        keep = [_f32(a) for a in weights]
        wp = (_f32p * 6)(*[_p(a, _f32p) for a in keep])
        sub = None if subdivision is None else _f32(subdivision)
        oc = np.empty((8 * n, 4), np.int32)
        out = np.empty((8 * n, out_channels), np.float32)
        m = self.lib.orc_resblock_c2s(_p(coords, _i32p), n, _p(x, _f32p), x.shape[1],
                                      out_channels, eps, _p(sub, _f32p), wp, _p(oc, _i32p),
                                      _p(out, _f32p))
        return oc[:m].copy(), out[:m].copy()

    def thread_count(self) -> int:
        return int(self.lib.orc_thread_count())

    # -- flow Euler sampler ------------------------------------------------------
    def flow_schedule(self, steps, cfg_f, step):
        """(code, t, t_next, guidance); cfg_f = [sigma_min, rescale_t, strength,
        rescale, interval_min, interval_max]."""
        cf = _f32(cfg_f)
        t, tn, g = (np.zeros(1, np.float32) for _ in range(3))
        rc = self.lib.orc_flow_schedule(steps, _p(cf, _f32p), step, _p(t, _f32p), _p(tn, _f32p),
                                        _p(g, _f32p))
        return int(rc), t[0], tn[0], g[0]

    def flow_guidance(self, state, pos, neg, coords, batch_size, t, sigma_min, guidance, rescale):
        state, pos, neg = _f32(state), _f32(pos), _f32(neg)
        coords = _i32(coords).reshape(-1, 4)
        pred = np.empty_like(state)
        rc = self.lib.orc_flow_guidance(_p(state, _f32p), _p(pos, _f32p), _p(neg, _f32p),
                                        _p(coords, _i32p), coords.shape[0], state.shape[1],
                                        batch_size, t, sigma_min, guidance, rescale,
                                        _p(pred, _f32p))
        if rc:
            raise ValueError(f"orc_flow_guidance failed with code {rc}")
        return pred

    def flow_euler_sample(self, coords, batch_size, noise, steps, cfg_f, fn, record=False):
        """-> (samples, traj_xt or None, traj_x0 or None); fn as for velocity_callback."""
        coords, noise, cf = _i32(coords).reshape(-1, 4), _f32(noise), _f32(cfg_f)
        rows, ch = noise.shape
        out = np.empty_like(noise)
        xt = np.empty((steps, rows, ch), np.float32) if record else None
        x0 = np.empty((steps, rows, ch), np.float32) if record else None
        cb = velocity_callback(fn)
        rc = self.lib.orc_flow_euler_sample(_p(coords, _i32p), rows, ch, batch_size,
                                            _p(noise, _f32p), steps, _p(cf, _f32p), cb, None,
                                            _p(out, _f32p), _p(xt, _f32p), _p(x0, _f32p))
        if rc:
            raise ValueError(f"orc_flow_euler_sample failed with code {rc}")
        return out, xt, x0


class RefSparse:
    """An owned reference SparseTensorF32 handle."""

    def __init__(self, ref: "Reference", handle):
        self.ref, self.h = ref, handle

    def __del__(self):
        try:
            self.ref.lib.ref_sparse_free(self.h)
        except Exception:
            pass

    def shape(self):
        s = np.zeros(6, np.int64)
        self.ref.lib.ref_sparse_shape(self.h, _p(s, _i64p))
        return s

    def read(self):
        s = self.shape()
        n, ch = int(s[0]), int(s[1])
        coords = np.empty((n, 4), np.int32)
        feats = np.empty((n, ch), np.float32)
        self.ref.lib.ref_sparse_read(self.h, _p(coords, _i32p), _p(feats, _f32p))
        return coords, feats


class RefVarLen:
    def __init__(self, ref: "Reference", handle):
        self.ref, self.h = ref, handle

    def __del__(self):
        try:
            self.ref.lib.ref_varlen_free(self.h)
        except Exception:
            pass

    def read(self):
        s = np.zeros(3, np.int64)
        self.ref.lib.ref_varlen_shape(self.h, _p(s, _i64p))
        out = np.empty((int(s[0]), int(s[1])), np.float32)
        self.ref.lib.ref_varlen_read(self.h, _p(out, _f32p))
        return out


class ReferenceError(RuntimeError):
    pass


class Reference:
    """The reference's compiled CPU primitives (oracle/_ref/libpixal3d_ref.so)."""

    def __init__(self, path: Path = REF_LIB):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} is not built (needs /root/reference)")
        self.lib = L = C.CDLL(str(path))
        L.ref_sparse_new.restype = _vp
        L.ref_sparse_new.argtypes = [_i32p, C.c_int64, C.c_int, C.c_int, C.c_int, C.c_int, _f32p,
                                     C.c_int]
        L.ref_sparse_empty.restype = _vp
        L.ref_sparse_free.argtypes = [_vp]
        L.ref_sparse_shape.argtypes = [_vp, _i64p]
        L.ref_sparse_read.argtypes = [_vp, _i32p, _f32p]
        L.ref_varlen_new.restype = _vp
        L.ref_varlen_new.argtypes = [C.c_int, C.c_int, _i64p, _f32p]
        L.ref_varlen_empty.restype = _vp
        L.ref_varlen_free.argtypes = [_vp]
        L.ref_varlen_shape.argtypes = [_vp, _i64p]
        L.ref_varlen_read.argtypes = [_vp, _f32p]
        # The drop-in build of the shim has no thread or timestep entry points.
        self.has_threads = hasattr(L, "ref_cpu_thread_count")
        if self.has_threads:
            L.ref_cpu_thread_count.restype = C.c_int
            L.ref_set_cpu_threads.argtypes = [C.c_int]
        eb = [C.c_char_p, C.c_int]
        L.ref_sparse_valid.argtypes = [_vp] + eb
        L.ref_varlen_valid.argtypes = [_vp] + eb
        L.ref_sparse_linear.argtypes = [_vp, _f32p, _f32p, C.c_int, _vp] + eb
        L.ref_varlen_linear.argtypes = [_vp, _f32p, _f32p, C.c_int, _vp] + eb
        L.ref_sparse_layer_norm.argtypes = [_vp, C.c_float, _f32p, _f32p, _vp] + eb
        L.ref_sparse_downsample_mean.argtypes = [_vp, C.c_int, _vp] + eb
        L.ref_sparse_channel_to_spatial.argtypes = [_vp, C.c_int, _vp, _vp] + eb
        L.ref_sparse_sdpa.argtypes = [_vp, _vp, _vp, C.c_int, C.c_int, C.c_float, _vp] + eb
        L.ref_sparse_cross_attention.argtypes = [_vp, _vp, _vp, C.c_int, C.c_int, C.c_float,
                                                 _vp] + eb
        L.ref_sparse_rope.argtypes = [_vp, C.c_int, C.c_int, C.c_float, C.c_float, _vp] + eb
        L.ref_sparse_mh_rms_norm.argtypes = [_vp, C.c_int, C.c_int, _f32p, _vp] + eb
        L.ref_varlen_mh_rms_norm.argtypes = [_vp, C.c_int, C.c_int, _f32p, _vp] + eb
        L.ref_sparse_submanifold_conv3d.argtypes = [_vp, _f32p, _f32p, C.c_int, _vp] + eb
        L.ref_transformer_block.argtypes = [_vp, _f32p, _vp, _vp, _intp, _f32p,
                                            C.POINTER(_f32p), _vp] + eb
        L.ref_flow_euler_sample.argtypes = [_vp, _intp, _f32p, VELOCITY_FN, _vp, _vp, _f32p,
                                            _f32p] + eb
        if self.has_threads:
            L.ref_timestep_embedding.argtypes = [_f32p, C.c_int64, C.c_int, C.c_int, _f32p] + eb
            L.ref_timestep_embed_mlp.argtypes = [_f32p, C.c_int64, C.c_int, C.c_int, _f32p,
                                                 _f32p, _f32p, _f32p, _f32p] + eb
        for name in ("ref_sparse_valid", "ref_varlen_valid", "ref_sparse_linear",
                     "ref_varlen_linear", "ref_sparse_layer_norm", "ref_sparse_downsample_mean",
                     "ref_sparse_channel_to_spatial", "ref_sparse_sdpa",
                     "ref_sparse_cross_attention", "ref_sparse_rope", "ref_sparse_mh_rms_norm",
                     "ref_varlen_mh_rms_norm", "ref_sparse_submanifold_conv3d",
                     "ref_transformer_block", "ref_timestep_embedding",
                     "ref_timestep_embed_mlp", "ref_flow_euler_sample"):
            if hasattr(L, name):
                getattr(L, name).restype = C.c_int

    # -- handles ---------------------------------------------------------------
    def sparse(self, coords, feats, batch_size, shape, channels=None):
        coords = _i32(coords).reshape(-1, 4)
        f = None if feats is None else _f32(feats).reshape(coords.shape[0], -1)
        ch = channels if channels is not None else (f.shape[1] if f is not None else 0)
        h = self.lib.ref_sparse_new(_p(coords, _i32p), coords.shape[0], batch_size, shape[0],
                                    shape[1], shape[2], _p(f, _f32p), ch)
        return RefSparse(self, h)

    def empty(self):
        return RefSparse(self, self.lib.ref_sparse_empty())

    def varlen(self, offsets, feats, batch_size=None):
        offsets = _i64(offsets)
        f = _f32(feats)
        b = batch_size if batch_size is not None else offsets.size - 1
        return RefVarLen(self, self.lib.ref_varlen_new(b, f.shape[1], _p(offsets, _i64p),
                                                       _p(f, _f32p)))

    def varlen_empty(self):
        return RefVarLen(self, self.lib.ref_varlen_empty())

    def set_threads(self, threads: int) -> None:
        self.lib.ref_set_cpu_threads(threads)

    def thread_count(self) -> int:
        return int(self.lib.ref_cpu_thread_count())

    def _call(self, name, *args):
        err = C.create_string_buffer(512)
        ok = getattr(self.lib, name)(*args, err, 512)
        if not ok:
            raise ReferenceError(err.value.decode())

    # -- operations --------------------------------------------------------------
    def valid(self, t: RefSparse):
        err = C.create_string_buffer(512)
        ok = self.lib.ref_sparse_valid(t.h, err, 512)
        return bool(ok), err.value.decode()

    def varlen_valid(self, t: RefVarLen):
        err = C.create_string_buffer(512)
        ok = self.lib.ref_varlen_valid(t.h, err, 512)
        return bool(ok), err.value.decode()

    def linear(self, t, weight, bias, out=None):
        weight, bias = _f32(weight), _f32(bias)
        out = self.empty() if out is None else out
        self._call("ref_sparse_linear", t.h, _p(weight, _f32p), _p(bias, _f32p), bias.size, out.h)
        return out

    def varlen_linear(self, t, weight, bias):
        weight, bias = _f32(weight), _f32(bias)
        out = self.varlen_empty()
        self._call("ref_varlen_linear", t.h, _p(weight, _f32p), _p(bias, _f32p), bias.size, out.h)
        return out

    def layer_norm(self, t, eps, gamma=None, beta=None):
        g = None if gamma is None else _f32(gamma)
        b = None if beta is None else _f32(beta)
        out = self.empty()
        self._call("ref_sparse_layer_norm", t.h, eps, _p(g, _f32p), _p(b, _f32p), out.h)
        return out

    def downsample_mean(self, t, factor):
        out = self.empty()
        self._call("ref_sparse_downsample_mean", t.h, factor, out.h)
        return out

    def channel_to_spatial(self, t, factor, subdivision=None):
        out = self.empty()
        self._call("ref_sparse_channel_to_spatial", t.h, factor,
                   None if subdivision is None else subdivision.h, out.h)
        return out

    def sdpa(self, q, k, v, heads, head_dim, scale):
        out = self.empty()
        self._call("ref_sparse_sdpa", q.h, k.h, v.h, heads, head_dim, scale, out.h)
        return out

    def cross_attention(self, q, k, v, heads, head_dim, scale):
        out = self.empty()
        self._call("ref_sparse_cross_attention", q.h, k.h, v.h, heads, head_dim, scale, out.h)
        return out

    def rope(self, t, heads, head_dim, fmin=1.0, fbase=10000.0):
        out = self.empty()
        self._call("ref_sparse_rope", t.h, heads, head_dim, fmin, fbase, out.h)
        return out

    def mh_rms_norm(self, t, heads, head_dim, gamma):
        gamma = _f32(gamma)
        out = self.empty()
        self._call("ref_sparse_mh_rms_norm", t.h, heads, head_dim, _p(gamma, _f32p), out.h)
        return out

    def varlen_mh_rms_norm(self, t, heads, head_dim, gamma):
        gamma = _f32(gamma)
        out = self.varlen_empty()
        self._call("ref_varlen_mh_rms_norm", t.h, heads, head_dim, _p(gamma, _f32p), out.h)
        return out

    def subm_conv3d(self, t, weight, bias):
        weight, bias = _f32(weight), _f32(bias)
        out = self.empty()
        self._call("ref_sparse_submanifold_conv3d", t.h, _p(weight, _f32p), _p(bias, _f32p),
                   bias.size, out.h)
        return out

    def transformer_block(self, t, t_mod, ctx: RefVarLen, cfg_i, cfg_f, weights, projected=None,
                          out=None):
        t_mod = _f32(t_mod)
        cfg_i_a = (C.c_int * 9)(*cfg_i)
        cfg_f_a = (C.c_float * 3)(*cfg_f)
        keep = [None if w is None else _f32(w) for w in weights]
        wp = (_f32p * 23)(*[None if w is None else _p(w, _f32p) for w in keep])
        out = self.empty() if out is None else out
        self._call("ref_transformer_block", t.h, _p(t_mod, _f32p), ctx.h,
                   None if projected is None else projected.h, cfg_i_a, cfg_f_a, wp, out.h)
        return out

    def flow_euler_sample(self, noise: "RefSparse", steps, cfg_f, fn, record=False):
        """flow_euler_sample_f32 with fn as the velocity (see velocity_callback);
        -> (samples RefSparse, traj_xt or None, traj_x0 or None)."""
        shape = noise.shape()
        rows, ch = int(shape[0]), int(shape[1])
        cfg_i = (C.c_int * 2)(steps, 1 if record else 0)
        cf = _f32(cfg_f)
        xt = np.empty((max(steps, 1), rows, ch), np.float32) if record else None
        x0 = np.empty((max(steps, 1), rows, ch), np.float32) if record else None
        out = self.empty()
        cb = velocity_callback(fn) if fn is not None else VELOCITY_FN()
        self._call("ref_flow_euler_sample", noise.h, cfg_i, _p(cf, _f32p), cb, None, out.h,
                   _p(xt, _f32p), _p(x0, _f32p))
        return out, xt, x0

    def timestep_embedding(self, t, dim, max_period=10000):
        t = _f32(t)
        out = np.empty((t.size, dim), np.float32)
        self._call("ref_timestep_embedding", _p(t, _f32p), t.size, dim, max_period,
                   _p(out, _f32p))
        return out

    def timestep_embed_mlp(self, t, hidden, freq_dim, w0, b0, w2, b2):
        t = _f32(t)
        ws = [_f32(a) for a in (w0, b0, w2, b2)]
        out = np.empty((t.size, hidden), np.float32)
        self._call("ref_timestep_embed_mlp", _p(t, _f32p), t.size, hidden, freq_dim,
                   *[_p(a, _f32p) for a in ws], _p(out, _f32p))
        return out


class DropIn(Reference):
    """The MI355X drop-in (libpxs.so) behind the same shim
    (build/libdropin_shim.so).  Calls need a GPU; loading does not."""

    def __init__(self, path: Path = DROPIN_LIB):
        super().__init__(path)

    def pack_reader_case(self, path, tensor, u32_key, capacity=1 << 20):
        """dropin_pack_reader_case (host only, no GPU): the drop-in
        Pixal3DPackReader driven as tests/test_pack_reader.cpp drives the
        reference's -> ({key: (flag, text) or value}, tensor bytes)."""
        fn = self.lib.dropin_pack_reader_case
        fn.restype = C.c_int
        fn.argtypes = [C.c_char_p, C.c_char_p, C.c_char_p, _vp, C.c_size_t, C.c_char_p, C.c_int]
        out = C.create_string_buffer(capacity)
        report = C.create_string_buffer(1 << 16)
        fn(str(path).encode(), tensor.encode(), u32_key.encode(), out, capacity, report,
           len(report))
        result = {}
        for line in report.value.decode().splitlines():
            key, _, value = line.partition("=")
            flag, colon, text = value.partition(":")
            result[key] = (int(flag), text) if colon else int(value)
        n = result.get("bytes", 0)
        return result, out.raw[:n]
