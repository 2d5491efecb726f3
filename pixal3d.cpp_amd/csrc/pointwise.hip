// Row-wise HBM-bound kernels: layer norm (+ adaLN modulation), multi-head RMS
// norm, 3-D RoPE, the fused QKV prologue, and activations.
//
// One wavefront per row; per-row reductions use wavefront shuffles.  These
// kernels read each row once from HBM (later passes over the same row hit
// L1/L2), so their bound is HBM bandwidth: bytes = rows * C * (in + out).

#include "pxs_common.h"

#include <cmath>
#include <vector>

namespace pxs {
namespace {

constexpr int kRowsPerBlock = 4;  // 4 wavefronts of 64 lanes

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

template <typename TX, typename TY, bool kModulate>
__global__ void __launch_bounds__(64 * kRowsPerBlock)
layer_norm_kernel(const TX * __restrict__ x, int64_t rows, int channels, float eps,
                  const float * __restrict__ gamma, const float * __restrict__ beta,
                  const int32_t * __restrict__ coords, const float * __restrict__ block_mod,
                  const float * __restrict__ time_mod, int mod_offset, TY * __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const TX * src = x + row * channels;
    float s = 0.0f;
    for (int c = lane; c < channels; c += 64) s += load_f32(src + c);
    const float mean = wave_sum(s) / static_cast<float>(channels);
    float v = 0.0f;
    for (int c = lane; c < channels; c += 64) {
        const float d = load_f32(src + c) - mean;
        v += d * d;
    }
    const float var = wave_sum(v) / static_cast<float>(channels);
    const float inv = 1.0f / sqrtf(var + eps);
    TY * dst = y + row * channels;
    const float * tm = nullptr;
    if constexpr (kModulate) tm = time_mod + static_cast<int64_t>(coords[row * 4]) * 6 * channels;
    for (int c = lane; c < channels; c += 64) {
        float val = (load_f32(src + c) - mean) * inv;
        if (gamma) val = val * gamma[c] + beta[c];
        if constexpr (kModulate) {
            const float scale = block_mod[mod_offset + channels + c] + tm[mod_offset + channels + c];
            const float shift = block_mod[mod_offset + c] + tm[mod_offset + c];
            val = val * (1.0f + scale) + shift;
        }
        store_f32(dst + c, val);
    }
}

// Layer norm of rows that are L x NV 16-byte vectors wide: L lanes own a row
// (64 / L rows per wave), each lane loads NV vectors of 16 bytes, keeps them
// in registers and reduces over its L-lane group.  Rows of 64 bf16 channels
// (the decoder's finest levels, millions of rows) get 8 rows per wave instead
// of one, with 16-byte accesses.  Same two passes and formulas as
// layer_norm_kernel (mean, then the mean of squared deviations, then
// 1 / sqrt(var + eps)); only the summation order within a row differs.
template <int L>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int d = L / 2; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

template <typename T> struct Vec16;
template <> struct Vec16<float> {
    static constexpr int kN = 4;
    __device__ static void load(const float * p, float (&v)[4]) {
        const float4 q = *reinterpret_cast<const float4 *>(p);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    }
};
template <> struct Vec16<uint16_t> {
    static constexpr int kN = 8;
    __device__ static void load(const uint16_t * p, float (&v)[8]) {
        const uint4 q = *reinterpret_cast<const uint4 *>(p);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
};

template <typename TY, int N>
__device__ __forceinline__ void store_vec(TY * p, const float (&v)[N]) {
    if constexpr (sizeof(TY) == 4) {
#pragma unroll
        for (int i = 0; i < N; i += 4)
            *reinterpret_cast<float4 *>(p + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
    } else if constexpr (N == 8) {
        *reinterpret_cast<uint4 *>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                   pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
    } else {
        *reinterpret_cast<uint2 *>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
}

template <typename TX, typename TY, int L, int NV, bool kModulate>
__global__ void __launch_bounds__(256)
layer_norm_rows_kernel(const TX * __restrict__ x, int64_t rows, float eps,
                       const float * __restrict__ gamma, const float * __restrict__ beta,
                       const int32_t * __restrict__ coords, const float * __restrict__ block_mod,
                       const float * __restrict__ time_mod, int mod_offset, TY * __restrict__ y) {
    constexpr int V = Vec16<TX>::kN;
    constexpr int C = L * NV * V;
    const int lane = threadIdx.x & 63;
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * (64 / L) + lane / L;
    const int part = lane % L;
    const bool live = row < rows;  // every lane takes part in the group shuffles
    float v[NV][V];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (live) {
            Vec16<TX>::load(x + row * C + (j * L + part) * V, v[j]);
        } else {
#pragma unroll
            for (int e = 0; e < V; ++e) v[j][e] = 0.0f;
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < V; ++e) s += v[j][e];
    const float mean = group_sum<L>(s) / static_cast<float>(C);
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int e = 0; e < V; ++e) {
            const float d = v[j][e] - mean;
            q += d * d;
        }
    const float var = group_sum<L>(q) / static_cast<float>(C);
    const float inv = 1.0f / sqrtf(var + eps);
    if (!live) return;
    const float * tm = nullptr;
    if constexpr (kModulate) tm = time_mod + static_cast<int64_t>(coords[row * 4]) * 6 * C;
    // Per-channel vectors in 16-byte pieces that match the lane's data (the
    // row is 16-byte aligned and so are the channel offsets used here).
    auto load_v = [&](const float * p, float (&w)[V]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < V; q += 4) {
            const float4 f = *reinterpret_cast<const float4 *>(p + q);
            w[q] = f.x; w[q + 1] = f.y; w[q + 2] = f.z; w[q + 3] = f.w;
        }
    };
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int c0 = (j * L + part) * V;
        float o[V], ga[V], be[V], bs[V], ts[V], bh[V], th[V];
        if (gamma) {
            load_v(gamma + c0, ga);
            load_v(beta + c0, be);
        }
        if constexpr (kModulate) {
            load_v(block_mod + mod_offset + C + c0, bs);
            load_v(tm + mod_offset + C + c0, ts);
            load_v(block_mod + mod_offset + c0, bh);
            load_v(tm + mod_offset + c0, th);
        }
#pragma unroll
        for (int e = 0; e < V; ++e) {
            float val = (v[j][e] - mean) * inv;
            if (gamma) val = val * ga[e] + be[e];
            if constexpr (kModulate) {
                const float scale = bs[e] + ts[e];
                const float shift = bh[e] + th[e];
                val = val * (1.0f + scale) + shift;
            }
            o[e] = val;
        }
        store_vec<TY, V>(y + row * C + c0, o);
    }
}

// RoPE frequency table computed on the host exactly as the reference does
// (std::pow in float), passed by value.
struct RopeTable {
    int fdim;
    float freq[32];
};

RopeTable make_rope_table(int head_dim, float fmin, float fbase) {
    RopeTable t{};
    const int pairs = head_dim / 2;
    t.fdim = pairs / 3;
    for (int i = 0; i < t.fdim && i < 32; ++i) {
        t.freq[i] = fmin / std::pow(fbase, static_cast<float>(i) / static_cast<float>(t.fdim));
    }
    return t;
}

__device__ __forceinline__ void rope_pair(float e, float o, float phase, float & re, float & ro) {
    const float cs = cosf(phase), sn = sinf(phase);
    re = e * cs - o * sn;
    ro = e * sn + o * cs;
}

// Generic per-(row, head) kernel: optional RMS norm then optional RoPE.
// Handles any head_dim; used for the standalone entry points.
template <typename T>
__global__ void head_norm_rope_kernel(const T * __restrict__ x, int64_t ld_x, int64_t rows,
                                      int heads, int head_dim, const float * __restrict__ gamma,
                                      const int32_t * __restrict__ coords, RopeTable rope,
                                      T * __restrict__ y, int64_t ld_y) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= rows * heads) return;
    const int64_t row = t / heads;
    const int head = static_cast<int>(t - row * heads);
    const T * src = x + row * ld_x + head * head_dim;
    T * dst = y + row * ld_y + head * head_dim;
    float inv = 1.0f;
    const float mult = sqrtf(static_cast<float>(head_dim));
    if (gamma) {
        float sq = 0.0f;
        for (int d = 0; d < head_dim; ++d) {
            const float v = load_f32(src + d);
            sq += v * v;
        }
        inv = 1.0f / fmaxf(sqrtf(sq), 1e-12f);
    }
    const float * g = gamma ? gamma + head * head_dim : nullptr;
    if (coords) {
        const int xyz[3] = {coords[row * 4 + 1], coords[row * 4 + 2], coords[row * 4 + 3]};
        for (int p = 0; p < head_dim / 2; ++p) {
            float e = load_f32(src + 2 * p), o = load_f32(src + 2 * p + 1);
            if (g) {
                e = e * inv * mult * g[2 * p];
                o = o * inv * mult * g[2 * p + 1];
            }
            float phase = 0.0f;
            if (p < 3 * rope.fdim) phase = static_cast<float>(xyz[p / rope.fdim]) * rope.freq[p % rope.fdim];
            float re, ro;
            rope_pair(e, o, phase, re, ro);
            store_f32(dst + 2 * p, re);
            store_f32(dst + 2 * p + 1, ro);
        }
    } else {
        for (int d = 0; d < head_dim; ++d) {
            float v = load_f32(src + d);
            if (g) v = v * inv * mult * g[d];
            store_f32(dst + d, v);
        }
    }
}

// Fast path of the QKV prologue for head_dim == 64: one wavefront per row;
// each lane owns 8 consecutive dimensions (one 16-byte bf16 load, two for
// fp32), so 8 lanes hold a head and a wave covers 8 heads per pass.  The RMS
// norm reduces over the head's 8 lanes; RoPE pairs (2i, 2i+1) sit inside a
// lane, and the lane's 4 pair phases depend only on the row, so their
// sin/cos are computed once per row for every head of q and k.
template <typename T> struct Vec8;
template <> struct Vec8<uint16_t> {
    static __device__ __forceinline__ void load(const uint16_t * p, float (&v)[8]) {
        const uint4 u = *reinterpret_cast<const uint4 *>(p);
        const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    }
    static __device__ __forceinline__ void store(uint16_t * p, const float (&v)[8]) {
        uint4 u;
        u.x = pack_bf16x2(v[0], v[1]);
        u.y = pack_bf16x2(v[2], v[3]);
        u.z = pack_bf16x2(v[4], v[5]);
        u.w = pack_bf16x2(v[6], v[7]);
        *reinterpret_cast<uint4 *>(p) = u;
    }
    static __device__ __forceinline__ void copy(const uint16_t * src, uint16_t * dst) {
        *reinterpret_cast<uint4 *>(dst) = *reinterpret_cast<const uint4 *>(src);
    }
};
template <> struct Vec8<float> {
    static __device__ __forceinline__ void load(const float * p, float (&v)[8]) {
        const float4 a = *reinterpret_cast<const float4 *>(p);
        const float4 b = *reinterpret_cast<const float4 *>(p + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    static __device__ __forceinline__ void store(float * p, const float (&v)[8]) {
        *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4 *>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    static __device__ __forceinline__ void copy(const float * src, float * dst) {
        *reinterpret_cast<float4 *>(dst) = *reinterpret_cast<const float4 *>(src);
        *reinterpret_cast<float4 *>(dst + 4) = *reinterpret_cast<const float4 *>(src + 4);
    }
};

template <typename T>
__global__ void __launch_bounds__(64 * kRowsPerBlock)
qkv_prepare64_kernel(const T * __restrict__ qkv, int64_t rows, int heads,
                     const float * __restrict__ q_gamma, const float * __restrict__ k_gamma,
                     const int32_t * __restrict__ coords, RopeTable rope, T * __restrict__ q,
                     T * __restrict__ k, T * __restrict__ v) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int C = heads * 64;
    const T * src = qkv + row * 3 * C;
    const int sub = lane & 7;       // 8-dim slice of the head
    const int hl = lane >> 3;       // head within the pass
    float cs[4] = {1.0f, 1.0f, 1.0f, 1.0f}, sn[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (coords) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = sub * 4 + i;
            if (p < 3 * rope.fdim) {
                const float phase = static_cast<float>(coords[row * 4 + 1 + p / rope.fdim]) *
                                    rope.freq[p % rope.fdim];
                cs[i] = cosf(phase);
                sn[i] = sinf(phase);
            }
        }
    }
    for (int part = 0; part < 2; ++part) {
        const float * gamma = part == 0 ? q_gamma : k_gamma;
        T * dst = (part == 0 ? q : k) + row * C;
        for (int hb = 0; hb < heads; hb += 8) {
            const int h = hb + hl;
            // Heads past the end idle their lanes but still join the shuffles.
            const bool on = h < heads;
            const int d0 = (on ? h : 0) * 64 + sub * 8;
            float val[8];
            Vec8<T>::load(src + part * C + d0, val);
            if (gamma) {
                float sq = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) sq += val[i] * val[i];
                sq += __shfl_xor(sq, 1, 64);
                sq += __shfl_xor(sq, 2, 64);
                sq += __shfl_xor(sq, 4, 64);
                const float inv = 1.0f / fmaxf(sqrtf(sq), 1e-12f);
#pragma unroll
                for (int i = 0; i < 8; ++i) val[i] = val[i] * inv * 8.0f * gamma[d0 + i];  // sqrt(64) = 8
            }
            if (coords) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = val[2 * i], o = val[2 * i + 1];
                    val[2 * i] = e * cs[i] - o * sn[i];
                    val[2 * i + 1] = e * sn[i] + o * cs[i];
                }
            }
            if (on) Vec8<T>::store(dst + d0, val);
        }
    }
    T * vd = v + row * C;
    for (int c = lane * 8; c < C; c += 512) Vec8<T>::copy(src + 2 * C + c, vd + c);
}

// The standalone head RMS norm / RoPE (pxs_mh_rms_norm, pxs_rope) at
// head_dim 64: the QKV prologue's layout (one wavefront per row, 8 lanes of
// 8 dims per head, 8 heads per pass, the RMS over the head's 8 lanes, RoPE
// pairs lane-local with per-row sin/cos).  x may be y.
template <typename T>
__global__ void __launch_bounds__(64 * kRowsPerBlock)
head_op64_kernel(const T * __restrict__ x, int64_t ld_x, int64_t rows, int heads,
                 const float * __restrict__ gamma, const int32_t * __restrict__ coords,
                 RopeTable rope, T * __restrict__ y, int64_t ld_y) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int sub = lane & 7, hl = lane >> 3;
    float cs[4] = {1.0f, 1.0f, 1.0f, 1.0f}, sn[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (coords) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = sub * 4 + i;
            if (p < 3 * rope.fdim) {
                const float phase = static_cast<float>(coords[row * 4 + 1 + p / rope.fdim]) *
                                    rope.freq[p % rope.fdim];
                cs[i] = cosf(phase);
                sn[i] = sinf(phase);
            }
        }
    }
    for (int hb = 0; hb < heads; hb += 8) {
        const int h = hb + hl;
        const bool on = h < heads;  // idle lanes still join the shuffles
        const int d0 = (on ? h : 0) * 64 + sub * 8;
        float val[8];
        Vec8<T>::load(x + row * ld_x + d0, val);
        if (gamma) {
            float sq = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) sq += val[i] * val[i];
            sq += __shfl_xor(sq, 1, 64);
            sq += __shfl_xor(sq, 2, 64);
            sq += __shfl_xor(sq, 4, 64);
            const float inv = 1.0f / fmaxf(sqrtf(sq), 1e-12f);
#pragma unroll
            for (int i = 0; i < 8; ++i) val[i] = val[i] * inv * 8.0f * gamma[d0 + i];  // sqrt(64) = 8
        }
        if (coords) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = val[2 * i], o = val[2 * i + 1];
                val[2 * i] = e * cs[i] - o * sn[i];
                val[2 * i + 1] = e * sn[i] + o * cs[i];
            }
        }
        if (on) Vec8<T>::store(y + row * ld_y + d0, val);
    }
}

template <typename T>
__global__ void split_copy_kernel(const T * __restrict__ qkv, int64_t rows, int C, int part,
                                  T * __restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows * C;
         i += stride) {
        const int64_t r = i / C;
        out[i] = qkv[r * 3 * C + part * C + (i - r * C)];
    }
}

// 8 consecutive elements through 16-byte accesses (two for fp32): the
// elementwise kernels below take this path when the count is a multiple of 8
// and the buffers are 16-byte aligned, with the same per-element arithmetic
// as their one-element loops (so the same bits).
template <typename T> __device__ __forceinline__ void load8(const T * p, float (&v)[8]);
template <> __device__ __forceinline__ void load8<float>(const float * p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <> __device__ __forceinline__ void load8<uint16_t>(const uint16_t * p, float (&v)[8]) {
    const uint4 q = *reinterpret_cast<const uint4 *>(p);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
template <typename T> __device__ __forceinline__ void store8(T * p, const float (&v)[8]);
template <> __device__ __forceinline__ void store8<float>(float * p, const float (&v)[8]) {
    reinterpret_cast<float4 *>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4 *>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
template <> __device__ __forceinline__ void store8<uint16_t>(uint16_t * p, const float (&v)[8]) {
    *reinterpret_cast<uint4 *>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                               pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
}

inline bool vec8_ok(int64_t count, const void * a, const void * b = nullptr) {
    return count % 8 == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(b) & 15) == 0;
}

inline unsigned vec8_blocks(int64_t count) {
    return static_cast<unsigned>(std::min<int64_t>((count / 8 + 255) / 256, 16384));
}

template <typename T>
__global__ void activation8_kernel(T * __restrict__ x, int64_t nvec, int act) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nvec;
         i += stride) {
        float v[8];
        load8(x + 8 * i, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = act == PXS_ACT_GELU_TANH ? gelu_tanh_f(v[e]) : silu_f(v[e]);
        store8(x + 8 * i, v);
    }
}

template <typename T>
__global__ void activation_kernel(T * __restrict__ x, int64_t count, int act) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const float v = load_f32(x + i);
        store_f32(x + i, act == PXS_ACT_GELU_TANH ? gelu_tanh_f(v) : silu_f(v));
    }
}

// First non-finite element: status = row * 8 + 7 (the code pxs_sparse_validate
// uses for features), min-reduced over rows.
template <typename T>
__global__ void check_finite_kernel(const T * __restrict__ x, int64_t rows, int channels,
                                    int64_t ld, unsigned long long * __restrict__ status) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t count = rows * channels;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const int64_t r = i / channels;
        const float v = load_f32(x + r * ld + (i - r * channels));
        if (!isfinite(v)) atomicMin(status, static_cast<unsigned long long>(r * 8 + 7));
    }
}

// Value statistics (pxs_value_stats_f32): each workgroup folds a grid-stride
// slice into one partial, a single workgroup then folds the partials in
// workgroup order, so the result does not depend on scheduling.
struct StatsPartial {
    double sum;
    long long nonfinite;
    long long first_bad;
    float lo, hi, max_abs, pad;
};

__device__ __forceinline__ void stats_fold(StatsPartial & a, const StatsPartial & b) {
    a.sum += b.sum;
    a.nonfinite += b.nonfinite;
    a.first_bad = b.first_bad < a.first_bad ? b.first_bad : a.first_bad;
    a.lo = fminf(a.lo, b.lo);
    a.hi = fmaxf(a.hi, b.hi);
    a.max_abs = fmaxf(a.max_abs, b.max_abs);
}

constexpr int kStatsThreads = 256;

// Tree over the workgroup's 256 partials in LDS; thread 0 holds the result.
__device__ void stats_block_fold(StatsPartial & mine, StatsPartial * lds) {
    lds[threadIdx.x] = mine;
    __syncthreads();
    for (int span = kStatsThreads / 2; span >= 1; span >>= 1) {
        if (static_cast<int>(threadIdx.x) < span) {
            stats_fold(lds[threadIdx.x], lds[threadIdx.x + span]);
        }
        __syncthreads();
    }
    mine = lds[0];
}

__device__ __forceinline__ StatsPartial stats_empty(long long count) {
    StatsPartial p;
    p.sum = 0.0;
    p.nonfinite = 0;
    p.first_bad = count;
    p.lo = INFINITY;
    p.hi = -INFINITY;
    p.max_abs = 0.0f;
    p.pad = 0.0f;
    return p;
}

__global__ void __launch_bounds__(kStatsThreads)
value_stats_partial_kernel(const float * __restrict__ x, int64_t count,
                           StatsPartial * __restrict__ partials) {
    __shared__ StatsPartial lds[kStatsThreads];
    StatsPartial p = stats_empty(count);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const float v = x[i];
        if (!isfinite(v)) {
            ++p.nonfinite;
            if (i < p.first_bad) p.first_bad = i;
            continue;
        }
        p.sum += static_cast<double>(v);
        p.lo = fminf(p.lo, v);
        p.hi = fmaxf(p.hi, v);
        p.max_abs = fmaxf(p.max_abs, fabsf(v));
    }
    stats_block_fold(p, lds);
    if (threadIdx.x == 0) partials[blockIdx.x] = p;
}

__global__ void __launch_bounds__(kStatsThreads)
value_stats_final_kernel(const float * __restrict__ x, int64_t count,
                         const StatsPartial * __restrict__ partials, int nparts,
                         pxs_value_stats * __restrict__ out) {
    __shared__ StatsPartial lds[kStatsThreads];
    StatsPartial p = stats_empty(count);
    for (int i = threadIdx.x; i < nparts; i += kStatsThreads) stats_fold(p, partials[i]);
    stats_block_fold(p, lds);
    if (threadIdx.x == 0) {
        out->nonfinite = p.nonfinite;
        out->first_bad = p.first_bad;
        out->sum = p.sum;
        out->first_bad_value = p.first_bad < count ? x[p.first_bad] : 0.0f;
        out->min = p.lo;
        out->max = p.hi;
        out->max_abs = p.max_abs;
    }
}

constexpr int kStatsMaxParts = 1024;

template <typename TS, typename TD>
__global__ void convert8_kernel(const TS * __restrict__ x, int64_t nvec, TD * __restrict__ y) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < nvec;
         i += stride) {
        float v[8];
        load8(x + 8 * i, v);
        store8(y + 8 * i, v);
    }
}

// add_repeat over 8-element pieces of a row (channels % 8 == 0); the row
// index is 32-bit (the caller checks rows * channels / 8 < 2^32).
template <typename T>
__global__ void add_repeat8_kernel(const T * a, uint32_t nvec, uint32_t vpr,
                                   const float * __restrict__ skip, int skip_channels, int repeats,
                                   float * y) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
        const uint32_t r = i / vpr;
        const int j0 = static_cast<int>(i - r * vpr) * 8;
        const float * sk = skip + static_cast<int64_t>(r) * skip_channels;
        float v[8];
        load8(a + static_cast<int64_t>(i) * 8, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = v[e] + sk[(j0 + e) / repeats];
        store8(y + static_cast<int64_t>(i) * 8, v);
    }
}

template <typename TS, typename TD>
__global__ void convert_kernel(const TS * __restrict__ x, int64_t count, TD * __restrict__ y) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        store_f32(y + i, load_f32(x + i));
    }
}

// repeat_channels followed by add_in_place (src/slat_decoder.cpp:44-107):
// y[r, j] = a[r, j] + skip[r, j / repeats].  a and y may be the same fp32
// buffer: each element is read and written by one thread.
template <typename T>
__global__ void add_repeat_kernel(const T * a, int64_t rows, int channels,
                                  const float * __restrict__ skip, int skip_channels, int repeats,
                                  float * y) {
    const int64_t count = rows * channels;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const int64_t r = i / channels;
        const int j = static_cast<int>(i - r * channels);
        y[i] = load_f32(a + i) + skip[r * skip_channels + j / repeats];
    }
}

// Sinusoidal timestep embedding (src/flow.cpp:92-123): cos half then sin
// half, frequency exp(-ln(max_period) * i / half); a trailing odd column is 0.
__global__ void timestep_embedding_kernel(const float * __restrict__ t, int64_t batch, int dim,
                                          float log_period, float * __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int half = dim / 2;
    if (i >= batch * dim) return;
    const int64_t row = i / dim;
    const int col = static_cast<int>(i - row * dim);
    float v = 0.0f;
    if (col < 2 * half) {
        const int idx = col < half ? col : col - half;
        const float fraction = static_cast<float>(idx) / static_cast<float>(half);
        const float arg = t[row] * expf(-log_period * fraction);
        v = col < half ? cosf(arg) : sinf(arg);
    }
    out[i] = v;
}

int check_dtype(int dtype) { return dtype == PXS_F32 || dtype == PXS_BF16; }

template <typename TX, typename TY, int L, int NV, bool kMod>
void launch_ln_rows(const void * x, int64_t rows, float eps, const float * gamma,
                    const float * beta, const int32_t * coords, const float * bm, const float * tm,
                    int off, void * y, hipStream_t s) {
    hipLaunchKernelGGL((layer_norm_rows_kernel<TX, TY, L, NV, kMod>),
                       dim3(grid_for(rows, 4 * (64 / L))), dim3(256), 0, s,
                       static_cast<const TX *>(x), rows, eps, gamma, beta, coords, bm, tm, off,
                       static_cast<TY *>(y));
}

// The row-group kernel when a row is 2^k 16-byte vectors (up to 64 lanes of
// one vector, or 64 lanes of 2 or 4) and both buffers are 16-byte aligned.
template <typename TX, typename TY, bool kMod>
bool try_ln_rows(const void * x, int64_t rows, int channels, float eps, const float * gamma,
                 const float * beta, const int32_t * coords, const float * bm, const float * tm,
                 int off, void * y, hipStream_t s) {
    constexpr int V = Vec16<TX>::kN;
    auto a16 = [](const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (channels % V != 0 || !a16(x) || !a16(y) || (gamma && (!a16(gamma) || !a16(beta))))
        return false;
    if (kMod && (!a16(bm) || !a16(tm) || off % 4 != 0)) return false;
    switch (channels / V) {
    case 1: launch_ln_rows<TX, TY, 1, 1, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    case 2: launch_ln_rows<TX, TY, 2, 1, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    case 4: launch_ln_rows<TX, TY, 4, 1, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    case 8: launch_ln_rows<TX, TY, 8, 1, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    case 16: launch_ln_rows<TX, TY, 16, 1, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    case 32: launch_ln_rows<TX, TY, 32, 1, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    case 64: launch_ln_rows<TX, TY, 64, 1, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    case 128: launch_ln_rows<TX, TY, 64, 2, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    case 256: launch_ln_rows<TX, TY, 64, 4, kMod>(x, rows, eps, gamma, beta, coords, bm, tm, off, y, s); return true;
    default: return false;
    }
}

template <typename TX, typename TY, bool kMod>
void launch_ln(const void * x, int64_t rows, int channels, float eps, const float * gamma,
               const float * beta, const int32_t * coords, const float * bm, const float * tm,
               int off, void * y, hipStream_t s) {
#ifndef PXS_LN_ROWS
#define PXS_LN_ROWS 1
#endif
    if (PXS_LN_ROWS &&
        try_ln_rows<TX, TY, kMod>(x, rows, channels, eps, gamma, beta, coords, bm, tm, off, y, s))
        return;
    hipLaunchKernelGGL((layer_norm_kernel<TX, TY, kMod>), dim3(grid_for(rows, kRowsPerBlock)),
                       dim3(64 * kRowsPerBlock), 0, s, static_cast<const TX *>(x), rows, channels,
                       eps, gamma, beta, coords, bm, tm, off, static_cast<TY *>(y));
}

template <bool kMod>
int run_ln(int xd, const void * x, int64_t rows, int channels, float eps, const float * gamma,
           const float * beta, const int32_t * coords, const float * bm, const float * tm, int off,
           int yd, void * y, hipStream_t s) {
    if (xd == PXS_F32 && yd == PXS_F32)
        launch_ln<float, float, kMod>(x, rows, channels, eps, gamma, beta, coords, bm, tm, off, y, s);
    else if (xd == PXS_F32 && yd == PXS_BF16)
        launch_ln<float, uint16_t, kMod>(x, rows, channels, eps, gamma, beta, coords, bm, tm, off, y, s);
    else if (xd == PXS_BF16 && yd == PXS_F32)
        launch_ln<uint16_t, float, kMod>(x, rows, channels, eps, gamma, beta, coords, bm, tm, off, y, s);
    else
        launch_ln<uint16_t, uint16_t, kMod>(x, rows, channels, eps, gamma, beta, coords, bm, tm, off, y, s);
    return check_launch("layer norm");
}

template <typename T>
int run_head_op(const void * x, int64_t ld_x, int64_t rows, int heads, int head_dim,
                const float * gamma, const int32_t * coords, const RopeTable & rope, void * y,
                int64_t ld_y, hipStream_t s) {
    if (head_dim == 64 && ld_x % 8 == 0 && ld_y % 8 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
        hipLaunchKernelGGL(head_op64_kernel<T>, dim3(grid_for(rows, kRowsPerBlock)),
                           dim3(64 * kRowsPerBlock), 0, s, static_cast<const T *>(x), ld_x, rows,
                           heads, gamma, coords, rope, static_cast<T *>(y), ld_y);
        return check_launch("head norm/rope");
    }
    const int64_t items = rows * heads;
    hipLaunchKernelGGL(head_norm_rope_kernel<T>, dim3(grid_for(items, 256)), dim3(256), 0, s,
                       static_cast<const T *>(x), ld_x, rows, heads, head_dim, gamma, coords, rope,
                       static_cast<T *>(y), ld_y);
    return check_launch("head norm/rope");
}

} // namespace
} // namespace pxs

using namespace pxs;

extern "C" {

int pxs_layer_norm(int x_dtype, const void * x, int64_t rows, int channels, float eps,
                   const float * gamma, const float * beta, int y_dtype, void * y, void * stream) {
    PXS_CHECK(check_dtype(x_dtype) && check_dtype(y_dtype), PXS_ERR_ARG, "pxs_layer_norm: bad dtype");
    PXS_CHECK(rows >= 0 && channels > 0, PXS_ERR_ARG, "pxs_layer_norm: bad shape");
    PXS_CHECK(eps > 0.0f && std::isfinite(eps), PXS_ERR_ARG,
              "sparse layer norm epsilon must be finite and positive");
    PXS_CHECK((gamma == nullptr) == (beta == nullptr), PXS_ERR_ARG,
              "sparse layer norm affine parameters must be both null or non-null");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x && y, PXS_ERR_ARG, "pxs_layer_norm: null pointer");
    return run_ln<false>(x_dtype, x, rows, channels, eps, gamma, beta, nullptr, nullptr, nullptr,
                         0, y_dtype, y, as_stream(stream));
}

int pxs_layer_norm_modulate(int x_dtype, const void * x, int64_t rows, int channels, float eps,
                            const int32_t * coords, const float * block_mod,
                            const float * time_mod, int mod_offset, int y_dtype, void * y,
                            void * stream) {
    PXS_CHECK(check_dtype(x_dtype) && check_dtype(y_dtype), PXS_ERR_ARG,
              "pxs_layer_norm_modulate: bad dtype");
    PXS_CHECK(rows >= 0 && channels > 0 && mod_offset >= 0, PXS_ERR_ARG,
              "pxs_layer_norm_modulate: bad shape");
    PXS_CHECK(eps > 0.0f && std::isfinite(eps), PXS_ERR_ARG,
              "sparse layer norm epsilon must be finite and positive");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x && y && coords && block_mod && time_mod, PXS_ERR_ARG,
              "pxs_layer_norm_modulate: null pointer");
    return run_ln<true>(x_dtype, x, rows, channels, eps, nullptr, nullptr, coords, block_mod,
                        time_mod, mod_offset, y_dtype, y, as_stream(stream));
}

int pxs_mh_rms_norm(int dtype, const void * x, int64_t ld_x, int64_t rows, int heads,
                    int head_dim, const float * gamma, void * y, int64_t ld_y, void * stream) {
    PXS_CHECK(check_dtype(dtype), PXS_ERR_ARG, "pxs_mh_rms_norm: bad dtype");
    PXS_CHECK(rows >= 0 && heads > 0 && head_dim > 0 && ld_x >= heads * head_dim &&
                  ld_y >= heads * head_dim,
              PXS_ERR_ARG, "sparse RMS norm head dimensions are invalid");
    PXS_CHECK(gamma, PXS_ERR_ARG, "sparse RMS norm gamma pointer is null");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x && y, PXS_ERR_ARG, "pxs_mh_rms_norm: null pointer");
    RopeTable none{};
    return dtype == PXS_F32
               ? run_head_op<float>(x, ld_x, rows, heads, head_dim, gamma, nullptr, none, y, ld_y,
                                    as_stream(stream))
               : run_head_op<uint16_t>(x, ld_x, rows, heads, head_dim, gamma, nullptr, none, y,
                                       ld_y, as_stream(stream));
}

int pxs_rope(int dtype, const int32_t * coords, const void * x, int64_t ld_x, int64_t rows,
             int heads, int head_dim, float freq_min, float freq_base, void * y, int64_t ld_y,
             void * stream) {
    PXS_CHECK(check_dtype(dtype), PXS_ERR_ARG, "pxs_rope: bad dtype");
    PXS_CHECK(rows >= 0 && heads > 0 && head_dim > 0 && head_dim % 2 == 0 &&
                  ld_x >= heads * head_dim && ld_y >= heads * head_dim,
              PXS_ERR_ARG, "sparse RoPE head dimensions are invalid");
    PXS_CHECK(freq_min > 0.0f && std::isfinite(freq_min) && freq_base > 0.0f &&
                  std::isfinite(freq_base),
              PXS_ERR_ARG, "sparse RoPE frequencies must be finite and positive");
    PXS_CHECK(head_dim / 2 / 3 <= 32, PXS_ERR_ARG, "pxs_rope: head_dim above 192 unsupported");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(coords && x && y, PXS_ERR_ARG, "pxs_rope: null pointer");
    const RopeTable t = make_rope_table(head_dim, freq_min, freq_base);
    return dtype == PXS_F32
               ? run_head_op<float>(x, ld_x, rows, heads, head_dim, nullptr, coords, t, y, ld_y,
                                    as_stream(stream))
               : run_head_op<uint16_t>(x, ld_x, rows, heads, head_dim, nullptr, coords, t, y,
                                       ld_y, as_stream(stream));
}

int pxs_qkv_prepare(int dtype, const void * qkv, int64_t rows, int heads, int head_dim,
                    const float * q_gamma, const float * k_gamma, const int32_t * coords,
                    float freq_min, float freq_base, void * q, void * k, void * v,
                    void * stream) {
    PXS_CHECK(check_dtype(dtype), PXS_ERR_ARG, "pxs_qkv_prepare: bad dtype");
    PXS_CHECK(rows >= 0 && heads > 0 && head_dim > 0 && (head_dim % 2 == 0 || !coords),
              PXS_ERR_ARG, "pxs_qkv_prepare: bad shape");
    PXS_CHECK((q_gamma == nullptr) == (k_gamma == nullptr), PXS_ERR_ARG,
              "pxs_qkv_prepare: q_gamma and k_gamma must be both set or both null");
    PXS_CHECK(head_dim / 2 / 3 <= 32, PXS_ERR_ARG, "pxs_qkv_prepare: head_dim above 192 unsupported");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(qkv && q && k && v, PXS_ERR_ARG, "pxs_qkv_prepare: null pointer");
    hipStream_t s = as_stream(stream);
    RopeTable t{};
    if (coords) {
        PXS_CHECK(freq_min > 0.0f && freq_base > 0.0f, PXS_ERR_ARG,
                  "sparse RoPE frequencies must be finite and positive");
        t = make_rope_table(head_dim, freq_min, freq_base);
    }
    const int C = heads * head_dim;
    const bool aligned = (reinterpret_cast<uintptr_t>(qkv) & 15u) == 0 &&
                         (reinterpret_cast<uintptr_t>(q) & 15u) == 0 &&
                         (reinterpret_cast<uintptr_t>(k) & 15u) == 0 &&
                         (reinterpret_cast<uintptr_t>(v) & 15u) == 0;
    if (head_dim == 64 && aligned) {
        if (dtype == PXS_F32) {
            hipLaunchKernelGGL(qkv_prepare64_kernel<float>, dim3(grid_for(rows, kRowsPerBlock)),
                               dim3(64 * kRowsPerBlock), 0, s, static_cast<const float *>(qkv),
                               rows, heads, q_gamma, k_gamma, coords, t, static_cast<float *>(q),
                               static_cast<float *>(k), static_cast<float *>(v));
        } else {
            hipLaunchKernelGGL(qkv_prepare64_kernel<uint16_t>, dim3(grid_for(rows, kRowsPerBlock)),
                               dim3(64 * kRowsPerBlock), 0, s, static_cast<const uint16_t *>(qkv),
                               rows, heads, q_gamma, k_gamma, coords, t,
                               static_cast<uint16_t *>(q), static_cast<uint16_t *>(k),
                               static_cast<uint16_t *>(v));
        }
        return check_launch("pxs_qkv_prepare");
    }
    // Generic head_dim: per-(row, head) kernels reading the interleaved qkv.
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((rows * C + 255) / 256, 16384));
    int rc;
    if (dtype == PXS_F32) {
        rc = run_head_op<float>(qkv, 3 * C, rows, heads, head_dim, q_gamma, coords, t, q, C, s);
        if (!rc) rc = run_head_op<float>(static_cast<const float *>(qkv) + C, 3 * C, rows, heads,
                                         head_dim, k_gamma, coords, t, k, C, s);
        if (!rc) hipLaunchKernelGGL(split_copy_kernel<float>, dim3(blocks), dim3(256), 0, s,
                                    static_cast<const float *>(qkv), rows, C, 2,
                                    static_cast<float *>(v));
    } else {
        rc = run_head_op<uint16_t>(qkv, 3 * C, rows, heads, head_dim, q_gamma, coords, t, q, C, s);
        if (!rc) rc = run_head_op<uint16_t>(static_cast<const uint16_t *>(qkv) + C, 3 * C, rows,
                                            heads, head_dim, k_gamma, coords, t, k, C, s);
        if (!rc) hipLaunchKernelGGL(split_copy_kernel<uint16_t>, dim3(blocks), dim3(256), 0, s,
                                    static_cast<const uint16_t *>(qkv), rows, C, 2,
                                    static_cast<uint16_t *>(v));
    }
    return rc ? rc : check_launch("pxs_qkv_prepare");
}

int pxs_activation(int dtype, void * x, int64_t count, int act, void * stream) {
    PXS_CHECK(check_dtype(dtype), PXS_ERR_ARG, "pxs_activation: bad dtype");
    PXS_CHECK(act == PXS_ACT_GELU_TANH || act == PXS_ACT_SILU || act == PXS_ACT_NONE, PXS_ERR_ARG,
              "pxs_activation: bad activation");
    if (count <= 0 || act == PXS_ACT_NONE) return PXS_OK;
    PXS_CHECK(x, PXS_ERR_ARG, "pxs_activation: null pointer");
    if (vec8_ok(count, x)) {
        if (dtype == PXS_F32)
            hipLaunchKernelGGL(activation8_kernel<float>, dim3(vec8_blocks(count)), dim3(256), 0,
                               as_stream(stream), static_cast<float *>(x), count / 8, act);
        else
            hipLaunchKernelGGL(activation8_kernel<uint16_t>, dim3(vec8_blocks(count)), dim3(256), 0,
                               as_stream(stream), static_cast<uint16_t *>(x), count / 8, act);
        return check_launch("pxs_activation");
    }
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((count + 255) / 256, 16384));
    if (dtype == PXS_F32) {
        hipLaunchKernelGGL(activation_kernel<float>, dim3(blocks), dim3(256), 0, as_stream(stream),
                           static_cast<float *>(x), count, act);
    } else {
        hipLaunchKernelGGL(activation_kernel<uint16_t>, dim3(blocks), dim3(256), 0,
                           as_stream(stream), static_cast<uint16_t *>(x), count, act);
    }
    return check_launch("pxs_activation");
}

int pxs_check_finite(int dtype, const void * x, int64_t rows, int channels, int64_t ld,
                     int64_t * status, void * stream) {
    PXS_CHECK(check_dtype(dtype), PXS_ERR_ARG, "pxs_check_finite: bad dtype");
    PXS_CHECK(rows >= 0 && channels > 0 && ld >= channels, PXS_ERR_ARG,
              "pxs_check_finite: bad shape");
    PXS_CHECK(status, PXS_ERR_ARG, "pxs_check_finite: null status");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x, PXS_ERR_ARG, "pxs_check_finite: null pointer");
    const unsigned blocks =
        static_cast<unsigned>(std::min<int64_t>((rows * channels + 255) / 256, 4096));
    auto * st = reinterpret_cast<unsigned long long *>(status);
    if (dtype == PXS_F32) {
        hipLaunchKernelGGL(check_finite_kernel<float>, dim3(blocks), dim3(256), 0,
                           as_stream(stream), static_cast<const float *>(x), rows, channels, ld, st);
    } else {
        hipLaunchKernelGGL(check_finite_kernel<uint16_t>, dim3(blocks), dim3(256), 0,
                           as_stream(stream), static_cast<const uint16_t *>(x), rows, channels, ld,
                           st);
    }
    return check_launch("pxs_check_finite");
}

size_t pxs_value_stats_workspace_bytes(int64_t count) {
    (void)count;
    return kStatsMaxParts * sizeof(StatsPartial);
}

int pxs_value_stats_f32(const float * x, int64_t count, pxs_value_stats * stats, void * workspace,
                        void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_value_stats_f32");
    PXS_CHECK(count >= 0, PXS_ERR_ARG, "pxs_value_stats_f32: negative count");
    PXS_CHECK(stats && workspace && (x || count == 0), PXS_ERR_ARG,
              "pxs_value_stats_f32: null pointer");
    const int parts = static_cast<int>(
        std::max<int64_t>(1, std::min<int64_t>((count + 4 * kStatsThreads - 1) / (4 * kStatsThreads),
                                               kStatsMaxParts)));
    auto * partials = static_cast<StatsPartial *>(workspace);
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(value_stats_partial_kernel, dim3(parts), dim3(kStatsThreads), 0, s, x, count,
                       partials);
    hipLaunchKernelGGL(value_stats_final_kernel, dim3(1), dim3(kStatsThreads), 0, s, x, count,
                       partials, parts, stats);
    return check_launch("pxs_value_stats_f32");
}

int pxs_convert(int src_dtype, const void * x, int64_t count, int dst_dtype, void * y,
                void * stream) {
    PXS_CHECK(check_dtype(src_dtype) && check_dtype(dst_dtype), PXS_ERR_ARG,
              "pxs_convert: bad dtype");
    PXS_CHECK(count >= 0, PXS_ERR_ARG, "pxs_convert: negative count");
    if (count == 0) return PXS_OK;
    PXS_CHECK(x && y, PXS_ERR_ARG, "pxs_convert: null pointer");
    hipStream_t s = as_stream(stream);
    if (vec8_ok(count, x, y)) {
        const unsigned vb = vec8_blocks(count);
        const int64_t nv = count / 8;
        if (src_dtype == PXS_F32 && dst_dtype == PXS_BF16)
            hipLaunchKernelGGL((convert8_kernel<float, uint16_t>), dim3(vb), dim3(256), 0, s,
                               static_cast<const float *>(x), nv, static_cast<uint16_t *>(y));
        else if (src_dtype == PXS_BF16 && dst_dtype == PXS_F32)
            hipLaunchKernelGGL((convert8_kernel<uint16_t, float>), dim3(vb), dim3(256), 0, s,
                               static_cast<const uint16_t *>(x), nv, static_cast<float *>(y));
        else if (src_dtype == PXS_F32)
            hipLaunchKernelGGL((convert8_kernel<float, float>), dim3(vb), dim3(256), 0, s,
                               static_cast<const float *>(x), nv, static_cast<float *>(y));
        else
            hipLaunchKernelGGL((convert8_kernel<uint16_t, uint16_t>), dim3(vb), dim3(256), 0, s,
                               static_cast<const uint16_t *>(x), nv, static_cast<uint16_t *>(y));
        return check_launch("pxs_convert");
    }
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((count + 255) / 256, 16384));
    if (src_dtype == PXS_F32 && dst_dtype == PXS_BF16) {
        hipLaunchKernelGGL((convert_kernel<float, uint16_t>), dim3(blocks), dim3(256), 0, s,
                           static_cast<const float *>(x), count, static_cast<uint16_t *>(y));
    } else if (src_dtype == PXS_BF16 && dst_dtype == PXS_F32) {
        hipLaunchKernelGGL((convert_kernel<uint16_t, float>), dim3(blocks), dim3(256), 0, s,
                           static_cast<const uint16_t *>(x), count, static_cast<float *>(y));
    } else if (src_dtype == PXS_F32) {
        hipLaunchKernelGGL((convert_kernel<float, float>), dim3(blocks), dim3(256), 0, s,
                           static_cast<const float *>(x), count, static_cast<float *>(y));
    } else {
        hipLaunchKernelGGL((convert_kernel<uint16_t, uint16_t>), dim3(blocks), dim3(256), 0, s,
                           static_cast<const uint16_t *>(x), count, static_cast<uint16_t *>(y));
    }
    return check_launch("pxs_convert");
}

int pxs_add_repeat(int a_dtype, const void * a, int64_t rows, int channels, const float * skip,
                   int skip_channels, float * y, void * stream) {
    PXS_CHECK(check_dtype(a_dtype), PXS_ERR_ARG, "pxs_add_repeat: bad dtype");
    PXS_CHECK(rows >= 0 && channels > 0 && skip_channels > 0 && channels % skip_channels == 0,
              PXS_ERR_ARG, "SLat decoder skip channels are not repeatable");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(a && skip && y, PXS_ERR_ARG, "pxs_add_repeat: null pointer");
    const int64_t count = rows * channels;
    const int repeats = channels / skip_channels;
    if (channels % 8 == 0 && count / 8 <= UINT32_MAX && vec8_ok(count, a, y)) {
        const uint32_t nv = static_cast<uint32_t>(count / 8), vpr = static_cast<uint32_t>(channels / 8);
        if (a_dtype == PXS_F32)
            hipLaunchKernelGGL(add_repeat8_kernel<float>, dim3(vec8_blocks(count)), dim3(256), 0,
                               as_stream(stream), static_cast<const float *>(a), nv, vpr, skip,
                               skip_channels, repeats, y);
        else
            hipLaunchKernelGGL(add_repeat8_kernel<uint16_t>, dim3(vec8_blocks(count)), dim3(256), 0,
                               as_stream(stream), static_cast<const uint16_t *>(a), nv, vpr, skip,
                               skip_channels, repeats, y);
        return check_launch("pxs_add_repeat");
    }
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((count + 255) / 256, 16384));
    if (a_dtype == PXS_F32) {
        hipLaunchKernelGGL(add_repeat_kernel<float>, dim3(blocks), dim3(256), 0, as_stream(stream),
                           static_cast<const float *>(a), rows, channels, skip, skip_channels,
                           repeats, y);
    } else {
        hipLaunchKernelGGL(add_repeat_kernel<uint16_t>, dim3(blocks), dim3(256), 0,
                           as_stream(stream), static_cast<const uint16_t *>(a), rows, channels,
                           skip, skip_channels, repeats, y);
    }
    return check_launch("pxs_add_repeat");
}

int pxs_timestep_embedding(const float * timesteps, int64_t batch, int dim, int max_period,
                           float * out, void * stream) {
    PXS_CHECK(batch >= 0 && dim > 0 && max_period > 0, PXS_ERR_ARG,
              "pxs_timestep_embedding: bad shape");
    if (batch == 0) return PXS_OK;
    PXS_CHECK(timesteps && out, PXS_ERR_ARG, "pxs_timestep_embedding: null pointer");
    const float log_period = static_cast<float>(std::log(static_cast<double>(max_period)));
    hipLaunchKernelGGL(timestep_embedding_kernel, dim3(grid_for(batch * dim, 256)), dim3(256), 0,
                       as_stream(stream), timesteps, batch, dim, log_period, out);
    return check_launch("pxs_timestep_embedding");
}

} // extern "C"
