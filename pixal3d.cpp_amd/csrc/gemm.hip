// Gather-GEMM on MFMA: submanifold conv, stride-2 conv and sparse linear.
//
// One kernel computes Y[p, :] = sum_k W_k X[rowmap[k][p], :] (+ bias, then an
// epilogue) for a tile of BM output rows x BN output channels:
//   * submanifold conv: rowmap = the dense [27][n] neighbor map;
//   * stride-2 conv:    rowmap = the [8][ld] child map;
//   * linear:           no rowmap (identity, one offset).
// Output-stationary: a workgroup owns its output rows for every offset, so
// there is no scatter and no atomic.  Offsets absent from every row of a tile
// are skipped as whole stages.
//
// Per stage the workgroup stages a 128-byte chunk of every gathered input row
// (A) and of every weight row (B) in LDS (double buffered, padded rows for
// conflict-free 16-byte reads), then each of the 4 waves runs a 2x2 (or
// smaller) grid of 32x32 MFMA tiles:
//   bf16: v_mfma_f32_32x32x16_bf16, 4 K-steps per 64-channel chunk;
//   fp32: v_mfma_f32_32x32x2_f32, 16 K-steps per 32-channel chunk.
// The K order inside a chunk is permuted identically for A and B so that each
// lane reads 16 contiguous bytes per LDS access.

#include "pxs_common.h"

namespace pxs {
namespace {

constexpr int kGemmThreads = 256;
constexpr int kChunkBytes = 128;
constexpr int kPitch = kChunkBytes + 16;

enum Epilogue { kEpiStore = 0, kEpiGateResidual = 1 };

struct GemmArgs {
    const void * x;
    int64_t rows_in;
    int64_t ldx;
    int cin;
    const void * w;
    const float * bias;
    int cout;
    int64_t m;
    const int32_t * rowmap;
    int64_t ld_map;
    int noff;
    const uint32_t * masks;
    void * y;
    int64_t ldy;
    int act;
    int vec_ok;
    const int32_t * coords;
    const float * block_mod;
    const float * time_mod;
    int gate_offset;
    float * residual;
};

template <typename T> struct Mfma;

template <> struct Mfma<uint16_t> {
    static constexpr int kVec = 8;            // elements per 16 bytes
    static constexpr int kChunk = 64;         // elements per 128-byte chunk
};

template <> struct Mfma<float> {
    static constexpr int kVec = 4;
    static constexpr int kChunk = 32;
};

__device__ __forceinline__ int remap_xcd(int bid, int blocks) {
    // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
    // contiguous range of logical tiles so neighbouring tiles (which share
    // gathered rows and weights) share one L2.
    const int q = blocks / 8, rem = blocks % 8;
    const int xcd = bid % 8, slot = bid / 8;
    return (xcd < rem) ? xcd * (q + 1) + slot : rem * (q + 1) + (xcd - rem) * q + slot;
}

template <typename T>
__device__ __forceinline__ uint4 load_chunk16(const T * base, int64_t row, int64_t ld, int col,
                                              int limit, bool vec_ok) {
    constexpr int kVec = Mfma<T>::kVec;
    if (vec_ok) {
        if (col < limit) return *reinterpret_cast<const uint4 *>(base + row * ld + col);
        return make_uint4(0, 0, 0, 0);
    }
    T tmp[kVec];
#pragma unroll
    for (int e = 0; e < kVec; ++e) tmp[e] = (col + e < limit) ? base[row * ld + col + e] : T(0);
    return *reinterpret_cast<const uint4 *>(tmp);
}

template <typename T, int BM, int BN, int EPI>
__global__ void __launch_bounds__(kGemmThreads)
gather_gemm_kernel(GemmArgs a) {
    constexpr int kVec = Mfma<T>::kVec;
    constexpr int kChunk = Mfma<T>::kChunk;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TI = WM / 32, TJ = WN / 32;
    constexpr int APASS = BM / 32, BPASS = BN / 32;
    constexpr int kStageBytes = (BM + BN) * kPitch;

    extern __shared__ __align__(16) char smem[];
    __shared__ uint32_t tile_mask;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int h = lane >> 5, r = lane & 31;

    const int tiles_n = (a.cout + BN - 1) / BN;
    const int logical = remap_xcd(blockIdx.x, gridDim.x);
    const int64_t p0 = static_cast<int64_t>(logical / tiles_n) * BM;
    const int n0 = (logical % tiles_n) * BN;

    const T * __restrict__ x = static_cast<const T *>(a.x);
    const T * __restrict__ w = static_cast<const T *>(a.w);

    // Offsets present in this tile.
    if (tid == 0) tile_mask = 0;
    __syncthreads();
    {
        uint32_t local = 0;
        if (tid < BM && p0 + tid < a.m) {
            const int64_t p = p0 + tid;
            if (a.masks) {
                local = a.masks[p];
            } else if (a.rowmap) {
                for (int k = 0; k < a.noff; ++k) {
                    const int32_t src = a.rowmap[k * a.ld_map + p];
                    if (src >= 0 && src < a.rows_in) local |= 1u << k;
                }
            } else {
                local = 1u;
            }
        }
        if (local) atomicOr(&tile_mask, local);
    }
    __syncthreads();
    uint32_t pending = tile_mask & (a.noff >= 32 ? ~0u : ((1u << a.noff) - 1u));
    const int chunks = (a.cin + kChunk - 1) / kChunk;
    const int stages = __popc(pending) * chunks;

    // Per-thread staging slots: row (pass * 32 + tid / 8), 16-byte piece tid % 8.
    const int srow = tid >> 3;
    const int spiece = tid & 7;
    uint4 ra[APASS], rb[BPASS];

    int cur_k = pending ? __ffs(pending) - 1 : 0;
    int cur_chunk = 0;

    auto load_stage = [&](int k, int chunk) {
        const int col = chunk * kChunk + spiece * kVec;
#pragma unroll
        for (int i = 0; i < APASS; ++i) {
            const int64_t p = p0 + i * 32 + srow;
            int64_t src = -1;
            if (p < a.m) {
                src = a.rowmap ? static_cast<int64_t>(a.rowmap[k * a.ld_map + p]) : p;
                if (src >= a.rows_in) src = -1;
            }
            ra[i] = src >= 0 ? load_chunk16<T>(x, src, a.ldx, col, a.cin, a.vec_ok)
                             : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < BPASS; ++j) {
            const int o = n0 + j * 32 + srow;
            rb[j] = o < a.cout
                        ? load_chunk16<T>(w, static_cast<int64_t>(k) * a.cout + o, a.cin, col,
                                          a.cin, a.vec_ok)
                        : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_stage = [&](int buf) {
        char * sa = smem + buf * kStageBytes;
        char * sb = sa + BM * kPitch;
#pragma unroll
        for (int i = 0; i < APASS; ++i) {
            *reinterpret_cast<uint4 *>(sa + (i * 32 + srow) * kPitch + spiece * 16) = ra[i];
        }
#pragma unroll
        for (int j = 0; j < BPASS; ++j) {
            *reinterpret_cast<uint4 *>(sb + (j * 32 + srow) * kPitch + spiece * 16) = rb[j];
        }
    };
    auto advance = [&]() {
        if (++cur_chunk == chunks) {
            cur_chunk = 0;
            pending &= pending - 1;
            cur_k = pending ? __ffs(pending) - 1 : 0;
        }
    };

    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    if (stages > 0) {
        load_stage(cur_k, cur_chunk);
        advance();
        store_stage(0);
        __syncthreads();
    }
    for (int s = 0; s < stages; ++s) {
        const bool more = s + 1 < stages;
        if (more) {
            load_stage(cur_k, cur_chunk);
            advance();
        }
        const char * sa = smem + (s & 1) * kStageBytes;
        const char * sb = sa + BM * kPitch;
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                bf16x8 af[TI], bfr[TJ];
#pragma unroll
                for (int i = 0; i < TI; ++i)
                    af[i] = *reinterpret_cast<const bf16x8 *>(
                        sa + (wm * WM + i * 32 + r) * kPitch + h * 64 + ks * 16);
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    bfr[j] = *reinterpret_cast<const bf16x8 *>(
                        sb + (wn * WN + j * 32 + r) * kPitch + h * 64 + ks * 16);
#pragma unroll
                for (int i = 0; i < TI; ++i)
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j],
                                                                            acc[i][j], 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                f32x4 af[TI], bfr[TJ];
#pragma unroll
                for (int i = 0; i < TI; ++i)
                    af[i] = *reinterpret_cast<const f32x4 *>(
                        sa + (wm * WM + i * 32 + r) * kPitch + h * 64 + u * 16);
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    bfr[j] = *reinterpret_cast<const f32x4 *>(
                        sb + (wn * WN + j * 32 + r) * kPitch + h * 64 + u * 16);
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int i = 0; i < TI; ++i)
#pragma unroll
                        for (int j = 0; j < TJ; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][e], bfr[j][e],
                                                                             acc[i][j], 0, 0, 0);
            }
        }
        if (more) store_stage((s + 1) & 1);
        __syncthreads();
    }

    // Epilogue.  32x32 accumulator layout: lane (h, r), register v holds
    // row 8*(v/4) + 4*h + v%4, column r of the tile.
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int col = n0 + wn * WN + j * 32 + r;
            if (col >= a.cout) continue;
            const float b = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t row = p0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                if (row >= a.m) continue;
                float val = acc[i][j][v] + b;
                if constexpr (EPI == kEpiStore) {
                    if (a.act == PXS_ACT_GELU_TANH) val = gelu_tanh_f(val);
                    else if (a.act == PXS_ACT_SILU) val = silu_f(val);
                    store_f32(static_cast<T *>(a.y) + row * a.ldy + col, val);
                } else {
                    const int batch = a.coords[row * 4];
                    const float g = a.block_mod[a.gate_offset + col] +
                                    a.time_mod[static_cast<int64_t>(batch) * 6 * a.cout +
                                               a.gate_offset + col];
                    float * res = a.residual + row * a.cout + col;
                    *res = *res + val * g;
                }
            }
        }
    }
}

template <typename T, int BM, int BN, int EPI>
int launch_tile(const GemmArgs & args, hipStream_t stream) {
    constexpr int kStageBytes = (BM + BN) * kPitch;
    constexpr int kSmem = 2 * kStageBytes;
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&gather_gemm_kernel<T, BM, BN, EPI>),
            hipFuncAttributeMaxDynamicSharedMemorySize, kSmem);
        if (e != hipSuccess) return check_hip(e, "hipFuncSetAttribute(gather_gemm)");
        configured = true;
    }
    const int64_t tiles_m = (args.m + BM - 1) / BM;
    const int64_t tiles_n = (args.cout + BN - 1) / BN;
    const int64_t blocks = tiles_m * tiles_n;
    if (blocks > INT32_MAX) return fail(PXS_ERR_ARG, "gather GEMM grid too large");
    hipLaunchKernelGGL((gather_gemm_kernel<T, BM, BN, EPI>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kGemmThreads), kSmem, stream, args);
    return check_launch("gather GEMM");
}

template <typename T, int EPI>
int dispatch(const GemmArgs & args, hipStream_t stream) {
    if (args.m == 0 || args.cout == 0) return PXS_OK;
    const bool narrow = args.cout <= 64;
    const int64_t tiles_n = (args.cout + (narrow ? 63 : 127)) / (narrow ? 64 : 128);
    // Prefer 128-row tiles when they still give every CU two workgroups.
    const bool tall = ((args.m + 127) / 128) * tiles_n >= 512;
    if (narrow) {
        return tall ? launch_tile<T, 128, 64, EPI>(args, stream)
                    : launch_tile<T, 64, 64, EPI>(args, stream);
    }
    return tall ? launch_tile<T, 128, 128, EPI>(args, stream)
                : launch_tile<T, 64, 128, EPI>(args, stream);
}

int check_dtype(int dtype, const char * who) {
    if (dtype != PXS_F32 && dtype != PXS_BF16) {
        return fail(PXS_ERR_ARG, std::string(who) + ": dtype must be PXS_F32 or PXS_BF16");
    }
    return PXS_OK;
}

bool aligned16(const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int run_gemm(int dtype, GemmArgs & args, int epi, hipStream_t stream) {
    const int vec = dtype == PXS_BF16 ? 8 : 4;
    args.vec_ok = (args.cin % vec == 0) && (args.ldx % vec == 0) && aligned16(args.x) &&
                  aligned16(args.w);
    if (dtype == PXS_BF16) {
        return epi == kEpiStore ? dispatch<uint16_t, kEpiStore>(args, stream)
                                : dispatch<uint16_t, kEpiGateResidual>(args, stream);
    }
    return epi == kEpiStore ? dispatch<float, kEpiStore>(args, stream)
                            : dispatch<float, kEpiGateResidual>(args, stream);
}

// Mean of present children in ascending input-row order (the order the
// reference's per-group sums visit rows).
template <typename T>
__global__ void downsample_mean_kernel(const T * __restrict__ x, int channels,
                                       const int32_t * __restrict__ child_map, int64_t ld_map,
                                       int64_t m, T * __restrict__ y) {
    const int64_t q = blockIdx.x;
    if (q >= m) return;
    int32_t rows[8];
    int count = 0;
    for (int c = 0; c < 8; ++c) {
        const int32_t r = child_map[c * ld_map + q];
        if (r >= 0) rows[count++] = r;
    }
    // insertion sort (<= 8 entries)
    for (int i = 1; i < count; ++i) {
        const int32_t v = rows[i];
        int j = i - 1;
        while (j >= 0 && rows[j] > v) {
            rows[j + 1] = rows[j];
            --j;
        }
        rows[j + 1] = v;
    }
    for (int ch = threadIdx.x; ch < channels; ch += blockDim.x) {
        float s = 0.0f;
        for (int i = 0; i < count; ++i) s += load_f32(x + static_cast<int64_t>(rows[i]) * channels + ch);
        store_f32(y + q * channels + ch, s / static_cast<float>(count));
    }
}

} // namespace
} // namespace pxs

using namespace pxs;

extern "C" {

int pxs_subm_conv3d(int dtype, const void * x, int64_t n, int cin, const void * weight,
                    const float * bias, int cout, const int32_t * nbr, const uint32_t * masks,
                    void * y, void * stream) {
    if (int rc = check_dtype(dtype, "pxs_subm_conv3d")) return rc;
    PXS_CHECK(n >= 0 && cin > 0 && cout > 0, PXS_ERR_ARG, "pxs_subm_conv3d: bad shape");
    if (n == 0) return PXS_OK;
    PXS_CHECK(x && weight && nbr && y, PXS_ERR_ARG, "pxs_subm_conv3d: null pointer");
    GemmArgs a{};
    a.x = x; a.rows_in = n; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = n; a.rowmap = nbr; a.ld_map = n; a.noff = 27; a.masks = masks;
    a.y = y; a.ldy = cout; a.act = PXS_ACT_NONE;
    return run_gemm(dtype, a, kEpiStore, as_stream(stream));
}

int pxs_sparse_conv3d_s2(int dtype, const void * x, int64_t n_in, int cin, const void * weight,
                         const float * bias, int cout, const int32_t * child_map, int64_t ld_map,
                         int64_t m, void * y, void * stream) {
    if (int rc = check_dtype(dtype, "pxs_sparse_conv3d_s2")) return rc;
    PXS_CHECK(n_in >= 0 && m >= 0 && cin > 0 && cout > 0 && ld_map >= m, PXS_ERR_ARG,
              "pxs_sparse_conv3d_s2: bad shape");
    if (m == 0) return PXS_OK;
    PXS_CHECK(x && weight && child_map && y, PXS_ERR_ARG, "pxs_sparse_conv3d_s2: null pointer");
    GemmArgs a{};
    a.x = x; a.rows_in = n_in; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = m; a.rowmap = child_map; a.ld_map = ld_map; a.noff = 8;
    a.masks = nullptr; a.y = y; a.ldy = cout; a.act = PXS_ACT_NONE;
    return run_gemm(dtype, a, kEpiStore, as_stream(stream));
}

int pxs_linear(int dtype, const void * x, int64_t rows, int cin, const void * weight,
               const float * bias, int cout, int act, void * y, void * stream) {
    if (int rc = check_dtype(dtype, "pxs_linear")) return rc;
    PXS_CHECK(rows >= 0 && cin > 0 && cout > 0, PXS_ERR_ARG, "pxs_linear: bad shape");
    PXS_CHECK(act == PXS_ACT_NONE || act == PXS_ACT_GELU_TANH || act == PXS_ACT_SILU,
              PXS_ERR_ARG, "pxs_linear: bad activation");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x && weight && y, PXS_ERR_ARG, "pxs_linear: null pointer");
    GemmArgs a{};
    a.x = x; a.rows_in = rows; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = rows; a.rowmap = nullptr; a.ld_map = 0; a.noff = 1; a.masks = nullptr;
    a.y = y; a.ldy = cout; a.act = act;
    return run_gemm(dtype, a, kEpiStore, as_stream(stream));
}

int pxs_linear_gate_residual(int dtype, const void * x, int64_t rows, int cin,
                             const void * weight, const float * bias, int cout,
                             const int32_t * coords, const float * block_mod,
                             const float * time_mod, int gate_offset, float * residual,
                             void * stream) {
    if (int rc = check_dtype(dtype, "pxs_linear_gate_residual")) return rc;
    PXS_CHECK(rows >= 0 && cin > 0 && cout > 0 && gate_offset >= 0, PXS_ERR_ARG,
              "pxs_linear_gate_residual: bad shape");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x && weight && coords && block_mod && time_mod && residual, PXS_ERR_ARG,
              "pxs_linear_gate_residual: null pointer");
    GemmArgs a{};
    a.x = x; a.rows_in = rows; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = rows; a.noff = 1; a.y = nullptr; a.ldy = cout;
    a.coords = coords; a.block_mod = block_mod; a.time_mod = time_mod;
    a.gate_offset = gate_offset; a.residual = residual;
    return run_gemm(dtype, a, kEpiGateResidual, as_stream(stream));
}

int pxs_downsample_mean_s2(int dtype, const void * x, int channels, const int32_t * child_map,
                           int64_t ld_map, int64_t m, void * y, void * stream) {
    if (int rc = check_dtype(dtype, "pxs_downsample_mean_s2")) return rc;
    PXS_CHECK(channels > 0 && m >= 0 && ld_map >= m, PXS_ERR_ARG, "pxs_downsample_mean_s2: bad shape");
    if (m == 0) return PXS_OK;
    PXS_CHECK(x && child_map && y, PXS_ERR_ARG, "pxs_downsample_mean_s2: null pointer");
    PXS_CHECK(m <= INT32_MAX, PXS_ERR_ARG, "pxs_downsample_mean_s2: too many rows");
    const int threads = channels >= 256 ? 256 : 64;
    if (dtype == PXS_F32) {
        hipLaunchKernelGGL(downsample_mean_kernel<float>, dim3(static_cast<unsigned>(m)),
                           dim3(threads), 0, as_stream(stream), static_cast<const float *>(x),
                           channels, child_map, ld_map, m, static_cast<float *>(y));
    } else {
        hipLaunchKernelGGL(downsample_mean_kernel<uint16_t>, dim3(static_cast<unsigned>(m)),
                           dim3(threads), 0, as_stream(stream), static_cast<const uint16_t *>(x),
                           channels, child_map, ld_map, m, static_cast<uint16_t *>(y));
    }
    return check_launch("pxs_downsample_mean_s2");
}

} // extern "C"
