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
#include "s2emit.h"
#include "scan.h"

#include <type_traits>

namespace pxs {
namespace {

constexpr int kGemmThreads = 256;
constexpr int kChunkBytes = 128;
constexpr int kPitch = kChunkBytes + 16;

enum Epilogue { kEpiStore = 0, kEpiGateResidual = 1, kEpiAddResidual = 2 };

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
    // Neighbours from a dense voxel grid instead of rowmap (SubMConv3d only,
    // noff = 27): output row p's source at offset k is the grid cell next to
    // coords[p] (voxel_grid_row; generation 0 = plain grid).
    const uint32_t * grid;
    int grid_b, grid_x, grid_y, grid_z;
    uint32_t grid_gen;
    // Side work carried by the launch (LDS-pipeline kernels only): workgroups
    // [0, s2.blocks) run the stride-2 emit (s2emit.h) instead of a tile.
    int side_blocks;
    S2EmitArgs s2;
};

// Source row of output row p (coordinates c) at 3x3x3 offset k = kd*9 + kh*3
// + kw, looked up in the grid, or -1: the entry pxs_neighbor_map_k3_grid
// (or _tagged) would write, computed where the convolution needs it.  The
// centre is the row itself, as in the map.
__device__ __forceinline__ int32_t grid_src(const GemmArgs & a, int4 c, int k, int64_t p) {
    if (k == 13) return static_cast<int32_t>(p);
    const int x = c.y + k / 9 - 1, y = c.z + (k / 3) % 3 - 1, z = c.w + k % 3 - 1;
    if (static_cast<unsigned>(c.x) >= static_cast<unsigned>(a.grid_b) ||
        static_cast<unsigned>(x) >= static_cast<unsigned>(a.grid_x) ||
        static_cast<unsigned>(y) >= static_cast<unsigned>(a.grid_y) ||
        static_cast<unsigned>(z) >= static_cast<unsigned>(a.grid_z))
        return -1;
    const int64_t cell = ((static_cast<int64_t>(c.x) * a.grid_x + x) * a.grid_y + y) * a.grid_z + z;
    const int32_t s = voxel_grid_row(a.grid[cell], a.grid_gen);
    return s < a.rows_in ? s : -1;
}

// Grid mode prologue: all 27 sources of the tile's rows into idx[k * BM +
// row] (-1 absent or past the end), OR-ing each row's present offsets into
// *tile_mask.  Each thread takes one row and a quarter of the offsets, so a
// row's coordinates are read once per thread.
//
// Over a grid at least 3 cells deep in z, the 3 offsets kw of a kh row q =
// (kd, kh) are the cells z - 1, z, z + 1 of one grid column: each thread takes
// one row and the kh rows q = part, part + 4, part + 8, one 12-byte load each.
template <int BM>
__device__ __forceinline__ void grid_tile_sources(const GemmArgs & a, int64_t p0, int tid,
                                                  int nthreads, int32_t * idx,
                                                  uint32_t * tile_mask) {
    const int4 * crd = reinterpret_cast<const int4 *>(a.coords);
    uint32_t local = 0;
    if (a.grid_z >= 3) {
        for (int t = tid; t < 4 * BM; t += nthreads) {
            const int row = t % BM, part = t / BM;
            const int64_t p = p0 + row;
            const bool live = p < a.m;
            const int4 c = live ? crd[p] : make_int4(0, 0, 0, 0);
            const int z0 = min(max(c.w - 1, 0), a.grid_z - 3);  // first cell loaded
#pragma unroll
            for (int u = 0; u < 3; ++u) {
                const int q = part + 4 * u;
                if (q >= 9) break;
                const int x = c.y + q / 3 - 1, y = c.z + q % 3 - 1;
                const bool ok = live && static_cast<unsigned>(c.x) < static_cast<unsigned>(a.grid_b) &&
                                static_cast<unsigned>(x) < static_cast<unsigned>(a.grid_x) &&
                                static_cast<unsigned>(y) < static_cast<unsigned>(a.grid_y);
                uint32_t cell[3] = {kVoxelGridEmpty, kVoxelGridEmpty, kVoxelGridEmpty};
                if (ok) {
                    typedef uint32_t u32x3 __attribute__((ext_vector_type(3), aligned(4)));
                    const u32x3 v = *reinterpret_cast<const u32x3 *>(
                        a.grid + ((static_cast<int64_t>(c.x) * a.grid_x + x) * a.grid_y + y) * a.grid_z + z0);
                    cell[0] = v.x;
                    cell[1] = v.y;
                    cell[2] = v.z;
                }
#pragma unroll
                for (int dz = 0; dz < 3; ++dz) {
                    const int k = 3 * q + dz, z = c.w + dz - 1;
                    int32_t src = -1;
                    if (ok && static_cast<unsigned>(z) < static_cast<unsigned>(a.grid_z)) {
                        const int e = z - z0;  // 0..2, selected without indexing the registers
                        const uint32_t v = e == 0 ? cell[0] : (e == 1 ? cell[1] : cell[2]);
                        src = k == 13 ? static_cast<int32_t>(p) : voxel_grid_row(v, a.grid_gen);
                        if (src >= a.rows_in) src = -1;
                    }
                    idx[k * BM + row] = src;
                    if (src >= 0) local |= 1u << k;
                }
            }
        }
        if (local) atomicOr(tile_mask, local);
        return;
    }
    for (int t = tid; t < 4 * BM; t += nthreads) {
        const int row = t % BM, kb = (t / BM) * 7, ke = kb + 7 < 27 ? kb + 7 : 27;
        const int64_t p = p0 + row;
        if (p < a.m) {
            const int4 c = crd[p];
            for (int k = kb; k < ke; ++k) {
                const int32_t src = grid_src(a, c, k, p);
                idx[k * BM + row] = src;
                if (src >= 0) local |= 1u << k;
            }
        } else {
            for (int k = kb; k < ke; ++k) idx[k * BM + row] = -1;
        }
    }
    if (local) atomicOr(tile_mask, local);
}

template <typename T> struct Mfma;

template <> struct Mfma<uint16_t> {
    static constexpr int kVec = 8;            // elements per 16 bytes
    static constexpr int kChunk = 64;         // elements per 128-byte chunk
};

template <> struct Mfma<float> {
    static constexpr int kVec = 4;
    static constexpr int kChunk = 32;
};

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

// Epilogue.  32x32 accumulator layout: lane (h, r), register v holds row
// 8*(v/4) + 4*h + v%4, column r of the 32x32 tile.
template <typename T, int TI, int TJ, int WM, int WN, int EPI, bool COHERENT = false>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs & a, const f32x16 (&acc)[TI][TJ],
                                              int64_t p0, int n0, int wm, int wn, int h, int r) {
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
                    if constexpr (COHERENT)
                        store_f32_coherent(static_cast<T *>(a.y) + row * a.ldy + col, val);
                    else
                        store_f32(static_cast<T *>(a.y) + row * a.ldy + col, val);
                } else if constexpr (EPI == kEpiAddResidual) {
                    float * res = a.residual + row * a.cout + col;
                    *res = *res + val;
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

// The bf16 store epilogue through LDS.  Each lane writes its 32x32 blocks
// (bias and activation applied) into a BM x BN tile staged at `stage`; tile
// rows row0 + wm*WM + i*32 + ... come from this call's accumulators.  Then the
// workgroup writes whole 16-byte row pieces, where 2-byte element stores
// would take eight times the store instructions.  The caller has made
// `stage` free; cout and ldy are multiples of 8 and y is 16-byte aligned.
template <int BM, int BN, int TI, int TJ, int WM, int WN, int NT, bool COHERENT>
__device__ __forceinline__ void gemm_epilogue_staged(const GemmArgs & a, const f32x16 (&acc)[TI][TJ],
                                                     char * stage, int64_t p0, int n0, int row0,
                                                     int wm, int wn, int h, int r, int tid) {
    constexpr int kPitch = BN * 2 + 16;
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int cl = wn * WN + j * 32 + r;
            const float b = (a.bias && n0 + cl < a.cout) ? a.bias[n0 + cl] : 0.0f;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int rl = row0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                float val = acc[i][j][v] + b;
                if (a.act == PXS_ACT_GELU_TANH) val = gelu_tanh_f(val);
                else if (a.act == PXS_ACT_SILU) val = silu_f(val);
                *reinterpret_cast<uint16_t *>(stage + rl * kPitch + cl * 2) = f32_to_bf16(val);
            }
        }
    barrier_no_fence();
    uint16_t * y = static_cast<uint16_t *>(a.y);
    for (int q = tid; q < BM * (BN / 8); q += NT) {
        const int rl = q / (BN / 8), piece = q % (BN / 8);
        const int64_t row = p0 + rl;
        const int col = n0 + piece * 8;
        if (row < a.m && col < a.cout) {
            const uint4 v = *reinterpret_cast<const uint4 *>(stage + rl * kPitch + piece * 16);
            if constexpr (COHERENT) store16_coherent(y + row * a.ldy + col, v);
            else *reinterpret_cast<uint4 *>(y + row * a.ldy + col) = v;
        }
    }
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
            if (a.grid) {
                const int4 c = reinterpret_cast<const int4 *>(a.coords)[p];
                for (int k = 0; k < 27; ++k)
                    if (grid_src(a, c, k, p) >= 0) local |= 1u << k;
            } else if (a.masks) {
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
                if (a.grid) src = grid_src(a, reinterpret_cast<const int4 *>(a.coords)[p], k, p);
                else src = a.rowmap ? static_cast<int64_t>(a.rowmap[k * a.ld_map + p]) : p;
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

    gemm_epilogue<T, TI, TJ, WM, WN, EPI>(a, acc, p0, n0, wm, wn, h, r);
}


// ---------------------------------------------------------------------------
// Pipelined variant for 16-byte-aligned operands: tiles stream from HBM/L2
// straight into LDS with global_load_lds_dwordx4 (no VGPR staging), NSTAGE
// stages in flight.  Each wavefront instruction fills 1 KiB of LDS = 8 rows x
// 128 bytes, lane l landing at offset 16*l; the 16-byte piece a lane fetches
// is XOR-swizzled so that the MFMA fragment reads (32 rows, one piece) hit
// distinct banks.  The gathered row indices of the tile (for every present
// offset) are staged in LDS once at the start, so a stage issues its loads
// without waiting on an index load.

__device__ __align__(16) uint4 g_zero_chunk[8];  // 128 zero bytes for absent rows

// Measured on MI355X (SubMConv3d 128->128 / 256->256, linear 1024->3072):
// the kernel is bound by the latency of the gathered loads, so resident waves
// matter most.  128x128 tiles in two stages (64 KiB + indices, two
// workgroups per CU) with 8 waves of 64x32 each beat 4 waves of 64x64,
// 256-row tiles and 3-4 stage pipelines (which fit only one workgroup per CU).
// Loading gathered rows straight into VGPRs (64 bytes per lane, weights alone
// through LDS) lost 15-20% in the U-Net stage: its 32-byte row pieces per
// instruction coalesce worse than these 8 full 128-byte row chunks.  Staging
// them through VGPRs with this kernel's own load pattern, two steps ahead of
// the LDS ring (twice the gathers in flight), lost 10%: the kernel is not
// bound by load latency; each stage moves 128 KiB through LDS per workgroup
// (fragment reads plus DMA writes) with the matrix cores about a third busy.
// Splitting each stage's four K steps between two groups of 4 waves with
// 64x64 blocks (KSPLIT = 2) cuts that to 96 KiB: U-Net stage +3.5%.
// Reordering rows so that 128-row tiles share neighbour masks (buckets of the
// face offsets, or of the x-1/x+1 planes: up to 20% fewer offset stages)
// lost 2-15% to the lost locality of the gathered rows.
#ifndef PXS_GEMM_STAGES
#define PXS_GEMM_STAGES 2
#endif
#ifndef PXS_GEMM_BM
#define PXS_GEMM_BM 128
#endif
#ifndef PXS_GEMM_BN
#define PXS_GEMM_BN 128
#endif
#ifndef PXS_GEMM_WAVES
#define PXS_GEMM_WAVES 8
#endif
#ifndef PXS_GEMM_WAVES_M
#define PXS_GEMM_WAVES_M 2
#endif
#ifndef PXS_GEMM_KSPLIT
#define PXS_GEMM_KSPLIT 2
#endif
#ifndef PXS_GEMM_WIDE
#define PXS_GEMM_WIDE 1
#endif

#ifndef PXS_GEMM_ISSUE_LATE
#define PXS_GEMM_ISSUE_LATE 0
#endif
// Late issue: queue the next stage's loads after this stage's MFMAs (the
// buffer they fill was released by the barrier at the top of the iteration).
constexpr bool kIssueLate = PXS_GEMM_ISSUE_LATE != 0;

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// Absent gathered rows (a neighbour missing for this output row, or a row
// past the tile end): with PXS_GEMM_MASK_ABSENT their lanes are left out of
// the LDS DMA, and the fragment reads replace their stale LDS bytes with
// zeros in registers, so no bytes travel for them.
#ifndef PXS_GEMM_MASK_ABSENT
#define PXS_GEMM_MASK_ABSENT 0
#endif
constexpr bool kMaskAbsent = PXS_GEMM_MASK_ABSENT != 0;


template <int BM, int BN, int NSTAGE>
constexpr int lds_gemm_bytes(int noff) {
    return NSTAGE * (BM + BN) * kChunkBytes + noff * BM * 4;
}

// Dependencies between the workgroups of one launch (the chained U-Net
// level): flags in global memory set to the launch's generation when a
// producer's results are visible to the device.  A producer writes what
// consumers read with device-coherent stores (sc1) and waits for them to
// complete before it sets its flag; a consumer reads the flag and then the
// produced data with device-coherent loads.  So no L2 is written back or
// invalidated, which would stall, or cost every other tile on that XCD its
// cached operands.  A consumer
// workgroup only waits for workgroups with a lower index, which the
// dispatcher places before it on every XCD, so the waits end.  The spin is
// bounded all the same: a wait that gives up (after about a second) sets
// *error and goes on, so the launch always completes and the caller can see
// that its results are void.
struct TileSync {
    const uint32_t * emit_flags;  // wait for emit_flags[0, emit_count) == gen
    int emit_count;
    const uint32_t * src_flags;   // wait for the producer tiles holding this tile's sources
    int src_bm, src_tiles_n;      // producer rows per tile, producer column tiles
    uint32_t * done_flags;        // set done_flags[logical] = gen when this tile is stored
    uint32_t gen;
    uint32_t * error;
};

__device__ __forceinline__ void spin_until(const uint32_t * flag, uint32_t gen, uint32_t * error) {
    for (int it = 0; it < (1 << 20); ++it) {
        if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) return;
        __builtin_amdgcn_s_sleep(4);
    }
    atomicOr(error, 1u);
}

// NW waves per workgroup in KSPLIT groups; the waves of a group form a
// WAVES_M x (NW / KSPLIT / WAVES_M) grid, each owning a block of the output
// tile.  With KSPLIT = 2 the two groups take alternate 16-element K steps
// of every stage and add their partial sums once at the end: 8 waves of
// 64x64 blocks read each LDS fragment for two MFMAs instead of 1.5.
template <typename T, int BM, int BN, int EPI, int NSTAGE, int NW, int WAVES_M, int KSPLIT, bool SYNC>
__device__ __forceinline__ void gemm_lds_tile(const GemmArgs & a, int logical, const TileSync & sync,
                                              char * smem) {
    constexpr int kVec = Mfma<T>::kVec;
    constexpr int kChunk = Mfma<T>::kChunk;
    constexpr int kThreads = NW * 64;
    constexpr int NWG = NW / KSPLIT;
    constexpr int WAVES_N = NWG / WAVES_M;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int TI = WM / 32, TJ = WN / 32;
    constexpr int KSTEPS = 4 / KSPLIT;  // 16-element K steps per stage and group
    static_assert(KSPLIT == 1 || (KSPLIT == 2 && sizeof(T) == 2 && TI % 2 == 0),
                  "K split: bf16 only, an even number of 32-row blocks per wave");
    constexpr int kStageBytes = (BM + BN) * kChunkBytes;
    constexpr int AI = BM / (8 * NW);  // A instructions per wave per stage (8 rows each)
    constexpr int BI = BN / (8 * NW);
    constexpr int kPerStage = AI + BI;
    static_assert(AI * 8 * NW == BM && BI * 8 * NW == BN, "tile rows must split over the waves");

    int32_t * idx_lds = reinterpret_cast<int32_t *>(smem + NSTAGE * kStageBytes);
    __shared__ uint32_t tile_mask;
    __shared__ int koff[32];
    __shared__ int src_lo, src_hi;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int kg = wave / NWG, wl = wave % NWG;
    const int wm = wl / WAVES_N, wn = wl % WAVES_N;
    const int h = lane >> 5, r = lane & 31;

    const int tiles_n = (a.cout + BN - 1) / BN;
    const int64_t p0 = static_cast<int64_t>(logical / tiles_n) * BM;
    const int n0 = (logical % tiles_n) * BN;
    const T * __restrict__ x = static_cast<const T *>(a.x);
    const T * __restrict__ w = static_cast<const T *>(a.w);

    if constexpr (SYNC) {
        // A consumer waits for the side workgroups that wrote its map.
        if (sync.emit_flags) {
            for (int i = tid; i < sync.emit_count; i += kThreads) spin_until(sync.emit_flags + i, sync.gen, sync.error);
            __syncthreads();
        }
    }
    if (tid == 0) tile_mask = 0;
    __syncthreads();
    // A map without masks (the stride-2 conv's child map) is read once: every
    // offset's sources go into idx_lds[k * BM + row] while the mask is formed,
    // as in grid mode, instead of a mask pass and then a pass over the
    // present offsets.
    const bool full_table = a.grid || (a.rowmap && !a.masks);
    if (a.grid) {
        grid_tile_sources<BM>(a, p0, tid, kThreads, idx_lds, &tile_mask);
    } else if (full_table) {
        uint32_t local = 0;
        for (int e = tid; e < a.noff * BM; e += kThreads) {
            const int k = e / BM, row = e % BM;
            int32_t src = -1;
            if (p0 + row < a.m) {
                const int32_t * q = a.rowmap + k * a.ld_map + p0 + row;
                int32_t s;
                if constexpr (SYNC) {
                    // a map written in this launch: a device-coherent load
                    s = sync.emit_flags ? __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                        : *q;
                } else {
                    s = *q;
                }
                src = (s >= 0 && s < a.rows_in) ? s : -1;
            }
            idx_lds[e] = src;
            if (src >= 0) local |= 1u << k;
        }
        if (local) atomicOr(&tile_mask, local);
    } else {
        uint32_t local = 0;
        for (int row = tid; row < BM; row += kThreads) {
            if (p0 + row >= a.m) break;
            const int64_t p = p0 + row;
            if (a.masks) {
                local |= a.masks[p];
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
    const uint32_t present = tile_mask & (a.noff >= 32 ? ~0u : ((1u << a.noff) - 1u));
    const int kcount = __popc(present);
    if (tid == 0) {
        uint32_t m = present;
        for (int i = 0; i < kcount; ++i) {
            koff[i] = __ffs(m) - 1;
            m &= m - 1;
        }
    }
    __syncthreads();
    // idx_lds rows: the tile's present offsets in order (i), or with a full
    // table every offset (k = koff[i]).
    for (int e = tid; !full_table && e < kcount * BM; e += kThreads) {
        const int i = e / BM, row = e % BM;
        int32_t src = -1;
        if (p0 + row < a.m) {
            const int64_t p = p0 + row;
            const int64_t s = a.rowmap ? static_cast<int64_t>(a.rowmap[koff[i] * a.ld_map + p]) : p;
            src = (s >= 0 && s < a.rows_in) ? static_cast<int32_t>(s) : -1;
        }
        idx_lds[e] = src;
    }
    __syncthreads();
    if constexpr (SYNC) {
        // A consumer waits for the producer tiles that wrote its source rows
        // (rows [t * src_bm, (t + 1) * src_bm) of producer row tile t).
        if (sync.src_flags) {
            if (tid == 0) {
                src_lo = INT_MAX;
                src_hi = -1;
            }
            __syncthreads();
            int lo = INT_MAX, hi = -1;
            const int entries = (full_table ? a.noff : kcount) * BM;
            for (int e = tid; e < entries; e += kThreads) {
                const int src = idx_lds[e];
                if (src >= 0) {
                    lo = min(lo, src);
                    hi = max(hi, src);
                }
            }
            if (hi >= 0) {
                atomicMin(&src_lo, lo);
                atomicMax(&src_hi, hi);
            }
            __syncthreads();
            if (src_hi >= 0) {
                const int t0 = src_lo / sync.src_bm, t1 = src_hi / sync.src_bm;
                const int count = (t1 - t0 + 1) * sync.src_tiles_n;
                for (int i = tid; i < count; i += kThreads)
                    spin_until(sync.src_flags + static_cast<int64_t>(t0) * sync.src_tiles_n + i, sync.gen,
                               sync.error);
            }
            __syncthreads();
        }
    }
    // Sources written in this launch are read with device-coherent loads.
    bool coherent_x = false;
    if constexpr (SYNC) coherent_x = sync.src_flags != nullptr;

    const int chunks = (a.cin + kChunk - 1) / kChunk;
    const int stages = kcount * chunks;
    const int lrow = lane >> 3, lslot = lane & 7;
    const void * zero = static_cast<const void *>(g_zero_chunk);

    // Per-lane constant parts of the load addresses: the row this lane fills
    // in each of its instructions and the swizzled 16-byte piece it fetches.
    int a_row[AI], a_piece[AI];
#pragma unroll
    for (int j = 0; j < AI; ++j) {
        a_row[j] = (wave * AI + j) * 8 + lrow;
        a_piece[j] = lslot ^ swz(a_row[j]);
    }
    int64_t b_off[BI];
    int b_piece[BI];
    bool b_ok[BI];
#pragma unroll
    for (int j = 0; j < BI; ++j) {
        const int row = (wave * BI + j) * 8 + lrow;
        b_piece[j] = lslot ^ swz(row);
        b_ok[j] = n0 + row < a.cout;
        b_off[j] = static_cast<int64_t>(n0 + row) * a.cin + b_piece[j] * kVec;
    }

    auto issue = [&](int s) {
        const int i = s / chunks, chunk = s - i * chunks;
        const int k = koff[i];
        char * base = smem + (s % NSTAGE) * kStageBytes;
        int32_t src[AI];
        const int slot = full_table ? k : i;
#pragma unroll
        for (int j = 0; j < AI; ++j) src[j] = idx_lds[slot * BM + a_row[j]];
#pragma unroll
        for (int j = 0; j < AI; ++j) {
            const int col = chunk * kChunk + a_piece[j] * kVec;
            const void * g = (src[j] >= 0 && col < a.cin)
                                 ? static_cast<const void *>(x + static_cast<int64_t>(src[j]) * a.ldx + col)
                                 : zero;
            if constexpr (kMaskAbsent) {
                // lane 0 always issues (zero line when its row is absent)
                const uint64_t lanes = __ballot(src[j] >= 0) | 1ull;
                lds_dma16_masked(g, lds_offset(base + (wave * AI + j) * 8 * kChunkBytes), lanes);
            } else if (SYNC && coherent_x) {
                lds_dma16_coherent(g, lds_offset(base + (wave * AI + j) * 8 * kChunkBytes));
            } else {
                lds_dma16(g, lds_offset(base + (wave * AI + j) * 8 * kChunkBytes));
            }
        }
        const int64_t kbase = static_cast<int64_t>(k) * a.cout * a.cin + chunk * kChunk;
#pragma unroll
        for (int j = 0; j < BI; ++j) {
            const int col = chunk * kChunk + b_piece[j] * kVec;
            const void * g = (b_ok[j] && col < a.cin) ? static_cast<const void *>(w + kbase + b_off[j]) : zero;
            lds_dma16(g, lds_offset(base + (BM + (wave * BI + j) * 8) * kChunkBytes));
        }
    };

    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

#pragma unroll
    for (int s = 0; s < NSTAGE - 1; ++s)
        if (s < stages) issue(s);

    for (int s = 0; s < stages; ++s) {
        const int after = min(NSTAGE - 2, stages - 1 - s);
        wait_vmcnt(after * kPerStage);
        barrier_no_fence();
        if constexpr (!kIssueLate) {
            if (s + NSTAGE - 1 < stages) issue(s + NSTAGE - 1);
        }
        const char * sa = smem + (s % NSTAGE) * kStageBytes;
        const char * sb = sa + BM * kChunkBytes;
        bool row_ok[TI];
#pragma unroll
        for (int i = 0; i < TI; ++i) {
            row_ok[i] = true;
            if constexpr (kMaskAbsent)
                row_ok[i] = idx_lds[(full_table ? koff[s / chunks] : s / chunks) * BM + wm * WM + i * 32 + r] >= 0;
        }
        if constexpr (sizeof(T) == 2) {
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) {
                const int piece = 4 * h + kg * KSTEPS + kk;
                bf16x8 af[TI], bfr[TJ];
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const int row = wm * WM + i * 32 + r;
                    uint4 raw = *reinterpret_cast<const uint4 *>(sa + row * kChunkBytes +
                                                                 ((piece ^ swz(row)) << 4));
                    if constexpr (kMaskAbsent) {
                        if (!row_ok[i]) raw = make_uint4(0, 0, 0, 0);
                    }
                    af[i] = __builtin_bit_cast(bf16x8, raw);
                }
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const int row = wn * WN + j * 32 + r;
                    bfr[j] = *reinterpret_cast<const bf16x8 *>(sb + row * kChunkBytes +
                                                               ((piece ^ swz(row)) << 4));
                }
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
                const int piece = 4 * h + u;
                f32x4 af[TI], bfr[TJ];
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const int row = wm * WM + i * 32 + r;
                    uint4 raw = *reinterpret_cast<const uint4 *>(sa + row * kChunkBytes +
                                                                 ((piece ^ swz(row)) << 4));
                    if constexpr (kMaskAbsent) {
                        if (!row_ok[i]) raw = make_uint4(0, 0, 0, 0);
                    }
                    af[i] = __builtin_bit_cast(f32x4, raw);
                }
#pragma unroll
                for (int j = 0; j < TJ; ++j) {
                    const int row = wn * WN + j * 32 + r;
                    bfr[j] = *reinterpret_cast<const f32x4 *>(sb + row * kChunkBytes +
                                                              ((piece ^ swz(row)) << 4));
                }
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
        if constexpr (kIssueLate) {
            if (s + NSTAGE - 1 < stages) issue(s + NSTAGE - 1);
        }
    }
    // A producer of the chained launch stores device-coherently.
    bool coherent_y = false;
    if constexpr (SYNC) coherent_y = sync.done_flags != nullptr;
    // bf16 stores go through a tile staged in the stage buffers when it fits
    // there and whole 16-byte row pieces are aligned (the same for every
    // thread of the launch).
    constexpr int kStagedPitch = BN * 2 + 16;
    constexpr bool kStageable =
        EPI == kEpiStore && sizeof(T) == 2 && BM * kStagedPitch <= NSTAGE * kStageBytes;
    const bool staged = kStageable && a.cout % 8 == 0 && a.ldy % 8 == 0 &&
                        (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;
    if constexpr (KSPLIT == 1) {
        if (kStageable && staged) {
            barrier_no_fence();  // every wave is done reading the stage buffers
            if (SYNC && coherent_y)
                gemm_epilogue_staged<BM, BN, TI, TJ, WM, WN, kThreads, true>(a, acc, smem, p0, n0, 0, wm, wn,
                                                                           h, r, tid);
            else
                gemm_epilogue_staged<BM, BN, TI, TJ, WM, WN, kThreads, false>(a, acc, smem, p0, n0, 0, wm, wn,
                                                                            h, r, tid);
        } else if (SYNC && coherent_y) {
            gemm_epilogue<T, TI, TJ, WM, WN, EPI, true>(a, acc, p0, n0, wm, wn, h, r);
        } else {
            gemm_epilogue<T, TI, TJ, WM, WN, EPI>(a, acc, p0, n0, wm, wn, h, r);
        }
    } else {
        // Group 0 finishes the upper 32-row blocks of each wave's tile and
        // group 1 the lower ones; each hands the other half of its partial
        // sums over through the (now idle) stage buffers.  A lane's slot is
        // its own register index, so the exchange is conflict-free, and the
        // sum a + b is the same whichever group adds it.
        constexpr int HI = TI / 2;
        // The exchange runs in PASSES rounds over the 32-column blocks j when
        // the whole of it does not fit in the stage buffers.
        constexpr int kXchBytes = NW * HI * TJ * 16 * 64 * 4;
        constexpr int PASSES = (kXchBytes + NSTAGE * kStageBytes - 1) / (NSTAGE * kStageBytes);
        constexpr int TJP = TJ / PASSES;
        static_assert(TJP * PASSES == TJ, "exchange passes must split the column blocks");
        float * xch = reinterpret_cast<float *>(smem);
        auto slot = [&](int group, int i, int j, int v) {
            return ((((group * NWG + wl) * HI + i) * TJP + j) * 16 + v) * 64 + lane;
        };
        auto finish = [&](auto keep_tag) {
            constexpr int KEEP = decltype(keep_tag)::value, GIVE = HI - KEEP;
            f32x16 fin[HI][TJ];
#pragma unroll
            for (int pass = 0; pass < PASSES; ++pass) {
                if (pass > 0) barrier_no_fence();  // the previous pass's sums are read
#pragma unroll
                for (int i = 0; i < HI; ++i)
#pragma unroll
                    for (int j = 0; j < TJP; ++j)
#pragma unroll
                        for (int v = 0; v < 16; ++v)
                            xch[slot(kg, i, j, v)] = acc[GIVE + i][pass * TJP + j][v];
                barrier_no_fence();
#pragma unroll
                for (int i = 0; i < HI; ++i)
#pragma unroll
                    for (int j = 0; j < TJP; ++j)
#pragma unroll
                        for (int v = 0; v < 16; ++v)
                            fin[i][pass * TJP + j][v] =
                                acc[KEEP + i][pass * TJP + j][v] + xch[slot(1 - kg, i, j, v)];
            }
            if (kStageable && staged) {
                // A producer of the chained launch writes whole 16-byte
                // pieces device-coherently (2-byte write-through stores would
                // each go to memory on their own).
                barrier_no_fence();  // the partner's sums are read: the exchange area is free
                if (SYNC && coherent_y)
                    gemm_epilogue_staged<BM, BN, HI, TJ, WM, WN, kThreads, true>(a, fin, smem, p0, n0, KEEP * 32,
                                                                               wm, wn, h, r, tid);
                else
                    gemm_epilogue_staged<BM, BN, HI, TJ, WM, WN, kThreads, false>(a, fin, smem, p0, n0, KEEP * 32,
                                                                                wm, wn, h, r, tid);
            } else if (SYNC && coherent_y) {
                gemm_epilogue<T, HI, TJ, WM, WN, EPI, true>(a, fin, p0 + KEEP * 32, n0, wm, wn, h, r);
            } else {
                gemm_epilogue<T, HI, TJ, WM, WN, EPI>(a, fin, p0 + KEEP * 32, n0, wm, wn, h, r);
            }
        };
        barrier_no_fence();  // every wave is done reading the stage buffers
        if (kg == 0) finish(std::integral_constant<int, 0>{});
        else finish(std::integral_constant<int, HI>{});
    }
    if constexpr (SYNC) {
        // A producer publishes the tile: every thread's stores made visible
        // to the device, then the tile's flag set to this launch's value.
        if (sync.done_flags) {
            release_stores();
            __syncthreads();
            if (tid == 0)
                __hip_atomic_store(sync.done_flags + logical, sync.gen, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <typename T, int BM, int BN, int EPI, int NSTAGE, int NW, int WAVES_M, int KSPLIT>
__global__ void __launch_bounds__(NW * 64)
gather_gemm_lds_kernel(GemmArgs a) {
    extern __shared__ __align__(16) char smem[];
    // Side workgroups last: dispatched in order, they take the slots the
    // tiles' last, partial round leaves free.
    const int tiles = static_cast<int>(gridDim.x) - a.side_blocks;
    if (static_cast<int>(blockIdx.x) >= tiles) {
        s2_emit_block(a.s2, blockIdx.x - tiles, threadIdx.x, NW * 64, smem);
        return;
    }
    gemm_lds_tile<T, BM, BN, EPI, NSTAGE, NW, WAVES_M, KSPLIT, false>(
        a, remap_xcd(blockIdx.x, tiles), TileSync{}, smem);
}

// One U-Net level in one launch (pxs_unet_s2_level): workgroups [0, tiles_a)
// are SubMConv3d tiles (a), then `side` workgroups emit the stride-2
// topology (a.s2), then tiles_b stride-2 convolution tiles (b), which read
// the child map the emit writes and the rows conv a's tiles write.  Each
// consumer waits only on its own producers (TileSync), so the strided conv's
// tiles run in the slots conv a's last round leaves free.  tiles_a + side is
// a multiple of 8, so every role keeps its XCD mapping.
struct ChainArgs {
    int tiles_a, side, tiles_b, tiles_n_a;
    uint32_t * emit_flags;
    uint32_t * a_flags;
    uint32_t gen;
    uint32_t * error;
};

template <typename T, int BM, int BN, int NSTAGE, int NW, int WAVES_M, int KSPLIT>
__global__ void __launch_bounds__(NW * 64)
gather_gemm_lds_chain_kernel(GemmArgs a, GemmArgs b, ChainArgs c) {
    extern __shared__ __align__(16) char smem[];
    const int bid = blockIdx.x;
    if (bid < c.tiles_a) {
        TileSync sync{};
        sync.done_flags = c.a_flags;
        sync.gen = c.gen;
        sync.error = c.error;
        gemm_lds_tile<T, BM, BN, kEpiStore, NSTAGE, NW, WAVES_M, KSPLIT, true>(
            a, remap_xcd(bid, c.tiles_a), sync, smem);
        return;
    }
    if (bid < c.tiles_a + c.side) {
        s2_emit_block(a.s2, bid - c.tiles_a, threadIdx.x, NW * 64, smem);
        release_stores();
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_store(c.emit_flags + (bid - c.tiles_a), c.gen, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    TileSync sync{};
    sync.emit_flags = c.emit_flags;
    sync.emit_count = c.side;
    sync.src_flags = c.a_flags;
    sync.src_bm = BM;
    sync.src_tiles_n = c.tiles_n_a;
    sync.gen = c.gen;
    sync.error = c.error;
    gemm_lds_tile<T, BM, BN, kEpiStore, NSTAGE, NW, WAVES_M, KSPLIT, true>(
        b, remap_xcd(bid - c.tiles_a - c.side, c.tiles_b), sync, smem);
}

// ---------------------------------------------------------------------------
// SubMConv3d (bf16, 27 offsets) over neighbourhood ranges.  The 9 offsets
// (kh, kw) of one x-plane kd take their sources for a tile of 128
// consecutive output rows from an almost contiguous range of input rows: rows
// are sorted by (b, x, y, z), so the neighbours in plane x + kd - 1 of a run
// of rows lie between those of its first and last row (163 rows at the
// median on the U-Net shells, against 9 x 128 gathered row chunks).  A tile
// stages each plane's range [lo, hi] once per 64-channel chunk (one
// contiguous DMA, no index table) and then streams only the weights W_k of
// that plane's offsets; the MFMA operand of output row p at offset k is the
// staged row src(k, p) - lo, or a zero row where the neighbour is absent.
// A plane whose range exceeds kRangeCap rows is split into its three kh rows
// of offsets; a kh row that still exceeds it is staged per offset as the
// offset's 128 gathered rows.  The vector-memory instructions per tile fall
// from 1,728 to about 1,000 (the weights are now most of them).
//
// Pipeline: a ring of WS weight stages (each stage's weights issued WS - 1
// stages ahead) and one halo buffer, which the next (group, chunk) refills
// after every wave has read its operands of the group's last stage (a
// barrier inside that stage, the DMA then overlapping its MFMAs); 8 waves in
// two K groups of 2 x 2 blocks (64 x BN/2 each).  As launched: BN = 128, a
// 320-row halo and WS = 2, 80.8 KB of LDS, so two workgroups share a CU
// (outputs wider than 128 channels take one tile per 128 columns).  Stages
// run chunk by chunk, within a chunk group by group (planes ascending),
// within a group offsets ascending.  The tile is written through LDS as
// whole 16-byte row pieces.
#ifndef PXS_GEMM_RANGE
#define PXS_GEMM_RANGE 1
#endif
// Outputs of 65..PXS_GEMM_RANGE_MAXN channels run on range tiles (256: the
// U-Net's conv A and conv C; 128 keeps wider ones on gather tiles).
#ifndef PXS_GEMM_RANGE_MAXN
#define PXS_GEMM_RANGE_MAXN 256
#endif
// Weight ring slots: 2 (weights one stage ahead) leaves room for a 320-row
// halo at two workgroups per CU (81.4 KB with the static tables); 3 (two
// stages ahead) for 192 rows.
#ifndef PXS_GEMM_RANGE_WS
#define PXS_GEMM_RANGE_WS 2
#endif
constexpr int kRangeBM = 128, kRangeNW = 8, kRangeWS = PXS_GEMM_RANGE_WS;
constexpr int kRangeCap = kRangeWS == 2 ? 320 : 192;
template <int CAP> constexpr int range_halo_bytes() { return (CAP + 1) * kChunkBytes; }  // its zero row last
template <int BN, int CAP, int WS> constexpr int range_lds_bytes() {
    return WS * BN * kChunkBytes + range_halo_bytes<CAP>() + 27 * kRangeBM * 2;
}

// Tile of workgroup `bid`.  PXS_GEMM_RANGE_ORDER 1: chunks of
// PXS_GEMM_RANGE_CHUNK consecutive tiles dealt to the XCDs (bid % 8) in turn,
// so every XCD's share samples the whole volume and the XCDs finish together
// (the last partial block of 8 chunks in reverse order).  Conv A (1,268 tiles), one
// box: 0.1588-0.1596 ms with 0 (each XCD a contiguous range of tiles,
// remap_xcd, whose last tiles ended up to 13 us apart); chunks of 8
// 0.1547-0.1552 ms, then on another box chunks of 4 and 8 0.1538-0.1539 ms,
// of 16 0.1520-0.1525 ms, and on a third chunks of 16 0.1560-0.1563 ms, of 32
// 0.1544-0.1547 ms, of 64 0.1601-0.1605 ms.  Dealing tiles out fetches the
// rows of neighbouring planes into several XCDs' L2s: the launch reads
// 114.4 MB from HBM with chunks of 32 (126.8 MB with 16, 103.9 MB with 64,
// 77.3 MB with contiguous ranges), far from what binds it.
#ifndef PXS_GEMM_RANGE_ORDER
#define PXS_GEMM_RANGE_ORDER 1
#endif
#ifndef PXS_GEMM_RANGE_CHUNK
#define PXS_GEMM_RANGE_CHUNK 32
#endif
__device__ __forceinline__ int range_tile_order(int bid, int tiles) {
    constexpr int C = PXS_GEMM_RANGE_CHUNK;
    if (PXS_GEMM_RANGE_ORDER == 0) return remap_xcd(bid, tiles);
    const int full = tiles / (8 * C) * (8 * C);
    // the rest in reverse: the tiles at the end of the volume (the shells'
    // caps, whose wide planes refill the halo stage by stage) start first
    // instead of last (conv A 0.1530-0.1532 against 0.1538-0.1542 ms)
    if (bid >= full) return tiles - 1 - (bid - full);
    const int x = bid & 7, i = bid >> 3;
    return ((i / C) * 8 + x) * C + i % C;
}

// Min, max and or over each 16-lane row by DPP row shifts (VALU, no LDS
// round trip): lane 15 of every row ends with its row's result.
__device__ __forceinline__ int dpp_row_min(int v) {
    v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x111, 0xf, 0xf, false));  // row_shr:1
    v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x114, 0xf, 0xf, false));  // row_shr:4
    return min(v, __builtin_amdgcn_update_dpp(INT_MAX, v, 0x118, 0xf, 0xf, false));  // row_shr:8
}
__device__ __forceinline__ int dpp_row_max(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x111, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x112, 0xf, 0xf, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x114, 0xf, 0xf, false));
    return max(v, __builtin_amdgcn_update_dpp(-1, v, 0x118, 0xf, 0xf, false));
}
__device__ __forceinline__ uint32_t dpp_row_or(uint32_t v) {
    v |= __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xf, 0xf, false);
    v |= __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xf, 0xf, false);
    v |= __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xf, 0xf, false);
    return v | __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xf, 0xf, false);
}

template <int BN, int CAP, int WS>
__global__ void __launch_bounds__(kRangeNW * 64)
range_conv_bf16_kernel(GemmArgs a) {
    constexpr int BM = kRangeBM, NW = kRangeNW, NT = NW * 64;
    constexpr int L = WS - 1;  // weight stages issued ahead
    constexpr int NWG = NW / 2;               // waves per K group
    constexpr int WAVES_N = 2;                // each group: 2 x 2 blocks
    constexpr int WM = BM / 2, WN = BN / WAVES_N;
    constexpr int TI = WM / 32, TJ = WN / 32, HI = TI / 2;
    constexpr int BI = BN / (8 * NW);         // weight DMA instructions per wave per stage
    constexpr int kWBytes = BN * kChunkBytes;
    constexpr int kStagePitch = BN * 2 + 16;  // the output tile staged in LDS
    static_assert(BI >= 1 && TJ >= 1 && TI == 2, "tile shape");
    static_assert((WS == 2 || WS == 3) && 27 * BM * 4 <= kWBytes, "source table inside the last weight slot");
    // the K groups' partial sums are exchanged in XP passes over the column blocks
    constexpr int XP = (NW * HI * TJ * 16 * 64 * 4 + range_lds_bytes<BN, CAP, WS>() - 1) / range_lds_bytes<BN, CAP, WS>();
    constexpr int TJP = TJ / XP;
    static_assert(TJP * XP == TJ, "exchange passes split the column blocks");
    static_assert(BM * kStagePitch <= range_lds_bytes<BN, CAP, WS>(), "staged tile fits");
    extern __shared__ __align__(16) char smem[];
    const int tiles = static_cast<int>(gridDim.x) - a.side_blocks;
    if (static_cast<int>(blockIdx.x) >= tiles) {
        s2_emit_block(a.s2, blockIdx.x - tiles, threadIdx.x, NT, smem);
        return;
    }
    char * wring = smem;
    char * halo = smem + WS * kWBytes;
    // slots[k][p]: byte address in the halo of output row p's operand at
    // offset k, row * 128 + (swz(row) << 4), so a lane's 16-byte piece P is at
    // slots ^ (P << 4)
    uint16_t * slots = reinterpret_cast<uint16_t *>(halo + range_halo_bytes<CAP>());
    // prologue only, in the ring slot the stages issued before the loop do not use
    int32_t * idx = reinterpret_cast<int32_t *>(smem + L * kWBytes);
    __shared__ uint32_t tile_mask;
    __shared__ int rlo[9], rhi[9];        // source range of each kh row q = k / 3
    __shared__ int g_lo[27], g_rows[27];  // range start (-1 - k: offset k gathered), rows staged
    __shared__ uint32_t g_mask[27];       // offsets of each group
    __shared__ int g_of[27];              // group of each present offset
    // The stages of a chunk: the present offsets in ascending k (the group
    // order), entry i = {k * BM | group << 12 | first << 17 | last << 18, k * W_k bytes}.
    __shared__ uint2 ent[27];
    __shared__ int n_pos;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave / NWG, wl = wave % NWG;
    const int wm = wl / WAVES_N, wn = wl % WAVES_N;
    const int h = lane >> 5, r = lane & 31;
    const int lrow = lane >> 3, lslot = lane & 7;
    const int tiles_n = (a.cout + BN - 1) / BN;
    const int logical = range_tile_order(blockIdx.x, tiles);
    const int64_t p0 = static_cast<int64_t>(logical / tiles_n) * BM;
    const int n0 = (logical % tiles_n) * BN;
    const uint16_t * __restrict__ x = static_cast<const uint16_t *>(a.x);
    const int4 * crd = reinterpret_cast<const int4 *>(a.coords);

    // ---- the tile's sources and the range of each kh row ----
    if (tid == 0) tile_mask = 0;
    if (tid < 9) {
        rlo[tid] = INT_MAX;
        rhi[tid] = -1;
    }
    if (tid < 8) *reinterpret_cast<uint4 *>(halo + CAP * kChunkBytes + tid * 16) = make_uint4(0, 0, 0, 0);
    __syncthreads();
    if (a.grid && a.grid_z >= 3) {
        // Over a grid, the 3 offsets kw of a kh row q = (kd, kh) are the cells
        // z - 1, z, z + 1 of one grid column: one 12-byte load each.  Thread:
        // one row, kh rows q = part, part + 4, part + 8 (part wave-uniform).
        const int row = tid % BM, part = tid / BM;
        const int64_t p = p0 + row;
        const bool live = p < a.m;
        const int4 c = live ? crd[p] : make_int4(0, 0, 0, 0);
        const int z0 = min(max(c.w - 1, 0), a.grid_z - 3);  // first cell loaded
        uint32_t cell[3][3];
        bool col_ok[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int q = part + 4 * u;
            const int x = c.y + q / 3 - 1, y = c.z + q % 3 - 1;
            col_ok[u] = live && q < 9 && static_cast<unsigned>(c.x) < static_cast<unsigned>(a.grid_b) &&
                        static_cast<unsigned>(x) < static_cast<unsigned>(a.grid_x) &&
                        static_cast<unsigned>(y) < static_cast<unsigned>(a.grid_y);
            if (col_ok[u]) {
                typedef uint32_t u32x3 __attribute__((ext_vector_type(3), aligned(4)));
                const u32x3 v = *reinterpret_cast<const u32x3 *>(
                    a.grid + ((static_cast<int64_t>(c.x) * a.grid_x + x) * a.grid_y + y) * a.grid_z + z0);
                cell[u][0] = v.x;
                cell[u][1] = v.y;
                cell[u][2] = v.z;
            } else {
                cell[u][0] = cell[u][1] = cell[u][2] = kVoxelGridEmpty;
            }
        }
        uint32_t local = 0;
#pragma unroll
        for (int u = 0; u < 3; ++u) {
            const int q = part + 4 * u;
            if (q >= 9) break;  // wave-uniform
            int lo = INT_MAX, hi = -1;
#pragma unroll
            for (int dz = 0; dz < 3; ++dz) {
                const int k = 3 * q + dz, z = c.w + dz - 1;
                int32_t src = -1;
                if (col_ok[u] && static_cast<unsigned>(z) < static_cast<unsigned>(a.grid_z)) {
                    const int e = z - z0;  // 0..2, selected without indexing the registers
                    const uint32_t v = e == 0 ? cell[u][0] : (e == 1 ? cell[u][1] : cell[u][2]);
                    src = k == 13 ? static_cast<int32_t>(p) : voxel_grid_row(v, a.grid_gen);
                    if (src >= a.rows_in) src = -1;
                }
                idx[k * BM + row] = src;
                if (src >= 0) {
                    local |= 1u << k;
                    lo = min(lo, src);
                    hi = max(hi, src);
                }
            }
            lo = dpp_row_min(lo);
            hi = dpp_row_max(hi);
            if ((lane & 15) == 15 && hi >= 0) {
                atomicMin(&rlo[q], lo);
                atomicMax(&rhi[q], hi);
            }
        }
        local = dpp_row_or(local);
        if ((lane & 15) == 15 && local) atomicOr(&tile_mask, local);
    } else {
        // Thread: one row, offsets [kb, kb + 7) (kb wave-uniform); all its
        // lookups are issued before any is used.
        const int row = tid % BM, kb = 7 * (tid / BM);
        const int64_t p = p0 + row;
        const bool live = p < a.m;
        int32_t src[7];
        if (a.grid) {
            const int4 c = live ? crd[p] : make_int4(0, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 7; ++i) src[i] = (live && kb + i < 27) ? grid_src(a, c, kb + i, p) : -1;
        } else {
            const uint32_t pm = (live && a.masks) ? a.masks[p] : ~0u;
#pragma unroll
            for (int i = 0; i < 7; ++i) {
                const int k = kb + i;
                int32_t s = -1;
                if (live && k < 27 && ((pm >> k) & 1u)) {
                    s = a.rowmap[k * a.ld_map + p];
                    if (s < 0 || s >= a.rows_in) s = -1;
                }
                src[i] = s;
            }
        }
        uint32_t local = 0;
        int lo = INT_MAX, hi = -1;
#pragma unroll
        for (int i = 0; i < 7; ++i) {
            const int k = kb + i;
            if (k >= 27) break;  // wave-uniform
            idx[k * BM + row] = src[i];
            if (src[i] >= 0) {
                local |= 1u << k;
                lo = min(lo, src[i]);
                hi = max(hi, src[i]);
            }
            if (k % 3 == 2 || i == 6) {  // the end of a kh row or of this thread's offsets
                lo = dpp_row_min(lo);
                hi = dpp_row_max(hi);
                if ((lane & 15) == 15 && hi >= 0) {
                    atomicMin(&rlo[k / 3], lo);
                    atomicMax(&rhi[k / 3], hi);
                }
                lo = INT_MAX;
                hi = -1;
            }
        }
        local = dpp_row_or(local);
        if ((lane & 15) == 15 && local) atomicOr(&tile_mask, local);
    }
    __syncthreads();
    // ---- the groups and the stage sequence (wave 0, every lane the same
    // scalar decisions) ----
    if (wave == 0) {
        const uint32_t present = tile_mask;
        int ng = 0;
        auto add = [&](int lo, int rows, uint32_t mask) {
            if (lane == 0) {
                g_lo[ng] = lo;
                g_rows[ng] = rows;
                g_mask[ng] = mask;
            }
            if (lane < 27 && ((mask >> lane) & 1u)) g_of[lane] = ng;
            ++ng;
        };
        const int rows_here = static_cast<int>(min<int64_t>(BM, a.m - p0));
        for (int kd = 0; kd < 3; ++kd) {
            const uint32_t pm = present & (0x1FFu << (9 * kd));
            if (!pm) continue;
            const int plo = min(rlo[3 * kd], min(rlo[3 * kd + 1], rlo[3 * kd + 2]));
            const int phi = max(rhi[3 * kd], max(rhi[3 * kd + 1], rhi[3 * kd + 2]));
            if (phi - plo < CAP) {
                add(plo, phi - plo + 1, pm);
                continue;
            }
            for (int kh = 0; kh < 3; ++kh) {
                const int q = 3 * kd + kh;
                const uint32_t hm = present & (0x7u << (3 * q));
                if (!hm) continue;
                if (rhi[q] - rlo[q] < CAP) {
                    add(rlo[q], rhi[q] - rlo[q] + 1, hm);
                    continue;
                }
                for (uint32_t m = hm; m; m &= m - 1) add(-1 - (__ffs(m) - 1), rows_here, 1u << (__ffs(m) - 1));
            }
        }
        // every lane k < 27 writes its offset's entry (g_of is this wave's own writes)
        if (lane < 27 && ((present >> lane) & 1u)) {
            const uint32_t below = present & ((1u << lane) - 1u);
            const uint32_t above = present & ~((2u << lane) - 1u);
            const int g = g_of[lane];
            const bool first = below == 0 || g_of[31 - __clz(below)] != g;
            const bool last = above == 0 || g_of[__ffs(above) - 1] != g;
            ent[__popc(below)] = make_uint2(static_cast<uint32_t>(lane * BM) | (static_cast<uint32_t>(g) << 12) |
                                                (first ? 1u << 17 : 0u) | (last ? 1u << 18 : 0u),
                                            static_cast<uint32_t>(lane) * static_cast<uint32_t>(a.cout) *
                                                static_cast<uint32_t>(a.cin) * 2u);
        }
        if (lane == 0) n_pos = __popc(present);
    }
    __syncthreads();

    const int kcount = __builtin_amdgcn_readfirstlane(n_pos);  // stages per chunk
    const int total = (a.cin / 64) * kcount;

    // Weight stage (k, c): rows n0 .. n0 + BN - 1 of W_k (rows past cout
    // repeat the last row: their products land in columns never stored),
    // bytes 128 c .. 128 c + 127 of each; a scalar base and fixed lane offsets.
    const char * wbase = static_cast<const char *>(a.w);
    uint32_t b_voff[BI];
#pragma unroll
    for (int j = 0; j < BI; ++j) {
        const int row = (wave * BI + j) * 8 + lrow;
        b_voff[j] = static_cast<uint32_t>(min(n0 + row, a.cout - 1)) * static_cast<uint32_t>(a.cin) * 2u +
                    static_cast<uint32_t>((lslot ^ swz(row)) << 4);
    }
    auto issue_w = [&](uint32_t wk, int c, int ring) __attribute__((always_inline)) {
        const char * sb = uniform_ptr(wbase + (wk + static_cast<uint32_t>(c) * 128u));
        char * dst = wring + ring * kWBytes;
#pragma unroll
        for (int j = 0; j < BI; ++j) lds_dma16_sbase(sb, b_voff[j], lds_offset(dst + (wave * BI + j) * 8 * kChunkBytes));
    };
    // The halo of group g, chunk c.  Halo row hr holds input row lo + hr, or
    // for a gathered offset k tile row hr's source; rows no slot refers to
    // (past the range, absent sources) load row lo or row 0.
    auto issue_h = [&](int g, int c) __attribute__((always_inline)) {
        const int lo = g_lo[g], rows = g_rows[g];
        if (lo >= 0) {
            const char * sb = uniform_ptr(reinterpret_cast<const char *>(x + static_cast<int64_t>(lo) * a.ldx + c * 64));
            const uint32_t pitch = static_cast<uint32_t>(a.ldx) * 2u;
            for (int q = wave; q * 8 < rows; q += NW) {
                const int hr = min(q * 8 + lrow, rows - 1);
                lds_dma16_sbase(sb, static_cast<uint32_t>(hr) * pitch + static_cast<uint32_t>((lslot ^ swz(q * 8 + lrow)) << 4),
                                lds_offset(halo + q * 8 * kChunkBytes));
            }
        } else {
            const int k = -1 - lo;
            for (int q = wave; q * 8 < rows; q += NW) {
                const int hr = q * 8 + lrow;
                int64_t src = -1;
                if (hr < rows) {
                    const int64_t p = p0 + hr;
                    src = a.grid ? grid_src(a, crd[p], k, p)
                                 : ((!a.masks || ((a.masks[p] >> k) & 1u)) ? a.rowmap[k * a.ld_map + p] : -1);
                    if (src >= a.rows_in) src = -1;
                }
                lds_dma16(x + (src > 0 ? src : int64_t{0}) * a.ldx + c * 64 + (lslot ^ swz(hr)) * 8,
                          lds_offset(halo + q * 8 * kChunkBytes));
            }
        }
    };

    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // Stage s is position i0 of chunk c0; info0, info1 describe stages s and
    // s + 1; (i2, c2) is the position of the next stage to issue (s + L), into
    // ring slot r2, its table entry e2 read one stage ahead.
    int i0 = 0, c0 = 0, i2 = 0, c2 = 0, r2 = L;
    uint32_t info0 = 0, info1 = 0;
    uint2 e2 = make_uint2(0, 0);
    const uint32_t pmask = static_cast<uint32_t>((4 * h + kg * 2) << 4);  // this lane's first piece
    uint32_t slot_nx[TI];
    auto adv = [&](int & i, int & c) __attribute__((always_inline)) {
        if (++i == kcount) {
            i = 0;
            ++c;
        }
    };
    auto rd = [&](int i) __attribute__((always_inline)) {
        const uint2 v = ent[i];
        return make_uint2(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y));
    };
    if (total > 0) {
        const uint2 e0 = rd(0);
        info0 = e0.x;
        issue_h((info0 >> 12) & 31, 0);
        issue_w(e0.y, 0, 0);
        adv(i2, c2);
        if (total > 1) {
            const uint2 e1 = rd(i2);
            info1 = e1.x;
            if constexpr (L == 2) {
                issue_w(e1.y, c2, 1);
                adv(i2, c2);
            }
        }
        if (total > L) e2 = ent[i2];
    }
    for (int e = tid; e < 27 * BM; e += NT) {
        const int k = e / BM, row = e % BM;  // k wave-uniform
        if (!((tile_mask >> k) & 1u)) continue;
        const int32_t src = idx[e];
        const int lo = g_lo[g_of[k]];
        const int sl = src < 0 ? CAP : (lo < 0 ? row : src - lo);
        slots[e] = static_cast<uint16_t>(sl * kChunkBytes + (swz(sl) << 4));
    }
    barrier_no_fence();  // the slot table is complete (no fence: the first DMAs stay in flight)
    if (total > 0) {
#pragma unroll
        for (int i = 0; i < TI; ++i) slot_nx[i] = slots[(info0 & 4095) + wm * WM + i * 32 + r];
        if (L == 2 && total > 1) wait_vmcnt(BI);
        else wait_vmcnt(0);
        barrier_no_fence();
    }
    bool wait_all = false;  // stage s starts a halo issued in stage s - 1
    for (int s = 0; s < total; ++s) {
        if (s > 0) {
            // this stage's weights (and halo) are in; with L = 2 the next
            // stage's weights may still be in flight
            if (L == 1 || wait_all || s + 1 >= total) wait_vmcnt(0);
            else wait_vmcnt(BI);
            barrier_no_fence();
        }
        uint32_t slot[TI];
#pragma unroll
        for (int i = 0; i < TI; ++i) slot[i] = slot_nx[i];
        if (s + 1 < total) {
#pragma unroll
            for (int i = 0; i < TI; ++i) slot_nx[i] = slots[(info1 & 4095) + wm * WM + i * 32 + r];
        }
        uint32_t info2 = 0;  // stage s + 2
        if (s + L < total) {
            // stage s + L into the ring slot stage s - 1 used
            const uint32_t ex = __builtin_amdgcn_readfirstlane(e2.x);
            issue_w(__builtin_amdgcn_readfirstlane(e2.y), c2, r2);
            adv(i2, c2);
            r2 = r2 == WS - 1 ? 0 : r2 + 1;
            if (s + L + 1 < total) e2 = ent[i2];
            if constexpr (L == 2) info2 = ex;
            else if (s + 2 < total) info2 = __builtin_amdgcn_readfirstlane(e2.x);
        }
        bf16x8 af[2][TI];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int i = 0; i < TI; ++i)
                af[kk][i] = *reinterpret_cast<const bf16x8 *>(halo + (slot[i] ^ pmask ^ (kk << 4)));
        const bool last = ((info0 >> 18) & 1) && s + 1 < total;  // the halo is refilled in this stage
        if (last) {
            barrier_no_fence();  // every wave holds its operands from the halo
            issue_h((info1 >> 12) & 31, i0 + 1 == kcount ? c0 + 1 : c0);
        }
        wait_all = last;
        const char * wb = wring + (s % WS) * kWBytes;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int piece = 4 * h + kg * 2 + kk;
            bf16x8 bfr[TJ];
#pragma unroll
            for (int jn = 0; jn < TJ; ++jn) {
                const int row = wn * WN + jn * 32 + r;
                bfr[jn] = *reinterpret_cast<const bf16x8 *>(wb + row * kChunkBytes + ((piece ^ swz(row)) << 4));
            }
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int jn = 0; jn < TJ; ++jn)
                    acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[kk][i], bfr[jn], acc[i][jn], 0, 0, 0);
        }
        info0 = info1;
        info1 = info2;
        adv(i0, c0);
    }

    // Group 0 finishes the upper 32-row block of each wave's 64 rows, group 1
    // the lower one; each hands the other half of its partial sums over
    // through the (now idle) buffers, then the tile is staged in LDS as bf16
    // and written as whole 16-byte row pieces.  (The kept block is a
    // compile-time index in each branch: a run-time index into acc would put
    // the accumulators in scratch memory.)
    float * xch = reinterpret_cast<float *>(smem);
    auto xslot = [&](int group, int jn, int v) { return (((group * NWG + wl) * TJP + jn) * 16 + v) * 64 + lane; };
    auto finish = [&](auto keep_tag) __attribute__((always_inline)) {
        constexpr int KEEP = decltype(keep_tag)::value, GIVE = 1 - KEEP;
        f32x16 fin[TJ];
#pragma unroll
        for (int pass = 0; pass < XP; ++pass) {
#pragma unroll
            for (int jn = 0; jn < TJP; ++jn)
#pragma unroll
                for (int v = 0; v < 16; ++v) xch[xslot(KEEP, jn, v)] = acc[GIVE][pass * TJP + jn][v];
            barrier_no_fence();
#pragma unroll
            for (int jn = 0; jn < TJP; ++jn)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    fin[pass * TJP + jn][v] = acc[KEEP][pass * TJP + jn][v] + xch[xslot(GIVE, jn, v)];
            barrier_no_fence();  // the exchange is read: the area may take the next pass or the staged tile
        }
#pragma unroll
        for (int jn = 0; jn < TJ; ++jn) {
            const int cl = wn * WN + jn * 32 + r;
            const float b = (a.bias && n0 + cl < a.cout) ? a.bias[n0 + cl] : 0.0f;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int rl = KEEP * 32 + wm * WM + 8 * (v >> 2) + 4 * h + (v & 3);
                float val = fin[jn][v] + b;
                if (a.act == PXS_ACT_GELU_TANH) val = gelu_tanh_f(val);
                else if (a.act == PXS_ACT_SILU) val = silu_f(val);
                *reinterpret_cast<uint16_t *>(smem + rl * kStagePitch + cl * 2) = f32_to_bf16(val);
            }
        }
    };
    barrier_no_fence();
    if (kg == 0) finish(std::integral_constant<int, 0>{});
    else finish(std::integral_constant<int, 1>{});
    barrier_no_fence();
    uint16_t * y = static_cast<uint16_t *>(a.y);
    for (int q = tid; q < BM * (BN / 8); q += NT) {
        const int rl = q / (BN / 8), piece = q % (BN / 8);
        const int64_t row = p0 + rl;
        const int col = n0 + piece * 8;
        if (row < a.m && col < a.cout)
            *reinterpret_cast<uint4 *>(y + row * a.ldy + col) =
                *reinterpret_cast<const uint4 *>(smem + rl * kStagePitch + piece * 16);
    }
}

template <int BN, int CAP, int WS>
int launch_range_conv(const GemmArgs & args, hipStream_t stream) {
    constexpr int smem = range_lds_bytes<BN, CAP, WS>();
    static bool configured = false;
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&range_conv_bf16_kernel<BN, CAP, WS>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, smem);
        if (e != hipSuccess) return check_hip(e, "hipFuncSetAttribute(range_conv)");
        configured = true;
    }
    const int64_t tiles = ((args.m + kRangeBM - 1) / kRangeBM) * ((args.cout + BN - 1) / BN);
    const int64_t blocks = tiles + args.side_blocks;
    if (blocks > INT32_MAX) return fail(PXS_ERR_ARG, "range conv grid too large");
    if (args.side_blocks > 0 && smem < s2_emit_lds_bytes(args.s2.words_per_block, kRangeNW * 64))
        return fail(PXS_ERR_ARG, "range conv: side work needs more LDS than the tile");
    hipLaunchKernelGGL((range_conv_bf16_kernel<BN, CAP, WS>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kRangeNW * 64), smem, stream, args);
    return check_launch("SubMConv3d (neighbourhood ranges)");
}

// ---------------------------------------------------------------------------
// fp32 split-K gather GEMM (SubMConv3d and linears in fp32).  A workgroup
// owns 32*TI output rows x 64 output channels; its (offset, 32-channel chunk)
// steps are dealt round-robin to the 4 waves, so even a few hundred tiles
// keep every CU busy.  Each wave loads its operands straight into VGPRs --
// lane (h, r) takes the 64 contiguous bytes k = 16h .. 16h+15 of A row r (of
// each 32-row block) and of weight row r, the same K permutation on both
// sides of v_mfma_f32_32x32x2_f32 -- with the next step's loads in flight
// during the current step's MFMAs, and no barrier until the end, where waves
// 1-3 hand their partial sums to wave 0 through LDS (a fixed summation order:
// deterministic).  The operand loads return through the per-CU vector-memory
// path, which bounds the kernel: TI = 2 reads each weight chunk once for 64
// rows instead of 32 (16 KB per 64x64x32 step instead of 24 KB), at 64
// accumulator registers per lane.

template <int EPI, int TI>
__global__ void __launch_bounds__(256)
split_gemm_f32_kernel(GemmArgs a) {
    constexpr int BM = 32 * TI, BN = 64, NW = 4;
    __shared__ float red[NW - 1][TI * 2][16][64];
    __shared__ int32_t idx_lds[32 * BM];
    __shared__ uint32_t tile_mask;
    __shared__ int koff[32];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, r = lane & 31;

    const int tiles_n = (a.cout + BN - 1) / BN;
    const int logical = remap_xcd(blockIdx.x, gridDim.x);
    const int64_t p0 = static_cast<int64_t>(logical / tiles_n) * BM;
    const int n0 = (logical % tiles_n) * BN;
    const float * __restrict__ x = static_cast<const float *>(a.x);
    const float * __restrict__ w = static_cast<const float *>(a.w);

    if (tid == 0) tile_mask = 0;
    __syncthreads();
    if (a.grid) {
        grid_tile_sources<BM>(a, p0, tid, NW * 64, idx_lds, &tile_mask);
    } else if (tid < BM && p0 + tid < a.m) {
        const int64_t p = p0 + tid;
        uint32_t local = 0;
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
        if (local) atomicOr(&tile_mask, local);
    }
    __syncthreads();
    const uint32_t present = tile_mask & (a.noff >= 32 ? ~0u : ((1u << a.noff) - 1u));
    const int kcount = __popc(present);
    if (tid == 0) {
        uint32_t m = present;
        for (int i = 0; i < kcount; ++i) {
            koff[i] = __ffs(m) - 1;
            m &= m - 1;
        }
    }
    __syncthreads();
    for (int e = tid; !a.grid && e < kcount * BM; e += NW * 64) {
        const int i = e / BM, row = e % BM;
        int32_t src = -1;
        if (p0 + row < a.m) {
            const int64_t p = p0 + row;
            const int64_t s = a.rowmap ? static_cast<int64_t>(a.rowmap[koff[i] * a.ld_map + p]) : p;
            src = (s >= 0 && s < a.rows_in) ? static_cast<int32_t>(s) : -1;
        }
        idx_lds[e] = src;
    }
    __syncthreads();

    const int chunks = (a.cin + 31) / 32;
    const int steps = kcount * chunks;
    const int my_steps = steps > wave ? (steps - wave + NW - 1) / NW : 0;
    const float4 * zero4 = reinterpret_cast<const float4 *>(g_zero_chunk);

    // Operands of one step: A (16 floats of row r of each 32-row block) and B
    // (16 floats of each of the two 32-column weight tiles).  Steps past the
    // end load zeros, so every iteration issues the same loads and the
    // compiler's waits count exactly one step in flight.
    struct Ops {
        float4 av[TI][4];
        float4 bv[2][4];
    };
    auto load = [&](int t, Ops & o) __attribute__((always_inline)) {
        const int s = wave + t * NW;
        const bool live = t < my_steps;
        const int i = live ? s / chunks : 0, chunk = live ? s - i * chunks : 0;
        const int k = live ? koff[i] : 0;
        const int col0 = chunk * 32 + 16 * h;
#pragma unroll
        for (int ti = 0; ti < TI; ++ti) {
            const int32_t src = live ? idx_lds[(a.grid ? k : i) * BM + ti * 32 + r] : -1;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = col0 + 4 * q;
                o.av[ti][q] = (src >= 0 && col < a.cin)
                                  ? *reinterpret_cast<const float4 *>(x + static_cast<int64_t>(src) * a.ldx + col)
                                  : *zero4;
            }
        }
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int c = n0 + ct * 32 + r;
            const bool ok = live && c < a.cout;
            const float * wrow = w + (static_cast<int64_t>(k) * a.cout + c) * a.cin;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int col = col0 + 4 * q;
                o.bv[ct][q] = (ok && col < a.cin) ? *reinterpret_cast<const float4 *>(wrow + col) : *zero4;
            }
        }
    };

    f32x16 acc[TI][2];
#pragma unroll
    for (int ti = 0; ti < TI; ++ti)
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[ti][ct][v] = 0.0f;
    auto compute = [&](const Ops & o) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ti = 0; ti < TI; ++ti)
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
                        acc[ti][ct] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            o.av[ti][q][e], o.bv[ct][q][e], acc[ti][ct], 0, 0, 0);
    };

    Ops o0, o1;
    load(0, o0);
    for (int t = 0; t < my_steps; t += 2) {
        load(t + 1, o1);
        compute(o0);
        load(t + 2, o0);
        if (t + 1 < my_steps) compute(o1);
    }

    if (wave > 0) {
#pragma unroll
        for (int ti = 0; ti < TI; ++ti)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int v = 0; v < 16; ++v) red[wave - 1][ti * 2 + ct][v][lane] = acc[ti][ct][v];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int wv = 0; wv < NW - 1; ++wv)
#pragma unroll
        for (int ti = 0; ti < TI; ++ti)
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[ti][ct][v] += red[wv][ti * 2 + ct][v][lane];
    gemm_epilogue<float, TI, 2, 32 * TI, 64, EPI>(a, acc, p0, n0, 0, 0, h, r);
}

#ifndef PXS_SPLIT_F32
#define PXS_SPLIT_F32 1
#endif
// 64-row tiles (one workgroup, one wave per SIMD, per CU) for grids of
// about one to four rounds over the 256 CUs; past that, 32-row tiles at two
// workgroups per CU hide more latency.  Measured on SubMConv3d over shell
// voxels: 64 -> 64 at 16k rows 57 against 67 us, 128 -> 128 at 8k-32k rows
// 0.79-0.89x; at 8k rows 64 -> 64 (128 wide tiles) 1.66x slower, at 96k rows
// 1.03-1.12x slower.
#ifndef PXS_SPLIT_F32_WIDE_MIN
#define PXS_SPLIT_F32_WIDE_MIN 224
#endif
#ifndef PXS_SPLIT_F32_WIDE_MAX
#define PXS_SPLIT_F32_WIDE_MAX 1024
#endif

template <int EPI, int TI>
int launch_split_f32_ti(const GemmArgs & args, hipStream_t stream) {
    const int64_t tiles_m = (args.m + 32 * TI - 1) / (32 * TI);
    const int64_t tiles_n = (args.cout + 63) / 64;
    const int64_t blocks = tiles_m * tiles_n;
    if (blocks > INT32_MAX) return fail(PXS_ERR_ARG, "gather GEMM grid too large");
    hipLaunchKernelGGL((split_gemm_f32_kernel<EPI, TI>), dim3(static_cast<unsigned>(blocks)),
                       dim3(256), 0, stream, args);
    return check_launch("gather GEMM (fp32 split-K)");
}

template <int EPI>
int launch_split_f32(const GemmArgs & args, hipStream_t stream) {
    const int64_t wide = ((args.m + 63) / 64) * ((args.cout + 63) / 64);
    // (Only for the 27-offset gathers: plain linears, with 2 K steps per
    // tile, run 1.5x slower on 64-row tiles, 19 against 13 us at 16k x 64.)
    if ((args.rowmap || args.grid) && args.noff >= 27 && wide >= PXS_SPLIT_F32_WIDE_MIN &&
        wide <= PXS_SPLIT_F32_WIDE_MAX)
        return launch_split_f32_ti<EPI, 2>(args, stream);
    return launch_split_f32_ti<EPI, 1>(args, stream);
}

template <typename T, int BM, int BN, int EPI, int NSTAGE, int NW, int WAVES_M, int KSPLIT>
int launch_lds_tile(const GemmArgs & args, hipStream_t stream) {
    const int smem = lds_gemm_bytes<BM, BN, NSTAGE>(args.noff);
    static int configured = 0;
    if (configured < smem) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void *>(&gather_gemm_lds_kernel<T, BM, BN, EPI, NSTAGE, NW, WAVES_M, KSPLIT>),
            hipFuncAttributeMaxDynamicSharedMemorySize, lds_gemm_bytes<BM, BN, NSTAGE>(27));
        if (e != hipSuccess) return check_hip(e, "hipFuncSetAttribute(gather_gemm_lds)");
        configured = lds_gemm_bytes<BM, BN, NSTAGE>(27);
    }
    const int64_t tiles_m = (args.m + BM - 1) / BM;
    const int64_t tiles_n = (args.cout + BN - 1) / BN;
    const int64_t blocks = tiles_m * tiles_n + args.side_blocks;
    if (blocks > INT32_MAX) return fail(PXS_ERR_ARG, "gather GEMM grid too large");
    if (args.side_blocks > 0 &&
        smem < s2_emit_lds_bytes(args.s2.words_per_block, NW * 64))
        return fail(PXS_ERR_ARG, "gather GEMM: side work needs more LDS than the tile");
    hipLaunchKernelGGL((gather_gemm_lds_kernel<T, BM, BN, EPI, NSTAGE, NW, WAVES_M, KSPLIT>),
                       dim3(static_cast<unsigned>(blocks)), dim3(NW * 64), smem, stream, args);
    return check_launch("gather GEMM (LDS pipeline)");
}

// The chained level runs the default bf16 tile of both convolutions
// (128 x 128, 2 stages, 8 waves in two K groups), the one dispatch picks for
// them.
int launch_unet_chain(const GemmArgs & a, const GemmArgs & b, ChainArgs c, hipStream_t stream) {
    constexpr int BM = 128, BN = 128, NSTAGE = 2, NW = 8, WAVES_M = 2, KSPLIT = 2;
    const int smem = lds_gemm_bytes<BM, BN, NSTAGE>(27);
    static bool configured = false;
    if (!configured) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void *>(
                &gather_gemm_lds_chain_kernel<uint16_t, BM, BN, NSTAGE, NW, WAVES_M, KSPLIT>),
            hipFuncAttributeMaxDynamicSharedMemorySize, smem);
        if (e != hipSuccess) return check_hip(e, "hipFuncSetAttribute(gather_gemm_lds_chain)");
        configured = true;
    }
    c.tiles_a = static_cast<int>((a.m + BM - 1) / BM) * ((a.cout + BN - 1) / BN);
    c.tiles_n_a = (a.cout + BN - 1) / BN;
    c.tiles_b = static_cast<int>((b.m + BM - 1) / BM) * ((b.cout + BN - 1) / BN);
    c.side = a.s2.blocks;
    while ((c.tiles_a + c.side) % 8 != 0) ++c.side;
    const int64_t blocks = static_cast<int64_t>(c.tiles_a) + c.side + c.tiles_b;
    if (blocks > INT32_MAX) return fail(PXS_ERR_ARG, "chained level: grid too large");
    if (smem < s2_emit_lds_bytes(a.s2.words_per_block, NW * 64))
        return fail(PXS_ERR_ARG, "chained level: side work needs more LDS than the tile");
    hipLaunchKernelGGL((gather_gemm_lds_chain_kernel<uint16_t, BM, BN, NSTAGE, NW, WAVES_M, KSPLIT>),
                       dim3(static_cast<unsigned>(blocks)), dim3(NW * 64), smem, stream, a, b, c);
    return check_launch("chained U-Net level");
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
    if (args.noff > 32) return fail(PXS_ERR_ARG, "gather GEMM supports at most 32 offsets");
    const bool narrow = args.cout <= 64;
    if (args.vec_ok) {
        // 128-row tiles: the row count only changes the grid, not the tile.
        constexpr int ksplit = sizeof(T) == 2 ? PXS_GEMM_KSPLIT : 1;
        constexpr int waves_m = ksplit == 2 ? 2 : PXS_GEMM_WAVES_M;
        if constexpr (sizeof(T) == 2) {
            // Long gathers wider than 128 channels: one 256-channel tile
            // gathers each row chunk once instead of once per 128-channel
            // tile (one workgroup per CU; SubMConv3d 256->256 at 64^3 -6%).
            // Short ones (the 8-offset stride-2 conv, 16 K stages) lose 6%:
            // with one workgroup per CU nothing hides a tile's prologue.
            const int64_t kstages = static_cast<int64_t>(args.noff) * ((args.cin + 63) / 64);
            // (192-row tiles, which put SubMConv3d 256->256 on ~40k rows in
            // one round of tiles instead of 1.2, measured the same: the
            // chip-wide operand rate bounds it, not the last round.)
            // Long gathers of at least 512 output channels, with two or more
            // rounds of 256x256 tiles: each stage's 64 KB feed 2x the MACs
            // of a 128x256 stage's 48 KB (one workgroup per CU either way;
            // 155.6 KB of LDS with the 27-offset source table).  The C2S
            // up-convolution 768 -> 1536 at 64^3: 1.97 -> 1.61 ms; the SLat
            // decoder 27.3 -> 25.6 ms.  Sixteen waves (4 x 4, a 64x64 block
            // of the tile each, 100 VGPRs) instead of eight (2 x 4, 128x64
            // each) keep more loads in flight per CU and take half the
            // epilogue per wave: the up-convolution 1.62 -> 1.56 ms, the
            // decoder 25.1 -> 24.8 ms.
#ifndef PXS_GEMM_SQUARE256
#define PXS_GEMM_SQUARE256 1
#endif
#ifndef PXS_GEMM_SQUARE256_TILES
#define PXS_GEMM_SQUARE256_TILES 512
#endif
            if (PXS_GEMM_SQUARE256 && (args.rowmap || args.grid) && args.cout >= 512 &&
                kstages >= 32 && ((args.m + 255) / 256) * ((args.cout + 255) / 256) >= PXS_GEMM_SQUARE256_TILES)
            {
#ifndef PXS_GEMM_SQUARE256_WAVES
#define PXS_GEMM_SQUARE256_WAVES 16
#endif
                if constexpr (PXS_GEMM_SQUARE256_WAVES == 16)
                    return launch_lds_tile<T, 256, 256, EPI, 2, 16, 4, 1>(args, stream);
                else
                    return launch_lds_tile<T, 256, 256, EPI, 2, 8, 2, 1>(args, stream);
            }
            // (Sixteen waves on the 128x256 tile -- two K groups with 2 or 3
            // stages, or 4 x 4 blocks of 32x64 -- measured the same as eight
            // on the U-Net stage's 256-channel conv; four waves of 128x128 on
            // the 256x256 tile, one per SIMD, ran the up-convolution 26%
            // slower.)
            if (PXS_GEMM_WIDE && (args.rowmap || args.grid) && args.cout > 128 && kstages >= 32)
                return launch_lds_tile<T, 128, 256, EPI, 2, 8, 2, 1>(args, stream);
        }
#ifndef PXS_GEMM_NARROW_KSPLIT
#define PXS_GEMM_NARROW_KSPLIT 2
#endif
        constexpr int narrow_ks = sizeof(T) == 2 ? PXS_GEMM_NARROW_KSPLIT : 1;
        return narrow ? launch_lds_tile<T, 128, 64, EPI, PXS_GEMM_STAGES, 4 * narrow_ks, 2, narrow_ks>(args, stream)
                      : launch_lds_tile<T, PXS_GEMM_BM, PXS_GEMM_BN, EPI, PXS_GEMM_STAGES,
                                        PXS_GEMM_WAVES, waves_m, ksplit>(args, stream);
    }
    const int64_t tiles_n = (args.cout + (narrow ? 63 : 127)) / (narrow ? 64 : 128);
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
    if (dtype == PXS_F32 && args.vec_ok && PXS_SPLIT_F32 && args.m > 0 && args.cout > 0 &&
        args.noff <= 32 && (args.ldx % 4 == 0)) {
        if (epi == kEpiStore) return launch_split_f32<kEpiStore>(args, stream);
        if (epi == kEpiAddResidual) return launch_split_f32<kEpiAddResidual>(args, stream);
        return launch_split_f32<kEpiGateResidual>(args, stream);
    }
    if (dtype == PXS_BF16) {
        // SubMConv3d over a voxel grid: neighbourhood ranges, 128-column
        // tiles with a 320-row halo and a 2-slot weight ring (80.8 KB, two
        // workgroups per CU).  Measured on one box against the forms before
        // it: the U-Net's conv A (128 -> 128 at 128^3) 0.1629-0.1640 ms
        // against 0.1709-0.1714 ms with a 256-row halo and 0.1745 ms with a
        // 192-row halo and a 3-slot ring (planes wider than the halo fall
        // back to kh rows or single offsets, whose refills the tile then
        // waits for); its conv C (256 -> 256 at 64^3) 0.1136-0.1139 ms
        // against 0.1172-0.1175 ms on one 256-column tile per CU (256-row
        // halo, 3 slots) and 0.128-0.129 ms on 128 x 256 gather tiles.  (Over a neighbour map,
        // the SLat decoder's 128-channel levels at up to 1024^3 ran 3.7%
        // slower on ranges.)
        if (PXS_GEMM_RANGE && epi == kEpiStore && args.noff == 27 && args.grid && args.vec_ok &&
            args.cin % 64 == 0 && args.m > 0 && args.cout > 64 && args.cout <= PXS_GEMM_RANGE_MAXN &&
            args.cout % 8 == 0 && args.ldy % 8 == 0 && aligned16(args.y))
            return launch_range_conv<128, kRangeCap, kRangeWS>(args, stream);
        if (epi == kEpiStore) return dispatch<uint16_t, kEpiStore>(args, stream);
        if (epi == kEpiAddResidual) return dispatch<uint16_t, kEpiAddResidual>(args, stream);
        return dispatch<uint16_t, kEpiGateResidual>(args, stream);
    }
    if (epi == kEpiStore) return dispatch<float, kEpiStore>(args, stream);
    if (epi == kEpiAddResidual) return dispatch<float, kEpiAddResidual>(args, stream);
    return dispatch<float, kEpiGateResidual>(args, stream);
}

// Mean of each group's rows, summed in the group's (ascending) row order, the
// order src/sparse.cpp:566-572 accumulates them; then one division
// (src/sparse.cpp:594-597).
template <typename T>
__global__ void downsample_mean_kernel(const T * __restrict__ x, int channels,
                                       const int64_t * __restrict__ offsets,
                                       const int32_t * __restrict__ rows, int64_t m,
                                       T * __restrict__ y) {
    const int64_t q = blockIdx.x;
    if (q >= m) return;
    const int64_t begin = offsets[q], end = offsets[q + 1];
    for (int ch = threadIdx.x; ch < channels; ch += blockDim.x) {
        float s = 0.0f;
        for (int64_t i = begin; i < end; ++i) {
            s += load_f32(x + static_cast<int64_t>(rows[i]) * channels + ch);
        }
        store_f32(y + q * channels + ch, s / static_cast<float>(end - begin));
    }
}

// fp32 linear in sparse_linear's own operation order (src/sparse.cpp:436-446):
// value = bias[o], then value += w[o][i] * x[i] for i ascending, every product
// and sum rounded alone.  One thread per (row, output); the x row is read in
// 16-byte pieces.  For a handful of outputs whose signs decide a topology
// (the subdivision logits), where the MFMA linear's different summation
// order could flip a logit within rounding of zero.
__global__ void ordered_linear_kernel(const float * __restrict__ x, int64_t rows, int cin,
                                      const float * __restrict__ weight,
                                      const float * __restrict__ bias, int cout,
                                      float * __restrict__ y) {
#pragma clang fp contract(off)
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= rows * cout) return;
    const int64_t row = t / cout;
    const int o = static_cast<int>(t - row * cout);
    const float * xr = x + row * cin;
    const float * wr = weight + static_cast<int64_t>(o) * cin;
    float value = bias ? bias[o] : 0.0f;
    int i = 0;
    if ((cin & 3) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(weight) & 15) == 0) {
        for (; i < cin; i += 4) {
            const float4 xv = *reinterpret_cast<const float4 *>(xr + i);
            const float4 wv = *reinterpret_cast<const float4 *>(wr + i);
            value += wv.x * xv.x;
            value += wv.y * xv.y;
            value += wv.z * xv.z;
            value += wv.w * xv.w;
        }
    }
    for (; i < cin; ++i) value += wr[i] * xr[i];
    y[t] = value;
}

// The same order with one thread per row for up to 8 outputs: the row is
// read once and each output keeps its own running sum (interleaving the
// outputs does not change any one sum's order).  Weights come from LDS.
constexpr int kOrderedRowOut = 8;
constexpr int kOrderedRowCin = 2048;
constexpr int kOrderedRows = 256;                  // rows per workgroup, one per thread
constexpr int kOrderedChunk = 32;                  // input channels staged per pass
constexpr int kOrderedPitch = kOrderedChunk + 1;   // odd pitch: lane l reads bank (l + j) % 32

// Rows pass through LDS 32 channels at a time, loaded by the whole workgroup
// with coalesced (16-byte where possible) reads, so each thread walks its own
// row from LDS instead of striding 4 x cin bytes between lanes in global
// memory.  The weights are read at wave-uniform addresses (scalar loads into
// SGPRs, 8 inputs at a time), so the multiply-adds take them as operands.
template <int COUT>
__global__ void __launch_bounds__(kOrderedRows)
ordered_linear_rows_kernel(const float * __restrict__ x, int64_t rows, int cin,
                           const float * __restrict__ weight, const float * __restrict__ bias,
                           bool vec4, float * __restrict__ y) {
#pragma clang fp contract(off)
    __shared__ float x_lds[kOrderedRows * kOrderedPitch];
    const int t = threadIdx.x;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kOrderedRows;
    const int nrows = static_cast<int>(rows - row0 < kOrderedRows ? rows - row0 : kOrderedRows);
    float acc[COUT];
#pragma unroll
    for (int o = 0; o < COUT; ++o) acc[o] = bias ? bias[o] : 0.0f;
    for (int k0 = 0; k0 < cin; k0 += kOrderedChunk) {
        const int kw = cin - k0 < kOrderedChunk ? cin - k0 : kOrderedChunk;
        __syncthreads();  // the previous chunk is consumed
        if (vec4) {
            for (int e = t; e < kOrderedRows * (kOrderedChunk / 4); e += kOrderedRows) {
                const int r = e / (kOrderedChunk / 4), c = (e % (kOrderedChunk / 4)) * 4;
                float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (r < nrows && c < kw)
                    v = *reinterpret_cast<const float4 *>(x + (row0 + r) * cin + k0 + c);
                float * d = x_lds + r * kOrderedPitch + c;
                d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
            }
        } else {
            for (int e = t; e < kOrderedRows * kOrderedChunk; e += kOrderedRows) {
                const int r = e / kOrderedChunk, c = e % kOrderedChunk;
                x_lds[r * kOrderedPitch + c] =
                    (r < nrows && c < kw) ? x[(row0 + r) * cin + k0 + c] : 0.0f;
            }
        }
        __syncthreads();
        if (t < nrows) {
            const float * xr = x_lds + t * kOrderedPitch;
            const float * wk = weight + k0;  // row o of this chunk starts at wk + o * cin
            int j = 0;
            for (; j + 8 <= kw; j += 8) {
                float xv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) xv[e] = xr[j + e];
#pragma unroll
                for (int o = 0; o < COUT; ++o) {
                    const float * wo = wk + o * cin + j;
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[o] += wo[e] * xv[e];
                }
            }
            for (; j < kw; ++j) {
                const float xv = xr[j];
#pragma unroll
                for (int o = 0; o < COUT; ++o) acc[o] += wk[o * cin + j] * xv;
            }
        }
    }
    if (t >= nrows) return;
#pragma unroll
    for (int o = 0; o < COUT; ++o) y[(row0 + t) * COUT + o] = acc[o];
}

int launch_ordered_rows(const float * x, int64_t rows, int cin, const float * weight,
                        const float * bias, int cout, float * y, hipStream_t s) {
    const bool vec4 = cin % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const dim3 grid(static_cast<unsigned>((rows + kOrderedRows - 1) / kOrderedRows));
    switch (cout) {
#define PXS_ORDERED_ROWS(N)                                                                       \
    case N:                                                                                    \
        hipLaunchKernelGGL(ordered_linear_rows_kernel<N>, grid, dim3(kOrderedRows), 0, s, x, rows, \
                           cin, weight, bias, vec4, y);                                       \
        break;
        PXS_ORDERED_ROWS(1) PXS_ORDERED_ROWS(2) PXS_ORDERED_ROWS(3) PXS_ORDERED_ROWS(4)
        PXS_ORDERED_ROWS(5) PXS_ORDERED_ROWS(6) PXS_ORDERED_ROWS(7) PXS_ORDERED_ROWS(8)
#undef PXS_ORDERED_ROWS
    default: return fail(PXS_ERR_ARG, "ordered linear (rows): at most 8 outputs");
    }
    return check_launch("ordered linear (rows)");
}

} // namespace

// The plain linears: the dense MFMA kernels (csrc/dense.hip) for operands of
// whole 16-byte pieces, the gather-GEMM kernels (one offset, no row map)
// otherwise.
int linear_rows(int dtype, const void * x, int64_t rows, int cin, const void * weight,
                const float * bias, int cout, int act, void * y, hipStream_t s) {
    if (int rc = check_dtype(dtype, "pxs_linear")) return rc;
    PXS_CHECK(rows >= 0 && cin > 0 && cout > 0, PXS_ERR_ARG, "pxs_linear: bad shape");
    PXS_CHECK(act == PXS_ACT_NONE || act == PXS_ACT_GELU_TANH || act == PXS_ACT_SILU,
              PXS_ERR_ARG, "pxs_linear: bad activation");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x && weight && y, PXS_ERR_ARG, "pxs_linear: null pointer");
    // A few fp32 outputs over narrow rows (the decoder's output layer, 64 -> 7
    // over millions of rows): the reference's own operation order, one thread
    // per row, HBM-bound, instead of MFMA tiles 7/8 empty.
    if (dtype == PXS_F32 && act == PXS_ACT_NONE && cout <= kOrderedRowOut && cin <= 256)
        return launch_ordered_rows(static_cast<const float *>(x), rows, cin,
                                   static_cast<const float *>(weight), bias, cout,
                                   static_cast<float *>(y), s);
    bool done = false;
    if (int rc = dense_linear(dtype, x, rows, cin, weight, bias, cout, act, y, s, &done)) return rc;
    if (done) return PXS_OK;
    GemmArgs a{};
    a.x = x; a.rows_in = rows; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = rows; a.rowmap = nullptr; a.ld_map = 0; a.noff = 1; a.masks = nullptr;
    a.y = y; a.ldy = cout; a.act = act;
    return run_gemm(dtype, a, kEpiStore, s);
}

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

int pxs_subm_conv3d_grid(int dtype, const void * x, const int32_t * coords, int64_t n, int cin,
                         const void * weight, const float * bias, int cout, int batch_size,
                         int sx, int sy, int sz, const void * grid, uint32_t generation, void * y,
                         void * stream) {
    if (int rc = check_dtype(dtype, "pxs_subm_conv3d_grid")) return rc;
    PXS_CHECK(n >= 0 && cin > 0 && cout > 0, PXS_ERR_ARG, "pxs_subm_conv3d_grid: bad shape");
    PXS_CHECK(batch_size > 0 && sx > 0 && sy > 0 && sz > 0, PXS_ERR_ARG,
              "pxs_subm_conv3d_grid: invalid extents");
    PXS_CHECK(generation <= kVoxelTagMax, PXS_ERR_ARG,
              "pxs_subm_conv3d_grid: generation must be 0 (plain grid) or 1..255");
    PXS_CHECK(generation == 0 || n < (int64_t{1} << kVoxelTagShift), PXS_ERR_ARG,
              "pxs_subm_conv3d_grid: a tagged grid holds at most 2^24 - 1 rows");
    PXS_CHECK(n <= INT32_MAX, PXS_ERR_ARG, "pxs_subm_conv3d_grid: bad row count");
    if (n == 0) return PXS_OK;
    PXS_CHECK(x && coords && weight && grid && y, PXS_ERR_ARG,
              "pxs_subm_conv3d_grid: null pointer");
    PXS_CHECK((reinterpret_cast<uintptr_t>(coords) & 15u) == 0, PXS_ERR_ARG,
              "pxs_subm_conv3d_grid: coordinates must be 16-byte aligned");
    PXS_CHECK((reinterpret_cast<uintptr_t>(grid) & 3u) == 0, PXS_ERR_ARG,
              "pxs_subm_conv3d_grid: the grid must be 4-byte aligned");
    GemmArgs a{};
    a.x = x; a.rows_in = n; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = n; a.rowmap = nullptr; a.ld_map = 0; a.noff = 27; a.masks = nullptr;
    a.y = y; a.ldy = cout; a.act = PXS_ACT_NONE; a.coords = coords;
    a.grid = static_cast<const uint32_t *>(grid);
    a.grid_b = batch_size; a.grid_x = sx; a.grid_y = sy; a.grid_z = sz; a.grid_gen = generation;
    return run_gemm(dtype, a, kEpiStore, as_stream(stream));
}

int pxs_subm_conv3d_grid_s2_emit(int dtype, const void * x, const int32_t * coords, int64_t n,
                                 int cin, const void * weight, const float * bias, int cout,
                                 int batch_size, int sx, int sy, int sz, const void * grid,
                                 uint32_t generation, void * y, int32_t * out_coords,
                                 int32_t * child_map, int64_t ld_map, int64_t * m_out,
                                 void * coarse_grid, void * s2_workspace, void * stream) {
    const char * who = "pxs_subm_conv3d_grid_s2_emit";
    if (int rc = check_dtype(dtype, who)) return rc;
    PXS_CHECK(n >= 0 && cin > 0 && cout > 0, PXS_ERR_ARG, std::string(who) + ": bad shape");
    PXS_CHECK(pxs_downsample_s2_tagged_workspace_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              std::string(who) + ": invalid extents");
    PXS_CHECK(generation >= 1 && generation <= kVoxelTagMax, PXS_ERR_ARG,
              std::string(who) + ": generation must be in 1..255");
    PXS_CHECK(n < (int64_t{1} << kVoxelTagShift), PXS_ERR_ARG,
              std::string(who) + ": bad row count (at most 2^24 - 1 rows)");
    PXS_CHECK(ld_map >= n, PXS_ERR_ARG, std::string(who) + ": child map stride below the row count");
    PXS_CHECK_WORKSPACE(s2_workspace, who);
    PXS_CHECK(m_out && s2_workspace, PXS_ERR_ARG, std::string(who) + ": null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) return fill_i64(m_out, 1, 0, s);
    PXS_CHECK(x && coords && weight && grid && y && out_coords && child_map && coarse_grid,
              PXS_ERR_ARG, std::string(who) + ": null pointer");
    PXS_CHECK((reinterpret_cast<uintptr_t>(coords) & 15u) == 0, PXS_ERR_ARG,
              std::string(who) + ": coordinates must be 16-byte aligned");
    PXS_CHECK((reinterpret_cast<uintptr_t>(grid) & 3u) == 0, PXS_ERR_ARG,
              std::string(who) + ": the grid must be 4-byte aligned");
    GemmArgs a{};
    a.x = x; a.rows_in = n; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = n; a.rowmap = nullptr; a.ld_map = 0; a.noff = 27; a.masks = nullptr;
    a.y = y; a.ldy = cout; a.act = PXS_ACT_NONE; a.coords = coords;
    a.grid = static_cast<const uint32_t *>(grid);
    a.grid_b = batch_size; a.grid_x = sx; a.grid_y = sy; a.grid_z = sz; a.grid_gen = generation;
    // The bf16 16-byte path runs on the LDS-pipeline or neighbourhood-range
    // kernel, both of which carry the emit in side workgroups; otherwise the
    // emit follows as its own launch.
    const bool fuse = dtype == PXS_BF16 && cin % 8 == 0 && aligned16(x) && aligned16(weight);
    if (fuse) {
        a.s2 = make_s2_emit_args(batch_size, sx, sy, sz, grid, generation, out_coords, child_map,
                                 ld_map, m_out, coarse_grid, s2_workspace, kS2SideWords);
        a.side_blocks = a.s2.blocks;
        return run_gemm(dtype, a, kEpiStore, s);
    }
    if (int rc = run_gemm(dtype, a, kEpiStore, s)) return rc;
    return pxs_s2_tagged_emit(n, batch_size, sx, sy, sz, grid, generation, out_coords, child_map,
                              ld_map, m_out, coarse_grid, s2_workspace, stream);
}

int pxs_unet_s2_level(int dtype, const void * x, const int32_t * coords, int64_t n, int cin,
                      const void * w_a, const float * b_a, int cout_a, int batch_size, int sx,
                      int sy, int sz, const void * grid, uint32_t generation, void * y_a,
                      const void * w_b, const float * b_b, int cout_b, int64_t m, void * y_b,
                      int32_t * out_coords, int32_t * child_map, int64_t ld_map, int64_t * m_out,
                      void * coarse_grid, void * s2_workspace, void * stream) {
    const char * who = "pxs_unet_s2_level";
    if (int rc = check_dtype(dtype, who)) return rc;
    PXS_CHECK(n >= 0 && cin > 0 && cout_a > 0 && cout_b > 0 && m >= 0 && m <= n, PXS_ERR_ARG,
              std::string(who) + ": bad shape");
    PXS_CHECK(pxs_downsample_s2_tagged_workspace_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              std::string(who) + ": invalid extents");
    PXS_CHECK(generation >= 1 && generation <= kVoxelTagMax, PXS_ERR_ARG,
              std::string(who) + ": generation must be in 1..255");
    PXS_CHECK(n < (int64_t{1} << kVoxelTagShift), PXS_ERR_ARG,
              std::string(who) + ": bad row count (at most 2^24 - 1 rows)");
    PXS_CHECK(ld_map >= n, PXS_ERR_ARG, std::string(who) + ": child map stride below the row count");
    PXS_CHECK_WORKSPACE(s2_workspace, who);
    PXS_CHECK(m_out && s2_workspace, PXS_ERR_ARG, std::string(who) + ": null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) return fill_i64(m_out, 1, 0, s);
    PXS_CHECK(x && coords && w_a && grid && y_a && w_b && y_b && out_coords && child_map &&
                  coarse_grid, PXS_ERR_ARG, std::string(who) + ": null pointer");
    PXS_CHECK((reinterpret_cast<uintptr_t>(coords) & 15u) == 0, PXS_ERR_ARG,
              std::string(who) + ": coordinates must be 16-byte aligned");
    PXS_CHECK((reinterpret_cast<uintptr_t>(grid) & 3u) == 0, PXS_ERR_ARG,
              std::string(who) + ": the grid must be 4-byte aligned");
    // The chain runs both convolutions on the default bf16 tile, the one
    // dispatch picks for a 27-offset gather of 65..128 outputs and an
    // 8-offset gather of 16 K stages over more than 64 outputs.  Inputs of a
    // multiple of 64 channels, whose SubMConv3d runs on neighbourhood ranges,
    // take the two launches instead.
    constexpr bool kDefaultTile = PXS_GEMM_BM == 128 && PXS_GEMM_BN == 128 &&
                                  PXS_GEMM_STAGES == 2 && PXS_GEMM_WAVES == 8 &&
                                  PXS_GEMM_KSPLIT == 2;
    const bool ranged = PXS_GEMM_RANGE && cin % 64 == 0 && cout_a > 64 && cout_a <= PXS_GEMM_RANGE_MAXN;
    const bool chain = kDefaultTile && !ranged && dtype == PXS_BF16 && cin % 8 == 0 && cout_a % 8 == 0 &&
                       cout_a > 64 && cout_a <= 128 && cout_b > 64 && m > 0 && aligned16(x) &&
                       aligned16(w_a) && aligned16(y_a) && aligned16(w_b);
    if (!chain) {
        if (int rc = pxs_subm_conv3d_grid_s2_emit(dtype, x, coords, n, cin, w_a, b_a, cout_a,
                                                  batch_size, sx, sy, sz, grid, generation, y_a,
                                                  out_coords, child_map, ld_map, m_out,
                                                  coarse_grid, s2_workspace, stream))
            return rc;
        return pxs_sparse_conv3d_s2(dtype, y_a, n, cout_a, w_b, b_b, cout_b, child_map, ld_map, m,
                                    y_b, stream);
    }
    GemmArgs a{};
    a.x = x; a.rows_in = n; a.ldx = cin; a.cin = cin; a.w = w_a; a.bias = b_a;
    a.cout = cout_a; a.m = n; a.rowmap = nullptr; a.ld_map = 0; a.noff = 27; a.masks = nullptr;
    a.y = y_a; a.ldy = cout_a; a.act = PXS_ACT_NONE; a.coords = coords; a.vec_ok = 1;
    a.grid = static_cast<const uint32_t *>(grid);
    a.grid_b = batch_size; a.grid_x = sx; a.grid_y = sy; a.grid_z = sz; a.grid_gen = generation;
    a.s2 = make_s2_emit_args(batch_size, sx, sy, sz, grid, generation, out_coords, child_map,
                             ld_map, m_out, coarse_grid, s2_workspace, kS2SideWords);
    a.s2.coherent_children = 1;  // read by the strided conv's tiles of the same launch
    GemmArgs b{};
    b.x = y_a; b.rows_in = n; b.ldx = cout_a; b.cin = cout_a; b.w = w_b; b.bias = b_b;
    b.cout = cout_b; b.m = m; b.rowmap = child_map; b.ld_map = ld_map; b.noff = 8;
    b.masks = nullptr; b.y = y_b; b.ldy = cout_b; b.act = PXS_ACT_NONE; b.vec_ok = 1;
    const S2ChainFlags f = s2_chain_flags(s2_workspace, batch_size, sx, sy, sz);
    ChainArgs c{};
    c.emit_flags = f.emit;
    c.a_flags = f.tiles;
    c.gen = generation;
    c.error = f.error;
    PXS_CHECK((n + 127) / 128 <= f.tiles_cap && a.s2.blocks + 7 <= f.emit_cap, PXS_ERR_ARG,
              std::string(who) + ": flag space exceeded");
    return launch_unet_chain(a, b, c, s);
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
    return linear_rows(dtype, x, rows, cin, weight, bias, cout, act, y, as_stream(stream));
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
    bool done = false;
    if (int rc = dense_linear_gate(dtype, x, rows, cin, weight, bias, cout, coords, block_mod,
                                   time_mod, gate_offset, residual, as_stream(stream), &done))
        return rc;
    if (done) return PXS_OK;
    GemmArgs a{};
    a.x = x; a.rows_in = rows; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = rows; a.noff = 1; a.y = nullptr; a.ldy = cout;
    a.coords = coords; a.block_mod = block_mod; a.time_mod = time_mod;
    a.gate_offset = gate_offset; a.residual = residual;
    return run_gemm(dtype, a, kEpiGateResidual, as_stream(stream));
}

int pxs_linear_residual(int dtype, const void * x, int64_t rows, int cin, const void * weight,
                        const float * bias, int cout, float * residual, void * stream) {
    if (int rc = check_dtype(dtype, "pxs_linear_residual")) return rc;
    PXS_CHECK(rows >= 0 && cin > 0 && cout > 0, PXS_ERR_ARG, "pxs_linear_residual: bad shape");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x && weight && residual, PXS_ERR_ARG, "pxs_linear_residual: null pointer");
    bool done = false;
    if (int rc = dense_linear_residual(dtype, x, rows, cin, weight, bias, cout, residual,
                                       as_stream(stream), &done))
        return rc;
    if (done) return PXS_OK;
    GemmArgs a{};
    a.x = x; a.rows_in = rows; a.ldx = cin; a.cin = cin; a.w = weight; a.bias = bias;
    a.cout = cout; a.m = rows; a.noff = 1; a.y = nullptr; a.ldy = cout; a.residual = residual;
    return run_gemm(dtype, a, kEpiAddResidual, as_stream(stream));
}

int pxs_downsample_mean(int dtype, const void * x, int channels, const int64_t * group_offsets,
                        const int32_t * group_rows, int64_t m, void * y, void * stream) {
    if (int rc = check_dtype(dtype, "pxs_downsample_mean")) return rc;
    PXS_CHECK(channels > 0 && m >= 0 && m <= INT32_MAX, PXS_ERR_ARG,
              "pxs_downsample_mean: bad shape");
    if (m == 0) return PXS_OK;
    PXS_CHECK(x && group_offsets && group_rows && y, PXS_ERR_ARG,
              "pxs_downsample_mean: null pointer");
    const int threads = channels >= 256 ? 256 : 64;
    if (dtype == PXS_F32) {
        hipLaunchKernelGGL(downsample_mean_kernel<float>, dim3(static_cast<unsigned>(m)),
                           dim3(threads), 0, as_stream(stream), static_cast<const float *>(x),
                           channels, group_offsets, group_rows, m, static_cast<float *>(y));
    } else {
        hipLaunchKernelGGL(downsample_mean_kernel<uint16_t>, dim3(static_cast<unsigned>(m)),
                           dim3(threads), 0, as_stream(stream), static_cast<const uint16_t *>(x),
                           channels, group_offsets, group_rows, m, static_cast<uint16_t *>(y));
    }
    return check_launch("pxs_downsample_mean");
}

int pxs_linear_ordered(const float * x, int64_t rows, int cin, const float * weight,
                       const float * bias, int cout, float * y, void * stream) {
    PXS_CHECK(rows >= 0 && cin > 0 && cout > 0, PXS_ERR_ARG, "pxs_linear_ordered: bad shape");
    if (rows == 0) return PXS_OK;
    PXS_CHECK(x && weight && y, PXS_ERR_ARG, "pxs_linear_ordered: null pointer");
    if (cout <= kOrderedRowOut && cin <= kOrderedRowCin)
        return launch_ordered_rows(x, rows, cin, weight, bias, cout, y, as_stream(stream));
    const int64_t count = rows * cout;
    hipLaunchKernelGGL(ordered_linear_kernel, dim3(static_cast<unsigned>((count + 255) / 256)),
                       dim3(256), 0, as_stream(stream), x, rows, cin, weight, bias, cout, y);
    return check_launch("pxs_linear_ordered");
}

} // extern "C"
