// Varlen flash attention on MFMA (sparse self-, cross- and window attention).
//
// Work item = (segment, 32*NW-query tile, head).  NW wavefronts each own 32
// queries and share 64-key K/V tiles staged in LDS.  For every key tile a
// wave computes S^T = K Q^T (keys x queries) so that each lane owns one query
// (lane % 32) and 32 of its 64 scores; the online-softmax statistics are then
// lane-local plus one exchange with the partner lane (lane ^ 32).  The output
// is accumulated transposed, O^T = V^T P^T, so the running rescale is
// lane-local too.  P feeds the second MFMA straight from registers (the
// 32x32 accumulator layout of S^T is the B-operand layout of the next MFMA
// for the key order it implies); V is staged transposed in LDS so the matching
// A-operand fragments are two 8-byte reads.
//
//   bf16: v_mfma_f32_32x32x16_bf16 (8 for S^T + 8 for O^T per wave per tile)
//   fp32: v_mfma_f32_32x32x2_f32   (64 + 64 per wave per tile)
// head_dim and value_dim up to 64 (zero padded to 64 inside the kernel).

#include "pxs_common.h"
#include "scan.h"

#include <cmath>
#include <atomic>
#include <type_traits>

namespace pxs {
namespace {

constexpr int kKeys = 64;  // keys per tile
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ void wait_vmcnt0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// s_waitcnt with only vmcnt bounded (expcnt/lgkmcnt at their maxima); n above
// 15 waits for everything.
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
    case 1: __builtin_amdgcn_s_waitcnt(0x0F71); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F72); break;
    case 3: __builtin_amdgcn_s_waitcnt(0x0F73); break;
    case 4: __builtin_amdgcn_s_waitcnt(0x0F74); break;
    case 5: __builtin_amdgcn_s_waitcnt(0x0F75); break;
    case 6: __builtin_amdgcn_s_waitcnt(0x0F76); break;
    case 7: __builtin_amdgcn_s_waitcnt(0x0F77); break;
    case 8: __builtin_amdgcn_s_waitcnt(0x0F78); break;
    case 9: __builtin_amdgcn_s_waitcnt(0x0F79); break;
    case 10: __builtin_amdgcn_s_waitcnt(0x0F7A); break;
    case 11: __builtin_amdgcn_s_waitcnt(0x0F7B); break;
    case 12: __builtin_amdgcn_s_waitcnt(0x0F7C); break;
    case 13: __builtin_amdgcn_s_waitcnt(0x0F7D); break;
    case 14: __builtin_amdgcn_s_waitcnt(0x0F7E); break;
    case 15: __builtin_amdgcn_s_waitcnt(0x0F7F); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    }
}

__device__ __forceinline__ int64_t remap_xcd64(int64_t bid, int64_t blocks) {
    // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
    // contiguous range of logical work items.
    const int64_t q = blocks / 8, rem = blocks % 8;
    const int64_t xcd = bid % 8, slot = bid / 8;
    return (xcd < rem) ? xcd * (q + 1) + slot : rem * (q + 1) + (xcd - rem) * q + slot;
}

// The segment owning query tile t: the largest s with tile_start[s] <= t
// (tile_start is non-decreasing; empty segments repeat a value).  The wave
// samples 64 evenly spaced entries per round and keeps the last interval whose
// start is <= t, so nseg <= 64 takes one dependent load and nseg <= 4096 two.
__device__ __forceinline__ int find_segment(const int64_t * __restrict__ tile_start, int nseg,
                                            int64_t t, int lane) {
    int lo = 0, len = nseg;
    while (len > 1) {
        const int stride = (len + 63) >> 6;
        const int off = lane * stride;
        const bool le = off < len && tile_start[lo + off] <= t;
        const int cnt = __popcll(__ballot(le));  // >= 1: tile_start[lo] <= t
        lo += (cnt - 1) * stride;
        len = min(stride, len - (cnt - 1) * stride);
    }
    return __builtin_amdgcn_readfirstlane(lo);
}

// Mean segment length (queries per segment, from the host-known total and
// segment count) up to which bf16 head_dim-64 attention runs the per-segment
// window kernel, and that kernel's waves per workgroup.
#ifndef PXS_ATTN_WINDOW_MEAN
#define PXS_ATTN_WINDOW_MEAN 512
#endif
#ifndef PXS_ATTN_WINDOW_WAVES
#define PXS_ATTN_WINDOW_WAVES 4
#endif
#ifndef PXS_ATTN_WINDOW_ORDER
#define PXS_ATTN_WINDOW_ORDER 1  // segments costliest first (one 1024-thread sort launch)
#endif
#ifndef PXS_ATTN_WINDOW_HPG
#define PXS_ATTN_WINDOW_HPG 1  // heads per workgroup; 0 = from the segment count
#endif

// Mean segment length from which the generic kernel runs 4 waves per
// workgroup instead of one.
#ifndef PXS_ATTN_NW4_MIN
#define PXS_ATTN_NW4_MIN 256
#endif

struct AttnArgs {
    const void * q;
    const void * k;
    const void * v;
    int64_t ldq, ldk, ldv;
    const int64_t * cu_q;
    const int64_t * cu_k;
    int nseg;
    const int64_t * tile_start;  // [nseg + 1]; tile_start[nseg] = total tiles
    const int32_t * row_map;
    int hd, vd;
    float scale_log2;
    void * o;
    int64_t ldo;
    int vec_ok;
    const int32_t * seg_order;  // short-segment kernel: segments, costliest first (or null)
};

template <typename T> struct AttnTraits;
template <> struct AttnTraits<uint16_t> {
    static constexpr int kVec = 8;                  // elements per 16 bytes
    static constexpr int kRowBytes = 64 * 2;        // one padded head row
    static constexpr int kKPitch = kRowBytes + 16;  // K tile row pitch (bytes)
    static constexpr int kVPitch = kKeys * 2 + 8;   // V^T row pitch (bytes)
};
template <> struct AttnTraits<float> {
    static constexpr int kVec = 4;
    static constexpr int kRowBytes = 64 * 4;
    static constexpr int kKPitch = kRowBytes + 16;
    static constexpr int kVPitch = kKeys * 4 + 16;
};

template <typename T>
__device__ __forceinline__ void load16(const T * base, int64_t row, int64_t ld, int col,
                                       int limit, bool vec_ok, T (&out)[16 / sizeof(T)]) {
    constexpr int kVec = 16 / sizeof(T);
    if (vec_ok && col + kVec <= limit) {
        *reinterpret_cast<uint4 *>(out) = *reinterpret_cast<const uint4 *>(base + row * ld + col);
        return;
    }
#pragma unroll
    for (int e = 0; e < kVec; ++e) out[e] = (col + e < limit) ? base[row * ld + col + e] : T(0);
}

__global__ void attn_tiles_kernel(const int64_t * __restrict__ cu_q, int nseg, int bq,
                                  int32_t * __restrict__ tiles) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nseg) return;
    const int64_t len = cu_q[s + 1] - cu_q[s];
    tiles[s] = static_cast<int32_t>((len + bq - 1) / bq);
}

template <typename T, int NW>
__global__ void __launch_bounds__(NW * 64)
flash_attn_kernel(AttnArgs a) {
    using Tr = AttnTraits<T>;
    constexpr int kVec = Tr::kVec;
    constexpr int kThreads = NW * 64;
    constexpr int kChunksPerRow = Tr::kRowBytes / 16;
    __shared__ __align__(16) char k_lds[kKeys * Tr::kKPitch];
    __shared__ __align__(16) char vt_lds[64 * Tr::kVPitch];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, r = lane & 31;
    const int head = blockIdx.y;

    const int64_t t = blockIdx.x;
    if (t >= a.tile_start[a.nseg]) return;
    const int seg = find_segment(a.tile_start, a.nseg, t, lane);
    const int64_t q_begin = a.cu_q[seg] + (t - a.tile_start[seg]) * (32 * NW);
    const int64_t q_end = a.cu_q[seg + 1];
    const int64_t k_begin = a.cu_k[seg], k_end = a.cu_k[seg + 1];

    const T * __restrict__ qp = static_cast<const T *>(a.q);
    const T * __restrict__ kp = static_cast<const T *>(a.k);
    const T * __restrict__ vp = static_cast<const T *>(a.v);

    // This lane's query and its Q fragment (dims 32h .. 32h+31).
    const int64_t qi = q_begin + wave * 32 + r;
    const bool q_valid = qi < q_end;
    const int64_t q_row = q_valid ? (a.row_map ? a.row_map[qi] : qi) : -1;
    T qv[32];
#pragma unroll
    for (int c = 0; c < 32 / kVec; ++c) {
        T tmp[kVec];
        if (q_valid) {
            load16<T>(qp + head * a.hd, q_row, a.ldq, 32 * h + c * kVec, a.hd, a.vec_ok, tmp);
        } else {
#pragma unroll
            for (int e = 0; e < kVec; ++e) tmp[e] = T(0);
        }
#pragma unroll
        for (int e = 0; e < kVec; ++e) qv[c * kVec + e] = tmp[e];
    }

    f32x16 oacc[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) oacc[dt][v] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    for (int64_t kt0 = k_begin; kt0 < k_end; kt0 += kKeys) {
        __syncthreads();
        // Stage K (row layout) and V (transposed) for keys kt0 .. kt0+63.
        for (int c = tid; c < kKeys * kChunksPerRow; c += kThreads) {
            const int key = c / kChunksPerRow, piece = c % kChunksPerRow;
            const int64_t kidx = kt0 + key;
            T kk[kVec], vv[kVec];
            if (kidx < k_end) {
                const int64_t row = a.row_map ? a.row_map[kidx] : kidx;
                load16<T>(kp + head * a.hd, row, a.ldk, piece * kVec, a.hd, a.vec_ok, kk);
                load16<T>(vp + head * a.vd, row, a.ldv, piece * kVec, a.vd, a.vec_ok, vv);
            } else {
#pragma unroll
                for (int e = 0; e < kVec; ++e) kk[e] = vv[e] = T(0);
            }
            *reinterpret_cast<uint4 *>(k_lds + key * Tr::kKPitch + piece * 16) =
                *reinterpret_cast<const uint4 *>(kk);
#pragma unroll
            for (int e = 0; e < kVec; ++e) {
                *reinterpret_cast<T *>(vt_lds + (piece * kVec + e) * Tr::kVPitch +
                                       key * static_cast<int>(sizeof(T))) = vv[e];
            }
        }
        __syncthreads();

        // S^T for two 32-key sub-tiles.
        f32x16 sacc[2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int v = 0; v < 16; ++v) sacc[kt][v] = 0.0f;
            const char * krow = k_lds + (kt * 32 + r) * Tr::kKPitch;
            if constexpr (sizeof(T) == 2) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const bf16x8 af = *reinterpret_cast<const bf16x8 *>(krow + h * 64 + s * 16);
                    bf16x8 bq;
#pragma unroll
                    for (int e = 0; e < 8; ++e) bq[e] = __builtin_bit_cast(__bf16, qv[s * 8 + e]);
                    sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bq, sacc[kt], 0, 0, 0);
                }
            } else {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    const f32x4 af = *reinterpret_cast<const f32x4 *>(krow + (32 * h + 4 * u) * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        sacc[kt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            af[e], __builtin_bit_cast(float, qv[4 * u + e]), sacc[kt], 0, 0, 0);
                    }
                }
            }
        }

        // Online softmax (log2 domain).  Register v of sub-tile kt holds key
        // kt*32 + 8*(v/4) + 4h + v%4.
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t key = kt0 + kt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                const float sv = key < k_end ? sacc[kt][v] * a.scale_log2 : -INFINITY;
                sacc[kt][v] = sv;
                mx = fmaxf(mx, sv);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = (m_new == -INFINITY) ? 1.0f : exp2f(m_run - m_new);
        float rs = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float p = (m_new == -INFINITY) ? 0.0f : exp2f(sacc[kt][v] - m_new);
                sacc[kt][v] = p;
                rs += p;
            }
        }
        rs += __shfl_xor(rs, 32, 64);
        l_run = l_run * alpha + rs;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int v = 0; v < 16; ++v) oacc[dt][v] *= alpha;

        // O^T += V^T P^T.
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            if constexpr (sizeof(T) == 2) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    bf16x8 pb;
#pragma unroll
                    for (int e = 0; e < 8; ++e) pb[e] = static_cast<__bf16>(sacc[kt][8 * u + e]);
#pragma unroll
                    for (int dt = 0; dt < 2; ++dt) {
                        const char * vrow = vt_lds + (dt * 32 + r) * Tr::kVPitch;
                        const int key0 = kt * 32 + 16 * u + 4 * h;
                        const uint2 lo4 = *reinterpret_cast<const uint2 *>(vrow + key0 * 2);
                        const uint2 hi4 = *reinterpret_cast<const uint2 *>(vrow + (key0 + 8) * 2);
                        const uint4 packed = make_uint4(lo4.x, lo4.y, hi4.x, hi4.y);
                        const bf16x8 va = __builtin_bit_cast(bf16x8, packed);
                        oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, oacc[dt], 0, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int dt = 0; dt < 2; ++dt) {
                        const char * vrow = vt_lds + (dt * 32 + r) * Tr::kVPitch;
                        const f32x4 va = *reinterpret_cast<const f32x4 *>(
                            vrow + (kt * 32 + 8 * i + 4 * h) * 4);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                va[j], sacc[kt][4 * i + j], oacc[dt], 0, 0, 0);
                        }
                    }
                }
            }
        }
    }

    if (!q_valid) return;
    const float inv_l = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    T * op = static_cast<T *>(a.o) + q_row * a.ldo + head * a.vd;
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = dt * 32 + 8 * i + 4 * h + j;
                if (d < a.vd) store_f32(op + d, oacc[dt][4 * i + j] * inv_l);
            }
        }
    }
}


// ---------------------------------------------------------------------------
// bf16, head_dim 64 fast path: K/V tiles stream HBM -> LDS with
// global_load_lds_dwordx4 into a double buffer (the next tile loads while the
// current one is consumed), and V stays row-major in LDS: the V^T operand
// fragments are read with ds_read_b64_tr_b16, whose 16-lane transpose hands
// lane (G, i) element i%4 of the rows addressed by lanes i/4 + 4t.  Rows are
// XOR-swizzled in 16-byte pieces (kswz for the K fragment reads, vswz for the
// transposed V reads) so neither read pattern conflicts on LDS banks.

__device__ __align__(16) uint4 g_attn_zero[8];

__device__ __forceinline__ int kswz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int vswz(int row) { return (2 * (row & 3)) ^ ((row >> 2) & 1); }

typedef short v4i16 __attribute__((ext_vector_type(4)));

// Scores are kept in the raw (unscaled) domain; p = exp2(s * c - m * c) with
// c = scale * log2(e) costs one FMA and one exp per score.  The running max m
// is only raised when a tile's max exceeds it by more than kLazyLog2 / c
// (p <= 2^kLazyLog2 meanwhile), so the O rescale runs on few tiles.
constexpr float kLazyLog2 = 8.0f;

__device__ __forceinline__ float lane_pair_max(float v) {
    // max over lanes l and l ^ 32 (v_permlane32_swap exchanges the halves).
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                     false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
}

__device__ __forceinline__ float lane_pair_sum(float v) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                     false, false);
    return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
}

// Software-pipelined bf16 kernel (head_dim 64).  Each wave owns 32 queries.
// Iteration j of the key loop issues 16 MFMAs that do not depend on tile j's
// softmax -- S for tile j+1 (K_{j+1} Q^T) and O += V_{j-1}^T P_{j-1} -- and
// then runs tile j's softmax on the VALU while they execute, so the matrix
// cores and the VALU work at the same time.  K/V tiles stream HBM -> LDS with
// global_load_lds through a ring of 4 stages (tiles j-1 .. j+2 live).
constexpr int kAttnStages = 4;
// PXS_ATTN_W3=1 builds the three-waves-per-SIMD form: K and V in rings of
// their own, 2 K stages (tile j+1 read while j+2 lands in the slot tile j
// left) and 4 V stages (tiles j-1 .. j+2), 48 KB of tiles instead of 64, so
// three workgroups fit a CU, and the register budget capped at 168 VGPRs.
#ifndef PXS_ATTN_W3
#define PXS_ATTN_W3 0
#endif
constexpr bool kAttnW3 = PXS_ATTN_W3 != 0;
// PXS_ATTN_OACC_AGPR=1 keeps the O accumulators in AGPRs: the PV products are
// issued as inline-asm MFMAs whose C/D operands are accumulation registers,
// so their 32 accumulator reads and writes per MFMA stay off the VGPR file
// the softmax works in.  Inline asm hides the MFMA from the compiler's hazard
// checks, so the asm carries its own wait states: 2 before each MFMA (VALU or
// accvgpr write of an operand, then an MFMA read of it) and 24 before the
// accumulators are read back (an MFMA result read by a VALU).
#ifndef PXS_ATTN_OACC_AGPR
#define PXS_ATTN_OACC_AGPR 0
#endif
constexpr int kAttnWavesPerEu = kAttnW3 ? 3 : 2;
constexpr int kAttnTileSlots = kAttnW3 ? 6 : 2 * kAttnStages;  // 8 KB K or V tile slots
// Raise the wave's issue priority while it queues a tile's MFMAs, so the
// SIMD's other wave fills the matrix core's shadow with its VALU softmax.
// Instruction interleave of one steady-state step (PV of the previous tile,
// QK of the next, this tile's exponentials): 0 leaves it to the compiler,
// 1..3 impose MFMA/VALU/LDS-read groups with sched_group_barrier.
#ifndef PXS_ATTN_SCHED
#define PXS_ATTN_SCHED 0
#endif
__device__ __forceinline__ void attn_step_schedule() {
    // masks: 0x008 MFMA, 0x002 VALU, 0x100 LDS read
#if PXS_ATTN_SCHED == 1
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
#elif PXS_ATTN_SCHED == 2
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
#elif PXS_ATTN_SCHED == 3
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
#endif
}

#ifndef PXS_ATTN_SETPRIO
#define PXS_ATTN_SETPRIO 0
#endif
constexpr bool kSetPrio = PXS_ATTN_SETPRIO != 0;
constexpr int kKeyRowsLds = 1024;  // longest permuted segment whose key rows are staged in LDS
#ifndef PXS_ATTN_SADDR
#define PXS_ATTN_SADDR 1
#endif

template <int NW, int DH>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(kAttnWavesPerEu)))
flash_attn_bf16_kernel(AttnArgs a, int heads, int64_t tiles_bound) {
    // DH = 64: 64-key tiles (two 32-key sub-tiles); DH = 128: 32-key tiles of
    // two 64-dim halves.  Either way a K or V tile is 8 KB and a step issues
    // 16 MFMAs; a tile row is stored as DH / 64 halves of 128 bytes, each
    // half laid out (and swizzled) as the 64-dim tile.
    static_assert(DH == 64 || DH == 128, "head dim 64 or 128");
    constexpr int KT = DH == 64 ? 2 : 1;              // 32-key sub-tiles per tile
    constexpr int kKeysT = 32 * KT;                   // keys per tile
    constexpr int NHALF = DH / 64;                    // 64-dim halves of a row
    constexpr int NST = DH / 16;                      // K steps of K Q^T
    constexpr int NDT = DH / 32;                      // 32-dim blocks of O
    constexpr int kHalfBytes = kKeysT * 128;          // one half of a tile
    constexpr int kTileBytes = NHALF * kHalfBytes;    // one K or V tile (8 KB)
    constexpr int kUnitsHalf = kKeysT / 8;            // 8-row load units per half
    constexpr int kInstr = 2 * NHALF * kUnitsHalf / NW;  // K + V wave instructions per tile
    // Load unit u (8 rows of one half of the K or V tile): its half and first
    // row.  (For one half, the plain forms, so the 64-dim code is as before.)
    auto unit_half = [](int u) {
        if constexpr (NHALF == 1) return 0;
        else return (u % (NHALF * kUnitsHalf)) / kUnitsHalf;
    };
    auto unit_row0 = [](int u) {
        if constexpr (NHALF == 1) return (u % kUnitsHalf) * 8;
        else return ((u % (NHALF * kUnitsHalf)) % kUnitsHalf) * 8;
    };
    __shared__ __align__(16) char lds[kAttnTileSlots * kTileBytes];
    // Byte offsets of tile t's K and V slots.
    auto k_slot = [](int t) { return kAttnW3 ? (t & 1) * kTileBytes : (t % kAttnStages) * 2 * kTileBytes; };
    auto v_slot = [](int t) {
        return kAttnW3 ? (2 + (t & 3)) * kTileBytes : (t % kAttnStages) * 2 * kTileBytes + kTileBytes;
    };
    __shared__ int32_t key_rows[kKeyRowsLds];  // row_map of the segment's keys

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, kept in an SGPR
    const int h = lane >> 5, r = lane & 31;

    const int64_t total = tiles_bound * heads;
    const int64_t logical = remap_xcd64(blockIdx.x, total);
    const int head = static_cast<int>(logical / tiles_bound);
    const int64_t t = logical - static_cast<int64_t>(head) * tiles_bound;
    if (t >= a.tile_start[a.nseg]) return;
    const int seg = find_segment(a.tile_start, a.nseg, t, lane);
    const int64_t q_begin = a.cu_q[seg] + (t - a.tile_start[seg]) * (32 * NW);
    const int64_t q_end = a.cu_q[seg + 1];
    const int64_t k_begin = a.cu_k[seg], k_end = a.cu_k[seg + 1];

    const uint16_t * __restrict__ qp = static_cast<const uint16_t *>(a.q);
    const uint16_t * __restrict__ kp = static_cast<const uint16_t *>(a.k);
    const uint16_t * __restrict__ vp = static_cast<const uint16_t *>(a.v);

    // This lane's query and its Q^T fragments (B operand): dims 32h + 8st ..
    const int64_t qi = q_begin + wave * 32 + r;
    const bool q_valid = qi < q_end;
    const int64_t q_row = q_valid ? (a.row_map ? a.row_map[qi] : qi) : -1;
    bf16x8 qf[NST];
#pragma unroll
    for (int st = 0; st < NST; ++st) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (q_valid)
            v = *reinterpret_cast<const uint4 *>(qp + q_row * a.ldq + head * DH + (st / 4) * 64 +
                                                 32 * h + 8 * (st % 4));
        qf[st] = __builtin_bit_cast(bf16x8, v);
    }

    const int ntiles = static_cast<int>((k_end - k_begin + kKeysT - 1) / kKeysT);
    const int lrow = lane >> 3, lslot = lane & 7;
    // Permuted keys (windows): stage the segment's row indices in LDS, so the
    // tile loads below need no global index load (whose wait would also wait
    // for the K/V prefetches in flight).  Longer segments read row_map
    // directly.
    const int64_t klen_all = k_end - k_begin;
    const bool keys_in_lds = a.row_map != nullptr && klen_all <= kKeyRowsLds;
    if (keys_in_lds) {
        for (int64_t i = tid; i < klen_all; i += NW * 64) key_rows[i] = a.row_map[k_begin + i];
        __syncthreads();
    }
    const uint32_t lds_base = lds_offset(&lds[0]);
    // The zero source of masked rows, kept in registers across the loop.
    uint64_t zero_addr = reinterpret_cast<uint64_t>(&g_attn_zero[0]);
    asm volatile("" : "+s"(zero_addr));
#if !PXS_ATTN_SADDR
    // Per-lane source pointers of this wave's kInstr load units for tile 0;
    // a full tile of unpermuted keys advances them by 64 rows.
    const uint16_t * src0[kInstr];
    int64_t src_step[kInstr];
#pragma unroll
    for (int j = 0; j < kInstr; ++j) {
        const int unit = wave * kInstr + j;           // 0..15: 8 K blocks then 8 V blocks
        const bool is_v = unit >= NHALF * kUnitsHalf;
        const int half = unit_half(unit);
        const int row = unit_row0(unit) + lrow;
        const int piece = lslot ^ (is_v ? vswz(row) : kswz(row));
        const int64_t ld = is_v ? a.ldv : a.ldk;
        src0[j] = (is_v ? vp : kp) + (k_begin + row) * ld + head * DH + half * 64 + piece * 8;
        src_step[j] = kKeysT * ld;
    }
#else
    // Full unpermuted tiles: the K and V tile bases (wave-uniform, scalar
    // registers) advance by 64 rows per tile; each lane's byte offset within
    // a tile (row * ld + piece) stays fixed, so a tile's loads need no vector
    // address arithmetic.  Offsets fit 32 bits for rows of up to 2^25 bytes.
    const char * kbase = reinterpret_cast<const char *>(kp + k_begin * a.ldk + head * DH);
    const char * vbase = reinterpret_cast<const char *>(vp + k_begin * a.ldv + head * DH);
    const int64_t kstep = static_cast<int64_t>(kKeysT) * a.ldk * 2;
    const int64_t vstep = static_cast<int64_t>(kKeysT) * a.ldv * 2;
    uint32_t voff[kInstr];
#pragma unroll
    for (int j = 0; j < kInstr; ++j) {
        const int unit = wave * kInstr + j;
        const bool is_v = unit >= NHALF * kUnitsHalf;
        const int half = unit_half(unit);
        const int row = unit_row0(unit) + lrow;
        const int piece = lslot ^ (is_v ? vswz(row) : kswz(row));
        if constexpr (NHALF == 1)
            voff[j] = static_cast<uint32_t>((row * (is_v ? a.ldv : a.ldk) + piece * 8) * 2);
        else
            voff[j] = static_cast<uint32_t>((row * (is_v ? a.ldv : a.ldk) + half * 64 + piece * 8) * 2);
    }
    const bool saddr_ok = a.ldk < (int64_t(1) << 24) && a.ldv < (int64_t(1) << 24);
#endif
    auto issue = [&](int tile) __attribute__((always_inline)) {
        const uint32_t kbase_lds = lds_base + k_slot(tile), vbase_lds = lds_base + v_slot(tile);
        const int64_t kt0 = k_begin + static_cast<int64_t>(tile) * kKeysT;
        if (a.row_map == nullptr && kt0 + kKeysT <= k_end) {
#if PXS_ATTN_SADDR
            if (saddr_ok) {
                const char * kt_base = kbase + tile * kstep;
                const char * vt_base = vbase + tile * vstep;
#pragma unroll
                for (int j = 0; j < kInstr; ++j) {
                    const int unit = wave * kInstr + j;
                    const bool is_v = unit >= NHALF * kUnitsHalf;
                    const int half = unit_half(unit);
                    const int row0 = unit_row0(unit);
                    lds_dma16_sbase(is_v ? vt_base : kt_base, voff[j],
                                    (is_v ? vbase_lds : kbase_lds) + half * kHalfBytes + row0 * 128);
                    (void)half;
                }
                return;
            }
            // Row strides of 2^24 elements or more: the per-row loads below.
#else
#pragma unroll
            for (int j = 0; j < kInstr; ++j) {
                const int unit = wave * kInstr + j;
                const bool is_v = unit >= NHALF * kUnitsHalf;
                const int half = unit_half(unit);
                const int row0 = unit_row0(unit);
                lds_dma16(src0[j] + tile * src_step[j],
                          (is_v ? vbase_lds : kbase_lds) + half * kHalfBytes + row0 * 128);
            }
            return;
#endif
        }
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
            const int unit = wave * kInstr + j;
            const bool is_v = unit >= NHALF * kUnitsHalf;
            const int half = unit_half(unit);
            const int row0 = unit_row0(unit);
            const int row = row0 + lrow;
            const int piece = lslot ^ (is_v ? vswz(row) : kswz(row));
            const int64_t kidx = kt0 + row;
            const void * g = reinterpret_cast<const void *>(zero_addr);
            if (kidx < k_end) {
                const int64_t prow = keys_in_lds ? key_rows[kidx - k_begin]
                                                 : (a.row_map ? a.row_map[kidx] : kidx);
                if constexpr (NHALF == 1) {
                    g = is_v ? static_cast<const void *>(vp + prow * a.ldv + head * 64 + piece * 8)
                             : static_cast<const void *>(kp + prow * a.ldk + head * 64 + piece * 8);
                } else {
                    const int col = head * DH + half * 64 + piece * 8;
                    g = is_v ? static_cast<const void *>(vp + prow * a.ldv + col)
                             : static_cast<const void *>(kp + prow * a.ldk + col);
                }
            }
            lds_dma16(g, (is_v ? vbase_lds : kbase_lds) + half * kHalfBytes + row0 * 128);
        }
    };

    // S^T (keys x queries) for one tile: 2 sub-tiles of 32 keys, 4 K-steps each.
    auto qk = [&](int tile, f32x16 (&s)[KT]) {
        const char * kl = lds + k_slot(tile);
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            const int row = kt * 32 + r;
#pragma unroll
            for (int st = 0; st < NST; ++st) {
                const bf16x8 kf = *reinterpret_cast<const bf16x8 *>(
                    kl + (st / 4) * kHalfBytes + row * 128 + (((4 * h + st % 4) ^ kswz(row)) << 4));
                if (st == 0) {
                    const f32x16 zero = {};
                    s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[0], zero, 0, 0, 0);
                } else {
                    s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[kt], 0, 0, 0);
                }
            }
        }
    };

    // Lane-constant parts of the transposed V reads: source row t = j / 4 of
    // the 4-key group and the 4 dims starting at 16*(G%2) + 4*(j%4).
    const int G = lane >> 4, jl = lane & 15;
    const int v_key_off = 4 * (G >> 1) + (jl >> 2);
    const int v_dim_off = 16 * (G & 1) + 4 * (jl & 3);

    f32x16 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int v = 0; v < 16; ++v) oacc[dt][v] = 0.0f;
    // Orders VALU reads of the accumulators after the last PV MFMA's result
    // (a no-op unless they live in AGPRs).
    auto oacc_ready = [&]() __attribute__((always_inline)) {
#if PXS_ATTN_OACC_AGPR
        static_assert(NDT == 2, "the AGPR form covers two O blocks");
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(oacc[0]), "+a"(oacc[1]));
#endif
    };

    // O^T += V^T P^T for one tile (P^T fragments pb[kt][u] from softmax).
    auto pv = [&](int tile, const bf16x8 (&pb)[KT][2]) {
        const char * vl = lds + v_slot(tile);
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int key_a = kt * 32 + 16 * u + v_key_off;
                const int key_b = key_a + 8;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    const int dbyte = ((dt % 2) * 32 + v_dim_off) * 2;
                    const int piece = dbyte >> 4, within = dbyte & 15;
                    const char * vh = vl + (dt / 2) * kHalfBytes;
                    const char * pa = vh + key_a * 128 + ((piece ^ vswz(key_a)) << 4) + within;
                    const char * pbp = vh + key_b * 128 + ((piece ^ vswz(key_b)) << 4) + within;
                    const v4i16 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (v4i16 __attribute__((address_space(3))) *)(pa));
                    const v4i16 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (v4i16 __attribute__((address_space(3))) *)(pbp));
                    const uint2 lo2 = __builtin_bit_cast(uint2, lo4);
                    const uint2 hi2 = __builtin_bit_cast(uint2, hi4);
                    const bf16x8 va = __builtin_bit_cast(bf16x8, make_uint4(lo2.x, lo2.y, hi2.x, hi2.y));
#if PXS_ATTN_OACC_AGPR
                    asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                        : "+a"(oacc[dt]) : "v"(va), "v"(pb[kt][u]));
#else
                    oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[kt][u], oacc[dt], 0, 0, 0);
#endif
                }
            }
        }
    };

    float m_run = -INFINITY;  // running max of raw scores (lazy, see kLazyLog2)
    float l_part = 0.0f;      // this lane's half of the row sum
    const float c = a.scale_log2;
    const float lazy = kLazyLog2 / c;
    const bf16x2 ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};

    // Softmax of one tile's scores into bf16 P^T fragments, in two parts so
    // that independent MFMAs can be interleaved with each: the max (and the
    // rare lazy rescale of O), then the exponentials and row sums.  valid < 64
    // masks the keys past the segment end (only the last tile).
    auto softmax_max = [&](f32x16 (&s)[KT], int valid) {
        if (valid < kKeysT) {
#pragma unroll
            for (int kt = 0; kt < KT; ++kt)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = kt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
                    if (key >= valid) s[kt][v] = -INFINITY;
                }
        }
        float mx = fmaxf(s[0][0], s[0][1]);
#pragma unroll
        for (int v = 2; v < 16; ++v) mx = fmaxf(mx, s[0][v]);
#pragma unroll
        for (int kt = 1; kt < KT; ++kt)
#pragma unroll
            for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kt][v]);
        return lane_pair_max(mx);
    };
    // Raise the running max only when this tile would overflow the lazy
    // headroom somewhere in the wave (a uniform branch).  O must already hold
    // every earlier tile's PV product.
    auto rescale = [&](float mx) __attribute__((always_inline)) {
        if (__builtin_expect(__ballot(mx > m_run + lazy) != 0, 0)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
            m_run = m_new;
            l_part *= alpha;
            oacc_ready();
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int v = 0; v < 16; ++v) oacc[dt][v] *= alpha;
        }
    };
    auto softmax_exp = [&](const f32x16 (&s)[KT], bf16x8 (&pb)[KT][2]) {
        const float mc = m_run * c;
        float lsum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                bf16x8 p8;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    bf16x2 pp;
                    pp[0] = static_cast<__bf16>(__builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][8 * u + e], c, -mc)));
                    pp[1] = static_cast<__bf16>(__builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][8 * u + e + 1], c, -mc)));
                    p8[e] = pp[0];
                    p8[e + 1] = pp[1];
                    lsum = __builtin_amdgcn_fdot2_f32_bf16(pp, ones, lsum, false);
                }
                pb[kt][u] = p8;
            }
        }
        return lsum;  // this lane's share of the tile's row sum
    };
    // Full tiles after the first skip the max: m_run (the first tile's max,
    // raised only by the lazy rescale of a partial last tile) stays in place,
    // and a tile whose scores exceed it by enough to push a row sum past
    // kTileSumLimit (or to inf) is redone with its true max.  p then stays
    // below 2^40, far from fp32 and bf16 overflow in O and l.
    constexpr float kTileSumLimit = 1099511627776.0f;  // 2^40
    auto softmax_exp_checked = [&](f32x16 (&s)[KT], bf16x8 (&pb)[KT][2]) __attribute__((always_inline)) {
        float ts = softmax_exp(s, pb);
        attn_step_schedule();
        if (__builtin_expect(__ballot(!(ts <= kTileSumLimit)) != 0, 0)) {
            const float mx = softmax_max(s, kKeysT);
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
            m_run = m_new;
            l_part *= alpha;
            oacc_ready();
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int v = 0; v < 16; ++v) oacc[dt][v] *= alpha;
            ts = softmax_exp(s, pb);
        }
        l_part += ts;
    };

    // One steady-state step for tile j (full, not the last): PV(j-1) with the
    // max of S_j, then the rescale, then QK(j+1) with the exponentials of S_j.
    // One steady-state step for full tile j > 0: PV(j-1), QK(j+1), then tile
    // j's exponentials (overflow-checked) while those MFMAs run.  The first
    // tile (step_first) takes its max to set m_run.
    auto step = [&](int j, f32x16 (&s_cur)[KT], f32x16 (&s_next)[KT], bf16x8 (&p)[KT][2]) {
        // Tile j+1 has landed (it is the newest load); the barrier also frees
        // the stage of tile j-2 for tile j+2.
        wait_vmcnt0();
        barrier_no_fence();
        if (j + 2 < ntiles) issue(j + 2);
        if constexpr (kSetPrio) __builtin_amdgcn_s_setprio(1);
        pv(j - 1, p);
        qk(j + 1, s_next);
        if constexpr (kSetPrio) __builtin_amdgcn_s_setprio(0);
        softmax_exp_checked(s_cur, p);
    };
    auto step_first = [&](f32x16 (&s_cur)[KT], f32x16 (&s_next)[KT], bf16x8 (&p)[KT][2]) {
        wait_vmcnt0();
        barrier_no_fence();
        if (2 < ntiles) issue(2);
        rescale(softmax_max(s_cur, kKeysT));
        qk(1, s_next);
        softmax_exp_checked(s_cur, p);
    };

    const int64_t klen = k_end - k_begin;
    if (ntiles > 0) {
        issue(0);
        if (ntiles > 1) issue(1);
        if (ntiles > 1) wait_vmcnt(kInstr);
        else wait_vmcnt0();
        barrier_no_fence();
        f32x16 s_a[KT], s_b[KT];
        bf16x8 p_prev[KT][2];
        qk(0, s_a);
        // Steady state over tiles 0 .. ntiles-2 (only the last can be
        // partial): the first tile peeled, the rest unrolled by two so the S
        // registers alternate roles.
        int j = 1;
        if (ntiles > 1) {
            step_first(s_a, s_b, p_prev);
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) s_a[kt] = s_b[kt];
        }
        for (; j + 2 < ntiles; j += 2) {
            step(j, s_a, s_b, p_prev);
            step(j + 1, s_b, s_a, p_prev);
        }
        if (j + 1 < ntiles) {
            step(j, s_a, s_b, p_prev);
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) s_a[kt] = s_b[kt];
        }
        // Last tile (possibly partial), then the two outstanding PV products.
        const int last = ntiles - 1;
        if (last > 0) pv(last - 1, p_prev);
        const float mx = softmax_max(s_a, static_cast<int>(klen - static_cast<int64_t>(last) * kKeysT));
        rescale(mx);
        l_part += softmax_exp(s_a, p_prev);
        pv(last, p_prev);
    }

    const float l_tot = lane_pair_sum(l_part);
    if (!q_valid) return;
    oacc_ready();
    const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    uint16_t * op = static_cast<uint16_t *>(a.o) + q_row * a.ldo + head * DH;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = dt * 32 + 8 * i + 4 * h;
            uint2 packed;
            packed.x = pack_bf16x2(oacc[dt][4 * i + 0] * inv_l, oacc[dt][4 * i + 1] * inv_l);
            packed.y = pack_bf16x2(oacc[dt][4 * i + 2] * inv_l, oacc[dt][4 * i + 3] * inv_l);
            *reinterpret_cast<uint2 *>(op + d) = packed;
        }
    }
}

// ---------------------------------------------------------------------------
// Short segments (windows of a few hundred rows, bf16, head_dim 64): one
// workgroup owns a segment and a group of heads and walks its (head, query
// pass, 64-key chunk) items with one continuous DMA pipeline, so the
// segment's setup (bounds, row-map staging) and the pipeline fill are paid
// once per segment and head group, not once per head; each item is an exact
// online-softmax step (the chunk's own max).  A pass covers 32 * NW queries.
//
// Every global read in the item loop is an LDS DMA whose completion the
// kernel counts itself: the K/V chunks go through a ring of kWinStages
// stages shared by the waves, and each wave DMAs its own 32 query rows into
// a private slot (kWinStages slots per wave) with the first chunk of each
// (head, pass), and reads its fragments from there at every item of it.
// Chunk t + kWinStages is issued at the end of item t, once a barrier shows
// every wave has finished reading stage t % kWinStages.  The kernel is
// latency bound (a workgroup's chain is segment bounds -> row map -> DMA ->
// compute -> store), so what it is tuned for is workgroups per CU: one stage
// and re-read query fragments keep it at 36 KB of LDS and 128 VGPRs, four
// workgroups per CU.
#ifndef PXS_ATTN_WINDOW_STAGES
#define PXS_ATTN_WINDOW_STAGES 1
#endif
constexpr int kWinStages = PXS_ATTN_WINDOW_STAGES;
static_assert(kWinStages >= 1 && kWinStages <= 3, "window ring depth");
constexpr int kWinRowsLds = 512;  // longest segment whose row map is staged in LDS (8^3)

#ifndef PXS_ATTN_WINDOW_WAVES_PER_EU
#define PXS_ATTN_WINDOW_WAVES_PER_EU 4
#endif

template <int NW>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(PXS_ATTN_WINDOW_WAVES_PER_EU)))
window_attn_bf16_kernel(AttnArgs a, int heads, int heads_per_group, int groups) {
    constexpr int kTileBytes = kKeys * 128;       // 64 keys x 64 dims, bf16
    constexpr int kInstr = 2 * (kKeys / 8) / NW;  // K + V DMA instructions per wave per chunk
    constexpr int kQInstr = 4;                    // 32 query rows x 8 pieces / 64 lanes
    constexpr int kQSlotBytes = 32 * 128;
    static_assert(kInstr >= 1 && kInstr * NW * 8 == 2 * kKeys, "chunk rows must split over waves");
    static_assert((kWinStages - 1) * (kInstr + kQInstr) <= 15, "vmcnt bookkeeping range");
    __shared__ __align__(16) char lds[kWinStages][2 * kTileBytes];
    __shared__ __align__(16) char qlds[kWinStages][NW][kQSlotBytes];
    __shared__ int32_t q_rows[kWinRowsLds];
    __shared__ int32_t k_rows[kWinRowsLds];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5, r = lane & 31;
    // Workgroups take the segments costliest first (seg_order, when given:
    // the last to start then are the shortest, which trims the tail);
    // consecutive workgroups land on different XCDs, and segments share no
    // rows, so there is no L2 locality to keep.
    const int64_t logical = blockIdx.x;
    const int slot = static_cast<int>(logical / groups);
    const int grp = static_cast<int>(logical - static_cast<int64_t>(slot) * groups);
    const int seg = a.seg_order ? a.seg_order[slot] : slot;
    const int head0 = grp * heads_per_group;
    const int nheads = min(heads_per_group, heads - head0);
    const int64_t q0 = a.cu_q[seg], k0 = a.cu_k[seg];
    const int64_t nq = a.cu_q[seg + 1] - q0, nk = a.cu_k[seg + 1] - k0;
    if (nq <= 0 || nheads <= 0) return;  // uniform over the workgroup

    const char * __restrict__ qp = static_cast<const char *>(a.q);
    const char * __restrict__ kp = static_cast<const char *>(a.k);
    const char * __restrict__ vp = static_cast<const char *>(a.v);
    uint16_t * __restrict__ op = static_cast<uint16_t *>(a.o);
    // Row strides in bytes; the drop-in's strides are far below 2^32 bytes.
    const uint32_t ldq_b = static_cast<uint32_t>(a.ldq) * 2u;
    const uint32_t ldk_b = static_cast<uint32_t>(a.ldk) * 2u;
    const uint32_t ldv_b = static_cast<uint32_t>(a.ldv) * 2u;
    const uint64_t q_addr = reinterpret_cast<uint64_t>(qp);
    // Each wave DMAs only K rows or only V rows of a chunk (NW >= 2): its
    // source and stride are chosen once here, as values.
    static_assert(NW >= 2, "a wave's chunk DMAs must be all K or all V");
    const bool dma_v = wave * kInstr >= kKeys / 8;
    const uint32_t dma_ld = dma_v ? ldv_b : ldk_b;
    const uint64_t dma_base = dma_v ? reinterpret_cast<uint64_t>(vp) : reinterpret_cast<uint64_t>(kp);

    const int passes = static_cast<int>((nq + 32 * NW - 1) / (32 * NW));
    const int chunks = static_cast<int>((nk + kKeys - 1) / kKeys);
    const int per_head = passes * chunks;
    const int items = nheads * per_head;
    const int lrow = lane >> 3, lslot = lane & 7;
    const uint32_t lds_base = lds_offset(&lds[0][0]);
    const uint32_t q_base = lds_offset(&qlds[0][wave][0]);
    uint64_t zero_addr = reinterpret_cast<uint64_t>(&g_attn_zero[0]);
    asm volatile("" : "+s"(zero_addr));
    const int G = lane >> 4, jl = lane & 15;
    const int v_key_off = 4 * (G >> 1) + (jl >> 2);
    const int v_dim_off = 16 * (G & 1) + 4 * (jl & 3);
    const float c = a.scale_log2;

    // The item loop, for a row map staged in LDS (the segment's physical rows,
    // row_map or identity) or read from global memory (longer segments).
    auto run = [&](auto rows_in_lds) __attribute__((always_inline)) {
        constexpr bool kLds = decltype(rows_in_lds)::value;
        auto q_row_of = [&](int i) -> uint32_t {
            if constexpr (kLds) return static_cast<uint32_t>(q_rows[i]);
            else return static_cast<uint32_t>(a.row_map ? a.row_map[q0 + i] : q0 + i);
        };
        auto k_row_of = [&](int i) -> uint32_t {
            if constexpr (kLds) return static_cast<uint32_t>(k_rows[i]);
            else return static_cast<uint32_t>(a.row_map ? a.row_map[k0 + i] : k0 + i);
        };
        if (chunks == 0) {
            // queries without keys: zeros, as the tiled kernels write
            for (int hh = 0; hh < nheads; ++hh)
                for (int i = wave * 32 + r; i < nq; i += 32 * NW) {
                    if (h) continue;
                    uint4 * dst = reinterpret_cast<uint4 *>(
                        op + static_cast<int64_t>(q_row_of(i)) * a.ldo + (head0 + hh) * 64);
#pragma unroll
                    for (int j = 0; j < 8; ++j) dst[j] = make_uint4(0, 0, 0, 0);
                }
            return;
        }

        // DMA instructions per wave that item t issues: its K/V chunk, plus
        // this wave's query rows when it is the first chunk of a (head, pass).
        auto instrs = [&](int t) -> int { return kInstr + (t % chunks == 0 ? kQInstr : 0); };
        auto issue = [&](int t) __attribute__((always_inline)) {
            const int hh = t / per_head;
            const int rem = t - hh * per_head;
            const int kc = rem % chunks;
            const uint32_t head_b = static_cast<uint32_t>(head0 + hh) * 128u;
            const uint32_t base = lds_base + (t % kWinStages) * (2 * kTileBytes);
            // the lane's rows first, then the addresses: one LDS round trip
            int32_t kidx[kInstr];
            uint32_t prow[kInstr];
#pragma unroll
            for (int j = 0; j < kInstr; ++j) {
                const int unit = wave * kInstr + j;  // 0..15: 8 K blocks then 8 V blocks
                kidx[j] = kc * kKeys + (unit % (kKeys / 8)) * 8 + lrow;
                prow[j] = kidx[j] < nk ? k_row_of(kidx[j]) : 0u;
            }
#pragma unroll
            for (int j = 0; j < kInstr; ++j) {
                const int unit = wave * kInstr + j;
                const int row0 = (unit % (kKeys / 8)) * 8;
                const int row = row0 + lrow;
                const uint32_t piece_b = static_cast<uint32_t>(lslot ^ (dma_v ? vswz(row) : kswz(row))) * 16u;
                const uint64_t addr = static_cast<uint64_t>(prow[j]) * dma_ld + dma_base + (head_b + piece_b);
                lds_dma16(reinterpret_cast<const void *>(kidx[j] < nk ? addr : zero_addr),
                          base + (dma_v ? kTileBytes : 0) + row0 * 128);
            }
            if (kc == 0) {
                // this wave's 32 query rows of (head, pass), K-swizzled like a key tile
                const int pass = rem / chunks;
                const uint32_t qb = q_base + ((t / chunks) % kWinStages) * (NW * kQSlotBytes);
                int32_t qi[kQInstr];
                uint32_t qrow[kQInstr];
#pragma unroll
                for (int j = 0; j < kQInstr; ++j) {
                    qi[j] = pass * 32 * NW + wave * 32 + j * 8 + lrow;
                    qrow[j] = qi[j] < nq ? q_row_of(qi[j]) : 0u;
                }
#pragma unroll
                for (int j = 0; j < kQInstr; ++j) {
                    const uint32_t piece_b = static_cast<uint32_t>(lslot ^ kswz(j * 8 + lrow)) * 16u;
                    const uint64_t addr = static_cast<uint64_t>(qrow[j]) * ldq_b + q_addr + (head_b + piece_b);
                    lds_dma16(reinterpret_cast<const void *>(qi[j] < nq ? addr : zero_addr),
                              qb + j * 8 * 128);
                }
            }
        };

#pragma unroll
        for (int t = 0; t < kWinStages; ++t)
            if (t < items) issue(t);

        // Zeroed once: each group's first item rescales the accumulators by
        // exp2(-inf) = 0 (the scale is positive), which clears what the
        // previous group left (finite).
        f32x16 oacc[2];
#pragma unroll
        for (int dt = 0; dt < 2; ++dt)
#pragma unroll
            for (int v = 0; v < 16; ++v) oacc[dt][v] = 0.0f;
        float m_run = -INFINITY, l_part = 0.0f;
        for (int t = 0; t < items; ++t) {
            const int hh = t / per_head;
            const int rem = t - hh * per_head;
            const int pass = rem / chunks, kc = rem - (rem / chunks) * chunks;
            // Item t's DMAs have landed: only those of the items issued after
            // it (t+1 .. t+kWinStages-1) may be in flight; loads return in order.
            int after = 0;
#pragma unroll
            for (int u = 1; u < kWinStages; ++u)
                if (t + u < items) after += instrs(t + u);
            wait_vmcnt(after);
            barrier_no_fence();
            // A wave whose 32 queries all lie past the segment's end (the last
            // pass of a segment that is not a multiple of 32 * NW) only keeps
            // the pipeline going: its DMAs and barriers, no compute.
            const bool active = pass * 32 * NW + wave * 32 < nq;
            if (kc == 0) m_run = -INFINITY;
            if (active) {
                // This wave's query fragments, read again for every item (its
                // slot holds them until the group's last item ends), so no
                // registers stay tied up with them across items.
                bf16x8 qf[4];
                const char * qs = &qlds[(t / chunks) % kWinStages][wave][0];
#pragma unroll
                for (int st = 0; st < 4; ++st)
                    qf[st] = *reinterpret_cast<const bf16x8 *>(qs + r * 128 + (((4 * h + st) ^ kswz(r)) << 4));

                const char * kl = lds[t % kWinStages];
                const char * vl = kl + kTileBytes;
                f32x16 sc[2];
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
                    const int row = kt * 32 + r;
#pragma unroll
                    for (int st = 0; st < 4; ++st) {
                        const bf16x8 kf = *reinterpret_cast<const bf16x8 *>(
                            kl + row * 128 + (((4 * h + st) ^ kswz(row)) << 4));
                        if (st == 0) {
                            const f32x16 zero = {};
                            sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[0], zero, 0, 0, 0);
                        } else {
                            sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], sc[kt], 0, 0, 0);
                        }
                    }
                }
                // Keys past the segment's end: register v of sub-tile kt holds
                // key kt*32 + 8*(v/4) + 4h + v%4, so each block of four
                // registers spans keys base .. base+7 over the two lane halves
                // and is wholly valid, wholly masked or split (one block).
                const int valid = static_cast<int>(min<int64_t>(nk - static_cast<int64_t>(kc) * kKeys, kKeys));
                if (valid < kKeys) {
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const int base = kt * 32 + 8 * b;
                            if (base >= valid) {
#pragma unroll
                                for (int i = 0; i < 4; ++i) sc[kt][4 * b + i] = -INFINITY;
                            } else if (base + 8 > valid) {
#pragma unroll
                                for (int i = 0; i < 4; ++i)
                                    if (base + 4 * h + i >= valid) sc[kt][4 * b + i] = -INFINITY;
                            }
                        }
                }
                float mx = sc[0][0];
#pragma unroll
                for (int v = 1; v < 16; ++v) mx = fmaxf(mx, sc[0][v]);
#pragma unroll
                for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sc[1][v]);
                mx = lane_pair_max(mx);
                const float m_new = fmaxf(m_run, mx);  // finite: every chunk has a valid key
                const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c);
                m_run = m_new;
                l_part *= alpha;
#pragma unroll
                for (int dt = 0; dt < 2; ++dt)
#pragma unroll
                    for (int v = 0; v < 16; ++v) oacc[dt][v] *= alpha;
                const float mc = m_run * c;
                const bf16x2 ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
                bf16x8 pb[2][2];
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        bf16x8 p8;
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            bf16x2 pp;
                            pp[0] = static_cast<__bf16>(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][8 * u + e], c, -mc)));
                            pp[1] = static_cast<__bf16>(__builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][8 * u + e + 1], c, -mc)));
                            p8[e] = pp[0];
                            p8[e + 1] = pp[1];
                            l_part = __builtin_amdgcn_fdot2_f32_bf16(pp, ones, l_part, false);
                        }
                        pb[kt][u] = p8;
                    }
                }
#pragma unroll
                for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int key_a = kt * 32 + 16 * u + v_key_off;
                        const int key_b = key_a + 8;
#pragma unroll
                        for (int dt = 0; dt < 2; ++dt) {
                            const int dbyte = (dt * 32 + v_dim_off) * 2;
                            const int piece = dbyte >> 4, within = dbyte & 15;
                            const char * pa = vl + key_a * 128 + ((piece ^ vswz(key_a)) << 4) + within;
                            const char * pbp = vl + key_b * 128 + ((piece ^ vswz(key_b)) << 4) + within;
                            const v4i16 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                (v4i16 __attribute__((address_space(3))) *)(pa));
                            const v4i16 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                (v4i16 __attribute__((address_space(3))) *)(pbp));
                            const uint2 lo2 = __builtin_bit_cast(uint2, lo4);
                            const uint2 hi2 = __builtin_bit_cast(uint2, hi4);
                            const bf16x8 va = __builtin_bit_cast(bf16x8, make_uint4(lo2.x, lo2.y, hi2.x, hi2.y));
                            oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[kt][u], oacc[dt], 0, 0, 0);
                        }
                    }
                }
            }  // active
            // Every wave has read stage t % kWinStages (and its own query
            // slot): refill them with item t + kWinStages.
            if (t + kWinStages < items) {
                barrier_no_fence();
                issue(t + kWinStages);
            }
            if (active && kc == chunks - 1) {
                const float l_tot = lane_pair_sum(l_part);
                const int qi = pass * 32 * NW + wave * 32 + r;
                if (qi < nq) {
                    const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
                    uint16_t * dst = op + static_cast<int64_t>(q_row_of(qi)) * a.ldo + (head0 + hh) * 64;
#pragma unroll
                    for (int dt = 0; dt < 2; ++dt) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int d = dt * 32 + 8 * i + 4 * h;
                            uint2 packed;
                            packed.x = pack_bf16x2(oacc[dt][4 * i + 0] * inv_l, oacc[dt][4 * i + 1] * inv_l);
                            packed.y = pack_bf16x2(oacc[dt][4 * i + 2] * inv_l, oacc[dt][4 * i + 3] * inv_l);
                            *reinterpret_cast<uint2 *>(dst + d) = packed;
                        }
                    }
                }
            }
        }
    };

    // Physical rows of the segment's queries and keys (row_map or identity).
    if (nq <= kWinRowsLds && nk <= kWinRowsLds) {
        for (int i = tid; i < nq; i += NW * 64)
            q_rows[i] = static_cast<int32_t>(a.row_map ? a.row_map[q0 + i] : q0 + i);
        for (int i = tid; i < nk; i += NW * 64)
            k_rows[i] = static_cast<int32_t>(a.row_map ? a.row_map[k0 + i] : k0 + i);
        __syncthreads();
        run(std::true_type{});
    } else {
        run(std::false_type{});
    }
}

// Segments in the order the short-segment kernel takes them: a counting sort
// by item count (query passes x key chunks, the same for every head group),
// costliest class first, empty segments last.  The order within a class is
// whatever the LDS atomics give; every segment's output rows are its own, so
// results do not depend on it.
constexpr int kOrderClasses = 17;
constexpr int kOrderMaxSegments = 65536;
__global__ void __launch_bounds__(1024)
window_order_kernel(const int64_t * __restrict__ cu_q, const int64_t * __restrict__ cu_k, int nseg,
                    int q_pass, int32_t * __restrict__ order) {
    __shared__ int next[kOrderClasses];
    const int tid = threadIdx.x;
    auto cls = [&](int s) -> int {
        const int64_t nq = cu_q[s + 1] - cu_q[s], nk = cu_k[s + 1] - cu_k[s];
        if (nq <= 0) return 0;
        const int64_t work = ((nq + q_pass - 1) / q_pass) * ((nk + kKeys - 1) / kKeys);
        return static_cast<int>(min<int64_t>(max<int64_t>(work, 1), kOrderClasses - 1));
    };
    if (tid < kOrderClasses) next[tid] = 0;
    __syncthreads();
    for (int s = tid; s < nseg; s += 1024) atomicAdd(&next[cls(s)], 1);
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int c = kOrderClasses - 1; c >= 0; --c) {
            const int n = next[c];
            next[c] = run;
            run += n;
        }
    }
    __syncthreads();
    for (int s = tid; s < nseg; s += 1024) order[atomicAdd(&next[cls(s)], 1)] = s;
}

template <int NW>
int launch_attn_window(const AttnArgs & args, int heads, hipStream_t stream) {
    // Head groups: enough workgroups to give every CU a few (256 CUs).
    const int64_t want = (4 * 256 + args.nseg - 1) / std::max(args.nseg, 1);
    const int groups0 = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(heads, want)));
    const int hpg = PXS_ATTN_WINDOW_HPG > 0 ? std::min(heads, PXS_ATTN_WINDOW_HPG)
                                            : (heads + groups0 - 1) / groups0;
    const int groups = (heads + hpg - 1) / hpg;
    const int64_t blocks = static_cast<int64_t>(args.nseg) * groups;
    if (blocks > INT32_MAX) return fail(PXS_ERR_ARG, "attention grid too large");
    hipLaunchKernelGGL((window_attn_bf16_kernel<NW>), dim3(static_cast<unsigned>(blocks)),
                       dim3(NW * 64), 0, stream, args, heads, hpg, groups);
    return check_launch("window attention (bf16)");
}

template <int NW, int DH>
int launch_attn_bf16(const AttnArgs & args, int64_t total_q, int heads, hipStream_t stream) {
    const int64_t bound = total_q / (32 * NW) + args.nseg + 1;
    if (bound * heads > INT32_MAX) return fail(PXS_ERR_ARG, "attention grid too large");
    hipLaunchKernelGGL((flash_attn_bf16_kernel<NW, DH>), dim3(static_cast<unsigned>(bound * heads)),
                       dim3(NW * 64), 0, stream, args, heads, bound);
    return check_launch("flash attention (bf16)");
}

template <typename T, int NW>
int launch_attn(const AttnArgs & args, int64_t total_q, int heads, hipStream_t stream) {
    const int64_t bound = total_q / (32 * NW) + args.nseg + 1;
    if (bound > INT32_MAX) return fail(PXS_ERR_ARG, "attention grid too large");
    hipLaunchKernelGGL((flash_attn_kernel<T, NW>), dim3(static_cast<unsigned>(bound), heads),
                       dim3(NW * 64), 0, stream, args);
    return check_launch("flash attention");
}

bool aligned16(const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Scratch of pxs_varlen_attention_noalloc: the segment tile counts, their
// prefix sums and the scan partials of up to PXS_ATTN_NOALLOC_MAX_SEGMENTS
// segments.  Each device holds its own copy for the life of the process.
constexpr size_t kNoAllocScratchBytes = 1u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up once per
// device (the host-side symbol is only a stand-in and must never reach a
// kernel).
int noalloc_scratch(void ** out) {
    int dev = 0;
    if (int rc = check_hip(hipGetDevice(&dev), "pxs_varlen_attention_noalloc: hipGetDevice"))
        return rc;
    PXS_CHECK(dev >= 0 && dev < kMaxDevices, PXS_ERR_ARG,
              "pxs_varlen_attention_noalloc: device index out of range");
    // Racing first calls look up the same address and store the same value.
    void * cached = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!cached) {
        void * ptr = nullptr;
        if (int rc = check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)),
                               "pxs_varlen_attention_noalloc: hipGetSymbolAddress"))
            return rc;
        PXS_CHECK(ptr != nullptr, PXS_ERR_HIP,
                  "pxs_varlen_attention_noalloc: no device address for the scratch array");
        g_scratch_ptr[dev].store(ptr, std::memory_order_release);
        cached = ptr;
    }
    *out = cached;
    return PXS_OK;
}

// Heads wider than the tiled kernels take (head_dim or value_dim above 64, up
// to kWideMaxDim): one wavefront per (query row, head) walks the segment's
// keys in order with an online softmax.  Lane l owns dims l, l + 64, ... of
// q, k and the output; a key's score is the wavefront sum of the lanes'
// partial dot products.  Latency-bound (every key costs a 6-step shuffle
// reduction), but it keeps the drop-in's attention free of a head-size limit.
constexpr int kWideMaxDim = 512;
constexpr int kWidePerLane = kWideMaxDim / 64;

template <typename T>
__global__ void __launch_bounds__(64)
attn_wide_kernel(AttnArgs a, int64_t total_q, float scale) {
    const int64_t qi = blockIdx.x;
    const int head = blockIdx.y;
    const int lane = threadIdx.x;
    if (qi >= total_q) return;
    // segment of query qi: the last s with cu_q[s] <= qi
    int lo = 0, hi = a.nseg;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (a.cu_q[mid] <= qi) lo = mid; else hi = mid;
    }
    const int64_t k_begin = a.cu_k[lo], k_end = a.cu_k[lo + 1];
    const T * q = static_cast<const T *>(a.q);
    const T * k = static_cast<const T *>(a.k);
    const T * v = static_cast<const T *>(a.v);
    const int64_t q_row = a.row_map ? a.row_map[qi] : qi;
    float qv[kWidePerLane];
#pragma unroll
    for (int c = 0; c < kWidePerLane; ++c) {
        const int d = lane + 64 * c;
        qv[c] = d < a.hd ? load_f32(q + q_row * a.ldq + static_cast<int64_t>(head) * a.hd + d) : 0.0f;
    }
    float acc[kWidePerLane];
#pragma unroll
    for (int c = 0; c < kWidePerLane; ++c) acc[c] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    for (int64_t j = k_begin; j < k_end; ++j) {
        const int64_t row = a.row_map ? a.row_map[j] : j;
        const T * kr = k + row * a.ldk + static_cast<int64_t>(head) * a.hd;
        float part = 0.0f;
#pragma unroll
        for (int c = 0; c < kWidePerLane; ++c) {
            const int d = lane + 64 * c;
            if (d < a.hd) part += qv[c] * load_f32(kr + d);
        }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
        const float sc = part * scale;
        const float m_new = fmaxf(m, sc);
        const float corr = expf(m - m_new);  // 0 on the first key (m = -inf)
        const float p = expf(sc - m_new);
        l = l * corr + p;
        const T * vr = v + row * a.ldv + static_cast<int64_t>(head) * a.vd;
#pragma unroll
        for (int c = 0; c < kWidePerLane; ++c) {
            const int d = lane + 64 * c;
            if (d < a.vd) acc[c] = acc[c] * corr + p * load_f32(vr + d);
        }
        m = m_new;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;  // no keys: zeros
    T * o = static_cast<T *>(a.o);
#pragma unroll
    for (int c = 0; c < kWidePerLane; ++c) {
        const int d = lane + 64 * c;
        if (d < a.vd) store_f32(o + q_row * a.ldo + static_cast<int64_t>(head) * a.vd + d, acc[c] * inv);
    }
}

} // namespace
} // namespace pxs

using namespace pxs;

extern "C" {

size_t pxs_attention_workspace_bytes(int nseg) {
    const int64_t n = std::max(nseg, 1);
    return static_cast<size_t>(n + 1) * sizeof(int64_t) + static_cast<size_t>(n) * sizeof(int32_t) +
           scan_workspace_bytes(n) + 64;
}

int pxs_varlen_attention(int dtype, const void * q, int64_t ld_q, const void * k, int64_t ld_k,
                         const void * v, int64_t ld_v, const int64_t * cu_q,
                         const int64_t * cu_k, int nseg, int64_t total_q,
                         const int32_t * row_map, int heads, int head_dim, int value_dim,
                         float scale, void * o, int64_t ld_o, void * workspace, void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_varlen_attention");
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG, "pxs_varlen_attention: bad dtype");
    PXS_CHECK(heads > 0 && head_dim > 0 && head_dim <= kWideMaxDim && value_dim > 0 &&
                  value_dim <= kWideMaxDim,
              PXS_ERR_ARG, "pxs_varlen_attention: head_dim and value_dim must be in 1..512");
    PXS_CHECK(heads <= 65535, PXS_ERR_ARG, "pxs_varlen_attention: too many heads");
    PXS_CHECK(scale > 0.0f && std::isfinite(scale), PXS_ERR_ARG,
              "sparse attention scale must be finite and positive");
    PXS_CHECK(nseg >= 0 && total_q >= 0, PXS_ERR_ARG, "pxs_varlen_attention: bad segment count");
    PXS_CHECK(ld_q >= heads * head_dim && ld_k >= heads * head_dim && ld_v >= heads * value_dim &&
                  ld_o >= heads * value_dim,
              PXS_ERR_ARG, "pxs_varlen_attention: row stride smaller than heads * head_dim");
    if (nseg == 0 || total_q == 0) return PXS_OK;
    PXS_CHECK(q && k && v && o && cu_q && cu_k && workspace, PXS_ERR_ARG,
              "pxs_varlen_attention: null pointer");
    hipStream_t s = as_stream(stream);
    // bf16 head_dim 128 runs the tiled kernel too (32-key tiles of two 64-dim halves)
    const bool fast128 = dtype == PXS_BF16 && head_dim == 128 && value_dim == 128 &&
                         (ld_q % 8 == 0) && (ld_k % 8 == 0) && (ld_v % 8 == 0) && (ld_o % 4 == 0) &&
                         aligned16(q) && aligned16(k) && aligned16(v) &&
                         (reinterpret_cast<uintptr_t>(o) & 7u) == 0;
    if ((head_dim > 64 || value_dim > 64) && !fast128) {
        PXS_CHECK(total_q <= INT32_MAX, PXS_ERR_ARG, "attention grid too large");
        AttnArgs a{};
        a.q = q; a.k = k; a.v = v; a.ldq = ld_q; a.ldk = ld_k; a.ldv = ld_v;
        a.cu_q = cu_q; a.cu_k = cu_k; a.nseg = nseg; a.row_map = row_map;
        a.hd = head_dim; a.vd = value_dim; a.o = o; a.ldo = ld_o;
        const dim3 grid(static_cast<unsigned>(total_q), heads);
        if (dtype == PXS_BF16) {
            hipLaunchKernelGGL(attn_wide_kernel<uint16_t>, grid, dim3(64), 0, s, a, total_q, scale);
        } else {
            hipLaunchKernelGGL(attn_wide_kernel<float>, grid, dim3(64), 0, s, a, total_q, scale);
        }
        return check_launch("flash attention (wide heads)");
    }
    const bool fast = dtype == PXS_BF16 && head_dim == 64 && value_dim == 64 && (ld_q % 8 == 0) &&
                      (ld_k % 8 == 0) && (ld_v % 8 == 0) && (ld_o % 4 == 0) && aligned16(q) &&
                      aligned16(k) && aligned16(v) && (reinterpret_cast<uintptr_t>(o) & 7u) == 0;
    if (fast && total_q <= static_cast<int64_t>(PXS_ATTN_WINDOW_MEAN) * nseg) {
        AttnArgs a{};
        a.q = q; a.k = k; a.v = v; a.ldq = ld_q; a.ldk = ld_k; a.ldv = ld_v;
        a.cu_q = cu_q; a.cu_k = cu_k; a.nseg = nseg; a.row_map = row_map;
        a.hd = head_dim; a.vd = value_dim; a.scale_log2 = scale * kLog2e; a.o = o; a.ldo = ld_o;
        if (PXS_ATTN_WINDOW_ORDER && nseg <= kOrderMaxSegments) {
            // the workspace's tile list holds the order (nseg entries)
            int32_t * order = reinterpret_cast<int32_t *>(static_cast<int64_t *>(workspace) + nseg + 1);
            hipLaunchKernelGGL(window_order_kernel, dim3(1), dim3(1024), 0, s, cu_q, cu_k, nseg,
                               32 * PXS_ATTN_WINDOW_WAVES, order);
            if (int rc = check_launch("attention segment order")) return rc;
            a.seg_order = order;
        }
        return launch_attn_window<PXS_ATTN_WINDOW_WAVES>(a, heads, s);
    }
    // Waves per workgroup (32 queries each, sharing the K/V tiles).  The bf16
    // kernel always runs 4: its 4-stage K/V ring takes 64 KB of LDS per
    // workgroup whatever the wave count, so fewer waves only lower occupancy
    // (windows of ~100 rows run 3.6x faster with 4 waves than with 1).  The
    // generic kernel drops to one wave for short segments.
    const int nw = (fast || fast128 || total_q / nseg >= PXS_ATTN_NW4_MIN) ? 4 : 1;
    const int q_tile = 32 * nw;
    int64_t * tile_start = static_cast<int64_t *>(workspace);
    int32_t * tiles = reinterpret_cast<int32_t *>(tile_start + nseg + 1);
    void * scan_ws = reinterpret_cast<void *>(
        (reinterpret_cast<uintptr_t>(tiles + nseg) + 7) & ~uintptr_t(7));
    hipLaunchKernelGGL(attn_tiles_kernel, dim3(grid_for(nseg, 256)), dim3(256), 0, s, cu_q, nseg,
                       q_tile, tiles);
    int rc = exclusive_scan_i32(tiles, tile_start, nseg, tile_start + nseg, scan_ws, s);
    if (rc) return rc;
    AttnArgs a{};
    a.q = q; a.k = k; a.v = v; a.ldq = ld_q; a.ldk = ld_k; a.ldv = ld_v;
    a.cu_q = cu_q; a.cu_k = cu_k; a.nseg = nseg; a.tile_start = tile_start;
    a.row_map = row_map; a.hd = head_dim; a.vd = value_dim;
    a.scale_log2 = scale * kLog2e; a.o = o; a.ldo = ld_o;
    const int vec = dtype == PXS_BF16 ? 8 : 4;
    a.vec_ok = (head_dim % vec == 0) && (value_dim % vec == 0) && (ld_q % vec == 0) && (ld_k % vec == 0) &&
               (ld_v % vec == 0) && aligned16(q) && aligned16(k) && aligned16(v);
    if (dtype == PXS_BF16) {
        if (fast) return launch_attn_bf16<4, 64>(a, total_q, heads, s);
        if (fast128) return launch_attn_bf16<4, 128>(a, total_q, heads, s);
        return nw == 4 ? launch_attn<uint16_t, 4>(a, total_q, heads, s)
                       : launch_attn<uint16_t, 1>(a, total_q, heads, s);
    }
    return nw == 4 ? launch_attn<float, 4>(a, total_q, heads, s)
                   : launch_attn<float, 1>(a, total_q, heads, s);
}

int pxs_varlen_attention_noalloc(int dtype, const void * q, int64_t ld_q, const void * k,
                                 int64_t ld_k, const void * v, int64_t ld_v, const int64_t * cu_q,
                                 const int64_t * cu_k, int nseg, int64_t total_q,
                                 const int32_t * row_map, int heads, int head_dim, int value_dim,
                                 float scale, void * o, int64_t ld_o, void * stream) {
    PXS_CHECK(nseg <= PXS_ATTN_NOALLOC_MAX_SEGMENTS, PXS_ERR_ARG,
              "pxs_varlen_attention_noalloc: more than PXS_ATTN_NOALLOC_MAX_SEGMENTS (65536) "
              "segments; use pxs_varlen_attention with a workspace");
    PXS_CHECK(pxs_attention_workspace_bytes(nseg) <= kNoAllocScratchBytes, PXS_ERR_ARG,
              "pxs_varlen_attention_noalloc: scratch too small for this segment count");
    void * ws = nullptr;
    if (int rc = noalloc_scratch(&ws)) return rc;
    return pxs_varlen_attention(dtype, q, ld_q, k, ld_k, v, ld_v, cu_q, cu_k, nseg, total_q,
                                row_map, heads, head_dim, value_dim, scale, o, ld_o, ws, stream);
}

} // extern "C"
