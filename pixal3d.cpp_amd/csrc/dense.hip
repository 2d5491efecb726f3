// Dense GEMM on MFMA for the plain linears: sparse_linear / varlen_linear
// (src/sparse.cpp:337-488) and the transformer block's gated and residual
// linears (src/sparse_transformer.cpp:229-235), in bf16 or fp32.
//
//   Y[m, n] = sum_k X[m, k] W[n, k] + bias[n]   then one epilogue:
//     store        y[m, n] = act(Y)                 (y in the operands' dtype)
//     add residual r[m, n] = r[m, n] + Y            (r fp32)
//     gate         r[m, n] = r[m, n] + Y * (block_mod[o + n] + time_mod[b(m), o + n])
//
// X rows and W rows are both contiguous along K, so a workgroup's BM x BN
// output tile streams 128-byte K chunks of BM rows of X and BN rows of W
// from L2 into LDS with global_load_lds_dwordx4 (no VGPR staging, no row
// map), two chunks in flight.  The loads use the instruction's scalar-base
// form: the tile's base address advances by 128 bytes per chunk in SGPRs and
// every lane keeps one fixed 32-bit offset per instruction, so the K loop
// issues no vector address arithmetic.  Rows past the end of X or W are
// clamped to the last row (valid memory; their outputs are not stored).
//
// MFMA operands are swapped relative to the output: the W fragment is the
// instruction's A operand and the X fragment its B operand, so D = Y^T per
// 32 x 32 block and lane (h, r) holds output row r, channels 8g + 4h + 0..3
// for g = 0..3: four consecutive channels per lane.
//   bf16: v_mfma_f32_32x32x16_bf16, 4 K steps of 16 per chunk;
//   fp32: v_mfma_f32_32x32x2_f32, 16 K steps of 2 per chunk.
// The K order inside a chunk is permuted identically for both operands so a
// lane reads 16 contiguous bytes per LDS access; pieces are XOR-swizzled by
// row so the 16 rows one LDS cycle serves read 16 different bank groups.
// The fragments of K step u + 1 are read while step u multiplies.
//
// Plain stores go through LDS (each wave's block is written there and read
// back as whole 16-byte row pieces, so a store instruction covers 128-byte
// row segments); the residual forms read, add and write 4 channels per lane.
// Tile shapes (measured on MI355X against hipBLASLt's 256 x 256 kernels on
// the flow block's, the window workload's and the decoder's shapes):
//   256 x 256, 16 waves of 64 x 64, each wave issuing its share of the next
//     chunk's DMA one part per K step (one instruction burst per chunk left
//     the vector-memory return path idle between chunks);
//   128 x 128, 8 waves of 64 x 32 (two workgroups per CU);
//   128 x 64, 4 waves of 64 x 32 (three workgroups per CU; 64 outputs);
// chosen per shape by the number of rounds of tiles over the 256 CUs.

#include "pxs_common.h"

namespace pxs {
namespace {

enum DenseEpi { kDenseStore = 0, kDenseAddResidual = 1, kDenseGate = 2 };

struct DenseArgs {
    const void * x;        // [m, k]
    const void * w;        // [n, k]
    const float * bias;    // [n] or null
    int64_t m;
    int k;
    int n;
    void * y;              // [m, n], store epilogue
    int act;
    float * residual;      // [m, n] fp32, residual epilogues
    const int32_t * coords;      // [m, 4], gate epilogue: batch of each row
    const float * block_mod;     // gate = block_mod[gate_offset + c] + time_mod[b, gate_offset + c]
    const float * time_mod;      // [batch, 6 n]
    int gate_offset;
    int vec_out;           // 1: 4-channel vector accesses; 2: also whole 16-byte row pieces
    int group_m;           // tile order: groups of group_m row tiles, each walked down its rows first
};

// Output tile (row tile, column tile) of logical tile t: groups of g row
// tiles share their column tiles, and inside a group consecutive t walk the
// rows, so the tiles one XCD runs at a time cover g row tiles x (32 / g)
// column tiles of operands instead of one row tile x every column tile.
__device__ __forceinline__ void tile_of(int t, int tiles_m, int tiles_n, int g, int & tm, int & tn) {
    if (g <= 1) {
        tm = t / tiles_n;
        tn = t % tiles_n;
        return;
    }
    const int per_group = g * tiles_n;
    const int grp = t / per_group, in = t % per_group;
    const int rows = min(g, tiles_m - grp * g);  // the last group may be short
    tm = grp * g + in % rows;
    tn = in / rows;
}

__device__ __align__(16) uint4 g_dense_zero[8];  // 128 zero bytes: K pieces past the end

template <typename T> struct Store4;
template <> struct Store4<uint16_t> {
    static __device__ __forceinline__ void put(uint16_t * p, const float (&v)[4]) {
        uint2 u;
        u.x = pack_bf16x2(v[0], v[1]);
        u.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2 *>(p) = u;
    }
};
template <> struct Store4<float> {
    static __device__ __forceinline__ void put(float * p, const float (&v)[4]) {
        *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
    }
};

// Epilogue of one wave: acc[i][j] is the 32 x 32 block (rows i, channels j);
// lane (h, r) holds row r and channels 8 g + 4 h + e at acc[i][j][4 g + e].
// The per-element arithmetic is the gather-GEMM epilogue's (value = acc +
// bias, then the activation; residual + value; residual + value * gate).
template <typename T, int TI, int TJ, int EPI>
__device__ __forceinline__ void dense_epilogue(const DenseArgs & a, const f32x16 (&acc)[TI][TJ],
                                               int64_t row0, int col0, int h, int r) {
#pragma unroll
    for (int i = 0; i < TI; ++i) {
        const int64_t row = row0 + i * 32 + r;
        if (row >= a.m) continue;
        int batch = 0;
        if constexpr (EPI == kDenseGate) batch = a.coords[row * 4];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = col0 + j * 32 + 8 * g + 4 * h;
                if (c >= a.n) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e];
                if (a.vec_out && c + 3 < a.n) {
                    if (a.bias) {
                        const float4 b = *reinterpret_cast<const float4 *>(a.bias + c);
                        v[0] = v[0] + b.x; v[1] = v[1] + b.y; v[2] = v[2] + b.z; v[3] = v[3] + b.w;
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] = v[e] + 0.0f;
                    }
                    if constexpr (EPI == kDenseStore) {
                        if (a.act == PXS_ACT_GELU_TANH) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = gelu_tanh_f(v[e]);
                        } else if (a.act == PXS_ACT_SILU) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] = silu_f(v[e]);
                        }
                        Store4<T>::put(static_cast<T *>(a.y) + row * a.n + c, v);
                    } else if constexpr (EPI == kDenseAddResidual) {
                        float4 * res = reinterpret_cast<float4 *>(a.residual + row * a.n + c);
                        float4 o = *res;
                        o.x = o.x + v[0]; o.y = o.y + v[1]; o.z = o.z + v[2]; o.w = o.w + v[3];
                        *res = o;
                    } else {
                        const float4 bm = *reinterpret_cast<const float4 *>(a.block_mod + a.gate_offset + c);
                        const float4 tm = *reinterpret_cast<const float4 *>(
                            a.time_mod + static_cast<int64_t>(batch) * 6 * a.n + a.gate_offset + c);
                        float4 * res = reinterpret_cast<float4 *>(a.residual + row * a.n + c);
                        float4 o = *res;
                        o.x = o.x + v[0] * (bm.x + tm.x);
                        o.y = o.y + v[1] * (bm.y + tm.y);
                        o.z = o.z + v[2] * (bm.z + tm.z);
                        o.w = o.w + v[3] * (bm.w + tm.w);
                        *res = o;
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int ce = c + e;
                        if (ce >= a.n) break;
                        float val = v[e] + (a.bias ? a.bias[ce] : 0.0f);
                        if constexpr (EPI == kDenseStore) {
                            if (a.act == PXS_ACT_GELU_TANH) val = gelu_tanh_f(val);
                            else if (a.act == PXS_ACT_SILU) val = silu_f(val);
                            store_f32(static_cast<T *>(a.y) + row * a.n + ce, val);
                        } else if constexpr (EPI == kDenseAddResidual) {
                            float * res = a.residual + row * a.n + ce;
                            *res = *res + val;
                        } else {
                            const float gate = a.block_mod[a.gate_offset + ce] +
                                               a.time_mod[static_cast<int64_t>(batch) * 6 * a.n +
                                                          a.gate_offset + ce];
                            float * res = a.residual + row * a.n + ce;
                            *res = *res + val * gate;
                        }
                    }
                }
            }
        }
    }
}

// Row pitch in LDS of a wave's block in the staged store epilogue: 16 bytes
// of padding keep the 32 rows one fragment write covers on distinct banks
// (two-way at most).
template <typename T, int WN> constexpr int staged_pitch() { return WN * static_cast<int>(sizeof(T)) + 16; }

// Store epilogue through LDS: each wave writes its WM x WN block (bias and
// activation applied, rounded to T) into its own LDS region, then reads it
// back row by row, 16 contiguous bytes per lane, so every store instruction
// covers whole 128-byte row segments instead of 16 bytes in each of 32 rows.
// Same per-element arithmetic as dense_epilogue.  Needs n a multiple of 16 /
// sizeof(T) and y 16-byte aligned (vec_out with that n).
template <typename T, int TI, int TJ>
__device__ __forceinline__ void dense_store_staged(const DenseArgs & a, const f32x16 (&acc)[TI][TJ],
                                                   char * region, int64_t row0, int col0, int h,
                                                   int r, int lane) {
    constexpr int WM = TI * 32, WN = TJ * 32;
    constexpr int kPitch = staged_pitch<T, WN>();
    constexpr int kRowBytes = WN * static_cast<int>(sizeof(T));
    constexpr int kLanesPerRow = kRowBytes / 16;
    constexpr int kRowsPerPass = 64 / kLanesPerRow;
    constexpr int kElems = 16 / static_cast<int>(sizeof(T));
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int cl = j * 32 + 8 * g + 4 * h;  // column inside the block
            const int c = col0 + cl;
            float b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (a.bias && c < a.n) {
                const float4 bv = *reinterpret_cast<const float4 *>(a.bias + c);
                b[0] = bv.x; b[1] = bv.y; b[2] = bv.z; b[3] = bv.w;
            }
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = acc[i][j][4 * g + e] + b[e];
                    if (a.act == PXS_ACT_GELU_TANH) v[e] = gelu_tanh_f(v[e]);
                    else if (a.act == PXS_ACT_SILU) v[e] = silu_f(v[e]);
                }
                Store4<T>::put(reinterpret_cast<T *>(region + (i * 32 + r) * kPitch + cl * sizeof(T)), v);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave's own writes are in LDS
    const int lr = lane / kLanesPerRow, lc = lane % kLanesPerRow;
#pragma unroll
    for (int pass = 0; pass < WM / kRowsPerPass; ++pass) {
        const int rl = pass * kRowsPerPass + lr;
        const int64_t row = row0 + rl;
        const uint4 v = *reinterpret_cast<const uint4 *>(region + rl * kPitch + lc * 16);
        const int c = col0 + lc * kElems;
        if (row < a.m && c < a.n)
            *reinterpret_cast<uint4 *>(static_cast<T *>(a.y) + row * a.n + c) = v;
    }
}

// Rows of KB = 128 bytes per K chunk in LDS: 8 pieces of 16 bytes,
// XOR-swizzled by row so that the 16 rows one LDS cycle serves (64 banks of
// 4 bytes) read 16 different bank groups.
template <int KB> __device__ __forceinline__ int piece_swz(int row);
template <> __device__ __forceinline__ int piece_swz<128>(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// NW waves in a WAVES_M x (NW / WAVES_M) grid, each owning a (BM / WAVES_M) x
// (BN / WAVES_N) block of the tile; NSTAGE K chunks of KB bytes per row in
// flight (one DMA instruction fills 1 KiB: 1024 / KB rows).
template <typename T, int BM, int BN, int NW, int WAVES_M, int NSTAGE, int KB, int EPI, bool SPREAD,
          bool STAGED>
__global__ void __launch_bounds__(NW * 64)
dense_gemm_kernel(DenseArgs a) {
    constexpr int kVec = 16 / static_cast<int>(sizeof(T));  // elements per piece
    constexpr int P = KB / 16;                              // pieces per chunk row
    constexpr int kChunk = P * kVec;                        // elements per chunk row
    constexpr int RPI = 1024 / KB;                          // rows per DMA instruction
    constexpr int WAVES_N = NW / WAVES_M;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int TI = WM / 32, TJ = WN / 32;
    static_assert(TI * 32 * WAVES_M == BM && TJ * 32 * WAVES_N == BN, "wave blocks must tile");
    constexpr int kStage = (BM + BN) * KB;
    constexpr int AI = BM / (RPI * NW);  // DMA instructions per wave per stage
    constexpr int BI = BN / (RPI * NW);
    static_assert(AI * RPI * NW == BM && BI * RPI * NW == BN, "tile rows must split over the waves");
    constexpr int kPerStage = AI + BI;

    extern __shared__ __align__(16) char smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int h = lane >> 5, r = lane & 31;

    const int tiles_n = (a.n + BN - 1) / BN;
    const int tiles_m = static_cast<int>((a.m + BM - 1) / BM);
    const int logical = remap_xcd(blockIdx.x, gridDim.x);
    int tm, tn;
    tile_of(logical, tiles_m, tiles_n, a.group_m, tm, tn);
    const int64_t p0 = static_cast<int64_t>(tm) * BM;
    const int n0 = tn * BN;

    const char * xs = static_cast<const char *>(a.x) + p0 * a.k * static_cast<int64_t>(sizeof(T));
    const char * wsb = static_cast<const char *>(a.w) + static_cast<int64_t>(n0) * a.k * sizeof(T);
    const int stages = (a.k + kChunk - 1) / kChunk;
    const bool ragged = a.k % kChunk != 0;  // the last chunk holds pieces past k
    // Fixed per-lane parts of the loads: row lane / P of each instruction,
    // clamped into the operand, and the swizzled piece it fetches.
    const int lrow = lane / P, lslot = lane % P;
    const int64_t last_x = a.m - 1 - p0;
    const int last_w = a.n - 1 - n0;
    uint32_t a_off[AI], b_off[BI];
#pragma unroll
    for (int j = 0; j < AI; ++j) {
        const int row = (wave * AI + j) * RPI + lrow;
        const int64_t rr = row < last_x ? row : last_x;
        a_off[j] = static_cast<uint32_t>(rr * a.k * static_cast<int64_t>(sizeof(T)) +
                                         (lslot ^ piece_swz<KB>(row)) * 16);
    }
#pragma unroll
    for (int j = 0; j < BI; ++j) {
        const int row = (wave * BI + j) * RPI + lrow;
        const int rr = row < last_w ? row : last_w;
        b_off[j] = static_cast<uint32_t>(static_cast<int64_t>(rr) * a.k * sizeof(T) +
                                         (lslot ^ piece_swz<KB>(row)) * 16);
    }

    // DMA instruction q of stage s: q < AI fills X rows, the rest W rows.
    auto issue_one = [&](int s, int q) __attribute__((always_inline)) {
        char * base = smem + (s % NSTAGE) * kStage;
        const int64_t kb = static_cast<int64_t>(s) * KB;
        const bool is_x = q < AI;
        const int j = is_x ? q : q - AI;
        const int row = (wave * (is_x ? AI : BI) + j) * RPI + lrow;
        const uint32_t lds = lds_offset(base + ((is_x ? 0 : BM) + (wave * (is_x ? AI : BI) + j) * RPI) * KB);
        const char * src = is_x ? xs : wsb;
        const uint32_t off = is_x ? a_off[j] : b_off[j];
        if (ragged && s == stages - 1) {
            // Pieces past k come from the zero line.
            const bool in = s * kChunk + (lslot ^ piece_swz<KB>(row)) * kVec < a.k;
            lds_dma16(in ? static_cast<const void *>(src + kb + off) : static_cast<const void *>(g_dense_zero), lds);
        } else {
            lds_dma16_sbase(src + kb, off, lds);
        }
    };
    auto issue = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < kPerStage; ++q) issue_one(s, q);
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
        const bool more = s + NSTAGE - 1 < stages;
        if (!SPREAD && more) issue(s + NSTAGE - 1);
        const char * sx = smem + (s % NSTAGE) * kStage;
        const char * sw = sx + BM * KB;
        // Half h of the wave's lanes reads pieces (P / 2) h .. (P / 2) h + P / 2 - 1;
        // the fragments of K step u + 1 are read while step u multiplies.
        uint4 xr[2][TI], wr[2][TJ];
        auto read_frags = [&](int u, uint4 (&xo)[TI], uint4 (&wo)[TJ]) __attribute__((always_inline)) {
            const int piece = (P / 2) * h + u;
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const int row = wm * WM + i * 32 + r;
                xo[i] = *reinterpret_cast<const uint4 *>(sx + row * KB + ((piece ^ piece_swz<KB>(row)) << 4));
            }
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const int row = wn * WN + j * 32 + r;
                wo[j] = *reinterpret_cast<const uint4 *>(sw + row * KB + ((piece ^ piece_swz<KB>(row)) << 4));
            }
        };
        read_frags(0, xr[0], wr[0]);
#pragma unroll
        for (int u = 0; u < P / 2; ++u) {
            if constexpr (SPREAD) {
                // The next stage's DMA in P / 2 parts, one per K step.
#pragma unroll
                for (int q = 0; q < kPerStage; ++q)
                    if (more && q * (P / 2) / kPerStage == u) issue_one(s + NSTAGE - 1, q);
            }
            if (u + 1 < P / 2) read_frags(u + 1, xr[(u + 1) & 1], wr[(u + 1) & 1]);
            const uint4 (&xc)[TI] = xr[u & 1];
            const uint4 (&wc)[TJ] = wr[u & 1];
            if constexpr (sizeof(T) == 2) {
#pragma unroll
                for (int i = 0; i < TI; ++i)
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, wc[j]), __builtin_bit_cast(bf16x8, xc[i]),
                            acc[i][j], 0, 0, 0);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int i = 0; i < TI; ++i)
#pragma unroll
                        for (int j = 0; j < TJ; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                                __builtin_bit_cast(f32x4, wc[j])[e], __builtin_bit_cast(f32x4, xc[i])[e],
                                acc[i][j], 0, 0, 0);
            }
        }
    }
    if constexpr (STAGED && EPI == kDenseStore) {
        if (a.vec_out == 2) {
            barrier_no_fence();  // every wave is done with the stage buffers
            dense_store_staged<T, TI, TJ>(a, acc, smem + wave * WM * staged_pitch<T, WN>(), p0 + wm * WM,
                                          n0 + wn * WN, h, r, lane);
            return;
        }
    }
    dense_epilogue<T, TI, TJ, EPI>(a, acc, p0 + wm * WM, n0 + wn * WN, h, r);
}

template <typename T, int BM, int BN, int NW, int WAVES_M, int NSTAGE, int KB, int EPI,
          bool SPREAD, bool STAGED>
int launch_dense(const DenseArgs & a, hipStream_t stream) {
    constexpr int kStage = (BM + BN) * KB;
    constexpr int kChunk = KB / static_cast<int>(sizeof(T));
    constexpr int WN = BN / (NW / WAVES_M);
    constexpr int kStagedBytes = STAGED && EPI == kDenseStore ? NW * (BM / WAVES_M) * staged_pitch<T, WN>() : 0;
    constexpr int kMaxSmem = NSTAGE * kStage > kStagedBytes ? NSTAGE * kStage : kStagedBytes;
    static_assert(kMaxSmem <= 160 * 1024, "LDS");
    auto kernel = &dense_gemm_kernel<T, BM, BN, NW, WAVES_M, NSTAGE, KB, EPI, SPREAD, STAGED>;
    static bool configured = false;
    if (!configured) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, kMaxSmem);
        if (e != hipSuccess) return check_hip(e, "hipFuncSetAttribute(dense_gemm)");
        configured = true;
    }
    const int stages = (a.k + kChunk - 1) / kChunk;
    int smem = (stages < NSTAGE ? stages : NSTAGE) * kStage;
    if (a.vec_out == 2 && smem < kStagedBytes) smem = kStagedBytes;
    const int64_t blocks = ((a.m + BM - 1) / BM) * ((a.n + BN - 1) / BN);
    if (blocks > INT32_MAX) return fail(PXS_ERR_ARG, "dense GEMM grid too large");
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(NW * 64), smem, stream, a);
    return check_launch("dense GEMM");
}

// Tile shape by the estimated time of the whole grid: rounds of tiles over
// the 256 CUs (workgroups resident per CU in parallel) times the time of one
// round, from each shape's measured rate (bf16: 256 x 256 tiles about 1000
// TFLOP/s, 128 x 128 about 880, 128 x 64 about 700; fp32: 128 x 128 about
// 130, 128 x 64 about 128).  256 x 256 tiles go down 8-row-tile groups, the
// others down groups of 16 when a row holds at most 4 column tiles, else 8.
template <typename T, int EPI>
int dispatch_dense(DenseArgs a, hipStream_t s) {
    constexpr bool bf16 = sizeof(T) == 2;
    auto rounds = [&](int bm, int bn, int per_cu) {
        const int64_t tiles = ((a.m + bm - 1) / bm) * ((a.n + bn - 1) / bn);
        return static_cast<double>((tiles + 256 * per_cu - 1) / (256 * per_cu));
    };
    const double t_b = rounds(128, 128, 2) * 2.0 * 128 * 128 / (bf16 ? 880.0 : 130.0);
    const double t_c = rounds(128, 64, 3) * 3.0 * 128 * 64 / (bf16 ? 700.0 : 128.0);
    if constexpr (bf16) {
        const double t_a = rounds(256, 256, 1) * 256.0 * 256 / 1000.0;
        if (a.n > 128 && t_a <= t_b) {
            a.group_m = 8;
            return launch_dense<T, 256, 256, 16, 4, 2, 128, EPI, true, true>(a, s);
        }
    }
    if (a.n <= 64 || t_c < t_b) {
        a.group_m = (a.n + 63) / 64 <= 4 ? 16 : 8;
        return launch_dense<T, 128, 64, 4, 2, 2, 128, EPI, false, true>(a, s);
    }
    a.group_m = (a.n + 127) / 128 <= 4 ? 16 : 8;
    return launch_dense<T, 128, 128, 8, 2, 2, 128, EPI, false, true>(a, s);
}

bool aligned_to(const void * p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// Common checks; false when the kernel does not take the shape (rows of X or
// W not whole 16-byte pieces, or operands not 16-byte aligned).
bool dense_takes(int dtype, const void * x, int cin, const void * w) {
    const int vec = dtype == PXS_BF16 ? 8 : 4;
    return (dtype == PXS_BF16 || dtype == PXS_F32) && cin % vec == 0 && aligned_to(x, 16) &&
           aligned_to(w, 16);
}

template <int EPI>
int run_dense(int dtype, const DenseArgs & a, hipStream_t s) {
    return dtype == PXS_BF16 ? dispatch_dense<uint16_t, EPI>(a, s) : dispatch_dense<float, EPI>(a, s);
}

} // namespace

int dense_linear(int dtype, const void * x, int64_t rows, int cin, const void * w,
                 const float * bias, int cout, int act, void * y, hipStream_t s, bool * done) {
    *done = false;
    if (!dense_takes(dtype, x, cin, w)) return PXS_OK;
    DenseArgs a{};
    a.x = x; a.w = w; a.bias = bias; a.m = rows; a.k = cin; a.n = cout; a.y = y; a.act = act;
    a.vec_out = cout % 4 == 0 && aligned_to(y, dtype == PXS_BF16 ? 8 : 16) &&
                (!bias || aligned_to(bias, 16));
    // Whole 16-byte pieces of output rows: the store goes through LDS.
    if (a.vec_out && cout % (dtype == PXS_BF16 ? 8 : 4) == 0 && aligned_to(y, 16)) a.vec_out = 2;
    *done = true;
    return run_dense<kDenseStore>(dtype, a, s);
}

int dense_linear_residual(int dtype, const void * x, int64_t rows, int cin, const void * w,
                          const float * bias, int cout, float * residual, hipStream_t s,
                          bool * done) {
    *done = false;
    if (!dense_takes(dtype, x, cin, w)) return PXS_OK;
    DenseArgs a{};
    a.x = x; a.w = w; a.bias = bias; a.m = rows; a.k = cin; a.n = cout; a.residual = residual;
    a.vec_out = cout % 4 == 0 && aligned_to(residual, 16) && (!bias || aligned_to(bias, 16));
    *done = true;
    return run_dense<kDenseAddResidual>(dtype, a, s);
}

int dense_linear_gate(int dtype, const void * x, int64_t rows, int cin, const void * w,
                      const float * bias, int cout, const int32_t * coords,
                      const float * block_mod, const float * time_mod, int gate_offset,
                      float * residual, hipStream_t s, bool * done) {
    *done = false;
    if (!dense_takes(dtype, x, cin, w)) return PXS_OK;
    DenseArgs a{};
    a.x = x; a.w = w; a.bias = bias; a.m = rows; a.k = cin; a.n = cout; a.residual = residual;
    a.coords = coords; a.block_mod = block_mod; a.time_mod = time_mod; a.gate_offset = gate_offset;
    a.vec_out = cout % 4 == 0 && gate_offset % 4 == 0 && aligned_to(residual, 16) &&
                (!bias || aligned_to(bias, 16)) && aligned_to(block_mod, 16) &&
                aligned_to(time_mod, 16);
    *done = true;
    return run_dense<kDenseGate>(dtype, a, s);
}

} // namespace pxs
