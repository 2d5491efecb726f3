// Stride-2 topology emit from a generation-tagged occupancy bitmap, shared by
// the standalone emit kernel (topology.hip) and the side workgroups that carry
// the emit inside a SubMConv3d launch (gemm.hip).
//
// The coarse cell of fine voxel (b, x, y, z) is (b, x/2, y/2, z/2), linearised
// ((b*cx + X)*cy + Y)*cz + Z.  That order is lexicographic, so ranking the
// occupied cells by a popcount prefix over the bitmap gives the coarse rows in
// the order the reference sorts them (src/sparse.cpp:575-593); child
// c = (x&1) + 2(y&1) + 4(z&1) (src/sparse.cpp:682-686).
#pragma once

#include "pxs_common.h"

namespace pxs {

// The occupancy bitmap of the fused form is a pair of plain bitmaps used by
// generation parity: the build of generation g marks bitmap g & 1, and its
// emit clears bitmap (g + 1) & 1, which the build before it used and which
// the next build marks.  No workgroup clears a bitmap another may still be
// reading, and no pass of its own clears either.  Successive builds on one
// workspace therefore use successive generations, and the workspace is reset
// when the generations start again (as the tagged voxel grid is).
struct S2EmitArgs {
    const uint32_t * bits;       // occupancy words of this generation's bitmap
    uint32_t * clear_bits;       // the other bitmap, cleared word range by word range
    int64_t words, cells;        // words = ceil(cells / 32)
    int b, fx, fy, fz;           // fine extents (batch, x, y, z)
    int cx, cy, cz;              // coarse extents
    const uint32_t * fine_grid;  // the generation-tagged fine voxel grid
    uint32_t generation;         // of both the fine grid and the bitmap
    int32_t * coarse_grid;       // dense coarse grid: rank or kVoxelGridEmpty per cell
    int4 * out_coords;
    int32_t * child_map;         // [8, ld_map]
    int64_t ld_map;
    int64_t * m_out;
    int blocks;                  // workgroups sharing the emit
    int words_per_block;         // a multiple of 4, at most the workgroup's thread count
    int coherent_children;       // child map stored device-coherently (read in the same launch)
};

// The emit's arguments over a workspace of pxs_downsample_s2_tagged_workspace_bytes
// (the bitmap pair is its last region); blocks = the workgroups for
// words_per_block words each, rounded up to a multiple of 8.
S2EmitArgs make_s2_emit_args(int batch_size, int sx, int sy, int sz, const void * fine_grid,
                             uint32_t generation, int32_t * out_coords, int32_t * child_map,
                             int64_t ld_map, int64_t * m_out, void * coarse_grid,
                             void * s2_workspace, int words_per_block);

// Bitmap words per emit workgroup when the emit rides in a convolution's
// launch (1,024 cells: short workgroups that fill the launch's tail).
constexpr int kS2SideWords = 32;

// The flags of the chained U-Net level (pxs_unet_s2_level) in the same
// workspace: one per emit workgroup and one per row tile of the first
// convolution, each set to the generation when its results are visible.
struct S2ChainFlags {
    uint32_t * emit;
    int64_t emit_cap;
    uint32_t * tiles;
    int64_t tiles_cap;
    uint32_t * error;  // nonzero once a dependency wait gave up (cleared by the reset)
};
S2ChainFlags s2_chain_flags(void * s2_workspace, int batch_size, int sx, int sy, int sz);

// Bytes of LDS s2_emit_block needs.
constexpr int s2_emit_lds_bytes(int words_per_block, int threads) {
    return words_per_block * 8 + (threads / 64) * 12 + 16;
}

// One coarse cell: its dense grid entry and, if occupied, its coordinate and
// its 8 children looked up in the fine grid (-1 when absent).
__device__ __forceinline__ void s2_emit_cell(const S2EmitArgs & e, int64_t cell, bool occupied,
                                             int64_t rank) {
    if (cell >= e.cells) return;
    e.coarse_grid[cell] = occupied ? static_cast<int32_t>(rank)
                                   : static_cast<int32_t>(kVoxelGridEmpty);
    // (a rank past the child map's stride only comes from a bitmap holding
    // another build of the same generation: nothing is written for it)
    if (!occupied || rank >= e.ld_map) return;
    const int64_t per_item = static_cast<int64_t>(e.cx) * e.cy * e.cz;
    const int b = static_cast<int>(cell / per_item);
    int64_t rem = cell - static_cast<int64_t>(b) * per_item;
    const int X = static_cast<int>(rem / (static_cast<int64_t>(e.cy) * e.cz));
    rem -= static_cast<int64_t>(X) * e.cy * e.cz;
    const int Y = static_cast<int>(rem / e.cz);
    const int Z = static_cast<int>(rem - static_cast<int64_t>(Y) * e.cz);
    e.out_coords[rank] = make_int4(b, X, Y, Z);
    int32_t child[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int x = 2 * X + (c & 1), y = 2 * Y + ((c >> 1) & 1), z = 2 * Z + (c >> 2);
        child[c] = -1;
        if (x < e.fx && y < e.fy && z < e.fz) {
            const int64_t f = ((static_cast<int64_t>(b) * e.fx + x) * e.fy + y) * e.fz + z;
            child[c] = voxel_grid_row(e.fine_grid[f], e.generation);
        }
    }
    if (e.coherent_children) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
            __hip_atomic_store(e.child_map + c * e.ld_map + rank, child[c], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) e.child_map[c * e.ld_map + rank] = child[c];
    }
}

// Workgroup sb of e.blocks emits the cells of bitmap words [w0, w1),
// w0 = sb * words_per_block.  Its first rank is the popcount of all words
// before w0, which it sums itself, so no workgroup waits for another.  The
// workgroup holding the last word writes *m_out.  Called by every thread of
// the workgroup (it synchronises the workgroup); lds holds
// s2_emit_lds_bytes(words_per_block, nthreads) bytes.
__device__ __forceinline__ void s2_emit_block(const S2EmitArgs & e, int sb, int tid, int nthreads,
                                              char * lds) {
    uint32_t * bits = reinterpret_cast<uint32_t *>(lds);
    int32_t * pre = reinterpret_cast<int32_t *>(lds + 4 * e.words_per_block);
    int64_t * wave_base = reinterpret_cast<int64_t *>(lds + 8 * e.words_per_block);
    int32_t * wave_own = reinterpret_cast<int32_t *>(lds + 8 * e.words_per_block + 8 * (nthreads / 64));
    const int lane = tid & 63, wave = tid >> 6, nw = nthreads / 64;
    const int64_t w0 = static_cast<int64_t>(sb) * e.words_per_block;
    if (w0 >= e.words) return;  // workgroup-uniform: nothing to emit
    const int L = static_cast<int>(e.words - w0 < e.words_per_block ? e.words - w0
                                                                     : e.words_per_block);
    // The words before w0 in 16-byte pieces (w0 is a multiple of
    // words_per_block, itself a multiple of 4; the bitmap is 256-byte
    // aligned), all of a thread's loads issued before their sums.
    int64_t before = 0;
    const uint4 * q4 = reinterpret_cast<const uint4 *>(e.bits);
#pragma unroll 4
    for (int64_t q = tid; q < w0 / 4; q += nthreads) {
        const uint4 v = q4[q];
        before += __popc(v.x) + __popc(v.y) + __popc(v.z) + __popc(v.w);
    }
    const uint32_t mine_bits = tid < L ? e.bits[w0 + tid] : 0u;
    if (tid < L) {
        bits[tid] = mine_bits;
        e.clear_bits[w0 + tid] = 0u;
    }
    const int32_t mine = __popc(mine_bits);
    int32_t inc = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t o = __shfl_up(inc, d, 64);
        if (lane >= d) inc += o;
        before += __shfl_xor(before, d, 64);
    }
    if (lane == 63) wave_own[wave] = inc;
    if (lane == 0) wave_base[wave] = before;
    __syncthreads();
    int64_t base = 0;
    int32_t own_before = 0, own_total = 0;
    for (int w = 0; w < nw; ++w) {
        base += wave_base[w];
        if (w < wave) own_before += wave_own[w];
        own_total += wave_own[w];
    }
    if (tid < L) pre[tid] = own_before + inc - mine;
    if (tid == 0 && w0 + L == e.words) *e.m_out = base + own_total;
    __syncthreads();
    const int64_t c_end = (w0 + L) * 32;
    for (int64_t cell = w0 * 32 + tid; cell < c_end; cell += nthreads) {
        const int i = static_cast<int>((cell >> 5) - w0);
        const uint32_t wb = bits[i];
        const int bit = static_cast<int>(cell & 31);
        s2_emit_cell(e, cell, (wb >> bit) & 1u, base + pre[i] + __popc(wb & ((1u << bit) - 1u)));
    }
}

}  // namespace pxs
