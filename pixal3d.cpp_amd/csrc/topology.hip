// Integer/topology kernels: voxel hash, validation, neighbor maps, pair lists,
// stride-2 topology, window partition, cu_seqlens, channel-to-spatial.
//
// All of these are HBM/latency-bound integer work; they are written for
// coalesced row-parallel access (one thread per voxel row, offset-major
// outputs so a wavefront writes 64 consecutive entries of one offset).

#include "pxs_common.h"
#include "s2emit.h"
#include "scan.h"

#include <algorithm>
#include <climits>

namespace pxs {
namespace {

constexpr int kThreads = 256;

// Slots: the next power of two >= PXS_HASH_LOAD_INV * n (load <= 1/that).
// Measured on MI355X (162k and 32k voxels): load 1/4 with plain mix64 homes
// halves the neighbor-map time against load 1/2, and grouping consecutive z
// into shared slot groups loses (shell surfaces have short z runs, so groups
// mostly add collisions).
#ifndef PXS_HASH_LOAD_INV
#define PXS_HASH_LOAD_INV 4
#endif
int64_t hash_capacity(int64_t n) {
    int64_t cap = 64;
    while (cap < PXS_HASH_LOAD_INV * n) cap <<= 1;
    return cap;
}

// A slot holds the packed key and the owning row in one 16-byte line piece,
// so a probe is a single 16-byte load.
struct __align__(16) HashSlot {
    unsigned long long key;
    int32_t val;
    int32_t pad;
};

struct HashView {
    HashSlot * slots;
    uint64_t mask;
};

HashView hash_view(void * table, int64_t n) {
    HashView h;
    h.slots = static_cast<HashSlot *>(table);
    h.mask = static_cast<uint64_t>(hash_capacity(n) - 1);
    return h;
}

#ifndef PXS_HASH_GROUP_BITS
#define PXS_HASH_GROUP_BITS 0
#endif
// Home slot.  With G = PXS_HASH_GROUP_BITS > 0, the 2^G voxels that differ
// only in the low G bits of z share 2^G consecutive slots.
__device__ __forceinline__ uint64_t home_slot(uint64_t key, uint64_t mask) {
    constexpr int G = PXS_HASH_GROUP_BITS;
    if constexpr (G == 0) return mix64(key) & mask;
    return ((mix64(key >> G) << G) | (key & ((1u << G) - 1))) & mask;
}

__device__ __forceinline__ HashSlot load_slot(const HashSlot * slots, uint64_t i) {
    const uint4 v = *reinterpret_cast<const uint4 *>(slots + i);
    HashSlot s;
    s.key = static_cast<unsigned long long>(v.x) | (static_cast<unsigned long long>(v.y) << 32);
    s.val = static_cast<int32_t>(v.z);
    s.pad = 0;
    return s;
}

// Linear probing from the home slot; the table has at least 2n slots, so
// every probe sequence meets an empty slot.
__device__ __forceinline__ int32_t probe_from(const HashSlot * __restrict__ slots, uint64_t mask,
                                              uint64_t key, uint64_t slot, HashSlot s) {
    for (uint64_t probe = 0; probe <= mask; ++probe) {
        if (s.key == key) return s.val;
        if (s.key == kEmptyKey) return -1;
        slot = (slot + 1) & mask;
        s = load_slot(slots, slot);
    }
    return -1;
}

__device__ __forceinline__ int32_t hash_find(const HashSlot * __restrict__ slots, uint64_t mask,
                                             uint64_t key) {
    const uint64_t slot = home_slot(key, mask);
    return probe_from(slots, mask, key, slot, load_slot(slots, slot));
}

__global__ void hash_init_kernel(HashSlot * slots, int64_t cap, int32_t * counters = nullptr,
                                 int ncounters = 0) {
    // (counters: the brick table's, zeroed in the same launch)
    if (counters && blockIdx.x == 0 && static_cast<int>(threadIdx.x) < ncounters) counters[threadIdx.x] = 0;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < cap;
         i += stride) {
        *reinterpret_cast<uint4 *>(slots + i) = make_uint4(0xFFFFFFFFu, 0xFFFFFFFFu, INT_MAX, 0u);
    }
}

// Lock-free insert: claim a slot with a 64-bit CAS (or find the key already
// there), then keep the smallest inserting row with atomicMin.
__global__ void hash_insert_kernel(const int4 * __restrict__ coords, int64_t n, HashSlot * slots,
                                   uint64_t mask) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    const uint64_t key = voxel_key(c.x, c.y, c.z, c.w);
    uint64_t slot = home_slot(key, mask);
    for (uint64_t probe = 0; probe <= mask; ++probe) {
        const unsigned long long prev = atomicCAS(&slots[slot].key,
                                                  static_cast<unsigned long long>(kEmptyKey),
                                                  static_cast<unsigned long long>(key));
        if (prev == kEmptyKey || prev == key) {
            atomicMin(&slots[slot].val, static_cast<int32_t>(p));
            return;
        }
        slot = (slot + 1) & mask;
    }
}

__global__ void status_init_kernel(int64_t * status) { *status = LLONG_MAX; }

// Row checks in the reference's order at one row: outside shape (4),
// duplicate (5: a smaller row owns the key), not contiguous by batch (6).
__global__ void validate_coords_kernel(const int4 * __restrict__ coords, int64_t n,
                                       int batch_size, int sx, int sy, int sz,
                                       const HashSlot * __restrict__ slots, uint64_t mask,
                                       int64_t * status) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    int code = 0;
    if (c.x < 0 || c.x >= batch_size || c.y < 0 || c.y >= sx || c.z < 0 || c.z >= sy ||
        c.w < 0 || c.w >= sz) {
        code = 4;
    } else if (hash_find(slots, mask, voxel_key(c.x, c.y, c.z, c.w)) !=
               static_cast<int32_t>(p)) {
        code = 5;
    } else if (p > 0 && coords[p - 1].x > c.x) {
        code = 6;
    }
    if (code) {
        atomicMin(reinterpret_cast<unsigned long long *>(status),
                  static_cast<unsigned long long>(p * 8 + code));
    }
}

template <typename T>
__global__ void validate_feats_kernel(const T * __restrict__ feats, int64_t count, int channels,
                                      int64_t * status) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        const float v = load_f32(feats + i);
        if (!isfinite(v)) {
            atomicMin(reinterpret_cast<unsigned long long *>(status),
                      static_cast<unsigned long long>((i / channels) * 8 + 7));
        }
    }
}

// One thread per (row, kd): the 9 neighbours with that x offset.  All 9 home
// slots are loaded before any is resolved, so a thread keeps 9 probes in
// flight; the rare collision chains are walked afterwards.  Thread index
// kd * n + p writes nbr[(9 kd + 3 kh + kw) * n + p], so a wavefront's stores of
// one offset are contiguous.  masks must be zero on entry (bits are ORed in).
__global__ void __launch_bounds__(kThreads)
neighbor_map_kernel(const int4 * __restrict__ coords, int64_t n,
                    const HashSlot * __restrict__ slots, uint64_t mask,
                    int32_t * __restrict__ nbr, uint32_t * __restrict__ masks) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= 3 * n) return;
    const int kd = static_cast<int>(t / n);
    const int64_t p = t - static_cast<int64_t>(kd) * n;
    const int4 c = coords[p];
    const int x = c.y + kd - 1;
    uint64_t key[9], slot[9];
    HashSlot first[9];
    bool probe[9];
#pragma unroll
    for (int j = 0; j < 9; ++j) {
        const int y = c.z + j / 3 - 1;
        const int z = c.w + j % 3 - 1;
        // The centre is the row itself; negative coordinates never exist.
        probe[j] = !(kd == 1 && j == 4) && x >= 0 && y >= 0 && z >= 0;
        key[j] = voxel_key(c.x, x, y, z);
        slot[j] = home_slot(key[j], mask);
        if (probe[j]) first[j] = load_slot(slots, slot[j]);
    }
    uint32_t present = 0;
#pragma unroll
    for (int j = 0; j < 9; ++j) {
        int32_t row = -1;
        if (kd == 1 && j == 4) row = static_cast<int32_t>(p);
        else if (probe[j]) row = probe_from(slots, mask, key[j], slot[j], first[j]);
        const int k = kd * 9 + j;
        if (row >= 0) present |= 1u << k;
        nbr[static_cast<int64_t>(k) * n + p] = row >= 0 ? row : static_cast<int32_t>(n);
    }
    if (masks && present) atomicOr(masks + p, present);
}

// ---- voxel bricks: a locality-preserving hash --------------------------------------
// The voxel hash puts the 27 neighbours of a row in 27 unrelated 128-byte
// lines.  Here the hash holds 4x4x4 bricks: a slot keys brick (b, x>>2,
// y>>2, z>>2) to its id, and brick id owns 64 consecutive int32 entries of a
// pool, entry ((x&3)*4 + (y&3))*4 + (z&3) holding the row at that voxel (the
// smallest, as in the voxel hash) or INT_MAX.  A row's 3x3x3 neighbourhood
// spans 1..8 bricks (3.4 on average), found with as many probes, and its 27
// entries sit in those bricks' 256 bytes, shared with the rows around it.
// Brick ids come from kBrickCounters counters: wavefront w (64 rows) takes
// its new bricks' ids from counter w % kBrickCounters, which owns the ids
// [k * per, (k + 1) * per), per = 64 * ceil(waves / kBrickCounters), enough
// for every brick of its wavefronts.  So no single counter serialises the
// claims.  Layout of the table: hash slots (hash_capacity(n), as the voxel
// hash), then the pool (kBrickCounters * per bricks of 256 bytes, about one
// per row, the worst case), then the counters.
constexpr int kBrickShift = 2;
constexpr int kBrickCells = 64;
constexpr int kBrickCounters = 64;

int64_t bricks_per_counter(int64_t n) {
    const int64_t waves = (std::max<int64_t>(n, 1) + 63) / 64;
    return 64 * ((waves + kBrickCounters - 1) / kBrickCounters);
}

struct BrickView {
    HashSlot * slots;
    uint64_t mask;
    int32_t * pool;
    int32_t * counters;
    int32_t per;
};

BrickView brick_view(void * table, int64_t n) {
    BrickView v;
    const int64_t cap = hash_capacity(n);
    v.slots = static_cast<HashSlot *>(table);
    v.mask = static_cast<uint64_t>(cap - 1);
    v.pool = reinterpret_cast<int32_t *>(static_cast<char *>(table) + cap * sizeof(HashSlot));
    v.per = static_cast<int32_t>(bricks_per_counter(n));
    v.counters = v.pool + static_cast<int64_t>(kBrickCounters) * v.per * kBrickCells;
    return v;
}

__device__ __forceinline__ uint64_t brick_key(int b, int x, int y, int z) {
    return voxel_key(b, x >> kBrickShift, y >> kBrickShift, z >> kBrickShift);
}
__device__ __forceinline__ int brick_local(int x, int y, int z) {
    return ((x & 3) * 4 + (y & 3)) * 4 + (z & 3);
}

// Claim each brick once: every lane whose key differs from the lane before
// it (sorted rows repeat a brick in runs) inserts it, all at once, with a
// plain load first (a key already there never changes, so seeing it skips
// the compare-and-swap); the lanes that won a new slot take consecutive ids
// from one add per wavefront on the wavefront's counter, and fill their
// brick's 64 pool entries with INT_MAX.
__global__ void brick_claim_kernel(const int4 * __restrict__ coords, int64_t n, HashSlot * slots,
                                   uint64_t mask, int32_t * __restrict__ pool,
                                   int32_t * __restrict__ counters, int32_t per) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int lane = threadIdx.x & 63;
    const bool live = p < n;
    uint64_t key = kEmptyKey;
    if (live) {
        const int4 c = coords[p];
        key = brick_key(c.x, c.y, c.z, c.w);
    }
    const uint64_t before = __shfl_up(key, 1, 64);
    bool won = false;
    uint64_t slot = 0;
    if (live && (lane == 0 || before != key)) {
        slot = home_slot(key, mask);
        for (uint64_t probe = 0; probe <= mask; ++probe) {
            const unsigned long long seen = slots[slot].key;
            if (seen == key) break;
            if (seen == kEmptyKey) {
                const unsigned long long prev =
                    atomicCAS(&slots[slot].key, static_cast<unsigned long long>(kEmptyKey),
                              static_cast<unsigned long long>(key));
                if (prev == kEmptyKey) {
                    won = true;
                    break;
                }
                if (prev == key) break;
            }
            slot = (slot + 1) & mask;
        }
    }
    const uint64_t winners = __ballot(won);
    if (winners == 0) return;
    const int leader = __ffsll(static_cast<unsigned long long>(winners)) - 1;
    const int k = static_cast<int>((p >> 6) % kBrickCounters);
    int32_t base = 0;
    if (lane == leader) base = k * per + atomicAdd(counters + k, __popcll(winners));
    base = __shfl(base, leader, 64);
    if (!won) return;
    const int32_t id = base + __popcll(winners & ((1ull << lane) - 1ull));
    slots[slot].val = id;
    uint4 * b = reinterpret_cast<uint4 *>(pool + static_cast<int64_t>(id) * kBrickCells);
#pragma unroll
    for (int i = 0; i < kBrickCells / 4; ++i) b[i] = make_uint4(INT_MAX, INT_MAX, INT_MAX, INT_MAX);
}

// Each row into its brick's entry (the smallest row when coordinates repeat).
__global__ void brick_place_kernel(const int4 * __restrict__ coords, int64_t n,
                                   const HashSlot * __restrict__ slots, uint64_t mask,
                                   int32_t * __restrict__ pool) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    const int32_t id = hash_find(slots, mask, brick_key(c.x, c.y, c.z, c.w));
    if (id < 0) return;
    atomicMin(pool + static_cast<int64_t>(id) * kBrickCells + brick_local(c.y, c.z, c.w),
              static_cast<int32_t>(p));
}

// One thread per row: the ids of the (up to 8) bricks its 3x3x3 window
// touches, then its 27 entries; the same map and masks as neighbor_map_kernel
// (masks written, not ORed).
__global__ void __launch_bounds__(kThreads)
neighbor_map_bricks_kernel(const int4 * __restrict__ coords, int64_t n,
                           const HashSlot * __restrict__ slots, uint64_t mask,
                           const int32_t * __restrict__ pool, int32_t * __restrict__ nbr,
                           uint32_t * __restrict__ masks) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    // per axis: the window's first brick and whether it spans a second one
    const int bx = (c.y - 1) >> kBrickShift, by = (c.z - 1) >> kBrickShift, bz = (c.w - 1) >> kBrickShift;
    const int nx = ((c.y + 1) >> kBrickShift) - bx, ny = ((c.z + 1) >> kBrickShift) - by,
              nz = ((c.w + 1) >> kBrickShift) - bz;
    int32_t id[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int ix = q >> 2, iy = (q >> 1) & 1, iz = q & 1;
        const int X = bx + ix, Y = by + iy, Z = bz + iz;
        id[q] = -1;
        if (ix <= nx && iy <= ny && iz <= nz && X >= 0 && Y >= 0 && Z >= 0)
            id[q] = hash_find(slots, mask, voxel_key(c.x, X, Y, Z));
    }
    uint32_t present = 0;
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const int x = c.y + k / 9 - 1, y = c.z + (k / 3) % 3 - 1, z = c.w + k % 3 - 1;
        int32_t row = -1;
        if (k == 13) {
            row = static_cast<int32_t>(p);
        } else {
            // id[q] by selects on q's bits, so the ids stay in registers
            const int qx = (x >> kBrickShift) - bx, qy = (y >> kBrickShift) - by,
                      qz = (z >> kBrickShift) - bz;
            const int32_t l0 = qz ? id[1] : id[0], l1 = qz ? id[3] : id[2];
            const int32_t l2 = qz ? id[5] : id[4], l3 = qz ? id[7] : id[6];
            const int32_t m0 = qy ? l1 : l0, m1 = qy ? l3 : l2;
            const int32_t b = qx ? m1 : m0;
            if (b >= 0) {
                const int32_t v = pool[static_cast<int64_t>(b) * kBrickCells + brick_local(x, y, z)];
                if (v != INT_MAX) row = v;
            }
        }
        if (row >= 0) present |= 1u << k;
        nbr[static_cast<int64_t>(k) * n + p] = row >= 0 ? row : static_cast<int32_t>(n);
    }
    if (masks) masks[p] = present;
}

// ---- dense voxel grid -----------------------------------------------------------
// An int32 cell per (b, x, y, z) of the extents, holding the smallest row at
// that coordinate or kGridEmpty.  Building it is a fill and a scatter; a
// neighbour lookup is one load from a cell next to the row's own (z
// neighbours are adjacent words, y neighbours sz words away), with no probe
// chain.  Rows outside the extents are not entered.
constexpr int32_t kGridEmpty = INT_MAX;

struct GridDims {
    int b, x, y, z;
};

__device__ __forceinline__ bool grid_inside(const GridDims & g, int b, int x, int y, int z) {
    return static_cast<unsigned>(b) < static_cast<unsigned>(g.b) &&
           static_cast<unsigned>(x) < static_cast<unsigned>(g.x) &&
           static_cast<unsigned>(y) < static_cast<unsigned>(g.y) &&
           static_cast<unsigned>(z) < static_cast<unsigned>(g.z);
}

__device__ __forceinline__ int64_t grid_cell(const GridDims & g, int b, int x, int y, int z) {
    return ((static_cast<int64_t>(b) * g.x + x) * g.y + y) * g.z + z;
}

__global__ void grid_scatter_kernel(const int4 * __restrict__ coords, int64_t n, GridDims g,
                                    int32_t * __restrict__ grid) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    if (grid_inside(g, c.x, c.y, c.z, c.w)) atomicMin(grid + grid_cell(g, c.x, c.y, c.z, c.w), static_cast<int32_t>(p));
}

// One thread per row: all 27 lookups in flight at once; nbr[k * n + p] is
// written with a wavefront's rows contiguous for each k, and the row's mask
// is stored whole (no atomics, no zero fill).
__global__ void __launch_bounds__(kThreads)
neighbor_map_grid_kernel(const int4 * __restrict__ coords, int64_t n, GridDims g,
                         const int32_t * __restrict__ grid, int32_t * __restrict__ nbr,
                         uint32_t * __restrict__ masks) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    int32_t row[27];
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const int x = c.y + k / 9 - 1, y = c.z + (k / 3) % 3 - 1, z = c.w + k % 3 - 1;
        row[k] = grid_inside(g, c.x, x, y, z) ? grid[grid_cell(g, c.x, x, y, z)] : kGridEmpty;
    }
    row[13] = static_cast<int32_t>(p);  // the centre is the row itself
    uint32_t present = 0;
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const bool hit = row[k] != kGridEmpty;
        if (hit) present |= 1u << k;
        nbr[static_cast<int64_t>(k) * n + p] = hit ? row[k] : static_cast<int32_t>(n);
    }
    if (masks) masks[p] = present;
}

// ---- generation-tagged voxel grid ---------------------------------------------
// One 32-bit cell per (b, x, y, z): the top 8 bits hold 255 - generation
// (generations 1 .. 255), the low 24 the row.  A cell belongs to the current
// build only when its tag matches, so the grid is not refilled per build: a
// reset (all ones, the tag of generation 0) once per 255 generations, and
// between resets every build passes a larger generation, so old entries stop
// matching.  Insertion is an atomicMin: within a generation the smallest row
// wins, and a newer generation has a smaller tag and always replaces an
// older entry.  Same cell size as the plain grid, so a map's lookups move the
// same bytes as pxs_neighbor_map_k3_grid.
constexpr uint32_t kTagRowBits = 24;
constexpr uint32_t kTagMaxGeneration = 255;
constexpr int64_t kTagMaxRows = (int64_t{1} << kTagRowBits) - 1;
static_assert(kTagRowBits == kVoxelTagShift && kTagMaxGeneration == kVoxelTagMax &&
                  static_cast<uint32_t>(kGridEmpty) == kVoxelGridEmpty,
              "grid cell layout shared with voxel_grid_row");

__device__ __forceinline__ uint32_t tag_cell(uint32_t generation, uint32_t row) {
    return ((kTagMaxGeneration - generation) << kTagRowBits) | row;
}

__device__ __forceinline__ int32_t tag_lookup(uint32_t cell, uint32_t generation) {
    return (cell >> kTagRowBits) == kTagMaxGeneration - generation
               ? static_cast<int32_t>(cell & ((1u << kTagRowBits) - 1u))
               : kGridEmpty;
}

__global__ void tagged_scatter_kernel(const int4 * __restrict__ coords, int64_t n, GridDims g,
                                      uint32_t * __restrict__ grid, uint32_t generation) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    if (grid_inside(g, c.x, c.y, c.z, c.w)) {
        atomicMin(grid + grid_cell(g, c.x, c.y, c.z, c.w),
                  tag_cell(generation, static_cast<uint32_t>(p)));
    }
}

// neighbor_map_grid_kernel over a tagged grid: the same map and masks.
__device__ __forceinline__ void map_row_tagged(int64_t p, const int4 * __restrict__ coords,
                                               int64_t n, GridDims g,
                                               const uint32_t * __restrict__ grid,
                                               uint32_t generation, int32_t * __restrict__ nbr,
                                               uint32_t * __restrict__ masks) {
    if (p >= n) return;
    const int4 c = coords[p];
    int32_t row[27];
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const int x = c.y + k / 9 - 1, y = c.z + (k / 3) % 3 - 1, z = c.w + k % 3 - 1;
        row[k] = grid_inside(g, c.x, x, y, z)
                     ? tag_lookup(grid[grid_cell(g, c.x, x, y, z)], generation)
                     : kGridEmpty;
    }
    row[13] = static_cast<int32_t>(p);
    uint32_t present = 0;
#pragma unroll
    for (int k = 0; k < 27; ++k) {
        const bool hit = row[k] != kGridEmpty;
        if (hit) present |= 1u << k;
        nbr[static_cast<int64_t>(k) * n + p] = hit ? row[k] : static_cast<int32_t>(n);
    }
    if (masks) masks[p] = present;
}

__global__ void __launch_bounds__(kThreads)
neighbor_map_tagged_kernel(const int4 * __restrict__ coords, int64_t n, GridDims g,
                           const uint32_t * __restrict__ grid, uint32_t generation,
                           int32_t * __restrict__ nbr, uint32_t * __restrict__ masks) {
    map_row_tagged(static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x, coords, n, g, grid,
                   generation, nbr, masks);
}

template <typename T>
__global__ void fill_value_kernel(T * p, int64_t count, T value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        p[i] = value;
    }
}

// Pair lists: counts per (offset, block of kThreads rows).
__global__ void __launch_bounds__(kThreads)
pair_count_kernel(const int32_t * __restrict__ nbr, int64_t n, int32_t * __restrict__ counts,
                  int64_t blocks) {
    __shared__ int32_t wave_counts[27][kThreads / 64];
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int k = 0; k < 27; ++k) {
        const bool present = p < n && nbr[static_cast<int64_t>(k) * n + p] != n;
        const uint64_t ballot = __ballot(present);
        if (lane == 0) wave_counts[k][wave] = __popcll(ballot);
    }
    __syncthreads();
    if (threadIdx.x < 27) {
        int32_t s = 0;
        for (int w = 0; w < kThreads / 64; ++w) s += wave_counts[threadIdx.x][w];
        counts[static_cast<int64_t>(threadIdx.x) * blocks + blockIdx.x] = s;
    }
}

__global__ void __launch_bounds__(kThreads)
pair_emit_kernel(const int32_t * __restrict__ nbr, int64_t n, const int64_t * __restrict__ base,
                 int64_t blocks, int32_t * __restrict__ pair_in, int32_t * __restrict__ pair_out) {
    __shared__ int32_t wave_counts[27][kThreads / 64];
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int32_t in_row[27];
    uint64_t ballots[27];
    for (int k = 0; k < 27; ++k) {
        in_row[k] = p < n ? nbr[static_cast<int64_t>(k) * n + p] : static_cast<int32_t>(n);
        ballots[k] = __ballot(in_row[k] != n);
        if (lane == 0) wave_counts[k][wave] = __popcll(ballots[k]);
    }
    __syncthreads();
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int k = 0; k < 27; ++k) {
        if (in_row[k] == n) continue;
        int64_t pos = base[static_cast<int64_t>(k) * blocks + blockIdx.x];
        for (int w = 0; w < wave; ++w) pos += wave_counts[k][w];
        pos += __popcll(ballots[k] & below);
        pair_in[pos] = in_row[k];
        pair_out[pos] = static_cast<int32_t>(p);
    }
}

__global__ void pair_offsets_kernel(const int64_t * __restrict__ base, int64_t blocks,
                                    const int64_t * __restrict__ total, int64_t * offsets28) {
    const int k = threadIdx.x;
    if (k < 27) offsets28[k] = base[static_cast<int64_t>(k) * blocks];
    if (k == 27) offsets28[27] = *total;
}

// ---- factor-f topology via an occupancy bitmap over the coarse grid -------
// The dense linearisation ((b*cx + x/f)*cy + y/f)*cz + z/f is lexicographic,
// so a popcount prefix over the bitmap ranks occupied coarse cells in exactly
// the order the reference sorts them (src/sparse.cpp:575-580).
__device__ __forceinline__ int64_t coarse_cell(int4 c, int f, int cx, int cy, int cz) {
    return ((static_cast<int64_t>(c.x) * cx + c.y / f) * cy + c.z / f) * cz + c.w / f;
}

// Rows that share a bitmap word (the f^3 children of a cell and their
// neighbours along z) are merged inside the wavefront first: one atomic per
// distinct word instead of one per row.  Sorted input gives a handful of
// words per wavefront.  Called by every lane of the wavefront.
__device__ __forceinline__ void mark_bits(bool live, int64_t word, uint32_t bit,
                                          uint32_t * __restrict__ bitmap) {
    uint64_t pending = __ballot(live);
    while (pending) {
        const int leader = __ffsll(static_cast<unsigned long long>(pending)) - 1;
        const int64_t w0 = __shfl(word, leader, 64);
        const bool mine = live && word == w0;
        uint32_t v = mine ? bit : 0u;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) v |= __shfl_xor(v, d, 64);
        if ((threadIdx.x & 63) == leader) atomicOr(bitmap + w0, v);
        pending &= ~__ballot(mine);
    }
}

// It also sets clear[k * n + p] = value for k < clear_rows (the child map or
// the group counts the next kernels fill in), saving a fill launch.
__global__ void coarse_mark_kernel(const int4 * __restrict__ coords, int64_t n, int f, int cx,
                                   int cy, int cz, int64_t words, uint32_t * __restrict__ bitmap,
                                   int32_t * __restrict__ clear, int clear_rows, int32_t value) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    bool live = p < n;
    if (live) {
        for (int k = 0; k < clear_rows; ++k) clear[k * n + p] = value;
    }
    int64_t word = -1;
    uint32_t bit = 0;
    if (live) {
        const int4 c = coords[p];
        const int64_t cell = coarse_cell(c, f, cx, cy, cz);
        // a row outside the extents (invalid input) marks nothing
        live = c.x >= 0 && c.y >= 0 && c.z >= 0 && c.w >= 0 && cell >= 0 && (cell >> 5) < words;
        word = live ? cell >> 5 : -1;
        bit = 1u << (cell & 31);
    }
    mark_bits(live, word, bit, bitmap);
}

// pxs_voxel_grid_tagged_insert that also marks each row's stride-2 cell in
// the occupancy bitmap (coarse_mark_kernel's work for factor 2), in the same
// pass over the coordinates.
__global__ void tagged_scatter_mark_kernel(const int4 * __restrict__ coords, int64_t n, GridDims g,
                                           uint32_t * __restrict__ grid, uint32_t generation,
                                           int cx, int cy, int cz, int64_t words,
                                           uint32_t * __restrict__ bitmap) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    bool live = p < n;
    int64_t word = -1;
    uint32_t bit = 0;
    if (live) {
        const int4 c = coords[p];
        if (grid_inside(g, c.x, c.y, c.z, c.w)) {
            atomicMin(grid + grid_cell(g, c.x, c.y, c.z, c.w),
                      tag_cell(generation, static_cast<uint32_t>(p)));
        }
        const int64_t cell = coarse_cell(c, 2, cx, cy, cz);
        live = c.x >= 0 && c.y >= 0 && c.z >= 0 && c.w >= 0 && cell >= 0 && (cell >> 5) < words;
        word = live ? cell >> 5 : -1;
        bit = 1u << (cell & 31);
    }
    mark_bits(live, word, bit, bitmap);
}

constexpr int kEmitWords = 256;  // bitmap words per emit workgroup

// Flag counts of the chained level: every emit workgroup of kS2SideWords
// words (rounded up to 8, plus up to 7 more that align the next role to an
// XCD boundary), and every 128-row tile of at most min(fine cells, 2^24 - 1)
// rows.
int64_t s2_emit_flag_cap(int64_t words) { return (words + kS2SideWords - 1) / kS2SideWords + 16; }
int64_t s2_tile_flag_cap(int batch_size, int sx, int sy, int sz) {
    const int64_t cells = static_cast<int64_t>(batch_size) * sx * sy * sz;
    return (std::min<int64_t>(cells, kTagMaxRows) + 127) / 128 + 1;
}
__global__ void __launch_bounds__(kThreads) s2_emit_tagged_kernel(S2EmitArgs e) {
    __shared__ __align__(16) char lds[s2_emit_lds_bytes(kEmitWords, kThreads)];
    s2_emit_block(e, blockIdx.x, threadIdx.x, kThreads, lds);
}

__device__ __forceinline__ int64_t coarse_rank(int64_t cell, const uint32_t * __restrict__ bitmap,
                                               const int64_t * __restrict__ word_prefix) {
    const int64_t w = cell >> 5;
    const uint32_t bit = static_cast<uint32_t>(cell & 31);
    return word_prefix[w] + __popc(bitmap[w] & ((1u << bit) - 1u));
}

// Factor 2: child c = (x&1) + 2(y&1) + 4(z&1) of output q is row child_map[c*n + q].
__global__ void coarse_emit_kernel(const int4 * __restrict__ coords, int64_t n, int cx, int cy,
                                   int cz, const uint32_t * __restrict__ bitmap,
                                   const int64_t * __restrict__ word_prefix,
                                   int4 * __restrict__ out_coords, int32_t * __restrict__ child_map) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    const int64_t rank = coarse_rank(coarse_cell(c, 2, cx, cy, cz), bitmap, word_prefix);
    const int child = (c.y & 1) + 2 * (c.z & 1) + 4 * (c.w & 1);
    child_map[static_cast<int64_t>(child) * n + rank] = static_cast<int32_t>(p);
    // Every child of the cell writes the same coarse coordinate.
    out_coords[rank] = make_int4(c.x, c.y >> 1, c.z >> 1, c.w >> 1);
}

// ---- stride-2 topology from the fine tagged grid ---------------------------------
// Bitmap words are scanned in blocks of kWordBlock: block-local exclusive
// prefixes plus one total per block, which the emit adds up (at most a few
// dozen totals per block of words).
constexpr int kWordBlock = 1024;

__device__ __forceinline__ void word_block_scan(int64_t block, const uint32_t * __restrict__ bitmap,
                                                int64_t words, int32_t * __restrict__ local_prefix,
                                                int32_t * __restrict__ block_totals) {
    constexpr int kPer = kWordBlock / kThreads;  // 4 words per thread
    __shared__ int32_t wave_sums[kThreads / 64];
    const int64_t base = block * kWordBlock;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    int32_t cnt[kPer];
    int32_t mine = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int64_t w = base + t * kPer + j;
        cnt[j] = w < words ? __popc(bitmap[w]) : 0;
        mine += cnt[j];
    }
    int32_t inc = mine;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t o = __shfl_up(inc, d, 64);
        if (lane >= d) inc += o;
    }
    if (lane == 63) wave_sums[wave] = inc;
    __syncthreads();
    int32_t before = inc - mine;
    for (int w = 0; w < wave; ++w) before += wave_sums[w];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int64_t w = base + t * kPer + j;
        if (w < words) local_prefix[w] = before;
        before += cnt[j];
    }
    if (t == kThreads - 1) block_totals[block] = before;
}

__global__ void __launch_bounds__(kThreads)
word_block_scan_kernel(const uint32_t * __restrict__ bitmap, int64_t words,
                       int32_t * __restrict__ local_prefix, int32_t * __restrict__ block_totals) {
    word_block_scan(blockIdx.x, bitmap, words, local_prefix, block_totals);
}

// The fine neighbour map and the blocked scan of the stride-2 occupancy
// counts in one launch: both need only the insert's results, so workgroups
// [0, map_blocks) map rows and the rest scan bitmap blocks.
__global__ void __launch_bounds__(kThreads)
map_tagged_and_scan_kernel(const int4 * __restrict__ coords, int64_t n, GridDims g,
                           const uint32_t * __restrict__ grid, uint32_t generation,
                           int32_t * __restrict__ nbr, uint32_t * __restrict__ masks,
                           int64_t map_blocks, const uint32_t * __restrict__ bitmap, int64_t words,
                           int32_t * __restrict__ local_prefix,
                           int32_t * __restrict__ block_totals) {
    const int64_t b = blockIdx.x;
    if (b < map_blocks) {
        map_row_tagged(b * kThreads + threadIdx.x, coords, n, g, grid, generation, nbr, masks);
    } else {
        word_block_scan(b - map_blocks, bitmap, words, local_prefix, block_totals);
    }
}

// One thread per coarse cell (32 per bitmap word).  Every cell writes its
// entry of the dense coarse grid (its rank, or kGridEmpty), so that grid needs
// no fill and is freshly cached for the coarse neighbour map that follows.  An
// occupied cell also writes its rank's coordinate and its 8 children looked
// up in the fine tagged grid (child c = (x&1) + 2(y&1) + 4(z&1), -1 when
// absent).  Lane 0 of each word's 32 clears the word once the wavefront has
// read it, so the bitmap is zero again for the next call.
__global__ void __launch_bounds__(kThreads)
coarse_emit_grid_kernel(uint32_t * __restrict__ bitmap, int64_t words, int64_t cells,
                        const int32_t * __restrict__ local_prefix,
                        const int32_t * __restrict__ block_totals, int nblocks, GridDims fine,
                        GridDims coarse, const uint32_t * __restrict__ fine_grid,
                        uint32_t fine_gen, int32_t * __restrict__ coarse_grid,
                        int4 * __restrict__ out_coords, int32_t * __restrict__ child_map,
                        int64_t ld_map, int64_t * m_out) {
    __shared__ int64_t partial[kThreads];
    const int64_t cell = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t w = cell >> 5;
    // The workgroup's 8 words lie in one scan block (kWordBlock words, a
    // multiple of 8); its base is the sum of the earlier blocks' totals
    // (workgroup 0 sums all of them, for m_out).
    const int64_t first_word = static_cast<int64_t>(blockIdx.x) * (kThreads / 32);
    const int64_t sb = blockIdx.x == 0 ? nblocks : first_word / kWordBlock;
    int64_t acc = 0;
    for (int64_t b = threadIdx.x; b < sb; b += kThreads) acc += block_totals[b];
    partial[threadIdx.x] = acc;
    __syncthreads();
    for (int span = kThreads / 2; span >= 1; span >>= 1) {
        if (static_cast<int>(threadIdx.x) < span) partial[threadIdx.x] += partial[threadIdx.x + span];
        __syncthreads();
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) *m_out = partial[0];
    const int64_t block_base = blockIdx.x == 0 ? 0 : partial[0];
    if (w >= words) return;
    const uint32_t bits = bitmap[w];
    const int bit = static_cast<int>(cell & 31);
    // every lane of the word has read it (wavefront-wide loads precede this)
    __builtin_amdgcn_wave_barrier();
    if (bit == 0 && bits) bitmap[w] = 0u;
    const bool occupied = (bits >> bit) & 1u;
    const int64_t rank = block_base + local_prefix[w] + __popc(bits & ((1u << bit) - 1u));
    if (cell < cells) coarse_grid[cell] = occupied ? static_cast<int32_t>(rank) : kGridEmpty;
    if (!occupied) return;
    const int64_t per_item = static_cast<int64_t>(coarse.x) * coarse.y * coarse.z;
    const int b = static_cast<int>(cell / per_item);
    int64_t rem = cell - static_cast<int64_t>(b) * per_item;
    const int X = static_cast<int>(rem / (static_cast<int64_t>(coarse.y) * coarse.z));
    rem -= static_cast<int64_t>(X) * coarse.y * coarse.z;
    const int Y = static_cast<int>(rem / coarse.z);
    const int Z = static_cast<int>(rem - static_cast<int64_t>(Y) * coarse.z);
    out_coords[rank] = make_int4(b, X, Y, Z);
    int32_t child[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int x = 2 * X + (c & 1), y = 2 * Y + ((c >> 1) & 1), z = 2 * Z + (c >> 2);
        child[c] = grid_inside(fine, b, x, y, z)
                       ? tag_lookup(fine_grid[grid_cell(fine, b, x, y, z)], fine_gen)
                       : kGridEmpty;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) child_map[c * ld_map + rank] = child[c] == kGridEmpty ? -1 : child[c];
}

// Any factor: group rows by output cell.  Pass 1 ranks each row's cell and
// takes a slot in its group (atomic, so slot order is arbitrary); pass 2
// places rows; pass 3 sorts each group by row so a group lists its rows in
// ascending input order, the order the reference accumulates them
// (src/sparse.cpp:553-573).
__global__ void group_assign_kernel(const int4 * __restrict__ coords, int64_t n, int f, int cx,
                                    int cy, int cz, const uint32_t * __restrict__ bitmap,
                                    const int64_t * __restrict__ word_prefix,
                                    int4 * __restrict__ out_coords, int32_t * __restrict__ group_of,
                                    int32_t * __restrict__ counts, int32_t * __restrict__ slot) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int4 c = coords[p];
    const int64_t q = coarse_rank(coarse_cell(c, f, cx, cy, cz), bitmap, word_prefix);
    group_of[p] = static_cast<int32_t>(q);
    slot[p] = atomicAdd(counts + q, 1);
    out_coords[q] = make_int4(c.x, c.y / f, c.z / f, c.w / f);
}

__global__ void group_place_kernel(int64_t n, const int32_t * __restrict__ group_of,
                                   const int32_t * __restrict__ slot,
                                   const int64_t * __restrict__ offsets,
                                   int32_t * __restrict__ rows) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    rows[offsets[group_of[p]] + slot[p]] = static_cast<int32_t>(p);
}

__global__ void group_sort_kernel(int64_t groups, const int64_t * __restrict__ offsets,
                                  int32_t * __restrict__ rows) {
    const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (q >= groups) return;
    const int64_t begin = offsets[q], end = offsets[q + 1];
    for (int64_t i = begin + 1; i < end; ++i) {
        const int32_t v = rows[i];
        int64_t j = i - 1;
        while (j >= begin && rows[j] > v) {
            rows[j + 1] = rows[j];
            --j;
        }
        rows[j + 1] = v;
    }
}

// ---- window partition (counting sort by window id, stable per window) -----
struct WindowGrid {
    int64_t nx, ny, nz;
};

__device__ __forceinline__ int64_t window_id(int4 c, int window, int shift, WindowGrid g) {
    const int64_t wx = (c.y + shift) / window;
    const int64_t wy = (c.z + shift) / window;
    const int64_t wz = (c.w + shift) / window;
    return ((static_cast<int64_t>(c.x) * g.nx + wx) * g.ny + wy) * g.nz + wz;
}

__global__ void window_count_kernel(const int4 * __restrict__ coords, int64_t n, int window,
                                    int shift, WindowGrid g, int32_t * __restrict__ counts,
                                    int32_t * __restrict__ slot) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int64_t wid = window_id(coords[p], window, shift, g);
    slot[p] = atomicAdd(counts + wid, 1);
}

// The same counts with each workgroup's rows aggregated first: an LDS table
// (open addressing, load <= 1/2) gives every row a rank among the
// workgroup's rows of its window, and each distinct window then takes one
// global atomic for all of them, which returns the base of its slots.
// slot[p] is unique within the window (in no particular order; the stable
// order comes from window_sort_kernel).  Window ids fit in int32 here.
constexpr int kWinTable = 2 * kThreads;
__global__ void __launch_bounds__(kThreads)
window_count_agg_kernel(const int4 * __restrict__ coords, int64_t n, int window, int shift,
                        WindowGrid g, int32_t * __restrict__ counts, int32_t * __restrict__ slot) {
    __shared__ int32_t keys[kWinTable];
    __shared__ int32_t cnt[kWinTable];
    const int tid = threadIdx.x;
    for (int i = tid; i < kWinTable; i += kThreads) {
        keys[i] = -1;
        cnt[i] = 0;
    }
    __syncthreads();
    const int64_t p = static_cast<int64_t>(blockIdx.x) * kThreads + tid;
    int h = 0, local = 0;
    if (p < n) {
        const int32_t wid = static_cast<int32_t>(window_id(coords[p], window, shift, g));
        h = static_cast<int>((static_cast<uint32_t>(wid) * 2654435761u) >> 23) & (kWinTable - 1);
        for (;;) {
            const int32_t prev = atomicCAS(&keys[h], -1, wid);
            if (prev == -1 || prev == wid) break;
            h = (h + 1) & (kWinTable - 1);
        }
        local = atomicAdd(&cnt[h], 1);
    }
    __syncthreads();
    for (int i = tid; i < kWinTable; i += kThreads)
        if (keys[i] >= 0) cnt[i] = atomicAdd(counts + keys[i], cnt[i]);
    __syncthreads();
    if (p < n) slot[p] = cnt[h] + local;
}

// start (exclusive scan of the counts), cu of the non-empty windows in
// ascending id, *nwin and cu[nwin .. cap] = n, by one workgroup walking the
// windows 1024 at a time (used up to kWinOffsetsMax windows).
constexpr int64_t kWinOffsetsMax = 65536;
__global__ void __launch_bounds__(1024)
window_offsets_kernel(const int32_t * __restrict__ counts, int64_t windows, int64_t n, int64_t cap,
                      int64_t * __restrict__ start, int64_t * __restrict__ cu,
                      int64_t * __restrict__ nwin) {
    __shared__ int32_t wave_tot[16][2];
    __shared__ int64_t carry[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) {
        carry[0] = 0;
        carry[1] = 0;
    }
    __syncthreads();
    for (int64_t w0 = 0; w0 < windows; w0 += 1024) {
        const int64_t w = w0 + tid;
        const int c = w < windows ? counts[w] : 0;
        const int f = c > 0 ? 1 : 0;
        int sc = c, sf = f;  // inclusive wave scans (a chunk's rows are at most n <= INT_MAX)
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int oc = __shfl_up(sc, d, 64), of = __shfl_up(sf, d, 64);
            if (lane >= d) {
                sc += oc;
                sf += of;
            }
        }
        if (lane == 63) {
            wave_tot[wave][0] = sc;
            wave_tot[wave][1] = sf;
        }
        __syncthreads();
        int64_t bc = carry[0], bf = carry[1];
        for (int j = 0; j < wave; ++j) {
            bc += wave_tot[j][0];
            bf += wave_tot[j][1];
        }
        const int64_t excl_c = bc + sc - c, excl_f = bf + sf - f;
        if (w < windows) {
            start[w] = excl_c;
            if (f) cu[excl_f] = excl_c;
        }
        __syncthreads();  // carry and wave_tot read by every thread
        if (tid == 1023) {
            carry[0] = excl_c + c;
            carry[1] = excl_f + f;
        }
        __syncthreads();
    }
    const int64_t nw = carry[1];
    if (tid == 0) *nwin = nw;
    for (int64_t i = nw + tid; i <= cap; i += 1024) cu[i] = n;
}

__global__ void window_flags_kernel(const int32_t * __restrict__ counts, int64_t windows,
                                    int32_t * __restrict__ flags) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < windows) flags[i] = counts[i] > 0 ? 1 : 0;
}

// cu[rank] = start of each non-empty window; cu[nwin .. cap] = n, so that
// any segment count between nwin and cap = min(n, windows) describes the same
// partition (the extra segments are empty).
__global__ void window_cu_kernel(const int32_t * __restrict__ counts, int64_t windows,
                                 const int64_t * __restrict__ start,
                                 const int64_t * __restrict__ rank, const int64_t * __restrict__ nwin,
                                 int64_t n, int64_t cap, int64_t * __restrict__ cu) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < windows && counts[i] > 0) cu[rank[i]] = start[i];
    const int64_t nw = *nwin;
    if (i >= nw && i <= cap) cu[i] = n;
}

__global__ void window_place_kernel(const int4 * __restrict__ coords, int64_t n, int window,
                                    int shift, WindowGrid g, const int64_t * __restrict__ start,
                                    const int32_t * __restrict__ slot, int32_t * __restrict__ tmp) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    const int64_t wid = window_id(coords[p], window, shift, g);
    tmp[start[wid] + slot[p]] = static_cast<int32_t>(p);
}

// One workgroup per window: rank each member by counting smaller row
// indices (rows are unique), giving the stable order.  Windows hold at most
// window^3 rows; larger segments are ranked in LDS chunks.
__global__ void __launch_bounds__(kThreads)
window_sort_kernel(const int32_t * __restrict__ tmp, const int64_t * __restrict__ cu,
                   const int64_t * __restrict__ nwin, int32_t * __restrict__ fwd,
                   int32_t * __restrict__ bwd) {
    __shared__ int32_t members[1024];
    const int64_t w = blockIdx.x;
    if (w >= *nwin) return;
    const int64_t begin = cu[w], end = cu[w + 1];
    const int64_t len = end - begin;
    for (int64_t i0 = 0; i0 < len; i0 += kThreads) {
        const int64_t i = i0 + threadIdx.x;
        const int32_t mine = i < len ? tmp[begin + i] : INT_MAX;
        int64_t rank = 0;
        for (int64_t c0 = 0; c0 < len; c0 += 1024) {
            __syncthreads();
            for (int64_t j = threadIdx.x; j < 1024 && c0 + j < len; j += kThreads) {
                members[j] = tmp[begin + c0 + j];
            }
            __syncthreads();
            const int64_t cnt = min<int64_t>(1024, len - c0);
            for (int64_t j = 0; j < cnt; ++j) rank += members[j] < mine ? 1 : 0;
        }
        if (i < len) {
            fwd[begin + rank] = mine;
            bwd[mine] = static_cast<int32_t>(begin + rank);
        }
    }
}

// ---- per-batch cu_seqlens ----------------------------------------------------
__global__ void batch_cu_kernel(const int4 * __restrict__ coords, int64_t n, int batch_size,
                                int64_t * __restrict__ cu) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (n == 0) {
        if (p <= batch_size) cu[p] = 0;
        return;
    }
    if (p >= n) return;
    const int b = coords[p].x;
    const int prev = p == 0 ? -1 : coords[p - 1].x;
    for (int bb = prev + 1; bb <= b && bb <= batch_size; ++bb) cu[bb] = p;
    if (p == n - 1) {
        for (int bb = b + 1; bb <= batch_size; ++bb) cu[bb] = n;
    }
}

// ---- channel to spatial (factor f, cc = f^3 children) --------------------------
__global__ void c2s_count_kernel(const float * __restrict__ sub, int64_t n, int cc,
                                 int32_t * __restrict__ counts) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (p >= n) return;
    int c = 0;
    for (int j = 0; j < cc; ++j) c += sub[p * cc + j] > 0.0f ? 1 : 0;
    counts[p] = c;
}

// One thread per (parent, child); the channel copy is done by the feature
// kernel below.  Child c sits at (c % f, (c / f) % f, c / f^2) inside the
// parent (src/sparse.cpp:682-686).
__global__ void c2s_coords_kernel(const int4 * __restrict__ coords, int64_t n, int f, int cc,
                                  const float * __restrict__ sub,
                                  const int64_t * __restrict__ prefix,
                                  int4 * __restrict__ out_coords, int64_t * __restrict__ src_of) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= n * cc) return;
    const int64_t p = t / cc;
    const int child = static_cast<int>(t - p * cc);
    int64_t dst;
    if (sub) {
        if (!(sub[p * cc + child] > 0.0f)) return;
        int before = 0;
        for (int j = 0; j < child; ++j) before += sub[p * cc + j] > 0.0f ? 1 : 0;
        dst = prefix[p] + before;
    } else {
        dst = t;
    }
    const int4 c = coords[p];
    out_coords[dst] = make_int4(c.x, f * c.y + child % f, f * c.z + (child / f) % f,
                                f * c.w + child / (f * f));
    src_of[dst] = t;  // source (parent * cc + child)
}

// The same copy in 16-byte pieces (8 elements; c_out % 8 == 0, 16-byte
// aligned buffers): one source-row lookup per piece, 32-bit indices (the
// caller bounds rows * cc by INT_MAX).
template <typename T>
__global__ void c2s_feats8_kernel(const T * __restrict__ x, int channels, int cc,
                                  const int64_t * __restrict__ src_of,
                                  const int64_t * __restrict__ m_dev, int64_t m_max,
                                  T * __restrict__ y) {
    constexpr int kWords = sizeof(T) == 4 ? 2 : 1;  // 16-byte words per 8 elements
    const uint32_t vpr = static_cast<uint32_t>(channels / cc / 8);
    const int64_t m = m_dev ? *m_dev : m_max;
    const uint32_t total = static_cast<uint32_t>(m) * vpr;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const uint32_t r = i / vpr;
        const uint32_t piece = i - r * vpr;
        const uint32_t s = static_cast<uint32_t>(src_of[r]);
        const uint32_t parent = s / static_cast<uint32_t>(cc);
        const uint32_t slot = s - parent * static_cast<uint32_t>(cc);
        const uint4 * src = reinterpret_cast<const uint4 *>(
            x + static_cast<int64_t>(parent) * channels + (static_cast<int64_t>(slot) * vpr + piece) * 8);
        uint4 * dst = reinterpret_cast<uint4 *>(y + static_cast<int64_t>(i) * 8);
#pragma unroll
        for (int w = 0; w < kWords; ++w) dst[w] = src[w];
    }
}

template <typename T>
__global__ void c2s_feats_kernel(const T * __restrict__ x, int channels, int cc,
                                 const int64_t * __restrict__ src_of,
                                 const int64_t * __restrict__ m_dev, int64_t m_max,
                                 T * __restrict__ y) {
    // The child slice of parent p is channels / cc wide.
    const int c_out = channels / cc;
    const int64_t m = m_dev ? *m_dev : m_max;
    const int64_t total = m * c_out;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += stride) {
        const int64_t r = i / c_out;
        const int ch = static_cast<int>(i - r * c_out);
        const int64_t s = src_of[r];
        const int64_t parent = s / cc;
        y[i] = x[parent * channels + (s - parent * cc) * c_out + ch];
    }
}

} // namespace

} // namespace pxs

using namespace pxs;

extern "C" {

size_t pxs_voxel_hash_bytes(int64_t n) {
    return static_cast<size_t>(hash_capacity(n)) * sizeof(HashSlot);
}

int pxs_voxel_hash_build(const int32_t * coords, int64_t n, void * table, void * stream) {
    PXS_CHECK(n >= 0, PXS_ERR_ARG, "pxs_voxel_hash_build: negative row count");
    PXS_CHECK(n <= INT_MAX, PXS_ERR_ARG, "pxs_voxel_hash_build: row count exceeds int32");
    PXS_CHECK(table != nullptr, PXS_ERR_ARG, "pxs_voxel_hash_build: null table");
    PXS_CHECK(n == 0 || coords != nullptr, PXS_ERR_ARG, "pxs_voxel_hash_build: null coords");
    const HashView h = hash_view(table, n);
    const int64_t cap = static_cast<int64_t>(h.mask) + 1;
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(hash_init_kernel, dim3(static_cast<unsigned>(std::min<int64_t>((cap + 255) / 256, 8192))),
                       dim3(256), 0, s, h.slots, cap, nullptr, 0);
    if (n > 0) {
        hipLaunchKernelGGL(hash_insert_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                           reinterpret_cast<const int4 *>(coords), n, h.slots, h.mask);
    }
    return check_launch("pxs_voxel_hash_build");
}

int pxs_sparse_validate(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                        int sz, int dtype, const void * feats, int channels,
                        const void * table, int64_t * status, void * stream) {
    PXS_CHECK(status != nullptr, PXS_ERR_ARG, "pxs_sparse_validate: null status");
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_sparse_validate: bad row count");
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG, "pxs_sparse_validate: bad dtype");
    PXS_CHECK(batch_size <= PXS_MAX_EXTENT && sx <= PXS_MAX_EXTENT && sy <= PXS_MAX_EXTENT &&
                  sz <= PXS_MAX_EXTENT,
              PXS_ERR_ARG, "pxs_sparse_validate: extent exceeds PXS_MAX_EXTENT");
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(status_init_kernel, dim3(1), dim3(1), 0, s, status);
    if (n > 0) {
        PXS_CHECK(coords && table, PXS_ERR_ARG, "pxs_sparse_validate: null coords or table");
        const HashView h = hash_view(const_cast<void *>(table), n);
        hipLaunchKernelGGL(validate_coords_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0,
                           s, reinterpret_cast<const int4 *>(coords), n, batch_size, sx, sy, sz,
                           h.slots, h.mask, status);
        if (feats && channels > 0) {
            const int64_t count = n * channels;
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((count + 255) / 256, 8192));
            if (dtype == PXS_F32) {
                hipLaunchKernelGGL(validate_feats_kernel<float>, dim3(blocks), dim3(256), 0, s,
                                   static_cast<const float *>(feats), count, channels, status);
            } else {
                hipLaunchKernelGGL(validate_feats_kernel<uint16_t>, dim3(blocks), dim3(256), 0, s,
                                   static_cast<const uint16_t *>(feats), count, channels, status);
            }
        }
    }
    return check_launch("pxs_sparse_validate");
}

int pxs_status_reset(int64_t * status, void * stream) {
    PXS_CHECK(status != nullptr, PXS_ERR_ARG, "pxs_status_reset: null status");
    hipLaunchKernelGGL(status_init_kernel, dim3(1), dim3(1), 0, as_stream(stream), status);
    return check_launch("pxs_status_reset");
}

const char * pxs_validation_message(int code) {
    switch (code) {
    case 1: return "invalid sparse tensor shape";
    case 2: return "sparse coordinates must have four columns";
    case 3: return "sparse feature count does not match coordinates";
    case 4: return "sparse coordinate is outside its shape";
    case 5: return "sparse coordinates contain a duplicate point";
    case 6: return "sparse coordinates must be contiguous by batch";
    case 7: return "sparse features contain a non-finite value";
    default: return "";
    }
}

int pxs_neighbor_map_k3(const int32_t * coords, int64_t n, const void * table, int32_t * nbr,
                        uint32_t * masks, void * stream) {
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_neighbor_map_k3: bad row count");
    if (n == 0) return PXS_OK;
    PXS_CHECK(coords && table && nbr, PXS_ERR_ARG, "pxs_neighbor_map_k3: null pointer");
    const HashView h = hash_view(const_cast<void *>(table), n);
    hipStream_t s = as_stream(stream);
    if (masks) {
        if (int rc = fill_u32(masks, n, 0u, s)) return rc;
    }
    hipLaunchKernelGGL(neighbor_map_kernel, dim3(grid_for(3 * n, kThreads)), dim3(kThreads), 0, s,
                       reinterpret_cast<const int4 *>(coords), n, h.slots, h.mask, nbr, masks);
    return check_launch("pxs_neighbor_map_k3");
}

size_t pxs_voxel_bricks_bytes(int64_t n) {
    if (n < 0) return 0;
    return static_cast<size_t>(hash_capacity(n)) * sizeof(HashSlot) +
           static_cast<size_t>(kBrickCounters) * bricks_per_counter(n) * kBrickCells *
               sizeof(int32_t) +
           kBrickCounters * sizeof(int32_t);
}

int pxs_voxel_bricks_build(const int32_t * coords, int64_t n, void * table, void * stream) {
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_voxel_bricks_build: bad row count");
    PXS_CHECK(table != nullptr, PXS_ERR_ARG, "pxs_voxel_bricks_build: null table");
    PXS_CHECK(n == 0 || coords != nullptr, PXS_ERR_ARG, "pxs_voxel_bricks_build: null coords");
    PXS_CHECK((reinterpret_cast<uintptr_t>(table) & 15u) == 0, PXS_ERR_ARG,
              "pxs_voxel_bricks_build: the table must be 16-byte aligned");
    const BrickView v = brick_view(table, n);
    const int64_t cap = static_cast<int64_t>(v.mask) + 1;
    hipStream_t s = as_stream(stream);
    hipLaunchKernelGGL(hash_init_kernel, dim3(static_cast<unsigned>(std::min<int64_t>((cap + 255) / 256, 8192))),
                       dim3(256), 0, s, v.slots, cap, v.counters, kBrickCounters);
    if (n > 0) {
        const int4 * c4 = reinterpret_cast<const int4 *>(coords);
        hipLaunchKernelGGL(brick_claim_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                           c4, n, v.slots, v.mask, v.pool, v.counters, v.per);
        hipLaunchKernelGGL(brick_place_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                           c4, n, v.slots, v.mask, v.pool);
    }
    return check_launch("pxs_voxel_bricks_build");
}

int pxs_neighbor_map_k3_bricks(const int32_t * coords, int64_t n, const void * table, int32_t * nbr,
                               uint32_t * masks, void * stream) {
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_neighbor_map_k3_bricks: bad row count");
    if (n == 0) return PXS_OK;
    PXS_CHECK(coords && table && nbr, PXS_ERR_ARG, "pxs_neighbor_map_k3_bricks: null pointer");
    const BrickView v = brick_view(const_cast<void *>(table), n);
    hipLaunchKernelGGL(neighbor_map_bricks_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0,
                       as_stream(stream), reinterpret_cast<const int4 *>(coords), n, v.slots,
                       v.mask, v.pool, nbr, masks);
    return check_launch("pxs_neighbor_map_k3_bricks");
}

size_t pxs_voxel_grid_bytes(int batch_size, int sx, int sy, int sz) {
    if (batch_size <= 0 || sx <= 0 || sy <= 0 || sz <= 0) return 0;
    const double cells = static_cast<double>(batch_size) * sx * sy * sz;
    if (cells * 4.0 > 9.0e18) return 0;
    return static_cast<size_t>(batch_size) * sx * sy * sz * sizeof(int32_t);
}

int pxs_voxel_grid_build(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                         int sz, void * grid, void * stream) {
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_voxel_grid_build: bad row count");
    const size_t bytes = pxs_voxel_grid_bytes(batch_size, sx, sy, sz);
    PXS_CHECK(bytes > 0, PXS_ERR_ARG, "pxs_voxel_grid_build: invalid extents");
    PXS_CHECK(grid != nullptr && (n == 0 || coords != nullptr), PXS_ERR_ARG,
              "pxs_voxel_grid_build: null pointer");
    hipStream_t s = as_stream(stream);
    int32_t * cells = static_cast<int32_t *>(grid);
    if (int rc = fill_i32(cells, static_cast<int64_t>(bytes / sizeof(int32_t)), kGridEmpty, s)) return rc;
    if (n > 0) {
        hipLaunchKernelGGL(grid_scatter_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                           reinterpret_cast<const int4 *>(coords), n,
                           GridDims{batch_size, sx, sy, sz}, cells);
    }
    return check_launch("pxs_voxel_grid_build");
}

int pxs_neighbor_map_k3_grid(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                             int sz, const void * grid, int32_t * nbr, uint32_t * masks,
                             void * stream) {
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_neighbor_map_k3_grid: bad row count");
    PXS_CHECK(pxs_voxel_grid_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              "pxs_neighbor_map_k3_grid: invalid extents");
    if (n == 0) return PXS_OK;
    PXS_CHECK(coords && grid && nbr, PXS_ERR_ARG, "pxs_neighbor_map_k3_grid: null pointer");
    hipLaunchKernelGGL(neighbor_map_grid_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0,
                       as_stream(stream), reinterpret_cast<const int4 *>(coords), n,
                       GridDims{batch_size, sx, sy, sz}, static_cast<const int32_t *>(grid), nbr,
                       masks);
    return check_launch("pxs_neighbor_map_k3_grid");
}

size_t pxs_voxel_grid_tagged_bytes(int batch_size, int sx, int sy, int sz) {
    return pxs_voxel_grid_bytes(batch_size, sx, sy, sz);
}

int pxs_voxel_grid_tagged_reset(void * grid, int batch_size, int sx, int sy, int sz,
                                void * stream) {
    const size_t bytes = pxs_voxel_grid_tagged_bytes(batch_size, sx, sy, sz);
    PXS_CHECK(bytes > 0, PXS_ERR_ARG, "pxs_voxel_grid_tagged_reset: invalid extents");
    PXS_CHECK(grid, PXS_ERR_ARG, "pxs_voxel_grid_tagged_reset: null pointer");
    const int64_t cells = static_cast<int64_t>(bytes / 4);
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((cells + kThreads - 1) / kThreads, 16384));
    hipLaunchKernelGGL(fill_value_kernel<uint32_t>, dim3(blocks), dim3(kThreads), 0,
                       as_stream(stream), static_cast<uint32_t *>(grid), cells, ~0u);
    return check_launch("pxs_voxel_grid_tagged_reset");
}

int pxs_voxel_grid_tagged_insert(const int32_t * coords, int64_t n, int batch_size, int sx,
                                 int sy, int sz, void * grid, uint32_t generation, void * stream) {
    PXS_CHECK(n >= 0 && n <= kTagMaxRows, PXS_ERR_ARG,
              "pxs_voxel_grid_tagged_insert: bad row count (at most 2^24 - 1 rows)");
    PXS_CHECK(pxs_voxel_grid_tagged_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              "pxs_voxel_grid_tagged_insert: invalid extents");
    PXS_CHECK(generation >= 1 && generation <= kTagMaxGeneration, PXS_ERR_ARG,
              "pxs_voxel_grid_tagged_insert: generation must be in 1..255");
    if (n == 0) return PXS_OK;
    PXS_CHECK(grid && coords, PXS_ERR_ARG, "pxs_voxel_grid_tagged_insert: null pointer");
    hipLaunchKernelGGL(tagged_scatter_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0,
                       as_stream(stream), reinterpret_cast<const int4 *>(coords), n,
                       GridDims{batch_size, sx, sy, sz}, static_cast<uint32_t *>(grid),
                       generation);
    return check_launch("pxs_voxel_grid_tagged_insert");
}

int pxs_neighbor_map_k3_grid_tagged(const int32_t * coords, int64_t n, int batch_size, int sx,
                                    int sy, int sz, const void * grid, uint32_t generation,
                                    int32_t * nbr, uint32_t * masks, void * stream) {
    PXS_CHECK(n >= 0 && n <= kTagMaxRows, PXS_ERR_ARG,
              "pxs_neighbor_map_k3_grid_tagged: bad row count (at most 2^24 - 1 rows)");
    PXS_CHECK(pxs_voxel_grid_tagged_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              "pxs_neighbor_map_k3_grid_tagged: invalid extents");
    PXS_CHECK(generation >= 1 && generation <= kTagMaxGeneration, PXS_ERR_ARG,
              "pxs_neighbor_map_k3_grid_tagged: generation must be in 1..255");
    if (n == 0) return PXS_OK;
    PXS_CHECK(coords && grid && nbr, PXS_ERR_ARG, "pxs_neighbor_map_k3_grid_tagged: null pointer");
    hipLaunchKernelGGL(neighbor_map_tagged_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0,
                       as_stream(stream), reinterpret_cast<const int4 *>(coords), n,
                       GridDims{batch_size, sx, sy, sz},
                       static_cast<const uint32_t *>(grid), generation, nbr, masks);
    return check_launch("pxs_neighbor_map_k3_grid_tagged");
}

size_t pxs_neighbor_pairs_workspace_bytes(int64_t n) {
    const int64_t blocks = std::max<int64_t>((n + kThreads - 1) / kThreads, 1);
    const int64_t count = 27 * blocks;
    return static_cast<size_t>(count) * (sizeof(int32_t) + sizeof(int64_t)) + sizeof(int64_t) +
           scan_workspace_bytes(count) + 64;
}

int pxs_neighbor_pairs(const int32_t * nbr, int64_t n, int32_t * pair_in, int32_t * pair_out,
                       int64_t * offsets28, void * workspace, void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_neighbor_pairs");
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_neighbor_pairs: bad row count");
    PXS_CHECK(offsets28 && workspace, PXS_ERR_ARG, "pxs_neighbor_pairs: null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) return fill_i64(offsets28, 28, 0, s);
    PXS_CHECK(nbr && pair_in && pair_out, PXS_ERR_ARG, "pxs_neighbor_pairs: null pointer");
    const int64_t blocks = (n + kThreads - 1) / kThreads;
    const int64_t count = 27 * blocks;
    char * ws = static_cast<char *>(workspace);
    int64_t * base = reinterpret_cast<int64_t *>(ws);
    int64_t * total = base + count;
    int32_t * counts = reinterpret_cast<int32_t *>(total + 1);
    void * scan_ws = reinterpret_cast<char *>(counts + count) + 8;  // keep 8-byte alignment
    scan_ws = reinterpret_cast<void *>((reinterpret_cast<uintptr_t>(scan_ws) + 7) & ~uintptr_t(7));
    hipLaunchKernelGGL(pair_count_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                       nbr, n, counts, blocks);
    int rc = exclusive_scan_i32(counts, base, count, total, scan_ws, s);
    if (rc != PXS_OK) return rc;
    hipLaunchKernelGGL(pair_emit_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                       nbr, n, base, blocks, pair_in, pair_out);
    hipLaunchKernelGGL(pair_offsets_kernel, dim3(1), dim3(64), 0, s, base, blocks, total,
                       offsets28);
    return check_launch("pxs_neighbor_pairs");
}

size_t pxs_downsample_workspace_bytes(int64_t n, int batch_size, int sx, int sy, int sz,
                                      int factor) {
    if (factor <= 0) return 0;
    const int64_t cells = static_cast<int64_t>(std::max(batch_size, 1)) *
                          ((sx + factor - 1) / factor) * ((sy + factor - 1) / factor) *
                          ((sz + factor - 1) / factor);
    const int64_t words = (cells + 31) / 32;
    const int64_t rows = std::max<int64_t>(n, 1);
    return static_cast<size_t>(words) * (sizeof(uint32_t) + sizeof(int64_t)) +
           static_cast<size_t>(rows) * 3 * sizeof(int32_t) +
           scan_workspace_bytes(std::max(words, rows)) + 128;
}

namespace {
struct CoarseGrid {
    int cx, cy, cz;
    int64_t words;
    uint32_t * bitmap;
    int64_t * prefix;
    char * rest;  // 8-byte aligned scratch after the bitmap scan
};

CoarseGrid coarse_grid(void * workspace, int batch_size, int sx, int sy, int sz, int f) {
    CoarseGrid g;
    g.cx = (sx + f - 1) / f;
    g.cy = (sy + f - 1) / f;
    g.cz = (sz + f - 1) / f;
    g.words = (static_cast<int64_t>(batch_size) * g.cx * g.cy * g.cz + 31) / 32;
    g.bitmap = static_cast<uint32_t *>(workspace);
    g.prefix = reinterpret_cast<int64_t *>(
        (reinterpret_cast<uintptr_t>(g.bitmap + g.words) + 7) & ~uintptr_t(7));
    g.rest = reinterpret_cast<char *>(g.prefix + g.words);
    return g;
}
} // namespace

int pxs_downsample_s2_topology(const int32_t * coords, int64_t n, int batch_size, int sx,
                               int sy, int sz, int32_t * out_coords, int32_t * child_map,
                               int64_t * m_out, void * workspace, void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_downsample_s2_topology");
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_downsample_s2_topology: bad row count");
    PXS_CHECK(batch_size > 0 && sx > 0 && sy > 0 && sz > 0, PXS_ERR_ARG,
              "pxs_downsample_s2_topology: invalid shape");
    PXS_CHECK(m_out && workspace, PXS_ERR_ARG, "pxs_downsample_s2_topology: null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) return fill_i64(m_out, 1, 0, s);
    PXS_CHECK(coords && out_coords && child_map, PXS_ERR_ARG,
              "pxs_downsample_s2_topology: null pointer");
    const CoarseGrid g = coarse_grid(workspace, batch_size, sx, sy, sz, 2);
    int rc = fill_u32(g.bitmap, g.words, 0u, s);
    if (rc) return rc;
    hipLaunchKernelGGL(coarse_mark_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                       reinterpret_cast<const int4 *>(coords), n, 2, g.cx, g.cy, g.cz, g.words,
                       g.bitmap, child_map, 8, -1);
    rc = exclusive_scan_popcount(g.bitmap, g.prefix, g.words, m_out, g.rest, s);
    if (rc) return rc;
    hipLaunchKernelGGL(coarse_emit_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                       reinterpret_cast<const int4 *>(coords), n, g.cx, g.cy, g.cz, g.bitmap,
                       g.prefix, reinterpret_cast<int4 *>(out_coords), child_map);
    return check_launch("pxs_downsample_s2_topology");
}

size_t pxs_downsample_s2_tagged_workspace_bytes(int batch_size, int sx, int sy, int sz) {
    if (batch_size <= 0 || sx <= 0 || sy <= 0 || sz <= 0) return 0;
    const int64_t cells = static_cast<int64_t>(batch_size) * ((sx + 1) / 2) * ((sy + 1) / 2) *
                          ((sz + 1) / 2);
    const int64_t words = (cells + 31) / 32;
    const int64_t blocks = (words + kWordBlock - 1) / kWordBlock;
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    // bitmap, word prefixes, block totals; then the bitmap pair of the fused
    // emit (pxs_s2_tagged_insert / pxs_subm_conv3d_grid_s2_emit) and the flags
    // of the chained level (pxs_unet_s2_level)
    return static_cast<size_t>(up(words * 4) + up(words * 4) + up(blocks * 4) + 2 * up(words * 4) +
                               up(s2_emit_flag_cap(words) * 4) +
                               up(s2_tile_flag_cap(batch_size, sx, sy, sz) * 4) + 256);
}

}  // extern "C"

namespace pxs {
// The emit's arguments over a workspace of pxs_downsample_s2_tagged_workspace_bytes.
S2EmitArgs make_s2_emit_args(int batch_size, int sx, int sy, int sz, const void * fine_grid,
                             uint32_t generation, int32_t * out_coords, int32_t * child_map,
                             int64_t ld_map, int64_t * m_out, void * coarse_grid,
                             void * s2_workspace, int words_per_block) {
    const int cx = (sx + 1) / 2, cy = (sy + 1) / 2, cz = (sz + 1) / 2;
    const int64_t cells = static_cast<int64_t>(batch_size) * cx * cy * cz;
    const int64_t words = (cells + 31) / 32;
    const int64_t blocks = (words + kWordBlock - 1) / kWordBlock;
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    S2EmitArgs e{};
    char * pair = static_cast<char *>(s2_workspace) + 2 * up(words * 4) + up(blocks * 4);
    e.bits = reinterpret_cast<const uint32_t *>(pair + (generation & 1) * up(words * 4));
    e.clear_bits = reinterpret_cast<uint32_t *>(pair + ((generation + 1) & 1) * up(words * 4));
    e.words = words;
    e.cells = cells;
    e.b = batch_size; e.fx = sx; e.fy = sy; e.fz = sz;
    e.cx = cx; e.cy = cy; e.cz = cz;
    e.fine_grid = static_cast<const uint32_t *>(fine_grid);
    e.generation = generation;
    e.coarse_grid = static_cast<int32_t *>(coarse_grid);
    e.out_coords = reinterpret_cast<int4 *>(out_coords);
    e.child_map = child_map;
    e.ld_map = ld_map;
    e.m_out = m_out;
    e.words_per_block = words_per_block;
    // a multiple of 8, so that workgroups after the emit's keep their XCD
    e.blocks = static_cast<int>(((words + words_per_block - 1) / words_per_block + 7) / 8 * 8);
    return e;
}

S2ChainFlags s2_chain_flags(void * s2_workspace, int batch_size, int sx, int sy, int sz) {
    const int64_t cells = static_cast<int64_t>(batch_size) * ((sx + 1) / 2) * ((sy + 1) / 2) *
                          ((sz + 1) / 2);
    const int64_t words = (cells + 31) / 32;
    const int64_t blocks = (words + kWordBlock - 1) / kWordBlock;
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    char * base = static_cast<char *>(s2_workspace) + 2 * up(words * 4) + up(blocks * 4) +
                  2 * up(words * 4);
    S2ChainFlags f;
    f.emit = reinterpret_cast<uint32_t *>(base);
    f.emit_cap = s2_emit_flag_cap(words);
    f.tiles = reinterpret_cast<uint32_t *>(base + up(f.emit_cap * 4));
    f.tiles_cap = s2_tile_flag_cap(batch_size, sx, sy, sz);
    f.error = reinterpret_cast<uint32_t *>(base + up(f.emit_cap * 4) + up(f.tiles_cap * 4));
    return f;
}
}  // namespace pxs

extern "C" {

int pxs_downsample_s2_tagged_workspace_reset(void * workspace, int batch_size, int sx, int sy,
                                             int sz, void * stream) {
    const size_t bytes = pxs_downsample_s2_tagged_workspace_bytes(batch_size, sx, sy, sz);
    PXS_CHECK(bytes > 0, PXS_ERR_ARG, "pxs_downsample_s2_tagged_workspace_reset: invalid shape");
    PXS_CHECK_WORKSPACE(workspace, "pxs_downsample_s2_tagged_workspace_reset");
    PXS_CHECK(workspace, PXS_ERR_ARG, "pxs_downsample_s2_tagged_workspace_reset: null pointer");
    return fill_u32(static_cast<uint32_t *>(workspace), static_cast<int64_t>(bytes / 4), 0u,
                    as_stream(stream));
}

int pxs_downsample_s2_topology_tagged(const int32_t * coords, int64_t n, int batch_size, int sx,
                                      int sy, int sz, const void * fine_grid,
                                      uint32_t fine_generation, int32_t * out_coords,
                                      int32_t * child_map, int64_t ld_map, int64_t * m_out,
                                      void * coarse_grid, void * workspace, void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_downsample_s2_topology_tagged");
    PXS_CHECK(n >= 0 && n <= kTagMaxRows, PXS_ERR_ARG,
              "pxs_downsample_s2_topology_tagged: bad row count (at most 2^24 - 1 rows)");
    PXS_CHECK(pxs_downsample_s2_tagged_workspace_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              "pxs_downsample_s2_topology_tagged: invalid shape");
    PXS_CHECK(fine_generation >= 1 && fine_generation <= kTagMaxGeneration, PXS_ERR_ARG,
              "pxs_downsample_s2_topology_tagged: generation must be in 1..255");
    PXS_CHECK(ld_map >= n, PXS_ERR_ARG,
              "pxs_downsample_s2_topology_tagged: child map stride below the row count");
    PXS_CHECK(m_out && workspace, PXS_ERR_ARG, "pxs_downsample_s2_topology_tagged: null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) return fill_i64(m_out, 1, 0, s);
    PXS_CHECK(coords && fine_grid && out_coords && child_map && coarse_grid, PXS_ERR_ARG,
              "pxs_downsample_s2_topology_tagged: null pointer");
    const int cx = (sx + 1) / 2, cy = (sy + 1) / 2, cz = (sz + 1) / 2;
    const int64_t cells = static_cast<int64_t>(batch_size) * cx * cy * cz;
    const int64_t words = (cells + 31) / 32;
    const int64_t blocks = (words + kWordBlock - 1) / kWordBlock;
    char * ws = static_cast<char *>(workspace);
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    uint32_t * bitmap = reinterpret_cast<uint32_t *>(ws);
    int32_t * local_prefix = reinterpret_cast<int32_t *>(ws + up(words * 4));
    int32_t * totals = reinterpret_cast<int32_t *>(ws + 2 * up(words * 4));
    PXS_CHECK(blocks <= INT_MAX, PXS_ERR_ARG, "pxs_downsample_s2_topology_tagged: grid too large");
    hipLaunchKernelGGL(coarse_mark_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                       reinterpret_cast<const int4 *>(coords), n, 2, cx, cy, cz, words, bitmap,
                       nullptr, 0, 0);
    hipLaunchKernelGGL(word_block_scan_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                       0, s, bitmap, words, local_prefix, totals);
    hipLaunchKernelGGL(coarse_emit_grid_kernel, dim3(grid_for(words * 32, kThreads)), dim3(kThreads), 0,
                       s, bitmap, words, cells, local_prefix, totals, static_cast<int>(blocks),
                       GridDims{batch_size, sx, sy, sz}, GridDims{batch_size, cx, cy, cz},
                       static_cast<const uint32_t *>(fine_grid), fine_generation,
                       static_cast<int32_t *>(coarse_grid), reinterpret_cast<int4 *>(out_coords),
                       child_map, ld_map, m_out);
    return check_launch("pxs_downsample_s2_topology_tagged");
}

int pxs_s2_tagged_insert(const int32_t * coords, int64_t n, int batch_size, int sx, int sy, int sz,
                         void * grid, uint32_t generation, void * s2_workspace, void * stream) {
    PXS_CHECK_WORKSPACE(s2_workspace, "pxs_s2_tagged_insert");
    PXS_CHECK(n >= 0 && n <= kTagMaxRows, PXS_ERR_ARG,
              "pxs_s2_tagged_insert: bad row count (at most 2^24 - 1 rows)");
    PXS_CHECK(pxs_downsample_s2_tagged_workspace_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              "pxs_s2_tagged_insert: invalid extents");
    PXS_CHECK(generation >= 1 && generation <= kTagMaxGeneration, PXS_ERR_ARG,
              "pxs_s2_tagged_insert: generation must be in 1..255");
    if (n == 0) return PXS_OK;
    PXS_CHECK(coords && grid && s2_workspace, PXS_ERR_ARG, "pxs_s2_tagged_insert: null pointer");
    const S2EmitArgs e = make_s2_emit_args(batch_size, sx, sy, sz, grid, generation, nullptr,
                                           nullptr, 0, nullptr, nullptr, s2_workspace, kEmitWords);
    hipLaunchKernelGGL(tagged_scatter_mark_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads),
                       0, as_stream(stream), reinterpret_cast<const int4 *>(coords), n,
                       GridDims{batch_size, sx, sy, sz}, static_cast<uint32_t *>(grid), generation,
                       e.cx, e.cy, e.cz, e.words, const_cast<uint32_t *>(e.bits));
    return check_launch("pxs_s2_tagged_insert");
}

int pxs_s2_tagged_emit(int64_t n, int batch_size, int sx, int sy, int sz, const void * grid,
                       uint32_t generation, int32_t * out_coords, int32_t * child_map,
                       int64_t ld_map, int64_t * m_out, void * coarse_grid, void * s2_workspace,
                       void * stream) {
    PXS_CHECK_WORKSPACE(s2_workspace, "pxs_s2_tagged_emit");
    PXS_CHECK(n >= 0 && n <= kTagMaxRows, PXS_ERR_ARG,
              "pxs_s2_tagged_emit: bad row count (at most 2^24 - 1 rows)");
    PXS_CHECK(pxs_downsample_s2_tagged_workspace_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              "pxs_s2_tagged_emit: invalid extents");
    PXS_CHECK(generation >= 1 && generation <= kTagMaxGeneration, PXS_ERR_ARG,
              "pxs_s2_tagged_emit: generation must be in 1..255");
    PXS_CHECK(ld_map >= n, PXS_ERR_ARG, "pxs_s2_tagged_emit: child map stride below the row count");
    PXS_CHECK(m_out && s2_workspace, PXS_ERR_ARG, "pxs_s2_tagged_emit: null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) return fill_i64(m_out, 1, 0, s);
    PXS_CHECK(grid && out_coords && child_map && coarse_grid, PXS_ERR_ARG,
              "pxs_s2_tagged_emit: null pointer");
    const S2EmitArgs e = make_s2_emit_args(batch_size, sx, sy, sz, grid, generation, out_coords,
                                           child_map, ld_map, m_out, coarse_grid, s2_workspace,
                                           kEmitWords);
    hipLaunchKernelGGL(s2_emit_tagged_kernel, dim3(static_cast<unsigned>(e.blocks)), dim3(kThreads),
                       0, s, e);
    return check_launch("pxs_s2_tagged_emit");
}

int pxs_unet_s2_level_error(const void * s2_workspace, int batch_size, int sx, int sy, int sz,
                            uint32_t * error_out, void * stream) {
    PXS_CHECK(pxs_downsample_s2_tagged_workspace_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              "pxs_unet_s2_level_error: invalid extents");
    PXS_CHECK(s2_workspace && error_out, PXS_ERR_ARG, "pxs_unet_s2_level_error: null pointer");
    const S2ChainFlags f = s2_chain_flags(const_cast<void *>(s2_workspace), batch_size, sx, sy, sz);
    return check_hip(hipMemcpyAsync(error_out, f.error, sizeof(uint32_t), hipMemcpyDefault,
                                    as_stream(stream)),
                     "pxs_unet_s2_level_error");
}

int pxs_map_s2_topology_tagged(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                               int sz, void * grid, uint32_t generation, int32_t * nbr,
                               uint32_t * masks, int32_t * out_coords, int32_t * child_map,
                               int64_t ld_map, int64_t * m_out, void * coarse_grid,
                               void * s2_workspace, void * stream) {
    PXS_CHECK_WORKSPACE(s2_workspace, "pxs_map_s2_topology_tagged");
    PXS_CHECK(n >= 0 && n <= kTagMaxRows, PXS_ERR_ARG,
              "pxs_map_s2_topology_tagged: bad row count (at most 2^24 - 1 rows)");
    PXS_CHECK(pxs_downsample_s2_tagged_workspace_bytes(batch_size, sx, sy, sz) > 0, PXS_ERR_ARG,
              "pxs_map_s2_topology_tagged: invalid extents");
    PXS_CHECK(generation >= 1 && generation <= kTagMaxGeneration, PXS_ERR_ARG,
              "pxs_map_s2_topology_tagged: generation must be in 1..255");
    PXS_CHECK(ld_map >= n, PXS_ERR_ARG,
              "pxs_map_s2_topology_tagged: child map stride below the row count");
    PXS_CHECK(m_out && s2_workspace, PXS_ERR_ARG, "pxs_map_s2_topology_tagged: null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) return fill_i64(m_out, 1, 0, s);
    PXS_CHECK(coords && grid && out_coords && child_map && coarse_grid, PXS_ERR_ARG,
              "pxs_map_s2_topology_tagged: null pointer");
    PXS_CHECK(nbr || !masks, PXS_ERR_ARG,
              "pxs_map_s2_topology_tagged: masks without a neighbour map");
    const int cx = (sx + 1) / 2, cy = (sy + 1) / 2, cz = (sz + 1) / 2;
    const int64_t cells = static_cast<int64_t>(batch_size) * cx * cy * cz;
    const int64_t words = (cells + 31) / 32;
    const int64_t blocks = (words + kWordBlock - 1) / kWordBlock;
    const int64_t map_blocks = (n + kThreads - 1) / kThreads;
    PXS_CHECK(blocks + map_blocks <= INT_MAX, PXS_ERR_ARG, "pxs_map_s2_topology_tagged: grid too large");
    char * ws = static_cast<char *>(s2_workspace);
    auto up = [](int64_t b) { return (b + 255) / 256 * 256; };
    uint32_t * bitmap = reinterpret_cast<uint32_t *>(ws);
    int32_t * local_prefix = reinterpret_cast<int32_t *>(ws + up(words * 4));
    int32_t * totals = reinterpret_cast<int32_t *>(ws + 2 * up(words * 4));
    const GridDims fine{batch_size, sx, sy, sz};
    const int4 * c4 = reinterpret_cast<const int4 *>(coords);
    hipLaunchKernelGGL(tagged_scatter_mark_kernel, dim3(static_cast<unsigned>(map_blocks)),
                       dim3(kThreads), 0, s, c4, n, fine, static_cast<uint32_t *>(grid), generation,
                       cx, cy, cz, words, bitmap);
    // Without nbr only the bitmap scan runs (the map's workgroups are left out).
    const int64_t row_blocks = nbr ? map_blocks : 0;
    hipLaunchKernelGGL(map_tagged_and_scan_kernel, dim3(static_cast<unsigned>(row_blocks + blocks)),
                       dim3(kThreads), 0, s, c4, n, fine, static_cast<const uint32_t *>(grid),
                       generation, nbr, masks, row_blocks, bitmap, words, local_prefix, totals);
    hipLaunchKernelGGL(coarse_emit_grid_kernel, dim3(grid_for(words * 32, kThreads)), dim3(kThreads), 0,
                       s, bitmap, words, cells, local_prefix, totals, static_cast<int>(blocks), fine,
                       GridDims{batch_size, cx, cy, cz}, static_cast<const uint32_t *>(grid),
                       generation, static_cast<int32_t *>(coarse_grid),
                       reinterpret_cast<int4 *>(out_coords), child_map, ld_map, m_out);
    return check_launch("pxs_map_s2_topology_tagged");
}

int pxs_downsample_topology(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                            int sz, int factor, int32_t * out_coords, int64_t * group_offsets,
                            int32_t * group_rows, int64_t * m_out, void * workspace,
                            void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_downsample_topology");
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_downsample_topology: bad row count");
    PXS_CHECK(factor > 0, PXS_ERR_ARG, "sparse downsample factor must be positive");
    PXS_CHECK(batch_size > 0 && sx > 0 && sy > 0 && sz > 0, PXS_ERR_ARG,
              "pxs_downsample_topology: invalid shape");
    PXS_CHECK(m_out && group_offsets && workspace, PXS_ERR_ARG,
              "pxs_downsample_topology: null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) {
        int rc = fill_i64(m_out, 1, 0, s);
        return rc ? rc : fill_i64(group_offsets, 1, 0, s);
    }
    PXS_CHECK(coords && out_coords && group_rows, PXS_ERR_ARG,
              "pxs_downsample_topology: null pointer");
    const CoarseGrid g = coarse_grid(workspace, batch_size, sx, sy, sz, factor);
    int32_t * group_of = reinterpret_cast<int32_t *>(g.rest);
    int32_t * slot = group_of + n;
    int32_t * counts = slot + n;
    void * scan_ws = reinterpret_cast<void *>(
        (reinterpret_cast<uintptr_t>(counts + n) + 7) & ~uintptr_t(7));
    const int4 * c4 = reinterpret_cast<const int4 *>(coords);
    int rc = fill_u32(g.bitmap, g.words, 0u, s);
    if (rc) return rc;
    hipLaunchKernelGGL(coarse_mark_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, c4,
                       n, factor, g.cx, g.cy, g.cz, g.words, g.bitmap, counts, 1, 0);
    rc = exclusive_scan_popcount(g.bitmap, g.prefix, g.words, m_out, scan_ws, s);
    if (rc) return rc;
    hipLaunchKernelGGL(group_assign_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, c4,
                       n, factor, g.cx, g.cy, g.cz, g.bitmap, g.prefix,
                       reinterpret_cast<int4 *>(out_coords), group_of, counts, slot);
    // counts past the last group are zero, so offsets[m .. n] all equal n.
    rc = exclusive_scan_i32(counts, group_offsets, n, group_offsets + n, scan_ws, s);
    if (rc) return rc;
    hipLaunchKernelGGL(group_place_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, n,
                       group_of, slot, group_offsets, group_rows);
    hipLaunchKernelGGL(group_sort_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, n,
                       group_offsets, group_rows);
    return check_launch("pxs_downsample_topology");
}

size_t pxs_window_partition_workspace_bytes(int batch_size, int sx, int sy, int sz, int window,
                                            int shift, int64_t n) {
    if (window <= 0) return 0;
    const int64_t nx = (sx + shift + window - 1) / window;
    const int64_t ny = (sy + shift + window - 1) / window;
    const int64_t nz = (sz + shift + window - 1) / window;
    const int64_t windows = static_cast<int64_t>(std::max(batch_size, 1)) * nx * ny * nz;
    // counts + flags (int32), start + rank (int64), slot + tmp (int32 per row), scan.
    return static_cast<size_t>(windows) * (2 * sizeof(int32_t) + 2 * sizeof(int64_t)) +
           static_cast<size_t>(std::max<int64_t>(n, 1)) * 2 * sizeof(int32_t) + sizeof(int64_t) +
           scan_workspace_bytes(windows) + 128;
}

int pxs_window_partition(const int32_t * coords, int64_t n, int batch_size, int sx, int sy,
                         int sz, int window, int shift, int32_t * fwd, int32_t * bwd,
                         int64_t * cu_seqlens, int64_t * nwin_out, void * workspace,
                         void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_window_partition");
    PXS_CHECK(n >= 0 && n <= INT_MAX, PXS_ERR_ARG, "pxs_window_partition: bad row count");
    PXS_CHECK(window > 0 && shift >= 0 && batch_size > 0 && sx > 0 && sy > 0 && sz > 0,
              PXS_ERR_ARG, "pxs_window_partition: invalid window or shape");
    PXS_CHECK(cu_seqlens && nwin_out && workspace, PXS_ERR_ARG,
              "pxs_window_partition: null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) {
        int rc = fill_i64(nwin_out, 1, 0, s);
        return rc ? rc : fill_i64(cu_seqlens, 1, 0, s);
    }
    PXS_CHECK(coords && fwd && bwd, PXS_ERR_ARG, "pxs_window_partition: null pointer");
    WindowGrid g;
    g.nx = (sx + shift + window - 1) / window;
    g.ny = (sy + shift + window - 1) / window;
    g.nz = (sz + shift + window - 1) / window;
    const int64_t windows = static_cast<int64_t>(batch_size) * g.nx * g.ny * g.nz;
    char * ws = static_cast<char *>(workspace);
    int64_t * start = reinterpret_cast<int64_t *>(ws);
    int64_t * rank = start + windows;
    int64_t * nwin_scratch = rank + windows;
    int32_t * counts = reinterpret_cast<int32_t *>(nwin_scratch + 1);
    int32_t * flags = counts + windows;
    int32_t * slot = flags + windows;
    int32_t * tmp = slot + n;
    void * scan_ws = reinterpret_cast<void *>(
        (reinterpret_cast<uintptr_t>(tmp + n) + 7) & ~uintptr_t(7));
    (void)nwin_scratch;
    const int4 * c4 = reinterpret_cast<const int4 *>(coords);
    int rc = fill_i32(counts, windows, 0, s);
    if (rc) return rc;
    const int64_t cap = std::min<int64_t>(n, windows);
    if (windows <= kWinOffsetsMax) {
        // aggregated counts, then one workgroup for starts, cu and nwin
        hipLaunchKernelGGL(window_count_agg_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0,
                           s, c4, n, window, shift, g, counts, slot);
        hipLaunchKernelGGL(window_offsets_kernel, dim3(1), dim3(1024), 0, s, counts, windows, n, cap,
                           start, cu_seqlens, nwin_out);
    } else {
        hipLaunchKernelGGL(window_count_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                           c4, n, window, shift, g, counts, slot);
        rc = exclusive_scan_i32(counts, start, windows, nullptr, scan_ws, s);
        if (rc) return rc;
        hipLaunchKernelGGL(window_flags_kernel, dim3(grid_for(windows, kThreads)), dim3(kThreads), 0,
                           s, counts, windows, flags);
        rc = exclusive_scan_i32(flags, rank, windows, nwin_out, scan_ws, s);
        if (rc) return rc;
        hipLaunchKernelGGL(window_cu_kernel, dim3(grid_for(windows + 1, kThreads)), dim3(kThreads),
                           0, s, counts, windows, start, rank, nwin_out, n, cap, cu_seqlens);
    }
    hipLaunchKernelGGL(window_place_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s, c4,
                       n, window, shift, g, start, slot, tmp);
    // At most cap non-empty windows; workgroups past *nwin exit at once.
    hipLaunchKernelGGL(window_sort_kernel, dim3(static_cast<unsigned>(cap)), dim3(kThreads), 0, s,
                       tmp, cu_seqlens, nwin_out, fwd, bwd);
    return check_launch("pxs_window_partition");
}

int pxs_batch_cu_seqlens(const int32_t * coords, int64_t n, int batch_size, int64_t * cu,
                         void * stream) {
    PXS_CHECK(n >= 0 && batch_size > 0 && cu, PXS_ERR_ARG, "pxs_batch_cu_seqlens: bad argument");
    const int64_t items = std::max<int64_t>(n, batch_size + 1);
    hipLaunchKernelGGL(batch_cu_kernel, dim3(grid_for(items, kThreads)), dim3(kThreads), 0,
                       as_stream(stream), reinterpret_cast<const int4 *>(coords), n, batch_size,
                       cu);
    return check_launch("pxs_batch_cu_seqlens");
}

size_t pxs_channel_to_spatial_workspace_bytes(int64_t n, int factor) {
    if (factor <= 0 || factor > 1024) return 0;
    const int64_t cc = static_cast<int64_t>(factor) * factor * factor;
    const int64_t rows = std::max<int64_t>(n, 1);
    return static_cast<size_t>(rows) * (sizeof(int32_t) + sizeof(int64_t)) +
           static_cast<size_t>(rows * cc) * sizeof(int64_t) + scan_workspace_bytes(rows) + 64;
}

int pxs_channel_to_spatial(int dtype, const int32_t * coords, int64_t n, const void * x,
                           int channels, int factor, const float * subdivision,
                           int32_t * out_coords, void * y, int64_t * m_out, void * workspace,
                           void * stream) {
    PXS_CHECK_WORKSPACE(workspace, "pxs_channel_to_spatial");
    PXS_CHECK(factor > 0 && factor <= 1024, PXS_ERR_ARG,
              "pxs_channel_to_spatial: factor must be in 1..1024");
    const int64_t cc = static_cast<int64_t>(factor) * factor * factor;
    PXS_CHECK(n >= 0 && n * cc <= INT_MAX, PXS_ERR_ARG, "pxs_channel_to_spatial: bad row count");
    PXS_CHECK(channels > 0 && channels % cc == 0, PXS_ERR_ARG,
              "sparse channel-to-spatial channels are not divisible by factor^3");
    PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG, "pxs_channel_to_spatial: bad dtype");
    PXS_CHECK(m_out && workspace, PXS_ERR_ARG, "pxs_channel_to_spatial: null pointer");
    hipStream_t s = as_stream(stream);
    if (n == 0) return fill_i64(m_out, 1, 0, s);
    PXS_CHECK(coords && x && out_coords && y, PXS_ERR_ARG, "pxs_channel_to_spatial: null pointer");
    const int icc = static_cast<int>(cc);
    char * ws = static_cast<char *>(workspace);
    int64_t * prefix = reinterpret_cast<int64_t *>(ws);
    int64_t * src_of = prefix + n;
    int32_t * counts = reinterpret_cast<int32_t *>(src_of + n * cc);
    void * scan_ws = reinterpret_cast<void *>(
        (reinterpret_cast<uintptr_t>(counts + n) + 7) & ~uintptr_t(7));
    int rc;
    if (subdivision) {
        hipLaunchKernelGGL(c2s_count_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, s,
                           subdivision, n, icc, counts);
        rc = exclusive_scan_i32(counts, prefix, n, m_out, scan_ws, s);
        if (rc) return rc;
    } else {
        rc = fill_i64(m_out, 1, n * cc, s);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(c2s_coords_kernel, dim3(grid_for(n * cc, kThreads)), dim3(kThreads), 0, s,
                       reinterpret_cast<const int4 *>(coords), n, factor, icc, subdivision, prefix,
                       reinterpret_cast<int4 *>(out_coords), src_of);
    const int64_t max_elems = n * channels;
    if ((channels / icc) % 8 == 0 && max_elems / 8 <= UINT32_MAX &&
        (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
        const unsigned vb = static_cast<unsigned>(std::min<int64_t>((max_elems / 8 + 255) / 256, 16384));
        if (dtype == PXS_F32)
            hipLaunchKernelGGL(c2s_feats8_kernel<float>, dim3(vb), dim3(256), 0, s,
                               static_cast<const float *>(x), channels, icc, src_of, m_out, n * cc,
                               static_cast<float *>(y));
        else
            hipLaunchKernelGGL(c2s_feats8_kernel<uint16_t>, dim3(vb), dim3(256), 0, s,
                               static_cast<const uint16_t *>(x), channels, icc, src_of, m_out,
                               n * cc, static_cast<uint16_t *>(y));
        return check_launch("pxs_channel_to_spatial");
    }
    const unsigned blocks = static_cast<unsigned>(std::min<int64_t>((max_elems + 255) / 256, 16384));
    if (dtype == PXS_F32) {
        hipLaunchKernelGGL(c2s_feats_kernel<float>, dim3(blocks), dim3(256), 0, s,
                           static_cast<const float *>(x), channels, icc, src_of, m_out, n * cc,
                           static_cast<float *>(y));
    } else {
        hipLaunchKernelGGL(c2s_feats_kernel<uint16_t>, dim3(blocks), dim3(256), 0, s,
                           static_cast<const uint16_t *>(x), channels, icc, src_of, m_out, n * cc,
                           static_cast<uint16_t *>(y));
    }
    return check_launch("pxs_channel_to_spatial");
}

} // extern "C"
