// Device-wide exclusive prefix sums and fills for the topology kernels.
//
// Scan layout: tiles of kScanTile consecutive items; phase 1 reduces each
// tile into partials[t]; phase 2 scans the partials in one workgroup (looping
// over chunks of 256); phase 3 rescans each tile with its partial offset.

#include "scan.h"

namespace pxs {
namespace {

template <bool kPopcount>
__device__ __forceinline__ int64_t scan_value(const void * in, int64_t i) {
    if constexpr (kPopcount) {
        return __popc(static_cast<const uint32_t *>(in)[i]);
    } else {
        return static_cast<const int32_t *>(in)[i];
    }
}

// Block-wide inclusive scan of one int64 per thread (256 threads).
__device__ __forceinline__ int64_t block_inclusive_scan(int64_t v, int64_t * smem) {
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    // Wave-level scan with shuffles.
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    if (lane == 63) smem[wave] = v;
    __syncthreads();
    if (t == 0) {
        int64_t run = 0;
        for (int w = 0; w < kScanBlock / 64; ++w) {
            const int64_t s = smem[w];
            smem[w] = run;
            run += s;
        }
    }
    __syncthreads();
    v += smem[wave];
    __syncthreads();
    return v;
}

template <bool kPopcount>
__global__ void __launch_bounds__(kScanBlock)
scan_tile_sums(const void * in, int64_t count, int64_t * partials) {
    __shared__ int64_t smem[kScanBlock / 64];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile;
    int64_t s = 0;
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + static_cast<int64_t>(j) * kScanBlock + threadIdx.x;
        if (i < count) s += scan_value<kPopcount>(in, i);
    }
    const int64_t total = block_inclusive_scan(s, smem);
    if (threadIdx.x == kScanBlock - 1) partials[blockIdx.x] = total;
}

__global__ void __launch_bounds__(kScanBlock)
scan_partials(int64_t * partials, int64_t tiles, int64_t * total) {
    __shared__ int64_t smem[kScanBlock / 64];
    int64_t carry = 0;
    for (int64_t base = 0; base < tiles; base += kScanBlock) {
        const int64_t i = base + threadIdx.x;
        const int64_t v = i < tiles ? partials[i] : 0;
        const int64_t inc = block_inclusive_scan(v, smem);
        if (i < tiles) partials[i] = carry + inc - v;
        __shared__ int64_t chunk_total;
        if (threadIdx.x == kScanBlock - 1) chunk_total = inc;
        __syncthreads();
        carry += chunk_total;
        __syncthreads();
    }
    if (threadIdx.x == 0 && total) *total = carry;
}

template <bool kPopcount>
__global__ void __launch_bounds__(kScanBlock)
scan_tiles(const void * in, int64_t count, const int64_t * partials, int64_t * out) {
    __shared__ int64_t smem[kScanBlock / 64];
    // Each thread owns kScanItems consecutive items of the tile.
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanTile +
                         static_cast<int64_t>(threadIdx.x) * kScanItems;
    int64_t vals[kScanItems];
    int64_t s = 0;
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        vals[j] = i < count ? scan_value<kPopcount>(in, i) : 0;
        s += vals[j];
    }
    const int64_t inc = block_inclusive_scan(s, smem);
    int64_t run = partials[blockIdx.x] + inc - s;
    for (int j = 0; j < kScanItems; ++j) {
        const int64_t i = base + j;
        if (i < count) out[i] = run;
        run += vals[j];
    }
}

// Counts up to kSingleItems: one workgroup of 1024 threads scans everything
// in a single launch (the three-phase scan costs three launches even for a
// few thousand items).  The items are read coalesced into LDS (one pad word
// per 16, so that thread t's 16 consecutive items at 17t.. hit distinct
// banks), then each thread scans its own 16.
constexpr int kSingleThreads = 1024;
constexpr int kSinglePer = 16;
constexpr int64_t kSingleItems = static_cast<int64_t>(kSinglePer) * kSingleThreads;
constexpr int kSingleLdsBytes = static_cast<int>((kSingleItems + kSingleItems / 16) * 4);

template <bool kPopcount>
__global__ void __launch_bounds__(kSingleThreads)
scan_single(const void * in, int64_t count, int64_t * out, int64_t * total) {
    extern __shared__ int32_t stage[];
    __shared__ int64_t wave_sums[kSingleThreads / 64];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    {
        // All 16 loads in flight at once, then the LDS stores.
        int32_t v[kSinglePer];
#pragma unroll
        for (int j = 0; j < kSinglePer; ++j) {
            const int i = j * kSingleThreads + t;
            v[j] = i < count ? static_cast<int32_t>(scan_value<kPopcount>(in, i)) : 0;
        }
#pragma unroll
        for (int j = 0; j < kSinglePer; ++j) {
            const int i = j * kSingleThreads + t;
            stage[i + (i >> 4)] = v[j];
        }
    }
    __syncthreads();
    const int base = t * kSinglePer;
    int64_t vals[kSinglePer];
    int64_t s = 0;
#pragma unroll
    for (int j = 0; j < kSinglePer; ++j) {
        vals[j] = base + j < count ? stage[t * (kSinglePer + 1) + j] : 0;
        s += vals[j];
    }
    int64_t inc = s;
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t o = __shfl_up(inc, d, 64);
        if (lane >= d) inc += o;
    }
    if (lane == 63) wave_sums[wave] = inc;
    __syncthreads();
    if (wave == 0) {
        int64_t w = lane < kSingleThreads / 64 ? wave_sums[lane] : 0;
        for (int d = 1; d < 64; d <<= 1) {
            const int64_t o = __shfl_up(w, d, 64);
            if (lane >= d) w += o;
        }
        if (lane < kSingleThreads / 64) wave_sums[lane] = w;  // inclusive over waves
    }
    __syncthreads();
    // Thread t's exclusive base in LDS; its items become their offsets from
    // it (a partial sum of 16 items fits in int32, the total does too).
    __shared__ int64_t thread_base[kSingleThreads];
    thread_base[t] = inc - s + (wave > 0 ? wave_sums[wave - 1] : 0);
    int32_t part = 0;
#pragma unroll
    for (int j = 0; j < kSinglePer; ++j) {
        stage[t * (kSinglePer + 1) + j] = part;
        part += static_cast<int32_t>(vals[j]);
    }
    __syncthreads();
    // Coalesced stores: item i = j * 1024 + t.
#pragma unroll
    for (int j = 0; j < kSinglePer; ++j) {
        const int i = j * kSingleThreads + t;
        if (i < count) out[i] = thread_base[i >> 4] + stage[i + (i >> 4)];
    }
    if (t == kSingleThreads - 1 && total) *total = wave_sums[kSingleThreads / 64 - 1];
}

template <typename T>
__global__ void fill_kernel(T * p, int64_t count, T value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
         i += stride) {
        p[i] = value;
    }
}

template <bool kPopcount>
int run_scan(const void * in, int64_t * out, int64_t count, int64_t * total, void * workspace,
             hipStream_t stream) {
    const int64_t tiles = (count + kScanTile - 1) / kScanTile;
    int64_t * partials = static_cast<int64_t *>(workspace);
    if (count <= 0) {
        if (total) return fill_i64(total, 1, 0, stream);
        return PXS_OK;
    }
    if (count <= kSingleItems) {
        static bool configured = false;
        if (!configured) {
            hipError_t e = hipFuncSetAttribute(
                reinterpret_cast<const void *>(&scan_single<kPopcount>),
                hipFuncAttributeMaxDynamicSharedMemorySize, kSingleLdsBytes);
            if (e != hipSuccess) return check_hip(e, "hipFuncSetAttribute(scan_single)");
            configured = true;
        }
        hipLaunchKernelGGL(scan_single<kPopcount>, dim3(1), dim3(kSingleThreads), kSingleLdsBytes,
                           stream, in, count, out, total);
        return check_launch("exclusive scan (single workgroup)");
    }
    hipLaunchKernelGGL(scan_tile_sums<kPopcount>, dim3(static_cast<unsigned>(tiles)),
                       dim3(kScanBlock), 0, stream, in, count, partials);
    hipLaunchKernelGGL(scan_partials, dim3(1), dim3(kScanBlock), 0, stream, partials, tiles,
                       total);
    hipLaunchKernelGGL(scan_tiles<kPopcount>, dim3(static_cast<unsigned>(tiles)),
                       dim3(kScanBlock), 0, stream, in, count, partials, out);
    return check_launch("exclusive scan");
}

template <typename T>
int run_fill(T * p, int64_t count, T value, hipStream_t stream) {
    if (count <= 0) return PXS_OK;
    const int64_t blocks = std::min<int64_t>((count + 255) / 256, 4096);
    hipLaunchKernelGGL(fill_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                       p, count, value);
    return check_launch("fill");
}

} // namespace

size_t scan_workspace_bytes(int64_t count) {
    const int64_t tiles = (count + kScanTile - 1) / kScanTile;
    return static_cast<size_t>(std::max<int64_t>(tiles, 1)) * sizeof(int64_t);
}

int exclusive_scan_i32(const int32_t * in, int64_t * out, int64_t count, int64_t * total,
                       void * workspace, hipStream_t stream) {
    return run_scan<false>(in, out, count, total, workspace, stream);
}

int exclusive_scan_popcount(const uint32_t * in, int64_t * out, int64_t count, int64_t * total,
                            void * workspace, hipStream_t stream) {
    return run_scan<true>(in, out, count, total, workspace, stream);
}

int fill_i32(int32_t * p, int64_t count, int32_t value, hipStream_t stream) {
    return run_fill<int32_t>(p, count, value, stream);
}
int fill_i64(int64_t * p, int64_t count, int64_t value, hipStream_t stream) {
    return run_fill<int64_t>(p, count, value, stream);
}
int fill_u32(uint32_t * p, int64_t count, uint32_t value, hipStream_t stream) {
    return run_fill<uint32_t>(p, count, value, stream);
}

} // namespace pxs
