// Shared device/host helpers for the pxs HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "pxs.h"

namespace pxs {

// ---- error reporting (thread-local last error, see pxs_last_error) ---------
void set_error(const std::string & message);
int fail(int code, const std::string & message) noexcept;
int fail_workspace(const char * what) noexcept;
int check_hip(hipError_t status, const char * what);
int check_launch(const char * what);

// Dense linears on MFMA (csrc/dense.hip): x [rows, cin] and w [cout, cin],
// both PXS_BF16 or both PXS_F32.  Each sets *done when it ran the product and
// leaves it false for operands it does not take (rows of x or w not whole
// 16-byte pieces, or not 16-byte aligned), which the caller then runs on the
// gather-GEMM kernels.
//   dense_linear:          y (dtype) = act(x w^T + bias)
//   dense_linear_residual: residual (fp32) += x w^T + bias
//   dense_linear_gate:     residual += (x w^T + bias) * (block_mod[o + c] + time_mod[b, o + c])
int dense_linear(int dtype, const void * x, int64_t rows, int cin, const void * w,
                 const float * bias, int cout, int act, void * y, hipStream_t s, bool * done);
int dense_linear_residual(int dtype, const void * x, int64_t rows, int cin, const void * w,
                          const float * bias, int cout, float * residual, hipStream_t s,
                          bool * done);
int dense_linear_gate(int dtype, const void * x, int64_t rows, int cin, const void * w,
                      const float * bias, int cout, const int32_t * coords,
                      const float * block_mod, const float * time_mod, int gate_offset,
                      float * residual, hipStream_t s, bool * done);

#define PXS_CHECK(expr, code, msg)            \
    do {                                      \
        if (!(expr)) return ::pxs::fail((code), (msg)); \
    } while (0)

// Caller workspaces are carved into 256-byte-aligned sub-buffers that hold
// 16-byte vectors and 64-bit counters, so a workspace must start 256-byte
// aligned (as hipMalloc returns); a null workspace passes, for calls that
// need none.
// The message is composed inside fail_workspace, which cannot throw.
#define PXS_CHECK_WORKSPACE(ws, what)                                   \
    do {                                                                \
        if (reinterpret_cast<uintptr_t>(ws) % 256 != 0)                 \
            return ::pxs::fail_workspace(what);                         \
    } while (0)

inline hipStream_t as_stream(void * s) { return static_cast<hipStream_t>(s); }

inline unsigned grid_for(int64_t items, int per_block) {
    return static_cast<unsigned>((items + per_block - 1) / per_block);
}

// ---- bf16 storage ------------------------------------------------------------
// bf16 values live in HBM as raw uint16_t bit patterns; device code converts
// with the hardware round-to-nearest-even conversion.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t bits) {
    return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    __bf16 b = static_cast<__bf16>(v);
    return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    bf16x2 v;
    v[0] = static_cast<__bf16>(lo);
    v[1] = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

// Element load/store helpers templated on storage type (float or uint16_t=bf16).
template <typename T> __device__ __forceinline__ float load_f32(const T * p);
template <> __device__ __forceinline__ float load_f32<float>(const float * p) { return *p; }
template <> __device__ __forceinline__ float load_f32<uint16_t>(const uint16_t * p) {
    return bf16_to_f32(*p);
}
template <typename T> __device__ __forceinline__ void store_f32(T * p, float v);
template <> __device__ __forceinline__ void store_f32<float>(float * p, float v) { *p = v; }
template <> __device__ __forceinline__ void store_f32<uint16_t>(uint16_t * p, float v) {
    *p = f32_to_bf16(v);
}

// Device-coherent stores (sc1): written through to the level every XCD reads
// with device-coherent loads, for data that other workgroups of the same
// launch consume.  A wave that has issued them waits with release_stores()
// before the workgroup publishes a flag.
template <typename T> __device__ __forceinline__ void store_f32_coherent(T * p, float v);
template <> __device__ __forceinline__ void store_f32_coherent<float>(float * p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <> __device__ __forceinline__ void store_f32_coherent<uint16_t>(uint16_t * p, float v) {
    const uint32_t bits = f32_to_bf16(v);
    asm volatile("global_store_short %0, %1, off sc1" : : "v"(p), "v"(bits) : "memory");
}
__device__ __forceinline__ void store16_coherent(void * p, uint4 v) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 d = {v.x, v.y, v.z, v.w};
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(d) : "memory");
}
__device__ __forceinline__ void release_stores() { asm volatile("s_waitcnt vmcnt(0)" : : : "memory"); }

// ---- LDS DMA pipelines ----------------------------------------------------------
// LDS byte offset of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_offset(const void * p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
        (const __attribute__((address_space(3))) char *)(p)));
}

// 16 bytes per lane from global memory into LDS (global_load_lds_dwordx4):
// lane l writes lds_base + 16 l, lds_base wave-uniform.  Written as inline
// asm: the compiler then neither counts it nor makes later LDS reads wait for
// it (it cannot prove that a read of one ring stage misses the stage being
// filled, and would drain the whole pipeline); the caller waits with
// s_waitcnt vmcnt and a workgroup barrier before reading the data.
// No "memory" clobber: the stage it fills was released by a barrier_no_fence
// (whose clobbers keep earlier LDS reads before it), and the source is never
// written by the kernels that use it.
__device__ __forceinline__ void lds_dma16(const void * g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(g), "s"(lds_base)
                 : "m0");
}

// lds_dma16 as a device-coherent load (sc1): it reads the level where data
// that other workgroups of the same launch, on other XCDs, have released
// (written back and flagged) is visible, instead of a line this XCD's L2 may
// still hold from before.
__device__ __forceinline__ void lds_dma16_coherent(const void * g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1"
                 :
                 : "v"(g), "s"(lds_base)
                 : "m0");
}

// A wave-uniform pointer the compiler cannot prove uniform, as a scalar value
// (lane 0's, which every lane holds): the operand lds_dma16_sbase needs in
// SGPRs.
__device__ __forceinline__ const char * uniform_ptr(const char * p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<const char *>((static_cast<uint64_t>(hi) << 32) | lo);
}

// lds_dma16 with a wave-uniform base in SGPRs and a per-lane 32-bit byte
// offset (the instruction's saddr form): a loop that walks the base keeps its
// per-lane offsets fixed and advances the base with scalar arithmetic.
__device__ __forceinline__ void lds_dma16_sbase(const void * sbase, uint32_t voff,
                                                uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds_base)
                 : "m0");
}

// lds_dma16 for the lanes set in `lanes` only (EXEC narrowed inside the asm
// and restored after it); the other lanes leave their 16 LDS bytes as they
// were.  `lanes` must not be empty: the instruction is then always issued, so
// the caller's vmcnt bookkeeping holds.
__device__ __forceinline__ void lds_dma16_masked(const void * g, uint32_t lds_base,
                                                 uint64_t lanes) {
    uint64_t saved;
    asm volatile("s_mov_b64 %0, exec\n\ts_and_b64 exec, exec, %3\n\ts_mov_b32 m0, %2\n\t"
                 "s_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b64 exec, %0"
                 : "=&s"(saved)
                 : "v"(g), "s"(lds_base), "s"(lanes)
                 : "m0", "scc");
}

// Workgroup barrier without __syncthreads' release/acquire fences (which wait
// for every outstanding global load, prefetches included).  It waits for the
// wave's own LDS accesses (lgkmcnt 0), so no wave refills a stage another is
// still reading; callers wait for their LDS DMA (vmcnt) first.  The empty asm
// statements keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void barrier_no_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt unbounded
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) with expcnt/lgkmcnt at their maxima: waits until at most
// n of the wave's vector-memory instructions (LDS DMA included) are in flight.
__device__ __forceinline__ void wait_vmcnt(int n) {
    switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
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
    case 16: __builtin_amdgcn_s_waitcnt(0x4F70); break;
    case 17: __builtin_amdgcn_s_waitcnt(0x4F71); break;
    case 18: __builtin_amdgcn_s_waitcnt(0x4F72); break;
    case 19: __builtin_amdgcn_s_waitcnt(0x4F73); break;
    case 20: __builtin_amdgcn_s_waitcnt(0x4F74); break;
    case 21: __builtin_amdgcn_s_waitcnt(0x4F75); break;
    case 22: __builtin_amdgcn_s_waitcnt(0x4F76); break;
    case 23: __builtin_amdgcn_s_waitcnt(0x4F77); break;
    case 24: __builtin_amdgcn_s_waitcnt(0x4F78); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    }
}

// Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
// contiguous range of logical tiles so neighbouring tiles (which share
// operand rows and weights) share one L2.
__device__ __forceinline__ int remap_xcd(int bid, int blocks) {
    const int q = blocks / 8, rem = blocks % 8;
    const int xcd = bid % 8, slot = bid / 8;
    return (xcd < rem) ? xcd * (q + 1) + slot : rem * (q + 1) + (xcd - rem) * q + slot;
}

// ---- dense voxel grid cells ---------------------------------------------------
// The row a cell of a dense voxel grid holds, or -1.  generation 0: a plain
// grid (pxs_voxel_grid_build), each cell the row or INT_MAX; 1..255: a
// generation-tagged grid (pxs_voxel_grid_tagged_insert), each cell
// (255 - generation) << 24 | row, other tags being other builds.
constexpr uint32_t kVoxelGridEmpty = 0x7FFFFFFFu;
constexpr uint32_t kVoxelTagShift = 24;
constexpr uint32_t kVoxelTagMax = 255;
__device__ __forceinline__ int32_t voxel_grid_row(uint32_t cell, uint32_t generation) {
    if (generation == 0) return cell == kVoxelGridEmpty ? -1 : static_cast<int32_t>(cell);
    return (cell >> kVoxelTagShift) == kVoxelTagMax - generation
               ? static_cast<int32_t>(cell & ((1u << kVoxelTagShift) - 1u))
               : -1;
}

// ---- math helpers ------------------------------------------------------------
__device__ __forceinline__ float gelu_tanh_f(float v) {
    const float k = 0.7978845608028654f;
    const float cubic = v * v * v;
    return 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * cubic)));
}

__device__ __forceinline__ float silu_f(float v) { return v * (1.0f / (1.0f + expf(-v))); }

// Voxel key packing: (batch, x, y, z) -> 16 bits each.  Lexicographic order
// of (b, x, y, z) equals numeric order of the key.  All-ones is the empty
// slot marker; it is unreachable because batch and spatial extents are
// limited to PXS_MAX_EXTENT (< 0xFFFF).
__host__ __device__ __forceinline__ uint64_t voxel_key(int32_t b, int32_t x, int32_t y, int32_t z) {
    return (static_cast<uint64_t>(static_cast<uint32_t>(b) & 0xFFFFu) << 48) |
           (static_cast<uint64_t>(static_cast<uint32_t>(x) & 0xFFFFu) << 32) |
           (static_cast<uint64_t>(static_cast<uint32_t>(y) & 0xFFFFu) << 16) |
           static_cast<uint64_t>(static_cast<uint32_t>(z) & 0xFFFFu);
}

constexpr uint64_t kEmptyKey = ~0ull;

__device__ __forceinline__ uint64_t mix64(uint64_t k) {
    // MurmurHash3 fmix64 finalizer.
    k ^= k >> 33;
    k *= 0xff51afd7ed558ccdull;
    k ^= k >> 33;
    k *= 0xc4ceb9fe1a85ec53ull;
    k ^= k >> 33;
    return k;
}

} // namespace pxs
