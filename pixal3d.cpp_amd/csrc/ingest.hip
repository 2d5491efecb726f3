// Pack tensor upload with conversion on the device (the ingestion half of
// SLatFlowModel::load / SLatDecoderModel::load, src/slat_flow.cpp:1239-1281,
// src/slat_decoder.cpp:3392-3467, whose read_tensor_f32 widens F16 / BF16
// payloads on the host: src/slat_flow.cpp:360-395).
//
// Payloads stream in 16 MiB chunks that consecutive tensors share: one file
// read into pinned host staging (split over four reader threads when large),
// one DMA to HBM staging, one conversion launch per tensor piece, with the
// next chunk's read overlapping the previous chunk's DMA and conversions
// (two chunks in flight).  The kernel is HBM-bound elementwise work: 8
// elements per thread, 16-byte loads and stores.
//
// Conversions are exact or round to nearest even, independent of the
// device's denormal modes: F16 is widened with integer operations (a
// subnormal half m * 2^-24 is the exact product of two floats), BF16 is the
// high half of a float, F32 -> BF16 rounds to nearest even with the carry
// trick on the bit pattern (NaN stays a quiet NaN).  A non-finite value sets
// the tensor's flag; the host reports the first flagged tensor.

#include "ingest.h"

#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <thread>

#pragma clang fp contract(off)

namespace pxs {
namespace {

constexpr int kIngestThreads = 256;

__device__ __forceinline__ uint32_t f16_to_f32_bits(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0x1fu) return sign | 0x7f800000u | (m << 13);
    if (e != 0u) return sign | ((e + 112u) << 23) | (m << 13);
    if (m == 0u) return sign;
    return sign | __float_as_uint(static_cast<float>(m) * 0x1p-24f);
}

__device__ __forceinline__ uint32_t f32_bits_to_bf16(uint32_t b) {
    if ((b & 0x7fffffffu) > 0x7f800000u) return (b >> 16) | 0x40u;
    return (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
}

// SRC: storage of the payload (kGgmlF32, kGgmlF16, kGgmlBf16);
// DST: PXS_F32 or PXS_BF16.  n elements of src -> dst; flag set if any is
// non-finite.
template <uint32_t SRC, int DST>
__global__ void __launch_bounds__(kIngestThreads)
ingest_convert_kernel(const uint8_t * __restrict__ src, int64_t n, void * __restrict__ dst,
                      int32_t * __restrict__ flag) {
    const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kIngestThreads + threadIdx.x) * 8;
    if (i0 >= n) return;
    const int cnt = static_cast<int>(min<int64_t>(8, n - i0));
    uint32_t v[8];
    if (cnt == 8) {
        if constexpr (SRC == kGgmlF32) {
            const uint4 a = *reinterpret_cast<const uint4 *>(src + i0 * 4);
            const uint4 b = *reinterpret_cast<const uint4 *>(src + i0 * 4 + 16);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
            const uint4 a = *reinterpret_cast<const uint4 *>(src + i0 * 2);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[2 * k] = w[k] & 0xffffu;
                v[2 * k + 1] = w[k] >> 16;
            }
        }
    } else {
        for (int k = 0; k < 8; ++k) {
            if (k < cnt) {
                if constexpr (SRC == kGgmlF32) {
                    v[k] = reinterpret_cast<const uint32_t *>(src)[i0 + k];
                } else {
                    v[k] = reinterpret_cast<const uint16_t *>(src)[i0 + k];
                }
            } else {
                v[k] = 0u;
            }
        }
    }
    bool bad = false;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        if constexpr (SRC == kGgmlF16) v[k] = f16_to_f32_bits(v[k]);
        if constexpr (SRC == kGgmlBf16) v[k] <<= 16;
        bad = bad || (k < cnt && (v[k] & 0x7f800000u) == 0x7f800000u);
    }
    if constexpr (DST == PXS_F32) {
        uint32_t * out = static_cast<uint32_t *>(dst) + i0;
        if (cnt == 8) {
            reinterpret_cast<uint4 *>(out)[0] = make_uint4(v[0], v[1], v[2], v[3]);
            reinterpret_cast<uint4 *>(out)[1] = make_uint4(v[4], v[5], v[6], v[7]);
        } else {
            for (int k = 0; k < cnt; ++k) out[k] = v[k];
        }
    } else {
        uint16_t * out = static_cast<uint16_t *>(dst) + i0;
        uint32_t h[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            h[k] = SRC == kGgmlBf16 ? (v[k] >> 16) : f32_bits_to_bf16(v[k]);
            // a finite F32 above the bf16 range rounds to infinity
            bad = bad || (k < cnt && (h[k] & 0x7f80u) == 0x7f80u);
        }
        if (cnt == 8) {
            *reinterpret_cast<uint4 *>(out) =
                make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                           h[6] | (h[7] << 16));
        } else {
            for (int k = 0; k < cnt; ++k) out[k] = static_cast<uint16_t>(h[k]);
        }
    }
    if (bad) *flag = 1;
}

template <uint32_t SRC>
int launch_convert(const uint8_t * src, int64_t n, int dtype, void * dst, int32_t * flag,
                   hipStream_t stream) {
    const unsigned grid = grid_for((n + 7) / 8, kIngestThreads);
    if (dtype == PXS_F32) {
        ingest_convert_kernel<SRC, PXS_F32><<<grid, kIngestThreads, 0, stream>>>(src, n, dst, flag);
    } else {
        ingest_convert_kernel<SRC, PXS_BF16><<<grid, kIngestThreads, 0, stream>>>(src, n, dst,
                                                                                 flag);
    }
    return check_launch("ingest_convert_kernel");
}

size_t stage_bytes() { return 2 * kIngestChunk; }

} // namespace

size_t ingest_workspace_bytes(size_t flags) {
    return stage_bytes() + (std::max<size_t>(flags, 1) * sizeof(int32_t) + 255) / 256 * 256;
}

Ingest::~Ingest() {
    for (int s = 0; s < 2; ++s) {
        if (done_[s]) {
            if (pending_[s]) (void)hipEventSynchronize(done_[s]);
            (void)hipEventDestroy(done_[s]);
        }
    }
}

int Ingest::begin() {
    if (!pack_->host_stage) {
        int rc = check_hip(hipHostMalloc(&pack_->host_stage, stage_bytes(), hipHostMallocDefault),
                           "hipHostMalloc(pack staging)");
        if (rc != PXS_OK) {
            pack_->host_stage = nullptr;
            return rc;
        }
    }
    for (int s = 0; s < 2; ++s) {
        if (!done_[s]) {
            int rc = check_hip(hipEventCreateWithFlags(&done_[s], hipEventDisableTiming),
                               "hipEventCreate(pack staging)");
            if (rc != PXS_OK) return rc;
        }
    }
    auto * flags = reinterpret_cast<int32_t *>(static_cast<uint8_t *>(workspace_) + stage_bytes());
    return check_hip(hipMemsetAsync(flags, 0, flags_ * sizeof(int32_t), stream_),
                     "hipMemsetAsync(pack flags)");
}

namespace {

// pread of [offset, offset + n) into dst, retried on short reads.
bool read_range(int fd, uint64_t offset, uint8_t * dst, size_t n) {
    while (n > 0) {
        const ssize_t got = ::pread(fd, dst, n, static_cast<off_t>(offset));
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return false;
        dst += got;
        offset += static_cast<uint64_t>(got);
        n -= static_cast<size_t>(got);
    }
    return true;
}

// A large read is split over reader threads: one thread copying out of the
// page cache tops out well below the host link's DMA rate.
constexpr int kReaders = 4;
constexpr size_t kSplitBytes = size_t(4) << 20;

bool read_parallel(int fd, uint64_t offset, uint8_t * dst, size_t n) {
    if (n < kSplitBytes) return read_range(fd, offset, dst, n);
    const size_t part = (n / kReaders + 4095) / 4096 * 4096;
    bool ok[kReaders] = {};
    std::thread workers[kReaders - 1];
    int started = 1;  // parts [0, started) have a reader; the rest are read here
    try {
        for (int r = 1; r < kReaders; ++r, ++started) {
            const size_t a = std::min(n, r * part), b = std::min(n, (r + 1) * part);
            workers[r - 1] = std::thread([&, r, a, b] { ok[r] = read_range(fd, offset + a, dst + a, b - a); });
        }
    } catch (...) {
        // No thread to be had: the parts without one are read on this thread.
    }
    ok[0] = read_range(fd, offset, dst, std::min(n, part));
    for (int r = started; r < kReaders; ++r) {
        const size_t a = std::min(n, r * part), b = std::min(n, (r + 1) * part);
        ok[r] = read_range(fd, offset + a, dst + a, b - a);
    }
    for (int r = 1; r < started; ++r) workers[r - 1].join();
    for (bool v : ok) {
        if (!v) return false;
    }
    return true;
}

size_t elem_size(uint32_t type) { return type == kGgmlF32 ? 4 : 2; }

} // namespace

int Ingest::run(const std::vector<IngestItem> & items) {
    for (const IngestItem & it : items) {
        const GgufTensor & t = *it.tensor;
        PXS_CHECK(t.type == kGgmlF32 || t.type == kGgmlF16 || t.type == kGgmlBf16, PXS_ERR_ARG,
                  "pack upload: unsupported tensor type: " + t.name);
        PXS_CHECK(it.dtype == PXS_F32 || it.dtype == PXS_BF16, PXS_ERR_ARG,
                  "pack upload: bad dtype");
        PXS_CHECK(it.flag < flags_, PXS_ERR_ARG, "pack upload: flag slot out of range");
        PXS_CHECK(reinterpret_cast<uintptr_t>(it.dst) % 16 == 0, PXS_ERR_ARG,
                  "pack upload: destination must be 16-byte aligned: " + t.name);
        PXS_CHECK(t.n_bytes % elem_size(t.type) == 0, PXS_ERR_ARG,
                  "pack upload: misaligned payload: " + t.name);
    }
    const uint64_t base = pack_->file.data_offset;
    std::vector<Segment> segs;
    uint64_t chunk_begin = 0, chunk_end = 0;
    for (size_t i = 0; i < items.size(); ++i) {
        const GgufTensor & t = *items[i].tensor;
        const uint64_t es = elem_size(t.type);
        uint64_t done = 0;
        while (done < t.n_bytes) {
            const uint64_t at = base + t.offset + done;
            // Pieces keep the kernel's 16-byte accesses aligned: each starts
            // 16-byte aligned in the chunk (the chunk's first piece at 0) and
            // every split falls on a multiple of 8 elements.  A piece opens a
            // new chunk when it is misaligned in the current one, would not
            // fit, or lies before its end (an out-of-order table).
            const uint64_t step = 8 * es;
            if (!segs.empty() &&
                (at < chunk_end || (at - chunk_begin) % 16 != 0 ||
                 (chunk_begin + kIngestChunk - at) / step * step == 0 ||
                 at + std::min<uint64_t>(t.n_bytes - done, step) > chunk_begin + kIngestChunk)) {
                const int rc = flush(chunk_begin, chunk_end, items, segs);
                if (rc != PXS_OK) return rc;
                segs.clear();
            }
            if (segs.empty()) chunk_begin = at;
            const uint64_t room = (chunk_begin + kIngestChunk - at) / step * step;
            const uint64_t take = std::min<uint64_t>(t.n_bytes - done, room);
            segs.push_back({i, at - chunk_begin, done / es, static_cast<int64_t>(take / es)});
            chunk_end = at + take;
            done += take;
        }
    }
    if (!segs.empty()) return flush(chunk_begin, chunk_end, items, segs);
    return PXS_OK;
}

int Ingest::flush(uint64_t begin, uint64_t end, const std::vector<IngestItem> & items,
                  const std::vector<Segment> & segs) {
    const int s = slot_;
    slot_ ^= 1;
    if (pending_[s]) {
        int rc = check_hip(hipEventSynchronize(done_[s]), "hipEventSynchronize(pack staging)");
        if (rc != PXS_OK) return rc;
        pending_[s] = false;
    }
    const size_t bytes = static_cast<size_t>(end - begin);
    auto * host = static_cast<uint8_t *>(pack_->host_stage) + s * kIngestChunk;
    auto * dev = static_cast<uint8_t *>(workspace_) + s * kIngestChunk;
    if (!read_parallel(pack_->fd, begin, host, bytes)) {
        // Name the first tensor the failed range covers.
        return fail(PXS_ERR_ARG, "short read for tensor: " + items[segs.front().item].tensor->name);
    }
    int rc = check_hip(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, stream_),
                       "hipMemcpyAsync(pack staging)");
    if (rc != PXS_OK) return rc;
    auto * flags = reinterpret_cast<int32_t *>(static_cast<uint8_t *>(workspace_) + stage_bytes());
    for (const Segment & g : segs) {
        const IngestItem & it = items[g.item];
        const uint32_t type = it.tensor->type;
        const uint8_t * src = dev + g.chunk_offset;
        void * out = static_cast<uint8_t *>(it.dst) +
                     g.first_element * (it.dtype == PXS_F32 ? 4 : 2);
        int32_t * flag = flags + it.flag;
        rc = type == kGgmlF32   ? launch_convert<kGgmlF32>(src, g.elements, it.dtype, out, flag, stream_)
             : type == kGgmlF16 ? launch_convert<kGgmlF16>(src, g.elements, it.dtype, out, flag, stream_)
                                : launch_convert<kGgmlBf16>(src, g.elements, it.dtype, out, flag, stream_);
        if (rc != PXS_OK) return rc;
    }
    rc = check_hip(hipEventRecord(done_[s], stream_), "hipEventRecord(pack staging)");
    if (rc != PXS_OK) return rc;
    pending_[s] = true;
    return PXS_OK;
}

int Ingest::finish(std::vector<int32_t> & nonfinite) {
    int rc = check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize(pack upload)");
    if (rc != PXS_OK) return rc;
    pending_[0] = pending_[1] = false;
    nonfinite.assign(flags_, 0);
    return check_hip(hipMemcpy(nonfinite.data(), static_cast<uint8_t *>(workspace_) + stage_bytes(),
                               flags_ * sizeof(int32_t), hipMemcpyDeviceToHost),
                     "hipMemcpy(pack flags)");
}

} // namespace pxs

using namespace pxs;

extern "C" {

size_t pxs_pack_upload_workspace_bytes(const pxs_pack * pack) {
    return ingest_workspace_bytes(pack ? pack->file.tensors.size() : 1);
}

int pxs_pack_upload(pxs_pack * pack, const char * name, int dtype, void * dst, int64_t count,
                    void * workspace, void * stream) {
    return pxs::guarded("pxs_pack_upload", [&]() -> int {
        PXS_CHECK(pack && name && workspace, PXS_ERR_ARG, "pxs_pack_upload: null argument");
        PXS_CHECK_WORKSPACE(workspace, "pxs_pack_upload");
        const GgufTensor * t = pack->file.tensor(name);
        PXS_CHECK(t, PXS_ERR_ARG, std::string("tensor not found: ") + name);
        PXS_CHECK(t->type == kGgmlF32 || t->type == kGgmlF16 || t->type == kGgmlBf16, PXS_ERR_ARG,
                  std::string("pxs_pack_upload: tensor ") + name + " has type " +
                      ggml_type_name(t->type) + ", not f32, f16 or bf16");
        PXS_CHECK(dtype == PXS_F32 || dtype == PXS_BF16, PXS_ERR_ARG, "pxs_pack_upload: bad dtype");
        const uint64_t esize = t->type == kGgmlF32 ? 4 : 2;
        const int64_t elements = static_cast<int64_t>(t->n_bytes / esize);
        PXS_CHECK(count == elements, PXS_ERR_ARG,
                  std::string("pxs_pack_upload: ") + name + " holds " + std::to_string(elements) +
                      " elements, not " + std::to_string(count));
        PXS_CHECK(dst || elements == 0, PXS_ERR_ARG, "pxs_pack_upload: null destination");
        if (elements == 0) return PXS_OK;
        Ingest ingest(pack, workspace, 1, as_stream(stream));
        int rc = ingest.begin();
        if (rc != PXS_OK) return rc;  // nothing enqueued
        rc = ingest.run({IngestItem{t, dtype, dst, 0}});
        std::vector<int32_t> flags;
        const int frc = ingest.finish(flags);
        if (rc != PXS_OK) return rc;
        if (frc != PXS_OK) return frc;
        PXS_CHECK(!flags[0], PXS_ERR_DATA, std::string("tensor contains a non-finite value: ") + name);
        return PXS_OK;
    });
}

} // extern "C"
