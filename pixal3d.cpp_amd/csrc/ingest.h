// The pack upload path: tensor payloads stream file -> pinned host staging
// -> HBM staging -> conversion kernel -> destination, two chunks in flight.
#pragma once

#include "pack_file.h"
#include "pxs_common.h"

#include <vector>

namespace pxs {

// Bytes per staging chunk (host and device, two of each).
constexpr size_t kIngestChunk = size_t(16) << 20;

// Device workspace of an upload session with room for `flags` per-tensor
// non-finite flags.
size_t ingest_workspace_bytes(size_t flags);

// One upload session over an open pack.  upload() enqueues a tensor's
// conversion (F32, F16 or BF16 payload -> PXS_F32 or PXS_BF16 at dst) on the
// stream, reading the file while the previous chunk is in flight; finish()
// waits for the stream and returns, per flag slot, whether any converted
// value was non-finite.  The destination of every upload must be 16-byte
// aligned and hold the tensor's element count in the target dtype.
class Ingest {
public:
    Ingest(pxs_pack * pack, void * workspace, size_t flags, hipStream_t stream)
        : pack_(pack), workspace_(workspace), flags_(flags), stream_(stream) {}
    ~Ingest();

    int begin();
    int upload(const GgufTensor & t, int dtype, void * dst, size_t flag);
    int finish(std::vector<int32_t> & nonfinite);

private:
    pxs_pack * pack_;
    void * workspace_;
    size_t flags_;
    hipStream_t stream_;
    hipEvent_t done_[2] = {nullptr, nullptr};
    bool pending_[2] = {false, false};
    int slot_ = 0;
};

} // namespace pxs
