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

// One tensor to upload: its payload (F32, F16 or BF16) converted to dtype
// (PXS_F32 or PXS_BF16) at dst (16-byte aligned, the tensor's element count
// in dtype); flag is its non-finite flag slot.
struct IngestItem {
    const GgufTensor * tensor;
    int dtype;
    void * dst;
    size_t flag;
};

// One upload session over an open pack.  run() streams the items (in
// increasing file order, as the tensor table lists them): consecutive
// payloads share 16 MiB chunks, each chunk is one file read (split over
// reader threads when large) and one DMA, the next chunk's read overlapping
// the previous chunk's DMA and conversions.  finish() waits for the stream
// and returns, per flag slot, whether any converted value was non-finite.
class Ingest {
public:
    Ingest(pxs_pack * pack, void * workspace, size_t flags, hipStream_t stream)
        : pack_(pack), workspace_(workspace), flags_(flags), stream_(stream) {}
    ~Ingest();

    int begin();
    int run(const std::vector<IngestItem> & items);
    int finish(std::vector<int32_t> & nonfinite);

private:
    struct Segment {
        size_t item;
        uint64_t chunk_offset;    // bytes into the chunk
        uint64_t first_element;   // element offset within the tensor
        int64_t elements;
    };
    int flush(uint64_t begin, uint64_t end, const std::vector<IngestItem> & items,
              const std::vector<Segment> & segs);

    pxs_pack * pack_;
    void * workspace_;
    size_t flags_;
    hipStream_t stream_;
    hipEvent_t done_[2] = {nullptr, nullptr};
    bool pending_[2] = {false, false};
    int slot_ = 0;
};

} // namespace pxs
