// Host-side helpers shared by the device compositions (transformer block, flow
// forward, decoder blocks): workspace carving and status propagation.
#pragma once

#include <cstddef>
#include <cstdint>

#include "pxs.h"

namespace pxs {

constexpr size_t kCarveAlign = 256;

inline size_t align_up(size_t v) { return (v + kCarveAlign - 1) / kCarveAlign * kCarveAlign; }

inline size_t dtype_bytes(int dtype) { return dtype == PXS_BF16 ? 2 : 4; }

// Carves aligned sub-buffers out of a caller workspace, in a fixed order, so
// the size query (constructed with nullptr) and the call agree by construction.
class Carver {
public:
    explicit Carver(void * base) : base_(static_cast<char *>(base)) {}
    void * take(size_t bytes) {
        void * p = base_ ? base_ + used_ : nullptr;
        used_ += align_up(bytes);
        return p;
    }
    size_t used() const { return used_; }

private:
    char * base_;
    size_t used_ = 0;
};

} // namespace pxs

#define PXS_TRY(expr)                     \
    do {                                  \
        if (int rc_ = (expr)) return rc_; \
    } while (0)
